"""Weight stores on the CPU: pinning requests, staging order, checkpoint
loading and the seeded random filler.

The first three tests restate the reference's (tests/test_weight_store.py:
67-108) with the same tiny plan, recording factory and fake event.
"""

import pytest
import torch

from layer_streaming.plan import (
    ModelPlan,
    ResidentPlacement,
    TensorSpec,
    TransferUnit,
    UnitPiece,
)
from layer_streaming.weight_store import (
    FullPinnedWeightStore,
    PinnedStagingWeightStore,
    create_weight_store,
    tensor_seed,
)


def tiny_plan():
    streamed = TensorSpec("stream.weight", (2, 2))
    resident = TensorSpec("resident.weight", (2,), resident=True)
    unit = TransferUnit(
        unit_id="unit", layer_index=0, operation="q_proj",
        pieces=(UnitPiece(streamed, 0),), elements=4, host_offset_elements=0,
    )
    placement = ResidentPlacement(tensor=resident, host_offset_elements=4,
                                  device_offset_elements=0)
    return ModelPlan(
        model_id="tiny", granularity="matrix",
        tensors={streamed.key: streamed, resident.key: resident},
        units=(unit,), resident=(placement,), aliases={},
        host_arena_elements=6, resident_arena_elements=2, slot_elements=4,
    )


class RecordingFactory:
    def __init__(self):
        self.pin_flags = []

    def __call__(self, elements, **kwargs):
        self.pin_flags.append(bool(kwargs.pop("pin_memory")))
        return torch.empty(elements, **kwargs)


class FakeEvent:
    def __init__(self, log=None):
        self.synchronized = False
        self.log = log

    def synchronize(self):
        self.synchronized = True
        if self.log is not None:
            self.log.append("wait")


def test_full_pinned_requests_one_pinned_arena():
    factory = RecordingFactory()
    store = FullPinnedWeightStore(tiny_plan(), tensor_factory=factory)
    assert factory.pin_flags == [True]
    assert store.pinned_cpu_bytes == 12
    store.close()


def test_staging_has_pageable_store_and_two_pinned_slots():
    factory = RecordingFactory()
    plan = tiny_plan()
    store = PinnedStagingWeightStore(plan, tensor_factory=factory)
    assert factory.pin_flags == [False, True, True]
    assert store.pinned_cpu_bytes == plan.two_slot_bytes
    store.close()


def test_staging_copies_unit_and_waits_before_reuse():
    plan = tiny_plan()
    store = PinnedStagingWeightStore(plan, tensor_factory=RecordingFactory())
    store.arena[:4] = torch.tensor([1.0, 2.0, 3.0, 4.0], dtype=torch.bfloat16)
    event = FakeEvent()
    staged = store.prepare_unit(plan.units[0], 0, reuse_event=event).result()
    assert event.synchronized
    assert staged.float().tolist() == [1.0, 2.0, 3.0, 4.0]
    assert store.profile_stats()["staging_copy_count"] == 1
    store.close()


def test_staging_waits_before_it_overwrites_the_slot():
    # the copy into the slot must come after the reuse event's wait
    plan = tiny_plan()
    store = PinnedStagingWeightStore(plan, tensor_factory=RecordingFactory())
    log = []
    store.arena[:4] = 7.0
    slot = store.staging_slots[0]
    slot.fill_(-1.0)

    class OrderedEvent(FakeEvent):
        def synchronize(self):
            log.append(("wait", float(slot[0])))

    store.prepare_unit(plan.units[0], 0, reuse_event=OrderedEvent()).result()
    assert log == [("wait", -1.0)]  # slot untouched at the time of the wait
    assert float(slot[0]) == 7.0
    store.close()


def test_full_pinned_prepare_unit_is_a_resolved_arena_view():
    plan = tiny_plan()
    store = FullPinnedWeightStore(plan, tensor_factory=RecordingFactory())
    fut = store.prepare_unit(plan.units[0], 1)
    assert fut.done()
    assert fut.result().data_ptr() == store.arena.data_ptr()
    store.close()


def test_tensor_views_and_unit_source():
    plan = tiny_plan()
    store = create_weight_store(plan, "full_pinned", tensor_factory=RecordingFactory())
    store.arena.copy_(torch.arange(6, dtype=torch.bfloat16))
    assert store.tensor("stream.weight").tolist() == [[0.0, 1.0], [2.0, 3.0]]
    assert store.tensor("resident.weight").tolist() == [4.0, 5.0]
    assert store.unit_source(plan.units[0]).tolist() == [0.0, 1.0, 2.0, 3.0]
    with pytest.raises(KeyError):
        store.tensor("missing.weight")
    store.close()
    with pytest.raises(RuntimeError):
        store.tensor("stream.weight")


def test_load_checkpoint_checks_keys_and_shapes(tmp_path):
    from safetensors.torch import save_file

    plan = tiny_plan()
    store = create_weight_store(plan, "pinned_staging", tensor_factory=RecordingFactory())
    good = {
        "stream.weight": torch.tensor([[1.0, 2.0], [3.0, 4.0]]),
        "resident.weight": torch.tensor([5.0, 6.0]),
    }
    save_file(good, str(tmp_path / "model.safetensors"))
    store.load_checkpoint(tmp_path)
    assert store.loaded
    assert store.arena.float().tolist() == [1, 2, 3, 4, 5, 6]

    bad = tmp_path / "bad"
    bad.mkdir()
    save_file({"stream.weight": torch.zeros(2, 2)}, str(bad / "model.safetensors"))
    with pytest.raises(KeyError):
        store.load_checkpoint(bad)
    wrong = tmp_path / "wrong"
    wrong.mkdir()
    save_file({"stream.weight": torch.zeros(4), "resident.weight": torch.zeros(2)},
              str(wrong / "model.safetensors"))
    with pytest.raises(ValueError):
        store.load_checkpoint(wrong)
    with pytest.raises(FileNotFoundError):
        store.load_checkpoint(tmp_path / "nothing")
    store.close()


def test_fill_random_is_seeded_per_tensor():
    plan = tiny_plan()
    a = create_weight_store(plan, "full_pinned", tensor_factory=RecordingFactory())
    b = create_weight_store(plan, "full_pinned", tensor_factory=RecordingFactory())
    a.fill_random(seed=3, norm="random")
    b.fill_random(seed=3, norm="random")
    assert torch.equal(a.arena, b.arena)
    gen = torch.Generator().manual_seed(tensor_seed(3, 0))
    expected = (torch.randn(4, generator=gen) * 0.02).to(torch.bfloat16)
    assert torch.equal(a.tensor("stream.weight").reshape(-1), expected)
    c = create_weight_store(plan, "full_pinned", tensor_factory=RecordingFactory())
    c.fill_random(seed=3)  # norms = 1
    assert c.tensor("resident.weight").tolist() == [1.0, 1.0]


def test_staging_ring_packs_small_units_and_waits_for_copies():
    # two 100-byte slots: units of 30, 30, 30 share slot 0; 60 moves on to
    # slot 1; 50 wraps to slot 0 over the first two (their copies must be
    # enqueued, and are waited for); a unit larger than a slot is refused
    from layer_streaming.weight_store import StagingRing

    ring = StagingRing([torch.empty(50, dtype=torch.bfloat16) for _ in range(2)])
    assert ring.place(30, "a")[:2] == (0, 0)
    assert ring.place(30, "b")[:2] == (0, 30)
    assert ring.place(30, "c")[:2] == (0, 60)
    assert ring.place(60, "d")[:2] == (1, 0)
    assert ring.place(50, "e") is None  # a and b not copied yet
    ev_a, ev_b = FakeEvent(), FakeEvent()
    ring.copied("a", ev_a)
    assert ring.place(50, "e") is None  # b still holds bytes 30-59
    ring.copied("b", ev_b)
    slot, start, waits = ring.place(50, "e")
    assert (slot, start) == (0, 0) and waits == [ev_a, ev_b]
    # a (0-29) is wholly covered by e (0-49) and drops out; b (30-59) is
    # only partly covered and stays, as do c and d
    assert [entry[3] for entry in ring.live] == ["b", "c", "d", "e"]
    # the rest of b's bytes: a unit there waits for b's copy again
    # (dropping b on the first overlap let such a unit overwrite bytes
    # whose copy was still in flight)
    slot, start, waits = ring.place(8, "f")
    assert (slot, start) == (0, 50) and waits == [ev_b]
    with pytest.raises(ValueError):
        ring.place(101, "g")
    ring.reset()
    assert ring.place(10, "h")[:2] == (0, 0) and ring.live[0][3] == "h"


def test_staging_in_ring_waits_then_copies():
    plan = tiny_plan()
    store = PinnedStagingWeightStore(plan, tensor_factory=RecordingFactory())
    store.arena[:4] = torch.tensor([1.0, 2.0, 3.0, 4.0], dtype=torch.bfloat16)
    log = []
    slot_index, start, waits = store.staging_ring.place(plan.units[0].nbytes, 0)
    staged = store.stage_in_ring(plan.units[0], slot_index, start,
                                 [FakeEvent(log), FakeEvent(log)]).result()
    assert log == ["wait", "wait"]
    assert staged.float().tolist() == [1.0, 2.0, 3.0, 4.0]
    assert staged.data_ptr() == store.staging_slots[slot_index].data_ptr()
    store.close()
