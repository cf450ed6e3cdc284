"""DoubleBufferRuntime's copy / compute ordering on the CPU, with streams,
events and the H2D copy replaced by recording doubles (copies complete at
once, so a compute that runs before its copy sees stale slot bytes).

Checked: every unit computes on its own weights; the host waits for copy i
before it enqueues compute i; a copy into a slot waits for the event of the
slot's last reader (with one slot: copy i + 1 waits for compute i); the next
call's first units are copied ahead (full_pinned) and reused, not copied
again, unless the store reloaded, refilled or freed its arena since (its
generation), in which case the store first drains the copy stream; a run
that raises part-way is drained (staging jobs, both streams) before the next
run reuses the slots, which then compute on the right weights (reference
ordering: runtime.py:93-106, :185-236).
"""

import contextlib

import pytest
import torch

from layer_streaming import _hip
from layer_streaming import runtime as rt
from layer_streaming.plan import build_llama31_8b_plan
from layer_streaming.weight_store import (
    FullPinnedWeightStore,
    PinnedStagingWeightStore,
)


class Log(list):
    pass


class FakeStream:
    def __init__(self, log, name):
        self.log, self.name = log, name
        self.cuda_stream = 0

    def synchronize(self):
        self.log.append(("stream_sync", self.name))


class FakeEvent:
    count = 0

    def __init__(self, log, enable_timing=False):
        FakeEvent.count += 1
        self.id = FakeEvent.count
        self.log = log

    def record(self, stream=None):
        self.log.append(("record", self.id, getattr(stream, "name", None)))

    def wait(self, stream=None):
        self.log.append(("wait", self.id, getattr(stream, "name", None)))

    def synchronize(self):
        self.log.append(("sync", self.id))

    def query(self):
        return True

    def elapsed_time(self, other):
        return 1.0


@pytest.fixture
def doubles(monkeypatch):
    log = Log()
    streams = {}

    def stream_factory(device=None):
        name = "copy" if "copy" not in streams else "compute"
        streams[name] = FakeStream(log, name)
        return streams[name]

    coordinator = FakeStream(log, "coordinator")
    monkeypatch.setattr(rt, "_require_gpu", lambda device: torch.device("cpu"))
    monkeypatch.setattr(rt.torch.cuda, "Stream", stream_factory)
    monkeypatch.setattr(rt.torch.cuda, "current_stream", lambda device=None: coordinator)
    monkeypatch.setattr(rt.torch.cuda, "stream", lambda s: contextlib.nullcontext())
    monkeypatch.setattr(_hip, "HipEvent", lambda enable_timing=False: FakeEvent(log))

    def copy(dst, src, nbytes, stream):
        n = nbytes // 2
        dst.view(-1)[:n].copy_(src.reshape(-1)[:n])
        log.append(("copy", dst.data_ptr(), src.data_ptr(), stream.name))

    monkeypatch.setattr(_hip, "memcpy_h2d_async", copy)
    return log


def cpu_factory(n, **kw):
    kw.pop("pin_memory")
    return torch.empty(n, **kw)


def tiny_plan():
    # one full-width layer: the arena is allocated lazily and only the ends
    # of each tensor are written
    return build_llama31_8b_plan("matrix_group", num_layers=1, stream_vocab=True)


class UnitChecker:
    """compute_unit double: each unit's first and last weight elements must
    be that unit's host bytes (a copy not yet done would leave old bytes)."""

    def __init__(self, store, log, fail_at=None):
        self.store, self.log, self.fail_at = store, log, fail_at
        self.seen = []

    def __call__(self, unit, views, state):
        self.log.append(("compute", unit.unit_id))
        for piece in unit.pieces:
            key = piece.tensor.key
            got = views[key].reshape(-1)
            want = self.store.tensor(key).reshape(-1)
            assert torch.equal(got[:4], want[:4]) and torch.equal(got[-4:], want[-4:]), key
        if self.fail_at == len(self.seen):
            self.seen.append(unit.unit_id)
            raise RuntimeError("planted failure")
        self.seen.append(unit.unit_id)
        return state


def mark_units(store, base=0):
    # distinct values at both ends of every tensor (the rest stays as is)
    for index, (key, spec) in enumerate(store.plan.tensors.items()):
        if spec.alias_of is None:
            flat = store.tensor(key).reshape(-1)
            flat[:4] = float(base + index + 1)
            flat[-4:] = -float(base + index + 1)


def events_of(log, kind):
    return [entry for entry in log if entry[0] == kind]


def test_host_handoff_and_slot_waits(doubles):
    plan = tiny_plan()
    store = FullPinnedWeightStore(plan, tensor_factory=cpu_factory)
    mark_units(store)
    runtime = rt.DoubleBufferRuntime(plan, store, resident=None, device="cpu")
    check = UnitChecker(store, doubles)
    runtime.run(check, state=None)
    assert check.seen == [u.unit_id for u in plan.units]
    # compute i comes after the host waited for copy i's event, and no
    # compute-stream wait on a copy-stream event exists
    computes = [i for i, e in enumerate(doubles) if e[0] == "compute"]
    syncs = [i for i, e in enumerate(doubles) if e[0] == "sync"]
    assert len(syncs) >= len(plan.units)
    for c, s in zip(computes, syncs):
        assert s < c
    assert not [e for e in doubles if e[0] == "wait" and e[2] == "compute"
                and e[1] in {ev.id for ev in runtime._ready}]
    # unit i + 2 waits for unit i's free event before its copy
    free_ids = [ev.id for ev in runtime._free]
    waits = [e[1] for e in doubles if e[0] == "wait" and e[2] == "copy"]
    assert waits[:2] == free_ids[:2]
    store.close()


def test_next_call_first_units_are_prefetched_and_reused(doubles):
    plan = tiny_plan()
    store = FullPinnedWeightStore(plan, tensor_factory=cpu_factory)
    mark_units(store)
    runtime = rt.DoubleBufferRuntime(plan, store, resident=None, device="cpu")
    runtime.run(UnitChecker(store, doubles), state=None)
    first_call_copies = len(events_of(doubles, "copy"))
    # the last units released the slots: units 0 and 1 are copied ahead
    assert first_call_copies == len(plan.units) + 2
    assert runtime.slot_holding(0, "unit", 0) is runtime._ready[0]
    del doubles[:]
    check = UnitChecker(store, doubles)
    runtime.run(check, state=None)
    assert check.seen == [u.unit_id for u in plan.units]
    # this call copied units 2.. only (0 and 1 were in place), then the
    # next call's 0 and 1 again
    assert len(events_of(doubles, "copy")) == len(plan.units)
    # weights changed on the host: forget the slots, copy again
    runtime.discard_slots()
    del doubles[:]
    runtime.run(UnitChecker(store, doubles), state=None)
    assert len(events_of(doubles, "copy")) == len(plan.units) + 2
    store.close()


def test_run_that_raised_is_drained_before_reuse(doubles):
    plan = build_llama31_8b_plan("matrix", num_layers=1, stream_vocab=True)
    store = PinnedStagingWeightStore(plan, tensor_factory=cpu_factory)
    mark_units(store)
    runtime = rt.DoubleBufferRuntime(plan, store, resident=None, device="cpu",
                                     profile=False)
    with pytest.raises(RuntimeError, match="planted"):
        runtime.run(UnitChecker(store, doubles, fail_at=3), state=None)
    del doubles[:]
    check = UnitChecker(store, doubles)
    runtime.run(check, state=None)
    # both streams were drained before the first copy, and every unit
    # computed on its bytes
    first_copy = next(i for i, e in enumerate(doubles) if e[0] == "copy")
    drained = [e for e in doubles[:first_copy] if e[0] == "stream_sync"]
    assert drained == [("stream_sync", "copy"), ("stream_sync", "compute")]
    assert check.seen == [u.unit_id for u in plan.units]
    # a clean run leaves nothing to drain
    del doubles[:]
    runtime.run(UnitChecker(store, doubles), state=None)
    assert ("stream_sync", "copy") not in doubles
    store.close()


@pytest.mark.parametrize("mode", ["full_pinned", "pinned_staging"])
def test_single_slot_copy_waits_for_previous_compute(doubles, mode):
    # reference runtime.py:93-106 accepts one slot: unit i + 1 then reuses
    # unit i's slot, so its copy must wait for compute i
    plan = build_llama31_8b_plan("matrix_group", num_layers=1, stream_vocab=False)
    store_cls = FullPinnedWeightStore if mode == "full_pinned" else PinnedStagingWeightStore
    store = store_cls(plan, tensor_factory=cpu_factory)
    mark_units(store)
    runtime = rt.DoubleBufferRuntime(plan, store, resident=None, device="cpu",
                                     slot_count=1)
    assert len(runtime.device_slots) == 1 and runtime.stats.device_slot_count == 1
    for call in range(2):
        del doubles[:]
        check = UnitChecker(store, doubles)
        runtime.run(check, state=None)
        assert check.seen == [u.unit_id for u in plan.units]
        # every copy-stream wait names the free event of a unit whose
        # compute is already recorded: earlier in this call, or (the first
        # copy of a call) the previous call's last unit
        free_ids = {ev.id: i for i, ev in enumerate(runtime._free)}
        waits = [(index, entry) for index, entry in enumerate(doubles)
                 if entry[0] == "wait" and entry[2] == "copy"]
        copies = [index for index, entry in enumerate(doubles) if entry[0] == "copy"]
        # one slot: every copy waits, except the very first copy into the
        # fresh slot
        if call == 0:
            assert copies[0] < waits[0][0]
            copies = copies[1:]
        assert len(waits) == len(copies)
        for (index, entry), copy_at in zip(waits, copies):
            assert index < copy_at
            unit = free_ids[entry[1]]
            record = ("record", entry[1], "compute")
            if record in doubles[:index]:
                computed = doubles.index(("compute", plan.units[unit].unit_id))
                assert computed < doubles.index(record) < index
            else:
                assert index == waits[0][0] and unit == len(plan.units) - 1
    store.close()


def _loading(monkeypatch, log, base):
    # a checkpoint "load" that writes new bytes at the marked positions
    from layer_streaming import weight_store as ws

    def load_into(store, checkpoint):
        log.append(("load", checkpoint))
        mark_units(store, base=base)

    monkeypatch.setattr(ws._checkpoint, "load_into", load_into)


def test_reloaded_store_is_not_served_from_prefetched_slots(doubles, monkeypatch):
    # units 0 and 1 sit in the slots after a run; a checkpoint load (no
    # discard_slots) must drain the copy stream first and make the next run
    # copy them again, computing on the new bytes
    plan = tiny_plan()
    store = FullPinnedWeightStore(plan, tensor_factory=cpu_factory)
    mark_units(store)
    runtime = rt.DoubleBufferRuntime(plan, store, resident=None, device="cpu")
    runtime.run(UnitChecker(store, doubles), state=None)
    assert runtime.slot_holding(0, "unit", 0) is not None
    generation = store.generation
    del doubles[:]
    _loading(monkeypatch, doubles, base=1000)
    store.load_checkpoint("weights.safetensors")
    assert store.generation > generation
    # the runtime's prefetch reading the arena finished before the new bytes
    assert doubles.index(("stream_sync", "copy")) < doubles.index(
        ("load", "weights.safetensors"))
    assert runtime.slot_holding(0, "unit", 0) is None
    del doubles[:]
    check = UnitChecker(store, doubles)
    runtime.run(check, state=None)
    assert check.seen == [u.unit_id for u in plan.units]
    assert len(events_of(doubles, "copy")) == len(plan.units) + 2
    store.close()


def test_store_close_drains_the_runtime_copies(doubles):
    plan = tiny_plan()
    store = FullPinnedWeightStore(plan, tensor_factory=cpu_factory)
    mark_units(store)
    runtime = rt.DoubleBufferRuntime(plan, store, resident=None, device="cpu")
    runtime.run(UnitChecker(store, doubles), state=None)
    del doubles[:]
    store.close()
    # the copies of the next call's first units (still reading the arena)
    # were waited for before the arena was dropped
    assert doubles == [("stream_sync", "copy")]
    assert store.arena is None and runtime.slot_holding(0, "unit", 0) is None


def _staged_runtime(doubles):
    plan = build_llama31_8b_plan("matrix", num_layers=1, stream_vocab=True)
    store = PinnedStagingWeightStore(plan, tensor_factory=cpu_factory)
    mark_units(store)
    runtime = rt.DoubleBufferRuntime(plan, store, resident=None, device="cpu")
    return plan, store, runtime


def _stage_and_copy_ahead(runtime):
    # what VocabStreamingRuntime does at the end of a call: stage the next
    # call's first units, then copy them as the last chunks free the slots
    runtime.stage_call_ahead()
    for i in (0, 1):
        runtime._ahead.staged[i].result()
        runtime.prefetch_next_call(i)


def test_staged_next_call_is_staged_and_copied_ahead(doubles):
    plan, store, runtime = _staged_runtime(doubles)
    runtime.run(UnitChecker(store, doubles), state=None)
    del doubles[:]
    _stage_and_copy_ahead(runtime)
    assert len(events_of(doubles, "copy")) == 2
    assert runtime.slot_holding(0, "unit", 0) is runtime._ready[0]
    # a second request changes nothing
    runtime.stage_call_ahead()
    runtime.prefetch_next_call(0)
    assert len(events_of(doubles, "copy")) == 2
    del doubles[:]
    check = UnitChecker(store, doubles)
    runtime.run(check, state=None)
    assert check.seen == [u.unit_id for u in plan.units]
    # units 0 and 1 were in place: this call copied the others only, and
    # every unit was staged exactly once for it
    assert len(events_of(doubles, "copy")) == len(plan.units) - 2
    assert store.profile_stats()["staging_copy_count"] == len(plan.units)
    # and the next call again
    _stage_and_copy_ahead(runtime)
    del doubles[:]
    check = UnitChecker(store, doubles)
    runtime.run(check, state=None)
    assert check.seen == [u.unit_id for u in plan.units]
    store.close()


def test_staged_ahead_units_are_dropped_when_the_store_reloads(doubles, monkeypatch):
    plan, store, runtime = _staged_runtime(doubles)
    runtime.run(UnitChecker(store, doubles), state=None)
    _stage_and_copy_ahead(runtime)
    del doubles[:]
    _loading(monkeypatch, doubles, base=500)
    store.load_checkpoint("weights.safetensors")
    # the copies made ahead were waited for before the new bytes
    assert doubles.index(("stream_sync", "copy")) < doubles.index(
        ("load", "weights.safetensors"))
    assert runtime._ahead is None
    del doubles[:]
    check = UnitChecker(store, doubles)  # compares with the new bytes
    runtime.run(check, state=None)
    assert check.seen == [u.unit_id for u in plan.units]
    assert len(events_of(doubles, "copy")) == len(plan.units)
    store.close()


def test_staged_ahead_units_whose_slot_was_taken_are_staged_again(doubles):
    plan, store, runtime = _staged_runtime(doubles)
    runtime.run(UnitChecker(store, doubles), state=None)
    _stage_and_copy_ahead(runtime)
    # an LM-head chunk copied into slot 0 between the calls
    chunk = torch.zeros(64, dtype=torch.bfloat16)
    runtime.slot_copy(0, "chunk", 0, chunk, chunk.numel() * 2, FakeEvent(doubles))
    del doubles[:]
    check = UnitChecker(store, doubles)
    runtime.run(check, state=None)
    assert check.seen == [u.unit_id for u in plan.units]
    assert len(events_of(doubles, "copy")) == len(plan.units)
    store.close()
