"""DoubleBufferRuntime's copy / compute ordering on the CPU, with streams,
events and the H2D copy replaced by recording doubles (copies complete at
once, so a compute that runs before its copy sees stale slot bytes).

Checked: every unit computes on its own weights; the host waits for copy i
before it enqueues compute i; a copy into a slot waits for the event of the
slot's last reader; the next call's first units are copied ahead (full_pinned)
and reused, not copied again; a run that raises part-way is drained (staging
jobs, both streams) before the next run reuses the slots, which then compute
on the right weights (reference ordering: runtime.py:185-236).
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


def mark_units(store):
    # distinct values at both ends of every tensor (the rest stays as is)
    for index, (key, spec) in enumerate(store.plan.tensors.items()):
        if spec.alias_of is None:
            flat = store.tensor(key).reshape(-1)
            flat[:4] = float(index + 1)
            flat[-4:] = -float(index + 1)


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
