"""Device arenas and the two-slot H2D / compute pipeline.

* ``ResidentDeviceArena`` -- device copy of the plan's resident tensors
  (norms, plus embedding / LM head when the vocabulary is resident);
  reference layer_streaming/runtime.py:33-64.
* ``DoubleBufferRuntime`` -- the per-token transfer loop of the reference
  (runtime.py:67-268): unit i is copied host->device into slot i % slots on
  a copy stream while the compute stream runs unit i-1.  The copies are
  hipMemcpyAsync calls and the ready / free handoff uses hipEvents, all
  through libcascade_hip (cascade_memcpy_h2d_async, cascade_event_*).
  Ordering invariants (runtime.py:70-74, :194-230):
    - copy i waits for free[i - slots] (the compute that last read slot i);
    - compute i waits for ready[i];
    - a staging worker may refill host slot i % slots once ready[i] fired.
  In addition both streams wait for the caller's stream at the start of
  run(), so device work the caller enqueued before (e.g. the embedding
  gather) is ordered before the first unit.
* ``ResidentTransformerRuntime`` -- same ``run`` contract with every transfer
  unit resident in HBM (no streaming); the configuration used to measure
  the decode kernels against the HBM roofline.

compute_unit(unit, weight_views, state) enqueues its work on the current
stream and returns the next state; views must not escape the call because a
slot is reused ``slot_count`` units later.
"""

from dataclasses import dataclass
import time

import torch

from . import _hip
from .plan import ModelPlan

__all__ = [
    "RuntimeStats",
    "ResidentDeviceArena",
    "DoubleBufferRuntime",
    "ResidentTransformerRuntime",
]


@dataclass
class RuntimeStats:
    transfer_units: int
    slot_bytes: int
    two_slot_bytes: int
    device_slot_count: int
    device_slots_bytes: int
    resident_bytes: int
    weight_gpu_bytes: int

    def as_dict(self):
        return dict(self.__dict__)


def _require_gpu(device):
    _hip.load()
    if not torch.cuda.is_available():
        raise RuntimeError("no HIP device is available")
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError("the runtime requires a GPU device, got {}".format(device))
    return device


def _copy_to_device(dst, src, stream):
    """H2D copy of a host tensor into a device view (C-ABI hipMemcpyAsync)."""

    src = src.contiguous()
    _hip.memcpy_h2d_async(dst, src, src.numel() * src.element_size(), stream)


class ResidentDeviceArena:
    """GPU allocation for the plan's resident tensors and their aliases."""

    def __init__(self, plan, store, device, fill=True):
        if not isinstance(plan, ModelPlan):
            raise TypeError("plan must be a ModelPlan")
        self.plan = plan
        self.store = store
        self.device = _require_gpu(device)
        self.arena = torch.empty(
            plan.resident_arena_elements, dtype=torch.bfloat16, device=self.device
        )
        self.views = {}
        for placement in plan.resident:
            spec = placement.tensor
            start = placement.device_offset_elements
            self.views[spec.key] = self.arena[start : start + spec.numel].view(
                spec.shape
            )
        for alias, target in plan.aliases.items():
            self.views[alias] = self.views[target]
        if fill and store is not None:
            stream = torch.cuda.current_stream(self.device)
            for placement in plan.resident:
                key = placement.tensor.key
                _copy_to_device(self.views[key], store.tensor(key), stream)
            stream.synchronize()

    @property
    def nbytes(self):
        return self.plan.resident_bytes

    def fill_random(self, seed=0, std=0.02, norm="ones"):
        """Synthetic resident tensors drawn on the device: matrices
        N(0, std) seeded base*1000 + plan index, norm weights 1 (or
        1 + N(0, 0.1) with norm="random")."""

        with torch.inference_mode():
            for placement in self.plan.resident:
                key = placement.tensor.key
                view = self.views[key]
                if view.dim() == 1 and norm == "ones":
                    view.fill_(1.0)
                    continue
                gen = torch.Generator(device=self.device)
                gen.manual_seed(int(seed) * 1000 + self.plan.tensor_index(key))
                flat = view.reshape(-1)
                scale, shift = (0.1, 1.0) if view.dim() == 1 else (std, 0.0)
                step = 1 << 28
                for start in range(0, flat.numel(), step):
                    piece = flat[start : start + step]
                    piece.copy_(torch.randn(piece.numel(), generator=gen,
                                            device=self.device) * scale + shift)
        torch.cuda.synchronize(self.device)
        return self

    def __getitem__(self, key):
        return self.views[key]

    def __contains__(self, key):
        return key in self.views


def _unit_views(unit, base):
    views = {}
    for piece in unit.pieces:
        spec = piece.tensor
        start = piece.unit_offset_elements
        views[spec.key] = base[start : start + spec.numel].view(spec.shape)
    return views


class DoubleBufferRuntime:
    """Two device slots with a copy stream and a compute stream."""

    def __init__(self, plan, store, resident, device="cuda:0", slot_count=None,
                 profile=False):
        self.device = _require_gpu(device)
        self.plan = plan
        self.store = store
        self.resident = resident
        self.slot_count = plan.slot_count if slot_count is None else int(slot_count)
        if self.slot_count not in (1, 2):
            raise ValueError("slot_count must be 1 or 2")
        self.profile = bool(profile)
        self.last_profile = None
        self.device_slots = [
            torch.empty(plan.slot_elements, dtype=torch.bfloat16, device=self.device)
            for _ in range(self.slot_count)
        ]
        self.copy_stream = torch.cuda.Stream(device=self.device)
        self.compute_stream = torch.cuda.Stream(device=self.device)
        # pinned_staging: units staged ahead of the one being copied (ring
        # room permitting)
        self.stage_lookahead = 8
        self._staging_left = {}
        self.coordinator = torch.cuda.current_stream(self.device)
        count = len(plan.units)
        # Events are created once and re-recorded every token (each run()
        # ends with a full synchronisation, so reuse is safe).
        self._ready = [_hip.HipEvent() for _ in range(count)]
        self._free = [_hip.HipEvent() for _ in range(count)]
        self._start = _hip.HipEvent()
        self._timing = None

    @property
    def stats(self):
        return RuntimeStats(
            transfer_units=len(self.plan.units),
            slot_bytes=self.plan.slot_bytes,
            two_slot_bytes=self.plan.two_slot_bytes,
            device_slot_count=self.slot_count,
            device_slots_bytes=self.slot_count * self.plan.slot_bytes,
            resident_bytes=self.plan.resident_bytes,
            weight_gpu_bytes=self.slot_count * self.plan.slot_bytes
            + self.plan.resident_bytes,
        )

    def _timing_events(self):
        if self._timing is None:
            count = len(self.plan.units)

            def make(n):
                return [_hip.HipEvent(enable_timing=True) for _ in range(n)]

            self._timing = {
                "pipeline": make(2),
                "copy_start": make(count),
                "copy_end": make(count),
                "compute_start": make(count),
                "compute_end": make(count),
            }
        return self._timing

    def _unit_views(self, unit, slot):
        return _unit_views(unit, slot)

    def run(self, compute_unit, state):
        wall_started = time.perf_counter()
        units = self.plan.units
        if not units:
            return state
        slots = self.slot_count
        copy_stream = self.copy_stream
        compute_stream = self.compute_stream
        timing = self._timing_events() if self.profile else None

        self._start.record(self.coordinator)
        self._start.wait(copy_stream)
        self._start.wait(compute_stream)
        if timing:
            timing["pipeline"][0].record(self.coordinator)

        self.store.reset_profile()
        staging = self.store.mode.value == "pinned_staging"
        ring = getattr(self.store, "staging_ring", None) if staging else None
        staged = {}
        next_stage = 0
        if ring is None:
            staged = {i: self.store.prepare_unit(units[i], i)
                      for i in range(min(slots, len(units)))}
        else:
            # The ring starts empty: every copy of the previous run is done
            # (a normal run ends synchronised; the copy stream is then idle
            # and this costs nothing), and so is every staging job it left
            # behind if it ended in an exception.
            for future in self._staging_left.values():
                try:
                    future.result()
                except Exception:  # that run already raised
                    pass
            self._staging_left = {}
            copy_stream.synchronize()
            ring.reset()

        def stage_ahead(done):
            # ring staging: units after ``done`` (whose copy is enqueued)
            # go to the staging workers while the ring has room for them
            nonlocal next_stage
            while next_stage < len(units) and next_stage - done <= self.stage_lookahead:
                placed = ring.place(units[next_stage].nbytes, next_stage)
                if placed is None:
                    break
                staged[next_stage] = self.store.stage_in_ring(units[next_stage], *placed)
                next_stage += 1

        if ring is not None:
            self._staging_left = staged  # drained by the next run if this one raises
            stage_ahead(-1)

        source_wait_ms = 0.0
        submit_started = time.perf_counter()
        for index, unit in enumerate(units):
            slot_index = index % slots
            slot = self.device_slots[slot_index]
            waited = time.perf_counter()
            source = staged.pop(index).result()
            source_wait_ms += (time.perf_counter() - waited) * 1000.0

            if index >= slots:
                self._free[index - slots].wait(copy_stream)
            if timing:
                timing["copy_start"][index].record(copy_stream)
            _hip.memcpy_h2d_async(slot, source, unit.nbytes, copy_stream)
            if timing:
                timing["copy_end"][index].record(copy_stream)
            self._ready[index].record(copy_stream)

            ahead = index + slots
            if ring is not None:
                ring.copied(index, self._ready[index])
                stage_ahead(index)
            elif ahead < len(units):
                # The staging worker may overwrite host slot `slot_index` as
                # soon as this H2D copy has completed; it need not wait for
                # the compute, which reads the device slot.
                staged[ahead] = self.store.prepare_unit(
                    units[ahead],
                    slot_index,
                    reuse_event=self._ready[index] if staging else None,
                )

            self._ready[index].wait(compute_stream)
            with torch.cuda.stream(compute_stream):
                if timing:
                    timing["compute_start"][index].record(compute_stream)
                state = compute_unit(unit, self._unit_views(unit, slot), state)
                if timing:
                    timing["compute_end"][index].record(compute_stream)
                self._free[index].record(compute_stream)

        submit_ms = (time.perf_counter() - submit_started) * 1000.0
        self._free[len(units) - 1].wait(self.coordinator)
        if timing:
            timing["pipeline"][1].record(self.coordinator)
        self.coordinator.synchronize()
        wall_ms = (time.perf_counter() - wall_started) * 1000.0
        if timing:
            h2d_ms = sum(
                a.elapsed_time(b)
                for a, b in zip(timing["copy_start"], timing["copy_end"])
            )
            compute_ms = sum(
                a.elapsed_time(b)
                for a, b in zip(timing["compute_start"], timing["compute_end"])
            )
            nbytes = self.plan.stream_bytes_per_token
            self.last_profile = {
                "wall_ms": wall_ms,
                "host_submit_ms": submit_ms,
                "source_wait_ms": source_wait_ms,
                "gpu_pipeline_ms": timing["pipeline"][0].elapsed_time(
                    timing["pipeline"][1]
                ),
                "h2d_event_sum_ms": h2d_ms,
                "compute_event_sum_ms": compute_ms,
                "h2d_bytes": nbytes,
                "h2d_effective_gbps": (nbytes / 1e9) / (h2d_ms / 1000.0),
            }
            self.last_profile.update(self.store.profile_stats())
        return state


class ResidentTransformerRuntime:
    """Every transfer unit resident in HBM; ``run`` has the DoubleBufferRuntime
    contract without any copies.

    Units keep their plan layout inside one device arena.  Fill it from a
    host store (``store`` given) or, with ``store=None``, draw synthetic
    weights on the device via :meth:`fill_random`.  ``synchronize=False``
    lets ``run`` return without waiting for the GPU, so a token loop whose
    next input stays on the device can run ahead of the GPU.
    """

    def __init__(self, plan, store, resident, device="cuda:0", synchronize=True):
        self.device = _require_gpu(device)
        self.plan = plan
        self.store = store
        self.resident = resident
        self.synchronize = bool(synchronize)
        self.profile = False
        self.last_profile = None
        total = sum(unit.elements for unit in plan.units)
        self.arena = torch.empty(total, dtype=torch.bfloat16, device=self.device)
        self._bases = []
        offset = 0
        for unit in plan.units:
            self._bases.append(self.arena[offset : offset + unit.elements])
            offset += unit.elements
        self._views = [_unit_views(u, b) for u, b in zip(plan.units, self._bases)]
        self.compute_stream = torch.cuda.current_stream(self.device)
        self.device_slots = []
        if store is not None:
            stream = torch.cuda.current_stream(self.device)
            for unit, base in zip(plan.units, self._bases):
                _copy_to_device(base, store.unit_source(unit), stream)
            stream.synchronize()

    @property
    def stats(self):
        return RuntimeStats(
            transfer_units=len(self.plan.units),
            slot_bytes=0,
            two_slot_bytes=0,
            device_slot_count=0,
            device_slots_bytes=0,
            resident_bytes=self.plan.resident_bytes,
            weight_gpu_bytes=self.arena.numel() * 2 + self.plan.resident_bytes,
        )

    def fill_random(self, seed=0, std=0.02):
        """Synthetic N(0, std) weights drawn on the device, per unit piece
        with seed base*1000 + plan index (not byte-identical to a CPU draw)."""

        with torch.inference_mode():
            for unit, views in zip(self.plan.units, self._views):
                for key, view in views.items():
                    gen = torch.Generator(device=self.device)
                    gen.manual_seed(int(seed) * 1000 + self.plan.tensor_index(key))
                    flat = view.reshape(-1)
                    step = 1 << 28
                    for start in range(0, flat.numel(), step):
                        piece = flat[start : start + step]
                        piece.copy_(
                            torch.randn(piece.numel(), generator=gen,
                                        device=self.device).mul_(std)
                        )
        torch.cuda.synchronize(self.device)
        return self

    def unit_views(self, index):
        return self._views[index]

    def run(self, compute_unit, state):
        for unit, views in zip(self.plan.units, self._views):
            state = compute_unit(unit, views, state)
        if self.synchronize:
            torch.cuda.current_stream(self.device).synchronize()
        return state
