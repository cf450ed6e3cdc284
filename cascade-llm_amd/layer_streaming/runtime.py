"""Device arenas and the two-slot H2D / compute pipeline.

* ``ResidentDeviceArena`` -- device copy of the plan's resident tensors
  (norms, plus embedding / LM head when the vocabulary is resident);
  reference layer_streaming/runtime.py:33-64.
* ``DoubleBufferRuntime`` -- the per-token transfer loop of the reference
  (runtime.py:67-268): unit i is copied host->device into slot i % slots on
  a copy stream while the compute stream runs the units before it.  The
  copies are hipMemcpyAsync calls and the hand-off uses hipEvents, all
  through libcascade_hip (cascade_memcpy_h2d_async, cascade_event_*).
  Ordering invariants (runtime.py:70-74, :194-230):
    - a copy into a slot waits for the compute that last read the slot;
    - compute i is enqueued once copy i is complete (the host waits for
      its event; the reference makes the compute stream wait for it);
    - a staging worker may refill pinned bytes once the copies that read
      them fired.
  Slots remember what they hold, so copies run ahead across calls (the LM
  head's first chunks behind the last units, the next call's first units
  behind the last chunks); they also remember the store generation the
  bytes came from, and the store drains the runtime's copies (``quiesce``)
  before it reloads, refills or frees its arena.
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


class _CallStaging:
    """Ring staging of one call's units (pinned_staging): futures of the
    staged pinned sources, the next unit to stage, and the units whose
    copies were made ahead of the call.  Ring keys are (serial, unit), so
    placements of successive calls never share a key."""

    def __init__(self, serial, generation):
        self.serial = serial
        self.generation = generation
        self.staged = {}
        self.next = 0
        self.copied = set()

    def drain(self):
        for future in list(self.staged.values()):
            try:
                future.result()
            except Exception:  # the call that used it already raised
                pass
        self.staged = {}


def _unit_views(unit, base):
    views = {}
    for piece in unit.pieces:
        spec = piece.tensor
        start = piece.unit_offset_elements
        views[spec.key] = base[start : start + spec.numel].view(spec.shape)
    return views


class DoubleBufferRuntime:
    """Device slots filled on a copy stream, read on a compute stream.

    Unit i goes to slot i % slot_count, as in the reference's loop
    (runtime.py:137-268): its copy waits until the slot's last reader is
    done, and its compute follows its copy.  Two things differ:

    * The copy -> compute hand-off is made by the host.  The host waits for
      copy i's event, then enqueues ``compute_unit(unit i)`` on the compute
      stream, so the compute stream never waits on a copy-stream event.  On
      MI355X such a cross-stream wait slowed every copy by about 0.6% (56.30
      against 56.64 GB/s for a 48/32/224/112 MiB layer sequence); a copy
      stream waiting for compute events costs nothing measurable.  The host
      is idle otherwise: copy i + 1 is already queued while it waits.
    * Slots are owned.  Each slot remembers the last transfer it received
      (a unit of this runtime or an LM-head chunk of the vocabulary runtime
      that shares the slots) and that copy's ready event, and a consumer
      that finds its transfer already in the slot skips the copy.  Copies can
      therefore run ahead of the calls that use them: as the last units free
      their slots, the first LM-head chunks are copied in (``release_hook``,
      set by VocabStreamingRuntime); as the last chunks (or, with a resident
      vocabulary, the last units) free theirs, the next call's first units
      are (``prefetch_across_calls``): from the arena when the store is
      full_pinned; for pinned_staging, from the staging ring once
      ``stage_call_ahead`` (called by the vocabulary runtime behind its last
      chunk, and again when the next call gathers its embedding rows) has
      staged them.  The copy engine then never waits for the host between
      calls.

    run() returns once every unit's work is enqueued; the coordinator
    (caller's) stream waits for the last unit, without a host
    synchronisation (with profile=True run() synchronises to read its
    events).  After a run that raised, the next run first waits for every
    copy, kernel and staging job the failed one left in flight.
    """

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
        self.coordinator = torch.cuda.current_stream(self.device)
        # pinned_staging: units staged ahead of the one being copied (ring
        # room permitting)
        self.stage_lookahead = 8
        self.prefetch_across_calls = True
        # called with a slot index when the last unit of a call that uses
        # that slot has been enqueued (VocabStreamingRuntime copies its
        # first chunks from here); a hook that returns False has no owner
        # left, and the slot goes to the next call's prefetch instead
        self.release_hook = None
        # pinned_staging: called once per call, when the call's last unit has
        # gone to the staging workers (VocabStreamingRuntime queues the
        # staging of its first chunks behind it)
        self.staging_done_hook = None
        # pinned_staging: the next call's staging, started ahead of it by
        # stage_call_ahead (None: not started)
        self._ahead = None
        self._serial = 0
        # (kind, index, ready event, store generation of the bytes)
        self._owner = [None] * self.slot_count
        self._last_free = [None] * self.slot_count  # event of the last reader
        self._failed = False
        self._staging_left = {}
        self._timed_copies = {}
        count = len(plan.units)
        self._ready = [_hip.HipEvent() for _ in range(count)]
        self._free = [_hip.HipEvent() for _ in range(count)]
        self._start = _hip.HipEvent()
        self._timing = None
        add_reader = getattr(store, "add_reader", None)
        if add_reader is not None:
            add_reader(self)  # the store drains our copies before its bytes change

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

    # ------------------------------------------------------ slot ownership

    def slot_copy(self, slot, kind, index, source, nbytes, ready, timing=None):
        """Copy ``nbytes`` of pinned ``source`` into device slot ``slot`` on
        the copy stream once the slot's last reader is done; ``ready`` is
        recorded after the copy, and the slot now holds (kind, index)."""

        stream = self.copy_stream
        if self._last_free[slot] is not None:
            self._last_free[slot].wait(stream)
        if timing is not None:
            timing[0].record(stream)
        _hip.memcpy_h2d_async(self.device_slots[slot], source, nbytes, stream)
        if timing is not None:
            timing[1].record(stream)
        ready.record(stream)
        self._owner[slot] = (kind, index, ready, self._store_generation())

    def _store_generation(self):
        return getattr(self.store, "generation", 0)

    def slot_holding(self, slot, kind, index):
        """Ready event of the copy that put (kind, index) in ``slot``, or
        None when the slot holds something else, or bytes the store has
        replaced since (load_checkpoint, fill_random, close)."""

        owner = self._owner[slot]
        if (owner is not None and owner[0] == kind and owner[1] == index
                and owner[3] == self._store_generation()):
            return owner[2]
        return None

    def quiesce(self):
        """Wait until no copy or staging job of this runtime reads the
        store's arena (called by the store before its bytes change)."""

        for future in list(self._staging_left.values()):
            try:
                future.result()
            except Exception:  # the run that made it already raised
                pass
        self.copy_stream.synchronize()
        self._drop_ahead()

    def slot_released(self, slot, free):
        """``free`` (a compute-stream event) marks the end of the last
        reader of ``slot``: later copies into the slot wait for it."""

        self._last_free[slot] = free

    def discard_slots(self):
        """Forget what the slots hold.  Not needed after the store's own
        load_checkpoint / fill_random / close, which the slots notice by the
        store's generation."""

        self._owner = [None] * self.slot_count

    def prefetch_next_call(self, slot):
        """Copy the first unit a call reads from ``slot`` ahead of that
        call: from the store's arena when it needs no staging (full_pinned),
        or, for pinned_staging, from the ring once stage_call_ahead has
        staged it (a unit still staging is left to the call)."""

        units = self.plan.units
        if not self.prefetch_across_calls or slot >= len(units):
            return
        if self.slot_holding(slot, "unit", slot) is not None:
            return
        unit = units[slot]
        mode = self.store.mode.value
        if mode == "full_pinned":
            self.slot_copy(slot, "unit", slot, self.store.unit_source(unit),
                           unit.nbytes, self._ready[slot])
            return
        call = self._ahead
        if mode != "pinned_staging" or call is None or slot in call.copied:
            return
        future = call.staged.get(slot)
        if future is None or not future.done() or future.exception() is not None:
            return
        self.slot_copy(slot, "unit", slot, future.result(), unit.nbytes,
                       self._ready[slot])
        self.store.staging_ring.copied((call.serial, slot), self._ready[slot])
        del call.staged[slot]
        call.copied.add(slot)

    # ------------------------------------------------------ ahead staging

    def _ring(self):
        if self.store.mode.value != "pinned_staging":
            return None
        return getattr(self.store, "staging_ring", None)

    def _stage_ahead(self, call, done):
        """Ring staging: units after ``done`` (whose copy is enqueued) go to
        the staging workers while the ring has room for them."""

        units = self.plan.units
        count = len(units)
        ring = self.store.staging_ring
        while call.next < count and call.next - done <= self.stage_lookahead:
            i = call.next
            placed = ring.place(units[i].nbytes, (call.serial, i))
            if placed is None:
                break
            call.staged[i] = self.store.stage_in_ring(units[i], *placed)
            call.next += 1
            if call.next == count and self.staging_done_hook is not None:
                self.staging_done_hook()

    def _new_call(self):
        self._serial += 1
        return _CallStaging(self._serial, self._store_generation())

    def stage_call_ahead(self):
        """pinned_staging: start staging the next run's first units now, into
        the ring behind the copies that last read it, so they stage while
        the caller finishes this call (VocabStreamingRuntime calls this once
        the LM head's last chunk is queued) or gathers the next call's
        embedding rows.  prefetch_next_call may then copy them ahead too.
        No-op in other modes, after a run that raised, or when already
        started."""

        if self._ring() is None or self._ahead is not None or self._failed:
            return
        self.store.reset_profile()  # the staging profile counts the next call
        call = self._new_call()
        self._ahead = call
        self._stage_ahead(call, -1)

    def _take_ahead(self):
        """The call staged ahead, if it can serve this run: the store's bytes
        unchanged, and every unit copied ahead still in its slot (an LM-head
        call between runs may have taken the slot back).  Otherwise it is
        drained and dropped."""

        call = self._ahead
        if call is None:
            return None
        if call.generation == self._store_generation() and all(
                self.slot_holding(i % self.slot_count, "unit", i) is not None
                for i in call.copied):
            self._ahead = None
            return call
        self._drop_ahead()
        return None

    def _drop_ahead(self):
        """Forget the call staged ahead once nothing of it is in flight
        (staging jobs done, copies done): its ring placements go too."""

        call, self._ahead = self._ahead, None
        if call is None:
            return
        call.drain()
        self.copy_stream.synchronize()
        ring = self._ring()
        if ring is not None:
            ring.reset()

    # ----------------------------------------------------------------- run

    def _recover(self):
        """Wait for what a run that raised left in flight."""

        for future in self._staging_left.values():
            try:
                future.result()
            except Exception:  # that run already raised
                pass
        self._staging_left = {}
        self.copy_stream.synchronize()
        self.compute_stream.synchronize()
        self._drop_ahead()
        ring = getattr(self.store, "staging_ring", None)
        if ring is not None:
            ring.reset()
        self._failed = False

    def run(self, compute_unit, state):
        if not self.plan.units:
            return state
        if self._failed:
            self._recover()
        self._failed = True
        state = self._run(compute_unit, state)
        self._failed = False
        return state

    def _run(self, compute_unit, state):
        wall_started = time.perf_counter()
        units = self.plan.units
        count = len(units)
        slots = self.slot_count
        compute_stream = self.compute_stream
        timing = self._timing_events() if self.profile else None
        self._timed_copies = {}

        # work the caller enqueued before (the embedding) precedes the units
        self._start.record(self.coordinator)
        self._start.wait(compute_stream)
        if timing:
            timing["pipeline"][0].record(self.coordinator)

        staging = self.store.mode.value == "pinned_staging"
        ring = self._ring()
        call = None
        if ring is not None:
            call = self._take_ahead()
            if call is None:
                ring.reset()  # every copy that read the pinned slots is done
                self.store.reset_profile()
                call = self._new_call()
            staged = call.staged
        else:
            self.store.reset_profile()
            staged = {}
        self._staging_left = staged

        source_wait_ms = 0.0

        def copy_unit(i):
            # the source (staged for pinned_staging), then the copy
            nonlocal source_wait_ms
            slot = i % slots
            if staging:
                waited = time.perf_counter()
                source = staged.pop(i).result()
                source_wait_ms += (time.perf_counter() - waited) * 1000.0
            else:
                source = self.store.unit_source(units[i])
            pair = None
            if timing:
                pair = (timing["copy_start"][i], timing["copy_end"][i])
                self._timed_copies[i] = units[i].nbytes
            self.slot_copy(slot, "unit", i, source, units[i].nbytes,
                           self._ready[i], pair)
            if ring is not None:
                ring.copied((call.serial, i), self._ready[i])
                self._stage_ahead(call, i)
            elif staging and i + slots < count:
                # the staging worker may refill this pinned slot once this
                # copy has read it (it need not wait for the compute)
                staged[i + slots] = self.store.prepare_unit(
                    units[i + slots], slot, reuse_event=self._ready[i])

        if ring is not None:
            self._stage_ahead(call, -1)
        elif staging:
            for i in range(min(slots, count)):
                staged[i] = self.store.prepare_unit(units[i], i)
        ready = {}
        for i in range(min(slots, count)):
            held = self.slot_holding(i % slots, "unit", i)
            if held is not None and (not staging
                                     or (call is not None and i in call.copied)):
                ready[i] = held  # copied ahead of this call
            else:
                copy_unit(i)
                ready[i] = self._ready[i]

        submit_started = time.perf_counter()
        for i, unit in enumerate(units):
            slot = i % slots
            ready.pop(i).synchronize()  # host hand-off: copy i is in HBM
            with torch.cuda.stream(compute_stream):
                if timing:
                    timing["compute_start"][i].record(compute_stream)
                state = compute_unit(unit, self._unit_views(unit, self.device_slots[slot]),
                                     state)
                if timing:
                    timing["compute_end"][i].record(compute_stream)
                self._free[i].record(compute_stream)
            self.slot_released(slot, self._free[i])
            following = i + slots
            if following < count:
                copy_unit(following)
                ready[following] = self._ready[following]
            elif self.release_hook is not None and self.release_hook(slot) is not False:
                pass
            else:
                self.prefetch_next_call(slot)

        submit_ms = (time.perf_counter() - submit_started) * 1000.0
        self._free[count - 1].wait(self.coordinator)
        if timing:
            timing["pipeline"][1].record(self.coordinator)
            timing["pipeline"][1].synchronize()
            wall_ms = (time.perf_counter() - wall_started) * 1000.0
            timed = self._timed_copies
            h2d_ms = sum(timing["copy_start"][i].elapsed_time(timing["copy_end"][i])
                         for i in timed)
            compute_ms = sum(
                a.elapsed_time(b)
                for a, b in zip(timing["compute_start"], timing["compute_end"])
            )
            nbytes = sum(timed.values())
            self.last_profile = {
                "wall_ms": wall_ms,
                "host_submit_ms": submit_ms,
                "source_wait_ms": source_wait_ms,
                "gpu_pipeline_ms": timing["pipeline"][0].elapsed_time(
                    timing["pipeline"][1]
                ),
                "h2d_event_sum_ms": h2d_ms,
                "compute_event_sum_ms": compute_ms,
                "h2d_bytes": self.plan.stream_bytes_per_token,
                "h2d_timed_bytes": nbytes,
                "h2d_effective_gbps": (nbytes / 1e9) / (h2d_ms / 1000.0)
                if h2d_ms else 0.0,
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
