"""Host weight stores: one packed bf16 arena, fully pinned or staged.

API and behaviour follow the reference (layer_streaming/weight_store.py):

* ``FullPinnedWeightStore`` page-locks the whole arena; ``prepare_unit``
  returns an already-resolved future over the arena view (:184-206).
* ``PinnedStagingWeightStore`` keeps a pageable arena plus ``slot_count``
  page-locked staging slots filled by worker threads; a worker first waits on
  ``reuse_event`` (the H2D copy that last read its slot) and then copies the
  unit in (:209-298) with the library's multi-threaded non-temporal memcpy
  (``cascade_host_copy``; ``copy_threads`` threads, default this process's
  CPUs up to 8) instead of one tensor copy.
* Staging ring (added): the runtime stages units at consecutive byte ranges
  of the same pinned slots, so several small units can be staged ahead of
  their copies (``StagingRing``); ``prepare_unit`` keeps the reference's
  one-unit-per-slot behaviour.
* ``load_checkpoint`` fills the arena from a local safetensors file or
  sharded index with key and shape checks (:20-38, :109-171).
* ``tensor_factory`` is injectable for tests (:55).

Added here: ``fill_random`` writes the seeded synthetic weights the
benchmark configurations use (there is no checkpoint on the GPU hosts).
"""

import json
from concurrent.futures import Future, ThreadPoolExecutor
from enum import Enum
from pathlib import Path
import threading
import time

import torch

from . import _hip
from .plan import ModelPlan

__all__ = [
    "WeightStoreMode",
    "BaseWeightStore",
    "FullPinnedWeightStore",
    "PinnedStagingWeightStore",
    "create_weight_store",
    "tensor_seed",
]


class WeightStoreMode(str, Enum):
    FULL_PINNED = "full_pinned"
    PINNED_STAGING = "pinned_staging"


def _checkpoint_files(checkpoint):
    """key -> file map of a sharded checkpoint, or None for a single file."""

    root = Path(checkpoint)
    index = root / "model.safetensors.index.json"
    if index.exists():
        with index.open("r", encoding="utf-8") as handle:
            weight_map = json.load(handle).get("weight_map")
        if not isinstance(weight_map, dict):
            raise ValueError("{} has no weight_map".format(index))
        return {key: root / name for key, name in weight_map.items()}
    if (root / "model.safetensors").exists():
        return None
    raise FileNotFoundError(
        "expected model.safetensors or model.safetensors.index.json in "
        "{}".format(root)
    )


def tensor_seed(base_seed, tensor_index):
    """Seed of one tensor in the synthetic weights: base*1000 + index."""

    return int(base_seed) * 1000 + int(tensor_index)


class BaseWeightStore:
    """Packed CPU arena shared by both memory modes."""

    def __init__(self, plan, pin_full_arena, allocate=True, tensor_factory=None):
        if not isinstance(plan, ModelPlan):
            raise TypeError("plan must be a ModelPlan")
        self.plan = plan
        self.pin_full_arena = bool(pin_full_arena)
        self.tensor_factory = tensor_factory or torch.empty
        self.arena = None
        self._loaded = False
        if allocate:
            self.allocate()

    @property
    def mode(self):
        raise NotImplementedError

    @property
    def pinned_cpu_bytes(self):
        raise NotImplementedError

    @property
    def allocated(self):
        return self.arena is not None

    @property
    def loaded(self):
        return self._loaded

    def allocate(self):
        if self.arena is None:
            self.arena = self.tensor_factory(
                self.plan.host_arena_elements,
                dtype=torch.bfloat16,
                device="cpu",
                pin_memory=self.pin_full_arena,
            )
        return self.arena

    def _require_arena(self):
        if self.arena is None:
            raise RuntimeError("weight arena has not been allocated")
        return self.arena

    def _view(self, key):
        spec = self.plan.tensors[key]
        if spec.alias_of is not None:
            return self._view(spec.alias_of)
        start = self.plan.tensor_host_offset(key)
        return self._require_arena()[start : start + spec.numel].view(spec.shape)

    def tensor(self, key):
        self._require_arena()
        return self._view(self.plan.aliases.get(key, key))

    def unit_source(self, unit, slot_index=None):
        arena = self._require_arena()
        start = unit.host_offset_elements
        return arena[start : start + unit.elements]

    def required_keys(self):
        return sorted(
            key for key, spec in self.plan.tensors.items()
            if spec.alias_of is None
        )

    def load_checkpoint(self, checkpoint):
        """Load a local safetensors checkpoint into the packed CPU arena."""

        self.allocate()
        try:
            from safetensors import safe_open
        except ImportError as error:
            raise RuntimeError(
                "safetensors is required to load a checkpoint"
            ) from error
        weight_map = _checkpoint_files(checkpoint)
        required = set(self.required_keys())
        if weight_map is None:
            files = [Path(checkpoint) / "model.safetensors"]
        else:
            missing = required.difference(weight_map)
            if missing:
                raise KeyError(
                    "checkpoint index misses required tensors: {}".format(
                        ", ".join(sorted(missing)[:8])
                    )
                )
            files = sorted({weight_map[key] for key in required})
        loaded = set()
        with torch.inference_mode():
            for filename in files:
                with safe_open(str(filename), framework="pt", device="cpu") as src:
                    for key in sorted(required.intersection(src.keys())):
                        value = src.get_tensor(key)
                        target = self._view(key)
                        if tuple(value.shape) != tuple(target.shape):
                            raise ValueError(
                                "{} shape {} != expected {}".format(
                                    key, tuple(value.shape), tuple(target.shape)
                                )
                            )
                        target.copy_(value.to(dtype=torch.bfloat16))
                        loaded.add(key)
        missing = required.difference(loaded)
        if missing:
            raise KeyError(
                "checkpoint misses required tensors: {}".format(
                    ", ".join(sorted(missing)[:8])
                )
            )
        self._loaded = True
        return self

    def fill_random(self, seed=0, std=0.02, norm="ones", device=None):
        """Write seeded synthetic weights into the arena.

        Matrices are N(0, std) drawn in fp32 from a generator seeded with
        ``tensor_seed(seed, plan index)`` and rounded to bf16.  Norm weights
        are 1.0 (``norm="ones"``) or 1 + N(0, 0.1) (``norm="random"``).
        ``device=None`` draws on the CPU, so the bytes are reproducible
        anywhere; a CUDA device draws there (much faster for 16 GB, but the
        bytes differ from the CPU draw).
        """

        self.allocate()
        gen_device = torch.device(device) if device is not None else None
        with torch.inference_mode():
            for index, (key, spec) in enumerate(self.plan.tensors.items()):
                if spec.alias_of is not None:
                    continue
                target = self._view(key)
                is_norm = len(spec.shape) == 1
                if is_norm and norm == "ones":
                    target.fill_(1.0)
                    continue
                generator = torch.Generator(
                    device=gen_device if gen_device is not None else "cpu"
                )
                generator.manual_seed(tensor_seed(seed, index))
                scale = 0.1 if is_norm else float(std)
                self._fill_normal(target, generator, gen_device, scale,
                                  1.0 if is_norm else 0.0)
        self._loaded = True
        return self

    @staticmethod
    def _fill_normal(target, generator, gen_device, scale, shift):
        flat = target.view(-1)
        # Draw in bounded pieces so 16 GB of weights never needs a full fp32
        # copy in memory.
        step = 1 << 26
        for start in range(0, flat.numel(), step):
            piece = flat[start : start + step]
            values = torch.randn(
                piece.numel(),
                generator=generator,
                dtype=torch.float32,
                device=gen_device if gen_device is not None else "cpu",
            )
            values.mul_(scale).add_(shift)
            piece.copy_(values.to(torch.bfloat16))

    def close(self):
        self.arena = None
        self._loaded = False

    def reset_profile(self):
        return None

    def profile_stats(self):
        return {}


class FullPinnedWeightStore(BaseWeightStore):
    """All checkpoint weights remain in page-locked CPU memory."""

    def __init__(self, plan, allocate=True, tensor_factory=None):
        super().__init__(plan, True, allocate=allocate,
                         tensor_factory=tensor_factory)

    @property
    def mode(self):
        return WeightStoreMode.FULL_PINNED

    @property
    def pinned_cpu_bytes(self):
        return self.plan.host_arena_bytes

    def prepare_unit(self, unit, slot_index, reuse_event=None):
        future = Future()
        future.set_result(self.unit_source(unit))
        return future


class StagingRing:
    """Byte ring over the pinned staging slots.

    The reference stages unit i into slot i % 2 once the copy that last read
    that slot is done (weight_store.py:209-298, runtime.py:194-230).  After
    a short copy (an 8 MiB k_proj) the next slot frees too late to stage the
    following unit before the link runs dry.  Here units take consecutive
    byte ranges of the slots, in order, a unit moving on to the next slot
    (after the last, the first) when it does not fit in what is left of the
    current one.  A range is placed once every unit still holding part of
    it has had its copy enqueued, and the staging worker waits for those
    copies' events before writing.  Several small units are then staged
    ahead within the same pinned slots; units as large as a slot alternate
    between them as before.  Used from the runtime's host thread only.
    """

    def __init__(self, slots):
        self.slots = slots
        self.slot_bytes = slots[0].numel() * slots[0].element_size()
        self.reset()

    def reset(self):
        """Forget every placement (all copies reading the slots are done)."""

        self.slot = 0
        self.head = 0
        self.live = []  # [slot, start, end, unit key, ready event or None]

    def place(self, nbytes, key):
        """(slot, byte start, events to wait for) for ``nbytes``, or None
        while a unit whose copy is not yet enqueued holds part of the range."""

        if nbytes > self.slot_bytes:
            raise ValueError("unit larger than a staging slot")
        slot, start = self.slot, self.head
        if start + nbytes > self.slot_bytes:
            slot, start = (slot + 1) % len(self.slots), 0
        end = start + nbytes
        waits, keep = [], []
        for entry in self.live:
            if entry[0] == slot and entry[1] < end and start < entry[2]:
                if entry[4] is None:
                    return None
                waits.append(entry[4])
                if start <= entry[1] and entry[2] <= end:
                    continue  # wholly covered: the new unit owns its bytes
            # kept, partial overlaps included: the rest of their range may
            # be written by a later unit, which must wait for them too
            keep.append(entry)
        self.live = keep + [[slot, start, end, key, None]]
        self.slot, self.head = slot, end
        return slot, start, waits

    def copied(self, key, event):
        """The copy of unit ``key`` is enqueued; ``event`` marks its end."""

        for entry in self.live:
            if entry[3] == key:
                entry[4] = event
                return
        raise KeyError(key)


class PinnedStagingWeightStore(BaseWeightStore):
    """Pageable full store plus reusable page-locked staging slots."""

    def __init__(self, plan, allocate=True, tensor_factory=None, worker_count=2,
                 copy_threads=None):
        self.staging_slots = None
        self.staging_ring = None
        self.worker_count = int(worker_count)
        self.copy_threads = int(copy_threads or _hip.default_copy_threads())
        self._executor = None
        self._profile_lock = threading.Lock()
        self._stage_durations_ms = []
        super().__init__(plan, False, allocate=allocate,
                         tensor_factory=tensor_factory)

    @property
    def mode(self):
        return WeightStoreMode.PINNED_STAGING

    @property
    def pinned_cpu_bytes(self):
        return self.plan.two_slot_bytes

    def allocate(self):
        arena = super().allocate()
        if self.staging_slots is None:
            self.staging_slots = [
                self.tensor_factory(
                    self.plan.slot_elements,
                    dtype=torch.bfloat16,
                    device="cpu",
                    pin_memory=True,
                )
                for _ in range(self.plan.slot_count)
            ]
            self.staging_ring = StagingRing(self.staging_slots)
        if self._executor is None:
            self._executor = ThreadPoolExecutor(
                max_workers=self.worker_count, thread_name_prefix="weight-stage"
            )
        return arena

    def _stage(self, unit, slot_index, reuse_event):
        started = time.perf_counter()
        if reuse_event is not None:
            # The slot is free once the H2D copy that last read it is done.
            reuse_event.synchronize()
        target = self.staging_slots[slot_index][: unit.elements]
        _hip.host_copy(target, self.unit_source(unit), self.copy_threads)
        elapsed = (time.perf_counter() - started) * 1000.0
        with self._profile_lock:
            self._stage_durations_ms.append(elapsed)
        return target

    def prepare_unit(self, unit, slot_index, reuse_event=None):
        if self.staging_slots is None or self._executor is None:
            raise RuntimeError("staging store has not been allocated")
        return self._executor.submit(self._stage, unit, slot_index, reuse_event)

    def _stage_at(self, unit, slot_index, start, waits):
        started = time.perf_counter()
        for event in waits:
            event.synchronize()
        slot = self.staging_slots[slot_index]
        first = start // slot.element_size()
        target = slot[first:first + unit.elements]
        _hip.host_copy(target, self.unit_source(unit), self.copy_threads)
        elapsed = (time.perf_counter() - started) * 1000.0
        with self._profile_lock:
            self._stage_durations_ms.append(elapsed)
        return target

    def stage_in_ring(self, unit, slot_index, start, waits):
        """Stage ``unit`` at byte ``start`` of staging slot ``slot_index``
        once ``waits`` (the copies that last read those bytes) are done;
        returns a future of the pinned source view."""

        if self._executor is None:
            raise RuntimeError("staging store has not been allocated")
        return self._executor.submit(self._stage_at, unit, slot_index, start, waits)

    def close(self):
        if self._executor is not None:
            self._executor.shutdown(wait=True)
            self._executor = None
        self.staging_slots = None
        super().close()

    def reset_profile(self):
        with self._profile_lock:
            self._stage_durations_ms = []

    def profile_stats(self):
        with self._profile_lock:
            durations = list(self._stage_durations_ms)
        return {
            "staging_copy_count": len(durations),
            "staging_event_sum_ms": sum(durations),
            "staging_event_max_ms": max(durations) if durations else 0.0,
        }


def create_weight_store(plan, mode=WeightStoreMode.FULL_PINNED, allocate=True,
                        tensor_factory=None):
    if WeightStoreMode(mode) == WeightStoreMode.FULL_PINNED:
        return FullPinnedWeightStore(plan, allocate=allocate,
                                     tensor_factory=tensor_factory)
    return PinnedStagingWeightStore(plan, allocate=allocate,
                                    tensor_factory=tensor_factory)
