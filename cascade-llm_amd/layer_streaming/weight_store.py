"""Host weight stores: one packed bf16 arena, page-locked whole or staged.

Public surface as in the reference (layer_streaming/weight_store.py):
``WeightStoreMode``, ``BaseWeightStore``, ``FullPinnedWeightStore``,
``PinnedStagingWeightStore`` and ``create_weight_store``, with the same
constructor arguments, ``tensor`` / ``unit_source`` / ``prepare_unit`` /
``load_checkpoint`` / ``close`` / ``profile_stats`` and error types.

* The arena follows the plan's packed layout; a key -> (offset, shape)
  table with aliases resolved is built once per store.
* full_pinned page-locks the arena; a unit's source is its arena view
  (``prepare_unit`` hands back a completed future).
* pinned_staging keeps the arena pageable and moves units through pinned
  staging buffers.  A ``_Stager`` owns those buffers, their byte ring
  (``StagingRing``), its own worker threads and a copy pool of the library
  (``cascade_copy_pool_*``, helpers bound to the GPU's NUMA node when the
  host has several); each job waits for the copies that last read its
  bytes, then copies with that pool's multi-threaded non-temporal memcpy,
  where the reference makes one tensor copy per unit (:258-268).
* ``load_checkpoint`` parses safetensors headers and reads every tensor
  straight into its arena bytes (``checkpoint.load_into``).
* ``fill_random`` writes the seeded synthetic weights of the benchmark
  configurations (there is no checkpoint on the GPU hosts).
* ``generation`` counts the times the arena's bytes changed (a load, a
  fill, ``close``).  Runtimes that copy out of the arena asynchronously
  register with ``add_reader``; before the bytes change, the store calls
  each reader's ``quiesce()`` (which waits for its copies in flight), and
  a runtime's device slots remember the generation they were filled from,
  so a slot filled before a reload is never taken for the new weights.
* ``tensor_factory`` stays injectable for tests, called as
  ``factory(elements, dtype=torch.bfloat16, device="cpu", pin_memory=...)``.
"""

from concurrent.futures import Future
from enum import Enum
import queue
import threading
import time
import weakref

import torch

from . import _hip
from . import checkpoint as _checkpoint
from .plan import ModelPlan

__all__ = [
    "WeightStoreMode",
    "BaseWeightStore",
    "FullPinnedWeightStore",
    "PinnedStagingWeightStore",
    "StagingRing",
    "create_weight_store",
    "tensor_seed",
]


class WeightStoreMode(str, Enum):
    FULL_PINNED = "full_pinned"
    PINNED_STAGING = "pinned_staging"


def tensor_seed(base_seed, tensor_index):
    """Seed of one tensor in the synthetic weights: base*1000 + index."""

    return int(base_seed) * 1000 + int(tensor_index)


def _layout_table(plan):
    """key -> (first element, element count, shape) for every tensor key and
    alias of ``plan``, each alias resolved to the tensor that owns the
    bytes."""

    table = {}
    for key, spec in plan.tensors.items():
        owner = spec
        while owner.alias_of is not None:
            owner = plan.tensors[owner.alias_of]
        table[key] = (plan.tensor_host_offset(owner.key), owner.numel,
                      tuple(owner.shape))
    for alias, target in plan.aliases.items():
        table[alias] = table[target]
    return table


class BaseWeightStore:
    """The packed host arena of a plan; subclasses decide whether it is
    page-locked and how a unit reaches a pinned source for its copy."""

    def __init__(self, plan, pin_full_arena, allocate=True, tensor_factory=None):
        if not isinstance(plan, ModelPlan):
            raise TypeError("expected a ModelPlan, got {}".format(
                type(plan).__name__))
        self.plan = plan
        self.pin_full_arena = bool(pin_full_arena)
        self.tensor_factory = tensor_factory or torch.empty
        self.arena = None
        self._loaded = False
        self._layout = _layout_table(plan)
        self.generation = 0
        self._readers = weakref.WeakSet()
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

    def add_reader(self, reader):
        """Register an object whose ``quiesce()`` waits for its reads of the
        arena in flight (held weakly)."""

        self._readers.add(reader)

    def _bytes_changing(self):
        # every asynchronous reader of the old bytes is done before they
        # change, and the generation tells cached copies of them apart
        for reader in list(self._readers):
            reader.quiesce()
        self.generation += 1

    def _host_buffer(self, elements, pinned):
        return self.tensor_factory(elements, dtype=torch.bfloat16, device="cpu",
                                   pin_memory=bool(pinned))

    def allocate(self):
        if self.arena is None:
            self._bytes_changing()
            self.arena = self._host_buffer(self.plan.host_arena_elements,
                                           self.pin_full_arena)
        return self.arena

    def _allocated_arena(self):
        if self.arena is None:
            raise RuntimeError("the host arena is not allocated (allocate() "
                               "first)")
        return self.arena

    def tensor(self, key):
        arena = self._allocated_arena()
        first, count, shape = self._layout[key]
        return arena[first:first + count].view(shape)

    def unit_source(self, unit, slot_index=None):
        first = unit.host_offset_elements
        return self._allocated_arena()[first:first + unit.elements]

    def required_keys(self):
        """Keys a checkpoint must provide (aliases share their target)."""

        return sorted(key for key, spec in self.plan.tensors.items()
                      if spec.alias_of is None)

    def load_checkpoint(self, checkpoint):
        """Load a local safetensors checkpoint into the packed CPU arena."""

        self.allocate()
        self._bytes_changing()
        _checkpoint.load_into(self, checkpoint)
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
        self._bytes_changing()
        draw_on = torch.device(device) if device is not None else torch.device("cpu")
        with torch.inference_mode():
            for index, (key, spec) in enumerate(self.plan.tensors.items()):
                if spec.alias_of is not None:
                    continue
                target = self.tensor(key)
                is_norm = len(spec.shape) == 1
                if is_norm and norm == "ones":
                    target.fill_(1.0)
                    continue
                generator = torch.Generator(device=draw_on)
                generator.manual_seed(tensor_seed(seed, index))
                scale, shift = (0.1, 1.0) if is_norm else (float(std), 0.0)
                flat = target.view(-1)
                # bounded pieces: 16 GB of weights never needs an fp32 copy
                step = 1 << 26
                for first in range(0, flat.numel(), step):
                    piece = flat[first:first + step]
                    values = torch.randn(piece.numel(), generator=generator,
                                         dtype=torch.float32, device=draw_on)
                    piece.copy_(values.mul_(scale).add_(shift).to(torch.bfloat16))
        self._loaded = True
        return self

    def close(self):
        if self.arena is not None:
            self._bytes_changing()
        self.arena = None
        self._loaded = False

    def reset_profile(self):
        return None

    def profile_stats(self):
        return {}


class FullPinnedWeightStore(BaseWeightStore):
    """All checkpoint weights remain in page-locked CPU memory."""

    mode = WeightStoreMode.FULL_PINNED

    def __init__(self, plan, allocate=True, tensor_factory=None):
        super().__init__(plan, True, allocate=allocate,
                         tensor_factory=tensor_factory)

    @property
    def pinned_cpu_bytes(self):
        return self.plan.host_arena_bytes

    def prepare_unit(self, unit, slot_index, reuse_event=None):
        # the arena itself is the pinned source: nothing to stage or wait for
        done = Future()
        done.set_result(self.unit_source(unit))
        return done


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


def _staging_summary(durations_ms):
    """The reference's staging profile keys (weight_store.py:285-298)."""

    return {
        "staging_copy_count": len(durations_ms),
        "staging_event_sum_ms": sum(durations_ms),
        "staging_event_max_ms": max(durations_ms) if durations_ms else 0.0,
    }


class _Stager:
    """Pinned staging buffers, their byte ring and the threads that fill
    them.  A job names a source, a buffer, a byte offset and the events of
    the copies that last read those bytes; a worker waits for the events,
    copies, and resolves the job's future with the pinned view."""

    def __init__(self, buffers, workers, copy_threads, numa_node):
        self.buffers = buffers
        self.ring = StagingRing(buffers)
        self.pool = _hip.CopyPool(copy_threads, numa_node)
        self._jobs = queue.SimpleQueue()
        self._lock = threading.Lock()
        self._durations_ms = []
        self._threads = [
            threading.Thread(target=self._serve, name="weight-stage-{}".format(i),
                             daemon=True)
            for i in range(max(1, int(workers)))
        ]
        for thread in self._threads:
            thread.start()

    def submit(self, source, buffer_index, byte_start, waits):
        result = Future()
        self._jobs.put((result, source, buffer_index, byte_start, tuple(waits)))
        return result

    def submit_into(self, target, source, waits):
        """A job that copies ``source`` into the pinned ``target`` (a buffer
        the caller owns) once ``waits`` are done."""

        result = Future()
        self._jobs.put((result, source, target, None, tuple(waits)))
        return result

    def _serve(self):
        while True:
            job = self._jobs.get()
            if job is None:
                return
            result, source, buffer_index, byte_start, waits = job
            if not result.set_running_or_notify_cancel():
                continue
            try:
                result.set_result(self._stage(source, buffer_index, byte_start,
                                              waits))
            except BaseException as error:  # handed to the waiting runtime
                result.set_exception(error)

    def _stage(self, source, buffer_index, byte_start, waits):
        started = time.perf_counter()
        for event in waits:
            event.synchronize()  # the copies that read these bytes are done
        if byte_start is None:  # submit_into: buffer_index is the target view
            target = buffer_index
        else:
            buffer = self.buffers[buffer_index]
            first = byte_start // buffer.element_size()
            target = buffer[first:first + source.numel()]
        self.pool.copy(target, source)
        if byte_start is not None:  # the unit staging the profile reports
            with self._lock:
                self._durations_ms.append((time.perf_counter() - started) * 1000.0)
        return target

    def stats(self, reset=False):
        with self._lock:
            durations = self._durations_ms
            if reset:
                self._durations_ms = []
        return _staging_summary(durations)

    def close(self):
        for _ in self._threads:
            self._jobs.put(None)
        for thread in self._threads:
            thread.join()
        self.pool.close()


class PinnedStagingWeightStore(BaseWeightStore):
    """Pageable full store plus reusable page-locked staging slots."""

    mode = WeightStoreMode.PINNED_STAGING

    def __init__(self, plan, allocate=True, tensor_factory=None, worker_count=2,
                 copy_threads=None, numa_node=None):
        self.worker_count = int(worker_count)
        self.copy_threads = int(copy_threads or _hip.default_copy_threads())
        # None: the current GPU's node, looked up when the slots are made
        self.numa_node = numa_node
        self._stager = None
        super().__init__(plan, False, allocate=allocate,
                         tensor_factory=tensor_factory)

    @property
    def pinned_cpu_bytes(self):
        return self.plan.two_slot_bytes

    @property
    def staging_slots(self):
        return None if self._stager is None else self._stager.buffers

    @property
    def staging_ring(self):
        return None if self._stager is None else self._stager.ring

    def allocate(self):
        arena = super().allocate()
        if self._stager is None:
            buffers = [self._host_buffer(self.plan.slot_elements, True)
                       for _ in range(self.plan.slot_count)]
            if self.numa_node is None:
                self.numa_node = _hip.device_numa_node()
            self._stager = _Stager(buffers, self.worker_count, self.copy_threads,
                                   self.numa_node)
        return arena

    def _running_stager(self):
        if self._stager is None:
            raise RuntimeError("the staging slots are not allocated (allocate() "
                               "first)")
        return self._stager

    def prepare_unit(self, unit, slot_index, reuse_event=None):
        """Stage ``unit`` at the start of pinned slot ``slot_index`` once
        ``reuse_event`` (the copy that last read the slot) is done."""

        waits = () if reuse_event is None else (reuse_event,)
        return self._running_stager().submit(self.unit_source(unit), slot_index,
                                             0, waits)

    def stage_in_ring(self, unit, slot_index, start, waits):
        """Stage ``unit`` at byte ``start`` of staging slot ``slot_index``
        once ``waits`` (the copies that last read those bytes) are done;
        returns a future of the pinned source view."""

        return self._running_stager().submit(self.unit_source(unit), slot_index,
                                             start, waits)

    def stage_into(self, target, source, waits=()):
        """Copy ``source`` into the caller's pinned ``target`` on the staging
        workers once ``waits`` (the copies that last read ``target``) are
        done; returns a future of ``target``.  The streamed LM head stages
        its chunks ahead this way (vocab.py)."""

        return self._running_stager().submit_into(target, source, waits)

    def copy_to_pinned(self, target, source):
        """``target.copy_(source)`` on the staging copy pool (the streamed
        LM head stages its chunks through it, vocab.py)."""

        return self._running_stager().pool.copy(target, source)

    def close(self):
        if self._stager is not None:
            if self.arena is not None:
                self._bytes_changing()  # before the staging buffers go
            self._stager.close()
            self._stager = None
        super().close()

    def reset_profile(self):
        if self._stager is not None:
            self._stager.stats(reset=True)

    def profile_stats(self):
        if self._stager is None:
            return _staging_summary(())
        return self._stager.stats()


_STORE_CLASSES = {
    WeightStoreMode.FULL_PINNED: FullPinnedWeightStore,
    WeightStoreMode.PINNED_STAGING: PinnedStagingWeightStore,
}


def create_weight_store(plan, mode=WeightStoreMode.FULL_PINNED, allocate=True,
                        tensor_factory=None):
    return _STORE_CLASSES[WeightStoreMode(mode)](plan, allocate=allocate,
                                                 tensor_factory=tensor_factory)
