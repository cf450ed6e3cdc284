"""Host-only vocabulary of a streamed-vocabulary plan (reference
layer_streaming/vocab.py).

* ``embedding(ids)`` gathers the requested rows of the host embedding into a
  page-locked row buffer and copies them to the device on the caller's
  stream (vocab.py:100-131).  The buffer's two halves take turns, so one
  group of rows is gathered while the previous group's copy runs; an event
  per half guards it until the copy that reads it is done.
* ``lm_head_topk(h, top_k, return_full_logits)`` streams the LM head in row
  chunks through the transformer runtime's two device slots and keeps an
  exact running top-k on the device (vocab.py:149-300).  Per chunk there is
  one kernel launch (cascade_lm_head_topk_bf16: fp32 logits GEMV, block
  top-k and the merge with the running list).  Hand-off and slot ownership
  follow DoubleBufferRuntime: the host waits for a chunk's copy, then
  enqueues its kernel; the first two chunks are copied while the
  transformer's last units still run, and the next call's first units while
  the last chunks run.  With a pinned_staging store the chunks pass through
  two pinned halves, staged on the store's staging workers ahead of their
  copies: the first two queued behind the call's last unit, chunk c + 2 as
  soon as chunk c's copy is enqueued (the reference stages each chunk on
  the calling thread, vocab.py:133-147); behind the last chunk the next
  call's first units are staged into the transformer's ring
  (DoubleBufferRuntime.stage_call_ahead).  The call
  returns when the top-k is in HBM (the reference synchronises there too,
  vocab.py:268-271).
* ``merge_topk`` is the reference's public helper (vocab.py:11-32) with a
  deterministic order on ties (value descending, index ascending).

Logits are fp32 and not rounded to bf16 (the reference rounds them through
bf16 first, which ties inside the top-10 for almost every step at this
shape); the top-k order equals a stable descending sort of them.
"""

import time
import weakref

import torch

from . import _hip
from .weight_store import WeightStoreMode

__all__ = ["merge_topk", "VocabStreamingRuntime"]


def merge_topk(current_values, current_indices, candidate_values,
               candidate_indices, top_k):
    """Merge two candidate sets into the exact top-k.

    Ties are broken towards the lower index, so the result does not depend
    on the order in which the candidates arrive.
    """

    if current_values is None:
        values, indices = candidate_values, candidate_indices
    else:
        values = torch.cat((current_values, candidate_values), dim=-1)
        indices = torch.cat((current_indices, candidate_indices), dim=-1)
    keep = min(int(top_k), values.shape[-1])
    # stable two-key sort: index ascending, then value descending
    by_index = torch.argsort(indices, dim=-1, stable=True)
    values = torch.gather(values, -1, by_index)
    indices = torch.gather(indices, -1, by_index)
    order = torch.argsort(values, dim=-1, descending=True, stable=True)[..., :keep]
    return torch.gather(values, -1, order), torch.gather(indices, -1, order)


def _pinned_rows(count, width):
    return torch.empty((count, width), dtype=torch.bfloat16, device="cpu",
                       pin_memory=True)


def _weak_hook(method):
    """``method`` as a hook for the transformer runtime that holds its owner
    weakly (the owner holds that runtime, so a strong reference back would
    keep both, and the owner's device buffers, alive until a cyclic garbage
    collection); once the owner is gone the hook returns False."""

    ref = weakref.WeakMethod(method)

    def hook(*args):
        target = ref()
        if target is None:
            return False
        target(*args)
        return None

    return hook


class VocabStreamingRuntime:
    """Embedding rows and LM-head chunks of a host-only vocabulary, sharing
    the transformer runtime's two device slots and streams."""

    def __init__(self, plan, store, transformer_runtime,
                 embedding_staging_rows=256, profile=False):
        layout = plan.vocab
        if layout is None:
            raise ValueError("the plan keeps the vocabulary resident "
                             "(build it with stream_vocab=True)")
        row_buffer = int(embedding_staging_rows)
        if row_buffer < 1:
            raise ValueError("embedding_staging_rows must be at least 1, got "
                             "{}".format(row_buffer))
        runtime = transformer_runtime
        if len(runtime.device_slots) != 2:
            raise ValueError("the LM head streams through two device slots, the "
                             "runtime has {}".format(len(runtime.device_slots)))
        smallest = min(slot.numel() for slot in runtime.device_slots)
        if smallest < layout.chunk_elements:
            raise ValueError("a device slot of {} elements cannot take a "
                             "{}-element LM-head chunk".format(
                                 smallest, layout.chunk_elements))
        _hip.load()
        self.plan = plan
        self.vocab = layout
        self.store = store
        self.transformer_runtime = runtime
        self.device = runtime.device
        self.device_slots = runtime.device_slots
        self.copy_stream = runtime.copy_stream
        self.compute_stream = runtime.compute_stream
        self.coordinator = runtime.coordinator
        self.profile = bool(profile)
        self.last_profile = None
        self.last_embedding_bytes = 0
        self.embedding_staging_rows = row_buffer
        self.embedding_staging = _pinned_rows(row_buffer, layout.hidden_size)
        # pinned_staging: the pageable LM head passes through two pinned
        # chunk buffers (one allocation, split in halves)
        self._staged = store.mode == WeightStoreMode.PINNED_STAGING
        self.head_staging_slots = None
        if self._staged:
            both = torch.empty(2 * layout.chunk_elements, dtype=torch.bfloat16,
                               device="cpu", pin_memory=True)
            self.head_staging_slots = list(both.split(layout.chunk_elements))
        chunks = layout.chunk_count
        self._ready = [_hip.HipEvent() for _ in range(chunks)]
        self._free = [_hip.HipEvent() for _ in range(chunks)]
        self._staging_read = [None, None]  # copy that last read a pinned half
        self._prestaged = {}  # chunk -> future of its staged pinned half
        self._start = _hip.HipEvent()
        # gather groups alternate between the two halves of the row buffer
        # (one group of its single row when it holds one)
        group = max(1, row_buffer // 2)
        self._row_halves = [self.embedding_staging[h * group:(h + 1) * group]
                            for h in range(min(2, row_buffer))]
        self._rows_free = [_hip.HipEvent() for _ in self._row_halves]
        self._timers = None
        self._timed = {}
        self._workspaces = {}
        # the first chunks follow the transformer's last units directly; a
        # pageable store's chunks are staged on its staging workers, the
        # first two queued behind the call's last unit
        runtime.release_hook = _weak_hook(self._copy_first_chunk)
        if self._staged:
            runtime.staging_done_hook = _weak_hook(self._prestage_first_chunks)
            add_reader = getattr(store, "add_reader", None)
            if add_reader is not None:
                add_reader(self)  # staging jobs read the arena

    @property
    def gpu_slot_bytes(self):
        return sum(slot.numel() * slot.element_size() for slot in self.device_slots)

    @property
    def extra_pinned_cpu_bytes(self):
        buffers = [self.embedding_staging] + list(self.head_staging_slots or ())
        return sum(b.numel() * b.element_size() for b in buffers)

    # --------------------------------------------------------- embedding

    def embedding(self, input_ids):
        """Gather only the requested CPU rows and copy them to the GPU."""

        # pinned_staging: the call's first units stage while the rows are
        # gathered (no-op if the last call already started them)
        self.transformer_runtime.stage_call_ahead()
        shape = tuple(input_ids.shape)
        ids = input_ids.detach().reshape(-1).to(device="cpu", dtype=torch.long)
        count = ids.numel()
        vocab, width = self.vocab.vocab_size, self.vocab.hidden_size
        if count and (int(ids.min()) < 0 or int(ids.max()) >= vocab):
            raise IndexError("token id outside [0, {})".format(vocab))
        table = self.store.tensor(self.vocab.embedding_key)
        out = torch.empty((count, width), dtype=torch.bfloat16, device=self.device)
        self.last_embedding_bytes = count * width * 2
        stream = torch.cuda.current_stream(self.device)
        # the row buffer's halves take turns: one is gathered into while the
        # other's copy runs
        halves = self._row_halves
        group = halves[0].shape[0]
        for n, first in enumerate(range(0, count, group)):
            rows = min(group, count - first)
            half = n % len(halves)
            # the half is free once the copy that last read it is done
            self._rows_free[half].synchronize()
            buffer = halves[half][:rows]
            torch.index_select(table, 0, ids[first:first + rows], out=buffer)
            _hip.memcpy_h2d_async(out[first:first + rows], buffer,
                                  rows * width * 2, stream)
            self._rows_free[half].record(stream)
        return out.view(shape + (width,))

    # ----------------------------------------------------------- LM head

    def _chunk_rows(self, chunk):
        first, end = self.vocab.chunk_bounds(chunk)
        return self.store.tensor(self.vocab.lm_head_key)[first:end].reshape(-1)

    def _prestage(self, chunk):
        """pinned_staging: queue the staging of ``chunk`` into its pinned half
        on the store's staging workers, behind the copy that last read the
        half.  Called for chunk c + 2 once chunk c's copy is enqueued, and
        for the first two chunks behind a call's last unit."""

        if chunk >= self.vocab.chunk_count or chunk in self._prestaged:
            return
        rows = self._chunk_rows(chunk)
        half = chunk % 2
        reader = self._staging_read[half]
        target = self.head_staging_slots[half][: rows.numel()]
        self._prestaged[chunk] = self.store.stage_into(
            target, rows, () if reader is None else (reader,))
        if chunk == self.vocab.chunk_count - 1:
            # the next call's first units stage behind the last chunk, and
            # are copied as the last chunks free their slots
            self.transformer_runtime.stage_call_ahead()

    def _prestage_first_chunks(self):
        for chunk in range(min(2, self.vocab.chunk_count)):
            self._prestage(chunk)

    def _chunk_source(self, chunk):
        """Pinned host rows of one chunk (staged first for pinned_staging)."""

        if not self._staged:
            rows = self._chunk_rows(chunk)
            if not rows.is_pinned():
                raise RuntimeError("a full_pinned store must hold the LM head "
                                   "in page-locked memory")
            return rows
        self._prestage(chunk)  # no-op when already queued
        return self._prestaged.pop(chunk).result()

    def quiesce(self):
        """Wait for the staging jobs still reading the store's arena (called
        by the store before its bytes change)."""

        for future in list(self._prestaged.values()):
            try:
                future.result()
            except Exception:  # the call that queued it already raised
                pass
        self._prestaged = {}

    def _copy_chunk(self, chunk):
        first, end = self.vocab.chunk_bounds(chunk)
        nbytes = (end - first) * self.vocab.hidden_size * 2
        pair = None
        if self.profile:
            timers = self._timing()
            pair = (timers["copy_start"][chunk], timers["copy_end"][chunk])
            self._timed[chunk] = nbytes
        self.transformer_runtime.slot_copy(chunk % 2, "chunk", chunk,
                                           self._chunk_source(chunk), nbytes,
                                           self._ready[chunk], pair)
        if self._staged:
            # this copy reads the chunk's pinned half; the chunk two ahead
            # is staged there once it is done
            self._staging_read[chunk % 2] = self._ready[chunk]
            self._prestage(chunk + 2)

    def _copy_first_chunk(self, slot):
        """Release hook of the transformer runtime: its last unit in
        ``slot`` is enqueued, so chunk ``slot`` can follow it there."""

        if slot < self.vocab.chunk_count:
            self._copy_chunk(slot)

    def _chunk_ready(self, chunk):
        held = self.transformer_runtime.slot_holding(chunk % 2, "chunk", chunk)
        if held is not None:
            return held
        self._copy_chunk(chunk)
        return self._ready[chunk]

    def _workspace(self, top_k):
        ws = self._workspaces.get(top_k)
        if ws is None:
            size = _hip.lm_head_workspace_bytes(self.vocab.chunk_rows, top_k)
            # zero-filled once; the kernel returns its ticket counter to 0
            ws = torch.zeros(size, dtype=torch.uint8, device=self.device)
            self._workspaces[top_k] = ws
        return ws

    def _timing(self):
        if self._timers is None:
            n = self.vocab.chunk_count

            def events(k):
                return [_hip.HipEvent(enable_timing=True) for _ in range(k)]

            self._timers = {
                "pipeline": events(2), "copy_start": events(n), "copy_end": events(n),
                "compute_start": events(n), "compute_end": events(n),
            }
        return self._timers

    def lm_head_topk(self, hidden_states, top_k=10, return_full_logits=False):
        """Stream row shards and maintain an exact global top-k."""

        width, vocab = self.vocab.hidden_size, self.vocab.vocab_size
        if hidden_states.shape[-1] != width:
            raise ValueError("hidden width {} does not match the vocabulary's "
                             "{}".format(hidden_states.shape[-1], width))
        if top_k < 1 or top_k > vocab:
            raise ValueError("top_k must lie in [1, {}], got {}".format(vocab, top_k))
        if top_k > 64:
            raise ValueError("the LM-head kernel keeps at most 64 candidates "
                             "(top_k {})".format(top_k))
        rows = hidden_states.reshape(-1, width)
        if rows.shape[0] != 1:
            raise ValueError("the streamed LM head scores one position, got "
                             "{}".format(rows.shape[0]))
        hidden = rows[0].contiguous()
        started = time.perf_counter()
        top_k = int(top_k)
        runtime = self.transformer_runtime
        chunks = self.vocab.chunk_count
        timers = self._timing() if self.profile else None
        workspace = self._workspace(top_k)
        lead = hidden_states.shape[:-1]
        values = torch.empty(lead + (top_k,), dtype=torch.float32, device=self.device)
        indices = torch.empty(lead + (top_k,), dtype=torch.int64, device=self.device)
        logits = None
        if return_full_logits:
            logits = torch.empty(lead + (vocab,), dtype=torch.float32,
                                 device=self.device)
        flat_logits = None if logits is None else logits.view(-1)

        # the hidden state (written on the caller's stream) precedes the kernels
        self._start.record(self.coordinator)
        self._start.wait(self.compute_stream)
        if timers:
            timers["pipeline"][0].record(self.coordinator)
        try:
            ready = {c: self._chunk_ready(c) for c in range(min(2, chunks))}
            for chunk in range(chunks):
                first, end = self.vocab.chunk_bounds(chunk)
                slot = chunk % 2
                ready.pop(chunk).synchronize()  # host hand-off: the chunk is in HBM
                weight = self.device_slots[slot][: (end - first) * width].view(-1, width)
                with torch.cuda.stream(self.compute_stream):
                    if timers:
                        timers["compute_start"][chunk].record(self.compute_stream)
                    _hip.lm_head_topk(
                        weight, hidden, top_k, first, chunk == 0, workspace, values,
                        indices,
                        logits_out=None if flat_logits is None else flat_logits[first:end],
                        stream=self.compute_stream,
                    )
                    if timers:
                        timers["compute_end"][chunk].record(self.compute_stream)
                    self._free[chunk].record(self.compute_stream)
                runtime.slot_released(slot, self._free[chunk])
                if chunk + 2 < chunks:
                    ready[chunk + 2] = self._chunk_ready(chunk + 2)
                else:
                    runtime.prefetch_next_call(slot)
        except BaseException:
            # staging jobs left in flight must not land in a half that a
            # later call stages again: wait for them, and for the copies
            self.quiesce()
            self.copy_stream.synchronize()
            self._staging_read = [None, None]
            raise

        last = self._free[chunks - 1]
        last.wait(self.coordinator)
        if timers:
            timers["pipeline"][1].record(self.coordinator)
        last.synchronize()  # values / indices are in HBM on return
        if timers:
            timers["pipeline"][1].synchronize()
            wall_ms = (time.perf_counter() - started) * 1000.0
            h2d_ms = sum(timers["copy_start"][c].elapsed_time(timers["copy_end"][c])
                         for c in self._timed)
            compute_ms = sum(a.elapsed_time(b) for a, b in
                             zip(timers["compute_start"], timers["compute_end"]))
            timed_bytes = sum(self._timed.values())
            self.last_profile = {
                "wall_ms": wall_ms,
                "pipeline_ms": timers["pipeline"][0].elapsed_time(timers["pipeline"][1]),
                "h2d_event_sum_ms": h2d_ms,
                "compute_event_sum_ms": compute_ms,
                "h2d_bytes": vocab * width * 2,
                "h2d_timed_bytes": timed_bytes,
                "h2d_effective_gbps": (timed_bytes / 1e9) / (h2d_ms / 1000.0)
                if h2d_ms else 0.0,
                "chunk_count": chunks,
                "chunk_rows": self.vocab.chunk_rows,
                "requested_top_k": top_k,
            }
        # chunks copied from here on (ahead of the next call) count there
        self._timed = {}
        return {"values": values, "indices": indices, "logits": logits}
