"""Row lookup and vocabulary-sharded LM head (reference layer_streaming/vocab.py).

* ``embedding(ids)`` gathers the requested rows of the host-only embedding
  into a page-locked staging buffer and copies them to the device
  (vocab.py:100-131).
* ``lm_head_topk(h, top_k, return_full_logits)`` streams the LM head in row
  chunks through the transformer runtime's two device slots and keeps an
  exact running top-k on the device (vocab.py:149-300).  Per chunk there is
  one kernel launch (cascade_lm_head_topk_bf16: GEMV to fp32 logits, block
  top-k and the merge with the running list), and no host synchronisation
  until the end of the call.
* ``merge_topk`` is the reference's public helper (vocab.py:11-32) with a
  deterministic order on ties (value descending, index ascending).

Logits are fp32 and not rounded to bf16 (the reference rounds them through
bf16 first, which creates ties inside the top-10 for almost every step at
this shape); the top-k order equals a stable descending sort of them.
"""

import time

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


class VocabStreamingRuntime:
    """Share the transformer runtime's slots for the LM-head chunks."""

    def __init__(self, plan, store, transformer_runtime,
                 embedding_staging_rows=256, profile=False):
        if plan.vocab is None:
            raise ValueError("plan does not enable vocabulary streaming")
        _hip.load()
        self.plan = plan
        self.vocab = plan.vocab
        self.store = store
        self.transformer_runtime = transformer_runtime
        self.device = transformer_runtime.device
        self.device_slots = transformer_runtime.device_slots
        self.copy_stream = transformer_runtime.copy_stream
        self.compute_stream = transformer_runtime.compute_stream
        self.coordinator = transformer_runtime.coordinator
        self.profile = bool(profile)
        self.last_profile = None
        self.last_embedding_bytes = 0
        self.embedding_staging_rows = int(embedding_staging_rows)
        if self.embedding_staging_rows < 1:
            raise ValueError("embedding_staging_rows must be positive")
        if len(self.device_slots) != 2:
            raise ValueError("vocabulary streaming requires two GPU slots")
        if self.device_slots[0].numel() < self.vocab.chunk_elements:
            raise ValueError("shared GPU slot is smaller than vocab chunk")
        self.embedding_staging = torch.empty(
            (self.embedding_staging_rows, self.vocab.hidden_size),
            dtype=torch.bfloat16, device="cpu", pin_memory=True,
        )
        self.head_staging_slots = None
        if self.store.mode == WeightStoreMode.PINNED_STAGING:
            self.head_staging_slots = [
                torch.empty(self.vocab.chunk_elements, dtype=torch.bfloat16,
                            device="cpu", pin_memory=True)
                for _ in range(2)
            ]
        count = self.vocab.chunk_count
        self._ready = [_hip.HipEvent() for _ in range(count)]
        self._free = [_hip.HipEvent() for _ in range(count)]
        self._start = _hip.HipEvent()
        self._embed_done = _hip.HipEvent()
        self._timing = None
        self._workspaces = {}

    @property
    def gpu_slot_bytes(self):
        return sum(s.numel() * s.element_size() for s in self.device_slots)

    @property
    def extra_pinned_cpu_bytes(self):
        total = self.embedding_staging.numel() * self.embedding_staging.element_size()
        if self.head_staging_slots is not None:
            total += sum(s.numel() * s.element_size() for s in self.head_staging_slots)
        return total

    def embedding(self, input_ids):
        """Gather only the requested CPU rows and transfer them to the GPU."""

        shape = tuple(input_ids.shape)
        ids = input_ids.detach().reshape(-1).to(device="cpu", dtype=torch.long)
        if ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= self.vocab.vocab_size):
            raise IndexError("token id outside the vocabulary")
        table = self.store.tensor(self.vocab.embedding_key)
        out = torch.empty((ids.numel(), self.vocab.hidden_size),
                          dtype=torch.bfloat16, device=self.device)
        self.last_embedding_bytes = ids.numel() * self.vocab.hidden_size * 2
        group = self.embedding_staging_rows
        for start in range(0, ids.numel(), group):
            end = min(start + group, ids.numel())
            staging = self.embedding_staging[: end - start]
            torch.index_select(table, 0, ids[start:end], out=staging)
            _hip.memcpy_h2d_async(out[start:end], staging,
                                  staging.numel() * 2, self.copy_stream)
            self._embed_done.record(self.copy_stream)
            # the staging rows are reused by the next group
            self._embed_done.synchronize()
        return out.view(shape + (self.vocab.hidden_size,))

    def _head_source(self, start_row, end_row, slot_index, ready_event):
        source = self.store.tensor(self.vocab.lm_head_key)[start_row:end_row].reshape(-1)
        if self.head_staging_slots is None:
            if not source.is_pinned():
                raise RuntimeError("full_pinned LM-head source unexpectedly is not pinned")
            return source
        if ready_event is not None:
            ready_event.synchronize()
        target = self.head_staging_slots[slot_index][: source.numel()]
        _hip.host_copy(target, source, getattr(self.store, "copy_threads", None))
        return target

    def _workspace(self, top_k):
        ws = self._workspaces.get(top_k)
        if ws is None:
            size = _hip.lm_head_workspace_bytes(self.vocab.chunk_rows, top_k)
            # zero-filled once; the kernel returns its ticket counter to 0
            ws = torch.zeros(size, dtype=torch.uint8, device=self.device)
            self._workspaces[top_k] = ws
        return ws

    def _timing_events(self):
        if self._timing is None:
            n = self.vocab.chunk_count

            def make(k):
                return [_hip.HipEvent(enable_timing=True) for _ in range(k)]

            self._timing = {
                "pipeline": make(2), "copy_start": make(n), "copy_end": make(n),
                "compute_start": make(n), "compute_end": make(n),
            }
        return self._timing

    def lm_head_topk(self, hidden_states, top_k=10, return_full_logits=False):
        """Stream row shards and maintain an exact global top-k."""

        if hidden_states.shape[-1] != self.vocab.hidden_size:
            raise ValueError("hidden state width does not match vocabulary")
        if top_k < 1 or top_k > self.vocab.vocab_size:
            raise ValueError("top_k is outside vocabulary range")
        if top_k > 64:
            raise ValueError("top_k above 64 is not supported by the LM-head kernel")
        hidden = hidden_states.reshape(-1, self.vocab.hidden_size)
        if hidden.shape[0] != 1:
            raise ValueError("the streamed LM head takes one position")
        hidden = hidden[0].contiguous()
        wall_started = time.perf_counter()
        chunks = self.vocab.chunk_count
        timing = self._timing_events() if self.profile else None
        workspace = self._workspace(int(top_k))
        lead = hidden_states.shape[:-1]
        values = torch.empty(lead + (int(top_k),), dtype=torch.float32, device=self.device)
        indices = torch.empty(lead + (int(top_k),), dtype=torch.int64, device=self.device)
        logits = None
        if return_full_logits:
            logits = torch.empty(lead + (self.vocab.vocab_size,),
                                 dtype=torch.float32, device=self.device)
        flat_logits = None if logits is None else logits.view(-1)

        self._start.record(self.coordinator)
        self._start.wait(self.copy_stream)
        self._start.wait(self.compute_stream)
        if timing:
            timing["pipeline"][0].record(self.coordinator)
        transferred = 0
        for c in range(chunks):
            slot_index = c % 2
            start_row, end_row = self.vocab.chunk_bounds(c)
            rows = end_row - start_row
            elements = rows * self.vocab.hidden_size
            source = self._head_source(start_row, end_row, slot_index,
                                       self._ready[c - 2] if c >= 2 else None)
            slot = self.device_slots[slot_index]
            if c >= 2:
                self._free[c - 2].wait(self.copy_stream)
            if timing:
                timing["copy_start"][c].record(self.copy_stream)
            _hip.memcpy_h2d_async(slot, source, elements * 2, self.copy_stream)
            if timing:
                timing["copy_end"][c].record(self.copy_stream)
            self._ready[c].record(self.copy_stream)
            transferred += elements * 2

            self._ready[c].wait(self.compute_stream)
            if timing:
                timing["compute_start"][c].record(self.compute_stream)
            weight = slot[:elements].view(rows, self.vocab.hidden_size)
            _hip.lm_head_topk(
                weight, hidden, int(top_k), start_row, c == 0, workspace,
                values, indices,
                logits_out=None if flat_logits is None else flat_logits[start_row:end_row],
                stream=self.compute_stream,
            )
            if timing:
                timing["compute_end"][c].record(self.compute_stream)
            self._free[c].record(self.compute_stream)

        self._free[chunks - 1].wait(self.coordinator)
        if timing:
            timing["pipeline"][1].record(self.coordinator)
        self.coordinator.synchronize()
        wall_ms = (time.perf_counter() - wall_started) * 1000.0
        if timing:
            h2d_ms = sum(a.elapsed_time(b) for a, b in
                         zip(timing["copy_start"], timing["copy_end"]))
            compute_ms = sum(a.elapsed_time(b) for a, b in
                             zip(timing["compute_start"], timing["compute_end"]))
            self.last_profile = {
                "wall_ms": wall_ms,
                "pipeline_ms": timing["pipeline"][0].elapsed_time(timing["pipeline"][1]),
                "h2d_event_sum_ms": h2d_ms,
                "compute_event_sum_ms": compute_ms,
                "h2d_bytes": transferred,
                "h2d_effective_gbps": (transferred / 1e9) / (h2d_ms / 1000.0),
                "chunk_count": chunks,
                "chunk_rows": self.vocab.chunk_rows,
                "requested_top_k": int(top_k),
            }
        return {"values": values, "indices": indices, "logits": logits}
