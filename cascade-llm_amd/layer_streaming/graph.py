"""Greedy batch-1 decode of an HBM-resident model as one replayed HIP graph
per token.

The reference's token loop (tools/run_llama31.py:105-121) runs
``executor.begin`` / ``runtime.run`` / ``executor.finish`` per token, feeds
``topk_indices[..., 0]`` back as the next input, and derives every kernel's
position from the host (position_ids from the cache length,
layer_streaming/llama31.py:131-143).  Here the cached length lives in a
device word instead:

- the step's first launch (cascade_decode_step_begin_bf16) gathers the
  embedding of the previous step's top-1 id, records that id in ``history``
  at its position, and advances the word;
- the q|k|v launches (cascade_qkv_rope_at_bf16) take RoPE row and KV slot
  from the word, and the attention launches
  (cascade_decode_attention_fused_at_bf16, or cascade_decode_attention_at_bf16
  where the fused form does not apply) their length;
- the LM head writes its top-k into fixed buffers, whose first id is the
  next step's input.

So one captured graph of the whole step (every launch of the 32 layers and
the head) serves every token; a token costs the host one replay call, and
no host value changes between tokens.  Everything the graph touches is
allocated before capture; a replay refuses to run if the executor has since
moved any of it (a KV cache, RoPE table or workspace that grew).
"""

import torch

from . import _hip
from .runtime import ResidentTransformerRuntime


class DeviceStep:
    """Device words and fixed buffers of a device-position decode step.

    ``length`` (int64 [1]) is the cached length: tokens at positions
    [0, length) are in the KV cache.  ``history[p]`` is the token id at
    position p for every position a step has consumed.  ``indices[0, 0, 0]``
    (``ids``) is the last step's top-1 id, i.e. the next step's input.
    """

    def __init__(self, device, capacity, vocab, top_k):
        self.capacity = int(capacity)
        self.length = torch.zeros(1, dtype=torch.int64, device=device)
        self.history = torch.full((self.capacity,), -1, dtype=torch.int64,
                                  device=device)
        self.error = torch.zeros(1, dtype=torch.int32, device=device)
        self.logits = torch.empty((1, 1, vocab), dtype=torch.float32,
                                  device=device)
        self.values = torch.empty((1, 1, top_k), dtype=torch.float32,
                                  device=device)
        self.indices = torch.zeros((1, 1, top_k), dtype=torch.int64,
                                   device=device)
        self.ids = self.indices.view(1, -1)[:, :1]
        # True only while the owning DecodeGraph runs or captures a step:
        # the executor refuses other calls meanwhile (they would advance
        # the device length behind the graph's back)
        self.active = False


class DecodeGraph:
    """Greedy decode of up to ``max_new_tokens`` tokens after the cached
    prompt, one HIP-graph replay per token.

    ``token`` ([1, 1] int64) is the first input: the token at position
    ``past`` (the prompt's argmax after a prefill, or any id).  Construction
    runs that first step eagerly through the same kernels (it fills the
    executor's lazily made buffers) and captures the second; ``step()``
    replays it.  ``tokens()`` returns the ids generated so far, in order.

    Requires an executor without a streamed vocabulary (the LM head is
    resident) and a ResidentTransformerRuntime: streamed weights would put
    host copies and cross-stream events in the step.
    """

    def __init__(self, executor, runtime, token, max_new_tokens):
        if not isinstance(runtime, ResidentTransformerRuntime):
            raise TypeError("DecodeGraph needs a ResidentTransformerRuntime")
        if executor.vocab_runtime is not None:
            raise ValueError("DecodeGraph needs the resident LM head")
        if executor._device_step is not None:
            raise RuntimeError("the executor already runs a DecodeGraph")
        if executor.capture is not None:
            # its hidden-state clones would be captured and replayed into
            # the graph's own memory pool
            raise ValueError("DecodeGraph needs executor.capture = None")
        if int(max_new_tokens) < 2:
            raise ValueError("max_new_tokens must be at least 2")
        # a bad id in the eager steps before raises here, not in the graph
        executor.check_errors()
        self.executor = executor
        self.runtime = runtime
        self.device = executor.device
        self.past = executor.kv_cache.sequence_length()
        self.max_new_tokens = int(max_new_tokens)
        capacity = self.past + self.max_new_tokens
        executor.reserve(capacity)
        executor._ensure_attention_workspace(capacity)
        head = executor.resident["lm_head.weight"]
        step = DeviceStep(self.device, capacity, head.shape[0], executor.top_k)
        _hip.require_device(token, "token", torch.int64, 1, contiguous=False)
        step.length.fill_(self.past)
        step.indices.view(-1)[:1].copy_(token.reshape(-1)[:1])
        self.step_buffers = step
        self.graph = None
        self._sync = runtime.synchronize
        runtime.synchronize = False
        executor._device_step = step
        try:
            self._run_step()  # first token, eagerly
            self.decoded = 1
            self._set_host_length()
            torch.cuda.synchronize(self.device)
            self._pins = self._buffers()
            # kernel timing events are per launch call, not per replay
            timed = (executor._instrumented, executor._instrument_next)
            executor._instrumented, executor._instrument_next = {}, {}
            self.graph = torch.cuda.CUDAGraph()
            try:
                with torch.cuda.graph(self.graph):
                    self._run_step()
            finally:
                executor._instrumented, executor._instrument_next = timed
            # capture ran no kernels: the host view of the cache is one
            # step ahead of the device
            self._set_host_length()
        except BaseException:
            self.close()
            raise

    # ---------------------------------------------------------------- steps

    def _run_step(self):
        ex = self.executor
        self.step_buffers.active = True
        try:
            state = ex.begin(self.step_buffers.ids)
            state = self.runtime.run(ex, state)
            ex.finish(state)
        finally:
            self.step_buffers.active = False

    def _set_host_length(self):
        cache = self.executor.kv_cache
        for layer in range(cache.layer_count):
            cache.set_length(layer, self.past + self.decoded)

    def _buffers(self):
        ex = self.executor
        return (ex.kv_cache.buffer.data_ptr(), ex.kv_cache.capacity,
                ex.rope.cos.data_ptr(), ex.rope.sin.data_ptr(),
                ex._attn_ws.data_ptr(), ex._attn_sync.data_ptr(),
                ex._head_ws.data_ptr(), ex._q_ptr,
                ex._attn_ptr, ex._normed_ptr, ex._gate_ptr, ex._inter_ptr)

    def step(self, count=1):
        """Decode ``count`` more tokens (graph replays on the current
        stream; nothing waits for them)."""

        if self.graph is None:
            raise RuntimeError("DecodeGraph is closed")
        if self.decoded + count > self.max_new_tokens:
            raise RuntimeError("DecodeGraph holds {} tokens".format(
                self.max_new_tokens))
        if self._buffers() != self._pins:
            raise RuntimeError("executor buffers moved since capture")
        for _ in range(count):
            self.graph.replay()
            self.decoded += 1
        self._set_host_length()

    def tokens(self):
        """Generated ids so far ([1, decoded] int64 on the device): the
        inputs of steps 2..n, which history holds by position, and the last
        step's top-1."""

        step = self.step_buffers
        start = self.past + 1
        return torch.cat([step.history[start:self.past + self.decoded],
                          step.indices.view(-1)[:1]]).view(1, -1)

    def check(self):
        """Raise if a step saw an id outside the vocabulary or ran out of
        positions (waits for the GPU)."""

        value = int(self.step_buffers.error.item())
        if value != 0:
            if value & (_hip.ATTN_EPLACEMENT | _hip.ATTN_ETIMEOUT):
                # the fused attention's counters are no longer at zero
                self.executor._attn_sync.zero_()
            raise RuntimeError("decode step error flag set ({})".format(value))

    def close(self):
        self.executor._device_step = None
        self.runtime.synchronize = self._sync
        self.graph = None
