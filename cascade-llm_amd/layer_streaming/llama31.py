"""Llama-3.1-8B decode executor running on the libcascade_hip kernels.

Public surface as in the reference (layer_streaming/llama31.py):
``Llama31DecodeExecutor(config, resident, kv_cache, vocab_runtime, top_k,
return_full_logits)`` with ``begin`` / ``__call__`` / ``finish``,
``SimpleKVCache`` and ``DecodeState``.  The executor is the ``compute_unit``
callback of the runtimes: each call enqueues the kernels of one transfer
unit on the current (compute) stream.

Operation -> kernels (reference lines in parentheses):
  qkv / q_proj / k_proj / v_proj   cascade_qkv_rope_bf16: input RMSNorm,
      the projection(s), RoPE and the KV-cache write in one launch per
      token (:169-180, :206-218, :241-245)
  o_proj     cascade_decode_attention_fused_bf16 (split merge inside the
      launch; cascade_decode_attention_bf16 below 225 positions) then
      cascade_gemv_residual_bf16 (:182-234, :246-251)
  gate_up    cascade_gate_up_swiglu_bf16 (post-attention RMSNorm, both
      projections, SiLU and the product; :252-275)
  gate_proj / up_proj   cascade_gate_silu_bf16 / cascade_up_mul_bf16
  down_proj  cascade_gemv_residual_bf16 (:272-279)
  finish     cascade_rmsnorm_bf16 + the LM head (cascade_lm_head_topk_bf16,
      resident head or VocabStreamingRuntime) (:324-349)
A call with S > 1 tokens at consecutive positions (every prefill the
reference makes) runs each matrix once over all S token rows on the matrix
cores: cascade_rmsnorm_bf16 over the rows, then
  qkv        cascade_qkv_rope_gemm_bf16 (projections, RoPE, KV write)
  o_proj     cascade_prefill_attention_bf16 (causal: token t attends to
      positions <= past + t, the is_causal SDPA of :223-229) then
      cascade_gemm_residual_bf16
  gate_up    cascade_gate_up_swiglu_gemm_bf16 (or the silu / mul halves)
  down_proj  cascade_gemm_residual_bf16
  finish     (resident head) cascade_gemm_f32out_bf16 for the logits of
      every position, as the reference's F.linear over [1, S, H]
Position ids with gaps run the per-token kernels for t = 0..S-1 instead.
"""

import inspect
import weakref
from dataclasses import dataclass, field

import torch

from . import _hip
from .rope import RopeTable, rope_parameters

__all__ = [
    "LLAMA31_8B_MODEL_ID",
    "MATRIX_ORDER",
    "Llama31Config",
    "SimpleKVCache",
    "DecodeState",
    "Llama31DecodeExecutor",
]

LLAMA31_8B_MODEL_ID = "meta-llama/Llama-3.1-8B"
MATRIX_ORDER = (
    "q_proj",
    "k_proj",
    "v_proj",
    "o_proj",
    "gate_proj",
    "up_proj",
    "down_proj",
)


@dataclass
class Llama31Config:
    """The Llama-3.1-8B config fields the executor reads (stand-in for a
    transformers LlamaConfig when there is no checkpoint directory)."""

    hidden_size: int = 4096
    intermediate_size: int = 14336
    num_hidden_layers: int = 32
    num_attention_heads: int = 32
    num_key_value_heads: int = 8
    vocab_size: int = 128256
    rms_norm_eps: float = 1e-5
    rope_theta: float = 500000.0
    rope_scaling: dict = field(
        default_factory=lambda: {
            "rope_type": "llama3",
            "factor": 8.0,
            "low_freq_factor": 1.0,
            "high_freq_factor": 4.0,
            "original_max_position_embeddings": 8192,
        }
    )
    max_position_embeddings: int = 131072
    tie_word_embeddings: bool = False


class SimpleKVCache:
    """Single-request KV cache, preallocated in HBM and grown by doubling.

    Layout: one bf16 buffer [layers, 2 (K, V), kv_heads, capacity, head_dim];
    the attention kernel reads KV head g of a layer at
    ``g * head_stride`` elements.  ``entries[layer]`` gives the reference's
    (key, value) pair of [1, kv_heads, length, head_dim] views
    (reference llama31.py:34-54).
    """

    def __init__(self, layer_count=32, num_kv_heads=8, head_dim=128,
                 capacity=0, device=None):
        self.layer_count = int(layer_count)
        self.num_kv_heads = int(num_kv_heads)
        self.head_dim = int(head_dim)
        self.device = None if device is None else torch.device(device)
        self.capacity = 0
        self.buffer = None
        self.lengths = [0] * self.layer_count
        if capacity:
            self.reserve(capacity)

    @property
    def head_stride(self):
        return self.capacity * self.head_dim

    def reserve(self, length, device=None):
        """Make room for ``length`` positions (copies existing entries)."""

        if device is not None and self.device is None:
            self.device = torch.device(device)
        if length <= self.capacity:
            return
        if self.device is None:
            raise RuntimeError("KV cache device is unknown")
        capacity = max(int(length), 2 * self.capacity, 256)
        capacity = -(-capacity // 256) * 256
        buffer = torch.empty(
            (self.layer_count, 2, self.num_kv_heads, capacity, self.head_dim),
            dtype=torch.bfloat16,
            device=self.device,
        )
        if self.buffer is not None:
            used = max(self.lengths)
            if used:
                buffer[:, :, :, :used].copy_(self.buffer[:, :, :, :used])
        self.buffer = buffer
        self.capacity = capacity

    def layer_base(self, layer_index, which):
        """Flat view from position 0 of KV head 0 (which: 0 = K, 1 = V)."""

        return self.buffer[layer_index, which].view(-1)

    def sequence_length(self):
        return self.lengths[0]

    @property
    def entries(self):
        out = []
        for layer in range(self.layer_count):
            n = self.lengths[layer]
            if n == 0:
                out.append(None)
            else:
                out.append(
                    (
                        self.buffer[layer, 0, :, :n].unsqueeze(0),
                        self.buffer[layer, 1, :, :n].unsqueeze(0),
                    )
                )
        return out

    def append(self, layer_index, key, value):
        """Append [1, kv_heads, S, head_dim] key / value tensors."""

        n = key.shape[-2]
        start = self.lengths[layer_index]
        self.reserve(start + n, device=key.device)
        self.buffer[layer_index, 0, :, start : start + n].copy_(key[0])
        self.buffer[layer_index, 1, :, start : start + n].copy_(value[0])
        self.lengths[layer_index] = start + n
        return self.entries[layer_index]

    def set_length(self, layer_index, length):
        self.lengths[layer_index] = int(length)

    def clear(self):
        self.lengths = [0] * self.layer_count


@dataclass
class DecodeState:
    hidden_states: torch.Tensor
    position_ids: torch.Tensor
    layer_values: dict = field(default_factory=dict)
    logits: object = None
    topk_values: object = None
    topk_indices: object = None
    positions: tuple = ()


_EXPECTED = {
    "hidden_size": 4096,
    "intermediate_size": 14336,
    "num_attention_heads": 32,
    "num_key_value_heads": 8,
    "vocab_size": 128256,
}

# Kernel groups whose entry point launches exactly one kernel.
_KERNEL_TIMED_GROUPS = frozenset((
    "gate_up", "qkv", "o_proj", "down_proj",
    # prefill (S > 1 tokens): one MFMA GEMM / attention launch per unit
    "gemm_qkv", "gemm_o", "gemm_gate_up", "gemm_gate", "gemm_up", "gemm_down",
    "gemm_lm_head", "prefill_attention"))


def _check_ids(ids, vocab):
    if ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= vocab):
        raise IndexError("token id outside [0, {})".format(vocab))


class _ErrorWord:
    """An int32 device flag that kernels set on bad input, read back without
    blocking: ``publish`` copies it to pinned memory behind the step's work,
    ``raise_if_set`` raises once that copy has landed (or waits for it).

    The embedding gather stores 1 for an id outside the vocabulary
    (IndexError); the fused decode attention ors in _hip.ATTN_EPLACEMENT /
    ATTN_ETIMEOUT (RuntimeError, after ``on_attention_error(value)`` has
    run)."""

    def __init__(self, device, message, on_attention_error=None):
        self.message = message
        # a method of the word's owner is held weakly: the owner holds the
        # word, and a strong reference back would keep the owner and its
        # device buffers alive until a cyclic garbage collection
        if inspect.ismethod(on_attention_error):
            self._on_attention_error = weakref.WeakMethod(on_attention_error)
        else:
            self._on_attention_error = lambda cb=on_attention_error: cb
        self.flag = torch.zeros(1, dtype=torch.int32, device=device)
        self.host = torch.zeros(1, dtype=torch.int32,
                                pin_memory=device.type == "cuda")
        self.event = _hip.HipEvent() if device.type == "cuda" else None
        self.pending = False

    def publish(self):
        """Copy the flag to the host behind the current stream's work."""

        self.host.copy_(self.flag, non_blocking=True)
        if self.event is not None:
            self.event.record()
        self.pending = True

    def raise_if_set(self, block=False):
        if not self.pending:
            return
        if self.event is not None:
            if block:
                self.event.synchronize()
            elif not self.event.query():
                return
        self.pending = False
        value = int(self.host[0])
        if value != 0:
            self.flag.zero_()
            self.host.zero_()
            if value & ~1:
                callback = self._on_attention_error()
                if callback is not None:
                    callback(value)
                raise RuntimeError(_attention_error_message(value))
            raise IndexError(self.message)


def _attention_error_message(value):
    if value & _hip.ATTN_EPLACEMENT:
        return ("fused decode attention: the device did not deal the "
                "workgroups evenly over 8 XCDs")
    return "fused decode attention: a split-merge wait ran out"


class Llama31DecodeExecutor:
    """Stateful callbacks consumed by the runtimes (one unpadded request: a
    multi-token prefill, then one-token decode calls)."""

    def __init__(self, config, resident, kv_cache=None, vocab_runtime=None,
                 top_k=10, return_full_logits=False):
        _hip.load()  # no kernels, no executor
        layers = getattr(resident, "plan", None)
        layers = layers.num_layers if layers is not None else 32
        expected = dict(_EXPECTED, num_hidden_layers=layers)
        for name, value in expected.items():
            if getattr(config, name, None) != value:
                raise ValueError(
                    "config {}={} is not Llama-3.1-8B value {}".format(
                        name, getattr(config, name, None), value
                    )
                )
        self.config = config
        self.resident = resident
        self.vocab_runtime = vocab_runtime
        self.top_k = int(top_k)
        self.return_full_logits = bool(return_full_logits)
        if self.top_k < 1:
            raise ValueError("top_k must be positive")
        if self.top_k > 64:
            raise ValueError("top_k above 64 is not supported by the LM-head kernel")
        self.device = resident.device
        self.hidden = config.hidden_size
        self.head_dim = config.hidden_size // config.num_attention_heads
        self.n_heads = config.num_attention_heads
        self.n_kv_heads = config.num_key_value_heads
        self.kv_groups = self.n_heads // self.n_kv_heads
        self.eps = float(config.rms_norm_eps)
        self.scale = self.head_dim ** -0.5
        self.kv_cache = kv_cache or SimpleKVCache(
            config.num_hidden_layers, self.n_kv_heads, self.head_dim,
            device=self.device,
        )
        if self.kv_cache.device is None:
            self.kv_cache.device = self.device
        self.rope = RopeTable(self.head_dim, rope_parameters(config), self.device)
        self.intermediate = config.intermediate_size
        self._norms = [
            (
                resident["model.layers.{}.input_layernorm.weight".format(i)],
                resident["model.layers.{}.post_attention_layernorm.weight".format(i)],
            )
            for i in range(config.num_hidden_layers)
        ]
        for pair in self._norms:
            for norm in pair:
                _hip.require_device(norm, "norm weight", torch.bfloat16, self.hidden)
        self._norm_ptrs = [(a.data_ptr(), b.data_ptr()) for a, b in self._norms]
        lib = _hip.load()
        self._k_qkv = lib.cascade_qkv_rope_bf16
        self._k_attn = lib.cascade_decode_attention_bf16
        self._k_residual = lib.cascade_gemv_residual_bf16
        self._k_swiglu = lib.cascade_gate_up_swiglu_bf16
        self._k_silu = lib.cascade_gate_silu_bf16
        self._k_mul = lib.cascade_up_mul_bf16
        self._k_rmsnorm = lib.cascade_rmsnorm_bf16
        self._k_head = lib.cascade_lm_head_topk_bf16
        self._k_qkv_gemm = lib.cascade_qkv_rope_gemm_bf16
        self._k_prefill_attn = lib.cascade_prefill_attention_bf16
        self._k_gemm_residual = lib.cascade_gemm_residual_bf16
        self._k_gemm_residual_ws = lib.cascade_gemm_residual_ws_bf16
        self._k_swiglu_gemm = lib.cascade_gate_up_swiglu_gemm_bf16
        self._k_silu_gemm = lib.cascade_gate_silu_gemm_bf16
        self._k_mul_gemm = lib.cascade_up_mul_gemm_bf16
        self._k_f32_gemm = lib.cascade_gemm_f32out_bf16
        self._k_topk = lib.cascade_topk_f32
        self._k_qkv_at = lib.cascade_qkv_rope_at_bf16
        self._k_attn_at = lib.cascade_decode_attention_at_bf16
        self._k_attn_fused = lib.cascade_decode_attention_fused_bf16
        self._k_attn_fused_at = lib.cascade_decode_attention_fused_at_bf16
        self._k_step_begin = lib.cascade_decode_step_begin_bf16
        # Set by DecodeGraph (layer_streaming/graph.py): decode steps take
        # their position from a device word instead of host values.
        self._device_step = None
        self._batched = False
        self._first_slot = 0
        self._unit_cache = {}
        self._instrumented = {}
        self._instrument_next = {}
        # Debug hook: a list receives (layer, hidden copy) after the
        # embedding (layer -1) and after every decoder layer.
        self.capture = None
        self._tokens_cap = 0
        self._gemm_ws, self._gemm_ws_rows, self._gemm_ws_need = None, -1, 0
        self._attn_ws = None
        self._attn_ws_len = 0
        self._head_ws = None
        # decode attention merges its splits inside the attention launch
        # where the shape allows (one KV head per XCD, >= 8 splits); its
        # counters live in this zero-filled buffer, reset after an error
        self._fused_attention = self.n_kv_heads == _hip.FUSED_ATTENTION_KV_HEADS
        self._attn_sync = torch.zeros(_hip.ATTENTION_SYNC_BYTES, dtype=torch.uint8,
                                      device=self.device)
        self._id_errors = _ErrorWord(self.device, "token id outside [0, {})".format(
            config.vocab_size), on_attention_error=self._attention_failed)
        self._ensure_buffers(1)

    def _attention_failed(self, value):
        """The fused attention flagged ``value``: its counters are zero-filled
        for the next call, and a device that does not deal workgroups evenly
        over 8 XCDs (another partition mode or part) gets the two-launch
        attention from then on."""

        self._attn_sync.zero_()
        if value & _hip.ATTN_EPLACEMENT:
            self._fused_attention = False

    # ------------------------------------------------------------ buffers

    def _ensure_buffers(self, tokens):
        if tokens <= self._tokens_cap:
            return
        dev = self.device
        bf16 = torch.bfloat16
        self._q = torch.empty((tokens, self.hidden), dtype=bf16, device=dev)
        self._attn = torch.empty((tokens, self.hidden), dtype=bf16, device=dev)
        self._gate_buf = torch.empty(
            (tokens, self.config.intermediate_size), dtype=bf16, device=dev)
        self._inter = torch.empty(
            (tokens, self.config.intermediate_size), dtype=bf16, device=dev)
        self._normed = torch.empty((tokens, self.hidden), dtype=bf16, device=dev)
        self._q_ptr = self._q.data_ptr()
        self._normed_ptr = self._normed.data_ptr()
        self._attn_ptr = self._attn.data_ptr()
        self._gate_ptr = self._gate_buf.data_ptr()
        self._inter_ptr = self._inter.data_ptr()
        self._tokens_cap = tokens

    def _gemm_workspace(self, tokens):
        """(pointer, bytes) of the split-K workspace for o_proj / down_proj
        over `tokens` rows ((0, 0) where those shapes run in one pass)."""

        if tokens != self._gemm_ws_rows:
            need = max(_hip.gemm_workspace_bytes(tokens, self.hidden, self.hidden),
                       _hip.gemm_workspace_bytes(tokens, self.hidden,
                                                 self.intermediate))
            have = 0 if self._gemm_ws is None else self._gemm_ws.numel()
            if need > have:
                self._gemm_ws = torch.empty(need, dtype=torch.uint8,
                                            device=self.device)
            self._gemm_ws_rows, self._gemm_ws_need = tokens, need
        if self._gemm_ws_need == 0:
            return 0, 0
        return self._gemm_ws.data_ptr(), self._gemm_ws.numel()

    def _ensure_attention_workspace(self, length):
        if length <= self._attn_ws_len:
            return
        target = max(length, 2 * self._attn_ws_len, 4096)
        size = _hip.attention_workspace_bytes(
            target, self.n_heads, self.n_kv_heads, self.head_dim)
        # zero-filled once: the kernel's completion counters start at 0 and
        # every call leaves them at 0
        self._attn_ws = torch.zeros(size, dtype=torch.uint8, device=self.device)
        self._attn_ws_len = target

    def reserve(self, length):
        """Pre-size the KV cache, RoPE table and workspaces for ``length``
        positions (avoids growth inside a timed loop)."""

        self.kv_cache.reserve(length, device=self.device)
        self.rope.reserve(length)
        self._ensure_attention_workspace(length)

    # --------------------------------------------------------------- API

    def begin(self, input_ids, position_ids=None):
        if self._device_step is not None and not self._device_step.active:
            raise RuntimeError("the executor belongs to an open DecodeGraph "
                               "(decode with DecodeGraph.step, or close it)")
        if input_ids.ndim != 2 or input_ids.shape[0] != 1:
            raise ValueError("first runtime supports one unpadded request")
        past = self.kv_cache.sequence_length()
        sequence = int(input_ids.shape[1])
        if past and sequence != 1:
            raise ValueError("after prefill, only one-token decode calls are supported")
        if position_ids is None:
            positions = tuple(range(past, past + sequence))
            position_ids = torch.arange(past, past + sequence,
                                        dtype=torch.long).unsqueeze(0)
        else:
            positions = tuple(int(p) for p in position_ids.reshape(-1).tolist())
            if len(positions) != sequence:
                raise ValueError("position_ids must match input_ids")
        if positions and min(positions) < 0:
            raise ValueError("negative position id")
        # Token t attends to cache positions [0, past + t]; its K/V land at
        # slot past + t (the reference appends in order, llama31.py:44-50).
        self.reserve(past + sequence)
        self.rope.reserve(max(positions) + 1)
        self._ensure_buffers(sequence)
        if self.vocab_runtime is None:
            if self._device_step is None:
                self._id_errors.raise_if_set()
            hidden = torch.empty((1, sequence, self.hidden),
                                 dtype=torch.bfloat16, device=self.device)
            ids = input_ids.reshape(-1)
            table = self.resident["model.embed_tokens.weight"]
            if ids.device.type == "cpu" or sequence > 1:
                # ids the host has (or a prompt, read back once): checked
                # here, as F.embedding raises on them
                _check_ids(ids.to("cpu"), table.shape[0])
            if ids.device != self.device or ids.dtype != torch.long:
                ids = ids.to(device=self.device, dtype=torch.long)
            step = self._device_step
            if step is None:
                # a device-held id (the previous step's top-1) is checked by
                # the gather kernel, which flags it; finish() publishes the
                # flag and the next begin() / finish() raises
                _hip.embedding_gather(table, ids, hidden, self._id_errors.flag)
            else:
                if sequence != 1:
                    raise ValueError("a device-position step decodes one token")
                _hip.check("cascade_decode_step_begin_bf16", self._k_step_begin(
                    table.data_ptr(), table.shape[0], self.hidden,
                    ids.data_ptr(), hidden.data_ptr(), step.length.data_ptr(),
                    step.history.data_ptr(), step.capacity,
                    step.error.data_ptr(), self._stream()))
        else:
            hidden = self.vocab_runtime.embedding(input_ids)
        _hip.require_device(hidden, "hidden_states", torch.bfloat16,
                            sequence * self.hidden)
        if self.capture is not None:
            self.capture.append((-1, hidden.detach().clone()))
        return DecodeState(hidden_states=hidden, position_ids=position_ids,
                           positions=positions)

    def _token_rows(self, state):
        return state.hidden_states.view(-1, self.hidden)

    # ------------------------------------------------------ unit launches
    # Units launch on raw pointers.  A unit's weight views are validated
    # (device, dtype, shape, alignment) the first time a (unit, slot) pair is
    # seen; per-token pointers are byte offsets into buffers that begin()
    # sized: the hidden rows, the q / attention / intermediate scratch rows,
    # the KV cache slots and the RoPE rows.

    def _stream(self):
        """Raw handle of the current stream (kernels launch there)."""

        return torch.cuda.current_stream(self.device).cuda_stream

    def _unit_pointers(self, unit, weights):
        first = weights[unit.pieces[0].tensor.key]
        key = (unit.unit_id, first.data_ptr())
        entry = self._unit_cache.get(key)
        if entry is None:
            if len(self._unit_cache) > 4096:
                self._unit_cache.clear()
            entry = {}
            for piece in unit.pieces:
                spec = piece.tensor
                view = weights[spec.key]
                _hip.bf16_weight(view, spec.key, *spec.shape)
                entry[spec.key.rsplit(".", 2)[-2]] = view.data_ptr()
            self._unit_cache[key] = entry
        return entry

    def _slots(self, state):
        """Cache slots of the state's tokens (past .. past + S - 1)."""

        first = self._first_slot
        return range(first, first + len(state.positions))

    def _kv_pointer(self, layer, which, slot):
        cache = self.kv_cache
        element = ((layer * 2 + which) * cache.num_kv_heads * cache.capacity
                   + slot) * cache.head_dim
        return cache.buffer.data_ptr() + 2 * element

    def _qkv(self, layer, ptrs, state, stream):
        wq = ptrs.get("q_proj", 0)
        wk = ptrs.get("k_proj", 0)
        wv = ptrs.get("v_proj", 0)
        nq = self.hidden if wq else 0
        nkv = self.n_kv_heads * self.head_dim
        nk = nkv if wk else 0
        nv = nkv if wv else 0
        x = state.hidden_states.data_ptr()
        row = 2 * self.hidden
        norm = self._norm_ptrs[layer][0]
        stride = self.kv_cache.head_stride
        cos = self.rope.cos.data_ptr()
        sin = self.rope.sin.data_ptr()
        half = self.head_dim // 2
        step = self._device_step
        if step is not None:
            # position = *length - 1 on the device; tables and cache from row 0
            ev = self._mark_begin("qkv")
            rc = self._k_qkv_at(
                wq, wk, wv, nq, nk, nv, self.hidden, x, norm, self.eps, cos, sin,
                self._q_ptr if wq else 0,
                self._kv_pointer(layer, 0, 0) if wk else 0,
                self._kv_pointer(layer, 1, 0) if wv else 0,
                stride, step.length.data_ptr(), step.capacity, stream)
            self._mark_end("qkv", ev, rc)
            _hip.check("cascade_qkv_rope_at_bf16", rc)
            return
        for t, slot in enumerate(self._slots(state)):
            pos = state.positions[t]
            ev = self._mark_begin("qkv")
            rc = self._k_qkv(
                wq, wk, wv, nq, nk, nv, self.hidden, x + t * row, norm, self.eps,
                cos + 2 * half * pos, sin + 2 * half * pos,
                self._q_ptr + t * row if wq else 0,
                self._kv_pointer(layer, 0, slot) if wk else 0,
                self._kv_pointer(layer, 1, slot) if wv else 0,
                stride, stream)
            self._mark_end("qkv", ev, rc)
            _hip.check("cascade_qkv_rope_bf16", rc)

    def _attention_o(self, layer, ptrs, state, stream, with_o=True):
        row = 2 * self.hidden
        k0 = self._kv_pointer(layer, 0, 0)
        v0 = self._kv_pointer(layer, 1, 0)
        stride = self.kv_cache.head_stride
        ws, ws_bytes = self._attn_ws.data_ptr(), self._attn_ws.numel()
        step = self._device_step
        sync = self._attn_sync.data_ptr()
        min_len = _hip.FUSED_ATTENTION_MIN_LEN
        for t, slot in enumerate(self._slots(state)):
            ev = self._mark_begin("attention")
            if step is not None:
                if self._fused_attention and step.capacity >= min_len:
                    name = "cascade_decode_attention_fused_at_bf16"
                    rc = self._k_attn_fused_at(
                        self._q_ptr, k0, v0, stride, step.length.data_ptr(),
                        step.capacity, self.n_heads, self.n_kv_heads,
                        self.head_dim, self.scale, self._attn_ptr, ws, ws_bytes,
                        sync, step.error.data_ptr(), stream)
                else:
                    name = "cascade_decode_attention_at_bf16"
                    rc = self._k_attn_at(
                        self._q_ptr, k0, v0, stride, step.length.data_ptr(),
                        step.capacity, self.n_heads, self.n_kv_heads,
                        self.head_dim, self.scale, self._attn_ptr, ws, ws_bytes,
                        stream)
                self._mark_end("attention", ev, rc)
                _hip.check(name, rc)
                if with_o:
                    self._o_residual(ptrs, state, t, stream)
                continue
            if self._fused_attention and slot + 1 >= min_len:
                name = "cascade_decode_attention_fused_bf16"
                rc = self._k_attn_fused(
                    self._q_ptr + t * row, k0, v0, stride, slot + 1, self.n_heads,
                    self.n_kv_heads, self.head_dim, self.scale,
                    self._attn_ptr + t * row, ws, ws_bytes, sync,
                    self._id_errors.flag.data_ptr(), stream)
            else:
                name = "cascade_decode_attention_bf16"
                rc = self._k_attn(self._q_ptr + t * row, k0, v0, stride, slot + 1,
                                  self.n_heads, self.n_kv_heads, self.head_dim,
                                  self.scale, self._attn_ptr + t * row, ws,
                                  ws_bytes, stream)
            self._mark_end("attention", ev, rc)
            _hip.check(name, rc)
            if with_o:
                self._o_residual(ptrs, state, t, stream)
        self.kv_cache.set_length(layer, self._first_slot + len(state.positions))

    def _o_residual(self, ptrs, state, t, stream):
        row = 2 * self.hidden
        xt = state.hidden_states.data_ptr() + t * row
        ev = self._mark_begin("o_proj")
        rc = self._k_residual(ptrs["o_proj"], self._attn_ptr + t * row, xt, xt,
                              self.hidden, self.hidden, stream)
        self._mark_end("o_proj", ev, rc)
        _hip.check("cascade_gemv_residual_bf16", rc)

    def instrument(self, name, launches, stride=1, offset=0):
        """Time ``launches`` launches of kernel group ``name`` ("gate_up",
        "qkv", "attention", "o_proj", "down_proj", "lm_head"; at prefill
        "gemm_qkv", "gemm_o", "gemm_gate_up", "gemm_gate", "gemm_up",
        "gemm_down", "gemm_lm_head", "topk", "prefill_attention"): of the group's
        coming launches, numbers offset, offset + stride, ...; read them back
        with :meth:`kernel_times_ms` after a synchronize.  The one-kernel
        groups (gate_up, qkv, o_proj, down_proj) bind the events to the
        kernel's own execution; attention, lm_head (GEMV + two top-k
        kernels) and topk (two kernels) are bracketed by events recorded on the
        launching stream, which include dispatch time.  A timed launch costs
        a few microseconds of extra queue time (the timestamp packets), so a
        stride spreads a few samples over a long run."""

        if int(stride) < 1 or int(offset) < 0:
            raise ValueError("stride must be >= 1 and offset >= 0")
        self._instrumented[name] = [
            (_hip.HipEvent(enable_timing=True), _hip.HipEvent(enable_timing=True))
            for _ in range(int(launches))
        ]
        self._instrument_next[name] = [0, 0, int(stride), int(offset)]

    def kernel_times_ms(self, name):
        pairs = self._instrumented.get(name, [])
        used = self._instrument_next[name][0] if pairs else 0
        return [a.elapsed_time(b) for a, b in pairs[:used]]

    def _events(self, name):
        pairs = self._instrumented.get(name)
        if not pairs:
            return None
        state = self._instrument_next[name]  # [timed, seen, stride, offset]
        index, seen, stride, offset = state
        state[1] = seen + 1
        if index >= len(pairs) or seen < offset or (seen - offset) % stride:
            return None
        state[0] = index + 1
        return pairs[index]

    def _mark_begin(self, name):
        ev = self._events(name)
        if ev is not None:
            if name in _KERNEL_TIMED_GROUPS:
                _hip.time_next_launch(ev[0], ev[1])
            else:
                ev[0].record()
        return ev

    def _mark_end(self, name, ev, rc):
        if ev is None:
            return
        if name not in _KERNEL_TIMED_GROUPS:
            ev[1].record()
        elif rc != 0:
            _hip.time_next_launch(None, None)

    def _gate_up(self, layer, ptrs, state, stream):
        x = state.hidden_states.data_ptr()
        row = 2 * self.hidden
        inter_row = 2 * self.intermediate
        norm = self._norm_ptrs[layer][1]
        wg, wu = ptrs["gate_proj"], ptrs["up_proj"]
        for t in range(len(state.positions)):
            ev = self._mark_begin("gate_up")
            rc = self._k_swiglu(wg, wu, self.intermediate, self.hidden, x + t * row,
                                norm, self.eps, self._inter_ptr + t * inter_row,
                                stream)
            self._mark_end("gate_up", ev, rc)
            _hip.check("cascade_gate_up_swiglu_bf16", rc)

    def _gate(self, layer, ptrs, state, stream):
        x = state.hidden_states.data_ptr()
        row, inter_row = 2 * self.hidden, 2 * self.intermediate
        norm = self._norm_ptrs[layer][1]
        for t in range(len(state.positions)):
            rc = self._k_silu(ptrs["gate_proj"], self.intermediate, self.hidden,
                              x + t * row, norm, self.eps,
                              self._gate_ptr + t * inter_row, stream)
            _hip.check("cascade_gate_silu_bf16", rc)

    def _up(self, layer, ptrs, state, stream):
        x = state.hidden_states.data_ptr()
        row, inter_row = 2 * self.hidden, 2 * self.intermediate
        norm = self._norm_ptrs[layer][1]
        for t in range(len(state.positions)):
            rc = self._k_mul(ptrs["up_proj"], self.intermediate, self.hidden,
                             x + t * row, norm, self.eps,
                             self._gate_ptr + t * inter_row,
                             self._inter_ptr + t * inter_row, stream)
            _hip.check("cascade_up_mul_bf16", rc)

    def _down(self, layer, ptrs, state, stream):
        x = state.hidden_states.data_ptr()
        row, inter_row = 2 * self.hidden, 2 * self.intermediate
        wd = ptrs["down_proj"]
        for t in range(len(state.positions)):
            ev = self._mark_begin("down_proj")
            xt = x + t * row
            rc = self._k_residual(wd, self._inter_ptr + t * inter_row, xt, xt,
                                  self.hidden, self.intermediate, stream)
            self._mark_end("down_proj", ev, rc)
            _hip.check("cascade_gemv_residual_bf16", rc)
        if self.capture is not None:
            self.capture.append((layer, state.hidden_states.detach().clone()))

    # ------------------------------------------- batched (S > 1) launches
    # One launch per matrix over all S token rows (MFMA GEMMs).  The
    # normalised rows are computed by the unit that opens a block (q_proj /
    # qkv / layer for the input norm, gate_proj / gate_up for the
    # post-attention norm) and reused by the matrices that follow it, as the
    # reference reuses layer_values["normalized"] (llama31.py:169-180,
    # :252-271).

    def _norm_rows(self, state, norm_ptr, stream):
        rc = self._k_rmsnorm(state.hidden_states.data_ptr(), norm_ptr,
                             self._normed_ptr, len(state.positions),
                             self.hidden, self.eps, stream)
        _hip.check("cascade_rmsnorm_bf16", rc)

    def _qkv_rows(self, layer, ptrs, state, stream):
        wq = ptrs.get("q_proj", 0)
        wk = ptrs.get("k_proj", 0)
        wv = ptrs.get("v_proj", 0)
        if wq:
            self._norm_rows(state, self._norm_ptrs[layer][0], stream)
        nkv = self.n_kv_heads * self.head_dim
        rope = self.rope
        ev = self._mark_begin("gemm_qkv")
        rc = self._k_qkv_gemm(
            self._normed_ptr, len(state.positions), wq, wk, wv,
            self.hidden if wq else 0, nkv if wk else 0, nkv if wv else 0,
            self.hidden, rope.cos.data_ptr(), rope.sin.data_ptr(),
            rope.capacity, state.positions[0], self._q_ptr if wq else 0,
            self._kv_pointer(layer, 0, 0) if wk else 0,
            self._kv_pointer(layer, 1, 0) if wv else 0,
            self.kv_cache.head_stride, self._first_slot, stream)
        self._mark_end("gemm_qkv", ev, rc)
        _hip.check("cascade_qkv_rope_gemm_bf16", rc)

    def _attention_o_rows(self, layer, ptrs, state, stream):
        tokens = len(state.positions)
        ev = self._mark_begin("prefill_attention")
        rc = self._k_prefill_attn(
            self._q_ptr, self._kv_pointer(layer, 0, 0),
            self._kv_pointer(layer, 1, 0), self.kv_cache.head_stride,
            self._first_slot, tokens, self.n_heads, self.n_kv_heads,
            self.head_dim, self.scale, self._attn_ptr, stream)
        self._mark_end("prefill_attention", ev, rc)
        _hip.check("cascade_prefill_attention_bf16", rc)
        x = state.hidden_states.data_ptr()
        ws, ws_bytes = self._gemm_workspace(tokens)
        ev = self._mark_begin("gemm_o")
        rc = self._k_gemm_residual_ws(self._attn_ptr, ptrs["o_proj"], x, x,
                                      tokens, self.hidden, self.hidden, ws,
                                      ws_bytes, stream)
        self._mark_end("gemm_o", ev, rc)
        _hip.check("cascade_gemm_residual_ws_bf16", rc)
        self.kv_cache.set_length(layer, self._first_slot + tokens)

    def _gate_up_rows(self, layer, ptrs, state, stream):
        tokens = len(state.positions)
        wg, wu = ptrs.get("gate_proj", 0), ptrs.get("up_proj", 0)
        if wg:
            self._norm_rows(state, self._norm_ptrs[layer][1], stream)
        if wg and wu:
            ev = self._mark_begin("gemm_gate_up")
            rc = self._k_swiglu_gemm(self._normed_ptr, wg, wu, self._inter_ptr,
                                     tokens, self.intermediate, self.hidden,
                                     stream)
            self._mark_end("gemm_gate_up", ev, rc)
            _hip.check("cascade_gate_up_swiglu_gemm_bf16", rc)
        elif wg:
            ev = self._mark_begin("gemm_gate")
            rc = self._k_silu_gemm(self._normed_ptr, wg, self._gate_ptr, tokens,
                                   self.intermediate, self.hidden, stream)
            self._mark_end("gemm_gate", ev, rc)
            _hip.check("cascade_gate_silu_gemm_bf16", rc)
        else:
            ev = self._mark_begin("gemm_up")
            rc = self._k_mul_gemm(self._normed_ptr, wu, self._gate_ptr,
                                  self._inter_ptr, tokens, self.intermediate,
                                  self.hidden, stream)
            self._mark_end("gemm_up", ev, rc)
            _hip.check("cascade_up_mul_gemm_bf16", rc)

    def _down_rows(self, layer, ptrs, state, stream):
        x = state.hidden_states.data_ptr()
        tokens = len(state.positions)
        ws, ws_bytes = self._gemm_workspace(tokens)
        ev = self._mark_begin("gemm_down")
        rc = self._k_gemm_residual_ws(self._inter_ptr, ptrs["down_proj"], x, x,
                                      tokens, self.hidden, self.intermediate, ws,
                                      ws_bytes, stream)
        self._mark_end("gemm_down", ev, rc)
        _hip.check("cascade_gemm_residual_ws_bf16", rc)
        if self.capture is not None:
            self.capture.append((layer, state.hidden_states.detach().clone()))

    def _call_batched(self, layer, op, ptrs, state, stream):
        if op == "layer":
            self._qkv_rows(layer, ptrs, state, stream)
            self._attention_o_rows(layer, ptrs, state, stream)
            self._gate_up_rows(layer, ptrs, state, stream)
            self._down_rows(layer, ptrs, state, stream)
        elif op in ("qkv", "q_proj", "k_proj", "v_proj"):
            self._qkv_rows(layer, ptrs, state, stream)
        elif op == "o_proj":
            self._attention_o_rows(layer, ptrs, state, stream)
        elif op in ("gate_up", "gate_proj", "up_proj"):
            self._gate_up_rows(layer, ptrs, state, stream)
        elif op == "down_proj":
            self._down_rows(layer, ptrs, state, stream)
        else:
            raise ValueError("unknown Llama operation {}".format(op))
        return state

    def __call__(self, unit, weights, state):
        layer = unit.layer_index
        op = unit.operation
        ptrs = self._unit_pointers(unit, weights)
        stream = self._stream()
        if layer == 0 and op in ("qkv", "q_proj", "layer"):
            # slot of the first token of this call, fixed for all layers
            self._first_slot = self.kv_cache.sequence_length()
            positions = state.positions
            self._batched = len(positions) > 1 and positions == tuple(
                range(positions[0], positions[0] + len(positions)))
        if self._batched:
            return self._call_batched(layer, op, ptrs, state, stream)
        if op == "layer":
            self._qkv(layer, ptrs, state, stream)
            self._attention_o(layer, ptrs, state, stream)
            self._gate_up(layer, ptrs, state, stream)
            self._down(layer, ptrs, state, stream)
        elif op in ("qkv", "q_proj", "k_proj", "v_proj"):
            self._qkv(layer, ptrs, state, stream)
        elif op == "o_proj":
            self._attention_o(layer, ptrs, state, stream)
        elif op == "gate_up":
            self._gate_up(layer, ptrs, state, stream)
        elif op == "gate_proj":
            self._gate(layer, ptrs, state, stream)
        elif op == "up_proj":
            self._up(layer, ptrs, state, stream)
        elif op == "down_proj":
            self._down(layer, ptrs, state, stream)
        else:
            raise ValueError("unknown Llama operation {}".format(op))
        return state

    def finish(self, state):
        rows = self._token_rows(state)
        count = rows.shape[0]
        stream = self._stream()
        final_norm = self.resident["model.norm.weight"]
        if self.vocab_runtime is not None:
            # the flag carries only the fused attention's bits here (the
            # streamed embedding checks ids on the host)
            self._id_errors.raise_if_set()
            last = self._normed[:1]
            _hip.rmsnorm(rows[count - 1 :], final_norm, last, self.eps)
            result = self.vocab_runtime.lm_head_topk(
                last.view(1, 1, self.hidden),
                top_k=self.top_k,
                return_full_logits=self.return_full_logits,
            )
            state.topk_values = result["values"]
            state.topk_indices = result["indices"]
            state.logits = result["logits"]
            self._id_errors.publish()
            return state
        step = self._device_step
        if step is None:
            self._id_errors.raise_if_set()
        normed = self._normed[:count]
        _hip.check("cascade_rmsnorm_bf16", self._k_rmsnorm(
            rows.data_ptr(), final_norm.data_ptr(), normed.data_ptr(), count,
            self.hidden, self.eps, stream))
        if self._head_ws is None:
            head = self.resident["lm_head.weight"]
            vocab, _ = _hip.bf16_weight(head, "lm_head.weight", k=self.hidden)
            size = _hip.lm_head_workspace_bytes(vocab, self.top_k)
            self._head_ws = torch.zeros(size, dtype=torch.uint8, device=self.device)
            self._head = (head.data_ptr(), vocab)
        head_ptr, vocab = self._head
        step = self._device_step
        if step is not None and count == 1:
            # fixed buffers: the next step's input is indices[0, 0, 0]
            logits, values, indices = step.logits, step.values, step.indices
        else:
            logits = torch.empty((1, count, vocab), dtype=torch.float32,
                                 device=self.device)
            values = torch.empty((1, 1, self.top_k), dtype=torch.float32,
                                 device=self.device)
            indices = torch.empty((1, 1, self.top_k), dtype=torch.int64,
                                  device=self.device)
        ws, ws_bytes = self._head_ws.data_ptr(), self._head_ws.numel()
        if count > 1:
            # every position's logits in one GEMM (the reference's F.linear
            # over [1, S, H]), then the top-k of the last row's logits
            # (torch.topk(state.logits[:, -1:, :]), llama31.py:335-339)
            ev = self._mark_begin("gemm_lm_head")
            rc = self._k_f32_gemm(normed.data_ptr(), head_ptr, logits.data_ptr(),
                                  count, vocab, self.hidden, stream)
            self._mark_end("gemm_lm_head", ev, rc)
            _hip.check("cascade_gemm_f32out_bf16", rc)
            ev = self._mark_begin("topk")
            rc = self._k_topk(logits.data_ptr() + 4 * vocab * (count - 1), vocab,
                              self.top_k, ws, ws_bytes, values.data_ptr(),
                              indices.data_ptr(), stream)
            self._mark_end("topk", ev, rc)
            _hip.check("cascade_topk_f32", rc)
        else:
            # one position: its logits and their top-k in one call
            ev = self._mark_begin("lm_head")
            rc = self._k_head(head_ptr, vocab, self.hidden, 0, normed.data_ptr(),
                              self.top_k, 1, logits.data_ptr(), ws, ws_bytes,
                              values.data_ptr(), indices.data_ptr(), stream)
            self._mark_end("lm_head", ev, rc)
            _hip.check("cascade_lm_head_topk_bf16", rc)
        state.logits = logits
        state.topk_values = values
        state.topk_indices = indices
        if step is None:
            self._id_errors.publish()
        return state

    def check_errors(self):
        """Wait for the last step's error flags and raise if one is set
        (begin() / finish() check them without waiting, one step late)."""

        self._id_errors.raise_if_set(block=True)
