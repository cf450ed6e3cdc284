"""CPU oracle for the batch=1 Llama-3.1-8B decode path.

TEST INFRASTRUCTURE.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only as the checker (or, for
the baseline, as the timed CPU restatement).  The product path
(layer_streaming) never imports it.

It restates the reference's math with torch CPU ops, op for op and with the
same bf16 rounding points (reference = lianghan224-cloud/Cascade-LLM;
TF = transformers, the library the reference calls for RoPE):

  rms_norm            layer_streaming/llama31.py:21-25
  linear              F.linear on bf16 tensors (fp32 accumulate, bf16 out),
                      llama31.py:241-279, vocab.py:247
  llama3_inv_freq     TF modeling_rope_utils.py:580-661
  rope_cos_sin        TF models/llama/modeling_llama.py:111-127
  apply_rope          TF models/llama/modeling_llama.py:130-160,
                      called at llama31.py:206-212
  attention           _repeat_kv + F.scaled_dot_product_attention,
                      llama31.py:28-31,213-234 (fp32 scores, softmax
                      numerator rounded to bf16 as bf16 SDPA does, bf16
                      output)
  decoder_layer       llama31.py:169-283 (one whole layer, all S tokens)
  lm_head_logits      llama31.py:330-334, vocab.py:247 (fp32 logits; the
                      reference's bf16 rounding is optional)
  topk / merge_topk   vocab.py:11-32,248-261 with the canonical tie order
                      (value descending, index ascending)
  streamed_lm_head    vocab.py:207-266 (chunked logits + online merge)
  OracleLlama         Llama31DecodeExecutor begin / units / finish,
                      llama31.py:128-154,285-349, and the reference's CPU
                      reference path (benchmarks/real_llama31_correctness.py:
                      87-129: greedy argmax, lowest index on ties)

How each function is pinned (tests/test_oracle.py): golden vectors from the
reference's own tests (merge_topk known answer), golden RoPE / decoder /
model fixtures written from transformers (tests/golden/), library routines
(torch F.rms_norm, F.scaled_dot_product_attention, numpy float64 matmul),
closed forms (RoPE at position 0, attention over one position, constant
vectors) and brute force (full stable sorts for top-k).
"""

import math

import numpy as np
import torch
import torch.nn.functional as F

BF16 = torch.bfloat16

LLAMA31_ROPE = {
    "rope_type": "llama3",
    "rope_theta": 500000.0,
    "factor": 8.0,
    "low_freq_factor": 1.0,
    "high_freq_factor": 4.0,
    "original_max_position_embeddings": 8192,
}


# ----------------------------------------------------------------- layers


def rms_norm(hidden, weight, eps):
    """llama31.py:21-25: w * bf16(x32 * rsqrt(mean(x32^2) + eps))."""

    dtype = hidden.dtype
    variance = hidden.float().pow(2).mean(-1, keepdim=True)
    normalized = hidden.float() * torch.rsqrt(variance + eps)
    return weight * normalized.to(dtype)


def linear(x, weight):
    """F.linear on bf16 operands: fp32 accumulation, bf16 result."""

    return F.linear(x, weight)


def linear_exact(x, weight):
    """float64 reference product of the same bf16 operands (pins linear)."""

    a = x.float().numpy().astype(np.float64)
    b = weight.float().numpy().astype(np.float64)
    return torch.from_numpy(a @ b.T)


def llama3_inv_freq(head_dim=128, params=None):
    """Inverse frequencies, TF modeling_rope_utils.py:580-661 (and the
    default RoPE of modeling_llama.py:93-109 when rope_type is default)."""

    params = dict(LLAMA31_ROPE if params is None else params)
    base = float(params["rope_theta"])
    inv_freq = 1.0 / (
        base ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim)
    )
    if params.get("rope_type", "default") == "default":
        return inv_freq
    factor = float(params["factor"])
    low = float(params["low_freq_factor"])
    high = float(params["high_freq_factor"])
    old_context = float(params["original_max_position_embeddings"])
    low_wavelen = old_context / low
    high_wavelen = old_context / high
    wavelen = 2 * math.pi / inv_freq
    out = torch.where(wavelen > low_wavelen, inv_freq / factor, inv_freq)
    smooth = (old_context / wavelen - low) / (high - low)
    smoothed = (1 - smooth) * out / factor + smooth * out
    medium = ~(wavelen < high_wavelen) * ~(wavelen > low_wavelen)
    return torch.where(medium, smoothed, out)


def rope_cos_sin(inv_freq, positions, dtype=BF16):
    """cos / sin [S, head_dim], TF modeling_llama.py:111-127."""

    pos = torch.as_tensor(positions, dtype=torch.long).reshape(1, -1)
    inv = inv_freq[None, :, None].float()
    freqs = (inv @ pos[:, None, :].float()).transpose(1, 2)[0]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def rotate_half(x):
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rope(x, cos, sin):
    """x [heads, S, D]; cos / sin [S, D]: x*cos + rotate_half(x)*sin with
    the operands' dtype (bf16 in the model)."""

    return (x * cos[None]) + (rotate_half(x) * sin[None])


def attention(q, k, v, past, round_numerator=True):
    """q [H, S, D]; k / v [Hkv, past + S, D] (all bf16).  Query token t sees
    positions <= past + t (no mask at decode, causal at prefill, as
    llama31.py:221-229).  fp32 scores; output [S, H*D] in q's dtype.

    The softmax numerator p = exp(s - rowmax) is rounded to q's dtype
    before the product with V, and the denominator sums the unrounded p:
    the rounding point of F.scaled_dot_product_attention on bf16 operands
    (llama31.py:223-229; the reference's CPU path reaches it through
    transformers' sdpa attention, benchmarks/real_llama31_correctness.py:
    87-129).  Bit-exact against bf16 SDPA on the CPU for a prompt whose keys
    fit one block of that kernel (tests/golden/tiny_llama_bf16.json); no-op
    for fp32 operands.  ``round_numerator=False`` keeps p in fp32 (fp32
    SDPA)."""

    heads, seq, dim = q.shape
    groups = heads // k.shape[0]
    kf = k.float().repeat_interleave(groups, dim=0)
    vf = v.float().repeat_interleave(groups, dim=0)
    scores = (q.float() @ kf.transpose(1, 2)) / math.sqrt(dim)
    length = k.shape[1]
    allowed = torch.arange(length)[None, :] <= (past + torch.arange(seq))[:, None]
    scores = scores.masked_fill(~allowed[None], float("-inf"))
    numerator = torch.exp(scores - scores.amax(dim=-1, keepdim=True))
    denominator = numerator.sum(dim=-1, keepdim=True)
    if round_numerator:
        numerator = numerator.to(q.dtype).float()
    out = (numerator @ vf) / denominator
    return out.transpose(0, 1).reshape(seq, heads * dim).to(q.dtype)


def decoder_layer(hidden, w, cache, past, cos, sin, eps, n_heads=32,
                  n_kv_heads=8, linear_fn=None, attention_fn=None, trace=None):
    """One decoder layer for S tokens, llama31.py:169-283.

    hidden [S, H] bf16; w: dict with q, k, v, o, gate, up, down, ln1, ln2;
    cache: dict with "k" / "v" tensors [Hkv, past, D] (or None), updated in
    place.  Returns the new hidden [S, H].  ``linear_fn`` / ``attention_fn``
    replace the GEMV / attention restatements (default: ``linear``,
    ``attention``).  A ``trace`` dict receives the intermediates: attn,
    o (o_proj output), h_attn (after the first residual add), inter
    (silu(gate) * up) and down (down_proj output).
    """

    linear = globals()["linear"] if linear_fn is None else linear_fn
    attend = globals()["attention"] if attention_fn is None else attention_fn
    seq, width = hidden.shape
    dim = width // n_heads
    residual = hidden
    normalized = rms_norm(hidden, w["ln1"], eps)
    q = linear(normalized, w["q"]).view(seq, n_heads, dim).transpose(0, 1)
    k = linear(normalized, w["k"]).view(seq, n_kv_heads, dim).transpose(0, 1)
    v = linear(normalized, w["v"]).view(seq, n_kv_heads, dim).transpose(0, 1)
    q = apply_rope(q, cos, sin)
    k = apply_rope(k, cos, sin)
    if cache.get("k") is not None:
        k = torch.cat((cache["k"], k), dim=1)
        v = torch.cat((cache["v"], v), dim=1)
    cache["k"], cache["v"] = k, v
    attn = attend(q, k, v, past)
    o = linear(attn, w["o"])
    hidden = residual + o
    residual = hidden
    normalized = rms_norm(hidden, w["ln2"], eps)
    gate = F.silu(linear(normalized, w["gate"]))
    up = linear(normalized, w["up"])
    inter = gate * up
    down = linear(inter, w["down"])
    if trace is not None:
        trace.update(attn=attn, o=o, h_attn=hidden, inter=inter, down=down)
    return residual + down


# --------------------------------------------------------------- LM head


def lm_head_logits(hidden, weight, round_to_bf16=False, chunk_rows=16384):
    """fp32 logits of one hidden vector [H] against weight [V, H]."""

    h = hidden.reshape(1, -1).float()
    parts = []
    for start in range(0, weight.shape[0], chunk_rows):
        part = h @ weight[start : start + chunk_rows].float().t()
        parts.append(part.to(BF16).float() if round_to_bf16 else part)
    return torch.cat(parts, dim=-1).reshape(-1)


def topk(values, k):
    """Exact top-k, value descending then index ascending (a stable sort)."""

    order = torch.sort(values, descending=True, stable=True).indices[:k]
    return values[order], order


def merge_topk(current_values, current_indices, candidate_values,
               candidate_indices, top_k):
    """vocab.py:11-32 with a deterministic tie order."""

    if current_values is None:
        values, indices = candidate_values, candidate_indices
    else:
        values = torch.cat((current_values, candidate_values))
        indices = torch.cat((current_indices, candidate_indices))
    keep = min(int(top_k), values.numel())
    by_index = torch.argsort(indices, stable=True)
    values, indices = values[by_index], indices[by_index]
    order = torch.argsort(values, descending=True, stable=True)[:keep]
    return values[order], indices[order]


def streamed_lm_head(hidden, weight, chunk_rows, top_k):
    """Chunked logits + local top-k + online merge, vocab.py:207-266."""

    values = indices = None
    logits = []
    for start in range(0, weight.shape[0], chunk_rows):
        part = lm_head_logits(hidden, weight[start : start + chunk_rows])
        logits.append(part)
        lv, li = topk(part, min(top_k, part.numel()))
        values, indices = merge_topk(values, indices, lv, li + start, top_k)
    return values, indices, torch.cat(logits)


# ----------------------------------------------------------------- model


def layer_weights(tensor, layer):
    """Gather one layer's tensors through ``tensor(key)`` (store.tensor)."""

    p = "model.layers.{}.".format(layer)
    return {
        "q": tensor(p + "self_attn.q_proj.weight"),
        "k": tensor(p + "self_attn.k_proj.weight"),
        "v": tensor(p + "self_attn.v_proj.weight"),
        "o": tensor(p + "self_attn.o_proj.weight"),
        "gate": tensor(p + "mlp.gate_proj.weight"),
        "up": tensor(p + "mlp.up_proj.weight"),
        "down": tensor(p + "mlp.down_proj.weight"),
        "ln1": tensor(p + "input_layernorm.weight"),
        "ln2": tensor(p + "post_attention_layernorm.weight"),
    }


class OracleLlama:
    """Greedy batch=1 decoding of a Llama-3.1-8B-shaped model on the CPU.

    ``tensor(key)`` returns the bf16 CPU tensor of a checkpoint key (e.g. a
    weight store's ``tensor``); ``linear_fn`` / ``attention_fn`` replace the
    GEMV / attention restatements in every layer (default ``linear``,
    ``attention``).  Mirrors Llama31DecodeExecutor: begin
    (embedding row gather), the layers, finish (final norm, fp32 logits of
    the last position, top-k).
    """

    def __init__(self, tensor, num_layers=32, eps=1e-5, rope=None,
                 n_heads=32, n_kv_heads=8, head_dim=128, linear_fn=None,
                 attention_fn=None):
        self.tensor = tensor
        self.linear_fn = linear_fn
        self.attention_fn = attention_fn
        self.num_layers = int(num_layers)
        self.eps = float(eps)
        self.n_heads = n_heads
        self.n_kv_heads = n_kv_heads
        self.inv_freq = llama3_inv_freq(head_dim, rope)
        # cos / sin take the activations' dtype (bf16 for the 8B model; fp32
        # when the oracle runs a fp32 model against a fp32 golden)
        self.dtype = tensor("model.embed_tokens.weight").dtype
        self.caches = [dict() for _ in range(self.num_layers)]
        self.length = 0

    def step(self, ids, top_k=10, round_logits=False):
        """Run S = len(ids) tokens; returns (fp32 logits of the last token,
        top-k values, top-k indices)."""

        ids = torch.as_tensor(ids, dtype=torch.long).reshape(-1)
        past = self.length
        positions = list(range(past, past + ids.numel()))
        cos, sin = rope_cos_sin(self.inv_freq, positions, self.dtype)
        hidden = self.tensor("model.embed_tokens.weight")[ids]
        for layer in range(self.num_layers):
            hidden = decoder_layer(
                hidden, layer_weights(self.tensor, layer), self.caches[layer],
                past, cos, sin, self.eps, self.n_heads, self.n_kv_heads,
                linear_fn=self.linear_fn, attention_fn=self.attention_fn,
            )
        self.length = past + ids.numel()
        normalized = rms_norm(hidden[-1:], self.tensor("model.norm.weight"), self.eps)
        logits = lm_head_logits(normalized[0], self.tensor("lm_head.weight"),
                                round_to_bf16=round_logits)
        values, indices = topk(logits, top_k)
        return logits, values, indices

    def generate(self, prompt_ids, new_tokens, top_k=10):
        """Greedy tokens plus the per-step logits / top-k."""

        steps = []
        logits, values, indices = self.step(prompt_ids, top_k)
        steps.append((logits, values, indices))
        tokens = [int(indices[0])]
        for _ in range(new_tokens - 1):
            logits, values, indices = self.step([tokens[-1]], top_k)
            steps.append((logits, values, indices))
            tokens.append(int(indices[0]))
        return tokens, steps
