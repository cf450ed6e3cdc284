"""Rotary position tables for the fused QKV kernel.

The reference takes cos/sin from transformers' LlamaRotaryEmbedding
(layer_streaming/llama31.py:84-87,125,206-212; transformers
models/llama/modeling_llama.py:73-127 and modeling_rope_utils.py:580-661):

  inv_freq[i] = 1 / theta^(2i / d)                       (fp32, i < d/2)
  llama3 scaling (rope_type "llama3"):
    wavelen = 2 pi / inv_freq
    wavelen > orig/low   -> inv_freq / factor
    wavelen < orig/high  -> inv_freq
    otherwise            -> (1 - s) inv_freq / factor + s inv_freq,
                            s = (orig / wavelen - low) / (high - low)
  freqs = inv_freq * position (fp32), emb = cat(freqs, freqs)
  cos = bf16(cos(emb)), sin = bf16(sin(emb))   (attention_scaling = 1)

The table is built once per capacity on the host in fp32 with exactly these
steps and kept in HBM as bf16 [capacity, d/2] (the two halves of emb are
equal, so half the table suffices).  It is a constant of the model, like the
reference's inv_freq buffer; the rotation itself runs in the QKV kernel.
"""

import math

import torch

__all__ = ["rope_parameters", "inverse_frequencies", "RopeTable"]

_LLAMA31_ROPE = {
    "rope_type": "llama3",
    "rope_theta": 500000.0,
    "factor": 8.0,
    "low_freq_factor": 1.0,
    "high_freq_factor": 4.0,
    "original_max_position_embeddings": 8192,
}


def rope_parameters(config):
    """RoPE settings of a Llama config (transformers 4.x or 5.x layout)."""

    params = getattr(config, "rope_parameters", None)
    if isinstance(params, dict) and "rope_theta" in params:
        out = dict(params)
    else:
        scaling = getattr(config, "rope_scaling", None) or {}
        out = dict(scaling)
        out["rope_theta"] = float(getattr(config, "rope_theta", 500000.0))
    out.setdefault("rope_type", out.get("type", "default"))
    return out


def inverse_frequencies(head_dim, params):
    """fp32 inverse frequencies, llama3-scaled when rope_type is llama3."""

    base = float(params["rope_theta"])
    exponent = torch.arange(0, head_dim, 2, dtype=torch.int64).to(torch.float32)
    inv_freq = 1.0 / (base ** (exponent / head_dim))
    rope_type = params.get("rope_type", "default")
    if rope_type == "default":
        return inv_freq
    if rope_type != "llama3":
        raise ValueError("unsupported rope_type {}".format(rope_type))
    factor = float(params["factor"])
    low = float(params["low_freq_factor"])
    high = float(params["high_freq_factor"])
    original = float(params["original_max_position_embeddings"])
    wavelen = 2 * math.pi / inv_freq
    scaled = torch.where(wavelen > original / low, inv_freq / factor, inv_freq)
    smooth = (original / wavelen - low) / (high - low)
    blended = (1 - smooth) * scaled / factor + smooth * scaled
    medium = ~(wavelen < original / high) * ~(wavelen > original / low)
    return torch.where(medium, blended, scaled)


def cos_sin_rows(inv_freq, start, end):
    """bf16 cos / sin rows [end - start, d/2] for positions start..end-1."""

    positions = torch.arange(start, end, dtype=torch.int64).to(torch.float32)
    freqs = positions[:, None] * inv_freq[None, :]
    return freqs.cos().to(torch.bfloat16), freqs.sin().to(torch.bfloat16)


class RopeTable:
    """Device-resident bf16 cos / sin rows, grown on demand."""

    def __init__(self, head_dim, params, device, capacity=4096):
        self.head_dim = int(head_dim)
        self.inv_freq = inverse_frequencies(self.head_dim, params)
        self.device = torch.device(device)
        self.capacity = 0
        self.cos = None
        self.sin = None
        self.reserve(capacity)

    def reserve(self, positions):
        if positions <= self.capacity:
            return
        capacity = max(int(positions), 2 * self.capacity, 256)
        capacity = -(-capacity // 256) * 256
        cos, sin = cos_sin_rows(self.inv_freq, 0, capacity)
        self.cos = cos.to(self.device)
        self.sin = sin.to(self.device)
        self.capacity = capacity

    def row(self, position):
        """(cos, sin) views of one position (64 bf16 each)."""

        if position >= self.capacity:
            self.reserve(position + 1)
        return self.cos[position], self.sin[position]
