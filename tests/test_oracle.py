"""Pins of the CPU oracle (oracle/llama_oracle.py).

Each oracle function is checked against something that fixes it
independently -- golden fixtures written from transformers
(tests/golden/make_golden.py), library routines (torch F.rms_norm,
F.scaled_dot_product_attention, numpy float64 matmul), closed forms and
brute force -- and the planted-mistake tests show the pins fail for the
plausible errors (sign of rotate_half, GQA head map, gate/up swap, eps
placement, missing residual).
"""

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import cases
from oracle import llama_oracle as ref

GOLDEN = Path(__file__).resolve().parent / "golden"
BF16 = torch.bfloat16


def from_bits(bits, shape):
    arr = torch.tensor(bits, dtype=torch.int32).to(torch.int16)
    return arr.view(BF16).reshape(shape)


# ---------------------------------------------------------------- RMSNorm


def test_rms_norm_matches_library_rms_norm():
    x = torch.randn(3, 4096, generator=torch.Generator().manual_seed(1))
    ours = ref.rms_norm(x, torch.ones(4096), 1e-5)
    lib = F.rms_norm(x, (4096,), eps=1e-5)
    assert torch.allclose(ours, lib, atol=1e-6, rtol=1e-6)


def test_rms_norm_closed_form_constant_vector():
    # x = c everywhere: mean(x^2) = c^2 -> x / sqrt(c^2 + eps)
    for c in (0.5, 3.0, -2.0):
        x = torch.full((4096,), c)
        out = ref.rms_norm(x, torch.ones(4096), 1e-5)
        assert torch.allclose(out, torch.full((4096,), c / math.sqrt(c * c + 1e-5)))


def test_rms_norm_rounds_before_the_weight_multiply():
    # bf16 path: w * bf16(x * r) -- differs from bf16(w * x * r) in general
    x = cases.normal_bf16((4096,), 5)
    w = cases.normal_bf16((4096,), 6, 0.1, 1.0)
    r = torch.rsqrt(x.float().pow(2).mean() + 1e-5)
    expected = w * (x.float() * r).to(BF16)
    assert torch.equal(ref.rms_norm(x, w, 1e-5), expected)


# ----------------------------------------------------------------- linear


def test_linear_is_fp32_accumulated_bf16():
    w = cases.normal_bf16((512, 4096), 7, 0.02)
    x = cases.normal_bf16((1, 4096), 8)
    out = ref.linear(x, w).float()
    exact = ref.linear_exact(x, w).float()
    # within one bf16 ulp of the float64 product (bf16 accumulation would
    # be off by many ulps at K = 4096)
    ulp = torch.exp2(torch.floor(torch.log2(exact.abs().clamp_min(1e-30))) - 7)
    assert bool(((out - exact).abs() <= ulp).all())


# ------------------------------------------------------------------- RoPE


@pytest.fixture(scope="module")
def rope_golden():
    return json.loads((GOLDEN / "rope_llama3.json").read_text())


def test_llama3_inverse_frequencies_match_golden(rope_golden):
    inv = ref.llama3_inv_freq(128, rope_golden["rope"])
    assert torch.equal(inv, torch.tensor(rope_golden["inv_freq"], dtype=torch.float32))


def test_cos_sin_match_golden(rope_golden):
    inv = ref.llama3_inv_freq(128, rope_golden["rope"])
    cos, sin = ref.rope_cos_sin(inv, rope_golden["positions"])
    n = len(rope_golden["positions"])
    assert torch.equal(cos, from_bits(rope_golden["cos_bf16_bits"], (n, 128)))
    assert torch.equal(sin, from_bits(rope_golden["sin_bf16_bits"], (n, 128)))


def test_apply_rope_matches_golden(rope_golden):
    inv = ref.llama3_inv_freq(128, rope_golden["rope"])
    cos, sin = ref.rope_cos_sin(inv, [rope_golden["apply_position"]])
    q = from_bits(rope_golden["q_bf16_bits"], (4, 1, 128))
    k = from_bits(rope_golden["k_bf16_bits"], (2, 1, 128))
    assert torch.equal(ref.apply_rope(q, cos, sin),
                       from_bits(rope_golden["q_out_bf16_bits"], (4, 1, 128)))
    assert torch.equal(ref.apply_rope(k, cos, sin),
                       from_bits(rope_golden["k_out_bf16_bits"], (2, 1, 128)))


def test_rope_closed_forms():
    # textbook default RoPE: 1 / theta^(2i/d)
    inv = ref.llama3_inv_freq(128, {"rope_type": "default", "rope_theta": 10000.0})
    i = torch.arange(64, dtype=torch.float64)
    assert torch.allclose(inv.double(), 1.0 / 10000.0 ** (2 * i / 128), rtol=1e-6)
    # llama3: high-frequency band untouched, low-frequency band / 8
    base = ref.llama3_inv_freq(128, dict(ref.LLAMA31_ROPE, rope_type="default"))
    scaled = ref.llama3_inv_freq(128)
    wavelen = 2 * math.pi / base
    assert torch.equal(scaled[wavelen < 2048], base[wavelen < 2048])
    assert torch.allclose(scaled[wavelen > 8192], base[wavelen > 8192] / 8)
    # position 0 is the identity; rotation keeps pair norms (fp32)
    cos, sin = ref.rope_cos_sin(scaled, [0])
    x = cases.normal_bf16((2, 1, 128), 9)
    assert torch.equal(ref.apply_rope(x, cos, sin), x)
    cos, sin = ref.rope_cos_sin(scaled, [1234], torch.float32)
    y = torch.randn(1, 1, 128)
    r = ref.apply_rope(y, cos, sin)
    pair = lambda t: t[..., :64] ** 2 + t[..., 64:] ** 2  # noqa: E731
    assert torch.allclose(pair(r), pair(y), atol=1e-5)


# -------------------------------------------------------------- attention


@pytest.mark.parametrize("length", [1, 5, 300])
def test_attention_matches_library_sdpa(length):
    q = cases.normal_bf16((32, 1, 128), 10)
    k = cases.normal_bf16((8, length, 128), 11)
    v = cases.normal_bf16((8, length, 128), 12)
    ours = ref.attention(q, k, v, length - 1)
    lib = cases.softmax_attention_reference(q, k, v).to(BF16)
    assert torch.equal(ours, lib) or torch.allclose(ours.float(), lib.float(), atol=8e-3)


def test_attention_single_position_returns_value():
    q = cases.normal_bf16((32, 1, 128), 13)
    v = cases.normal_bf16((8, 1, 128), 14)
    out = ref.attention(q, cases.normal_bf16((8, 1, 128), 15), v, 0)
    assert torch.equal(out.reshape(32, 128), v[:, 0].repeat_interleave(4, 0))


def test_attention_prefill_is_causal():
    # row t of a prefill equals a decode over the first t + 1 positions
    q = cases.normal_bf16((4, 6, 16), 16)
    k = cases.normal_bf16((2, 6, 16), 17)
    v = cases.normal_bf16((2, 6, 16), 18)
    full = ref.attention(q, k, v, 0)
    for t in range(6):
        step = ref.attention(q[:, t : t + 1], k[:, : t + 1], v[:, : t + 1], t)
        assert torch.equal(full[t], step[0])


# ------------------------------------------------------ whole-model golden


@pytest.fixture(scope="module")
def tiny():
    data = np.load(GOLDEN / "tiny_llama.npz")
    return {k: data[k] for k in data.files}


def tiny_oracle(tiny):
    def tensor(key):
        return torch.from_numpy(tiny[key])

    return ref.OracleLlama(tensor, num_layers=2, eps=1e-5, n_heads=4,
                           n_kv_heads=2, head_dim=16)


def test_oracle_model_matches_transformers_golden(tiny):
    tokens, steps = tiny_oracle(tiny).generate(tiny["__prompt"].tolist(), 4)
    assert tokens == tiny["__tokens"].tolist()
    for (logits, _, _), gold in zip(steps, tiny["__logits"]):
        assert torch.allclose(logits, torch.from_numpy(gold), atol=2e-4, rtol=1e-4)


def _mutated_logits(tiny, monkeypatch, target, replacement):
    with monkeypatch.context() as m:
        m.setattr(ref, target, replacement)
        _, steps = tiny_oracle(tiny).generate(tiny["__prompt"].tolist(), 2)
    return steps[0][0]


@pytest.mark.parametrize("mistake", ["rotate_sign", "gqa_map", "eps_outside",
                                     "gate_up_swap", "no_causal_mask"])
def test_planted_mistakes_fail_the_golden(tiny, monkeypatch, mistake):
    gold = torch.from_numpy(tiny["__logits"][0])
    original = {name: getattr(ref, name) for name in
                ("rotate_half", "attention", "rms_norm", "linear")}
    if mistake == "rotate_sign":
        repl = ("rotate_half", lambda x: -original["rotate_half"](x))
    elif mistake == "gqa_map":
        # wrong head map: repeat instead of repeat_interleave
        repl = ("attention", _bad_gqa)
    elif mistake == "eps_outside":
        def rms_norm(h, w, eps):
            var = h.float().pow(2).mean(-1, keepdim=True)
            return w * (h.float() * torch.rsqrt(var) + eps).to(h.dtype)
        repl = ("rms_norm", rms_norm)
    elif mistake == "gate_up_swap":
        swapped = {}

        def linear(x, w):
            return original["linear"](x, w)
        repl = ("linear", linear)
        # swap the two MLP input matrices in the weights the oracle reads
        for layer in range(2):
            p = "model.layers.{}.mlp.".format(layer)
            swapped[p + "gate_proj.weight"] = tiny[p + "up_proj.weight"]
            swapped[p + "up_proj.weight"] = tiny[p + "gate_proj.weight"]
        tiny = dict(tiny, **swapped)
    else:
        def attention(q, k, v, past):
            return original["attention"](q, k, v, past + k.shape[1])
        repl = ("attention", attention)
    logits = _mutated_logits(tiny, monkeypatch, *repl)
    assert not torch.allclose(logits, gold, atol=2e-4, rtol=1e-4)


def _bad_gqa(q, k, v, past):
    heads = q.shape[0]
    groups = heads // k.shape[0]
    kk = k.repeat(groups, 1, 1)  # head h -> kv h % n_kv (wrong)
    vv = v.repeat(groups, 1, 1)
    qf, kf, vf = q.float(), kk.float(), vv.float()
    scores = (qf @ kf.transpose(1, 2)) / math.sqrt(q.shape[-1])
    seq, length = q.shape[1], k.shape[1]
    allowed = torch.arange(length)[None, :] <= (past + torch.arange(seq))[:, None]
    scores = scores.masked_fill(~allowed[None], float("-inf"))
    out = torch.softmax(scores, -1) @ vf
    return out.transpose(0, 1).reshape(seq, -1).to(q.dtype)


# ------------------------------------------------- bf16 layer composition


def test_layer_steps_equal_composed_layer():
    case = cases.layer_case(5, 40, hidden=256, intermediate=512, n_heads=4,
                            n_kv_heads=1, head_dim=64)
    steps = cases.layer_expected(case)["out"]
    composed = cases.layer_expected_composed(case)
    assert torch.equal(steps, composed)
