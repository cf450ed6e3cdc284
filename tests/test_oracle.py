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


@pytest.mark.parametrize("length,seq", [(2, 2), (6, 6), (64, 1), (300, 1),
                                        (2049, 1), (256, 256)])
def test_attention_within_one_ulp_of_bf16_sdpa(length, seq):
    # The numerator's bf16 rounding point is the library's (bf16
    # F.scaled_dot_product_attention, causal, GQA by repeat_interleave);
    # the library's vectorised exp moves some numerators across a bf16
    # rounding boundary, so outputs agree within one bf16 ulp of the largest
    # output, and dropping the rounding point lands further away.  (The
    # whole-model fixture's 6-token prompt is bit-exact.)
    q = cases.normal_bf16((32, seq, 128), 50 + length)
    k = cases.normal_bf16((8, length, 128), 51 + length)
    v = cases.normal_bf16((8, length, 128), 52 + length)
    lib = F.scaled_dot_product_attention(
        q[None], k.repeat_interleave(4, 0)[None], v.repeat_interleave(4, 0)[None],
        is_causal=seq > 1)[0].transpose(0, 1).reshape(seq, -1).float()
    ulp = cases.bf16_ulp(lib.abs().max())
    past = length - seq
    ours = ref.attention(q, k, v, past).float()
    assert float((ours - lib).abs().max()) <= ulp
    unrounded = ref.attention(q, k, v, past, round_numerator=False).float()
    assert float((ours - lib).abs().sum()) < float((unrounded - lib).abs().sum())


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


# ------------------------- the reference's CPU path in bf16 (transformers)


@pytest.fixture(scope="module")
def bf16_golden():
    data = json.loads((GOLDEN / "tiny_llama_bf16.json").read_text())
    weights = {}
    for index, (name, shape, checksum) in enumerate(zip(
            data["weight_names"], data["weight_shapes"], data["weight_checksums"])):
        # the fixture's recipe (tests/golden/make_golden.py bf16_weight)
        gen = torch.Generator().manual_seed(1000 + index)
        values = torch.randn(tuple(shape), generator=gen)
        values = 1.0 + 0.1 * values if len(shape) == 1 else 0.04 * values
        weights[name] = values.to(BF16)
        # the generator still draws what the fixture was written from
        assert float(weights[name].double().sum()) == checksum, name
    data["weights"] = weights
    return data


def _bf16_oracle_step(golden, caches, past, ids, composition=None):
    """One step of the oracle's decoder stack on the fixture's weights;
    returns the per-layer outputs, the final norm and the bf16 logits
    (F.linear, the reference's LM head).  ``composition`` swaps oracle
    functions (planted mistakes)."""

    cfg, w = golden["config"], golden["weights"]
    tensor = w.__getitem__
    heads, kv_heads = cfg["num_attention_heads"], cfg["num_key_value_heads"]
    cos, sin = ref.rope_cos_sin(ref.llama3_inv_freq(cfg["head_dim"]),
                                list(range(past, past + len(ids))))
    hidden = tensor("model.embed_tokens.weight")[torch.tensor(ids)]
    outs = []
    for layer in range(cfg["num_hidden_layers"]):
        hidden = ref.decoder_layer(hidden, ref.layer_weights(tensor, layer),
                                   caches[layer], past, cos, sin,
                                   cfg["rms_norm_eps"], heads, kv_heads)
        outs.append(hidden)
    normed = ref.rms_norm(hidden, tensor("model.norm.weight"), cfg["rms_norm_eps"])
    logits = ref.linear(normed[-1:], tensor("lm_head.weight"))[0]
    return outs, normed, logits


def _bf16_run(golden):
    cfg = golden["config"]
    caches = [dict() for _ in range(cfg["num_hidden_layers"])]
    past, results = 0, []
    for step in golden["steps"]:
        results.append(_bf16_oracle_step(golden, caches, past, step["ids"]))
        past += len(step["ids"])
    return results


def test_oracle_prompt_step_equals_transformers_bf16_bit_for_bit(bf16_golden):
    # Every bf16 rounding point of the oracle's composition -- RMSNorm
    # rounding before the weight multiply, q / k / v / o / gate / up / down
    # as bf16 F.linear, RoPE products and sum in bf16, the SDPA numerator
    # rounded to bf16, SiLU and the gate * up product in bf16, both
    # residual adds in bf16, the final norm and the bf16 LM head -- equals
    # transformers' LlamaForCausalLM in bf16 on the CPU (the reference's
    # CPU path) for the whole 6-token prompt.
    cfg = bf16_golden["config"]
    h = cfg["hidden_size"]
    step = bf16_golden["steps"][0]
    outs, normed, logits = _bf16_run(bf16_golden)[0]
    seq = len(step["ids"])
    for layer, expected in enumerate(step["layer_out_bf16_bits"]):
        assert torch.equal(outs[layer], from_bits(expected, (seq, h))), layer
    assert torch.equal(normed, from_bits(step["final_norm_bf16_bits"], (seq, h)))
    assert torch.equal(logits, from_bits(step["logits_bf16_bits"], (cfg["vocab_size"],)))


def test_oracle_decode_steps_match_transformers_bf16(bf16_golden):
    # Single-token steps attend over 7..9 positions.  There torch's bf16
    # SDPA kernel computes the softmax numerator with its own vectorised
    # exp, so the numerator's bf16 rounding can land one ulp apart from the
    # oracle's (the one rounding point that differs); everything after it
    # inherits that.  Each layer output stays within 2 bf16 ulps of its
    # largest element, the greedy tokens are equal and the logits are within
    # the north-star tolerance.
    cfg = bf16_golden["config"]
    h = cfg["hidden_size"]
    tokens = []
    for index, (step, (outs, normed, logits)) in enumerate(
            zip(bf16_golden["steps"], _bf16_run(bf16_golden))):
        seq = len(step["ids"])
        for layer, expected in enumerate(step["layer_out_bf16_bits"]):
            want = from_bits(expected, (seq, h)).float()
            diff = float((outs[layer].float() - want).abs().max())
            assert diff <= 2 * cases.bf16_ulp(want.abs().max()), (index, layer, diff)
        want = from_bits(step["logits_bf16_bits"], (cfg["vocab_size"],)).float()
        assert cases.compare(logits, want)["ok"], index
        tokens.append(int(torch.sort(logits.float(), descending=True,
                                     stable=True).indices[0]))
    assert tokens == bf16_golden["tokens"]


@pytest.mark.parametrize("mistake", ["fp32_numerator", "norm_rounding",
                                     "silu_two_roundings", "residual_fp32"])
def test_planted_bf16_mistakes_break_the_prompt_step(bf16_golden, monkeypatch,
                                                     mistake):
    # each rounding point, moved, changes the prompt step's bits
    original_attention = ref.attention
    if mistake == "fp32_numerator":
        monkeypatch.setattr(ref, "attention", lambda q, k, v, past:
                            original_attention(q, k, v, past, round_numerator=False))
    elif mistake == "norm_rounding":
        def rms_norm(hidden, weight, eps):  # multiply before rounding
            var = hidden.float().pow(2).mean(-1, keepdim=True)
            return (weight.float() * hidden.float() * torch.rsqrt(var + eps)).to(hidden.dtype)
        monkeypatch.setattr(ref, "rms_norm", rms_norm)
    elif mistake == "silu_two_roundings":
        # x * sigmoid(x) in bf16: the sigmoid rounded before the product
        monkeypatch.setattr(ref.F, "silu", lambda x: x * torch.sigmoid(x))
    else:
        def linear(x, w):  # fp32 GEMV outputs: the residual adds stay fp32
            return F.linear(x.float(), w.float())
        monkeypatch.setattr(ref, "linear", linear)
    step = bf16_golden["steps"][0]
    outs, _, _ = _bf16_oracle_step(bf16_golden,
                                   [dict(), dict()], 0, step["ids"])
    want = from_bits(step["layer_out_bf16_bits"][-1],
                     (len(step["ids"]), bf16_golden["config"]["hidden_size"]))
    assert not torch.equal(outs[-1].to(BF16), want)


# ------------------------------------ per-element bound of the layer checks


def _layer_check(seq, past, seed):
    case = cases.layer_case(seed, past, hidden=4096)
    s = seed * 100
    x = cases.normal_bf16((seq, 4096), s + 21)
    w = {name: case[name] for name in
         ("q", "k", "v", "o", "gate", "up", "down", "ln1", "ln2")}
    cos, sin = ref.rope_cos_sin(ref.llama3_inv_freq(128), list(range(past, past + seq)))
    prefix = {"k": case["k_cache"], "v": case["v_cache"]} if past else {}
    trace = {}
    expected = ref.decoder_layer(x, w, dict(prefix), past, cos, sin, 1e-5, trace=trace)
    alternative = cases.alternative_layer(x, w, dict(prefix), past, cos, sin, 1e-5)
    return x, w, prefix, cos, sin, trace, expected, alternative


@pytest.mark.parametrize("seq,past", [(1, 544), (256, 0)])
def test_rounding_bound_calibration(seq, past):
    # the alternative restatement sits within half of the per-element bound
    # (the calibration LAYER_ULPS rests on), for a decode step and a prefill
    x, w, prefix, cos, sin, trace, expected, alternative = _layer_check(seq, past, 3)
    scales = cases.layer_rounding_scales(x, trace, w)
    r = cases.within_rounding_bound(alternative, expected, scales["out"])
    assert r["ok"] and r["worst_ratio"] <= 0.5, r
    # and the bound is not loose: a plausible mistake in any stage exceeds it
    mistakes = {
        # one KV head's keys shifted by a position (a wrong cache slot)
        "kv_slot": lambda w_: dict(w_),
        # one 64-deep slab of down_proj's reduction dropped
        "down_slab": lambda w_: dict(w_, down=w_["down"].clone().index_fill_(
            1, torch.arange(640, 704), 0)),
        # gate and up rows of one 512-row block swapped
        "gate_up_rows": lambda w_: dict(w_, gate=torch.cat(
            (w_["up"][:512], w_["gate"][512:])), up=torch.cat(
            (w_["gate"][:512], w_["up"][512:]))),
        # one query head's o_proj columns dropped (a head left out)
        "head_dropped": lambda w_: dict(w_, o=w_["o"].clone().index_fill_(
            1, torch.arange(128 * 5, 128 * 6), 0)),
        # the post-attention norm weight ignored
        "norm_weight": lambda w_: dict(w_, ln2=torch.ones_like(w_["ln2"])),
    }
    for name, mutate in mistakes.items():
        bad_prefix = dict(prefix)
        if name == "kv_slot":
            if not past:
                continue
            bad_prefix = {"k": prefix["k"].roll(1, dims=1), "v": prefix["v"]}
        bad = ref.decoder_layer(x, mutate(w), bad_prefix, past, cos, sin, 1e-5)
        r = cases.within_rounding_bound(bad, expected, scales["out"])
        assert not r["ok"], (name, r)
