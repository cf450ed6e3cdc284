"""GPU side of the parity cases: runs the C-ABI kernels on the inputs of
oracle/cases.py and reports against the oracle's expectations.

Used by the gpu-marked tests and by __graft_entry__.smoke().  Every GPU
step prints what it runs before it runs (flushed), so a failure names its
case.
"""

import torch

from layer_streaming import _hip
from layer_streaming.rope import RopeTable
from layer_streaming.llama31 import Llama31Config
from layer_streaming.rope import rope_parameters
from oracle import cases


def _say(*parts):
    print("[gpu-case]", *parts, flush=True)


def run_layer_gpu(case, device="cuda:0", capacity_pad=256):
    """One decode step of one layer through the kernels; CPU outputs."""

    dev = torch.device(device)
    past = case["past"]
    n_kv, dim = case["n_kv_heads"], case["head_dim"]
    hidden = case["x"].numel()
    w = {k: case[k].to(dev) for k in ("q", "k", "v", "o", "gate", "up", "down",
                                      "ln1", "ln2")}
    capacity = past + capacity_pad
    k_cache = torch.zeros((n_kv, capacity, dim), dtype=torch.bfloat16, device=dev)
    v_cache = torch.zeros_like(k_cache)
    if past:
        k_cache[:, :past].copy_(case["k_cache"].to(dev))
        v_cache[:, :past].copy_(case["v_cache"].to(dev))
    rope = RopeTable(dim, rope_parameters(Llama31Config()), dev, capacity)
    cos, sin = rope.row(past)
    x = case["x"].to(dev)
    q = torch.empty(hidden, dtype=torch.bfloat16, device=dev)
    attn = torch.empty_like(q)
    h = x.clone()
    inter = torch.empty(w["gate"].shape[0], dtype=torch.bfloat16, device=dev)
    ws = torch.zeros(_hip.attention_workspace_bytes(past + 1, case["n_heads"],
                                                    n_kv, dim),
                     dtype=torch.uint8, device=dev)
    stride = capacity * dim
    kb, vb = k_cache.view(-1), v_cache.view(-1)
    _say("qkv_rope past={}".format(past))
    _hip.qkv_rope(w["q"], w["k"], w["v"], x, w["ln1"], case["eps"], cos, sin,
                  q, kb[past * dim:], vb[past * dim:], stride)
    torch.cuda.synchronize(dev)
    _say("decode_attention len={}".format(past + 1))
    _hip.decode_attention(q, kb, vb, stride, past + 1, attn, ws,
                          dim ** -0.5, case["n_heads"], n_kv, dim)
    torch.cuda.synchronize(dev)
    _say("o_proj residual")
    _hip.gemv_residual(w["o"], attn, h, h)
    h_attn = h.clone()
    _say("gate_up swiglu")
    _hip.gate_up_swiglu(w["gate"], w["up"], h, w["ln2"], case["eps"], inter)
    _say("down residual")
    _hip.gemv_residual(w["down"], inter, h, h)
    torch.cuda.synchronize(dev)
    return {
        "q": q.cpu(),
        "k_new": k_cache[:, past].cpu(),
        "v_new": v_cache[:, past].cpu(),
        "attn": attn.cpu(),
        "h_attn": h_attn.cpu(),
        "inter": inter.cpu(),
        "out": h.cpu(),
        "cos": cos.cpu(),
        "sin": sin.cpu(),
        "k_cache_prefix_intact": bool(torch.equal(
            k_cache[:, :past].cpu(), case["k_cache"])) if past else True,
    }


def run_layer_case(seed, past, device="cuda:0"):
    """Config-2 layer.  q, the new K / V rows, the attention output and
    silu(gate) * up within the north-star tolerance, or twice the deviation
    of the alternative restatement (sgemm_linear, blocked_attention;
    cases.within_noise_floor); the two bf16 residual sums (h_attn, out)
    element by element within cases.LAYER_ULPS bf16 ulps of their rounding
    scales (cases.within_rounding_bound)."""

    case = cases.layer_case(seed, past)
    expected = cases.layer_expected(case)
    alternative = cases.layer_expected(case, cases.sgemm_linear,
                                       cases.blocked_attention)
    got = run_layer_gpu(case, device)
    report = {"seed": seed, "past": past}
    ok = got["k_cache_prefix_intact"]
    trace = {"attn": expected["attn"], "o": expected["o"],
             "h_attn": expected["h_attn"], "inter": expected["inter"],
             "down": expected["down"]}
    scales = cases.layer_rounding_scales(case["x"], trace, case)
    for key in ("q", "k_new", "v_new", "attn", "h_attn", "inter", "out"):
        if key in scales:
            r = cases.within_rounding_bound(got[key], expected[key], scales[key])
            r["alternative_worst_ratio"] = cases.within_rounding_bound(
                alternative[key], expected[key], scales[key])["worst_ratio"]
        else:
            r = cases.compare(got[key], expected[key])
            f = cases.within_noise_floor(got[key], expected[key], alternative[key])
            r["ratio_to_noise_floor"] = f["ratio_to_floor"]
            r["ok"] = r["ok"] or f["ok"]
        report[key] = {k: round(v, 6) if isinstance(v, float) else v
                       for k, v in r.items()}
        ok = ok and r["ok"]
    rope_exact = bool(torch.equal(got["cos"], expected["cos"])) and bool(
        torch.equal(got["sin"], expected["sin"]))
    report["rope_table_exact"] = rope_exact
    report["ok"] = bool(ok and rope_exact)
    return report


def run_lm_head_gpu(case, chunk_rows, top_k=10, device="cuda:0"):
    dev = torch.device(device)
    w = case["w"].to(dev)
    h = case["h"].to(dev)
    rows = w.shape[0]
    ws = torch.zeros(_hip.lm_head_workspace_bytes(min(chunk_rows, rows), top_k),
                     dtype=torch.uint8, device=dev)
    values = torch.empty(top_k, dtype=torch.float32, device=dev)
    indices = torch.empty(top_k, dtype=torch.int64, device=dev)
    logits = torch.empty(rows, dtype=torch.float32, device=dev)
    for c, start in enumerate(range(0, rows, chunk_rows)):
        end = min(start + chunk_rows, rows)
        _say("lm_head chunk {} rows {}..{} top_k={}".format(c, start, end, top_k))
        _hip.lm_head_topk(w[start:end], h, top_k, start, c == 0, ws, values,
                          indices, logits_out=logits[start:end])
    torch.cuda.synchronize(dev)
    return values.cpu(), indices.cpu(), logits.cpu()


def run_lm_head_case(seed, rows, chunk_rows, top_k=10, device="cuda:0"):
    case = cases.lm_head_case(seed, rows)
    expected = cases.lm_head_expected(case, chunk_rows, top_k)
    values, indices, logits = run_lm_head_gpu(case, chunk_rows, top_k, device)
    report = {"seed": seed, "rows": rows, "chunk_rows": chunk_rows, "top_k": top_k}
    lr = cases.compare(logits, expected["logits"])
    report["logits"] = {k: round(v, 7) if isinstance(v, float) else v
                        for k, v in lr.items()}
    report["topk"] = cases.topk_contract(values, indices, logits,
                                         expected["logits"], top_k)
    report["ok"] = bool(lr["ok"] and report["topk"]["ok"])
    return report
