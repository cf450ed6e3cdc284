#!/usr/bin/env python3
"""Decode benchmark of the MI355X layer_streaming path (one GPU).

Headline (the JSON ``value``): BASELINE config 4 -- the 32-layer
Llama-3.1-8B-shaped model with all 16 GB of bf16 weights resident in HBM,
batch 1, greedy decode at context 32768 (KV cache 4 GiB ~ N(0, 1), synthetic
N(0, 0.02) weights drawn on the device).  A step is one decode token; the
timed region covers exactly --steps tokens between two synchronisations,
inputs already resident in HBM.

Also reported (extra keys, not ``value``):
  * hbm: the achievable HBM read bandwidth on this GPU, measured live (a
    streaming-read kernel over 4 GiB, sweep of launch widths), beside the
    8 TB/s vendor peak; rooflines are given against both;
  * roofline of the dominant kernel (the fused gate/up SwiGLU GEMV, 224 MiB
    per launch), timed live in the timed region with HIP events bound to
    launches of the kernel on its stream (hipExtLaunchKernel start/stop
    events: kernel execution only; one launch per token, layer 16, by
    default, since a timed launch adds a few microseconds of queue time),
    HBM traffic per launch from the committed FETCH_SIZE / WRITE_SIZE
    counter summary;
  * decode_graph: config 4 again, the same number of steps continuing the
    same sequence, replayed as one HIP graph per token (the position held
    on the device; layer_streaming.DecodeGraph; skip: --no-decode-graph);
  * streamed: BASELINE config 3 -- full_pinned 16 GB host arena,
    matrix_group units through two 224 MiB slots, streamed vocabulary, the
    configuration of the reference's published 624.16 ms/token;
    decode ms/token (1 warm-up + 7 timed tokens, p10 / median / p90), the
    PCIe-inclusive H2D GB/s, and the copy time the same transfers take in
    isolation at each size (measured live from the same arena): the H2D
    roofline of the streamed path (skip: --no-streamed);
  * prefill: BASELINE config 5 -- a 2048-token random-ID prompt through the
    pinned_staging store with matrix granularity and the streamed
    vocabulary (pageable arena -> pinned staging slots -> two 128 MiB device
    slots), prefill ms and H2D GB/s timed without events, then one
    profiled prefill whose every GEMM / attention launch is bound to HIP
    events: per-matrix TFLOP/s and the fraction of the bf16 dense MFMA
    peak (skip: --no-prefill);
  * cpu_baseline: the CPU oracle on this host's cores, per the reference's
    protocol (benchmarks/real_llama31_benchmark.py:83-104): 1 warm-up + 7
    repeats, p10 / median / p90, for config 4 whole tokens (the value),
    config 1 (the full streamed-vocabulary LM head step) and config 2 (one
    decoder layer at context 2048); CPU model and thread count stated
    (skip: --no-cpu-baseline).

Run: python bench.py [--steps K] [--warmup W] [--context L]
"""

import argparse
import gc
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "cascade-llm_amd"))
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E, vendor peak
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 matrix peak, vendor figure
PCIE_PEAK_GBPS = 63.0   # PCIe Gen5 x16 per direction, vendor figure
HIDDEN, INTER, VOCAB, LAYERS = 4096, 14336, 128256, 32
KV_BYTES_PER_POS_LAYER = 2 * 8 * 128 * 2
REFERENCE_STREAMED_MS = 624.162  # README.md:25-29, RTX 3080 Ti, PCIe Gen4


def log(*parts):
    print("[bench]", *parts, file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=32)
    p.add_argument("--warmup", type=int, default=4)
    p.add_argument("--context", type=int, default=32768)
    p.add_argument("--no-decode-graph", action="store_true",
                   help="config 4: skip the second timed run, which replays "
                        "the same number of decode steps as one HIP graph per "
                        "token (layer_streaming.DecodeGraph) after the eager "
                        "timed steps")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--no-streamed", action="store_true")
    p.add_argument("--streamed-steps", type=int, default=7)
    p.add_argument("--no-prefill", action="store_true")
    p.add_argument("--prefill-tokens", type=int, default=2048)
    p.add_argument("--prefill-repeats", type=int, default=3)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-repeats", type=int, default=7)
    p.add_argument("--roofline-stride", type=int, default=LAYERS,
                   help="time every N-th gate/up launch of the timed region "
                        "(default: one per token, layer 16; 1 = all; each "
                        "timed launch adds ~5 us of queue time)")
    p.add_argument("--probe", action="store_true",
                   help="only run the HBM-counter probe: 4 plain device copies "
                        "of 256 MiB, then 12 launches of each decode kernel "
                        "over 3 rotating operand copies (for rocprofv3 --pmc "
                        "runs)")
    p.add_argument("--hbm-only", action="store_true",
                   help="only measure and print the achievable HBM read "
                        "bandwidth sweep")
    return p.parse_args()


PROBE_COPY_BYTES = 256 << 20
TRAFFIC_FILE = ROOT / "profiles" / "gate_up_traffic.txt"


def counter_probe():
    """Known-size copies (counter calibration), then each decode kernel at
    its config-4 shape over 3 rotating operand copies (beyond the 256 MB
    MALL), 12 launches each, in this order: gate/up SwiGLU, q|k|v + RoPE,
    o_proj + residual, down_proj + residual, decode attention at L = 32769
    (main kernel + split merge, then the fused form that merges inside
    the attention launch)."""

    import torch
    from layer_streaming import _hip
    from layer_streaming.llama31 import Llama31Config
    from layer_streaming.rope import RopeTable, rope_parameters

    dev = torch.device("cuda:0")
    src = torch.randn(PROBE_COPY_BYTES // 4, device=dev)
    dst = torch.empty_like(src)
    for _ in range(4):
        _hip.device_copy(dst, src)
    torch.cuda.synchronize(dev)
    log("probe: 4 device copies of {} bytes done".format(PROBE_COPY_BYTES))
    del src, dst

    def weights(rows, k):
        return [torch.randn(rows, k, device=dev).mul_(0.02).to(torch.bfloat16)
                for _ in range(3)]

    x = torch.randn(INTER, device=dev).to(torch.bfloat16)
    norm = torch.ones(HIDDEN, dtype=torch.bfloat16, device=dev)
    y = torch.empty(INTER, dtype=torch.bfloat16, device=dev)
    gates, ups = weights(INTER, HIDDEN), weights(INTER, HIDDEN)
    for i in range(12):
        _hip.gate_up_swiglu(gates[i % 3], ups[i % 3], x[:HIDDEN], norm, 1e-5, y)
    torch.cuda.synchronize(dev)
    log("probe: 12 gate/up launches done")
    del gates, ups

    length = 32769
    capacity = 32800
    kv = [torch.randn(2, 8, capacity, 128, device=dev).to(torch.bfloat16)
          for _ in range(3)]
    rope = RopeTable(128, rope_parameters(Llama31Config()), dev, capacity)
    cos, sin = rope.row(length - 1)
    q = torch.empty(HIDDEN, dtype=torch.bfloat16, device=dev)
    wqs, wks, wvs = weights(HIDDEN, HIDDEN), weights(1024, HIDDEN), weights(1024, HIDDEN)
    stride = capacity * 128
    for i in range(12):
        cache = kv[i % 3]
        _hip.qkv_rope(wqs[i % 3], wks[i % 3], wvs[i % 3], x[:HIDDEN], norm, 1e-5,
                      cos, sin, q, cache[0].view(-1)[(length - 1) * 128:],
                      cache[1].view(-1)[(length - 1) * 128:], stride)
    torch.cuda.synchronize(dev)
    log("probe: 12 q|k|v launches done")
    del wqs, wks, wvs
    h = torch.randn(HIDDEN, device=dev).to(torch.bfloat16)
    wos = weights(HIDDEN, HIDDEN)
    for i in range(12):
        _hip.gemv_residual(wos[i % 3], x[:HIDDEN], h, h)
    torch.cuda.synchronize(dev)
    log("probe: 12 o_proj launches done")
    del wos
    wds = weights(HIDDEN, INTER)
    for i in range(12):
        _hip.gemv_residual(wds[i % 3], x, h, h)
    torch.cuda.synchronize(dev)
    log("probe: 12 down_proj launches done")
    del wds
    out = torch.empty(HIDDEN, dtype=torch.bfloat16, device=dev)
    ws = torch.zeros(_hip.attention_workspace_bytes(length), dtype=torch.uint8,
                     device=dev)
    for i in range(12):
        cache = kv[i % 3]
        _hip.decode_attention(q, cache[0].view(-1), cache[1].view(-1), stride,
                              length, out, ws, 128 ** -0.5)
    torch.cuda.synchronize(dev)
    log("probe: 12 attention launches done")
    sync = torch.zeros(_hip.ATTENTION_SYNC_BYTES, dtype=torch.uint8, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    for i in range(12):
        cache = kv[i % 3]
        _hip.decode_attention_fused(q, cache[0].view(-1), cache[1].view(-1),
                                    stride, length, out, ws, sync, err,
                                    128 ** -0.5)
    torch.cuda.synchronize(dev)
    if int(err.item()) != 0:
        raise RuntimeError("fused attention error word {}".format(int(err.item())))
    log("probe: 12 fused attention launches done")


def measured_traffic(path):
    """HBM bytes per launch from a committed counter summary."""

    try:
        for line in path.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch="):
                return int(line.split("=", 1)[1])
    except OSError:
        return None
    return None


def percentiles(values):
    ordered = sorted(values)
    return {
        "median": statistics.median(ordered),
        "p10": ordered[int(0.1 * (len(ordered) - 1))],
        "p90": ordered[int(round(0.9 * (len(ordered) - 1)))],
    }


# ------------------------------------------------------------ HBM plateau

HBM_SWEEP_BYTES = 4 << 30


def hbm_plateau():
    """Achievable HBM read bandwidth: a nontemporal streaming read of 4 GiB
    (16x the 256 MB MALL) at several launch widths, kernel-bound events,
    median of 8 launches each; the best width's median is the plateau."""

    import torch
    from layer_streaming import _hip

    dev = torch.device("cuda:0")
    buf = torch.empty(HBM_SWEEP_BYTES, dtype=torch.uint8, device=dev)
    buf.view(torch.int32).random_(0, 1 << 30)
    sink = torch.zeros(1, dtype=torch.float32, device=dev)
    sweep = {}
    for blocks in (512, 1024, 2048, 4096, 8192, 16384, 32768):
        times = []
        for rep in range(10):
            start = _hip.HipEvent(enable_timing=True)
            stop = _hip.HipEvent(enable_timing=True)
            _hip.time_next_launch(start, stop)
            _hip.hbm_read(buf, sink, blocks=blocks)
            if rep >= 2:
                times.append((start, stop))
        torch.cuda.synchronize(dev)
        ms = statistics.median(a.elapsed_time(b) for a, b in times)
        sweep[blocks] = round(HBM_SWEEP_BYTES / 1e9 / (ms / 1e3), 1)
    best = max(sweep, key=sweep.get)
    del buf
    torch.cuda.empty_cache()
    return {
        "read_gbps": sweep[best],
        "blocks": best,
        "sweep_gbps_by_blocks": sweep,
        "bytes": HBM_SWEEP_BYTES,
        "peak_gbps": HBM_PEAK_GBPS,
        "frac_of_peak": round(sweep[best] / HBM_PEAK_GBPS, 4),
        "method": "cascade_hbm_read: nontemporal 16-byte loads, 8 in flight per "
                  "thread, 32 KiB contiguous per 256-thread workgroup and step; "
                  "kernel-bound events, median of 8 launches per width",
    }


# ------------------------------------------------- config 4 (HBM resident)


def token_bytes(context):
    """Algorithmic HBM bytes of one decode token at a given context."""

    weights = LAYERS * 436207616 + VOCAB * HIDDEN * 2
    norms = (2 * LAYERS + 1) * HIDDEN * 2
    kv_read = LAYERS * context * KV_BYTES_PER_POS_LAYER
    kv_write = LAYERS * KV_BYTES_PER_POS_LAYER
    embedding_row = HIDDEN * 2
    return weights + norms + kv_read + kv_write + embedding_row


def gate_up_bytes():
    # W (gate | up) + input vector + norm weight + output (bf16)
    return 2 * INTER * HIDDEN * 2 + HIDDEN * 2 + HIDDEN * 2 + INTER * 2


def resident_decode(args):
    import torch
    from layer_streaming import (
        Llama31Config,
        Llama31DecodeExecutor,
        ResidentDeviceArena,
        ResidentTransformerRuntime,
        build_llama31_8b_plan,
    )

    dev = torch.device("cuda:0")
    plan = build_llama31_8b_plan("matrix_group", stream_vocab=False)
    log("config 4: drawing 16 GB of synthetic weights in HBM")
    resident = ResidentDeviceArena(plan, None, dev, fill=False).fill_random(args.seed)
    runtime = ResidentTransformerRuntime(plan, None, resident, dev,
                                         synchronize=False).fill_random(args.seed)
    executor = Llama31DecodeExecutor(Llama31Config(), resident, top_k=10)
    head_steps = 8  # config 1 with the head resident, after the timed steps
    total = args.context + args.warmup + args.steps + head_steps + 1
    graphed = not args.no_decode_graph
    if graphed:
        total += args.warmup + args.steps + 1
    executor.reserve(total)
    cache = executor.kv_cache
    log("config 4: KV cache {} positions x 32 layers ~ N(0,1)".format(args.context))
    gen = torch.Generator(device=dev).manual_seed(args.seed + 2)
    for layer in range(LAYERS):
        cache.buffer[layer, :, :, : args.context].normal_(generator=gen)
        cache.set_length(layer, args.context)
    torch.cuda.synchronize(dev)

    token = torch.tensor([[int(args.seed * 7919 % VOCAB)]], device=dev)
    group = "gate_up"
    with torch.inference_mode():
        for _ in range(args.warmup):
            state = executor.finish(runtime.run(executor, executor.begin(token)))
            token = state.topk_indices.reshape(1, -1)[:, :1]
        torch.cuda.synchronize(dev)
        stride = args.roofline_stride
        executor.instrument(group, (args.steps * LAYERS + stride - 1) // stride,
                            stride=stride, offset=(LAYERS // 2) % stride)
        log("config 4: timing {} decode steps".format(args.steps))
        start = time.perf_counter()
        for _ in range(args.steps):
            state = executor.finish(runtime.run(executor, executor.begin(token)))
            token = state.topk_indices.reshape(1, -1)[:, :1]
        torch.cuda.synchronize(dev)
        elapsed = time.perf_counter() - start
        executor.instrument("lm_head", head_steps)
        for _ in range(head_steps):
            state = executor.finish(runtime.run(executor, executor.begin(token)))
            token = state.topk_indices.reshape(1, -1)[:, :1]
        torch.cuda.synchronize(dev)
    executor.check_errors()
    timed_ms = executor.kernel_times_ms(group)
    head_us = 1000.0 * statistics.median(executor.kernel_times_ms("lm_head"))
    ms_per_step = elapsed * 1000.0 / args.steps
    graph = None
    if graphed:
        from layer_streaming import DecodeGraph

        with torch.inference_mode():
            decoder = DecodeGraph(executor, runtime, token,
                                  args.warmup + args.steps + 1)
            decoder.step(args.warmup)
            torch.cuda.synchronize(dev)
            log("config 4: timing {} graph-replayed decode steps".format(args.steps))
            start = time.perf_counter()
            decoder.step(args.steps)
            torch.cuda.synchronize(dev)
            g_elapsed = time.perf_counter() - start
            decoder.check()
            graph = {
                "ms_per_step": round(g_elapsed * 1000.0 / args.steps, 4),
                "tokens": args.steps,
                "launches_per_step": "one graph replay (165 kernel nodes)",
                "last_token": int(decoder.tokens()[0, -1]),
            }
            decoder.close()
    prefill = None
    if not args.no_prefill:
        prefill = resident_prefill(args, executor, runtime, dev)
    mean_context = args.context + args.warmup + (args.steps - 1) / 2.0
    result = {
        "ms_per_step": ms_per_step,
        "tokens": args.steps,
        "timed_group": group,
        "timed_launches": len(timed_ms),
        "timed_avg_us": 1000.0 * statistics.mean(timed_ms),
        "timed_median_us": 1000.0 * statistics.median(timed_ms),
        "mean_attended": mean_context + 1,
        "token_hbm_bytes": token_bytes(int(mean_context)),
        "last_token": int(token.reshape(-1)[0]),
        "config1_lm_head_resident": {
            "workload": "BASELINE config 1 with the LM head resident in HBM: "
                        "128256 x 4096 bf16 GEMV to fp32 logits, block top-k "
                        "and merge (3 launches) on the final hidden state of "
                        "{} decode steps, between stream events (dispatch "
                        "included)".format(head_steps),
            "median_us": round(head_us, 2),
            "bytes": VOCAB * HIDDEN * 2,
            "gbps": round(VOCAB * HIDDEN * 2 / (head_us * 1e-6) / 1e9, 1),
        },
    }
    if graph is not None:
        result["decode_graph"] = graph
    if prefill is not None:
        result["prefill_resident"] = prefill
    del executor, runtime, resident, cache
    torch.cuda.empty_cache()
    return result


# Resident prefill launch groups of the matrix_group granularity: fused
# q|k|v (+ RoPE + KV write) and gate|up (+ SwiGLU) GEMMs, and their
# multiply-accumulates per token row.
RESIDENT_PREFILL_GEMMS = (
    ("qkv_rope", "gemm_qkv", (HIDDEN + 2 * 1024) * HIDDEN),
    ("o_proj", "gemm_o", HIDDEN * HIDDEN),
    ("gate_up_swiglu", "gemm_gate_up", 2 * INTER * HIDDEN),
    ("down_proj", "gemm_down", HIDDEN * INTER),
)


def resident_prefill(args, executor, runtime, dev):
    """A 2048-token prefill through the config-4 executor, weights resident:
    the prefill GEMMs and causal attention back to back (no H2D waits
    between launches), as a compute-bound counterpart of config 5."""

    import torch

    tokens = args.prefill_tokens
    gen = torch.Generator().manual_seed(args.seed + 3)
    prompt = torch.randint(0, VOCAB, (1, tokens), generator=gen).to(dev)
    groups = {name: LAYERS for _, name, _ in RESIDENT_PREFILL_GEMMS}
    groups["prefill_attention"] = LAYERS
    walls = []
    with torch.inference_mode():
        # warm-up, timed prefills, then one with every launch timed
        for rep in range(1 + args.prefill_repeats + 1):
            executor.kv_cache.clear()
            last = rep == args.prefill_repeats + 1
            if last:
                for name, count in groups.items():
                    executor.instrument(name, count)
            torch.cuda.synchronize(dev)
            t0 = time.perf_counter()
            executor.finish(runtime.run(executor, executor.begin(prompt)))
            torch.cuda.synchronize(dev)
            wall = (time.perf_counter() - t0) * 1000.0
            log("resident prefill {} {:.1f} ms{}".format(rep, wall, " (profiled)" if last else ""))
            if 0 < rep and not last:
                walls.append(wall)
    executor.check_errors()
    gemms = {}
    for label, group, macs in RESIDENT_PREFILL_GEMMS:
        avg = statistics.mean(executor.kernel_times_ms(group))
        tflops = 2.0 * tokens * macs / (avg * 1e-3) / 1e12
        gemms[label] = {"avg_us": round(1000 * avg, 1), "tflops": round(tflops, 1),
                        "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4)}
    attn = statistics.mean(executor.kernel_times_ms("prefill_attention"))
    attn_tflops = 4.0 * 32 * 128 * tokens * (tokens + 1) / 2 / (attn * 1e-3) / 1e12
    median = statistics.median(walls)
    return {
        "workload": "{}-token random-ID prompt through the config-4 executor "
                    "(matrix_group, all weights HBM-resident): 1 warm-up + {} "
                    "timed prefills + 1 with every GEMM and attention launch "
                    "timed; wall time from begin() to finish(): 32 layers, the "
                    "fp32 logits of every position (the reference's resident "
                    "finish) and the last row's top-k".format(tokens, args.prefill_repeats),
        "prefill_ms_median": round(median, 2),
        "prompt_tokens_per_s": round(tokens / (median / 1e3), 1),
        "gemm": gemms,
        "attention": {"avg_us": round(1000 * attn, 1), "tflops": round(attn_tflops, 1),
                      "mfma_frac": round(attn_tflops / MFMA_BF16_PEAK_TFLOPS, 4)},
        "mfma_peak_tflops": MFMA_BF16_PEAK_TFLOPS,
    }


# One decoder layer's seven projections, as the prefill's matrix-granularity
# launches: (name, [N, K], epilogue).
SWEEP_ROWS = (16, 64, 128, 256, 512, 1024, 2048, 4096, 8192, 16384, 32768)
LAYER_MACS = (HIDDEN + 2 * 1024 + HIDDEN + 3 * INTER) * HIDDEN  # 218,103,808


# Prefill projection shapes at M = 2048 (N, K): the per-matrix units of
# config 5 and the fused units of the resident prefill.
VENDOR_SHAPES = (
    ("q_proj / o_proj", HIDDEN, HIDDEN),
    ("k_proj / v_proj", 1024, HIDDEN),
    ("gate_proj / up_proj", INTER, HIDDEN),
    ("down_proj", HIDDEN, INTER),
    ("q|k|v fused", HIDDEN + 2 * 1024, HIDDEN),
    ("gate|up fused", 2 * INTER, HIDDEN),
)


def prefill_vs_vendor(m=2048, copies=4, rounds=6, per_round=4):
    """Each prefill projection shape at M = 2048: this library's bf16 GEMM
    (cascade_gemm_bf16, the tile schedule the fused epilogues use) against
    torch's F.linear (hipBLASLt on this image), both on cold weights (weight
    copies rotating over >= 512 MiB, twice the 256 MB MALL),
    alternating rounds, each launch between stream events; medians."""
    import torch
    import torch.nn.functional as F
    from layer_streaming import _hip

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(11)
    x = (torch.randn((m, INTER), device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    out = {}
    for name, n, k in VENDOR_SHAPES:
        ncopy = max(copies, -(-(512 << 20) // (n * k * 2)))
        ws = [(torch.randn((n, k), device=dev, generator=gen) * 0.02).to(torch.bfloat16)
              for _ in range(ncopy)]
        xk = x[:, :k].contiguous()
        y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        times = {"ours": [], "vendor": []}
        idx = 0
        for _ in range(rounds):
            for who in ("ours", "vendor"):
                for _ in range(per_round):
                    w = ws[idx % ncopy]
                    idx += 1
                    start = torch.cuda.Event(enable_timing=True)
                    stop = torch.cuda.Event(enable_timing=True)
                    start.record()
                    if who == "ours":
                        _hip.gemm(xk, w, y)
                    else:
                        F.linear(xk, w)
                    stop.record()
                    times[who].append((start, stop))
        torch.cuda.synchronize(dev)
        flops = 2.0 * m * n * k
        row = {"m_n_k": [m, n, k], "weight_copies": ncopy}
        for who, evs in times.items():
            us = statistics.median(a.elapsed_time(b) * 1000.0 for a, b in evs)
            row[who + "_us"] = round(us, 1)
            row[who + "_tflops"] = round(flops / (us * 1e-6) / 1e12, 1)
        row["ours_over_vendor"] = round(row["ours_us"] / row["vendor_us"], 3)
        out[name] = row
        del ws, y
    torch.cuda.empty_cache()
    return {
        "workload": "prefill projection GEMMs at M = 2048 rows, bf16 in / out, "
                    "fp32 accumulation; this library's cascade_gemm_bf16 against "
                    "torch F.linear (hipBLASLt), cold weights, stream events "
                    "around each launch (dispatch included), medians of "
                    "{} launches each".format(rounds * per_round),
        "shapes": out,
    }


def prefill_sweep(args):
    """The copy/compute crossover of a streamed prefill, measured the way the
    reference measures it (an M sweep of one layer's projections,
    benchmarks/torch_llama32_1b_bench.py:351-385): one layer's seven
    projections through this library's prefill GEMMs at M prompt rows --
    q, k, v, o (+ residual), gate (+ SiLU), up (* gate), down (+ residual),
    each weight ~ N(0, 0.02) and read from HBM -- timed back to back with
    HIP events (2 warm-up + 5 timed passes, median), against the time one
    layer's 436 MB take over PCIe from pinned host memory (5 timed copies
    with this library's hipMemcpyAsync, median)."""

    import torch
    from layer_streaming import _hip

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(args.seed + 4)

    def draw(*shape, scale=0.02):
        return (torch.randn(*shape, generator=gen, device=dev) * scale).to(torch.bfloat16)

    wq, wk, wv, wo = draw(HIDDEN, HIDDEN), draw(1024, HIDDEN), draw(1024, HIDDEN), draw(HIDDEN, HIDDEN)
    wg, wu, wd = draw(INTER, HIDDEN), draw(INTER, HIDDEN), draw(HIDDEN, INTER)
    layer_bytes = LAYER_MACS * 2
    # the layer's copy time over PCIe
    host = torch.empty(LAYER_MACS, dtype=torch.bfloat16, pin_memory=True)
    slot = torch.empty(LAYER_MACS, dtype=torch.bfloat16, device=dev)
    stream = torch.cuda.Stream(dev)
    copies = []
    for rep in range(2 + 5):
        a = _hip.HipEvent(enable_timing=True)
        b = _hip.HipEvent(enable_timing=True)
        a.record(stream)
        _hip.memcpy_h2d_async(slot, host, layer_bytes, stream)
        b.record(stream)
        b.synchronize()
        if rep >= 2:
            copies.append(a.elapsed_time(b))
    copy_ms = statistics.median(copies)
    del host, slot
    rows = []
    for m in SWEEP_ROWS:
        x = draw(m, HIDDEN, scale=1.0)
        q = torch.empty(m, HIDDEN, dtype=torch.bfloat16, device=dev)
        k = torch.empty(m, 1024, dtype=torch.bfloat16, device=dev)
        v = torch.empty_like(k)
        h = torch.zeros(m, HIDDEN, dtype=torch.bfloat16, device=dev)
        g = torch.empty(m, INTER, dtype=torch.bfloat16, device=dev)
        u = torch.empty_like(g)
        # split-K workspace for o_proj / down_proj, as the executor passes
        ws_bytes = max(_hip.gemm_workspace_bytes(m, HIDDEN, HIDDEN),
                       _hip.gemm_workspace_bytes(m, HIDDEN, INTER))
        ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)

        def layer():
            _hip.gemm(x, wq, q)
            _hip.gemm(x, wk, k)
            _hip.gemm(x, wv, v)
            _hip.gemm_residual(q, wo, h, h, workspace=ws)
            _hip.gate_silu_gemm(x, wg, g)
            _hip.up_mul_gemm(x, wu, g, u)
            _hip.gemm_residual(u, wd, h, h, workspace=ws)

        times = []
        for rep in range(2 + 5):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            layer()
            b.record()
            b.synchronize()
            if rep >= 2:
                times.append(a.elapsed_time(b))
        ms = statistics.median(times)
        tflops = 2.0 * LAYER_MACS * m / (ms * 1e-3) / 1e12
        rows.append({"rows_M": m, "gpu_elapsed_ms": round(ms, 4),
                     "effective_tflops": round(tflops, 1),
                     "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                     "nominal_weight_gbps": round(layer_bytes / 1e9 / (ms / 1e3), 1),
                     "compute_over_copy": round(ms / copy_ms, 4)})
        log("prefill sweep M={}: {:.3f} ms, {:.1f} TFLOP/s".format(m, ms, tflops))
        del x, q, k, v, h, g, u, ws
    crossover = None
    for lo, hi in zip(rows, rows[1:]):
        if lo["compute_over_copy"] < 1.0 <= hi["compute_over_copy"]:
            # compute time is linear in M between the two sweep points
            f = (1.0 - lo["compute_over_copy"]) / (hi["compute_over_copy"] - lo["compute_over_copy"])
            crossover = int(round(lo["rows_M"] + f * (hi["rows_M"] - lo["rows_M"])))
    del wq, wk, wv, wo, wg, wu, wd
    torch.cuda.empty_cache()
    return {
        "workload": "one layer's seven projections (q, k, v, o + residual, "
                    "gate + SiLU, up * gate, down + residual) at M prompt rows, "
                    "weights read from HBM, o/down with the split-K workspace; "
                    "2 warm-up + 5 timed passes per M",
        "layer_weight_bytes": layer_bytes,
        "layer_copy_ms": round(copy_ms, 3),
        "layer_copy_gbps": round(layer_bytes / 1e9 / (copy_ms / 1e3), 2),
        "rows": rows,
        "crossover_rows_M": crossover,
    }


# ------------------------------------------------- config 3 (H2D streamed)


def copy_rates(samples, stream, slot, reps=5, rounds=2):
    """H2D GB/s of each (nbytes -> pinned source) copied alone into ``slot``
    on ``stream``: per round 2 warm-up + ``reps`` timed copies per size, each
    bracketed by events, median per round; the best round per size (a
    transient stall of the host link in one round is not the link's rate)."""

    from layer_streaming import _hip

    rates = {}
    for _ in range(rounds):
        for nbytes, source in samples.items():
            pairs = []
            for rep in range(2 + reps):
                a = _hip.HipEvent(enable_timing=True)
                b = _hip.HipEvent(enable_timing=True)
                a.record(stream)
                _hip.memcpy_h2d_async(slot, source, nbytes, stream)
                b.record(stream)
                if rep >= 2:
                    pairs.append((a, b))
            stream.synchronize()
            ms = statistics.median(x.elapsed_time(y) for x, y in pairs)
            rates[nbytes] = max(rates.get(nbytes, 0.0), nbytes / 1e9 / (ms / 1e3))
    return rates


def size_label(n):
    return str(n >> 20) + " MiB" if n % (1 << 20) == 0 else str(n)


def h2d_ideal(plan, store, runtime, reps=5):
    """Copy time of one streamed token's transfers when each runs alone:
    every distinct transfer size is copied from the token's own arena rows
    into a device slot on the copy stream (copy_rates), and the token's
    transfers are priced at their size's rate."""

    import torch

    vocab = plan.vocab
    transfers = [(u.nbytes, store.unit_source(u)) for u in plan.units]
    head = store.tensor(vocab.lm_head_key)
    for c in range(vocab.chunk_count):
        first, end = vocab.chunk_bounds(c)
        transfers.append(((end - first) * vocab.hidden_size * 2,
                          head[first:end].reshape(-1)))
    samples = {}
    for nbytes, source in transfers:
        samples.setdefault(nbytes, source)
    rates = copy_rates(samples, runtime.copy_stream, runtime.device_slots[0], reps)
    ideal_ms = sum(n / 1e9 / rates[n] * 1e3 for n, _ in transfers)
    runtime.discard_slots()  # slot 0 now holds a probe copy
    torch.cuda.synchronize()
    return ideal_ms, {size_label(n): round(r, 2) for n, r in sorted(rates.items())}


def streamed_decode(args):
    import torch
    from layer_streaming import (
        DoubleBufferRuntime,
        Llama31Config,
        Llama31DecodeExecutor,
        ResidentDeviceArena,
        VocabStreamingRuntime,
        build_llama31_8b_plan,
        create_weight_store,
    )

    dev = torch.device("cuda:0")
    plan = build_llama31_8b_plan("matrix_group", stream_vocab=True)
    log("config 3: pinning a {:.1f} GB host arena".format(plan.host_arena_bytes / 1e9))
    t0 = time.perf_counter()
    store = create_weight_store(plan, "full_pinned")
    store.fill_random(seed=args.seed, device=dev)
    setup_s = time.perf_counter() - t0
    # the peak counts from here: the synthetic weights are drawn on the GPU
    # in fp32 (GBs of temporaries a checkpoint load does not have); earlier
    # legs' objects that only a cycle still holds are collected first
    torch.cuda.synchronize(dev)
    gc.collect()
    torch.cuda.empty_cache()
    torch.cuda.reset_peak_memory_stats(dev)
    allocated_before = torch.cuda.memory_allocated(dev)  # earlier legs' leftovers
    resident = ResidentDeviceArena(plan, store, dev)
    runtime = DoubleBufferRuntime(plan, store, resident, dev)
    vocab = VocabStreamingRuntime(plan, store, runtime)
    executor = Llama31DecodeExecutor(Llama31Config(), resident, vocab_runtime=vocab,
                                     top_k=10)
    ideal_ms, size_rates = h2d_ideal(plan, store, runtime)
    log("config 3: isolated copies of the token's transfers: {:.2f} ms".format(ideal_ms))
    prompt = torch.tensor([[128000, 791, 7438, 315, 2324, 374]], device=dev)
    walls, h2d, lm, profiled = [], [], [], []
    with torch.inference_mode():
        t0 = time.perf_counter()
        state = executor.finish(runtime.run(executor, executor.begin(prompt)))
        prefill_ms = (time.perf_counter() - t0) * 1000.0
        token = state.topk_indices[..., 0]
        # 1 warm-up, timed decodes without timing events, then two decodes
        # with per-copy / per-unit events for the H2D and compute figures.
        # A token is timed from the previous token's return to its own: the
        # runtime keeps copying ahead across that boundary (a device-wide
        # synchronise per token would stop it), and finish() returns once
        # the top-k is in HBM.
        timed = args.streamed_steps
        torch.cuda.current_stream(dev).synchronize()
        t0 = time.perf_counter()
        for step in range(1 + timed + 2):
            runtime.profile = vocab.profile = step > timed
            state = executor.begin(token)
            state = runtime.run(executor, state)
            state = executor.finish(state)
            token = state.topk_indices[..., 0]
            torch.cuda.current_stream(dev).synchronize()
            now = time.perf_counter()
            wall = (now - t0) * 1000.0
            t0 = now
            if step == 0:
                continue  # warm-up decode, as the reference's protocol
            log("config 3: decode {} {:.1f} ms{}".format(
                step, wall, " (profiled)" if step > timed else ""))
            if step > timed:
                profiled.append(wall)
                h2d.append(runtime.last_profile)
                lm.append(vocab.last_profile)
            else:
                walls.append(wall)
    peak_allocated = torch.cuda.max_memory_allocated(dev)
    peak_reserved = torch.cuda.max_memory_reserved(dev)
    lm_head = config1_lm_head(executor, vocab, runtime, state, dev)
    bytes_token = plan.stream_bytes_per_token + VOCAB * HIDDEN * 2 + HIDDEN * 2
    spread = percentiles(walls)
    median = spread["median"]
    result = {
        "ms_per_token_median": median,
        "ms_per_token_p10": spread["p10"],
        "ms_per_token_p90": spread["p90"],
        "tokens_per_s": 1000.0 / median,
        "profiled_ms_per_token": statistics.median(profiled),
        "prefill_6_tokens_ms": prefill_ms,
        "h2d_bytes_per_token": bytes_token,
        "pcie_inclusive_gbps": bytes_token / 1e9 / (median / 1e3),
        "isolated_copy_ms_per_token": ideal_ms,
        "frac_of_isolated_copy_time": ideal_ms / median,
        "isolated_copy_gbps_by_size": size_rates,
        "transformer_h2d_gbps_median": statistics.median(
            p["h2d_effective_gbps"] for p in h2d),
        "transformer_compute_event_sum_ms": statistics.median(
            p["compute_event_sum_ms"] for p in h2d),
        "lm_head_h2d_gbps_median": statistics.median(
            p["h2d_effective_gbps"] for p in lm),
        "lm_head_compute_event_sum_ms": statistics.median(
            p["compute_event_sum_ms"] for p in lm),
        "host_setup_s": setup_s,
        "memory": {
            "cuda_peak_allocated_bytes": peak_allocated,
            "cuda_peak_allocated_gib": round(peak_allocated / 2 ** 30, 4),
            "cuda_peak_reserved_bytes": peak_reserved,
            "allocated_before_bytes": allocated_before,
            "planned_weight_gpu_bytes": runtime.stats.weight_gpu_bytes,
            "pinned_host_bytes": store.pinned_cpu_bytes + vocab.extra_pinned_cpu_bytes,
            "reference_cuda_peak_allocated_bytes": 481369088,
            "reference_source": "real_results/vocab_streaming_summary.json "
                                "matrix_group_streamed_vocab (0.448 GiB, RTX 3080 Ti)",
            "note": "peak since the host store was filled (the runtime objects "
                    "were built after it): two 224 MiB slots, resident norms, "
                    "KV cache, scratch and workspaces",
        },
        "config1_lm_head_streamed": lm_head,
    }
    store.close()
    del executor, vocab, runtime, resident, store
    torch.cuda.empty_cache()
    return result


def config1_lm_head(executor, vocab, runtime, state, dev, repeats=5):
    """BASELINE config 1 on the GPU: the streamed-vocabulary LM-head step
    alone (8 chunks of 16384 rows, the last 13568, copied from the pinned
    arena through the two device slots; one GEMV + top-k launch per chunk),
    the figures the reference reports for its vocab profile
    (real_results/vocab_streaming_summary.json "profiles.vocab": H2D event
    sum, GEMV + top-k event sum, pipeline).  Each step starts with no chunk
    in the slots (they hold the next call's first units)."""

    import torch

    hidden = torch.randn(1, 1, HIDDEN, device=dev).to(torch.bfloat16)
    profiles = []
    with torch.inference_mode():
        vocab.profile = True
        for step in range(1 + repeats):
            torch.cuda.synchronize(dev)
            runtime.discard_slots()
            out = vocab.lm_head_topk(hidden, top_k=10)
            torch.cuda.synchronize(dev)
            if step:
                profiles.append(dict(vocab.last_profile))
        vocab.profile = False
    del out

    def med(key):
        return round(statistics.median(p[key] for p in profiles), 4)

    return {
        "workload": "hidden [1, 4096] bf16 ~ N(0,1); LM head [128256, 4096] bf16 "
                    "in the pinned arena; 7 x 16384 + 13568 rows; top-10; "
                    "{} steps after 1 warm-up, medians".format(repeats),
        "pipeline_ms": med("pipeline_ms"),
        "h2d_event_sum_ms": med("h2d_event_sum_ms"),
        "gemv_topk_event_sum_ms": med("compute_event_sum_ms"),
        "h2d_gbps": med("h2d_effective_gbps"),
        "h2d_bytes": VOCAB * HIDDEN * 2,
        "reference_ms": {"pipeline": 44.01, "h2d_event_sum": 43.70,
                         "gemv_topk_event_sum": 2.18,
                         "source": "real_results/vocab_streaming_summary.json:68-78 "
                                   "(RTX 3080 Ti, PCIe Gen4)"},
    }


# ------------------------------------------------- config 2 (one layer)

# Algorithmic bytes of the decode kernels of one layer (weights, the input
# vector, the norm weight and the epilogue operands they read, and what they
# write); attention: the K / V rows read for L attended positions, q and the
# output.
def layer_kernel_bytes(attended):
    return {
        "qkv": (HIDDEN + 2 * 1024) * HIDDEN * 2 + HIDDEN * 2 * 2 + (HIDDEN + 2 * 1024) * 2,
        "attention": 2 * attended * 8 * 128 * 2 + 32 * 128 * 2 * 2,
        "o_proj": HIDDEN * HIDDEN * 2 + HIDDEN * 2 + 2 * HIDDEN * 2,
        "gate_up": 2 * INTER * HIDDEN * 2 + 2 * HIDDEN * 2 + INTER * 2,
        "down_proj": HIDDEN * INTER * 2 + INTER * 2 + 2 * HIDDEN * 2,
    }


def config2_layer(args, past=2048, repeats=20):
    """BASELINE config 2 on the GPU: one Llama-3.1-8B-shaped decoder layer,
    one decode token over a KV cache pre-filled at 2048 positions ~ N(0, 1),
    weights resident in HBM.  The layer (the runtime's four matrix_group
    units: q|k|v + RoPE + KV write, attention + o_proj, gate/up, down) is
    timed with events around runtime.run, the embedding gather and the LM
    head outside them; then each kernel group with its own events
    (Llama31DecodeExecutor.instrument)."""

    import torch
    from layer_streaming import (
        Llama31Config,
        Llama31DecodeExecutor,
        ResidentDeviceArena,
        ResidentTransformerRuntime,
        build_llama31_8b_plan,
    )

    dev = torch.device("cuda:0")
    plan = build_llama31_8b_plan("matrix_group", stream_vocab=False, num_layers=1)
    resident = ResidentDeviceArena(plan, None, dev, fill=False).fill_random(args.seed)
    runtime = ResidentTransformerRuntime(plan, None, resident, dev,
                                         synchronize=False).fill_random(args.seed)
    executor = Llama31DecodeExecutor(Llama31Config(num_hidden_layers=1), resident,
                                     top_k=10)
    executor.reserve(past + 2 * repeats + 8)
    cache = executor.kv_cache
    gen = torch.Generator(device=dev).manual_seed(args.seed + 2)
    cache.buffer[0, :, :, :past].normal_(generator=gen)
    cache.set_length(0, past)
    groups = ("qkv", "attention", "o_proj", "gate_up", "down_proj")
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    token = torch.tensor([[int(args.seed * 7919 % VOCAB)]], device=dev)
    layer_ms, attended = [], []
    log("config 2: one layer at KV {}".format(past))
    with torch.inference_mode():
        for phase in ("layer", "kernels"):
            if phase == "kernels":
                for group in groups:
                    executor.instrument(group, repeats)
            for step in range(repeats + (1 if phase == "layer" else 0)):
                state = executor.begin(token)
                start.record()
                state = runtime.run(executor, state)
                stop.record()
                state = executor.finish(state)
                token = state.topk_indices.reshape(1, -1)[:, :1]
                torch.cuda.synchronize(dev)
                if phase == "layer" and step:
                    layer_ms.append(start.elapsed_time(stop))
                    attended.append(cache.sequence_length())
    executor.check_errors()
    mean_attended = statistics.mean(attended)
    kernel_bytes = layer_kernel_bytes(mean_attended)
    kernels = {}
    for group in groups:
        times = executor.kernel_times_ms(group)
        avg_us = 1000.0 * statistics.mean(times)
        kernels[group] = {
            "avg_us": round(avg_us, 3),
            "bytes": int(kernel_bytes[group]),
            "gbps": round(kernel_bytes[group] / (avg_us * 1e-6) / 1e9, 1),
            "frac_of_peak": round(kernel_bytes[group] / (avg_us * 1e-6) / 1e9
                                  / HBM_PEAK_GBPS, 4),
        }
    kernels["attention"]["timing"] = ("one launch, split merge inside, between "
                                      "stream events (dispatch included)")
    layer_bytes = (436207616 + 2 * HIDDEN * 2 + 2 * mean_attended * 8 * 128 * 2
                   + 8 * 128 * 2 * 2)
    median = statistics.median(layer_ms)
    result = {
        "workload": "BASELINE config 2: one 8B-shaped decoder layer, weights "
                    "~ N(0,0.02) resident in HBM, KV pre-filled at {} positions "
                    "~ N(0,1), one decode token per step; 1 warm-up + {} timed "
                    "steps, then {} steps with per-kernel events".format(
                        past, repeats, repeats),
        "layer_us_median": round(1000.0 * median, 2),
        "layer_us_p10": round(1000.0 * percentiles(layer_ms)["p10"], 2),
        "layer_bytes": int(layer_bytes),
        "layer_gbps": round(layer_bytes / (median * 1e-3) / 1e9, 1),
        "layer_frac_of_peak": round(layer_bytes / (median * 1e-3) / 1e9
                                    / HBM_PEAK_GBPS, 4),
        "mean_attended": round(mean_attended, 1),
        "kernels": kernels,
    }
    del executor, runtime, resident, cache
    torch.cuda.empty_cache()
    return result


# ------------------------------------------------- config 5 (prefill)

# Prefill launch groups of the matrix granularity and their [N, K] shapes.
# The q / k / v projections share the "gemm_qkv" group (launch order q, k, v
# in every layer).
PREFILL_GEMMS = (
    ("q_proj", "gemm_qkv", 0, (HIDDEN, HIDDEN)),
    ("k_proj", "gemm_qkv", 1, (1024, HIDDEN)),
    ("v_proj", "gemm_qkv", 2, (1024, HIDDEN)),
    ("o_proj", "gemm_o", None, (HIDDEN, HIDDEN)),
    ("gate_proj", "gemm_gate", None, (INTER, HIDDEN)),
    ("up_proj", "gemm_up", None, (INTER, HIDDEN)),
    ("down_proj", "gemm_down", None, (HIDDEN, INTER)),
)


def unit_copy_gaps(runtime, plan):
    """Idle time of the copy engine between consecutive unit copies of the
    profiled call (copy i + 1's start event minus copy i's end event), in
    total and by the operation of the unit whose copy waited."""

    timing = runtime._timing_events()
    units = plan.units
    by_op = {}
    gaps = []
    timed = runtime._timed_copies  # units copied ahead of the call have no events
    for i in range(len(units) - 1):
        if i not in timed or i + 1 not in timed:
            continue
        gap = timing["copy_end"][i].elapsed_time(timing["copy_start"][i + 1])
        gaps.append(gap)
        op = units[i + 1].operation
        by_op[op] = by_op.get(op, 0.0) + gap
    return {"sum_ms": round(sum(gaps), 3),
            "max_ms": round(max(gaps), 3),
            "by_next_unit_ms": {k: round(v, 3) for k, v in sorted(by_op.items())}}


def prefill_streamed(args):
    """one 2048-token prefill in pinned_staging mode."""

    import torch
    from layer_streaming import (
        DoubleBufferRuntime,
        Llama31Config,
        Llama31DecodeExecutor,
        ResidentDeviceArena,
        VocabStreamingRuntime,
        build_llama31_8b_plan,
        create_weight_store,
    )

    dev = torch.device("cuda:0")
    tokens = args.prefill_tokens
    plan = build_llama31_8b_plan("matrix", stream_vocab=True)
    log("config 5: pageable {:.1f} GB arena, {} MiB slots".format(
        plan.host_arena_bytes / 1e9, plan.slot_bytes >> 20))
    store = create_weight_store(plan, "pinned_staging")
    store.fill_random(seed=args.seed, device=dev)
    resident = ResidentDeviceArena(plan, store, dev)
    runtime = DoubleBufferRuntime(plan, store, resident, dev)
    vocab = VocabStreamingRuntime(plan, store, runtime)
    executor = Llama31DecodeExecutor(Llama31Config(), resident, vocab_runtime=vocab,
                                     top_k=10)
    executor.reserve(tokens + 1)
    gen = torch.Generator().manual_seed(args.seed + 1)
    prompt = torch.randint(0, VOCAB, (1, tokens), generator=gen).to(dev)
    walls, profiles = [], []
    groups = {"gemm_qkv": 3 * LAYERS, "gemm_o": LAYERS, "gemm_gate": LAYERS,
              "gemm_up": LAYERS, "gemm_down": LAYERS,
              "prefill_attention": LAYERS}
    repeats = args.prefill_repeats
    profiled = None
    phases = []  # host ms of begin (embedding), run (the units), finish (LM head)
    head_profile = {}
    copy_gaps = {}
    with torch.inference_mode():
        # warm-up, timed prefills without timing events, then one prefill
        # with copy / unit events and every GEMM and attention launch timed
        for rep in range(1 + repeats + 1):
            executor.kv_cache.clear()
            last = rep == repeats + 1
            runtime.profile = vocab.profile = last
            if last:
                for name, count in groups.items():
                    executor.instrument(name, count)
            torch.cuda.synchronize(dev)
            t0 = time.perf_counter()
            state = executor.begin(prompt)
            t1 = time.perf_counter()
            state = runtime.run(executor, state)
            t2 = time.perf_counter()
            state = executor.finish(state)
            torch.cuda.synchronize(dev)
            t3 = time.perf_counter()
            wall = (t3 - t0) * 1000.0
            if rep and not last:
                phases.append(((t1 - t0) * 1e3, (t2 - t1) * 1e3, (t3 - t2) * 1e3))
            log("config 5: prefill {} {:.1f} ms{}".format(
                rep, wall, " (profiled)" if last else ""))
            if rep == 0:
                continue  # warm-up
            if last:
                profiled = wall
                profiles.append(runtime.last_profile)
                head_profile = dict(vocab.last_profile)
                copy_gaps = unit_copy_gaps(runtime, plan)
            else:
                walls.append(wall)
    times = {name: executor.kernel_times_ms(name) for name in groups}
    gemms = {}
    total_ms = 0.0
    for name, group, phase, (n, k) in PREFILL_GEMMS:
        ms = times[group]
        if phase is not None:
            ms = ms[phase::3]
        avg = statistics.mean(ms)
        total_ms += sum(ms)
        tflops = 2.0 * tokens * n * k / (avg * 1e-3) / 1e12
        gemms[name] = {"m_n_k": [tokens, n, k], "avg_us": round(1000 * avg, 1),
                       "tflops": round(tflops, 1),
                       "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4)}
    attn = times["prefill_attention"]
    attn_flops = 4.0 * 32 * 128 * tokens * (tokens + 1) / 2
    attn_tflops = attn_flops / (statistics.mean(attn) * 1e-3) / 1e12
    bytes_prefill = plan.stream_bytes_per_token + VOCAB * HIDDEN * 2
    median = statistics.median(walls)
    # the H2D roofline of this path: the prefill's transfers (224 matrix
    # units, 8 LM-head chunks) priced at the rate each size reaches alone,
    # copied from a pinned staging slot
    sizes = [u.nbytes for u in plan.units] + [
        (e - f) * HIDDEN * 2 for f, e in
        (plan.vocab.chunk_bounds(c) for c in range(plan.vocab.chunk_count))]
    pinned = store.staging_slots[0].view(-1)
    rates = copy_rates({n: pinned for n in sorted(set(sizes))},
                       runtime.copy_stream, runtime.device_slots[0])
    runtime.discard_slots()
    torch.cuda.synchronize(dev)
    ideal_ms = sum(n / 1e9 / rates[n] * 1e3 for n in sizes)
    result = {
        "workload": "BASELINE config 5: {}-token random-ID prompt, pinned_staging "
                    "(pageable arena + pinned staging slots), matrix granularity, "
                    "2 x {} MiB device slots, streamed vocab; 1 warm-up + {} "
                    "timed prefills + 1 profiled prefill (copy / kernel "
                    "events)".format(tokens, plan.slot_bytes >> 20, repeats),
        "prefill_ms_median": round(median, 2),
        "profiled_prefill_ms": round(profiled, 2),
        "prefill_ms_min": round(min(walls), 2),
        "prompt_tokens_per_s": round(tokens / (median / 1e3), 1),
        "h2d_bytes": bytes_prefill,
        "pcie_inclusive_gbps": round(bytes_prefill / 1e9 / (median / 1e3), 2),
        "isolated_copy_ms": round(ideal_ms, 2),
        "frac_of_isolated_copy_time": round(ideal_ms / median, 4),
        "isolated_copy_gbps_by_size": {size_label(n): round(r, 2)
                                       for n, r in sorted(rates.items())},
        "transformer_h2d_gbps_median": round(statistics.median(
            p["h2d_effective_gbps"] for p in profiles), 2),
        "transformer_compute_event_sum_ms": round(statistics.median(
            p["compute_event_sum_ms"] for p in profiles), 2),
        "staging_copy_sum_ms": round(statistics.median(
            p.get("staging_event_sum_ms", 0.0) for p in profiles), 1),
        "host_phase_ms_median": {
            name: round(statistics.median(ph[i] for ph in phases), 2)
            for i, name in enumerate(("begin_embedding", "run_units",
                                      "finish_lm_head"))},
        "lm_head_profiled": {k: round(head_profile[k], 3) for k in
                             ("pipeline_ms", "h2d_event_sum_ms",
                              "h2d_effective_gbps", "compute_event_sum_ms")
                             if k in head_profile},
        "transformer_gpu_pipeline_ms": round(statistics.median(
            p["gpu_pipeline_ms"] for p in profiles), 2),
        "unit_copy_gaps": copy_gaps,
        "gemm": gemms,
        "gemm_sum_ms": round(total_ms, 2),
        "gemm_tflops": round(2.0 * tokens * 218103808 * LAYERS / (total_ms * 1e-3)
                             / 1e12, 1),
        "attention": {"avg_us": round(1000 * statistics.mean(attn), 1),
                      "tflops": round(attn_tflops, 1),
                      "mfma_frac": round(attn_tflops / MFMA_BF16_PEAK_TFLOPS, 4)},
        "mfma_peak_tflops": MFMA_BF16_PEAK_TFLOPS,
        "last_token": int(state.topk_indices.reshape(-1)[0]),
    }
    store.close()
    del executor, vocab, runtime, resident, store
    torch.cuda.empty_cache()
    return result


# ------------------------------------------------------------ CPU baseline

CPU_DISTINCT_LAYERS = 4


def cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(args):
    """The CPU oracle on this host, per the reference's protocol (1 warm-up +
    ``--cpu-repeats`` repeats, p10 / median / p90):

    * config 4, the value: whole decode tokens -- 32 decoder layers at
      context 32768 then the final norm and the 128256-row LM head with
      top-10.  The layers cycle through 4 distinct sets of weights and KV
      cache (2.3 GB, several times any CPU cache), so no layer reads warm
      data, and the CPU's time equals that of 32 distinct layers;
    * config 1: the streamed-vocabulary LM head step (8 chunks, online top-10
      merge);
    * config 2: one decoder layer at context 2048.
    """

    import torch
    from oracle import llama_oracle as ref

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    gen = torch.Generator().manual_seed(5)

    def draw(shape, scale=0.02):
        t = torch.empty(shape, dtype=torch.bfloat16)
        return t.uniform_(-scale * 1.7, scale * 1.7, generator=gen)

    def layer_weights():
        return {"q": draw((4096, 4096)), "k": draw((1024, 4096)),
                "v": draw((1024, 4096)), "o": draw((4096, 4096)),
                "gate": draw((INTER, 4096)), "up": draw((INTER, 4096)),
                "down": draw((4096, INTER)),
                "ln1": torch.ones(4096, dtype=torch.bfloat16),
                "ln2": torch.ones(4096, dtype=torch.bfloat16)}

    ctx = args.context
    log("cpu baseline: drawing {} distinct layers at context {}".format(
        CPU_DISTINCT_LAYERS, ctx))
    layers = [(layer_weights(), {"k": draw((8, ctx, 128), 1.0),
                                 "v": draw((8, ctx, 128), 1.0)})
              for _ in range(CPU_DISTINCT_LAYERS)]
    head = draw((VOCAB, 4096))
    norm = torch.ones(4096, dtype=torch.bfloat16)
    inv = ref.llama3_inv_freq(128)
    cos, sin = ref.rope_cos_sin(inv, [ctx])

    def token(hidden):
        for layer in range(LAYERS):
            w, kv = layers[layer % CPU_DISTINCT_LAYERS]
            hidden = ref.decoder_layer(hidden, w, dict(kv), ctx, cos, sin, 1e-5)
        normalized = ref.rms_norm(hidden, norm, 1e-5)
        logits = ref.lm_head_logits(normalized[0], head)
        return ref.topk(logits, 10)

    def timed(fn, repeats):
        fn()  # warm-up
        out = []
        for _ in range(repeats):
            t0 = time.perf_counter()
            fn()
            out.append((time.perf_counter() - t0) * 1000.0)
        return percentiles(out)

    h = draw((1, 4096), 1.0)
    log("cpu baseline: config 4 tokens")
    config4 = timed(lambda: token(h), args.cpu_repeats)
    log("cpu baseline: config 1 LM head")
    config1 = timed(lambda: ref.streamed_lm_head(h[0], head, 16384, 10),
                    args.cpu_repeats)
    kv2 = {"k": layers[0][1]["k"][:, :2048].contiguous(),
           "v": layers[0][1]["v"][:, :2048].contiguous()}
    cos2, sin2 = ref.rope_cos_sin(inv, [2048])
    log("cpu baseline: config 2 layer")
    config2 = timed(lambda: ref.decoder_layer(h, layers[0][0], dict(kv2), 2048,
                                              cos2, sin2, 1e-5),
                    args.cpu_repeats)
    model = cpu_model()
    return {
        "value": round(config4["median"], 2),
        "unit": "ms/token",
        "cores": cores,
        "kind": "port",
        "cpu_model": model,
        "p10": round(config4["p10"], 2),
        "p90": round(config4["p90"], 2),
        "sample": "CPU oracle (torch bf16 ops, fp32 softmax, {} threads on {}): "
                  "BASELINE config 4 whole decode tokens, 1 warm-up + {} repeats "
                  "(32 layers at context {} cycling {} distinct weight / KV sets, "
                  "final norm, 128256-row LM head, top-10)".format(
                      cores, model, args.cpu_repeats, ctx, CPU_DISTINCT_LAYERS),
        "config1_lm_head_ms": {k: round(v, 2) for k, v in config1.items()},
        "config2_layer_ctx2048_ms": {k: round(v, 2) for k, v in config2.items()},
    }


def main():
    args = parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(--gpus {} requested); run with --gpus 1".format(args.gpus),
              file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    from layer_streaming import _hip

    _hip.load()
    if args.probe:
        counter_probe()
        return
    log("achievable HBM read bandwidth sweep")
    hbm = hbm_plateau()
    if args.hbm_only:
        print(json.dumps(hbm), flush=True)
        return
    resident = resident_decode(args)
    ms = resident["ms_per_step"]
    t_us = resident["timed_avg_us"]
    per_launch = gate_up_bytes()
    achieved = per_launch / (t_us * 1e-6) / 1e9
    token_gbps = resident["token_hbm_bytes"] / 1e9 / (ms / 1e3)
    line = {
        "metric": "decode ms/token, 8B-shape bf16 b=1; achieved HBM & H2D GB/s vs peak",
        "value": round(ms, 4),
        "unit": "ms/token",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) weights drawn in HBM; KV ~ N(0,1))",
        "config": {
            "workload": "BASELINE config 4: 32-layer Llama-3.1-8B-shaped model, "
                        "all weights HBM-resident, batch 1 greedy decode at "
                        "context {}".format(args.context),
            "context": args.context,
            "units": "matrix_group",
            "layer_launches": "5 per layer: q|k|v, attention (split merge inside), o_proj, gate/up, down",
            "batch": 1,
            "layers": LAYERS,
            "vocab": VOCAB,
            "parallelism": "single GPU",
        },
        "tokens_per_s": round(1000.0 / ms, 3),
        "token_hbm_gbps": round(token_gbps, 2),
        "token_hbm_frac_of_peak": round(token_gbps / HBM_PEAK_GBPS, 4),
        "token_hbm_frac_of_achievable": round(token_gbps / hbm["read_gbps"], 4),
        "hbm": hbm,
        "roofline": {
            "kernel": "gate_up_swiglu GEMV (gemv_kernel<8,2,4,kSwiglu>), "
                      "2x[14336,4096] bf16",
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": measured_traffic(TRAFFIC_FILE),
            "achievable": hbm["read_gbps"],
            "frac_of_achievable": round(achieved / hbm["read_gbps"], 4),
            "bytes_per_launch": int(per_launch),
            "avg_launch_us": round(t_us, 3),
            "median_launch_us": round(resident["timed_median_us"], 3),
            "launches_timed": resident["timed_launches"],
        },
    }
    if "decode_graph" in resident:
        line["decode_graph"] = resident["decode_graph"]
    if "prefill_resident" in resident:
        line["prefill_resident"] = resident["prefill_resident"]
    line["config1_lm_head_resident"] = resident["config1_lm_head_resident"]
    line["config2_layer"] = config2_layer(args)
    if not args.no_streamed:
        s = streamed_decode(args)
        line["streamed"] = {
            "workload": "BASELINE config 3: full_pinned, matrix_group, 2 x 224 MiB "
                        "slots, streamed vocab, 6-token prompt, 1 warm-up + {} "
                        "timed decodes + 2 profiled decodes (copy / unit "
                        "events)".format(args.streamed_steps),
            **{k: round(v, 4) if isinstance(v, float) else v for k, v in s.items()},
            "pcie_peak_gbps": PCIE_PEAK_GBPS,
        }
        line["comparable_to_reference"] = {
            "key": "streamed.ms_per_token_median",
            "this_ms_per_token": round(s["ms_per_token_median"], 3),
            "reference_ms_per_token": REFERENCE_STREAMED_MS,
            "reference_setup": "RTX 3080 Ti, PCIe Gen4 x16, full_pinned, "
                               "matrix_group, streamed vocab, 2 slots "
                               "(README.md:25-29); a different machine, so "
                               "vs_baseline stays null",
        }
    if not args.no_prefill:
        line["prefill"] = prefill_streamed(args)
        line["prefill_sweep"] = prefill_sweep(args)
        line["prefill_vs_vendor"] = prefill_vs_vendor()
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(args)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
