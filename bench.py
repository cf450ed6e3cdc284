#!/usr/bin/env python3
"""Decode benchmark of the MI355X layer_streaming path (one GPU).

Headline (the JSON ``value``): BASELINE config 4 -- the 32-layer
Llama-3.1-8B-shaped model with all 16 GB of bf16 weights resident in HBM,
batch 1, greedy decode at context 32768 (KV cache 4 GiB ~ N(0, 1), synthetic
N(0, 0.02) weights drawn on the device).  A step is one decode token; the
timed region covers exactly --steps tokens between two synchronisations,
inputs already resident in HBM.

Also reported (extra keys, not ``value``):
  * roofline of the dominant kernel (the fused gate/up SwiGLU GEMV, 224 MiB
    per launch), timed live in the timed region with HIP events bound to
    launches of the kernel on its stream (hipExtLaunchKernel start/stop
    events: kernel execution only; one launch per token, layer 16, by
    default, since a timed launch adds a few microseconds of queue time), HBM traffic per launch from the
    committed FETCH_SIZE / WRITE_SIZE counter summary;
  * decode_graph: config 4 again, the same number of steps continuing the
    same sequence, replayed as one HIP graph per token (the position held
    on the device; layer_streaming.DecodeGraph; skip: --no-decode-graph);
  * streamed: BASELINE config 3 -- full_pinned 16 GB host arena,
    matrix_group units through two 224 MiB slots, streamed vocabulary;
    decode ms/token and the PCIe-inclusive H2D GB/s, timed without copy /
    unit events, which two further decodes carry for the per-copy rates
    (skip: --no-streamed);
  * prefill: BASELINE config 5 -- a 2048-token random-ID prompt through the
    pinned_staging store with matrix granularity and the streamed
    vocabulary (pageable arena -> pinned staging slots -> two 128 MiB device
    slots), prefill ms and H2D GB/s timed without events, then one
    profiled prefill whose every GEMM / attention launch is bound to HIP
    events: per-matrix TFLOP/s and the fraction of the bf16 dense MFMA
    peak (skip: --no-prefill);
  * cpu_baseline: the CPU oracle on this host's cores on a bounded sample
    (skip: --no-cpu-baseline).

Config 4 runs the six per-stage kernels per layer by default; --layer-mode
mlp / one switch to the one-launch MLP half / whole layer
(cascade_decode_mlp_bf16 / cascade_decode_layer_bf16, on par with the
default), and the roofline then describes that launch.

Run: python bench.py [--steps K] [--warmup W] [--context L] [--layer-mode M]
"""

import argparse
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


def log(*parts):
    print("[bench]", *parts, file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=32)
    p.add_argument("--warmup", type=int, default=4)
    p.add_argument("--context", type=int, default=32768)
    p.add_argument("--layer-mode", default="stages", choices=("stages", "mlp", "one"),
                   help="config 4 launches per decoder layer: stages = six "
                        "per-stage kernels (matrix_group units); mlp = q|k|v and "
                        "attention per stage, o_proj..down_proj as one launch "
                        "(layer units); one = the whole layer as one launch")
    p.add_argument("--no-decode-graph", action="store_true",
                   help="config 4: skip the second timed run, which replays "
                        "the same number of decode steps as one HIP graph per "
                        "token (layer_streaming.DecodeGraph, per-stage "
                        "launches) after the eager timed steps")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--no-streamed", action="store_true")
    p.add_argument("--streamed-steps", type=int, default=7)
    p.add_argument("--no-prefill", action="store_true")
    p.add_argument("--prefill-tokens", type=int, default=2048)
    p.add_argument("--prefill-repeats", type=int, default=3)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-sample-seconds", type=float, default=15.0)
    p.add_argument("--roofline-stride", type=int, default=LAYERS,
                   help="time every N-th gate/up launch of the timed region "
                        "(default: one per token, layer 16; 1 = all; each "
                        "timed launch adds ~5 us of queue time)")
    p.add_argument("--probe", action="store_true",
                   help="only run the HBM-counter probe: 4 plain device copies "
                        "of 256 MiB, then 12 gate/up SwiGLU launches over 3 "
                        "rotating weight copies (for rocprofv3 --pmc runs)")
    return p.parse_args()


PROBE_COPY_BYTES = 256 << 20
TRAFFIC_FILE = ROOT / "profiles" / "gate_up_traffic.txt"
LAYER_TRAFFIC_FILE = ROOT / "profiles" / "decode_layer_traffic.txt"
MLP_TRAFFIC_FILE = ROOT / "profiles" / "decode_mlp_traffic.txt"


def counter_probe():
    """Known-size copies (counter calibration) then the dominant kernel."""

    import torch
    from layer_streaming import _hip

    dev = torch.device("cuda:0")
    src = torch.randn(PROBE_COPY_BYTES // 4, device=dev)
    dst = torch.empty_like(src)
    for _ in range(4):
        _hip.device_copy(dst, src)
    torch.cuda.synchronize(dev)
    log("probe: 4 device copies of {} bytes done".format(PROBE_COPY_BYTES))
    mats = [(torch.randn(INTER, HIDDEN, device=dev).mul_(0.02).to(torch.bfloat16),
             torch.randn(INTER, HIDDEN, device=dev).mul_(0.02).to(torch.bfloat16))
            for _ in range(3)]
    x = torch.randn(HIDDEN, device=dev).to(torch.bfloat16)
    norm = torch.ones(HIDDEN, dtype=torch.bfloat16, device=dev)
    y = torch.empty(INTER, dtype=torch.bfloat16, device=dev)
    for i in range(12):
        g, u = mats[i % 3]
        _hip.gate_up_swiglu(g, u, x, norm, 1e-5, y)
    torch.cuda.synchronize(dev)
    log("probe: 12 gate/up launches done")


def measured_traffic(path):
    """HBM bytes per launch from a committed counter summary."""

    try:
        for line in path.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch="):
                return int(line.split("=", 1)[1])
    except OSError:
        return None
    return None


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


def mlp_bytes():
    """Algorithmic HBM bytes of the one-launch MLP half of a layer: o_proj,
    gate, up and down weights, the post-attention norm weight, the attention
    output read, the hidden state read and written."""

    weights = HIDDEN * HIDDEN * 2 + 3 * INTER * HIDDEN * 2
    return weights + HIDDEN * 2 + HIDDEN * 2 + 2 * HIDDEN * 2


def layer_bytes(length):
    """Algorithmic HBM bytes of one decoder layer at attended length L:
    the seven weight matrices, two norm weights, K and V rows [0, L) read,
    the new K / V row written, the hidden state read and written."""

    weights = 436207616
    norms = 2 * HIDDEN * 2
    kv = length * KV_BYTES_PER_POS_LAYER + KV_BYTES_PER_POS_LAYER
    return weights + norms + kv + 2 * HIDDEN * 2


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
    granularity = "matrix_group" if args.layer_mode == "stages" else "layer"
    plan = build_llama31_8b_plan(granularity, stream_vocab=False)
    log("config 4: drawing 16 GB of synthetic weights in HBM")
    resident = ResidentDeviceArena(plan, None, dev, fill=False).fill_random(args.seed)
    runtime = ResidentTransformerRuntime(plan, None, resident, dev,
                                         synchronize=False).fill_random(args.seed)
    executor = Llama31DecodeExecutor(Llama31Config(), resident, top_k=10,
                                     layer_mode=args.layer_mode)
    total = args.context + args.warmup + args.steps + 1
    graphed = not args.no_decode_graph and args.layer_mode == "stages"
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
    with torch.inference_mode():
        for _ in range(args.warmup):
            state = executor.finish(runtime.run(executor, executor.begin(token)))
            token = state.topk_indices.reshape(1, -1)[:, :1]
        torch.cuda.synchronize(dev)
        # the dominant launch: the whole layer where it runs as one launch,
        # else the gate/up GEMV
        fused = executor._fused_ok is True
        group = {"one": "layer", "mlp": "mlp"}.get(args.layer_mode, "gate_up")
        group = group if fused else "gate_up"
        log("config 4: {} units, timing {} launches".format(granularity, group))
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
    timed_ms = executor.kernel_times_ms(group)
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
                "launches_per_step": "one graph replay (197 kernel nodes)",
                "last_token": int(decoder.tokens()[0, -1]),
            }
            decoder.close()
    mean_context = args.context + args.warmup + (args.steps - 1) / 2.0
    result = {
        "ms_per_step": ms_per_step,
        "tokens": args.steps,
        "timed_group": group,
        "units": granularity,
        "timed_launches": len(timed_ms),
        "timed_avg_us": 1000.0 * statistics.mean(timed_ms),
        "timed_median_us": 1000.0 * statistics.median(timed_ms),
        "mean_attended": mean_context + 1,
        "token_hbm_bytes": token_bytes(int(mean_context)),
        "last_token": int(token.reshape(-1)[0]),
    }
    if graph is not None:
        result["decode_graph"] = graph
    del executor, runtime, resident, cache
    torch.cuda.empty_cache()
    return result


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
    resident = ResidentDeviceArena(plan, store, dev)
    runtime = DoubleBufferRuntime(plan, store, resident, dev)
    vocab = VocabStreamingRuntime(plan, store, runtime)
    executor = Llama31DecodeExecutor(Llama31Config(), resident, vocab_runtime=vocab,
                                     top_k=10)
    prompt = torch.tensor([[128000, 791, 7438, 315, 2324, 374]], device=dev)
    walls, h2d, lm, profiled = [], [], [], []
    with torch.inference_mode():
        t0 = time.perf_counter()
        state = executor.finish(runtime.run(executor, executor.begin(prompt)))
        prefill_ms = (time.perf_counter() - t0) * 1000.0
        token = state.topk_indices[..., 0]
        # warm-up, timed decodes without timing events, then two decodes
        # with per-copy / per-unit events for the H2D and compute figures
        # (the events cost about 1% of the token)
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
    bytes_token = plan.stream_bytes_per_token + VOCAB * HIDDEN * 2 + HIDDEN * 2
    result = {
        "ms_per_token_median": statistics.median(walls),
        "ms_per_token_p10": sorted(walls)[max(0, int(0.1 * (len(walls) - 1)))],
        "ms_per_token_p90": sorted(walls)[int(0.9 * (len(walls) - 1))],
        "profiled_ms_per_token": statistics.median(profiled),
        "prefill_6_tokens_ms": prefill_ms,
        "h2d_bytes_per_token": bytes_token,
        "pcie_inclusive_gbps": bytes_token / 1e9 / (statistics.median(walls) / 1e3),
        "transformer_h2d_gbps_median": statistics.median(
            p["h2d_effective_gbps"] for p in h2d),
        "transformer_compute_event_sum_ms": statistics.median(
            p["compute_event_sum_ms"] for p in h2d),
        "lm_head_h2d_gbps_median": statistics.median(
            p["h2d_effective_gbps"] for p in lm),
        "lm_head_compute_event_sum_ms": statistics.median(
            p["compute_event_sum_ms"] for p in lm),
        "host_setup_s": setup_s,
    }
    store.close()
    del executor, vocab, runtime, resident, store
    torch.cuda.empty_cache()
    return result


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
    walls, profiles, staging = [], [], []
    groups = {"gemm_qkv": 3 * LAYERS, "gemm_o": LAYERS, "gemm_gate": LAYERS,
              "gemm_up": LAYERS, "gemm_down": LAYERS,
              "prefill_attention": LAYERS}
    repeats = args.prefill_repeats
    profiled = None
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
            state = executor.finish(runtime.run(executor, executor.begin(prompt)))
            torch.cuda.synchronize(dev)
            wall = (time.perf_counter() - t0) * 1000.0
            log("config 5: prefill {} {:.1f} ms{}".format(
                rep, wall, " (profiled)" if last else ""))
            if rep == 0:
                continue  # warm-up
            if last:
                profiled = wall
                profiles.append(runtime.last_profile)
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
        "transformer_h2d_gbps_median": round(statistics.median(
            p["h2d_effective_gbps"] for p in profiles), 2),
        "transformer_compute_event_sum_ms": round(statistics.median(
            p["compute_event_sum_ms"] for p in profiles), 2),
        "staging_copy_sum_ms": round(statistics.median(
            p.get("staging_event_sum_ms", 0.0) for p in profiles), 1),
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


def cpu_baseline(args):
    """The CPU oracle on this host: one decode token at context 32768 is
    timed as (32 x one decoder layer) + the full LM head, on a bounded
    sample of repeated layer steps."""

    import torch
    from oracle import llama_oracle as ref

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    gen = torch.Generator().manual_seed(5)

    def draw(shape, std=0.02):
        return (torch.randn(shape, generator=gen) * std).to(torch.bfloat16)

    w = {"q": draw((4096, 4096)), "k": draw((1024, 4096)), "v": draw((1024, 4096)),
         "o": draw((4096, 4096)), "gate": draw((INTER, 4096)),
         "up": draw((INTER, 4096)), "down": draw((4096, INTER)),
         "ln1": torch.ones(4096, dtype=torch.bfloat16),
         "ln2": torch.ones(4096, dtype=torch.bfloat16)}
    ctx = args.context
    kv = {"k": draw((8, ctx, 128), 1.0), "v": draw((8, ctx, 128), 1.0)}
    head = draw((VOCAB, 4096))
    inv = ref.llama3_inv_freq(128)
    cos, sin = ref.rope_cos_sin(inv, [ctx])
    h = draw((1, 4096), 1.0)
    layer_times = []
    deadline = time.perf_counter() + args.cpu_sample_seconds * 0.8
    while time.perf_counter() < deadline or len(layer_times) < 2:
        cache = dict(kv)
        t0 = time.perf_counter()
        ref.decoder_layer(h, w, cache, ctx, cos, sin, 1e-5)
        layer_times.append(time.perf_counter() - t0)
    t0 = time.perf_counter()
    logits = ref.lm_head_logits(h[0], head)
    ref.topk(logits, 10)
    head_s = time.perf_counter() - t0
    token_ms = (LAYERS * statistics.median(layer_times) + head_s) * 1000.0
    return {
        "value": token_ms,
        "unit": "ms/token",
        "cores": cores,
        "kind": "port",
        "sample": "CPU oracle (torch bf16 ops, fp32 softmax) on {} cores: {} "
                  "repeats of one full-width decoder layer at context {} "
                  "(median {:.1f} ms) x 32 layers + one 128256-row LM head "
                  "with top-10 ({:.1f} ms)".format(
                      cores, len(layer_times), ctx,
                      1000 * statistics.median(layer_times), 1000 * head_s),
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
    resident = resident_decode(args)
    ms = resident["ms_per_step"]
    t_us = resident["timed_avg_us"]
    if resident["timed_group"] == "mlp":
        kernel = ("decode_layer_kernel<true>: o_proj + residual, RMSNorm + "
                  "gate/up + SwiGLU, down_proj + residual of one layer in one launch")
        per_launch = mlp_bytes()
        traffic = measured_traffic(MLP_TRAFFIC_FILE)
    elif resident["timed_group"] == "layer":
        kernel = ("decode_layer_kernel: one decoder layer per launch (q|k|v, "
                  "attention, merge, o, gate/up, down), attended length {:.1f}"
                  .format(resident["mean_attended"]))
        per_launch = layer_bytes(resident["mean_attended"])
        traffic = measured_traffic(LAYER_TRAFFIC_FILE)
    else:
        kernel = "gate_up_swiglu GEMV (gemv_kernel<8,2,4,3,true>), 2x[14336,4096] bf16"
        per_launch = gate_up_bytes()
        traffic = measured_traffic(TRAFFIC_FILE)
    achieved = per_launch / (t_us * 1e-6) / 1e9
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
            "units": resident["units"],
            "layer_launches": {"stages": "6 per-stage kernels",
                               "mlp": "q|k|v, attention (+ split merge), one MLP launch",
                               "one": "one launch per layer"}[args.layer_mode],
            "batch": 1,
            "layers": LAYERS,
            "vocab": VOCAB,
            "parallelism": "single GPU",
        },
        "tokens_per_s": round(1000.0 / ms, 3),
        "token_hbm_gbps": round(resident["token_hbm_bytes"] / 1e9 / (ms / 1e3), 2),
        "token_hbm_frac_of_peak": round(
            resident["token_hbm_bytes"] / 1e9 / (ms / 1e3) / HBM_PEAK_GBPS, 4),
        "roofline": {
            "kernel": kernel,
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "bytes_per_launch": int(per_launch),
            "avg_launch_us": round(t_us, 3),
            "median_launch_us": round(resident["timed_median_us"], 3),
            "launches_timed": resident["timed_launches"],
        },
    }
    if "decode_graph" in resident:
        line["decode_graph"] = resident["decode_graph"]
    if not args.no_streamed:
        s = streamed_decode(args)
        line["streamed"] = {
            "workload": "BASELINE config 3: full_pinned, matrix_group, 2 x 224 MiB "
                        "slots, streamed vocab, 6-token prompt, 1 warm-up + {} "
                        "timed decodes + 2 profiled decodes (copy / unit "
                        "events)".format(args.streamed_steps),
            **{k: round(v, 3) if isinstance(v, float) else v for k, v in s.items()},
            "pcie_peak_gbps": PCIE_PEAK_GBPS,
        }
    if not args.no_prefill:
        line["prefill"] = prefill_streamed(args)
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(args)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
