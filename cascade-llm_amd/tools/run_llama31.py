#!/usr/bin/env python3
"""Run Llama-3.1-8B-shaped weights through the streaming runtime.

Same flags and JSON result as the reference CLI (tools/run_llama31.py:27-154):
--checkpoint --prompt --max-new-tokens --weight-store --granularity
--vocab-mode --top-k --device --output.  Without a checkpoint directory
(there is none on the GPU hosts) use --random-init: seeded synthetic weights
(--seed), prompt ids from --prompt-ids, optionally fewer decoder layers
(--layers) for quick runs.

--decode-graph (not in the reference) keeps every weight resident in HBM
and, after the prefill, decodes by replaying one captured HIP graph per
token (layer_streaming.DecodeGraph; needs --vocab-mode resident).  Its
decode_token_latencies_ms lists the replays; the first decode step runs
eagerly while the graph is captured (decode_graph_setup_ms).
"""

import argparse
import json
import sys
import time
from pathlib import Path

import torch

PACKAGE_ROOT = Path(__file__).resolve().parents[1]
if str(PACKAGE_ROOT) not in sys.path:
    sys.path.insert(0, str(PACKAGE_ROOT))

from layer_streaming import (  # noqa: E402
    DecodeGraph,
    DoubleBufferRuntime,
    Llama31Config,
    Llama31DecodeExecutor,
    ResidentDeviceArena,
    ResidentTransformerRuntime,
    VocabStreamingRuntime,
    build_llama31_8b_plan,
    create_weight_store,
)


def parse_args(argv=None):
    parser = argparse.ArgumentParser()
    parser.add_argument("--checkpoint", type=Path)
    parser.add_argument("--prompt", default="The meaning of life is")
    parser.add_argument("--max-new-tokens", type=int, default=8)
    parser.add_argument("--weight-store", choices=("full_pinned", "pinned_staging"),
                        default="full_pinned")
    parser.add_argument("--granularity", choices=("matrix", "matrix_group", "layer"),
                        default="matrix_group")
    parser.add_argument("--vocab-mode", choices=("resident", "streamed"),
                        default="streamed")
    parser.add_argument("--top-k", type=int, default=10)
    parser.add_argument("--device", default="cuda:0")
    parser.add_argument("--output", type=Path)
    parser.add_argument("--random-init", action="store_true",
                        help="seeded synthetic weights instead of a checkpoint")
    parser.add_argument("--seed", type=int, default=0)
    parser.add_argument("--layers", type=int, default=32)
    parser.add_argument("--prompt-ids", default="128000,791,7438,315,2324,374",
                        help="comma-separated prompt ids for --random-init")
    parser.add_argument("--decode-graph", action="store_true",
                        help="weights resident in HBM; decode by replaying one "
                             "captured HIP graph per token (needs --vocab-mode "
                             "resident)")
    args = parser.parse_args(argv)
    if args.checkpoint is None and not args.random_init:
        parser.error("either --checkpoint or --random-init is required")
    if args.decode_graph and args.vocab_mode != "resident":
        parser.error("--decode-graph needs --vocab-mode resident")
    return args


def main(argv=None):
    args = parse_args(argv)
    if args.max_new_tokens <= 0:
        raise SystemExit("--max-new-tokens must be positive")
    if not torch.cuda.is_available():
        raise SystemExit("no HIP device is available")

    tokenizer = None
    if args.checkpoint is not None:
        from transformers import AutoConfig, AutoTokenizer

        config = AutoConfig.from_pretrained(args.checkpoint, local_files_only=True)
        tokenizer = AutoTokenizer.from_pretrained(args.checkpoint,
                                                  local_files_only=True)
        tied = bool(config.tie_word_embeddings)
    else:
        config = Llama31Config(num_hidden_layers=args.layers)
        tied = False
    plan = build_llama31_8b_plan(args.granularity, tie_word_embeddings=tied,
                                 stream_vocab=(args.vocab_mode == "streamed"),
                                 num_layers=config.num_hidden_layers)
    store = create_weight_store(plan, args.weight_store)
    load_started = time.perf_counter()
    if args.checkpoint is not None:
        store.load_checkpoint(args.checkpoint)
    else:
        store.fill_random(seed=args.seed, device=args.device)
    load_seconds = time.perf_counter() - load_started

    device = torch.device(args.device)
    torch.cuda.set_device(device)
    resident = ResidentDeviceArena(plan, store, device)
    if args.decode_graph:
        runtime = ResidentTransformerRuntime(plan, store, resident, device,
                                             synchronize=False)
    else:
        runtime = DoubleBufferRuntime(plan, store, resident, device)
    vocab_runtime = None
    if plan.vocab is not None:
        vocab_runtime = VocabStreamingRuntime(plan, store, runtime)
    executor = Llama31DecodeExecutor(config, resident, vocab_runtime=vocab_runtime,
                                     top_k=args.top_k)
    if tokenizer is not None:
        input_ids = tokenizer(args.prompt, return_tensors="pt",
                              add_special_tokens=True).input_ids.to(device)
    else:
        ids = [int(t) for t in args.prompt_ids.split(",") if t.strip()]
        input_ids = torch.tensor([ids], device=device)

    generated = []
    token_latencies = []
    graph_setup_ms = None
    with torch.inference_mode():
        state = executor.begin(input_ids)
        state = runtime.run(executor, state)
        state = executor.finish(state)
        next_token = state.topk_indices[..., 0]
        generated.append(next_token)
        eager_steps = args.max_new_tokens - 1
        if args.decode_graph and args.max_new_tokens >= 3:
            started = time.perf_counter()
            graph = DecodeGraph(executor, runtime, next_token, args.max_new_tokens - 1)
            torch.cuda.synchronize(device)
            graph_setup_ms = (time.perf_counter() - started) * 1000.0
            for _ in range(args.max_new_tokens - 2):
                started = time.perf_counter()
                graph.step()
                torch.cuda.synchronize(device)
                token_latencies.append((time.perf_counter() - started) * 1000.0)
            graph.check()
            generated.append(graph.tokens())
            graph.close()
            eager_steps = 0
        for _ in range(eager_steps):
            started = time.perf_counter()
            state = executor.begin(next_token)
            state = runtime.run(executor, state)
            state = executor.finish(state)
            next_token = state.topk_indices[..., 0]
            # the token is on the device once the caller's stream is done;
            # a device-wide synchronise would also wait for the copies the
            # streamed runtime already runs for the next token
            torch.cuda.current_stream(device).synchronize()
            token_latencies.append((time.perf_counter() - started) * 1000.0)
            generated.append(next_token)

    generated_ids = torch.cat(generated, dim=-1).cpu()
    text = (tokenizer.decode(generated_ids[0], skip_special_tokens=True)
            if tokenizer is not None else None)
    result = {
        "model_id": plan.model_id,
        "checkpoint": str(args.checkpoint) if args.checkpoint else None,
        "random_init_seed": None if args.checkpoint else args.seed,
        "weight_store": args.weight_store,
        "granularity": args.granularity,
        "vocab_mode": args.vocab_mode,
        "top_k": args.top_k,
        "prompt_tokens": int(input_ids.numel()),
        "generated_tokens": args.max_new_tokens,
        "generated_ids": generated_ids[0].tolist(),
        "generated_text": text,
        "checkpoint_load_seconds": load_seconds,
        "decode_token_latencies_ms": token_latencies,
        "decode_graph_setup_ms": graph_setup_ms,
        "runtime": runtime.stats.as_dict(),
        "cpu_pinned_bytes": store.pinned_cpu_bytes,
        "vocab_extra_pinned_cpu_bytes": (
            vocab_runtime.extra_pinned_cpu_bytes if vocab_runtime is not None else 0
        ),
        "plan": {
            "host_arena_bytes": plan.host_arena_bytes,
            "stream_bytes_per_token": plan.stream_bytes_per_token,
        },
        "cuda_peak_allocated_bytes": torch.cuda.max_memory_allocated(device),
    }
    rendered = json.dumps(result, indent=2, ensure_ascii=False)
    if args.output is not None:
        args.output.parent.mkdir(parents=True, exist_ok=True)
        args.output.write_text(rendered + "\n", encoding="utf-8")
    print(rendered)
    store.close()
    return result


if __name__ == "__main__":
    main()
