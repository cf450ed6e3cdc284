"""The run_llama31 CLI end to end on the GPU (the reference's
tools/run_llama31.py:27-154 flags and JSON result), with seeded synthetic
weights on 2 full-width layers: the MFMA prefill of the prompt, then greedy
decode through the two-slot pipeline and the streamed vocabulary.

The same seeded weights go through every store mode and granularity; the
kernels of the matrix granularity (split q / k / v, gate / up halves) are
bit-identical to the fused ones, so the greedy tokens must agree exactly.
"""

import pytest

pytestmark = pytest.mark.gpu

# keys of the reference CLI's JSON result (tools/run_llama31.py:125-154)
RESULT_KEYS = {
    "model_id", "checkpoint", "weight_store", "granularity", "vocab_mode",
    "top_k", "prompt_tokens", "generated_tokens", "generated_ids",
    "generated_text", "checkpoint_load_seconds", "decode_token_latencies_ms",
    "runtime", "cpu_pinned_bytes", "vocab_extra_pinned_cpu_bytes", "plan",
    "cuda_peak_allocated_bytes",
}


def run_cli(tmp_path, *flags):
    from tools import run_llama31

    out = tmp_path / "result.json"
    argv = ["--random-init", "--seed", "3", "--layers", "2",
            "--max-new-tokens", "3", "--output", str(out), *flags]
    print("run_llama31", " ".join(argv), flush=True)
    result = run_llama31.main(argv)
    assert out.exists()
    return result


def test_cli_tokens_agree_across_modes(gpu_device, tmp_path):
    a = run_cli(tmp_path, "--weight-store", "full_pinned",
                "--granularity", "matrix_group", "--vocab-mode", "streamed")
    b = run_cli(tmp_path, "--weight-store", "pinned_staging",
                "--granularity", "matrix", "--vocab-mode", "streamed")
    c = run_cli(tmp_path, "--weight-store", "full_pinned",
                "--granularity", "layer", "--vocab-mode", "resident")
    for r in (a, b, c):
        assert RESULT_KEYS <= set(r), RESULT_KEYS - set(r)
        assert r["prompt_tokens"] == 6 and r["generated_tokens"] == 3
        assert len(r["generated_ids"]) == 3
        assert len(r["decode_token_latencies_ms"]) == 2
    print("generated", a["generated_ids"], b["generated_ids"], c["generated_ids"],
          flush=True)
    assert a["generated_ids"] == b["generated_ids"] == c["generated_ids"]
    assert b["cpu_pinned_bytes"] < a["cpu_pinned_bytes"]  # staging pins 2 slots only


def test_cli_decode_graph_equals_eager(gpu_device, tmp_path):
    # weights resident, decode as graph replays: the same kernels at the same
    # split plan as the eager resident-vocabulary run, so the same tokens
    eager = run_cli(tmp_path, "--granularity", "matrix_group", "--vocab-mode",
                    "resident", "--max-new-tokens", "5")
    graph = run_cli(tmp_path, "--granularity", "matrix_group", "--vocab-mode",
                    "resident", "--max-new-tokens", "5", "--decode-graph")
    print("eager", eager["generated_ids"], "graph", graph["generated_ids"],
          flush=True)
    assert graph["generated_ids"] == eager["generated_ids"]
    assert len(graph["generated_ids"]) == 5
    assert len(graph["decode_token_latencies_ms"]) == 3
    assert graph["decode_graph_setup_ms"] > 0
