"""The one-launch decoder layer (cascade_decode_layer_bf16) on the GPU.

Parity: every stage output of one decode step against the CPU oracle (the
north-star tolerance, or twice the oracle's own summation-order noise floor
for the bf16 hidden states, as the per-stage layer test), and q / k / v bit
for bit against the per-stage kernels.  Lengths cover the attention split
edges: one position, one and two 32-row blocks, splits of one and two blocks
with a last split holding a single position, and uneven splits.
"""

import pytest
import torch

import gpu_cases
from layer_streaming import _hip
from layer_streaming.llama31 import Llama31Config
from layer_streaming.rope import RopeTable, rope_parameters
from oracle import cases

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("past", [0, 31, 32, 1024, 2048, 4100])
def test_decode_layer_matches_oracle_and_per_stage(gpu_device, past):
    report = gpu_cases.run_layer_fused_case(seed=11 + past, past=past,
                                            device=gpu_device)
    if report is None:
        pytest.skip("device cannot run the one-launch layer (needs 256 CUs)")
    print(report, flush=True)
    assert report["ok"], report


def test_decode_layer_repeated_launches_are_identical(gpu_device):
    # 24 launches on one workspace: the barrier counters carry over from
    # launch to launch; every launch must give the same bits, and no barrier
    # may run out
    case = cases.layer_case(7, 300)
    dev = torch.device(gpu_device)
    ws = torch.zeros(_hip.decode_layer_workspace_bytes(), dtype=torch.uint8,
                     device=dev)
    first = gpu_cases.run_layer_fused_gpu(case, gpu_device, workspace=ws)
    if first is None:
        pytest.skip("device cannot run the one-launch layer (needs 256 CUs)")
    print("launch 0 error word", first["error"], flush=True)
    assert first["error"] == 0
    w = {k: case[k].to(dev) for k in ("q", "k", "v", "o", "gate", "up", "down",
                                      "ln1", "ln2")}
    n_kv, dim, past = case["n_kv_heads"], case["head_dim"], case["past"]
    capacity = past + 64
    k_cache = torch.zeros((n_kv, capacity, dim), dtype=torch.bfloat16, device=dev)
    v_cache = torch.zeros_like(k_cache)
    k_cache[:, :past].copy_(case["k_cache"].to(dev))
    v_cache[:, :past].copy_(case["v_cache"].to(dev))
    rope = RopeTable(dim, rope_parameters(Llama31Config()), dev, capacity)
    cos, sin = rope.row(past)
    x0 = case["x"].to(dev)
    outs = torch.empty((24, x0.numel()), dtype=torch.bfloat16, device=dev)
    for i in range(24):
        x = x0.clone()
        _hip.decode_layer(w, x, cos, sin, k_cache.view(-1), v_cache.view(-1),
                          capacity * dim, past + 1, ws, case["eps"], dim ** -0.5)
        outs[i].copy_(x)
    torch.cuda.synchronize(dev)
    print("24 launches done, error word", _hip.decode_layer_error(ws), flush=True)
    assert _hip.decode_layer_error(ws) == 0
    assert torch.equal(outs.cpu(), first["out"].expand(24, -1).contiguous())


@pytest.mark.parametrize("past", [0, 2048])
def test_decode_mlp_equals_per_stage_kernels(gpu_device, past):
    # q|k|v and attention per stage, then the one-launch MLP half: the hidden
    # state must equal the per-stage o_proj / gate_up / down path bit for bit
    # (same GEMV rows, same RMSNorm order), and match the oracle
    case = cases.layer_case(23 + past, past)
    staged = gpu_cases.run_layer_gpu(case, gpu_device)
    dev = torch.device(gpu_device)
    w = {k: case[k].to(dev) for k in ("o", "gate", "up", "down", "ln2")}
    ws = torch.zeros(_hip.decode_layer_workspace_bytes(), dtype=torch.uint8,
                     device=dev)
    x = case["x"].to(dev).clone()
    attn = staged["attn"].to(dev)
    print("decode_mlp past={}".format(past), flush=True)
    code = _hip.decode_mlp(w, attn, x, ws, case["eps"])
    if code != 0:
        pytest.skip("device cannot run the one-launch MLP (needs 256 CUs)")
    torch.cuda.synchronize(dev)
    inter = ws[_hip.DECODE_LAYER_INTER:_hip.DECODE_LAYER_INTER + 2 * 14336]
    assert _hip.decode_layer_error(ws) == 0
    assert torch.equal(inter.view(torch.bfloat16).cpu(), staged["inter"])
    assert torch.equal(x.cpu(), staged["out"])
    expected = cases.layer_expected(case)
    alternative = cases.layer_expected(case, cases.sgemm_linear)
    r = cases.within_noise_floor(x.cpu(), expected["out"], alternative["out"])
    assert r["ok"], r
