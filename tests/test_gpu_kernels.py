"""Kernel parity: every libcascade_hip kernel against the CPU oracle on
seeded inputs at the BASELINE shapes (bf16 weights, fp32 accumulation).

Tolerances: bf16 results within 1 bf16 ulp of the oracle (fp32 summation
order differs), composed results within |a-b| <= 2e-2 + 1e-2|b| (the
north-star logit tolerance); integer / index results bit-exact.
"""

import math

import pytest
import torch

import gpu_cases
from layer_streaming import _hip
from oracle import cases
from oracle import llama_oracle as ref

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def ulp_close(actual, expected, ulps=1):
    """|a - b| <= ulps * ulp_bf16(b) (ulp of 2^-7 relative, floor 1e-30)."""

    a = actual.float().cpu()
    b = expected.float().cpu()
    mag = b.abs().clamp_min(1e-30)
    ulp = torch.exp2(torch.floor(torch.log2(mag)) - 7)
    return bool(((a - b).abs() <= ulps * ulp + 1e-30).all())


def test_residual_add_rounding_is_torch_bf16(gpu_device):
    # W = I turns the GEMV into y = bf16(res + x): must equal torch's bf16 add
    n = 4096
    w = torch.eye(n, dtype=BF16)
    x = cases.normal_bf16((n,), 11, 3.0)
    res = cases.normal_bf16((n,), 12, 3.0)
    y = torch.empty(n, dtype=BF16, device=gpu_device)
    _hip.gemv_residual(w.to(gpu_device), x.to(gpu_device), res.to(gpu_device), y)
    assert torch.equal(y.cpu(), res + x)


@pytest.mark.parametrize(
    "n,k", [(4096, 4096), (6144, 4096), (4096, 14336), (1000, 4096),
            (100, 200), (3, 8), (1, 4096)])
def test_gemv_matches_oracle(gpu_device, n, k):
    print("gemv n={} k={}".format(n, k), flush=True)
    w = cases.normal_bf16((n, k), 21, 0.02)
    x = cases.normal_bf16((k,), 22)
    y = torch.empty(n, dtype=BF16, device=gpu_device)
    _hip.gemv(w.to(gpu_device), x.to(gpu_device), y)
    expected = ref.linear(x.reshape(1, -1), w).reshape(-1)
    assert ulp_close(y, expected)


@pytest.mark.parametrize("n,k", [(4096, 4096), (4096, 14336), (250, 520)])
def test_gemv_residual_matches_oracle(gpu_device, n, k):
    w = cases.normal_bf16((n, k), 31, 0.02)
    x = cases.normal_bf16((k,), 32)
    res = cases.normal_bf16((n,), 33)
    y = res.to(gpu_device)  # in place, as the executor uses it
    _hip.gemv_residual(w.to(gpu_device), x.to(gpu_device), y, y)
    expected = res.reshape(1, -1) + ref.linear(x.reshape(1, -1), w)
    r = cases.compare(y, expected)
    assert r["ok"], r


@pytest.mark.parametrize("rows,n", [(1, 4096), (6, 4096), (2, 256)])
def test_rmsnorm_matches_oracle(gpu_device, rows, n):
    x = cases.normal_bf16((rows, n), 41)
    w = cases.normal_bf16((n,), 42, 0.1, 1.0)
    y = torch.empty_like(x, device=gpu_device)
    _hip.rmsnorm(x.to(gpu_device), w.to(gpu_device), y, 1e-5)
    assert ulp_close(y, ref.rms_norm(x, w, 1e-5))


@pytest.mark.parametrize("position", [0, 1, 77, 2047, 8191, 32767, 32768])
def test_qkv_rope_matches_oracle(gpu_device, position):
    print("qkv_rope position={}".format(position), flush=True)
    case = cases.layer_case(51, 0)
    dev = gpu_device
    dim = 128
    x = case["x"].to(dev)
    capacity = position + 1
    kc = torch.zeros((8, capacity, dim), dtype=BF16, device=dev)
    vc = torch.zeros_like(kc)
    q = torch.empty(4096, dtype=BF16, device=dev)
    inv = ref.llama3_inv_freq(dim)
    cos, sin = ref.rope_cos_sin(inv, [position])
    _hip.qkv_rope(case["q"].to(dev), case["k"].to(dev), case["v"].to(dev), x,
                  case["ln1"].to(dev), 1e-5, cos[0, :64].contiguous().to(dev),
                  sin[0, :64].contiguous().to(dev), q,
                  kc.view(-1)[position * dim:], vc.view(-1)[position * dim:],
                  capacity * dim)
    n = ref.rms_norm(case["x"].reshape(1, -1), case["ln1"], 1e-5)
    eq = ref.apply_rope(ref.linear(n, case["q"]).view(1, 32, dim).transpose(0, 1), cos, sin)
    ek = ref.apply_rope(ref.linear(n, case["k"]).view(1, 8, dim).transpose(0, 1), cos, sin)
    ev = ref.linear(n, case["v"]).view(8, dim)
    for got, exp in ((q.cpu(), eq.reshape(-1)), (kc[:, position].cpu(), ek[:, 0]),
                     (vc[:, position].cpu(), ev)):
        r = cases.compare(got, exp)
        assert r["ok"], r
    # nothing but the new position was written
    if position:
        assert int(kc[:, :position].abs().sum()) == 0


def test_qkv_rope_split_matrices_equal_fused(gpu_device):
    # matrix granularity: q, k, v in three launches == one fused launch
    case = cases.layer_case(52, 0)
    dev = gpu_device
    dim, pos = 128, 5
    cos, sin = ref.rope_cos_sin(ref.llama3_inv_freq(dim), [pos])
    c, s = cos[0, :64].contiguous().to(dev), sin[0, :64].contiguous().to(dev)
    wq, wk, wv = (case[k].to(dev) for k in ("q", "k", "v"))
    x, ln = case["x"].to(dev), case["ln1"].to(dev)
    outs = []
    for split in (False, True):
        kc = torch.zeros((8, 16, dim), dtype=BF16, device=dev)
        vc = torch.zeros_like(kc)
        q = torch.zeros(4096, dtype=BF16, device=dev)
        kb, vb = kc.view(-1)[pos * dim:], vc.view(-1)[pos * dim:]
        if split:
            _hip.qkv_rope(wq, None, None, x, ln, 1e-5, c, s, q, None, None, 16 * dim)
            _hip.qkv_rope(None, wk, None, x, ln, 1e-5, c, s, None, kb, None, 16 * dim)
            _hip.qkv_rope(None, None, wv, x, ln, 1e-5, c, s, None, None, vb, 16 * dim)
        else:
            _hip.qkv_rope(wq, wk, wv, x, ln, 1e-5, c, s, q, kb, vb, 16 * dim)
        outs.append((q.cpu(), kc.cpu(), vc.cpu()))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("length,q_scale", [
    (1, 1), (2, 1), (17, 1), (32, 1), (33, 1), (64, 1), (65, 1), (129, 1),
    (1000, 1), (2048, 1), (2049, 1), (4100, 1), (8192, 1), (8193, 1),
    (32769, 1), (34000, 1),
    # sharp softmax: the running maximum moves between blocks and splits
    (4097, 8), (32769, 8)])
def test_decode_attention_matches_oracle(gpu_device, length, q_scale):
    print("attention length={} q_scale={}".format(length, q_scale), flush=True)
    dev = gpu_device
    dim = 128
    q = cases.normal_bf16((32, 1, dim), 61)
    if q_scale != 1:
        q = (q.float() * q_scale).to(BF16)
    k = cases.normal_bf16((8, length, dim), 62)
    v = cases.normal_bf16((8, length, dim), 63)
    capacity = length + 3
    kc = torch.zeros((8, capacity, dim), dtype=BF16, device=dev)
    vc = torch.zeros_like(kc)
    kc[:, :length].copy_(k.to(dev))
    vc[:, :length].copy_(v.to(dev))
    out = torch.empty(32 * dim, dtype=BF16, device=dev)
    ws = torch.zeros(_hip.attention_workspace_bytes(length), dtype=torch.uint8,
                     device=dev)
    _hip.decode_attention(q.reshape(-1).to(dev), kc.view(-1), vc.view(-1),
                          capacity * dim, length, out, ws, dim ** -0.5)
    expected = ref.attention(q, k, v, length - 1).reshape(-1)
    r = cases.compare(out, expected, atol=1e-2, rtol=1e-2)
    assert r["ok"], r
    # a second call on the same workspace gives the same bits
    out2 = torch.empty_like(out)
    _hip.decode_attention(q.reshape(-1).to(dev), kc.view(-1), vc.view(-1),
                          capacity * dim, length, out2, ws, dim ** -0.5)
    assert torch.equal(out.cpu(), out2.cpu())


def _attention_inputs(dev, length, capacity, q_scale, seed=71):
    dim = 128
    q = cases.normal_bf16((32 * dim,), seed)
    if q_scale != 1:
        q = (q.float() * q_scale).to(BF16)
    kc = torch.zeros((8, capacity, dim), dtype=BF16, device=dev)
    vc = torch.zeros_like(kc)
    kc[:, :length].copy_(cases.normal_bf16((8, length, dim), seed + 1).to(dev))
    vc[:, :length].copy_(cases.normal_bf16((8, length, dim), seed + 2).to(dev))
    return q.to(dev), kc, vc


@pytest.mark.parametrize("length,q_scale", [
    (225, 1), (256, 1), (300, 1), (2048, 1), (2049, 1), (32769, 1), (34000, 1),
    (4097, 8), (32769, 8)])
def test_fused_decode_attention_equals_two_launch_form(gpu_device, length, q_scale):
    # the split merge inside the attention launch reproduces the merge
    # launch's arithmetic: bit-identical outputs, counters back at zero
    print("fused attention length={} q_scale={}".format(length, q_scale), flush=True)
    dev = gpu_device
    capacity = length + 5
    q, kc, vc = _attention_inputs(dev, length, capacity, q_scale)
    stride = capacity * 128
    ws = torch.zeros(_hip.attention_workspace_bytes(length), dtype=torch.uint8,
                     device=dev)
    sync = torch.zeros(_hip.ATTENTION_SYNC_BYTES, dtype=torch.uint8, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    scale = 128 ** -0.5
    expected = torch.empty(32 * 128, dtype=BF16, device=dev)
    _hip.decode_attention(q, kc.view(-1), vc.view(-1), stride, length, expected,
                          ws, scale)
    for _ in range(2):  # a second call finds the counters it left at zero
        out = torch.empty_like(expected)
        _hip.decode_attention_fused(q, kc.view(-1), vc.view(-1), stride, length,
                                    out, ws, sync, err, scale)
        assert torch.equal(out.cpu(), expected.cpu())
        assert int(err.item()) == 0
        assert int(sync.count_nonzero().item()) == 0


@pytest.mark.parametrize("length_word", [1, 5, 224, 225, 4097, 33000])
def test_fused_decode_attention_at_equals_two_launch_form(gpu_device, length_word):
    print("fused attention at length word {}".format(length_word), flush=True)
    dev = gpu_device
    capacity = 33000
    q, kc, vc = _attention_inputs(dev, capacity, capacity, 1, seed=81)
    stride = capacity * 128
    ws = torch.zeros(_hip.attention_workspace_bytes(capacity), dtype=torch.uint8,
                     device=dev)
    sync = torch.zeros(_hip.ATTENTION_SYNC_BYTES, dtype=torch.uint8, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    length = torch.tensor([length_word], dtype=torch.int64, device=dev)
    scale = 128 ** -0.5
    expected = torch.empty(32 * 128, dtype=BF16, device=dev)
    out = torch.empty_like(expected)
    _hip.decode_attention_at(q, kc.view(-1), vc.view(-1), stride, length, capacity,
                             expected, ws, scale)
    _hip.decode_attention_fused_at(q, kc.view(-1), vc.view(-1), stride, length,
                                   capacity, out, ws, sync, err, scale)
    assert torch.equal(out.cpu(), expected.cpu())
    assert int(err.item()) == 0
    assert int(sync.count_nonzero().item()) == 0


def test_fused_decode_attention_flags_a_counter_left_set(gpu_device):
    # A counter left at 1 (a phantom arrival: the state an interrupted call
    # could leave) gives one ticket past the split count; the launch flags
    # it instead of merging silently, every workgroup exits, and once the
    # caller zero-fills the sync buffer the next call is exact again.
    dev = gpu_device
    length = 4097
    q, kc, vc = _attention_inputs(dev, length, length, 1, seed=91)
    stride = length * 128
    ws = torch.zeros(_hip.attention_workspace_bytes(length), dtype=torch.uint8,
                     device=dev)
    sync = torch.zeros(_hip.ATTENTION_SYNC_BYTES, dtype=torch.uint8, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    scale = 128 ** -0.5
    expected = torch.empty(32 * 128, dtype=BF16, device=dev)
    _hip.decode_attention(q, kc.view(-1), vc.view(-1), stride, length, expected,
                          ws, scale)
    sync.view(torch.int32)[0] = 1  # KV head 0's arrival counter
    out = torch.empty_like(expected)
    _hip.decode_attention_fused(q, kc.view(-1), vc.view(-1), stride, length, out,
                                ws, sync, err, scale)
    torch.cuda.synchronize(dev)
    assert int(err.item()) & _hip.ATTN_EPLACEMENT
    sync.zero_()
    err.zero_()
    _hip.decode_attention_fused(q, kc.view(-1), vc.view(-1), stride, length, out,
                                ws, sync, err, scale)
    assert torch.equal(out.cpu(), expected.cpu())
    assert int(err.item()) == 0


def test_fused_decode_attention_rejects_unsupported_shapes(gpu_device):
    dev = gpu_device
    q, kc, vc = _attention_inputs(dev, 300, 300, 1)
    ws = torch.zeros(_hip.attention_workspace_bytes(300), dtype=torch.uint8, device=dev)
    sync = torch.zeros(_hip.ATTENTION_SYNC_BYTES, dtype=torch.uint8, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    out = torch.empty(32 * 128, dtype=BF16, device=dev)
    with pytest.raises(ValueError):  # 7 splits: fewer than one per merger
        _hip.decode_attention_fused(q, kc.view(-1), vc.view(-1), 300 * 128, 224, out,
                                    ws, sync, err, 0.1)
    # the C entry point refuses the same call with nothing launched
    lib = _hip.load()
    rc = lib.cascade_decode_attention_fused_bf16(
        q.data_ptr(), kc.data_ptr(), vc.data_ptr(), 300 * 128, 224, 32, 8, 128, 0.1,
        out.data_ptr(), ws.data_ptr(), ws.numel(), sync.data_ptr(), err.data_ptr(), None)
    assert rc == _hip.ESHAPE
    with pytest.raises(ValueError):  # a sync buffer short of one line per head
        _hip.decode_attention_fused(q, kc.view(-1), vc.view(-1), 300 * 128, 300, out,
                                    ws, sync[:512], err, 0.1)
    assert int(sync.count_nonzero().item()) == 0 and int(err.item()) == 0


def test_attention_single_position_is_value_row(gpu_device):
    # softmax over one position is 1: the output is V itself (bit-exact)
    dev = gpu_device
    q = cases.normal_bf16((32 * 128,), 64)
    v = cases.normal_bf16((8, 1, 128), 65)
    kc = cases.normal_bf16((8, 1, 128), 66).to(dev)
    out = torch.empty(32 * 128, dtype=BF16, device=dev)
    ws = torch.zeros(_hip.attention_workspace_bytes(1), dtype=torch.uint8, device=dev)
    _hip.decode_attention(q.to(dev), kc.view(-1), v.to(dev).view(-1), 128, 1, out,
                          ws, 128 ** -0.5)
    expected = v[:, 0].repeat_interleave(4, dim=0).reshape(-1)
    assert torch.equal(out.cpu(), expected)


def test_swiglu_fused_and_split_match_oracle(gpu_device):
    dev = gpu_device
    case = cases.layer_case(71, 0)
    x = case["x"].to(dev)
    ln = case["ln2"].to(dev)
    wg, wu = case["gate"].to(dev), case["up"].to(dev)
    n = ref.rms_norm(case["x"].reshape(1, -1), case["ln2"], 1e-5)
    gate = torch.nn.functional.silu(ref.linear(n, case["gate"]))
    expected = (gate * ref.linear(n, case["up"])).reshape(-1)
    fused = torch.empty(14336, dtype=BF16, device=dev)
    _hip.gate_up_swiglu(wg, wu, x, ln, 1e-5, fused)
    assert cases.compare(fused, expected)["ok"]
    g = torch.empty(14336, dtype=BF16, device=dev)
    split = torch.empty(14336, dtype=BF16, device=dev)
    _hip.gate_silu(wg, x, ln, 1e-5, g)
    _hip.up_mul(wu, x, ln, 1e-5, g, split)
    assert ulp_close(g, gate.reshape(-1))
    assert torch.equal(fused.cpu(), split.cpu())


@pytest.mark.parametrize("past", [0, 2048])
def test_decoder_layer_config2(gpu_device, past):
    report = gpu_cases.run_layer_case(seed=3 + past, past=past, device=gpu_device)
    print(report, flush=True)
    assert report["ok"], report


@pytest.mark.parametrize(
    "rows,chunk,top_k",
    [(128256, 16384, 10), (128256, 128256, 10), (16384, 16384, 1),
     (16384, 16384, 64), (13568, 16384, 10), (37, 16384, 10), (1000, 100, 7)])
def test_lm_head_topk_matches_oracle(gpu_device, rows, chunk, top_k):
    report = gpu_cases.run_lm_head_case(seed=rows % 97, rows=rows,
                                        chunk_rows=chunk, top_k=top_k,
                                        device=gpu_device)
    print(report, flush=True)
    assert report["ok"], report


def test_lm_head_fewer_rows_than_top_k(gpu_device):
    # 5 rows, top-10: the 5 real entries in order, then -inf / -1
    case = cases.lm_head_case(4, 5)
    values, indices, logits = gpu_cases.run_lm_head_gpu(case, 16384, 10,
                                                        gpu_device)
    ev, ei = ref.topk(logits, 5)
    assert torch.equal(indices[:5], ei) and torch.equal(values[:5], ev)
    assert indices[5:].tolist() == [-1] * 5
    assert bool(torch.isinf(values[5:]).all())


@pytest.mark.parametrize("rows,top_k", [(128256, 10), (5, 10), (3000, 1),
                                         (65536, 64)])
def test_topk_f32_matches_oracle(gpu_device, rows, top_k):
    # top-k of a row of logits already in memory (the resident finish after
    # its GEMM over every position): exact ties, -0.0 / +0.0 and fewer rows
    # than top_k; the workspace is left dirty (no zero-fill is needed)
    g = torch.Generator().manual_seed(rows + top_k)
    logits = torch.randn(rows, generator=g)
    logits[::7] = logits[min(3, rows - 1)].item()
    if rows > 8:
        logits[1] = -0.0
        logits[2] = 0.0
    dev = gpu_device
    ws = torch.full((_hip.lm_head_workspace_bytes(rows, top_k),), 0xAB,
                    dtype=torch.uint8, device=dev)
    values = torch.empty(top_k, dtype=torch.float32, device=dev)
    indices = torch.empty(top_k, dtype=torch.int64, device=dev)
    _hip.topk_f32(logits.to(dev), top_k, ws, values, indices)
    n = min(rows, top_k)
    ev, ei = ref.topk(logits, n)
    assert torch.equal(indices[:n].cpu(), ei)
    assert torch.equal(values[:n].cpu(), ev)
    if n < top_k:
        assert indices[n:].cpu().tolist() == [-1] * (top_k - n)
        assert bool(torch.isinf(values[n:].cpu()).all())


def test_lm_head_ties_break_to_lower_index(gpu_device):
    # duplicated rows give exactly equal logits: order must be index-ascending
    dev = gpu_device
    base = cases.normal_bf16((64, 4096), 81, 0.02)
    w = base.repeat(40, 1)  # 2560 rows, every logit appears 40 times
    h = cases.normal_bf16((4096,), 82)
    ws = torch.zeros(_hip.lm_head_workspace_bytes(1024, 10), dtype=torch.uint8,
                     device=dev)
    values = torch.empty(10, dtype=torch.float32, device=dev)
    indices = torch.empty(10, dtype=torch.int64, device=dev)
    logits = torch.empty(2560, dtype=torch.float32, device=dev)
    wd, hd = w.to(dev), h.to(dev)
    for c, start in enumerate(range(0, 2560, 1024)):
        end = min(start + 1024, 2560)
        _hip.lm_head_topk(wd[start:end], hd, 10, start, c == 0, ws, values,
                          indices, logits_out=logits[start:end])
    best = int(torch.argmax(logits[:64].cpu()))
    expected = [best + 64 * i for i in range(10)]
    assert indices.cpu().tolist() == expected
    ev, ei = ref.topk(logits.cpu(), 10)
    assert torch.equal(indices.cpu(), ei)


def test_embedding_gather(gpu_device):
    dev = gpu_device
    table = cases.normal_bf16((1000, 4096), 91).to(dev)
    ids = torch.tensor([3, 999, 0, 3, 1000, -1], dtype=torch.int64, device=dev)
    out = torch.empty((6, 4096), dtype=BF16, device=dev)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    _hip.embedding_gather(table, ids, out, flag)
    out, table_cpu = out.cpu(), table.cpu()
    for i, idx in enumerate([3, 999, 0, 3]):
        assert torch.equal(out[i], table_cpu[idx])
    assert int(out[4:].abs().sum()) == 0
    assert int(flag.item()) == 1


def test_argument_errors_raise(gpu_device):
    dev = gpu_device
    w = torch.zeros((16, 4096), dtype=BF16, device=dev)
    x = torch.zeros(4096, dtype=BF16, device=dev)
    y = torch.zeros(16, dtype=BF16, device=dev)
    with pytest.raises(ValueError):
        _hip.gemv(w, x.cpu(), y)  # host tensor never reaches a kernel
    with pytest.raises(_hip.HipCallError):  # misaligned: rejected, no launch
        _hip.call("cascade_gemv_bf16", w.data_ptr() + 2, x.data_ptr(),
                  y.data_ptr(), 16, 4096, _hip.stream_handle())
    ws = torch.zeros(8, dtype=torch.uint8, device=dev)
    with pytest.raises(_hip.HipCallError):
        _hip.decode_attention(torch.zeros(4096, dtype=BF16, device=dev),
                              torch.zeros(8 * 4096 * 128, dtype=BF16, device=dev),
                              torch.zeros(8 * 4096 * 128, dtype=BF16, device=dev),
                              4096 * 128, 4096, torch.zeros(4096, dtype=BF16, device=dev),
                              ws, 0.1)


def test_hbm_read_and_copy_kernels(gpu_device):
    dev = gpu_device
    src = torch.arange(1 << 20, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    sink = torch.zeros(1, dtype=torch.float32, device=dev)
    _hip.device_copy(dst, src)
    _hip.hbm_read(src, sink)
    torch.cuda.synchronize(dev)
    assert torch.equal(dst, src)
    assert math.isfinite(float(sink.item()))
