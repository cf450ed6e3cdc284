"""Prefill kernels (S > 1 token rows): the MFMA GEMM family and causal GQA
attention against the CPU oracle on seeded inputs.

Tolerances: a bf16 GEMM result is a bf16 rounding of an fp32 accumulation,
so it must lie within one bf16 ulp plus an fp32 accumulation bound of the
float64 product of the same bf16 operands:
    |y - exact| <= ulp_bf16(exact) + 2^-22 * sum_k |x_k w_k|
(the oracle's F.linear is held to the same bound in the same test, so the
bound pins nothing that a correct CPU restatement would fail); fp32 logits
within 1e-4 absolute + 1e-4 relative of a float64 product; composed bf16
results
(residual, SwiGLU, RoPE, attention) within the north-star bound
|a - b| <= 2e-2 + 1e-2 |b| (attention: 1e-2 + 1e-2 |b|, as the decode
kernel's test); integer placement (which KV slots are written) exact.
"""

import pytest
import torch
import torch.nn.functional as F

from layer_streaming import _hip
from oracle import cases
from oracle import llama_oracle as ref

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
DIM = 128


def linear_bound_report(actual, x, w):
    """Worst ratio of |actual - exact| to ulp_bf16(exact) + 2^-22 sum|x w|."""

    exact = ref.linear_exact(x, w)
    absdot = x.float().abs() @ w.float().abs().t()
    mag = exact.abs().clamp_min(1e-30)
    ulp = torch.exp2(torch.floor(torch.log2(mag)) - 7)
    bound = ulp + absdot.double() * 2.0 ** -22
    ratio = (actual.double().cpu().reshape(exact.shape) - exact).abs() / bound
    return float(ratio.max())


@pytest.mark.parametrize("m,n,k", [
    (2048, 4096, 4096), (6, 6144, 4096), (130, 1024, 4096), (2, 128, 64),
    (257, 4096, 14336), (1, 256, 4096), (300, 28672, 4096),
    (5, 1000, 4096), (129, 200, 128), (7, 1001, 128),
    (2048, 4096, 192), (2048, 4096, 320), (2048, 1024, 384),
    (2048, 1024, 448), (40, 512, 1088), (16, 4096, 4096), (11, 1024, 14336),
    (17, 384, 4096), (64, 4096, 4096), (65, 1024, 4096), (128, 4096, 14336),
    (192, 14336, 256), (256, 14336, 192)])
def test_gemm_matches_oracle(gpu_device, m, n, k):
    # m <= 16 and m <= 64: the two skinny kernels; m <= 256 over at most 64
    # column pairs per 64-row block: blocks of the 64-row skinny kernel
    # (130 x 1024, 128 x 4096, 65 x 1024, 129 x 200); else tiles (128-row
    # tiles short of a round where 64-row ones would take two: 192 / 256 x
    # 14336);
    # n = 1001: rows not 16-byte aligned, the element-wise epilogue runs.
    # Slab counts (K / 64): odd and even counts (1, 2, 3, 5, 6, 7, 17, 64,
    # 224) below and above the ring depth of each tile shape (256-row
    # tiles: 3 buffers; 128-row: 4; 64-row: 6)
    print("gemm m={} n={} k={}".format(m, n, k), flush=True)
    dev = gpu_device
    x = cases.normal_bf16((m, k), 101)
    w = cases.normal_bf16((n, k), 102, 0.02)
    y = torch.empty((m, n), dtype=BF16, device=dev)
    _hip.gemm(x.to(dev), w.to(dev), y)
    oracle = ref.linear(x, w)
    gpu_ratio = linear_bound_report(y, x, w)
    oracle_ratio = linear_bound_report(oracle, x, w)
    print("bound ratio gpu {:.3f} oracle {:.3f}".format(gpu_ratio, oracle_ratio),
          flush=True)
    assert oracle_ratio <= 1.0
    assert gpu_ratio <= 1.0
    # and against the oracle itself
    r = cases.compare(y, oracle)
    assert r["ok"], r


@pytest.mark.parametrize("m", [3, 16, 40, 64])
def test_skinny_single_fragment_equals_column_pairs(gpu_device, m):
    # At N = 4096 the short-prompt kernels give each 16-column fragment its
    # own workgroup (the column pairs would fill half the CUs); at
    # N = 14336 they keep the pairs.  The first 4096 columns of the wide
    # product are the narrow product, so the two forms must agree bit for
    # bit, for the plain, residual and fp32 epilogues.
    print("skinny single-fragment m={}".format(m), flush=True)
    dev = gpu_device
    k = 4096
    x = cases.normal_bf16((m, k), 121).to(dev)
    w = cases.normal_bf16((14336, k), 122, 0.02).to(dev)
    res = cases.normal_bf16((m, 14336), 123).to(dev)
    narrow = torch.empty((m, 4096), dtype=BF16, device=dev)
    wide = torch.empty((m, 14336), dtype=BF16, device=dev)
    _hip.gemm(x, w[:4096], narrow)
    _hip.gemm(x, w, wide)
    assert torch.equal(narrow, wide[:, :4096])
    res_narrow = res[:, :4096].contiguous()
    _hip.gemm_residual(x, w[:4096], res_narrow, narrow)
    _hip.gemm_residual(x, w, res, wide)
    assert torch.equal(narrow, wide[:, :4096])
    f_narrow = torch.empty((m, 4096), dtype=torch.float32, device=dev)
    f_wide = torch.empty((m, 14336), dtype=torch.float32, device=dev)
    _hip.gemm_f32out(x, w[:4096], f_narrow)
    _hip.gemm_f32out(x, w, f_wide)
    assert torch.equal(f_narrow, f_wide[:, :4096])


def _random_split_shapes(count, seed):
    # shapes the split plan takes: 17..1024 rows, N a multiple of 8 up to
    # 4096 (so 256-row tiles fill at most half of 256 CUs), K a multiple of
    # 64 with at least 16 slabs, K >= 8192 past 128 rows
    import random
    rng = random.Random(seed)
    shapes = []
    for _ in range(count):
        m = rng.randint(17, 1024)
        n = 8 * rng.randint(16, 512)
        k = 64 * (rng.randint(16, 200) if m <= 128 else rng.randint(128, 200))
        while m * n * k > 12e9:  # keeps the float64 bound quick
            n = max(128, (n // 2) // 8 * 8)
        shapes.append((m, n, k))
    return shapes


@pytest.mark.parametrize("m,n,k", [(m, 4096, k) for m, k in (
    (17, 4096), (40, 14336), (64, 4096), (65, 4096), (128, 4096),
    (100, 14336), (256, 14336), (300, 14336), (512, 14336), (1000, 14336))]
    + _random_split_shapes(6, 23))
def test_gemm_split_k_matches_oracle(gpu_device, m, n, k):
    # Prompts of 17..1000 rows over N = 4096 (down_proj; o_proj up to 128
    # rows: past that its one-pass tiles are faster and no split is
    # planned, checked at the end) split K
    # over workgroup rows with fp32 partials in the caller's workspace: the
    # plain and residual (in place, as the executor calls it) products stay
    # within the float64 product bound and the oracle's tolerance; a
    # workspace one byte short is refused before any launch.
    print("split-K m={} n={} k={}".format(m, n, k), flush=True)
    dev = gpu_device
    need = _hip.gemm_workspace_bytes(m, n, k)
    assert need >= 2 * m * n * 4  # the shape splits on this device
    x = cases.normal_bf16((m, k), 131)
    w = cases.normal_bf16((n, k), 132, 0.02)
    res = cases.normal_bf16((m, n), 133)
    xd, wd = x.to(dev), w.to(dev)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    y = torch.empty((m, n), dtype=BF16, device=dev)
    _hip.gemm(xd, wd, y, workspace=ws)
    assert linear_bound_report(y, x, w) <= 1.0
    r = cases.compare(y, ref.linear(x, w))
    assert r["ok"], r
    h = res.to(dev)
    _hip.gemm_residual(xd, wd, h, h, workspace=ws)
    r = cases.compare(h, res + ref.linear(x, w))
    assert r["ok"], r
    # the one-pass form of the same product agrees within one bf16 place
    # (plus a small absolute slack for outputs whose exact value is ~0)
    one = torch.empty_like(y)
    _hip.gemm(xd, wd, one)
    diff = (one.float() - y.float()).abs()
    mag = torch.maximum(one.float().abs(), y.float().abs()).clamp_min(1e-30)
    ulp = torch.exp2(torch.floor(torch.log2(mag)) - 7)
    assert bool((diff <= ulp + 2.0 ** -14).all())
    with pytest.raises(_hip.HipCallError):
        _hip.gemm(xd, wd, y, workspace=ws[: need - 16])
    assert _hip.gemm_workspace_bytes(256, 4096, 4096) == 0
    assert _hip.gemm_workspace_bytes(16, 4096, 14336) == 0
    assert _hip.gemm_workspace_bytes(2048, 4096, 14336) == 0


@pytest.mark.parametrize("m", [5, 37])
def test_gemm_f32out_matches_float64(gpu_device, m):
    # m = 5: the skinny kernel's fp32 epilogue; m = 37: 64-row tiles
    dev = gpu_device
    n, k = 128256 // 8, 4096
    x = cases.normal_bf16((m, k), 103)
    w = cases.normal_bf16((n, k), 104, 0.02)
    y = torch.empty((m, n), dtype=torch.float32, device=dev)
    _hip.gemm_f32out(x.to(dev), w.to(dev), y)
    expected = ref.linear_exact(x, w).float()
    r = cases.compare(y, expected, atol=1e-4, rtol=1e-4)
    assert r["ok"], r


@pytest.mark.parametrize("m,n,k", [(2048, 4096, 4096), (6, 4096, 14336),
                                   (129, 4096, 14336), (100, 1024, 4096),
                                   (256, 1024, 4096)])
def test_gemm_residual_matches_oracle(gpu_device, m, n, k):
    dev = gpu_device
    x = cases.normal_bf16((m, k), 111)
    w = cases.normal_bf16((n, k), 112, 0.02)
    res = cases.normal_bf16((m, n), 113)
    y = res.to(dev)  # in place, as the executor uses it
    _hip.gemm_residual(x.to(dev), w.to(dev), y, y)
    expected = res + ref.linear(x, w)
    r = cases.compare(y, expected)
    assert r["ok"], r
    # W = I: y = bf16(res + x) exactly, torch's bf16 add
    eye = torch.eye(n, dtype=BF16, device=dev)
    xs = cases.normal_bf16((m, n), 114, 3.0)
    out = torch.empty((m, n), dtype=BF16, device=dev)
    _hip.gemm_residual(xs.to(dev), eye, res.to(dev), out)
    assert torch.equal(out.cpu(), res + xs)


@pytest.mark.parametrize("m", [2, 6, 16, 192, 200, 700])
def test_swiglu_gemm_fused_and_split_match_oracle(gpu_device, m):
    dev = gpu_device
    inter, hidden = 14336, 4096
    x = cases.normal_bf16((m, hidden), 121)
    wg = cases.normal_bf16((inter, hidden), 122, 0.02)
    wu = cases.normal_bf16((inter, hidden), 123, 0.02)
    gate = F.silu(ref.linear(x, wg))
    expected = gate * ref.linear(x, wu)
    xd, wgd, wud = x.to(dev), wg.to(dev), wu.to(dev)
    fused = torch.empty((m, inter), dtype=BF16, device=dev)
    _hip.gate_up_swiglu_gemm(xd, wgd, wud, fused)
    r = cases.compare(fused, expected)
    assert r["ok"], r
    g = torch.empty((m, inter), dtype=BF16, device=dev)
    split = torch.empty((m, inter), dtype=BF16, device=dev)
    _hip.gate_silu_gemm(xd, wgd, g)
    _hip.up_mul_gemm(xd, wud, g, split)
    r = cases.compare(g, gate)
    assert r["ok"], r
    assert torch.equal(fused.cpu(), split.cpu())


# Shapes whose last round of full tiles would leave at least half of the
# 256 CUs idle: the last tile columns run as half-height tiles in the same
# launch (256-row tiles with 128-row halves; 128-row tiles with 64-row
# halves), through every epilogue.
@pytest.mark.parametrize("m,n,k", [(512, 20480, 256), (200, 18432, 128),
                                   (1100, 14336, 128)])
def test_gemm_half_tile_tail_matches_oracle(gpu_device, m, n, k):
    print("half-tile tail m={} n={} k={}".format(m, n, k), flush=True)
    dev = gpu_device
    x = cases.normal_bf16((m, k), 161)
    w = cases.normal_bf16((n, k), 162, 0.05)
    w2 = cases.normal_bf16((n, k), 163, 0.05)
    res = cases.normal_bf16((m, n), 164)
    xd, wd, w2d = x.to(dev), w.to(dev), w2.to(dev)
    lin = ref.linear(x, w)
    y = torch.empty((m, n), dtype=BF16, device=dev)
    _hip.gemm(xd, wd, y)
    assert linear_bound_report(y, x, w) <= 1.0
    r = cases.compare(y, lin)
    assert r["ok"], r
    yf = torch.empty((m, n), dtype=torch.float32, device=dev)
    _hip.gemm_f32out(xd, wd, yf)
    r = cases.compare(yf, ref.linear_exact(x, w).float(), atol=1e-4, rtol=1e-4)
    assert r["ok"], r
    out = torch.empty((m, n), dtype=BF16, device=dev)
    _hip.gemm_residual(xd, wd, res.to(dev), out)
    r = cases.compare(out, res + lin)
    assert r["ok"], r
    gate = F.silu(lin)
    g = torch.empty((m, n), dtype=BF16, device=dev)
    split = torch.empty((m, n), dtype=BF16, device=dev)
    _hip.gate_silu_gemm(xd, wd, g)
    _hip.up_mul_gemm(xd, w2d, g, split)
    r = cases.compare(g, gate)
    assert r["ok"], r
    r = cases.compare(split, gate * ref.linear(x, w2))
    assert r["ok"], r
    fused = torch.empty((m, n), dtype=BF16, device=dev)
    _hip.gate_up_swiglu_gemm(xd, wd, w2d, fused)
    assert torch.equal(fused.cpu(), split.cpu())


# Outputs whose schedule of 256 x 256 tiles (two 128-column sub-tiles per
# workgroup, 32-deep slabs) is shorter than that of 256 x 128 tiles run on
# them: 8000 columns (63 128-column tiles, the last one partial, so the last
# workgroup's second sub-tile lies past the output; k = 64: fewer slabs
# than the ring holds), 8192 (one whole round), 600 x 28672 and 2048 x
# 28672 (a last round of 128 x 256 half-height tiles; SwiGLU over 2 x 28672
# rows: whole rounds, and at m = 600 a partial last round).  The split
# SwiGLU halves of 8192 / 28672 run on 256 x 128 or 256 x 256 tiles by the
# same rule, and the fused result equals the split one bit for bit either
# way (the K order of the MFMAs does not depend on the slab depth).
@pytest.mark.parametrize("m,n,k", [(2048, 8000, 64), (2048, 8192, 128),
                                   (600, 28672, 320), (2048, 28672, 64)])
def test_gemm_wide_tiles_match_oracle(gpu_device, m, n, k):
    print("wide tiles m={} n={} k={}".format(m, n, k), flush=True)
    dev = gpu_device
    x = cases.normal_bf16((m, k), 181)
    w = cases.normal_bf16((n, k), 182, 0.05)
    w2 = cases.normal_bf16((n, k), 183, 0.05)
    res = cases.normal_bf16((m, n), 184)
    xd, wd, w2d = x.to(dev), w.to(dev), w2.to(dev)
    lin = ref.linear(x, w)
    y = torch.empty((m, n), dtype=BF16, device=dev)
    _hip.gemm(xd, wd, y)
    assert linear_bound_report(y, x, w) <= 1.0
    r = cases.compare(y, lin)
    assert r["ok"], r
    yf = torch.empty((m, n), dtype=torch.float32, device=dev)
    _hip.gemm_f32out(xd, wd, yf)
    r = cases.compare(yf, ref.linear_exact(x, w).float(), atol=1e-4, rtol=1e-4)
    assert r["ok"], r
    out = torch.empty((m, n), dtype=BF16, device=dev)
    _hip.gemm_residual(xd, wd, res.to(dev), out)
    r = cases.compare(out, res + lin)
    assert r["ok"], r
    if n % 128:
        return  # fused SwiGLU pairs whole 128-column gate / up groups
    g = torch.empty((m, n), dtype=BF16, device=dev)
    split = torch.empty((m, n), dtype=BF16, device=dev)
    _hip.gate_silu_gemm(xd, wd, g)
    _hip.up_mul_gemm(xd, w2d, g, split)
    r = cases.compare(g, F.silu(lin))
    assert r["ok"], r
    r = cases.compare(split, F.silu(lin) * ref.linear(x, w2))
    assert r["ok"], r
    fused = torch.empty((m, n), dtype=BF16, device=dev)
    _hip.gate_up_swiglu_gemm(xd, wd, w2d, fused)
    assert torch.equal(fused.cpu(), split.cpu())


# Seeded random shapes across the tile-shape rule (256 x 128 or 256 x 256
# tiles by their schedule of rounds, half-height tails, 128- and 64-row
# tiles): every epilogue output stays within the float64 product bound and
# the fused SwiGLU equals the split one.
def _random_gemm_shapes(count, seed):
    import random
    rng = random.Random(seed)
    shapes = []
    for _ in range(count):
        m = rng.choice([rng.randint(129, 700), rng.randint(700, 3100)])
        n = rng.choice([8 * rng.randint(32, 5000), 128 * rng.randint(2, 300)])
        n = min(n, (24_000_000 // m) // 128 * 128)  # keeps the oracle quick
        shapes.append((m, n, 64 * rng.randint(1, 3)))
    return shapes


# seed 11: 256 x 256 tiles, 256 x 128 tiles with and without a
# half-height round, 128- and 64-row tiles, and SwiGLU on 256 x 256,
# 256 x 128 (with and without a half-height round) and 128-row tiles; the
# 256 x 256 tiles with a half-height round are tested below
@pytest.mark.parametrize("m,n,k", _random_gemm_shapes(8, 11))
def test_gemm_random_shapes_match_oracle(gpu_device, m, n, k):
    print("random shape m={} n={} k={}".format(m, n, k), flush=True)
    dev = gpu_device
    x = cases.normal_bf16((m, k), 191)
    w = cases.normal_bf16((n, k), 192, 0.05)
    res = cases.normal_bf16((m, n), 193)
    xd, wd = x.to(dev), w.to(dev)
    y = torch.empty((m, n), dtype=BF16, device=dev)
    _hip.gemm(xd, wd, y)
    assert linear_bound_report(y, x, w) <= 1.0
    out = torch.empty((m, n), dtype=BF16, device=dev)
    _hip.gemm_residual(xd, wd, res.to(dev), out)
    r = cases.compare(out, res + ref.linear(x, w))
    assert r["ok"], r
    yf = torch.empty((m, n), dtype=torch.float32, device=dev)
    _hip.gemm_f32out(xd, wd, yf)
    r = cases.compare(yf, ref.linear_exact(x, w).float(), atol=1e-4, rtol=1e-4)
    assert r["ok"], r
    if n % 128:
        return
    w2d = cases.normal_bf16((n, k), 194, 0.05).to(dev)
    g = torch.empty((m, n), dtype=BF16, device=dev)
    split = torch.empty_like(g)
    fused = torch.empty_like(g)
    _hip.gate_silu_gemm(xd, wd, g)
    _hip.up_mul_gemm(xd, w2d, g, split)
    _hip.gate_up_swiglu_gemm(xd, wd, w2d, fused)
    assert torch.equal(fused.cpu(), split.cpu())


def test_swiglu_gemm_wide_tiles_with_half_round(gpu_device):
    # The smallest shapes that still run 256 x 256 tiles with a last round
    # of 128 x 256 half-height tiles are large SwiGLUs such as this one
    # (M = 1537, 2 x 52736 columns).  The fused launch equals the split
    # silu / mul launches bit for bit, and the gate GEMM's first rows stay
    # within the float64 product bound.
    m, n, k = 1537, 52736, 64
    print("swiglu wide tiles m={} n={} k={}".format(m, n, k), flush=True)
    dev = gpu_device
    x = cases.normal_bf16((m, k), 201)
    wg = cases.normal_bf16((n, k), 202, 0.05)
    wu = cases.normal_bf16((n, k), 203, 0.05)
    xd, wgd, wud = x.to(dev), wg.to(dev), wu.to(dev)
    g = torch.empty((m, n), dtype=BF16, device=dev)
    split = torch.empty_like(g)
    fused = torch.empty_like(g)
    _hip.gate_silu_gemm(xd, wgd, g)
    _hip.up_mul_gemm(xd, wud, g, split)
    _hip.gate_up_swiglu_gemm(xd, wgd, wud, fused)
    assert torch.equal(fused, split)
    y = torch.empty((m, n), dtype=BF16, device=dev)
    _hip.gemm(xd, wgd, y)
    assert linear_bound_report(y[:64], x[:64], wg) <= 1.0


def _rope_tables(positions):
    inv = ref.llama3_inv_freq(DIM)
    cos, sin = ref.rope_cos_sin(inv, list(range(positions)))
    return cos[:, :64].contiguous(), sin[:, :64].contiguous()


@pytest.mark.parametrize("m,pos0", [(6, 0), (16, 100), (2048, 0), (33, 4000), (2, 32766)])
def test_qkv_rope_gemm_matches_oracle(gpu_device, m, pos0):
    print("qkv_rope_gemm m={} pos0={}".format(m, pos0), flush=True)
    dev = gpu_device
    hidden, kv = 4096, 1024
    x = cases.normal_bf16((m, hidden), 131)
    wq = cases.normal_bf16((hidden, hidden), 132, 0.02)
    wk = cases.normal_bf16((kv, hidden), 133, 0.02)
    wv = cases.normal_bf16((kv, hidden), 134, 0.02)
    table_cos, table_sin = _rope_tables(pos0 + m + 5)
    slot0 = 3  # cache slots are not positions: a different offset on purpose
    capacity = slot0 + m + 7
    kc = torch.zeros((8, capacity, DIM), dtype=BF16, device=dev)
    vc = torch.zeros_like(kc)
    q = torch.empty((m, hidden), dtype=BF16, device=dev)
    _hip.qkv_rope_gemm(x.to(dev), wq.to(dev), wk.to(dev), wv.to(dev),
                       table_cos.to(dev), table_sin.to(dev), pos0, q,
                       kc.view(-1), vc.view(-1), capacity * DIM, slot0)
    cos, sin = ref.rope_cos_sin(ref.llama3_inv_freq(DIM),
                                list(range(pos0, pos0 + m)))
    eq = ref.apply_rope(ref.linear(x, wq).view(m, 32, DIM).transpose(0, 1), cos, sin)
    ek = ref.apply_rope(ref.linear(x, wk).view(m, 8, DIM).transpose(0, 1), cos, sin)
    ev = ref.linear(x, wv).view(m, 8, DIM).transpose(0, 1)
    kcpu, vcpu = kc.cpu(), vc.cpu()
    for got, exp in ((q.cpu(), eq.transpose(0, 1).reshape(m, -1)),
                     (kcpu[:, slot0:slot0 + m], ek), (vcpu[:, slot0:slot0 + m], ev)):
        r = cases.compare(got, exp)
        assert r["ok"], r
    # only slots slot0 .. slot0 + m - 1 were written
    for buf in (kcpu, vcpu):
        assert int(buf[:, :slot0].abs().sum()) == 0
        assert int(buf[:, slot0 + m:].abs().sum()) == 0


# matrix granularity: q, k, v in three launches == one fused launch; at
# m = 2048 the fused launch takes three heads per tile (32-deep slabs) and
# the split ones 256 x 128 / 64 x 128 tiles (64-deep), in the same K order
@pytest.mark.parametrize("m", [70, 2048])
def test_qkv_rope_gemm_split_matrices_equal_fused(gpu_device, m):
    dev = gpu_device
    hidden, kv = 4096, 1024
    x = cases.normal_bf16((m, hidden), 141).to(dev)
    wq = cases.normal_bf16((hidden, hidden), 142, 0.02).to(dev)
    wk = cases.normal_bf16((kv, hidden), 143, 0.02).to(dev)
    wv = cases.normal_bf16((kv, hidden), 144, 0.02).to(dev)
    c, s = (t.to(dev) for t in _rope_tables(m + 10))
    outs = []
    for split in (False, True):
        cap = m + 58
        kc = torch.zeros((8, cap, DIM), dtype=BF16, device=dev)
        vc = torch.zeros_like(kc)
        q = torch.zeros((m, hidden), dtype=BF16, device=dev)
        args = (c, s, 10)
        if split:
            _hip.qkv_rope_gemm(x, wq, None, None, *args, q, None, None, cap * DIM, 5)
            _hip.qkv_rope_gemm(x, None, wk, None, *args, None, kc.view(-1), None,
                               cap * DIM, 5)
            _hip.qkv_rope_gemm(x, None, None, wv, *args, None, None, vc.view(-1),
                               cap * DIM, 5)
        else:
            _hip.qkv_rope_gemm(x, wq, wk, wv, *args, q, kc.view(-1), vc.view(-1),
                               cap * DIM, 5)
        outs.append((q.cpu(), kc.cpu(), vc.cpu()))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_gemm_row_matches_gemv_rounding(gpu_device):
    # one token through the GEMM and through the GEMV: both are valid fp32
    # summation orders of the same bf16 products, so they agree to 1 ulp
    dev = gpu_device
    x = cases.normal_bf16((1, 4096), 151).to(dev)
    w = cases.normal_bf16((4096, 4096), 152, 0.02).to(dev)
    a = torch.empty((1, 4096), dtype=BF16, device=dev)
    b = torch.empty(4096, dtype=BF16, device=dev)
    _hip.gemm(x, w, a)
    _hip.gemv(w, x.reshape(-1), b)
    xc, wc = x.cpu(), w.cpu()
    assert linear_bound_report(a, xc, wc) <= 1.0
    assert linear_bound_report(b.reshape(1, -1), xc, wc) <= 1.0


# 32-token units are paired (unit p with unit U - 1 - p); 96 tokens leave a
# middle unit that walks alone, past > 0 makes every walk long, slack 0 puts
# the last cache row at the very end of the allocation
@pytest.mark.parametrize("past,tokens,q_scale,slack", [
    (0, 1, 1, 9), (0, 2, 1, 9), (0, 5, 1, 9), (0, 33, 1, 9), (0, 96, 1, 9),
    (0, 130, 1, 9), (0, 2048, 1, 9), (0, 2048, 8, 9), (100, 7, 1, 9),
    (4000, 45, 4, 9), (1000, 300, 1, 0), (0, 77, 1, 0)])
def test_prefill_attention_matches_oracle(gpu_device, past, tokens, q_scale,
                                          slack):
    print("prefill attention past={} tokens={} q_scale={} slack={}".format(
        past, tokens, q_scale, slack), flush=True)
    dev = gpu_device
    length = past + tokens
    q = cases.normal_bf16((32, tokens, DIM), 161)
    if q_scale != 1:
        q = (q.float() * q_scale).to(BF16)
    k = cases.normal_bf16((8, length, DIM), 162)
    v = cases.normal_bf16((8, length, DIM), 163)
    capacity = length + slack
    kc = torch.zeros((8, capacity, DIM), dtype=BF16, device=dev)
    vc = torch.zeros_like(kc)
    kc[:, :length].copy_(k.to(dev))
    vc[:, :length].copy_(v.to(dev))
    qrows = q.transpose(0, 1).reshape(tokens, 32 * DIM).contiguous()
    out = torch.empty((tokens, 32 * DIM), dtype=BF16, device=dev)
    _hip.prefill_attention(qrows.to(dev), kc.view(-1), vc.view(-1),
                           capacity * DIM, past, tokens, out, DIM ** -0.5)
    expected = ref.attention(q, k, v, past)
    r = cases.compare(out, expected, atol=1e-2, rtol=1e-2)
    assert r["ok"], r


def test_prefill_attention_first_token_is_value_row(gpu_device):
    # token 0 of a prefill sees position 0 only: its output is V[0] exactly
    dev = gpu_device
    tokens = 40
    q = cases.normal_bf16((tokens, 32 * DIM), 171).to(dev)
    kc = cases.normal_bf16((8, tokens, DIM), 172).to(dev)
    vc = cases.normal_bf16((8, tokens, DIM), 173).to(dev)
    out = torch.empty((tokens, 32 * DIM), dtype=BF16, device=dev)
    _hip.prefill_attention(q, kc.view(-1), vc.view(-1), tokens * DIM, 0, tokens,
                           out, DIM ** -0.5)
    expected = vc[:, 0].repeat_interleave(4, dim=0).reshape(-1)
    assert torch.equal(out[0].cpu(), expected.cpu())


def test_prefill_argument_errors_raise(gpu_device):
    dev = gpu_device
    x = torch.zeros((4, 4096), dtype=BF16, device=dev)
    w = torch.zeros((128, 4000), dtype=BF16, device=dev)  # K not a multiple of 64
    y = torch.zeros((4, 128), dtype=BF16, device=dev)
    with pytest.raises(_hip.HipCallError):
        _hip.gemm(torch.zeros((4, 4000), dtype=BF16, device=dev), w, y)
    with pytest.raises(_hip.HipCallError):  # n_half not a multiple of 64
        wg = torch.zeros((100, 4096), dtype=BF16, device=dev)
        _hip.gate_up_swiglu_gemm(x, wg, wg, torch.zeros((4, 100), dtype=BF16,
                                                        device=dev))
    w = torch.zeros((128, 4096), dtype=BF16, device=dev)
    y = torch.zeros((4, 128), dtype=BF16, device=dev)
    with pytest.raises(ValueError):
        _hip.gemm(x.cpu(), w, y)  # host tensor never reaches a kernel
    # a RoPE table too short for the rows: rejected before any launch
    c = torch.zeros((3, 64), dtype=BF16, device=dev)
    kc = torch.zeros((8, 16, DIM), dtype=BF16, device=dev)
    q = torch.zeros((4, 4096), dtype=BF16, device=dev)
    wq = torch.zeros((4096, 4096), dtype=BF16, device=dev)
    with pytest.raises(_hip.HipCallError):
        _hip.qkv_rope_gemm(x, wq, None, None, c, c, 0, q, None, None, 16 * DIM, 0)
    # KV slots beyond the head stride: rejected
    wk = torch.zeros((1024, 4096), dtype=BF16, device=dev)
    with pytest.raises(ValueError):
        _hip.qkv_rope_gemm(x, None, wk, None, c, c, 0, None, kc.view(-1), None,
                           16 * DIM, 14)
