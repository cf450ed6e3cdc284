"""cascade_decode_attention_noalloc_bf16 (split partials in the library's
static device scratch, no workspace argument) against
cascade_decode_attention_bf16 (caller's workspace) through the C ABI: bit for
bit on two calls in a row, the second with a smaller input (shorter cache,
fewer heads), so the second call reuses scratch the first one filled."""

import ctypes

import pytest
import torch

from layer_streaming import _hip

pytestmark = pytest.mark.gpu

D = 128
ESCRATCH = 1005


def _case(seed, n_kv, length, capacity, device):
    gen = torch.Generator().manual_seed(seed)
    n_q = 4 * n_kv
    q = torch.randn(n_q * D, generator=gen).to(torch.bfloat16)
    k = torch.randn(n_kv, capacity, D, generator=gen).to(torch.bfloat16)
    v = torch.randn(n_kv, capacity, D, generator=gen).to(torch.bfloat16)
    return q.to(device), k.to(device), v.to(device), n_q


def _both(lib, q, k, v, n_q, n_kv, length, capacity, device):
    stream = torch.cuda.current_stream(device).cuda_stream
    scale = D ** -0.5
    out_ws = torch.empty(n_q * D, dtype=torch.bfloat16, device=device)
    out_na = torch.full((n_q * D,), float("nan"), dtype=torch.bfloat16,
                        device=device)
    ws = torch.zeros(_hip.attention_workspace_bytes(length, n_q, n_kv, D),
                     dtype=torch.uint8, device=device)
    stride = capacity * D
    print("[no-alloc] workspace form n_kv={} len={}".format(n_kv, length),
          flush=True)
    rc = lib.cascade_decode_attention_bf16(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), stride, length, n_q, n_kv, D,
        ctypes.c_float(scale), out_ws.data_ptr(), ws.data_ptr(), ws.numel(),
        stream)
    assert rc == 0, _hip.load().cascade_error_string(rc)
    print("[no-alloc] static-scratch form n_kv={} len={}".format(n_kv, length),
          flush=True)
    rc = lib.cascade_decode_attention_noalloc_bf16(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), stride, length, n_q, n_kv, D,
        ctypes.c_float(scale), out_na.data_ptr(), stream)
    assert rc == 0, _hip.load().cascade_error_string(rc)
    torch.cuda.synchronize(device)
    return out_ws.cpu(), out_na.cpu()


def test_noalloc_attention_matches_workspace_form(gpu_device):
    lib = _hip.load()
    # larger first (8 KV heads, 64 splits: the whole scratch), then smaller
    for seed, n_kv, length, capacity in ((3, 8, 32769, 32800),
                                         (4, 2, 1000, 1024)):
        q, k, v, n_q = _case(seed, n_kv, length, capacity, gpu_device)
        expected, got = _both(lib, q, k, v, n_q, n_kv, length, capacity,
                              gpu_device)
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got.view(torch.int16), expected.view(torch.int16)), (
            n_kv, length)


def test_noalloc_attention_rejects_more_kv_heads_than_the_scratch_holds():
    lib = _hip.load()
    # refused on the host before any device work (pointers are never read)
    rc = lib.cascade_decode_attention_noalloc_bf16(16, 16, 16, 128 * 8, 8, 36,
                                                   9, D, ctypes.c_float(0.1),
                                                   16, None)
    assert rc == ESCRATCH
    assert b"static scratch" in lib.cascade_error_string(rc)
