"""The C ABI boundary, checked on a CPU-only host: the library loads, every
function include/cascade_hip.h declares is exported and typed by the
binding, and argument checks reject bad calls before anything is launched
(no kernel runs here)."""

import ctypes
import re
from pathlib import Path

import pytest

from layer_streaming import _hip

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "cascade_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cascade_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    assert "cascade_qkv_rope_bf16" in names
    assert "cascade_lm_head_topk_bf16" in names
    assert len(names) == len(set(names)) >= 20


def test_library_exports_every_declared_function():
    lib = ctypes.CDLL(_hip.library_path())
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert missing == []


def test_binding_types_exactly_the_declared_functions():
    assert sorted(_hip.exported_symbols()) == declared_functions()


def test_abi_version_and_error_strings():
    lib = _hip.load()
    assert lib.cascade_abi_version() == _hip.ABI_VERSION
    for code in (0, 1001, 1002, 1003, 1004, 1005):
        assert lib.cascade_error_string(code)


def test_argument_checks_reject_without_launching():
    lib = _hip.load()
    # null pointers / zero sizes / misalignment are refused host-side
    assert lib.cascade_gemv_bf16(None, None, None, 16, 4096, None) == 1001
    assert lib.cascade_gemv_bf16(16, 32, 48, 16, 4095, None) == 1002
    assert lib.cascade_rmsnorm_bf16(None, None, None, 1, 4096, 1e-5, None) == 1001
    assert lib.cascade_qkv_rope_bf16(16, 16, 16, 100, 0, 0, 4096, 16, None,
                                     1e-5, 16, 16, 16, None, None, 0, None) == 1003
    assert lib.cascade_decode_attention_bf16(16, 16, 16, 128, 4, 32, 8, 64,
                                             0.1, 16, 16, 1 << 20, None) == 1003
    assert lib.cascade_lm_head_topk_bf16(16, 100, 4096, 0, 16, 65, 1, None, 16,
                                         1 << 20, 16, 16, None) == 1001
    assert lib.cascade_memcpy_h2d_async(None, None, 0, None) == 1001
    # top-k of a logits row: pointers, 1 <= top_k <= 64, workspace size and
    # alignment
    ws_bytes = _hip.lm_head_workspace_bytes(1000, 10)
    assert lib.cascade_topk_f32(None, 1000, 10, 16, ws_bytes, 16, 16, None) == 1001
    assert lib.cascade_topk_f32(16, 1000, 65, 16, ws_bytes, 16, 16, None) == 1001
    assert lib.cascade_topk_f32(16, 0, 10, 16, ws_bytes, 16, 16, None) == 1001
    assert lib.cascade_topk_f32(16, 1000, 10, 16, ws_bytes - 4, 16, 16, None) == 1004
    assert lib.cascade_topk_f32(16, 1000, 10, 20, ws_bytes, 16, 16, None) == 1002
    # split-K GEMM forms, at a shape the plan splits (64 x 4096 x 14336):
    # pointers, alignment and the workspace size are checked before launching
    need = lib.cascade_gemm_workspace_bytes(64, 4096, 14336)
    assert need >= 2 * 64 * 4096 * 4
    assert lib.cascade_gemm_residual_ws_bf16(16, 16, 16, 16, 64, 4096, 14336,
                                             None, need, None) == 1001
    assert lib.cascade_gemm_residual_ws_bf16(16, 16, None, 16, 64, 4096, 14336,
                                             16, need, None) == 1001
    assert lib.cascade_gemm_residual_ws_bf16(16, 16, 16, 16, 64, 4096, 14336,
                                             20, need, None) == 1002
    assert lib.cascade_gemm_ws_bf16(16, 16, 16, 64, 4096, 14336, 16, need - 4,
                                    None) == 1004
    # prefill attention: cache positions past + tokens are limited to 2^24,
    # head_dim to 128 and n_q_heads to 4 n_kv_heads
    pos = 1 << 24
    assert lib.cascade_prefill_attention_bf16(16, 16, 16, pos * 128, pos - 2, 4,
                                              32, 8, 128, 0.1, 16, None) == 1001
    assert lib.cascade_prefill_attention_bf16(16, 16, 16, 64 * 128, 0, 4,
                                              32, 8, 64, 0.1, 16, None) == 1003
    assert lib.cascade_prefill_attention_bf16(16, 16, 16, 64 * 128, 0, 4,
                                              16, 8, 128, 0.1, 16, None) == 1003
    # device-position forms: the length word must be given and 8-byte
    # aligned, the capacity positive, the cache stride >= capacity * 128
    def qkv_at(length=16, capacity=10, stride=128 * 10):
        return lib.cascade_qkv_rope_at_bf16(16, 16, 16, 4096, 1024, 1024, 4096, 16,
                                            16, 1e-5, 16, 16, 16, 16, 16, stride,
                                            length, capacity, None)

    assert qkv_at(length=None) == 1001
    assert qkv_at(length=20) == 1002
    assert qkv_at(capacity=0) == 1001
    assert qkv_at(stride=128 * 9) == 1001
    attn_ws = _hip.attention_workspace_bytes(10)

    def attn_at(length=16, capacity=10, stride=128 * 10, ws_bytes=attn_ws):
        return lib.cascade_decode_attention_at_bf16(16, 16, 16, stride, length,
                                                    capacity, 32, 8, 128, 0.1, 16,
                                                    16, ws_bytes, None)

    assert attn_at(length=None) == 1001
    assert attn_at(length=12) == 1002
    assert attn_at(capacity=0) == 1001
    assert attn_at(stride=128 * 9) == 1001
    assert attn_at(ws_bytes=16) == 1004

    def begin(ids=16, length=16, history=16, capacity=8):
        return lib.cascade_decode_step_begin_bf16(16, 100, 64, ids, 16, length,
                                                  history, capacity, None, None)

    assert begin(ids=None) == 1001
    assert begin(history=None) == 1001
    assert begin(capacity=0) == 1001
    assert begin(length=12) == 1002
    assert begin(ids=20) == 1002


def test_workspace_sizes():
    # attention: header + (m, l, acc[128]) per (kv head, split, q head),
    # sized for the maximum of 64 splits whatever the length
    for length in (1, 2048, 32769, 1 << 20):
        assert _hip.attention_workspace_bytes(length) == 256 + 8 * 64 * 4 * (2 + 128) * 4
    # LM head: counter, running top-64 keys, 4096 candidate keys, fp32 logits
    assert _hip.lm_head_workspace_bytes(16384, 10) == 256 + 512 + 4096 * 8 + 16384 * 4
    assert _hip.lm_head_workspace_bytes(128256, 64) == 256 + 512 + 4096 * 8 + 128256 * 4
    with pytest.raises(ValueError):
        _hip.lm_head_workspace_bytes(16384, 65)
    with pytest.raises(ValueError):
        _hip.attention_workspace_bytes(100, 32, 8, 64)


def test_host_tensors_never_reach_a_kernel():
    import torch

    w = torch.zeros(16, 4096, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        _hip.gemv(w, w[0], w[0])
