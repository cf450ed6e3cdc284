"""ctypes binding to libcascade_hip.so, the gfx950 kernels of the decode path.

The C ABI is declared in ``include/cascade_hip.h``.  This module is the only
place that touches the library; everything above it passes torch tensors.
Every wrapper validates device, dtype, contiguity and size before launching,
because a host pointer or a short buffer reaching a kernel would fault the
GPU.  ``torch`` is imported first so the library binds to the HIP runtime
torch already loaded (both carry the same SONAME), which makes torch's
streams and device pointers valid here.

There is no fallback: if the library is missing or fails to load, every
entry point raises :class:`HipLibraryError`.
"""

import ctypes
import os
import threading
import weakref

import torch

__all__ = [
    "HipLibraryError",
    "HipCallError",
    "HipEvent",
    "library_path",
    "load",
    "exported_symbols",
]

_PACKAGE_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBRARY_NAME = "libcascade_hip.so"

_I64 = ctypes.c_int64
_P = ctypes.c_void_p
_F = ctypes.c_float
_INT = ctypes.c_int
_SZ = ctypes.c_size_t
_U64 = ctypes.c_uint64

# name -> (restype, argtypes); mirrors include/cascade_hip.h exactly.
_SIGNATURES = {
    "cascade_abi_version": (_INT, []),
    "cascade_error_string": (ctypes.c_char_p, [_INT]),
    "cascade_rmsnorm_bf16": (_INT, [_P, _P, _P, _I64, _I64, _F, _P]),
    "cascade_gemv_bf16": (_INT, [_P, _P, _P, _I64, _I64, _P]),
    "cascade_gemv_residual_bf16": (_INT, [_P, _P, _P, _P, _I64, _I64, _P]),
    "cascade_qkv_rope_bf16": (
        _INT,
        [_P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _F, _P, _P, _P, _P, _P,
         _I64, _P],
    ),
    "cascade_qkv_rope_at_bf16": (
        _INT,
        [_P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _F, _P, _P, _P, _P, _P,
         _I64, _P, _I64, _P],
    ),
    "cascade_gate_up_swiglu_bf16": (
        _INT, [_P, _P, _I64, _I64, _P, _P, _F, _P, _P]),
    "cascade_gate_silu_bf16": (_INT, [_P, _I64, _I64, _P, _P, _F, _P, _P]),
    "cascade_up_mul_bf16": (_INT, [_P, _I64, _I64, _P, _P, _F, _P, _P, _P]),
    "cascade_decode_attention_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64]),
    "cascade_decode_attention_bf16": (
        _INT,
        [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _P, _P, _SZ, _P],
    ),
    "cascade_decode_attention_at_bf16": (
        _INT,
        [_P, _P, _P, _I64, _P, _I64, _I64, _I64, _I64, _F, _P, _P, _SZ, _P],
    ),
    "cascade_decode_attention_fused_bf16": (
        _INT,
        [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _P, _P, _SZ, _P, _P, _P],
    ),
    "cascade_decode_attention_fused_at_bf16": (
        _INT,
        [_P, _P, _P, _I64, _P, _I64, _I64, _I64, _I64, _F, _P, _P, _SZ, _P, _P,
         _P],
    ),
    "cascade_decode_attention_noalloc_bf16": (
        _INT, [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _P, _P]),
    "cascade_gemm_bf16": (_INT, [_P, _P, _P, _I64, _I64, _I64, _P]),
    "cascade_gemm_residual_bf16": (
        _INT, [_P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "cascade_gemm_f32out_bf16": (_INT, [_P, _P, _P, _I64, _I64, _I64, _P]),
    "cascade_gate_up_swiglu_gemm_bf16": (
        _INT, [_P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "cascade_gate_silu_gemm_bf16": (_INT, [_P, _P, _P, _I64, _I64, _I64, _P]),
    "cascade_up_mul_gemm_bf16": (
        _INT, [_P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "cascade_qkv_rope_gemm_bf16": (
        _INT,
        [_P, _I64, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _I64, _P,
         _P, _P, _I64, _I64, _P],
    ),
    "cascade_prefill_attention_bf16": (
        _INT, [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _F, _P, _P]),
    "cascade_lm_head_workspace_bytes": (_SZ, [_I64, _I64]),
    "cascade_lm_head_topk_bf16": (
        _INT,
        [_P, _I64, _I64, _I64, _P, _I64, _INT, _P, _P, _SZ, _P, _P, _P],
    ),
    "cascade_topk_f32": (_INT, [_P, _I64, _I64, _P, _SZ, _P, _P, _P]),
    "cascade_gemm_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "cascade_gemm_ws_bf16": (_INT, [_P, _P, _P, _I64, _I64, _I64, _P, _SZ, _P]),
    "cascade_gemm_residual_ws_bf16": (
        _INT, [_P, _P, _P, _P, _I64, _I64, _I64, _P, _SZ, _P]),
    "cascade_embedding_gather_bf16": (
        _INT, [_P, _I64, _I64, _P, _I64, _P, _P, _P]),
    "cascade_decode_step_begin_bf16": (
        _INT, [_P, _I64, _I64, _P, _P, _P, _P, _I64, _P, _P]),
    "cascade_memcpy_h2d_async": (_INT, [_P, _P, _SZ, _P]),
    "cascade_memcpy_d2d_async": (_INT, [_P, _P, _SZ, _P]),
    "cascade_event_create": (_INT, [ctypes.POINTER(_U64), _INT]),
    "cascade_event_destroy": (_INT, [_U64]),
    "cascade_event_record": (_INT, [_U64, _P]),
    "cascade_stream_wait_event": (_INT, [_P, _U64]),
    "cascade_event_synchronize": (_INT, [_U64]),
    "cascade_event_query": (_INT, [_U64]),
    "cascade_event_elapsed_ms": (_INT, [_U64, _U64, ctypes.POINTER(_F)]),
    "cascade_host_copy": (_INT, [_P, _P, _SZ, _INT]),
    "cascade_copy_pool_create": (_INT, [_INT, _INT, ctypes.POINTER(_U64)]),
    "cascade_copy_pool_copy": (_INT, [_U64, _P, _P, _SZ]),
    "cascade_copy_pool_info": (
        _INT, [_U64, ctypes.POINTER(_INT), ctypes.POINTER(_INT)]),
    "cascade_copy_pool_destroy": (_INT, [_U64]),
    "cascade_hbm_read": (_INT, [_P, _SZ, _P, _I64, _P]),
    "cascade_device_copy": (_INT, [_P, _P, _SZ, _P]),
    "cascade_time_next_launch": (_INT, [_U64, _U64]),
}

ABI_VERSION = 5
ESHAPE = 1003  # CASCADE_ESHAPE
# fused decode attention: sync buffer size and the bits it ors into the
# caller's error word (include/cascade_hip.h)
ATTENTION_SYNC_BYTES = 1024
ATTN_EPLACEMENT = 2
ATTN_ETIMEOUT = 4
# the fused form needs one KV head per XCD and at least 8 splits of 32 rows
FUSED_ATTENTION_KV_HEADS = 8
FUSED_ATTENTION_MIN_LEN = 225


class HipLibraryError(RuntimeError):
    """libcascade_hip.so is missing, stale or failed to load."""


class HipCallError(RuntimeError):
    """A libcascade_hip entry point returned a non-zero status."""

    def __init__(self, name, code, message):
        super().__init__("{} failed ({}): {}".format(name, code, message))
        self.code = code


_lock = threading.Lock()
_lib = None


def library_path():
    """Absolute path of the in-tree library (``<package>/lib``)."""

    override = os.environ.get("CASCADE_HIP_LIBRARY")
    if override:
        return override
    return os.path.join(_PACKAGE_ROOT, "lib", LIBRARY_NAME)


def exported_symbols():
    """Names every build of the library must export."""

    return tuple(_SIGNATURES)


def load():
    """Load and type the library once; raise HipLibraryError if impossible."""

    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not os.path.exists(path):
            raise HipLibraryError(
                "{} is missing; build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` "
                "from the repository root".format(path)
            )
        try:
            lib = ctypes.CDLL(path)
        except OSError as error:
            raise HipLibraryError(
                "cannot load {}: {}".format(path, error)
            ) from error
        for name, (restype, argtypes) in _SIGNATURES.items():
            try:
                fn = getattr(lib, name)
            except AttributeError as error:
                raise HipLibraryError(
                    "{} does not export {}".format(path, name)
                ) from error
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.cascade_abi_version()
        if version != ABI_VERSION:
            raise HipLibraryError(
                "{} has ABI version {}, expected {}".format(
                    path, version, ABI_VERSION
                )
            )
        _lib = lib
    return _lib


def _check(name, code):
    if code != 0:
        message = load().cascade_error_string(int(code))
        raise HipCallError(
            name, int(code), message.decode() if message else "unknown"
        )


def call(name, *args):
    """Call an entry point by name and raise HipCallError on failure."""

    _check(name, getattr(load(), name)(*args))


def check(name, code):
    """Raise HipCallError when a raw entry-point call returned non-zero."""

    if code != 0:
        _check(name, code)


def bf16_weight(tensor, name, rows=None, k=None):
    """Validate a weight view once (device, dtype, layout, shape) and return
    its (rows, K); the executor then launches on raw pointers."""

    _bf16(tensor, name)
    if tensor.dim() != 2:
        raise ValueError("{} must be 2-D [rows, K]".format(name))
    n, kk = tensor.shape
    if (rows is not None and n != rows) or (k is not None and kk != k):
        raise ValueError("{} has shape {}, expected [{}, {}]".format(
            name, tuple(tensor.shape), rows, k))
    if tensor.data_ptr() % 16 or kk % 8:
        raise ValueError("{} is not 16-byte aligned".format(name))
    return n, kk


def stream_handle(stream=None, device=None):
    """Raw hipStream_t (as int) of a torch stream; default: current stream."""

    if stream is None:
        stream = torch.cuda.current_stream(device)
    return stream.cuda_stream


# --------------------------------------------------------------- validation


def require_device(tensor, name, dtype=None, min_numel=None, contiguous=True):
    if not isinstance(tensor, torch.Tensor):
        raise TypeError("{} must be a torch.Tensor".format(name))
    if tensor.device.type != "cuda":
        raise ValueError(
            "{} must live on the GPU, got {}".format(name, tensor.device)
        )
    if dtype is not None and tensor.dtype != dtype:
        raise TypeError(
            "{} must be {}, got {}".format(name, dtype, tensor.dtype)
        )
    if contiguous and not tensor.is_contiguous():
        raise ValueError("{} must be contiguous".format(name))
    if min_numel is not None and tensor.numel() < min_numel:
        raise ValueError(
            "{} holds {} elements, needs at least {}".format(
                name, tensor.numel(), min_numel
            )
        )
    return tensor


def _bf16(tensor, name, min_numel=None):
    return require_device(tensor, name, torch.bfloat16, min_numel)


def _matrix(tensor, name):
    _bf16(tensor, name)
    if tensor.dim() != 2:
        raise ValueError("{} must be 2-D [rows, K]".format(name))
    return tensor.shape


# ------------------------------------------------------------------ kernels


def rmsnorm(x, weight, out, eps, stream=None):
    """out[r] = rmsnorm(x[r]) for every row of x (last dim = hidden)."""

    n = weight.numel()
    _bf16(weight, "weight")
    _bf16(x, "x")
    if x.numel() % n:
        raise ValueError("x width does not match the norm weight")
    rows = x.numel() // n
    _bf16(out, "out", x.numel())
    call("cascade_rmsnorm_bf16", x.data_ptr(), weight.data_ptr(),
         out.data_ptr(), rows, n, float(eps), stream_handle(stream))
    return out


def gemv(weight, x, out, stream=None):
    n, k = _matrix(weight, "weight")
    _bf16(x, "x", k)
    _bf16(out, "out", n)
    call("cascade_gemv_bf16", weight.data_ptr(), x.data_ptr(),
         out.data_ptr(), n, k, stream_handle(stream))
    return out


def gemv_residual(weight, x, residual, out, stream=None):
    n, k = _matrix(weight, "weight")
    _bf16(x, "x", k)
    _bf16(residual, "residual", n)
    _bf16(out, "out", n)
    call("cascade_gemv_residual_bf16", weight.data_ptr(), x.data_ptr(),
         residual.data_ptr(), out.data_ptr(), n, k, stream_handle(stream))
    return out


def qkv_rope(wq, wk, wv, x, norm_weight, eps, rope_cos, rope_sin, q_out,
             k_out, v_out, kv_head_stride, stream=None):
    """Fused RMSNorm + Q/K/V GEMVs + RoPE + KV write for one token.

    Any of wq / wk / wv may be None (matrix granularity).  rope_cos /
    rope_sin are the 64-entry bf16 rows of this position; k_out / v_out are
    views starting at this position of KV head 0 of the layer's cache.
    """

    k = None
    sizes = []
    for name, w in (("wq", wq), ("wk", wk), ("wv", wv)):
        if w is None:
            sizes.append(0)
            continue
        n, kk = _matrix(w, name)
        if k is not None and kk != k:
            raise ValueError("q/k/v matrices disagree on K")
        k = kk
        sizes.append(n)
    if k is None:
        raise ValueError("at least one of wq, wk, wv is required")
    nq, nk, nv = sizes
    _bf16(x, "x", k)
    if norm_weight is not None:
        _bf16(norm_weight, "norm_weight", k)
    if nq or nk:
        _bf16(rope_cos, "rope_cos", 64)
        _bf16(rope_sin, "rope_sin", 64)
    heads_k = nk // 128
    heads_v = nv // 128
    if nq:
        _bf16(q_out, "q_out", nq)
    for name, buf, heads in (("k_out", k_out, heads_k), ("v_out", v_out, heads_v)):
        if heads:
            require_device(buf, name, torch.bfloat16, contiguous=False)
            if buf.storage_offset() + (heads - 1) * kv_head_stride + 128 > (
                buf.untyped_storage().nbytes() // 2
            ):
                raise ValueError("{} cannot hold {} heads".format(name, heads))

    def ptr(t):
        return 0 if t is None else t.data_ptr()

    call(
        "cascade_qkv_rope_bf16",
        ptr(wq), ptr(wk), ptr(wv), nq, nk, nv, k,
        x.data_ptr(), ptr(norm_weight), float(eps),
        ptr(rope_cos) if (nq or nk) else 0,
        ptr(rope_sin) if (nq or nk) else 0,
        ptr(q_out) if nq else 0,
        ptr(k_out) if nk else 0,
        ptr(v_out) if nv else 0,
        int(kv_head_stride), stream_handle(stream),
    )


def gate_up_swiglu(w_gate, w_up, x, norm_weight, eps, out, stream=None):
    n, k = _matrix(w_gate, "w_gate")
    if tuple(_matrix(w_up, "w_up")) != (n, k):
        raise ValueError("gate and up matrices differ in shape")
    _bf16(x, "x", k)
    if norm_weight is not None:
        _bf16(norm_weight, "norm_weight", k)
    _bf16(out, "out", n)
    call("cascade_gate_up_swiglu_bf16", w_gate.data_ptr(), w_up.data_ptr(),
         n, k, x.data_ptr(),
         0 if norm_weight is None else norm_weight.data_ptr(), float(eps),
         out.data_ptr(), stream_handle(stream))
    return out


def gate_silu(w_gate, x, norm_weight, eps, out, stream=None):
    n, k = _matrix(w_gate, "w_gate")
    _bf16(x, "x", k)
    if norm_weight is not None:
        _bf16(norm_weight, "norm_weight", k)
    _bf16(out, "out", n)
    call("cascade_gate_silu_bf16", w_gate.data_ptr(), n, k, x.data_ptr(),
         0 if norm_weight is None else norm_weight.data_ptr(), float(eps),
         out.data_ptr(), stream_handle(stream))
    return out


def up_mul(w_up, x, norm_weight, eps, gate, out, stream=None):
    n, k = _matrix(w_up, "w_up")
    _bf16(x, "x", k)
    if norm_weight is not None:
        _bf16(norm_weight, "norm_weight", k)
    _bf16(gate, "gate", n)
    _bf16(out, "out", n)
    call("cascade_up_mul_bf16", w_up.data_ptr(), n, k, x.data_ptr(),
         0 if norm_weight is None else norm_weight.data_ptr(), float(eps),
         gate.data_ptr(), out.data_ptr(), stream_handle(stream))
    return out


# ------------------------------------------------------ prefill (M > 1)


def _rows(x, name, k):
    """Validate a token-row operand [.., M, K] and return M."""

    _bf16(x, name)
    if x.numel() % k or x.numel() == 0:
        raise ValueError("{} is not a whole number of {}-wide rows".format(name, k))
    return x.numel() // k


def gemm_workspace_bytes(m, n, k):
    """Workspace bytes of the split-K forms for this shape on the current
    device (0: these shapes run the one-pass GEMM)."""

    return int(load().cascade_gemm_workspace_bytes(int(m), int(n), int(k)))


def _ws(workspace):
    if workspace is None:
        return 0, 0
    require_device(workspace, "workspace", torch.uint8)
    return workspace.data_ptr(), workspace.numel()


def gemm(x, weight, out, stream=None, workspace=None):
    """out[M, N] = bf16(x[M, K] . weight[N, K]^T) on the matrix cores; with
    a workspace (gemm_workspace_bytes) K may be split where the tiles would
    leave CUs idle."""

    n, k = _matrix(weight, "weight")
    m = _rows(x, "x", k)
    _bf16(out, "out", m * n)
    if workspace is None:
        call("cascade_gemm_bf16", x.data_ptr(), weight.data_ptr(), out.data_ptr(),
             m, n, k, stream_handle(stream))
    else:
        ws, ws_bytes = _ws(workspace)
        call("cascade_gemm_ws_bf16", x.data_ptr(), weight.data_ptr(),
             out.data_ptr(), m, n, k, ws, ws_bytes, stream_handle(stream))
    return out


def gemm_residual(x, weight, residual, out, stream=None, workspace=None):
    """out = bf16(residual + bf16(x . weight^T)); out may be residual; with a
    workspace K may be split as in gemm()."""

    n, k = _matrix(weight, "weight")
    m = _rows(x, "x", k)
    _bf16(residual, "residual", m * n)
    _bf16(out, "out", m * n)
    if workspace is None:
        call("cascade_gemm_residual_bf16", x.data_ptr(), weight.data_ptr(),
             residual.data_ptr(), out.data_ptr(), m, n, k, stream_handle(stream))
    else:
        ws, ws_bytes = _ws(workspace)
        call("cascade_gemm_residual_ws_bf16", x.data_ptr(), weight.data_ptr(),
             residual.data_ptr(), out.data_ptr(), m, n, k, ws, ws_bytes,
             stream_handle(stream))
    return out


def gemm_f32out(x, weight, out, stream=None):
    """fp32 out[M, N] = x . weight^T (no rounding; LM-head logits)."""

    n, k = _matrix(weight, "weight")
    m = _rows(x, "x", k)
    require_device(out, "out", torch.float32, m * n)
    call("cascade_gemm_f32out_bf16", x.data_ptr(), weight.data_ptr(),
         out.data_ptr(), m, n, k, stream_handle(stream))
    return out


def gate_up_swiglu_gemm(x, w_gate, w_up, out, stream=None):
    n, k = _matrix(w_gate, "w_gate")
    if tuple(_matrix(w_up, "w_up")) != (n, k):
        raise ValueError("gate and up matrices differ in shape")
    m = _rows(x, "x", k)
    _bf16(out, "out", m * n)
    call("cascade_gate_up_swiglu_gemm_bf16", x.data_ptr(), w_gate.data_ptr(),
         w_up.data_ptr(), out.data_ptr(), m, n, k, stream_handle(stream))
    return out


def gate_silu_gemm(x, w_gate, out, stream=None):
    n, k = _matrix(w_gate, "w_gate")
    m = _rows(x, "x", k)
    _bf16(out, "out", m * n)
    call("cascade_gate_silu_gemm_bf16", x.data_ptr(), w_gate.data_ptr(),
         out.data_ptr(), m, n, k, stream_handle(stream))
    return out


def up_mul_gemm(x, w_up, gate, out, stream=None):
    n, k = _matrix(w_up, "w_up")
    m = _rows(x, "x", k)
    _bf16(gate, "gate", m * n)
    _bf16(out, "out", m * n)
    call("cascade_up_mul_gemm_bf16", x.data_ptr(), w_up.data_ptr(),
         gate.data_ptr(), out.data_ptr(), m, n, k, stream_handle(stream))
    return out


def _kv_span_ok(buf, name, heads, kv_head_stride, end_slot, head_dim=128):
    require_device(buf, name, torch.bfloat16, contiguous=False)
    if kv_head_stride < end_slot * head_dim:
        raise ValueError("{}: slot {} is outside the head stride".format(
            name, end_slot - 1))
    end = buf.storage_offset() + (heads - 1) * kv_head_stride + end_slot * head_dim
    if end > buf.untyped_storage().nbytes() // 2:
        raise ValueError("{} cannot hold {} heads up to slot {}".format(
            name, heads, end_slot))


def qkv_rope_gemm(x, wq, wk, wv, rope_cos, rope_sin, pos0, q_out, k_out,
                  v_out, kv_head_stride, slot0, stream=None):
    """Q/K/V GEMMs of M token rows + RoPE + KV write.

    rope_cos / rope_sin are whole [positions, 64] bf16 tables; row r uses
    position pos0 + r and cache slot slot0 + r; k_out / v_out start at
    position 0 of KV head 0 of the layer's cache.
    """

    k = None
    sizes = []
    for name, w in (("wq", wq), ("wk", wk), ("wv", wv)):
        if w is None:
            sizes.append(0)
            continue
        n, kk = _matrix(w, name)
        if k is not None and kk != k:
            raise ValueError("q/k/v matrices disagree on K")
        k = kk
        sizes.append(n)
    if k is None:
        raise ValueError("at least one of wq, wk, wv is required")
    nq, nk, nv = sizes
    m = _rows(x, "x", k)
    positions = 0
    if nq or nk:
        _bf16(rope_cos, "rope_cos")
        _bf16(rope_sin, "rope_sin", rope_cos.numel())
        positions = rope_cos.numel() // 64
    if nq:
        _bf16(q_out, "q_out", m * nq)
    if nk:
        _kv_span_ok(k_out, "k_out", nk // 128, kv_head_stride, slot0 + m)
    if nv:
        _kv_span_ok(v_out, "v_out", nv // 128, kv_head_stride, slot0 + m)

    def ptr(t, used=True):
        return t.data_ptr() if (used and t is not None) else 0

    call("cascade_qkv_rope_gemm_bf16", x.data_ptr(), m, ptr(wq), ptr(wk),
         ptr(wv), nq, nk, nv, k, ptr(rope_cos, nq or nk),
         ptr(rope_sin, nq or nk), positions, int(pos0), ptr(q_out, nq),
         ptr(k_out, nk), ptr(v_out, nv), int(kv_head_stride), int(slot0),
         stream_handle(stream))


def prefill_attention(q, k_cache, v_cache, kv_head_stride, past, tokens, out,
                      scale, n_q_heads=32, n_kv_heads=8, head_dim=128,
                      stream=None):
    """Causal GQA attention of ``tokens`` query rows at slots past .. past +
    tokens - 1 over a layer cache (views from position 0 of KV head 0)."""

    width = n_q_heads * head_dim
    _bf16(q, "q", tokens * width)
    _bf16(out, "out", tokens * width)
    for name, buf in (("k_cache", k_cache), ("v_cache", v_cache)):
        _kv_span_ok(buf, name, n_kv_heads, kv_head_stride, past + tokens,
                    head_dim)
    call("cascade_prefill_attention_bf16", q.data_ptr(), k_cache.data_ptr(),
         v_cache.data_ptr(), int(kv_head_stride), int(past), int(tokens),
         n_q_heads, n_kv_heads, head_dim, float(scale), out.data_ptr(),
         stream_handle(stream))
    return out


def attention_workspace_bytes(max_len, n_q_heads=32, n_kv_heads=8,
                              head_dim=128):
    size = load().cascade_decode_attention_workspace_bytes(
        int(max_len), int(n_q_heads), int(n_kv_heads), int(head_dim)
    )
    if size == 0:
        raise ValueError("unsupported attention shape")
    return int(size)


def decode_attention(q, k_cache, v_cache, kv_head_stride, length, out,
                     workspace, scale, n_q_heads=32, n_kv_heads=8,
                     head_dim=128, stream=None):
    """One-token GQA attention over positions [0, length) of a layer cache.

    k_cache / v_cache are views starting at position 0 of KV head 0.
    """

    _bf16(q, "q", n_q_heads * head_dim)
    _bf16(out, "out", n_q_heads * head_dim)
    for name, buf in (("k_cache", k_cache), ("v_cache", v_cache)):
        require_device(buf, name, torch.bfloat16, contiguous=False)
        end = buf.storage_offset() + (n_kv_heads - 1) * kv_head_stride + (
            length * head_dim
        )
        if end > buf.untyped_storage().nbytes() // 2:
            raise ValueError("{} is too small for length {}".format(name, length))
    require_device(workspace, "workspace", torch.uint8)
    call("cascade_decode_attention_bf16", q.data_ptr(), k_cache.data_ptr(),
         v_cache.data_ptr(), int(kv_head_stride), int(length), n_q_heads,
         n_kv_heads, head_dim, float(scale), out.data_ptr(),
         workspace.data_ptr(), workspace.numel(), stream_handle(stream))
    return out


def _length_word(length, capacity):
    require_device(length, "length", torch.int64, 1)
    if int(capacity) <= 0:
        raise ValueError("capacity must be positive")


def qkv_rope_at(wq, wk, wv, x, norm_weight, eps, rope_cos, rope_sin, q_out,
                k_cache, v_cache, kv_head_stride, length, capacity,
                stream=None):
    """q|k|v + RoPE + KV write at the position *length - 1 held on the device.

    rope_cos / rope_sin are the [capacity, 64] tables; k_cache / v_cache are
    views at position 0 of KV head 0 of the layer cache.
    """

    _length_word(length, capacity)
    nq = 0 if wq is None else _matrix(wq, "wq")[0]
    nk = 0 if wk is None else _matrix(wk, "wk")[0]
    nv = 0 if wv is None else _matrix(wv, "wv")[0]
    k = _matrix(next(w for w in (wq, wk, wv) if w is not None), "w")[1]
    _bf16(x, "x", k)
    if norm_weight is not None:
        _bf16(norm_weight, "norm_weight", k)
    if nq or nk:
        _bf16(rope_cos, "rope_cos", capacity * 64)
        _bf16(rope_sin, "rope_sin", capacity * 64)
    if nq:
        _bf16(q_out, "q_out", nq)
    for name, buf, heads in (("k_cache", k_cache, nk // 128),
                             ("v_cache", v_cache, nv // 128)):
        if heads:
            require_device(buf, name, torch.bfloat16, contiguous=False)
            if buf.storage_offset() + (heads - 1) * kv_head_stride + (
                capacity * 128
            ) > buf.untyped_storage().nbytes() // 2:
                raise ValueError("{} cannot hold {} positions".format(name, capacity))

    def ptr(t):
        return 0 if t is None else t.data_ptr()

    call("cascade_qkv_rope_at_bf16", ptr(wq), ptr(wk), ptr(wv), nq, nk, nv, k,
         x.data_ptr(), ptr(norm_weight), float(eps),
         ptr(rope_cos) if (nq or nk) else 0,
         ptr(rope_sin) if (nq or nk) else 0,
         ptr(q_out) if nq else 0, ptr(k_cache) if nk else 0,
         ptr(v_cache) if nv else 0, int(kv_head_stride), length.data_ptr(),
         int(capacity), stream_handle(stream))


def decode_attention_at(q, k_cache, v_cache, kv_head_stride, length, capacity,
                        out, workspace, scale, n_q_heads=32, n_kv_heads=8,
                        head_dim=128, stream=None):
    """decode_attention over positions [0, *length) held on the device; the
    split plan follows ``capacity``."""

    _length_word(length, capacity)
    _bf16(q, "q", n_q_heads * head_dim)
    _bf16(out, "out", n_q_heads * head_dim)
    for name, buf in (("k_cache", k_cache), ("v_cache", v_cache)):
        require_device(buf, name, torch.bfloat16, contiguous=False)
        end = buf.storage_offset() + (n_kv_heads - 1) * kv_head_stride + (
            capacity * head_dim
        )
        if end > buf.untyped_storage().nbytes() // 2:
            raise ValueError("{} is too small for capacity {}".format(name, capacity))
    require_device(workspace, "workspace", torch.uint8)
    call("cascade_decode_attention_at_bf16", q.data_ptr(), k_cache.data_ptr(),
         v_cache.data_ptr(), int(kv_head_stride), length.data_ptr(),
         int(capacity), n_q_heads, n_kv_heads, head_dim, float(scale),
         out.data_ptr(), workspace.data_ptr(), workspace.numel(),
         stream_handle(stream))
    return out


def _fused_attention_args(sync, error_flag, n_kv_heads):
    require_device(sync, "sync", torch.uint8, ATTENTION_SYNC_BYTES)
    require_device(error_flag, "error_flag", torch.int32, 1)
    if n_kv_heads != FUSED_ATTENTION_KV_HEADS:
        raise ValueError("the fused attention needs {} KV heads".format(
            FUSED_ATTENTION_KV_HEADS))


def decode_attention_fused(q, k_cache, v_cache, kv_head_stride, length, out,
                           workspace, sync, error_flag, scale, n_q_heads=32,
                           n_kv_heads=8, head_dim=128, stream=None):
    """decode_attention with the split merge inside the attention launch
    (bit-identical results).  ``sync``: ATTENTION_SYNC_BYTES zero-filled
    bytes, left zeroed; ``error_flag``: int32 word that receives
    ATTN_EPLACEMENT / ATTN_ETIMEOUT.  length >= FUSED_ATTENTION_MIN_LEN."""

    if int(length) < FUSED_ATTENTION_MIN_LEN:
        raise ValueError("the fused attention needs length >= {}".format(
            FUSED_ATTENTION_MIN_LEN))
    _fused_attention_args(sync, error_flag, n_kv_heads)
    _bf16(q, "q", n_q_heads * head_dim)
    _bf16(out, "out", n_q_heads * head_dim)
    for name, buf in (("k_cache", k_cache), ("v_cache", v_cache)):
        require_device(buf, name, torch.bfloat16, contiguous=False)
        end = buf.storage_offset() + (n_kv_heads - 1) * kv_head_stride + (
            length * head_dim
        )
        if end > buf.untyped_storage().nbytes() // 2:
            raise ValueError("{} is too small for length {}".format(name, length))
    require_device(workspace, "workspace", torch.uint8)
    call("cascade_decode_attention_fused_bf16", q.data_ptr(), k_cache.data_ptr(),
         v_cache.data_ptr(), int(kv_head_stride), int(length), n_q_heads,
         n_kv_heads, head_dim, float(scale), out.data_ptr(),
         workspace.data_ptr(), workspace.numel(), sync.data_ptr(),
         error_flag.data_ptr(), stream_handle(stream))
    return out


def decode_attention_fused_at(q, k_cache, v_cache, kv_head_stride, length,
                              capacity, out, workspace, sync, error_flag, scale,
                              n_q_heads=32, n_kv_heads=8, head_dim=128,
                              stream=None):
    """decode_attention_at with the split merge inside the attention launch;
    capacity >= FUSED_ATTENTION_MIN_LEN."""

    _length_word(length, capacity)
    if int(capacity) < FUSED_ATTENTION_MIN_LEN:
        raise ValueError("the fused attention needs capacity >= {}".format(
            FUSED_ATTENTION_MIN_LEN))
    _fused_attention_args(sync, error_flag, n_kv_heads)
    _bf16(q, "q", n_q_heads * head_dim)
    _bf16(out, "out", n_q_heads * head_dim)
    for name, buf in (("k_cache", k_cache), ("v_cache", v_cache)):
        require_device(buf, name, torch.bfloat16, contiguous=False)
        end = buf.storage_offset() + (n_kv_heads - 1) * kv_head_stride + (
            capacity * head_dim
        )
        if end > buf.untyped_storage().nbytes() // 2:
            raise ValueError("{} is too small for capacity {}".format(name, capacity))
    require_device(workspace, "workspace", torch.uint8)
    call("cascade_decode_attention_fused_at_bf16", q.data_ptr(),
         k_cache.data_ptr(), v_cache.data_ptr(), int(kv_head_stride),
         length.data_ptr(), int(capacity), n_q_heads, n_kv_heads, head_dim,
         float(scale), out.data_ptr(), workspace.data_ptr(), workspace.numel(),
         sync.data_ptr(), error_flag.data_ptr(), stream_handle(stream))
    return out


def decode_step_begin(table, ids, out, length, history, error_flag=None,
                      stream=None):
    """Gather table[ids[0]] into out, then history[L] = ids[0] and
    *length = L + 1 (L = *length on entry, 0 <= L < history.numel())."""

    vocab, hidden = _matrix(table, "table")
    require_device(ids, "ids", torch.int64, contiguous=False)
    _bf16(out, "out", hidden)
    require_device(history, "history", torch.int64)
    _length_word(length, history.numel())
    if error_flag is not None:
        require_device(error_flag, "error_flag", torch.int32, 1)
    call("cascade_decode_step_begin_bf16", table.data_ptr(), vocab, hidden,
         ids.data_ptr(), out.data_ptr(), length.data_ptr(), history.data_ptr(),
         history.numel(), 0 if error_flag is None else error_flag.data_ptr(),
         stream_handle(stream))
    return out


def lm_head_workspace_bytes(rows, top_k):
    size = load().cascade_lm_head_workspace_bytes(int(rows), int(top_k))
    if size == 0:
        raise ValueError("unsupported LM-head shape (rows={}, top_k={})".format(
            rows, top_k))
    return int(size)


def lm_head_topk(weight, hidden, top_k, row_offset, first_chunk, workspace,
                 out_values, out_indices, logits_out=None, stream=None):
    rows, k = _matrix(weight, "weight")
    _bf16(hidden, "hidden", k)
    require_device(workspace, "workspace", torch.uint8)
    require_device(out_values, "out_values", torch.float32, top_k)
    require_device(out_indices, "out_indices", torch.int64, top_k)
    if logits_out is not None:
        require_device(logits_out, "logits_out", torch.float32, rows)
    call("cascade_lm_head_topk_bf16", weight.data_ptr(), rows, k,
         int(row_offset), hidden.data_ptr(), int(top_k),
         1 if first_chunk else 0,
         0 if logits_out is None else logits_out.data_ptr(),
         workspace.data_ptr(), workspace.numel(), out_values.data_ptr(),
         out_indices.data_ptr(), stream_handle(stream))


def topk_f32(logits, top_k, workspace, out_values, out_indices, stream=None):
    """Exact top-k of one row of fp32 logits already on the device (value
    descending, index ascending; lm_head_topk's order) into out_values /
    out_indices.  workspace: lm_head_workspace_bytes(rows, top_k) bytes."""

    require_device(logits, "logits", torch.float32)
    rows = logits.numel()
    require_device(workspace, "workspace", torch.uint8)
    require_device(out_values, "out_values", torch.float32, top_k)
    require_device(out_indices, "out_indices", torch.int64, top_k)
    call("cascade_topk_f32", logits.data_ptr(), rows, int(top_k),
         workspace.data_ptr(), workspace.numel(), out_values.data_ptr(),
         out_indices.data_ptr(), stream_handle(stream))


def embedding_gather(table, ids, out, error_flag=None, stream=None):
    vocab, hidden = _matrix(table, "table")
    require_device(ids, "ids", torch.int64)
    _bf16(out, "out", ids.numel() * hidden)
    if error_flag is not None:
        require_device(error_flag, "error_flag", torch.int32, 1)
    call("cascade_embedding_gather_bf16", table.data_ptr(), vocab, hidden,
         ids.data_ptr(), ids.numel(), out.data_ptr(),
         0 if error_flag is None else error_flag.data_ptr(),
         stream_handle(stream))
    return out


def hbm_read(src, sink, blocks=0, stream=None):
    require_device(src, "src")
    require_device(sink, "sink", torch.float32, 1)
    call("cascade_hbm_read", src.data_ptr(),
         src.numel() * src.element_size(), sink.data_ptr(), int(blocks),
         stream_handle(stream))


def device_copy(dst, src, stream=None):
    require_device(src, "src")
    require_device(dst, "dst", src.dtype, src.numel())
    call("cascade_device_copy", dst.data_ptr(), src.data_ptr(),
         src.numel() * src.element_size(), stream_handle(stream))


# ------------------------------------------------------------ copy pipeline


def memcpy_h2d_async(dst, src, nbytes, stream):
    """hipMemcpyAsync host->device of nbytes; src must be page-locked."""

    require_device(dst, "dst", contiguous=False)
    if src.device.type != "cpu":
        raise ValueError("src must be a host tensor")
    if nbytes > src.numel() * src.element_size():
        raise ValueError("copy larger than the source")
    if nbytes > dst.numel() * dst.element_size():
        raise ValueError("copy larger than the destination")
    call("cascade_memcpy_h2d_async", dst.data_ptr(), src.data_ptr(),
         int(nbytes), stream_handle(stream))


def default_copy_threads():
    """Threads for host staging copies: this process's CPUs, at most 8.

    Eight threads stage at about twice the link rate.  More slow the H2D
    copies that read host memory at the same time: on MI355X, config 5
    prefill took 286 ms with 16 threads, 277 ms with 6 to 10, and 281 ms
    with 4."""

    try:
        cpus = len(os.sched_getaffinity(0))
    except AttributeError:  # not Linux
        cpus = os.cpu_count() or 1
    return max(1, min(8, cpus))


def _host_copy_bytes(dst, src):
    for name, t in (("dst", dst), ("src", src)):
        if not isinstance(t, torch.Tensor) or t.device.type != "cpu":
            raise ValueError("{} must be a host tensor".format(name))
        if not t.is_contiguous():
            raise ValueError("{} must be contiguous".format(name))
    nbytes = src.numel() * src.element_size()
    if dst.numel() * dst.element_size() != nbytes:
        raise ValueError("host_copy needs equal byte sizes")
    return nbytes


def host_copy(dst, src, threads=None):
    """dst.copy_(src) for contiguous host tensors of equal byte size, with
    the library's multi-threaded non-temporal memcpy (threads started for
    this call only; the GIL is released for the duration of the copy)."""

    nbytes = _host_copy_bytes(dst, src)
    call("cascade_host_copy", dst.data_ptr(), src.data_ptr(), nbytes,
         int(threads or default_copy_threads()))
    return dst


def device_numa_node(device=None):
    """NUMA node of the host bridge a GPU sits behind, from the PCI
    device's sysfs entry; -1 when there is no GPU, the platform reports
    none (a one-node host writes -1 there too) or the entry is missing."""

    if not torch.cuda.is_available():
        return -1
    props = torch.cuda.get_device_properties(
        torch.cuda.current_device() if device is None else device)
    path = "/sys/bus/pci/devices/{:04x}:{:02x}:{:02x}.0/numa_node".format(
        props.pci_domain_id, props.pci_bus_id, props.pci_device_id)
    try:
        with open(path) as f:
            return int(f.read().strip())
    except (OSError, ValueError):
        return -1


class _PoolState:
    """The native pool handle and the count of copies running on it, shared
    by a CopyPool and its finalizer."""

    __slots__ = ("handle", "busy", "lock")

    def __init__(self, handle):
        self.handle = handle
        self.busy = 0
        self.lock = threading.Lock()


def _destroy_copy_pool(state):
    with state.lock:
        handle, state.handle = state.handle, 0
        if not handle or state.busy:
            # A copy is still running on the pool: only a daemon staging
            # thread at interpreter exit can be inside one when the pool is
            # finalized.  New copies are refused from here on, and the
            # native pool, whose helpers that copy is using, is left to the
            # process exit.
            return
    call("cascade_copy_pool_destroy", handle)


class CopyPool:
    """A caller-owned pool for the multi-threaded host copy: ``threads``
    threads in all (the caller and threads - 1 helpers), the helpers bound
    to the CPUs of ``numa_node`` when it is >= 0.  ``close`` joins them (as
    does garbage collection, or interpreter exit, of an unclosed pool).  A
    pool closed or finalized while a copy runs on it refuses new copies and
    leaves the native pool alive for that copy (it is not destroyed then)."""

    def __init__(self, threads=None, numa_node=-1):
        handle = _U64(0)
        call("cascade_copy_pool_create", int(threads or default_copy_threads()),
             int(numa_node), ctypes.byref(handle))
        self._state = _PoolState(handle.value)
        self._finalizer = weakref.finalize(self, _destroy_copy_pool, self._state)
        threads_out, bound = _INT(0), _INT(0)
        call("cascade_copy_pool_info", handle.value, ctypes.byref(threads_out),
             ctypes.byref(bound))
        self.threads = threads_out.value
        self.bound_cpus = bound.value
        self.numa_node = int(numa_node)

    @property
    def handle(self):
        return self._state.handle

    def copy(self, dst, src):
        nbytes = _host_copy_bytes(dst, src)
        state = self._state
        with state.lock:
            handle = state.handle
            if not handle:
                raise RuntimeError("the copy pool is closed")
            state.busy += 1
        try:
            call("cascade_copy_pool_copy", handle, dst.data_ptr(),
                 src.data_ptr(), nbytes)
        finally:
            with state.lock:
                state.busy -= 1
        return dst

    def close(self):
        self._finalizer()  # destroys the native pool, once

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class HipEvent:
    """A hipEvent_t created through the C ABI (duck-types torch.cuda.Event
    for ``record``, ``wait``, ``synchronize``, ``query`` and
    ``elapsed_time``)."""

    __slots__ = ("handle", "timing")

    def __init__(self, enable_timing=False):
        handle = _U64(0)
        call("cascade_event_create", ctypes.byref(handle),
             1 if enable_timing else 0)
        self.handle = handle.value
        self.timing = bool(enable_timing)

    def record(self, stream=None):
        call("cascade_event_record", self.handle, stream_handle(stream))

    def wait(self, stream=None):
        """Make ``stream`` wait for this event (hipStreamWaitEvent)."""

        call("cascade_stream_wait_event", stream_handle(stream), self.handle)

    def synchronize(self):
        call("cascade_event_synchronize", self.handle)

    def query(self):
        code = load().cascade_event_query(self.handle)
        if code in (0, 1):
            return code == 0
        _check("cascade_event_query", code)
        return False

    def elapsed_time(self, end):
        ms = _F(0.0)
        call("cascade_event_elapsed_ms", self.handle, end.handle,
             ctypes.byref(ms))
        return float(ms.value)

    def __del__(self):
        lib = _lib
        if lib is not None and self.handle:
            try:
                lib.cascade_event_destroy(self.handle)
            except Exception:  # interpreter shutdown
                pass
            self.handle = 0


def time_next_launch(start, stop):
    """Bind two timing HipEvents (or None) to this thread's next kernel
    launch through the library: their elapsed time is that kernel's own
    duration.  ``time_next_launch(None, None)`` clears pending events."""

    call("cascade_time_next_launch", start.handle if start else 0,
         stop.handle if stop else 0)


def stream_wait(stream, event):
    """stream waits for event (either a HipEvent or a torch.cuda.Event)."""

    if isinstance(event, HipEvent):
        event.wait(stream)
    else:
        stream.wait_event(event)
