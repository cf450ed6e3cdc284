// MFMA bf16 GEMM family for prefill (M = prompt tokens > 1) on gfx950.
//
//   Y[M, N] = epilogue(X[M, K] . W[N, K]^T)
//
// X holds the (already RMS-normalised) token rows, W is a weight matrix in
// the reference's row-major [out_features, in_features] layout, so both
// operands are read along K.  This replaces F.linear with a [1, S, 4096]
// input (layer_streaming/llama31.py:241-279 during the prefill call, and the
// resident LM head, llama31.py:330-334).
//
// Tiling.  A workgroup of 4 waves computes a 128 x 128 output tile; K is
// walked in 64-deep slabs staged through LDS (double buffered, one barrier
// per slab: the next slab's global loads are issued before the current
// slab's MFMAs and written to the other buffer after them).  Each wave owns
// 64 rows x 64 columns = 4 x 4 v_mfma_f32_16x16x32_bf16 tiles; per slab it
// reads 8 A and 8 B fragments (16 bytes a lane) from LDS and issues 32
// MFMAs.  LDS rows are padded to 72 bf16 (144 bytes) so the 16 rows a
// fragment read touches start 4 banks apart.
//
// A wave's 64 columns are not contiguous: column block j (16 wide) of wave
// wn is at 32 wn + 16 (j & 1) + 64 (j >> 1) of the tile, so blocks j and
// j + 2 of one lane hold columns c and c + 64.  That pairs the two halves
// of a head (RoPE's rotate_half) and, with gate rows in tile columns 0..63
// and up rows in 64..127, a gate and its up value, so those epilogues need
// no data exchange.
//
// Tile order.  Workgroups are dispatched round-robin over the 8 XCDs (each
// with its own L2); workgroup b runs logical tile (b % 8) * (grid / 8) +
// b / 8, so an XCD walks a contiguous range of logical tiles, which are
// ordered in groups of 8 M-tiles (column-major inside a group).  An XCD's
// first 64 tiles then form an 8 x 8 block that reuses every X and W slab it
// loads 8 times from its L2.
//
// Epilogues reproduce the reference's bf16 rounding points (the GEMV family
// in gemv.hip applies the same ones):
//   store     y = bf16(acc)                               F.linear
//   residual  y = bf16(res + bf16(acc))                   residual + F.linear
//   qkv_rope  q/k heads: bf16 RoPE at position pos0 + row, then the q rows
//             or the layer's KV cache at slot slot0 + row;  v heads: cache
//   swiglu    bf16(bf16(silu(bf16(g))) * bf16(u))
//   silu / mul  the matrix-granularity halves of swiglu
//   f32       fp32 output (LM-head logits, not rounded)
#include "cascade_device.h"
#include "cascade_internal.h"

namespace cascade {

enum GemmEpilogue : int {
  kGemmStore = 0,
  kGemmResidual = 1,
  kGemmQkvRope = 2,
  kGemmSwiglu = 3,
  kGemmSilu = 4,
  kGemmMul = 5,
  kGemmF32 = 6,
};

constexpr int kTileM = 128;
constexpr int kTileN = 128;
constexpr int kTileK = 64;
constexpr int kGemmWaves = 4;
constexpr int kGemmThreads = kGemmWaves * kWave;
constexpr int kLdsRow = kTileK + 8;           // bf16 elements per LDS row
constexpr int kLdsTile = kTileM * kLdsRow;    // one operand tile (128 rows)
constexpr int kRowsPerPass = kGemmThreads / 8;  // 8 x 16 B pieces per row
constexpr int kPasses = kTileM / kRowsPerPass;  // 4 loads per operand
constexpr int kGroupM = 8;
constexpr int kXcds = 8;
constexpr int kGemmHead = 128;
constexpr int kGemmHalfHead = 64;

struct GemmArgs {
  const uint16_t *x;  // [m, k]
  const uint16_t *w0;  // store/residual/silu/mul/f32: W; qkv: Wq; swiglu: Wgate
  const uint16_t *w1;  // qkv: Wk; swiglu: Wup
  const uint16_t *w2;  // qkv: Wv
  int64_t n0, n1, n2;  // rows of w0 / w1 / w2 (swiglu: n0 = n_half)
  int64_t m, k;
  uint16_t *y;  // [m, ldy] (qkv: the q rows, ldy = n0)
  int64_t ldy;
  float *yf;    // kGemmF32 output [m, ldy]
  const uint16_t *aux;  // residual (kGemmResidual) or gate (kGemmMul), [m, ldy]
  const uint16_t *rope_cos;  // [positions, 64] bf16
  const uint16_t *rope_sin;
  int64_t pos0;
  uint16_t *k_out;  // position 0 of KV head 0 of this layer's K cache
  uint16_t *v_out;
  int64_t kv_head_stride;
  int64_t slot0;
  int32_t tiles_m, tiles_n, tiles;
};

__device__ __forceinline__ float gemm_silu(float g) {
  return g / (1.0f + expf(-g));
}

// Logical tile of this workgroup (false: padding workgroup, no work).
__device__ __forceinline__ bool gemm_tile(const GemmArgs &a, int &tm, int &tn) {
  const int per = static_cast<int>(gridDim.x) / kXcds;
  const int t = static_cast<int>(blockIdx.x % kXcds) * per +
                static_cast<int>(blockIdx.x / kXcds);
  if (t >= a.tiles) return false;
  const int group_size = kGroupM * a.tiles_n;
  const int group = t / group_size;
  const int first = group * kGroupM;
  const int gm = min(kGroupM, a.tiles_m - first);
  const int r = t - group * group_size;
  tm = first + r % gm;
  tn = r / gm;
  return true;
}

// Weight row feeding tile column r (0..127) of tile column-block tn.
template <int EPI>
__device__ __forceinline__ const uint16_t *gemm_w_row(const GemmArgs &a,
                                                      int tn, int r) {
  if constexpr (EPI == kGemmSwiglu) {
    const int64_t i = static_cast<int64_t>(tn) * kGemmHalfHead + (r & 63);
    return (r < 64 ? a.w0 : a.w1) + i * a.k;
  } else if constexpr (EPI == kGemmQkvRope) {
    const int64_t hq = a.n0 / kGemmHead, hk = a.n1 / kGemmHead;
    const uint16_t *base;
    int64_t lh;
    if (tn < hq) {
      base = a.w0;
      lh = tn;
    } else if (tn < hq + hk) {
      base = a.w1;
      lh = tn - hq;
    } else {
      base = a.w2;
      lh = tn - hq - hk;
    }
    return base + (lh * kGemmHead + r) * a.k;
  } else {
    // rows past n (a partial last tile) repeat row n - 1; not stored
    int64_t row = static_cast<int64_t>(tn) * kTileN + r;
    row = row < a.n0 ? row : a.n0 - 1;
    return a.w0 + row * a.k;
  }
}

// Column of tile column-block j (0..3) of wave column wn for lane row lr.
__device__ __forceinline__ int gemm_col(int wn, int j, int lr) {
  return 32 * wn + 16 * (j & 1) + 64 * (j >> 1) + lr;
}

template <int EPI>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs &a, int tm, int tn,
                                              int wm, int wn, int lane,
                                              const f32x4 (&acc)[4][4]) {
  const int lr = lane & 15;
  const int lq = lane >> 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t row = static_cast<int64_t>(tm) * kTileM + 64 * wm + 16 * i +
                          4 * lq + r;
      if (row >= a.m) continue;
      if constexpr (EPI == kGemmQkvRope) {
        const int64_t hq = a.n0 / kGemmHead, hk = a.n1 / kGemmHead;
        const int64_t pos = a.pos0 + row;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int d = gemm_col(wn, j, lr);  // 0..63
          const float xa = round_bf16(acc[i][j][r]);
          const float xb = round_bf16(acc[i][j + 2][r]);
          uint16_t oa, ob;
          if (tn < hq + hk) {
            // x*cos + rotate_half(x)*sin, products and sum rounded to bf16
            // (apply_rotary_pos_emb on bf16 tensors)
            const float c = bf16_to_f32(a.rope_cos[pos * kGemmHalfHead + d]);
            const float s = bf16_to_f32(a.rope_sin[pos * kGemmHalfHead + d]);
            oa = f32_to_bf16(round_bf16(xa * c) + round_bf16(-xb * s));
            ob = f32_to_bf16(round_bf16(xb * c) + round_bf16(xa * s));
          } else {
            oa = f32_to_bf16(xa);
            ob = f32_to_bf16(xb);
          }
          uint16_t *dst;
          if (tn < hq) {
            dst = a.y + row * a.ldy + static_cast<int64_t>(tn) * kGemmHead;
          } else if (tn < hq + hk) {
            dst = a.k_out + (tn - hq) * a.kv_head_stride +
                  (a.slot0 + row) * kGemmHead;
          } else {
            dst = a.v_out + (tn - hq - hk) * a.kv_head_stride +
                  (a.slot0 + row) * kGemmHead;
          }
          dst[d] = oa;
          dst[d + kGemmHalfHead] = ob;
        }
      } else if constexpr (EPI == kGemmSwiglu) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int64_t col =
              static_cast<int64_t>(tn) * kGemmHalfHead + gemm_col(wn, j, lr);
          const float g = round_bf16(acc[i][j][r]);
          const float u = round_bf16(acc[i][j + 2][r]);
          const float s = round_bf16(gemm_silu(g));
          a.y[row * a.ldy + col] = f32_to_bf16(s * u);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t col =
              static_cast<int64_t>(tn) * kTileN + gemm_col(wn, j, lr);
          if (col >= a.n0) continue;
          const int64_t at = row * a.ldy + col;
          if constexpr (EPI == kGemmF32) {
            a.yf[at] = acc[i][j][r];
            continue;
          }
          const float v = round_bf16(acc[i][j][r]);
          float out;
          if constexpr (EPI == kGemmStore) {
            out = v;
          } else if constexpr (EPI == kGemmResidual) {
            out = bf16_to_f32(a.aux[at]) + v;
          } else if constexpr (EPI == kGemmSilu) {
            out = gemm_silu(v);
          } else {  // kGemmMul
            out = bf16_to_f32(a.aux[at]) * v;
          }
          a.y[at] = f32_to_bf16(out);
        }
      }
    }
  }
}

template <int EPI>
__global__ __launch_bounds__(kGemmThreads) void gemm_kernel(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[2][2][kLdsTile];
  int tm, tn;
  if (!gemm_tile(a, tm, tn)) return;  // whole workgroup: no barrier skipped
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int lr = lane & 15;
  const int lk = (lane >> 4) * 8;

  // Global -> LDS staging: thread t moves 16-byte piece t % 8 of rows
  // t / 8 + 32 p (p = 0..3) of both operands.  X rows past m repeat row
  // m - 1 (valid memory; their results are not stored).
  const int piece = tid & 7;
  const int srow = tid >> 3;
  const uint16_t *xrow[kPasses];
  const uint16_t *wrow[kPasses];
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    const int r = srow + kRowsPerPass * p;
    int64_t xr = static_cast<int64_t>(tm) * kTileM + r;
    xr = xr < a.m ? xr : a.m - 1;
    xrow[p] = a.x + xr * a.k + piece * 8;
    wrow[p] = gemm_w_row<EPI>(a, tn, r) + piece * 8;
  }

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  u32x4 rx[kPasses], rw[kPasses];
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    rx[p] = *reinterpret_cast<const u32x4 *>(xrow[p]);
    rw[p] = *reinterpret_cast<const u32x4 *>(wrow[p]);
  }
  const int lds_at = srow * kLdsRow + piece * 8;
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    *reinterpret_cast<u32x4 *>(&lds[0][0][lds_at + p * kRowsPerPass * kLdsRow]) = rx[p];
    *reinterpret_cast<u32x4 *>(&lds[0][1][lds_at + p * kRowsPerPass * kLdsRow]) = rw[p];
  }
  __syncthreads();

  const int slabs = static_cast<int>(a.k / kTileK);
  for (int s = 0; s < slabs; ++s) {
    const int cur = s & 1;
    const bool more = s + 1 < slabs;
    if (more) {
      const int64_t k0 = static_cast<int64_t>(s + 1) * kTileK;
#pragma unroll
      for (int p = 0; p < kPasses; ++p) {
        rx[p] = *reinterpret_cast<const u32x4 *>(xrow[p] + k0);
        rw[p] = *reinterpret_cast<const u32x4 *>(wrow[p] + k0);
      }
    }
    const uint16_t *la = lds[cur][0];
    const uint16_t *lb = lds[cur][1];
#pragma unroll
    for (int ks = 0; ks < kTileK / 32; ++ks) {
      u32x4 af[4], bfr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = *reinterpret_cast<const u32x4 *>(
            la + (64 * wm + 16 * i + lr) * kLdsRow + 32 * ks + lk);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bfr[j] = *reinterpret_cast<const u32x4 *>(
            lb + gemm_col(wn, j, lr) * kLdsRow + 32 * ks + lk);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = mfma_16x16x32_bf16(af[i], bfr[j], acc[i][j]);
    }
    if (more) {
      const int nxt = cur ^ 1;
#pragma unroll
      for (int p = 0; p < kPasses; ++p) {
        *reinterpret_cast<u32x4 *>(&lds[nxt][0][lds_at + p * kRowsPerPass * kLdsRow]) = rx[p];
        *reinterpret_cast<u32x4 *>(&lds[nxt][1][lds_at + p * kRowsPerPass * kLdsRow]) = rw[p];
      }
    }
    __syncthreads();
  }
  gemm_epilogue<EPI>(a, tm, tn, wm, wn, lane, acc);
}

template <int EPI>
static hipError_t launch_gemm(GemmArgs &a, int64_t tiles_n, hipStream_t s) {
  const int64_t tiles_m = (a.m + kTileM - 1) / kTileM;
  const int64_t tiles = tiles_m * tiles_n;
  if (tiles > (int64_t{1} << 30)) return static_cast<hipError_t>(CASCADE_ESHAPE);
  a.tiles_m = static_cast<int32_t>(tiles_m);
  a.tiles_n = static_cast<int32_t>(tiles_n);
  a.tiles = static_cast<int32_t>(tiles);
  const int64_t grid = (tiles + kXcds - 1) / kXcds * kXcds;
  return launch_kernel(gemm_kernel<EPI>, dim3(static_cast<unsigned>(grid)),
                       dim3(kGemmThreads), 0, s, a);
}

// Shared argument checks: X [m, k], K a multiple of the 64-deep slab.
static int gemm_check_x(const void *x, int64_t m, int64_t k) {
  if (x == nullptr || m <= 0 || k <= 0 || m > (int64_t{1} << 24))
    return CASCADE_EINVAL;
  if (!aligned16(x)) return CASCADE_EALIGN;
  if (k % kTileK) return CASCADE_ESHAPE;
  return 0;
}

static int gemm_check_w(const void *w, int64_t n, int64_t granule) {
  if (w == nullptr || n <= 0) return CASCADE_EINVAL;
  if (!aligned16(w)) return CASCADE_EALIGN;
  if (n % granule) return CASCADE_ESHAPE;
  return 0;
}

}  // namespace cascade

using namespace cascade;

static int gemm_plain(int epi, const void *x, const void *w, const void *aux,
                      void *y, int64_t m, int64_t n, int64_t k, void *stream) {
  if (int e = gemm_check_x(x, m, k)) return e;
  if (int e = gemm_check_w(w, n, 1)) return e;
  if (y == nullptr) return CASCADE_EINVAL;
  if (!aligned16(y)) return CASCADE_EALIGN;
  if ((epi == kGemmResidual || epi == kGemmMul) && aux == nullptr)
    return CASCADE_EINVAL;
  GemmArgs a{};
  a.x = static_cast<const uint16_t *>(x);
  a.w0 = static_cast<const uint16_t *>(w);
  a.n0 = n;
  a.m = m;
  a.k = k;
  a.y = static_cast<uint16_t *>(y);
  a.yf = static_cast<float *>(y);
  a.ldy = n;
  a.aux = static_cast<const uint16_t *>(aux);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t tiles_n = (n + kTileN - 1) / kTileN;
  switch (epi) {
    case kGemmStore: return launch_gemm<kGemmStore>(a, tiles_n, s);
    case kGemmResidual: return launch_gemm<kGemmResidual>(a, tiles_n, s);
    case kGemmSilu: return launch_gemm<kGemmSilu>(a, tiles_n, s);
    case kGemmMul: return launch_gemm<kGemmMul>(a, tiles_n, s);
    default: return launch_gemm<kGemmF32>(a, tiles_n, s);
  }
}

extern "C" int cascade_gemm_bf16(const void *x, const void *w, void *y,
                                 int64_t m, int64_t n, int64_t k,
                                 void *stream) {
  return gemm_plain(kGemmStore, x, w, nullptr, y, m, n, k, stream);
}

extern "C" int cascade_gemm_f32out_bf16(const void *x, const void *w,
                                        float *y, int64_t m, int64_t n,
                                        int64_t k, void *stream) {
  return gemm_plain(kGemmF32, x, w, nullptr, y, m, n, k, stream);
}

extern "C" int cascade_gemm_residual_bf16(const void *x, const void *w,
                                          const void *residual, void *y,
                                          int64_t m, int64_t n, int64_t k,
                                          void *stream) {
  return gemm_plain(kGemmResidual, x, w, residual, y, m, n, k, stream);
}

extern "C" int cascade_gate_silu_gemm_bf16(const void *x, const void *w_gate,
                                           void *y, int64_t m, int64_t n,
                                           int64_t k, void *stream) {
  return gemm_plain(kGemmSilu, x, w_gate, nullptr, y, m, n, k, stream);
}

extern "C" int cascade_up_mul_gemm_bf16(const void *x, const void *w_up,
                                        const void *gate, void *y, int64_t m,
                                        int64_t n, int64_t k, void *stream) {
  return gemm_plain(kGemmMul, x, w_up, gate, y, m, n, k, stream);
}

extern "C" int cascade_gate_up_swiglu_gemm_bf16(const void *x,
                                                const void *w_gate,
                                                const void *w_up, void *y,
                                                int64_t m, int64_t n_half,
                                                int64_t k, void *stream) {
  if (int e = gemm_check_x(x, m, k)) return e;
  if (int e = gemm_check_w(w_gate, n_half, kGemmHalfHead)) return e;
  if (int e = gemm_check_w(w_up, n_half, kGemmHalfHead)) return e;
  if (y == nullptr) return CASCADE_EINVAL;
  if (!aligned16(y)) return CASCADE_EALIGN;
  GemmArgs a{};
  a.x = static_cast<const uint16_t *>(x);
  a.w0 = static_cast<const uint16_t *>(w_gate);
  a.w1 = static_cast<const uint16_t *>(w_up);
  a.n0 = n_half;
  a.m = m;
  a.k = k;
  a.y = static_cast<uint16_t *>(y);
  a.ldy = n_half;
  return launch_gemm<kGemmSwiglu>(a, n_half / kGemmHalfHead,
                                  static_cast<hipStream_t>(stream));
}

extern "C" int cascade_qkv_rope_gemm_bf16(
    const void *x, int64_t m, const void *wq, const void *wk, const void *wv,
    int64_t nq, int64_t nk, int64_t nv, int64_t k, const void *rope_cos,
    const void *rope_sin, int64_t rope_positions, int64_t pos0, void *q_out,
    void *k_out, void *v_out, int64_t kv_head_stride, int64_t slot0,
    void *stream) {
  if (int e = gemm_check_x(x, m, k)) return e;
  if (nq < 0 || nk < 0 || nv < 0 || nq + nk + nv == 0) return CASCADE_EINVAL;
  if ((nq % kGemmHead) || (nk % kGemmHead) || (nv % kGemmHead))
    return CASCADE_ESHAPE;
  if (nq && (wq == nullptr || q_out == nullptr)) return CASCADE_EINVAL;
  if (nk && (wk == nullptr || k_out == nullptr)) return CASCADE_EINVAL;
  if (nv && (wv == nullptr || v_out == nullptr)) return CASCADE_EINVAL;
  if ((nq && (!aligned16(wq) || !aligned16(q_out))) ||
      (nk && (!aligned16(wk) || !aligned16(k_out))) ||
      (nv && (!aligned16(wv) || !aligned16(v_out))))
    return CASCADE_EALIGN;
  if (nq || nk) {
    // every row's position must have a cos / sin row
    if (rope_cos == nullptr || rope_sin == nullptr || pos0 < 0 ||
        pos0 + m > rope_positions)
      return CASCADE_EINVAL;
  }
  if (nk || nv) {
    // every row's slot must lie inside each KV head's span
    if (slot0 < 0 || kv_head_stride < (slot0 + m) * kGemmHead ||
        (kv_head_stride & 7))
      return CASCADE_EINVAL;
  }
  GemmArgs a{};
  a.x = static_cast<const uint16_t *>(x);
  a.w0 = static_cast<const uint16_t *>(wq);
  a.w1 = static_cast<const uint16_t *>(wk);
  a.w2 = static_cast<const uint16_t *>(wv);
  a.n0 = nq;
  a.n1 = nk;
  a.n2 = nv;
  a.m = m;
  a.k = k;
  a.y = static_cast<uint16_t *>(q_out);
  a.ldy = nq;
  a.rope_cos = static_cast<const uint16_t *>(rope_cos);
  a.rope_sin = static_cast<const uint16_t *>(rope_sin);
  a.pos0 = pos0;
  a.k_out = static_cast<uint16_t *>(k_out);
  a.v_out = static_cast<uint16_t *>(v_out);
  a.kv_head_stride = kv_head_stride;
  a.slot0 = slot0;
  return launch_gemm<kGemmQkvRope>(a, (nq + nk + nv) / kGemmHead,
                                   static_cast<hipStream_t>(stream));
}
