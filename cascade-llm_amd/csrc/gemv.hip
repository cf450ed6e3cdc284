// M=1 bf16 GEMV family for the batch=1 decode path on gfx950.
//
// One wavefront owns a tile of R weight rows and the whole reduction
// dimension K.  Lane l reads 16-byte pieces l, l+64, l+128, ... of each row,
// so every load instruction of a wave covers 1 KiB of one row, fully
// coalesced.  A wave issues its loads of the input vector (and of the norm
// weight), then those of the epilogue's operands (residual, gate, RoPE
// cos / sin), then every weight load of its tile; loads complete in issue
// order, so the workgroup builds its copy of the (optionally
// RMS-normalised) input vector in LDS while the weights stream in, and the
// epilogue finds its operands in registers.  Products use v_dot2_f32_bf16 (two bf16
// products accumulated into fp32 per instruction); the row sums are reduced
// across the wave and finished by an epilogue that reproduces the reference's
// bf16 rounding points:
//   plain     y = bf16(acc)                          F.linear
//   residual  y = bf16(res + bf16(acc))              residual + F.linear
//   qkv_rope  rows (d, d+64) of one head per tile -> RoPE in bf16, then the
//             q buffer or the layer's KV cache       llama31.py:206-218
//   swiglu    gate row i and up row i per tile ->
//             bf16(bf16(silu(bf16(g))) * bf16(u))    llama31.py:264-275
//   silu / mul  the matrix-granularity halves of swiglu.
#include "cascade_device.h"
#include "cascade_internal.h"

namespace cascade {

enum GemvEpilogue : int {
  kPlain = 0,
  kResidual = 1,
  kQkvRope = 2,
  kSwiglu = 3,
  kSilu = 4,
  kMul = 5,
  kLogits = 6,  // fp32 output, no rounding (LM head)
};

struct GemvArgs {
  const uint16_t *w0;  // plain/residual/silu/mul: W; qkv: Wq; swiglu: Wgate
  const uint16_t *w1;  // qkv: Wk; swiglu: Wup
  const uint16_t *w2;  // qkv: Wv
  int64_t n0, n1, n2;  // rows of w0 / w1 / w2 (swiglu: n0 = n_half)
  int64_t k;
  const uint16_t *x;
  const uint16_t *norm_w;  // nullable: RMSNorm weight applied to x first
  float eps;
  uint16_t *y;
  const uint16_t *aux;  // residual (kResidual) or gate (kMul)
  float *yf;            // kLogits output
  const uint16_t *rope_cos;
  const uint16_t *rope_sin;
  uint16_t *k_out;
  uint16_t *v_out;
  int64_t kv_head_stride;
  int64_t n_tiles;
  // qkv at a device-held position (nullable): the token's position is
  // *length - 1, clamped to [0, capacity); rope_cos / rope_sin then point at
  // row 0 of the tables and k_out / v_out at position 0 of the cache
  const int64_t *length;
  int64_t capacity;
};

constexpr int kHeadDim = 128;
constexpr int kHalfHead = 64;

template <bool NT>
__device__ __forceinline__ u32x4 load16(const uint16_t *p) {
  // NT: streaming weights that are read once (nontemporal hint)
  if constexpr (NT)
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
  else
    return *reinterpret_cast<const u32x4 *>(p);
}

// Builds the GEMV input vector in LDS.  With a norm weight it applies
// _rms_norm (llama31.py:21-25): fp32 mean of squares, 1/sqrt(var + eps),
// x * r rounded to bf16, times the bf16 weight rounded to bf16.
template <int THREADS>
__device__ void stage_input(const GemvArgs &a, u32x4 *xs) {
  const int64_t nvec = a.k >> 3;
  const u32x4 *xg = reinterpret_cast<const u32x4 *>(a.x);
  if (a.norm_w == nullptr) {
    for (int64_t j = threadIdx.x; j < nvec; j += THREADS) xs[j] = xg[j];
    return;
  }
  __shared__ float red[THREADS / kWave];
  float ss = 0.0f;
  for (int64_t j = threadIdx.x; j < nvec; j += THREADS) {
    const u32x4 v = xg[j];
    xs[j] = v;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = lo_bf16(v[e]);
      const float hi = hi_bf16(v[e]);
      ss = fmaf(lo, lo, ss);
      ss = fmaf(hi, hi, ss);
    }
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = ss;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int i = 0; i < THREADS / kWave; ++i) total += red[i];
  const float variance = total * (1.0f / static_cast<float>(a.k));
  const float r = 1.0f / __builtin_sqrtf(variance + a.eps);
  const u32x4 *wg = reinterpret_cast<const u32x4 *>(a.norm_w);
  for (int64_t j = threadIdx.x; j < nvec; j += THREADS) {
    const u32x4 v = xs[j];
    const u32x4 w = wg[j];
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float nlo = round_bf16(lo_bf16(v[e]) * r);
      const float nhi = round_bf16(hi_bf16(v[e]) * r);
      const uint32_t olo = f32_to_bf16(lo_bf16(w[e]) * nlo);
      const uint32_t ohi = f32_to_bf16(hi_bf16(w[e]) * nhi);
      o[e] = olo | (ohi << 16);
    }
    xs[j] = o;
  }
}

// The same input vector built in two phases, for K = KC * 512 with NV =
// ceil(KC / WAVES) 16-byte pieces per thread: load_input issues the loads of
// x (and of the norm weight) before the weight loads, so that, loads
// completing in issue order, the vector can be normalised and staged while
// the weights stream in (store_input) instead of after they have landed.
template <int NV>
struct InputRegs {
  u32x4 x[NV];
  u32x4 w[NV];  // loaded only with a norm weight
};

template <int NV, int THREADS, bool EARLY_W>
__device__ __forceinline__ void load_input(const GemvArgs &a, InputRegs<NV> &in) {
  // unconditional loads at a clamped index (a load under a per-lane
  // predicate is waited for on the spot, to merge it with the other path)
  const int64_t nvec = a.k >> 3;
  const u32x4 *xg = reinterpret_cast<const u32x4 *>(a.x);
  const u32x4 *wg = reinterpret_cast<const u32x4 *>(a.norm_w);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t j = min(threadIdx.x + static_cast<int64_t>(i) * THREADS, nvec - 1);
    in.x[i] = xg[j];
  }
  if (EARLY_W && wg != nullptr) {  // workgroup-uniform; in.w is read only on this path
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int64_t j = min(threadIdx.x + static_cast<int64_t>(i) * THREADS, nvec - 1);
      in.w[i] = wg[j];
    }
  }
}

template <int NV, int THREADS, bool EARLY_W>
__device__ __forceinline__ void store_input(const GemvArgs &a, InputRegs<NV> &in,
                                            u32x4 *xs) {
  const int64_t nvec = a.k >> 3;
  if (a.norm_w == nullptr) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int64_t j = threadIdx.x + static_cast<int64_t>(i) * THREADS;
      if (j < nvec) xs[j] = in.x[i];
    }
    return;
  }
  if constexpr (!EARLY_W) {
    const u32x4 *wg = reinterpret_cast<const u32x4 *>(a.norm_w);
#pragma unroll
    for (int i = 0; i < NV; ++i)
      in.w[i] = wg[min(threadIdx.x + static_cast<int64_t>(i) * THREADS, nvec - 1)];
  }
  __shared__ float red[THREADS / kWave];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    // a clamped index repeats the last piece: it counts once
    if (threadIdx.x + static_cast<int64_t>(i) * THREADS >= nvec) continue;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = lo_bf16(in.x[i][e]);
      const float hi = hi_bf16(in.x[i][e]);
      ss = fmaf(lo, lo, ss);
      ss = fmaf(hi, hi, ss);
    }
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = ss;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int i = 0; i < THREADS / kWave; ++i) total += red[i];
  const float variance = total * (1.0f / static_cast<float>(a.k));
  const float r = 1.0f / __builtin_sqrtf(variance + a.eps);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t j = threadIdx.x + static_cast<int64_t>(i) * THREADS;
    if (j >= nvec) continue;
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float nlo = round_bf16(lo_bf16(in.x[i][e]) * r);
      const float nhi = round_bf16(hi_bf16(in.x[i][e]) * r);
      const uint32_t olo = f32_to_bf16(lo_bf16(in.w[i][e]) * nlo);
      const uint32_t ohi = f32_to_bf16(hi_bf16(in.w[i][e]) * nhi);
      o[e] = olo | (ohi << 16);
    }
    xs[j] = o;
  }
}

__device__ __forceinline__ float silu_f32(float g) {
  return g / (1.0f + expf(-g));
}

// Row addressing of one tile.  Returns, per tile row, the row's weight
// pointer and whether the row exists.
template <int EPI, int R>
__device__ __forceinline__ void tile_rows(const GemvArgs &a, int64_t tile,
                                          bool tile_ok,
                                          const uint16_t *(&wrow)[R],
                                          bool (&ok)[R]) {
  if constexpr (EPI == kQkvRope) {
    constexpr int P = R / 2;
    constexpr int kTilesPerHead = kHalfHead / P;
    const int64_t head = tile / kTilesPerHead;
    const int d0 = static_cast<int>(tile % kTilesPerHead) * P;
    const int64_t hq = a.n0 / kHeadDim, hk = a.n1 / kHeadDim;
    const uint16_t *base;
    int64_t lh;
    if (head < hq) {
      base = a.w0;
      lh = head;
    } else if (head < hq + hk) {
      base = a.w1;
      lh = head - hq;
    } else {
      base = a.w2;
      lh = head - hq - hk;
    }
    // a padding tile reads row 0 of a matrix the launch has (unused)
    const uint16_t *any = a.w0 != nullptr ? a.w0 : (a.w1 != nullptr ? a.w1 : a.w2);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int d = d0 + (r % P) + (r >= P ? kHalfHead : 0);
      ok[r] = tile_ok;
      wrow[r] = tile_ok ? base + (lh * kHeadDim + d) * a.k : any;
    }
  } else if constexpr (EPI == kSwiglu) {
    constexpr int P = R / 2;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t i = tile * P + (r % P);
      ok[r] = tile_ok && i < a.n0;
      wrow[r] = ok[r] ? (r < P ? a.w0 : a.w1) + i * a.k : a.w0;
    }
  } else {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t row = tile * R + r;
      ok[r] = tile_ok && row < a.n0;
      wrow[r] = ok[r] ? a.w0 + row * a.k : a.w0;
    }
  }
}

// The memory operands of the epilogue (the residual or gate element of
// each row; RoPE's cos / sin at the token's position), loaded with the
// input vector ahead of the weights (right after them where registers are
// short), so that their latency hides under the weight stream instead of
// following the reduction.
template <int EPI, int R>
__device__ __forceinline__ void epilogue_operands(const GemvArgs &a, int64_t tile,
                                                  int64_t length_word,
                                                  float (&pre0)[R], float (&pre1)[R]) {
#pragma unroll
  for (int r = 0; r < R; ++r) pre0[r] = pre1[r] = 0.0f;
  if constexpr (EPI == kResidual || EPI == kMul) {
    // rows past the matrix read its last row (unused)
#pragma unroll
    for (int r = 0; r < R; ++r)
      pre0[r] = bf16_to_f32(a.aux[min(tile * R + r, a.n0 - 1)]);
  } else if constexpr (EPI == kQkvRope) {
    constexpr int P = R / 2;
    constexpr int kTilesPerHead = kHalfHead / P;
    const int d0 = static_cast<int>(tile % kTilesPerHead) * P;
    // a launch of v rows only may pass no tables (kernel-uniform test)
    if (a.rope_cos != nullptr && a.rope_sin != nullptr) {
      const uint16_t *rope_cos = a.rope_cos, *rope_sin = a.rope_sin;
      if (a.length != nullptr) {
        const int64_t pos = min(max(length_word - 1, int64_t{0}), a.capacity - 1);
        rope_cos += pos * kHalfHead;
        rope_sin += pos * kHalfHead;
      }
#pragma unroll
      for (int p = 0; p < P; ++p) {
        pre0[p] = bf16_to_f32(rope_cos[d0 + p]);
        pre1[p] = bf16_to_f32(rope_sin[d0 + p]);
      }
    }
  }
}

template <int EPI, int R>
__device__ __forceinline__ void epilogue(const GemvArgs &a, int64_t tile,
                                         const float (&acc)[R],
                                         const bool (&ok)[R],
                                         int64_t length_word,
                                         const float (&pre0)[R],
                                         const float (&pre1)[R]) {
  if constexpr (EPI == kQkvRope) {
    constexpr int P = R / 2;
    constexpr int kTilesPerHead = kHalfHead / P;
    const int64_t head = tile / kTilesPerHead;
    const int d0 = static_cast<int>(tile % kTilesPerHead) * P;
    const int64_t hq = a.n0 / kHeadDim, hk = a.n1 / kHeadDim;
    uint16_t *k_out = a.k_out, *v_out = a.v_out;
    if (a.length != nullptr) {
      const int64_t pos =
          min(max(length_word - 1, int64_t{0}), a.capacity - 1);
      k_out += pos * kHeadDim;
      v_out += pos * kHeadDim;
    }
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int d = d0 + p;
      const float xa = round_bf16(acc[p]);      // element d of the head
      const float xb = round_bf16(acc[p + P]);  // element d + 64
      uint16_t oa, ob;
      if (head < hq + hk) {
        // apply_rotary_pos_emb: x*cos + rotate_half(x)*sin, every product
        // and the sum rounded to bf16; cos/sin are bf16 and identical for
        // d and d + 64 (emb = cat(freqs, freqs)).
        const float c = pre0[p];
        const float s = pre1[p];
        oa = f32_to_bf16(round_bf16(xa * c) + round_bf16(-xb * s));
        ob = f32_to_bf16(round_bf16(xb * c) + round_bf16(xa * s));
      } else {
        oa = f32_to_bf16(xa);
        ob = f32_to_bf16(xb);
      }
      if (head < hq) {
        a.y[head * kHeadDim + d] = oa;
        a.y[head * kHeadDim + d + kHalfHead] = ob;
      } else if (head < hq + hk) {
        uint16_t *dst = k_out + (head - hq) * a.kv_head_stride;
        dst[d] = oa;
        dst[d + kHalfHead] = ob;
      } else {
        uint16_t *dst = v_out + (head - hq - hk) * a.kv_head_stride;
        dst[d] = oa;
        dst[d + kHalfHead] = ob;
      }
    }
  } else if constexpr (EPI == kSwiglu) {
    constexpr int P = R / 2;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      if (!ok[p]) continue;
      const float g = round_bf16(acc[p]);
      const float u = round_bf16(acc[p + P]);
      const float s = round_bf16(silu_f32(g));
      a.y[tile * P + p] = f32_to_bf16(s * u);
    }
  } else {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (!ok[r]) continue;
      const int64_t row = tile * R + r;
      if constexpr (EPI == kLogits) {
        a.yf[row] = acc[r];
        continue;
      }
      const float v = round_bf16(acc[r]);
      float out;
      if constexpr (EPI == kPlain) {
        out = v;
      } else if constexpr (EPI == kResidual) {
        out = pre0[r] + v;
      } else if constexpr (EPI == kSilu) {
        out = silu_f32(v);
      } else {  // kMul
        out = pre0[r] * v;
      }
      a.y[row] = f32_to_bf16(out);
    }
  }
}

// KC > 0: K == KC * 512, loads fully unrolled and issued up front.
// KC == 0: any K that is a multiple of 8 (loop over 16-byte pieces).
template <int KC, int R, int WAVES, int EPI, bool NT>
__global__ __launch_bounds__(WAVES *kWave) void gemv_kernel(GemvArgs a) {
  extern __shared__ u32x4 xs[];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t tile = static_cast<int64_t>(blockIdx.x) * WAVES + wave;
  const bool tile_ok = tile < a.n_tiles;

  // A device-held position is loaded up front and unconditionally (x, 16
  // readable bytes, stands in when the position came from the host), so the
  // load is in flight with the weight loads instead of waited for on the
  // spot at the end of a branch.
  int64_t length_word = 0;
  if constexpr (EPI == kQkvRope)
    length_word = *(a.length != nullptr
                        ? a.length
                        : reinterpret_cast<const int64_t *>(a.x));

  const uint16_t *wrow[R];
  bool ok[R];
  tile_rows<EPI, R>(a, tile, tile_ok, wrow, ok);

  float acc[R], pre0[R], pre1[R];
  if constexpr (KC > 0) {
    constexpr int NV = (KC + WAVES - 1) / WAVES;
    // the input (and the norm weight, K = 4096) ahead of the weights where
    // the registers allow; down_proj's 56 loads per lane leave no room
    constexpr bool kEarly = R * KC <= 32;
    constexpr bool kEarlyW = kEarly && KC <= 8;
    InputRegs<NV> in;
    if constexpr (kEarly) {
      load_input<NV, WAVES * kWave, kEarlyW>(a, in);
      epilogue_operands<EPI, R>(a, tile, length_word, pre0, pre1);
    }
    // unconditional: a row past the matrix reads row 0 of a matrix the
    // launch has (tile_rows) and its sum is never stored
    u32x4 wv[R][KC];
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int c = 0; c < KC; ++c) wv[r][c] = load16<NT>(wrow[r] + (c * kWave + lane) * 8);
    }
    // every load above is issued before any use of the input (the waits
    // for the input then leave the weight loads in flight)
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kEarly) {
      store_input<NV, WAVES * kWave, kEarlyW>(a, in, xs);
    } else {
      epilogue_operands<EPI, R>(a, tile, length_word, pre0, pre1);
      stage_input<WAVES * kWave>(a, xs);
    }
    __syncthreads();
    float acc2[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      acc[r] = 0.0f;
      acc2[r] = 0.0f;
    }
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      const u32x4 xv = xs[c * kWave + lane];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (c & 1)
          acc2[r] = dot8_bf16(wv[r][c], xv, acc2[r]);
        else
          acc[r] = dot8_bf16(wv[r][c], xv, acc[r]);
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] += acc2[r];
  } else {
    epilogue_operands<EPI, R>(a, tile, length_word, pre0, pre1);
    stage_input<WAVES * kWave>(a, xs);
    __syncthreads();
    const int64_t nvec = a.k >> 3;
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    for (int64_t j = lane; j < nvec; j += kWave) {
      const u32x4 xv = xs[j];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (ok[r]) acc[r] = dot8_bf16(load16<NT>(wrow[r] + j * 8), xv, acc[r]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
  if (lane == 0 && tile_ok) epilogue<EPI, R>(a, tile, acc, ok, length_word, pre0, pre1);
}

template <int KC, int R, int WAVES, int EPI, bool NT>
static hipError_t launch_gemv(const GemvArgs &a, hipStream_t stream) {
  const int64_t blocks = (a.n_tiles + WAVES - 1) / WAVES;
  const size_t lds = static_cast<size_t>(a.k) * 2;
  return launch_kernel(gemv_kernel<KC, R, WAVES, EPI, NT>, dim3(blocks),
                       dim3(WAVES * kWave), lds, stream, a);
}

// Launch shapes, from MI355X sweeps of back-to-back launches over rotating
// weight copies (so no launch is served by the 256 MB MALL).  K = 4096 rows
// are 8 KiB (8 loads per lane), K = 14336 rows 28 KiB (28 loads per lane).
// Where a matrix is only one workgroup deep per CU, the grid is sized to
// exactly 256 workgroups -- one per CU, so no CU reads twice the share of
// another: q|k|v (6144 rows) as 12 waves x 2 rows, o_proj and down_proj
// (4096 rows) as 16 waves x 1 row.  Deep grids: gate/up (3584 workgroups)
// uses 4 waves x 2 rows, the LM head 2 waves x 1 row (64128 workgroups,
// launch_logits_gemv); everything else 8 waves x 2 rows.
// Nontemporal weight loads everywhere (every weight byte is read once per
// token).  Other K use the looped kernel.
template <int EPI>
struct GemvShape {
  static constexpr int WAVES = (EPI == kSwiglu || EPI == kLogits) ? 4
                               : EPI == kQkvRope                 ? 12
                                                                 : 8;
  static constexpr bool NT = true;
};

template <int R, int EPI>
static hipError_t dispatch_gemv(const GemvArgs &a, hipStream_t stream) {
  constexpr int W = GemvShape<EPI>::WAVES;
  constexpr bool NT = GemvShape<EPI>::NT;
  if constexpr (R == 1 && EPI == kResidual) {
    // o_proj / down_proj: 4096 rows -> 256 workgroups of 16 rows, as 16
    // one-row waves (K = 4096) or 8 two-row waves (K = 14336: 56 loads per
    // lane in flight, within the register file at 2 waves per SIMD)
    if (a.k == 4096) return launch_gemv<8, 1, 16, EPI, NT>(a, stream);
    if (a.k == 14336) {
      GemvArgs b = a;
      b.n_tiles = (a.n0 + 1) / 2;
      return launch_gemv<28, 2, 8, EPI, NT>(b, stream);
    }
  }
  if (a.k == 4096) return launch_gemv<8, R, W, EPI, NT>(a, stream);
  if constexpr (R == 1) {
    if (a.k == 14336) return launch_gemv<28, 1, 8, EPI, NT>(a, stream);
  }
  return launch_gemv<0, R, 4, EPI, NT>(a, stream);
}

static int check_common(const void *w, const void *x, int64_t n, int64_t k) {
  if (w == nullptr || x == nullptr || n <= 0 || k <= 0) return CASCADE_EINVAL;
  if ((k & 7) != 0 || !aligned16(w) || !aligned16(x)) return CASCADE_EALIGN;
  if (k * 2 > kMaxGemvLdsBytes) return CASCADE_ESHAPE;
  return 0;
}

hipError_t launch_logits_gemv(const uint16_t *w, int64_t rows, int64_t k,
                              const uint16_t *h, float *logits,
                              hipStream_t stream) {
  GemvArgs a{};
  a.w0 = w;
  a.n0 = rows;
  a.k = k;
  a.x = h;
  a.yf = logits;
  if (k == 4096) {
    // one row per wave, two waves per workgroup: 7.4 TB/s over the 1 GB
    // head on MI355X (2 rows x 4 waves: 6.8 TB/s)
    a.n_tiles = rows;
    return launch_gemv<8, 1, 2, kLogits, true>(a, stream);
  }
  a.n_tiles = (rows + 1) / 2;
  return dispatch_gemv<2, kLogits>(a, stream);
}

}  // namespace cascade

using namespace cascade;

extern "C" int cascade_gemv_bf16(const void *w, const void *x, void *y,
                                 int64_t n, int64_t k, void *stream) {
  if (int e = check_common(w, x, n, k)) return e;
  if (y == nullptr) return CASCADE_EINVAL;
  GemvArgs a{};
  a.w0 = static_cast<const uint16_t *>(w);
  a.n0 = n;
  a.k = k;
  a.x = static_cast<const uint16_t *>(x);
  a.y = static_cast<uint16_t *>(y);
  a.n_tiles = (n + 1) / 2;
  return dispatch_gemv<2, kPlain>(a, static_cast<hipStream_t>(stream));
}

extern "C" int cascade_gemv_residual_bf16(const void *w, const void *x,
                                          const void *residual, void *y,
                                          int64_t n, int64_t k, void *stream) {
  if (int e = check_common(w, x, n, k)) return e;
  if (y == nullptr || residual == nullptr) return CASCADE_EINVAL;
  GemvArgs a{};
  a.w0 = static_cast<const uint16_t *>(w);
  a.n0 = n;
  a.k = k;
  a.x = static_cast<const uint16_t *>(x);
  a.y = static_cast<uint16_t *>(y);
  a.aux = static_cast<const uint16_t *>(residual);
  hipStream_t s = static_cast<hipStream_t>(stream);
  a.n_tiles = n;
  return dispatch_gemv<1, kResidual>(a, s);
}

// Argument checks and packing shared by the two q|k|v entry points.
static int qkv_rope_args(const void *wq, const void *wk, const void *wv,
                         int64_t nq, int64_t nk, int64_t nv, int64_t k,
                         const void *x, const void *norm_weight, float eps,
                         const void *rope_cos, const void *rope_sin,
                         void *q_out, void *k_out, void *v_out,
                         int64_t kv_head_stride, GemvArgs &a) {
  if (nq < 0 || nk < 0 || nv < 0) return CASCADE_EINVAL;
  if ((nq % kHeadDim) || (nk % kHeadDim) || (nv % kHeadDim))
    return CASCADE_ESHAPE;
  const int64_t total = nq + nk + nv;
  if (total == 0 || x == nullptr || k <= 0) return CASCADE_EINVAL;
  if ((k & 7) != 0 || !aligned16(x) || !aligned16(norm_weight))
    return CASCADE_EALIGN;
  if (k * 2 > kMaxGemvLdsBytes) return CASCADE_ESHAPE;
  if (nq && (wq == nullptr || q_out == nullptr || !aligned16(wq)))
    return wq == nullptr || q_out == nullptr ? CASCADE_EINVAL : CASCADE_EALIGN;
  if (nk && (wk == nullptr || k_out == nullptr || !aligned16(wk)))
    return wk == nullptr || k_out == nullptr ? CASCADE_EINVAL : CASCADE_EALIGN;
  if (nv && (wv == nullptr || v_out == nullptr || !aligned16(wv)))
    return wv == nullptr || v_out == nullptr ? CASCADE_EINVAL : CASCADE_EALIGN;
  if ((nq || nk) && (rope_cos == nullptr || rope_sin == nullptr))
    return CASCADE_EINVAL;
  if ((nk || nv) && kv_head_stride < kHeadDim) return CASCADE_EINVAL;
  a.w0 = static_cast<const uint16_t *>(wq);
  a.w1 = static_cast<const uint16_t *>(wk);
  a.w2 = static_cast<const uint16_t *>(wv);
  a.n0 = nq;
  a.n1 = nk;
  a.n2 = nv;
  a.k = k;
  a.x = static_cast<const uint16_t *>(x);
  a.norm_w = static_cast<const uint16_t *>(norm_weight);
  a.eps = eps;
  a.y = static_cast<uint16_t *>(q_out);
  a.rope_cos = static_cast<const uint16_t *>(rope_cos);
  a.rope_sin = static_cast<const uint16_t *>(rope_sin);
  a.k_out = static_cast<uint16_t *>(k_out);
  a.v_out = static_cast<uint16_t *>(v_out);
  a.kv_head_stride = kv_head_stride;
  a.n_tiles = total / 2;  // two rows (d, d + 64) per tile
  return 0;
}

extern "C" int cascade_qkv_rope_bf16(const void *wq, const void *wk,
                                     const void *wv, int64_t nq, int64_t nk,
                                     int64_t nv, int64_t k, const void *x,
                                     const void *norm_weight, float eps,
                                     const void *rope_cos,
                                     const void *rope_sin, void *q_out,
                                     void *k_out, void *v_out,
                                     int64_t kv_head_stride, void *stream) {
  GemvArgs a{};
  if (int e = qkv_rope_args(wq, wk, wv, nq, nk, nv, k, x, norm_weight, eps,
                            rope_cos, rope_sin, q_out, k_out, v_out,
                            kv_head_stride, a))
    return e;
  return dispatch_gemv<2, kQkvRope>(a, static_cast<hipStream_t>(stream));
}

extern "C" int cascade_qkv_rope_at_bf16(
    const void *wq, const void *wk, const void *wv, int64_t nq, int64_t nk,
    int64_t nv, int64_t k, const void *x, const void *norm_weight, float eps,
    const void *rope_cos_table, const void *rope_sin_table, void *q_out,
    void *k_cache, void *v_cache, int64_t kv_head_stride,
    const int64_t *length, int64_t capacity, void *stream) {
  if (length == nullptr || capacity <= 0 || capacity > (int64_t{1} << 30))
    return CASCADE_EINVAL;
  if (reinterpret_cast<uintptr_t>(length) & 7) return CASCADE_EALIGN;
  if ((nk || nv) && kv_head_stride < capacity * kHeadDim) return CASCADE_EINVAL;
  GemvArgs a{};
  if (int e = qkv_rope_args(wq, wk, wv, nq, nk, nv, k, x, norm_weight, eps,
                            rope_cos_table, rope_sin_table, q_out, k_cache,
                            v_cache, kv_head_stride, a))
    return e;
  a.length = length;
  a.capacity = capacity;
  return dispatch_gemv<2, kQkvRope>(a, static_cast<hipStream_t>(stream));
}

extern "C" int cascade_gate_up_swiglu_bf16(const void *w_gate,
                                           const void *w_up, int64_t n_half,
                                           int64_t k, const void *x,
                                           const void *norm_weight, float eps,
                                           void *y, void *stream) {
  if (int e = check_common(w_gate, x, n_half, k)) return e;
  if (w_up == nullptr || y == nullptr) return CASCADE_EINVAL;
  if (!aligned16(w_up) || !aligned16(norm_weight)) return CASCADE_EALIGN;
  GemvArgs a{};
  a.w0 = static_cast<const uint16_t *>(w_gate);
  a.w1 = static_cast<const uint16_t *>(w_up);
  a.n0 = n_half;
  a.k = k;
  a.x = static_cast<const uint16_t *>(x);
  a.norm_w = static_cast<const uint16_t *>(norm_weight);
  a.eps = eps;
  a.y = static_cast<uint16_t *>(y);
  a.n_tiles = n_half;  // one gate row + one up row per tile
  return dispatch_gemv<2, kSwiglu>(a, static_cast<hipStream_t>(stream));
}

extern "C" int cascade_gate_silu_bf16(const void *w_gate, int64_t n, int64_t k,
                                      const void *x, const void *norm_weight,
                                      float eps, void *y, void *stream) {
  if (int e = check_common(w_gate, x, n, k)) return e;
  if (y == nullptr) return CASCADE_EINVAL;
  if (!aligned16(norm_weight)) return CASCADE_EALIGN;
  GemvArgs a{};
  a.w0 = static_cast<const uint16_t *>(w_gate);
  a.n0 = n;
  a.k = k;
  a.x = static_cast<const uint16_t *>(x);
  a.norm_w = static_cast<const uint16_t *>(norm_weight);
  a.eps = eps;
  a.y = static_cast<uint16_t *>(y);
  a.n_tiles = (n + 1) / 2;
  return dispatch_gemv<2, kSilu>(a, static_cast<hipStream_t>(stream));
}

extern "C" int cascade_up_mul_bf16(const void *w_up, int64_t n, int64_t k,
                                   const void *x, const void *norm_weight,
                                   float eps, const void *gate, void *y,
                                   void *stream) {
  if (int e = check_common(w_up, x, n, k)) return e;
  if (y == nullptr || gate == nullptr) return CASCADE_EINVAL;
  if (!aligned16(norm_weight)) return CASCADE_EALIGN;
  GemvArgs a{};
  a.w0 = static_cast<const uint16_t *>(w_up);
  a.n0 = n;
  a.k = k;
  a.x = static_cast<const uint16_t *>(x);
  a.norm_w = static_cast<const uint16_t *>(norm_weight);
  a.eps = eps;
  a.y = static_cast<uint16_t *>(y);
  a.aux = static_cast<const uint16_t *>(gate);
  a.n_tiles = (n + 1) / 2;
  return dispatch_gemv<2, kMul>(a, static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------------
// Standalone RMSNorm, one workgroup per row (the final norm before the LM
// head, llama31.py:325-329, and any caller that wants the normalised vector).
namespace cascade {

constexpr int kNormThreads = 256;

__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(
    const uint16_t *x, const uint16_t *w, uint16_t *y, int64_t n, float eps) {
  __shared__ float red[kNormThreads / kWave];
  const int64_t row = blockIdx.x;
  const u32x4 *xr = reinterpret_cast<const u32x4 *>(x + row * n);
  const u32x4 *wr = reinterpret_cast<const u32x4 *>(w);
  u32x4 *yr = reinterpret_cast<u32x4 *>(y + row * n);
  const int64_t nvec = n >> 3;
  float ss = 0.0f;
  for (int64_t j = threadIdx.x; j < nvec; j += kNormThreads) {
    const u32x4 v = xr[j];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = lo_bf16(v[e]);
      const float hi = hi_bf16(v[e]);
      ss = fmaf(lo, lo, ss);
      ss = fmaf(hi, hi, ss);
    }
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = ss;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormThreads / kWave; ++i) total += red[i];
  const float r =
      1.0f / __builtin_sqrtf(total * (1.0f / static_cast<float>(n)) + eps);
  for (int64_t j = threadIdx.x; j < nvec; j += kNormThreads) {
    const u32x4 v = xr[j];
    const u32x4 wv = wr[j];
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float nlo = round_bf16(lo_bf16(v[e]) * r);
      const float nhi = round_bf16(hi_bf16(v[e]) * r);
      o[e] = static_cast<uint32_t>(f32_to_bf16(lo_bf16(wv[e]) * nlo)) |
             (static_cast<uint32_t>(f32_to_bf16(hi_bf16(wv[e]) * nhi)) << 16);
    }
    yr[j] = o;
  }
}

}  // namespace cascade

extern "C" int cascade_rmsnorm_bf16(const void *x, const void *weight, void *y,
                                    int64_t rows, int64_t n, float eps,
                                    void *stream) {
  if (x == nullptr || weight == nullptr || y == nullptr || rows <= 0 ||
      n <= 0 || rows > 0x7fffffff)
    return CASCADE_EINVAL;
  if ((n & 7) || !aligned16(x) || !aligned16(weight) || !aligned16(y))
    return CASCADE_EALIGN;
  return launch_kernel(rmsnorm_kernel, dim3(static_cast<unsigned>(rows)),
                       dim3(kNormThreads), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint16_t *>(x),
                       static_cast<const uint16_t *>(weight),
                       static_cast<uint16_t *>(y), n, eps);
}
