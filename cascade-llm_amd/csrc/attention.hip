// GQA decode attention for one query token on gfx950 (split over the
// sequence, "flash-decoding" style).
//
// Grid: (splits, kv_heads).  A workgroup of 8 waves owns one span of
// consecutive positions of one KV head and the G = 4 query heads that share
// it (q head h uses kv head h / G: the repeat_interleave of _repeat_kv,
// layer_streaming/llama31.py:28-31).
//
// Inside a workgroup every wave runs its own online softmax over rows of
// the span: per pass a wave reads 4*RPL rows of K and V (a 256-byte row is
// 16 lanes x 16 bytes, so one load instruction covers four rows and every
// load of the pass is issued before any arithmetic).  The q.k dot of a row
// is reduced across its 16 lanes with DPP, so every lane of the row holds
// the score and multiplies its own 8 dims of V: scores, probabilities and
// the running (max, sum, P.V) stay in registers.  Scores carry
// scale * log2(e) so exp2 replaces exp.  The waves merge through LDS; with
// more than one split a second launch merges the splits:
//   out = sum_s 2^(m_s - M) acc_s / sum_s 2^(m_s - M) l_s,  M = max_s m_s
// which is exactly softmax(q K^T * scale) V (F.scaled_dot_product_attention
// without a mask, llama31.py:223-229; is_causal is False at decode).
#include "cascade_device.h"
#include "cascade_internal.h"

namespace cascade {

constexpr int kAttnG = 4;
constexpr int kAttnD = 128;
constexpr int kAttnWaves = 8;  // waves per workgroup (4 waves per SIMD)
constexpr int kAttnMaxSplits = 64;
constexpr size_t kAttnHeaderBytes = 256;
constexpr float kLog2e = 1.4426950408889634f;

// 2^x with the bare v_exp_f32 (no denormal-range fix-up: arguments are
// s - max <= 0, and results below 2^-126 are negligible in a softmax sum;
// 2^-inf = 0).
__device__ __forceinline__ float exp2_fast(float x) {
  return __builtin_amdgcn_exp2f(x);
}

struct AttnArgs {
  const uint16_t *q;
  const uint16_t *k;
  const uint16_t *v;
  int64_t head_stride;
  int32_t len;
  int32_t span;     // positions per split
  int32_t nsplits;
  float scale_log2;  // scale * log2(e)
  uint16_t *out;
  float *part_ml;      // [kv_heads][nsplits][G][2]  (max in log2 units, sum)
  float *part_acc;     // [kv_heads][nsplits][G][D]
};

template <int RPL>
struct KvTile {
  u32x4 k[RPL];
  u32x4 v[RPL];
};

// Loads the K / V pieces of one wave pass (rows base + 4i + grp).
template <int RPL>
__device__ __forceinline__ void load_tile(KvTile<RPL> &t, const uint16_t *kb,
                                          const uint16_t *vb, int base, int grp,
                                          int end) {
#pragma unroll
  for (int i = 0; i < RPL; ++i) {
    const int row = base + 4 * i + grp;
    if (row < end) {
      t.k[i] = *reinterpret_cast<const u32x4 *>(kb + static_cast<int64_t>(row) * kAttnD);
      t.v[i] = *reinterpret_cast<const u32x4 *>(vb + static_cast<int64_t>(row) * kAttnD);
    } else {
      t.k[i] = u32x4{0u, 0u, 0u, 0u};
      t.v[i] = u32x4{0u, 0u, 0u, 0u};
    }
  }
}

// Online-softmax update of a wave's (m, l, acc) with one pass of rows.
template <int RPL>
__device__ __forceinline__ void attend_tile(const KvTile<RPL> &t,
                                            const u32x4 (&qv)[kAttnG],
                                            float scale_log2, int base, int grp,
                                            int end, float (&m)[kAttnG],
                                            float (&l)[kAttnG],
                                            float (&acc)[kAttnG][8]) {
  constexpr int G = kAttnG;
  float s[G][RPL];
  float pmax[G];
#pragma unroll
  for (int h = 0; h < G; ++h) pmax[h] = -INFINITY;
#pragma unroll
  for (int i = 0; i < RPL; ++i) {
    const bool valid = base + 4 * i + grp < end;
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float d = row16_sum(dot8_bf16(t.k[i], qv[h], 0.0f)) * scale_log2;
      s[h][i] = valid ? d : -INFINITY;
      pmax[h] = fmaxf(pmax[h], s[h][i]);
    }
  }
#pragma unroll
  for (int h = 0; h < G; ++h) {
    // lanes of one row agree; combine the 4 rows of the wave
    pmax[h] = fmaxf(pmax[h], __shfl_xor(pmax[h], 16, kWave));
    pmax[h] = fmaxf(pmax[h], __shfl_xor(pmax[h], 32, kWave));
    const float mnew = fmaxf(m[h], pmax[h]);
    // mnew is finite: row `base` of this pass is valid
    const float alpha = exp2_fast(m[h] - mnew);
    m[h] = mnew;
    l[h] *= alpha;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] *= alpha;
  }
#pragma unroll
  for (int i = 0; i < RPL; ++i) {
    float vf[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t pair = t.v[i][e];
      vf[2 * e] = lo_bf16(pair);
      vf[2 * e + 1] = hi_bf16(pair);
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float p = exp2_fast(s[h][i] - m[h]);
      l[h] += p;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[h][e] = fmaf(p, vf[e], acc[h][e]);
    }
  }
}

// WAVES waves per workgroup; PREFETCH: the next pass's loads are issued
// before the current pass is computed (two tiles of registers per wave).
template <int RPL, int WAVES, bool PREFETCH>
__global__ __launch_bounds__(WAVES *kWave) void decode_attention_kernel(
    AttnArgs a) {
  constexpr int G = kAttnG, D = kAttnD;
  constexpr int kWaveRows = 4 * RPL;          // rows per wave per pass
  constexpr int kPassRows = WAVES * kWaveRows;
  const int split = blockIdx.x;
  const int g = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int grp = lane >> 4;  // row of a load instruction (0..3)
  const int sub = lane & 15;  // 16-byte piece of the row (dims 8*sub ..)
  const int begin = split * a.span;
  const int end = min(begin + a.span, a.len);

  __shared__ float s_ml[WAVES][G][2];
  __shared__ float s_acc[WAVES][G][D];

  u32x4 qv[G];
  {
    const u32x4 *qg = reinterpret_cast<const u32x4 *>(a.q) + g * G * (D / 8);
#pragma unroll
    for (int h = 0; h < G; ++h) qv[h] = qg[h * (D / 8) + sub];
  }
  const uint16_t *kb = a.k + g * a.head_stride + sub * 8;
  const uint16_t *vb = a.v + g * a.head_stride + sub * 8;

  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.0f;
  }

  int base = begin + wave * kWaveRows;
  if constexpr (PREFETCH) {
    KvTile<RPL> cur;
    if (base < end) load_tile<RPL>(cur, kb, vb, base, grp, end);
    for (; base < end; base += kPassRows) {
      KvTile<RPL> nxt;
      const int nb = base + kPassRows;
      if (nb < end) load_tile<RPL>(nxt, kb, vb, nb, grp, end);
      attend_tile<RPL>(cur, qv, a.scale_log2, base, grp, end, m, l, acc);
      cur = nxt;
    }
  } else {
    for (; base < end; base += kPassRows) {
      KvTile<RPL> cur;
      load_tile<RPL>(cur, kb, vb, base, grp, end);
      attend_tile<RPL>(cur, qv, a.scale_log2, base, grp, end, m, l, acc);
    }
  }

  // Sum the wave's 4 row groups (their maxima already agree).
#pragma unroll
  for (int h = 0; h < G; ++h) {
    l[h] += __shfl_xor(l[h], 16, kWave);
    l[h] += __shfl_xor(l[h], 32, kWave);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      acc[h][e] += __shfl_xor(acc[h][e], 16, kWave);
      acc[h][e] += __shfl_xor(acc[h][e], 32, kWave);
    }
  }
  if (lane < 16) {
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) s_acc[wave][h][sub * 8 + e] = acc[h][e];
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      s_ml[wave][h][0] = m[h];
      s_ml[wave][h][1] = l[h];
    }
  }
  __syncthreads();

  // Merge the waves; output o = (query head h, dim d).  A wave that saw no
  // rows has m = -inf, l = 0 and weight 0 (wave 0 always sees one).
  for (int o = tid; o < G * D; o += WAVES * kWave) {
    const int h = o / D;
    const int d = o % D;
    float mm = -INFINITY;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) mm = fmaxf(mm, s_ml[w][h][0]);
    float den = 0.0f, r = 0.0f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      const float wt = exp2_fast(s_ml[w][h][0] - mm);
      den = fmaf(wt, s_ml[w][h][1], den);
      r = fmaf(wt, s_acc[w][h][d], r);
    }
    if (a.nsplits == 1) {
      a.out[(static_cast<int64_t>(g) * G + h) * D + d] = f32_to_bf16(r / den);
    } else {
      const int64_t slot =
          (static_cast<int64_t>(g) * a.nsplits + split) * G + h;
      a.part_acc[slot * D + d] = r;
      if (d == 0) {
        a.part_ml[slot * 2] = mm;
        a.part_ml[slot * 2 + 1] = den;
      }
    }
  }
}

// Merge of the splits, one workgroup per (KV head, query head): lane c of
// wave 0 reads split c's (m, l), so the maximum and the denominator are
// wave reductions; then each quarter of the workgroup sums every dim over
// its quarter of the splits (at most 16 independent loads per thread) and
// the quarters add up in LDS.  A separate launch (rather than a
// last-workgroup ticket) lets the kernel boundary publish the partials
// with one L2 writeback instead of one per workgroup.
constexpr int kMergeQuarters = 4;
constexpr int kMergeThreads = kMergeQuarters * kAttnD;
constexpr int kMergePerQuarter = kAttnMaxSplits / kMergeQuarters;

__global__ __launch_bounds__(kMergeThreads) void decode_attention_merge_kernel(
    AttnArgs a) {
  constexpr int G = kAttnG, D = kAttnD;
  const int g = blockIdx.x / G;
  const int h = blockIdx.x % G;
  const int t = threadIdx.x;
  const int d = t % D;
  const int quarter = t / D;
  __shared__ float s_w[kAttnMaxSplits];
  __shared__ float s_part[kMergeQuarters][D];
  __shared__ float s_den;
  const int64_t base = static_cast<int64_t>(g) * a.nsplits * G + h;
  // The partial sums do not depend on the weights: their loads are issued
  // first, so they are in flight together with wave 0's (m, l) loads.
  float v[kMergePerQuarter];
#pragma unroll
  for (int i = 0; i < kMergePerQuarter; ++i) {
    const int c = quarter * kMergePerQuarter + i;
    v[i] = c < a.nsplits
               ? a.part_acc[(base + static_cast<int64_t>(c) * G) * D + d]
               : 0.0f;
  }
  if (t < kWave) {
    const float mc = t < a.nsplits ? a.part_ml[(base + t * G) * 2] : -INFINITY;
    const float lc = t < a.nsplits ? a.part_ml[(base + t * G) * 2 + 1] : 0.0f;
    const float mx = wave_max(mc);
    const float wc = t < a.nsplits ? exp2_fast(mc - mx) : 0.0f;
    s_w[t] = wc;
    const float den = wave_sum(wc * lc);
    if (t == 0) s_den = den;
  }
  __syncthreads();
  // s_w[c] = 0 and v = 0 past the last split
  float r = 0.0f;
#pragma unroll
  for (int i = 0; i < kMergePerQuarter; ++i)
    r = fmaf(s_w[quarter * kMergePerQuarter + i], v[i], r);
  s_part[quarter][d] = r;
  __syncthreads();
  if (quarter == 0) {
    r = s_part[0][d] + s_part[1][d] + s_part[2][d] + s_part[3][d];
    a.out[(static_cast<int64_t>(g) * G + h) * D + d] = f32_to_bf16(r / s_den);
  }
}

struct AttnShape {
  int64_t span;
  int64_t nsplits;
};

// Split policy: kAttnMaxSplits splits per KV head (512 workgroups for 8
// heads) once the sequence is long enough, spans of at least 16 rows.
static AttnShape attention_shape(int64_t len) {
  AttnShape s;
  int64_t span = (len + kAttnMaxSplits - 1) / kAttnMaxSplits;
  if (span < 16) span = 16;
  s.span = span;
  s.nsplits = (len + span - 1) / span;
  return s;
}

static size_t attention_workspace(int64_t nsplits, int64_t n_kv_heads) {
  const size_t per = static_cast<size_t>(n_kv_heads) * nsplits * kAttnG;
  return kAttnHeaderBytes + per * 2 * sizeof(float) +
         per * kAttnD * sizeof(float);
}

}  // namespace cascade

using namespace cascade;

extern "C" size_t cascade_decode_attention_workspace_bytes(
    int64_t max_len, int64_t n_q_heads, int64_t n_kv_heads, int64_t head_dim) {
  if (max_len <= 0 || n_kv_heads <= 0 || n_q_heads != n_kv_heads * kAttnG ||
      head_dim != kAttnD)
    return 0;
  // the split count never exceeds kAttnMaxSplits, whatever the length
  return attention_workspace(kAttnMaxSplits, n_kv_heads);
}

extern "C" int cascade_decode_attention_bf16(
    const void *q, const void *k_cache, const void *v_cache,
    int64_t kv_head_stride, int64_t len, int64_t n_q_heads, int64_t n_kv_heads,
    int64_t head_dim, float scale, void *out, void *workspace,
    size_t workspace_bytes, void *stream) {
  if (q == nullptr || k_cache == nullptr || v_cache == nullptr ||
      out == nullptr || workspace == nullptr)
    return CASCADE_EINVAL;
  if (len <= 0 || len > (int64_t{1} << 30) || n_kv_heads <= 0 ||
      n_kv_heads > 65535)
    return CASCADE_EINVAL;
  if (head_dim != kAttnD || n_q_heads != n_kv_heads * kAttnG)
    return CASCADE_ESHAPE;
  if (kv_head_stride < len * head_dim) return CASCADE_EINVAL;
  if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) ||
      !aligned16(out) || !aligned16(workspace) || (kv_head_stride & 7))
    return CASCADE_EALIGN;
  const AttnShape shape = attention_shape(len);
  if (workspace_bytes < attention_workspace(shape.nsplits, n_kv_heads))
    return CASCADE_EWORKSPACE;
  AttnArgs a{};
  a.q = static_cast<const uint16_t *>(q);
  a.k = static_cast<const uint16_t *>(k_cache);
  a.v = static_cast<const uint16_t *>(v_cache);
  a.head_stride = kv_head_stride;
  a.len = static_cast<int32_t>(len);
  a.span = static_cast<int32_t>(shape.span);
  a.nsplits = static_cast<int32_t>(shape.nsplits);
  a.scale_log2 = scale * kLog2e;
  a.out = static_cast<uint16_t *>(out);
  char *ws = static_cast<char *>(workspace);
  const size_t per = static_cast<size_t>(n_kv_heads) * shape.nsplits * kAttnG;
  a.part_ml = reinterpret_cast<float *>(ws + kAttnHeaderBytes);
  a.part_acc = reinterpret_cast<float *>(ws + kAttnHeaderBytes +
                                         per * 2 * sizeof(float));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(shape.nsplits),
                  static_cast<unsigned>(n_kv_heads));
  const hipError_t e =
      launch_kernel(decode_attention_kernel<4, kAttnWaves, false>, grid,
                    dim3(kAttnWaves * kWave), 0, s, a);
  if (e != hipSuccess || shape.nsplits == 1) return e;
  return launch_kernel(decode_attention_merge_kernel,
                       dim3(static_cast<unsigned>(n_kv_heads * kAttnG)),
                       dim3(kMergeThreads), 0, s, a);
}
