// GQA decode attention for one query token on gfx950 (split over the
// sequence, "flash-decoding" style).
//
// Grid: (splits, kv_heads).  A workgroup of 4 waves owns one span of
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
// scale * log2(e) so exp2 replaces exp.  The 4 waves merge through LDS; with
// more than one split a second launch merges the splits:
//   out = sum_s 2^(m_s - M) acc_s / sum_s 2^(m_s - M) l_s,  M = max_s m_s
// which is exactly softmax(q K^T * scale) V (F.scaled_dot_product_attention
// without a mask, llama31.py:223-229; is_causal is False at decode).
#include "cascade_device.h"
#include "cascade_internal.h"

namespace cascade {

constexpr int kAttnG = 4;
constexpr int kAttnD = 128;
constexpr int kAttnWaves = 4;
constexpr int kAttnThreads = kAttnWaves * kWave;
constexpr int kAttnMaxSplits = 64;
constexpr int64_t kAttnLongContext = 8192;  // RPL 8 above, 4 at or below
constexpr size_t kAttnHeaderBytes = 256;
constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
  const uint16_t *q;
  const uint16_t *k;
  const uint16_t *v;
  int64_t head_stride;
  int32_t len;
  int32_t span;     // positions per split (multiple of 16 * RPL)
  int32_t nsplits;
  float scale_log2;  // scale * log2(e)
  uint16_t *out;
  float *part_ml;      // [kv_heads][nsplits][G][2]  (max in log2 units, sum)
  float *part_acc;     // [kv_heads][nsplits][G][D]
};

template <int RPL>
__global__ __launch_bounds__(kAttnThreads) void decode_attention_kernel(
    AttnArgs a) {
  constexpr int G = kAttnG, D = kAttnD;
  constexpr int kWaveRows = 4 * RPL;          // rows per wave per pass
  constexpr int kPassRows = kAttnWaves * kWaveRows;
  const int split = blockIdx.x;
  const int g = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int grp = lane >> 4;  // row of a load instruction (0..3)
  const int sub = lane & 15;  // 16-byte piece of the row (dims 8*sub ..)
  const int begin = split * a.span;
  const int end = min(begin + a.span, a.len);

  __shared__ float s_ml[kAttnWaves][G][2];
  __shared__ float s_acc[kAttnWaves][G][D];

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

  for (int base = begin + wave * kWaveRows; base < end; base += kPassRows) {
    u32x4 kr[RPL], vr[RPL];
#pragma unroll
    for (int i = 0; i < RPL; ++i) {
      const int row = base + 4 * i + grp;
      if (row < end) {
        kr[i] = *reinterpret_cast<const u32x4 *>(kb + static_cast<int64_t>(row) * D);
        vr[i] = *reinterpret_cast<const u32x4 *>(vb + static_cast<int64_t>(row) * D);
      } else {
        kr[i] = u32x4{0u, 0u, 0u, 0u};
        vr[i] = u32x4{0u, 0u, 0u, 0u};
      }
    }
    float s[G][RPL];
    float pmax[G];
#pragma unroll
    for (int h = 0; h < G; ++h) pmax[h] = -INFINITY;
#pragma unroll
    for (int i = 0; i < RPL; ++i) {
      const bool valid = base + 4 * i + grp < end;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float d = row16_sum(dot8_bf16(kr[i], qv[h], 0.0f)) * a.scale_log2;
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
      const float alpha = exp2f(m[h] - mnew);
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
        const uint32_t pair = vr[i][e];
        vf[2 * e] = lo_bf16(pair);
        vf[2 * e + 1] = hi_bf16(pair);
      }
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float p = exp2f(s[h][i] - m[h]);
        l[h] += p;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = fmaf(p, vf[e], acc[h][e]);
      }
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

  // Merge the 4 waves: thread -> (query head h, dims d, d + 1).  A wave that
  // saw no rows has m = -inf, l = 0 and weight 0 (wave 0 always sees one).
  const int h = tid / kWave;
  const int d = (tid & (kWave - 1)) * 2;
  float mm = -INFINITY;
#pragma unroll
  for (int w = 0; w < kAttnWaves; ++w) mm = fmaxf(mm, s_ml[w][h][0]);
  float den = 0.0f, o0 = 0.0f, o1 = 0.0f;
#pragma unroll
  for (int w = 0; w < kAttnWaves; ++w) {
    const float wt = exp2f(s_ml[w][h][0] - mm);
    den = fmaf(wt, s_ml[w][h][1], den);
    o0 = fmaf(wt, s_acc[w][h][d], o0);
    o1 = fmaf(wt, s_acc[w][h][d + 1], o1);
  }
  uint16_t *out = a.out + (static_cast<int64_t>(g) * G + h) * D + d;
  if (a.nsplits == 1) {
    const float inv = 1.0f / den;
    out[0] = f32_to_bf16(o0 * inv);
    out[1] = f32_to_bf16(o1 * inv);
    return;
  }

  const int64_t slot = (static_cast<int64_t>(g) * a.nsplits + split) * G + h;
  a.part_acc[slot * D + d] = o0;
  a.part_acc[slot * D + d + 1] = o1;
  if ((tid & (kWave - 1)) == 0) {
    a.part_ml[slot * 2] = mm;
    a.part_ml[slot * 2 + 1] = den;
  }
}

// Merge of the splits, one workgroup per (KV head, query head): lane c of
// wave 0 reads split c's (m, l), so the maximum and the denominator are
// wave reductions; thread t then sums dim t over the splits.  A separate
// launch (rather than a last-workgroup ticket) lets the kernel boundary
// publish the partials with one L2 writeback instead of one per workgroup.
__global__ __launch_bounds__(kAttnD) void decode_attention_merge_kernel(
    AttnArgs a) {
  constexpr int G = kAttnG, D = kAttnD;
  const int g = blockIdx.x / G;
  const int h = blockIdx.x % G;
  const int t = threadIdx.x;
  __shared__ float s_w[kAttnMaxSplits];
  __shared__ float s_den;
  const int64_t base = static_cast<int64_t>(g) * a.nsplits * G + h;
  if (t < kWave) {
    const float mc = t < a.nsplits ? a.part_ml[(base + t * G) * 2] : -INFINITY;
    const float lc = t < a.nsplits ? a.part_ml[(base + t * G) * 2 + 1] : 0.0f;
    const float mx = wave_max(mc);
    const float wc = t < a.nsplits ? exp2f(mc - mx) : 0.0f;
    s_w[t] = wc;
    const float den = wave_sum(wc * lc);
    if (t == 0) s_den = den;
  }
  __syncthreads();
  float r = 0.0f;
#pragma unroll 16
  for (int c = 0; c < a.nsplits; ++c)
    r = fmaf(s_w[c], a.part_acc[(base + static_cast<int64_t>(c) * G) * D + t], r);
  a.out[(static_cast<int64_t>(g) * G + h) * D + t] = f32_to_bf16(r / s_den);
}

struct AttnShape {
  int rpl;
  int64_t span;
  int64_t nsplits;
};

// Split policy: about 64 splits per KV head (512 workgroups for 8 heads) for
// long sequences, never more than kAttnMaxSplits, spans rounded to a whole
// workgroup pass.
static AttnShape attention_shape(int64_t len) {
  AttnShape s;
  s.rpl = len > kAttnLongContext ? 8 : 4;
  const int64_t pass = int64_t{kAttnWaves} * 4 * s.rpl;
  int64_t span = (len + kAttnMaxSplits - 1) / kAttnMaxSplits;
  span = ((span + pass - 1) / pass) * pass;
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
  if (shape.rpl == 8)
    hipLaunchKernelGGL(decode_attention_kernel<8>, grid, dim3(kAttnThreads), 0,
                       s, a);
  else
    hipLaunchKernelGGL(decode_attention_kernel<4>, grid, dim3(kAttnThreads), 0,
                       s, a);
  if (shape.nsplits > 1) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(decode_attention_merge_kernel,
                       dim3(static_cast<unsigned>(n_kv_heads * kAttnG)),
                       dim3(kAttnD), 0, s, a);
  }
  return hipGetLastError();
}
