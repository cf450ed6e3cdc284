// GQA decode attention for one query token on gfx950 (split over the
// sequence, "flash-decoding" style).
//
// Grid: (chunks, kv_heads).  A workgroup of 4 waves owns C consecutive
// positions of one KV head and the G = 4 query heads that share it
// (q head h uses kv head h / G, the repeat_interleave of _repeat_kv,
// layer_streaming/llama31.py:28-31).  A 256-byte K or V row is read by 16
// lanes with 16-byte loads, so each load instruction of a wave covers four
// rows; every K and V load of the chunk is issued before any arithmetic.
// Scores and probabilities live in LDS; the chunk's partial softmax state
// (running max m, sum l, unnormalised P.V) goes to the workspace and the
// last workgroup to finish for a KV head merges the chunks:
//   out = sum_c e^(m_c - M) acc_c / sum_c e^(m_c - M) l_c,  M = max_c m_c
// which is exactly softmax(q K^T * scale) V (F.scaled_dot_product_attention
// without a mask, llama31.py:223-229; is_causal is False at decode).
#include "cascade_device.h"
#include "cascade_internal.h"

namespace cascade {

constexpr int kAttnG = 4;
constexpr int kAttnD = 128;
constexpr int kAttnThreads = 256;
constexpr int64_t kAttnSmallChunk = 64;
constexpr int64_t kAttnLargeChunk = 256;
constexpr int64_t kAttnSmallMaxLen = 8192;
constexpr size_t kAttnCounterBytes = 256;

struct AttnArgs {
  const uint16_t *q;
  const uint16_t *k;
  const uint16_t *v;
  int64_t head_stride;
  int32_t len;
  int32_t nchunks;
  float scale;
  uint16_t *out;
  uint32_t *counters;  // [kv_heads]
  float *part_ml;      // [kv_heads][nchunks][G][2]
  float *part_acc;     // [kv_heads][nchunks][G][D]
};

template <int C>
__global__ __launch_bounds__(kAttnThreads) void decode_attention_kernel(
    AttnArgs a) {
  constexpr int G = kAttnG, D = kAttnD, PPL = C / 16;
  const int chunk = blockIdx.x;
  const int g = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int grp = lane >> 4;  // which of the 4 rows a load instruction covers
  const int sub = lane & 15;  // which 16-byte piece (8 dims) of the row
  const int p0 = chunk * C;
  const int n = min(C, a.len - p0);

  __shared__ float s_p[G][C];
  __shared__ float s_acc[4][G][D];
  __shared__ float s_m[G];
  __shared__ float s_l[G];
  __shared__ int s_last;

  u32x4 qv[G];
  const u32x4 *qg = reinterpret_cast<const u32x4 *>(a.q) + g * G * (D / 8);
#pragma unroll
  for (int h = 0; h < G; ++h) qv[h] = qg[h * (D / 8) + sub];

  const uint16_t *kb = a.k + g * a.head_stride + static_cast<int64_t>(p0) * D;
  const uint16_t *vb = a.v + g * a.head_stride + static_cast<int64_t>(p0) * D;
  u32x4 kr[PPL], vr[PPL];
#pragma unroll
  for (int i = 0; i < PPL; ++i) {
    const int pl = wave * 4 + grp + 16 * i;
    if (pl < n) {
      kr[i] = *reinterpret_cast<const u32x4 *>(kb + pl * D + sub * 8);
      vr[i] = *reinterpret_cast<const u32x4 *>(vb + pl * D + sub * 8);
    } else {
      kr[i] = u32x4{0u, 0u, 0u, 0u};
      vr[i] = u32x4{0u, 0u, 0u, 0u};
    }
  }

  // Scores.
#pragma unroll
  for (int i = 0; i < PPL; ++i) {
    const int pl = wave * 4 + grp + 16 * i;
    float d[G];
#pragma unroll
    for (int h = 0; h < G; ++h) d[h] = row16_sum(dot8_bf16(kr[i], qv[h], 0.0f));
    if (sub == 0 && pl < n) {
#pragma unroll
      for (int h = 0; h < G; ++h) s_p[h][pl] = d[h] * a.scale;
    }
  }
  __syncthreads();

  // Softmax statistics of the chunk: wave h owns query head h.
  {
    const int h = wave;
    float m = -INFINITY;
    for (int pl = lane; pl < n; pl += kWave) m = fmaxf(m, s_p[h][pl]);
    m = wave_max(m);
    float l = 0.0f;
    for (int pl = lane; pl < n; pl += kWave) {
      const float e = expf(s_p[h][pl] - m);
      s_p[h][pl] = e;
      l += e;
    }
    l = wave_sum(l);
    if (lane == 0) {
      s_m[h] = m;
      s_l[h] = l;
    }
  }
  __syncthreads();

  // P . V over this lane's rows, for 8 dims and all G heads.
  float acc[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.0f;
#pragma unroll
  for (int i = 0; i < PPL; ++i) {
    const int pl = wave * 4 + grp + 16 * i;
    if (pl < n) {
      float vf[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vf[2 * e] = lo_bf16(vr[i][e]);
        vf[2 * e + 1] = hi_bf16(vr[i][e]);
      }
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float p = s_p[h][pl];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = fmaf(p, vf[e], acc[h][e]);
      }
    }
  }
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      acc[h][e] += __shfl_xor(acc[h][e], 16, kWave);
      acc[h][e] += __shfl_xor(acc[h][e], 32, kWave);
    }
  if (grp == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) s_acc[wave][h][sub * 8 + e] = acc[h][e];
  }
  __syncthreads();

  const int h = tid / kWave;        // query head within the group
  const int d = (tid & (kWave - 1)) * 2;  // two dims per thread
  const float o0 = s_acc[0][h][d] + s_acc[1][h][d] + s_acc[2][h][d] +
                   s_acc[3][h][d];
  const float o1 = s_acc[0][h][d + 1] + s_acc[1][h][d + 1] +
                   s_acc[2][h][d + 1] + s_acc[3][h][d + 1];
  uint16_t *out = a.out + (static_cast<int64_t>(g) * G + h) * D + d;
  if (a.nchunks == 1) {
    const float inv = 1.0f / s_l[h];
    out[0] = f32_to_bf16(o0 * inv);
    out[1] = f32_to_bf16(o1 * inv);
    return;
  }

  const int64_t slot = (static_cast<int64_t>(g) * a.nchunks + chunk) * G + h;
  a.part_acc[slot * D + d] = o0;
  a.part_acc[slot * D + d + 1] = o1;
  if ((tid & (kWave - 1)) == 0) {
    a.part_ml[slot * 2] = s_m[h];
    a.part_ml[slot * 2 + 1] = s_l[h];
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = atomicAdd(&a.counters[g], 1u);
    s_last = (prev == static_cast<uint32_t>(a.nchunks - 1));
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  const int64_t base = static_cast<int64_t>(g) * a.nchunks * G + h;
  float mmax = -INFINITY;
  for (int c = 0; c < a.nchunks; ++c)
    mmax = fmaxf(mmax, a.part_ml[(base + c * G) * 2]);
  float den = 0.0f, r0 = 0.0f, r1 = 0.0f;
  for (int c = 0; c < a.nchunks; ++c) {
    const int64_t s = base + c * G;
    const float w = expf(a.part_ml[s * 2] - mmax);
    den = fmaf(w, a.part_ml[s * 2 + 1], den);
    r0 = fmaf(w, a.part_acc[s * D + d], r0);
    r1 = fmaf(w, a.part_acc[s * D + d + 1], r1);
  }
  out[0] = f32_to_bf16(r0 / den);
  out[1] = f32_to_bf16(r1 / den);
  if (tid == 0) a.counters[g] = 0u;  // ready for the next call
}

static int64_t attention_chunk(int64_t len) {
  return len <= kAttnSmallMaxLen ? kAttnSmallChunk : kAttnLargeChunk;
}

static int64_t attention_chunks(int64_t len) {
  const int64_t c = attention_chunk(len);
  return (len + c - 1) / c;
}

static size_t attention_workspace(int64_t nchunks, int64_t n_kv_heads) {
  const size_t per = static_cast<size_t>(n_kv_heads) * nchunks * kAttnG;
  return kAttnCounterBytes + per * 2 * sizeof(float) +
         per * kAttnD * sizeof(float);
}

}  // namespace cascade

using namespace cascade;

extern "C" size_t cascade_decode_attention_workspace_bytes(
    int64_t max_len, int64_t n_q_heads, int64_t n_kv_heads, int64_t head_dim) {
  if (max_len <= 0 || n_kv_heads <= 0 || n_q_heads != n_kv_heads * kAttnG ||
      head_dim != kAttnD)
    return 0;
  const int64_t small = attention_chunks(
      max_len < kAttnSmallMaxLen ? max_len : kAttnSmallMaxLen);
  const int64_t large = attention_chunks(max_len);
  const int64_t nchunks = small > large ? small : large;
  return attention_workspace(nchunks, n_kv_heads);
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
  const int64_t chunk = attention_chunk(len);
  const int64_t nchunks = attention_chunks(len);
  if (workspace_bytes < attention_workspace(nchunks, n_kv_heads))
    return CASCADE_EWORKSPACE;
  AttnArgs a{};
  a.q = static_cast<const uint16_t *>(q);
  a.k = static_cast<const uint16_t *>(k_cache);
  a.v = static_cast<const uint16_t *>(v_cache);
  a.head_stride = kv_head_stride;
  a.len = static_cast<int32_t>(len);
  a.nchunks = static_cast<int32_t>(nchunks);
  a.scale = scale;
  a.out = static_cast<uint16_t *>(out);
  char *ws = static_cast<char *>(workspace);
  a.counters = reinterpret_cast<uint32_t *>(ws);
  const size_t per = static_cast<size_t>(n_kv_heads) * nchunks * kAttnG;
  a.part_ml = reinterpret_cast<float *>(ws + kAttnCounterBytes);
  a.part_acc = reinterpret_cast<float *>(ws + kAttnCounterBytes +
                                         per * 2 * sizeof(float));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(nchunks),
                  static_cast<unsigned>(n_kv_heads));
  if (chunk == kAttnSmallChunk)
    hipLaunchKernelGGL(decode_attention_kernel<kAttnSmallChunk>, grid,
                       dim3(kAttnThreads), 0, s, a);
  else
    hipLaunchKernelGGL(decode_attention_kernel<kAttnLargeChunk>, grid,
                       dim3(kAttnThreads), 0, s, a);
  return hipGetLastError();
}
