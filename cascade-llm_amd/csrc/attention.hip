// GQA decode attention for one query token on gfx950 (split over the
// sequence, "flash-decoding" style), both products on the matrix cores.
//
// Grid: (splits, kv_heads).  A workgroup of 4 waves owns one span of
// consecutive positions of one KV head and the G = 4 query heads that share
// it (q head h uses kv head h / G: the repeat_interleave of _repeat_kv,
// layer_streaming/llama31.py:28-31).  Each wave runs its own online softmax
// over 32-row blocks of the span (blocks wave, wave + 4, ...), the waves
// merge through LDS, and with more than one split a second launch merges the
// splits:
//   out = sum_s 2^(m_s - M) acc_s / sum_s 2^(m_s - M) l_s,  M = max_s m_s
// which is exactly softmax(q K^T * scale) V (F.scaled_dot_product_attention
// without a mask, llama31.py:223-229; is_causal is False at decode).  Scores
// carry scale * log2(e) so exp2 replaces exp.
//
// One 32-row block is 16 v_mfma_f32_16x16x32_bf16, with the G = 4 query
// heads as the 16-wide N dimension (12 columns of zeros):
//   S = K_blk q^T   two 16-row halves x four 32-dim chunks = 8 MFMAs
//   O += V_blk^T P  eight 16-dim slots, K = the 32 rows      = 8 MFMAs
// Lane l (c = l % 16, g4 = l / 16) ends up owning the scores of query head c
// for rows 8 g4 .. 8 g4 + 7 of the block; that is exactly its piece of the
// P operand, so the softmax moves no data beyond the max over the four lanes
// of a head.  The row order inside a half (row 8 (i / 4) + 4 hf + i % 4 for
// MFMA row i) is chosen for that.  V is loaded as whole 256-byte rows (16
// lanes a row) and transposed in registers with byte permutes: lane l holds
// dims 8 c .. 8 c + 7 of rows 8 g4 + j, and operand e takes dim 8 c + e of
// its 8 rows.  P enters the MFMA rounded to bf16; the sum l is kept from the
// fp32 values.  Rows past the end of the span are loaded from the span's last
// row (always valid memory) and given a score of -inf.  K and V are read
// once, with the nontemporal hint.
#include "cascade_device.h"
#include "cascade_internal.h"

namespace cascade {

constexpr int kAttnG = 4;
constexpr int kAttnD = 128;
constexpr int kAttnWaves = 4;   // waves per workgroup
constexpr int kAttnBlock = 32;  // rows per wave step (the MFMA K of P V)
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
  int32_t span;     // positions per split (a multiple of kAttnBlock)
  int32_t nsplits;
  float scale_log2;  // scale * log2(e)
  uint16_t *out;
  float *part_ml;      // [kv_heads][nsplits][G][2]  (max in log2 units, sum)
  float *part_acc;     // [kv_heads][nsplits][G][D]
};

template <bool NT>
__device__ __forceinline__ u32x4 kv_load(const uint16_t *p) {
  if constexpr (NT)
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
  else
    return *reinterpret_cast<const u32x4 *>(p);
}

// Operand e of the transposed V block: dword p = (row 2p, row 2p + 1) of
// dim 8 c + e, from the lane's 8 loaded rows.
__device__ __forceinline__ u32x4 v_operand(const u32x4 (&vt)[8], int e) {
  // v_perm_b32 selectors: low halves / high halves of (src1, src0)
  const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
  u32x4 r;
#pragma unroll
  for (int p = 0; p < 4; ++p)
    r[p] = __builtin_amdgcn_perm(vt[2 * p + 1][e >> 1], vt[2 * p][e >> 1], sel);
  return r;
}

template <int WAVES, bool NT>
__global__ __launch_bounds__(WAVES *kWave) void decode_attention_kernel(
    AttnArgs a) {
  constexpr int G = kAttnG, D = kAttnD;
  constexpr int kPassRows = WAVES * kAttnBlock;
  const int split = blockIdx.x;
  const int g = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int c16 = lane & 15;
  const int g4 = lane >> 4;
  const int begin = split * a.span;
  const int end = min(begin + a.span, a.len);

  __shared__ float s_ml[WAVES][G][2];
  __shared__ float s_acc[WAVES][G][D];

  // q operand of dim chunk c: B[8 g4 + j][c16] = q[head c16][32 c + 8 g4 + j]
  u32x4 qop[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
    qop[c] = c16 < G ? *reinterpret_cast<const u32x4 *>(
                           a.q + (g * G + c16) * D + 32 * c + 8 * g4)
                     : u32x4{0u, 0u, 0u, 0u};
  const uint16_t *kb = a.k + g * a.head_stride;
  const uint16_t *vb = a.v + g * a.head_stride;
  const int krow = 8 * (c16 >> 2) + (c16 & 3);  // + 4 hf
  const int last = end - 1;
  const uint32_t head_mask = c16 < G ? 0xffffffffu : 0u;  // zero P columns

  float m = -INFINITY, l = 0.0f;
  f32x4 o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // K rows of the block as two MFMA halves, V rows as 8 whole rows per lane
  auto load_block = [&](int r0, u32x4 (&kt)[2][4], u32x4 (&vt)[8]) {
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int row = min(r0 + krow + 4 * hf, last);
#pragma unroll
      for (int c = 0; c < 4; ++c)
        kt[hf][c] = kv_load<NT>(kb + static_cast<int64_t>(row) * D + 32 * c +
                                8 * g4);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int row = min(r0 + 8 * g4 + j, last);
      vt[j] = kv_load<NT>(vb + static_cast<int64_t>(row) * D + 8 * c16);
    }
  };

  auto block_step = [&](int r0, const u32x4 (&kt)[2][4], const u32x4 (&vt)[8]) {
    f32x4 s0 = {0.0f, 0.0f, 0.0f, 0.0f}, s1 = s0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      s0 = mfma_16x16x32_bf16(kt[0][c], qop[c], s0);
      s1 = mfma_16x16x32_bf16(kt[1][c], qop[c], s1);
    }
    // s[j]: row r0 + 8 g4 + j, query head c16
    float s[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
    float bmax = -INFINITY;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      s[j] = r0 + 8 * g4 + j < end ? s[j] * a.scale_log2 : -INFINITY;
      bmax = fmaxf(bmax, s[j]);
    }
    bmax = xor32_max(xor16_max(bmax));
    // finite: row r0 (lane group 0, j = 0) is valid
    const float mnew = fmaxf(m, bmax);
    const float alpha = exp2_fast(m - mnew);
    m = mnew;
    float p[8], psum = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      p[j] = exp2_fast(s[j] - mnew);
      psum += p[j];
    }
    l = fmaf(l, alpha, psum);
    u32x4 pop;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      pop[i] = pack_bf16x2(p[2 * i], p[2 * i + 1]) & head_mask;
    if (alpha != 1.0f) {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] *= alpha;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e)
      o[e] = mfma_16x16x32_bf16(v_operand(vt, e), pop, o[e]);
  };

  for (int r0 = begin + wave * kAttnBlock; r0 < end; r0 += kPassRows) {
    u32x4 kt[2][4];
    u32x4 vt[8];
    load_block(r0, kt, vt);
    block_step(r0, kt, vt);
  }

  // The four lanes of a head share m; sum their l.
  l = xor32_sum(xor16_sum(l));
  if (c16 < G) {
    // o[e][r] = O[dim 8 (4 g4 + r) + e][head c16]
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        s_acc[wave][c16][8 * (4 * g4 + r) + e] = o[e][r];
    if (g4 == 0) {
      s_ml[wave][c16][0] = m;
      s_ml[wave][c16][1] = l;
    }
  }
  __syncthreads();

  // Merge the waves; output (query head h, dim d).  A wave that saw no rows
  // has m = -inf, l = 0, acc = 0 and weight 0 (wave 0 always sees one).
  for (int o_idx = tid; o_idx < G * D; o_idx += WAVES * kWave) {
    const int h = o_idx / D;
    const int d = o_idx % D;
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
// wave reductions; each quarter of the workgroup sums every dim over its
// quarter of the splits (at most 16 independent loads per thread, issued
// before the weights are known) and the quarters add up in LDS.  A separate
// launch (rather than a last-workgroup ticket) lets the kernel boundary
// publish the partials with one L2 writeback instead of one per workgroup.
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

// ---------------------------------------------------------------------------
// Causal GQA prefill attention (the is_causal=True SDPA of the prefill call,
// layer_streaming/llama31.py:223-229): query token t (cache slot past + t)
// attends to cache positions [0, past + t].
//
// One wave owns one KV head and NB x 4 consecutive query tokens: NB blocks
// of 16 MFMA columns, column c of block b being (token t0 + 4 b + c / 4,
// query head 4 g + c % 4), so the 4 query heads sharing the KV head and the
// NB token groups reuse every K / V fragment the wave loads.  The wave walks
// 32-row blocks from position 0 to its last token's position with the
// decode kernel's block step (scores S = K_blk Q^T, online softmax in
// registers, O += V_blk^T P, P rounded to bf16 for the MFMA); positions
// beyond a column's own limit score -inf.  No split and no merge: a wave
// finishes its columns and writes them.  Workgroups run the latest tokens
// (the longest walks) first.
// Two column blocks per wave, at most 256 registers (2 waves per SIMD):
// 150 us per layer at S = 2048 on MI355X (one block: 240 us; four blocks:
// 157 us at one wave per SIMD, spills when held to two).
constexpr int kPrefillBlocks = 2;                    // MFMA column blocks per wave
constexpr int kPrefillTokens = 4 * kPrefillBlocks;  // query tokens per wave
constexpr int kPrefillWavesPerSimd = 2;

struct PrefillArgs {
  const uint16_t *q;  // [tokens, n_q_heads * D]
  const uint16_t *k;  // position 0 of KV head 0
  const uint16_t *v;
  int64_t head_stride;
  int32_t past;
  int32_t tokens;
  int32_t q_row;  // n_q_heads * D
  int32_t groups;  // ceil(tokens / (4 NB))
  float scale_log2;
  uint16_t *out;  // [tokens, n_q_heads * D]
};

template <bool NT, int NB, int WPE>
__global__ __launch_bounds__(kAttnWaves *kWave)
__attribute__((amdgpu_waves_per_eu(WPE))) void prefill_attention_kernel(
    PrefillArgs a) {
  constexpr int G = kAttnG, D = kAttnD, TOK = 4 * NB;
  const int g = blockIdx.y;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int group =
      (static_cast<int>(gridDim.x) - 1 - static_cast<int>(blockIdx.x)) *
          kAttnWaves + wave;
  if (group >= a.groups) return;  // no barriers in this kernel
  const int c16 = lane & 15;
  const int g4 = lane >> 4;
  const int hq = g * G + (c16 & 3);
  const int t_last = min(group * TOK + TOK - 1, a.tokens - 1);
  const int end = a.past + t_last + 1;
  const int last = end - 1;

  int tq[NB], limit[NB];
  u32x4 qop[NB][4];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    tq[b] = group * TOK + 4 * b + (c16 >> 2);
    limit[b] = a.past + tq[b];  // inclusive
    const int tq_load = min(tq[b], a.tokens - 1);
    const uint16_t *qrow =
        a.q + static_cast<int64_t>(tq_load) * a.q_row + hq * D;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      qop[b][c] = *reinterpret_cast<const u32x4 *>(qrow + 32 * c + 8 * g4);
  }
  const uint16_t *kb = a.k + g * a.head_stride;
  const uint16_t *vb = a.v + g * a.head_stride;
  const int krow = 8 * (c16 >> 2) + (c16 & 3);  // + 4 hf

  float m[NB], l[NB];
  f32x4 o[NB][8];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    m[b] = -INFINITY;
    l[b] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[b][e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  for (int r0 = 0; r0 < end; r0 += kAttnBlock) {
    u32x4 kt[2][4];
    u32x4 vt[8];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int row = min(r0 + krow + 4 * hf, last);
#pragma unroll
      for (int c = 0; c < 4; ++c)
        kt[hf][c] = kv_load<NT>(kb + static_cast<int64_t>(row) * D + 32 * c +
                                8 * g4);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int row = min(r0 + 8 * g4 + j, last);
      vt[j] = kv_load<NT>(vb + static_cast<int64_t>(row) * D + 8 * c16);
    }
    u32x4 vop[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) vop[e] = v_operand(vt, e);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      f32x4 s0 = {0.0f, 0.0f, 0.0f, 0.0f}, s1 = s0;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        s0 = mfma_16x16x32_bf16(kt[0][c], qop[b][c], s0);
        s1 = mfma_16x16x32_bf16(kt[1][c], qop[b][c], s1);
      }
      // s[j]: position r0 + 8 g4 + j, column c16 of block b
      float s[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
      float bmax = -INFINITY;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        s[j] = r0 + 8 * g4 + j <= limit[b] ? s[j] * a.scale_log2 : -INFINITY;
        bmax = fmaxf(bmax, s[j]);
      }
      bmax = xor32_max(xor16_max(bmax));
      // finite from the first block on: position 0 is valid for every column
      const float mnew = fmaxf(m[b], bmax);
      const float alpha = exp2_fast(m[b] - mnew);
      m[b] = mnew;
      float p[8], psum = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        p[j] = exp2_fast(s[j] - mnew);
        psum += p[j];
      }
      l[b] = fmaf(l[b], alpha, psum);
      u32x4 pop;
#pragma unroll
      for (int i = 0; i < 4; ++i) pop[i] = pack_bf16x2(p[2 * i], p[2 * i + 1]);
      if (alpha != 1.0f) {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[b][e] *= alpha;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e)
        o[b][e] = mfma_16x16x32_bf16(vop[e], pop, o[b][e]);
    }
  }

#pragma unroll
  for (int b = 0; b < NB; ++b) {
    float lb = l[b];
    lb = xor32_sum(xor16_sum(lb));
    if (tq[b] >= a.tokens) continue;
    const float inv = 1.0f / lb;
    // o[b][e][r] = O[dim 8 (4 g4 + r) + e][column c16 of block b]
    uint16_t *orow = a.out + static_cast<int64_t>(tq[b]) * a.q_row + hq * D;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      u32x4 packed;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        packed[i] = pack_bf16x2(o[b][2 * i][r] * inv, o[b][2 * i + 1][r] * inv);
      *reinterpret_cast<u32x4 *>(orow + 8 * (4 * g4 + r)) = packed;
    }
  }
}

struct AttnShape {
  int64_t span;
  int64_t nsplits;
};

// Split policy: at most kAttnMaxSplits splits per KV head (512 workgroups
// for 8 heads at long contexts), spans a multiple of the 32-row block.  At
// context 32769 this gives 61 spans of 544 rows (an MI355X sweep of spans
// 544 .. 1024 rows and 4 / 8 waves per workgroup put this within 0.5 us of
// the best).
static AttnShape attention_shape(int64_t len) {
  AttnShape s;
  int64_t span = (len + kAttnMaxSplits - 1) / kAttnMaxSplits;
  span = (span + kAttnBlock - 1) / kAttnBlock * kAttnBlock;
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
      launch_kernel(decode_attention_kernel<kAttnWaves, true>, grid,
                    dim3(kAttnWaves * kWave), 0, s, a);
  if (e != hipSuccess || shape.nsplits == 1) return e;
  return launch_kernel(decode_attention_merge_kernel,
                       dim3(static_cast<unsigned>(n_kv_heads * kAttnG)),
                       dim3(kMergeThreads), 0, s, a);
}

extern "C" int cascade_prefill_attention_bf16(
    const void *q, const void *k_cache, const void *v_cache,
    int64_t kv_head_stride, int64_t past, int64_t tokens, int64_t n_q_heads,
    int64_t n_kv_heads, int64_t head_dim, float scale, void *out,
    void *stream) {
  if (q == nullptr || k_cache == nullptr || v_cache == nullptr ||
      out == nullptr)
    return CASCADE_EINVAL;
  if (tokens <= 0 || past < 0 || past + tokens > (int64_t{1} << 30) ||
      n_kv_heads <= 0 || n_kv_heads > 65535)
    return CASCADE_EINVAL;
  if (head_dim != kAttnD || n_q_heads != n_kv_heads * kAttnG)
    return CASCADE_ESHAPE;
  if (kv_head_stride < (past + tokens) * head_dim) return CASCADE_EINVAL;
  if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) ||
      !aligned16(out) || (kv_head_stride & 7))
    return CASCADE_EALIGN;
  PrefillArgs a{};
  a.q = static_cast<const uint16_t *>(q);
  a.k = static_cast<const uint16_t *>(k_cache);
  a.v = static_cast<const uint16_t *>(v_cache);
  a.head_stride = kv_head_stride;
  a.past = static_cast<int32_t>(past);
  a.tokens = static_cast<int32_t>(tokens);
  a.q_row = static_cast<int32_t>(n_q_heads * head_dim);
  a.groups = static_cast<int32_t>((tokens + kPrefillTokens - 1) / kPrefillTokens);
  a.scale_log2 = scale * kLog2e;
  a.out = static_cast<uint16_t *>(out);
  const int64_t blocks = (a.groups + kAttnWaves - 1) / kAttnWaves;
  const dim3 grid(static_cast<unsigned>(blocks),
                  static_cast<unsigned>(n_kv_heads));
  // K / V rows are re-read by every later query token: keep them cached
  return launch_kernel(prefill_attention_kernel<false, kPrefillBlocks, kPrefillWavesPerSimd>, grid,
                       dim3(kAttnWaves * kWave), 0,
                       static_cast<hipStream_t>(stream), a);
}
