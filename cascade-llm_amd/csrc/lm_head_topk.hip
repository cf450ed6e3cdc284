// Vocabulary-chunk LM head with an exact on-device top-k (gfx950).
//
// One launch handles one chunk of `rows` LM-head rows (a streamed 128 MiB
// slot, or the whole resident head):
//   1. each workgroup (8 waves) computes the fp32 logits of its block of
//      rows with the same wave-per-row-pair GEMV as gemv.hip, keeping them in
//      LDS (and optionally writing them out);
//   2. wave 0 selects the block's top-k with k passes of a wave-wide
//      maximum over (value, index) keys;
//   3. the last workgroup to finish (atomic ticket) merges every block's
//      candidates with the running list of earlier chunks and publishes the
//      running top-k.
// Keys order by value descending then index ascending (see topk_key), so the
// result is the exact top-k of the fp32 logits with lower-index-first ties:
// the reference's per-chunk torch.topk + merge_topk (layer_streaming/
// vocab.py:11-32,239-261) made deterministic on ties.
#include "cascade_device.h"
#include "cascade_internal.h"

namespace cascade {

constexpr int kLmWaves = 8;
constexpr int kLmThreads = kLmWaves * kWave;
constexpr int kLmRowsPerWaveIter = 2;
constexpr int kLmMaxRowsPerBlock = 1024;   // 16 keys per lane in step 2
constexpr int kLmMergeSlots = 16;          // keys per thread in step 3
constexpr int kLmMaxMerge = kLmMergeSlots * kLmThreads;  // 8192
constexpr int kLmMaxTopK = 64;
constexpr size_t kLmHeaderBytes = 256;     // ticket counter
constexpr size_t kLmRunningBytes = kLmMaxTopK * sizeof(uint64_t);

struct LmArgs {
  const uint16_t *w;
  int64_t rows;
  int64_t k;
  int64_t row_offset;
  const uint16_t *h;
  int top_k;
  int first;
  int rows_per_block;
  int nblocks;
  float *logits_out;
  uint32_t *counter;
  uint64_t *running;
  uint64_t *cand;
  float *out_values;
  int64_t *out_indices;
};

template <int KC>
__global__ __launch_bounds__(kLmThreads) void lm_head_topk_kernel(LmArgs a) {
  constexpr int R = kLmRowsPerWaveIter;
  extern __shared__ u32x4 xs[];
  __shared__ float s_logit[kLmMaxRowsPerBlock];
  __shared__ uint64_t s_red[2][kLmWaves];
  __shared__ int s_last;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int64_t rb = static_cast<int64_t>(blockIdx.x) * a.rows_per_block;
  const int nrows =
      static_cast<int>(min(static_cast<int64_t>(a.rows_per_block), a.rows - rb));

  {
    const int64_t nvec = a.k >> 3;
    const u32x4 *hg = reinterpret_cast<const u32x4 *>(a.h);
    for (int64_t j = tid; j < nvec; j += kLmThreads) xs[j] = hg[j];
  }
  __syncthreads();

  // 1. logits of this block's rows.
  for (int base = wave * R; base < nrows; base += kLmWaves * R) {
    float acc[R];
    bool ok[R];
    const uint16_t *wrow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      ok[r] = base + r < nrows;
      wrow[r] = a.w + (rb + base + (ok[r] ? r : 0)) * a.k;
      acc[r] = 0.0f;
    }
    if constexpr (KC > 0) {
      u32x4 wv[R][KC];
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < KC; ++c)
          wv[r][c] = ok[r] ? *reinterpret_cast<const u32x4 *>(
                                 wrow[r] + (c * kWave + lane) * 8)
                           : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int c = 0; c < KC; ++c) {
        const u32x4 xv = xs[c * kWave + lane];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = dot8_bf16(wv[r][c], xv, acc[r]);
      }
    } else {
      const int64_t nvec = a.k >> 3;
      for (int64_t j = lane; j < nvec; j += kWave) {
        const u32x4 xv = xs[j];
#pragma unroll
        for (int r = 0; r < R; ++r)
          if (ok[r])
            acc[r] = dot8_bf16(
                *reinterpret_cast<const u32x4 *>(wrow[r] + j * 8), xv, acc[r]);
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (!ok[r]) continue;
        s_logit[base + r] = acc[r];
        if (a.logits_out != nullptr) a.logits_out[rb + base + r] = acc[r];
      }
    }
  }
  __syncthreads();

  // 2. block top-k (wave 0): k passes of "largest key below the previous".
  if (wave == 0) {
    uint64_t keys[kLmMaxRowsPerBlock / kWave];
#pragma unroll
    for (int t = 0; t < kLmMaxRowsPerBlock / kWave; ++t) {
      const int li = t * kWave + lane;
      keys[t] = li < nrows
                    ? topk_key(s_logit[li],
                               static_cast<uint32_t>(a.row_offset + rb + li))
                    : 0ull;
    }
    uint64_t thr = ~0ull;
    for (int j = 0; j < a.top_k; ++j) {
      uint64_t best = 0ull;
#pragma unroll
      for (int t = 0; t < kLmMaxRowsPerBlock / kWave; ++t)
        if (keys[t] < thr && keys[t] > best) best = keys[t];
      best = wave_max_u64(best);
      if (lane == 0)
        a.cand[static_cast<int64_t>(blockIdx.x) * a.top_k + j] = best;
      thr = best;
    }
  }

  // 3. the last block merges all candidates with the running list.
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = atomicAdd(a.counter, 1u);
    s_last = (prev == static_cast<uint32_t>(a.nblocks - 1));
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  const int ncand = a.nblocks * a.top_k;
  const int ntot = ncand + (a.first ? 0 : a.top_k);
  uint64_t keys[kLmMergeSlots];
#pragma unroll
  for (int t = 0; t < kLmMergeSlots; ++t) {
    const int i = t * kLmThreads + tid;
    keys[t] = i < ncand ? a.cand[i] : (i < ntot ? a.running[i - ncand] : 0ull);
  }
  uint64_t thr = ~0ull;
  for (int j = 0; j < a.top_k; ++j) {
    uint64_t best = 0ull;
#pragma unroll
    for (int t = 0; t < kLmMergeSlots; ++t)
      if (keys[t] < thr && keys[t] > best) best = keys[t];
    best = wave_max_u64(best);
    if (lane == 0) s_red[j & 1][wave] = best;
    __syncthreads();
    best = 0ull;
#pragma unroll
    for (int w = 0; w < kLmWaves; ++w)
      best = s_red[j & 1][w] > best ? s_red[j & 1][w] : best;
    thr = best;
    if (tid == 0) {
      a.running[j] = best;
      a.out_values[j] = best ? key_value(best) : -INFINITY;
      a.out_indices[j] = best ? key_index(best) : int64_t{-1};
    }
  }
  if (tid == 0) *a.counter = 0u;  // ready for the next chunk
}

static int lm_rows_per_block(int64_t rows, int64_t top_k) {
  // Smallest multiple of 16 rows (>= 64) such that every block's candidates
  // plus the running list fit the single-block merge.
  const int64_t budget = kLmMaxMerge - top_k;
  int64_t rpb = (rows * top_k + budget - 1) / budget;
  rpb = ((rpb + 15) / 16) * 16;
  if (rpb < 64) rpb = 64;
  while (rpb <= kLmMaxRowsPerBlock &&
         ((rows + rpb - 1) / rpb) * top_k + top_k > kLmMaxMerge)
    rpb += 16;
  return static_cast<int>(rpb);
}

static size_t lm_workspace(int64_t nblocks, int64_t top_k) {
  return kLmHeaderBytes + kLmRunningBytes +
         static_cast<size_t>(nblocks) * top_k * sizeof(uint64_t);
}

}  // namespace cascade

using namespace cascade;

extern "C" size_t cascade_lm_head_workspace_bytes(int64_t rows,
                                                  int64_t top_k) {
  if (rows <= 0 || top_k < 1 || top_k > kLmMaxTopK) return 0;
  const int rpb = lm_rows_per_block(rows, top_k);
  if (rpb > kLmMaxRowsPerBlock) return 0;
  return lm_workspace((rows + rpb - 1) / rpb, top_k);
}

extern "C" int cascade_lm_head_topk_bf16(const void *w, int64_t rows, int64_t k,
                                         int64_t row_offset, const void *h,
                                         int64_t top_k, int first_chunk,
                                         float *logits_out, void *workspace,
                                         size_t workspace_bytes,
                                         float *out_values,
                                         int64_t *out_indices, void *stream) {
  if (w == nullptr || h == nullptr || workspace == nullptr ||
      out_values == nullptr || out_indices == nullptr)
    return CASCADE_EINVAL;
  if (rows <= 0 || k <= 0 || row_offset < 0 || top_k < 1 ||
      top_k > kLmMaxTopK)
    return CASCADE_EINVAL;
  if (row_offset + rows > 0xffffffffll) return CASCADE_ESHAPE;
  if ((k & 7) != 0 || !aligned16(w) || !aligned16(h) || !aligned16(workspace))
    return CASCADE_EALIGN;
  if (k * 2 > kMaxGemvLdsBytes) return CASCADE_ESHAPE;
  const int rpb = lm_rows_per_block(rows, top_k);
  if (rpb > kLmMaxRowsPerBlock) return CASCADE_ESHAPE;
  const int64_t nblocks = (rows + rpb - 1) / rpb;
  if (workspace_bytes < lm_workspace(nblocks, top_k)) return CASCADE_EWORKSPACE;
  LmArgs a{};
  a.w = static_cast<const uint16_t *>(w);
  a.rows = rows;
  a.k = k;
  a.row_offset = row_offset;
  a.h = static_cast<const uint16_t *>(h);
  a.top_k = static_cast<int>(top_k);
  a.first = first_chunk ? 1 : 0;
  a.rows_per_block = rpb;
  a.nblocks = static_cast<int>(nblocks);
  a.logits_out = logits_out;
  char *ws = static_cast<char *>(workspace);
  a.counter = reinterpret_cast<uint32_t *>(ws);
  a.running = reinterpret_cast<uint64_t *>(ws + kLmHeaderBytes);
  a.cand = reinterpret_cast<uint64_t *>(ws + kLmHeaderBytes + kLmRunningBytes);
  a.out_values = out_values;
  a.out_indices = out_indices;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t lds = static_cast<size_t>(k) * 2;
  if (k == 4096)
    hipLaunchKernelGGL(lm_head_topk_kernel<8>, dim3(nblocks), dim3(kLmThreads),
                       lds, s, a);
  else
    hipLaunchKernelGGL(lm_head_topk_kernel<0>, dim3(nblocks), dim3(kLmThreads),
                       lds, s, a);
  return hipGetLastError();
}
