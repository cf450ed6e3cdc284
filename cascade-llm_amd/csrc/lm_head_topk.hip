// Vocabulary-chunk LM head with an exact on-device top-k (gfx950).
//
// One call handles one chunk of `rows` LM-head rows (a streamed 128 MiB
// slot, or the whole resident head) in three launches:
//   1. the logits GEMV (gemv.hip, fp32 output, nontemporal weight loads)
//      writes logits[r] = W[r] . h, unrounded;
//   2. topk_candidates_kernel: each workgroup takes a span of logits and
//      selects its top-k with k passes of a block-wide maximum over
//      (value, index) keys;
//   3. topk_merge_kernel (one workgroup) merges all spans' candidates with
//      the running list of earlier chunks and publishes the running top-k.
// Keys order by value descending then index ascending (see topk_key), so the
// result is the exact top-k of the fp32 logits with lower-index-first ties:
// the reference's per-chunk torch.topk + merge_topk (layer_streaming/
// vocab.py:11-32,239-261) made deterministic on ties.
#include "cascade_device.h"
#include "cascade_internal.h"

namespace cascade {

constexpr int kTopkThreads = 256;
constexpr int kTopkWaves = kTopkThreads / kWave;
constexpr int kTopkMaxSlots = 16;  // keys per thread, at most
constexpr int kTopkMaxSpan = kTopkMaxSlots * kTopkThreads;   // 4096 logits
constexpr int kTopkMaxMerge = kTopkMaxSlots * kTopkThreads;  // 4096 keys
constexpr int kTopkMinSpan = 1024;
constexpr int kLmMaxTopK = 64;
constexpr size_t kLmHeaderBytes = 256;  // reserved
constexpr size_t kLmRunningBytes = kLmMaxTopK * sizeof(uint64_t);
constexpr size_t kLmCandBytes = kTopkMaxMerge * sizeof(uint64_t);

struct TopkArgs {
  const float *logits;
  int64_t rows;
  int64_t row_offset;
  int top_k;
  int first;
  int span;
  int nblocks;
  uint64_t *running;
  uint64_t *cand;
  float *out_values;
  int64_t *out_indices;
};

// Largest key strictly below `thr` among a thread's keys, maximised over the
// workgroup.  `parity` alternates the LDS slot between passes so one barrier
// per pass suffices.  SLOTS (keys per thread) is the smallest of 4, 8, 16
// that holds the kernel's keys: the per-thread scan is most of a pass.
template <int SLOTS>
__device__ __forceinline__ uint64_t block_next_key(
    const uint64_t (&keys)[SLOTS], uint64_t thr,
    uint64_t (&red)[2][kTopkWaves], int parity) {
  uint64_t best = 0ull;
#pragma unroll
  for (int t = 0; t < SLOTS; ++t)
    if (keys[t] < thr && keys[t] > best) best = keys[t];
  best = wave_max_u64(best);
  if ((threadIdx.x & (kWave - 1)) == 0) red[parity][threadIdx.x / kWave] = best;
  __syncthreads();
  best = 0ull;
#pragma unroll
  for (int w = 0; w < kTopkWaves; ++w)
    best = red[parity][w] > best ? red[parity][w] : best;
  return best;
}

// Candidates: workgroup b selects the top-k of logits [b*span, (b+1)*span)
// (span <= SLOTS * kTopkThreads).
template <int SLOTS>
__global__ __launch_bounds__(kTopkThreads) void topk_candidates_kernel(
    TopkArgs a) {
  __shared__ uint64_t s_red[2][kTopkWaves];
  const int tid = threadIdx.x;
  const int64_t begin = static_cast<int64_t>(blockIdx.x) * a.span;
  const int n = static_cast<int>(min(static_cast<int64_t>(a.span), a.rows - begin));
  uint64_t keys[SLOTS];
#pragma unroll
  for (int t = 0; t < SLOTS; ++t) {
    const int i = t * kTopkThreads + tid;
    keys[t] = i < n ? topk_key(a.logits[begin + i],
                               static_cast<uint32_t>(a.row_offset + begin + i))
                    : 0ull;
  }
  uint64_t thr = ~0ull;
  for (int j = 0; j < a.top_k; ++j) {
    thr = block_next_key(keys, thr, s_red, j & 1);
    if (tid == 0) a.cand[static_cast<int64_t>(blockIdx.x) * a.top_k + j] = thr;
  }
}

// Merge (one workgroup): all spans' candidates plus the running list of
// earlier chunks (at most SLOTS * kTopkThreads keys).  A separate launch, so
// the kernel boundary publishes the candidates (no per-workgroup L2
// writeback for a ticket).
template <int SLOTS>
__global__ __launch_bounds__(kTopkThreads) void topk_merge_kernel(TopkArgs a) {
  __shared__ uint64_t s_red[2][kTopkWaves];
  const int tid = threadIdx.x;
  const int ncand = a.nblocks * a.top_k;
  const int ntot = ncand + (a.first ? 0 : a.top_k);
  uint64_t keys[SLOTS];
#pragma unroll
  for (int t = 0; t < SLOTS; ++t) {
    const int i = t * kTopkThreads + tid;
    keys[t] = i < ncand ? a.cand[i] : (i < ntot ? a.running[i - ncand] : 0ull);
  }
  __syncthreads();  // every read of the old running list precedes its rewrite
  uint64_t thr = ~0ull;
  for (int j = 0; j < a.top_k; ++j) {
    thr = block_next_key(keys, thr, s_red, j & 1);
    if (tid == 0) {
      a.running[j] = thr;
      a.out_values[j] = thr ? key_value(thr) : -INFINITY;
      a.out_indices[j] = thr ? key_index(thr) : int64_t{-1};
    }
  }
}

struct TopkShape {
  int span;
  int nblocks;
};

// Spans of 1024..4096 logits (whole multiples of the block size) such that
// every span's candidates plus the running list fit the single-block merge.
static bool topk_shape(int64_t rows, int64_t top_k, TopkShape *out) {
  const int64_t budget = kTopkMaxMerge - top_k;
  int64_t span = (rows * top_k + budget - 1) / budget;
  span = ((span + kTopkThreads - 1) / kTopkThreads) * kTopkThreads;
  if (span < kTopkMinSpan) span = kTopkMinSpan;
  while (span <= kTopkMaxSpan &&
         ((rows + span - 1) / span) * top_k + top_k > kTopkMaxMerge)
    span += kTopkThreads;
  if (span > kTopkMaxSpan) return false;
  out->span = static_cast<int>(span);
  out->nblocks = static_cast<int>((rows + span - 1) / span);
  return true;
}

// The candidates (CAND) or merge kernel with the fewest key slots per
// thread that hold `keys` keys.
template <bool CAND>
static hipError_t launch_topk(const TopkArgs &a, int keys, dim3 grid,
                              hipStream_t s) {
  if (keys <= 4 * kTopkThreads)
    return CAND ? launch_kernel(topk_candidates_kernel<4>, grid,
                                dim3(kTopkThreads), 0, s, a)
                : launch_kernel(topk_merge_kernel<4>, grid,
                                dim3(kTopkThreads), 0, s, a);
  if (keys <= 8 * kTopkThreads)
    return CAND ? launch_kernel(topk_candidates_kernel<8>, grid,
                                dim3(kTopkThreads), 0, s, a)
                : launch_kernel(topk_merge_kernel<8>, grid,
                                dim3(kTopkThreads), 0, s, a);
  return CAND ? launch_kernel(topk_candidates_kernel<kTopkMaxSlots>, grid,
                              dim3(kTopkThreads), 0, s, a)
              : launch_kernel(topk_merge_kernel<kTopkMaxSlots>, grid,
                              dim3(kTopkThreads), 0, s, a);
}

// Candidates then merge over logits[0..rows) (global index row_offset + r);
// first: start a new running list instead of merging with the stored one.
static int run_topk(const float *logits, int64_t rows, int64_t row_offset,
                    int64_t top_k, bool first, const TopkShape &shape, char *ws,
                    float *out_values, int64_t *out_indices, hipStream_t s) {
  TopkArgs a{};
  a.logits = logits;
  a.rows = rows;
  a.row_offset = row_offset;
  a.top_k = static_cast<int>(top_k);
  a.first = first ? 1 : 0;
  a.span = shape.span;
  a.nblocks = shape.nblocks;
  a.running = reinterpret_cast<uint64_t *>(ws + kLmHeaderBytes);
  a.cand = reinterpret_cast<uint64_t *>(ws + kLmHeaderBytes + kLmRunningBytes);
  a.out_values = out_values;
  a.out_indices = out_indices;
  hipError_t e = launch_topk<true>(a, a.span, dim3(shape.nblocks), s);
  if (e != hipSuccess) return e;
  return launch_topk<false>(a, shape.nblocks * a.top_k + a.top_k, dim3(1), s);
}

static size_t lm_workspace(int64_t rows) {
  const size_t logits = ((static_cast<size_t>(rows) * 4 + 255) / 256) * 256;
  return kLmHeaderBytes + kLmRunningBytes + kLmCandBytes + logits;
}

}  // namespace cascade

using namespace cascade;

extern "C" size_t cascade_lm_head_workspace_bytes(int64_t rows,
                                                  int64_t top_k) {
  if (rows <= 0 || top_k < 1 || top_k > kLmMaxTopK) return 0;
  TopkShape shape;
  if (!topk_shape(rows, top_k, &shape)) return 0;
  return lm_workspace(rows);
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
  TopkShape shape;
  if (!topk_shape(rows, top_k, &shape)) return CASCADE_ESHAPE;
  if (workspace_bytes < lm_workspace(rows)) return CASCADE_EWORKSPACE;
  char *ws = static_cast<char *>(workspace);
  float *logits = logits_out != nullptr
                      ? logits_out
                      : reinterpret_cast<float *>(ws + kLmHeaderBytes +
                                                  kLmRunningBytes + kLmCandBytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = launch_logits_gemv(static_cast<const uint16_t *>(w), rows, k,
                                    static_cast<const uint16_t *>(h), logits, s);
  if (e != hipSuccess) return e;
  return run_topk(logits, rows, row_offset, top_k, first_chunk != 0, shape, ws,
                  out_values, out_indices, s);
}

extern "C" int cascade_topk_f32(const float *logits, int64_t rows, int64_t top_k,
                                void *workspace, size_t workspace_bytes,
                                float *out_values, int64_t *out_indices,
                                void *stream) {
  if (logits == nullptr || workspace == nullptr || out_values == nullptr ||
      out_indices == nullptr)
    return CASCADE_EINVAL;
  if (rows <= 0 || top_k < 1 || top_k > kLmMaxTopK) return CASCADE_EINVAL;
  if (rows > 0xffffffffll) return CASCADE_ESHAPE;
  if (!aligned16(workspace)) return CASCADE_EALIGN;
  TopkShape shape;
  if (!topk_shape(rows, top_k, &shape)) return CASCADE_ESHAPE;
  if (workspace_bytes < lm_workspace(rows)) return CASCADE_EWORKSPACE;
  // first = 1: the merge reads no running list, so the workspace needs no
  // zero-fill
  return run_topk(logits, rows, 0, top_k, true, shape,
                  static_cast<char *>(workspace), out_values, out_indices,
                  static_cast<hipStream_t>(stream));
}
