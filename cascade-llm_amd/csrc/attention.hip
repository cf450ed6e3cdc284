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
#include <atomic>
#include <cfloat>
#include <mutex>

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

// Split plan.  The len positions of a KV head form ceil(len / 32) blocks of
// 32 rows; split_count(len) = min(kAttnMaxSplits, blocks) splits take
// consecutive runs of them, as evenly as whole blocks allow: each split gets
// blocks / used blocks and the last blocks % used splits one more.  The
// partial last block thus lands in a longer split: at len = 32769 (1025
// blocks) 63 splits hold 16 blocks and the last 17, the 17th a single row,
// so no wave of the 4 in a workgroup runs more than 4 full blocks.  (A
// fixed span of ceil(blocks / 64) blocks would give 61 splits of 17, whose
// first waves run a fifth full block while the other three idle.)
__host__ __device__ constexpr int split_count(int len) {
  return (len + kAttnBlock - 1) / kAttnBlock < kAttnMaxSplits
             ? (len + kAttnBlock - 1) / kAttnBlock
             : kAttnMaxSplits;
}

struct SplitRows {
  int used;   // split_count(len)
  int begin;  // rows [begin, end) of split `split` (split < used)
  int end;
};

__device__ __forceinline__ SplitRows split_rows(int len, int split) {
  const int blocks = (len + kAttnBlock - 1) / kAttnBlock;
  const int used = split_count(len);
  const int per = blocks / used;
  const int shorter = used - blocks % used;  // splits of `per` blocks
  const int first = split * per + max(0, split - shorter);
  const int count = per + (split >= shorter ? 1 : 0);
  SplitRows r;
  r.used = used;
  r.begin = first * kAttnBlock;
  r.end = min((first + count) * kAttnBlock, len);
  return r;
}

struct AttnArgs {
  const uint16_t *q;
  const uint16_t *k;
  const uint16_t *v;
  int64_t head_stride;
  int32_t len;
  int32_t nsplits;  // grid width and partial layout (split_count(len))
  float scale_log2;  // scale * log2(e)
  uint16_t *out;
  float *part_ml;      // [kv_heads][nsplits][G][2]  (max in log2 units, sum)
  float *part_acc;     // [kv_heads][nsplits][G][D]
  // AT kernels: the length is this device word, clamped to [1, len] (len
  // then holds the cache capacity, which sets nsplits; the splits follow
  // the word's length, and those past its plan write empty partials)
  const int64_t *len_word;
  // FUSED kernels: per-KV-head arrival / completion counters (one 128-byte
  // line per head, zero before and after every call) and the caller's
  // error word (kFusedErr* bits are or-ed in)
  uint32_t *sync;
  int32_t *error;
};

// Split merge inside the attention launch ("fused").  The grid is 1-D,
// nsplits x 8 workgroups: workgroup b serves split b / 8 of the KV head
// whose index is the XCC id of the XCD it runs on.  Workgroups are dealt to
// the 8 XCDs round-robin, so each XCD receives one workgroup of every
// index b / 8 -- whichever XCD the round starts at: eagerly launched
// workgroup b lands on XCD b % 8, graph-replayed launches were seen to start
// elsewhere -- and every split of head g runs on XCD g, sharing that XCD's
// L2.  Counters and partials of head g are therefore only touched through
// one L2, where the atomics are performed: after its
// partial stores are acknowledged, a workgroup takes an arrival ticket; the
// last kFusedMergers to arrive wait (bounded) until all nsplits have
// arrived, then each merges one eighth of the head's 4 x 128 outputs --
// the arithmetic, and so the result, of decode_attention_merge_kernel, bit
// for bit -- and the last of them to finish resets the counters.  No
// workgroup waits for one that has not started: only the last arrivals
// wait, for workgroups that already hold their CUs.
// decode_attention_merge_kernel's shape: four quarters of the splits per
// output dim (also the fused merge's)
constexpr int kMergeQuarters = 4;
constexpr int kMergeThreads = kMergeQuarters * kAttnD;
constexpr int kMergePerQuarter = kAttnMaxSplits / kMergeQuarters;
constexpr int kFusedHeads = 8;     // KV heads = XCDs
constexpr int kFusedMergers = 8;   // 4 query heads x 2 halves of 64 dims
constexpr int kFusedLineWords = 32;  // one 128-byte line per head
constexpr int kFusedSpinLimit = 1 << 16;
constexpr int32_t kFusedErrPlacement = 2;  // XCDs got unequal shares of the grid
constexpr int32_t kFusedErrTimeout = 4;    // a merger's wait ran out

static_assert(CASCADE_DECODE_ATTENTION_SYNC_BYTES >= kFusedHeads * kFusedLineWords * 4,
              "sync buffer holds one line per KV head");

template <bool NT>
__device__ __forceinline__ u32x4 kv_load(const uint16_t *p) {
  if constexpr (NT)
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
  else
    return *reinterpret_cast<const u32x4 *>(p);
}

// Atomics performed in the L2 of the calling XCD (workgroup scope: no
// write-back or bypass of the L2), for the fused merge's counters.
__device__ __forceinline__ uint32_t l2_fetch_add(uint32_t *p, uint32_t v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// The counter's current value by an atomic add of zero, issued as an
// instruction of its own: the compiler would turn a fetch_add(p, 0) into a
// plain load, whose hit in the CU's vector cache could return a stale value
// on every poll.
__device__ __forceinline__ uint32_t l2_atomic_read(uint32_t *p) {
  uint32_t old;
  const uint32_t zero = 0;
  asm volatile("global_atomic_add %0, %1, %2, off sc0\n\ts_waitcnt vmcnt(0)"
               : "=&v"(old)
               : "v"(p), "v"(zero)
               : "memory");
  return old;
}

__device__ __forceinline__ void l2_exchange(uint32_t *p, uint32_t v) {
  (void)__hip_atomic_exchange(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// A load that skips the CU's vector cache and reads the L2, where the other
// CUs' partial stores of this XCD landed (global_load ... sc0).
__device__ __forceinline__ float l2_load(const float *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ uint32_t xcc_id() {
  uint32_t v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v & 0xfu;
}

// The fused tail of one workgroup of KV head g (its partial already
// stored): arrival, and for the last kFusedMergers arrivals the merge of
// one slice of the head's outputs.  256 threads.
__device__ __forceinline__ void fused_merge_tail(const AttnArgs &a, int g, int tid) {
  constexpr int G = kAttnG, D = kAttnD;
  constexpr int kSlice = G * D / kFusedMergers;  // 64 dims of one query head
  __shared__ uint32_t s_ticket, s_ok;
  __shared__ float s_w[kAttnMaxSplits];
  __shared__ float s_part[kMergeQuarters][kSlice];
  __shared__ float s_den;
  uint32_t *line = a.sync + g * kFusedLineWords;
  // this wave's partial stores acknowledged by the L2 (stores count in
  // vmcnt on gfx9), then every wave's, before the ticket
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
  __syncthreads();
  if (tid == 0) s_ticket = l2_fetch_add(line, 1u);
  __syncthreads();
  const int first = a.nsplits - kFusedMergers;
  const int ticket = static_cast<int>(s_ticket);
  if (ticket < first) return;
  if (ticket >= a.nsplits) {
    // more workgroups of this head than splits: the XCDs did not receive
    // equal shares of the grid (workgroups not dealt round-robin)
    if (tid == 0)
      __hip_atomic_fetch_or(a.error, kFusedErrPlacement, __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  if (tid == 0) {
    uint32_t seen = 0;
    for (int n = 0; n < kFusedSpinLimit; ++n) {
      seen = l2_atomic_read(line);
      if (seen >= static_cast<uint32_t>(a.nsplits)) break;
      __builtin_amdgcn_s_sleep(1);
    }
    s_ok = seen >= static_cast<uint32_t>(a.nsplits);
    if (!s_ok)
      __hip_atomic_fetch_or(a.error, kFusedErrTimeout, __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_ok) return;

  // slice = (query head h, dims 64 hf ..): decode_attention_merge_kernel's
  // per-output arithmetic with the quarters over 64 instead of 128 dims
  const int slice = ticket - first;
  const int h = slice / 2;
  const int dl = tid % kSlice;
  const int d = kSlice * (slice % 2) + dl;
  const int quarter = tid / kSlice;
  const int64_t base = static_cast<int64_t>(g) * a.nsplits * G + h;
  float v[kMergePerQuarter];
#pragma unroll
  for (int i = 0; i < kMergePerQuarter; ++i) {
    const int c = quarter * kMergePerQuarter + i;
    v[i] = c < a.nsplits ? l2_load(a.part_acc + (base + static_cast<int64_t>(c) * G) * D + d)
                         : 0.0f;
  }
  if (tid < kWave) {
    const float mc = tid < a.nsplits ? l2_load(a.part_ml + (base + tid * G) * 2) : -INFINITY;
    const float lc = tid < a.nsplits ? l2_load(a.part_ml + (base + tid * G) * 2 + 1) : 0.0f;
    const float mx = wave_max(mc);
    const float wc = tid < a.nsplits ? exp2_fast(mc - mx) : 0.0f;
    s_w[tid] = wc;
    const float den = wave_sum(wc * lc);
    if (tid == 0) s_den = den;
  }
  __syncthreads();
  float r = 0.0f;
#pragma unroll
  for (int i = 0; i < kMergePerQuarter; ++i)
    r = fmaf(s_w[quarter * kMergePerQuarter + i], v[i], r);
  s_part[quarter][dl] = r;
  __syncthreads();
  if (quarter == 0) {
    r = s_part[0][dl];
#pragma unroll
    for (int q = 1; q < kMergeQuarters; ++q) r += s_part[q][dl];
    a.out[(static_cast<int64_t>(g) * G + h) * D + d] = f32_to_bf16(r / s_den);
  }
  // the last merger to finish leaves the counters at zero for the next
  // call (every merger has passed its wait by then)
  if (tid == 0 && l2_fetch_add(line + 16, 1u) == kFusedMergers - 1) {
    l2_exchange(line + 16, 0u);
    l2_exchange(line, 0u);
  }
}

template <int WAVES, bool NT, bool AT = false, bool FUSED = false>
__global__ __launch_bounds__(WAVES *kWave) void decode_attention_kernel(
    AttnArgs a) {
  constexpr int G = kAttnG, D = kAttnD;
  constexpr int kPassRows = WAVES * kAttnBlock;
  static_assert(!FUSED || WAVES * kWave == kMergeQuarters * kAttnD / 2,
                "the fused merge runs on 256 threads");
  // FUSED: the XCD the workgroup runs on picks its KV head, its index
  // picks the split (see "Split merge inside the attention launch")
  const int split = FUSED ? static_cast<int>(blockIdx.x) / kFusedHeads
                          : static_cast<int>(blockIdx.x);
  const int g = FUSED ? static_cast<int>(xcc_id()) : static_cast<int>(blockIdx.y);
  const int tid = threadIdx.x;
  if constexpr (FUSED) {
    if (g >= kFusedHeads) {  // a device with more XCDs than KV heads
      if (tid == 0)
        __hip_atomic_fetch_or(a.error, kFusedErrPlacement, __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
  }
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int c16 = lane & 15;
  const int g4 = lane >> 4;
  // AT: the length word is loaded first (the split's rows depend on it)
  int64_t len_word = a.len;
  if constexpr (AT) len_word = *a.len_word;
  // q operand of dim chunk c: B[8 g4 + j][c16] = q[head c16][32 c + 8 g4 + j]
  // (loaded before the length is used, so the two latencies overlap)
  u32x4 qop[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
    qop[c] = c16 < G ? *reinterpret_cast<const u32x4 *>(
                           a.q + (g * G + c16) * D + 32 * c + 8 * g4)
                     : u32x4{0u, 0u, 0u, 0u};
  const int len = static_cast<int>(
      min(max(len_word, int64_t{1}), static_cast<int64_t>(a.len)));
  const SplitRows rows = split_rows(len, split);
  if constexpr (AT) {
    if (split >= rows.used) {
      // A split past the current length's plan (the grid is sized for the
      // capacity): an empty partial, m = -inf and l = 0, which the merge
      // weighs 0.  Split 0 is always used, so nsplits > 1 here.
      const int64_t slot0 = (static_cast<int64_t>(g) * a.nsplits + split) * G;
      for (int i = tid; i < G * D; i += WAVES * kWave)
        a.part_acc[slot0 * D + i] = 0.0f;
      if (tid < G) {
        a.part_ml[(slot0 + tid) * 2] = -INFINITY;
        a.part_ml[(slot0 + tid) * 2 + 1] = 0.0f;
      }
      if constexpr (FUSED) fused_merge_tail(a, g, tid);
      return;
    }
  }
  const int begin = rows.begin;
  const int end = rows.end;
  const uint16_t *kb = a.k + g * a.head_stride;
  const uint16_t *vb = a.v + g * a.head_stride;
  const int krow = 8 * (c16 >> 2) + (c16 & 3);  // + 4 hf

  // K rows of the block as two MFMA halves, V rows as 8 whole rows per lane;
  // rows past last repeat row last
  auto load_block = [&](int r0, int last, u32x4 (&kt)[2][4], u32x4 (&vt)[8]) {
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

  __shared__ float s_ml[WAVES][G][2];
  __shared__ float s_acc[WAVES][G][D];

  const int last = end - 1;
  const uint32_t head_mask = c16 < G ? 0xffffffffu : 0u;  // zero P columns

  float m = -INFINITY, l = 0.0f;
  f32x4 o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

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
    load_block(r0, last, kt, vt);
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
  if constexpr (FUSED) fused_merge_tail(a, g, tid);
}

// Merge of the splits, one workgroup per (KV head, query head): lane c of
// wave 0 reads split c's (m, l), so the maximum and the denominator are
// wave reductions; each quarter of the workgroup sums every dim over its
// quarter of the splits (at most 16 independent loads per thread, issued
// before the weights are known) and the quarters add up in LDS.  A separate
// launch (rather than a last-workgroup ticket) lets the kernel boundary
// publish the partials with one L2 writeback instead of one per workgroup.

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
    r = s_part[0][d];
#pragma unroll
    for (int q = 1; q < kMergeQuarters; ++q) r += s_part[q][d];
    a.out[(static_cast<int64_t>(g) * G + h) * D + d] = f32_to_bf16(r / s_den);
  }
}

// ---------------------------------------------------------------------------
// Causal GQA prefill attention (the is_causal=True SDPA of the prefill call,
// layer_streaming/llama31.py:219-229 with _repeat_kv at :28-31): query token
// t (cache slot past + t) attends to cache positions [0, past + t].
//
// Columns.  A wave owns 4 NB consecutive query tokens of one KV head: NB
// blocks of 16 MFMA columns, column c of block b being (token t0 + 4 b +
// c / 4, query head 4 g + c % 4), so the 4 query heads sharing the KV head
// reuse every K / V fragment.  Per 32-row block of positions the wave runs
//   S = K_blk Q^T  (two 16-row tiles x four 32-dim chunks, per column block)
//   online softmax in registers (scores carry scale * log2 e; exp2)
//   O += V_blk^T P (eight 16-dim tiles; P rounded to bf16 for the MFMA)
// and positions past a column's own limit score -inf.
//
// Balance.  Tokens are cut into units of HW waves x 4 NB tokens; unit u
// needs blocks [0, len(u)), len growing along the causal triangle.
// Workgroup (pair p, KV head g) has 2 HW waves in two halves: half 0 walks
// unit A = p and then the first `split` blocks of unit B = U - 1 - p, half
// 1 walks B's blocks [split, len(B)); `split` evens the two walks, so all
// workgroups do about the same work.  B's two partial softmax states are merged through
// LDS at the end (m, l, o of half 0 rescaled onto half 1's).
//
// Staging.  A half walks its blocks in lockstep; each block is moved once
// into LDS by buffer loads straight to LDS (no staging registers), K two
// blocks ahead of use and V one block ahead, so that in step j a wave reads
// block j's V fragments while its K Q^T products run and block j + 1's K
// fragments while the P V products run.  Each buffer parity is its own
// __shared__ array and the loop is unrolled by two: the compiler can see
// that a step's LDS reads never alias the loads in flight, and waits for
// them only at the step's closing barrier.  LDS layout of a staged 32-row
// block (8 KB): 16-byte slot 32 ch + (r ^ 8 (ch & 1)) holds chunk ch (dims
// 8 ch .. 8 ch + 7) of block row r.  The K fragment reads (16 lanes: rows
// 0-15 or 16-31 of one chunk) and the transposed V reads (32 lanes: 8 rows x
// 2 adjacent chunks) then hit distinct banks, and each read of a step is one
// per-lane base plus an immediate offset.
//
// Softmax.  The running maximum moves only when a block's maximum exceeds it
// by more than kLazyRescale (log2 units); o and l share the stale maximum,
// so the result is unchanged and most rescales are skipped.
//
// MI355X, S = 2048 (config 5, one layer): 55 us with NB = 2, HW = 4 (two
// waves per SIMD), against 150 us for one wave per (4 NB tokens) reading
// K / V from L2 with no balancing, 74 us for NB = 4, HW = 2 (one wave per
// SIMD) and 96 us for NB = 1, HW = 8 (registers spilled).
constexpr int kPrefillBlocks = 2;     // MFMA column blocks per wave
constexpr int kPrefillHalfWaves = 4;  // waves per half of a workgroup
constexpr int kPrefillUnit = kPrefillHalfWaves * 4 * kPrefillBlocks;  // query tokens per unit
constexpr float kLazyRescale = 8.0f;

struct PrefillArgs {
  const uint16_t *q;  // [tokens, n_q_heads * D]
  const uint16_t *k;  // position 0 of KV head 0
  const uint16_t *v;
  int64_t head_stride;
  int32_t past;
  int32_t tokens;
  int32_t q_row;     // n_q_heads * D
  int32_t units;     // ceil(tokens / kPrefillUnit)
  int32_t kv_heads;
  float scale_log2;
  uint16_t *out;  // [tokens, n_q_heads * D]
};

typedef short i16x4 __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16: within each 16-lane group, result lane i element j is
// element i % 4 of the 8 bytes addressed by lane 4 j + i / 4 (checked on
// gfx950).
__device__ __forceinline__ uint2 lds_read_tr16(const uint16_t *p) {
  const i16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) i16x4 *)(p));
  return __builtin_bit_cast(uint2, r);
}

template <int NB, int HW>
__global__ __launch_bounds__(2 * HW * kWave)
__attribute__((amdgpu_waves_per_eu(HW / 2))) void prefill_attention_kernel(
    PrefillArgs a) {
  constexpr int G = kAttnG, D = kAttnD, TOK = 4 * NB;
  constexpr int UNIT = HW * TOK;
  constexpr int LPW = 8 / HW;  // block load instructions per wave
  static_assert(8 % HW == 0, "whole load instructions per wave");
  constexpr int BUF = kAttnBlock * D;
  __shared__ __attribute__((aligned(16))) uint16_t kbuf0[2][BUF];  // [half]
  __shared__ __attribute__((aligned(16))) uint16_t kbuf1[2][BUF];
  __shared__ __attribute__((aligned(16))) uint16_t vbuf0[2][BUF];
  __shared__ __attribute__((aligned(16))) uint16_t vbuf1[2][BUF];
  __shared__ f32x4 mo[HW][NB * 8][kWave];  // half 0's partial o of B
  __shared__ float2 mml[HW][NB][kWave];    // and its m, l

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int half = wave / HW;
  const int w4 = wave % HW;
  const int g = static_cast<int>(blockIdx.x) % a.kv_heads;
  const int pair = static_cast<int>(blockIdx.x) / a.kv_heads;
  const int c16 = lane & 15;
  const int g4 = lane >> 4;
  const int hq = g * G + (c16 & 3);
  const float c = a.scale_log2;

  const int ub = a.units - 1 - pair;
  const int ua = pair < ub ? pair : -1;  // the middle unit of an odd count walks alone
  auto unit_len = [&](int u) {
    return u < 0 ? 0
                 : (a.past + min(u * UNIT + UNIT - 1, a.tokens - 1)) / kAttnBlock + 1;
  };
  const int len_a = unit_len(ua), len_b = unit_len(ub);
  const int split = (len_b - len_a) / 2;
  const int steps = max(len_a + split, len_b - split);
  auto block_at = [&](int j) {
    if (half == 1) return j < len_b - split ? split + j : -1;
    if (j < len_a) return j;
    return j < len_a + split ? j - len_a : -1;
  };

  // block loads: instruction i (0..7) of a block fills slots 64 i .. 64 i + 63,
  // i.e. chunks 2 i, 2 i + 1 of all 32 rows; lane L takes chunk
  // 2 i + L / 32 of row (L % 32) ^ (8 (L / 32)).  Wave w4 issues i = LPW w4 ..
  // LPW w4 + LPW - 1.
  const int last_row = a.past + a.tokens - 1;
  const int ld_row = (lane & 31) ^ (8 * (lane >> 5));
  const int ld_chunk_bytes = 16 * (lane >> 5);
  const __amdgpu_buffer_rsrc_t k_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t *>(a.k + g * a.head_stride), 0, (last_row + 1) * D * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t v_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t *>(a.v + g * a.head_stride), 0, (last_row + 1) * D * 2, 0x00020000);
  auto load_block = [&](__amdgpu_buffer_rsrc_t rsrc, uint16_t *dst, int blk) __attribute__((always_inline)) {
    const int voff = min(blk * kAttnBlock + ld_row, last_row) * (D * 2) + ld_chunk_bytes;
#pragma unroll
    for (int h = 0; h < LPW; ++h) {
      const int i = LPW * w4 + h;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rsrc, (__attribute__((address_space(3))) void *)(dst + 64 * 8 * i), 16,
          voff, 32 * i, 0, 0);
    }
  };

  // fragment read bases (bytes within a block buffer)
  //  K: tile hf, dims 32 cc + 8 g4 ..: slot kv_slot(16 hf + c16, 4 cc + g4)
  //     = 128 cc + 16 hf + [32 g4 + (c16 ^ 8 (g4 & 1))]
  //  V: lane k = 4 j + q of group g4, half h, tile e: row 16 h + 4 g4 + j,
  //     dims 16 e + 4 q: slot kv_slot(16 h + 4 g4 + j, 2 e + q / 2), + 8 (q & 1) bytes
  //     = 64 e + 16 h + [32 (q / 2) + ((4 g4 + j) ^ 8 (q / 2))]
  const int k_base = 16 * (32 * g4 + (c16 ^ (8 * (g4 & 1))));
  const int vq = c16 & 3, vj = c16 >> 2;
  const int v_base = 16 * (32 * (vq >> 1) + ((4 * g4 + vj) ^ (8 * (vq >> 1)))) + 8 * (vq & 1);

  int tq[NB], limit[NB], lim_min = 0;
  u32x4 qop[NB][4];
  float m[NB], l[NB];
  f32x4 o[NB][8];
  auto begin_unit = [&](int u) __attribute__((always_inline)) {
    const int t0 = u * UNIT + w4 * TOK;
    lim_min = a.past + t0;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      tq[b] = t0 + 4 * b + (c16 >> 2);
      limit[b] = a.past + tq[b];
      const int tq_load = min(tq[b], a.tokens - 1);
      const uint16_t *qrow =
          a.q + static_cast<int64_t>(tq_load) * a.q_row + hq * D;
#pragma unroll
      for (int cc = 0; cc < 4; ++cc)
        qop[b][cc] = *reinterpret_cast<const u32x4 *>(qrow + 32 * cc + 8 * g4);
      m[b] = -FLT_MAX;  // finite: a column with no valid row yet keeps alpha = 1
      l[b] = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[b][e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  };
  auto write_out = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float lb = xor32_sum(xor16_sum(l[b]));
      if (tq[b] >= a.tokens) continue;
      const float inv = 1.0f / lb;
      // o[b][e][r] = O[dim 16 e + 4 g4 + r][column c16 of block b]
      uint16_t *orow = a.out + static_cast<int64_t>(tq[b]) * a.q_row + hq * D;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        uint2 packed;
        packed.x = pack_bf16x2(o[b][e][0] * inv, o[b][e][1] * inv);
        packed.y = pack_bf16x2(o[b][e][2] * inv, o[b][e][3] * inv);
        *reinterpret_cast<uint2 *>(orow + 16 * e + 4 * g4) = packed;
      }
    }
  };
  auto read_k = [&](const uint16_t *buf, u32x4 (&kt)[2][4]) __attribute__((always_inline)) {
    const char *base = reinterpret_cast<const char *>(buf) + k_base;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int cc = 0; cc < 4; ++cc)
        kt[hf][cc] = *reinterpret_cast<const u32x4 *>(base + 2048 * cc + 256 * hf);
  };
  auto read_v = [&](const uint16_t *buf, u32x4 (&vf)[8]) __attribute__((always_inline)) {
    const char *base = reinterpret_cast<const char *>(buf) + v_base;
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint2 t = lds_read_tr16(
            reinterpret_cast<const uint16_t *>(base + 1024 * e + 256 * h));
        vf[e][2 * h] = t.x;
        vf[e][2 * h + 1] = t.y;
      }
  };

  bool a_open = half == 0 && len_a > 0;
  begin_unit(a_open ? ua : ub);
  u32x4 kt[2][4];
  {
    const int b0 = block_at(0), b1 = block_at(1);
    if (b0 >= 0) {
      load_block(k_rsrc, kbuf0[half], b0);
      load_block(v_rsrc, vbuf0[half], b0);
    }
    if (b1 >= 0) load_block(k_rsrc, kbuf1[half], b1);
    __syncthreads();
    if (b0 >= 0) read_k(kbuf0[half], kt);
    __syncthreads();  // kbuf0 is refilled in step 0
  }
  // step j, parity P = j & 1: K_{j+2} -> kbuf[P], V_{j+1} -> vbuf[1-P];
  // reads V_j from vbuf[P] and K_{j+1} from kbuf[1-P]
  auto step = [&](int j, uint16_t *k_here, const uint16_t *k_next,
                  const uint16_t *v_here, uint16_t *v_next) __attribute__((always_inline)) {
    const int blk = block_at(j);
    const int nb1 = block_at(j + 1);
    const int nb2 = block_at(j + 2);
    if (nb2 >= 0) load_block(k_rsrc, k_here, nb2);
    if (nb1 >= 0) load_block(v_rsrc, v_next, nb1);
    if (blk >= 0) {
      const int r0 = blk * kAttnBlock;
      u32x4 vf[8];
      read_v(v_here, vf);
      // s[b][4 hf + r]: block row 16 hf + 4 g4 + r, column c16 of block b
      float s[NB][8];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        f32x4 s0 = {0.0f, 0.0f, 0.0f, 0.0f}, s1 = s0;
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
          s0 = mfma_16x16x32_bf16(kt[0][cc], qop[b][cc], s0);
          s1 = mfma_16x16x32_bf16(kt[1][cc], qop[b][cc], s1);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          s[b][r] = s0[r];
          s[b][4 + r] = s1[r];
        }
      }
      if (r0 + kAttnBlock - 1 > lim_min) {  // wave-uniform: a diagonal block
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
          for (int jj = 0; jj < 8; ++jj)
            if (r0 + 16 * (jj >> 2) + 4 * g4 + (jj & 3) > limit[b]) s[b][jj] = -INFINITY;
      }
      u32x4 pop[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        float bmax = max_f32(max_f32(max_f32(s[b][0], s[b][1]), max_f32(s[b][2], s[b][3])),
                             max_f32(max_f32(s[b][4], s[b][5]), max_f32(s[b][6], s[b][7])));
        bmax = xor32_max(xor16_max(bmax)) * c;
        if (bmax > m[b] + kLazyRescale) {
          const float alpha = exp2_fast(m[b] - bmax);
          m[b] = bmax;
          l[b] *= alpha;
#pragma unroll
          for (int e = 0; e < 8; ++e) o[b][e] *= alpha;
        }
        const float nm = -m[b];
        float p[8];
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) p[jj] = exp2_fast(fmaf(s[b][jj], c, nm));
        // P enters the MFMA rounded to bf16; l sums the fp32 values
#pragma unroll
        for (int i2 = 0; i2 < 4; ++i2) {
          pop[b][i2] = pack_bf16x2(p[2 * i2], p[2 * i2 + 1]);
          l[b] += p[2 * i2] + p[2 * i2 + 1];
        }
      }
      if (nb1 >= 0) read_k(k_next, kt);
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int b = 0; b < NB; ++b) o[b][e] = mfma_16x16x32_bf16(vf[e], pop[b], o[b][e]);
    }
    if (a_open && j + 1 == len_a) {  // half 0 leaves A; kt already holds B's block 0
      write_out();
      a_open = false;
      begin_unit(ub);
    }
    __syncthreads();
  };
  for (int j = 0; j < steps; j += 2) {
    step(j, kbuf0[half], kbuf1[half], vbuf0[half], vbuf1[half]);
    if (j + 1 < steps) step(j + 1, kbuf1[half], kbuf0[half], vbuf1[half], vbuf0[half]);
  }
  if (a_open) write_out();
  if (split > 0) {  // workgroup-uniform
    if (half == 0) {
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        mml[w4][b][lane] = make_float2(m[b], l[b]);
#pragma unroll
        for (int e = 0; e < 8; ++e) mo[w4][b * 8 + e][lane] = o[b][e];
      }
    }
    __syncthreads();
    if (half == 1) {
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const float2 ml = mml[w4][b][lane];
        const float mx = fmaxf(ml.x, m[b]);
        const float ax = exp2_fast(ml.x - mx), ay = exp2_fast(m[b] - mx);
        l[b] = ml.y * ax + l[b] * ay;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[b][e] = mo[w4][b * 8 + e][lane] * ax + o[b][e] * ay;
      }
    }
  }
  if (half == 1) write_out();
}

constexpr size_t attention_workspace(int64_t nsplits, int64_t n_kv_heads) {
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

// Argument checks and packing shared by the two decode entry points; len
// is the attended length (the capacity for the AT form).
static int decode_attention_args(const void *q, const void *k_cache,
                                 const void *v_cache, int64_t kv_head_stride,
                                 int64_t len, int64_t n_q_heads,
                                 int64_t n_kv_heads, int64_t head_dim,
                                 float scale, void *out, void *workspace,
                                 size_t workspace_bytes, AttnArgs &a) {
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
  const int nsplits = split_count(static_cast<int>(len));
  if (workspace_bytes < attention_workspace(nsplits, n_kv_heads))
    return CASCADE_EWORKSPACE;
  a.q = static_cast<const uint16_t *>(q);
  a.k = static_cast<const uint16_t *>(k_cache);
  a.v = static_cast<const uint16_t *>(v_cache);
  a.head_stride = kv_head_stride;
  a.len = static_cast<int32_t>(len);
  a.nsplits = nsplits;
  a.scale_log2 = scale * kLog2e;
  a.out = static_cast<uint16_t *>(out);
  char *ws = static_cast<char *>(workspace);
  const size_t per = static_cast<size_t>(n_kv_heads) * nsplits * kAttnG;
  a.part_ml = reinterpret_cast<float *>(ws + kAttnHeaderBytes);
  a.part_acc = reinterpret_cast<float *>(ws + kAttnHeaderBytes +
                                         per * 2 * sizeof(float));
  return 0;
}

template <bool AT>
static int launch_decode_attention(const AttnArgs &a, int64_t n_kv_heads,
                                   hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(a.nsplits),
                  static_cast<unsigned>(n_kv_heads));
  const hipError_t e =
      launch_kernel(decode_attention_kernel<kAttnWaves, true, AT>, grid,
                    dim3(kAttnWaves * kWave), 0, s, a);
  if (e != hipSuccess || a.nsplits == 1) return e;
  return launch_kernel(decode_attention_merge_kernel,
                       dim3(static_cast<unsigned>(n_kv_heads * kAttnG)),
                       dim3(kMergeThreads), 0, s, a);
}

// One launch of nsplits x 8 workgroups with the split merge inside.
template <bool AT>
static int launch_decode_attention_fused(AttnArgs &a, int64_t n_kv_heads, void *sync,
                                         int32_t *error_flag, hipStream_t s) {
  if (sync == nullptr || error_flag == nullptr) return CASCADE_EINVAL;
  if ((reinterpret_cast<uintptr_t>(sync) & 127) || (reinterpret_cast<uintptr_t>(error_flag) & 3))
    return CASCADE_EALIGN;
  if (n_kv_heads != kFusedHeads || a.nsplits < kFusedMergers) return CASCADE_ESHAPE;
  a.sync = static_cast<uint32_t *>(sync);
  a.error = error_flag;
  return launch_kernel(decode_attention_kernel<kAttnWaves, true, AT, true>,
                       dim3(static_cast<unsigned>(a.nsplits * kFusedHeads)),
                       dim3(kAttnWaves * kWave), 0, s, a);
}

extern "C" int cascade_decode_attention_fused_bf16(
    const void *q, const void *k_cache, const void *v_cache,
    int64_t kv_head_stride, int64_t len, int64_t n_q_heads, int64_t n_kv_heads,
    int64_t head_dim, float scale, void *out, void *workspace,
    size_t workspace_bytes, void *sync, int32_t *error_flag, void *stream) {
  AttnArgs a{};
  if (int e = decode_attention_args(q, k_cache, v_cache, kv_head_stride, len,
                                    n_q_heads, n_kv_heads, head_dim, scale,
                                    out, workspace, workspace_bytes, a))
    return e;
  return launch_decode_attention_fused<false>(a, n_kv_heads, sync, error_flag,
                                              static_cast<hipStream_t>(stream));
}

extern "C" int cascade_decode_attention_fused_at_bf16(
    const void *q, const void *k_cache, const void *v_cache,
    int64_t kv_head_stride, const int64_t *length, int64_t capacity,
    int64_t n_q_heads, int64_t n_kv_heads, int64_t head_dim, float scale,
    void *out, void *workspace, size_t workspace_bytes, void *sync,
    int32_t *error_flag, void *stream) {
  if (length == nullptr) return CASCADE_EINVAL;
  if (reinterpret_cast<uintptr_t>(length) & 7) return CASCADE_EALIGN;
  AttnArgs a{};
  if (int e = decode_attention_args(q, k_cache, v_cache, kv_head_stride,
                                    capacity, n_q_heads, n_kv_heads, head_dim,
                                    scale, out, workspace, workspace_bytes, a))
    return e;
  a.len_word = length;
  return launch_decode_attention_fused<true>(a, n_kv_heads, sync, error_flag,
                                             static_cast<hipStream_t>(stream));
}

extern "C" int cascade_decode_attention_bf16(
    const void *q, const void *k_cache, const void *v_cache,
    int64_t kv_head_stride, int64_t len, int64_t n_q_heads, int64_t n_kv_heads,
    int64_t head_dim, float scale, void *out, void *workspace,
    size_t workspace_bytes, void *stream) {
  AttnArgs a{};
  if (int e = decode_attention_args(q, k_cache, v_cache, kv_head_stride, len,
                                    n_q_heads, n_kv_heads, head_dim, scale,
                                    out, workspace, workspace_bytes, a))
    return e;
  return launch_decode_attention<false>(a, n_kv_heads,
                                        static_cast<hipStream_t>(stream));
}

extern "C" int cascade_decode_attention_at_bf16(
    const void *q, const void *k_cache, const void *v_cache,
    int64_t kv_head_stride, const int64_t *length, int64_t capacity,
    int64_t n_q_heads, int64_t n_kv_heads, int64_t head_dim, float scale,
    void *out, void *workspace, size_t workspace_bytes, void *stream) {
  if (length == nullptr) return CASCADE_EINVAL;
  if (reinterpret_cast<uintptr_t>(length) & 7) return CASCADE_EALIGN;
  AttnArgs a{};
  if (int e = decode_attention_args(q, k_cache, v_cache, kv_head_stride,
                                    capacity, n_q_heads, n_kv_heads, head_dim,
                                    scale, out, workspace, workspace_bytes, a))
    return e;
  a.len_word = length;
  return launch_decode_attention<true>(a, n_kv_heads,
                                       static_cast<hipStream_t>(stream));
}

// ------------------------------------------------- no-allocation variant
// The split partials of cascade_decode_attention_noalloc_bf16 live in this
// file-scope device array (one copy per GPU, held until the process ends).
// It covers up to kNoAllocMaxKvHeads KV heads at the largest split count.
// In host code `scratch` names a host-side stand-in; its device address on
// each GPU comes from hipGetSymbolAddress and is the only form host code
// hands to a kernel.
constexpr int64_t kNoAllocMaxKvHeads = CASCADE_DECODE_ATTENTION_NOALLOC_MAX_KV_HEADS;
constexpr size_t kNoAllocScratchBytes =
    attention_workspace(kAttnMaxSplits, kNoAllocMaxKvHeads);
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxScratchDevices = 64;
std::atomic<void *> g_scratch[kMaxScratchDevices];
std::mutex g_scratch_lock;

// Device address of `scratch` on the device that owns `s`, looked up once
// per device with that device current.
int scratch_on_stream_device(hipStream_t s, void **out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (s != nullptr) {
    hipDevice_t owner = 0;
    e = hipStreamGetDevice(s, &owner);
    if (e != hipSuccess) return e;
    dev = static_cast<int>(owner);
  }
  if (dev < 0 || dev >= kMaxScratchDevices) return CASCADE_EINVAL;
  void *p = g_scratch[dev].load(std::memory_order_acquire);
  if (p != nullptr) {
    *out = p;
    return 0;
  }
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  p = g_scratch[dev].load(std::memory_order_relaxed);
  if (p == nullptr) {
    int current = 0;
    e = hipGetDevice(&current);
    if (e != hipSuccess) return e;
    if (current != dev && (e = hipSetDevice(dev)) != hipSuccess) return e;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (current != dev) {
      const hipError_t back = hipSetDevice(current);
      if (e == hipSuccess) e = back;
    }
    if (e != hipSuccess) return e;
    if (p == nullptr) return hipErrorInvalidSymbol;
    g_scratch[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return 0;
}

}  // namespace

extern "C" int cascade_decode_attention_noalloc_bf16(
    const void *q, const void *k_cache, const void *v_cache,
    int64_t kv_head_stride, int64_t len, int64_t n_q_heads, int64_t n_kv_heads,
    int64_t head_dim, float scale, void *out, void *stream) {
  if (n_kv_heads > kNoAllocMaxKvHeads) return CASCADE_ESCRATCH;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  void *ws = nullptr;
  if (int e = scratch_on_stream_device(s, &ws)) return e;
  AttnArgs a{};
  if (int e = decode_attention_args(q, k_cache, v_cache, kv_head_stride, len,
                                    n_q_heads, n_kv_heads, head_dim, scale,
                                    out, ws, kNoAllocScratchBytes, a))
    return e;
  return launch_decode_attention<false>(a, n_kv_heads, s);
}

extern "C" int cascade_prefill_attention_bf16(
    const void *q, const void *k_cache, const void *v_cache,
    int64_t kv_head_stride, int64_t past, int64_t tokens, int64_t n_q_heads,
    int64_t n_kv_heads, int64_t head_dim, float scale, void *out,
    void *stream) {
  if (q == nullptr || k_cache == nullptr || v_cache == nullptr ||
      out == nullptr)
    return CASCADE_EINVAL;
  // positions < 2^24: per-head byte offsets of the buffer loads are 32-bit
  if (tokens <= 0 || past < 0 || past + tokens > (int64_t{1} << 24) ||
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
  a.units = static_cast<int32_t>((tokens + kPrefillUnit - 1) / kPrefillUnit);
  a.kv_heads = static_cast<int32_t>(n_kv_heads);
  a.scale_log2 = scale * kLog2e;
  a.out = static_cast<uint16_t *>(out);
  // one workgroup per (unit pair, KV head); consecutive workgroups take
  // consecutive KV heads
  const int64_t workgroups = (a.units + 1) / 2 * n_kv_heads;
  if (workgroups > 0x7fffffff) return CASCADE_EINVAL;
  return launch_kernel(prefill_attention_kernel<kPrefillBlocks, kPrefillHalfWaves>,
                       dim3(static_cast<unsigned>(workgroups)),
                       dim3(2 * kPrefillHalfWaves * kWave), 0,
                       static_cast<hipStream_t>(stream), a);
}
