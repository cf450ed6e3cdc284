// One Llama-3.1-8B-shaped decoder layer of batch-1 decode as one persistent
// launch on gfx950 (MI355X), or its MLP half (o_proj .. down_proj).
//
// The per-stage path (gemv.hip, attention.hip) runs a layer as six kernels:
// q|k|v, attention, split merge, o_proj, gate/up, down_proj, each paying a
// few microseconds of dispatch, ramp-up and drain.  This kernel runs the
// same stages in one launch of 256 workgroups (one per CU, all resident at
// once) with a grid barrier between stages, and issues each stage's first
// weight (or K / V) loads before the barrier that opens it, so the barrier
// overlaps HBM traffic the stage needs anyway.  Measured on config 4 it is
// on par with the per-stage kernels, not faster (the stage tails of uneven
// per-CU bandwidth and the hand-off latencies eat the launch savings), so
// callers select it explicitly.
//
// Stages (reference: layer_streaming/llama31.py).  Wave 0 of a workgroup is
// the control wave; waves 1..7 (workers) carry the rows:
//   A  RMSNorm + q|k|v rows + RoPE; q -> scratch, k / v -> cache slot
//      len - 1 (:169-180, :206-218, :241-245)    12 (d, d + 64) pairs / WG
//   B  attention over positions [0, len) (:219-229): KV head g = wg % 8,
//      split wg / 8 of 32; worker w walks 32-row blocks w, w + 7, ...
//   C  split merge -> attn (bf16), control wave       1 (head, 16 dims) / WG
//   D  o_proj + residual -> x (:246-251)              16 rows / WG
//   E  RMSNorm + gate/up + SwiGLU -> inter (:252-275) 56 row pairs / WG
//   F  down_proj + residual -> x (:276-279)           16 rows / WG
// Workgroup b takes rows b, b + 256, b + 512, ... of every matrix, so each
// XCD (b % 8) reads rows spread over the whole matrix: with contiguous
// blocks per workgroup, some XCDs were measured ~30% slower than others on
// the same stage, depending on where the matrix sits in memory.
// Each GEMV row is computed exactly as gemv.hip computes it (same loads,
// same dot8 order, same wave reduction and rounding points, same RMSNorm
// reduction order), so stages A, D, E and F give the per-stage path's
// results bit for bit on the same input.
//
// Coherence.  The 8 XCDs' L2 caches are not coherent with each other.
// Everything one stage hands to the next (q, the new K / V row, split
// partials, attn, x, inter) is written with device-scope (sc1) stores and
// read with sc1 loads, which go to the coherent level, so a barrier needs no
// L2 writeback or invalidate.  Weights and the older cache rows, written
// before the launch, are read with ordinary nontemporal loads.
//
// Grid barrier.  One counter per XCD (workgroup b runs on XCD b % 8), one
// counter over the XCDs and a generation word.  The last arrival of an XCD
// bumps the counter over the XCDs; the last XCD sets the generation; every
// workgroup's control wave spins (bounded) on the generation.  Counters only
// grow, so a launch takes the generation it finds at start as its base and
// needs no reset; a spin that runs out sets the error word and every later
// wait falls through, so the grid always drains.
#include "cascade_device.h"
#include "cascade_internal.h"

namespace cascade {
namespace {

constexpr int kLH = 4096;         // hidden size
constexpr int kLI = 14336;        // intermediate size
constexpr int kLQ = 32;           // query heads
constexpr int kLKV = 8;           // KV heads
constexpr int kLD = 128;          // head dim
constexpr int kLG = kLQ / kLKV;   // query heads per KV head
constexpr int kLWaves = 8;
constexpr int kLThreads = kLWaves * kWave;
constexpr int kLGrid = 256;       // one workgroup per CU
constexpr int kLSplits = kLGrid / kLKV;  // attention splits per KV head
constexpr int kLBlock = 32;       // attention rows per wave step
constexpr int kKcH = kLH / 512;   // 16-byte loads per lane, 4096-long row
constexpr int kKcI = kLI / 512;   // 16-byte loads per lane, 14336-long row
constexpr int kQkvPairs = (kLQ + 2 * kLKV) * kLD / 2;  // (d, d + 64) pairs
constexpr float kLLog2e = 1.4426950408889634f;
static_assert(kLGrid == kLQ * 8, "merge: one (head, 16 dims) per workgroup");

// Sync words (uint32), one 64-byte line each: 8 arrival counters (one per
// XCD), the counter over the XCDs, the generation, the error word.
constexpr int kSyncLine = 16;
constexpr int kSyncAll = 8 * kSyncLine;
constexpr int kSyncGen = 9 * kSyncLine;
constexpr int kSyncErr = 10 * kSyncLine;
constexpr int kPerXcd = kLGrid / 8;
static_assert((kPerXcd & (kPerXcd - 1)) == 0, "counters wrap cleanly");
constexpr uint32_t kSpinLimit = 1u << 21;

// Workspace layout (bytes; the public offsets are part of the C ABI).
constexpr size_t kWsQ = CASCADE_DECODE_LAYER_Q;
constexpr size_t kWsAttn = CASCADE_DECODE_LAYER_ATTN;
constexpr size_t kWsInter = CASCADE_DECODE_LAYER_INTER;
static_assert(kWsAttn == kWsQ + kLH * 2 && kWsInter == kWsAttn + kLH * 2, "layout");
static_assert(CASCADE_DECODE_LAYER_ERROR == kSyncErr * 4, "error word");
constexpr size_t kWsMl = kWsInter + kLI * 2;
constexpr size_t kWsAcc = kWsMl + size_t{kLKV} * kLSplits * kLG * 2 * 4;
constexpr size_t kWsBytes = kWsAcc + size_t{kLKV} * kLSplits * kLG * kLD * 4;

// Buffer-load cache policies: nontemporal (read once) and device-coherent.
constexpr int kPolicyNt = 2;
constexpr int kPolicySc1 = 16;
// s_waitcnt vmcnt(0) with expcnt / lgkmcnt left alone
constexpr int kWaitVm0 = (7 << 4) | (15 << 8);

struct LayerArgs {
  const uint16_t *wq, *wk, *wv, *wo, *wg, *wu, *wd;
  const uint16_t *norm_in, *norm_post;
  float eps;
  float scale_log2;
  uint16_t *x;                          // hidden state [kLH], updated in place
  const uint16_t *rope_cos, *rope_sin;  // this position's rows [64]
  uint16_t *k_cache, *v_cache;          // position 0 of KV head 0
  int64_t head_stride;
  int32_t len;     // positions attended; the new token sits at len - 1
  int32_t span;    // positions per split (a multiple of kLBlock)
  int32_t n_used;  // splits holding positions
  uint16_t *q, *attn, *inter;
  float *part_ml;   // [kv head][split][G][2]  (max in log2 units, sum)
  float *part_acc;  // [kv head][split][G][D]
  uint32_t *sync;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t whole_rsrc(const void *base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0,
                                           0x7fffffff, 0x00020000);
}

template <int POLICY>
__device__ __forceinline__ u32x4 bload(__amdgpu_buffer_rsrc_t r, int off, int soff = 0) {
  return __builtin_bit_cast(u32x4,
                            __builtin_amdgcn_raw_buffer_load_b128(r, off, soff, POLICY));
}

__device__ __forceinline__ uint32_t ld_agent(const uint32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t *p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint16_t ld_agent16(const uint16_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent16(uint16_t *p, uint16_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent_f32(const float *p) {
  return __uint_as_float(ld_agent(reinterpret_cast<const uint32_t *>(p)));
}
__device__ __forceinline__ void st_agent_f32(float *p, float v) {
  st_agent(reinterpret_cast<uint32_t *>(p), __float_as_uint(v));
}

// Arrival of this workgroup (control lane 0, after the workgroup's stores
// completed).  Polling a line that no arrival touches keeps the spinners
// off the counters' lines: polling the 8 counters themselves (256 waves x 8
// loads per spin) was measured to slow the arrivals and the release by
// 2-4 us.
__device__ __forceinline__ void grid_arrive(uint32_t *sync, uint32_t target) {
  const uint32_t old = __hip_atomic_fetch_add(
      sync + (blockIdx.x % 8) * kSyncLine, 1u, __ATOMIC_RELAXED,
      __HIP_MEMORY_SCOPE_AGENT);
  if (((old + 1) & (kPerXcd - 1)) != 0) return;
  const uint32_t old2 = __hip_atomic_fetch_add(sync + kSyncAll, 1u, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
  if (((old2 + 1) & 7) == 0) st_agent(sync + kSyncGen, target);
}

// Wait (control lane 0) until the generation reaches target; bounded.  On
// time-out the error word is set, and every later wait falls through.
__device__ __forceinline__ void grid_wait(uint32_t *sync, uint32_t target) {
  uint32_t spins = 0;
  while (static_cast<int32_t>(ld_agent(sync + kSyncGen) - target) < 0) {
    if (++spins >= kSpinLimit ||
        ((spins & 255) == 0 && ld_agent(sync + kSyncErr) != 0)) {
      st_agent(sync + kSyncErr, 1u);
      return;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// 16-byte loads of one weight row, lane l taking pieces l, l + 64, ...
template <int KC>
__device__ __forceinline__ void load_row(const uint16_t *row, int lane,
                                         u32x4 (&w)[KC]) {
  const __amdgpu_buffer_rsrc_t r = whole_rsrc(row);
  // 4 KiB steps in soffset (an SGPR), the rest in the 12-bit immediate: one
  // offset register per row instead of one per 4 KiB
#pragma unroll
  for (int c = 0; c < KC; ++c)
    w[c] = bload<kPolicyNt>(r, 16 * lane + 1024 * (c % 4), 4096 * (c / 4));
}

// Row sums against the staged vector: the dot8 order of gemv_kernel (two
// accumulators over alternate pieces), then the wave reduction.
template <int R, int KC>
__device__ __forceinline__ void gemv_rows(const u32x4 (&w)[R][KC], const u32x4 *xs,
                                          int lane, float (&acc)[R]) {
  float acc2[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = acc2[r] = 0.0f;
#pragma unroll
  for (int c = 0; c < KC; ++c) {
    const u32x4 xv = xs[c * kWave + lane];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (c & 1)
        acc2[r] = dot8_bf16(w[r][c], xv, acc2[r]);
      else
        acc[r] = dot8_bf16(w[r][c], xv, acc[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r] + acc2[r]);
}

// The control wave's copy of the N-element bf16 vector at src (sc1 loads)
// into xs, RMS-normalised with norm_w when given (_rms_norm,
// llama31.py:21-25).  The sum of squares is reduced in the order of
// gemv.hip's stage_input run with T threads (thread t sums pieces t, t + T,
// ... in turn, each wave reduces its threads, the waves add up in order), so
// the vector equals the per-stage kernel's bit for bit.
template <int N, int T>
__device__ __forceinline__ void ctl_stage(const uint16_t *src, const uint16_t *norm_w,
                                          float eps, u32x4 *xs, int lane) {
  constexpr int kVec = N / 8;
  constexpr int kPer = kVec / kWave;  // pieces per lane: lane + 64 i
  constexpr int kWavesT = T / kWave;
  static_assert(kVec % kWave == 0 && T % kWave == 0, "whole pieces per lane");
  const __amdgpu_buffer_rsrc_t r = whole_rsrc(src);
  if (norm_w == nullptr) {
    // straight into LDS (buffer_load ... lds: lane l of instruction i fills
    // xs[64 i + l]), no registers held; the per-instruction offset rides in
    // soffset, which does not move the LDS destination
#pragma unroll
    for (int i = 0; i < kPer; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          r, (__attribute__((address_space(3))) void *)(xs + kWave * i), 16, 16 * lane,
          1024 * i, 0, kPolicySc1);
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    return;
  }
  u32x4 v[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) v[i] = bload<kPolicySc1>(r, 16 * (lane + kWave * i));
  const u32x4 *wg = reinterpret_cast<const u32x4 *>(norm_w);
  u32x4 nw[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) nw[i] = wg[lane + kWave * i];
  // piece lane + 64 i belongs to wave i % kWavesT of the T-thread layout
  float total = 0.0f;
#pragma unroll
  for (int w = 0; w < kWavesT; ++w) {
    float ss = 0.0f;
#pragma unroll
    for (int i = w; i < kPer; i += kWavesT) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = lo_bf16(v[i][e]);
        const float hi = hi_bf16(v[i][e]);
        ss = fmaf(lo, lo, ss);
        ss = fmaf(hi, hi, ss);
      }
    }
    total += wave_sum(ss);
  }
  const float variance = total * (1.0f / static_cast<float>(N));
  const float rr = 1.0f / __builtin_sqrtf(variance + eps);
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float nlo = round_bf16(lo_bf16(v[i][e]) * rr);
      const float nhi = round_bf16(hi_bf16(v[i][e]) * rr);
      const uint32_t olo = f32_to_bf16(lo_bf16(nw[i][e]) * nlo);
      const uint32_t ohi = f32_to_bf16(hi_bf16(nw[i][e]) * nhi);
      o[e] = olo | (ohi << 16);
    }
    xs[lane + kWave * i] = o;
  }
}

__device__ __forceinline__ float layer_silu(float g) { return g / (1.0f + expf(-g)); }

// Roles inside a workgroup.  vmcnt, the counter a wave waits on for its
// vector loads and stores, completes in issue order on gfx950: a wave that
// still has weight loads in flight cannot see its spin load, its arrival
// atomic or its stores complete before those weights land.  So wave 0 (the
// control wave) never holds long loads: it spins at the barriers, stages
// each stage's input vector into LDS, runs the split merge and makes every
// store that leaves the workgroup.  Waves 1..7 (workers) only load weights
// and K / V -- ahead of the barriers, as deep as their registers allow --
// compute, and hand their results to the control wave through LDS.  The
// kernel branches once on the (wave-uniform) role; both paths pass the same
// 16 workgroup barriers in the same order, and their registers never
// overlap.
constexpr int kWorkers = kLWaves - 1;
constexpr int kQkvPerWg = kQkvPairs / kLGrid;   // 12 (d, d + 64) pairs
constexpr int kRowsPerWg = kLH / kLGrid;         // 16 o_proj / down_proj rows
constexpr int kPairsPerWg = kLI / kLGrid;        // 56 gate/up pairs
constexpr int kPairsPerWorker = kPairsPerWg / kWorkers;  // 8
static_assert(kQkvPairs % kLGrid == 0 && kPairsPerWg % kWorkers == 0, "even split");
static_assert(kRowsPerWg > 2 * kWorkers && kRowsPerWg <= 3 * kWorkers, "2-3 rows / worker");
static_assert(kQkvPerWg > kWorkers && kQkvPerWg <= 2 * kWorkers, "1-2 pairs / worker");
static_assert(kPairsPerWorker % 2 == 0, "pairs alternate between two buffers");

struct LayerShared {
  u32x4 xs[kLI / 8];  // staged GEMV input vector
  float ml[kLWaves][kLG][2];
  float acc[kLWaves][kLG][kLD];
  float out[kLG * kLD];  // worker results for the control wave
  float out_ml[kLG][2];
  float w[kLSplits];
  uint32_t pair[kQkvPerWg];
};

// Split geometry of stage B for workgroup b: KV head b % 8, split b / 8.
struct AttnSplit {
  int g, split, begin, end, nb;
  __device__ AttnSplit(const LayerArgs &a, int blk) {
    g = blk % kLKV;
    split = blk / kLKV;
    begin = split * a.span;
    end = min(begin + a.span, a.len);
    nb = begin < end ? (end - begin + kLBlock - 1) / kLBlock : 0;
  }
};

// The workgroup merge of stage B for output t (query head t / 128, dim
// t % 128): the waves' partial softmax states combined into this split's
// (m, l, acc).  Every wave takes part; a wave without rows has m = -inf,
// l = 0, acc = 0 and weight 0 (worker 0 always has rows).
__device__ __forceinline__ void attn_wg_merge(LayerShared &sh, int t) {
  const int h = t / kLD, d = t % kLD;
  float mm = -INFINITY;
#pragma unroll
  for (int w = 0; w < kLWaves; ++w) mm = fmaxf(mm, sh.ml[w][h][0]);
  float den = 0.0f, r = 0.0f;
#pragma unroll
  for (int w = 0; w < kLWaves; ++w) {
    const float wt = __builtin_amdgcn_exp2f(sh.ml[w][h][0] - mm);
    den = fmaf(wt, sh.ml[w][h][1], den);
    r = fmaf(wt, sh.acc[w][h][d], r);
  }
  sh.out[t] = r;
  if (d == 0) {
    sh.out_ml[h][0] = mm;
    sh.out_ml[h][1] = den;
  }
}

// ------------------------------------------------------------------ workers
template <bool MLP>
__device__ __forceinline__ void layer_worker(const LayerArgs &a, LayerShared &sh,
                                             int blk, int wave, int lane) {
  const int wi = wave - 1;

  if constexpr (!MLP) {
  // ------------------------------------------------------------ A: q|k|v
  {
    // pair p = b + 256 k (k < 12): rows (d, d + 64) of head p / 64,
    // d = p % 64; heads 0..31 are q, 32..39 k, 40..47 v.  Worker w takes
    // k = w and k = w + 7.
    auto row_ptr = [&](int p, int half) {
      const int head = p >> 6;
      const int d = (p & 63) + 64 * half;
      if (head < kLQ) return a.wq + static_cast<int64_t>(head * kLD + d) * kLH;
      if (head < kLQ + kLKV)
        return a.wk + static_cast<int64_t>((head - kLQ) * kLD + d) * kLH;
      return a.wv + static_cast<int64_t>((head - kLQ - kLKV) * kLD + d) * kLH;
    };
    const int k0 = wi, k1 = wi + kWorkers;
    const bool has1 = k1 < kQkvPerWg;
    const int p0 = blk + kLGrid * k0, p1 = blk + kLGrid * k1;
    u32x4 w0[2][kKcH], w1[2][kKcH];
    load_row<kKcH>(row_ptr(p0, 0), lane, w0[0]);
    load_row<kKcH>(row_ptr(p0, 1), lane, w0[1]);
    if (has1) {
      load_row<kKcH>(row_ptr(p1, 0), lane, w1[0]);
      load_row<kKcH>(row_ptr(p1, 1), lane, w1[1]);
    }
    __syncthreads();  // S1: input staged
    auto emit = [&](int k, int p, const float (&acc)[2]) {
      const int d = p & 63;
      const float xa = round_bf16(acc[0]);  // element d of the head
      const float xb = round_bf16(acc[1]);  // element d + 64
      uint32_t oa, ob;
      if ((p >> 6) < kLQ + kLKV) {
        // apply_rotary_pos_emb in bf16 (llama31.py:206-218)
        const float c = bf16_to_f32(a.rope_cos[d]);
        const float s = bf16_to_f32(a.rope_sin[d]);
        oa = f32_to_bf16(round_bf16(xa * c) + round_bf16(-xb * s));
        ob = f32_to_bf16(round_bf16(xb * c) + round_bf16(xa * s));
      } else {
        oa = f32_to_bf16(xa);
        ob = f32_to_bf16(xb);
      }
      sh.pair[k] = oa | (ob << 16);
    };
    {
      float acc[2];
      gemv_rows<2, kKcH>(w0, sh.xs, lane, acc);
      if (lane == 0) emit(k0, p0, acc);
    }
    if (has1) {
      float acc[2];
      gemv_rows<2, kKcH>(w1, sh.xs, lane, acc);
      if (lane == 0) emit(k1, p1, acc);
    }
    __syncthreads();  // S2: results to the control wave
  }

  // ------------------------------------------------------------ B: attention
  {
    constexpr int G = kLG, D = kLD;
    const AttnSplit sp(a, blk);
    const int c16 = lane & 15;
    const int g4 = lane >> 4;
    // worker w walks blocks w, w + 7, ... of the split
    const int nbw = sp.nb > wi ? (sp.nb - wi + kWorkers - 1) / kWorkers : 0;
    // the block holding the new row (len - 1) is the last block of the
    // last split, loaded coherently after the barrier
    const bool holds_new = sp.end == a.len && sp.nb > 0 && (sp.nb - 1) % kWorkers == wi;
    const int last = sp.end - 1;
    const __amdgpu_buffer_rsrc_t kr = whole_rsrc(a.k_cache + sp.g * a.head_stride);
    const __amdgpu_buffer_rsrc_t vr = whole_rsrc(a.v_cache + sp.g * a.head_stride);
    const int krow = 8 * (c16 >> 2) + (c16 & 3);  // + 4 hf
    auto block_r0 = [&](int i) { return sp.begin + kLBlock * (wi + kWorkers * i); };
    auto is_new = [&](int i) { return holds_new && i == nbw - 1; };
    auto load_block = [&](int i, u32x4 (&kt)[2][4], u32x4 (&vt)[8]) {
      const int r0 = block_r0(i);
      int koff[2], voff[8];
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
        koff[hf] = min(r0 + krow + 4 * hf, last) * (D * 2) + 16 * g4;
#pragma unroll
      for (int j = 0; j < 8; ++j) voff[j] = min(r0 + 8 * g4 + j, last) * (D * 2) + 16 * c16;
      if (is_new(i)) {
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
          for (int c = 0; c < 4; ++c) kt[hf][c] = bload<kPolicySc1>(kr, koff[hf] + 64 * c);
#pragma unroll
        for (int j = 0; j < 8; ++j) vt[j] = bload<kPolicySc1>(vr, voff[j]);
      } else {
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
          for (int c = 0; c < 4; ++c) kt[hf][c] = bload<kPolicyNt>(kr, koff[hf] + 64 * c);
#pragma unroll
        for (int j = 0; j < 8; ++j) vt[j] = bload<kPolicyNt>(vr, voff[j]);
      }
    };
    u32x4 ktA[2][4], vtA[8], ktB[2][4], vtB[8];
    // prefetch: the worker's first block, unless it holds the new row.  One
    // 16 KiB block per worker (112 KiB per CU) covers the barrier; more
    // would queue ahead of the control wave's stores and barrier traffic
    // in the CU's memory pipeline and delay them.
    if (0 < nbw && !is_new(0)) load_block(0, ktA, vtA);
    __syncthreads();  // S3: grid barrier 1 passed

    if (0 < nbw && is_new(0)) load_block(0, ktA, vtA);
    if (1 < nbw) load_block(1, ktB, vtB);
    // q operand of dim chunk c: B[8 g4 + j][c16] = q[head c16][32 c + 8 g4 + j]
    u32x4 qop[4];
    {
      const __amdgpu_buffer_rsrc_t qr = whole_rsrc(a.q);
#pragma unroll
      for (int c = 0; c < 4; ++c)
        qop[c] = c16 < G ? bload<kPolicySc1>(qr, 2 * ((sp.g * G + c16) * D + 32 * c + 8 * g4))
                         : u32x4{0u, 0u, 0u, 0u};
    }
    const uint32_t head_mask = c16 < G ? 0xffffffffu : 0u;
    float m = -INFINITY, l = 0.0f;
    f32x4 o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // one 32-row block: S = K q^T (8 MFMAs), online softmax, O += V^T P
    // (8 MFMAs), as attention.hip's decode kernel
    auto step = [&](int i, const u32x4 (&kt)[2][4], const u32x4 (&vt)[8]) {
      const int r0 = block_r0(i);
      f32x4 s0 = {0.0f, 0.0f, 0.0f, 0.0f}, s1 = s0;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        s0 = mfma_16x16x32_bf16(kt[0][c], qop[c], s0);
        s1 = mfma_16x16x32_bf16(kt[1][c], qop[c], s1);
      }
      float s[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
      float bmax = -INFINITY;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        s[j] = r0 + 8 * g4 + j < sp.end ? s[j] * a.scale_log2 : -INFINITY;
        bmax = fmaxf(bmax, s[j]);
      }
      bmax = xor32_max(xor16_max(bmax));
      const float mnew = fmaxf(m, bmax);
      const float alpha = __builtin_amdgcn_exp2f(m - mnew);
      m = mnew;
      float p[8], psum = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        p[j] = __builtin_amdgcn_exp2f(s[j] - mnew);
        psum += p[j];
      }
      l = fmaf(l, alpha, psum);
      u32x4 pop;
#pragma unroll
      for (int k = 0; k < 4; ++k) pop[k] = pack_bf16x2(p[2 * k], p[2 * k + 1]) & head_mask;
      if (alpha != 1.0f) {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] *= alpha;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = mfma_16x16x32_bf16(v_operand(vt, e), pop, o[e]);
    };
    for (int i = 0; i < nbw; i += 2) {
      step(i, ktA, vtA);
      if (i + 2 < nbw) load_block(i + 2, ktA, vtA);
      if (i + 1 < nbw) {
        step(i + 1, ktB, vtB);
        if (i + 3 < nbw) load_block(i + 3, ktB, vtB);
      }
    }
    l = xor32_sum(xor16_sum(l));
    if (c16 < G) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int e = 0; e < 8; ++e) sh.acc[wave][c16][8 * (4 * g4 + r) + e] = o[e][r];
      if (g4 == 0) {
        sh.ml[wave][c16][0] = m;
        sh.ml[wave][c16][1] = l;
      }
    }
    __syncthreads();  // S4: every wave's state in LDS
    if (sp.nb > 0) attn_wg_merge(sh, wave * kWave + lane);
    __syncthreads();  // S5: split partials to the control wave
  }
  }  // !MLP

  // D rows r(m) = b + 256 m (m < 16), F rows the same: worker w takes
  // m = w, w + 7 and, for w < 2, w + 14.  Their weights and gate/up pair 0
  // go out now and stay in flight through the merge.
  auto out_row = [&](int t) { return blk + kLGrid * (wi + kWorkers * t); };
  const bool row2 = wi + 2 * kWorkers < kRowsPerWg;
  u32x4 wo[3][kKcH];
  load_row<kKcH>(a.wo + static_cast<int64_t>(out_row(0)) * kLH, lane, wo[0]);
  load_row<kKcH>(a.wo + static_cast<int64_t>(out_row(1)) * kLH, lane, wo[1]);
  if (row2) load_row<kKcH>(a.wo + static_cast<int64_t>(out_row(2)) * kLH, lane, wo[2]);
  // gate/up pair j of worker w: gate and up row i = b + 256 (w + 7 j)
  auto load_pair = [&](int j, u32x4 (&w)[2][kKcH]) {
    const int64_t i = blk + kLGrid * (wi + kWorkers * j);
    load_row<kKcH>(a.wg + i * kLH, lane, w[0]);
    load_row<kKcH>(a.wu + i * kLH, lane, w[1]);
  };
  u32x4 pa[2][kKcH], pb[2][kKcH];
  if constexpr (!MLP) {
    __syncthreads();  // S6: grid barrier 2 passed (the control wave merges)
    __syncthreads();  // S7: the control wave's merge loads are out
    load_pair(0, pa);
    __syncthreads();  // S8: grid barrier 3 passed
  }

  // ------------------------------------------------------------ D: o_proj
  __syncthreads();  // S9: attn staged
#pragma unroll
  for (int t = 0; t < 3; ++t) {
    if (t < 2 || row2) {
      float acc[1];
      gemv_rows<1, kKcH>(*reinterpret_cast<const u32x4(*)[1][kKcH]>(&wo[t]), sh.xs, lane, acc);
      if (lane == 0) sh.out[wi + kWorkers * t] = acc[0];
    }
  }
  __syncthreads();  // S10: results to the control wave
  if constexpr (MLP) {
    load_pair(0, pa);
    __syncthreads();  // S11: grid barrier 4 passed
    load_pair(1, pb);
  } else {
    load_pair(1, pb);
    __syncthreads();  // S11: grid barrier 4 passed
  }

  // ------------------------------------------------------------ E: gate/up
  __syncthreads();  // S12: normalised x staged
  auto emit = [&](int j, const float (&acc)[2]) {
    // bf16(bf16(silu(bf16(g))) * bf16(u)) (llama31.py:264-275)
    const float gt = round_bf16(acc[0]);
    const float u = round_bf16(acc[1]);
    const float sg = round_bf16(layer_silu(gt));
    sh.out[wi + kWorkers * j] = sg * u;
  };
#pragma unroll
  for (int j = 0; j < kPairsPerWorker; j += 2) {
    float acc[2];
    gemv_rows<2, kKcH>(pa, sh.xs, lane, acc);
    if (lane == 0) emit(j, acc);
    if (j + 2 < kPairsPerWorker) load_pair(j + 2, pa);
    gemv_rows<2, kKcH>(pb, sh.xs, lane, acc);
    if (lane == 0) emit(j + 1, acc);
    if (j + 3 < kPairsPerWorker) load_pair(j + 3, pb);
  }
  __syncthreads();  // S13: results to the control wave
  // down row 0 in flight before the barrier, row 1 after it
  u32x4 da[1][kKcI], db[1][kKcI];
  load_row<kKcI>(a.wd + static_cast<int64_t>(out_row(0)) * kLI, lane, da[0]);
  __syncthreads();  // S14: grid barrier 5 passed
  load_row<kKcI>(a.wd + static_cast<int64_t>(out_row(1)) * kLI, lane, db[0]);

  // ------------------------------------------------------------ F: down
  __syncthreads();  // S15: inter staged
  {
    float acc[1];
    gemv_rows<1, kKcI>(da, sh.xs, lane, acc);
    if (lane == 0) sh.out[wi] = acc[0];
    // row 2 reuses row 0's registers: keep its loads below row 0's
    // products (hoisted, three rows would be live at once)
    __builtin_amdgcn_sched_barrier(0);
    if (row2) load_row<kKcI>(a.wd + static_cast<int64_t>(out_row(2)) * kLI, lane, da[0]);
    gemv_rows<1, kKcI>(db, sh.xs, lane, acc);
    if (lane == 0) sh.out[wi + kWorkers] = acc[0];
    if (row2) {
      gemv_rows<1, kKcI>(da, sh.xs, lane, acc);
      if (lane == 0) sh.out[wi + 2 * kWorkers] = acc[0];
    }
  }
  __syncthreads();  // S16: results to the control wave
}

// ------------------------------------------------------------ control wave
template <bool MLP>
__device__ __forceinline__ void layer_control(const LayerArgs &a, LayerShared &sh,
                                              int blk, int lane) {
  // generation of the last barrier passed (lane 0): the value found at
  // start -- no workgroup can complete barrier 1 before all have read it
  uint32_t gen = 0;
  if (lane == 0) gen = ld_agent(a.sync + kSyncGen);
  // residual values of the D / F rows (lane m < 16: row b + 256 m); x is not
  // written before stage D in this launch
  float xr = 0.0f;
  if (lane < kRowsPerWg) xr = bf16_to_f32(ld_agent16(a.x + blk + kLGrid * lane));
  // this wave's stores complete, then the workgroup arrives
  auto arrive = [&]() {
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    if (lane == 0) grid_arrive(a.sync, ++gen);
  };
  auto wait = [&]() {
    if (lane == 0) grid_wait(a.sync, gen);
    __syncthreads();
  };

  if constexpr (!MLP) {
  // ------------------------------------------------------------ A
  ctl_stage<kLH, kLThreads>(a.x, a.norm_in, a.eps, sh.xs, lane);
  __syncthreads();  // S1
  __syncthreads();  // S2
  if (lane < 2 * kQkvPerWg) {
    const int k = lane >> 1, half = lane & 1;
    const int p = blk + kLGrid * k;
    const int head = p >> 6;
    const uint16_t val = static_cast<uint16_t>(half ? sh.pair[k] >> 16 : sh.pair[k]);
    uint16_t *dst;
    if (head < kLQ)
      dst = a.q + head * kLD;
    else if (head < kLQ + kLKV)
      dst = a.k_cache + (head - kLQ) * a.head_stride + static_cast<int64_t>(a.len - 1) * kLD;
    else
      dst = a.v_cache + (head - kLQ - kLKV) * a.head_stride +
            static_cast<int64_t>(a.len - 1) * kLD;
    st_agent16(dst + (p & 63) + 64 * half, val);
  }
  arrive();

  // ------------------------------------------------------------ B
  const AttnSplit sp(a, blk);
  wait();  // S3
  // this wave walks no blocks: empty softmax state
  if ((lane & 15) < kLG) {
    const int h = lane & 15, g4 = lane >> 4;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int e = 0; e < 8; ++e) sh.acc[0][h][8 * (4 * g4 + r) + e] = 0.0f;
    if (g4 == 0) {
      sh.ml[0][h][0] = -INFINITY;
      sh.ml[0][h][1] = 0.0f;
    }
  }
  __syncthreads();  // S4
  if (sp.nb > 0) attn_wg_merge(sh, lane);
  __syncthreads();  // S5
  if (sp.nb > 0) {
    const int base = (sp.g * kLSplits + sp.split) * kLG;  // slot of query head 0
#pragma unroll
    for (int i = 0; i < kLG * kLD / kWave; ++i)
      st_agent_f32(a.part_acc + base * kLD + lane + kWave * i, sh.out[lane + kWave * i]);
    if (lane < 2 * kLG) st_agent_f32(a.part_ml + base * 2 + lane, sh.out_ml[lane >> 1][lane & 1]);
  }
  arrive();
  wait();  // S6

  // ------------------------------------------------------------ C: merge
  {
    const int qh = blk / 8;  // query head
    const int d0 = 16 * (blk % 8);
    const int g = qh / kLG, h = qh % kLG;
    const int d = d0 + (lane & 15);
    // lane: dim d, splits (lane >> 4) + 4 i
    float v[kLSplits / 4];
#pragma unroll
    for (int i = 0; i < kLSplits / 4; ++i) {
      const int s = (lane >> 4) + 4 * i;
      v[i] = s < a.n_used
                 ? ld_agent_f32(a.part_acc + ((g * kLSplits + s) * kLG + h) * kLD + d)
                 : 0.0f;
    }
    const int slot = (g * kLSplits + lane) * kLG + h;
    const float mc = lane < a.n_used ? ld_agent_f32(a.part_ml + slot * 2) : -INFINITY;
    const float lc = lane < a.n_used ? ld_agent_f32(a.part_ml + slot * 2 + 1) : 0.0f;
    __syncthreads();  // S7: loads out; the workers' gate/up loads queue behind
    const float mx = wave_max(mc);
    const float wc = lane < a.n_used ? __builtin_amdgcn_exp2f(mc - mx) : 0.0f;
    const float den = wave_sum(wc * lc);
    if (lane < kLSplits) sh.w[lane] = wc;  // read back by this wave only
    float r = 0.0f;
#pragma unroll
    for (int i = 0; i < kLSplits / 4; ++i) r = fmaf(sh.w[(lane >> 4) + 4 * i], v[i], r);
    r = xor32_sum(xor16_sum(r));
    if (lane < 16) st_agent16(a.attn + qh * kLD + d, f32_to_bf16(r / den));
  }
  arrive();
  wait();  // S8
  }  // !MLP

  // ------------------------------------------------------------ D
  ctl_stage<kLH, kLThreads>(a.attn, nullptr, 0.0f, sh.xs, lane);
  __syncthreads();  // S9
  __syncthreads();  // S10
  // residual + F.linear, rounded as bf16 tensors (llama31.py:246-251); xr
  // keeps the new value for stage F, which updates the same rows
  if (lane < kRowsPerWg) {
    xr = round_bf16(xr + round_bf16(sh.out[lane]));
    st_agent16(a.x + blk + kLGrid * lane, f32_to_bf16(xr));
  }
  arrive();
  wait();  // S11

  // ------------------------------------------------------------ E
  ctl_stage<kLH, 4 * kWave>(a.x, a.norm_post, a.eps, sh.xs, lane);
  __syncthreads();  // S12
  __syncthreads();  // S13
  if (lane < kPairsPerWg) st_agent16(a.inter + blk + kLGrid * lane, f32_to_bf16(sh.out[lane]));
  arrive();
  wait();  // S14

  // ------------------------------------------------------------ F
  ctl_stage<kLI, kLThreads>(a.inter, nullptr, 0.0f, sh.xs, lane);
  __syncthreads();  // S15
  __syncthreads();  // S16
  if (lane < kRowsPerWg)
    st_agent16(a.x + blk + kLGrid * lane, f32_to_bf16(round_bf16(xr + round_bf16(sh.out[lane]))));
}

// MLP = false: the whole layer (stages A..F).  MLP = true: stages D..F
// only, from an attention output the caller computed (a.attn): o_proj +
// residual, RMSNorm + gate/up + SwiGLU, down_proj + residual.
template <bool MLP>
__global__ __launch_bounds__(kLThreads) void decode_layer_kernel(LayerArgs a) {
  __shared__ LayerShared sh;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
  const int blk = static_cast<int>(blockIdx.x);
  if (wave == 0)
    layer_control<MLP>(a, sh, blk, lane);
  else
    layer_worker<MLP>(a, sh, blk, wave, lane);
}

struct DeviceInfo {
  int checked = 0;  // 0: not yet, 1: usable, -1: not usable
};
DeviceInfo g_devices[64];

// The grid barriers need all 256 workgroups resident at once: a device of
// 256 CUs, each able to hold a workgroup of this kernel (checked once per
// device).  A cooperative launch would guarantee residency too, but costs
// ~20 us per launch on MI355X (an empty cooperative launch, measured)
// against ~2.3 us for a plain one; with one workgroup per CU and nothing
// else holding the CUs, a plain launch makes all of them resident, and a
// barrier that still waits too long ends with the error word set.
bool layer_device_ok() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  DeviceInfo &info = g_devices[dev];
  if (info.checked == 0) {
    int cus = 0, blocks = 0;
    const bool ok =
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, decode_layer_kernel<false>,
                                                     kLThreads, 0) == hipSuccess &&
        blocks >= 1 && cus == kLGrid;
    info.checked = ok ? 1 : -1;
  }
  return info.checked == 1;
}

}  // namespace
}  // namespace cascade

using namespace cascade;

extern "C" size_t cascade_decode_layer_workspace_bytes(void) { return kWsBytes; }

extern "C" int cascade_decode_layer_bf16(
    const void *wq, const void *wk, const void *wv, const void *wo,
    const void *w_gate, const void *w_up, const void *w_down,
    const void *norm_in, const void *norm_post, float eps, void *x,
    const void *rope_cos, const void *rope_sin, void *k_cache, void *v_cache,
    int64_t kv_head_stride, int64_t len, float scale, void *workspace,
    size_t workspace_bytes, void *stream) {
  const void *in[] = {wq, wk, wv, wo, w_gate, w_up, w_down, norm_in, norm_post,
                      x, rope_cos, rope_sin, k_cache, v_cache, workspace};
  for (const void *p : in)
    if (p == nullptr) return CASCADE_EINVAL;
  for (const void *p : in)
    if (!aligned16(p)) return CASCADE_EALIGN;
  if (len < 1 || len > (int64_t{1} << 23)) return CASCADE_EINVAL;
  if (kv_head_stride < len * kLD || (kv_head_stride & 7)) return CASCADE_EINVAL;
  if (workspace_bytes < kWsBytes) return CASCADE_EWORKSPACE;
  if (!layer_device_ok()) return CASCADE_ESHAPE;
  // splits of whole 32-row blocks, as even as the block count allows
  const int64_t blocks = (len + kLBlock - 1) / kLBlock;
  const int64_t span = (blocks + kLSplits - 1) / kLSplits * kLBlock;
  char *ws = static_cast<char *>(workspace);
  LayerArgs a{};
  a.wq = static_cast<const uint16_t *>(wq);
  a.wk = static_cast<const uint16_t *>(wk);
  a.wv = static_cast<const uint16_t *>(wv);
  a.wo = static_cast<const uint16_t *>(wo);
  a.wg = static_cast<const uint16_t *>(w_gate);
  a.wu = static_cast<const uint16_t *>(w_up);
  a.wd = static_cast<const uint16_t *>(w_down);
  a.norm_in = static_cast<const uint16_t *>(norm_in);
  a.norm_post = static_cast<const uint16_t *>(norm_post);
  a.eps = eps;
  a.scale_log2 = scale * kLLog2e;
  a.x = static_cast<uint16_t *>(x);
  a.rope_cos = static_cast<const uint16_t *>(rope_cos);
  a.rope_sin = static_cast<const uint16_t *>(rope_sin);
  a.k_cache = static_cast<uint16_t *>(k_cache);
  a.v_cache = static_cast<uint16_t *>(v_cache);
  a.head_stride = kv_head_stride;
  a.len = static_cast<int32_t>(len);
  a.span = static_cast<int32_t>(span);
  a.n_used = static_cast<int32_t>((len + span - 1) / span);
  a.q = reinterpret_cast<uint16_t *>(ws + kWsQ);
  a.attn = reinterpret_cast<uint16_t *>(ws + kWsAttn);
  a.inter = reinterpret_cast<uint16_t *>(ws + kWsInter);
  a.part_ml = reinterpret_cast<float *>(ws + kWsMl);
  a.part_acc = reinterpret_cast<float *>(ws + kWsAcc);
  a.sync = reinterpret_cast<uint32_t *>(ws);
  return launch_kernel(decode_layer_kernel<false>, dim3(kLGrid), dim3(kLThreads), 0,
                       static_cast<hipStream_t>(stream), a);
}

extern "C" int cascade_decode_mlp_bf16(const void *wo, const void *w_gate,
                                       const void *w_up, const void *w_down,
                                       const void *norm_post, float eps,
                                       const void *attn, void *x, void *workspace,
                                       size_t workspace_bytes, void *stream) {
  const void *in[] = {wo, w_gate, w_up, w_down, norm_post, attn, x, workspace};
  for (const void *p : in)
    if (p == nullptr) return CASCADE_EINVAL;
  for (const void *p : in)
    if (!aligned16(p)) return CASCADE_EALIGN;
  if (workspace_bytes < kWsBytes) return CASCADE_EWORKSPACE;
  if (!layer_device_ok()) return CASCADE_ESHAPE;
  char *ws = static_cast<char *>(workspace);
  LayerArgs a{};
  a.wo = static_cast<const uint16_t *>(wo);
  a.wg = static_cast<const uint16_t *>(w_gate);
  a.wu = static_cast<const uint16_t *>(w_up);
  a.wd = static_cast<const uint16_t *>(w_down);
  a.norm_post = static_cast<const uint16_t *>(norm_post);
  a.eps = eps;
  a.x = static_cast<uint16_t *>(x);
  a.attn = const_cast<uint16_t *>(static_cast<const uint16_t *>(attn));
  a.inter = reinterpret_cast<uint16_t *>(ws + kWsInter);
  a.sync = reinterpret_cast<uint32_t *>(ws);
  return launch_kernel(decode_layer_kernel<true>, dim3(kLGrid), dim3(kLThreads), 0,
                       static_cast<hipStream_t>(stream), a);
}
