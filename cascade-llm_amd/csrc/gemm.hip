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
// Tiling.  A workgroup computes a BM x 128 output tile (or two side by
// side), K walked in 64-deep slabs (32-deep for the 256-column tiles); each
// wave owns 64 (or 128) rows x 64 (or 32) columns of
// v_mfma_f32_16x16x32_bf16 fragments and reads its A and B fragments (16
// bytes a lane) from LDS.  Shapes (launch_gemm picks one):
//   GemmTileWide 256 x 256 (two 128-column sub-tiles), 8 waves of 128 x 64,
//                32-deep slabs on a ring of 4: where its schedule of rounds
//                is shorter than GemmTile256's (the resident LM head over
//                every prompt row at M = 2048: 16 rounds);
//   GemmTile256  256 x 128, 8 waves, a ring of 3 slab buffers: the large
//                GEMMs (at least as many 256-row tiles as CUs: q, o, gate,
//                up, down and the fused gate|up at M = 2048);
//   GemmTile128  128 x 128, 4 waves, a ring of 4;
//   GemmTile64   64 x 128, 4 waves, a ring of 6: where 128-row tiles would
//                leave CUs idle (the N = 1024 K / V projections at M = 2048,
//                prompts of at most 64 tokens).
// When the last round of tiles would leave at least half of the CUs idle,
// the last tile columns run as tiles of half the height in the same launch
// (GemmTileWideHalf, 128 x 256, for GemmTileWide; GemmTile128x8 for
// GemmTile256; GemmTile64 for GemmTile128): M = 2048,
// N = 14336 runs 768 full tiles in three rounds, then 256 half tiles,
// instead of three and a half rounds of full tiles.
//
// Staging.  Slabs move global -> LDS by buffer loads that write LDS
// themselves (buffer_load_dwordx4 ... lds: no staging registers, no
// ds_write), issued from inline asm (dma_lds16) so that the compiler, which
// cannot tell which ring buffer such a load writes, adds no waits of its
// own.  Slab s lives in ring buffer s % STAGES.  Step s waits (explicit
// vmcnt) for this wave's loads of slab s + 1 only, one barrier publishes
// slab s + 1 and frees slab s's buffer, the first MFMAs of slab s issue,
// and the rest of the step runs in chunks, one per load instruction of
// slab s + STAGES (into the freed buffer): each chunk issues its load, then
// its share of slab s's MFMAs interleaved with its share of slab s + 1's
// fragment reads.  The MFMAs run from the registers filled one step
// earlier, so they never wait on an LDS read; and the loads leave one at a
// time over the step instead of all eight waves queueing theirs at the
// CU's load path right after the barrier, where a wave stuck behind its
// own burst held up its MFMAs (M = 2048, rotating weights, same bits:
// q/o_proj 61.3 -> 55.7 us, down_proj 190.5 -> 185.9, q|k|v-shaped
// N = 6144 95.8 -> 85.2, fused gate|up 407.0 -> 395.1).
//
// LDS layout of a slab: 128-byte rows (64 bf16) back to back; 16-byte
// chunk c of row r sits at chunk c ^ ((r / 2) % 8) (32-deep slabs: 64-byte
// rows, chunk c ^ ((r / 4) % 4)).  A fragment read (16
// lanes: 16 consecutive rows, one chunk) then hits 16 distinct 16-byte bank
// groups, each read is a per-lane base plus an immediate offset, and a load
// instruction (64 lanes x 16 bytes) fills 8 whole rows, so its lanes read
// whole 128-byte row segments.  Rows past m (X) or past a matrix's rows (W)
// read as zeros through the buffer bounds; their results are not stored.
//
// A wave's columns are not contiguous: its first-half fragments and its
// second-half fragments sit 64 columns apart, so fragment j and j + H of
// one lane hold columns c and c + 64.  That pairs the two halves of a head
// (RoPE's rotate_half) and, with gate rows in tile columns 0..63 and up
// rows in 64..127, a gate and its up value, so those epilogues need no data
// exchange.
//
// Tile order.  Workgroups are dispatched round-robin over the 8 XCDs (each
// with its own L2); workgroup b runs logical tile (b % 8) * (grid / 8) +
// b / 8, so an XCD walks a contiguous range of logical tiles, which are
// ordered in groups of 4 M-tiles (column-major inside a group).  A round of
// an XCD's 32 CUs then covers a 4 x 8 block of tiles, which loads each X
// slab line 8 times and each W slab line 4 times from the XCD's L2 (83% hit
// at best, against 79% for 8 x 4; measured 1-2% faster on q, down_proj,
// q|k|v and gate|up at M = 2048).
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
#include <algorithm>
#include <atomic>
#include <type_traits>

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

constexpr int kTileN = 128;
constexpr int kTileK = 64;
constexpr int kGroupM = 4;
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
  // full tiles: a tiles_m x tiles_n grid (tiles of them, per_xcd on each
  // XCD); half-height tiles: an htiles_m x htiles_n grid right of it
  int32_t tiles_m, tiles_n, tiles, per_xcd;
  int32_t htiles_m, htiles_n, htiles, hper_xcd;
  int32_t vec_out;  // row pitches and widths allow 16-byte output accesses
  // split K (fp32 partials, kGemmF32 only): workgroup row blockIdx.y runs
  // slabs [blockIdx.y * split_slabs, + split_slabs) of K and writes its
  // partial at yf + blockIdx.y * split_stride; 0: the whole K
  int32_t split_slabs;
  int64_t split_stride;
};

__device__ __forceinline__ float gemm_silu(float g) {
  return g / (1.0f + expf(-g));
}

// Tile (tm, tn) of logical tile t in a tiles_m x tiles_n grid (false:
// padding workgroup, no work).  Logical tiles run in groups of kGroupM
// tile rows, column-major inside a group.
__device__ __forceinline__ bool gemm_tile(int t, int tiles, int tiles_m, int tiles_n,
                                          int &tm, int &tn) {
  if (t >= tiles) return false;
  const int group_size = kGroupM * tiles_n;
  const int group = t / group_size;
  const int first = group * kGroupM;
  const int gm = min(kGroupM, tiles_m - first);
  const int r = t - group * group_size;
  tm = first + r % gm;
  tn = r / gm;
  return true;
}

// Tile shapes.  A tile is NSUB sub-tiles of 128 columns side by side (a
// sub-tile is one head of q|k|v, or 64 gate + 64 up rows); the BM rows of a
// sub-tile are split over WM x WN waves, each owning FM x FN fragments of
// 16 x 16.
template <int BM_, int WM_, int WN_, int NSUB_ = 1>
struct GemmTile {
  static constexpr int BM = BM_;
  static constexpr int WM = WM_;
  static constexpr int WN = WN_;
  static constexpr int NSUB = NSUB_;
  static constexpr int BN = kTileN * NSUB;
  static constexpr int SUBWAVES = WM * WN;  // waves of one sub-tile
  static constexpr int WAVES = SUBWAVES * NSUB;
  static constexpr int FM = BM / WM / 16;
  static constexpr int FN = kTileN / WN / 16;
  static constexpr int H = FN / 2;  // fragments per half sub-tile
  // staged epilogue: bf16 per staged column (BM rows + 8 pad; the column
  // stride is 4 banks mod 64, so 16 lanes writing 16 columns hit 16
  // distinct 4-bank groups)
  static constexpr int STAGE_COL = BM + 8;
  static_assert(WAVES == 4 || WAVES == 8, "4 or 8 waves");
};
using GemmTile256 = GemmTile<256, 4, 2>;  // 8 waves of 64 x 64
using GemmTile128 = GemmTile<128, 2, 2>;  // 4 waves of 64 x 64
using GemmTile64 = GemmTile<64, 1, 4>;    // 4 waves of 64 x 32
using GemmTile128x8 = GemmTile<128, 2, 4>;  // 8 waves of 64 x 32 (half of GemmTile256)
using GemmTileWide = GemmTile<256, 2, 2, 2>;      // 8 waves of 128 x 64, 256 columns
using GemmTileWideHalf = GemmTile<128, 2, 2, 2>;  // 8 waves of 64 x 64, 256 columns

// Tile column of fragment j of wave column wn for lane row lr.  A wave's
// first-half fragments (j < H) and second-half fragments (j >= H) sit 64
// columns apart, so fragment j and j + H of one lane hold columns c and
// c + 64: the two halves of a RoPE head, or a gate row and its up row.
template <class T>
__device__ __forceinline__ int gemm_col(int wn, int j, int lr) {
  return 16 * T::H * wn + 16 * (j % T::H) + 64 * (j / T::H) + lr;
}

// only_j >= 0: store only fragment column only_j (the element-wise
// epilogues; RoPE and SwiGLU pair fragment j with j + H and need both).
template <int EPI, class T>
__device__ __forceinline__ void gemm_epilogue(
    const GemmArgs &a, int tm, int tn, int wm, int wn, int lane,
    const f32x4 (&acc)[T::FM][T::FN], int only_j = -1) {
  const int lr = lane & 15;
  const int lq = lane >> 4;
#pragma unroll
  for (int i = 0; i < T::FM; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t row = static_cast<int64_t>(tm) * T::BM +
                          (T::BM / T::WM) * wm + 16 * i + 4 * lq + r;
      if (row >= a.m) continue;
      if constexpr (EPI == kGemmQkvRope) {
        const int64_t hq = a.n0 / kGemmHead, hk = a.n1 / kGemmHead;
        const int64_t pos = a.pos0 + row;
#pragma unroll
        for (int j = 0; j < T::H; ++j) {
          const int d = gemm_col<T>(wn, j, lr);  // 0..63
          const float xa = round_bf16(acc[i][j][r]);
          const float xb = round_bf16(acc[i][j + T::H][r]);
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
        for (int j = 0; j < T::H; ++j) {
          const int64_t col =
              static_cast<int64_t>(tn) * kGemmHalfHead + gemm_col<T>(wn, j, lr);
          const float g = round_bf16(acc[i][j][r]);
          const float u = round_bf16(acc[i][j + T::H][r]);
          const float s = round_bf16(gemm_silu(g));
          a.y[row * a.ldy + col] = f32_to_bf16(s * u);
        }
      } else {
#pragma unroll
        for (int j = 0; j < T::FN; ++j) {
          if (only_j >= 0 && j != only_j) continue;
          const int64_t col =
              static_cast<int64_t>(tn) * kTileN + gemm_col<T>(wn, j, lr);
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

// Vectorised epilogue.  The waves first write their fragments to LDS in
// column-major order (a lane's 4 rows of one column are 8 contiguous bytes:
// one ds_write_b64 per fragment), then read them back row-major with
// ds_read_b64_tr_b16, which hands lane i of a 16-lane group row i of the 4
// columns the group addresses, so every lane ends up with 8 consecutive
// columns of one row and loads aux / stores results 16 bytes at a time.
// Column stride (BM + 8) bf16 (GemmTile::STAGE_COL): the fragment writes
// of a lane group fall in distinct banks.  The values staged are those of
// the direct epilogue's rounding points (bf16(acc), or the final SwiGLU
// product), so results are the same bit for bit.

__device__ __forceinline__ uint2 stage_read_tr(const uint16_t *p) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4 *)(p));
  return __builtin_bit_cast(uint2, r);
}

__device__ __forceinline__ float lo_f(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float hi_f(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

template <int EPI, class T>
__device__ __forceinline__ void gemm_epilogue_staged(
    const GemmArgs &a, int tm, int tn, int wm, int wn, int lane, int wave,
    const f32x4 (&acc)[T::FM][T::FN], uint16_t *stage) {
  const int lr = lane & 15;
  const int lq = lane >> 4;
  const int arow = (T::BM / T::WM) * wm;
  // items: 16 rows x 32 columns of the output sub-tile; lane (g, i) of a
  // wave takes row i, columns 8 g .. 8 g + 7 of the item.  Wave w of the
  // sub-tile takes items w, w + SUBWAVES, ...
  constexpr int TW = EPI == kGemmSwiglu || EPI == kGemmQkvRope ? 64 : kTileN;
  constexpr int kItems = (T::BM / 16) * (TW / 32);
  constexpr int kPer = kItems / T::SUBWAVES;
  static_assert(kItems % T::SUBWAVES == 0, "whole items per wave");
  const int g = lq, li = lr;
  auto item_r0 = [&](int n) { return 16 * ((wave + T::SUBWAVES * n) / (TW / 32)); };
  auto item_c0 = [&](int n) { return 32 * ((wave + T::SUBWAVES * n) % (TW / 32)) + 8 * g; };
  const int64_t ncols = a.n0;  // output width (SwiGLU: n_half)

  // ---- inputs the epilogue reads from memory, issued first so their
  // latency overlaps the staging below
  u32x4 in0[kPer], in1[kPer];
#pragma unroll
  for (int n = 0; n < kPer; ++n) {
    const int64_t row = static_cast<int64_t>(tm) * T::BM + item_r0(n) + li;
    in0[n] = in1[n] = u32x4{0u, 0u, 0u, 0u};
    if (row >= a.m) continue;
    if constexpr (EPI == kGemmResidual || EPI == kGemmMul) {
      const int64_t col = static_cast<int64_t>(tn) * TW + item_c0(n);
      if (col + 8 <= ncols)
        in0[n] = *reinterpret_cast<const u32x4 *>(a.aux + row * a.ldy + col);
    } else if constexpr (EPI == kGemmQkvRope) {
      if (tn < (a.n0 + a.n1) / kGemmHead) {
        const int64_t pos = a.pos0 + row;
        in0[n] = *reinterpret_cast<const u32x4 *>(a.rope_cos + pos * kGemmHalfHead + item_c0(n));
        in1[n] = *reinterpret_cast<const u32x4 *>(a.rope_sin + pos * kGemmHalfHead + item_c0(n));
      }
    }
  }

  // ---- fragments -> LDS (column-major, 4 rows per 8-byte piece)
  if constexpr (EPI == kGemmSwiglu) {
    // column c (0..63) holds bf16(silu(bf16(gate c)) * bf16(up c))
#pragma unroll
    for (int i = 0; i < T::FM; ++i)
#pragma unroll
      for (int j = 0; j < T::H; ++j) {
        const int col = gemm_col<T>(wn, j, lr);
        uint2 v;
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float gt = round_bf16(acc[i][j][r]);
          const float u = round_bf16(acc[i][j + T::H][r]);
          o[r] = round_bf16(gemm_silu(gt)) * u;
        }
        v.x = pack_bf16x2(o[0], o[1]);
        v.y = pack_bf16x2(o[2], o[3]);
        *reinterpret_cast<uint2 *>(stage + col * T::STAGE_COL + arow + 16 * i + 4 * lq) = v;
      }
  } else {
#pragma unroll
    for (int i = 0; i < T::FM; ++i)
#pragma unroll
      for (int j = 0; j < T::FN; ++j) {
        const int col = gemm_col<T>(wn, j, lr);
        uint2 v;
        v.x = pack_bf16x2(acc[i][j][0], acc[i][j][1]);
        v.y = pack_bf16x2(acc[i][j][2], acc[i][j][3]);
        *reinterpret_cast<uint2 *>(stage + col * T::STAGE_COL + arow + 16 * i + 4 * lq) = v;
      }
  }
  __syncthreads();

  // ---- LDS -> rows
  const int qk = li >> 2, qq = li & 3;  // addressing lane k = 4 j + q of the group
  auto read8 = [&](int r0, int c0, uint32_t (&w)[4]) {
    // two transposed reads: columns c0 .. c0 + 3 and c0 + 4 .. c0 + 7
    const uint2 lo = stage_read_tr(stage + (c0 + qk) * T::STAGE_COL + r0 + 4 * qq);
    const uint2 hi = stage_read_tr(stage + (c0 + 4 + qk) * T::STAGE_COL + r0 + 4 * qq);
    w[0] = lo.x; w[1] = lo.y; w[2] = hi.x; w[3] = hi.y;
  };
#pragma unroll
  for (int n = 0; n < kPer; ++n) {
    const int r0 = item_r0(n), c0 = item_c0(n);
    const int64_t row = static_cast<int64_t>(tm) * T::BM + r0 + li;
    // the transposed reads need every addressing lane: read before any
    // lane drops out
    uint32_t w[4], w2[4];
    read8(r0, c0, w);  // bf16 pairs: columns c0 + 2 p, c0 + 2 p + 1
    if constexpr (EPI == kGemmQkvRope) read8(r0, c0 + kGemmHalfHead, w2);  // d + 64
    if (row >= a.m) continue;
    if constexpr (EPI == kGemmQkvRope) {
      const int64_t hq = a.n0 / kGemmHead, hk = a.n1 / kGemmHead;
      u32x4 oa, ob;
      if (tn < hq + hk) {
        const u32x4 cs = in0[n], sn = in1[n];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          // x*cos + rotate_half(x)*sin, products and sum rounded to bf16
          const float xa0 = lo_f(w[p]), xa1 = hi_f(w[p]);
          const float xb0 = lo_f(w2[p]), xb1 = hi_f(w2[p]);
          const float c0f = lo_f(cs[p]), c1f = hi_f(cs[p]);
          const float s0f = lo_f(sn[p]), s1f = hi_f(sn[p]);
          oa[p] = pack_bf16x2(round_bf16(xa0 * c0f) + round_bf16(-xb0 * s0f),
                              round_bf16(xa1 * c1f) + round_bf16(-xb1 * s1f));
          ob[p] = pack_bf16x2(round_bf16(xb0 * c0f) + round_bf16(xa0 * s0f),
                              round_bf16(xb1 * c1f) + round_bf16(xa1 * s1f));
        }
      } else {
        oa = u32x4{w[0], w[1], w[2], w[3]};
        ob = u32x4{w2[0], w2[1], w2[2], w2[3]};
      }
      uint16_t *dst;
      if (tn < hq) {
        dst = a.y + row * a.ldy + static_cast<int64_t>(tn) * kGemmHead;
      } else if (tn < hq + hk) {
        dst = a.k_out + (tn - hq) * a.kv_head_stride + (a.slot0 + row) * kGemmHead;
      } else {
        dst = a.v_out + (tn - hq - hk) * a.kv_head_stride + (a.slot0 + row) * kGemmHead;
      }
      *reinterpret_cast<u32x4 *>(dst + c0) = oa;
      *reinterpret_cast<u32x4 *>(dst + c0 + kGemmHalfHead) = ob;
    } else {
      const int64_t col = static_cast<int64_t>(tn) * TW + c0;
      const int64_t at = row * a.ldy + col;
      u32x4 out;
      if constexpr (EPI == kGemmStore || EPI == kGemmSwiglu) {
        out = u32x4{w[0], w[1], w[2], w[3]};
      } else {
        const u32x4 aux = in0[n];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const float v0 = lo_f(w[p]), v1 = hi_f(w[p]);
          float o0, o1;
          if constexpr (EPI == kGemmResidual) {
            o0 = lo_f(aux[p]) + v0; o1 = hi_f(aux[p]) + v1;
          } else if constexpr (EPI == kGemmSilu) {
            o0 = gemm_silu(v0); o1 = gemm_silu(v1);
          } else {  // kGemmMul
            o0 = lo_f(aux[p]) * v0; o1 = hi_f(aux[p]) * v1;
          }
          out[p] = pack_bf16x2(o0, o1);
        }
      }
      if (col + 8 <= ncols) {
        *reinterpret_cast<u32x4 *>(a.y + at) = out;
      } else if (col < ncols) {  // N tail: element stores (aux read element-wise)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if (col + e >= ncols) break;
          const uint32_t pr = w[e >> 1];
          const float v = (e & 1) ? hi_f(pr) : lo_f(pr);
          float o = v;
          if constexpr (EPI == kGemmResidual) o = bf16_to_f32(a.aux[at + e]) + v;
          else if constexpr (EPI == kGemmSilu) o = gemm_silu(v);
          else if constexpr (EPI == kGemmMul) o = bf16_to_f32(a.aux[at + e]) * v;
          a.y[at + e] = f32_to_bf16(o);
        }
      }
    }
  }
}

// Slab geometry (see the staging and layout notes at the top).
template <int BK>
struct DmaSlab {
  static constexpr int CH = BK / 8;         // 16-byte chunks per row
  static constexpr int ROWB = 2 * BK;       // bytes per row
  static constexpr int RPB = 256 / ROWB;    // rows per 256-byte bank cycle
  static constexpr int RPI = 1024 / ROWB;   // rows per load instruction
  static_assert(BK == 32 || BK == 64, "slab depth");
};

// Ring geometry of a tile shape: bf16 elements of one slab buffer (X rows,
// then W rows), and of the LDS a workgroup needs (the ring, or the staged
// output tile of the vectorised epilogue, which reuses it).
template <class T, int STAGES, int BK = kTileK>
struct GemmRing {
  static constexpr int XB = T::BM * BK;
  static constexpr int WB = T::BN * BK;
  static constexpr int SLAB = XB + WB;
  static constexpr int STAGE = T::NSUB * kTileN * T::STAGE_COL;
  static constexpr int LDS = STAGES * SLAB > STAGE ? STAGES * SLAB : STAGE;
};

// Output tile (tm, tn) of shape T: rows tm * BM .., 128-column sub-tiles
// tn * NSUB .. (q|k|v: head tn; SwiGLU: gate / up rows 64 per sub-tile).
// sb0 holds the ring.
template <int EPI, class T, int STAGES, int BK = kTileK>
__device__ __forceinline__ void gemm_tile_run(const GemmArgs &a, int tm, int tn,
                                              uint16_t *sb0) {
  static_assert(STAGES >= 3, "a ring of at least 3 slab buffers");
  static_assert(T::NSUB == 1 || EPI != kGemmQkvRope, "q|k|v: one head per tile");
  using L = DmaSlab<BK>;
  using R = GemmRing<T, STAGES, BK>;
  constexpr int XI = T::BM * L::ROWB / 1024;  // load instructions per X slab
  constexpr int WI = T::BN * L::ROWB / 1024;
  constexpr int XW = XI / T::WAVES, WW = WI / T::WAVES;  // per wave
  static_assert(XI % T::WAVES == 0 && WI % T::WAVES == 0, "whole loads per wave");
  constexpr int XB = R::XB, kSlab = R::SLAB;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int sub = wave / T::SUBWAVES;  // sub-tile of the wave
  const int sw = wave % T::SUBWAVES;
  const int wm = sw / T::WN;
  const int wn = sw % T::WN;
  const int lr = lane & 15;
  const int g4 = lane >> 4;
  const int64_t k_bytes = a.k * 2;

  // operands as buffer resources; W instruction i reads matrix wsel(i)
  const uint16_t *wbase0, *wbase1;
  int64_t wrows0, wrows1, wrow0, wrow1;  // rows of each matrix, first tile row in it
  if constexpr (EPI == kGemmSwiglu) {
    wbase0 = a.w0; wrows0 = a.n0; wrow0 = static_cast<int64_t>(tn) * T::NSUB * kGemmHalfHead;
    wbase1 = a.w1; wrows1 = a.n0; wrow1 = wrow0;
  } else if constexpr (EPI == kGemmQkvRope) {
    const int64_t hq = a.n0 / kGemmHead, hk = a.n1 / kGemmHead;
    if (tn < hq) {
      wbase0 = a.w0; wrows0 = a.n0; wrow0 = static_cast<int64_t>(tn) * kGemmHead;
    } else if (tn < hq + hk) {
      wbase0 = a.w1; wrows0 = a.n1; wrow0 = (tn - hq) * kGemmHead;
    } else {
      wbase0 = a.w2; wrows0 = a.n2; wrow0 = (tn - hq - hk) * kGemmHead;
    }
    wbase1 = wbase0; wrows1 = wrows0; wrow1 = wrow0;
  } else {
    wbase0 = a.w0; wrows0 = a.n0; wrow0 = static_cast<int64_t>(tn) * T::BN;
    wbase1 = wbase0; wrows1 = wrows0; wrow1 = wrow0;
  }
  const u32x4 xw = buffer_rsrc_words(a.x, a.m * k_bytes);
  const u32x4 ww0 = buffer_rsrc_words(wbase0, wrows0 * k_bytes);
  const u32x4 ww1 = buffer_rsrc_words(wbase1, wrows1 * k_bytes);

  // lane part of a load: row L / CH of the instruction's RPI rows, physical
  // chunk L % CH, i.e. logical chunk (L % CH) ^ f(row); f depends on the
  // instruction only through its parity (BK = 64)
  const int ld_r = lane / L::CH;
  auto ld_off = [&](int parity) {
    const int f = ((L::RPI * parity + ld_r) / L::RPB) % L::CH;
    return ld_r * static_cast<int>(k_bytes) + 16 * ((lane % L::CH) ^ f);
  };
  const int ld_off0 = ld_off(0), ld_off1 = ld_off(1);

  // fragment reads: rows 16 q + lr (q: fragment), chunk 4 ks + g4 at
  // physical chunk (4 ks + g4) ^ f(lr), f(lr) = (lr / RPB) % CH
  const int fl = (lr / L::RPB) % L::CH;
  const int rd_off0 = lr * L::ROWB + 16 * ((g4) ^ fl);
  const int rd_off1 = lr * L::ROWB + 16 * ((4 + g4) ^ fl);
  const int arow0 = (T::BM / T::WM) * wm;

  f32x4 acc[T::FM][T::FN];
#pragma unroll
  for (int i = 0; i < T::FM; ++i)
#pragma unroll
    for (int j = 0; j < T::FN; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const int slab0 = a.split_slabs ? static_cast<int>(blockIdx.y) * a.split_slabs : 0;
  const int slabs = a.split_slabs ? min(a.split_slabs, static_cast<int>(a.k / BK) - slab0)
                                  : static_cast<int>(a.k / BK);
  // LDS byte address of sb0 (the ring's buffer b starts kSlab * 2 b bytes
  // later)
  const uint32_t ring_lds = lds_address(sb0);
  // The whole byte offset goes in voffset: the buffer range check covers
  // voffset (not soffset), so rows past the end read as zeros instead of
  // leaving the allocation.  Offsets stay below 2^31 (checked on the host).
  // Load instruction h (0 .. XW + WW - 1) of this wave for slab `slab`
  // into ring buffer `buf`: X rows first, then W rows.
  auto ring_load_one = [&](int slab, int buf, int h) __attribute__((always_inline)) {
    const uint32_t dx = ring_lds + static_cast<uint32_t>(buf * kSlab * 2);
    const uint32_t dw = dx + XB * 2;
    const int kb = (slab0 + slab) * BK * 2;
    if (h < XW) {
      const int i = wave * XW + h;
      const int64_t row = static_cast<int64_t>(tm) * T::BM + L::RPI * i;
      dma_lds16(xw, ((i & 1) ? ld_off1 : ld_off0) + static_cast<int>(row * k_bytes) + kb,
                dx + i * 1024);
    } else {
      const int i = wave * WW + (h - XW);
      const int trow = L::RPI * i;  // tile row of the instruction
      // SwiGLU: sub-tile trow / 128 holds 64 gate rows, then their 64 up rows
      const int tt = trow % kTileN;
      const bool second = EPI == kGemmSwiglu && tt >= kGemmHalfHead;
      const int64_t row =
          EPI == kGemmSwiglu
              ? (second ? wrow1 : wrow0) + (trow / kTileN) * kGemmHalfHead + tt % kGemmHalfHead
              : wrow0 + trow;
      dma_lds16(second ? ww1 : ww0,
                ((i & 1) ? ld_off1 : ld_off0) + static_cast<int>(row * k_bytes) + kb,
                dw + i * 1024);
    }
  };
  auto ring_load = [&](int slab, int buf) {
#pragma unroll
    for (int h = 0; h < XW + WW; ++h) ring_load_one(slab, buf, h);
  };
  // Slab j lives in ring buffer j % STAGES.  Step s (one per slab):
  //   wait for this wave's loads of slab s + 1 (the loads of the
  //   STAGES - 2 slabs after it may stay in flight) and for its LDS reads
  //   of slab s (lgkmcnt 0); one barrier publishes slab s + 1 and frees
  //   slab s's buffer;
  //   slab s + STAGES goes out into that buffer, one load instruction at
  //   the head of each of the step's D chunks;
  //   slab s + 1's fragments are read into registers while slab s's
  //   MFMAs, whose fragments were read one step earlier, run: the MFMA
  //   queue never waits on an LDS read.
  // Steps past the end reload the last slab and read fragments that are
  // never used, so every step issues the same loads and a constant vmcnt
  // covers every wait.
  constexpr int D = XW + WW;
  constexpr int kAhead = (STAGES - 2) * D;
  constexpr int kAheadFirst = (STAGES - 1) * D;
  static_assert(kAheadFirst < 64, "vmcnt holds 6 bits");
  constexpr int kWaitStep = waitcnt_imm(kAhead, 0);
  constexpr int kWaitFirst = waitcnt_imm(kAheadFirst, 0);
  constexpr int kWaitAll = waitcnt_imm(0, 0);
  constexpr int KS = BK / 32;
  constexpr int kReads = KS * (T::FM + T::FN);
  constexpr int kMfmas = KS * T::FM * T::FN;
  // MFMAs issued right after the step barrier (at most 4, leaving one MFMA
  // for every fragment read in the chunks after them)
  constexpr int kLead = kMfmas - kReads < 4 ? kMfmas - kReads : 4;
  constexpr int kRest = kMfmas - kLead;
  // every chunk holds at least as many MFMAs as fragment reads
  static_assert(kRest >= kReads && kRest / D >= (kReads + D - 1) / D,
                "one MFMA ahead of every fragment read in each chunk");
  using FragA = u32x4[KS][T::FM];
  using FragB = u32x4[KS][T::FN];
  // Fragment read r (0 .. kReads - 1) of slab buffer `buf`: for each
  // 32-deep half ks of the slab, the FM A fragments, then the FN B ones.
  auto read_frag = [&](int buf, int r, FragA &fa, FragB &fb) __attribute__((always_inline)) {
    const char *ax = reinterpret_cast<const char *>(sb0 + buf * kSlab) + arow0 * L::ROWB;
    const char *aw = reinterpret_cast<const char *>(sb0 + buf * kSlab + XB);
    const int ks = r / (T::FM + T::FN), q = r % (T::FM + T::FN);
    const int off = ks ? rd_off1 : rd_off0;
    if (q < T::FM) {
      fa[ks][q] = *reinterpret_cast<const u32x4 *>(ax + off + 16 * q * L::ROWB);
    } else {
      const int j = q - T::FM;
      fb[ks][j] = *reinterpret_cast<const u32x4 *>(
          aw + off + (kTileN * sub + gemm_col<T>(wn, j, lr) - lr) * L::ROWB);
    }
  };
  // publish: every LDS read issued so far stays above the wait (the empty
  // asm pins memory accesses in program order)
  auto publish_step = [&]() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(kWaitStep);
    __builtin_amdgcn_s_barrier();
  };
  int cur = 0;  // buffer of slab s
  auto step = [&](int s, const FragA &fa, const FragB &fb, FragA &na, FragB &nb) {
    const int nxt = cur + 1 == STAGES ? 0 : cur + 1;
    publish_step();
    // the first kLead MFMAs of slab s go out right after the barrier, so
    // the matrix core restarts at once
#pragma unroll
    for (int idx = 0; idx < kLead; ++idx) {
      const int ks = idx / (T::FM * T::FN), i = (idx / T::FN) % T::FM, j = idx % T::FN;
      acc[i][j] = mfma_16x16x32_bf16(fa[ks][i], fb[ks][j], acc[i][j]);
    }
    __builtin_amdgcn_sched_barrier(0);
    // the rest of the step in D chunks, each opening with one load
    // instruction of slab s + STAGES, then its share of slab s's MFMAs
    // interleaved with its share of slab s + 1's fragment reads
    const int slab_next = min(s + STAGES, slabs - 1);
#pragma unroll
    for (int c = 0; c < D; ++c) {
      const int m0 = kLead + c * kRest / D, m1 = kLead + (c + 1) * kRest / D;
      const int r0 = c * kReads / D, r1 = (c + 1) * kReads / D;
      ring_load_one(slab_next, cur, c);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int idx = m0; idx < m1; ++idx) {
        const int ks = idx / (T::FM * T::FN), i = (idx / T::FN) % T::FM, j = idx % T::FN;
        acc[i][j] = mfma_16x16x32_bf16(fa[ks][i], fb[ks][j], acc[i][j]);
      }
#pragma unroll
      for (int r = r0; r < r1; ++r) read_frag(nxt, r, na, nb);
      // MFMA, read, MFMA, read, ..., then the chunk's remaining MFMAs
#pragma unroll
      for (int r = r0; r < r1; ++r) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
#pragma unroll
      for (int k = 0; k < (m1 - m0) - (r1 - r0); ++k)
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    cur = nxt;
  };
#pragma unroll
  for (int p = 0; p < STAGES; ++p) ring_load(min(p, slabs - 1), p);
  FragA fa0, fa1;
  FragB fb0, fb1;
  __builtin_amdgcn_s_waitcnt(kWaitFirst);
  __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int r = 0; r < kReads; ++r) read_frag(0, r, fa0, fb0);
  int s = 0;
  for (; s + 2 <= slabs; s += 2) {
    step(s, fa0, fb0, fa1, fb1);
    step(s + 1, fa1, fb1, fa0, fb0);
  }
  if (s < slabs) step(s, fa0, fb0, fa1, fb1);
  // every load landed and every LDS read done before the ring is reused
  // for the staged tile (or the workgroup leaves)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(kWaitAll);
  if (EPI != kGemmF32 && a.vec_out) {
    __builtin_amdgcn_s_barrier();  // every wave's loads landed, ring read
    gemm_epilogue_staged<EPI, T>(a, tm, tn * T::NSUB + sub, wm, wn, lane, sw, acc,
                                 sb0 + sub * (kTileN * T::STAGE_COL));
  } else {
    gemm_epilogue<EPI, T>(a, tm, tn * T::NSUB + sub, wm, wn, lane, acc);
  }
}

// One launch covers the output with tiles of shape T and, when the last
// round of T tiles would leave at least half of the CUs idle, the last
// tail_n tile columns with tiles of half the height (TH, the same wave
// count): those columns then take one round of half tiles instead of a
// partial round of full ones (M = 2048, N = 14336: 768 full tiles in 3
// rounds of 256, then 256 half tiles, instead of 3.5 rounds of full tiles).
// Workgroup b runs on XCD b % 8 (see "Tile order"); each XCD takes a
// contiguous range of full tiles first, then of half tiles, so the half
// tiles are dispatched last on every XCD.
template <int EPI, class T, int STAGES, class TH, int STAGES_H, int BK>
__global__ __launch_bounds__(T::WAVES *kWave) void gemm_kernel(GemmArgs a) {
  static_assert(TH::WAVES == T::WAVES, "one workgroup size");
  constexpr int kLds = GemmRing<T, STAGES, BK>::LDS > GemmRing<TH, STAGES_H, BK>::LDS
                           ? GemmRing<T, STAGES, BK>::LDS
                           : GemmRing<TH, STAGES_H, BK>::LDS;
  static_assert(kLds * 2 <= 160 * 1024, "LDS of one CU");
  __shared__ __attribute__((aligned(16))) uint16_t sb0[kLds];
  if constexpr (EPI == kGemmF32) {
    if (a.split_slabs) a.yf += static_cast<int64_t>(blockIdx.y) * a.split_stride;
  }
  const int xcd = static_cast<int>(blockIdx.x % kXcds);
  const int j = static_cast<int>(blockIdx.x / kXcds);
  int tm, tn;
  // padding workgroups leave as a whole: no barrier is skipped
  if (j < a.per_xcd) {
    if (!gemm_tile(xcd * a.per_xcd + j, a.tiles, a.tiles_m, a.tiles_n, tm, tn)) return;
    gemm_tile_run<EPI, T, STAGES, BK>(a, tm, tn, sb0);
    return;
  }
  if constexpr (!std::is_same<T, TH>::value) {
    if (!gemm_tile(xcd * a.hper_xcd + (j - a.per_xcd), a.htiles, a.htiles_m, a.htiles_n,
                   tm, tn))
      return;
    gemm_tile_run<EPI, TH, STAGES_H, BK>(a, tm, a.tiles_n + tn, sb0);
  }
}

// CUs of the device a stream runs on (cached per device; 256 on MI355X).
static int gemm_device_cus(hipStream_t s) {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cached[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (s != nullptr) {
    hipDevice_t owner = 0;
    if (hipStreamGetDevice(s, &owner) != hipSuccess) return 256;
    dev = static_cast<int>(owner);
  }
  if (dev < 0 || dev >= kMaxDevices) return 256;
  int cus = cached[dev].load(std::memory_order_relaxed);
  if (cus == 0) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cached[dev].store(cus, std::memory_order_relaxed);
  }
  return cus;
}

template <int EPI, int BK, class T, int STAGES, class TH = T, int STAGES_H = STAGES>
static hipError_t launch_tiles(GemmArgs &a, int64_t tiles_n, int cus, hipStream_t s,
                               int splits = 1) {
  const int64_t tiles_m = (a.m + T::BM - 1) / T::BM;
  const int64_t htiles_m = (a.m + TH::BM - 1) / TH::BM;
  int64_t tail_n = 0;
  if (!std::is_same<T, TH>::value) {
    const int64_t tiles = tiles_m * tiles_n;
    const int64_t rem = tiles % cus;
    if (tiles > cus && rem > 0 && 2 * rem <= cus) {
      const int64_t cols = (rem + tiles_m - 1) / tiles_m;
      if (cols < tiles_n && cols * htiles_m <= cus) tail_n = cols;
    }
  }
  const int64_t tiles = tiles_m * (tiles_n - tail_n);
  const int64_t htiles = htiles_m * tail_n;
  if (tiles + htiles > (int64_t{1} << 30)) return static_cast<hipError_t>(CASCADE_ESHAPE);
  a.tiles_m = static_cast<int32_t>(tiles_m);
  a.tiles_n = static_cast<int32_t>(tiles_n - tail_n);
  a.tiles = static_cast<int32_t>(tiles);
  a.per_xcd = static_cast<int32_t>((tiles + kXcds - 1) / kXcds);
  a.htiles_m = static_cast<int32_t>(htiles_m);
  a.htiles_n = static_cast<int32_t>(tail_n);
  a.htiles = static_cast<int32_t>(htiles);
  a.hper_xcd = static_cast<int32_t>((htiles + kXcds - 1) / kXcds);
  // 16-byte output accesses need 16-byte aligned rows in every buffer the
  // epilogue touches; otherwise the element-wise epilogue runs
  auto ok16 = [](const void *p) { return p == nullptr || aligned16(p); };
  a.vec_out = (a.ldy % 8 == 0) && ok16(a.y) && ok16(a.aux) && ok16(a.rope_cos) &&
              ok16(a.rope_sin) && ok16(a.k_out) && ok16(a.v_out) &&
              (a.kv_head_stride % 8 == 0);
  const int64_t grid = static_cast<int64_t>(kXcds) * (a.per_xcd + a.hper_xcd);
  return launch_kernel(gemm_kernel<EPI, T, STAGES, TH, STAGES_H, BK>,
                       dim3(static_cast<unsigned>(grid), static_cast<unsigned>(splits)),
                       dim3(T::WAVES * kWave), 0, s, a);
}

// Short prompts (M <= 64 rows, or up to 256 over few columns).  The weights are nearly all the traffic, so
// they must stream at HBM rate, which needs long runs of one row per load
// (64-byte pieces of 16 rows per instruction, the layout of an MFMA operand,
// stream at only 2-3 TB/s).  A workgroup computes one pair of 16-column
// fragments of a 128-column tile (the columns of wave column wn of a
// GemmTile<MR, 1, 4>, so the epilogues' pairing of column c with c + 64
// holds), or for the element-wise epilogues one fragment of it where the
// pairs would leave CUs idle (NF = 1: M = 16, o_proj 17.2 -> 12.2 us,
// down_proj 36.3 -> 28.5 us), for a block of MR rows (grid.y: the row block; M > 64 runs
// blocks of 64 rows side by side, each reading the column pair's W
// again, from the XCD's L2 when the blocks share an XCD).  K is walked in slabs through a ring of LDS
// buffers: every load instruction moves 1 KiB, one or two whole row runs
// of a slab (the 32 W rows and the MR X rows; rows past M or past a matrix
// read as zeros through the buffer bounds, and K past a short last slab
// is never used), each instruction's kilobyte lands after 16 bytes of
// padding so the fragment reads of 16 rows spread over the banks, and each
// wave runs the MFMAs of its quarter of a slab's K.  The waves' fp32 partials are summed through LDS in wave
// order and wave 0 runs the element-wise epilogue.
template <int MR, int NF = 2>
struct SkinnyShape {
  using T = GemmTile<MR, 1, 4>;  // one 16 x 32 column pair of MR rows per workgroup
  static_assert(NF == 1 || NF == 2, "a column pair or one fragment of it");
  static constexpr int SLAB_K = MR == 16 ? 512 : 256;
  static constexpr int RUN = SLAB_K * 2;          // bytes of one row in a slab
  static constexpr int RPI = 1024 / RUN;          // rows per load instruction (1 KiB)
  static constexpr int LINE = 1024 + 16;          // LDS pitch of one instruction's rows
  static constexpr int WROWS = 16 * NF;           // W rows of the fragment(s)
  static constexpr int SLAB_ROWS = WROWS + MR;    // W rows, then X rows
  static constexpr int STAGES = 3;
  static constexpr int WAVES = 4;
  static constexpr int LOADS = SLAB_ROWS / RPI / WAVES;  // per wave and slab
  static_assert(SLAB_ROWS % (RPI * WAVES) == 0, "whole instructions per wave");
  static_assert(16 % RPI == 0, "an instruction's rows stay in one operand");
};
// Prompt rows the skinny kernels cover.  A 128-row shape (128-deep slabs,
// 256-byte runs) measured slower than 64-row tiles at M = 128 (the layer
// of seven projections 0.460 against 0.311 ms).
constexpr int kSkinnyRows = 64;

// Slab row r (W rows of fragments 0 and 1, then X rows) sits at LDS byte
// (r / RPI) * LINE + (r % RPI) * RUN of its buffer.  With 512-byte runs two
// rows share one 1 KiB line, so a fragment read (16 rows) meets each bank
// group twice; with 1 KiB runs, once.
template <int EPI, int MR, int NF = 2>
__global__ __launch_bounds__(SkinnyShape<MR>::WAVES *kWave) void gemm_skinny_kernel(GemmArgs a) {
  using S = SkinnyShape<MR, NF>;
  using T = typename S::T;
  static_assert(S::WAVES == SkinnyShape<MR>::WAVES, "one workgroup size");
  static_assert(NF == 2 || (EPI != kGemmQkvRope && EPI != kGemmSwiglu),
                "RoPE and SwiGLU pair fragment j with j + 1");
  constexpr int kSlabBytes = S::SLAB_ROWS / S::RPI * S::LINE;
  __shared__ __attribute__((aligned(16))) unsigned char ring[S::STAGES * kSlabBytes];
  static_assert(S::WAVES * T::FM * NF * kWave * sizeof(f32x4) <= sizeof(ring),
                "the reduction fits in the ring");
  // NF = 2: workgroup x holds the fragment pair of wave column x % 4 of
  // tile x / 4; NF = 1: fragment (x / 4) % 2 of wave column x % 4 of tile
  // x / 8 (twice the workgroups for the same columns)
  constexpr int kPerTile = T::WN * (2 / NF);
  const int tn = static_cast<int>(blockIdx.x) / kPerTile;
  const int wn = static_cast<int>(blockIdx.x) % T::WN;
  const int jsel = NF == 2 ? 0 : (static_cast<int>(blockIdx.x) % kPerTile) / T::WN;
  const int rb = static_cast<int>(blockIdx.y);  // block of MR rows of X
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lr = lane & 15;
  const int g4 = lane >> 4;
  const int64_t row_bytes = a.k * 2;

  // the matrix, and the row in it, of W slab row r (r < 32: fragment r / 16,
  // tile column gemm_col(wn, r / 16, r % 16)); rows past a matrix read as
  // zeros through its buffer bounds
  auto w_row = [&](int r, const uint16_t *&base, int64_t &rows) -> int64_t {
    const int j = NF == 2 ? r / 16 : jsel;
    const int tc = gemm_col<T>(wn, j, r % 16);
    if constexpr (EPI == kGemmSwiglu) {
      base = tc < kGemmHalfHead ? a.w0 : a.w1;
      rows = a.n0;
      return static_cast<int64_t>(tn) * kGemmHalfHead + (tc % kGemmHalfHead);
    } else if constexpr (EPI == kGemmQkvRope) {
      const int64_t hq = a.n0 / kGemmHead, hk = a.n1 / kGemmHead;
      if (tn < hq) {
        base = a.w0; rows = a.n0; return static_cast<int64_t>(tn) * kGemmHead + tc;
      }
      if (tn < hq + hk) {
        base = a.w1; rows = a.n1; return (tn - hq) * kGemmHead + tc;
      }
      base = a.w2; rows = a.n2; return (tn - hq - hk) * kGemmHead + tc;
    } else {
      base = a.w0; rows = a.n0; return static_cast<int64_t>(tn) * kTileN + tc;
    }
  };
  // this wave's load instructions: a buffer over the operand's matrix and
  // the lane's byte offset of slab 0 (its row of the instruction, then
  // 16 bytes a lane along that row)
  constexpr int kLanesPerRow = kWave / S::RPI;
  u32x4 rsrc[S::LOADS];
  int voff[S::LOADS];
#pragma unroll
  for (int t = 0; t < S::LOADS; ++t) {
    const int r0 = (wave * S::LOADS + t) * S::RPI;
    const uint16_t *base;
    int64_t rows, row;
    if (r0 < S::WROWS) {
      row = w_row(r0, base, rows);
    } else {
      base = a.x; rows = a.m; row = static_cast<int64_t>(rb) * MR + r0 - S::WROWS;
    }
    rsrc[t] = buffer_rsrc_words(base, rows * row_bytes);
    voff[t] = static_cast<int>((row + lane / kLanesPerRow) * row_bytes) +
              16 * (lane % kLanesPerRow);
  }
  const uint32_t ring_lds = lds_address(ring);
  const int slabs = static_cast<int>((a.k + S::SLAB_K - 1) / S::SLAB_K);
  auto load_slab = [&](int slab, int buf) {
    const uint32_t dst = ring_lds + static_cast<uint32_t>(buf * kSlabBytes);
#pragma unroll
    for (int t = 0; t < S::LOADS; ++t)
      dma_lds16(rsrc[t], voff[t] + slab * S::RUN, dst + (wave * S::LOADS + t) * S::LINE);
  };

  // fragment reads: lane (lr, g4) of 32-deep chunk q reads row lr of the
  // operand's 16-row group, bytes 64 q + 16 g4 of its run
  auto row_at = [&](int r) { return (r / S::RPI) * S::LINE + (r % S::RPI) * S::RUN; };
  f32x4 acc[T::FM][NF];
#pragma unroll
  for (int i = 0; i < T::FM; ++i)
#pragma unroll
    for (int j = 0; j < NF; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  constexpr int kChunks = S::SLAB_K / 32 / S::WAVES;  // per wave and slab
  auto compute = [&](int slab, int buf) {
    const unsigned char *b0 = ring + buf * kSlabBytes + 16 * g4;
    const int valid = static_cast<int>(
        min<int64_t>(S::SLAB_K, a.k - static_cast<int64_t>(slab) * S::SLAB_K) / 32);
#pragma unroll
    for (int q = 0; q < kChunks; ++q) {
      const int chunk = wave * kChunks + q;
      if (chunk >= valid) break;  // wave-uniform: the last slab of a short K
      u32x4 xa[T::FM], wb[NF];
#pragma unroll
      for (int i = 0; i < T::FM; ++i)
        xa[i] = *reinterpret_cast<const u32x4 *>(b0 + row_at(S::WROWS + 16 * i + lr) +
                                                 64 * chunk);
#pragma unroll
      for (int j = 0; j < NF; ++j)
        wb[j] = *reinterpret_cast<const u32x4 *>(b0 + row_at(16 * j + lr) + 64 * chunk);
#pragma unroll
      for (int i = 0; i < T::FM; ++i)
#pragma unroll
        for (int j = 0; j < NF; ++j) acc[i][j] = mfma_16x16x32_bf16(xa[i], wb[j], acc[i][j]);
    }
  };
  // slab s in buffer s % STAGES; step s waits for this wave's loads of
  // slab s (the later slabs' loads may stay in flight), one barrier
  // publishes it and frees slab s - 1's buffer, which takes slab
  // s + STAGES - 1 (past the end: the last slab again, never read)
  constexpr int kWaitStep = waitcnt_imm((S::STAGES - 2) * S::LOADS, 0);
#pragma unroll
  for (int p = 0; p < S::STAGES - 1; ++p) load_slab(min(p, slabs - 1), p);
  int buf = 0;
  for (int slab = 0; slab < slabs; ++slab) {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(kWaitStep);
    __builtin_amdgcn_s_barrier();
    const int refill = buf == 0 ? S::STAGES - 1 : buf - 1;
    load_slab(min(slab + S::STAGES - 1, slabs - 1), refill);
    compute(slab, buf);
    buf = buf + 1 == S::STAGES ? 0 : buf + 1;
  }
  // every load landed and every LDS read done before the ring holds the
  // partials
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
  __syncthreads();
  f32x4(*partial)[T::FM * NF][kWave] =
      reinterpret_cast<f32x4(*)[T::FM * NF][kWave]>(ring);
#pragma unroll
  for (int i = 0; i < T::FM; ++i)
#pragma unroll
    for (int j = 0; j < NF; ++j) partial[wave][i * NF + j][lane] = acc[i][j];
  __syncthreads();
  if (wave != 0) return;
  // the wave partials in wave order, into the pair's fragment slots
  f32x4 out[T::FM][T::FN];
#pragma unroll
  for (int i = 0; i < T::FM; ++i)
#pragma unroll
    for (int j = 0; j < T::FN; ++j) out[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < T::FM; ++i)
#pragma unroll
    for (int j = 0; j < NF; ++j) {
      f32x4 sum = partial[0][i * NF + j][lane];
      for (int w = 1; w < S::WAVES; ++w) sum += partial[w][i * NF + j][lane];
      if (NF == 2) {
        out[i][j] = sum;
      } else {  // no register array indexed at run time
        out[i][0] = jsel == 0 ? sum : out[i][0];
        out[i][1] = jsel == 1 ? sum : out[i][1];
      }
    }
  gemm_epilogue<EPI, T>(a, rb, tn, 0, wn, lane, out, NF == 2 ? -1 : jsel);
}

template <int EPI>
static hipError_t launch_skinny(GemmArgs &a, int64_t tiles_n, hipStream_t s) {
  const int64_t pairs = tiles_n * 4;  // one workgroup per column pair
  if (pairs > (int64_t{1} << 29)) return static_cast<hipError_t>(CASCADE_ESHAPE);
  const unsigned blocks = a.m <= 16 ? 1u : static_cast<unsigned>((a.m + 63) / 64);
  // where the column pairs would leave CUs idle (o_proj / down_proj,
  // N = 4096: 128 pairs), the element-wise epilogues split each pair over
  // two workgroups, one fragment each; RoPE and SwiGLU keep their pairs
  constexpr bool kSplittable = EPI != kGemmQkvRope && EPI != kGemmSwiglu;
  const bool split = kSplittable && 2 * pairs * blocks <= gemm_device_cus(s);
  const unsigned grid = static_cast<unsigned>(split ? 2 * pairs : pairs);
  if constexpr (kSplittable) {
    if (split) {
      if (a.m <= 16)
        return launch_kernel(gemm_skinny_kernel<EPI, 16, 1>, dim3(grid),
                             dim3(SkinnyShape<16, 1>::WAVES * kWave), 0, s, a);
      return launch_kernel(gemm_skinny_kernel<EPI, 64, 1>, dim3(grid, blocks),
                           dim3(SkinnyShape<64, 1>::WAVES * kWave), 0, s, a);
    }
  }
  if (a.m <= 16)
    return launch_kernel(gemm_skinny_kernel<EPI, 16>, dim3(grid),
                         dim3(SkinnyShape<16>::WAVES * kWave), 0, s, a);
  // blocks of 64 rows side by side (grid.y); with an even pair count the
  // blocks of one column pair run on one XCD (linear index mod 8) and share
  // its W slabs through that XCD's L2
  return launch_kernel(gemm_skinny_kernel<EPI, 64>, dim3(grid, blocks),
                       dim3(SkinnyShape<64>::WAVES * kWave), 0, s, a);
}

// Schedule of launch_tiles in rounds: whole rounds of full tiles, then a
// round of half-height tiles (tail 1), a partial round of full tiles
// (tail 2) or nothing (tail 0).
struct TileRounds {
  int64_t full;
  int tail;
};
static TileRounds tile_rounds(int64_t tiles_m, int64_t tiles_n, int64_t htiles_m, int cus) {
  const int64_t tiles = tiles_m * tiles_n;
  const int64_t rem = tiles % cus;
  if (rem == 0) return {tiles / cus, 0};
  if (tiles > cus && 2 * rem <= cus) {
    const int64_t cols = (rem + tiles_m - 1) / tiles_m;
    if (cols < tiles_n && cols * htiles_m <= cus) return {tiles / cus, 1};
  }
  return {tiles / cus, 2};
}

// At most 64 rows of X, or at most 256 over few columns: the skinny
// kernels.  Else 256-row tiles when there are at least as many as CUs: 256
// columns wide where their schedule is shorter (below), else 128 wide (a
// partial last round runs as 128-row half tiles); else 128-row tiles (a
// partial last round as 64-row half tiles),
// unless there are fewer of those than CUs and 64-row tiles need no more
// than twice their rounds: then 64-row tiles (the K / V projections,
// N = 1024, at M = 2048, and short prompts).
template <int EPI>
static hipError_t launch_gemm(GemmArgs &a, int64_t tiles_n, hipStream_t s) {
  if (a.m <= kSkinnyRows) return launch_skinny<EPI>(a, tiles_n, s);
  const int cus = gemm_device_cus(s);
  // up to 256 rows over few columns: blocks of 64 rows through the skinny
  // kernel while that stays within one workgroup per CU (M = 128: q / o /
  // down_proj 30 -> 21, 32 -> 22, 103 -> 56 us; k / v up to M = 256 29 ->
  // 18 us); past that, tiles (M = 192, q_proj: 35 us skinny, 30 tiled).
  // Not for q|k|v, so that its per-matrix launches (matrix granularity)
  // sum in the same order as the fused one and match it bit for bit.
  if (EPI != kGemmQkvRope && a.m <= 4 * kSkinnyRows &&
      (a.m + kSkinnyRows - 1) / kSkinnyRows * tiles_n * 4 <= cus)
    return launch_skinny<EPI>(a, tiles_n, s);
  const int64_t tiles256 = (a.m + 255) / 256 * tiles_n;
  if (a.m > 128 && tiles256 >= cus) {
    // 256 x 256 tiles read a quarter less X and W per MFMA but need 32-deep
    // slabs (a ring of four 32 KiB slabs; 64-deep ones would not fit three
    // in the LDS), so twice the step barriers.  The schedule of rounds
    // decides, with round costs measured at M = 2048, K = 4096 (in rounds
    // of 256 x 128 tiles, about 58 us each): a round of 256 x 256 tiles
    // 1.98 (N = 16384: 230 us for 2 rounds against 244 us for 4), a round of
    // their 128 x 256 half-height tail tiles 1.2, a round of 128 x 128 tail
    // tiles 0.7.  So the fused gate|up (N = 2 x 14336) runs 7 rounds of
    // 256 x 128 tiles (405.8 us) rather than 3 rounds + a half-height round
    // of 256 x 256 (414.5 us), and the resident LM head (N = 128256) 16
    // rounds of 256 x 256 (1712 against 1784 us).  SwiGLU needs whole
    // pairs of 128-column gate / up groups; q|k|v keeps one head per tile.
    if constexpr (EPI != kGemmQkvRope) {
      const int64_t tm256 = (a.m + 255) / 256, tm128 = (a.m + 127) / 128;
      const int64_t wide_n = (tiles_n + 1) / 2;
      const TileRounds std_r = tile_rounds(tm256, tiles_n, tm128, cus);
      const TileRounds wide_r = tile_rounds(tm256, wide_n, tm128, cus);
      constexpr double kWideRound = 1.98;  // in rounds of 256 x 128 tiles
      constexpr double kWideHalfRound = 1.2;
      constexpr double kHalfRound = 0.7;
      const double std_t = static_cast<double>(std_r.full) +
                           (std_r.tail == 1 ? kHalfRound : std_r.tail == 2 ? 1.0 : 0.0);
      const double wide_t = kWideRound * static_cast<double>(wide_r.full) +
                            (wide_r.tail == 1 ? kWideHalfRound : wide_r.tail == 2 ? kWideRound : 0.0);
      if (wide_t < std_t && (EPI != kGemmSwiglu || tiles_n % 2 == 0))
        return launch_tiles<EPI, 32, GemmTileWide, 4, GemmTileWideHalf, 4>(a, wide_n, cus, s);
    }
    return launch_tiles<EPI, kTileK, GemmTile256, 3, GemmTile128x8, 4>(a, tiles_n, cus, s);
  }
  const int64_t tiles128 = (a.m + 127) / 128 * tiles_n;
  // fewer than one round of 128-row tiles still wins where it takes half
  // the rounds of 64-row tiles (M = 192 / 256, N = 14336: 61.8 -> 39.1 /
  // 62.6 -> 45.1 us)
  const int64_t rounds64 = ((a.m + 63) / 64 * tiles_n + cus - 1) / cus;
  const int64_t rounds128 = (tiles128 + cus - 1) / cus;
  if (a.m <= 64 || (tiles128 < cus && 2 * rounds128 > rounds64))
    return launch_tiles<EPI, kTileK, GemmTile64, 6>(a, tiles_n, cus, s);
  return launch_tiles<EPI, kTileK, GemmTile128, 4, GemmTile64, 6>(a, tiles_n, cus, s);
}

// Shared argument checks: X [m, k], K a multiple of the 64-deep slab.
// Byte offsets of the slab loads are 32-bit: X and every W stay below 2 GiB.
constexpr int64_t kGemmMaxBytes = int64_t{1} << 31;

static int gemm_check_x(const void *x, int64_t m, int64_t k) {
  if (x == nullptr || m <= 0 || k <= 0 || m > (int64_t{1} << 24))
    return CASCADE_EINVAL;
  if (!aligned16(x)) return CASCADE_EALIGN;
  if (k % kTileK) return CASCADE_ESHAPE;
  if (m * k * 2 >= kGemmMaxBytes) return CASCADE_ESHAPE;
  return 0;
}

static int gemm_check_w(const void *w, int64_t n, int64_t granule, int64_t k) {
  if (w == nullptr || n <= 0) return CASCADE_EINVAL;
  if (!aligned16(w)) return CASCADE_EALIGN;
  if (n % granule) return CASCADE_ESHAPE;
  if (n * k * 2 >= kGemmMaxBytes) return CASCADE_ESHAPE;
  return 0;
}

}  // namespace cascade

using namespace cascade;

// Split K.  Where 256-row tiles would keep at most half of the CUs busy
// (prompts of 17 to about 1000 rows over N = 4096: down_proj, and o_proj up
// to 128 rows; M = 256, down_proj: 102.7 -> 46.1 us, M = 1024: 136.5 ->
// 110.7 us, o_proj at M = 65: 28.5 -> 19.2 us), K is
// split over up to kSplitMax rows of workgroups (blockIdx.y), each writing
// an fp32 partial tile into the caller's workspace; a second launch sums
// the partials in split order and applies the element-wise epilogue at the
// same rounding points as the one-pass tile (bf16(sum), then the residual
// add).  The partials associate the K sum differently from one pass, so a
// result may differ from the one-pass tile in the last bf16 place, within
// the same rounding bound.
constexpr int kSplitMax = 8;
constexpr int kSplitMinSlabs = 8;  // 64-deep slabs per split, at least

struct SplitPlan {
  int splits;  // 1: no split
  int per;     // slabs per split
};

static SplitPlan split_plan(int64_t m, int64_t n, int64_t k, int cus) {
  SplitPlan p{1, 0};
  // 16 rows and fewer: one skinny block per column pair streams the weight
  // faster (M = 16, down_proj: 28.6 us one pass, 31.8 split; M = 24: 42.0
  // against 32.2, M = 64: 51.1 against 34.4)
  if (m <= 16 || n % 8 != 0 || k % kTileK != 0) return p;
  // short K past the skinny blocks: the one-pass 64-row tiles finish first
  // (o_proj, M = 192..1024: 22.0..33.8 us one pass, 23.3..42.8 split)
  if (k < 8192 && m > 2 * kSkinnyRows) return p;
  const int64_t tiles = (m + 255) / 256 * ((n + kTileN - 1) / kTileN);
  if (2 * tiles > cus) return p;
  const int64_t slabs = k / kTileK;
  const int64_t sp = std::min<int64_t>(std::min<int64_t>(kSplitMax, cus / tiles),
                                       slabs / kSplitMinSlabs);
  if (sp < 2) return p;
  const int64_t per = (slabs + sp - 1) / sp;
  p.splits = static_cast<int>((slabs + per - 1) / per);  // no empty split
  p.per = static_cast<int>(per);
  return p;
}

// y = epilogue(sum over s < splits of part[s]), 8 consecutive outputs per
// thread (n % 8 == 0, so a group never crosses a row).
template <int EPI>
__global__ __launch_bounds__(256) void gemm_split_reduce_kernel(GemmArgs a, int splits) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 8;
  if (i >= a.m * a.n0) return;
  const float *p = a.yf + i;
  f32x4 lo = *reinterpret_cast<const f32x4 *>(p);
  f32x4 hi = *reinterpret_cast<const f32x4 *>(p + 4);
  for (int sp = 1; sp < splits; ++sp) {
    p += a.split_stride;
    lo += *reinterpret_cast<const f32x4 *>(p);
    hi += *reinterpret_cast<const f32x4 *>(p + 4);
  }
  const float v[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  u32x4 aux = u32x4{0u, 0u, 0u, 0u};
  if constexpr (EPI == kGemmResidual) aux = *reinterpret_cast<const u32x4 *>(a.aux + i);
  u32x4 out;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float v0 = round_bf16(v[2 * q]), v1 = round_bf16(v[2 * q + 1]);
    if constexpr (EPI == kGemmResidual) {
      v0 = lo_f(aux[q]) + v0;
      v1 = hi_f(aux[q]) + v1;
    }
    out[q] = pack_bf16x2(v0, v1);
  }
  *reinterpret_cast<u32x4 *>(a.y + i) = out;
}

template <int EPI>
static int gemm_split_k(const GemmArgs &a, const SplitPlan &p, void *ws,
                        size_t ws_bytes, hipStream_t s) {
  static_assert(EPI == kGemmStore || EPI == kGemmResidual, "element-wise epilogues");
  const int64_t part = a.m * a.n0;
  if (ws_bytes < static_cast<size_t>(p.splits) * part * sizeof(float))
    return CASCADE_EWORKSPACE;
  GemmArgs b = a;
  b.yf = static_cast<float *>(ws);
  b.ldy = a.n0;
  b.split_slabs = p.per;
  b.split_stride = part;
  hipError_t e = launch_tiles<kGemmF32, kTileK, GemmTile256, 3>(
      b, (a.n0 + kTileN - 1) / kTileN, gemm_device_cus(s), s, p.splits);
  if (e != hipSuccess) return e;
  GemmArgs r = a;
  r.yf = static_cast<float *>(ws);
  r.split_stride = part;
  const int64_t groups = (part / 8 + 255) / 256;
  return launch_kernel(gemm_split_reduce_kernel<EPI>, dim3(static_cast<unsigned>(groups)),
                       dim3(256), 0, s, r, p.splits);
}

static int gemm_plain(int epi, const void *x, const void *w, const void *aux,
                      void *y, int64_t m, int64_t n, int64_t k, void *stream) {
  if (int e = gemm_check_x(x, m, k)) return e;
  if (int e = gemm_check_w(w, n, 1, k)) return e;
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

// The workspace forms: split K where the plan above applies (the workspace
// then needs cascade_gemm_workspace_bytes() bytes), else the one-pass GEMM.
static int gemm_ws(int epi, const void *x, const void *w, const void *aux,
                   void *y, int64_t m, int64_t n, int64_t k, void *workspace,
                   size_t workspace_bytes, void *stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  const SplitPlan p = split_plan(m, n, k, gemm_device_cus(s));
  if (p.splits == 1)
    return gemm_plain(epi, x, w, aux, y, m, n, k, stream);
  if (int e = gemm_check_x(x, m, k)) return e;
  if (int e = gemm_check_w(w, n, 1, k)) return e;
  if (y == nullptr || workspace == nullptr || (epi == kGemmResidual && aux == nullptr))
    return CASCADE_EINVAL;
  if (!aligned16(y) || !aligned16(workspace) || (aux != nullptr && !aligned16(aux)))
    return CASCADE_EALIGN;
  GemmArgs a{};
  a.x = static_cast<const uint16_t *>(x);
  a.w0 = static_cast<const uint16_t *>(w);
  a.n0 = n;
  a.m = m;
  a.k = k;
  a.y = static_cast<uint16_t *>(y);
  a.ldy = n;
  a.aux = static_cast<const uint16_t *>(aux);
  return epi == kGemmResidual
             ? gemm_split_k<kGemmResidual>(a, p, workspace, workspace_bytes, s)
             : gemm_split_k<kGemmStore>(a, p, workspace, workspace_bytes, s);
}

extern "C" size_t cascade_gemm_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0) return 0;
  const SplitPlan p = split_plan(m, n, k, gemm_device_cus(nullptr));
  return p.splits > 1 ? static_cast<size_t>(p.splits) * m * n * sizeof(float) : 0;
}

extern "C" int cascade_gemm_ws_bf16(const void *x, const void *w, void *y,
                                    int64_t m, int64_t n, int64_t k,
                                    void *workspace, size_t workspace_bytes,
                                    void *stream) {
  return gemm_ws(kGemmStore, x, w, nullptr, y, m, n, k, workspace,
                 workspace_bytes, stream);
}

extern "C" int cascade_gemm_residual_ws_bf16(const void *x, const void *w,
                                             const void *residual, void *y,
                                             int64_t m, int64_t n, int64_t k,
                                             void *workspace,
                                             size_t workspace_bytes,
                                             void *stream) {
  return gemm_ws(kGemmResidual, x, w, residual, y, m, n, k, workspace,
                 workspace_bytes, stream);
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
  if (int e = gemm_check_w(w_gate, n_half, kGemmHalfHead, k)) return e;
  if (int e = gemm_check_w(w_up, n_half, kGemmHalfHead, k)) return e;
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
  if (std::max(nq, std::max(nk, nv)) * k * 2 >= kGemmMaxBytes) return CASCADE_ESHAPE;
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
