// Device-side helpers shared by the gfx950 kernels of libcascade_hip.
//
// Conventions used throughout the library:
//   * bf16 tensors travel as raw uint16_t; arithmetic is fp32.
//   * float -> bf16 rounding is round-to-nearest-even (the hardware
//     v_cvt_pk_bf16_f32 conversion), the same rounding torch uses for
//     Tensor.to(torch.bfloat16).
//   * One wavefront is 64 lanes. A 16-byte load (u32x4) carries 8 bf16.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cascade {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// Buffer resource over [base, base + bytes) as four words (for inline asm):
// base, stride 0, num_records, raw-buffer flags.  Loads past num_records
// return zeros.
__device__ __forceinline__ u32x4 buffer_rsrc_words(const void *base, int64_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  u32x4 r;
  r.x = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p));
  r.y = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p >> 32) & 0xffffu);
  r.z = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(bytes));
  r.w = 0x00020000u;
  return r;
}

// LDS byte address of a __shared__ pointer.
__device__ __forceinline__ uint32_t lds_address(const void *p) {
  return __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
      (__attribute__((address_space(3))) const void *)p)));
}

// buffer_load_dwordx4 ... lds issued from inline asm: lane l's 16 bytes at
// voffset land at LDS byte address (lds + 16 l).  The compiler does not see
// these loads, so it adds no vmcnt waits of its own for them (the caller
// waits with an explicit s_waitcnt); the memory clobber keeps LDS accesses
// from moving across the issue.  The descriptor words pass through
// readfirstlane (a no-op on values the compiler already keeps in SGPRs):
// where it cannot prove a selected descriptor uniform it would otherwise
// hand the asm VGPRs.
__device__ __forceinline__ void dma_lds16(const u32x4 &rsrc, int voff, uint32_t lds) {
  u32x4 r;
  r.x = __builtin_amdgcn_readfirstlane(rsrc.x);
  r.y = __builtin_amdgcn_readfirstlane(rsrc.y);
  r.z = __builtin_amdgcn_readfirstlane(rsrc.z);
  r.w = __builtin_amdgcn_readfirstlane(rsrc.w);
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :: "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voff), "s"(r)
               : "memory", "m0");
}

// s_waitcnt immediate: vmcnt(vm) lgkmcnt(lgkm), expcnt left alone.
constexpr int waitcnt_imm(int vm, int lgkm) {
  return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | ((lgkm & 15) << 8);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Value of f after a round trip through bf16 (models a torch bf16 result).
__device__ __forceinline__ float round_bf16(float f) {
  return bf16_to_f32(f32_to_bf16(f));
}

__device__ __forceinline__ float lo_bf16(uint32_t pair) {
  return __uint_as_float(pair << 16);
}

__device__ __forceinline__ float hi_bf16(uint32_t pair) {
  return __uint_as_float(pair & 0xffff0000u);
}

// Reinterprets one packed dword as two bf16.  The dword is taken by value:
// hipcc (ROCm 7.2) miscompiles __builtin_bit_cast applied directly to an
// ext_vector element expression such as v.y (it reads element 0 instead).
__device__ __forceinline__ bf16x2_t as_bf16x2(uint32_t v) {
  return __builtin_bit_cast(bf16x2_t, v);
}

// acc + sum_{i<8} a[i] * b[i] for two 8 x bf16 vectors, fp32 accumulation
// (v_dot2_f32_bf16: two products per instruction).
__device__ __forceinline__ float dot8_bf16(u32x4 a, u32x4 b, float acc) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t ae = a[e];
    const uint32_t be = b[e];
    acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(ae), as_bf16x2(be), acc,
                                          false);
  }
  return acc;
}

// D = A B + C, A 16 x 32 and B 32 x 16 bf16, fp32 D and C
// (v_mfma_f32_16x16x32_bf16).  Lane l holds A[l % 16][8 (l / 16) + j] and
// B[8 (l / 16) + j][l % 16] as 8 bf16 (j = 0..7, one register quad) and
// D[4 (l / 16) + r][l % 16] in register r = 0..3.
__device__ __forceinline__ f32x4 mfma_16x16x32_bf16(u32x4 a, u32x4 b,
                                                     f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(
      __builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c, 0,
      0, 0);
}

// Operand e of a V block transposed in registers for the P.V MFMA (decode
// attention): lane (c, g4) holds dims 8 c .. 8 c + 7 of rows 8 g4 + j in
// vt[j]; dword p of the result = (row 2p, row 2p + 1) of dim 8 c + e.
__device__ __forceinline__ u32x4 v_operand(const u32x4 (&vt)[8], int e) {
  // v_perm_b32 selectors: low halves / high halves of (src1, src0)
  const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
  u32x4 r;
#pragma unroll
  for (int p = 0; p < 4; ++p)
    r[p] = __builtin_amdgcn_perm(vt[2 * p + 1][e >> 1], vt[2 * p][e >> 1], sel);
  return r;
}

// Two floats rounded to bf16 (round to nearest even), lo in bits 0..15.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two floats to a (lo, hi) bf16 pair, round-to-nearest-even: one
// v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(
      uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

// Wave-wide reductions.  Inside each 16-lane DPP row the values combine
// through four DPP moves (quad_perm [1,0,3,2] and [2,3,0,1] within each
// quad, row_half_mirror between the quads of a half row, row_mirror between
// the halves); the four row results are then read with v_readlane and
// combined in a fixed order.  Every lane returns the same (wave-uniform)
// result.  All 64 lanes must be active.  (A __shfl_xor butterfly lowers to
// six dependent LDS-crossbar permutes; these reductions sit on the tail of
// every GEMV and top-k pass.)
template <int CTRL>
__device__ __forceinline__ float dpp_float(float v) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
      0, static_cast<int>(v), CTRL, 0xF, 0xF, true));
}

__device__ __forceinline__ float lane_float(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Sum over the 16 lanes of a DPP row (lanes 16r .. 16r+15); every lane of
// the row receives the sum.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_float<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_float<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_float<0x141>(v);  // row_half_mirror
  v += dpp_float<0x140>(v);  // row_mirror
  return v;
}

__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_float<0xB1>(v));
  v = fmaxf(v, dpp_float<0x4E>(v));
  v = fmaxf(v, dpp_float<0x141>(v));
  v = fmaxf(v, dpp_float<0x140>(v));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  return (lane_float(v, 0) + lane_float(v, 16)) +
         (lane_float(v, 32) + lane_float(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  return fmaxf(fmaxf(lane_float(v, 0), lane_float(v, 16)),
               fmaxf(lane_float(v, 32), lane_float(v, 48)));
}

// Lane l combined with lane l ^ 16 (l ^ 32): v_permlane16_swap_b32 /
// v_permlane32_swap_b32 (gfx950) with one register as both operands return,
// in an order that depends on the lane, the lane's own value and its
// partner's, so a commutative combine gives the same result in both lanes.
// IEEE-754 2019 maximum (NaN-propagating): one v_maximum3_f32 on gfx950,
// with no quieting of the inputs that fmaxf's maxNum semantics needs.
// Softmax scores are finite or -inf, where both agree.
__device__ __forceinline__ float max_f32(float a, float b) {
  return __builtin_elementwise_maximum(a, b);
}

__device__ __forceinline__ float xor16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v),
                                                  __float_as_uint(v), false, false);
  return max_f32(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v),
                                                  __float_as_uint(v), false, false);
  return max_f32(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float xor16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v),
                                                  __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v),
                                                  __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <int CTRL>
__device__ __forceinline__ uint64_t dpp_max_u64(uint64_t v) {
  const uint32_t lo = dpp_u32<CTRL>(static_cast<uint32_t>(v));
  const uint32_t hi = dpp_u32<CTRL>(static_cast<uint32_t>(v >> 32));
  const uint64_t o = (static_cast<uint64_t>(hi) << 32) | lo;
  return o > v ? o : v;
}

__device__ __forceinline__ uint64_t lane_u64(uint64_t v, int lane) {
  const uint32_t lo = static_cast<uint32_t>(
      __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v)), lane));
  const uint32_t hi = static_cast<uint32_t>(
      __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v >> 32)), lane));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  v = dpp_max_u64<0xB1>(v);
  v = dpp_max_u64<0x4E>(v);
  v = dpp_max_u64<0x141>(v);
  v = dpp_max_u64<0x140>(v);
  uint64_t best = lane_u64(v, 0);
#pragma unroll
  for (int r = 1; r < 4; ++r) {
    const uint64_t o = lane_u64(v, 16 * r);
    best = o > best ? o : best;
  }
  return best;
}

// ---------------------------------------------------------------------------
// Top-k keys. A (value, index) pair maps to one uint64 whose unsigned order
// is "value descending, then index ascending", so selecting the k largest
// keys is an exact, deterministic top-k with lower-index-first tie breaking.
// -0.0 is folded into +0.0 and every NaN into one positive quiet NaN, which
// sorts above +inf (torch.topk also ranks NaN highest). Key 0 never encodes
// a real candidate and serves as the empty sentinel.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t ordered_bits(float v) {
  uint32_t u = __float_as_uint(v);
  if (v == 0.0f) u = 0u;
  if (v != v) u = 0x7fc00000u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float from_ordered_bits(uint32_t o) {
  uint32_t u = (o & 0x80000000u) ? (o & 0x7fffffffu) : ~o;
  return __uint_as_float(u);
}

__device__ __forceinline__ uint64_t topk_key(float v, uint32_t index) {
  return (static_cast<uint64_t>(ordered_bits(v)) << 32) |
         static_cast<uint64_t>(0xffffffffu - index);
}

__device__ __forceinline__ float key_value(uint64_t key) {
  return from_ordered_bits(static_cast<uint32_t>(key >> 32));
}

__device__ __forceinline__ int64_t key_index(uint64_t key) {
  return static_cast<int64_t>(0xffffffffu - static_cast<uint32_t>(key));
}

}  // namespace cascade
