// tq_mfma.h -- gfx950 building blocks shared by the attention kernels:
// f16 matrix-core operands with a two-part (hi/lo) split of f32 values,
// DPP wave reductions and the PQO decode constants.
#pragma once

#include <type_traits>
#include "tq_device.h"

namespace tqm {

using namespace tqd;

constexpr float kInvSqrt32 = 0x1.6a09e6p-3f;
constexpr float kLog2e = 1.44269504088896340736f;
// fl(fl(1/fl(sqrt 32)) * fl(sqrt 32)): the magnitude of every decode sign
// factor R_fwd[0][j] * sqrt(32) (wht_tensor.rs:28-41)
constexpr float kDecodeFactor = 0x1.fffffep-1f;

__device__ __forceinline__ float decode_sign(int j) {
  return ((kPqoSignMask >> j) & 1u) ? -kDecodeFactor : kDecodeFactor;
}
// Value of lane l ^ 1 (DPP quad permute [1, 0, 3, 2]) and of lane l ^ 2
// ([2, 3, 0, 1]).
__device__ __forceinline__ float dpp_quad_xor1(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
}
__device__ __forceinline__ float dpp_quad_xor2(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
}

// Value of lane l ^ 8 (DPP row_ror:8 inside rows of 16) and of lane l ^ 4 or
// l ^ 16 inside halves of 32 (ds_swizzle bit mode: source lane
// ((l & 31) ^ x), no address operand).
__device__ __forceinline__ float dpp_row_xor8(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xF, 0xF, true));
}
template <int X>
__device__ __forceinline__ float swizzle_xor(float v) {
  static_assert(X > 0 && X < 32, "inside 32 lanes");
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x1F | (X << 10)));
}
template <int X>
__device__ __forceinline__ float lane_xor(float v) {
  if constexpr (X == 1) return dpp_quad_xor1(v);
  else if constexpr (X == 2) return dpp_quad_xor2(v);
  else if constexpr (X == 8) return dpp_row_xor8(v);
  else return swizzle_xor<X>(v);
}
// The values of lane l and of lane l ^ 16 (l ^ 32), by one permlane swap of v
// with a copy of itself (v_permlane16_swap: the odd rows of the first
// operand trade places with the even rows of the second; v_permlane32_swap:
// the upper half of the first with the lower half of the second), so the
// two registers end as v of lane l and of its partner, in some order.  The
// swap is written in assembly: this toolchain's lowering of the
// __builtin_amdgcn_permlane*_swap pair result hands back the first register
// for both elements.  The s_nop gives the two wait states a VALU write needs
// before a permlane reads the register.
__device__ __forceinline__ void swap_pair16(float v, float &a, float &b) {
  a = v;
  b = v;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap_pair32(float v, float &a, float &b) {
  a = v;
  b = v;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
// Two registers' halves traded in place: afterwards a = (a of lanes 0-31,
// b of lanes 0-31) and b = (a of lanes 32-63, b of lanes 32-63), so a + b is
// a's sum over the halves in lanes 0-31 and b's in lanes 32-63.
__device__ __forceinline__ void trade_halves32(float &a, float &b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
// max(v, v of lane l ^ 16) and max(v, v of lane l ^ 32)
__device__ __forceinline__ float max_xor16(float v) {
  float a, b;
  swap_pair16(v, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float max_xor32(float v) {
  float a, b;
  swap_pair32(v, a, b);
  return fmaxf(a, b);
}

// Unnormalised 32-point Walsh-Hadamard transform across lanes: lane i (bits
// 0..4 of the lane index) ends with sum_j (-1)^popcount(i & j) v_j.
__device__ __forceinline__ float wht32_lanes(float v, int i) {
  auto stage = [&](float ov, int h) { return (i & h) ? (ov - v) : (v + ov); };
  v = stage(lane_xor<1>(v), 1);
  v = stage(lane_xor<2>(v), 2);
  v = stage(lane_xor<4>(v), 4);
  v = stage(lane_xor<8>(v), 8);
  v = stage(lane_xor<16>(v), 16);
  return v;
}

template <typename Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = op(v, __shfl_xor(v, o, 64));
  return v;
}

// DPP move: lanes whose source is outside the row (or whose row is masked
// off) take `id`.  Controls: row_shr:n = 0x110 + n, row_bcast:15 = 0x142,
// row_bcast:31 = 0x143.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp(float v, float id) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, id), __builtin_bit_cast(int, v),
                                                               CTRL, ROW_MASK, 0xf, false));
}

// Whole-wave reduction on the VALU (no LDS traffic): a row scan with
// row_shr 1/2/4/8 leaves each row's total in its lane 15, two row
// broadcasts fold the rows into lane 63, which is read back as a uniform.
template <typename Op>
__device__ __forceinline__ float wave_allreduce(float v, float id, Op op) {
  v = op(v, dpp<0x111>(v, id));
  v = op(v, dpp<0x112>(v, id));
  v = op(v, dpp<0x114>(v, id));
  v = op(v, dpp<0x118>(v, id));
  v = op(v, dpp<0x142, 0xa>(v, id));
  v = op(v, dpp<0x143, 0xc>(v, id));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
// Whole-wave max of non-NaN floats on order-preserving integer keys (the
// magnitude bits of negative values flipped), so every step is one integer
// max with a DPP operand and no float canonicalization.
__device__ __forceinline__ int order_key(int bits) { return bits ^ (int)((uint32_t)(bits >> 31) >> 1); }
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ int dpp_i(int v, int id) {
  return __builtin_amdgcn_update_dpp(id, v, CTRL, ROW_MASK, 0xf, false);
}
__device__ __forceinline__ float wave_max(float v) {
  constexpr int kMin = -2147483647 - 1;
  int k = order_key(__builtin_bit_cast(int, v));
  k = max(k, dpp_i<0x111>(k, kMin));
  k = max(k, dpp_i<0x112>(k, kMin));
  k = max(k, dpp_i<0x114>(k, kMin));
  k = max(k, dpp_i<0x118>(k, kMin));
  k = max(k, dpp_i<0x142, 0xa>(k, kMin));
  k = max(k, dpp_i<0x143, 0xc>(k, kMin));
  return __builtin_bit_cast(float, order_key(__builtin_amdgcn_readlane(k, 63)));
}
// Whole-wave integer sum and max (DPP row steps, two row broadcasts, lane
// 63 read back as a uniform), and the inclusive prefix sum over the lanes.
__device__ __forceinline__ int wave_sum_i(int v) {
  v += dpp_i<0x111>(v, 0);
  v += dpp_i<0x112>(v, 0);
  v += dpp_i<0x114>(v, 0);
  v += dpp_i<0x118>(v, 0);
  v += dpp_i<0x142, 0xa>(v, 0);
  v += dpp_i<0x143, 0xc>(v, 0);
  return __builtin_amdgcn_readlane(v, 63);
}
__device__ __forceinline__ int wave_max_i(int v) {
  constexpr int kMin = -2147483647 - 1;
  v = max(v, dpp_i<0x111>(v, kMin));
  v = max(v, dpp_i<0x112>(v, kMin));
  v = max(v, dpp_i<0x114>(v, kMin));
  v = max(v, dpp_i<0x118>(v, kMin));
  v = max(v, dpp_i<0x142, 0xa>(v, kMin));
  v = max(v, dpp_i<0x143, 0xc>(v, kMin));
  return __builtin_amdgcn_readlane(v, 63);
}
__device__ __forceinline__ int wave_incl_scan_i(int v) {
  v += dpp_i<0x111>(v, 0);  // row_shr:1 .. 8: inclusive sums inside each row of 16
  v += dpp_i<0x112>(v, 0);
  v += dpp_i<0x114>(v, 0);
  v += dpp_i<0x118>(v, 0);
  v += dpp_i<0x142, 0xa>(v, 0);  // row 15's total into rows 1 and 3
  v += dpp_i<0x143, 0xc>(v, 0);  // lane 31's total into rows 2 and 3
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
  return wave_allreduce(v, 0.f, [](float x, float y) { return x + y; });
}

// Device-coherent accesses to the split-K partials: relaxed atomics at agent
// scope bypass the non-coherent per-XCD caches.
__device__ __forceinline__ void st_agent(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- matrix-core operands ----
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// D + A B over 16 x 16 x 32 (f16 in, f32 accumulate).  Lane l holds A row
// l % 16 and B column l % 16, each at k = 8 (l / 16) .. 8 (l / 16) + 7 (two
// f16 per word, lower k in the low half), and D column l % 16 at rows
// 4 (l / 16) .. 4 (l / 16) + 3.
__device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 d) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), d, 0, 0,
                                                0);
}

// The same over bf16 operands (two per word, lower k in the low half).
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ f32x4 mfma_bf16(u32x4 a, u32x4 b, f32x4 d) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), d, 0,
                                                 0, 0);
}

// Transposing LDS read (ds_read_b64_tr_b16): inside each group of 16 lanes,
// lane 4 a + b receives item b (16-bit) of the 8-byte rows addressed by
// lanes a, a + 4, a + 8 and a + 12 of its group, in that order (item 0 in
// the low half of the first word).  p must point into LDS.
typedef short i16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2 lds_read_tr16(const void *p) {
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)p));
}

// Upper part of the two-part f16 split: x with its significand cut to 11
// bits (exact in f16 while |x| is in f16's normal range); x - hi is exact in
// f32 and is the lower part.
__device__ __forceinline__ float split_hi(float x) { return u2f(f2u(x) & 0xffffe000u); }
__device__ __forceinline__ uint32_t pack_f16(float lo_half, float hi_half) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo_half, hi_half));
}
// The same split from the f16 side: hi = pack_f16(x0, x1) (round toward zero
// is the 11-bit cut), and pack_rem(x0, x1, hi, k) = the f16 pair of x + k * hi,
// i.e. the lower parts for k = -1 (x - hi is exact in f32; the f16 -> f32
// widening folds into v_fma_mix_f32) and the upper parts again for k = 0.
__device__ __forceinline__ uint32_t pack_rem(float x0, float x1, uint32_t hi, float k) {
  const auto h = __builtin_bit_cast(__fp16 __attribute__((ext_vector_type(2))), hi);
  return pack_f16(__builtin_fmaf((float)h[0], k, x0), __builtin_fmaf((float)h[1], k, x1));
}
// E with m * 2^-E in [0.5, 1) for finite m > 0 (0 for m == 0), clamped so
// that 2^E and 2^-E are normal f32.
__device__ __forceinline__ int pow2_exponent(float m) {
  const int e = (int)((f2u(m) >> 23) & 0xffu);
  return e == 0 ? 0 : min(max(e - 126, -100), 100);
}
__device__ __forceinline__ float exp2i(int e) { return u2f((uint32_t)(127 + e) << 23); }

// Code pair p (codes 2p, 2p+1) of a qblock's BITS words, LSB-first: the
// 2 BITS-bit pair-table index (p must fold to a constant after unrolling).
template <int BITS>
__device__ __forceinline__ uint32_t pair_code(const uint32_t (&w)[BITS], int p) {
  constexpr int W = 2 * BITS;
  const int pos = W * p, wi = pos >> 5, sh = pos & 31;
  if (sh + W <= 32) return __builtin_amdgcn_ubfe(w[wi], sh, W);
  return __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh) & ((1u << W) - 1u);
}

// f(integral_constant<int, I>) for I = B .. E - 1, in order, at compile time.
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F &&f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

}  // namespace tqm
