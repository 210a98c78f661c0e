// tq_device.h -- device-side building blocks shared by the gfx950 kernels.
//
// All arithmetic that must agree bit-for-bit with the reference is written
// without contraction (the library is built with -ffp-contract=off); where a
// fused multiply-add is wanted it is spelled out with __builtin_fmaf.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tqd {

constexpr int kQBlock = 32;  // QUANT_BLOCK_SIZE (reference src/cache/config.rs:9)

__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }

// bf16 <-> f32.  bf16 -> f32 is exact; f32 -> bf16 rounds to nearest-even
// (the `half` crate's bf16::from_f32: (u + 0x7fff + lsb) >> 16, a NaN kept as
// (u >> 16) | 0x40).  gfx950's v_cvt_pk_bf16_f32 gives exactly that for every
// one of the 2^32 f32 inputs (both halves, checked exhaustively on MI355X);
// it is written in assembly because this toolchain's lowering of a
// two-element vector conversion fed the first element to both halves.
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }
// bf16(lo) in the low half, bf16(hi) in the high half
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  uint32_t r;
  asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(r) : "v"(lo), "v"(hi));
  return r;
}
__device__ __forceinline__ uint16_t f32_to_bf16(float x) { return (uint16_t)(pack_bf16x2(x, x) & 0xffffu); }

// f32 -> f16 round-to-nearest-even through the hardware conversion
// (v_cvt_f16_f32 in the default RNE mode, f16 denormals kept).
__device__ __forceinline__ uint16_t f32_to_f16(float x) {
  _Float16 h = (_Float16)x;
  return __builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

// Loads one element of the given storage type as f32 (exact).
enum DType : int { kF32 = 0, kBF16 = 1, kF16 = 2 };

// Next representable f32 toward +inf (finite inputs).
__device__ __forceinline__ float next_up(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) == 0) return u2f(1u);
  return u2f((int32_t)u >= 0 ? u + 1u : u - 1u);
}

// Smallest f32 x with fl(x / s) > b, given mu = (b + nextup(b)) / 2 (exact in
// f64) and strict = (b has an even significand, so a quotient exactly at mu
// rounds down to b).  mu * s is exact in f64 (25 x 24 significant bits), so
// the comparison x >= U is exactly the reference's fl(x/s) > b for every
// finite x when s is finite and positive.
__device__ __forceinline__ float div_threshold(double mu, bool strict, float s) {
  double p = mu * (double)s;
  float f = (float)p;
  double fd = (double)f;
  if (fd < p || (strict && fd == p)) f = next_up(f);
  return f;
}

// Unnormalized Sylvester butterfly over N registers, stages h = 1 .. N/2,
// pairing (j, j+h) as (x+y, x-y) -- the order of reference rotation.rs:24-35
// and wht_tensor.rs:44-59.
template <int N>
__device__ __forceinline__ void butterfly(float (&d)[N]) {
#pragma unroll
  for (int h = 1; h < N; h *= 2) {
#pragma unroll
    for (int i = 0; i < N; i += 2 * h) {
#pragma unroll
      for (int j = i; j < i + h; j++) {
        float x = d[j], y = d[j + h];
        d[j] = x + y;
        d[j + h] = x - y;
      }
    }
  }
}

// The reference's hardcoded 32-entry sign pattern for PQO blocks
// (src/cache/precomputed/rotation.rs:17-20), as a bit mask (bit j set <=> -1).
constexpr uint32_t kPqoSignMask =
    (0u << 0) | (1u << 1) | (0u << 2) | (0u << 3) | (1u << 4) | (1u << 5) | (0u << 6) | (1u << 7) |
    (0u << 8) | (0u << 9) | (1u << 10) | (0u << 11) | (1u << 12) | (0u << 13) | (1u << 14) | (1u << 15) |
    (0u << 16) | (1u << 17) | (1u << 18) | (0u << 19) | (0u << 20) | (1u << 21) | (0u << 22) | (1u << 23) |
    (1u << 24) | (0u << 25) | (0u << 26) | (0u << 27) | (1u << 28) | (1u << 29) | (0u << 30) | (1u << 31);

__host__ __device__ constexpr bool pqo_neg(int j) { return (kPqoSignMask >> j) & 1u; }

// PQO centroid i in f32 exactly as src/cache/precomputed/codebooks.rs:51-88
// evaluates it: 3-bit the fixed table, 4-bit -R + i * fl(2R / 15) with every
// step rounded to f32 (the library is built without contraction).  Written
// as a select chain so that device code indexes it by a lane-varying i
// without a memory table.
template <int BITS>
__host__ __device__ inline float pqo_centroid(int i) {
  static_assert(BITS == 2 || BITS == 3 || BITS == 4, "PQO codebooks are 2-, 3- or 4-bit");
  if constexpr (BITS == 4) {
    const float range = 2.1573f;
    const float step = (2.0f * range) / 15.0f;
    const float t = (float)i * step;
    return -range + t;
  } else {
    constexpr int NC = 1 << BITS;
    constexpr float c3[8] = {-2.1573f, -1.3336f, -0.7434f, -0.2428f, 0.2428f, 0.7434f, 1.3336f, 2.1573f};
    constexpr float c2[4] = {-2.1573f, -0.7434f, 0.7434f, 2.1573f};
    float v = BITS == 3 ? c3[0] : c2[0];
#pragma unroll
    for (int k = 1; k < NC; k++) v = (i == k) ? (BITS == 3 ? c3[k] : c2[k]) : v;
    return v;
  }
}

// Extracts the BITS-wide field i from a little-endian bitstream held in
// 32-bit words (fields may straddle a word boundary for BITS = 3).
template <int BITS, int NW>
__device__ __forceinline__ uint32_t field(const uint32_t (&w)[NW], int i) {
  const int pos = i * BITS;
  const int wi = pos >> 5, sh = pos & 31;
  if (sh + BITS <= 32) return (w[wi] >> sh) & ((1u << BITS) - 1u);
  return ((w[wi] >> sh) | (w[wi + 1] << (32 - sh))) & ((1u << BITS) - 1u);
}

}  // namespace tqd
