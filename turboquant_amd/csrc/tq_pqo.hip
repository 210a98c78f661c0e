// tq_pqo.hip -- PQO (block-32 MaxNorm) cache codec kernels for gfx950.
//
// Design: one lane owns one 32-element qblock.  The block's values live in
// 32 VGPRs, so the Walsh-Hadamard rotation is five in-register butterfly
// stages with no cross-lane traffic, the max-abs is a register reduction,
// and the bucketized codes are shifted straight into the packed words
// (12 B for 3-bit, 16 B for 4-bit) that the lane stores; nothing needs
// atomics or LDS.  A wave covers 64 consecutive qblocks, so its stores of
// packed codes and f16 scales are contiguous.
//
// Exactness: the reference computes v = fl(r / scale) and counts v > b_k
// (quantize_tensor.rs:107-108, 161-176).  Here each block turns its 2^b - 1
// boundaries into exact thresholds U_k in the input domain once
// (tqd::div_threshold, f64), and the per-element work is r >= U_k: the same
// codes for every finite input, without a division per element.
#include "tq_common.h"
#include "tq_device.h"

#include <algorithm>
#include <cmath>
#include <cstring>

namespace {

using namespace tqd;

constexpr float kInvSqrt32 = 0x1.6a09e6p-3f;  // fl(1 / fl(sqrt(32))) = 0.17677669f

struct QuantConsts {
  double mu[15];
  float b[15];
  float u[15];  // L2Norm: nextup(b), so x >= u <=> x > b
  uint32_t strict_mask;
  float mul;
  float scale_sign;
  int mixed_sign;  // scale sign per block: -1 for block % nb < eo
  int nb, eo;
  long long blk0;  // first block of this launch
  // Evenly spaced boundaries (the 4-bit MaxNorm codebook): b_k = b_0 + k D
  // up to a few ulps, and grid_step = fl(D), grid_off = fl(1 - b_0 / D).
  int grid;
  float grid_step, grid_off;
};

// Half-width of the band around an integer of the grid coordinate inside
// which the fast 4-bit path defers to the exact thresholds: 2^-16 = 256 u
// (u = 2^-24).  The coordinate's error is below 70 u (see quantize_grid).
constexpr float kGridBand = 0x1p-16f;

enum NormMode : int { kMaxNorm = 0, kL2Norm = 1 };

template <int BITS>
struct Packed {
  static constexpr int kWords = BITS;  // 32 * BITS / 32
  static constexpr int kBytes = 4 * BITS;
};

template <int IN_DT>
__device__ __forceinline__ void load_block(const void *__restrict__ x, long long blk, float (&r)[32]) {
  if constexpr (IN_DT == kF32) {
    const float4 *p = reinterpret_cast<const float4 *>(static_cast<const float *>(x) + blk * 32);
#pragma unroll
    for (int q = 0; q < 8; q++) {
      float4 v = p[q];
      r[4 * q + 0] = v.x;
      r[4 * q + 1] = v.y;
      r[4 * q + 2] = v.z;
      r[4 * q + 3] = v.w;
    }
  } else {
    const uint4 *p = reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(x) + blk * 32);
#pragma unroll
    for (int q = 0; q < 4; q++) {
      uint4 v = p[q];
      uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int k = 0; k < 4; k++) {
        if constexpr (IN_DT == kBF16) {
          r[8 * q + 2 * k] = u2f(w[k] << 16);
          r[8 * q + 2 * k + 1] = u2f(w[k] & 0xffff0000u);
        } else {
          r[8 * q + 2 * k] = f16_to_f32((uint16_t)(w[k] & 0xffffu));
          r[8 * q + 2 * k + 1] = f16_to_f32((uint16_t)(w[k] >> 16));
        }
      }
    }
  }
}

// #{t : U[t] <= x} for the 2^BITS - 1 ascending thresholds U: a binary search
// whose probe at each level is picked from the candidates by the decisions
// already made (a select tree), BITS compares per element instead of
// 2^BITS - 1.
template <int BITS>
__device__ __forceinline__ uint32_t bucket_sorted(float x, const float (&U)[(1 << BITS) - 1]) {
  if constexpr (BITS == 2) {
    const bool b1 = x >= U[1];
    const bool b0 = x >= (b1 ? U[2] : U[0]);
    return (b1 ? 2u : 0u) | (b0 ? 1u : 0u);
  } else if constexpr (BITS == 3) {
    const bool b2 = x >= U[3];
    const bool b1 = x >= (b2 ? U[5] : U[1]);
    const float lo = b1 ? U[2] : U[0], hi = b1 ? U[6] : U[4];
    const bool b0 = x >= (b2 ? hi : lo);
    return (b2 ? 4u : 0u) | (b1 ? 2u : 0u) | (b0 ? 1u : 0u);
  } else {
    const bool b3 = x >= U[7];
    const bool b2 = x >= (b3 ? U[11] : U[3]);
    const float l1 = b2 ? U[5] : U[1], h1 = b2 ? U[13] : U[9];
    const bool b1 = x >= (b3 ? h1 : l1);
    const float a0 = b1 ? U[2] : U[0], a1 = b1 ? U[6] : U[4], a2 = b1 ? U[10] : U[8], a3 = b1 ? U[14] : U[12];
    const float l0 = b2 ? a1 : a0, h0 = b2 ? a3 : a2;
    const bool b0 = x >= (b3 ? h0 : l0);
    return (b3 ? 8u : 0u) | (b2 ? 4u : 0u) | (b1 ? 2u : 0u) | (b0 ? 1u : 0u);
  }
}

// The code bits of x, most significant first, by the same binary search as
// bucket_sorted.
template <int BITS>
__device__ __forceinline__ void bucket_bits(float x, const float (&U)[(1 << BITS) - 1], bool (&bit)[BITS]) {
  if constexpr (BITS == 2) {
    bit[0] = x >= U[1];
    bit[1] = x >= (bit[0] ? U[2] : U[0]);
  } else if constexpr (BITS == 3) {
    bit[0] = x >= U[3];
    bit[1] = x >= (bit[0] ? U[5] : U[1]);
    const float lo = bit[1] ? U[2] : U[0], hi = bit[1] ? U[6] : U[4];
    bit[2] = x >= (bit[0] ? hi : lo);
  } else {
    bit[0] = x >= U[7];
    bit[1] = x >= (bit[0] ? U[11] : U[3]);
    const float l1 = bit[1] ? U[5] : U[1], h1 = bit[1] ? U[13] : U[9];
    bit[2] = x >= (bit[0] ? h1 : l1);
    const float a0 = bit[2] ? U[2] : U[0], a1 = bit[2] ? U[6] : U[4], a2 = bit[2] ? U[10] : U[8],
                a3 = bit[2] ? U[14] : U[12];
    const float l0 = bit[1] ? a1 : a0, h0 = bit[1] ? a3 : a2;
    bit[3] = x >= (bit[0] ? h0 : l0);
  }
}

// acc = 2 acc + bit, with the bit taken straight from the comparison's lane
// mask as the carry-in of one v_addc (LLVM would rebuild it as a select, a
// shift and an or).  The s_nop covers the wait after a VALU write of the
// mask's SGPRs.
__device__ __forceinline__ uint32_t push_bit(uint32_t acc, bool bit) {
  uint32_t r;
  uint64_t carry_out;
  asm("s_nop 1\n\tv_addc_co_u32_e64 %0, %1, %2, %2, %3"
      : "=v"(r), "=s"(carry_out)
      : "v"(acc), "s"(__builtin_amdgcn_ballot_w64(bit)));
  return r;
}

// MaxNorm scale, exact bucketize and pack of one rotated block.  The packed
// LSB-first bitstream is built from its most significant bit down: code j's
// bits go to stream bits 3j+2 .. 3j (for 3-bit codes) and each 32-bit word
// is the last 32 bits pushed into it, so codes that straddle words need no
// special case.  CB < BITS: CB-bit codes (the standard codebook) in BITS-wide
// slots, whose top bits stay zero (quantize_tensor.rs:73, config.rs:82-84).
template <int BITS, int CB>
__device__ __forceinline__ void pack_codes(const float (&r)[32], const float (&U)[(1 << CB) - 1],
                                           uint32_t (&w)[Packed<BITS>::kWords]) {
  uint32_t acc[Packed<BITS>::kWords];
#pragma unroll
  for (int q = 0; q < Packed<BITS>::kWords; q++) acc[q] = 0;
#pragma unroll
  for (int j = 31; j >= 0; j--) {
    bool bit[CB];
    bucket_bits<CB>(r[j], U, bit);
#pragma unroll
    for (int t = 0; t < BITS; t++) {
      const int pos = j * BITS + (BITS - 1 - t);
      if (t < BITS - CB) acc[pos >> 5] <<= 1;
      else acc[pos >> 5] = push_bit(acc[pos >> 5], bit[t - (BITS - CB)]);
    }
  }
#pragma unroll
  for (int q = 0; q < Packed<BITS>::kWords; q++) w[q] = acc[q];
}

template <int BITS, int CB = BITS>
__device__ __forceinline__ float quantize_block(const float (&r)[32], const QuantConsts &k,
                                                uint32_t (&w)[Packed<BITS>::kWords]) {
  static_assert(CB <= BITS, "codes fit their slots");
  constexpr int NB = (1 << CB) - 1;
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(r[j]));
  float s = amax * k.mul;
  if (s < 1e-10f) s = 1e-10f;

  uint32_t idx[32];
  if (__builtin_isfinite(s)) {
    float U[NB];
#pragma unroll
    for (int t = 0; t < NB; t++) U[t] = div_threshold(k.mu[t], (k.strict_mask >> t) & 1u, s);
    pack_codes<BITS, CB>(r, U, w);
    return s;
  } else {
    // Infinite scale (an infinite input): follow the reference's division.
#pragma unroll
    for (int j = 0; j < 32; j++) {
      float v = r[j] / s;
      uint32_t c = 0;
#pragma unroll
      for (int t = 0; t < NB; t++) c += (v > k.b[t]) ? 1u : 0u;
      idx[j] = c;
    }
  }
#pragma unroll
  for (int q = 0; q < Packed<BITS>::kWords; q++) w[q] = 0;
#pragma unroll
  for (int j = 0; j < 32; j++) {
    const int pos = j * BITS, wi = pos >> 5, sh = pos & 31;
    w[wi] |= idx[j] << sh;
    if (sh + BITS > 32) w[wi + 1] |= idx[j] >> (32 - sh);
  }
  return s;
}

// Fast MaxNorm bucketize for evenly spaced boundaries, on the butterfly
// outputs x_j before the sign and 1/sqrt(32) factor f_j = +-fl(1/sqrt(32)).
// The reference code is q_j = #{k : fl(fl(x_j f_j) / s) > b_k}.  With
// W = x_j f_j / s (real) and D the boundary spacing, boundary k sits at
// T = (v - b_0) / D + 1 = k + 1 + d_k, |d_k| <= 11 u for this codebook
// (checked on the host, which sets k.grid only below 16 u).  The lane
// computes t = fma(x_j, +-fl(fl(1/sqrt(32)) / fl(s D)), fl(1 - b_0 / D)):
// the scale carries <= 3 u, v's two roundings 2 u, |W / D| <= outer / D =
// 7.5, the offset's rounding 8 u (|1 - b_0 / D| < 8.5) and t's own rounding
// 8 u (t < 16 near a boundary), so |t - T| <= 7.5 * 5 u + 8 u + 8 u + 16 u
// (d_k) < 70 u.  Where t is more than
// kGridBand = 256 u from every integer, each comparison v > b_k equals
// t > k + 1, so q_j = min(floor(t), 15) (0 for t < 1).  Returns false when
// some element of the block falls inside the band (or t is NaN); the caller
// then takes the exact path for the whole block.
__device__ __forceinline__ bool quantize_grid(const float (&x)[32], float s, const QuantConsts &k,
                                              uint32_t (&w)[4]) {
  const float a = kInvSqrt32 / (s * k.grid_step);
  bool clear = true;
#pragma unroll
  for (int q = 0; q < 4; q++) w[q] = 0;
#pragma unroll
  for (int j = 0; j < 32; j++) {
    const float t = __builtin_fmaf(x[j], pqo_neg(j) ? -a : a, k.grid_off);
    const uint32_t c = (uint32_t)__builtin_amdgcn_fmed3f(t, 0.0f, 15.5f);
    const float f = __builtin_amdgcn_fractf(t);
    clear = clear && (fabsf(f - 0.5f) < 0.5f - kGridBand);
    w[j >> 3] |= c << (4 * (j & 7));
  }
  return clear;
}

template <int BITS>
__device__ __forceinline__ void store_packed(uint8_t *__restrict__ packed, long long blk,
                                             const uint32_t (&w)[Packed<BITS>::kWords]) {
  uint32_t *p = reinterpret_cast<uint32_t *>(packed + blk * Packed<BITS>::kBytes);
  if constexpr (BITS == 4) {
    *reinterpret_cast<uint4 *>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  } else if constexpr (BITS == 2) {
    *reinterpret_cast<uint2 *>(p) = make_uint2(w[0], w[1]);
  } else {
    p[0] = w[0];
    p[1] = w[1];
    p[2] = w[2];
  }
}

// Placement of contiguous [heads][tokens] vectors in a cache laid out
// [heads][head_stride] records (CompressedStorage, storage.rs:24-139):
// vector (h, t) <-> record h * head_stride + offset + t.
struct CacheMap {
  uint32_t qb_per_vec;  // head_dim / 32
  uint32_t tokens;
  long long head_stride;
  long long offset;
};

__device__ __forceinline__ long long cache_block(uint32_t blk, const CacheMap &m) {
  const uint32_t v = blk / m.qb_per_vec, j = blk - v * m.qb_per_vec;
  const uint32_t h = v / m.tokens, t = v - h * m.tokens;
  return ((long long)h * m.head_stride + m.offset + t) * m.qb_per_vec + j;
}

// ROTATE: input is raw activations (fused forward rotation, butterfly order).
// Otherwise input is already rotated f32 (the reference kernel's contract).
// MAP: outputs go to cache records (CacheMap) instead of block order.
// NORM = kL2Norm: the block's L2 norm (sum of squares in element order,
// sqrt, clamped to 1e-10) divides it before the rotation and is its scale;
// codes count the boundaries strictly below the rotated value
// (normalize_and_rotate, quantize_tensor.rs:90-101, 161-176).
// MIXED: one of the two launches of a mixed-outlier config (blocks from
// k.blk0, scale sign per block).
template <int BITS, int CB, int IN_DT, bool ROTATE, bool MAP, int NORM, bool MIXED>
__global__ __launch_bounds__(256) void pqo_quant_kernel(const void *__restrict__ x,
                                                        uint8_t *__restrict__ packed,
                                                        uint16_t *__restrict__ scales,
                                                        long long nblocks, QuantConsts k, CacheMap map) {
  const long long b0 = MIXED ? k.blk0 : 0;
  const long long blk = b0 + (long long)blockIdx.x * 256 + threadIdx.x;
  if (blk >= b0 + nblocks) return;
  const long long ob = MAP ? cache_block((uint32_t)blk, map) : blk;
  float r[32];
  load_block<IN_DT>(x, blk, r);
  float nrm = 0.f;
  if constexpr (NORM == kL2Norm) {
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++) ss = ss + r[j] * r[j];
    nrm = sqrtf(ss);
    nrm = nrm < 1e-10f ? 1e-10f : nrm;
#pragma unroll
    for (int j = 0; j < 32; j++) r[j] = r[j] / nrm;
  }
  uint32_t w[Packed<BITS>::kWords];
  float s = 0.0f;
  bool done = false;
  if constexpr (ROTATE) {
    butterfly<32>(r);
    if constexpr (NORM == kMaxNorm && BITS == 4 && CB == 4) {
      if (k.grid) {
        // max_j |fl(x_j f_j)| = fl(max_j |x_j| / sqrt(32)): rounding is monotone
        float am = 0.0f;
#pragma unroll
        for (int j = 0; j < 32; j++) am = fmaxf(am, fabsf(r[j]));
        s = (am * kInvSqrt32) * k.mul;
        if (s < 1e-10f) s = 1e-10f;
        done = __builtin_isfinite(s) && quantize_grid(r, s, k, w);
      }
    }
    if (!done) {
#pragma unroll
      for (int j = 0; j < 32; j++) r[j] = r[j] * (pqo_neg(j) ? -kInvSqrt32 : kInvSqrt32);
    }
  }
  if (done) {
  } else if constexpr (NORM == kL2Norm) {
    float U[(1 << CB) - 1];
#pragma unroll
    for (int t = 0; t < (1 << CB) - 1; t++) U[t] = k.u[t];
    pack_codes<BITS, CB>(r, U, w);
    s = nrm;
  } else {
    s = quantize_block<BITS, CB>(r, k, w);
  }
  store_packed<BITS>(packed, ob, w);
  const float sign = MIXED ? (((int)(blk % k.nb) < k.eo) ? -1.0f : 1.0f) : k.scale_sign;
  scales[ob] = f32_to_f16(s * sign);
}

// Reference-ABI variant: boundaries and outer centroid come from the caller
// (device boundaries), constants derived in-kernel per lane.
template <int BITS>
__global__ __launch_bounds__(256) void pqo_quant_rotated_dev_kernel(
    const float *__restrict__ rotated, const float *__restrict__ boundaries,
    uint8_t *__restrict__ packed, uint16_t *__restrict__ scales, long long nblocks, float outer,
    float scale_sign) {
  const long long blk = (long long)blockIdx.x * 256 + threadIdx.x;
  if (blk >= nblocks) return;
  constexpr int NB = (1 << BITS) - 1;
  QuantConsts k;
#pragma unroll
  for (int t = 0; t < NB; t++) {
    float b = boundaries[t];
    float up = next_up(b);
    k.b[t] = b;
    k.mu[t] = ((double)b + (double)up) * 0.5;
  }
  k.strict_mask = 0;
#pragma unroll
  for (int t = 0; t < NB; t++) k.strict_mask |= ((f2u(k.b[t]) & 1u) == 0 ? 1u : 0u) << t;
  k.mul = (float)(1.0 / (double)outer);
  k.scale_sign = scale_sign;
  float r[32];
  load_block<kF32>(rotated, blk, r);
  uint32_t w[Packed<BITS>::kWords];
  float s = quantize_block<BITS>(r, k, w);
  store_packed<BITS>(packed, blk, w);
  scales[blk] = f32_to_f16(s * scale_sign);
}

struct DequantConsts {
  float cb[16];   // codebook values (f32); the outlier codebook when mixed
  float cbn[16];  // mixed: the standard codebook
  // the reference's sign factor of element j is fl(R_fwd[0][j] * sqrt(32)) =
  // (pqo_neg(j) ? -sgm : sgm): one magnitude for every j
  float sgm;
  int mixed;      // codebook per block by the scale's sign (quantize_tensor.rs:242-260)
  int nn;         // mixed: standard codebook size (codes are clamped into it)
};

// out_j = fl(fl(W_j * fl(1/sqrt(32))) * |scale|), W = butterfly(cb[idx] * sign):
// butterfly_wht_inverse_cpu (wht_tensor.rs:38-64) then the broadcast_mul by
// |scale| (quantize_tensor.rs:203, 217-218).
// MAP: inputs come from cache records (CacheMap); outputs in block order.
// MIXED: the codebook per block from the scale's sign (else one codebook).
// With the library's constants the table holds fl(cb * |sg|) and element j
// takes it negated where sg[j] < 0: fl(c * -m) = -fl(c * m), the same value
// as the per-element product, one multiply per table entry instead of per
// element.
template <int BITS, int OUT_DT, bool DEV_CONSTS, bool MAP = false, bool MIXED = false>
__global__ __launch_bounds__(256) void pqo_dequant_kernel(const uint8_t *__restrict__ packed,
                                                          const uint16_t *__restrict__ scales,
                                                          void *__restrict__ out, long long nblocks,
                                                          DequantConsts dc,
                                                          const float *__restrict__ dev_cb,
                                                          const float *__restrict__ dev_sg, CacheMap map = {}) {
  __shared__ float lut[32];
  constexpr int NC = 1 << BITS;
  if (threadIdx.x < NC) lut[threadIdx.x] = DEV_CONSTS ? dev_cb[threadIdx.x] : dc.cb[threadIdx.x] * dc.sgm;
  if (MIXED && threadIdx.x >= 16 && threadIdx.x < 32) lut[threadIdx.x] = dc.cbn[threadIdx.x - 16] * dc.sgm;
  __syncthreads();
  const long long blk = (long long)blockIdx.x * 256 + threadIdx.x;
  // lanes past the end still take part in the wave's output staging
  const bool valid = blk < nblocks;
  const long long ib = !valid ? 0 : (MAP ? cache_block((uint32_t)blk, map) : blk);
  uint32_t w[Packed<BITS>::kWords];
#pragma unroll
  for (int q = 0; q < Packed<BITS>::kWords; q++) w[q] = 0u;
  uint16_t sbits = 0;
  if (valid) {
    const uint32_t *p = reinterpret_cast<const uint32_t *>(packed + ib * Packed<BITS>::kBytes);
    if constexpr (BITS == 4) {
      uint4 v = *reinterpret_cast<const uint4 *>(p);
      w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else if constexpr (BITS == 2) {
      uint2 v = *reinterpret_cast<const uint2 *>(p);
      w[0] = v.x; w[1] = v.y;
    } else {
#pragma unroll
      for (int q = 0; q < 3; q++) w[q] = p[q];
    }
    sbits = scales[ib];
  }
  const float ssig = f16_to_f32(sbits);
  const float s = fabsf(ssig);
  // mixed: a non-negative scale selects the standard codebook, codes clamped
  float z[32];
  if constexpr (MIXED) {
    const bool std_cb = !(ssig < 0.0f);
    const uint32_t base = std_cb ? 16u : 0u, cmax = std_cb ? (uint32_t)dc.nn - 1u : 15u;
#pragma unroll
    for (int j = 0; j < 32; j++) {
      const float c = lut[base + min(field<BITS>(w, j), cmax)];
      z[j] = pqo_neg(j) ? -c : c;
    }
  } else {
#pragma unroll
    for (int j = 0; j < 32; j++) {
      const float c = lut[field<BITS>(w, j)];
      if constexpr (DEV_CONSTS) z[j] = c * dev_sg[j];
      else z[j] = pqo_neg(j) ? -c : c;
    }
  }
  butterfly<32>(z);
#pragma unroll
  for (int j = 0; j < 32; j++) z[j] = (z[j] * kInvSqrt32) * s;
  // the block's output words
  constexpr int NDW = OUT_DT == kF32 ? 32 : 16;
  uint32_t v[NDW];
  if constexpr (OUT_DT == kF32) {
#pragma unroll
    for (int j = 0; j < 32; j++) v[j] = f2u(z[j]);
  } else {
#pragma unroll
    for (int k = 0; k < 16; k++) {
      const float a = z[2 * k], b = z[2 * k + 1];
      if constexpr (OUT_DT == kBF16) v[k] = pack_bf16x2(a, b);
      else v[k] = (uint32_t)f32_to_f16(a) | ((uint32_t)f32_to_f16(b) << 16);
    }
  }
  // A wave's 64 blocks are one contiguous run of 64 * NDW words: staged
  // through LDS (rows padded to RS words), each store instruction writes
  // 1 KB of it contiguously rather than 16 bytes into each of 64 lines.
  constexpr int RS = NDW + 4;
  __shared__ __attribute__((aligned(16))) uint32_t s_out[4][64 * RS];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t *row = s_out[wave] + lane * RS;
#pragma unroll
  for (int k = 0; k < NDW / 4; k++)
    *reinterpret_cast<uint4 *>(row + 4 * k) = make_uint4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const long long wb = (long long)blockIdx.x * 256 + wave * 64;  // the wave's first block
  uint32_t *dst = static_cast<uint32_t *>(out) + wb * NDW;
#pragma unroll
  for (int q = 0; q < NDW / 4; q++) {
    const int f = 256 * q + 4 * lane;  // word of the wave's run
    const int r = f / NDW, c = f % NDW;
    if (wb + r < nblocks)
      *reinterpret_cast<uint4 *>(dst + f) = *reinterpret_cast<const uint4 *>(s_out[wave] + r * RS + c);
  }
}

// One thread per output byte: gathers the codes overlapping bits [8i, 8i+8).
__global__ __launch_bounds__(256) void pack_indices_kernel(const uint8_t *__restrict__ idx,
                                                           uint8_t *__restrict__ out,
                                                           long long nvec, int block_size, int bits,
                                                           int bytes_per_block) {
  const long long g = (long long)blockIdx.x * 256 + threadIdx.x;
  if (g >= nvec * bytes_per_block) return;
  const long long v = g / bytes_per_block;
  const int byte = (int)(g % bytes_per_block);
  const uint8_t *src = idx + v * block_size;
  uint32_t acc = 0;
  const int lo = byte * 8, hi = lo + 8;
  const int mask = (1 << bits) - 1;
  for (int i = lo / bits; i * bits < hi && i < block_size; i++) {
    const int pos = i * bits - lo;  // may be negative for a code straddling in
    uint32_t c = (uint32_t)(src[i] & mask);
    acc |= pos >= 0 ? (c << pos) : (c >> -pos);
  }
  out[g] = (uint8_t)(acc & 0xffu);
}

// One launch of pqo_quant_kernel for (slot bits, codebook bits, input type):
// ROTATE for activations, MAP for cache placement.
template <bool ROTATE, bool MAP, int NORM, bool MIXED>
int launch_quant(const void *x, int dt, uint8_t *packed, uint16_t *scales, long long nblocks, int bits, int cb_bits,
                 const QuantConsts &k, const CacheMap &m, hipStream_t st) {
  if (nblocks <= 0) return TQ_OK;
  const dim3 grid((unsigned)((nblocks + 255) / 256)), block(256);
#define QL(B, C, D) hipLaunchKernelGGL((pqo_quant_kernel<B, C, D, ROTATE, MAP, NORM, MIXED>), grid, block, 0, st, x, \
                                       packed, scales, nblocks, k, m)
#define QD(B, C) \
  do {                                      \
    if (!ROTATE || dt == kF32) QL(B, C, kF32); \
    else if (dt == kBF16) QL(B, C, kBF16);  \
    else QL(B, C, kF16);                    \
  } while (0)
  if (bits == 2) QD(2, 2);
  else if (bits == 3 && cb_bits == 3) QD(3, 3);
  else if (bits == 3) QD(3, 2);
  else if (cb_bits == 4) QD(4, 4);
  else QD(4, 3);
#undef QD
#undef QL
  return tqh::check_launch("pqo_quant_kernel");
}

QuantConsts make_quant_consts(const tqh::PqoCodebook &cb, float outer, float scale_sign) {
  tqh::DivThresholds t = tqh::div_thresholds(cb.b, cb.nc - 1, outer);
  QuantConsts k{};
  for (int i = 0; i < t.nb; i++) {
    k.mu[i] = t.mu[i];
    k.b[i] = cb.b[i];
    uint32_t u;
    std::memcpy(&u, &cb.b[i], 4);  // nextup(b) for finite b
    if ((u & 0x7fffffffu) == 0) u = 1u;
    else u = ((int32_t)u >= 0) ? u + 1u : u - 1u;
    std::memcpy(&k.u[i], &u, 4);
  }
  k.strict_mask = t.strict_mask;
  k.mul = t.mul;
  k.scale_sign = scale_sign;
  // Evenly spaced 15 boundaries whose offsets from the grid stay below 16 u
  // in grid units (11 u for the 4-bit MaxNorm codebook) and whose spacing
  // keeps |W / D| <= outer / D near 7.5 (the error budget of quantize_grid).
  if (cb.nc == 16) {
    const double d = ((double)cb.b[14] - (double)cb.b[0]) / 14.0;
    double dev = 0.0;
    for (int i = 0; i < 15; i++) dev = std::max(dev, std::fabs(((double)cb.b[i] - (double)cb.b[0]) / d - i));
    if (d > 0.0 && dev < 16.0 * 0x1p-24 && (double)outer / d < 7.6 && std::fabs(1.0 - (double)cb.b[0] / d) < 8.5) {
      k.grid = 1;
      k.grid_step = (float)d;
      k.grid_off = (float)(1.0 - (double)cb.b[0] / d);
    }
  }
  return k;
}

// polar_quantize of nblocks blocks (vectors of codec.num_blocks blocks) in
// one launch per codebook: a mixed config's first nblocks / nb * eo blocks
// on the outlier codebook, the rest on the standard one.
template <bool MAP>
int launch_polar_quant(const void *x, int dt, uint8_t *packed, uint16_t *scales, long long nblocks,
                       const tqh::PolarCodec &codec, const CacheMap &m, hipStream_t st) {
  auto run = [&](const tqh::PqoCodebook &cb, int cb_bits, long long b0, long long n) {
    QuantConsts k = make_quant_consts(cb, codec.outer, codec.scale_sign);
    k.mixed_sign = codec.mixed ? 1 : 0;
    k.nb = codec.num_blocks;
    k.eo = codec.eo;
    k.blk0 = b0;
    if (codec.mixed) {
      if (codec.norm_mode == kL2Norm)
        return launch_quant<true, MAP, kL2Norm, true>(x, dt, packed, scales, n, codec.bits, cb_bits, k, m, st);
      return launch_quant<true, MAP, kMaxNorm, true>(x, dt, packed, scales, n, codec.bits, cb_bits, k, m, st);
    }
    if (codec.norm_mode == kL2Norm)
      return launch_quant<true, MAP, kL2Norm, false>(x, dt, packed, scales, n, codec.bits, cb_bits, k, m, st);
    return launch_quant<true, MAP, kMaxNorm, false>(x, dt, packed, scales, n, codec.bits, cb_bits, k, m, st);
  };
  if (!codec.mixed) return run(codec.cb, codec.cb_bits, 0, nblocks);
  const long long nout = nblocks / codec.num_blocks * codec.eo;  // bucketize_blocks' outlier rows
  int rc = run(codec.ocb, codec.bits, 0, nout);
  if (rc) return rc;
  return run(codec.ncb, codec.bits - 1, nout, nblocks - nout);
}

DequantConsts make_dequant_consts(const tqh::PqoCodebook &cb);

DequantConsts dequant_consts(const tqh::PolarCodec &codec) {
  DequantConsts dc = make_dequant_consts(codec.mixed ? codec.ocb : codec.cb);
  if (codec.mixed) {
    for (int i = 0; i < codec.ncb.nc; i++) dc.cbn[i] = codec.ncb.c[i];
    dc.nn = codec.ncb.nc;
    dc.mixed = 1;
  }
  return dc;
}

DequantConsts make_dequant_consts(const tqh::PqoCodebook &cb) {
  DequantConsts dc{};
  for (int i = 0; i < cb.nc; i++) dc.cb[i] = cb.c[i];
  dc.nn = cb.nc;
  // fl(R_fwd[0][j] * sqrt(32)) = fl(+-fl(1/sqrt(32)) * fl(sqrt(32))) (wht_tensor.rs:28-41)
  volatile float thirty_two = 32.0f;
  volatile float sq = sqrtf(thirty_two);  // fl(sqrt(32)), IEEE sqrt
  volatile float inv = 1.0f / sq;
  volatile float m = inv * sq;  // fl(+-inv * sq) = +-fl(inv * sq)
  dc.sgm = m;
  return dc;
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------

namespace {
int check_shape(int head_dim) {
  if (head_dim <= 0 || head_dim % 32 != 0)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "head_dim (%d) must be divisible by QUANT_BLOCK_SIZE (32)", head_dim);
  return TQ_OK;
}

template <bool MAP>
int launch_dequant(const uint8_t *packed, const uint16_t *scales, void *out, int out_dtype, long long nblocks,
                   int bits, const DequantConsts &dc, const CacheMap &m, hipStream_t stream) {
  const dim3 grid((unsigned)((nblocks + 255) / 256)), block(256);
#define DL(B, D)                                                                                                  \
  do {                                                                                                            \
    if (dc.mixed)                                                                                                 \
      hipLaunchKernelGGL((pqo_dequant_kernel<B, D, false, MAP, true>), grid, block, 0, stream, packed, scales, out, \
                         nblocks, dc, nullptr, nullptr, m);                                                       \
    else                                                                                                          \
      hipLaunchKernelGGL((pqo_dequant_kernel<B, D, false, MAP, false>), grid, block, 0, stream, packed, scales,     \
                         out, nblocks, dc, nullptr, nullptr, m);                                                  \
  } while (0)
  if (bits == 3) {
    if (out_dtype == kF32) DL(3, kF32);
    else if (out_dtype == kBF16) DL(3, kBF16);
    else DL(3, kF16);
  } else {
    if (out_dtype == kF32) DL(4, kF32);
    else if (out_dtype == kBF16) DL(4, kBF16);
    else DL(4, kF16);
  }
#undef DL
  return tqh::check_launch("pqo_dequant_kernel");
}
}  // namespace

extern "C" int tq_polar_quantize(const void *x, int x_dtype, uint8_t *packed_out, uint16_t *scales_out,
                                 size_t num_vectors, int head_dim, int bits, size_t outlier_blocks, int norm_mode,
                                 hipStream_t stream) {
  int rc = check_shape(head_dim);
  if (rc) return rc;
  tqh::PolarCodec codec;
  rc = tqh::polar_codec(bits, norm_mode, outlier_blocks, head_dim / 32, codec);
  if (rc) return rc;
  if (!tqh::valid_dtype(x_dtype)) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "unknown dtype %d", x_dtype);
  if (num_vectors == 0) return TQ_OK;
  if (!x || !packed_out || !scales_out) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
  const long long nblocks = (long long)num_vectors * (head_dim / 32);
  return launch_polar_quant<false>(x, x_dtype, packed_out, scales_out, nblocks, codec, CacheMap{}, stream);
}

extern "C" int tq_polar_dequantize(const uint8_t *packed, const uint16_t *scales, void *out, int out_dtype,
                                   size_t num_vectors, int head_dim, int bits, size_t outlier_blocks, int norm_mode,
                                   hipStream_t stream) {
  int rc = check_shape(head_dim);
  if (rc) return rc;
  tqh::PolarCodec codec;
  rc = tqh::polar_codec(bits, norm_mode, outlier_blocks, head_dim / 32, codec);
  if (rc) return rc;
  if (!tqh::valid_dtype(out_dtype)) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "unknown dtype %d", out_dtype);
  if (num_vectors == 0) return TQ_OK;
  if (!packed || !scales || !out) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
  const long long nblocks = (long long)num_vectors * (head_dim / 32);
  return launch_dequant<false>(packed, scales, out, out_dtype, nblocks, bits, dequant_consts(codec),
                               CacheMap{}, stream);
}

extern "C" int tq_pqo_quantize(const void *x, int x_dtype, uint8_t *packed_out, uint16_t *scales_out,
                               size_t num_vectors, int head_dim, int bits, hipStream_t stream) {
  return tq_polar_quantize(x, x_dtype, packed_out, scales_out, num_vectors, head_dim, bits, TQ_OUTLIER_ALL,
                           TQ_NORM_MAXNORM, stream);
}

extern "C" int tq_pqo_dequantize(const uint8_t *packed, const uint16_t *scales, void *out, int out_dtype,
                                 size_t num_vectors, int head_dim, int bits, hipStream_t stream) {
  return tq_polar_dequantize(packed, scales, out, out_dtype, num_vectors, head_dim, bits, TQ_OUTLIER_ALL,
                             TQ_NORM_MAXNORM, stream);
}

extern "C" int tq_quant_maxnorm_batch(const float *rotated_input, const float *boundaries, uint8_t *packed_out,
                                      uint16_t *scales_out, int num_blocks, int block_size, int bits,
                                      int num_boundaries, int bytes_per_block, float outer_centroid,
                                      float scale_sign, hipStream_t stream) {
  if (num_blocks == 0) return TQ_OK;  // tq_quant_kernel.cu:430
  if (num_blocks < 0) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "num_blocks < 0");
  if (block_size != 32) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "block_size must be QUANT_BLOCK_SIZE (32), got %d", block_size);
  if (bits < 2 || bits > 4) return tqh::fail(TQ_ERR_UNSUPPORTED_BITS, "unsupported bit width %d", bits);
  if (num_boundaries != (1 << bits) - 1)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "num_boundaries %d != 2^bits - 1", num_boundaries);
  if (bytes_per_block != 32 * bits / 8)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "bytes_per_block %d != 32*bits/8", bytes_per_block);
  if (!rotated_input || !boundaries || !packed_out || !scales_out)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
  const long long nb = num_blocks;
  const dim3 grid((unsigned)((nb + 255) / 256)), block(256);
  if (bits == 2)
    hipLaunchKernelGGL((pqo_quant_rotated_dev_kernel<2>), grid, block, 0, stream, rotated_input, boundaries,
                       packed_out, scales_out, nb, outer_centroid, scale_sign);
  else if (bits == 3)
    hipLaunchKernelGGL((pqo_quant_rotated_dev_kernel<3>), grid, block, 0, stream, rotated_input, boundaries,
                       packed_out, scales_out, nb, outer_centroid, scale_sign);
  else
    hipLaunchKernelGGL((pqo_quant_rotated_dev_kernel<4>), grid, block, 0, stream, rotated_input, boundaries,
                       packed_out, scales_out, nb, outer_centroid, scale_sign);
  return tqh::check_launch("pqo_quant_rotated_dev_kernel");
}

extern "C" int tq_dequant_batch(const uint8_t *packed_indices, const uint16_t *scales, const float *codebook,
                                const float *sign_pattern, float *output, int num_blocks, int block_size, int bits,
                                int bytes_per_block, hipStream_t stream) {
  if (num_blocks == 0) return TQ_OK;  // tq_dequant_kernel.cu:116
  if (num_blocks < 0) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "num_blocks < 0");
  if (block_size != 32) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "block_size must be QUANT_BLOCK_SIZE (32), got %d", block_size);
  if (bits < 2 || bits > 4) return tqh::fail(TQ_ERR_UNSUPPORTED_BITS, "unsupported bit width %d", bits);
  if (bytes_per_block != 32 * bits / 8)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "bytes_per_block %d != 32*bits/8", bytes_per_block);
  if (!packed_indices || !scales || !codebook || !sign_pattern || !output)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
  const long long nb = num_blocks;
  const dim3 grid((unsigned)((nb + 255) / 256)), block(256);
  DequantConsts dc{};
  if (bits == 2)
    hipLaunchKernelGGL((pqo_dequant_kernel<2, kF32, true>), grid, block, 0, stream, packed_indices, scales, output,
                       nb, dc, codebook, sign_pattern);
  else if (bits == 3)
    hipLaunchKernelGGL((pqo_dequant_kernel<3, kF32, true>), grid, block, 0, stream, packed_indices, scales, output,
                       nb, dc, codebook, sign_pattern);
  else
    hipLaunchKernelGGL((pqo_dequant_kernel<4, kF32, true>), grid, block, 0, stream, packed_indices, scales, output,
                       nb, dc, codebook, sign_pattern);
  return tqh::check_launch("pqo_dequant_kernel");
}

extern "C" int tq_pack_indices(const uint8_t *indices, uint8_t *packed_out, int num_vectors, int block_size,
                               int bits, int bytes_per_block, hipStream_t stream) {
  if (num_vectors == 0) return TQ_OK;
  if (num_vectors < 0 || block_size <= 0) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "negative size");
  if (bits < 2 || bits > 4) return tqh::fail(TQ_ERR_UNSUPPORTED_BITS, "unsupported bit width %d", bits);
  if (bytes_per_block * 8 < block_size * bits)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "bytes_per_block %d too small", bytes_per_block);
  if (!indices || !packed_out) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
  const long long total = (long long)num_vectors * bytes_per_block;
  hipLaunchKernelGGL(pack_indices_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, indices,
                     packed_out, (long long)num_vectors, block_size, bits, bytes_per_block);
  return tqh::check_launch("pack_indices_kernel");
}

// ---------------------------------------------------------------------------
// Cache placement (CompressedStorage append / full dequantize)
// ---------------------------------------------------------------------------

namespace {
int cache_map(int num_heads, int tokens, int head_dim, long long head_stride, long long offset, CacheMap &m) {
  if (num_heads < 0 || tokens < 0) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "negative shape");
  if (head_dim <= 0 || head_dim % 32 != 0)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "head_dim (%d) must be divisible by QUANT_BLOCK_SIZE (32)", head_dim);
  if (offset < 0 || head_stride < offset + tokens)
    return tqh::fail(TQ_ERR_RANGE_OUT_OF_BOUNDS, "cache rows [%lld, %lld) exceed head stride %lld", offset,
                     offset + tokens, head_stride);
  if ((long long)num_heads * tokens * (head_dim / 32) >= (1ll << 31))
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "too many blocks in one call");
  m.qb_per_vec = (uint32_t)(head_dim / 32);
  m.tokens = (uint32_t)(tokens > 0 ? tokens : 1);
  m.head_stride = head_stride;
  m.offset = offset;
  return TQ_OK;
}
}  // namespace

extern "C" int tq_polar_quantize_to_cache(const void *x, int x_dtype, int num_heads, int tokens,
                                          uint8_t *packed_cache, uint16_t *scales_cache, long long cache_head_stride,
                                          long long cache_offset, int head_dim, int bits, size_t outlier_blocks,
                                          int norm_mode, hipStream_t stream) {
  int rc = check_shape(head_dim);
  if (rc) return rc;
  tqh::PolarCodec codec;
  rc = tqh::polar_codec(bits, norm_mode, outlier_blocks, head_dim / 32, codec);
  if (rc) return rc;
  if (!tqh::valid_dtype(x_dtype)) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "unknown dtype %d", x_dtype);
  CacheMap m;
  rc = cache_map(num_heads, tokens, head_dim, cache_head_stride, cache_offset, m);
  if (rc) return rc;
  const long long nblocks = (long long)num_heads * tokens * (head_dim / 32);
  if (nblocks == 0) return TQ_OK;
  if (!x || !packed_cache || !scales_cache) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
  return launch_polar_quant<true>(x, x_dtype, packed_cache, scales_cache, nblocks, codec, m, stream);
}

extern "C" int tq_polar_dequantize_from_cache(const uint8_t *packed_cache, const uint16_t *scales_cache,
                                              long long cache_head_stride, int num_heads, int tokens, void *out,
                                              int out_dtype, int head_dim, int bits, size_t outlier_blocks,
                                              int norm_mode, hipStream_t stream) {
  int rc = check_shape(head_dim);
  if (rc) return rc;
  tqh::PolarCodec codec;
  rc = tqh::polar_codec(bits, norm_mode, outlier_blocks, head_dim / 32, codec);
  if (rc) return rc;
  if (!tqh::valid_dtype(out_dtype)) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "unknown dtype %d", out_dtype);
  CacheMap m;
  rc = cache_map(num_heads, tokens, head_dim, cache_head_stride, 0, m);
  if (rc) return rc;
  const long long nblocks = (long long)num_heads * tokens * (head_dim / 32);
  if (nblocks == 0) return TQ_OK;
  if (!packed_cache || !scales_cache || !out) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
  return launch_dequant<true>(packed_cache, scales_cache, out, out_dtype, nblocks, bits, dequant_consts(codec),
                              m, stream);
}

extern "C" int tq_pqo_quantize_to_cache(const void *x, int x_dtype, int num_heads, int tokens, uint8_t *packed_cache,
                                        uint16_t *scales_cache, long long cache_head_stride, long long cache_offset,
                                        int head_dim, int bits, hipStream_t stream) {
  return tq_polar_quantize_to_cache(x, x_dtype, num_heads, tokens, packed_cache, scales_cache, cache_head_stride,
                                    cache_offset, head_dim, bits, TQ_OUTLIER_ALL, TQ_NORM_MAXNORM, stream);
}

extern "C" int tq_pqo_dequantize_from_cache(const uint8_t *packed_cache, const uint16_t *scales_cache,
                                            long long cache_head_stride, int num_heads, int tokens, void *out,
                                            int out_dtype, int head_dim, int bits, hipStream_t stream) {
  return tq_polar_dequantize_from_cache(packed_cache, scales_cache, cache_head_stride, num_heads, tokens, out,
                                        out_dtype, head_dim, bits, TQ_OUTLIER_ALL, TQ_NORM_MAXNORM, stream);
}
