// tq_codec_dev.h -- lane-level core codec (quantize_vec / dequantize_vec,
// reference src/quantize.rs:142-316) shared by the codec and QJL kernels.
//
// One lane owns one vector (a lane pair for d = 256, each holding a half), so
// the reference's sequential parts stay sequential and bit-exact: the f32 sum
// of squares runs in element order (quantize.rs:51-53) and the Walsh-Hadamard
// butterflies run on registers in the reference's stage order
// (rotation.rs:22-40); only the last stage of d = 256 crosses the pair.
//
// Bucketize: the reference compares (f64)v > B_k against f64 boundaries
// (codebook/mod.rs:66-87).  For f32 v that is v >= T_k with T_k the smallest
// f32 above B_k (computed on the host), so the lanes do f32 compares only and
// produce the same codes for every input.
#pragma once

#include "tq_codebooks.h"
#include "tq_common.h"
#include "tq_device.h"

#include <cmath>

namespace tqd {

constexpr float kMinNorm = 1e-10f;  // MIN_NORM, quantize.rs

struct CodecConsts {
  float thr[15];      // smallest f32 T with (double)T > boundary k
  float cent[16];     // (f32) centroid k
  float wht_norm;     // fl(1 / fl(sqrt(d)))  (rotation.rs:36-39)
  float sign_even;    // sign of even elements: +1 if the rotation seed is even
};

template <int D>
struct Geo {
  static constexpr int LPV = D > 128 ? 2 : 1;  // lanes per vector
  static constexpr int E = D / LPV;            // elements per lane
};

// lane ^ 1 (DPP quad_perm [1,0,3,2]).  A DPP read from a lane that is
// switched off returns 0: call it only where both lanes of the pair are
// active (never as one arm of a conditional).
__device__ __forceinline__ float swap_pair(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
}

template <int BYTES>
struct StoreUnit {  // widest aligned store unit for a run of BYTES at a BYTES-aligned row offset
  static constexpr int value = (BYTES % 16 == 0) ? 16 : (BYTES % 8 == 0) ? 8 : 4;
};

template <int NW, int U>
__device__ __forceinline__ void store_words(uint8_t *dst, const uint32_t (&w)[NW]) {
  if constexpr (U == 16) {
#pragma unroll
    for (int k = 0; k < NW / 4; k++)
      reinterpret_cast<uint4 *>(dst)[k] = make_uint4(w[4 * k], w[4 * k + 1], w[4 * k + 2], w[4 * k + 3]);
  } else if constexpr (U == 8) {
#pragma unroll
    for (int k = 0; k < NW / 2; k++) reinterpret_cast<uint2 *>(dst)[k] = make_uint2(w[2 * k], w[2 * k + 1]);
  } else {
#pragma unroll
    for (int k = 0; k < NW; k++) reinterpret_cast<uint32_t *>(dst)[k] = w[k];
  }
}

template <int NW, int U>
__device__ __forceinline__ void load_words(const uint8_t *src, uint32_t (&w)[NW]) {
  if constexpr (U == 16) {
#pragma unroll
    for (int k = 0; k < NW / 4; k++) {
      const uint4 v = reinterpret_cast<const uint4 *>(src)[k];
      w[4 * k] = v.x; w[4 * k + 1] = v.y; w[4 * k + 2] = v.z; w[4 * k + 3] = v.w;
    }
  } else if constexpr (U == 8) {
#pragma unroll
    for (int k = 0; k < NW / 2; k++) {
      const uint2 v = reinterpret_cast<const uint2 *>(src)[k];
      w[2 * k] = v.x; w[2 * k + 1] = v.y;
    }
  } else {
#pragma unroll
    for (int k = 0; k < NW; k++) w[k] = reinterpret_cast<const uint32_t *>(src)[k];
  }
}

// Quantizes one lane's E elements of a vector (its half when LPV = 2) into
// packed words; returns the vector's L2 norm.  `w` is overwritten.
template <int E, int LPV, int BITS>
__device__ __forceinline__ float quantize_lane(float (&w)[E], int half, const CodecConsts &k,
                                               uint32_t (&pk)[E * BITS / 32]) {
  constexpr int NB = (1 << BITS) - 1;
  // l2_norm: f32 sum of squares in element order, from -0.0 (Rust's f32 sum)
  float norm;
  {
    float s = -0.0f;
#pragma unroll
    for (int e = 0; e < E; e++) s = s + w[e] * w[e];
    if constexpr (LPV == 2) {
      float s1 = swap_pair(s);  // the upper half continues from the lower half's sum
#pragma unroll
      for (int e = 0; e < E; e++) s1 = s1 + w[e] * w[e];
      const float u = swap_pair(s1);  // evaluated by both lanes of the pair
      s = half ? s1 : u;
    }
    norm = sqrtf(s);
  }
  // normalize_inplace (quantize.rs:60-71), then Forward rotation: sign, WHT
  if (norm < kMinNorm) {
#pragma unroll
    for (int e = 0; e < E; e++) w[e] = 0.0f;
  } else {
    const float inv = 1.0f / norm;
#pragma unroll
    for (int e = 0; e < E; e++) w[e] = w[e] * inv;
  }
  const float se = k.sign_even, so = -k.sign_even;  // E is even: parity of element = parity of e
#pragma unroll
  for (int e = 0; e < E; e++) w[e] = w[e] * ((e & 1) ? so : se);
  butterfly<E>(w);
  if constexpr (LPV == 2) {  // stage h = E across the pair: lower x + y, upper x - y
    const float sg = half ? -1.0f : 1.0f;
#pragma unroll
    for (int e = 0; e < E; e++) w[e] = swap_pair(w[e]) + w[e] * sg;
  }
#pragma unroll
  for (int i = 0; i < E * BITS / 32; i++) pk[i] = 0u;
#pragma unroll
  for (int e = 0; e < E; e++) {
    const float r = w[e] * k.wht_norm;
    uint32_t idx = 0;
#pragma unroll
    for (int b = 0; b < NB; b++) idx += (r >= k.thr[b]) ? 1u : 0u;
    const int bit = e * BITS, wi = bit >> 5, sh = bit & 31;
    pk[wi] |= idx << sh;
    if (sh + BITS > 32) pk[wi + 1] |= idx >> (32 - sh);
  }
  return norm;
}

// Dequantizes one lane's E elements: centroid lookup (s_cent in LDS), then,
// with ROTATE, the inverse rotation (WHT with its normalization, then sign,
// rotation.rs:137-150); finally times the f32 scale.
template <int E, int LPV, int BITS, bool ROTATE>
__device__ __forceinline__ void dequant_lane(const uint32_t (&pk)[E * BITS / 32], float sc, int half,
                                             const float *s_cent, const CodecConsts &k, float (&w)[E]) {
#pragma unroll
  for (int e = 0; e < E; e++) {
    const int bit = e * BITS, wi = bit >> 5, sh = bit & 31;
    uint32_t idx = pk[wi] >> sh;
    if (sh + BITS > 32) idx |= pk[wi + 1] << (32 - sh);
    w[e] = s_cent[idx & ((1u << BITS) - 1u)];
  }
  if constexpr (ROTATE) {
    butterfly<E>(w);
    if constexpr (LPV == 2) {
      const float sg = half ? -1.0f : 1.0f;
#pragma unroll
      for (int e = 0; e < E; e++) w[e] = swap_pair(w[e]) + w[e] * sg;
    }
    const float se = k.sign_even, so = -k.sign_even;
#pragma unroll
    for (int e = 0; e < E; e++) w[e] = (w[e] * k.wht_norm) * ((e & 1) ? so : se);
  }
#pragma unroll
  for (int e = 0; e < E; e++) w[e] = w[e] * sc;
}

}  // namespace tqd

namespace tqh {
// Host constants of a TurboQuantConfig{bits, dim, rotation_seed}; a status
// (with tq_last_error set) for a config without a codebook table.
inline int make_codec_consts(int bits, int dim, uint64_t seed, tqd::CodecConsts &k) {
  if (bits < 2 || bits > 4) return fail(TQ_ERR_UNSUPPORTED_BITS, "bits must be 2, 3 or 4 (got %d)", bits);
  if (dim <= 0 || (dim & (dim - 1)) != 0)
    return fail(TQ_ERR_INVALID_DIMENSION, "dim must be a power of two (got %d)", dim);
  const double *c, *b;
  int nc;
  if (!core_codebook(bits, dim, &c, &b, &nc))
    return fail(TQ_ERR_INVALID_DIMENSION, "no codebook table for bits=%d dim=%d (tables: d = 32..256)", bits, dim);
  k = tqd::CodecConsts{};
  for (int i = 0; i < nc; i++) k.cent[i] = (float)c[i];
  for (int i = 0; i < nc - 1; i++) {
    float t = (float)b[i];
    if (!((double)t > b[i])) t = std::nextafter(t, INFINITY);
    k.thr[i] = t;
  }
  for (int i = nc - 1; i < 15; i++) k.thr[i] = INFINITY;
  volatile float fd = (float)dim;
  volatile float sq = sqrtf(fd);
  k.wht_norm = 1.0f / sq;
  k.sign_even = (seed & 1u) ? -1.0f : 1.0f;  // generate_sign_pattern, rotation.rs:47-70
  return TQ_OK;
}
}  // namespace tqh
