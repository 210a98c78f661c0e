// tq_codec.hip -- core full-vector TurboQuant codec (quantize_vec /
// dequantize_vec / dequantize_rotated, reference src/quantize.rs:142-316),
// batched on gfx950.
//
// Design: one lane owns one vector (two adjacent lanes for d = 256, each
// holding a half), so the parts of the reference that are sequential stay
// sequential and bit-exact without cross-lane traffic: the f32 sum of
// squares runs element by element in order (quantize.rs:51-53), and the
// Walsh-Hadamard butterflies run on registers in the reference's stage
// order (rotation.rs:22-40); only the last stage of d = 256 crosses the lane
// pair (a DPP swap).  A wave covers 64 (or 32) consecutive vectors.
//
// Bucketize: the reference compares (f64)v > B_k against f64 boundaries
// (codebook/mod.rs:66-87).  For f32 v that is v >= T_k with T_k the smallest
// f32 above B_k, computed once on the host, so the kernel does f32
// compares only and produces the same codes for every input.
#include "tq_codebooks.h"
#include "tq_common.h"
#include "tq_device.h"

#include <cmath>

namespace {

using namespace tqd;

constexpr int kBlock = 256;
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
// switched off returns 0, so the move must run with both lanes of the pair
// active: the empty asm pins it before any select the compiler could turn
// into a branch.
__device__ __forceinline__ float swap_pair(float v) {
  float r = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  asm volatile("" : "+v"(r));
  return r;
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

// quantize_vec (quantize.rs:142-157) for `n` vectors of D f32.
template <int D, int BITS>
__global__ __launch_bounds__(kBlock) void codec_quant_kernel(const float *__restrict__ x, uint8_t *__restrict__ packed,
                                                             uint16_t *__restrict__ scales, long long n,
                                                             CodecConsts k) {
  using G = Geo<D>;
  constexpr int E = G::E, LPV = G::LPV, NB = (1 << BITS) - 1;
  constexpr int NW = E * BITS / 32;            // packed words per lane
  constexpr int RB = D * BITS / 8;             // packed bytes per vector
  constexpr int U = StoreUnit<E * BITS / 8>::value;
  static_assert(RB % U == 0, "row alignment");
  const long long t = (long long)blockIdx.x * kBlock + threadIdx.x;
  const long long v = t / LPV;
  const int half = (int)(t % LPV);
  if (v >= n) return;  // LPV divides kBlock, so lane pairs exit together

  float w[E];
  {
    const float4 *p = reinterpret_cast<const float4 *>(x + v * D + half * E);
#pragma unroll
    for (int q = 0; q < E / 4; q++) {
      const float4 f = p[q];
      w[4 * q] = f.x; w[4 * q + 1] = f.y; w[4 * q + 2] = f.z; w[4 * q + 3] = f.w;
    }
  }
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
  uint32_t pk[NW];
#pragma unroll
  for (int i = 0; i < NW; i++) pk[i] = 0u;
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
  store_words<NW, U>(packed + v * RB + half * (E * BITS / 8), pk);
  if (half == 0) scales[v] = f32_to_f16(norm < kMinNorm ? 0.0f : norm);
}

// dequantize_vec (quantize.rs:225-240) or, ROTATE = false, dequantize_rotated
// (quantize.rs:306-316).
template <int D, int BITS, bool ROTATE>
__global__ __launch_bounds__(kBlock) void codec_dequant_kernel(const uint8_t *__restrict__ packed,
                                                               const uint16_t *__restrict__ scales,
                                                               float *__restrict__ out, long long n, CodecConsts k) {
  using G = Geo<D>;
  constexpr int E = G::E, LPV = G::LPV;
  constexpr int NW = E * BITS / 32;
  constexpr int RB = D * BITS / 8;
  constexpr int U = StoreUnit<E * BITS / 8>::value;
  __shared__ float s_cent[16];
  if (threadIdx.x < 16) s_cent[threadIdx.x] = k.cent[threadIdx.x & ((1 << BITS) - 1)];
  __syncthreads();
  const long long t = (long long)blockIdx.x * kBlock + threadIdx.x;
  const long long v = t / LPV;
  const int half = (int)(t % LPV);
  if (v >= n) return;

  uint32_t pk[NW];
  load_words<NW, U>(packed + v * RB + half * (E * BITS / 8), pk);
  const float sc = f16_to_f32(scales[v]);
  float w[E];
#pragma unroll
  for (int e = 0; e < E; e++) {
    const int bit = e * BITS, wi = bit >> 5, sh = bit & 31;
    uint32_t idx = pk[wi] >> sh;
    if (sh + BITS > 32) idx |= pk[wi + 1] << (32 - sh);
    w[e] = s_cent[idx & ((1u << BITS) - 1u)];
  }
  if constexpr (ROTATE) {
    // Inverse rotation: WHT (with its normalization), then sign (rotation.rs:137-150)
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
  float4 *o = reinterpret_cast<float4 *>(out + v * D + half * E);
#pragma unroll
  for (int q = 0; q < E / 4; q++) o[q] = make_float4(w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3]);
}

int make_consts(int bits, int dim, uint64_t seed, CodecConsts &k) {
  if (bits < 2 || bits > 4) return tqh::fail(TQ_ERR_UNSUPPORTED_BITS, "bits must be 2, 3 or 4 (got %d)", bits);
  if (dim <= 0 || (dim & (dim - 1)) != 0)
    return tqh::fail(TQ_ERR_INVALID_DIMENSION, "dim must be a power of two (got %d)", dim);
  const double *c, *b;
  int nc;
  if (!tqh::core_codebook(bits, dim, &c, &b, &nc))
    return tqh::fail(TQ_ERR_INVALID_DIMENSION, "no codebook table for bits=%d dim=%d (tables: d = 32..256)", bits, dim);
  k = CodecConsts{};
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

template <template <int, int> class Launch, typename A>
int dispatch(int dim, int bits, const A &a) {
  switch (dim * 8 + bits) {
    case 32 * 8 + 2: return Launch<32, 2>::run(a);
    case 32 * 8 + 3: return Launch<32, 3>::run(a);
    case 32 * 8 + 4: return Launch<32, 4>::run(a);
    case 64 * 8 + 2: return Launch<64, 2>::run(a);
    case 64 * 8 + 3: return Launch<64, 3>::run(a);
    case 64 * 8 + 4: return Launch<64, 4>::run(a);
    case 128 * 8 + 2: return Launch<128, 2>::run(a);
    case 128 * 8 + 3: return Launch<128, 3>::run(a);
    case 128 * 8 + 4: return Launch<128, 4>::run(a);
    case 256 * 8 + 2: return Launch<256, 2>::run(a);
    case 256 * 8 + 3: return Launch<256, 3>::run(a);
    case 256 * 8 + 4: return Launch<256, 4>::run(a);
  }
  return tqh::fail(TQ_ERR_INVALID_DIMENSION, "unsupported dim %d", dim);
}

struct QuantArgs {
  const float *x;
  uint8_t *packed;
  uint16_t *scales;
  long long n;
  CodecConsts k;
  hipStream_t stream;
};

template <int D, int BITS>
struct QuantLaunch {
  static int run(const QuantArgs &a) {
    const long long threads = a.n * Geo<D>::LPV;
    hipLaunchKernelGGL((codec_quant_kernel<D, BITS>), dim3((unsigned)((threads + kBlock - 1) / kBlock)), dim3(kBlock),
                       0, a.stream, a.x, a.packed, a.scales, a.n, a.k);
    return tqh::check_launch("codec_quant_kernel");
  }
};

struct DequantArgs {
  const uint8_t *packed;
  const uint16_t *scales;
  float *out;
  long long n;
  CodecConsts k;
  bool rotate;
  hipStream_t stream;
};

template <int D, int BITS>
struct DequantLaunch {
  static int run(const DequantArgs &a) {
    const long long threads = a.n * Geo<D>::LPV;
    const dim3 grid((unsigned)((threads + kBlock - 1) / kBlock));
    if (a.rotate)
      hipLaunchKernelGGL((codec_dequant_kernel<D, BITS, true>), grid, dim3(kBlock), 0, a.stream, a.packed,
                         a.scales, a.out, a.n, a.k);
    else
      hipLaunchKernelGGL((codec_dequant_kernel<D, BITS, false>), grid, dim3(kBlock), 0, a.stream, a.packed,
                         a.scales, a.out, a.n, a.k);
    return tqh::check_launch("codec_dequant_kernel");
  }
};

constexpr long long kMaxVectors = (1ll << 31) / 2;  // grid.x bound with two lanes per vector

}  // namespace

extern "C" int tq_quantize_vec_batch(const float *data, uint8_t *packed_out, uint16_t *scales_out, size_t num_vectors,
                                     int bits, int dim, uint64_t rotation_seed, hipStream_t stream) {
  CodecConsts k;
  int rc = make_consts(bits, dim, rotation_seed, k);
  if (rc) return rc;
  if (num_vectors == 0) return TQ_OK;
  if ((long long)num_vectors > kMaxVectors) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "too many vectors");
  if (!data || !packed_out || !scales_out) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
  return dispatch<QuantLaunch>(dim, bits, QuantArgs{data, packed_out, scales_out, (long long)num_vectors, k, stream});
}

static int dequant_common(const uint8_t *packed, const uint16_t *scales, float *out, size_t num_vectors, int bits,
                          int dim, uint64_t seed, bool rotate, hipStream_t stream) {
  CodecConsts k;
  int rc = make_consts(bits, dim, seed, k);
  if (rc) return rc;
  if (num_vectors == 0) return TQ_OK;
  if ((long long)num_vectors > kMaxVectors) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "too many vectors");
  if (!packed || !scales || !out) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
  return dispatch<DequantLaunch>(dim, bits, DequantArgs{packed, scales, out, (long long)num_vectors, k, rotate, stream});
}

extern "C" int tq_dequantize_vec_batch(const uint8_t *packed, const uint16_t *scales, float *out, size_t num_vectors,
                                       int bits, int dim, uint64_t rotation_seed, hipStream_t stream) {
  return dequant_common(packed, scales, out, num_vectors, bits, dim, rotation_seed, true, stream);
}

extern "C" int tq_dequantize_rotated_batch(const uint8_t *packed, const uint16_t *scales, float *out,
                                           size_t num_vectors, int bits, int dim, hipStream_t stream) {
  return dequant_common(packed, scales, out, num_vectors, bits, dim, 0, false, stream);
}
