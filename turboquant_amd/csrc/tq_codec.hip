// tq_codec.hip -- core full-vector TurboQuant codec kernels (quantize_vec /
// dequantize_vec / dequantize_rotated, reference src/quantize.rs:142-316),
// batched on gfx950: one lane per vector (a lane pair for d = 256), see
// tq_codec_dev.h.  A wave covers 64 (or 32) consecutive vectors.
#include "tq_codec_dev.h"

namespace {

using namespace tqd;

constexpr int kBlock = 256;

// quantize_vec (quantize.rs:142-157) for `n` vectors of D f32.
template <int D, int BITS>
__global__ __launch_bounds__(kBlock) void codec_quant_kernel(const float *__restrict__ x, uint8_t *__restrict__ packed,
                                                             uint16_t *__restrict__ scales, long long n,
                                                             CodecConsts k) {
  using G = Geo<D>;
  constexpr int E = G::E, LPV = G::LPV;
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
  uint32_t pk[NW];
  const float norm = quantize_lane<E, LPV, BITS>(w, half, k, pk);
  store_words<NW, U>(packed + v * RB + half * (E * BITS / 8), pk);
  if (half == 0) scales[v] = f32_to_f16(norm < kMinNorm ? 0.0f : norm);  // select_scale, quantize.rs:123-126
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
  float w[E];
  dequant_lane<E, LPV, BITS, ROTATE>(pk, f16_to_f32(scales[v]), half, s_cent, k, w);
  float4 *o = reinterpret_cast<float4 *>(out + v * D + half * E);
#pragma unroll
  for (int q = 0; q < E / 4; q++) o[q] = make_float4(w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3]);
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
  int rc = tqh::make_codec_consts(bits, dim, rotation_seed, k);
  if (rc) return rc;
  if (num_vectors == 0) return TQ_OK;
  if ((long long)num_vectors > kMaxVectors) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "too many vectors");
  if (!data || !packed_out || !scales_out) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
  return dispatch<QuantLaunch>(dim, bits, QuantArgs{data, packed_out, scales_out, (long long)num_vectors, k, stream});
}

static int dequant_common(const uint8_t *packed, const uint16_t *scales, float *out, size_t num_vectors, int bits,
                          int dim, uint64_t seed, bool rotate, hipStream_t stream) {
  CodecConsts k;
  int rc = tqh::make_codec_consts(bits, dim, seed, k);
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
