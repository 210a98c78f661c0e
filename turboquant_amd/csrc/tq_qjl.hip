// tq_qjl.hip -- QJL inner-product estimator (reference src/qjl.rs,
// src/attention.rs) on gfx950: key quantization with the 1-bit sign sketch,
// query projections, batched score estimation, softmax and weighted values.
//
// The Rademacher matrix R[j][c] = sign(j, c) / sqrt(d) is implicit in the
// reference (a SplitMix64 hash per entry, qjl.rs:143-189).  Each workgroup
// hashes the d x d sign bits it needs into LDS once; a lane then forms a row
// product as d fused multiply-adds with a wave-uniform +-1 factor, which is
// exactly the reference's sequential sum of sign * value (the product is
// exact, so fma(sign, v, s) == fl(s + sign * v)).
//
// Scores use the rotated domain: <q, x_mse> = scale * <qt, c[idx]> with
// qt = H(s * q) / sqrt(d), the forward rotation of the query, so keys are
// never inverse-rotated.  Per block of queries the workgroup builds LDS
// tables of qt-pair x centroid-pair products and of +-rq nibble sums, so a
// score is one table read per two key elements plus one per four sign bits.
#include "tq_codec_dev.h"

#include <type_traits>

namespace {

using namespace tqd;

constexpr int kBlock = 256;
constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;

// qjl.rs:143-147
__device__ __forceinline__ uint64_t mix_seed(uint64_t seed, uint64_t row) {
  const uint64_t m = seed * 0x517CC1B727220A95ull + row;
  return m ^ (m >> 32) ^ 0x6C62272E07BB0142ull;
}

// qjl.rs:157-171: true where sign(row, col) = -1 (SplitMix64 finalizer odd)
__device__ __forceinline__ bool sign_negative(uint64_t row_seed, uint64_t row, uint64_t col) {
  uint64_t z = row_seed + row * kGolden + col;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z ^= z >> 31;
  return (z & 1u) != 0;
}

// Fills s_bits[j * D/32 + w] (bit b = sign(j, 32w + b) is -1) for all rows.
template <int D>
__device__ void build_sign_bits(uint32_t *s_bits, uint64_t seed) {
  for (int it = threadIdx.x; it < D * D / 32; it += blockDim.x) {
    const int j = it / (D / 32), w = it % (D / 32);
    const uint64_t rs = mix_seed(seed, (uint64_t)j);
    uint32_t bits = 0;
    for (int b = 0; b < 32; b++) bits |= (sign_negative(rs, (uint64_t)j, (uint64_t)(32 * w + b)) ? 1u : 0u) << b;
    s_bits[it] = bits;
  }
}

// rademacher_vector_product (qjl.rs:196-208): (sum_c sign(j,c) * v[c]) * inv,
// summed in column order from -0.0.
template <int D>
__device__ __forceinline__ float row_product(const float (&v)[D], const uint32_t *row_bits, float inv) {
  float s = -0.0f;
#pragma unroll
  for (int w = 0; w < D / 32; w++) {
    const uint32_t bits = __builtin_amdgcn_readfirstlane(row_bits[w]);
#pragma unroll
    for (int b = 0; b < 32; b++) s = __builtin_fmaf(((bits >> b) & 1u) ? -1.0f : 1.0f, v[32 * w + b], s);
  }
  return s * inv;
}

struct QjlConsts {
  CodecConsts polar;   // (total_bits - 1)-bit codec of the same dimension
  uint64_t qjl_seed;
  float inv_sqrt_d;    // fl(1 / fl(sqrt(d)))
  float sqrt_d;        // fl(sqrt(d))
};

// quantize_with_qjl (qjl.rs:355-377) per key, lane = key.
template <int D, int PB>
__global__ __launch_bounds__(kBlock) void qjl_quant_kernel(const float *__restrict__ x, uint8_t *__restrict__ polar,
                                                           uint16_t *__restrict__ polar_scales,
                                                           uint32_t *__restrict__ signs,
                                                           uint16_t *__restrict__ residual_norms, long long n,
                                                           QjlConsts k) {
  constexpr int NW = D * PB / 32;
  constexpr int U = StoreUnit<D * PB / 8>::value;
  __shared__ uint32_t s_bits[D * D / 32];
  __shared__ float s_cent[16];
  build_sign_bits<D>(s_bits, k.qjl_seed);
  if (threadIdx.x < 16) s_cent[threadIdx.x] = k.polar.cent[threadIdx.x & ((1 << PB) - 1)];
  __syncthreads();
  const long long v = (long long)blockIdx.x * kBlock + threadIdx.x;
  if (v >= n) return;
  const float4 *xp = reinterpret_cast<const float4 *>(x + v * D);
  float w[D];
#pragma unroll
  for (int q = 0; q < D / 4; q++) {
    const float4 f = xp[q];
    w[4 * q] = f.x; w[4 * q + 1] = f.y; w[4 * q + 2] = f.z; w[4 * q + 3] = f.w;
  }
  uint32_t pk[NW];
  const float norm = quantize_lane<D, 1, PB>(w, 0, k.polar, pk);
  const uint16_t sc = f32_to_f16(norm < kMinNorm ? 0.0f : norm);
  // x_mse = dequantize_vec(polar block), residual r = x - x_mse (qjl.rs:362-368)
  dequant_lane<D, 1, PB, true>(pk, f16_to_f32(sc), 0, s_cent, k.polar, w);
#pragma unroll
  for (int q = 0; q < D / 4; q++) {
    const float4 f = xp[q];
    w[4 * q] = f.x - w[4 * q]; w[4 * q + 1] = f.y - w[4 * q + 1];
    w[4 * q + 2] = f.z - w[4 * q + 2]; w[4 * q + 3] = f.w - w[4 * q + 3];
  }
  float rs = -0.0f;
#pragma unroll
  for (int e = 0; e < D; e++) rs = rs + w[e] * w[e];
  const float rn = sqrtf(rs);
  // compute_qjl_signs + pack_sign_bits (qjl.rs:305-319, 245-256): bit j = p_j >= 0
  uint32_t sw[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; i++) sw[i] = 0u;
  for (int j = 0; j < D; j++) {
    const float p = row_product<D>(w, s_bits + j * (D / 32), k.inv_sqrt_d);
    const uint32_t bit = (p >= 0.0f) ? 1u : 0u;
#pragma unroll
    for (int i = 0; i < D / 32; i++) sw[i] |= (i == (j >> 5)) ? (bit << (j & 31)) : 0u;
  }
  store_words<NW, U>(polar + v * (D * PB / 8), pk);
  polar_scales[v] = sc;
#pragma unroll
  for (int i = 0; i < D / 32; i++) signs[v * (D / 32) + i] = sw[i];
  residual_norms[v] = f32_to_f16(rn);
}

// EstimationContext for a batch of queries (qjl.rs:488-492, 561-572):
// ctx[q] = { qt[D] = forward rotation of q (no normalization), rq[D] = R q }.
template <int D>
__global__ __launch_bounds__(kBlock) void qjl_query_kernel(const float *__restrict__ queries, float *__restrict__ ctx,
                                                           long long nq, QjlConsts k) {
  __shared__ uint32_t s_bits[D * D / 32];
  build_sign_bits<D>(s_bits, k.qjl_seed);
  __syncthreads();
  const long long qi = (long long)blockIdx.x * kBlock + threadIdx.x;
  if (qi >= nq) return;
  float q[D];
  const float4 *qp = reinterpret_cast<const float4 *>(queries + qi * D);
#pragma unroll
  for (int i = 0; i < D / 4; i++) {
    const float4 f = qp[i];
    q[4 * i] = f.x; q[4 * i + 1] = f.y; q[4 * i + 2] = f.z; q[4 * i + 3] = f.w;
  }
  float *out = ctx + qi * 2 * D;
  for (int j = 0; j < D; j++) out[D + j] = row_product<D>(q, s_bits + j * (D / 32), k.inv_sqrt_d);
  const float se = k.polar.sign_even, so = -k.polar.sign_even;
#pragma unroll
  for (int e = 0; e < D; e++) q[e] = q[e] * ((e & 1) ? so : se);
  butterfly<D>(q);
#pragma unroll
  for (int e = 0; e < D; e++) out[e] = q[e] * k.polar.wht_norm;
}

// Scores of QB queries x 256 keys per workgroup (lane = key):
//   est = scale_k * sum_i qt_i c[idx_i] + c_k * sum_j rq_j (2 b_j - 1),
//   c_k = |r_k| * sqrt(pi/2) / sqrt(d)   (qjl.rs:263-265, 512-519, 585-606).
template <int D, int PB, int QB>
__global__ __launch_bounds__(kBlock) void qjl_scores_kernel(const float *__restrict__ ctx, long long nq,
                                                            const uint8_t *__restrict__ polar,
                                                            const uint16_t *__restrict__ polar_scales,
                                                            const uint32_t *__restrict__ signs,
                                                            const uint16_t *__restrict__ residual_norms, long long nk,
                                                            float *__restrict__ scores, QjlConsts k) {
  constexpr int PE = 1 << (2 * PB);        // entries per pair table
  constexpr int BT = (D / 2) * PE;         // pair tables per query
  constexpr int CT = (D / 4) * 16;         // sign-nibble tables per query
  constexpr int NW = D * PB / 32;
  constexpr int U = StoreUnit<D * PB / 8>::value;
  __shared__ float s_tab[QB * (BT + CT)];
  __shared__ float s_cent[16];
  if (threadIdx.x < 16) s_cent[threadIdx.x] = k.polar.cent[threadIdx.x & ((1 << PB) - 1)];
  __syncthreads();
  const long long q0 = (long long)blockIdx.y * QB;
  const int nql = (int)min<long long>(QB, nq - q0);
  // tables: pair (g, code) -> qt[2g] c[lo] + qt[2g+1] c[hi]; nibble (c, m) -> sum_b rq[4c+b] (m_b ? 1 : -1)
  for (int e = threadIdx.x; e < nql * (BT + CT); e += kBlock) {
    const int ql = e / (BT + CT), r = e % (BT + CT);
    const float *cq = ctx + (q0 + ql) * 2 * D;
    float val;
    if (r < BT) {
      const int g = r / PE, code = r % PE;
      val = cq[2 * g] * s_cent[code & ((1 << PB) - 1)] + cq[2 * g + 1] * s_cent[code >> PB];
    } else {
      const int c = (r - BT) / 16, m = (r - BT) % 16;
      const float *rq = cq + D + 4 * c;
      val = -0.0f;
#pragma unroll
      for (int b = 0; b < 4; b++) val = val + ((m >> b) & 1 ? rq[b] : -rq[b]);
    }
    s_tab[e] = val;
  }
  __syncthreads();
  const long long key = (long long)blockIdx.x * kBlock + threadIdx.x;
  if (key >= nk) return;
  uint32_t pk[NW], sg[D / 32];
  load_words<NW, U>(polar + key * (D * PB / 8), pk);
#pragma unroll
  for (int i = 0; i < D / 32; i++) sg[i] = signs[key * (D / 32) + i];
  const float scale = f16_to_f32(polar_scales[key]);
  const float ck = (f16_to_f32(residual_norms[key]) * 1.2533141f) / k.sqrt_d;
  for (int ql = 0; ql < nql; ql++) {
    const float *tb = s_tab + ql * (BT + CT);
    float base = 0.0f, corr = 0.0f;
#pragma unroll
    for (int g = 0; g < D / 2; g++) {
      const int bit = 2 * g * PB, wi = bit >> 5, sh = bit & 31;
      uint32_t code = pk[wi] >> sh;
      if (sh + 2 * PB > 32) code |= pk[wi + 1] << (32 - sh);
      base += tb[g * PE + (code & (PE - 1))];
    }
#pragma unroll
    for (int c = 0; c < D / 4; c++) corr += tb[BT + c * 16 + ((sg[c >> 3] >> ((c & 7) * 4)) & 15u)];
    scores[(q0 + ql) * nk + key] = scale * base + ck * corr;
  }
}

// Row softmax: probs = exp(scale * (s - max)) / sum (textbook; the reference
// returns raw scores, attention.rs:344-352).
__global__ __launch_bounds__(kBlock) void softmax_rows_kernel(const float *__restrict__ s, float *__restrict__ p,
                                                              long long cols, float scale) {
  __shared__ float red[kBlock / 64];
  const float *row = s + (long long)blockIdx.x * cols;
  float *out = p + (long long)blockIdx.x * cols;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float m = -INFINITY;
  for (long long c = threadIdx.x; c < cols; c += kBlock) m = fmaxf(m, row[c]);
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  if (lane == 0) red[wave] = m;
  __syncthreads();
  m = red[0];
  for (int w = 1; w < kBlock / 64; w++) m = fmaxf(m, red[w]);
  __syncthreads();
  float sum = 0.0f;
  for (long long c = threadIdx.x; c < cols; c += kBlock) sum += expf(scale * (row[c] - m));
  for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
  if (lane == 0) red[wave] = sum;
  __syncthreads();
  sum = 0.0f;
  for (int w = 0; w < kBlock / 64; w++) sum += red[w];
  const float inv = 1.0f / sum;
  for (long long c = threadIdx.x; c < cols; c += kBlock) out[c] = expf(scale * (row[c] - m)) * inv;
}

// weighted_values (attention.rs:371-408), rotated domain: a workgroup of D
// lanes (lane = element) accumulates sum_t w_t scale_t c[idx_t,e] over one
// chunk of values for one query; the finish kernel adds the chunks and
// applies the inverse rotation once.
constexpr int kWvChunk = 256;

template <int D, int PB>
__global__ __launch_bounds__(D) void qjl_wv_partial_kernel(const uint8_t *__restrict__ polar,
                                                           const uint16_t *__restrict__ polar_scales, long long nv,
                                                           const float *__restrict__ weights,
                                                           float *__restrict__ partial, QjlConsts k) {
  constexpr int RWORDS = D * PB / 32;  // packed words per value
  __shared__ uint32_t s_codes[kWvChunk * RWORDS];
  __shared__ float s_w[kWvChunk];
  __shared__ float s_cent[16];
  if (threadIdx.x < 16) s_cent[threadIdx.x] = k.polar.cent[threadIdx.x & ((1 << PB) - 1)];
  const long long t0 = (long long)blockIdx.x * kWvChunk;
  const long long qi = blockIdx.y;
  const int cnt = (int)min<long long>(kWvChunk, nv - t0);
  for (int i = threadIdx.x; i < cnt * RWORDS; i += D)
    s_codes[i] = reinterpret_cast<const uint32_t *>(polar + t0 * (D * PB / 8))[i];
  for (int i = threadIdx.x; i < cnt; i += D)
    s_w[i] = weights[qi * nv + t0 + i] * f16_to_f32(polar_scales[t0 + i]);
  __syncthreads();
  const int e = threadIdx.x;
  const int bit = e * PB, wi = bit >> 5, sh = bit & 31;
  float acc = 0.0f;
  for (int t = 0; t < cnt; t++) {
    const uint32_t *row = s_codes + t * RWORDS;
    uint32_t code = row[wi] >> sh;
    if (sh + PB > 32) code |= row[wi + 1] << (32 - sh);
    acc = __builtin_fmaf(s_w[t], s_cent[code & ((1u << PB) - 1u)], acc);
  }
  partial[(qi * gridDim.x + blockIdx.x) * D + e] = acc;
}

template <int D>
__global__ __launch_bounds__(kBlock) void qjl_wv_finish_kernel(const float *__restrict__ partial, int nchunks,
                                                               float *__restrict__ out, long long nq, QjlConsts k) {
  const long long qi = (long long)blockIdx.x * kBlock + threadIdx.x;
  if (qi >= nq) return;
  float a[D];
#pragma unroll
  for (int e = 0; e < D; e++) a[e] = 0.0f;
  for (int c = 0; c < nchunks; c++) {
    const float *p = partial + (qi * nchunks + c) * D;
#pragma unroll
    for (int e = 0; e < D; e++) a[e] += p[e];
  }
  butterfly<D>(a);
  const float se = k.polar.sign_even, so = -k.polar.sign_even;
#pragma unroll
  for (int e = 0; e < D; e++) out[qi * D + e] = (a[e] * k.polar.wht_norm) * ((e & 1) ? so : se);
}

int qjl_consts(int polar_bits, int dim, uint64_t rot_seed, uint64_t qjl_seed, QjlConsts &k) {
  if (dim != 32 && dim != 64 && dim != 128)
    return tqh::fail(TQ_ERR_INVALID_DIMENSION, "QJL kernels take dim 32, 64 or 128 (got %d)", dim);
  if (polar_bits != 2 && polar_bits != 3)
    return tqh::fail(TQ_ERR_UNSUPPORTED_BITS, "QJL total bits must be 3 or 4 (polar bits %d)", polar_bits);
  int rc = tqh::make_codec_consts(polar_bits, dim, rot_seed, k.polar);
  if (rc) return rc;
  k.qjl_seed = qjl_seed;
  volatile float fd = (float)dim;
  volatile float sq = sqrtf(fd);
  k.sqrt_d = sq;
  k.inv_sqrt_d = 1.0f / sq;
  return TQ_OK;
}

template <typename F>
int by_dim(int dim, F &&f) {
  switch (dim) {
    case 32: return f(std::integral_constant<int, 32>{});
    case 64: return f(std::integral_constant<int, 64>{});
    case 128: return f(std::integral_constant<int, 128>{});
  }
  return tqh::fail(TQ_ERR_INVALID_DIMENSION, "unsupported dim %d", dim);
}

template <typename F>
int by_dim_bits(int dim, int pb, F &&f) {
  return by_dim(dim, [&](auto d) {
    if (pb == 2) return f(d, std::integral_constant<int, 2>{});
    return f(d, std::integral_constant<int, 3>{});
  });
}

unsigned grid_for(long long n) { return (unsigned)((n + kBlock - 1) / kBlock); }

}  // namespace

extern "C" int tq_qjl_quantize_batch(const float *data, uint8_t *polar_packed, uint16_t *polar_scales,
                                     uint8_t *signs, uint16_t *residual_norms, size_t num_vectors, int total_bits,
                                     int dim, uint64_t rotation_seed, uint64_t qjl_seed, hipStream_t stream) {
  if (total_bits != 3 && total_bits != 4)
    return tqh::fail(TQ_ERR_UNSUPPORTED_BITS, "QJL total bits must be 3 or 4 (got %d)", total_bits);
  QjlConsts k;
  int rc = qjl_consts(total_bits - 1, dim, rotation_seed, qjl_seed, k);
  if (rc) return rc;
  if (num_vectors == 0) return TQ_OK;
  if (!data || !polar_packed || !polar_scales || !signs || !residual_norms)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
  const long long n = (long long)num_vectors;
  return by_dim_bits(dim, total_bits - 1, [&](auto d, auto pb) {
    hipLaunchKernelGGL((qjl_quant_kernel<decltype(d)::value, decltype(pb)::value>), dim3(grid_for(n)), dim3(kBlock),
                       0, stream, data, polar_packed, polar_scales, reinterpret_cast<uint32_t *>(signs),
                       residual_norms, n, k);
    return tqh::check_launch("qjl_quant_kernel");
  });
}

extern "C" int tq_qjl_query_context(const float *queries, float *ctx_out, size_t num_queries, int dim,
                                    uint64_t rotation_seed, uint64_t qjl_seed, hipStream_t stream) {
  QjlConsts k;
  int rc = qjl_consts(2, dim, rotation_seed, qjl_seed, k);
  if (rc) return rc;
  if (num_queries == 0) return TQ_OK;
  if (!queries || !ctx_out) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
  const long long nq = (long long)num_queries;
  return by_dim(dim, [&](auto d) {
    hipLaunchKernelGGL((qjl_query_kernel<decltype(d)::value>), dim3(grid_for(nq)), dim3(kBlock), 0, stream, queries,
                       ctx_out, nq, k);
    return tqh::check_launch("qjl_query_kernel");
  });
}

extern "C" int tq_qjl_scores(const float *ctx, size_t num_queries, const uint8_t *polar_packed,
                             const uint16_t *polar_scales, const uint8_t *signs, const uint16_t *residual_norms,
                             size_t num_keys, int polar_bits, int dim, uint64_t rotation_seed, float *scores,
                             hipStream_t stream) {
  QjlConsts k;
  int rc = qjl_consts(polar_bits, dim, rotation_seed, 0, k);
  if (rc) return rc;
  if (num_queries == 0 || num_keys == 0) return TQ_OK;
  if (!ctx || !polar_packed || !polar_scales || !signs || !residual_norms || !scores)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
  const long long nq = (long long)num_queries, nk = (long long)num_keys;
  return by_dim_bits(dim, polar_bits, [&](auto d, auto pb) {
    constexpr int D = decltype(d)::value, PB = decltype(pb)::value;
    constexpr int QB = PB == 2 ? 8 : 2;
    hipLaunchKernelGGL((qjl_scores_kernel<D, PB, QB>), dim3(grid_for(nk), (unsigned)((nq + QB - 1) / QB)),
                       dim3(kBlock), 0, stream, ctx, nq, polar_packed, polar_scales,
                       reinterpret_cast<const uint32_t *>(signs), residual_norms, nk, scores, k);
    return tqh::check_launch("qjl_scores_kernel");
  });
}

extern "C" int tq_softmax_rows(const float *scores, float *probs, size_t rows, size_t cols, float scale,
                               hipStream_t stream) {
  if (rows == 0 || cols == 0) return TQ_OK;
  if (!scores || !probs) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
  if (rows > 0x7fffffffu) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "too many rows");
  hipLaunchKernelGGL(softmax_rows_kernel, dim3((unsigned)rows), dim3(kBlock), 0, stream, scores, probs,
                     (long long)cols, scale);
  return tqh::check_launch("softmax_rows_kernel");
}

extern "C" size_t tq_qjl_weighted_values_workspace_size(size_t num_queries, size_t num_values, int dim) {
  if (dim <= 0) return 0;
  const size_t chunks = (num_values + kWvChunk - 1) / kWvChunk;
  return num_queries * chunks * (size_t)dim * sizeof(float);
}

extern "C" int tq_qjl_weighted_values(const uint8_t *polar_packed, const uint16_t *polar_scales, size_t num_values,
                                      const float *weights, size_t num_queries, int polar_bits, int dim,
                                      uint64_t rotation_seed, float *out, void *workspace, size_t workspace_bytes,
                                      hipStream_t stream) {
  QjlConsts k;
  int rc = qjl_consts(polar_bits, dim, rotation_seed, 0, k);
  if (rc) return rc;
  if (num_queries == 0) return TQ_OK;
  if (!out || (num_values && (!polar_packed || !polar_scales || !weights)))
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
  const size_t need = tq_qjl_weighted_values_workspace_size(num_queries, num_values, dim);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "workspace too small: %zu < %zu", workspace_bytes, need);
  const long long nv = (long long)num_values, nq = (long long)num_queries;
  const int nchunks = (int)((nv + kWvChunk - 1) / kWvChunk);
  if (nq > 65535) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "too many queries (%lld > 65535)", nq);
  float *partial = static_cast<float *>(workspace);
  return by_dim_bits(dim, polar_bits, [&](auto d, auto pb) {
    constexpr int D = decltype(d)::value, PB = decltype(pb)::value;
    if (nchunks > 0) {
      hipLaunchKernelGGL((qjl_wv_partial_kernel<D, PB>), dim3((unsigned)nchunks, (unsigned)nq), dim3(D), 0, stream,
                         polar_packed, polar_scales, nv, weights, partial, k);
      int rc2 = tqh::check_launch("qjl_wv_partial_kernel");
      if (rc2) return rc2;
    }
    hipLaunchKernelGGL((qjl_wv_finish_kernel<D>), dim3(grid_for(nq)), dim3(kBlock), 0, stream, partial, nchunks, out,
                       nq, k);
    return tqh::check_launch("qjl_wv_finish_kernel");
  });
}
