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
#include "tq_mfma.h"

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

// +-1 for the four sign bits of a nibble (bit i set <=> element i negative)
__device__ __forceinline__ float4 nibble_signs(int nib) {
  return make_float4((nib & 1) ? -1.0f : 1.0f, (nib & 2) ? -1.0f : 1.0f, (nib & 4) ? -1.0f : 1.0f,
                     (nib & 8) ? -1.0f : 1.0f);
}

// quantize_with_qjl (qjl.rs:355-377) for KB = 32 keys per workgroup.  One lane
// of each group of 8 quantizes its key (polar codes, scale, residual r = x -
// dequantized x, |r|) and stages r in LDS; then the 8 lanes of the key share
// its D sign projections, D / 8 rows each.  A row is summed in column order
// from -0.0 exactly as rademacher_vector_product (qjl.rs:196-208): the signs
// of four columns come from one table read by the nibble of the row's bits,
// and fma(+-1, r_c, s) is the reference's fl(s + sign * r_c).  Four rows at a
// time keep four independent sums in flight.
template <int D, int PB>
__global__ __launch_bounds__(kBlock) void qjl_quant_kernel(const float *__restrict__ x, uint8_t *__restrict__ polar,
                                                           uint16_t *__restrict__ polar_scales,
                                                           uint32_t *__restrict__ signs,
                                                           uint16_t *__restrict__ residual_norms, long long n,
                                                           QjlConsts k) {
  constexpr int LPK = 8, KB = kBlock / LPK, RPL = D / LPK, RI = RPL < 4 ? RPL : 4;
  constexpr int NW = D * PB / 32;
  constexpr int U = StoreUnit<D * PB / 8>::value;
  constexpr int RS = D + 4;  // residual row stride (floats): rows of different keys in different banks
  __shared__ uint32_t s_bits[D * D / 32];
  __shared__ float s_cent[16];
  __shared__ __attribute__((aligned(16))) float s_res[KB * RS];
  __shared__ __attribute__((aligned(16))) float4 s_sgn[16];
  __shared__ uint32_t s_sw[KB * (D / 32)];
  build_sign_bits<D>(s_bits, k.qjl_seed);
  const int tid = threadIdx.x, kk = tid / LPK, rq = tid % LPK;
  if (tid < 16) {
    s_cent[tid] = k.polar.cent[tid & ((1 << PB) - 1)];
    s_sgn[tid] = nibble_signs(tid);
  }
  for (int e = tid; e < KB * (D / 32); e += kBlock) s_sw[e] = 0u;
  __syncthreads();
  const long long v = (long long)blockIdx.x * KB + kk;
  const bool live = v < n;
  if (rq == 0 && live) {
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
#pragma unroll
    for (int q = 0; q < D / 4; q++)
      *reinterpret_cast<float4 *>(s_res + kk * RS + 4 * q) = make_float4(w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3]);
    store_words<NW, U>(polar + v * (D * PB / 8), pk);
    polar_scales[v] = sc;
    residual_norms[v] = f32_to_f16(sqrtf(rs));
  }
  __syncthreads();
  // compute_qjl_signs + pack_sign_bits (qjl.rs:305-319, 245-256): bit j = p_j >= 0
  if (live) {
    const float4 *res = reinterpret_cast<const float4 *>(s_res + kk * RS);
    uint32_t mine = 0u;  // bits of rows rq * RPL .. + RPL, at their place in the row's word
#pragma unroll
    for (int r0 = 0; r0 < RPL; r0 += RI) {
      const int j0 = rq * RPL + r0;
      float sum[RI];
#pragma unroll
      for (int i = 0; i < RI; i++) sum[i] = -0.0f;
#pragma unroll
      for (int w = 0; w < D / 32; w++) {
        uint32_t bw[RI];
#pragma unroll
        for (int i = 0; i < RI; i++) bw[i] = s_bits[(j0 + i) * (D / 32) + w];
#pragma unroll
        for (int nb = 0; nb < 8; nb++) {
          const float4 rv = res[8 * w + nb];
#pragma unroll
          for (int i = 0; i < RI; i++) {
            const float4 sg = s_sgn[(bw[i] >> (4 * nb)) & 15u];
            sum[i] = __builtin_fmaf(sg.x, rv.x, sum[i]);
            sum[i] = __builtin_fmaf(sg.y, rv.y, sum[i]);
            sum[i] = __builtin_fmaf(sg.z, rv.z, sum[i]);
            sum[i] = __builtin_fmaf(sg.w, rv.w, sum[i]);
          }
        }
      }
#pragma unroll
      for (int i = 0; i < RI; i++) {
        const float p = sum[i] * k.inv_sqrt_d;
        mine |= (p >= 0.0f ? 1u : 0u) << ((j0 + i) & 31);
      }
    }
    if (mine) atomicOr(&s_sw[kk * (D / 32) + (rq * RPL) / 32], mine);
  }
  __syncthreads();
  if (live && rq < D / 32) signs[v * (D / 32) + rq] = s_sw[kk * (D / 32) + rq];
}

// EstimationContext for a batch of queries (qjl.rs:488-492, 561-572):
// ctx[q] = { qt[D] = forward rotation of q (no normalization), rq[D] = R q }.
// A workgroup serves 8 queries x 32 projection rows, lane = (query, row): it
// hashes only its rows' sign bits; each lane sums its row in column order
// from -0.0 (rademacher_vector_product, qjl.rs:196-208).  The workgroups of
// the first row block also rotate their queries (one lane per query).
template <int D>
__global__ __launch_bounds__(kBlock) void qjl_query_kernel(const float *__restrict__ queries, float *__restrict__ ctx,
                                                           long long nq, QjlConsts k) {
  constexpr int RB = 32, QB = kBlock / RB;
  __shared__ uint32_t s_bits[RB * (D / 32)];
  __shared__ __attribute__((aligned(16))) float s_q[QB * D];
  __shared__ __attribute__((aligned(16))) float4 s_sgn[16];
  const int tid = threadIdx.x, qq = tid / RB, jj = tid % RB;
  if (tid < 16) s_sgn[tid] = nibble_signs(tid);
  const int jb = blockIdx.x * RB;
  const long long q0 = (long long)blockIdx.y * QB;
  // one sign per lane, 64 consecutive (row, column) entries per wave and step,
  // gathered into two words by a ballot
  for (int base = (tid >> 6) * 64; base < RB * D; base += kBlock) {
    const int f = base + (tid & 63), j = jb + f / D, col = f % D;
    const uint64_t m = __ballot(sign_negative(mix_seed(k.qjl_seed, (uint64_t)j), (uint64_t)j, (uint64_t)col));
    if ((tid & 63) == 0) {
      s_bits[base / 32] = (uint32_t)m;
      s_bits[base / 32 + 1] = (uint32_t)(m >> 32);
    }
  }
  for (int e = tid; e < QB * D; e += kBlock) {
    const long long qi = q0 + e / D;
    s_q[e] = qi < nq ? queries[qi * D + e % D] : 0.0f;
  }
  __syncthreads();
  const long long qi = q0 + qq;
  if (qi >= nq) return;
  const float *qv = s_q + qq * D;
  float s = -0.0f;
#pragma unroll
  for (int w = 0; w < D / 32; w++) {
    const uint32_t bits = s_bits[jj * (D / 32) + w];
#pragma unroll
    for (int nb = 0; nb < 8; nb++) {  // the signs of four columns by one table read
      const float4 sg = s_sgn[(bits >> (4 * nb)) & 15u];
      const float4 v = *reinterpret_cast<const float4 *>(qv + 32 * w + 4 * nb);
      s = __builtin_fmaf(sg.x, v.x, s);
      s = __builtin_fmaf(sg.y, v.y, s);
      s = __builtin_fmaf(sg.z, v.z, s);
      s = __builtin_fmaf(sg.w, v.w, s);
    }
  }
  float *out = ctx + qi * 2 * D;
  out[D + jb + jj] = s * k.inv_sqrt_d;
  if (blockIdx.x == 0) {
    // forward rotation, the query's 32 lanes holding E = D / 32 consecutive
    // elements each: butterfly stages h < E inside a lane, h >= E with the
    // lane jj ^ (h / E) (the lower element takes x + y, the upper x - y, in
    // the stage order of butterfly<D>, so every value is the same)
    constexpr int E = D / 32;
    const float se = k.polar.sign_even, so = -k.polar.sign_even;
    float q[E];
#pragma unroll
    for (int i = 0; i < E; i++) q[i] = qv[E * jj + i] * (((E * jj + i) & 1) ? so : se);
#pragma unroll
    for (int h = 1; h < E; h *= 2)
#pragma unroll
      for (int i = 0; i < E; i += 2 * h)
#pragma unroll
        for (int t = i; t < i + h; t++) {
          const float x = q[t], y = q[t + h];
          q[t] = x + y;
          q[t + h] = x - y;
        }
    auto cross = [&](auto xc) {
      constexpr int X = decltype(xc)::value;
      const bool upper = (jj & X) != 0;
#pragma unroll
      for (int i = 0; i < E; i++) {
        const float o = tqm::lane_xor<X>(q[i]);
        q[i] = upper ? o - q[i] : q[i] + o;
      }
    };
    cross(std::integral_constant<int, 1>{});
    cross(std::integral_constant<int, 2>{});
    cross(std::integral_constant<int, 4>{});
    cross(std::integral_constant<int, 8>{});
    cross(std::integral_constant<int, 16>{});
#pragma unroll
    for (int i = 0; i < E; i++) out[E * jj + i] = q[i] * k.polar.wht_norm;
  }
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
constexpr int kSoftmaxBlock = 1024;
// One workgroup per row: the max, then each exponential once (kept in the
// output) and their sum, then the scaling in place.
__global__ __launch_bounds__(kSoftmaxBlock) void softmax_rows_kernel(const float *__restrict__ s,
                                                                     float *__restrict__ p, long long cols,
                                                                     float scale) {
  __shared__ float red[kSoftmaxBlock / 64];
  const float *row = s + (long long)blockIdx.x * cols;
  float *out = p + (long long)blockIdx.x * cols;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float m = -INFINITY;
  for (long long c = threadIdx.x; c < cols; c += kSoftmaxBlock) m = fmaxf(m, row[c]);
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  if (lane == 0) red[wave] = m;
  __syncthreads();
  m = red[0];
  for (int w = 1; w < kSoftmaxBlock / 64; w++) m = fmaxf(m, red[w]);
  __syncthreads();
  float sum = 0.0f;
  for (long long c = threadIdx.x; c < cols; c += kSoftmaxBlock) {
    const float e = expf(scale * (row[c] - m));
    out[c] = e;
    sum += e;
  }
  for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
  if (lane == 0) red[wave] = sum;
  __syncthreads();
  sum = 0.0f;
  for (int w = 0; w < kSoftmaxBlock / 64; w++) sum += red[w];
  const float inv = 1.0f / sum;
  for (long long c = threadIdx.x; c < cols; c += kSoftmaxBlock) out[c] = out[c] * inv;
}

// weighted_values (attention.rs:371-408), rotated domain: a workgroup of D
// lanes (lane = element) accumulates sum_t w_t scale_t c[idx_t,e] over one
// chunk of values for one query; the finish kernel adds the chunks and
// applies the inverse rotation once.
constexpr int kWvChunk = 256;

constexpr int kWvQueries = 4;  // queries per partial workgroup: each code decoded once for all of them

template <int D, int PB>
__global__ __launch_bounds__(D) void qjl_wv_partial_kernel(const uint8_t *__restrict__ polar,
                                                           const uint16_t *__restrict__ polar_scales, long long nv,
                                                           long long nq, const float *__restrict__ weights,
                                                           float *__restrict__ partial, QjlConsts k) {
  constexpr int RWORDS = D * PB / 32;  // packed words per value
  constexpr int QW = kWvQueries;
  __shared__ uint32_t s_codes[kWvChunk * RWORDS];
  __shared__ float s_w[QW][kWvChunk];
  __shared__ float s_cent[16];
  if (threadIdx.x < 16) s_cent[threadIdx.x] = k.polar.cent[threadIdx.x & ((1 << PB) - 1)];
  const long long t0 = (long long)blockIdx.x * kWvChunk;
  const long long q0 = (long long)blockIdx.y * QW;
  const int cnt = (int)min<long long>(kWvChunk, nv - t0);
  for (int i = threadIdx.x; i < cnt * RWORDS; i += D)
    s_codes[i] = reinterpret_cast<const uint32_t *>(polar + t0 * (D * PB / 8))[i];
  for (int i = threadIdx.x; i < QW * cnt; i += D) {
    const int qq = i / cnt, t = i % cnt;
    const long long qi = q0 + qq;
    s_w[qq][t] = qi < nq ? weights[qi * nv + t0 + t] * f16_to_f32(polar_scales[t0 + t]) : 0.0f;
  }
  __syncthreads();
  const int e = threadIdx.x;
  const int bit = e * PB, wi = bit >> 5, sh = bit & 31;
  float acc[QW];
#pragma unroll
  for (int qq = 0; qq < QW; qq++) acc[qq] = 0.0f;
  for (int t = 0; t < cnt; t++) {
    const uint32_t *row = s_codes + t * RWORDS;
    uint32_t code = row[wi] >> sh;
    if (sh + PB > 32) code |= row[wi + 1] << (32 - sh);
    const float c = s_cent[code & ((1u << PB) - 1u)];
#pragma unroll
    for (int qq = 0; qq < QW; qq++) acc[qq] = __builtin_fmaf(s_w[qq][t], c, acc[qq]);
  }
#pragma unroll
  for (int qq = 0; qq < QW; qq++)
    if (q0 + qq < nq) partial[((q0 + qq) * gridDim.x + blockIdx.x) * D + e] = acc[qq];
}

// One workgroup of D lanes per query: lane e adds its element over the chunks
// (chunk order, from 0); then 32 lanes of E = D / 32 consecutive elements
// each apply the inverse rotation (butterfly<D>'s stages in its order: h < E
// inside a lane, h >= E with lane ^ (h / E); then the norm and the signs).
template <int D>
__global__ __launch_bounds__(D) void qjl_wv_finish_kernel(const float *__restrict__ partial, int nchunks,
                                                          float *__restrict__ out, long long nq, QjlConsts k) {
  constexpr int E = D / 32;
  __shared__ float s_a[D];
  const long long qi = blockIdx.x;
  const int e = threadIdx.x;
  float a = 0.0f;
  for (int c = 0; c < nchunks; c++) a += partial[(qi * nchunks + c) * D + e];
  s_a[e] = a;
  __syncthreads();
  if (e >= 32) return;
  float q[E];
#pragma unroll
  for (int i = 0; i < E; i++) q[i] = s_a[E * e + i];
#pragma unroll
  for (int h = 1; h < E; h *= 2)
#pragma unroll
    for (int i = 0; i < E; i += 2 * h)
#pragma unroll
      for (int t = i; t < i + h; t++) {
        const float x = q[t], y = q[t + h];
        q[t] = x + y;
        q[t + h] = x - y;
      }
  auto cross = [&](auto xc) {
    constexpr int X = decltype(xc)::value;
    const bool upper = (e & X) != 0;
#pragma unroll
    for (int i = 0; i < E; i++) {
      const float o = tqm::lane_xor<X>(q[i]);
      q[i] = upper ? o - q[i] : q[i] + o;
    }
  };
  cross(std::integral_constant<int, 1>{});
  cross(std::integral_constant<int, 2>{});
  cross(std::integral_constant<int, 4>{});
  cross(std::integral_constant<int, 8>{});
  cross(std::integral_constant<int, 16>{});
  const float se = k.polar.sign_even, so = -k.polar.sign_even;
#pragma unroll
  for (int i = 0; i < E; i++) {
    const int el = E * e + i;
    out[qi * D + el] = (q[i] * k.polar.wht_norm) * ((el & 1) ? so : se);
  }
}

// ---------------------------------------------------------------------------
// TqCache on the device (reference src/cache/tq.rs): the sign matrix of R,
// the sketch of cached keys' residuals, query projections and the logit bias.
// ---------------------------------------------------------------------------

// The d x d sign bits of R once, for kernels that read rather than hash them:
// out[j * D/32 + w] bit b set <=> sign(j, 32 w + b) = -1.
template <int D>
__global__ __launch_bounds__(kBlock) void qjl_sign_matrix_kernel(uint32_t *__restrict__ out, uint64_t seed) {
  const int it = blockIdx.x * kBlock + threadIdx.x;
  if (it >= D * D / 32) return;
  const int j = it / (D / 32), w = it % (D / 32);
  const uint64_t rs = mix_seed(seed, (uint64_t)j);
  uint32_t bits = 0;
  for (int b = 0; b < 32; b++) bits |= (sign_negative(rs, (uint64_t)j, (uint64_t)(32 * w + b)) ? 1u : 0u) << b;
  out[it] = bits;
}

// Lane j of a wave: p_j = (sum_c sign(j, c) v[c]) * inv for rows j = lane +
// 64 m (rademacher_vector_product, qjl.rs:196-208: column order, the +-v
// products exact), v read from LDS.
template <int D>
__device__ __forceinline__ void wave_row_products(const float *s_v, const uint32_t *__restrict__ rbits, float inv,
                                                  int lane, float (&p)[D / 64]) {
  constexpr int E = D / 64, NWR = D / 32;
  uint32_t rb[E][NWR];
#pragma unroll
  for (int m = 0; m < E; m++)
#pragma unroll
    for (int w = 0; w < NWR; w++) rb[m][w] = rbits[(lane + 64 * m) * NWR + w];
  float acc[E];
#pragma unroll
  for (int m = 0; m < E; m++) acc[m] = -0.0f;
#pragma unroll
  for (int c4 = 0; c4 < D / 4; c4++) {
    const float4 v = reinterpret_cast<const float4 *>(s_v)[c4];
    const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int c = 4 * c4 + i;
#pragma unroll
      for (int m = 0; m < E; m++)
        acc[m] = __builtin_fmaf(((rb[m][c >> 5] >> (c & 31)) & 1u) ? -1.0f : 1.0f, vv[i], acc[m]);
    }
  }
#pragma unroll
  for (int m = 0; m < E; m++) p[m] = acc[m] * inv;
}

struct SketchConsts {
  float cb[16];      // the cache codec's centroids
  uint32_t sign_mask;  // decode sign pattern (bit j set: -fl(R_fwd[0][j] * sqrt 32))
  float decode_factor;
  float inv_sqrt_d;
  long long head_stride, offset;
  int tokens;
};

// compute_qjl_signs_and_norms for keys just appended to a TqCache
// (tq.rs:154-182, 373-412), one wave per key vector (h, t): the key's cache
// record is dequantized exactly as polar_dequantize's CPU branch
// (quantize_tensor.rs:197-219, 32-lane butterflies), the residual
// r = k - k_hat is summed as sum r^2 in element order for the norm, and
// sign bit j = (R r)_j >= 0 (qjl.rs:305-319) is one wave ballot per 64 rows.
// Waves past the nvec keys project the nq query rows of `q` instead (rq = R q,
// as qjl_project_kernel), so a decode step's sketch and projection share one
// launch.
template <int D, int BITS, int IN_DT>
__global__ __launch_bounds__(kBlock) void qjl_cache_sketch_kernel(
    const void *__restrict__ x, const uint8_t *__restrict__ packed, const uint16_t *__restrict__ scales,
    const uint32_t *__restrict__ rbits, uint8_t *__restrict__ signs, uint16_t *__restrict__ norms, long long nvec,
    SketchConsts k, const void *__restrict__ q, int q_dtype, float *__restrict__ rq, long long nq) {
  constexpr int E = D / 64, NQB = D / 32, WB = 4 * BITS;
  __shared__ __attribute__((aligned(16))) float s_r[kBlock / 64][D];
  __shared__ float s_cb[16];
#pragma unroll
  for (int q = 0; q < 16; q++)
    if (threadIdx.x == q) s_cb[q] = k.cb[q];
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const long long v = (long long)blockIdx.x * (kBlock / 64) + wave;
  if (v >= nvec + nq) return;  // whole waves leave together
  if (v >= nvec) {
    const long long row = v - nvec;
#pragma unroll
    for (int m = 0; m < E; m++) {
      const long long xi = row * D + 64 * m + lane;
      float xv;
      if (q_dtype == kF32) xv = static_cast<const float *>(q)[xi];
      else if (q_dtype == kBF16) xv = bf16_to_f32(static_cast<const uint16_t *>(q)[xi]);
      else xv = f16_to_f32(static_cast<const uint16_t *>(q)[xi]);
      s_r[wave][64 * m + lane] = xv;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float p[E];
    wave_row_products<D>(s_r[wave], rbits, k.inv_sqrt_d, lane, p);
#pragma unroll
    for (int m = 0; m < E; m++) rq[row * D + 64 * m + lane] = p[m];
    return;
  }
  const long long h = v / k.tokens, t = v - h * k.tokens;
  const long long rec = h * k.head_stride + k.offset + t;
  const int i = lane & 31;
  const float sg = ((k.sign_mask >> i) & 1u) ? -k.decode_factor : k.decode_factor;
  float *r = s_r[wave];
#pragma unroll
  for (int m = 0; m < E; m++) {
    const int e = 64 * m + lane, qb = e >> 5;
    uint32_t w[BITS];
#pragma unroll
    for (int q = 0; q < BITS; q++) w[q] = reinterpret_cast<const uint32_t *>(packed + rec * (NQB * WB) + qb * WB)[q];
    // field i of the block's LSB-first bitstream (select chains: no
    // dynamically indexed registers)
    const int pos = i * BITS, wi = pos >> 5, sh = pos & 31;
    uint32_t lo = w[0], hi = w[1];
#pragma unroll
    for (int q = 1; q < BITS; q++) lo = (wi == q) ? w[q] : lo;
#pragma unroll
    for (int q = 2; q < BITS; q++) hi = (wi + 1 == q) ? w[q] : hi;
    hi = (wi + 1 < BITS) ? hi : 0u;
    const uint32_t code = __builtin_amdgcn_alignbit(hi, lo, sh) & ((1u << BITS) - 1u);
    float y = s_cb[code] * sg;
#pragma unroll
    for (int hh = 1; hh < 32; hh <<= 1) {
      const float o = __shfl_xor(y, hh, 64);
      y = (i & hh) ? (o - y) : (y + o);
    }
    const float s = fabsf(f16_to_f32(scales[rec * NQB + qb]));
    y = (y * 0x1.6a09e6p-3f) * s;
    const long long xi = v * D + e;
    float xv;
    if constexpr (IN_DT == kF32) xv = static_cast<const float *>(x)[xi];
    else if constexpr (IN_DT == kBF16) xv = bf16_to_f32(static_cast<const uint16_t *>(x)[xi]);
    else xv = f16_to_f32(static_cast<const uint16_t *>(x)[xi]);
    r[e] = xv - y;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float p[E];
  wave_row_products<D>(r, rbits, k.inv_sqrt_d, lane, p);
  uint64_t mask[E];
#pragma unroll
  for (int m = 0; m < E; m++) mask[m] = __builtin_amdgcn_ballot_w64(p[m] >= 0.0f);
  if (lane == 0) {
    float ss = 0.0f;
    for (int e = 0; e < D; e++) ss = ss + r[e] * r[e];
    norms[rec] = f32_to_f16(sqrtf(ss));
    uint32_t *sp = reinterpret_cast<uint32_t *>(signs + rec * (D / 8));
#pragma unroll
    for (int m = 0; m < E; m++) {
      sp[2 * m] = (uint32_t)mask[m];
      sp[2 * m + 1] = (uint32_t)(mask[m] >> 32);
    }
  }
}

// rq = R q per row (precompute_query_projections, qjl.rs:488-492; r_q = q R^T
// of tq.rs:233-234), one wave per row.
template <int D, int IN_DT>
__global__ __launch_bounds__(kBlock) void qjl_project_kernel(const void *__restrict__ q,
                                                             const uint32_t *__restrict__ rbits,
                                                             float *__restrict__ rq, long long nrows, float inv) {
  constexpr int E = D / 64;
  __shared__ __attribute__((aligned(16))) float s_q[kBlock / 64][D];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const long long row = (long long)blockIdx.x * (kBlock / 64) + wave;
  if (row >= nrows) return;
#pragma unroll
  for (int m = 0; m < E; m++) {
    const long long xi = row * D + 64 * m + lane;
    float xv;
    if constexpr (IN_DT == kF32) xv = static_cast<const float *>(q)[xi];
    else if constexpr (IN_DT == kBF16) xv = bf16_to_f32(static_cast<const uint16_t *>(q)[xi]);
    else xv = f16_to_f32(static_cast<const uint16_t *>(q)[xi]);
    s_q[wave][64 * m + lane] = xv;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float p[E];
  wave_row_products<D>(s_q[wave], rbits, inv, lane, p);
#pragma unroll
  for (int m = 0; m < E; m++) rq[row * D + 64 * m + lane] = p[m];
}

// compute_logit_bias (tq.rs:185-253): bias[h][i][t] = (sum_j rq[h][i][j]
// (2 b_tj - 1)) * (|r_t| * sf), sf = f32(sqrt(pi/2)) / sqrt(d), for query
// head h over KV head h / (H / H_kv).  Lane = token; per workgroup QB
// queries of one head, their +-rq nibble sums in LDS.
template <int D, int QB>
__global__ __launch_bounds__(kBlock) void qjl_logit_bias_kernel(const float *__restrict__ rq, int q_len,
                                                                const uint32_t *__restrict__ signs,
                                                                const uint16_t *__restrict__ norms, int kv_len,
                                                                long long head_stride, int n_rep, float sf,
                                                                void *__restrict__ out, int out_dtype) {
  constexpr int CT = (D / 4) * 16;
  __shared__ float s_tab[QB * CT];
  const int h = blockIdx.z;
  const int i0 = blockIdx.y * QB;
  const int nql = min(QB, q_len - i0);
  for (int e = threadIdx.x; e < nql * CT; e += kBlock) {
    const int ql = e / CT, rr = e % CT, c = rr / 16, m = rr % 16;
    const float *rp = rq + (((long long)h * q_len + i0 + ql) * D) + 4 * c;
    float val = -0.0f;
#pragma unroll
    for (int b = 0; b < 4; b++) val = val + (((m >> b) & 1) ? rp[b] : -rp[b]);
    s_tab[e] = val;
  }
  __syncthreads();
  const int t = blockIdx.x * kBlock + threadIdx.x;
  if (t >= kv_len) return;
  const long long rec = (long long)(h / n_rep) * head_stride + t;
  uint32_t sgn[D / 32];
#pragma unroll
  for (int w = 0; w < D / 32; w++) sgn[w] = signs[rec * (D / 32) + w];
  const float c = f16_to_f32(norms[rec]) * sf;
  for (int ql = 0; ql < nql; ql++) {
    const float *tb = s_tab + ql * CT;
    float raw = 0.0f;
#pragma unroll
    for (int cc = 0; cc < D / 4; cc++) raw += tb[cc * 16 + ((sgn[cc >> 3] >> ((cc & 7) * 4)) & 15u)];
    const float val = raw * c;
    const long long oi = ((long long)h * q_len + i0 + ql) * kv_len + t;
    if (out_dtype == kF32) static_cast<float *>(out)[oi] = val;
    else if (out_dtype == kBF16) static_cast<uint16_t *>(out)[oi] = f32_to_bf16(val);
    else static_cast<uint16_t *>(out)[oi] = f32_to_f16(val);
  }
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
    hipLaunchKernelGGL((qjl_quant_kernel<decltype(d)::value, decltype(pb)::value>), dim3((unsigned)((n + 31) / 32)),
                       dim3(kBlock), 0, stream, data, polar_packed, polar_scales, reinterpret_cast<uint32_t *>(signs),
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
  if (nq > 8LL * 65535) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "too many queries (%lld > %d)", nq, 8 * 65535);
  return by_dim(dim, [&](auto d) {
    constexpr int D = decltype(d)::value;
    hipLaunchKernelGGL((qjl_query_kernel<D>), dim3(D / 32, (unsigned)((nq + 7) / 8)), dim3(kBlock), 0, stream,
                       queries, ctx_out, nq, k);
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
  hipLaunchKernelGGL(softmax_rows_kernel, dim3((unsigned)rows), dim3(kSoftmaxBlock), 0, stream, scores, probs,
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
      hipLaunchKernelGGL((qjl_wv_partial_kernel<D, PB>), dim3((unsigned)nchunks, (unsigned)((nq + kWvQueries - 1) / kWvQueries)),
                         dim3(D), 0, stream, polar_packed, polar_scales, nv, nq, weights, partial, k);
      int rc2 = tqh::check_launch("qjl_wv_partial_kernel");
      if (rc2) return rc2;
    }
    hipLaunchKernelGGL((qjl_wv_finish_kernel<D>), dim3((unsigned)nq), dim3(D), 0, stream, partial, nchunks, out, nq, k);
    return tqh::check_launch("qjl_wv_finish_kernel");
  });
}

// ---------------------------------------------------------------------------
// TqCache building blocks
// ---------------------------------------------------------------------------

namespace {
float inv_sqrt_dim(int dim) { return tqh::inv_sqrt_dim(dim); }
int check_sketch_dim(int dim) {
  if (dim != 64 && dim != 128 && dim != 256)
    return tqh::fail(TQ_ERR_INVALID_DIMENSION, "cache QJL kernels take head_dim 64, 128 or 256 (got %d)", dim);
  return TQ_OK;
}
template <typename F>
int by_cache_dim(int dim, F &&f) {
  switch (dim) {
    case 64: return f(std::integral_constant<int, 64>{});
    case 128: return f(std::integral_constant<int, 128>{});
    case 256: return f(std::integral_constant<int, 256>{});
  }
  return tqh::fail(TQ_ERR_INVALID_DIMENSION, "unsupported head_dim %d", dim);
}
}  // namespace

extern "C" int tq_qjl_sign_matrix(uint32_t *bits_out, int dim, uint64_t qjl_seed, hipStream_t stream) {
  if (dim != 32 && dim != 64 && dim != 128 && dim != 256)
    return tqh::fail(TQ_ERR_INVALID_DIMENSION, "sign matrix dim must be 32, 64, 128 or 256 (got %d)", dim);
  if (!bits_out) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
  const unsigned grid = (unsigned)((dim * dim / 32 + kBlock - 1) / kBlock);
  switch (dim) {
    case 32: hipLaunchKernelGGL((qjl_sign_matrix_kernel<32>), dim3(grid), dim3(kBlock), 0, stream, bits_out, qjl_seed); break;
    case 64: hipLaunchKernelGGL((qjl_sign_matrix_kernel<64>), dim3(grid), dim3(kBlock), 0, stream, bits_out, qjl_seed); break;
    case 128: hipLaunchKernelGGL((qjl_sign_matrix_kernel<128>), dim3(grid), dim3(kBlock), 0, stream, bits_out, qjl_seed); break;
    default: hipLaunchKernelGGL((qjl_sign_matrix_kernel<256>), dim3(grid), dim3(kBlock), 0, stream, bits_out, qjl_seed); break;
  }
  return tqh::check_launch("qjl_sign_matrix_kernel");
}

extern "C" int tq_qjl_cache_sketch_project(const void *k, int k_dtype, int num_heads, int tokens,
                                           const uint8_t *packed_cache, const uint16_t *scales_cache,
                                           const uint32_t *sign_matrix, uint8_t *signs_cache, uint16_t *norms_cache,
                                           long long cache_head_stride, long long cache_offset, int head_dim, int bits,
                                           size_t outlier_blocks, int norm_mode, const void *q, int q_dtype, float *rq,
                                           size_t num_q_rows, hipStream_t stream) {
  int rc = check_sketch_dim(head_dim);
  if (rc) return rc;
  tqh::PolarCodec codec;
  rc = tqh::polar_codec(bits, norm_mode, outlier_blocks, head_dim / 32, codec);
  if (rc) return rc;
  if (!tqh::valid_dtype(k_dtype)) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "unknown dtype %d", k_dtype);
  if (num_heads < 0 || tokens < 0) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "negative shape");
  if (cache_offset < 0 || cache_head_stride < cache_offset + tokens)
    return tqh::fail(TQ_ERR_RANGE_OUT_OF_BOUNDS, "cache rows [%lld, %lld) exceed head stride %lld", cache_offset,
                     cache_offset + tokens, cache_head_stride);
  const long long nvec = (long long)num_heads * tokens, nq = (long long)num_q_rows;
  if (nvec + nq == 0) return TQ_OK;
  if (!sign_matrix || (nvec && (!k || !packed_cache || !scales_cache || !signs_cache || !norms_cache)))
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
  if (nq && (!q || !rq || !tqh::valid_dtype(q_dtype)))
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "query projection needs q (f32/bf16/f16) and rq");
  SketchConsts c{};
  for (int i = 0; i < codec.cb.nc; i++) c.cb[i] = codec.cb.c[i];
  c.sign_mask = kPqoSignMask;
  {
    volatile float thirty_two = 32.0f;
    volatile float sq = sqrtf(thirty_two);
    volatile float inv = 1.0f / sq;
    c.decode_factor = inv * sq;  // fl(fl(1/sqrt 32) * sqrt 32) (wht_tensor.rs:28-41)
  }
  c.inv_sqrt_d = inv_sqrt_dim(head_dim);
  c.head_stride = cache_head_stride;
  c.offset = cache_offset;
  c.tokens = tokens;
  const unsigned grid = (unsigned)((nvec + nq + kBlock / 64 - 1) / (kBlock / 64));
  return by_cache_dim(head_dim, [&](auto d) {
    constexpr int D = decltype(d)::value;
#define SK(B, T) hipLaunchKernelGGL((qjl_cache_sketch_kernel<D, B, T>), dim3(grid), dim3(kBlock), 0, stream, k, \
                                    packed_cache, scales_cache, sign_matrix, signs_cache, norms_cache, nvec, c, q, \
                                    q_dtype, rq, nq)
    if (bits == 3) {
      if (k_dtype == kF32) SK(3, kF32);
      else if (k_dtype == kBF16) SK(3, kBF16);
      else SK(3, kF16);
    } else {
      if (k_dtype == kF32) SK(4, kF32);
      else if (k_dtype == kBF16) SK(4, kBF16);
      else SK(4, kF16);
    }
#undef SK
    return tqh::check_launch("qjl_cache_sketch_kernel");
  });
}

extern "C" int tq_qjl_project(const void *q, int q_dtype, const uint32_t *sign_matrix, float *rq, size_t num_rows,
                              int dim, hipStream_t stream) {
  int rc = check_sketch_dim(dim);
  if (rc) return rc;
  if (!tqh::valid_dtype(q_dtype)) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "unknown dtype %d", q_dtype);
  if (num_rows == 0) return TQ_OK;
  if (!q || !sign_matrix || !rq) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
  const long long n = (long long)num_rows;
  const float inv = inv_sqrt_dim(dim);
  const unsigned grid = (unsigned)((n + kBlock / 64 - 1) / (kBlock / 64));
  return by_cache_dim(dim, [&](auto d) {
    constexpr int D = decltype(d)::value;
    if (q_dtype == kF32)
      hipLaunchKernelGGL((qjl_project_kernel<D, kF32>), dim3(grid), dim3(kBlock), 0, stream, q, sign_matrix, rq, n, inv);
    else if (q_dtype == kBF16)
      hipLaunchKernelGGL((qjl_project_kernel<D, kBF16>), dim3(grid), dim3(kBlock), 0, stream, q, sign_matrix, rq, n, inv);
    else
      hipLaunchKernelGGL((qjl_project_kernel<D, kF16>), dim3(grid), dim3(kBlock), 0, stream, q, sign_matrix, rq, n, inv);
    return tqh::check_launch("qjl_project_kernel");
  });
}

extern "C" float tq_qjl_bias_scale(int head_dim) {
  // tq.rs:213-214: f32(sqrt(pi / 2)) / sqrt(head_dim as f32)
  volatile float sp = (float)std::sqrt(3.14159265358979323846 / 2.0);
  volatile float fd = (float)head_dim;
  volatile float sq = sqrtf(fd);
  return sp / sq;
}

extern "C" int tq_qjl_logit_bias(const float *rq, int num_q_heads, int q_len, const uint8_t *signs_cache,
                                 const uint16_t *norms_cache, int num_kv_heads, int kv_len,
                                 long long cache_head_stride, int head_dim, void *out, int out_dtype,
                                 hipStream_t stream) {
  int rc = check_sketch_dim(head_dim);
  if (rc) return rc;
  if (!tqh::valid_dtype(out_dtype)) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "unknown dtype %d", out_dtype);
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads != 0)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "num_q_heads (%d) must be a multiple of num_kv_heads (%d)", num_q_heads,
                     num_kv_heads);
  if (q_len < 0 || kv_len < 0 || cache_head_stride < kv_len) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "bad shape");
  if (q_len == 0 || kv_len == 0) return TQ_OK;
  if (!rq || !signs_cache || !norms_cache || !out) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
  const float sf = tq_qjl_bias_scale(head_dim);
  const int n_rep = num_q_heads / num_kv_heads;
  return by_cache_dim(head_dim, [&](auto d) {
    constexpr int D = decltype(d)::value;
    constexpr int QB = 8;
    const dim3 grid((unsigned)((kv_len + kBlock - 1) / kBlock), (unsigned)((q_len + QB - 1) / QB), (unsigned)num_q_heads);
    hipLaunchKernelGGL((qjl_logit_bias_kernel<D, QB>), grid, dim3(kBlock), 0, stream, rq, q_len,
                       reinterpret_cast<const uint32_t *>(signs_cache), norms_cache, kv_len, cache_head_stride, n_rep,
                       sf, out, out_dtype);
    return tqh::check_launch("qjl_logit_bias_kernel");
  });
}

extern "C" int tq_qjl_cache_sketch(const void *k, int k_dtype, int num_heads, int tokens, const uint8_t *packed_cache,
                                   const uint16_t *scales_cache, const uint32_t *sign_matrix, uint8_t *signs_cache,
                                   uint16_t *norms_cache, long long cache_head_stride, long long cache_offset,
                                   int head_dim, int bits, size_t outlier_blocks, int norm_mode, hipStream_t stream) {
  return tq_qjl_cache_sketch_project(k, k_dtype, num_heads, tokens, packed_cache, scales_cache, sign_matrix,
                                     signs_cache, norms_cache, cache_head_stride, cache_offset, head_dim, bits,
                                     outlier_blocks, norm_mode, nullptr, TQ_DTYPE_F32, nullptr, 0, stream);
}
