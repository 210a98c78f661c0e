// tq_attention.hip -- fused PQO decode attention over the compressed cache.
//
// One workgroup (1024 lanes, 16 waves) owns a tile (sequence b, KV head g,
// chunk of CH = 1024 tokens) and serves all NR = num_heads / num_kv_heads
// query heads of that KV head, so every compressed byte is read from HBM
// exactly once (GQA sharing).  All of the tile's global loads (K and V codes
// and scales) are issued before any arithmetic and sit in VGPRs while the
// query tables are built, so each lane has ~25 loads in flight.
//
// Keys are never inverse-rotated.  With the block dequantization
//   k_j = |s| * inv * (H (cb[idx] * sg))_j               (wht_tensor.rs:38-64)
// the dot product is q.k = |s| * sum_i cb[idx_i] * qt_i, qt = inv * sg * (H q)
// (the rotated query), built once per tile.  The tile builds an LDS table of
// qt_i * cb[code] (times softmax scale * log2 e) for every code PAIR of
// adjacent elements (3-bit: 64 pair codes), so one 6-bit field extract and
// one LDS read cover two key elements for all NR heads at once.  Values are
// accumulated in the rotated domain, sum_t w_t |s_t| cb[idx_t], with a pair
// codebook (one LDS read per two elements), and inverse-rotated once per
// head after the split-K merge.
//
// Softmax is two-pass inside a tile (all CH scores staged in LDS, one max,
// one exp2 per score).  Split-K partials (m, l, acc) go to a workspace; with
// INLINE_MERGE the last tile of a (b, g) to finish (device-scope atomic
// counter) merges them and writes the output, then re-arms the counter, so
// one launch does the whole decode.
#include "tq_common.h"
#include "tq_device.h"

namespace {

using namespace tqd;

constexpr float kInvSqrt32 = 0x1.6a09e6p-3f;
constexpr float kLog2e = 1.44269504088896340736f;
// fl(fl(1/fl(sqrt 32)) * fl(sqrt 32)): the magnitude of every decode sign
// factor R_fwd[0][j] * sqrt(32) (wht_tensor.rs:28-41)
constexpr float kDecodeFactor = 0x1.fffffep-1f;

__device__ __forceinline__ float decode_sign(int j) {
  return ((kPqoSignMask >> j) & 1u) ? -kDecodeFactor : kDecodeFactor;
}
constexpr int kThreads = 1024;
constexpr int kChunk = 1024;
constexpr int kWaves = kThreads / 64;
// One split-K counter per (sequence, KV head), each on its own 256-byte line
// so the tiles' arrivals at different counters do not queue on one line.
constexpr int kCounterStride = 64;  // ints
#ifndef TQ_ATTN_LOAD_GROUPS
#define TQ_ATTN_LOAD_GROUPS 4
#endif
constexpr int kLoadGroups = TQ_ATTN_LOAD_GROUPS;  // staggered K/V fetch groups per tile
static_assert(kWaves % kLoadGroups == 0, "load groups split the waves evenly");

struct AttnArgs {
  const void *q;
  const uint8_t *k_idx;
  const uint16_t *k_sc;
  const uint8_t *v_idx;
  const uint16_t *v_sc;
  const int *kv_lens;        // device lengths, or null -> single_len
  int single_len;
  int max_len;               // host bound; device lengths are clamped to it
  int num_heads;
  int num_kv_heads;
  long long kv_head_stride;  // tokens
  long long seq_stride;      // tokens
  float softmax_scale;
  float *po;                 // partial acc  [(b*H + h) * P + c][head_dim]
  float *pm;                 // partial max  [(b*H + h) * P + c]   (base-2 logits)
  float *ps;                 // partial sum  [(b*H + h) * P + c]
  int *counters;             // [(b * Hkv + g) * kCounterStride], zero between launches
  int P;                     // chunk stride per (b, h) in the partial arrays
  void *out;
  int out_dtype;
  float cb[16];              // codebook
};

template <int QT>
__device__ __forceinline__ float load_q(const void *q, long long i) {
  if constexpr (QT == kF32) return static_cast<const float *>(q)[i];
  else if constexpr (QT == kBF16) return bf16_to_f32(static_cast<const uint16_t *>(q)[i]);
  else return f16_to_f32(static_cast<const uint16_t *>(q)[i]);
}

__device__ __forceinline__ float dpp_quad_xor1(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
}
__device__ __forceinline__ float dpp_quad_xor2(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
}

template <typename Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = op(v, __shfl_xor(v, o, 64));
  return v;
}

// DPP move: lanes whose source is outside the row (or whose row is masked
// off) take `id`.  Controls: row_shr:n = 0x110 + n, row_ror:n = 0x120 + n,
// row_bcast:15 = 0x142, row_bcast:31 = 0x143.
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
__device__ __forceinline__ float wave_max(float v) {
  return wave_allreduce(v, -INFINITY, [](float x, float y) { return fmaxf(x, y); });
}
__device__ __forceinline__ float wave_sum(float v) {
  return wave_allreduce(v, 0.f, [](float x, float y) { return x + y; });
}

// Sum of v over the lanes that differ only in lane bits 3..5 (the 8 lanes
// l ^ {0, 8, ..., 56}); every lane receives its group's total.  xor 8 is a
// DPP row rotate, xor 16 a swizzle inside each half-wave, xor 32 a permute.
__device__ __forceinline__ float xor16(float v) {
  // ds_swizzle bit mode: lane' = ((lane & 0x1f) | 0) ^ 0x10 within 32 lanes
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401f));
}
__device__ __forceinline__ float sum_lane_bits_4_5(float v) {
  v += xor16(v);
  return v + __shfl_xor(v, 32, 64);
}
__device__ __forceinline__ float sum_lane_bits_3_5(float v) {
  v += dpp<0x128>(v, 0.f);  // row_ror:8 == lane ^ 8 inside a row of 16
  return sum_lane_bits_4_5(v);
}

// Device-coherent accesses to the split-K partials: relaxed atomics at agent
// scope bypass the non-coherent per-XCD caches.
__device__ __forceinline__ void st_agent(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Reads `W` bits starting at bit `pos` of little-endian words (pos and the
// word indices must fold to constants after unrolling).
template <int W>
__device__ __forceinline__ uint32_t bits_at_p(const uint32_t *w, int pos) {
  const int wi = pos >> 5, sh = pos & 31;
  if (sh + W <= 32) return (w[wi] >> sh) & ((1u << W) - 1u);
  return __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh) & ((1u << W) - 1u);
}

// Reads `W` bits starting at bit `pos` of a little-endian word array.
template <int W, int NW>
__device__ __forceinline__ uint32_t bits_at(const uint32_t (&w)[NW], int pos) {
  const int wi = pos >> 5, sh = pos & 31;
  if (sh + W <= 32) return (w[wi] >> sh) & ((1u << W) - 1u);
  return __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh) & ((1u << W) - 1u);
}

template <int BITS>
struct Geo {
  static constexpr int NC = 1 << BITS;
  static constexpr int QB_BYTES = 4 * BITS;  // bytes per 32-element qblock
  // key table: 3-bit uses code pairs (64 entries per pair position),
  // 4-bit single codes (16 entries per element) to keep the table in LDS
  static constexpr bool KPAIR = (BITS == 3);
  static constexpr int KG = KPAIR ? 2 : 1;            // elements per key lookup
  static constexpr int KENT = KPAIR ? 64 : 16;        // entries per position
  static constexpr int KPOS = 32 / KG;                // positions per qblock
};

// ---------------------------------------------------------------------------
// Split-K merge and final inverse rotation for NR heads of one (b, g):
//   o = inv * H(sg * sum_c 2^(m_c - M) acc_c) / sum_c 2^(m_c - M) l_c
// All partial loads of a lane are independent (one latency round).
// ---------------------------------------------------------------------------
constexpr int kMergeCap = 2048;  // max NR * chunks merged (LDS floats)
constexpr int kMiscFloats = 2 * kMergeCap + kThreads + 8;

template <int NR>
__device__ void merge_and_store(const AttnArgs &a, int b, int g, int nchunks, float *lds) {
  constexpr int HD = 128;
  constexpr int OUTS = NR * HD;
  constexpr int PARTS = kThreads / OUTS;   // lanes sharing one output element
  constexpr int MAXC = 8;                  // partial values per lane per round
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  float *s_w = lds;                     // [NR][nchunks]: m_c, then weights 2^(m_c - M)
  float *s_ls = s_w + kMergeCap;        // [NR][nchunks]: l_c
  float *s_part = s_ls + kMergeCap;     // [kThreads] partial sums
  float *s_l = s_part + kThreads;       // [NR]
  const int o = tid % OUTS, part = tid / OUTS;
  const int r = o / HD, d = o % HD;
  const long long bh = (long long)b * a.num_heads + g * NR + r;
  // first round of this lane's partial accumulators, issued together with
  // the (m, l) loads so the whole merge costs one memory round trip when
  // nchunks <= MAXC * PARTS
  float pv[MAXC];
#pragma unroll
  for (int k = 0; k < MAXC; k++) {
    const int cc = part + k * PARTS;
    pv[k] = cc < nchunks ? ld_agent(&a.po[(bh * a.P + cc) * HD + d]) : 0.f;
  }
  for (int e = tid; e < NR * nchunks; e += kThreads) {
    const int rr = e / nchunks, cc = e % nchunks;
    const long long bh2 = (long long)b * a.num_heads + g * NR + rr;
    s_w[e] = ld_agent(&a.pm[bh2 * a.P + cc]);
    s_ls[e] = ld_agent(&a.ps[bh2 * a.P + cc]);
  }
  __syncthreads();
  if (wave < NR) {  // wave rr reduces head rr
    const int rr = wave;
    float M = -INFINITY;
    for (int cc = lane; cc < nchunks; cc += 64) M = fmaxf(M, s_w[rr * nchunks + cc]);
    M = wave_reduce(M, [](float x, float y) { return fmaxf(x, y); });
    float L = 0.f;
    for (int cc = lane; cc < nchunks; cc += 64) {
      const float w = exp2f(s_w[rr * nchunks + cc] - M);
      s_w[rr * nchunks + cc] = w;
      L = __builtin_fmaf(s_ls[rr * nchunks + cc], w, L);
    }
    L = wave_reduce(L, [](float x, float y) { return x + y; });
    if (lane == 0) s_l[rr] = L;
  }
  __syncthreads();
  float acc = 0.f;
#pragma unroll
  for (int k = 0; k < MAXC; k++) {
    const int cc = part + k * PARTS;
    if (cc < nchunks) acc = __builtin_fmaf(pv[k], s_w[r * nchunks + cc], acc);
  }
  for (int cc = part + MAXC * PARTS; cc < nchunks; cc += PARTS)  // long contexts only
    acc = __builtin_fmaf(ld_agent(&a.po[(bh * a.P + cc) * HD + d]), s_w[r * nchunks + cc], acc);
  s_part[tid] = acc;
  __syncthreads();
  if (tid < OUTS) {
    float A = 0.f;
#pragma unroll
    for (int p = 0; p < PARTS; p++) A += s_part[p * OUTS + tid];
    // inverse rotation over the 32 lanes of this block (lane bits 0..4 = i)
    const int i = d & 31;
    float v = A * decode_sign(i);
#pragma unroll
    for (int hh = 1; hh < 32; hh <<= 1) {
      float ov = __shfl_xor(v, hh, 64);
      v = (i & hh) ? (ov - v) : (v + ov);
    }
    const float L = s_l[r];
    const float res = (L > 0.f) ? v * kInvSqrt32 / L : 0.f;
    const long long oi = bh * HD + d;
    if (a.out_dtype == kF32) static_cast<float *>(a.out)[oi] = res;
    else if (a.out_dtype == kBF16) static_cast<uint16_t *>(a.out)[oi] = f32_to_bf16(res);
    else static_cast<uint16_t *>(a.out)[oi] = f32_to_f16(res);
  }
}

template <int BITS, int NR, int QT, bool INLINE_MERGE>
__global__ __launch_bounds__(kThreads) void attn_decode_kernel(AttnArgs a) {
  using G = Geo<BITS>;
  constexpr int NQB = 4, HD = 128, CH = kChunk;
  constexpr int QW = BITS;                       // 32-bit words per qblock
  constexpr int RW = NQB * QW;                   // words per token record (12 / 16)
  constexpr int PACKED = RW * 4;                 // bytes per token record
  constexpr int WT = 64;                         // tokens per wave: lane = token
  constexpr int EPL = NR <= 2 ? 16 : 8;          // V-pass elements per lane
  constexpr int GPQ = 32 / EPL;                  // V lanes per qblock of a token
  constexpr int VLPT = NQB * GPQ;                // V lanes per token
  constexpr int VSL = 64 / VLPT;                 // token slices per wave in the V pass
  constexpr int VTS = WT / VSL;                  // tokens per lane in the V pass
  constexpr int VCODES = 1 << (2 * BITS);        // pair-codebook entries
  constexpr int KV = NR == 1 ? 1 : 2;            // heads per key-table entry (one 4- or 8-byte read)
  constexpr int KNT = NR / KV;                   // key tables (entry reads per lookup)
  constexpr int KROW = G::KPOS * G::KENT;        // key-table entries per qblock
  constexpr int KTAB = NR * NQB * KROW;          // floats in all key tables
  constexpr int SPITCH = WT + 8;                 // V-scale rows: 4 qblock rows of 8 tokens on distinct banks
  constexpr int WSTAGE = WT * RW + NR * WT + NQB * SPITCH;  // per-wave staging: V records, p, |V scale|
  static_assert(kWaves * WT == CH, "one token per lane");
  static_assert(WSTAGE >= NR * HD + 2 * NR, "combine record fits the staging area");
  static_assert(KTAB * 4 <= 65536, "key-table offsets fit the ds_read immediate");
  // LDS carve (32-bit words).  Key tables [KNT][qblock][position][code] hold
  // KV heads per entry, so one lookup serves KV heads; the pair codebook holds
  // (cb[lo], cb[hi]) per 2*BITS-bit code.
  constexpr int OFF_CB2 = KTAB;
  constexpr int OFF_CB1 = OFF_CB2 + 2 * VCODES;
  constexpr int OFF_Q = OFF_CB1 + 16;
  constexpr int OFF_W = OFF_Q + NR * HD;
  constexpr int OFF_MISC = OFF_W;                       // merge scratch aliases the staging areas
  constexpr int TOTAL0 = OFF_W + kWaves * WSTAGE;
  constexpr int TOTAL = TOTAL0 > OFF_MISC + kMiscFloats ? TOTAL0 : OFF_MISC + kMiscFloats;
  __shared__ __attribute__((aligned(16))) float lds[TOTAL];
  __shared__ int s_flag;
  __shared__ int s_ready;  // waves whose K/V records have arrived (staggered loads)
  float *s_ktab = lds;
  float2 *s_cb2 = reinterpret_cast<float2 *>(lds + OFF_CB2);
  float *s_q = lds + OFF_Q;
  float *s_cb1 = lds + OFF_CB1;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int c = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int len = a.kv_lens ? min(max(a.kv_lens[b], 0), a.max_len) : a.single_len;
  const int t0 = c * CH;
  if (t0 >= len) return;  // empty tile: not counted by the merge
  const int nchunks = (len + CH - 1) / CH;
  const long long rec0 = (long long)b * a.seq_stride + (long long)g * a.kv_head_stride;
  uint32_t *stage = reinterpret_cast<uint32_t *>(lds + OFF_W + wave * WSTAGE);
  uint32_t *st_v = stage;                                     // [WT][RW]
  float *st_p = reinterpret_cast<float *>(stage + WT * RW);   // [WT][NR]: softmax numerators
  float *st_s = st_p + NR * WT;                               // [NQB][SPITCH]: |V scale|

  // ---- loads.  The query goes out alone, ahead of the code stream, so the
  // table build is not queued behind it.  The tile's waves then fetch their
  // K/V records in NGRP staggered groups: group g issues only once the
  // records of group g - 1 have arrived, so device-wide the early groups'
  // bytes come back first and their K/V passes overlap the later transfers
  // (all groups issuing at once would make every wave wait for the whole
  // tile). ----
  constexpr int GW = kWaves / kLoadGroups;  // waves per load group
  const int grp = wave / GW;
  // (every lane loads, clamped, so the wait for q lands at its first use)
  const float qv = load_q<QT>(a.q, ((long long)b * a.num_heads + g * NR) * HD + min(tid, NR * HD - 1));
  if (tid == 0) {  // codebook into LDS straight from the scalar kernel arguments
#pragma unroll
    for (int k = 0; k < 16; k++) s_cb1[k] = a.cb[k];
    s_ready = 0;
  }
  __syncthreads();
  const int tok = t0 + wave * WT + lane;
  const bool valid = tok < len;
  const long long rec = rec0 + min(tok, len - 1);
  uint32_t kr[RW], vr[RW];
  uint2 ksr, vsr;
  auto issue_loads = [&](long long r) {
    const uint4 *kp = reinterpret_cast<const uint4 *>(a.k_idx + r * PACKED);
    const uint4 *vp = reinterpret_cast<const uint4 *>(a.v_idx + r * PACKED);
#pragma unroll
    for (int q = 0; q < RW / 4; q++) {
      const uint4 v = kp[q];
      kr[4 * q] = v.x; kr[4 * q + 1] = v.y; kr[4 * q + 2] = v.z; kr[4 * q + 3] = v.w;
    }
    ksr = *reinterpret_cast<const uint2 *>(a.k_sc + r * NQB);
#pragma unroll
    for (int q = 0; q < RW / 4; q++) {
      const uint4 v = vp[q];
      vr[4 * q] = v.x; vr[4 * q + 1] = v.y; vr[4 * q + 2] = v.z; vr[4 * q + 3] = v.w;
    }
    vsr = *reinterpret_cast<const uint2 *>(a.v_sc + r * NQB);
  };
  // Every wave issues the same load sequence here (later groups fetch the
  // tile's first record, one cache line per instruction, as a placeholder),
  // so the number of loads in flight does not depend on the group and the
  // wait for the query below counts only the query.
  issue_loads(grp == 0 ? rec : rec0 + t0);

  // ---- rotated, scaled queries (32-lane butterflies) and the LDS tables ----
  const float qscale = a.softmax_scale * kLog2e * kInvSqrt32;
  if (tid < NR * HD) {
    const int d = tid % HD;
    float v = qv;
    const int i = d & 31;
#pragma unroll
    for (int hh = 1; hh < 32; hh <<= 1) {
      float ov = __shfl_xor(v, hh, 64);
      v = (i & hh) ? (ov - v) : (v + ov);
    }
    s_q[tid] = v * (decode_sign(i) * qscale);
  }
  if (tid < VCODES) {
    constexpr int NCm = G::NC - 1;
    s_cb2[tid] = make_float2(s_cb1[tid & NCm], s_cb1[(tid >> BITS) & NCm]);
  }
  __syncthreads();
  // Table entry (((t * NQB + qb) * KPOS + pos) * KENT + code) * KV + j holds,
  // for head r = t * KV + j, qt[2 pos] * cb[code & 7] + qt[2 pos + 1] * cb[code >> 3]
  // (3-bit pairs) or qt[pos] * cb[code] (4-bit).  Each work item fills four
  // consecutive codes of one row for its KV heads (one contiguous run).
  constexpr int ITEMS = KNT * NQB * G::KPOS * (G::KENT / 4);
  for (int it = tid; it < ITEMS; it += kThreads) {
    const int c4 = it % (G::KENT / 4), row = it / (G::KENT / 4);
    const int pos = row % G::KPOS, rq = row / G::KPOS;
    const int qb = rq % NQB, t = rq / NQB;
    float ov[4 * KV];
#pragma unroll
    for (int j = 0; j < KV; j++) {
      const int r = t * KV + j;
      if constexpr (G::KPAIR) {
        const float2 qt = *reinterpret_cast<const float2 *>(s_q + r * HD + qb * 32 + 2 * pos);
        const float hi = qt.y * s_cb1[(4 * c4) >> 3];
#pragma unroll
        for (int k = 0; k < 4; k++) ov[k * KV + j] = qt.x * s_cb1[(4 * c4 + k) & 7] + hi;
      } else {
        const float qt = s_q[r * HD + qb * 32 + pos];
#pragma unroll
        for (int k = 0; k < 4; k++) ov[k * KV + j] = qt * s_cb1[4 * c4 + k];
      }
    }
    float *dst = s_ktab + (row * G::KENT + 4 * c4) * KV;
#pragma unroll
    for (int k = 0; k < KV; k++)
      *reinterpret_cast<float4 *>(dst + 4 * k) = make_float4(ov[4 * k], ov[4 * k + 1], ov[4 * k + 2], ov[4 * k + 3]);
  }
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);  // keep the record-dependent code below the table build
  if (grp > 0) {
    // wait (acquire: the loads below cannot move above it) until every wave
    // of the previous group has its records, then fetch ours
    if (lane == 0)
      while (__hip_atomic_load(&s_ready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < grp * GW)
        __builtin_amdgcn_s_sleep(2);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    issue_loads(rec);
  }
  if constexpr (kLoadGroups > 1) {
    __builtin_amdgcn_s_waitcnt(0);  // this wave's records are in registers
    if (lane == 0) __hip_atomic_fetch_add(&s_ready, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  }

  // ---- K pass: lane = token, all qblocks in-lane (fully unrolled; the
  // scheduling barriers bound the LDS reads in flight to 16 positions) ----
  float score[NR];
#pragma unroll
  for (int r = 0; r < NR; r++) score[r] = 0.f;
#pragma unroll
  for (int qb = 0; qb < NQB; qb++) {
    float part[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) part[r] = 0.f;
    // groups of 16 positions: all table reads of a group are issued before
    // any is consumed, then summed as a tree (short dependency chains)
#pragma unroll
    for (int p0 = 0; p0 < G::KPOS; p0 += 16) {
      float ev[NR][16];
#pragma unroll
      for (int pos = p0; pos < p0 + 16; pos++) {
        const uint32_t code = bits_at_p<BITS * G::KG>(kr + qb * QW, pos * BITS * G::KG);
        const float *ent = s_ktab + ((qb * G::KPOS + pos) * G::KENT + code) * KV;
        if constexpr (KV == 1) {
          ev[0][pos - p0] = ent[0];
        } else {
#pragma unroll
          for (int t = 0; t < KNT; t++) {
            const float2 v = *reinterpret_cast<const float2 *>(ent + t * NQB * KROW * KV);
            ev[2 * t][pos - p0] = v.x;
            ev[2 * t + 1][pos - p0] = v.y;
          }
        }
      }
#pragma unroll
      for (int r = 0; r < NR; r++) {
#pragma unroll
        for (int w = 8; w > 0; w >>= 1)
#pragma unroll
          for (int i = 0; i < w; i++) ev[r][i] += ev[r][i + w];
        part[r] += ev[r][0];
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    const uint32_t sbits = (qb < 2 ? ksr.x : ksr.y) >> ((qb & 1) ? 16 : 0);
    const float ks = fabsf(f16_to_f32((uint16_t)(sbits & 0xffffu)));
#pragma unroll
    for (int r = 0; r < NR; r++) score[r] = __builtin_fmaf(part[r], ks, score[r]);
  }

  // ---- stage this wave's V records and scales (wave-private LDS) ----
#pragma unroll
  for (int q = 0; q < RW / 4; q++)
    *reinterpret_cast<uint4 *>(st_v + lane * RW + 4 * q) = make_uint4(vr[4 * q], vr[4 * q + 1], vr[4 * q + 2], vr[4 * q + 3]);
#pragma unroll
  for (int qb = 0; qb < NQB; qb++) {
    const uint32_t sbits = (qb < 2 ? vsr.x : vsr.y) >> ((qb & 1) ? 16 : 0);
    st_s[qb * SPITCH + lane] = fabsf(f16_to_f32((uint16_t)(sbits & 0xffffu)));
  }

  // ---- wave-local softmax (base 2): m = max over the wave's tokens ----
  float m_w[NR], p[NR];
#pragma unroll
  for (int r = 0; r < NR; r++) {
    const float sc = valid ? score[r] : -INFINITY;
    m_w[r] = wave_max(sc);
    p[r] = valid ? __builtin_amdgcn_exp2f(sc - m_w[r]) : 0.f;
  }
  if constexpr (NR == 1) {
    st_p[lane] = p[0];
  } else if constexpr (NR == 2) {
    *reinterpret_cast<float2 *>(st_p + 2 * lane) = make_float2(p[0], p[1]);
  } else {
    *reinterpret_cast<float4 *>(st_p + 4 * lane) = make_float4(p[0], p[1], p[2], p[3]);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // ---- V pass: lane = (token slice, qblock, group of EPL elements) ----
  const int vgrp = lane % GPQ, vqb = (lane / GPQ) % NQB, vsl = lane / VLPT;
  int vlo, vhi, vsh;
  if constexpr (BITS == 3 && EPL == 16) {
    vlo = (48 * vgrp) >> 5; vhi = vlo + 1; vsh = (48 * vgrp) & 31;
  } else if constexpr (BITS == 3) {
    vlo = (24 * vgrp) >> 5; vhi = min(vlo + 1, 2); vsh = (24 * vgrp) & 31;
  } else if constexpr (EPL == 16) {
    vlo = 2 * vgrp; vhi = vlo + 1; vsh = 0;
  } else {
    vlo = vgrp; vhi = vgrp; vsh = 0;
  }
  constexpr int VU = 4;  // V-pass unroll
  float acc[NR][EPL];
#pragma unroll
  for (int r = 0; r < NR; r++)
#pragma unroll
    for (int e = 0; e < EPL; e++) acc[r][e] = 0.f;
#pragma unroll VU
  for (int tk = 0; tk < VTS; tk++) {
    const int tl = vsl + tk * VSL;
    const uint32_t *rw = st_v + tl * RW + vqb * QW;
    uint64_t bits64;
    if constexpr (BITS == 3 && EPL == 16) {
      bits64 = (((uint64_t)rw[vhi] << 32) | rw[vlo]) >> vsh;
    } else if constexpr (BITS == 3) {
      bits64 = __builtin_amdgcn_alignbit(rw[vhi], rw[vlo], vsh);
    } else if constexpr (EPL == 16) {
      bits64 = ((uint64_t)rw[vhi] << 32) | rw[vlo];
    } else {
      bits64 = rw[vlo];
    }
    const float vs = st_s[vqb * SPITCH + tl];
    float wgt[NR];
    if constexpr (NR == 1) {
      wgt[0] = st_p[tl] * vs;
    } else if constexpr (NR == 2) {
      const float2 pp = *reinterpret_cast<const float2 *>(st_p + 2 * tl);
      wgt[0] = pp.x * vs; wgt[1] = pp.y * vs;
    } else {
      const float4 pp = *reinterpret_cast<const float4 *>(st_p + 4 * tl);
      wgt[0] = pp.x * vs; wgt[1] = pp.y * vs; wgt[2] = pp.z * vs; wgt[3] = pp.w * vs;
    }
#pragma unroll
    for (int pr = 0; pr < EPL / 2; pr++) {
      const uint32_t code = (uint32_t)(bits64 >> (pr * 2 * BITS)) & (VCODES - 1);
      const float2 cv = s_cb2[code];
#pragma unroll
      for (int r = 0; r < NR; r++) {
        acc[r][2 * pr] = __builtin_fmaf(wgt[r], cv.x, acc[r][2 * pr]);
        acc[r][2 * pr + 1] = __builtin_fmaf(wgt[r], cv.y, acc[r][2 * pr + 1]);
      }
    }
  }
  // reduce over the wave's token slices (lane bits above the V lane id)
  static_assert(VLPT == 8 || VLPT == 16, "token slices sit in lane bits 3..5 or 4..5");
#pragma unroll
  for (int r = 0; r < NR; r++)
#pragma unroll
    for (int e = 0; e < EPL; e++)
      acc[r][e] = VLPT == 8 ? sum_lane_bits_3_5(acc[r][e]) : sum_lane_bits_4_5(acc[r][e]);
  float l_w[NR];
#pragma unroll
  for (int r = 0; r < NR; r++) l_w[r] = wave_sum(p[r]);

  // ---- this wave's (m, l, acc) into its own staging area, then combine 16 waves ----
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  {
    float *comb = reinterpret_cast<float *>(stage);  // [HD][NR] acc, then m[NR], l[NR]
    if (lane < VLPT) {
#pragma unroll
      for (int r = 0; r < NR; r++)
#pragma unroll
        for (int e = 0; e < EPL; e++) comb[(vqb * 32 + vgrp * EPL + e) * NR + r] = acc[r][e];
    }
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < NR; r++) {
        comb[HD * NR + r] = m_w[r];
        comb[HD * NR + NR + r] = l_w[r];
      }
    }
  }
  __syncthreads();
  if (tid < NR * HD) {
    const int r = tid / HD, d = tid % HD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; w++) M = fmaxf(M, lds[OFF_W + w * WSTAGE + HD * NR + r]);
    float A = 0.f, L = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; w++) {
      const float *cw = lds + OFF_W + w * WSTAGE;
      const float mw = cw[HD * NR + r];
      const float f = (mw == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(mw - M);
      A = __builtin_fmaf(cw[d * NR + r], f, A);
      L = __builtin_fmaf(cw[HD * NR + NR + r], f, L);
    }
    const long long bh = (long long)b * a.num_heads + g * NR + r;
    st_agent(&a.po[(bh * a.P + c) * HD + d], A);
    if (d == 0) {
      st_agent(&a.pm[bh * a.P + c], M);
      st_agent(&a.ps[bh * a.P + c], L);
    }
  }

  if constexpr (INLINE_MERGE) {
    // The partials went out as agent-scope atomic stores, which are coherent
    // at device scope by themselves (no L2 writeback/invalidate needed).
    // Each wave waits until its stores have completed; after the barrier one
    // lane counts the tile in.  The last tile's merge reads the partials with
    // agent-scope atomic loads.
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __syncthreads();
    if (tid == 0) {
      const int prev = __hip_atomic_fetch_add(&a.counters[(b * a.num_kv_heads + g) * kCounterStride], 1, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
      s_flag = (prev == nchunks - 1);
    }
    __syncthreads();
    if (s_flag) {
      merge_and_store<NR>(a, b, g, nchunks, lds + OFF_MISC);
      if (tid == 0)
        __hip_atomic_store(&a.counters[(b * a.num_kv_heads + g) * kCounterStride], 0, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// Standalone split-K merge (the reference ABI's second launch).
template <int NR>
__global__ __launch_bounds__(kThreads) void attn_merge_kernel(AttnArgs a) {
  __shared__ float s_misc[kMiscFloats];
  const int g = blockIdx.x, b = blockIdx.y;
  const int len = a.kv_lens ? min(max(a.kv_lens[b], 0), a.max_len) : a.single_len;
  const int nchunks = (len + kChunk - 1) / kChunk;
  if (nchunks == 0) return;
  merge_and_store<NR>(a, b, g, nchunks, s_misc);
}

__global__ void fill_zero_kernel(int *p, long long n) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0;
}

// Workspace layout: po | pm | ps | counters (each 256-byte aligned).
struct WsLayout {
  size_t po, pm, ps, cnt, total;
  int P;
};

WsLayout ws_layout(int batch, int num_heads, int num_kv_heads, int head_dim, int max_len) {
  auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
  WsLayout w{};
  w.P = (max_len + kChunk - 1) / kChunk;
  const size_t bhp = (size_t)batch * num_heads * w.P;
  w.po = 0;
  w.pm = al(w.po + bhp * head_dim * sizeof(float));
  w.ps = al(w.pm + bhp * sizeof(float));
  w.cnt = al(w.ps + bhp * sizeof(float));
  w.total = al(w.cnt + (size_t)batch * num_kv_heads * kCounterStride * sizeof(int));
  return w;
}

AttnArgs base_args(int bits) {
  AttnArgs a{};
  tqh::PqoCodebook cb = tqh::pqo_codebook(bits);
  for (int i = 0; i < cb.nc; i++) a.cb[i] = cb.c[i];
  a.out_dtype = kF32;
  return a;
}

template <int BITS, int NR, bool INLINE>
int launch_decode_q(const AttnArgs &a, int qt, dim3 grid, hipStream_t st) {
  if (qt == kF32) hipLaunchKernelGGL((attn_decode_kernel<BITS, NR, kF32, INLINE>), grid, dim3(kThreads), 0, st, a);
  else if (qt == kBF16) hipLaunchKernelGGL((attn_decode_kernel<BITS, NR, kBF16, INLINE>), grid, dim3(kThreads), 0, st, a);
  else hipLaunchKernelGGL((attn_decode_kernel<BITS, NR, kF16, INLINE>), grid, dim3(kThreads), 0, st, a);
  return tqh::check_launch("attn_decode_kernel");
}

template <bool INLINE>
int launch_decode(const AttnArgs &a, int bits, int nr, int qt, dim3 grid, hipStream_t st) {
  if (bits == 3) {
    if (nr == 1) return launch_decode_q<3, 1, INLINE>(a, qt, grid, st);
    if (nr == 2) return launch_decode_q<3, 2, INLINE>(a, qt, grid, st);
    return launch_decode_q<3, 4, INLINE>(a, qt, grid, st);
  }
  if (nr == 1) return launch_decode_q<4, 1, INLINE>(a, qt, grid, st);
  if (nr == 2) return launch_decode_q<4, 2, INLINE>(a, qt, grid, st);
  return launch_decode_q<4, 4, INLINE>(a, qt, grid, st);
}

int check_common(int num_heads, int num_kv_heads, int head_dim, int bits) {
  if (bits != 3 && bits != 4) return tqh::fail(TQ_ERR_UNSUPPORTED_BITS, "unsupported bits=%d, expected 3 or 4", bits);
  if (head_dim != 128)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "fused decode attention supports head_dim 128, got %d", head_dim);
  if (num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads != 0)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "num_heads (%d) must be a multiple of num_kv_heads (%d)", num_heads,
                     num_kv_heads);
  const int nr = num_heads / num_kv_heads;
  if (nr != 1 && nr != 2 && nr != 4)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "GQA ratio %d not supported (1, 2 or 4)", nr);
  return TQ_OK;
}

}  // namespace

extern "C" size_t tq_attention_workspace_size(int batch, int num_heads, int num_kv_heads, int head_dim,
                                              int max_kv_len) {
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || max_kv_len < 0) return 0;
  return ws_layout(batch, num_heads, num_kv_heads, head_dim, max_kv_len).total;
}

extern "C" int tq_attention_workspace_init(void *workspace, size_t workspace_bytes, int batch, int num_heads,
                                           int num_kv_heads, int head_dim, int max_kv_len, hipStream_t stream) {
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || max_kv_len < 0)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "invalid workspace shape");
  const WsLayout w = ws_layout(batch, num_heads, num_kv_heads, head_dim, max_kv_len);
  if (!workspace || workspace_bytes < w.total)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "workspace too small: %zu < %zu", workspace_bytes, w.total);
  const long long n = (long long)batch * num_kv_heads * kCounterStride;
  hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                     reinterpret_cast<int *>(static_cast<char *>(workspace) + w.cnt), n);
  return tqh::check_launch("fill_zero_kernel");
}

extern "C" int tq_pqo_decode_attention(const void *q, int q_dtype, const uint8_t *k_indices, const uint16_t *k_scales,
                                       const uint8_t *v_indices, const uint16_t *v_scales, const int *kv_lens,
                                       int batch, int num_heads, int num_kv_heads, int head_dim, int bits,
                                       int max_kv_len, long long kv_head_stride, long long seq_stride,
                                       float softmax_scale, void *out, int out_dtype, void *workspace,
                                       size_t workspace_bytes, hipStream_t stream) {
  int rc = check_common(num_heads, num_kv_heads, head_dim, bits);
  if (rc) return rc;
  if (!tqh::valid_dtype(q_dtype) || !tqh::valid_dtype(out_dtype))
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "unknown dtype");
  if (batch <= 0 || max_kv_len <= 0) return TQ_OK;
  if (!q || !k_indices || !k_scales || !v_indices || !v_scales || !kv_lens || !out)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
  if (kv_head_stride < max_kv_len)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "kv_head_stride %lld < max_kv_len %d", kv_head_stride, max_kv_len);
  if (batch > 1 && seq_stride < (long long)num_kv_heads * kv_head_stride)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "seq_stride %lld overlaps the KV heads of a sequence", seq_stride);
  const WsLayout w = ws_layout(batch, num_heads, num_kv_heads, head_dim, max_kv_len);
  if (!workspace || workspace_bytes < w.total)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "workspace too small: %zu < %zu", workspace_bytes, w.total);
  if ((long long)(num_heads / num_kv_heads) * w.P > kMergeCap)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "max_kv_len %d too long for one merge", max_kv_len);
  AttnArgs a = base_args(bits);
  char *ws = static_cast<char *>(workspace);
  a.q = q;
  a.k_idx = k_indices;
  a.k_sc = k_scales;
  a.v_idx = v_indices;
  a.v_sc = v_scales;
  a.kv_lens = kv_lens;
  a.single_len = 0;
  a.max_len = max_kv_len;
  a.num_heads = num_heads;
  a.num_kv_heads = num_kv_heads;
  a.kv_head_stride = kv_head_stride;
  a.seq_stride = seq_stride;
  a.softmax_scale = softmax_scale;
  a.po = reinterpret_cast<float *>(ws + w.po);
  a.pm = reinterpret_cast<float *>(ws + w.pm);
  a.ps = reinterpret_cast<float *>(ws + w.ps);
  a.counters = reinterpret_cast<int *>(ws + w.cnt);
  a.P = w.P;
  a.out = out;
  a.out_dtype = out_dtype;
  const dim3 grid((unsigned)w.P, (unsigned)num_kv_heads, (unsigned)batch);
  return launch_decode<true>(a, bits, num_heads / num_kv_heads, q_dtype, grid, stream);
}

extern "C" int tq_fused_attention(const float *q, const uint8_t *k_indices, const uint16_t *k_scales,
                                  const uint8_t *v_indices, const uint16_t *v_scales, const float *codebook,
                                  const float *sign_pattern, float *output, float *partial_out, float *partial_max,
                                  float *partial_sum, const uint8_t *qjl_signs, const uint16_t *qjl_residual_norms,
                                  const float *rq, int qjl_enabled, int num_attention_heads, int num_kv_heads,
                                  int head_dim, int kv_len, int kv_stride, int packed_dim, int num_qblocks, int bits,
                                  float softmax_scale, int num_partitions, hipStream_t stream) {
  (void)qjl_signs;
  (void)qjl_residual_norms;
  (void)rq;
  if (kv_len == 0 || num_kv_heads == 0) return TQ_OK;  // tq_attention_kernel.cu:366
  if (qjl_enabled) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "QJL correction in fused attention is not enabled");
  int rc = check_common(num_attention_heads, num_kv_heads, head_dim, bits);
  if (rc) return rc;
  if (num_qblocks != head_dim / 32 || packed_dim != head_dim * bits / 8)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "num_qblocks/packed_dim inconsistent with head_dim and bits");
  if (kv_len < 0 || kv_stride < kv_len) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "kv_stride < kv_len");
  if (num_partitions < (kv_len + 511) / 512)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "num_partitions %d < ceil(kv_len/512)", num_partitions);
  if (!q || !k_indices || !k_scales || !v_indices || !v_scales || !codebook || !sign_pattern || !output ||
      !partial_out || !partial_max || !partial_sum)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
  // The codebook and sign pattern are device tensors in the reference
  // (pqo.rs:134-160) holding the PQO constants, which this entry applies from
  // its own copy.  The caller's partial buffers (sized for 512-token
  // partitions) hold this entry's 1024-token partials.
  (void)codebook;
  (void)sign_pattern;
  AttnArgs a = base_args(bits);
  a.q = q;
  a.k_idx = k_indices;
  a.k_sc = k_scales;
  a.v_idx = v_indices;
  a.v_sc = v_scales;
  a.kv_lens = nullptr;
  a.single_len = kv_len;
  a.max_len = kv_len;
  a.num_heads = num_attention_heads;
  a.num_kv_heads = num_kv_heads;
  a.kv_head_stride = kv_stride;
  a.seq_stride = 0;
  a.softmax_scale = softmax_scale;
  a.po = partial_out;
  a.pm = partial_max;
  a.ps = partial_sum;
  a.counters = nullptr;
  a.P = num_partitions;
  a.out = output;
  a.out_dtype = kF32;
  const int nr = num_attention_heads / num_kv_heads;
  const int P = (kv_len + kChunk - 1) / kChunk;
  if ((long long)nr * P > kMergeCap) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "kv_len %d too long for one merge", kv_len);
  rc = launch_decode<false>(a, bits, nr, kF32, dim3((unsigned)P, (unsigned)num_kv_heads, 1u), stream);
  if (rc) return rc;
  const dim3 mgrid((unsigned)num_kv_heads, 1u);
  if (nr == 1) hipLaunchKernelGGL((attn_merge_kernel<1>), mgrid, dim3(kThreads), 0, stream, a);
  else if (nr == 2) hipLaunchKernelGGL((attn_merge_kernel<2>), mgrid, dim3(kThreads), 0, stream, a);
  else hipLaunchKernelGGL((attn_merge_kernel<4>), mgrid, dim3(kThreads), 0, stream, a);
  return tqh::check_launch("attn_merge_kernel");
}
