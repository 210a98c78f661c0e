// tq_attention.hip -- fused PQO decode attention over the compressed cache.
//
// One workgroup (1024 lanes, 16 waves) owns a tile (sequence b, KV head g,
// chunk of CH = 1024 tokens) and serves all NR = num_heads / num_kv_heads
// query heads of that KV head, so every compressed byte is read from HBM
// exactly once (GQA sharing).  Each wave owns 64 tokens, fetched as four
// 16-token tiles, each load instruction one contiguous run of records (key
// codes: lane (t, q) loads qblock q of token t; value codes: lane l of a
// 16-lane group loads qblock l % 4 of token 4 g + l / 4).
//
// Keys are never inverse-rotated.  With the block dequantization
//   k_j = |s| * inv * (H (cb[idx] * sg))_j               (wht_tensor.rs:38-64)
// the dot product is q.k = |s| * sum_i cb[idx_i] * qt_i, qt = inv * sg * (H q)
// (the rotated query), built once per tile.  Both contractions run on the
// matrix cores (v_mfma_f32_16x16x32_f16) with every f32 operand split into
// two f16 parts (hi = the value cut to 11 significant bits, lo = the exact
// remainder), so the products carry 22 significant bits and accumulate in f32:
//   scores  D[(qblock, head, part)][token] = sum_k Q[..][k] K[k][token], the
//           query operand block-diagonal over qblocks so that the
//           per-(token, qblock) key scale applies after the contraction;
//   values  D[(qblock, value part)][(qblock, head, part)] = sum_t V W,
//           W = p * |s_V|, the value operand taken element-major straight
//           from the pair table through the transposing LDS read.
// A pair of codes is decoded by one 8-byte LDS read from a 2^(2 BITS)-entry
// table of (hi(cb[c0]), hi(cb[c1]), lo(cb[c0]), lo(cb[c1])).  Values are
// accumulated in the rotated domain and inverse-rotated once per head after
// the split-K merge.
//
// Softmax is two-pass inside a wave (all 64 scores, one max, one exp2 per
// score); the 16 waves' (m, l, acc) are combined in LDS.  Split-K partials go
// to a workspace; with INLINE_MERGE the last tile of a (b, g) to finish
// (device-scope atomic counter) merges them and writes the output, then
// re-arms the counter, so one launch does the whole decode.
#include "tq_common.h"
#include "tq_device.h"
#include "tq_mfma.h"

#include <mutex>
#include <type_traits>

namespace {

using namespace tqd;
using namespace tqm;

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

// Cache codec of the attended records: PQO (outlier codebook, CB = BITS),
// PQ (standard (BITS - 1)-bit codebook in BITS-wide slots) and TQ (PQ plus
// the QJL correction of the keys' residuals, tq.rs:185-253 and the QJL
// branch of tq_attention_kernel.cu:192-231).
enum Mode : int { kModePqo = 0, kModePq = 1, kModeTq = 2 };

struct AttnArgs {
  const void *q;
  int q_dtype;
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
  // Split-K arrival counters, one 256-byte line per (sequence, KV head),
  // zero between launches: counter i = b * Hkv + g sits at
  // cnt_top - (i + 1) * kCounterStride; *ws_hdr = the number of counters
  // below cnt_top that were zeroed.  A launch merges only if its ws_pairs =
  // batch * num_kv_heads counters were zeroed (ws_pairs <= *ws_hdr) and its
  // partials end below them (*ws_hdr <= ws_room, the counter lines between
  // its partials and cnt_top); otherwise it stores nothing and writes NaN
  // outputs.
  int *cnt_top;
  const int *ws_hdr;
  int ws_pairs;
  int ws_room;
  int P;                     // chunk stride per (b, h) in the partial arrays
  void *out;
  int out_dtype;
  // TQ: rq [b][h][head_dim] f32 = R q (precompute_query_projections); per
  // record, signs [16] u8 of R r and the f16 residual norm |r|; qjl_c =
  // f32(sqrt(pi/2)) / sqrt(head_dim)
  const float *rq;
  const uint32_t *qjl_signs;
  const uint16_t *qjl_norms;
  float qjl_c;
  // cb_args: the codebook comes from cb (L2Norm tables) instead of the
  // MaxNorm constants compiled in
  int cb_args;
  float cb[16];
  // reference ABI (tq_fused_attention): the caller's device codebook
  // (indexed by code, tq_attention_kernel.cu:129) and 32 decode signs
  // (applied before the WHT, tq_attention_kernel.cu:45), or null
  const float *cb_dev;
  const float *sg_dev;
};

// Query element as stored (f32 bits or a 16-bit pattern), converted
// separately so that the wait for the load lands at the first use.
__device__ __forceinline__ float q_value(uint32_t bits, int qt) {
  if (qt == kF32) return u2f(bits);
  if (qt == kBF16) return bf16_to_f32((uint16_t)bits);
  return f16_to_f32((uint16_t)bits);
}

// ---------------------------------------------------------------------------
// Split-K merge and final inverse rotation for NR heads of one (b, g):
//   o = inv * H(sg * sum_c 2^(m_c - M) acc_c) / sum_c 2^(m_c - M) l_c
// Each lane folds four consecutive elements of every PARTS-th chunk (one
// 16-byte device-coherent load per chunk) under a local maximum; the PARTS
// lane sets meet once in LDS.  The first-round loads of a lane are
// independent (one latency round); longer contexts continue with an online
// update.
// ---------------------------------------------------------------------------
constexpr int kMiscFloats = 2 * kThreads + 64;

// 16-byte load with the coherence of an agent-scope atomic load (SC1): the
// partials were written by other workgroups, possibly on other dies.
__device__ __forceinline__ float4 ld_agent16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 16));
}

template <int NR>
__device__ void merge_and_store(const AttnArgs &a, int b, int g, int nchunks, float *lds) {
  constexpr int HD = 128;
  constexpr int OUTS = NR * HD;
  constexpr int QUADS = OUTS / 4;          // four consecutive elements per lane
  constexpr int PARTS = 4;                 // lane sets, each folding every PARTS-th chunk
  constexpr int MAXC = 8;                  // chunks per lane in the first round
  static_assert(PARTS * OUTS <= 2 * kThreads && 2 * PARTS * NR <= 64, "merge scratch");
  const int tid = threadIdx.x;
  float *s_a = lds;                        // [PARTS][OUTS] partial sums
  float *s_ml = s_a + PARTS * OUTS;        // [PARTS][NR] (local max, local l)
  const int quad = tid % QUADS, part = tid / QUADS;
  const int r = quad / (HD / 4), d0 = 4 * (quad % (HD / 4));
  const long long bh0 = (long long)b * a.num_heads + g * NR;  // first head of this KV head
  const long long c0 = (bh0 + r) * a.P;
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      a.po + bh0 * a.P * HD, (short)0, NR * a.P * HD * (int)sizeof(float), 0x00020000);
  const bool active = tid < PARTS * QUADS;
  float4 pv[MAXC];
  float pm[MAXC], pl[MAXC];
#pragma unroll
  for (int k = 0; k < MAXC; k++) {
    const int cc = part + k * PARTS;
    const bool ok = active && cc < nchunks;
    pv[k] = ok ? ld_agent16(rsrc, (uint32_t)(((r * a.P + cc) * HD + d0) * 4)) : make_float4(0.f, 0.f, 0.f, 0.f);
    pm[k] = ok ? ld_agent(&a.pm[c0 + cc]) : -INFINITY;
    pl[k] = ok ? ld_agent(&a.ps[c0 + cc]) : 0.f;
  }
  float M = -INFINITY;
#pragma unroll
  for (int k = 0; k < MAXC; k++) M = fmaxf(M, pm[k]);
  float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
  float L = 0.f;
  auto fold = [&](const float4 &v, float l, float w) {
    A.x = __builtin_fmaf(v.x, w, A.x);
    A.y = __builtin_fmaf(v.y, w, A.y);
    A.z = __builtin_fmaf(v.z, w, A.z);
    A.w = __builtin_fmaf(v.w, w, A.w);
    L = __builtin_fmaf(l, w, L);
  };
#pragma unroll
  for (int k = 0; k < MAXC; k++) fold(pv[k], pl[k], pm[k] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(pm[k] - M));
  for (int cc = part + MAXC * PARTS; active && cc < nchunks; cc += PARTS) {  // long contexts only
    const float m = ld_agent(&a.pm[c0 + cc]), l = ld_agent(&a.ps[c0 + cc]);
    const float4 v = ld_agent16(rsrc, (uint32_t)(((r * a.P + cc) * HD + d0) * 4));
    if (m == -INFINITY) continue;
    if (m > M) {
      const float f = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M - m);
      A.x *= f;
      A.y *= f;
      A.z *= f;
      A.w *= f;
      L *= f;
      M = m;
    }
    fold(v, l, __builtin_amdgcn_exp2f(m - M));
  }
  if (active) *reinterpret_cast<float4 *>(s_a + part * OUTS + 4 * quad) = A;
  if (active && d0 == 0) {
    s_ml[2 * (part * NR + r)] = M;
    s_ml[2 * (part * NR + r) + 1] = L;
  }
  __syncthreads();
  if (tid < OUTS) {
    const int ro = tid / HD, d = tid % HD;
    float Mx = -INFINITY;
#pragma unroll
    for (int p = 0; p < PARTS; p++) Mx = fmaxf(Mx, s_ml[2 * (p * NR + ro)]);
    float At = 0.f, Lt = 0.f;
#pragma unroll
    for (int p = 0; p < PARTS; p++) {
      const float mp = s_ml[2 * (p * NR + ro)];
      const float f = mp == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mp - Mx);
      At = __builtin_fmaf(s_a[p * OUTS + tid], f, At);
      Lt = __builtin_fmaf(s_ml[2 * (p * NR + ro) + 1], f, Lt);
    }
    // inverse rotation over the 32 lanes of this block (lane bits 0..4 = i)
    const int i = d & 31;
    const float sg = a.sg_dev ? a.sg_dev[i] : decode_sign(i);
    const float v = wht32_lanes(At * sg, i);
    const float res = (Lt > 0.f) ? v * kInvSqrt32 / Lt : 0.f;
    const long long oi = (bh0 + ro) * HD + d;
    if (a.out_dtype == kF32) static_cast<float *>(a.out)[oi] = res;
    else if (a.out_dtype == kBF16) static_cast<uint16_t *>(a.out)[oi] = f32_to_bf16(res);
    else static_cast<uint16_t *>(a.out)[oi] = f32_to_f16(res);
  }
}

// The record pointers and strides also come as leading scalar arguments
// (copies of a's fields, plus the single length or -1 when the lengths are
// per sequence in device memory): the build preloads the first kernel-argument dwords
// into SGPRs at wave launch, so the first record loads need no kernel-argument
// fetch.
template <int BITS, int MODE, int NR, bool INLINE_MERGE>
__global__ __launch_bounds__(kThreads) void attn_decode_kernel(const uint8_t *k_idx, const uint8_t *v_idx,
                                                               const uint16_t *k_sc, const uint16_t *v_sc,
                                                               long long seq_stride, long long kv_head_stride,
                                                               int len_hint, AttnArgs a) {
  constexpr int CB = MODE == kModePqo ? BITS : BITS - 1;  // codebook bits
  constexpr bool QJL = MODE == kModeTq;
  constexpr int NQB = 4, HD = 128, CH = kChunk;
  constexpr int QW = BITS;                       // 32-bit words per qblock
  constexpr int PACKED = NQB * QW * 4;           // bytes per token record
  constexpr int NC = 1 << BITS;
  constexpr int NPAIR = 1 << (2 * BITS);         // pair-table entries
  // One pair table (512 B for 3-bit codes, 2 KB for 4-bit): per-lane copies
  // measured no faster, as 8-byte LDS reads are served 32 lanes at a time.
  constexpr int WT = 64;                         // tokens per wave
  constexpr int NT = WT / 16;                    // 16-token tiles per wave
  constexpr int NG = NR > 2 ? NR / 2 : 1;        // MFMA head groups: 16 rows = 4 qblocks x 2 heads x 2 parts
  // per-wave staging (32-bit words)
  constexpr int RA = NQB * WT * NR;              // K partial scores [qblock][token][head]
  constexpr int PW = NR * WT;                    // softmax numerators [head][token]
  constexpr int SW = NQB * WT;                   // |V scale| * 2^-Ev [qblock][token]
  constexpr int CW = (NR * HD + 2 * NR + 1 + 3) & ~3;  // combine record: acc [head][d], m, l, 2^Ev
  constexpr int WSTAGE = RA + PW + SW + CW;
  // LDS carve (32-bit words)
  constexpr int OFF_PAIR = 0;                    // uint2 [NPAIR]
  constexpr int OFF_QA = OFF_PAIR + 2 * NPAIR;   // u32x4 [NG][8][64]: key-pass query operands
  constexpr int OFF_Q = OFF_QA + NG * 8 * 64 * 4;
  constexpr int OFF_QMAX = OFF_Q + NR * HD;      // [2 NR] max |qt| per half head
  // QJL: u32x4 [4][64] correction operands, uint2 [16] +-1 f16 nibble table,
  // [2 NR] max |rq| per half head
  constexpr int OFF_RA = OFF_QMAX + 8;
  constexpr int OFF_NIB = OFF_RA + (QJL ? 4 * 64 * 4 : 0);
  constexpr int OFF_RQMAX = OFF_NIB + (QJL ? 32 : 0);
  constexpr int OFF_W = OFF_RQMAX + (QJL ? 8 : 0);
  constexpr int OFF_MISC = OFF_W;                // merge scratch aliases the staging areas
  constexpr int TOTAL0 = OFF_W + kWaves * WSTAGE;
  constexpr int TOTAL = TOTAL0 > OFF_MISC + kMiscFloats ? TOTAL0 : OFF_MISC + kMiscFloats;
  static_assert(kWaves * WT == CH, "64 tokens per wave");
  static_assert(TOTAL * 4 <= 160 * 1024, "fits the LDS of one CU");
  static_assert(NR * HD % 64 == 0, "whole waves rotate the query");
  __shared__ __attribute__((aligned(16))) float lds[TOTAL];
  __shared__ int s_flag;
  __shared__ int s_ready;  // waves whose K/V records have arrived (staggered loads)
  uint2 *s_pair = reinterpret_cast<uint2 *>(lds + OFF_PAIR);
  u32x4 *s_qa = reinterpret_cast<u32x4 *>(lds + OFF_QA);
  float *s_q = lds + OFF_Q;
  float *s_qmax = lds + OFF_QMAX;
  u32x4 *s_ra = reinterpret_cast<u32x4 *>(lds + OFF_RA);
  uint2 *s_nib = reinterpret_cast<uint2 *>(lds + OFF_NIB);
  float *s_rqmax = lds + OFF_RQMAX;
  float *s_rq = lds + OFF_W;  // scaled rq [NR][HD]: read before any wave stages its records here

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, lg = lane >> 4;  // matrix-core column / row group of this lane
  const int c = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int t0 = c * CH;
  const long long rec0 = (long long)b * seq_stride + (long long)g * kv_head_stride;
  const uint8_t *kbase = k_idx + rec0 * PACKED, *vbase = v_idx + rec0 * PACKED;

  // ---- the query goes out first (it does not depend on the sequence
  // length), loaded by the waves that rotate it, one element per lane (whole
  // waves: NR * HD % 64 == 0).  These waves rotate it before they queue any
  // record load, so the wait for it counts nothing else. ----
  const long long qidx = ((long long)b * a.num_heads + g * NR) * HD + tid;
  uint32_t qbits = 0;
  float rqv = 0.f;
  if (tid < NR * HD) {
    if (a.q_dtype == kF32) qbits = static_cast<const uint32_t *>(a.q)[qidx];
    else qbits = static_cast<const uint16_t *>(a.q)[qidx];
    if constexpr (QJL) rqv = a.rq[qidx];
  }
  float qsign = 0.f;  // decode sign of this lane's query element
  if (tid < NR * HD) qsign = a.sg_dev ? a.sg_dev[tid & 31] : decode_sign(tid & 31);
  // workspace header (inline merge): the counters the init zeroed
  int ws_hdr = 0;
  if (INLINE_MERGE && tid == 0) ws_hdr = *a.ws_hdr;
  // len_hint: the single length, or -1 for per-sequence device lengths
  const int len = len_hint >= 0 ? len_hint : min(max(a.kv_lens[b], 0), a.max_len);
  if (t0 >= len) {  // empty tile: not counted by the merge
    if (len == 0 && c == 0 && tid < NR * HD) {
      // an empty sequence attends to nothing: zero output (cuda/attention.rs:65-68)
      const long long oi = ((long long)b * a.num_heads + g * NR) * HD + tid;
      if (a.out_dtype == kF32) static_cast<float *>(a.out)[oi] = 0.f;
      else static_cast<uint16_t *>(a.out)[oi] = 0;
    }
    __builtin_amdgcn_s_waitcnt(0);
    return;
  }
  const int nchunks = (len + CH - 1) / CH;
  float *stage = lds + OFF_W + wave * WSTAGE;
  uint32_t *st_x = reinterpret_cast<uint32_t *>(stage);  // [NQB][WT][NR] K partial scores (f32 bits)
  float *st_p = stage + RA;                               // [NR][WT]
  float *st_s = st_p + PW;                                // [NQB][WT]
  float *comb = st_s + SW;                                // [NR][HD], m[NR], l[NR], 2^Ev

  // ---- K/V records.  The tile's waves fetch them in kLoadGroups staggered
  // groups: group k issues only once the records of group k - 1 have
  // arrived, so device-wide the early groups' bytes come back first and their
  // passes overlap the later transfers.  Group 0 is the highest waves (the
  // query waves fetch last).  Codes, tile tt of this wave: for the
  // keys lane (l16, lg) holds qblock lg of token 16 tt + l16, for the values
  // qblock l16 % 4 of token 16 tt + 4 lg + l16 / 4 (one contiguous run of
  // four records per 16 lanes); scales: lane = token, all
  // four qblock scales in one load.  Addresses are a per-(b, g) base plus a
  // 32-bit offset inside the head. ----
  constexpr int GW = kWaves / kLoadGroups;  // waves per load group
  const int grp = (kWaves - 1 - wave) / GW;
  using I0 = std::integral_constant<int, 0>;
  using INT = std::integral_constant<int, NT>;
  const int tw_a = t0 + wave * WT;
  const uint8_t *ksbase = reinterpret_cast<const uint8_t *>(k_sc + rec0 * NQB);
  const uint8_t *vsbase = reinterpret_cast<const uint8_t *>(v_sc + rec0 * NQB);
  uint32_t kq[NT][QW], vq[NT][QW];
  uint2 ksc, vsc;
  uint32_t sq[NT];   // QJL: sign word lg of token 16 tt + l16
  uint32_t nrm = 0;  // QJL: residual norm of token lane
  const uint8_t *sgbase = reinterpret_cast<const uint8_t *>(a.qjl_signs) + rec0 * 16;
  const uint16_t *nmbase = a.qjl_norms + rec0;
  // NTC tiles from token tw into tile registers TT0 ..
  auto issue_tiles = [&](const int tw, auto tt0c, auto ntc, uint2 &ks_, uint2 &vs_, uint32_t &nm_) {
    constexpr int TT0 = decltype(tt0c)::value, NTC = decltype(ntc)::value;
    const uint32_t soff = (uint32_t)min(tw + lane, len - 1) * (NQB * 2);
    uint32_t off[NTC], voff[NTC];
#pragma unroll
    for (int tt = 0; tt < NTC; tt++) {
      off[tt] = (uint32_t)min(tw + 16 * tt + l16, len - 1) * PACKED + lg * (QW * 4);
      voff[tt] = (uint32_t)min(tw + 16 * tt + 4 * lg + (l16 >> 2), len - 1) * PACKED + (l16 & 3) * (QW * 4);
    }
#pragma unroll
    for (int tt = 0; tt < NTC; tt++)
#pragma unroll
      for (int w = 0; w < QW; w++) kq[TT0 + tt][w] = *reinterpret_cast<const uint32_t *>(kbase + off[tt] + 4 * w);
    ks_ = *reinterpret_cast<const uint2 *>(ksbase + soff);
    if constexpr (QJL) {
#pragma unroll
      for (int tt = 0; tt < NTC; tt++)
        sq[TT0 + tt] = *reinterpret_cast<const uint32_t *>(
            sgbase + (uint32_t)min(tw + 16 * tt + l16, len - 1) * 16 + lg * 4);
      nm_ = nmbase[min(tw + lane, len - 1)];
    }
#pragma unroll
    for (int tt = 0; tt < NTC; tt++)
#pragma unroll
      for (int w = 0; w < QW; w++) vq[TT0 + tt][w] = *reinterpret_cast<const uint32_t *>(vbase + voff[tt] + 4 * w);
    vs_ = *reinterpret_cast<const uint2 *>(vsbase + soff);
  };
  // Group 0 fetches before the shared setup below, so its records are on the
  // way while the pair table and the query operands are built.
  if (grp == 0) issue_tiles(tw_a, I0{}, INT{}, ksc, vsc, nrm);

  // ---- pair table from the constant codebook ----
  for (int it = tid; it < NPAIR; it += kThreads) {
    const int e = it;
    constexpr int CM = (1 << CB) - 1;  // slot codes >= 2^CB never occur
    const int i0 = e & (NC - 1) & CM, i1 = (e >> BITS) & CM;
    float c0, c1;
    if (a.cb_dev) {
      c0 = a.cb_dev[i0];
      c1 = a.cb_dev[i1];
    } else if (a.cb_args) {
      c0 = a.cb[0];
      c1 = a.cb[0];
#pragma unroll
      for (int kk = 1; kk <= CM; kk++) {
        c0 = i0 == kk ? a.cb[kk] : c0;
        c1 = i1 == kk ? a.cb[kk] : c1;
      }
    } else {
      c0 = pqo_centroid<CB>(i0);
      c1 = pqo_centroid<CB>(i1);
    }
    const float h0 = split_hi(c0), h1 = split_hi(c1);
    s_pair[it] = make_uint2(pack_f16(h0, h1), pack_f16(c0 - h0, c1 - h1));
  }
  if (tid == 0) s_ready = 0;
  if constexpr (QJL) {
    // +-1 in f16 for the four sign bits of a nibble, LSB first
    if (tid < 16) {
      auto pm1 = [&](int bit) { return ((tid >> bit) & 1) ? 0x3C00u : 0xBC00u; };
      s_nib[tid] = make_uint2(pm1(0) | (pm1(1) << 16), pm1(2) | (pm1(3) << 16));
    }
  }

  // ---- rotated, scaled queries (32-lane butterflies), before these waves
  // queue their record loads behind the query ----
  const float qscale = a.softmax_scale * kLog2e * kInvSqrt32;
  if (tid < NR * HD) {
    const int d = tid % HD;
    const int i = d & 31;
    const float v = wht32_lanes(q_value(qbits, a.q_dtype), i);
    const float qt = v * (qsign * qscale);
    s_q[tid] = qt;
    const float am = wave_max(fabsf(qt));
    if (lane == 0) s_qmax[wave] = am;
    if constexpr (QJL) {
      const float rs = rqv * (a.softmax_scale * kLog2e);
      s_rq[tid] = rs;
      const float rm = wave_max(fabsf(rs));
      if (lane == 0) s_rqmax[wave] = rm;
    }
  }

  __syncthreads();
  // Key-pass query operands.  MFMA j covers elements 4 j .. 4 j + 3 of every
  // qblock, each twice along k (against the hi and the lo part of the key
  // value), so lane (m, kg) supplies k = 8 kg + (x0, x1, x0, x1, x2, x3, x2,
  // x3), x_i = part(Q[32 kg + 4 j + i]) for row m = (qblock qb, head
  // 2 gi + rl, part) when kg == qb, zero otherwise; Q = qt * 2^-Eq, scaled
  // per head into f16's range.
  if (tid < NG * 512) {
    const int gi = tid >> 9, j = (tid >> 6) & 7, m = lane & 15, kg = lane >> 4;
    const int qb = m >> 2, rl = (m >> 1) & 1, part = m & 1, r = 2 * gi + rl;
    u32x4 val = {0u, 0u, 0u, 0u};
    if (kg == qb && r < NR) {
      const float sc = exp2i(-pow2_exponent(fmaxf(s_qmax[2 * r], s_qmax[2 * r + 1])));
      const float4 q4 = *reinterpret_cast<const float4 *>(s_q + r * HD + 32 * kg + 4 * j);
      const float x0 = q4.x * sc, x1 = q4.y * sc, x2 = q4.z * sc, x3 = q4.w * sc;
      const float h0 = split_hi(x0), h1 = split_hi(x1), h2 = split_hi(x2), h3 = split_hi(x3);
      const uint32_t w01 = part ? pack_f16(x0 - h0, x1 - h1) : pack_f16(h0, h1);
      const uint32_t w23 = part ? pack_f16(x2 - h2, x3 - h3) : pack_f16(h2, h3);
      val = u32x4{w01, w01, w23, w23};
    }
    s_qa[(gi * 8 + j) * 64 + lane] = val;
  }
  if constexpr (QJL) {
    // Correction operands: MFMA s covers sign bits 32 kg + 8 s .. + 7 of a
    // token (k = 8 kg + i); row m = (head m / 2, part m % 2) holds part(rq)
    // of those projections, rq scaled per head by 2^-Er into f16's range.
    if (tid >= kThreads - 256) {
      const int e = tid - (kThreads - 256), sl = e >> 6, ln = e & 63, m = ln & 15, kg = ln >> 4;
      u32x4 val = {0u, 0u, 0u, 0u};
      if (m < 2 * NR) {
        const int r = m >> 1, part = m & 1;
        const float sc = exp2i(-pow2_exponent(fmaxf(s_rqmax[2 * r], s_rqmax[2 * r + 1])));
        const float *src = s_rq + r * HD + 32 * kg + 8 * sl;
        uint32_t wv[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const float x0 = src[2 * i] * sc, x1 = src[2 * i + 1] * sc;
          const float h0 = split_hi(x0), h1 = split_hi(x1);
          wv[i] = part ? pack_f16(x0 - h0, x1 - h1) : pack_f16(h0, h1);
        }
        val = u32x4{wv[0], wv[1], wv[2], wv[3]};
      }
      s_ra[sl * 64 + ln] = val;
    }
  }
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);  // keep the record-dependent code below the setup
  if (grp > 0) {
    // wait (acquire: the loads below cannot move above it) until every wave
    // of the previous group has its records, then fetch ours
    if (lane == 0)
      while (__hip_atomic_load(&s_ready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < grp * GW)
        __builtin_amdgcn_s_sleep(2);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    issue_tiles(tw_a, I0{}, INT{}, ksc, vsc, nrm);
  }
  if constexpr (kLoadGroups > 1) {
    __builtin_amdgcn_s_waitcnt(0);  // this wave's records are in registers
    if (lane == 0) __hip_atomic_fetch_add(&s_ready, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  }

  float escale[NR], erscale[NR];
#pragma unroll
  for (int r = 0; r < NR; r++) {
    escale[r] = exp2i(pow2_exponent(fmaxf(s_qmax[2 * r], s_qmax[2 * r + 1])));
    if constexpr (QJL) erscale[r] = exp2i(pow2_exponent(fmaxf(s_rqmax[2 * r], s_rqmax[2 * r + 1])));
  }

  // ---- the wave's NTB tiles from token tw (tile registers TT0 ..): its
  // record (m, l, acc in units of 2^-Ev) goes to comb ----
  float m_w[NR], l_w[NR];
#pragma unroll
  for (int r = 0; r < NR; r++) {
    m_w[r] = -INFINITY;
    l_w[r] = 0.f;
  }
  int ev = 0;
  const int bq = l16 >> 2, brl = (l16 >> 1) & 1, bpart = l16 & 1;
  auto run_batch = [&](const int tw, auto tt0c, auto ntbc, const uint2 ks_, const uint2 vs_, const uint32_t nm_) {
    constexpr int TT0 = decltype(tt0c)::value, NTB = decltype(ntbc)::value;
    // ---- K pass: D[tile][(qblock, head, part)][token] over the eight
    // 4-element slices j of every qblock.  The key operand of lane (t, q) for
    // slice j is (hi pair, lo pair) of codes 4j, 4j+1 and of codes 4j+2, 4j+3
    // of qblock q of token t: two pair-table reads.  Lane (t, q) ends with
    // token t's (unscaled) qblock-q partial of each head. ----
    f32x4 dk[NTB][NG];
#pragma unroll
    for (int tt = 0; tt < NTB; tt++)
#pragma unroll
      for (int gi = 0; gi < NG; gi++) dk[tt][gi] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 8; j++) {
      u32x4 qa[NG];
#pragma unroll
      for (int gi = 0; gi < NG; gi++) qa[gi] = s_qa[(gi * 8 + j) * 64 + lane];
#pragma unroll
      for (int tt = 0; tt < NTB; tt++) {
        const uint2 e0 = s_pair[pair_code<BITS>(kq[TT0 + tt], 2 * j)];
        const uint2 e1 = s_pair[pair_code<BITS>(kq[TT0 + tt], 2 * j + 1)];
        const u32x4 kb = {e0.x, e0.y, e1.x, e1.y};
#pragma unroll
        for (int gi = 0; gi < NG; gi++) dk[tt][gi] = mfma(qa[gi], kb, dk[tt][gi]);
      }
    }
    if constexpr (QJL) {
      // sum_j rq_j (2 b_j - 1) per (head, token) on the matrix core: the sign
      // operand of lane (t, kg) for MFMA s is the +-1 pairs of byte s of its
      // sign word; the (unscaled) sums go to st_p, which the softmax
      // overwrites only after they are read
      f32x4 dq[NTB];
#pragma unroll
      for (int tt = 0; tt < NTB; tt++) dq[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int sl = 0; sl < 4; sl++) {
        const u32x4 ra = s_ra[sl * 64 + lane];
#pragma unroll
        for (int tt = 0; tt < NTB; tt++) {
          const uint32_t byte = (sq[TT0 + tt] >> (8 * sl)) & 0xffu;
          const uint2 n0 = s_nib[byte & 15u], n1 = s_nib[byte >> 4];
          dq[tt] = mfma(ra, u32x4{n0.x, n0.y, n1.x, n1.y}, dq[tt]);
        }
      }
#pragma unroll
      for (int tt = 0; tt < NTB; tt++)
#pragma unroll
        for (int u = 0; u < 2; u++) {
          const int r = 2 * lg + u;
          if (r < NR) st_p[r * WT + 16 * tt + l16] = dq[tt][2 * u] + dq[tt][2 * u + 1];
        }
    }
#pragma unroll
    for (int tt = 0; tt < NTB; tt++) {
      uint32_t *dst = st_x + (lg * WT + 16 * tt + l16) * NR;
      uint32_t xv[NR];
#pragma unroll
      for (int r = 0; r < NR; r++) xv[r] = f2u(dk[tt][r >> 1][2 * (r & 1)] + dk[tt][r >> 1][2 * (r & 1) + 1]);
      if constexpr (NR == 1) {
        dst[0] = xv[0];
      } else if constexpr (NR == 2) {
        *reinterpret_cast<uint2 *>(dst) = make_uint2(xv[0], xv[1]);
      } else {
        *reinterpret_cast<uint4 *>(dst) = make_uint4(xv[0], xv[1], xv[2], xv[3]);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // lane = token: the four qblock partials times the token's key scales
    float score[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) score[r] = 0.f;
#pragma unroll
    for (int qb = 0; qb < NQB; qb++) {
      const uint32_t sbits = (qb < 2 ? ks_.x : ks_.y) >> ((qb & 1) ? 16 : 0);
      const float sk = fabsf(f16_to_f32((uint16_t)(sbits & 0xffffu)));
      const uint32_t *src = st_x + (qb * WT + lane) * NR;
      uint32_t xv[NR];
      if constexpr (NR == 1) {
        xv[0] = src[0];
      } else if constexpr (NR == 2) {
        const uint2 t = *reinterpret_cast<const uint2 *>(src);
        xv[0] = t.x; xv[1] = t.y;
      } else {
        const uint4 t = *reinterpret_cast<const uint4 *>(src);
        xv[0] = t.x; xv[1] = t.y; xv[2] = t.z; xv[3] = t.w;
      }
#pragma unroll
      for (int r = 0; r < NR; r++) score[r] = __builtin_fmaf(u2f(xv[r]), sk, score[r]);
    }

    // ---- softmax (base 2) of this batch's tokens ----
    const int tok = tw + lane;
    const bool valid = lane < 16 * NTB && tok < len;
    float mb[NR], p[NR], lb[NR];
    float corr[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) corr[r] = 0.f;
    if constexpr (QJL) {
      const float cn = f16_to_f32((uint16_t)nm_) * a.qjl_c;
#pragma unroll
      for (int r = 0; r < NR; r++) corr[r] = st_p[r * WT + lane] * (cn * erscale[r]);
    }
#pragma unroll
    for (int r = 0; r < NR; r++) {
      const float sc = valid ? (QJL ? __builtin_fmaf(score[r], escale[r], corr[r]) : score[r] * escale[r]) : -INFINITY;
      mb[r] = wave_max(sc);
      p[r] = valid ? __builtin_amdgcn_exp2f(sc - mb[r]) : 0.f;
      st_p[r * WT + lane] = p[r];
    }
#pragma unroll
    for (int r = 0; r < NR; r++) lb[r] = wave_sum(p[r]);

    // ---- V scales * 2^-Ev to LDS (lane = token) ----
    float sv[NQB];
    float smax = 0.f;
#pragma unroll
    for (int qb = 0; qb < NQB; qb++) {
      const uint32_t sbits = (qb < 2 ? vs_.x : vs_.y) >> ((qb & 1) ? 16 : 0);
      sv[qb] = fabsf(f16_to_f32((uint16_t)(sbits & 0xffffu)));
      smax = fmaxf(smax, sv[qb]);
    }
    const int evb = pow2_exponent(wave_max(smax));
    const float vinv = exp2i(-evb);
#pragma unroll
    for (int qb = 0; qb < NQB; qb++) st_s[qb * WT + lane] = sv[qb] * vinv;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- V pass.  Weight operands, one per pair of 16-token tiles: lane
    // (n, kg) holds for column n = (qblock bq, head 2 gi + brl, part) the
    // weights of tokens 4 kg .. 4 kg + 3 of tile 2 tp and of tile 2 tp + 1 ----
    static_assert(NTB % 2 == 0, "tiles pair up along the value contraction");
    u32x4 bw[NTB / 2][NG];
    const float kpart = bpart ? -1.f : 0.f;
#pragma unroll
    for (int tp = 0; tp < NTB / 2; tp++) {
#pragma unroll
      for (int gi = 0; gi < NG; gi++) {
        const int r = min(2 * gi + brl, NR - 1);  // NR == 1: the second head's columns are never read
        uint32_t w[4];
#pragma unroll
        for (int u = 0; u < 2; u++) {
          const int tt = 2 * tp + u;
          const float4 p4 = *reinterpret_cast<const float4 *>(st_p + r * WT + 16 * tt + 4 * lg);
          const float4 s4 = *reinterpret_cast<const float4 *>(st_s + bq * WT + 16 * tt + 4 * lg);
          const float x0 = p4.x * s4.x, x1 = p4.y * s4.y, x2 = p4.z * s4.z, x3 = p4.w * s4.w;
          w[2 * u] = pack_rem(x0, x1, pack_f16(x0, x1), kpart);          // hi (part 0) or lo (part 1)
          w[2 * u + 1] = pack_rem(x2, x3, pack_f16(x2, x3), kpart);
        }
        bw[tp][gi] = u32x4{w[0], w[1], w[2], w[3]};
      }
    }
    // The value codes are decoded by the same pair-table lookup as the keys,
    // read through the transposing LDS read: lane l of a 16-lane group holds
    // qblock l % 4 of token 4 g + l / 4 (g = lane group), so lane 4 a + b
    // receives part b (hi c0, hi c1, lo c0, lo c1) of the entries of qblock a
    // for tokens 4 g .. 4 g + 3 -- the value operand's row (a, b) at those
    // tokens, two tiles per 16 x 16 x 32 product.  D then holds rows =
    // (qblock, value part), columns (qblock, head, weight part); a lane's rows
    // count only under its own qblock's columns, and hi + lo of a value sum
    // inside the lane (rows 4 g + i and 4 g + i + 2).
    // Software-pipelined over the eight pair slices: slice j + 1's products
    // are issued before slice j's sums and store, so their latency overlaps.
    f32x4 dv[2][2][NG];  // [slice parity][h][gi]
    auto v_products = [&](auto jc) {
      constexpr int j = decltype(jc)::value, sl = j & 1;
#pragma unroll
      for (int h = 0; h < 2; h++)
#pragma unroll
        for (int gi = 0; gi < NG; gi++) dv[sl][h][gi] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int tp = 0; tp < NTB / 2; tp++) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const u32x2 r0 = lds_read_tr16(s_pair + pair_code<BITS>(vq[TT0 + 2 * tp], 2 * j + h));
          const u32x2 r1 = lds_read_tr16(s_pair + pair_code<BITS>(vq[TT0 + 2 * tp + 1], 2 * j + h));
          const u32x4 va = {r0[0], r0[1], r1[0], r1[1]};
#pragma unroll
          for (int gi = 0; gi < NG; gi++) dv[sl][h][gi] = mfma(va, bw[tp][gi], dv[sl][h][gi]);
        }
      }
    };
    // lane (n, lg) holds column n at rows (qblock lg, parts hi c0, hi c1,
    // lo c0, lo c1) of pairs 2 j and 2 j + 1; the weight parts of one head
    // sit in lanes n and n ^ 1
    auto v_store = [&](auto jc) {
      constexpr int j = decltype(jc)::value, sl = j & 1;
#pragma unroll
      for (int gi = 0; gi < NG; gi++) {
        f32x4 o;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const float x = dv[sl][i >> 1][gi][i & 1] + dv[sl][i >> 1][gi][(i & 1) + 2];
          o[i] = dpp_quad_xor1(x) + x;
          // keeps the add beside its DPP read (one v_add_f32_dpp), not sunk
          // into the store's branch
          asm volatile("" : "+v"(o[i]));
        }
        const int r = 2 * gi + brl;
        if (bpart == 0 && bq == lg && r < NR) {
          *reinterpret_cast<f32x4 *>(comb + r * HD + 32 * lg + 4 * j) = o;
        }
      }
    };
    v_products(std::integral_constant<int, 0>{});
    static_for<0, 8>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      if constexpr (j + 1 < 8) v_products(std::integral_constant<int, j + 1>{});
      v_store(jc);
    });
#pragma unroll
    for (int r = 0; r < NR; r++) {
      m_w[r] = mb[r];
      l_w[r] = lb[r];
    }
    ev = evb;
  };
  run_batch(tw_a, I0{}, INT{}, ksc, vsc, nrm);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < NR; r++) {
      comb[NR * HD + r] = m_w[r];
      comb[NR * HD + NR + r] = l_w[r];
    }
    comb[NR * HD + 2 * NR] = exp2i(ev);
  }
  // s_flag 2: the workspace was initialised for fewer (sequence, KV head)
  // pairs, or for so many that this launch's partials would reach their
  // counters: this tile stores no partial and touches no counter
  if (tid == 0) s_flag = (INLINE_MERGE && (ws_hdr < a.ws_pairs || ws_hdr > a.ws_room)) ? 2 : 0;

  // ---- combine the 16 waves' records: CP consecutive lanes share one output
  // (head r, element d), each folding kWaves / CP waves, then a DPP reduction
  // over the CP lanes ----
  __syncthreads();
  const bool ws_ok = s_flag != 2;
  {
    constexpr int OUTS = NR * HD;
    constexpr int CP = kThreads / OUTS;  // 8, 4 or 2 lanes per output
    constexpr int WPP = kWaves / CP;
    constexpr int COMB = RA + PW + SW;   // offset of the record inside a wave's staging
    static_assert(CP == 2 || CP == 4 || CP == 8, "lanes per output");
    const int o = tid / CP, part = tid % CP;
    const int r = o / HD, d = o % HD;
    float mw[WPP];
    float M = -INFINITY;
#pragma unroll
    for (int i = 0; i < WPP; i++) {
      mw[i] = lds[OFF_W + (part + i * CP) * WSTAGE + COMB + NR * HD + r];
      M = fmaxf(M, mw[i]);
    }
    M = fmaxf(M, dpp_quad_xor1(M));
    if constexpr (CP >= 4) M = fmaxf(M, dpp_quad_xor2(M));
    if constexpr (CP == 8) M = fmaxf(M, __shfl_xor(M, 4, 64));
    float A = 0.f, L = 0.f;
#pragma unroll
    for (int i = 0; i < WPP; i++) {
      const float *cw = lds + OFF_W + (part + i * CP) * WSTAGE + COMB;
      const float f = (mw[i] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(mw[i] - M);
      A = __builtin_fmaf(cw[r * HD + d], f * cw[NR * HD + 2 * NR], A);
      L = __builtin_fmaf(cw[NR * HD + NR + r], f, L);
    }
    A += dpp_quad_xor1(A);
    L += dpp_quad_xor1(L);
    if constexpr (CP >= 4) {
      A += dpp_quad_xor2(A);
      L += dpp_quad_xor2(L);
    }
    if constexpr (CP == 8) {
      A += __shfl_xor(A, 4, 64);
      L += __shfl_xor(L, 4, 64);
    }
    if (part == 0 && ws_ok) {
      const long long bh = (long long)b * a.num_heads + g * NR + r;
      st_agent(&a.po[(bh * a.P + c) * HD + d], A);
      if (d == 0) {
        st_agent(&a.pm[bh * a.P + c], M);
        st_agent(&a.ps[bh * a.P + c], L);
      }
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
    int *counter = a.cnt_top - (1 + b * a.num_kv_heads + g) * kCounterStride;
    if (tid == 0 && ws_ok) {
      const int prev = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_flag = (prev == nchunks - 1);
    }
    __syncthreads();
    if (!ws_ok) {
      if (tid < NR * HD) {
        const long long oi = ((long long)b * a.num_heads + g * NR) * HD + tid;
        if (a.out_dtype == kF32) static_cast<float *>(a.out)[oi] = __builtin_nanf("");
        else static_cast<uint16_t *>(a.out)[oi] = 0x7e00;  // quiet NaN in f16 and bf16 alike
      }
    } else if (s_flag) {
      merge_and_store<NR>(a, b, g, nchunks, lds + OFF_MISC);
      if (tid == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

// Zeroes `elems` outputs of the given dtype (a fill kernel, not a memset, so
// that a captured graph replays it faithfully).
int zero_output(void *out, long long elems, int dtype, hipStream_t stream) {
  const long long bytes = elems * (dtype == kF32 ? 4 : 2);
  const long long words = (bytes + 3) / 4;  // head_dim is a multiple of 32: whole words
  if (words == 0) return TQ_OK;
  hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, stream,
                     static_cast<int *>(out), words);
  return tqh::check_launch("fill_zero_kernel");
}

// Fills n ints with zeros, except the first of the last kCounterStride
// (the header line) = hdr.
__global__ void fill_header_kernel(int *p, long long n, int hdr) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = i == n - kCounterStride ? hdr : 0;
}

// Workspace layout: po | pm | ps from the start; the header in the last
// 256-byte line below end = workspace_bytes rounded down to 256, and the
// counters (one line per (sequence, KV head)) below it.  The counters'
// place depends on workspace_bytes only, so a workspace initialised for the
// largest batch and length serves every smaller call: their partials end
// lower and their counters are a subset of the zeroed ones.
constexpr size_t kLine = kCounterStride * sizeof(int);
struct WsLayout {
  size_t po, pm, ps, parts, total;
  int P;
};

WsLayout ws_layout(int batch, int num_heads, int num_kv_heads, int head_dim, int max_len) {
  auto al = [](size_t x) { return (x + kLine - 1) & ~(kLine - 1); };
  WsLayout w{};
  w.P = (max_len + kChunk - 1) / kChunk;
  const size_t bhp = (size_t)batch * num_heads * w.P;
  w.po = 0;
  w.pm = al(w.po + bhp * head_dim * sizeof(float));
  w.ps = al(w.pm + bhp * sizeof(float));
  w.parts = al(w.ps + bhp * sizeof(float));
  w.total = w.parts + ((size_t)batch * num_kv_heads + 1) * kLine;
  return w;
}

AttnArgs base_args() {
  AttnArgs a{};
  a.out_dtype = kF32;
  return a;
}

template <int BITS, int MODE, int NR, bool INLINE>
void launch_decode_nr(const AttnArgs &a, dim3 grid, hipStream_t st) {
  // len_hint: the single length, or -1 when the lengths are per sequence
  const int len_hint = a.kv_lens ? -1 : max(a.single_len, 0);
  hipLaunchKernelGGL((attn_decode_kernel<BITS, MODE, NR, INLINE>), grid, dim3(kThreads), 0, st, a.k_idx, a.v_idx,
                     a.k_sc, a.v_sc, a.seq_stride, a.kv_head_stride, len_hint, a);
}

template <int BITS, int MODE, bool INLINE>
int launch_decode_m(const AttnArgs &a, int nr, dim3 grid, hipStream_t st) {
  if (nr == 1) launch_decode_nr<BITS, MODE, 1, INLINE>(a, grid, st);
  else if (nr == 2) launch_decode_nr<BITS, MODE, 2, INLINE>(a, grid, st);
  else launch_decode_nr<BITS, MODE, 4, INLINE>(a, grid, st);
  return tqh::check_launch("attn_decode_kernel");
}

template <bool INLINE>
int launch_decode(const AttnArgs &a, int bits, int mode, int nr, dim3 grid, hipStream_t st) {
  if (bits == 3) {
    if (mode == kModePqo) return launch_decode_m<3, kModePqo, INLINE>(a, nr, grid, st);
    if (mode == kModePq) return launch_decode_m<3, kModePq, INLINE>(a, nr, grid, st);
    return launch_decode_m<3, kModeTq, INLINE>(a, nr, grid, st);
  }
  if (mode == kModePqo) return launch_decode_m<4, kModePqo, INLINE>(a, nr, grid, st);
  if (mode == kModePq) return launch_decode_m<4, kModePq, INLINE>(a, nr, grid, st);
  return launch_decode_m<4, kModeTq, INLINE>(a, nr, grid, st);
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
  // header = batch * num_kv_heads, the counters below it zero
  const size_t end = workspace_bytes & ~(kLine - 1);
  const int pairs = batch * num_kv_heads;
  const long long n = (long long)((size_t)(pairs + 1) * kLine / sizeof(int));
  int *hdr = reinterpret_cast<int *>(static_cast<char *>(workspace) + end - kLine);
  hipLaunchKernelGGL(fill_header_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                     hdr - (long long)pairs * kCounterStride, n, pairs);
  return tqh::check_launch("fill_header_kernel");
}

namespace {

// Where a decode launch keeps its split-K partials and counters: the
// partials from `base`, the counter of pair i at cnt_top - (i + 1) lines,
// *hdr = the number of zeroed counters below cnt_top.
struct DecodeWs {
  char *base = nullptr;
  int *cnt_top = nullptr;
  const int *hdr = nullptr;
  // host-side view of the same: bytes the partials may use (up to the lowest
  // zeroed counter a valid call can have), and the zeroed pairs (0: the
  // caller's workspace, known to the device only)
  size_t part_bytes = 0;
  int pairs = 0;
};

// A caller's workspace: header in the last line below the rounded-down end,
// counters below it.
DecodeWs caller_ws(void *workspace, size_t workspace_bytes) {
  DecodeWs d;
  d.base = static_cast<char *>(workspace);
  const size_t end = workspace_bytes & ~(kLine - 1);
  d.cnt_top = end >= kLine ? reinterpret_cast<int *>(d.base + end - kLine) : nullptr;
  d.hdr = d.cnt_top;
  d.part_bytes = end >= kLine ? end - kLine : 0;
  return d;
}

int decode_attention_ws(const void *q, int q_dtype, const uint8_t *k_indices, const uint16_t *k_scales,
                        const uint8_t *v_indices, const uint16_t *v_scales, const float *rq, const uint8_t *qjl_signs,
                        const uint16_t *qjl_norms, const int *kv_lens, int host_len, int batch, int num_heads,
                        int num_kv_heads, int head_dim, int bits, size_t outlier_blocks, int norm_mode,
                        int max_kv_len, long long kv_head_stride, long long seq_stride, float softmax_scale, void *out,
                        int out_dtype, const DecodeWs *wsd, size_t workspace_bytes, hipStream_t stream);

}  // namespace

// host_len >= 0 (with kv_lens null): every sequence holds host_len tokens;
// max_kv_len fixes the workspace layout either way.
int tqh::decode_attention(const void *q, int q_dtype, const uint8_t *k_indices, const uint16_t *k_scales,
                          const uint8_t *v_indices, const uint16_t *v_scales, const float *rq,
                          const uint8_t *qjl_signs, const uint16_t *qjl_norms, const int *kv_lens, int host_len,
                          int batch, int num_heads, int num_kv_heads, int head_dim, int bits, size_t outlier_blocks,
                          int norm_mode, int max_kv_len, long long kv_head_stride, long long seq_stride,
                          float softmax_scale, void *out, int out_dtype, void *workspace, size_t workspace_bytes,
                          hipStream_t stream) {
  const DecodeWs d = caller_ws(workspace, workspace_bytes);
  return decode_attention_ws(q, q_dtype, k_indices, k_scales, v_indices, v_scales, rq, qjl_signs, qjl_norms, kv_lens,
                             host_len, batch, num_heads, num_kv_heads, head_dim, bits, outlier_blocks, norm_mode,
                             max_kv_len, kv_head_stride, seq_stride, softmax_scale, out, out_dtype,
                             workspace ? &d : nullptr, workspace_bytes, stream);
}

namespace {

int decode_attention_ws(const void *q, int q_dtype, const uint8_t *k_indices, const uint16_t *k_scales,
                        const uint8_t *v_indices, const uint16_t *v_scales, const float *rq, const uint8_t *qjl_signs,
                        const uint16_t *qjl_norms, const int *kv_lens, int host_len, int batch, int num_heads,
                        int num_kv_heads, int head_dim, int bits, size_t outlier_blocks, int norm_mode,
                        int max_kv_len, long long kv_head_stride, long long seq_stride, float softmax_scale, void *out,
                        int out_dtype, const DecodeWs *wsd, size_t workspace_bytes, hipStream_t stream) {
  int rc = check_common(num_heads, num_kv_heads, head_dim, bits);
  if (rc) return rc;
  tqh::PolarCodec codec;
  rc = tqh::polar_codec(bits, norm_mode, outlier_blocks, head_dim / 32, codec);
  if (rc) return rc;
  if (codec.mixed)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT,
                     "fused decode takes outlier_blocks 0 or all (mixed configs: dequantize and attend)");
  const bool qjl = qjl_signs != nullptr;
  if (qjl && codec.outlier)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "QJL correction applies to the standard codebook (outlier_blocks 0)");
  if (!tqh::valid_dtype(q_dtype) || !tqh::valid_dtype(out_dtype))
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "unknown dtype");
  if (batch <= 0) return TQ_OK;
  if (max_kv_len <= 0) {
    // nothing to attend to: zero output (cuda/attention.rs:65-68)
    if (!out) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
    return zero_output(out, (long long)batch * num_heads * head_dim, out_dtype, stream);
  }
  if (!q || !k_indices || !k_scales || !v_indices || !v_scales || !out)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
  if (!kv_lens && host_len < 0) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null kv_lens");
  if (qjl && (!rq || !qjl_norms)) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "QJL needs rq, signs and norms");
  if (kv_head_stride < max_kv_len)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "kv_head_stride %lld < max_kv_len %d", kv_head_stride, max_kv_len);
  if (batch > 1 && seq_stride < (long long)num_kv_heads * kv_head_stride)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "seq_stride %lld overlaps the KV heads of a sequence", seq_stride);
  const WsLayout w = ws_layout(batch, num_heads, num_kv_heads, head_dim, max_kv_len);
  const long long pairs = (long long)batch * num_kv_heads;
  if (!wsd) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null workspace");
  if (wsd->pairs == 0) {  // the caller's workspace
    if (workspace_bytes < w.total)
      return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "workspace too small: %zu < %zu", workspace_bytes, w.total);
  } else if (pairs > wsd->pairs || w.parts > wsd->part_bytes) {
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT,
                     "decode needs %zu bytes of split-K partials and %lld counters; the library's scratch holds "
                     "%zu bytes and %d counters",
                     w.parts, pairs, wsd->part_bytes, wsd->pairs);
  }
  AttnArgs a = base_args();
  char *ws = wsd->base;
  a.q = q;
  a.q_dtype = q_dtype;
  a.k_idx = k_indices;
  a.k_sc = k_scales;
  a.v_idx = v_indices;
  a.v_sc = v_scales;
  a.kv_lens = kv_lens;
  a.single_len = kv_lens ? 0 : min(max(host_len, 0), max_kv_len);
  a.max_len = max_kv_len;
  a.num_heads = num_heads;
  a.num_kv_heads = num_kv_heads;
  a.kv_head_stride = kv_head_stride;
  a.seq_stride = seq_stride;
  a.softmax_scale = softmax_scale;
  a.po = reinterpret_cast<float *>(ws + w.po);
  a.pm = reinterpret_cast<float *>(ws + w.pm);
  a.ps = reinterpret_cast<float *>(ws + w.ps);
  a.cnt_top = wsd->cnt_top;
  a.ws_hdr = wsd->hdr;
  a.ws_pairs = (int)pairs;
  a.ws_room = (int)(((size_t)(reinterpret_cast<char *>(wsd->cnt_top) - ws) - w.parts) / kLine);
  a.P = w.P;
  a.out = out;
  a.out_dtype = out_dtype;
  a.rq = rq;
  a.qjl_signs = reinterpret_cast<const uint32_t *>(qjl_signs);
  a.qjl_norms = qjl_norms;
  a.qjl_c = tq_qjl_bias_scale(head_dim);
  if (codec.norm_mode == TQ_NORM_L2NORM) {
    a.cb_args = 1;
    for (int i = 0; i < codec.cb.nc; i++) a.cb[i] = codec.cb.c[i];
  }
  const int mode = codec.outlier ? kModePqo : (qjl ? kModeTq : kModePq);
  const dim3 grid((unsigned)w.P, (unsigned)num_kv_heads, (unsigned)batch);
  return launch_decode<true>(a, bits, mode, num_heads / num_kv_heads, grid, stream);
}

}  // namespace

extern "C" int tq_cache_decode_attention(const void *q, int q_dtype, const uint8_t *k_indices,
                                         const uint16_t *k_scales, const uint8_t *v_indices,
                                         const uint16_t *v_scales, const float *rq, const uint8_t *qjl_signs,
                                         const uint16_t *qjl_norms, const int *kv_lens, int batch, int num_heads,
                                         int num_kv_heads, int head_dim, int bits, size_t outlier_blocks,
                                         int norm_mode, int max_kv_len, long long kv_head_stride,
                                         long long seq_stride, float softmax_scale, void *out, int out_dtype,
                                         void *workspace, size_t workspace_bytes, hipStream_t stream) {
  return tqh::decode_attention(q, q_dtype, k_indices, k_scales, v_indices, v_scales, rq, qjl_signs, qjl_norms, kv_lens,
                               max_kv_len, batch, num_heads, num_kv_heads, head_dim, bits, outlier_blocks, norm_mode,
                               max_kv_len, kv_head_stride, seq_stride, softmax_scale, out, out_dtype, workspace,
                               workspace_bytes, stream);
}

extern "C" int tq_pqo_decode_attention(const void *q, int q_dtype, const uint8_t *k_indices, const uint16_t *k_scales,
                                       const uint8_t *v_indices, const uint16_t *v_scales, const int *kv_lens,
                                       int batch, int num_heads, int num_kv_heads, int head_dim, int bits,
                                       int max_kv_len, long long kv_head_stride, long long seq_stride,
                                       float softmax_scale, void *out, int out_dtype, void *workspace,
                                       size_t workspace_bytes, hipStream_t stream) {
  return tq_cache_decode_attention(q, q_dtype, k_indices, k_scales, v_indices, v_scales, nullptr, nullptr, nullptr,
                                   kv_lens, batch, num_heads, num_kv_heads, head_dim, bits, TQ_OUTLIER_ALL,
                                   TQ_NORM_MAXNORM, max_kv_len, kv_head_stride, seq_stride, softmax_scale, out,
                                   out_dtype, workspace, workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// Decode without a caller workspace and without any allocation: the split-K
// partials and counters live in a file-scope device array.  Static storage
// starts zeroed, so the counters are zero before the first call; every call
// leaves the counters it used at zero again (the merging tile re-arms them)
// and overwrites the partials it reads.  scratch_pairs holds the number of
// counters below the array's end (the kernels' workspace header), set by
// its static initializer.  All calls on one device share that device's
// copy: calls that overlap in time on one device race.
// ---------------------------------------------------------------------------
namespace {

constexpr size_t kScratchBytes = size_t(8) << 20;  // 8 MiB per device
constexpr int kScratchPairs = 1024;                // (sequence, KV head) pairs
static_assert(kScratchPairs * kLine < kScratchBytes, "room for partials");

__device__ __align__(256) int scratch[kScratchBytes / sizeof(int)];
__device__ int scratch_pairs = kScratchPairs;

constexpr int kMaxDevices = 64;
struct ScratchDev {
  char *base = nullptr;
  int *pairs = nullptr;
};
std::mutex g_scratch_mu;
ScratchDev g_scratch[kMaxDevices];

// The device addresses of scratch and scratch_pairs on the current device,
// looked up once per device (host code never passes the arrays' names).
int scratch_for_current_device(DecodeWs *d) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return tqh::fail(TQ_ERR_DEVICE, "no current device (or device index %d beyond %d)", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ScratchDev &s = g_scratch[dev];
  if (!s.base) {
    void *p = nullptr, *c = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return tqh::fail(TQ_ERR_DEVICE, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    e = hipGetSymbolAddress(&c, HIP_SYMBOL(scratch_pairs));
    if (e != hipSuccess || !c)
      return tqh::fail(TQ_ERR_DEVICE, "hipGetSymbolAddress(scratch_pairs) on device %d: %s", dev,
                       hipGetErrorString(e));
    s.base = static_cast<char *>(p);
    s.pairs = static_cast<int *>(c);
  }
  d->base = s.base;
  d->cnt_top = reinterpret_cast<int *>(s.base + kScratchBytes);
  d->hdr = s.pairs;
  d->part_bytes = kScratchBytes - (size_t)kScratchPairs * kLine;
  d->pairs = kScratchPairs;
  return TQ_OK;
}

}  // namespace

extern "C" int tq_pqo_decode_attention_noalloc(const void *q, int q_dtype, const uint8_t *k_indices,
                                               const uint16_t *k_scales, const uint8_t *v_indices,
                                               const uint16_t *v_scales, const int *kv_lens, int batch,
                                               int num_heads, int num_kv_heads, int head_dim, int bits,
                                               int max_kv_len, long long kv_head_stride, long long seq_stride,
                                               float softmax_scale, void *out, int out_dtype, hipStream_t stream) {
  DecodeWs d;
  int rc = scratch_for_current_device(&d);
  if (rc) return rc;
  return decode_attention_ws(q, q_dtype, k_indices, k_scales, v_indices, v_scales, nullptr, nullptr, nullptr, kv_lens,
                             max_kv_len, batch, num_heads, num_kv_heads, head_dim, bits, TQ_OUTLIER_ALL,
                             TQ_NORM_MAXNORM, max_kv_len, kv_head_stride, seq_stride, softmax_scale, out, out_dtype,
                             &d, 0, stream);
}

extern "C" int tq_fused_attention(const float *q, const uint8_t *k_indices, const uint16_t *k_scales,
                                  const uint8_t *v_indices, const uint16_t *v_scales, const float *codebook,
                                  const float *sign_pattern, float *output, float *partial_out, float *partial_max,
                                  float *partial_sum, const uint8_t *qjl_signs, const uint16_t *qjl_residual_norms,
                                  const float *rq, int qjl_enabled, int num_attention_heads, int num_kv_heads,
                                  int head_dim, int kv_len, int kv_stride, int packed_dim, int num_qblocks, int bits,
                                  float softmax_scale, int num_partitions, hipStream_t stream) {
  if (kv_len == 0 && output && num_attention_heads > 0 && head_dim > 0)  // attention.rs:65-68
    return zero_output(output, (long long)num_attention_heads * head_dim, kF32, stream);
  if (kv_len == 0 || num_kv_heads == 0) return TQ_OK;  // tq_attention_kernel.cu:366
  if (qjl_enabled && (!qjl_signs || !qjl_residual_norms || !rq))
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "qjl_enabled needs signs, residual norms and rq");
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
  // The codebook (indexed by code: 2^bits entries, 2^(bits-1) used by TQ
  // records) and the 32 decode signs are the caller's device tensors, read by
  // the kernels as tq_attention_kernel.cu:127-130 reads them (pqo.rs:134-160
  // passes pre.outlier_centroids, so an L2Norm cache brings its Beta tables);
  // with qjl_enabled the records are TQ records (standard (bits-1)-bit
  // codebook, the QJL branch of tq_attention_kernel.cu:192-231).  The
  // caller's partial buffers (sized for 512-token partitions) hold this
  // entry's 1024-token partials.
  AttnArgs a = base_args();
  a.cb_dev = codebook;
  a.sg_dev = sign_pattern;
  a.q = q;
  a.q_dtype = kF32;
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
  a.cnt_top = nullptr;
  a.ws_hdr = nullptr;
  a.P = num_partitions;
  a.out = output;
  a.out_dtype = kF32;
  a.rq = rq;
  a.qjl_signs = reinterpret_cast<const uint32_t *>(qjl_signs);
  a.qjl_norms = qjl_residual_norms;
  a.qjl_c = tq_qjl_bias_scale(head_dim);
  const int nr = num_attention_heads / num_kv_heads;
  const int P = (kv_len + kChunk - 1) / kChunk;
  rc = launch_decode<false>(a, bits, qjl_enabled ? kModeTq : kModePqo, nr, dim3((unsigned)P, (unsigned)num_kv_heads, 1u),
                            stream);
  if (rc) return rc;
  const dim3 mgrid((unsigned)num_kv_heads, 1u);
  if (nr == 1) hipLaunchKernelGGL((attn_merge_kernel<1>), mgrid, dim3(kThreads), 0, stream, a);
  else if (nr == 2) hipLaunchKernelGGL((attn_merge_kernel<2>), mgrid, dim3(kThreads), 0, stream, a);
  else hipLaunchKernelGGL((attn_merge_kernel<4>), mgrid, dim3(kThreads), 0, stream, a);
  return tqh::check_launch("attn_merge_kernel");
}
