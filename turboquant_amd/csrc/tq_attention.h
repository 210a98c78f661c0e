// tq_attention.h -- internal to the library: the fused decode's launch
// arguments, its configuration table (workgroup shape per head_dim, query
// heads per KV head and cache mode), the split-K merge shared by the decode
// kernel and the reference ABI's merge launch, and the per-(bits, mode)
// launchers.  tq_attention.hip holds the C-ABI entries and the workspace;
// each tq_attention_k<bits>_<mode>.hip compiles the decode kernels of one
// bit width and cache mode (separate units so they build in parallel).
#pragma once

#include "tq_common.h"
#include "tq_device.h"
#include "tq_mfma.h"

#include <type_traits>

namespace tqa {

using namespace tqd;
using namespace tqm;

// Tokens per partition of the reference ABI's partial buffers
// (cuda/attention.rs:13,70-77: num_partitions = ceil(kv_len / 512)).
constexpr int kRefPartition = 512;

// One split-K counter per (sequence, KV head), each on its own 256-byte line
// so the tiles' arrivals at different counters do not queue on one line.
constexpr int kCounterStride = 64;  // ints

// Cache codec of the attended records: PQO (outlier codebook, CB = BITS),
// PQ (standard (BITS - 1)-bit codebook in BITS-wide slots) and TQ (PQ plus
// the QJL correction of the keys' residuals, tq.rs:185-253 and the QJL
// branch of tq_attention_kernel.cu:192-231).
enum Mode : int { kModePqo = 0, kModePq = 1, kModeTq = 2 };

struct AttnArgs {
  // Read by every workgroup before its first record load, so kept together
  // at the head of the block (the kernel reads them in one batch).
  const void *q;
  // reference ABI (tq_fused_attention): the caller's device codebook
  // (indexed by code, tq_attention_kernel.cu:129) and 32 decode signs
  // (applied before the WHT, tq_attention_kernel.cu:45), or null
  const float *cb_dev;
  const float *sg_dev;
  const int *ws_hdr;         // see cnt_top
  const int *kv_lens;        // device lengths, or null -> single_len
  const float *rq;           // TQ: see below
  int q_dtype;
  int ngroups;               // head groups per KV head (grid.y = num_kv_heads * ngroups)
  int nr;                    // query heads per KV head
  int num_heads;
  int max_len;               // host bound; device lengths are clamped to it
  const uint8_t *k_idx;
  const uint16_t *k_sc;
  const uint8_t *v_idx;
  const uint16_t *v_sc;
  int single_len;
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
  int ws_pairs;
  int ws_room;
  int P;                     // chunk stride per (b, h) in the partial arrays
  int chunk;                 // tokens per chunk (a wave pass per TPW tokens)
  int cpr;                   // chunks per workgroup: workgroup c takes chunks [c cpr, (c + 1) cpr)
  // balanced split of a range launch (0: off): workgroups, sequences and
  // (KV head x head group) pairs per sequence; the grid is (bal_nwg, 1, 1)
  int bal_nwg;
  int bal_batch;
  int bal_ny;
  void *out;
  int out_dtype;
  // TQ: rq [b][h][head_dim] f32 = R q (precompute_query_projections); per
  // record, signs [16] u8 of R r and the f16 residual norm |r|; qjl_c =
  // f32(sqrt(pi/2)) / sqrt(head_dim)
  const uint32_t *qjl_signs;
  const uint16_t *qjl_norms;
  float qjl_c;
  // TQ without rq: the sign matrix (row j: head_dim / 32 words, bit c set =
  // -1, tq_qjl_sign_matrix) and 1 / sqrt(head_dim); the decode computes rq
  // = R q itself, summed in column order as tq_qjl_project (qjl.rs:196-208)
  const uint32_t *rmat;
  float qjl_inv;
  // cb_args: the codebook comes from cb (L2Norm tables) instead of the
  // MaxNorm constants compiled in
  int cb_args;
  float cb[16];
};

// Query element as stored (f32 bits or a 16-bit pattern), converted
// separately so that the wait for the load lands at the first use.
__device__ __forceinline__ float q_value(uint32_t bits, int qt) {
  if (qt == kF32) return u2f(bits);
  if (qt == kBF16) return bf16_to_f32((uint16_t)bits);
  return f16_to_f32((uint16_t)bits);
}

// Loads with the coherence of an agent-scope atomic load (SC1: read at the
// device-coherent level): the partials were written by other workgroups,
// possibly on other dies.  Buffer loads over a uniform descriptor, so a
// round's loads go out together with no per-lane address arithmetic.
__device__ __forceinline__ float4 ld_agent16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 16));
}
__device__ __forceinline__ float ld_agent4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, 16));
}


constexpr int dmin(int x, int y) { return x < y ? x : y; }
// LDS of the split-K merge (merge_heads) for a workgroup of `waves` waves
constexpr int merge_lds(int waves) { return waves * 256 * 4 + waves * 8 * 2 * 4; }

template <int BITS_, int MODE_, int NQB_, int HG_, int TPW_, int WAVES_>
struct DecCfg {
  static constexpr int BITS = BITS_, MODE = MODE_, NQB = NQB_, HG = HG_, TPW = TPW_, WAVES = WAVES_;
  static constexpr int CB = MODE == kModePqo ? BITS : BITS - 1;  // codebook bits
  static constexpr bool QJL = MODE == kModeTq;
  static constexpr int HD = 32 * NQB;
  static constexpr int QW = BITS;                // 32-bit words per qblock record
  static constexpr int PACKED = NQB * QW * 4;    // bytes per token record
  // qblocks per instruction (K and V) and heads per instruction
  static constexpr int QPM = dmin(NQB, HG <= 2 ? 4 : (HG <= 4 ? 2 : 1));
  static constexpr int HPM = 8 / QPM;
  static constexpr int QG = NQB / QPM;           // qblock groups (K) / sets (V)
  static constexpr int ES = 4 / QPM;             // parts of a qblock stream (lanes per qblock)
  static constexpr int KJ = 2 * QPM;             // K slices (4 elements each) per group
  static constexpr int PPL = 16 / ES;            // pairs per lane part (= V slices per set)
  static constexpr int NW = ES == 1 ? QW : 2;    // record words a lane holds per group
  static constexpr int NKT = TPW / 16, NVP = TPW / 32;
  // grid V pass: the row stride (bytes) of a staged V record, padded by 8 so
  // that the 16 rows a transposing read addresses fall in distinct banks
  static constexpr int VRS = PACKED + 8;
#ifndef TQ_DECODE_LOOKAHEAD
#define TQ_DECODE_LOOKAHEAD 2
#endif
  static constexpr int LOOKAHEAD = TQ_DECODE_LOOKAHEAD;  // load groups in flight per wave
  static constexpr int THREADS = 64 * WAVES, CHUNK = WAVES * TPW;
  static constexpr int NPAIR = 1 << (2 * BITS);
  static constexpr int SW4 = (NQB + 3) / 4;      // QJL: sign words per lane and tile
  static constexpr int TPL = TPW / 64;           // V-scale tokens per lane
  static constexpr bool QA_REGS = QG * KJ <= 8;  // query operands in registers (else LDS)
  // LDS carve (32-bit words)
  static constexpr int OFF_PAIR = 0;                                  // uint2 [NPAIR]
  static constexpr int OFF_NIB = OFF_PAIR + 2 * NPAIR;                // QJL uint2 [16]
  // the key-pass query operands, u32x4 [QG*KJ][64] (read per instruction,
  // or by QA_REGS configurations into registers at each chunk's K pass)
  static constexpr int OFF_QA = (OFF_NIB + (QJL ? 32 : 0) + 3) & ~3;
  static constexpr int OFF_W = OFF_QA + QG * KJ * 64 * 4;
  // the query setup lives in the wave staging area until the K pass starts
  static constexpr int OFF_Q = OFF_W;                                 // [HG][HD] scaled rotated query
  static constexpr int OFF_QMAX = OFF_Q + HG * HD;                    // [HG][NQB] block max |qt|
  static constexpr int OFF_RQ = OFF_QMAX + HG * NQB;                  // QJL [HG][HD]
  static constexpr int OFF_RQMAX = OFF_RQ + (QJL ? HG * HD : 0);      // QJL [HG][NQB]
  static constexpr int OFF_QSUM = OFF_RQMAX + (QJL ? HG * NQB : 0);   // [HG][NQB] block sums of the query
  static constexpr int SETUP_END = OFF_QSUM + (BITS == 4 && MODE == kModePqo ? HG * NQB : 0);
  // per wave: weights p [HG][TPW] and |s_V| 2^-Ev [NQB][TPW] of the current
  // chunk for the V pass; the wave's value sums acc [HG][HD] over its chunks;
  // then m [HG], l [HG], 2^Ev and the chunk's rescale factors [HG]
  // (rows PSTR words apart, padded by 16 bytes, so that the rows of
  // different heads and qblocks that one V-pass read touches sit in
  // different banks)
  static constexpr int PSTR = TPW + 4;
  static constexpr int WP = HG * PSTR;
  static constexpr int WS = NQB * PSTR;
  static constexpr int WC = WP + WS;
  static constexpr int WM = WC + HG * HD;
  static constexpr int WSTAGE = (WM + 3 * HG + 1 + 3) & ~3;
  static constexpr int TOTAL = OFF_W + WAVES * WSTAGE;
  static constexpr int MERGE_LDS = merge_lds(WAVES);
  static_assert(SETUP_END <= TOTAL, "the query setup fits the staging area");
  static_assert(HG >= 1 && HG <= 8, "heads per group");
  static_assert(TPW % 64 == 0, "whole V-scale loads per lane");
  static_assert(QPM * HPM == 8 && HPM >= HG, "one instruction serves every head");
  static_assert(WAVES == 4 || WAVES == 8 || WAVES == 16, "waves per workgroup");
  // does the workgroup's LDS (with the merge's scratch) fit 64 KiB (the
  // 8-wave form is taken only then), and gfx950's 160 KiB at all?
  static constexpr bool LDS_FITS = TOTAL * 4 + MERGE_LDS <= 64 * 1024;
  static constexpr bool LDS_OK = TOTAL * 4 + MERGE_LDS <= 160 * 1024;
  // The grid passes (4-bit codes on the MaxNorm codebook) read no codebook
  // table and take one query operand per qblock instead of per slice pair:
  // their layout starts the query operands at 0 and everything from OFF_W
  // on G_SHIFT words lower; each wave also stages a 64-token block of V
  // records (VSTAGE bytes for the workgroup, a separate array).
  static constexpr int G_OFF_W = QG * QPM * 64 * 4;
  static constexpr int G_SHIFT = OFF_W - G_OFF_W;
  static constexpr int VSTAGE = WAVES * 64 * VRS;
  static constexpr bool G_LDS_OK = (TOTAL - G_SHIFT) * 4 + MERGE_LDS + VSTAGE <= 160 * 1024;
};

// A buffer resource over the bytes [off, total) of the records at base:
// loads past the end return zeros.  The tile offset moves the base (scalar
// arithmetic) rather than riding in the instruction's scalar offset, so
// every byte a load touches is inside the range check.
// (The arguments are wave-uniform; readfirstlane keeps the descriptor in
// scalar registers, where a buffer instruction takes it.)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rec_rsrc(const void *base, uint32_t total, uint32_t off = 0) {
  const int d = (int)(total - off);  // both below 2^31 (the host bounds a sequence's records)
  const uint32_t n = (uint32_t)__builtin_amdgcn_readfirstlane(d > 0 ? d : 0);
  const uint64_t p = reinterpret_cast<uint64_t>(base) + off;
  const uint64_t ps = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(p >> 32)) << 32) |
                      (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)p);
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void *>(ps), (short)0, (int)n, 0x00020000);
}
// N consecutive 32-bit words at voff + soff of a buffer
template <int N>
__device__ __forceinline__ void buf_words(uint32_t (&w)[N], __amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  if constexpr (N == 1) {
    w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
  } else if constexpr (N == 2) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
    w[0] = v[0];
    w[1] = v[1];
  } else if constexpr (N == 3) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b96(r, voff, soff, 0);
    w[0] = v[0];
    w[1] = v[1];
    w[2] = v[2];
  } else {
    static_assert(N == 4, "1 to 4 words");
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    w[0] = v[0];
    w[1] = v[1];
    w[2] = v[2];
    w[3] = v[3];
  }
}

// ---------------------------------------------------------------------------
// Split-K merge and inverse rotation of the nr query heads of (b, g):
//   o = inv * H(sg * sum_c 2^(m_c - M) acc_c) / sum_c 2^(m_c - M) l_c
// (tq_attention_kernel.cu:299-332; 0 when the sum is 0).  Outputs go in
// rounds of 256; in a round each of the W waves is one lane set folding every
// W-th chunk of four consecutive outputs per lane (one 16-byte device-coherent
// load per chunk, MAXC chunks per lane in one latency round, an online
// update beyond); the W sets meet once in LDS.
// ---------------------------------------------------------------------------
template <int HD, int W>
__device__ void merge_heads(const AttnArgs &a, int b, int g, int nchunks) {
  constexpr int MAXC = 64 / W;
  __shared__ __attribute__((aligned(16))) float s_ma[W * 256];
  __shared__ float s_mml[W * 8 * 2];
  static_assert(sizeof(s_ma) + sizeof(s_mml) == merge_lds(W), "merge scratch");
  const int tid = threadIdx.x, part = tid >> 6, quad = tid & 63;
  const long long bh0 = (long long)b * a.num_heads + (long long)g * a.nr;
  const int outs = a.nr * HD;
  for (int o0 = 0; o0 < outs; o0 += 256) {
    const int oq = o0 + 4 * quad;  // this lane's first output
    const bool active = oq < outs;
    const int r = active ? oq / HD : 0, d0 = oq - r * HD;
    // one descriptor over the partial rows of the round's heads (uniform: a
    // per-lane descriptor would cost a waterfall loop per load); the lane's
    // head and chunk ride in the offset.  The round's heads hold hrn * HD <=
    // 256 outputs per chunk, so the range is at most 1 KiB x P (P below
    // 2^20, checked on the host).
    const int hr0 = o0 / HD, hrn = min(a.nr - hr0, (256 + HD - 1) / HD);
    const __amdgpu_buffer_rsrc_t rsrc =
        rec_rsrc(a.po + (bh0 + hr0) * a.P * HD, (uint32_t)(hrn * a.P * HD * (int)sizeof(float)));
    const uint32_t lane_off = (uint32_t)(((r - hr0) * a.P * HD + d0) * (int)sizeof(float));
    const __amdgpu_buffer_rsrc_t rm = rec_rsrc(a.pm + (bh0 + hr0) * a.P, (uint32_t)(hrn * a.P * (int)sizeof(float)));
    const __amdgpu_buffer_rsrc_t rl = rec_rsrc(a.ps + (bh0 + hr0) * a.P, (uint32_t)(hrn * a.P * (int)sizeof(float)));
    const uint32_t ml_off = (uint32_t)((r - hr0) * a.P * (int)sizeof(float));
    float4 pv[MAXC];
    float pm[MAXC], pl[MAXC];
#pragma unroll
    for (int k = 0; k < MAXC; k++) {
      const int cc = part + W * k;
      const bool ok = active && cc < nchunks;
      pv[k] = ok ? ld_agent16(rsrc, lane_off + (uint32_t)(cc * HD * 4)) : make_float4(0.f, 0.f, 0.f, 0.f);
      pm[k] = ok ? ld_agent4(rm, ml_off + (uint32_t)cc * 4u) : -INFINITY;
      pl[k] = ok ? ld_agent4(rl, ml_off + (uint32_t)cc * 4u) : 0.f;
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
    for (int cc = part + W * MAXC; active && cc < nchunks; cc += W) {  // long contexts only
      const float m = ld_agent4(rm, ml_off + (uint32_t)cc * 4u), l = ld_agent4(rl, ml_off + (uint32_t)cc * 4u);
      const float4 v = ld_agent16(rsrc, lane_off + (uint32_t)(cc * HD * 4));
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
    if (active) {
      *reinterpret_cast<float4 *>(s_ma + part * 256 + 4 * quad) = A;
      if (d0 == 0) {
        const int rl = (oq - o0) / HD;
        s_mml[2 * (part * 8 + rl)] = M;
        s_mml[2 * (part * 8 + rl) + 1] = L;
      }
    }
    __syncthreads();
    const int o = o0 + tid;
    if (tid < 256 && o < outs) {  // whole 32-lane blocks
      const int rl = tid / HD, d = o - (o / HD) * HD;
      float Mx = -INFINITY;
#pragma unroll
      for (int p = 0; p < W; p++) Mx = fmaxf(Mx, s_mml[2 * (p * 8 + rl)]);
      float At = 0.f, Lt = 0.f;
#pragma unroll
      for (int p = 0; p < W; p++) {
        const float mp = s_mml[2 * (p * 8 + rl)];
        const float f = mp == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mp - Mx);
        At = __builtin_fmaf(s_ma[p * 256 + tid], f, At);
        Lt = __builtin_fmaf(s_mml[2 * (p * 8 + rl) + 1], f, Lt);
      }
      const int i = d & 31;
      const float sg = a.sg_dev ? a.sg_dev[i] : decode_sign(i);
      const float v = wht32_lanes(At * sg, i);
      const float res = (Lt > 0.f) ? v * kInvSqrt32 / Lt : 0.f;
      const long long oi = bh0 * HD + o;
      if (a.out_dtype == kF32) static_cast<float *>(a.out)[oi] = res;
      else if (a.out_dtype == kBF16) static_cast<uint16_t *>(a.out)[oi] = f32_to_bf16(res);
      else static_cast<uint16_t *>(a.out)[oi] = f32_to_f16(res);
    }
    // the next round reuses the LDS scratch (after the last, nothing does: no
    // barrier, whose fence would wait for the output stores)
    if (o0 + 256 < outs) __syncthreads();
  }
}

// ---- streaming decode: configuration and dispatch ----
// Heads per group: the MFMA layouts take 2, 4 or 8 heads per instruction
// (fewer heads leave rows zero); more than 8 query heads per KV head run in
// several groups (each reading the KV head's records once).
inline int stream_hg(int nr) { return nr <= 2 ? 2 : (nr <= 4 ? 4 : 8); }
// Tokens per wave: 128, or 64 where 128 tokens' records and the wider
// operand sets would not fit the registers of two waves per SIMD (head_dim
// 256 with 4 or 8 heads per group; the QJL correction at head_dim 256 or 8
// heads) or the LDS staging of two workgroups per CU.
#ifndef TQ_DECODE_TPW
#define TQ_DECODE_TPW 128
#endif
constexpr int stream_tpw_c(int nqb, int hg, bool qjl) {
  return (nqb == 8 && hg >= 4) || (qjl && (nqb == 8 || hg == 8)) ? 64 : TQ_DECODE_TPW;
}
// Waves per workgroup: 8 where their LDS staging fits (a chunk of 8 TPW
// tokens halves the split-K partials of a long sequence, and the merge has
// twice the lanes to fetch them), else 4.
#ifndef TQ_DECODE_WAVES
#define TQ_DECODE_WAVES 8
#endif
template <int BITS, int MODE, int NQB, int HG>
constexpr int stream_waves_c() {
  return TQ_DECODE_WAVES == 16 && DecCfg<BITS, MODE, NQB, HG, stream_tpw_c(NQB, HG, MODE == kModeTq), 16>::LDS_FITS
             ? 16
             : (TQ_DECODE_WAVES >= 8 && DecCfg<BITS, MODE, NQB, HG, stream_tpw_c(NQB, HG, MODE == kModeTq), 8>::LDS_FITS ? 8 : 4);
}
template <int BITS, int MODE, int NQB, int HG>
using StreamCfg = DecCfg<BITS, MODE, NQB, HG, stream_tpw_c(NQB, HG, MODE == kModeTq), stream_waves_c<BITS, MODE, NQB, HG>()>;
template <int BITS, int MODE, int NQB, int HG>
using StreamCfg4 = DecCfg<BITS, MODE, NQB, HG, stream_tpw_c(NQB, HG, MODE == kModeTq), 4>;
// 64 tokens per wave in 8-wave workgroups (512-token chunks): each wave's
// key and value passes half as long, for grids that fit the compute units
// in one round even so (a sequence's KV heads over shorter contexts)
template <int BITS, int MODE, int NQB, int HG>
using StreamCfg64 = DecCfg<BITS, MODE, NQB, HG, 64, 8>;
// Compute units of the current device (cached per device).
int device_cus();

// Launches the streaming decode (grid: chunks or ranges, head groups x KV
// heads, batch) for BITS-bit records of cache mode MODE; a.chunk, a.cpr and
// grid.x are set from the launched configuration.  INLINE: the last
// workgroup of a (sequence, KV head) merges the split-K partials; else the
// caller launches stream_merge_kernel after it.  Defined in the
// tq_attention_k<BITS>_<mode>.hip units.
template <int BITS, int MODE, bool INLINE>
void launch_stream_bm(AttnArgs &a, int nqb, int hg, dim3 grid, hipStream_t st);

}  // namespace tqa
