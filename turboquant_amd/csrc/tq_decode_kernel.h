#pragma once

// tq_decode_kernel.h -- the streaming fused decode kernel and its launchers;
// included by the tq_attention_k<bits>_<mode>.hip units, each of which
// instantiates launch_stream_bm for its bit width and cache mode.
//
// One workgroup of WAVES waves (4 or 8) owns a chunk of CHUNK = WAVES * TPW tokens of
// one (sequence b, KV head g) for a group of HG query heads of that KV head;
// every compressed byte of the chunk is read once for all HG heads.  Wave w
// owns the TPW consecutive tokens starting at chunk + w * TPW, as NKT 16-token
// K tiles and NVP 32-token V tile pairs.
//
// Schedule.  At entry every lane issues the loads of its query and of the K
// records and scales of all its tiles; once the query setup has passed the
// workgroup barrier (every wave has requested its keys), the V scales and V
// records.  The keys thus arrive before the values chip-wide.  Each K tile is
// scored as soon as its records have arrived (the loads return in order), so
// the keys' arithmetic overlaps the transfer of the later keys; after the last
// K tile the wave's softmax weights are final (a two-pass softmax over the
// wave's tokens: no running rescale), and each V tile pair is accumulated as
// it arrives, overlapping the values' transfer.  What remains after the last
// byte is one tile pair's value products, the waves' combine and the split-K
// arrival.  When the launch has more chunks than one round of workgroups
// holds, a workgroup takes a range of consecutive chunks instead: the
// per-chunk step above repeats, the softmax state and the value sums are
// carried across chunks with an online rescale, and the next chunk's first K
// tiles are requested during the current chunk's last value tiles.
//
// Arithmetic (the same decomposition as the reference's per-qblock dequant,
// tq_attention_kernel.cu:33-53, k_j = |s| inv (H (cb[idx] d))_j): keys are
// never inverse-rotated; q.k = |s| sum_i cb[idx_i] qt_i with qt the rotated
// query.  Both contractions run on v_mfma_f32_16x16x32_f16 with every f32
// operand split into two f16 parts (hi = 11 significant bits, lo = the exact
// remainder), 22-bit products accumulated in f32; a pair of codes is decoded
// by one 8-byte LDS read of a 2^(2 BITS)-entry table (hi c0, hi c1, lo c0,
// lo c1).
//   K: D[(qblock, head, part)][token] = Q[..][k] K[k][token], the query
//      operand block-diagonal over QPM qblocks per instruction (so the
//      per-(token, qblock) key scale applies after the contraction).  QPM
//      and HPM = 8 / QPM heads per instruction follow from HG, so one
//      instruction serves every head of the group; lanes (token, k group)
//      hold the key stream of their qblock's ES-th part (ES = 4 / QPM).
//   V: D[(qblock, pair, part)][(qblock, head, weight part)] = V W, V through
//      the transposing LDS read (ds_read_b64_tr_b16) of the same table, W =
//      p |s_V| 2^-Ev; lanes (token, row set) hold the value stream of their
//      row set's qblock part.  Accumulated over the wave's tiles in MFMA
//      registers; the useful (block-diagonal) outputs are extracted once.

#include "tq_attention.h"

namespace tqa {
namespace {

// N (1, 2, 4 or 8) consecutive 32-bit words at voff of a buffer, and their
// store into LDS at p (4 N-byte aligned)
template <int N>
__device__ __forceinline__ void load_words(uint32_t (&w)[N], __amdgpu_buffer_rsrc_t r, uint32_t voff) {
  if constexpr (N == 8) {
    uint32_t a[4], b[4];
    buf_words<4>(a, r, voff, 0);
    buf_words<4>(b, r, voff + 16, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      w[i] = a[i];
      w[i + 4] = b[i];
    }
  } else {
    buf_words<N>(w, r, voff, 0);
  }
}
template <int N>
__device__ __forceinline__ void stage_words(uint8_t *p, const uint32_t (&w)[N]) {
  if constexpr (N == 1) {
    *reinterpret_cast<uint32_t *>(p) = w[0];
  } else if constexpr (N == 2) {
    *reinterpret_cast<uint2 *>(p) = make_uint2(w[0], w[1]);
  } else {
#pragma unroll
    for (int i = 0; i < N; i += 4) *reinterpret_cast<uint4 *>(p + 4 * i) = make_uint4(w[i], w[i + 1], w[i + 2], w[i + 3]);
  }
}
// Transposing 4-bit LDS read (ds_read_b64_tr_b4): inside each group of 16
// lanes, lane i receives 4-bit item i of the 8-byte rows addressed by lanes
// 0 .. 15 of its group, the row of lane j in bits 4 j .. 4 j + 3 (checked on
// MI355X).  p must point into LDS.
__device__ __forceinline__ u32x2 lds_read_tr4(const void *p) {
  typedef int v2i __attribute__((ext_vector_type(2)));
  typedef __attribute__((address_space(3))) v2i lds_v2i;
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr4_b64_v2i32((lds_v2i *)p));
}

// The 8 nibbles of w (4-bit codes, LSB first) as an f16 MFMA operand of
// exact subnormals, code r and r + 4 in register r: registers 0 and 2 hold
// i 2^-24 (the low nibble of each half), registers 1 and 3 i 2^-20 (the
// nibble left at bits 4..7 of its half), so the other operand's registers 0
// and 2 carry a factor 16 and every product is x i 2^-20.
__device__ __forceinline__ u32x4 nib_operand(uint32_t w) {
  const uint32_t h = w >> 8;
  return u32x4{w & 0x000F000Fu, w & 0x00F000F0u, h & 0x000F000Fu, h & 0x00F000F0u};
}

// BITS-bit code pair p of a lane's stream w (little-endian words), as the
// byte offset of its pair-table entry (code * 8): two VALU per pair.
template <int BITS, int NWD>
__device__ __forceinline__ uint32_t pair_off(const uint32_t (&w)[NWD], int p) {
  constexpr int W = 2 * BITS;
  constexpr uint32_t M = ((1u << W) - 1u) << 3;
  const int pos = W * p;
  if (pos < 3) return (w[0] << 3) & M;
  const int s = pos - 3, wi = s >> 5, sh = s & 31;
  if (sh + W + 3 <= 32) return (w[wi] >> sh) & M;
  return __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh) & M;
}

// Stream of part `es` (of ES) of a qblock record held in w: for ES > 1 the
// lane loaded the two words from word w0 = min(bo / 32, QW - 2); shift them so
// that its pairs start at bit 0.
template <class C>
__device__ __forceinline__ int part_word(int es) {
  if constexpr (C::ES == 1) return 0;
  else return dmin((es * C::PPL * 2 * C::BITS) >> 5, C::QW - 2);
}
template <class C>
__device__ __forceinline__ void align_part(uint32_t (&w)[C::NW], int es) {
  if constexpr (C::ES > 1) {
    const int sh = es * C::PPL * 2 * C::BITS - 32 * part_word<C>(es);
    const uint64_t x = ((((uint64_t)w[1]) << 32) | w[0]) >> sh;
    w[0] = (uint32_t)x;
    w[1] = (uint32_t)(x >> 32);
  }
}

__device__ __forceinline__ float row_max16(float v) {
  v = fmaxf(v, dpp_quad_xor1(v));
  v = fmaxf(v, dpp_quad_xor2(v));
  v = fmaxf(v, swizzle_xor<4>(v));
  return fmaxf(v, dpp_row_xor8(v));
}
__device__ __forceinline__ float row_sum16(float v) {
  v += dpp_quad_xor1(v);
  v += dpp_quad_xor2(v);
  v += swizzle_xor<4>(v);
  return v + dpp_row_xor8(v);
}
// v + v of lane l ^ 32 / l ^ 16
__device__ __forceinline__ float sum_xor32(float v) {
  float a, b;
  swap_pair32(v, a, b);
  return a + b;
}
__device__ __forceinline__ float sum_xor16(float v) {
  float a, b;
  swap_pair16(v, a, b);
  return a + b;
}

// MULTI: the launch gives workgroups ranges of several chunks (cpr > 1)
// PROJ (TQ only): no rq from the caller, R q is formed in the launch; an
// instance of its own, so that the launches given rq carry none of its code
template <class C, bool INLINE_MERGE, bool GRID, bool MULTI, bool PROJ = false>
#ifndef TQ_DECODE_WPE
#define TQ_DECODE_WPE 2
#endif
__global__ __launch_bounds__(C::THREADS, TQ_DECODE_WPE) void stream_decode_kernel(const uint8_t *k_idx, const uint8_t *v_idx,
                                                               const uint16_t *k_sc, const uint16_t *v_sc,
                                                               long long seq_stride, long long kv_head_stride,
                                                               int len_hint, AttnArgs a) {
  constexpr int BITS = C::BITS, HD = C::HD, NQB = C::NQB, HG = C::HG, TPW = C::TPW, QW = C::QW, NW = C::NW;
  static_assert(GRID ? C::G_LDS_OK : C::LDS_OK, "the workgroup's LDS (with the merge's scratch) fits 160 KiB");
  // word offset of the layout from OFF_W on (the grid passes need no
  // codebook table and fewer query operands)
  constexpr int LSH = GRID ? C::G_SHIFT : 0;
  constexpr int QPM = C::QPM, HPM = C::HPM, QG = C::QG, ES = C::ES, KJ = C::KJ, PPL = C::PPL;
  constexpr int NKT = C::NKT, NVP = C::NVP, PACKED = C::PACKED;
  // GRID: 4-bit codes on the evenly spaced MaxNorm codebook c_i = -R + i D.
  // Both passes then contract with the codes themselves (exact f16
  // subnormals, eight per word by masks: nib_operand) and apply
  // q.c = D sum q_j i_j - R sum q_j (and its value-pass counterpart) after
  // the product: no codebook reads, half the instructions of the two-part
  // codebook operand.
  static_assert(!GRID || (BITS == 4 && C::MODE == kModePqo), "the grid passes take 4-bit PQO codes");
  constexpr int KJA = GRID ? QPM : KJ;                  // key-pass instructions per qblock group
  constexpr bool QAR = GRID || C::QA_REGS;              // query operands in registers
  __shared__ __attribute__((aligned(16))) float lds[C::TOTAL - LSH];
  __shared__ int s_flag;
  // grid V pass: each wave's 64-token block of V records, token-major
  __shared__ __attribute__((aligned(16))) uint8_t vstage[GRID ? C::VSTAGE : 16];
  uint2 *s_pair = reinterpret_cast<uint2 *>(lds + C::OFF_PAIR);
  float *s_q = lds + C::OFF_Q - LSH;
  float *s_qmax = lds + C::OFF_QMAX - LSH;
  float *s_rq = lds + C::OFF_RQ - LSH;
  float *s_rqmax = lds + C::OFF_RQMAX - LSH;
  float *s_qsum = lds + C::OFF_QSUM - LSH;
  uint2 *s_nib = reinterpret_cast<uint2 *>(lds + C::OFF_NIB);
  u32x4 *s_qa = reinterpret_cast<u32x4 *>(lds + (GRID ? 0 : C::OFF_QA));

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: the wave's scalar offsets
  const int l16 = lane & 15, lg = lane >> 4;
  // (range c, head group y, sequence b).  Ranges: workgroups start in the
  // order of their linear index, so it is mapped range-major (range 0 of
  // every (sequence, head group) first): the ranges that the batch's lengths
  // leave empty come last instead of holding slots among the others (an
  // empty workgroup still waits for its first loads, queued behind the
  // records in flight), and consecutive workgroups, which go to different
  // XCDs, take different (sequence, KV head) pairs.
  int c = blockIdx.x, y = blockIdx.y, b = blockIdx.z;
  if constexpr (MULTI) {
    const int per = (int)(gridDim.y * gridDim.z);
    const int lin = blockIdx.x + (int)gridDim.x * (blockIdx.y + (int)gridDim.y * blockIdx.z);
    c = lin / per;
    const int rest = lin - c * per;
    b = rest / (int)gridDim.y;
    y = rest - b * (int)gridDim.y;
  }
  // The argument fields that the first loads depend on, all requested
  // before one wait (the empty asm makes them available together; left to
  // itself the compiler requests each behind the branch that uses it, and
  // each request after the first that misses the scalar cache costs a
  // memory round trip before any record load goes out).
  const void *const a_q = a.q;
  const float *const a_sg = a.sg_dev, *const a_cb = a.cb_dev, *const a_rq = a.rq;
  const int *const a_ws = a.ws_hdr, *const a_lens = a.kv_lens;
  const int a_qdt = a.q_dtype, a_ngroups = a.ngroups, a_nr = a.nr, a_heads = a.num_heads, a_max = a.max_len;
  const int a_cpr = a.cpr;
  asm volatile("" ::"s"(a_q), "s"(a_sg), "s"(a_cb), "s"(a_rq), "s"(a_ws), "s"(a_lens), "s"(a_qdt), "s"(a_ngroups),
               "s"(a_nr), "s"(a_heads), "s"(a_max), "s"(a_cpr));
  // ---- balanced split (range launches with a.bal_nwg > 0, one head group
  // per KV head, at most 64 sequences): the ranges' length S (in chunks) is
  // the smallest whose ranges, sequence b's chunks split into
  // R_b = ceil(n_b / S) near-equal ranges per KV head, number at most
  // bal_nwg.  Ragged batches then give every workgroup at most S chunks;
  // ranges of one fixed length would leave the compute units that hold the
  // long sequences' ranges setting the time.  A wave holds the batch's chunk
  // counts (one sequence per lane), so the split costs a few reductions and
  // a ballot, no LDS and no barrier before the first loads. ----
  int bal_ck0 = 0, bal_nck = 0, bal_nparts = 0;
  const bool bal = MULTI && a.bal_nwg > 0;
  if constexpr (MULTI) {
    if (bal) {
      const int nwg = a.bal_nwg, ny = a.bal_ny, nb = a.bal_batch;
      int n = 0;
      if (lane < nb) {
        const int lb = len_hint >= 0 ? len_hint : min(max(a_lens[lane], 0), a_max);
        n = (lb + C::CHUNK - 1) / C::CHUNK;
      }
      // S: the closed form ceil(ny T / (nwg - ny nb)) (feasible: sum_b
      // ceil(n_b / S) <= T / S + nb), or one less when that still fits
      const int T = wave_sum_i(n);
      int S = nwg > ny * nb ? (int)(((long long)T * ny + (nwg - ny * nb) - 1) / (nwg - ny * nb)) : wave_max_i(n);
      S = max(S, 1);
      if (S > 1 && (long long)wave_sum_i((n + S - 2) / (S - 1)) * ny <= nwg) S--;
      S = __builtin_amdgcn_readfirstlane(S);
      const int rb = (n + S - 1) / S;  // ranges per KV head of the lane's sequence
      const int incl = wave_incl_scan_i(rb);
      const int pre = incl - rb;  // ranges before the lane's sequence, per KV head
      const int wi = blockIdx.x;
      const int total = __builtin_amdgcn_readlane(incl, 63) * ny;
      // empty sequences attend to nothing: zero output (cuda/attention.rs:65-68)
      for (int bb = wi; bb < nb; bb += nwg)
        if (__builtin_amdgcn_readlane(n, bb) == 0)
          for (int e = tid; e < a_heads * HD; e += C::THREADS) {
            const long long oi = (long long)bb * a_heads * HD + e;
            if (a.out_dtype == kF32) static_cast<float *>(a.out)[oi] = 0.f;
            else static_cast<uint16_t *>(a.out)[oi] = 0;
          }
      if (wi >= total) {
        __builtin_amdgcn_s_waitcnt(0);
        return;
      }
      // workgroup wi: sequence b (the last whose ranges start at or before
      // it), KV head y, range r of its R_b
      const unsigned long long le = __ballot(lane < nb && pre * ny <= wi);
      b = __builtin_amdgcn_readfirstlane(63 - __builtin_clzll(le));
      const int pre_b = __builtin_amdgcn_readlane(pre, b), r_b = __builtin_amdgcn_readlane(rb, b);
      const int n_b = __builtin_amdgcn_readlane(n, b);
      const int k = wi - pre_b * ny;
      y = k / r_b;
      const int r = k - y * r_b;
      bal_ck0 = (int)((long long)r * n_b / r_b);
      bal_nck = (int)((long long)(r + 1) * n_b / r_b) - bal_ck0;
      bal_nparts = r_b;
      c = r;
    }
  }
  const int g = y / a_ngroups, gh = y - g * a_ngroups;
  const int nh = min(HG, a_nr - gh * HG);                    // heads of this group
  const long long hq0 = (long long)b * a_heads + (long long)g * a_nr + gh * HG;  // its first q head

  // ---- the query (and for TQ its projection) goes out first: later waits
  // for it count no record load ----
  constexpr int QE = HG * HD;                 // query elements of the group
  constexpr int QIT = (QE + C::THREADS - 1) / C::THREADS;
  uint32_t qbits[QIT];
  float rqv[QIT];
  // TQ without rq: the sign words of the rows of R whose products this lane
  // computes (row tile wave + WAVES t: row 16 (wave + WAVES t) + l16)
  constexpr int RT = C::QJL ? (HD / 16 + C::WAVES - 1) / C::WAVES : 1;
  uint32_t rsw[RT][C::QJL ? NQB : 1];
#pragma unroll
  for (int k = 0; k < QIT; k++) {
    const int e = tid + C::THREADS * k, hl = e / HD;
    qbits[k] = 0;
    rqv[k] = 0.f;
    if (e < QE && hl < nh) {
      const long long qi = hq0 * HD + e;
      if (a_qdt == kF32) qbits[k] = static_cast<const uint32_t *>(a_q)[qi];
      else qbits[k] = static_cast<const uint16_t *>(a_q)[qi];
      if constexpr (C::QJL) {
        if (a_rq) rqv[k] = a_rq[qi];
      }
    }
  }
  if constexpr (C::QJL) {
    if constexpr (PROJ) {
#pragma unroll
      for (int t = 0; t < RT; t++) {
        const int rt = wave + C::WAVES * t;
        const uint32_t *row = a.rmat + (16 * min(rt, HD / 16 - 1) + l16) * NQB;
#pragma unroll
        for (int w = 0; w < NQB; w++) rsw[t][w] = row[w];
      }
    }
  }
  // the caller's decode sign for this lane (selected at its use: a select
  // here would make the constant path wait for the load before any record
  // load goes out)
  float sgl = 0.f;
  if (a_sg) sgl = a_sg[tid & 31];
  // the caller's codebook entries for this lane's pair-table entry, also
  // before any record load (a wait for them then waits for nothing else)
  constexpr int CM = (1 << C::CB) - 1;  // slot codes >= 2^CB never occur
  const int pi0 = tid & ((1 << BITS) - 1) & CM, pi1 = (tid >> BITS) & CM;
  float pc0 = 0.f, pc1 = 0.f;
  if (a_cb && tid < C::NPAIR) {
    pc0 = a_cb[pi0];
    pc1 = a_cb[pi1];
  }
  // the workspace header, needed only at the split-K arrival: a vector load
  // (a scalar one would be waited for here, before the record loads)
  int ws_hdr = 0;
  if constexpr (INLINE_MERGE)
    ws_hdr = (int)__builtin_amdgcn_raw_buffer_load_b32(rec_rsrc(a_ws, 4u), 0u, 0u, 0);

  // the sequence's length through the scalar cache (constant address space):
  // a vector load would queue behind the records other workgroups on this
  // compute unit have in flight, and every record load here waits for it
  typedef __attribute__((address_space(4))) const int const_int;
  const int len = len_hint >= 0 ? len_hint : min(max(((const_int *)a_lens)[b], 0), a_max);
  // Workgroup c takes the range of cpr consecutive chunks from chunk c cpr
  // (the host picks cpr; the merge counts ranges): its waves keep one online
  // softmax state over the range's chunks, so the setup, the combine and the
  // split-K arrival are paid once per range.
  const int nchunks = (len + C::CHUNK - 1) / C::CHUNK;
  const int cpr = a_cpr;
  const int ck0 = bal ? bal_ck0 : c * cpr;
  if (ck0 >= nchunks) {  // an empty range is not counted by the merge
    if (len == 0 && c == 0) {
      // an empty sequence attends to nothing: zero output (cuda/attention.rs:65-68)
      for (int e = tid; e < nh * HD; e += C::THREADS) {
        const long long oi = hq0 * HD + e;
        if (a.out_dtype == kF32) static_cast<float *>(a.out)[oi] = 0.f;
        else static_cast<uint16_t *>(a.out)[oi] = 0;
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    return;
  }
  const int nck = bal ? bal_nck : (MULTI ? min(cpr, nchunks - ck0) : 1);  // chunks of this range
  const int nparts = bal ? bal_nparts : (nchunks + cpr - 1) / cpr;      // ranges the merge folds

  // ---- records.  Wave w's tokens of a chunk start at tw = chunk CHUNK +
  // w TPW.  K tile i, lane (l16, lg): token tw + 16 i + l16, for
  // group qg the stream part lg % ES of qblock qg * QPM + lg / ES; its key
  // scale.  V tile i, lane (l16, lg): token tw + 16 i + 4 lg + l16 / 4, row
  // set rs = l16 & 3 -> stream part rs % ES of qblock vs * QPM + rs / ES.
  // Buffer loads bounded by the sequence's len records: a token past the end
  // reads zeros (its score is masked and its weight is 0), and a tile's
  // offset is a scalar constant. ----
  const long long rec0 = (long long)b * seq_stride + (long long)g * kv_head_stride;
  const uint32_t nrec = (uint32_t)len;
  const uint8_t *kbase = k_idx + rec0 * PACKED, *vbase = v_idx + rec0 * PACKED;
  const uint16_t *ksbase = k_sc + rec0 * NQB, *vsbase = v_sc + rec0 * NQB;
  const int kes = lg % ES, kqb = lg / ES;
  const int rs = l16 & 3, ves = rs % ES, vqb = rs / ES;
  // per-lane offsets from the wave's first token tw
  const uint32_t kvo = (uint32_t)l16 * PACKED + (uint32_t)(kqb * QW + part_word<C>(kes)) * 4u;
  const uint32_t kso = ((uint32_t)l16 * NQB + kqb) * 2u;
  const uint32_t vvo = (uint32_t)(4 * lg + (l16 >> 2)) * PACKED + (uint32_t)(vqb * QW + part_word<C>(ves)) * 4u;
  const uint32_t tw_first = (uint32_t)(ck0 * C::CHUNK + wave * TPW);
  uint32_t kw[NKT][QG][NW], vw[GRID ? 1 : NKT][QG][NW];
  uint32_t vg[GRID ? NKT : 1][NQB];  // grid V pass: lane l's 4 NQB bytes of its tile
  uint32_t ksv[NKT][QG];
  uint32_t sgw[NKT][C::SW4];
  uint32_t nrm[NKT];
  uint32_t vsr[C::TPL][(NQB + 1) / 2];
  // The wave's loads form one stream of groups, consumed in order: K tile i
  // (records, scales, QJL signs and norms) is group i, the V scales group
  // NKT, V tile i group NKT + 1 + i.  Only a few groups are in flight at a
  // time (issued as earlier ones are consumed), so no load instruction waits
  // at issue for the CU's memory queue while arithmetic could run.
  auto issue = [&](int grp, uint32_t tw0) {
    if (grp < NKT) {
      const int i = grp;
      const uint32_t t16 = tw0 + 16u * i;  // the tile's first token
      const auto rk = rec_rsrc(kbase, nrec * PACKED, t16 * PACKED);
      const auto rks = rec_rsrc(ksbase, nrec * NQB * 2u, t16 * NQB * 2u);
#pragma unroll
      for (int qg = 0; qg < QG; qg++) {
        buf_words<NW>(kw[i][qg], rk, kvo + qg * QPM * QW * 4, 0);
        ksv[i][qg] = __builtin_amdgcn_raw_buffer_load_b16(rks, kso + qg * QPM * 2, 0, 0);
      }
      if constexpr (C::QJL) {
        const auto rsg = rec_rsrc(reinterpret_cast<const uint8_t *>(a.qjl_signs) + rec0 * (HD / 8), nrec * (HD / 8),
                                  t16 * (HD / 8));
        const auto rnm = rec_rsrc(a.qjl_norms + rec0, nrec * 2u, t16 * 2u);
#pragma unroll
        for (int s4 = 0; s4 < C::SW4; s4++) {
          const int wi = min(s4 * 4 + lg, NQB - 1);
          sgw[i][s4] = __builtin_amdgcn_raw_buffer_load_b32(rsg, (uint32_t)l16 * (HD / 8) + wi * 4, 0, 0);
        }
        nrm[i] = __builtin_amdgcn_raw_buffer_load_b16(rnm, (uint32_t)l16 * 2u, 0, 0);
      }
    } else if (grp == NKT) {
      // V scales of the wave: tokens tw + TPL lane + u, all NQB per token
      const auto rvs = rec_rsrc(vsbase, nrec * NQB * 2u, tw0 * NQB * 2u);
      const uint32_t vso = (uint32_t)(C::TPL * lane) * NQB * 2u;
#pragma unroll
      for (int u = 0; u < C::TPL; u++) {
        if constexpr (NQB == 1) vsr[u][0] = __builtin_amdgcn_raw_buffer_load_b16(rvs, vso + u * 2, 0, 0);
        else buf_words<NQB / 2>(vsr[u], rvs, vso + u * NQB * 2, 0);
      }
    } else {
      const int i = grp - NKT - 1;
      const auto rv = rec_rsrc(vbase, nrec * PACKED, (tw0 + 16u * i) * PACKED);
      if constexpr (GRID) {
        load_words<NQB>(vg[i], rv, (uint32_t)lane * (4u * NQB));
      } else {
#pragma unroll
        for (int qg = 0; qg < QG; qg++) buf_words<NW>(vw[i][qg], rv, vvo + qg * QPM * QW * 4, 0);
      }
    }
  };
  // Schedule: K tiles 0 .. LA-1 and the V scales (needed by the softmax)
  // of the first chunk before the setup; K tile i + LA as K tile i is
  // consumed; V tiles 0-3 during the last two K tiles, so the first values
  // are in flight before the softmax; then V tiles 2 vp + 4, 2 vp + 5 as V
  // pair vp is consumed, and the next chunk's first K tiles and V scales
  // two pairs before the chunk's last.
#ifndef TQ_DECODE_LOOKAHEAD_MULTI
#define TQ_DECODE_LOOKAHEAD_MULTI 4
#endif
#ifndef TQ_DECODE_LOOKAHEAD_PASS
#define TQ_DECODE_LOOKAHEAD_PASS TQ_DECODE_LOOKAHEAD
#endif
  // LA0 K tiles go out with the first chunk's prologue (more would hold the
  // waves at issue before their setup), LA during the K passes
  constexpr int LA = dmin(MULTI ? TQ_DECODE_LOOKAHEAD_MULTI : TQ_DECODE_LOOKAHEAD_PASS, NKT);
  constexpr int LA0 = MULTI ? LA : dmin(C::LOOKAHEAD, LA);
  constexpr int VP_NEXT = NVP >= 2 ? NVP - 2 : 0;
  auto issue_first = [&](uint32_t tw0, int n) {
#pragma unroll
    for (int grp = 0; grp < NKT; grp++)
      if (grp < n) issue(grp, tw0);
    issue(NKT, tw0);
  };
  issue_first(tw_first, LA0);
  auto issue_k = [&](int i, uint32_t tw0) {  // K tile i is being consumed
    if (i == 0) {
#pragma unroll
      for (int t = LA0; t < LA; t++) issue(t, tw0);
    }
    if (i + LA < NKT) issue(i + LA, tw0);
    if (i >= NKT - 2) {
      const int t = 2 * (i - (NKT - 2));
      issue(NKT + 1 + t, tw0);
      issue(NKT + 2 + t, tw0);
    }
  };
  auto issue_v = [&](int vp, uint32_t tw0) {  // V pair vp is being consumed
    if (2 * vp + 4 < NKT) {
      issue(NKT + 1 + 2 * vp + 4, tw0);
      issue(NKT + 2 + 2 * vp + 4, tw0);
    }
  };
  // ---- pair table (the caller's device codebook, L2Norm tables from the
  // arguments, or the PQO constants) ----
  static_assert(C::NPAIR <= 256, "one pair-table entry per lane");
  if (!GRID && tid < C::NPAIR) {  // the grid passes read no table (its words hold the query operands)
    const int e = tid, i0 = pi0, i1 = pi1;
    float c0, c1;
    if (a.cb_dev) {
      c0 = pc0;
      c1 = pc1;
    } else if (a.cb_args) {
      c0 = a.cb[0];
      c1 = a.cb[0];
#pragma unroll
      for (int kk = 1; kk <= CM; kk++) {
        c0 = i0 == kk ? a.cb[kk] : c0;
        c1 = i1 == kk ? a.cb[kk] : c1;
      }
    } else {
      c0 = pqo_centroid<C::CB>(i0);
      c1 = pqo_centroid<C::CB>(i1);
    }
    const float h0 = split_hi(c0), h1 = split_hi(c1);
    s_pair[e] = make_uint2(pack_f16(h0, h1), pack_f16(c0 - h0, c1 - h1));
  }
  if constexpr (C::QJL) {
    // +-1 in f16 for the four sign bits of a nibble, LSB first
    if (tid < 16) {
      auto pm1 = [&](int bit) { return ((tid >> bit) & 1) ? 0x3C00u : 0xBC00u; };
      s_nib[tid] = make_uint2(pm1(0) | (pm1(1) << 16), pm1(2) | (pm1(3) << 16));
    }
  }
  if constexpr (C::QJL) {
    if constexpr (PROJ) {
      // rq = R q (precompute_query_projections, qjl.rs:196-208) in the
      // launch, on the matrix cores: R's entries are +-1 (exact in bf16)
      // and the raw query is cut into bf16 parts that sum to it exactly
      // (one part for a bf16 query, two for f16, three for f32), so every
      // product is exact and only the f32 accumulation order differs from
      // the serial sum of tq_qjl_project (a few ulp).  Wave w takes the row
      // tiles w, w + WAVES, ..: A, lane (l16, lg), holds R[row][32 s + 8 lg
      // ..+7] expanded from one byte of sign bits through the nibble table
      // (f16 +-1 with bit 1 -> +1: its exponent bits flipped to bf16, and
      // the result negated, since R has bit 1 -> -1); B column h is head
      // h's query.  The rows land in s_q, which the rotated query below
      // overwrites element by element in the same lanes.
#pragma unroll
      for (int k = 0; k < QIT; k++) {
        const int e = tid + C::THREADS * k;
        if (e < QE) s_rq[e] = q_value(qbits[k], a_qdt);
      }
      __syncthreads();
      const int parts = a_qdt == kBF16 ? 1 : (a_qdt == kF16 ? 2 : 3);
#pragma unroll
      for (int t = 0; t < RT; t++) {
        const int rt = wave + C::WAVES * t;
        if (rt < HD / 16) {  // uniform per wave
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int sk = 0; sk < HD / 32; sk++) {
            const uint32_t byte = (rsw[t][sk] >> (8 * lg)) & 0xffu;
            const uint2 n0 = s_nib[byte & 15u], n1 = s_nib[byte >> 4];
            const u32x4 am = {n0.x ^ 0x03800380u, n0.y ^ 0x03800380u, n1.x ^ 0x03800380u, n1.y ^ 0x03800380u};
            float qv[8];
            if (l16 < HG) {
              const float4 *src = reinterpret_cast<const float4 *>(s_rq + l16 * HD + 32 * sk + 8 * lg);
              const float4 v0 = src[0], v1 = src[1];
              qv[0] = v0.x; qv[1] = v0.y; qv[2] = v0.z; qv[3] = v0.w;
              qv[4] = v1.x; qv[5] = v1.y; qv[6] = v1.z; qv[7] = v1.w;
            } else {
#pragma unroll
              for (int j = 0; j < 8; j++) qv[j] = 0.f;
            }
            for (int p = 0; p < parts; p++) {
              uint32_t cut[8];
#pragma unroll
              for (int j = 0; j < 8; j++) {
                cut[j] = f2u(qv[j]) & 0xffff0000u;  // the leading 8 significand bits
                qv[j] -= u2f(cut[j]);                // exact: the rest
              }
              const u32x4 bm = {__builtin_amdgcn_perm(cut[1], cut[0], 0x07060302u),
                                __builtin_amdgcn_perm(cut[3], cut[2], 0x07060302u),
                                __builtin_amdgcn_perm(cut[5], cut[4], 0x07060302u),
                                __builtin_amdgcn_perm(cut[7], cut[6], 0x07060302u)};
              acc = mfma_bf16(am, bm, acc);
            }
          }
          if (l16 < HG) {
#pragma unroll
            for (int i = 0; i < 4; i++) s_q[l16 * HD + 16 * rt + 4 * lg + i] = -acc[i] * a.qjl_inv;
          }
        }
      }
      __syncthreads();
#pragma unroll
      for (int k = 0; k < QIT; k++) {
        const int e = tid + C::THREADS * k;
        if (e < QE) rqv[k] = s_q[e];
      }
      __syncthreads();  // s_rq and s_q are rewritten below
    }
  }
  // ---- rotated, scaled query: 32-lane butterflies (elements of a qblock sit
  // in 32 consecutive lanes; absent heads are whole zero blocks) ----
  const float qscale = a.softmax_scale * kLog2e * kInvSqrt32;
  const float qsign = a.sg_dev ? sgl : decode_sign(tid & 31);
#pragma unroll
  for (int k = 0; k < QIT; k++) {
    const int e = tid + C::THREADS * k;
    if (e < QE) {  // uniform per 32-lane block
      const float v = wht32_lanes(q_value(qbits[k], a.q_dtype), e & 31);
      const float qt = v * (qsign * qscale);
      s_q[e] = qt;
      float m = fabsf(qt);
      m = fmaxf(m, lane_xor<1>(m));
      m = fmaxf(m, lane_xor<2>(m));
      m = fmaxf(m, lane_xor<4>(m));
      m = fmaxf(m, lane_xor<8>(m));
      m = fmaxf(m, lane_xor<16>(m));
      if ((e & 31) == 0) s_qmax[e >> 5] = m;
      if constexpr (GRID) {
        float sm = qt;
        sm += lane_xor<1>(sm);
        sm += lane_xor<2>(sm);
        sm += lane_xor<4>(sm);
        sm += lane_xor<8>(sm);
        sm += lane_xor<16>(sm);
        if ((e & 31) == 0) s_qsum[e >> 5] = sm;
      }
      if constexpr (C::QJL) {
        const float rsv = rqv[k] * (a.softmax_scale * kLog2e);
        s_rq[e] = rsv;
        float r = fabsf(rsv);
        r = fmaxf(r, lane_xor<1>(r));
        r = fmaxf(r, lane_xor<2>(r));
        r = fmaxf(r, lane_xor<4>(r));
        r = fmaxf(r, lane_xor<8>(r));
        r = fmaxf(r, lane_xor<16>(r));
        if ((e & 31) == 0) s_rqmax[e >> 5] = r;
      }
    }
  }
  __syncthreads();
  auto head_exp = [&](const float *mx, int hl) {
    float m = 0.f;
#pragma unroll
    for (int qb = 0; qb < NQB; qb++) m = fmaxf(m, mx[hl * NQB + qb]);
    return pow2_exponent(m);
  };
  // Key-pass query operands: for group qg and slice j, lane (m, kg) supplies
  // k = 8 kg + (x0, x1, x0, x1, x2, x3, x2, x3), x_i = part(Q[head][e + i])
  // with row m = (qbl, hl, part), e = element 4 j of stream part kg % ES of
  // qblock qg * QPM + qbl, when kg / ES == qbl and hl < nh; Q = qt * 2^-Eq,
  // scaled per head into f16's range.
  auto make_qa = [&](int qg, int j, int m, int kg) -> u32x4 {
    const int qbl = m / (2 * HPM), hl = (m >> 1) % HPM, part = m & 1;
    u32x4 val = {0u, 0u, 0u, 0u};
    if (kg / ES == qbl && hl < nh) {
      const float sc = exp2i(-head_exp(s_qmax, hl));
      const float4 q4 = *reinterpret_cast<const float4 *>(s_q + hl * HD + (qg * QPM + qbl) * 32 +
                                                          (kg % ES) * (32 / ES) + 4 * j);
      const float x0 = q4.x * sc, x1 = q4.y * sc, x2 = q4.z * sc, x3 = q4.w * sc;
      const float h0 = split_hi(x0), h1 = split_hi(x1), h2 = split_hi(x2), h3 = split_hi(x3);
      const uint32_t w01 = part ? pack_f16(x0 - h0, x1 - h1) : pack_f16(h0, h1);
      const uint32_t w23 = part ? pack_f16(x2 - h2, x3 - h3) : pack_f16(h2, h3);
      val = u32x4{w01, w01, w23, w23};
    }
    return val;
  };
  // Grid key pass: word j of the lane's stream part holds elements
  // 8 j + (0..7) as nibbles; B's register r carries nibbles r and r + 4
  // (nib_operand), so slot u = 2 r + h takes element 8 j + r + 4 h, and the
  // query operand follows that order.
  auto make_qa_grid = [&](int qg, int j, int m, int kg) -> u32x4 {
    const int qbl = m / (2 * HPM), hl = (m >> 1) % HPM, part = m & 1;
    u32x4 val = {0u, 0u, 0u, 0u};
    if (kg / ES == qbl && hl < nh) {
      const float sc = exp2i(-head_exp(s_qmax, hl));
      const float *src = s_q + hl * HD + (qg * QPM + qbl) * 32 + (kg % ES) * (32 / ES) + 8 * j;
      const float4 lo4 = *reinterpret_cast<const float4 *>(src), hi4 = *reinterpret_cast<const float4 *>(src + 4);
      // registers 0 and 2 meet codes i 2^-24, 1 and 3 codes i 2^-20
      // (nib_operand): the former take the factor 16 (exact)
      const float sc16 = sc * 16.f;
      const float xa[4] = {lo4.x * sc16, lo4.y * sc, lo4.z * sc16, lo4.w * sc};
      const float xb[4] = {hi4.x * sc16, hi4.y * sc, hi4.z * sc16, hi4.w * sc};
      uint32_t w[4];
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const float ha = split_hi(xa[r]), hb = split_hi(xb[r]);
        w[r] = part ? pack_f16(xa[r] - ha, xb[r] - hb) : pack_f16(ha, hb);
      }
      val = u32x4{w[0], w[1], w[2], w[3]};
    }
    return val;
  };
  // each operand is the same for every wave: the workgroup's lanes build
  // them once
  for (int e = tid; e < QG * KJA * 64; e += C::THREADS) {
    const int sl = e >> 6, ln = e & 63;
    s_qa[e] = GRID ? make_qa_grid(sl / KJA, sl % KJA, ln & 15, ln >> 4) : make_qa(sl / KJA, sl % KJA, ln & 15, ln >> 4);
  }
  // score rows of this lane's MFMA outputs: heads hl0 + u (u = 0, 1) of
  // qblock row qbl.  After the cross-qblock sum a lane keeps NS scores: both
  // heads (QPM 1, one qblock per row group: nothing to sum) or head hl0 + uh
  // (QPM 2 and 4: the sum trades the register halves, lanes 0-31 keep head
  // hl0 and lanes 32-63 head hl0 + 1).
  const int hl0 = (2 * lg) % HPM, uh = lane >> 5;
  constexpr int NS = QPM == 1 ? 2 : 1;
  // grid key pass: the lane's rows are qblock qg QPM + lg / ES of heads
  // hl0 + u; their R sum_j Q_j (Q as in the operand, exact power-of-two scale)
  float rqs[GRID ? QG : 1][2];
  constexpr float kGridR = 2.1573f;                       // -c_0 of the 4-bit MaxNorm codebook
  constexpr float kGridD20 = ((2.0f * kGridR) / 15.0f) * 1048576.0f;  // D 2^20 (products enter as x i 2^-20)
  constexpr float kGridR20 = kGridR * 1048576.0f;                     // R 2^20
  if constexpr (GRID) {
#pragma unroll
    for (int qg = 0; qg < QG; qg++)
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const int hl = min(hl0 + u, HG - 1);
        rqs[qg][u] = kGridR * s_qsum[hl * NQB + qg * QPM + lg / ES] * exp2i(-head_exp(s_qmax, hl));
      }
  }
  float escale[NS], erscale[NS];
#pragma unroll
  for (int v = 0; v < NS; v++) {
    const int hl = min(hl0 + (NS == 2 ? v : uh), HG - 1);
    escale[v] = exp2i(head_exp(s_qmax, hl));
    erscale[v] = C::QJL ? exp2i(head_exp(s_rqmax, hl)) : 0.f;
  }
  // QJL correction operands: MFMA s = 4 s4 + sb covers sign byte sb of sign
  // word 4 s4 + kg (k = 8 kg + i <-> element 32 (4 s4 + kg) + 8 sb + i); row
  // m = 4 r + 2 u + part holds part(rq) of head hl0(r) + u, so the sums land
  // in the lanes whose scores they correct
  u32x4 ra[C::QJL ? 4 * C::SW4 : 1];
  if constexpr (C::QJL) {
    const int r = l16 >> 2, u = (l16 >> 1) & 1, part = l16 & 1;
    const int hl = (2 * r) % HPM + u;
#pragma unroll
    for (int s = 0; s < 4 * C::SW4; s++) {
      const int wi = (s >> 2) * 4 + lg, sb = s & 3;
      u32x4 val = {0u, 0u, 0u, 0u};
      if (hl < nh && wi < NQB) {
        const float sc = exp2i(-head_exp(s_rqmax, hl));
        const float *src = s_rq + hl * HD + 32 * wi + 8 * sb;
        uint32_t wv[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const float x0 = src[2 * i] * sc, x1 = src[2 * i + 1] * sc;
          const float h0 = split_hi(x0), h1 = split_hi(x1);
          wv[i] = part ? pack_f16(x0 - h0, x1 - h1) : pack_f16(h0, h1);
        }
        val = u32x4{wv[0], wv[1], wv[2], wv[3]};
      }
      ra[s] = val;
    }
  }
  // the query setup is dead from here: the staging area it lives in is the waves' own
  __syncthreads();

  // ---- the range's chunks: per chunk a K pass, an online softmax step and a
  // V pass whose value sums are folded into the wave's running sums ----
  float *stage = lds + C::OFF_W - LSH + wave * C::WSTAGE;
  float *st_p = stage;                 // [HG][PSTR]
  float *st_s = stage + C::WP;         // [NQB][PSTR]
  float *comb = stage + C::WC;         // [HG][HD] value sums over the chunks
  float *cml = stage + C::WM;          // m[HG], l[HG], 2^Ev, the chunk's rescale [HG]
  // 16-lane rows holding the same head: R replicas (QPM 4: the row groups
  // lg and lg ^ 1; else one), replica ri stores every R-th tile's weights
  constexpr int R = QPM == 4 ? 2 : 1;
  const int ri = QPM == 4 ? (lg & 1) : 0;
  // V pass weight operand of lane (n, kg), column n = (qblock qsp of the
  // set, head hv, weight part): the weights of tokens 4 kg .. 4 kg + 3 of
  // both tiles
  const int qsp = l16 / (2 * HPM), hv = (l16 >> 1) % HPM, wpart = l16 & 1;
  const float kpart = wpart ? -1.f : 0.f;
  if constexpr (MULTI)
    for (int e = lane; e < HG * HD / 4; e += 64) reinterpret_cast<float4 *>(comb)[e] = make_float4(0.f, 0.f, 0.f, 0.f);
  // online softmax state of the lane's head rows (base 2) and the wave's
  // V-scale exponent
  float mrun[NS], lrun[NS];
#pragma unroll
  for (int v = 0; v < NS; v++) {
    mrun[v] = -INFINITY;
    lrun[v] = 0.f;
  }
  int evrun = 0;
  for (int ck = 0; ck < nck; ck++) {
  const int tw = (ck0 + ck) * C::CHUNK + wave * TPW;
  const uint32_t tw0 = (uint32_t)tw;
  // range launches: the K pass above the softmax in wave priority, the V
  // pass above both (C4 56.7 -> 55.5 us; single-chunk launches measured
  // no gain from the K-pass step)
  if constexpr (MULTI) __builtin_amdgcn_s_setprio(1);
  // ---- K pass, tile by tile as the records arrive ----
  // QA_REGS: the operands come into registers for the pass (a reload per
  // chunk through an opaque lane offset, so they do not occupy registers
  // through the V pass)
  u32x4 qa[QAR ? QG * KJA : 1];
  if constexpr (QAR) {
    int qoff = lane;
    if constexpr (MULTI) asm volatile("" : "+v"(qoff));
#pragma unroll
    for (int k = 0; k < QG * KJA; k++) qa[k] = s_qa[k * 64 + qoff];
  }
  float sc[NKT][NS];
#pragma unroll
  for (int i = 0; i < NKT; i++) {
    issue_k(i, tw0);
    f32x4 dk[QG];
#pragma unroll
    for (int qg = 0; qg < QG; qg++) {
      dk[qg] = f32x4{0.f, 0.f, 0.f, 0.f};
      align_part<C>(kw[i][qg], kes);
    }
    if constexpr (GRID) {
#pragma unroll
      for (int qg = 0; qg < QG; qg++)
#pragma unroll
        for (int j = 0; j < KJA; j++) {
          dk[qg] = mfma(qa[qg * KJA + j], nib_operand(kw[i][qg][j]), dk[qg]);
        }
    } else {
    // every pair-table read of the tile goes out before its first MFMA, so
    // the LDS latency is paid once per tile, not once per instruction
    uint2 e[QG][KJ][2];
#pragma unroll
    for (int qg = 0; qg < QG; qg++)
#pragma unroll
      for (int j = 0; j < 2 * KJ; j++)
        e[qg][j >> 1][j & 1] = *reinterpret_cast<const uint2 *>(reinterpret_cast<const char *>(s_pair) +
                                                                pair_off<BITS, NW>(kw[i][qg], j));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int qg = 0; qg < QG; qg++)
#pragma unroll
      for (int j = 0; j < KJ; j++) {
        const u32x4 qv = QAR ? qa[QAR ? qg * KJ + j : 0] : s_qa[(qg * KJ + j) * 64 + lane];
        dk[qg] = mfma(qv, u32x4{e[qg][j][0].x, e[qg][j][0].y, e[qg][j][1].x, e[qg][j][1].y}, dk[qg]);
      }
    }
    f32x4 dq = {0.f, 0.f, 0.f, 0.f};
    if constexpr (C::QJL) {
#pragma unroll
      for (int s = 0; s < 4 * C::SW4; s++) {
        const uint32_t byte = (sgw[i][s >> 2] >> (8 * (s & 3))) & 0xffu;
        const uint2 n0 = s_nib[byte & 15u], n1 = s_nib[byte >> 4];
        dq = mfma(ra[s], u32x4{n0.x, n0.y, n1.x, n1.y}, dq);
      }
    }
    // lane (token l16, row group lg): rows (qbl, head hl0 + u, part)
    float x[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
      x[u] = 0.f;
#pragma unroll
      for (int qg = 0; qg < QG; qg++) {
        const float sk = fabsf(f16_to_f32((uint16_t)ksv[i][qg]));
        float d = dk[qg][2 * u] + dk[qg][2 * u + 1];
        if constexpr (GRID) d = __builtin_fmaf(d, kGridD20, -rqs[qg][u]);
        x[u] = __builtin_fmaf(d, sk, x[u]);
      }
    }
    // sum over the qblocks of the instruction (row groups lg ^ 2 and, for
    // QPM 4, lg ^ 1): one trade of the register halves covers both heads
    float y[NS];
    if constexpr (NS == 2) {
      y[0] = x[0];
      y[1] = x[1];
    } else {
      trade_halves32(x[0], x[1]);
      y[0] = x[0] + x[1];
      if constexpr (QPM == 4) y[0] = sum_xor16(y[0]);
    }
    const bool tok_ok = tw + 16 * i + l16 < len;
#pragma unroll
    for (int v = 0; v < NS; v++) {
      float s = y[v] * escale[v];
      const int u = NS == 2 ? v : uh;
      if constexpr (C::QJL) {
        const float cn = f16_to_f32((uint16_t)nrm[i]) * a.qjl_c;
        const float dqs = NS == 2 ? dq[2 * v] + dq[2 * v + 1] : (uh ? dq[2] + dq[3] : dq[0] + dq[1]);
        s = __builtin_fmaf(dqs, cn * erscale[v], s);
      }
      sc[i][v] = (tok_ok && hl0 + u < nh) ? s : -INFINITY;
    }
  }

  if constexpr (MULTI) __builtin_amdgcn_s_setprio(0);
  // ---- online softmax step (base 2): the running row max of each head
  // moves to mn, the chunk's weights are 2^(s - mn) and the sums so far are
  // rescaled by 2^(m_old - mn) ----
  float alpha[NS];
#pragma unroll
  for (int v = 0; v < NS; v++) {
    float mc = -INFINITY;
#pragma unroll
    for (int i = 0; i < NKT; i++) mc = fmaxf(mc, sc[i][v]);
    const float mn = fmaxf(mrun[v], row_max16(mc));
    float l = 0.f;
    const int hl = hl0 + (NS == 2 ? v : uh);
#pragma unroll
    for (int i = 0; i < NKT; i++) {
      const float p = mn == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sc[i][v] - mn);
      l += p;
      if (hl < HG && i % R == ri) st_p[hl * C::PSTR + 16 * i + l16] = p;
    }
    alpha[v] = mrun[v] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mrun[v] - mn);
    lrun[v] = __builtin_fmaf(lrun[v], alpha[v], row_sum16(l));
    mrun[v] = mn;
  }
  // V scales (lane: tokens TPL lane + u) as |s| 2^-Ev, Ev from the wave's largest
  float svv[C::TPL][NQB];
  float smax = 0.f;
#pragma unroll
  for (int u = 0; u < C::TPL; u++)
#pragma unroll
    for (int qb = 0; qb < NQB; qb++) {
      const uint32_t bits = NQB == 1 ? vsr[u][0] : (vsr[u][qb >> 1] >> (16 * (qb & 1)));
      svv[u][qb] = fabsf(f16_to_f32((uint16_t)(bits & 0xffffu)));
      smax = fmaxf(smax, svv[u][qb]);
    }
  // the running exponent Ev is the largest of the range's chunks so far; the
  // sums so far are rescaled by 2^(Ev_old - Ev) with the softmax factor
  const int evc = pow2_exponent(wave_max(smax));
  const int ev = ck == 0 ? evc : max(evrun, evc);
  const float beta = ck == 0 ? 0.f : exp2i(evrun - ev);
  evrun = ev;
  const float vinv = exp2i(-ev);
#pragma unroll
  for (int u = 0; u < C::TPL; u++)
#pragma unroll
    for (int qb = 0; qb < NQB; qb++) {
      // the grid V pass: even tokens' weights meet codes i 2^-24 (nib_operand), so they take the factor 16
      const float f = GRID && ((C::TPL * lane + u) & 1) == 0 ? vinv * 16.f : vinv;
      st_s[qb * C::PSTR + C::TPL * lane + u] = svv[u][qb] * f;
    }
  if (MULTI && l16 == 0) {
#pragma unroll
    for (int v = 0; v < NS; v++) {
      const int hl = hl0 + (NS == 2 ? v : uh);
      if (hl < HG && ri == 0) cml[2 * HG + 1 + hl] = alpha[v] * beta;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // the V pass at raised wave priority: the other waves of the SIMD, in
  // their K passes or softmax, fill the gaps between its matrix products
  // instead of delaying them (C4 58.8 -> 56.7 us; C3 unchanged)
  __builtin_amdgcn_s_setprio(MULTI ? 3 : 1);
  if constexpr (GRID) {
  // ---- V pass on the grid, 64-token block by block: the block's records
  // are staged token-major in LDS; a transposing 4-bit read hands lane
  // (m, kg) code m of a 16-code chunk for 16 tokens, which become the A
  // operand as exact f16 subnormals (nib_operand; the weight operand takes
  // the same token order), so
  // sum_t W_t c_i = D 2^20 sum_t W_t (i 2^-20) - R 2^20 sum_t W_t 2^-20, the
  // last sum from one MFMA per weight operand over a constant code of 1
  // (nib_operand's scales: the weights of even tokens carry the factor 16). ----
  constexpr int NB = TPW / 64, NCH = 2 * NQB, RS = C::VRS;
  uint8_t *stg = vstage + wave * 64 * RS;
  f32x4 acc[NCH], acc1[QG];
#pragma unroll
  for (int cc = 0; cc < NCH; cc++) acc[cc] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int vs = 0; vs < QG; vs++) acc1[vs] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int bk = 0; bk < NB; bk++) {
    // tiles 4 bk + 4 .. 4 bk + 7 go out as this block's are consumed; the
    // next chunk's first K tiles and V scales with the last block
    if (4 * bk + 4 < NKT) {
#pragma unroll
      for (int u = 4; u < 8; u++)
        if (4 * bk + u < NKT) issue(NKT + 1 + 4 * bk + u, tw0);
    }
    if (MULTI && bk == NB - 1 && ck + 1 < nck) issue_first(tw0 + C::CHUNK, LA);
    // stage the block's four tiles: lane l holds token l / 4 of its tile,
    // bytes 4 NQB (l % 4) .. of the record
#pragma unroll
    for (int u = 0; u < 4; u++)
      stage_words<NQB>(stg + (16 * u + (lane >> 2)) * RS + 4 * NQB * (lane & 3), vg[4 * bk + u]);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // per qblock group: the weight operands for k = 8 kg + 2 r + e <-> token
    // 16 kg + 8 h + r + 4 e of the block (h: which half of the lane group's
    // 16 tokens), then the group's chunks (transposing reads ahead of the
    // MFMAs), so only one group's operands are live at a time
#pragma unroll
    for (int vs = 0; vs < QG; vs++) {
      u32x4 bw[2];
#pragma unroll
      for (int h = 0; h < 2; h++) {
        uint32_t w[4] = {0u, 0u, 0u, 0u};
        if (hv < nh) {
          const int t = 64 * bk + 16 * lg + 8 * h;
          const float4 pa = *reinterpret_cast<const float4 *>(st_p + hv * C::PSTR + t);
          const float4 pb = *reinterpret_cast<const float4 *>(st_p + hv * C::PSTR + t + 4);
          const float4 sa = *reinterpret_cast<const float4 *>(st_s + (vs * QPM + qsp) * C::PSTR + t);
          const float4 sb = *reinterpret_cast<const float4 *>(st_s + (vs * QPM + qsp) * C::PSTR + t + 4);
          const float xa[4] = {pa.x * sa.x, pa.y * sa.y, pa.z * sa.z, pa.w * sa.w};
          const float xb[4] = {pb.x * sb.x, pb.y * sb.y, pb.z * sb.z, pb.w * sb.w};
#pragma unroll
          for (int r = 0; r < 4; r++) w[r] = pack_rem(xa[r], xb[r], pack_f16(xa[r], xb[r]), kpart);
        }
        bw[h] = u32x4{w[0], w[1], w[2], w[3]};
      }
      constexpr int GC = 2 * QPM;  // 16-code chunks of a qblock group
      u32x2 cw[GC];
#pragma unroll
      for (int j = 0; j < GC; j++) cw[j] = lds_read_tr4(stg + (16 * lg + l16) * RS + 8 * (vs * GC + j));
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < GC; j++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
          acc[vs * GC + j] = mfma(nib_operand(cw[j][h]), bw[h], acc[vs * GC + j]);
        }
      // a code of 1 in nib_operand's scales: 2^-24 in registers 0 and 2, 2^-20 in 1 and 3
      constexpr uint32_t kOne = 0x00010001u, kOne16 = 0x00100010u;
#pragma unroll
      for (int h = 0; h < 2; h++) acc1[vs] = mfma(u32x4{kOne, kOne16, kOne, kOne16}, bw[h], acc1[vs]);
    }
  }
  // lane (n, lg) holds codes' dims 16 cc + 4 lg + (0..3) under column n; the
  // two weight parts of a head sit in lanes n, n ^ 1
  {
    const float rf = MULTI ? cml[2 * HG + 1 + dmin(hv, HG - 1)] : 0.f;
    float one[QG];
#pragma unroll
    for (int vs = 0; vs < QG; vs++) {
      const float xx = acc1[vs][0];
      one[vs] = dpp_quad_xor1(xx) + xx;
      asm volatile("" : "+v"(one[vs]));
    }
#pragma unroll
    for (int cc = 0; cc < NCH; cc++) {
      const int qb = cc >> 1, vs = qb / QPM;
      float o[4];
#pragma unroll
      for (int jj = 0; jj < 4; jj++) {
        const float xx = acc[cc][jj];
        float t = dpp_quad_xor1(xx) + xx;
        asm volatile("" : "+v"(t));
        o[jj] = __builtin_fmaf(t, kGridD20, -kGridR20 * one[vs]);
      }
      if (qsp == qb % QPM && wpart == 0 && hv < nh) {
        float4 *dst = reinterpret_cast<float4 *>(comb + hv * HD + 16 * cc + 4 * lg);
        if constexpr (MULTI) {
          const float4 old = *dst;
          *dst = make_float4(__builtin_fmaf(old.x, rf, o[0]), __builtin_fmaf(old.y, rf, o[1]),
                             __builtin_fmaf(old.z, rf, o[2]), __builtin_fmaf(old.w, rf, o[3]));
        } else {
          *dst = make_float4(o[0], o[1], o[2], o[3]);
        }
      }
    }
  }
  } else {
  // ---- V pass, tile pair by tile pair ----
  f32x4 dv[QG][PPL];
#pragma unroll
  for (int vs = 0; vs < QG; vs++)
#pragma unroll
    for (int j = 0; j < PPL; j++) dv[vs][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int vp = 0; vp < NVP; vp++) {
    issue_v(vp, tw0);
    if (MULTI && vp == VP_NEXT && ck + 1 < nck) issue_first(tw0 + C::CHUNK, LA);
    u32x4 bw[QG];
#pragma unroll
    for (int vs = 0; vs < QG; vs++) {
      uint32_t w[4] = {0u, 0u, 0u, 0u};
      if (hv < nh) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
          const int t = 32 * vp + 16 * u + 4 * lg;
          const float4 p4 = *reinterpret_cast<const float4 *>(st_p + hv * C::PSTR + t);
          const float4 s4 = *reinterpret_cast<const float4 *>(st_s + (vs * QPM + qsp) * C::PSTR + t);
          const float x0 = p4.x * s4.x, x1 = p4.y * s4.y, x2 = p4.z * s4.z, x3 = p4.w * s4.w;
          w[2 * u] = pack_rem(x0, x1, pack_f16(x0, x1), kpart);
          w[2 * u + 1] = pack_rem(x2, x3, pack_f16(x2, x3), kpart);
        }
      }
      bw[vs] = u32x4{w[0], w[1], w[2], w[3]};
    }
#pragma unroll
    for (int vs = 0; vs < QG; vs++) {
      align_part<C>(vw[2 * vp][vs], ves);
      align_part<C>(vw[2 * vp + 1][vs], ves);
      // the set's transposing reads all go out ahead of its MFMAs
      u32x2 r[PPL][2];
#pragma unroll
      for (int j = 0; j < PPL; j++) {
        r[j][0] = lds_read_tr16(reinterpret_cast<const char *>(s_pair) + pair_off<BITS, NW>(vw[2 * vp][vs], j));
        r[j][1] = lds_read_tr16(reinterpret_cast<const char *>(s_pair) + pair_off<BITS, NW>(vw[2 * vp + 1][vs], j));
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < PPL; j++) dv[vs][j] = mfma(u32x4{r[j][0][0], r[j][0][1], r[j][1][0], r[j][1][1]}, bw[vs], dv[vs][j]);
    }
  }
  // useful outputs: lane (n, lg) holds rows (row set lg: qblock lg / ES, pair
  // part lg % ES; parts hi c0, hi c1, lo c0, lo c1) under column n; the two
  // weight parts of a head sit in lanes n, n ^ 1.  They are added to the
  // wave's sums, rescaled for this chunk's max and exponent.
  {
    const int oqb = lg / ES, ops = lg % ES;
    const bool keep = qsp == oqb && wpart == 0 && hv < nh;
    const float rf = MULTI ? cml[2 * HG + 1 + dmin(hv, HG - 1)] : 0.f;
#pragma unroll
    for (int vs = 0; vs < QG; vs++)
#pragma unroll
      for (int j = 0; j < PPL; j++) {
        float o[2];
#pragma unroll
        for (int cc = 0; cc < 2; cc++) {
          const float xx = dv[vs][j][cc] + dv[vs][j][cc + 2];
          o[cc] = dpp_quad_xor1(xx) + xx;
          asm volatile("" : "+v"(o[cc]));  // keeps the add beside its DPP read
        }
        if (keep) {
          float2 *dst = reinterpret_cast<float2 *>(comb + hv * HD + (vs * QPM + oqb) * 32 + 2 * (ops * PPL + j));
          if constexpr (MULTI) {
            const float2 old = *dst;
            *dst = make_float2(__builtin_fmaf(old.x, rf, o[0]), __builtin_fmaf(old.y, rf, o[1]));
          } else {
            *dst = make_float2(o[0], o[1]);
          }
        }
      }
  }
  }  // V pass
  __builtin_amdgcn_s_setprio(0);
  }  // chunks
  if (l16 == 0) {
#pragma unroll
    for (int v = 0; v < NS; v++) {
      const int hl = hl0 + (NS == 2 ? v : uh);
      if (hl < HG && ri == 0) {
        cml[hl] = mrun[v];
        cml[HG + hl] = lrun[v];
      }
    }
    if (lane == 0) cml[2 * HG] = exp2i(evrun);
  }

  // ---- combine the waves' records; the workgroup's partial goes out (a
  // (sequence, KV head) of one chunk or range: its output, inverse-rotated
  // and normalized here, with no partial, counter or merge) ----
  if (tid == 0) s_flag = (INLINE_MERGE && (ws_hdr < a.ws_pairs || ws_hdr > a.ws_room)) ? 2 : 0;
  __syncthreads();
  const bool ws_ok = s_flag != 2;
  const bool direct = INLINE_MERGE && nparts == 1;
  const float osg = a_sg ? sgl : decode_sign(tid & 31);
  for (int e = tid; e < nh * HD; e += C::THREADS) {
    const int hl = e / HD, d = e - hl * HD;
    float mw[C::WAVES], M = -INFINITY;
#pragma unroll
    for (int w = 0; w < C::WAVES; w++) {
      mw[w] = lds[C::OFF_W - LSH + w * C::WSTAGE + C::WM + hl];
      M = fmaxf(M, mw[w]);
    }
    float A = 0.f, L = 0.f;
#pragma unroll
    for (int w = 0; w < C::WAVES; w++) {
      const float *cw = lds + C::OFF_W - LSH + w * C::WSTAGE;
      const float f = mw[w] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw[w] - M);
      A = __builtin_fmaf(cw[C::WC + hl * HD + d], f * cw[C::WM + 2 * HG], A);
      L = __builtin_fmaf(cw[C::WM + HG + hl], f, L);
    }
    if (direct) {
      if (ws_ok) {  // (uniform: whole 32-lane blocks of e take the butterfly)
        const float v = wht32_lanes(A * osg, e & 31);
        const float res = (L > 0.f) ? v * kInvSqrt32 / L : 0.f;
        const long long oi = hq0 * HD + e;
        if (a.out_dtype == kF32) static_cast<float *>(a.out)[oi] = res;
        else if (a.out_dtype == kBF16) static_cast<uint16_t *>(a.out)[oi] = f32_to_bf16(res);
        else static_cast<uint16_t *>(a.out)[oi] = f32_to_f16(res);
      }
    } else if (ws_ok) {
      const long long bh = hq0 + hl;
      st_agent(&a.po[(bh * a.P + c) * HD + d], A);
      if (d == 0) {
        st_agent(&a.pm[bh * a.P + c], M);
        st_agent(&a.ps[bh * a.P + c], L);
      }
    }
  }

  // ---- split-K arrival: the last of the (sequence, KV head)'s chunks x
  // head groups merges every head of the KV head.
  // Ordering (gfx942/gfx950 memory model, as LLVM's AMDGPU backend implements
  // it): the partials are agent-scope atomic stores (sc1: written through the
  // XCD's L2 to the device-coherent level) and every wave waits for its own to
  // be acknowledged (s_waitcnt 0) before the workgroup barrier; only then does
  // one lane add to the agent-scope counter, which is performed at the
  // coherent level.  The workgroup that reads the final count has every other
  // workgroup's increment, and so every partial, complete at that level; its
  // merge loads are agent-scope loads (sc1: they read the coherent level,
  // never a stale L2 line), issued after the counter's value has
  // returned and a barrier.  An acq_rel counter would add an L2 writeback and
  // invalidate per workgroup that this needs nowhere. ----
  if constexpr (!INLINE_MERGE) return;
  if (direct) {
    if (!ws_ok) {
      for (int e = tid; e < nh * HD; e += C::THREADS) {
        const long long oi = hq0 * HD + e;
        if (a.out_dtype == kF32) static_cast<float *>(a.out)[oi] = __builtin_nanf("");
        else static_cast<uint16_t *>(a.out)[oi] = 0x7e00;  // quiet NaN in f16 and bf16 alike
      }
    }
    return;
  }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __syncthreads();
  int *counter = a.cnt_top - (1 + b * a.num_kv_heads + g) * kCounterStride;
  if (tid == 0 && ws_ok) {
    const int prev = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_flag = (prev == nparts * a.ngroups - 1);
  }
  __syncthreads();
  if (!ws_ok) {
    for (int e = tid; e < nh * HD; e += C::THREADS) {
      const long long oi = hq0 * HD + e;
      if (a.out_dtype == kF32) static_cast<float *>(a.out)[oi] = __builtin_nanf("");
      else static_cast<uint16_t *>(a.out)[oi] = 0x7e00;  // quiet NaN in f16 and bf16 alike
    }
  } else if (s_flag) {
    if constexpr (INLINE_MERGE) {
      merge_heads<HD, C::WAVES>(a, b, g, nparts);
      if (tid == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

#ifndef TQ_BALANCE
#define TQ_BALANCE 1
#endif
#ifndef TQ_BAL_WGS
#define TQ_BAL_WGS 3  // at most this many balanced workgroups per compute unit
#endif

// 4-bit codes on the compiled-in MaxNorm codebook (evenly spaced) take the
// grid key pass; a caller's codebook or the L2Norm tables, the pair table
template <class C, bool INLINE, bool MULTI>
void launch_stream_k(AttnArgs &a, dim3 grid, hipStream_t st, int len_hint) {
  auto go = [&](auto kernel) {
    if (a.bal_nwg < 0) {
      // balanced split: as many workgroups as the compute units hold at once
      // (this kernel's occupancy, cached per device), at most one per task
      static int occ[64] = {};
      int dev = 0;
      (void)hipGetDevice(&dev);
      dev = dev >= 0 && dev < 64 ? dev : 0;
      if (occ[dev] == 0) {
        int n = 0;
        occ[dev] = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, C::THREADS, 0) == hipSuccess && n > 0
                       ? min(n, TQ_BAL_WGS)
                       : 2;
      }
      a.bal_nwg = (int)min((long long)-a.bal_nwg, (long long)occ[dev] * device_cus());
      grid = dim3((unsigned)a.bal_nwg, 1u, 1u);
    }
    hipLaunchKernelGGL(kernel, grid, dim3(C::THREADS), 0, st, a.k_idx, a.v_idx, a.k_sc, a.v_sc, a.seq_stride,
                       a.kv_head_stride, len_hint, a);
  };
  if constexpr (C::BITS == 4 && C::MODE == kModePqo) {
    if (!a.cb_dev && !a.cb_args) return go(stream_decode_kernel<C, INLINE, true, MULTI>);
  }
  if constexpr (C::QJL) {
    if (!a.rq) return go(stream_decode_kernel<C, INLINE, false, MULTI, true>);
  }
  go(stream_decode_kernel<C, INLINE, false, MULTI>);
}
template <class C, bool INLINE>
void launch_stream_c(AttnArgs &a, dim3 grid, hipStream_t st) {
  a.chunk = C::CHUNK;
  const int chunks = (a.max_len + C::CHUNK - 1) / C::CHUNK;
  // Chunks per workgroup: one while the grid of single chunks fits one round
  // of resident workgroups (three waves per SIMD); beyond that, ranges of
  // several chunks, so that each workgroup pays its setup, combine and
  // split-K arrival once per range and streams the next chunk's first tiles
  // during the current chunk's value pass.  The range length is sized for
  // one round of the range kernel (two workgroups per compute unit) with
  // every sequence at max_len.  Measured at C4 (16 sequences of 4096-16384
  // tokens, capacity 16384): 8 chunks per range 69.5 us; 7, 10, 12 and 16
  // chunks 79.0, 82.1, 81.4 and 93.7 us, so the batch's actual lengths do
  // not pick a shorter range.  The reference ABI's separate merge launch
  // takes single chunks.
  a.cpr = 1;
  if constexpr (INLINE) {
    const long long tasks = (long long)chunks * grid.y * grid.z;
    const long long cus = device_cus();
#ifndef TQ_RANGE_WGS
#define TQ_RANGE_WGS 2
#endif
    if (tasks > cus * (12 / C::WAVES)) {
      a.cpr = (int)min((long long)max(chunks, 1), (tasks + TQ_RANGE_WGS * cus - 1) / (TQ_RANGE_WGS * cus));
      // Balanced split: as many near-equal ranges as the compute units hold
      // at once (up to TQ_BAL_WGS per unit), for one head group per KV head
      // and at most 64 sequences (a wave holds their chunk counts).  Ragged
      // batches then load every compute unit alike; with ranges of a fixed
      // length, a unit that holds two full ranges of long sequences sets the
      // time.  Measured at C4: 64.3 -> 58.6 us; 16 sequences all at 16,384
      // tokens 66.6 -> 67.2 us.
      if (TQ_BALANCE && a.ngroups == 1 && grid.z <= 64u) {
        a.bal_nwg = (int)-min(tasks, (long long)1 << 30);  // negative: sized by launch_stream_k
        a.bal_batch = (int)grid.z;
        a.bal_ny = (int)grid.y;
        const int len_hint = a.kv_lens ? -1 : max(a.single_len, 0);
        return launch_stream_k<C, INLINE, true>(a, grid, st, len_hint);
      }
    }
  } else if constexpr (C::CHUNK < kRefPartition) {
    // The reference ABI's caller sizes its partials for 512-token partitions
    // (cuda/attention.rs:70-77): a configuration with shorter chunks takes
    // ranges of 512 tokens, one partial per range.
    static_assert(kRefPartition % C::CHUNK == 0, "whole chunks per reference partition");
    a.cpr = kRefPartition / C::CHUNK;
  }
  grid.x = (unsigned)((chunks + a.cpr - 1) / a.cpr);
  if (grid.x == 0) grid.x = 1;  // an empty batch still zeroes its outputs
  const int len_hint = a.kv_lens ? -1 : max(a.single_len, 0);
  if constexpr (INLINE || C::CHUNK < kRefPartition) {
    if (a.cpr > 1) return launch_stream_k<C, INLINE, true>(a, grid, st, len_hint);
  }
  launch_stream_k<C, INLINE, false>(a, grid, st, len_hint);
}
// The cache decode picks the workgroup size per launch: 8 waves while the
// grid of 8-wave workgroups leaves compute units idle (one long sequence:
// the halved split-K merge is on the critical path), else 4 waves (several
// workgroups per compute unit keep more waves per SIMD in flight).  The
// reference ABI (a separate merge launch) always takes the 8-wave form.
template <int BITS, int MODE, int NQB, int HG, bool INLINE>
void launch_stream_cfg(AttnArgs &a, dim3 grid, hipStream_t st) {
  using C = StreamCfg<BITS, MODE, NQB, HG>;
  using C4 = StreamCfg4<BITS, MODE, NQB, HG>;
  using C64 = StreamCfg64<BITS, MODE, NQB, HG>;
  if constexpr (INLINE && C::WAVES != 4) {
    const long long wgs = (long long)((a.max_len + C::CHUNK - 1) / C::CHUNK) * grid.y * grid.z;
    if (wgs > device_cus()) return launch_stream_c<C4, INLINE>(a, grid, st);
    // a grid that leaves compute units idle: 64 tokens per wave when that
    // grid still fits one round (C3's shape up to 16,384 tokens: 2,048 and
    // 4,096 tokens 11.8 / 12.0 -> 9.5 us; 32,768 stays at 128)
    if constexpr (C::TPW == 128 && C64::LDS_FITS) {
      const long long wgs64 = (long long)((a.max_len + C64::CHUNK - 1) / C64::CHUNK) * grid.y * grid.z;
      if (wgs64 <= device_cus()) return launch_stream_c<C64, INLINE>(a, grid, st);
    }
  }
  launch_stream_c<C, INLINE>(a, grid, st);
}
template <int BITS, int MODE, int NQB, bool INLINE>
void launch_stream_hg(AttnArgs &a, int hg, dim3 grid, hipStream_t st) {
  if (hg == 2) launch_stream_cfg<BITS, MODE, NQB, 2, INLINE>(a, grid, st);
  else if (hg == 4) launch_stream_cfg<BITS, MODE, NQB, 4, INLINE>(a, grid, st);
  else launch_stream_cfg<BITS, MODE, NQB, 8, INLINE>(a, grid, st);
}
template <int BITS, int MODE, bool INLINE>
void launch_stream_nqb(AttnArgs &a, int nqb, int hg, dim3 grid, hipStream_t st) {
  if constexpr (MODE != kModeTq) {
    if (nqb == 1) return launch_stream_hg<BITS, MODE, 1, INLINE>(a, hg, grid, st);
  }
  if (nqb == 2) launch_stream_hg<BITS, MODE, 2, INLINE>(a, hg, grid, st);
  else if (nqb == 4) launch_stream_hg<BITS, MODE, 4, INLINE>(a, hg, grid, st);
  else launch_stream_hg<BITS, MODE, 8, INLINE>(a, hg, grid, st);
}
}  // namespace

template <int BITS, int MODE, bool INLINE>
void launch_stream_bm(AttnArgs &a, int nqb, int hg, dim3 grid, hipStream_t st) {
  launch_stream_nqb<BITS, MODE, INLINE>(a, nqb, hg, grid, st);
}

}  // namespace tqa
