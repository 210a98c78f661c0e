// tq_prefill.hip -- multi-query (prefill) attention straight over the
// compressed cache, on the matrix cores.
//
// The reference hands prefill attention back to the caller as dequantized
// K/V (pqo.rs:184-200, tq.rs:258-273; SDPA runs in mistral.rs).  This kernel
// computes it without materializing K/V: out[h][i] = softmax_t(scale *
// (q_hi . k_t + corr_hit)) v_t over the tokens t a query may see (all, or
// t <= kv_len - q_len + i when causal), corr the QJL correction of a TQ
// cache (tq.rs:185-253).
//
// One workgroup serves 128 rows = (query, head) pairs of one KV head (8
// waves), query-major, so the NR query heads of a KV head share every
// decoded tile.  Per 64-token tile the
// workgroup decodes K and V (token-major, one K and one V exponent per
// 16-token slice folded out) into LDS as two-part f16 values (hi = 11
// significant bits, lo = the remainder), then each wave (16 rows) runs
//   S^T = K Q^T          16x16x32 MFMAs per 32-element slice: K hi x Q hi,
//                        K hi x Q lo, K lo x Q hi (22-bit products, lo x lo
//                        dropped, f32 accumulation; staged tiles with a bf16
//                        or f16 query: K hi x Q, K lo x Q)
//   corr^T = Sg RQ^T     TQ: the keys' +-1 sign bits against rq hi/lo
//   O^T += V^T P^T       16x16x32 MFMAs over two 16-token blocks whose B
//                        operand is S^T's accumulator layout (4 tokens per
//                        lane and block), the V operand read through the
//                        transposing LDS read, V hi/lo x P hi/lo (three
//                        products, lo x lo dropped)
// with an online base-2 softmax per row.  The four 16-token blocks of the
// key pass and pairs of 16-element blocks of the value pass run as
// independent accumulator chains, interleaved (each accumulator still sums
// its products in the same order); the value pass runs at raised wave
// priority.  Values stay in the rotated domain; each
// row is inverse-rotated once at the end.  Two tile buffers: tile t + 1 is
// decoded while tile t is computed (one barrier per tile), and the records of
// tile t + 2 are fetched meanwhile.
//
// Staged tiles (6 or more query blocks per KV head over 768 or more tokens):
// the query blocks of a KV head would each decode every tile again, so a
// staging pass (the same kernel, one workgroup per tile and KV head)
// decodes each tile once into an image of the tile buffer's LDS contents (TQ:
// with the sign words and scaled norms), and the attention workgroups copy
// the images into LDS in place of decoding.  The staging pass inverse-rotates
// K (original domain) and the attention takes the query unrotated, so a bf16
// or f16 query is exact in f16 and each key slice takes two products (K hi Q,
// K lo Q) instead of three; V stays rotated.  Both launches put KV head g on
// one XCD (g = linear index mod 8, workgroups being dealt to the 8 XCDs in
// turn): a head's images are written and read through one L2.
#include "tq_common.h"
#include "tq_device.h"
#include "tq_mfma.h"

#include <mutex>
#include <type_traits>

namespace {

using namespace tqd;
using namespace tqm;

// (query, head) rows per workgroup: 128 (8 waves) share each decoded tile,
// the TQ mode too (its waves fit 244 registers at 8 waves per workgroup)
constexpr int prefill_rows(int) { return 128; }
constexpr int kTile = 64;   // tokens per tile
constexpr int kKStride = 68;  // uint2 per token row of the K tile (32 chunks of 16 bytes + pad)
constexpr int kVRow = 144;    // halves per token row of the V tiles (128 elements + pad: the
                              // transposing reads of 4 tokens x 4 element quads hit 32 distinct banks)

// A K tile row holds, per 8-element group g, a 16-byte chunk of hi halves
// (2 g) and one of lo halves (2 g + 1).  Chunk c of row r sits at
// c ^ 2 ((c >> 3) & 3) ^ (r & 1), rows 34 chunks apart: the S^T reads (16
// rows x 4 chunks per 16-byte read) and the in-workgroup decode's stores (16
// tokens x 4 qblocks) are both free of LDS bank conflicts on gfx950 (measured
// with SQ_LDS_BANK_CONFLICT: the previous 33-chunk rows without the row term
// cost the reads 3.9 conflict cycles each, 2x their 4-cycle minimum).
__device__ __forceinline__ int kchunk(int c, int row) { return c ^ (2 * ((c >> 3) & 3)) ^ (row & 1); }
// The V rows' 16-byte chunk c (8 elements of one plane) sits at chunk
// c ^ ((c >> 3) & 1): rows are 18 chunks apart, and the 16-byte stores of
// tokens t, t + 1 (qblocks 0-3 each: chunks 0, 4, 8, 12 from the row start)
// then reach 8 distinct bank groups instead of 4; a transposing read (8
// bytes of one chunk per lane, 4 rows x 2 chunks per 16 lanes) stays
// distinct.
__device__ __forceinline__ int vchunk(int c) { return c ^ ((c >> 3) & 1); }
// Row strides of the staged query halves and the output floats, padded so
// that consecutive rows start 4 banks apart (the per-row accesses of 16 rows
// would otherwise all start in one bank)
constexpr int kQRow = 128 + 8;  // halves
constexpr int kORow = 128 + 4;  // floats

// Shapes whose tiles are decoded once, in a staging pass, instead of in every
// workgroup: at least this many query blocks per KV head and tokens (the
// second launch and writing the images have a cost that the decodes saved
// must repay: each tile is decoded by up to q_blocks workgroups otherwise;
// 16/8 heads, bf16 queries, both paths split over the tiles where the grid
// is small, in-workgroup vs staged, us: 128 causal queries at the end of
// 32768 tokens 135.8 vs 184.5, 256 x 32768 236.6 vs 261.8, 256 x 8192 80.9
// vs 80.0, 512 x 32768 450.7 vs 428.1; without splits 512 x 512 causal 36.1
// vs 36.1, 768 x 768 causal 49.1 vs 45.8, 2048 x 2048 causal 117.3 vs 93.8)
constexpr int kStagingMinQueryBlocks = 6;
constexpr int kStagingMinTokens = 768;
// A staged tile image: the tile buffer's K rows and V planes, then its
// exponent words (the slices' K exponents, the waves' V exponents), for a TQ
// cache then the sign words and the scaled residual norms, in 16-byte chunks
constexpr int kTileChunks = (kTile * kKStride * 2 + kTile * kVRow) / 4;
constexpr int kImgChunksPq = kTileChunks + 3;
// a TQ tile adds its tokens' sign words (64 x 4) and scaled norms (64)
constexpr int kImgChunksTq = kImgChunksPq + kTile + kTile / 4;
constexpr int img_chunks(int mode) { return mode == 2 ? kImgChunksTq : kImgChunksPq; }

// Stores 32 values split into f16 hi (11 significant bits) and lo (the
// exact remainder) at hi[0..31] and lo[0..31], 16 bytes per store.
__device__ __forceinline__ void stage_split32(const float (&x)[32], _Float16 *hi, _Float16 *lo) {
  uint32_t hw[16], lw[16];
#pragma unroll
  for (int k = 0; k < 16; k++) {
    const float h0 = split_hi(x[2 * k]), h1 = split_hi(x[2 * k + 1]);
    const _Float16 a0 = (_Float16)h0, a1 = (_Float16)h1;
    const _Float16 b0 = (_Float16)(x[2 * k] - h0), b1 = (_Float16)(x[2 * k + 1] - h1);
    hw[k] = (uint32_t)__builtin_bit_cast(uint16_t, a0) | ((uint32_t)__builtin_bit_cast(uint16_t, a1) << 16);
    lw[k] = (uint32_t)__builtin_bit_cast(uint16_t, b0) | ((uint32_t)__builtin_bit_cast(uint16_t, b1) << 16);
  }
  uint4 *dh = reinterpret_cast<uint4 *>(hi), *dl = reinterpret_cast<uint4 *>(lo);
#pragma unroll
  for (int k = 0; k < 4; k++) {
    dh[k] = make_uint4(hw[4 * k], hw[4 * k + 1], hw[4 * k + 2], hw[4 * k + 3]);
    dl[k] = make_uint4(lw[4 * k], lw[4 * k + 1], lw[4 * k + 2], lw[4 * k + 3]);
  }
}

enum PMode : int { kPPqo = 0, kPPq = 1, kPTq = 2 };

struct PrefillArgs {
  const void *q;
  int q_dtype;
  const uint8_t *k_idx;
  const uint16_t *k_sc;
  const uint8_t *v_idx;
  const uint16_t *v_sc;
  const float *rq;           // TQ: [H][q_len][128] = R q
  const uint32_t *signs;     // TQ: [record][4] sign words
  const uint16_t *norms;     // TQ: [record] f16 residual norms
  int num_heads, num_kv_heads, q_len, kv_len;
  long long kv_head_stride;  // records between KV heads
  int causal;
  float softmax_scale;
  float qjl_c;               // f32(sqrt(pi/2)) / sqrt(head_dim)
  void *out;
  int out_dtype;
  int cb_args;               // codebook from cb (L2Norm) instead of the MaxNorm constants
  float cb[16];
  // staged decode: per KV head, stage_tiles tile images of img_chunks(mode) 16-byte
  // chunks (the LDS contents of one decoded tile)
  const uint4 *stage;
  uint4 *stage_out;
  int stage_tiles;
  int stage_tpw;  // staging pass: consecutive tiles per workgroup
  // split-K over the tiles: workgroup z takes tiles [z tps, (z + 1) tps) of
  // its query block; with splits > 1 it writes partial rows to part
  int splits, tps;
  float *part;
};

// A partial row of a split: the inverse-rotated output sums (unnormalized,
// relative to the row maximum) [0, 128), the row maximum m (log2 domain)
// [128] and the row sum [129], padded to 16 bytes; rows [split][head][query]
constexpr int kPartRow = 132;

// Kernel phases: decode every tile in the workgroup (kDecode); the staging
// pass, one workgroup per tile and KV head, which writes the tile's image
// (kStage); read the tiles as those images (kStaged)
enum PPhase : int { kDecode = 0, kStaged = 1, kStage = 2 };

template <int BITS, int MODE, int NR, int PH>
__global__ __launch_bounds__(4 * prefill_rows(MODE)) void prefill_attn_kernel(PrefillArgs a) {
  constexpr int CB = MODE == kPPqo ? BITS : BITS - 1;
  constexpr bool QJL = MODE == kPTq;
  // staged tiles hold K in the original domain (the staging pass inverse-
  // rotates it) and the query is taken as it is: a bf16 or f16 query is then
  // exact in f16 and the key pass needs no product with its lo part
  constexpr bool ORIG = PH != kDecode;
  constexpr int HD = 128, QW = BITS, PACKED = 16 * QW;
  constexpr int kRows = prefill_rows(MODE);
  constexpr int NW = kRows / 16;            // waves
  constexpr int SPLIT = NW / 4;             // waves per 16-token slice of a tile's decode
  constexpr int NP = 16 / SPLIT;            // code pairs per decoding thread
  constexpr int QB = kRows / NR;  // queries per workgroup
  // LDS: K tile | V tiles (hi, lo) per buffer; slice exponents, TQ sign
  // words and norms, and per-row scalars beside them
  constexpr int K_WORDS = kTile * kKStride * 2;
  constexpr int V_HALVES = kTile * kVRow;
  constexpr int V_WORDS = V_HALVES;  // hi and lo planes, 2 halves per word each
  // K tile | V tiles; before the tiles the split query (and rq) rows, after
  // them the output rows
  // two tile buffers: tile t + 1 is decoded into one while tile t is read
  // from the other
  constexpr int TILE_WORDS = K_WORDS + V_WORDS;
  constexpr int IMG = img_chunks(MODE);
  static_assert(PH == kDecode || NW == 8, "staged tiles: 8 waves");
  static_assert(PH == kDecode || (TILE_WORDS / 4 == kTileChunks && kImgChunksPq == kTileChunks + 3),
                "the tile image is the LDS tile buffer plus its 12 exponent words (and the TQ arrays)");
  // (the staging pass decodes into one buffer, then copies it out)
  __shared__ __attribute__((aligned(16))) uint32_t s_tile[PH == kStage ? TILE_WORDS : 2 * TILE_WORDS];
  // per tile, read 4 at a time: [0..3] the K exponent E_k of each 16-token slice, [4 + w] the V
  // exponent E_v of decoding wave w's slice (the exponents folded out of the
  // decoded values)
  static_assert(NW <= 8 && kTile == 64, "4 slices, at most 8 decoding waves");
  __shared__ __attribute__((aligned(16))) int s_xe[2][12];
  __shared__ __attribute__((aligned(16))) float s_cn[2][kTile];       // TQ: |r_t| * qjl_c
  __shared__ __attribute__((aligned(16))) uint32_t s_sg[2][kTile * 4];  // TQ: sign words
  __shared__ float s_cb[16];
  __shared__ int s_eq[kRows], s_er[kRows];
  __shared__ uint2 s_nib[16];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // -1 in a register the compiler cannot see through, so x + (-1) * hi stays
  // one v_fma_mix_f32 instead of a widening convert and a subtraction
  float mone = -1.f;
  asm volatile("" : "+v"(mone));
  const int l16 = lane & 15, lg = lane >> 4;
  // Workgroups start in the order of their linear index.  Causal blocks'
  // work grows with the query block, so the linear index is mapped to the
  // longest blocks first (every KV head's last query block, then the blocks
  // before it): the short blocks fill in at the end instead of the long ones
  // starting last.  Either way KV head = linear index mod KV heads, so (with
  // 8 heads and workgroups dealt to the XCDs round-robin) a head's query
  // blocks share the XCD, and L2, that its staged tiles are written from and
  // read through (full attention, 1024 x 8192: 218.5 -> 210.5 us).
  int g = blockIdx.y, qblk = blockIdx.x;
  if (PH == kStage) {
    // staging pass, a 1-D grid: KV head g = linear index mod num_kv_heads,
    // so (with 8 heads) each head's tiles are decoded on the XCD whose
    // attention workgroups read them (-3.3 % at the bench shape); qblk is
    // the tile
    g = (int)blockIdx.x % a.num_kv_heads;
    qblk = (int)blockIdx.x / a.num_kv_heads;
  }
  if (PH != kStage) {
    const int lin = blockIdx.y * gridDim.x + blockIdx.x;
    g = lin % gridDim.y;
    qblk = a.causal ? (int)gridDim.x - 1 - lin / (int)gridDim.y : lin / (int)gridDim.y;
  }
  const int i0 = qblk * QB;
  const long long rec0 = (long long)g * a.kv_head_stride;
  const float lscale = a.softmax_scale * kLog2e;

  // the codebook (for decoding) and the sign-nibble table (QJL correction)
  if (tid < 16) {
    if (PH != kStaged) {
      constexpr int CM = (1 << CB) - 1;
      float c = a.cb[0];
      if (a.cb_args) {
#pragma unroll
        for (int kk = 1; kk <= CM; kk++) c = (tid == kk) ? a.cb[kk] : c;
      } else {
        c = pqo_centroid<CB>(tid & CM);
      }
      s_cb[tid] = c;
    }
    auto pm1 = [&](int bit) { return ((tid >> bit) & 1) ? 0x3C00u : 0xBC00u; };
    s_nib[tid] = make_uint2(pm1(0) | (pm1(1) << 16), pm1(2) | (pm1(3) << 16));
  }

  // thread (token, qblock) fetches one record of K and V per tile
  // thread (token, qblock, part): wave w decodes tokens 16 (w / SPLIT) ..
  // + 15, code pairs NP (w % SPLIT) .. + NP - 1 of every qblock
  // (staging pass: waves 0-3 take the K records of slices 0-3, waves 4-7 the
  // V records, whole qblocks)
  const int ftok = 16 * (PH == kStage ? (wave & 3) : wave / SPLIT) + (lane >> 2), fqb = lane & 3,
            fpart = wave % SPLIT;
  uint32_t kw[QW], vw[QW], sgw = 0;
  uint16_t ks = 0, vs = 0, nm = 0;
  // staged: thread tid moves chunks tid + 4 kRows r of a tile image
  constexpr int IMG_ROUNDS = (IMG + 4 * kRows - 1) / (4 * kRows);
  // (native vectors: an array of uint4 structs stays in scratch memory)
  u32x4 img[PH == kStaged ? IMG_ROUNDS : 1];
  // staged: KV head g's tile images as one buffer resource (scalar registers;
  // the host bounds a head's images below 2^31 bytes)
  auto make_img_rsrc = [&]() {
    const uint64_t p = reinterpret_cast<uint64_t>(a.stage + (long long)g * a.stage_tiles * IMG);
    const uint64_t ps = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(p >> 32)) << 32) |
                        (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)p);
    const int n = __builtin_amdgcn_readfirstlane(a.stage_tiles * IMG * 16);
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void *>(ps), (short)0, n, 0x00020000);
  };
  const __amdgpu_buffer_rsrc_t img_rsrc = make_img_rsrc();
  // staging pass: one K (waves 0-3) or V (waves 4-7) record of the tile at
  // t0 into w, sc (TQ: the sign word and norm)
  auto load_rec = [&](int t0, uint32_t(&w)[QW], uint16_t &sc, uint32_t &sg, uint16_t &n) {
    const long long rec = rec0 + min(t0 + ftok, a.kv_len - 1);
    const bool kwave = wave < 4;
    const uint32_t *src =
        reinterpret_cast<const uint32_t *>((kwave ? a.k_idx : a.v_idx) + rec * PACKED + fqb * 4 * QW);
#pragma unroll
    for (int i = 0; i < QW; i++) w[i] = src[i];
    sc = (kwave ? a.k_sc : a.v_sc)[rec * 4 + fqb];
    if constexpr (QJL) {
      if (kwave) {
        sg = a.signs[rec * 4 + fqb];
        n = a.norms[rec];
      }
    }
  };
  auto fetch = [&](int t0) {
    if constexpr (PH == kStaged) {
      // buffer loads: the lane's offset in a vector register (the same for
      // every tile), the tile's and the round's in a scalar register
      const uint32_t soff = (uint32_t)(t0 / kTile) * (uint32_t)(IMG * 16);
#pragma unroll
      for (int r = 0; r < IMG_ROUNDS; r++)
        if (r + 1 < IMG_ROUNDS || tid + 4 * kRows * r < IMG)
          img[r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                 img_rsrc, (uint32_t)tid * 16u, soff + (uint32_t)(r * 4 * kRows * 16), 0));
      return;
    }
    if constexpr (PH == kStage) {
      load_rec(t0, kw, ks, sgw, nm);
      return;
    }
    const int t = min(t0 + ftok, a.kv_len - 1);
    const long long rec = rec0 + t;
#pragma unroll
    for (int w = 0; w < QW; w++) {
      kw[w] = reinterpret_cast<const uint32_t *>(a.k_idx + rec * PACKED + fqb * 4 * QW)[w];
      vw[w] = reinterpret_cast<const uint32_t *>(a.v_idx + rec * PACKED + fqb * 4 * QW)[w];
    }
    ks = a.k_sc[rec * 4 + fqb];
    vs = a.v_sc[rec * 4 + fqb];
    if constexpr (QJL) {
      sgw = a.signs[rec * 4 + fqb];
      nm = a.norms[rec];
    }
  };
  // buffer b: K tile at s_tile + b TILE_WORDS, V hi plane after it, lo plane
  // after that
  auto tile_base = [&](int b) -> uint32_t * { return s_tile + b * TILE_WORDS; };
  auto ktile = [&](int b) { return reinterpret_cast<uint2 *>(tile_base(b)); };
  auto vhi = [&](int b) { return reinterpret_cast<_Float16 *>(tile_base(b) + K_WORDS); };
  auto xe = [&](int b) -> int * { return s_xe[b]; };
  // TQ: the tile's sign words and scaled norms
  auto sgp = [&](int b) -> uint32_t * { return s_sg[b]; };
  auto cnp = [&](int b) -> float * { return s_cn[b]; };
  static_assert(2 * V_HALVES <= 2 * V_WORDS, "both V planes fit");
  // (the query and rq staging precedes the tiles and may span both buffers)
  static_assert((QJL ? 2 : 1) * kRows * kQRow <= 2 * (K_WORDS + V_WORDS), "the split query (and rq) fit the tile region");
  static_assert(kRows * kORow + 2 * kRows <= K_WORDS + V_WORDS, "the output rows fit the tile region");

  // chunk c of tile buffer b's image: the K tile and V planes, then the
  // exponent words, then (TQ) the sign words and the scaled norms
  auto img_chunk = [&](int b, int c) -> uint4 * {
    if (c < kTileChunks) return reinterpret_cast<uint4 *>(s_tile + b * TILE_WORDS) + c;
    if (!QJL || c < kImgChunksPq) return reinterpret_cast<uint4 *>(s_xe[b]) + (c - kTileChunks);
    if (c < kImgChunksPq + kTile) return reinterpret_cast<uint4 *>(s_sg[b]) + (c - kImgChunksPq);
    return reinterpret_cast<uint4 *>(s_cn[b]) + (c - kImgChunksPq - kTile);
  };

  // ---- decode this thread's record into tile buffer b (staged: store the
  // fetched image chunks) ----
  auto decode_tile = [&](int b) {
    if constexpr (PH == kStaged) {
#pragma unroll
      for (int r = 0; r < IMG_ROUNDS; r++) {
        const int c = tid + 4 * kRows * r;
        if (r + 1 < IMG_ROUNDS || c < IMG) *reinterpret_cast<u32x4 *>(img_chunk(b, c)) = img[r];
      }
      return;
    }
    uint2 *kt = ktile(b);
    _Float16 *vth = vhi(b), *vtl = vth + V_HALVES;  // the lo plane follows the hi plane
    {
      // one exponent per 16-token slice for K and one for V: the wave's 64
      // lanes hold the slice's 16 tokens x 4 qblock scales (the SPLIT waves of
      // a slice reduce the same scales), so the softmax applies 4 factors per
      // tile instead of one per token
      const float sk = fabsf(f16_to_f32(ks)), sv = fabsf(f16_to_f32(vs));
      const int ek = pow2_exponent(wave_max(sk)), ev = pow2_exponent(wave_max(sv));
      const float kf = sk * exp2i(-ek), vf = sv * exp2i(-ev);
      if (lane == 0) {
        if (fpart == 0) xe(b)[wave / SPLIT] = ek;
        xe(b)[4 + wave] = ev;
      }
      if constexpr (QJL) {
        if (fqb == 0) cnp(b)[ftok] = f16_to_f32(nm) * a.qjl_c;
      }
      if constexpr (QJL) sgp(b)[ftok * 4 + fqb] = sgw;
      // this thread's code pairs P0 .. P0 + NP - 1 (a wave-uniform part, so
      // every pair index folds to a constant)
      auto decode_pairs = [&](auto p0c) {
        constexpr int P0 = decltype(p0c)::value;
        // every codebook value of the K and V codes first (the reads go out
        // together instead of in dependent groups), then the products
        constexpr uint32_t SM = (1u << BITS) - 1u, CMk = (1u << CB) - 1u;
        float ck[2 * NP], cv[2 * NP];
#pragma unroll
        for (int pp = 0; pp < NP; pp++) {
          const uint32_t code = pair_code<BITS>(kw, P0 + pp);
          ck[2 * pp] = s_cb[code & SM & CMk];
          ck[2 * pp + 1] = s_cb[(code >> BITS) & CMk];
        }
#pragma unroll
        for (int pp = 0; pp < NP; pp++) {
          const uint32_t code = pair_code<BITS>(vw, P0 + pp);
          cv[2 * pp] = s_cb[code & SM & CMk];
          cv[2 * pp + 1] = s_cb[(code >> BITS) & CMk];
        }
        uint32_t hw[NP], lw[NP];
#pragma unroll
        for (int pp = 0; pp < NP; pp++) {
          const float x0 = ck[2 * pp] * kf, x1 = ck[2 * pp + 1] * kf;
          hw[pp] = pack_f16(x0, x1);
          lw[pp] = pack_rem(x0, x1, hw[pp], mone);
        }
        // 8-element groups of qblock fqb: chunk 8 fqb + 2 g holds the hi
        // halves, the next chunk the lo halves
        uint4 *krow = reinterpret_cast<uint4 *>(kt + ftok * kKStride);
#pragma unroll
        for (int i = 0; i < NP / 4; i++) {
          const int c = 8 * fqb + 2 * (P0 / 4 + i);
          krow[kchunk(c, ftok)] = make_uint4(hw[4 * i], hw[4 * i + 1], hw[4 * i + 2], hw[4 * i + 3]);
          krow[kchunk(c + 1, ftok)] = make_uint4(lw[4 * i], lw[4 * i + 1], lw[4 * i + 2], lw[4 * i + 3]);
        }
#pragma unroll
        for (int pp = 0; pp < NP; pp++) {
          const float x0 = cv[2 * pp] * vf, x1 = cv[2 * pp + 1] * vf;
          hw[pp] = pack_f16(x0, x1);
          lw[pp] = pack_rem(x0, x1, hw[pp], mone);
        }
        // token-major rows: this thread's 2 NP elements, 16-byte stores per plane
        _Float16 *vrh = vth + ftok * kVRow, *vrl = vtl + ftok * kVRow;
#pragma unroll
        for (int i = 0; i < NP / 4; i++) {
          const int c = 8 * vchunk(4 * fqb + P0 / 4 + i);
          *reinterpret_cast<uint4 *>(vrh + c) = make_uint4(hw[4 * i], hw[4 * i + 1], hw[4 * i + 2], hw[4 * i + 3]);
          *reinterpret_cast<uint4 *>(vrl + c) = make_uint4(lw[4 * i], lw[4 * i + 1], lw[4 * i + 2], lw[4 * i + 3]);
        }
      };
      if constexpr (SPLIT == 1) {
        decode_pairs(std::integral_constant<int, 0>{});
      } else {
        if (fpart == 0) decode_pairs(std::integral_constant<int, 0>{});
        else decode_pairs(std::integral_constant<int, NP>{});
      }
    }
  };

  // ---- staging pass: decode tile qblk of KV head g once into LDS, then
  // copy it out as the tile's image (16 contiguous bytes per lane: each store
  // instruction writes 1 KiB in 16 lines, where the decode's own layout would
  // touch 64; the K rows' padding words are never read), for the attention
  // workgroups of every query block.  Thread (token, qblock) of waves 0-3
  // decodes a K record and inverse-rotates it, k = H (d . c s) / sqrt 32 per
  // 32-element block with d the decode signs (the transpose of the query's
  // rotation); waves 4-7 decode a V record, which stays rotated.  One K and
  // one V exponent per 16-token slice. ----
  if constexpr (PH == kStage) {
    // tiles [tile0, tile1) of KV head g; tile + 1's records are requested
    // before tile's decode
    const int tile0 = qblk * a.stage_tpw, tile1 = min(a.stage_tiles, tile0 + a.stage_tpw);
    if (tile0 >= tile1) return;
    fetch(tile0 * kTile);
    __syncthreads();  // codebook staged
    for (int tile = tile0; tile < tile1; tile++) {
      uint32_t nkw[QW];
      uint16_t nks = 0, nnm = 0;
      uint32_t nsg = 0;
      const bool more = tile + 1 < tile1;
      if (more) load_rec((tile + 1) * kTile, nkw, nks, nsg, nnm);
      const bool kwave = wave < 4;
      const int slice = wave & 3;
      const float sc = fabsf(f16_to_f32(ks));
      const int e = pow2_exponent(wave_max(sc));
      const float f = sc * exp2i(-e);
      if (lane == 0) {
        if (kwave) {
          xe(0)[slice] = e;
        } else {
          xe(0)[4 + 2 * slice] = e;
          xe(0)[5 + 2 * slice] = e;
        }
      }
      if constexpr (QJL) {
        if (kwave) {
          if (fqb == 0) cnp(0)[ftok] = f16_to_f32(nm) * a.qjl_c;
          sgp(0)[ftok * 4 + fqb] = sgw;
        }
      }
      constexpr uint32_t SM = (1u << BITS) - 1u, CMk = (1u << CB) - 1u;
      float y[32];
#pragma unroll
      for (int pp = 0; pp < 16; pp++) {
        const uint32_t code = pair_code<BITS>(kw, pp);
        y[2 * pp] = s_cb[code & SM & CMk];
        y[2 * pp + 1] = s_cb[(code >> BITS) & CMk];
      }
      uint32_t hw[16], lw[16];
      if (kwave) {
#pragma unroll
        for (int j = 0; j < 32; j++) y[j] = (y[j] * f) * decode_sign(j);
        butterfly<32>(y);
#pragma unroll
        for (int j = 0; j < 16; j++) {
          const float x0 = y[2 * j] * kInvSqrt32, x1 = y[2 * j + 1] * kInvSqrt32;
          hw[j] = pack_f16(x0, x1);
          lw[j] = pack_rem(x0, x1, hw[j], mone);
        }
        uint4 *krow = reinterpret_cast<uint4 *>(ktile(0) + ftok * kKStride);
#pragma unroll
        for (int gq = 0; gq < 4; gq++) {
          krow[kchunk(8 * fqb + 2 * gq, ftok)] = make_uint4(hw[4 * gq], hw[4 * gq + 1], hw[4 * gq + 2], hw[4 * gq + 3]);
          krow[kchunk(8 * fqb + 2 * gq + 1, ftok)] = make_uint4(lw[4 * gq], lw[4 * gq + 1], lw[4 * gq + 2], lw[4 * gq + 3]);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 16; j++) {
          const float x0 = y[2 * j] * f, x1 = y[2 * j + 1] * f;
          hw[j] = pack_f16(x0, x1);
          lw[j] = pack_rem(x0, x1, hw[j], mone);
        }
        _Float16 *vrh = vhi(0) + ftok * kVRow, *vrl = vrh + V_HALVES;
#pragma unroll
        for (int gq = 0; gq < 4; gq++) {
          const int c = 8 * vchunk(4 * fqb + gq);
          *reinterpret_cast<uint4 *>(vrh + c) = make_uint4(hw[4 * gq], hw[4 * gq + 1], hw[4 * gq + 2], hw[4 * gq + 3]);
          *reinterpret_cast<uint4 *>(vrl + c) = make_uint4(lw[4 * gq], lw[4 * gq + 1], lw[4 * gq + 2], lw[4 * gq + 3]);
        }
      }
      __syncthreads();
      u32x4 *dst = reinterpret_cast<u32x4 *>(a.stage_out + ((long long)g * a.stage_tiles + tile) * IMG);
#pragma unroll
      for (int r = 0; r < IMG_ROUNDS; r++) {
        const int c = tid + 4 * kRows * r;
        if (r + 1 < IMG_ROUNDS || c < IMG) dst[c] = *reinterpret_cast<const u32x4 *>(img_chunk(0, c));
      }
      if (more) {
        __syncthreads();  // the copy's reads of the buffer are done
#pragma unroll
        for (int i = 0; i < QW; i++) kw[i] = nkw[i];
        ks = nks;
        sgw = nsg;
        nm = nnm;
      }
    }
    return;
  }

  // the workgroup's tiles; the first tile's records (staged: image) are
  // requested before the query, so the two latencies overlap
  const int last_q = min(a.q_len - 1, i0 + QB - 1);
  const int kv_end = a.causal ? min(a.kv_len, a.kv_len - a.q_len + last_q + 1) : a.kv_len;
  const int ntiles = (kv_end + kTile - 1) / kTile;
  // this workgroup's split of the tiles
  const int tile_lo = min(ntiles, (int)blockIdx.z * a.tps), tile_hi = min(ntiles, tile_lo + a.tps);
  if (a.splits > 1 && tile_hi <= tile_lo) {
    // an empty split (a causal query block that ends before it): its partial
    // rows say so, m = -inf (the merge then reads nothing else of them)
    const int prow = tid >> 2, pq = tid & 3;
    const int qi = i0 + prow / NR, qh = g * NR + prow % NR;
    if (qi < a.q_len && pq == 0) {
      float *pr = a.part + (((long long)blockIdx.z * a.num_heads + qh) * a.q_len + qi) * kPartRow;
      pr[128] = -INFINITY;
      pr[129] = 0.f;
    }
    return;
  }
  if (tile_hi > tile_lo) fetch(tile_lo * kTile);

  // ---- query rows: thread (row, quarter) rotates one 32-element block ----
  // (the V tile region holds the split query until the operands are built)
  const int prow = tid >> 2, pq = tid & 3;
  const int qi = i0 + prow / NR, qh = g * NR + prow % NR;
  const bool row_ok = qi < a.q_len;
  _Float16 *s_qh = reinterpret_cast<_Float16 *>(s_tile);  // [row][kQRow] hi
  _Float16 *s_ql = s_qh + kRows * kQRow;              // [row][kQRow] lo
  {
    float x[32];
    const long long base = ((long long)qh * a.q_len + (row_ok ? qi : 0)) * HD + 32 * pq;
    // one dtype branch around all 32 loads (a branch per element keeps each
    // load behind its own test and wait)
    if (a.q_dtype == kF32) {
      const float *src = static_cast<const float *>(a.q) + base;
#pragma unroll
      for (int j = 0; j < 32; j++) x[j] = src[j];
    } else {
      const uint16_t *src = static_cast<const uint16_t *>(a.q) + base;
      uint16_t hb[32];
#pragma unroll
      for (int j = 0; j < 32; j++) hb[j] = src[j];
      if (a.q_dtype == kBF16) {
#pragma unroll
        for (int j = 0; j < 32; j++) x[j] = bf16_to_f32(hb[j]);
      } else {
#pragma unroll
        for (int j = 0; j < 32; j++) x[j] = f16_to_f32(hb[j]);
      }
    }
    // (staged tiles: the query as it is; the softmax scale joins the row's
    // exponent factor)
    if constexpr (!ORIG) butterfly<32>(x);
    float m = 0.f;
#pragma unroll
    for (int j = 0; j < 32; j++) {
      if constexpr (!ORIG) x[j] = x[j] * (decode_sign(j) * (kInvSqrt32 * lscale));
      m = fmaxf(m, fabsf(x[j]));
    }
    m = fmaxf(m, dpp_quad_xor1(m));
    m = fmaxf(m, dpp_quad_xor2(m));
    const int eq = pow2_exponent(m);
    const float sc = exp2i(-eq);
    if (pq == 0) s_eq[prow] = eq;
#pragma unroll
    for (int j = 0; j < 32; j++) x[j] = row_ok ? x[j] * sc : 0.f;
    stage_split32(x, s_qh + prow * kQRow + 32 * pq, s_ql + prow * kQRow + 32 * pq);
  }
  // TQ: rq rows the same way (no rotation), into the K tile region
  _Float16 *s_rh = reinterpret_cast<_Float16 *>(s_tile + kRows * kQRow);
  _Float16 *s_rl = s_rh + kRows * kQRow;
  if constexpr (QJL) {
    float x[32];
    const long long base = ((long long)qh * a.q_len + (row_ok ? qi : 0)) * HD + 32 * pq;
    float m = 0.f;
#pragma unroll
    for (int j = 0; j < 32; j++) {
      x[j] = a.rq[base + j] * lscale;
      m = fmaxf(m, fabsf(x[j]));
    }
    m = fmaxf(m, dpp_quad_xor1(m));
    m = fmaxf(m, dpp_quad_xor2(m));
    const int er = pow2_exponent(m);
    const float sc = exp2i(-er);
    if (pq == 0) s_er[prow] = er;
#pragma unroll
    for (int j = 0; j < 32; j++) x[j] = row_ok ? x[j] * sc : 0.f;
    stage_split32(x, s_rh + prow * kQRow + 32 * pq, s_rl + prow * kQRow + 32 * pq);
  }
  __syncthreads();

  // ---- per-wave operands for its 16 rows (lane column = row 16 wave + l16) ----
  const int myrow = 16 * wave + l16;
  // per 32-element slice s, lane (row, lg) holds elements 32 s + 8 lg .. + 7
  // of its row, hi and lo
  u32x4 qop[4][2];
#pragma unroll
  for (int s = 0; s < 4; s++) {
    const int e = myrow * kQRow + 32 * s + 8 * lg;
    const uint4 h = *reinterpret_cast<const uint4 *>(s_qh + e);
    const uint4 l = *reinterpret_cast<const uint4 *>(s_ql + e);
    qop[s][0] = u32x4{h.x, h.y, h.z, h.w};
    qop[s][1] = u32x4{l.x, l.y, l.z, l.w};
  }
  u32x4 rop[4][2];
  if constexpr (QJL) {
#pragma unroll
    for (int sl = 0; sl < 4; sl++) {
      const int e = myrow * kQRow + 32 * sl + 8 * lg;
      const uint4 h = *reinterpret_cast<const uint4 *>(s_rh + e);
      const uint4 l = *reinterpret_cast<const uint4 *>(s_rl + e);
      rop[sl][0] = u32x4{h.x, h.y, h.z, h.w};
      rop[sl][1] = u32x4{l.x, l.y, l.z, l.w};
    }
  }
  const int my_qi = i0 + myrow / NR;
  const bool my_ok = my_qi < a.q_len;
  const bool wave_rows_ok = __all(my_ok);  // every row of the wave is a query
  const float eq_scale = exp2i(s_eq[myrow]);
  // the row's factor on the key products: 2^E_q (staged: times the softmax
  // scale, which the unrotated query does not carry)
  const float eqz = ORIG ? eq_scale * lscale : eq_scale;
  // the product with the query's lo part: every query in the workgroup's
  // decode, f32 queries on staged tiles (a bf16 or f16 query scaled by 2^-E_q
  // is exact in f16 down to 2^-24 of the row's maximum)
  const bool q_lo = !ORIG || a.q_dtype == kF32;
  const float er_scale = QJL ? exp2i(s_er[myrow]) : 0.f;
  const int qpos = a.kv_len - a.q_len + my_qi;  // causal limit of this row
  const int qmin = a.kv_len - a.q_len + i0;     // the workgroup's first query position
  __syncthreads();  // operands built: the tiles may overwrite the query staging

  // ---- tiles ----


  float m_run = -INFINITY, l_run = 0.f;
  int ev_cur = -1000;
  f32x4 o[8];
#pragma unroll
  for (int eb = 0; eb < 8; eb++) o[eb] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (tile_hi > tile_lo) {
    decode_tile(0);
    if (tile_hi > tile_lo + 1) fetch((tile_lo + 1) * kTile);  // each tile's records arrive during the tile before
  }
  __syncthreads();
  // One barrier per tile: tile + 1 is decoded into the other buffer in the
  // same stretch as tile's products (the waves sharing a SIMD in opposite
  // orders, so that one's decode overlaps the other's matrix products); the
  // barrier then publishes tile + 1 and frees tile's buffer for tile + 2.
  const bool decode_first = (wave >> 2) & 1;
  for (int tile = tile_lo; tile < tile_hi; tile++) {
    const int t0 = tile * kTile, cur = (tile - tile_lo) & 1;
    const bool more = tile + 1 < tile_hi;
    if (decode_first && more) {
      decode_tile(cur ^ 1);
      if (tile + 2 < tile_hi) fetch(t0 + 2 * kTile);
    }
    const uint2 *kt = ktile(cur);
    const _Float16 *vth = vhi(cur), *vtl = vth + V_HALVES;

    // ---- S^T = K Q^T (+ corr), four 16-token blocks ----
    // a tile wholly before the workgroup's first query position (and inside
    // the sequence) is visible to every row: no per-element mask
    const bool open = t0 + kTile <= a.kv_len && (!a.causal || t0 + kTile - 1 <= qmin);
    float x[4][4];
    // the tile's slice exponents (wave-uniform)
    int ekt[4];
    {
      const int4 e4 = *reinterpret_cast<const int4 *>(s_xe[cur]);
      ekt[0] = __builtin_amdgcn_readfirstlane(e4.x);
      ekt[1] = __builtin_amdgcn_readfirstlane(e4.y);
      ekt[2] = __builtin_amdgcn_readfirstlane(e4.z);
      ekt[3] = __builtin_amdgcn_readfirstlane(e4.w);
    }
    f32x4 dk[4];
#pragma unroll
    for (int tb = 0; tb < 4; tb++) dk[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; s++) {
      u32x4 ah[4], al[4];
#pragma unroll
      for (int tb = 0; tb < 4; tb++) {
        const uint4 *krow = reinterpret_cast<const uint4 *>(kt + (16 * tb + l16) * kKStride);
        const uint4 kh = krow[kchunk(8 * s + 2 * lg, l16)], kl = krow[kchunk(8 * s + 2 * lg + 1, l16)];
        ah[tb] = u32x4{kh.x, kh.y, kh.z, kh.w};
        al[tb] = u32x4{kl.x, kl.y, kl.z, kl.w};
      }
#pragma unroll
      for (int tb = 0; tb < 4; tb++) dk[tb] = mfma(ah[tb], qop[s][0], dk[tb]);
      if (q_lo) {
#pragma unroll
        for (int tb = 0; tb < 4; tb++) dk[tb] = mfma(ah[tb], qop[s][1], dk[tb]);
      }
#pragma unroll
      for (int tb = 0; tb < 4; tb++) dk[tb] = mfma(al[tb], qop[s][0], dk[tb]);
    }
#pragma unroll
    for (int tb = 0; tb < 4; tb++) {
      const f32x4 d = dk[tb];
      f32x4 dc = f32x4{0.f, 0.f, 0.f, 0.f};
      if constexpr (QJL) {
        const uint32_t *sgrow = s_sg[cur] + (16 * tb + l16) * 4;
#pragma unroll
        for (int sl = 0; sl < 4; sl++) {
          const uint32_t byte = (sgrow[sl] >> (8 * lg)) & 0xffu;
          const uint2 n0 = s_nib[byte & 15u], n1 = s_nib[byte >> 4];
          const u32x4 sa = {n0.x, n0.y, n1.x, n1.y};
          dc = mfma(sa, rop[sl][0], dc);
          dc = mfma(sa, rop[sl][1], dc);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; i++) {
        // without QJL the slice's 2^E_k and the row's 2^E_q are applied in the softmax
        float v = QJL ? d[i] * (exp2i(ekt[tb]) * eqz) : d[i];
        if constexpr (QJL) v = __builtin_fmaf(dc[i], s_cn[cur][16 * tb + 4 * lg + i] * er_scale, v);
        x[tb][i] = v;
      }
      // the mask, in place, for tiles that are not open to every row
      if (!(open && wave_rows_ok)) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int tp = t0 + 16 * tb + 4 * lg + i;
          const bool ok = my_ok && (open || (tp < a.kv_len && (!a.causal || tp <= qpos)));
          x[tb][i] = ok ? x[tb][i] : -INFINITY;
        }
      }
    }
    // ---- online softmax of this row (its 64 logits sit in the 4 lanes l16 + 16 k) ----
    // logit = x z_tb, z_tb = 2^E_k,tb 2^E_q (a power of 2, exact; staged
    // tiles: times the softmax scale) (QJL: 1)
    float zt[4];
#pragma unroll
    for (int tb = 0; tb < 4; tb++) zt[tb] = QJL ? 1.f : exp2i(ekt[tb]) * eqz;
    float mt = -INFINITY;
#pragma unroll
    for (int tb = 0; tb < 4; tb++)
      mt = fmaxf(mt, fmaxf(fmaxf(x[tb][0], x[tb][1]), fmaxf(x[tb][2], x[tb][3])) * zt[tb]);
    mt = max_xor32(max_xor16(mt));
    const float m_new = fmaxf(m_run, mt);
    const float m_exp = m_new == -INFINITY ? 0.f : m_new;  // a row with nothing visible yet
    const float alpha = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
    // V exponent of the tile (each wave reads all 64)
    static_assert(NW % 4 == 0, "the wave exponents are read 4 at a time");
    int evw[NW];
#pragma unroll
    for (int w = 0; w < NW; w += 4) {
      const int4 e4 = *reinterpret_cast<const int4 *>(s_xe[cur] + 4 + w);
      evw[w] = __builtin_amdgcn_readfirstlane(e4.x);
      evw[w + 1] = __builtin_amdgcn_readfirstlane(e4.y);
      evw[w + 2] = __builtin_amdgcn_readfirstlane(e4.z);
      evw[w + 3] = __builtin_amdgcn_readfirstlane(e4.w);
    }
    int evt = -1000;
#pragma unroll
    for (int w = 0; w < NW; w++) evt = max(evt, evw[w]);
    const int ev_new = max(ev_cur, evt);
    const float rescale = alpha * exp2i(max(ev_cur - ev_new, -126));
    ev_cur = ev_new;
    m_run = m_new;
    float ls = 0.f;
    u32x2 pb[4][2];
#pragma unroll
    for (int tb = 0; tb < 4; tb++) {
      // p = e 2^(E_v,tb - Ev) with e = 2^(logit - m): the slice's V factor is
      // a shift of exp2's argument (E_v,tb - Ev in [-40, 0]: p stays normal
      // for every e above 2^-80), and e = p 2^(Ev - E_v,tb) for the row sum
      const int dv = evw[SPLIT * tb] - ev_new;
      const float cb = (float)dv - m_exp, gb = exp2i(-dv);
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(x[tb][i], zt[tb], cb));  // 2^-inf = 0 for masked tokens
        ls = __builtin_fmaf(p[i], gb, ls);
      }
      pb[tb][0] = u32x2{pack_f16(p[0], p[1]), pack_f16(p[2], p[3])};
      pb[tb][1] = u32x2{pack_rem(p[0], p[1], pb[tb][0][0], mone), pack_rem(p[2], p[3], pb[tb][0][1], mone)};
    }
    l_run = l_run * alpha + ls;
    // ---- O^T += V^T P^T, two 16-token blocks per 16x16x32 product.  The
    // value operand comes through the transposing LDS read: lane (4 a + b)
    // of group lg receives element 16 eb + 4 a + b of tokens 16 tb + 4 lg ..
    // + 3 from the token-major rows addressed by lanes a + 4 j. ----
    const int vrow = 4 * lg + (l16 >> 2), vcol = 4 * (l16 & 3);
    // the accumulators' rescale, skipped when every row's factor is 1
    if (!__all(rescale == 1.f)) {
#pragma unroll
      for (int eb = 0; eb < 8; eb++) o[eb] = o[eb] * rescale;
    }
    // the value pass at raised issue priority: the SIMD's other wave, often
    // in its softmax, fills the matrix products' gaps instead of delaying
    // them (0.2401 -> 0.2365 ms at the bench shape; the key pass gains nothing)
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int e2 = 0; e2 < 8; e2 += 2) {
#pragma unroll
      for (int tp = 0; tp < 2; tp++) {
        const u32x4 bh = {pb[2 * tp][0][0], pb[2 * tp][0][1], pb[2 * tp + 1][0][0], pb[2 * tp + 1][0][1]};
        const u32x4 bl = {pb[2 * tp][1][0], pb[2 * tp][1][1], pb[2 * tp + 1][1][0], pb[2 * tp + 1][1][1]};
        u32x4 ah[2], al[2];
#pragma unroll
        for (int j = 0; j < 2; j++) {
          const int eb = e2 + j;
          const int r0 = (32 * tp + vrow) * kVRow + 8 * vchunk(2 * eb + (vcol >> 3)) + (vcol & 7),
                    r1 = r0 + 16 * kVRow;
          const u32x2 h0 = lds_read_tr16(vth + r0), h1 = lds_read_tr16(vth + r1);
          const u32x2 q0 = lds_read_tr16(vtl + r0), q1 = lds_read_tr16(vtl + r1);
          ah[j] = u32x4{h0[0], h0[1], h1[0], h1[1]};
          al[j] = u32x4{q0[0], q0[1], q1[0], q1[1]};
        }
        o[e2] = mfma(ah[0], bh, o[e2]);
        o[e2 + 1] = mfma(ah[1], bh, o[e2 + 1]);
        o[e2] = mfma(ah[0], bl, o[e2]);
        o[e2 + 1] = mfma(ah[1], bl, o[e2 + 1]);
        o[e2] = mfma(al[0], bh, o[e2]);
        o[e2 + 1] = mfma(al[1], bh, o[e2 + 1]);
      }
    }
    __builtin_amdgcn_s_setprio(0);
    if (!decode_first && more) {
      decode_tile(cur ^ 1);
      if (tile + 2 < tile_hi) fetch(t0 + 2 * kTile);
    }
    __syncthreads();
  }

  // ---- finish: row sums, inverse rotation per 32-element block, store ----
  float L = l_run;
  L += __shfl_xor(L, 16, 64);
  L += __shfl_xor(L, 32, 64);
  float *s_o = reinterpret_cast<float *>(s_tile);  // [row][kORow] (rotated, in units of 2^ev_cur)
  const float ofac = exp2i(max(min(ev_cur, 126), -126));
#pragma unroll
  for (int eb = 0; eb < 8; eb++)
    *reinterpret_cast<float4 *>(s_o + myrow * kORow + 16 * eb + 4 * lg) =
        make_float4(o[eb][0] * ofac, o[eb][1] * ofac, o[eb][2] * ofac, o[eb][3] * ofac);
  float *s_rowl = s_o + kRows * kORow;  // [rows] (the tiles are done)
  float *s_rowm = s_rowl + kRows;
  if (lg == 0) {
    s_rowl[myrow] = L;
    s_rowm[myrow] = m_run;
  }
  __syncthreads();
  {
    float v[32];
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const float4 f = *reinterpret_cast<const float4 *>(s_o + prow * kORow + 32 * pq + 4 * k);
      v[4 * k] = f.x * decode_sign(4 * k);
      v[4 * k + 1] = f.y * decode_sign(4 * k + 1);
      v[4 * k + 2] = f.z * decode_sign(4 * k + 2);
      v[4 * k + 3] = f.w * decode_sign(4 * k + 3);
    }
    butterfly<32>(v);
    const float Lr = s_rowl[prow];
    if (row_ok && a.splits > 1) {
      // a split's partial row: the sums unnormalized, its maximum and sum
      float *pr = a.part + (((long long)blockIdx.z * a.num_heads + qh) * a.q_len + qi) * kPartRow;
#pragma unroll
      for (int k = 0; k < 8; k++)
        *reinterpret_cast<float4 *>(pr + 32 * pq + 4 * k) =
            make_float4(v[4 * k] * kInvSqrt32, v[4 * k + 1] * kInvSqrt32, v[4 * k + 2] * kInvSqrt32,
                        v[4 * k + 3] * kInvSqrt32);
      if (pq == 0) {
        pr[128] = s_rowm[prow];
        pr[129] = Lr;
      }
    } else if (row_ok) {
      const long long ob = ((long long)qh * a.q_len + qi) * HD + 32 * pq;
#pragma unroll
      for (int j = 0; j < 32; j++) v[j] = Lr > 0.f ? v[j] * kInvSqrt32 / Lr : 0.f;
      if (a.out_dtype == kF32) {
#pragma unroll
        for (int j = 0; j < 32; j++) static_cast<float *>(a.out)[ob + j] = v[j];
      } else if (a.out_dtype == kBF16) {
#pragma unroll
        for (int j = 0; j < 32; j++) static_cast<uint16_t *>(a.out)[ob + j] = f32_to_bf16(v[j]);
      } else {
#pragma unroll
        for (int j = 0; j < 32; j++) static_cast<uint16_t *>(a.out)[ob + j] = f32_to_f16(v[j]);
      }
    }
  }
}

// Split-K merge: out[row] = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) L_s
// over the splits' partial rows (M their maximum; 0 where no split saw a
// token), one workgroup of 128 lanes per (head, query) row.  The splits go
// in groups of 8 whose loads are all issued before the group is folded
// (one memory round trip per group), with a running maximum across groups.
__global__ __launch_bounds__(128) void prefill_merge_kernel(const float *part, int splits, long long rows, void *out,
                                                            int out_dtype) {
  constexpr int G = 8;
  const long long row = blockIdx.x;
  const int e = threadIdx.x;
  const float *p = part + row * kPartRow;
  const long long step = rows * kPartRow;
  float M = -INFINITY, O = 0.f, L = 0.f;
  for (int s0 = 0; s0 < splits; s0 += G) {
    float ms[G], ls[G], os[G];
#pragma unroll
    for (int k = 0; k < G; k++) {
      const bool ok = s0 + k < splits;
      const float *ps = p + (ok ? s0 + k : 0) * step;
      ms[k] = ok ? ps[128] : -INFINITY;
      ls[k] = ok ? ps[129] : 0.f;
      os[k] = ok ? ps[e] : 0.f;
    }
    float Mg = M;
#pragma unroll
    for (int k = 0; k < G; k++) Mg = fmaxf(Mg, ms[k]);
    if (Mg == -INFINITY) continue;  // nothing seen yet
    const float f = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M - Mg);
    O *= f;
    L *= f;
#pragma unroll
    for (int k = 0; k < G; k++) {
      // (a split that saw no token: m = -inf, weight 0, its sums ignored)
      const float w = ms[k] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ms[k] - Mg);
      O = __builtin_fmaf(ms[k] == -INFINITY ? 0.f : os[k], w, O);
      L = __builtin_fmaf(ms[k] == -INFINITY ? 0.f : ls[k], w, L);
    }
    M = Mg;
  }
  const float r = L > 0.f ? O / L : 0.f;
  const long long oi = row * 128 + e;
  if (out_dtype == kF32) static_cast<float *>(out)[oi] = r;
  else if (out_dtype == kBF16) static_cast<uint16_t *>(out)[oi] = f32_to_bf16(r);
  else static_cast<uint16_t *>(out)[oi] = f32_to_f16(r);
}

// Whether to decode each tile once into a staging buffer: the workgroups of
// q_blocks query blocks per KV head would otherwise decode a tile up to
// q_blocks times (causal: about half of that on average).  TQ_PREFILL_STAGING = 0 / 1 forces either path, except that a KV head's
// images must stay below 2^31 bytes (about 1.9 million tokens).
bool use_staging(int q_blocks, int kv_len, int mode) {
  // a KV head's images are read through one buffer resource: below 2^31 bytes
  const long long head_bytes = (long long)((kv_len + kTile - 1) / kTile) * img_chunks(mode) * 16;
  if (head_bytes >= (1ll << 31)) return false;
  if (const char *e = getenv("TQ_PREFILL_STAGING")) {
    if (e[0] == '0') return false;
    if (e[0] == '1') return true;
  }
  return q_blocks >= kStagingMinQueryBlocks && kv_len >= kStagingMinTokens;
}

// The staging buffers come from a memory pool of the library's own per
// device, which keeps up to kStagingPoolKeep bytes across synchronizations
// (the device's default pool, release threshold 0, would hand its memory
// back to the driver at each synchronization, and the next prefill would
// allocate it again).  nullptr: the pool could not be made; the caller then
// takes the device's default pool.
constexpr uint64_t kStagingPoolKeep = 1ull << 30;
hipMemPool_t staging_pool(int dev) {
  static std::mutex mu;
  static hipMemPool_t pools[64] = {};
  static bool tried[64] = {};
  if (dev < 0 || dev >= 64) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  if (!tried[dev]) {
    tried[dev] = true;
    hipMemPoolProps props{};
    props.allocType = hipMemAllocationTypePinned;
    props.location.type = hipMemLocationTypeDevice;
    props.location.id = dev;
    hipMemPool_t pool = nullptr;
    if (hipMemPoolCreate(&pool, &props) == hipSuccess) {
      uint64_t keep = kStagingPoolKeep;
      (void)hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep);
      pools[dev] = pool;
    } else {
      (void)hipGetLastError();
    }
  }
  return pools[dev];
}

// Compute units of device dev (cached; 0 if unknown)
int cu_count(int dev) {
  static std::mutex mu;
  static int n[64] = {};
  if (dev < 0 || dev >= 64) return 0;
  std::lock_guard<std::mutex> lock(mu);
  if (n[dev] == 0) {
    int c = 0;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
      (void)hipGetLastError();
      c = -1;
    }
    n[dev] = c;
  }
  return n[dev] > 0 ? n[dev] : 0;
}

// Splits of the attention's tiles: the attention runs one workgroup per
// compute unit (its LDS), so a grid of fewer workgroups than compute units (few query blocks per KV head: chunked prefill, multi-token decode)
// has each workgroup take 1 / splits of its query block's tiles, with
// floor(CUs / workgroups) splits (one round) of at least 2 tiles each;
// TQ_PREFILL_SPLITS = n forces n.
int prefill_splits(int wgs, int ntiles, int dev) {
  int s = 1;
  if (const char *e = getenv("TQ_PREFILL_SPLITS")) {
    s = atoi(e);
  } else {
    const int cus = cu_count(dev);
    if (cus > 0 && wgs > 0 && ntiles >= 4) s = min(cus / wgs, ntiles / 2);
  }
  return max(1, min(s, ntiles));
}

template <int BITS, int MODE, int PH>
void launch_attn(const PrefillArgs &a, int nr, dim3 grid, dim3 block, hipStream_t st) {
  grid.z = (unsigned)a.splits;
  if (nr == 1) hipLaunchKernelGGL((prefill_attn_kernel<BITS, MODE, 1, PH>), grid, block, 0, st, a);
  else if (nr == 2) hipLaunchKernelGGL((prefill_attn_kernel<BITS, MODE, 2, PH>), grid, block, 0, st, a);
  else hipLaunchKernelGGL((prefill_attn_kernel<BITS, MODE, 4, PH>), grid, block, 0, st, a);
}

template <int BITS, int MODE>
int launch_prefill_m(PrefillArgs &a, int nr, hipStream_t st) {
  const int qb = prefill_rows(MODE) / nr;
  const dim3 block((unsigned)(4 * prefill_rows(MODE)));
  const dim3 grid((unsigned)((a.q_len + qb - 1) / qb), (unsigned)a.num_kv_heads);
  const int ntiles = (a.kv_len + kTile - 1) / kTile;
  int dev = 0;
  (void)hipGetDevice(&dev);
  const bool staged = a.kv_len > 0 && use_staging((int)grid.x, a.kv_len, MODE);
  // the attention split over the tiles when its grid would leave compute
  // units idle
  const int splits = a.kv_len > 0 ? prefill_splits((int)(grid.x * grid.y), ntiles, dev) : 1;
  a.tps = max((ntiles + splits - 1) / splits, 1);
  a.splits = max((ntiles + a.tps - 1) / a.tps, 1);
  a.part = nullptr;
  a.stage_tiles = ntiles;
  // one stream-ordered buffer: the tile images (staged), then the splits'
  // partial rows; released in stream order after the launches
  const size_t img_bytes =
      staged ? (size_t)a.num_kv_heads * (size_t)a.stage_tiles * img_chunks(MODE) * sizeof(uint4) : 0;
  const size_t part_at = (img_bytes + 255) & ~(size_t)255;
  const size_t bytes = part_at + (a.splits > 1 ? (size_t)a.splits * a.num_heads * a.q_len * kPartRow * sizeof(float) : 0);
  void *buf = nullptr;
  if (bytes > 0) {
    hipMemPool_t pool = staging_pool(dev);
    const hipError_t ae = pool ? hipMallocFromPoolAsync(&buf, bytes, pool, st) : hipMallocAsync(&buf, bytes, st);
    if (ae != hipSuccess) {
      (void)hipGetLastError();
      return tqh::fail(TQ_ERR_DEVICE, "prefill staging buffer of %zu bytes not allocated", bytes);
    }
    if (a.splits > 1) a.part = reinterpret_cast<float *>(static_cast<char *>(buf) + part_at);
  }
  if (staged) {
    a.stage = static_cast<const uint4 *>(buf);
    a.stage_out = static_cast<uint4 *>(buf);
    // the staging pass in one round of workgroups (two per compute unit, its
    // LDS), each taking consecutive tiles of one KV head
    const int cus = cu_count(dev);
    const long long units = (long long)a.stage_tiles * grid.y;
    a.stage_tpw = cus > 0 ? (int)max(1ll, (units + 2ll * cus - 1) / (2ll * cus)) : 1;
    const unsigned stage_wgs = (unsigned)((a.stage_tiles + a.stage_tpw - 1) / a.stage_tpw) * grid.y;
    hipLaunchKernelGGL((prefill_attn_kernel<BITS, MODE, 1, kStage>), dim3(stage_wgs), block, 0, st, a);
    launch_attn<BITS, MODE, kStaged>(a, nr, grid, block, st);
  } else {
    launch_attn<BITS, MODE, kDecode>(a, nr, grid, block, st);
  }
  if (a.splits > 1) {
    const long long rows = (long long)a.num_heads * a.q_len;
    hipLaunchKernelGGL(prefill_merge_kernel, dim3((unsigned)rows), dim3(128), 0, st, a.part, a.splits, rows, a.out,
                       a.out_dtype);
  }
  const int rc = tqh::check_launch(staged ? "prefill_attn_kernel (staged)" : "prefill_attn_kernel");
  if (buf) (void)hipFreeAsync(buf, st);
  return rc;
}

}  // namespace

extern "C" int tq_cache_prefill_attention(const void *q, int q_dtype, const uint8_t *k_indices,
                                          const uint16_t *k_scales, const uint8_t *v_indices,
                                          const uint16_t *v_scales, const float *rq, const uint8_t *qjl_signs,
                                          const uint16_t *qjl_norms, int num_heads, int q_len, int num_kv_heads,
                                          int head_dim, int bits, size_t outlier_blocks, int norm_mode, int kv_len,
                                          long long kv_head_stride, int causal, float softmax_scale, void *out,
                                          int out_dtype, hipStream_t stream) {
  if (head_dim != 128)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "prefill attention supports head_dim 128, got %d", head_dim);
  if (num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads != 0)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "num_heads (%d) must be a multiple of num_kv_heads (%d)", num_heads,
                     num_kv_heads);
  const int nr = num_heads / num_kv_heads;
  if (nr != 1 && nr != 2 && nr != 4) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "GQA ratio %d not supported", nr);
  tqh::PolarCodec codec;
  int rc = tqh::polar_codec(bits, norm_mode, outlier_blocks, head_dim / 32, codec);
  if (rc) return rc;
  if (codec.mixed)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "prefill attention takes outlier_blocks 0 or all");
  const bool qjl = qjl_signs != nullptr;
  if (qjl && (codec.outlier || !rq || !qjl_norms))
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "QJL correction needs outlier_blocks 0, rq, signs and norms");
  if (!tqh::valid_dtype(q_dtype) || !tqh::valid_dtype(out_dtype))
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "unknown dtype");
  if (q_len < 0 || kv_len < 0 || kv_head_stride < kv_len) return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "bad shape");
  if (causal && q_len > kv_len)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "causal prefill needs q_len (%d) <= kv_len (%d)", q_len, kv_len);
  if (q_len == 0) return TQ_OK;
  if (!q || !out || (kv_len > 0 && (!k_indices || !k_scales || !v_indices || !v_scales)))
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "null pointer");
  PrefillArgs a{};
  a.q = q;
  a.q_dtype = q_dtype;
  a.k_idx = k_indices;
  a.k_sc = k_scales;
  a.v_idx = v_indices;
  a.v_sc = v_scales;
  a.rq = rq;
  a.signs = reinterpret_cast<const uint32_t *>(qjl_signs);
  a.norms = qjl_norms;
  a.num_heads = num_heads;
  a.num_kv_heads = num_kv_heads;
  a.q_len = q_len;
  a.kv_len = kv_len;
  a.kv_head_stride = kv_head_stride;
  a.causal = causal ? 1 : 0;
  a.softmax_scale = softmax_scale;
  a.qjl_c = tq_qjl_bias_scale(head_dim);
  a.out = out;
  a.out_dtype = out_dtype;
  if (norm_mode == TQ_NORM_L2NORM) {
    a.cb_args = 1;
    for (int i = 0; i < codec.cb.nc; i++) a.cb[i] = codec.cb.c[i];
  }
  const int mode = codec.outlier ? kPPqo : (qjl ? kPTq : kPPq);
  if (bits == 3) {
    if (mode == kPPqo) return launch_prefill_m<3, kPPqo>(a, nr, stream);
    if (mode == kPPq) return launch_prefill_m<3, kPPq>(a, nr, stream);
    return launch_prefill_m<3, kPTq>(a, nr, stream);
  }
  if (mode == kPPqo) return launch_prefill_m<4, kPPqo>(a, nr, stream);
  if (mode == kPPq) return launch_prefill_m<4, kPPq>(a, nr, stream);
  return launch_prefill_m<4, kPTq>(a, nr, stream);
}
