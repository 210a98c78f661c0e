// tq_attention.hip -- fused decode attention over the compressed cache:
// the launch configuration of the streaming decode kernel
// (tq_decode_kernel.h), the split-K workspace (layout, header, counters),
// and the C-ABI entry points (the batched cache decode, the reference ABI's
// tq_fused_attention, and the allocation-free variant over a per-device
// static scratch array).
//
// The kernel reads every compressed byte once for all the query heads of a
// KV head (GQA sharing), scores the keys against the rotated query without
// inverse-rotating them, and accumulates the values in the rotated domain;
// split-K partials of a long sequence go to the workspace, and the last
// workgroup of a (sequence, KV head) to arrive (device-scope counter) merges
// them, inverse-rotates and writes the output, then re-arms the counter, so
// one launch does the whole decode.
#include "tq_common.h"
#include "tq_device.h"
#include "tq_mfma.h"

#include <mutex>
#include <type_traits>

namespace {

using namespace tqd;
using namespace tqm;

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
  void *out;
  int out_dtype;
  // TQ: rq [b][h][head_dim] f32 = R q (precompute_query_projections); per
  // record, signs [16] u8 of R r and the f16 residual norm |r|; qjl_c =
  // f32(sqrt(pi/2)) / sqrt(head_dim)
  const uint32_t *qjl_signs;
  const uint16_t *qjl_norms;
  float qjl_c;
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

// 16-byte load with the coherence of an agent-scope atomic load (SC1): the
// partials were written by other workgroups, possibly on other dies.
__device__ __forceinline__ float4 ld_agent16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 16));
}

#include "tq_decode_kernel.h"

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

// ---- streaming decode: configuration and dispatch ----
// Heads per group: the MFMA layouts take 2, 4 or 8 heads per instruction
// (fewer heads leave rows zero); more than 8 query heads per KV head run in
// several groups (each reading the KV head's records once).
int stream_hg(int nr) { return nr <= 2 ? 2 : (nr <= 4 ? 4 : 8); }
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
// The workspace layout is fixed by the shape alone: its chunk is the
// smallest any bit width, mode or workgroup size uses (the 4-wave form), so
// every launch's chunks fit its partial rows.
template <int NQB, int HG>
constexpr int stream_chunk_c() {
  return dmin(dmin(dmin(StreamCfg4<3, kModePqo, NQB, HG>::CHUNK, StreamCfg4<4, kModePqo, NQB, HG>::CHUNK),
                   dmin(StreamCfg4<3, kModePq, NQB, HG>::CHUNK, StreamCfg4<4, kModePq, NQB, HG>::CHUNK)),
              dmin(StreamCfg4<3, kModeTq, NQB, HG>::CHUNK, StreamCfg4<4, kModeTq, NQB, HG>::CHUNK));
}
template <int NQB>
int stream_chunk_hg(int hg) {
  return hg == 2 ? stream_chunk_c<NQB, 2>() : (hg == 4 ? stream_chunk_c<NQB, 4>() : stream_chunk_c<NQB, 8>());
}
// The chunk of the configuration a launch takes
template <int BITS, int MODE, int NQB>
int cfg_chunk_hg(int hg) {
  return hg == 2 ? StreamCfg<BITS, MODE, NQB, 2>::CHUNK
                 : (hg == 4 ? StreamCfg<BITS, MODE, NQB, 4>::CHUNK : StreamCfg<BITS, MODE, NQB, 8>::CHUNK);
}
template <int BITS, int MODE>
int cfg_chunk_nqb(int nqb, int hg) {
  return nqb == 1 ? cfg_chunk_hg<BITS, MODE, 1>(hg)
                  : (nqb == 2 ? cfg_chunk_hg<BITS, MODE, 2>(hg)
                              : (nqb == 4 ? cfg_chunk_hg<BITS, MODE, 4>(hg) : cfg_chunk_hg<BITS, MODE, 8>(hg)));
}
int stream_cfg_chunk(int bits, int mode, int head_dim, int nr) {
  const int nqb = head_dim / 32, hg = stream_hg(nr);
  if (bits == 3)
    return mode == kModePqo ? cfg_chunk_nqb<3, kModePqo>(nqb, hg)
                            : (mode == kModePq ? cfg_chunk_nqb<3, kModePq>(nqb, hg) : cfg_chunk_nqb<3, kModeTq>(nqb, hg));
  return mode == kModePqo ? cfg_chunk_nqb<4, kModePqo>(nqb, hg)
                          : (mode == kModePq ? cfg_chunk_nqb<4, kModePq>(nqb, hg) : cfg_chunk_nqb<4, kModeTq>(nqb, hg));
}
int stream_chunk(int head_dim, int nr) {
  const int hg = stream_hg(nr), nqb = head_dim / 32;
  return nqb == 1 ? stream_chunk_hg<1>(hg)
                  : (nqb == 2 ? stream_chunk_hg<2>(hg) : (nqb == 4 ? stream_chunk_hg<4>(hg) : stream_chunk_hg<8>(hg)));
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
  const int chunk = stream_chunk(head_dim, num_heads / num_kv_heads);
  w.P = (max_len + chunk - 1) / chunk;
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
  a.cpr = 1;
  return a;
}

// Compute units of the current device (cached per device).
int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int n = 0;
    cus[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
  }
  return cus[dev];
}

// 4-bit codes on the compiled-in MaxNorm codebook (evenly spaced) take the
// grid key pass; a caller's codebook or the L2Norm tables, the pair table
template <class C, bool INLINE, bool MULTI>
void launch_stream_k(AttnArgs &a, dim3 grid, hipStream_t st, int len_hint) {
  if constexpr (C::BITS == 4 && C::MODE == kModePqo) {
    if (!a.cb_dev && !a.cb_args) {
      hipLaunchKernelGGL((stream_decode_kernel<C, INLINE, true, MULTI>), grid, dim3(C::THREADS), 0, st, a.k_idx,
                         a.v_idx, a.k_sc, a.v_sc, a.seq_stride, a.kv_head_stride, len_hint, a);
      return;
    }
  }
  hipLaunchKernelGGL((stream_decode_kernel<C, INLINE, false, MULTI>), grid, dim3(C::THREADS), 0, st, a.k_idx, a.v_idx,
                     a.k_sc, a.v_sc, a.seq_stride, a.kv_head_stride, len_hint, a);
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
    if (tasks > cus * (12 / C::WAVES))
      a.cpr = (int)min((long long)max(chunks, 1), (tasks + 2 * cus - 1) / (2 * cus));
  }
  grid.x = (unsigned)((chunks + a.cpr - 1) / a.cpr);
  if (grid.x == 0) grid.x = 1;  // an empty batch still zeroes its outputs
  const int len_hint = a.kv_lens ? -1 : max(a.single_len, 0);
  if constexpr (INLINE) {
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
  if constexpr (INLINE && C::WAVES != 4) {
    const long long wgs = (long long)((a.max_len + C::CHUNK - 1) / C::CHUNK) * grid.y * grid.z;
    if (wgs > device_cus()) return launch_stream_c<C4, INLINE>(a, grid, st);
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
// grid: (-, num_kv_heads, batch); the chunk count (grid.x), a.nr / a.ngroups
// and a.chunk are set here from the launched configuration
template <bool INLINE>
int launch_stream(AttnArgs &a, int bits, int mode, int head_dim, dim3 grid, hipStream_t st) {
  const int hg = stream_hg(a.nr);
  a.ngroups = (a.nr + hg - 1) / hg;
  grid.y *= (unsigned)a.ngroups;
  const int nqb = head_dim / 32;
  if (bits == 3) {
    if (mode == kModePqo) launch_stream_nqb<3, kModePqo, INLINE>(a, nqb, hg, grid, st);
    else if (mode == kModePq) launch_stream_nqb<3, kModePq, INLINE>(a, nqb, hg, grid, st);
    else launch_stream_nqb<3, kModeTq, INLINE>(a, nqb, hg, grid, st);
  } else {
    if (mode == kModePqo) launch_stream_nqb<4, kModePqo, INLINE>(a, nqb, hg, grid, st);
    else if (mode == kModePq) launch_stream_nqb<4, kModePq, INLINE>(a, nqb, hg, grid, st);
    else launch_stream_nqb<4, kModeTq, INLINE>(a, nqb, hg, grid, st);
  }
  return tqh::check_launch("stream_decode_kernel");
}
int launch_stream_merge(const AttnArgs &a, int head_dim, dim3 grid, hipStream_t st) {
  if (head_dim == 32) hipLaunchKernelGGL((stream_merge_kernel<32>), grid, dim3(256), 0, st, a);
  else if (head_dim == 64) hipLaunchKernelGGL((stream_merge_kernel<64>), grid, dim3(256), 0, st, a);
  else if (head_dim == 128) hipLaunchKernelGGL((stream_merge_kernel<128>), grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((stream_merge_kernel<256>), grid, dim3(256), 0, st, a);
  return tqh::check_launch("stream_merge_kernel");
}

// max_len: the longest sequence; the decode addresses one sequence's
// records of a KV head with 32-bit offsets below 2^31
int check_common(int num_heads, int num_kv_heads, int head_dim, int bits, long long max_len) {
  if (bits != 3 && bits != 4) return tqh::fail(TQ_ERR_UNSUPPORTED_BITS, "unsupported bits=%d, expected 3 or 4", bits);
  if (head_dim != 32 && head_dim != 64 && head_dim != 128 && head_dim != 256)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "fused decode attention supports head_dim 32, 64, 128 or 256, got %d",
                     head_dim);
  if (num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads != 0)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "num_heads (%d) must be a multiple of num_kv_heads (%d)", num_heads,
                     num_kv_heads);
  if (max_len * (head_dim * bits / 8) >= (1LL << 31))
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "%lld tokens of %d-byte records exceed 2 GiB per sequence and KV head",
                     max_len, head_dim * bits / 8);
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
  int rc = check_common(num_heads, num_kv_heads, head_dim, bits, max_kv_len);
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
  if (mode == kModeTq && head_dim == 32)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "the QJL-corrected decode takes head_dim 64, 128 or 256");
  a.nr = num_heads / num_kv_heads;
  const dim3 grid((unsigned)w.P, (unsigned)num_kv_heads, (unsigned)batch);
  return launch_stream<true>(a, bits, mode, head_dim, grid, stream);
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
  int rc = check_common(num_attention_heads, num_kv_heads, head_dim, bits, kv_len);
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
  if (qjl_enabled && head_dim == 32)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "the QJL-corrected decode takes head_dim 64, 128 or 256");
  a.nr = num_attention_heads / num_kv_heads;
  const int chunk = stream_cfg_chunk(bits, qjl_enabled ? kModeTq : kModePqo, head_dim, a.nr);
  const int P = (kv_len + chunk - 1) / chunk;
  if (P > num_partitions)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "num_partitions %d < the %d chunks of %d tokens", num_partitions, P,
                     chunk);
  if (num_partitions > (1 << 20))  // the merge addresses a round's partials with 32-bit offsets
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "num_partitions %d exceeds 2^20", num_partitions);
  rc = launch_stream<false>(a, bits, qjl_enabled ? kModeTq : kModePqo, head_dim,
                            dim3((unsigned)P, (unsigned)num_kv_heads, 1u), stream);
  if (rc) return rc;
  return launch_stream_merge(a, head_dim, dim3((unsigned)num_kv_heads, 1u), stream);
}
