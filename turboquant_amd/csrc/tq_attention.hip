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
#include "tq_attention.h"

#include <mutex>

namespace tqa {

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

}  // namespace tqa

namespace {

using namespace tqa;

// The reference ABI's second launch: the split-K merge alone.
template <int HD>
__global__ __launch_bounds__(256) void stream_merge_kernel(AttnArgs a) {
  const int g = blockIdx.x, b = blockIdx.y;
  const int len = a.kv_lens ? min(max(a.kv_lens[b], 0), a.max_len) : a.single_len;
  const int nchunks = (len + a.chunk - 1) / a.chunk;
  if (nchunks == 0) return;
  merge_heads<HD, 4>(a, b, g, (nchunks + a.cpr - 1) / a.cpr);
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

// grid: (-, num_kv_heads, batch); the chunk count (grid.x), a.nr / a.ngroups
// and a.chunk are set here from the launched configuration
template <bool INLINE>
int launch_stream(AttnArgs &a, int bits, int mode, int head_dim, dim3 grid, hipStream_t st) {
  const int hg = stream_hg(a.nr);
  a.ngroups = (a.nr + hg - 1) / hg;
  grid.y *= (unsigned)a.ngroups;
  const int nqb = head_dim / 32;
  if (bits == 3) {
    if (mode == kModePqo) launch_stream_bm<3, kModePqo, INLINE>(a, nqb, hg, grid, st);
    else if (mode == kModePq) launch_stream_bm<3, kModePq, INLINE>(a, nqb, hg, grid, st);
    else launch_stream_bm<3, kModeTq, INLINE>(a, nqb, hg, grid, st);
  } else {
    if (mode == kModePqo) launch_stream_bm<4, kModePqo, INLINE>(a, nqb, hg, grid, st);
    else if (mode == kModePq) launch_stream_bm<4, kModePq, INLINE>(a, nqb, hg, grid, st);
    else launch_stream_bm<4, kModeTq, INLINE>(a, nqb, hg, grid, st);
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
                        int out_dtype, const DecodeWs *wsd, size_t workspace_bytes, hipStream_t stream,
                        const uint32_t *rmat = nullptr);

}  // namespace

// host_len >= 0 (with kv_lens null): every sequence holds host_len tokens;
// max_kv_len fixes the workspace layout either way.
int tqh::decode_attention(const void *q, int q_dtype, const uint8_t *k_indices, const uint16_t *k_scales,
                          const uint8_t *v_indices, const uint16_t *v_scales, const float *rq,
                          const uint8_t *qjl_signs, const uint16_t *qjl_norms, const int *kv_lens, int host_len,
                          int batch, int num_heads, int num_kv_heads, int head_dim, int bits, size_t outlier_blocks,
                          int norm_mode, int max_kv_len, long long kv_head_stride, long long seq_stride,
                          float softmax_scale, void *out, int out_dtype, void *workspace, size_t workspace_bytes,
                          hipStream_t stream, const uint32_t *rmat) {
  const DecodeWs d = caller_ws(workspace, workspace_bytes);
  return decode_attention_ws(q, q_dtype, k_indices, k_scales, v_indices, v_scales, rq, qjl_signs, qjl_norms, kv_lens,
                             host_len, batch, num_heads, num_kv_heads, head_dim, bits, outlier_blocks, norm_mode,
                             max_kv_len, kv_head_stride, seq_stride, softmax_scale, out, out_dtype,
                             workspace ? &d : nullptr, workspace_bytes, stream, rmat);
}

namespace {

int decode_attention_ws(const void *q, int q_dtype, const uint8_t *k_indices, const uint16_t *k_scales,
                        const uint8_t *v_indices, const uint16_t *v_scales, const float *rq, const uint8_t *qjl_signs,
                        const uint16_t *qjl_norms, const int *kv_lens, int host_len, int batch, int num_heads,
                        int num_kv_heads, int head_dim, int bits, size_t outlier_blocks, int norm_mode,
                        int max_kv_len, long long kv_head_stride, long long seq_stride, float softmax_scale, void *out,
                        int out_dtype, const DecodeWs *wsd, size_t workspace_bytes, hipStream_t stream,
                        const uint32_t *rmat) {
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
  if (qjl && ((!rq && !rmat) || !qjl_norms))
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "QJL needs rq (or the sign matrix), signs and norms");
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
  a.rmat = rq ? nullptr : rmat;
  a.qjl_inv = tqh::inv_sqrt_dim(head_dim);
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

extern "C" int tq_tq_decode_attention(const void *q, int q_dtype, const uint8_t *k_indices, const uint16_t *k_scales,
                                      const uint8_t *v_indices, const uint16_t *v_scales, const uint8_t *qjl_signs,
                                      const uint16_t *qjl_norms, const uint32_t *qjl_sign_matrix, const int *kv_lens,
                                      int batch, int num_heads, int num_kv_heads, int head_dim, int bits,
                                      int norm_mode, int max_kv_len, long long kv_head_stride, long long seq_stride,
                                      float softmax_scale, void *out, int out_dtype, void *workspace,
                                      size_t workspace_bytes, hipStream_t stream) {
  if (!qjl_signs || !qjl_sign_matrix)
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "TQ decode needs the QJL signs and the sign matrix");
  return tqh::decode_attention(q, q_dtype, k_indices, k_scales, v_indices, v_scales, nullptr, qjl_signs, qjl_norms,
                               kv_lens, max_kv_len, batch, num_heads, num_kv_heads, head_dim, bits, 0, norm_mode,
                               max_kv_len, kv_head_stride, seq_stride, softmax_scale, out, out_dtype, workspace,
                               workspace_bytes, stream, qjl_sign_matrix);
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
  // caller's partial buffers are sized for 512-token partitions
  // (cuda/attention.rs:70-77): every partial of this entry covers at least
  // 512 tokens (1024-token chunks, 512-token chunks, or ranges of two
  // 256-token chunks where a shape's operands only fit 4-wave workgroups of
  // 64 tokens per wave), so ceil(kv_len / 512) partitions always suffice.
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
  const int span = chunk < kRefPartition ? kRefPartition : chunk;  // tokens per partial
  const int P = (kv_len + span - 1) / span;
  if (P > num_partitions)  // unreachable after the ceil(kv_len / 512) check: kept as the launch's own bound
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "num_partitions %d < the %d partials of %d tokens", num_partitions, P,
                     span);
  if (num_partitions > (1 << 20))  // the merge addresses a round's partials with 32-bit offsets
    return tqh::fail(TQ_ERR_INVALID_ARGUMENT, "num_partitions %d exceeds 2^20", num_partitions);
  rc = launch_stream<false>(a, bits, qjl_enabled ? kModeTq : kModePqo, head_dim,
                            dim3((unsigned)P, (unsigned)num_kv_heads, 1u), stream);
  if (rc) return rc;
  return launch_stream_merge(a, head_dim, dim3((unsigned)num_kv_heads, 1u), stream);
}
