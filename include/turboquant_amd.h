/*
 * turboquant_amd.h -- C ABI of the MI355X (gfx950) TurboQuant KV-cache path.
 *
 * All pointers are device pointers unless stated otherwise; the caller owns
 * every buffer (outputs and scratch alike), as in the reference's FFI
 * (src/cache/cuda/ffi.rs:10-79), where candle tensors own all memory.  f16
 * values cross as raw uint16_t bits.  Every entry point is stream-ordered on
 * the given hipStream_t (0 = the null stream) and does not synchronise the
 * host.  Entry points return a status (0 = success); tq_last_error() gives
 * the message of the calling thread's last failure.
 *
 * Layouts (bits = 3 or 4, head_dim = 32 * num_qblocks):
 *   packed indices : [num_vectors][head_dim * bits / 8] u8, each 32-element
 *                    qblock a little-endian bitstream of bits-wide codes
 *                    (reference src/packed/mod.rs:242-309)
 *   scales         : [num_vectors][head_dim / 32] f16 bits; a negative value
 *                    marks an outlier-codebook block (quantize_tensor.rs:68-70)
 *   cache          : token t of KV head g of sequence b at
 *                    ((b * seq_stride) + g * kv_head_stride + t) records
 *                    (CompressedStorage, src/cache/storage.rs:24-139)
 */
#ifndef TURBOQUANT_AMD_H
#define TURBOQUANT_AMD_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  1..5 mirror TurboQuantError (reference src/error.rs:5-29);
 * 6 covers the candle cache errors (cache_err, src/cache/mod.rs:30-32). */
enum {
    TQ_OK = 0,
    TQ_ERR_INVALID_DIMENSION = 1,
    TQ_ERR_UNSUPPORTED_BITS = 2,
    TQ_ERR_DIMENSION_MISMATCH = 3,
    TQ_ERR_LAYER_OUT_OF_RANGE = 4,
    TQ_ERR_RANGE_OUT_OF_BOUNDS = 5,
    TQ_ERR_INVALID_ARGUMENT = 6,
    TQ_ERR_DEVICE = 7
};

/* Element types of activations crossing the boundary. */
enum { TQ_DTYPE_F32 = 0, TQ_DTYPE_BF16 = 1, TQ_DTYPE_F16 = 2 };

/* QuantNormMode (src/cache/config.rs:20-31).  MaxNorm is the default. */
enum { TQ_NORM_MAXNORM = 0, TQ_NORM_L2NORM = 1 };
/* CacheConfig::outlier_blocks = usize::MAX: PQO, every block on the outlier
 * codebook.  0 selects the standard codebook (PQ, and TQ with QJL). */
#define TQ_OUTLIER_ALL ((size_t)-1)

/* Message of the calling thread's last failed call ("" if none). */
const char *tq_last_error(void);
/* Library version string. */
const char *tq_version(void);

/* =========================================================================
 * Reference FFI, same symbols and argument meaning as
 * src/cache/cuda/ffi.rs:10-79 with hipStream_t in place of CUstream.  The
 * reference declares them void; these return a status, which a caller that
 * declares them void simply ignores (x86-64 SysV: the value is in rax).
 * ========================================================================= */

/* Replaces tq_dequant_batch (ffi.rs:11-22; tq_dequant_kernel.cu:104-125).
 * out[num_blocks][block_size] f32 = |scale| * WHT^-1(codebook[idx] * sign). */
int tq_dequant_batch(const uint8_t *packed_indices, const uint16_t *scales,
                     const float *codebook, const float *sign_pattern, float *output,
                     int num_blocks, int block_size, int bits, int bytes_per_block,
                     hipStream_t stream);

/* Replaces tq_quant_maxnorm_batch (ffi.rs:24-37; tq_quant_kernel.cu:416-439).
 * Input is already rotated; MaxNorm scale, bucketize, pack, signed f16 scale. */
int tq_quant_maxnorm_batch(const float *rotated_input, const float *boundaries,
                           uint8_t *packed_out, uint16_t *scales_out, int num_blocks,
                           int block_size, int bits, int num_boundaries, int bytes_per_block,
                           float outer_centroid, float scale_sign, hipStream_t stream);

/* Replaces tq_pack_indices (ffi.rs:39-48; tq_quant_kernel.cu:441-456). */
int tq_pack_indices(const uint8_t *indices, uint8_t *packed_out, int num_vectors,
                    int block_size, int bits, int bytes_per_block, hipStream_t stream);

/* Replaces tq_fused_attention (ffi.rs:50-78; tq_attention_kernel.cu:337-392).
 * q [num_attention_heads][head_dim] f32, out the same shape.  partial_out
 * [num_attention_heads * num_partitions][head_dim], partial_max/sum
 * [num_attention_heads * num_partitions] are caller scratch, with
 * num_partitions = ceil(kv_len / 512) as in cuda/attention.rs:13,70.  The
 * codebook (device f32, indexed by code: 2^bits entries, or 2^(bits-1) for
 * TQ records) and the 32 decode signs (device f32, applied before the
 * inverse WHT) are read as tq_attention_kernel.cu:127-130 reads them, so an
 * L2Norm cache's Beta tables decode correctly.  kv_len 0 zeroes the output
 * (cuda/attention.rs:65-68).  qjl_enabled = 1 attends TQ records (standard
 * (bits-1)-bit codebook) with the QJL correction of the kernel's dormant
 * branch (tq_attention_kernel.cu:192-231): qjl_signs [num_kv_heads]
 * [kv_stride][head_dim/8], qjl_residual_norms [num_kv_heads][kv_stride] f16,
 * rq [num_attention_heads][head_dim] = R q. */
int tq_fused_attention(const float *q, const uint8_t *k_indices, const uint16_t *k_scales,
                       const uint8_t *v_indices, const uint16_t *v_scales,
                       const float *codebook, const float *sign_pattern, float *output,
                       float *partial_out, float *partial_max, float *partial_sum,
                       const uint8_t *qjl_signs, const uint16_t *qjl_residual_norms,
                       const float *rq, int qjl_enabled, int num_attention_heads,
                       int num_kv_heads, int head_dim, int kv_len, int kv_stride,
                       int packed_dim, int num_qblocks, int bits, float softmax_scale,
                       int num_partitions, hipStream_t stream);

/* =========================================================================
 * Fused MI355X entry points (no reference counterpart as single calls; each
 * replaces a chain of reference calls, named per entry).
 * ========================================================================= */

/* PQO quantize with the block rotation fused in.  Replaces polar_quantize's
 * CUDA path = candle matmul(R_fwd) + tq_quant_maxnorm_batch
 * (quantize_tensor.rs:54-60, cuda/quantize.rs:97-168).  x [num_vectors]
 * [head_dim] in x_dtype; packed_out [num_vectors][head_dim*bits/8];
 * scales_out [num_vectors][head_dim/32] (negative: PQO outlier blocks). */
int tq_pqo_quantize(const void *x, int x_dtype, uint8_t *packed_out, uint16_t *scales_out,
                    size_t num_vectors, int head_dim, int bits, hipStream_t stream);

/* PQO dequantize.  Replaces polar_dequantize (quantize_tensor.rs:179-220) /
 * tq_dequant_batch followed by to_dtype.  out [num_vectors][head_dim]. */
int tq_pqo_dequantize(const uint8_t *packed, const uint16_t *scales, void *out, int out_dtype,
                      size_t num_vectors, int head_dim, int bits, hipStream_t stream);

/* PQO quantize of contiguous x [num_heads][tokens][head_dim] straight into
 * cache records: vector (h, t) goes to record h * cache_head_stride +
 * cache_offset + t of packed_cache / scales_cache.  Replaces
 * quantize_kv_pair + CompressedStorage::append's slice_set
 * (pqo.rs:64-100, storage.rs:145-172). */
int tq_pqo_quantize_to_cache(const void *x, int x_dtype, int num_heads, int tokens,
                             uint8_t *packed_cache, uint16_t *scales_cache,
                             long long cache_head_stride, long long cache_offset, int head_dim,
                             int bits, hipStream_t stream);

/* Dequantize records [0, tokens) of every head of a cache into contiguous
 * out [num_heads][tokens][head_dim].  Replaces dequantize_full_impl
 * (common.rs:16-62). */
int tq_pqo_dequantize_from_cache(const uint8_t *packed_cache, const uint16_t *scales_cache,
                                 long long cache_head_stride, int num_heads, int tokens, void *out,
                                 int out_dtype, int head_dim, int bits, hipStream_t stream);

/* The cache codec of any supported CacheConfig mode: polar_quantize /
 * polar_dequantize (quantize_tensor.rs:40-76, 179-220) with
 * outlier_blocks = TQ_OUTLIER_ALL (PQO: bits-bit outlier codebook, negative
 * scales) or 0 (PQ and TQ: the standard (bits-1)-bit codebook in bits-wide
 * slots, positive scales), norm_mode TQ_NORM_MAXNORM.  The tq_pqo_* entries
 * above are these with TQ_OUTLIER_ALL. */
int tq_polar_quantize(const void *x, int x_dtype, uint8_t *packed_out, uint16_t *scales_out,
                      size_t num_vectors, int head_dim, int bits, size_t outlier_blocks,
                      int norm_mode, hipStream_t stream);
int tq_polar_dequantize(const uint8_t *packed, const uint16_t *scales, void *out, int out_dtype,
                        size_t num_vectors, int head_dim, int bits, size_t outlier_blocks,
                        int norm_mode, hipStream_t stream);
int tq_polar_quantize_to_cache(const void *x, int x_dtype, int num_heads, int tokens,
                               uint8_t *packed_cache, uint16_t *scales_cache,
                               long long cache_head_stride, long long cache_offset, int head_dim,
                               int bits, size_t outlier_blocks, int norm_mode, hipStream_t stream);
int tq_polar_dequantize_from_cache(const uint8_t *packed_cache, const uint16_t *scales_cache,
                                   long long cache_head_stride, int num_heads, int tokens,
                                   void *out, int out_dtype, int head_dim, int bits,
                                   size_t outlier_blocks, int norm_mode, hipStream_t stream);

/* Workspace for tq_pqo_decode_attention: split-K partials from its start;
 * a header line and one merge counter line per (sequence, KV head) below its
 * end (workspace_bytes rounded down to 256).  A workspace sized and
 * initialised for the largest (batch, num_heads, max_kv_len) serves every
 * call with no more sequences x KV heads and no larger partials, in any
 * order, given the same pointer and workspace_bytes each time.  A call whose
 * counters the init did not zero, or whose partials would reach them, stores
 * nothing and writes NaN outputs (the workspace stays usable). */
size_t tq_attention_workspace_size(int batch, int num_heads, int num_kv_heads, int head_dim,
                                   int max_kv_len);
/* Writes the header (batch * num_kv_heads) and zero-fills those merge
 * counters (once after allocation; every call leaves its counters zero
 * again).  Uses a fill kernel, no memset node. */
int tq_attention_workspace_init(void *workspace, size_t workspace_bytes, int batch,
                                int num_heads, int num_kv_heads, int head_dim, int max_kv_len,
                                hipStream_t stream);

/* Fused PQO decode attention over a compressed cache, batched over
 * sequences with per-sequence lengths, split-K over the context and GQA
 * sharing (each compressed byte is read once for all query heads of its KV
 * head).  Replaces PqoCache::decode_cuda -> fused_attention ->
 * tq_fused_attention (pqo.rs:106-174, cuda/attention.rs:41-174).
 *   q   [batch][num_heads][head_dim] in q_dtype
 *   out [batch][num_heads][head_dim] in out_dtype
 *   kv_lens: device int[batch]; max_kv_len: host bound on every kv_lens[b].
 *   kv_lens may be null when every sequence holds exactly max_kv_len tokens
 *   (a length the host knows): the kernel then reads no length from memory.
 *   record strides in tokens: kv_head_stride (capacity), seq_stride.
 *   A sequence of length 0 (and every sequence when max_kv_len is 0) gets
 *   zero outputs, as the reference's fused_attention zero-fills its output
 *   (cuda/attention.rs:65-68). */
int tq_pqo_decode_attention(const void *q, int q_dtype, const uint8_t *k_indices,
                            const uint16_t *k_scales, const uint8_t *v_indices,
                            const uint16_t *v_scales, const int *kv_lens, int batch,
                            int num_heads, int num_kv_heads, int head_dim, int bits,
                            int max_kv_len, long long kv_head_stride, long long seq_stride,
                            float softmax_scale, void *out, int out_dtype, void *workspace,
                            size_t workspace_bytes, hipStream_t stream);

/* tq_pqo_decode_attention without the workspace arguments, for callers that
 * cannot allocate (HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the reference.  The split-K partials
 * and merge counters live in the library's file-scope device array of 8 MiB
 * per device (held until the process ends; room for 1,024 (sequence, KV
 * head) pairs and 7.75 MiB of partials = batch * num_heads *
 * ceil(max_kv_len / chunk) * (head_dim + 2) * 4 bytes, each part rounded up
 * to 256, with chunk = 512 tokens, or 256 at head_dim 256 or with more than
 * 4 query heads per KV head); larger shapes are rejected with
 * TQ_ERR_INVALID_ARGUMENT.  No
 * hipMalloc, hipFree or other allocation.  Every call on a device shares that
 * device's array: calls that overlap in time on one device race. */
int tq_pqo_decode_attention_noalloc(const void *q, int q_dtype, const uint8_t *k_indices,
                                    const uint16_t *k_scales, const uint8_t *v_indices,
                                    const uint16_t *v_scales, const int *kv_lens, int batch,
                                    int num_heads, int num_kv_heads, int head_dim, int bits,
                                    int max_kv_len, long long kv_head_stride, long long seq_stride,
                                    float softmax_scale, void *out, int out_dtype,
                                    hipStream_t stream);

/* Fused decode attention over any cache mode: outlier_blocks TQ_OUTLIER_ALL
 * (PQO) or 0 (PQ), norm_mode TQ_NORM_MAXNORM; arguments as
 * tq_pqo_decode_attention.  qjl_signs non-null selects TQ: the logits get
 * the QJL correction softmax_scale * |r_t| sqrt(pi/2)/sqrt(d) *
 * sum_j rq_j (2 b_tj - 1) (tq_attention_kernel.cu:192-231; tq.rs:185-253),
 * with rq [batch][num_heads][head_dim] f32 = R q (tq_qjl_project),
 * qjl_signs [..records..][head_dim/8] and qjl_norms [..records..] f16 laid
 * out by record like the codes.  Replaces TqCache::decode's dequantize +
 * logit bias + SDPA (tq.rs:275-297). */
/* tq_cache_decode_attention for TQ records (outlier_blocks 0) with the query
 * projection rq = R q computed inside the decode launch from the sign
 * matrix (tq_qjl_sign_matrix: row j = head_dim / 32 words, bit c set = -1)
 * instead of a separate tq_qjl_project launch.  rq is formed on the matrix
 * cores from exact products (+-1 times the query cut into bf16 parts that
 * sum to it); only the f32 accumulation order differs from tq_qjl_project's
 * serial column-order sum (precompute_query_projections, qjl.rs:196-208),
 * so the outputs agree with tq_qjl_project + tq_cache_decode_attention to
 * rounding (within 1e-5 in the tests).  No reference counterpart as
 * one call: replaces the projection and TqCache::decode's attention
 * (tq.rs:185-297). */
int tq_tq_decode_attention(const void *q, int q_dtype, const uint8_t *k_indices,
                           const uint16_t *k_scales, const uint8_t *v_indices,
                           const uint16_t *v_scales, const uint8_t *qjl_signs,
                           const uint16_t *qjl_norms, const uint32_t *qjl_sign_matrix,
                           const int *kv_lens, int batch, int num_heads, int num_kv_heads,
                           int head_dim, int bits, int norm_mode, int max_kv_len,
                           long long kv_head_stride, long long seq_stride, float softmax_scale,
                           void *out, int out_dtype, void *workspace, size_t workspace_bytes,
                           hipStream_t stream);

int tq_cache_decode_attention(const void *q, int q_dtype, const uint8_t *k_indices,
                              const uint16_t *k_scales, const uint8_t *v_indices,
                              const uint16_t *v_scales, const float *rq, const uint8_t *qjl_signs,
                              const uint16_t *qjl_norms, const int *kv_lens, int batch,
                              int num_heads, int num_kv_heads, int head_dim, int bits,
                              size_t outlier_blocks, int norm_mode, int max_kv_len,
                              long long kv_head_stride, long long seq_stride, float softmax_scale,
                              void *out, int out_dtype, void *workspace, size_t workspace_bytes,
                              hipStream_t stream);

/* Multi-query (prefill) attention straight over a compressed cache, on the
 * matrix cores (no dequantized K/V): q [num_heads][q_len][head_dim] in
 * q_dtype, out the same shape in out_dtype; query i sits at position
 * kv_len - q_len + i and, when causal, sees tokens t <= that position.
 * Records as tq_cache_decode_attention (one sequence, kv_head_stride);
 * qjl_signs non-null selects TQ (rq [num_heads][q_len][head_dim] f32 = R q,
 * logits scale * (q.k + correction)).  head_dim 128, GQA 1/2/4, outlier_blocks
 * 0 or all.  Replaces the reference's prefill result (dequantized K/V for
 * SDPA, pqo.rs:184-200, tq.rs:258-273).  Calls with 6 or more query blocks
 * (64 queries at GQA 2) per KV head over 768 or more tokens decode each
 * 64-token tile once
 * into a stream-ordered staging buffer (hipMallocFromPoolAsync /
 * hipFreeAsync on stream, from a memory pool of the library's own per device
 * that keeps up to 1 GiB between calls; about 72 KB per tile and KV head,
 * 73 KB for TQ);
 * the environment variable
 * TQ_PREFILL_STAGING=0 or 1 forces either path (never staged when a KV
 * head's images would reach 2^31 bytes, about 1.9 M tokens; both within the tolerance;
 * staged tiles hold K inverse-rotated, so the two differ by rounding).  When
 * the attention's grid (one workgroup per 128 (query, head) rows of a KV
 * head) would leave compute units idle, each query block's tiles are split
 * over several workgroups and a last launch merges the splits' partial rows
 * (132 floats per split, head and query, in a buffer taken the same way);
 * TQ_PREFILL_SPLITS=n forces n splits (1: none). */
int tq_cache_prefill_attention(const void *q, int q_dtype, const uint8_t *k_indices,
                               const uint16_t *k_scales, const uint8_t *v_indices,
                               const uint16_t *v_scales, const float *rq, const uint8_t *qjl_signs,
                               const uint16_t *qjl_norms, int num_heads, int q_len,
                               int num_kv_heads, int head_dim, int bits, size_t outlier_blocks,
                               int norm_mode, int kv_len, long long kv_head_stride, int causal,
                               float softmax_scale, void *out, int out_dtype, hipStream_t stream);

/* =========================================================================
 * Core full-vector codec (TurboQuantConfig{bits, dim, rotation_seed}),
 * batched over vectors.  A PackedBlock maps to one row of packed_out
 * (packed/mod.rs:149-233: LSB-first bits-wide indices, dim*bits/8 bytes) plus
 * its f16 scale (the vector's L2 norm).  dim: 32, 64, 128 or 256 (the
 * dimensions with codebook tables, codebook/tables.rs:89-105); bits 2..4.
 * ========================================================================= */

/* Replaces quantize_vec (quantize.rs:142-157) applied to each row of
 * data[num_vectors][dim] f32.  packed_out [num_vectors][dim*bits/8],
 * scales_out [num_vectors] f16 bits. */
int tq_quantize_vec_batch(const float *data, uint8_t *packed_out, uint16_t *scales_out,
                          size_t num_vectors, int bits, int dim, uint64_t rotation_seed,
                          hipStream_t stream);

/* Replaces dequantize_vec (quantize.rs:207-240) per row: centroid lookup,
 * inverse rotation, times the f16 scale.  out [num_vectors][dim] f32. */
int tq_dequantize_vec_batch(const uint8_t *packed, const uint16_t *scales, float *out,
                            size_t num_vectors, int bits, int dim, uint64_t rotation_seed,
                            hipStream_t stream);

/* Replaces dequantize_rotated (quantize.rs:306-316): centroids times scale,
 * left in the rotated domain. */
int tq_dequantize_rotated_batch(const uint8_t *packed, const uint16_t *scales, float *out,
                                size_t num_vectors, int bits, int dim, hipStream_t stream);

/* =========================================================================
 * QJL estimator (TurboQuant_prod): (total_bits-1)-bit polar codec plus a
 * 1-bit sign sketch of the residual under the implicit hash-Rademacher
 * matrix R (qjl.rs:143-208).  dim: 32, 64 or 128; total_bits 3 or 4.
 * A QjlBlock maps to one row of polar_packed [dim*(total_bits-1)/8] u8, its
 * polar f16 scale, one row of signs [dim/8] u8 (bit j of byte j/8 =
 * (R r)_j >= 0) and the f16 residual norm (qjl.rs:111-134).
 * ========================================================================= */

/* Replaces quantize_with_qjl (qjl.rs:355-377) over the rows of
 * data[num_vectors][dim] f32 (QuantizedKVCache::push_batch, attention.rs:274-301,
 * uses one qjl_seed for the whole cache). */
int tq_qjl_quantize_batch(const float *data, uint8_t *polar_packed, uint16_t *polar_scales,
                          uint8_t *signs, uint16_t *residual_norms, size_t num_vectors,
                          int total_bits, int dim, uint64_t rotation_seed, uint64_t qjl_seed,
                          hipStream_t stream);

/* EstimationContext for a batch of queries (qjl.rs:488-492, 561-572):
 * ctx_out[q] = { qt[dim] = forward rotation of query q, rq[dim] =
 * precompute_query_projections(q) }, f32 [num_queries][2*dim]. */
int tq_qjl_query_context(const float *queries, float *ctx_out, size_t num_queries, int dim,
                         uint64_t rotation_seed, uint64_t qjl_seed, hipStream_t stream);

/* Replaces estimate_inner_product_with_codebook over all (query, key) pairs
 * (qjl.rs:585-606; attention_scores, attention.rs:319-353):
 * scores[q][k] = <q, x_mse_k> + |r_k| sqrt(pi/2)/sqrt(d) * sum_j rq_j (2 b_kj - 1). */
int tq_qjl_scores(const float *ctx, size_t num_queries, const uint8_t *polar_packed,
                  const uint16_t *polar_scales, const uint8_t *signs,
                  const uint16_t *residual_norms, size_t num_keys, int polar_bits, int dim,
                  uint64_t rotation_seed, float *scores, hipStream_t stream);

/* Row softmax probs = exp(scale (s - max)) / sum over cols; no reference
 * counterpart (attention_scores returns raw scores, attention.rs:344-352). */
int tq_softmax_rows(const float *scores, float *probs, size_t rows, size_t cols, float scale,
                    hipStream_t stream);

/* Workspace bytes for tq_qjl_weighted_values. */
size_t tq_qjl_weighted_values_workspace_size(size_t num_queries, size_t num_values, int dim);

/* Replaces QuantizedKVCache::weighted_values (attention.rs:371-408) for a
 * batch of weight rows: out[q] = sum_t weights[q][t] * dequantize(value_t),
 * weights f32 [num_queries][num_values], out f32 [num_queries][dim]. */
int tq_qjl_weighted_values(const uint8_t *polar_packed, const uint16_t *polar_scales,
                           size_t num_values, const float *weights, size_t num_queries,
                           int polar_bits, int dim, uint64_t rotation_seed, float *out,
                           void *workspace, size_t workspace_bytes, hipStream_t stream);

/* ---- TqCache building blocks (reference src/cache/tq.rs) ----
 * head_dim 64, 128 or 256 (32 also for the sign matrix). */

/* The d x d sign bits of the Rademacher matrix R (qjl.rs:143-189) for
 * qjl_seed: bits_out[j * dim/32 + w] bit b set <=> R[j][32 w + b] < 0
 * (build_rademacher_matrix, precomputed/mod.rs:116-125). */
int tq_qjl_sign_matrix(uint32_t *bits_out, int dim, uint64_t qjl_seed, hipStream_t stream);

/* compute_qjl_signs_and_norms for keys just stored in a TQ cache
 * (tq.rs:154-182, 373-412): k [num_heads][tokens][head_dim] as appended;
 * its records h * cache_head_stride + cache_offset + t are dequantized, the
 * residual r = k - k_hat gives norms_cache[record] = f16(|r|) and
 * signs_cache[record][head_dim/8] = bits (R r)_j >= 0 (LSB first). */
int tq_qjl_cache_sketch(const void *k, int k_dtype, int num_heads, int tokens,
                        const uint8_t *packed_cache, const uint16_t *scales_cache,
                        const uint32_t *sign_matrix, uint8_t *signs_cache, uint16_t *norms_cache,
                        long long cache_head_stride, long long cache_offset, int head_dim, int bits,
                        size_t outlier_blocks, int norm_mode, hipStream_t stream);

/* tq_qjl_cache_sketch plus rq = R q for num_q_rows rows of q (q_dtype) in
 * the same launch (a TQ decode step's sketch and projection). */
int tq_qjl_cache_sketch_project(const void *k, int k_dtype, int num_heads, int tokens,
                                const uint8_t *packed_cache, const uint16_t *scales_cache,
                                const uint32_t *sign_matrix, uint8_t *signs_cache,
                                uint16_t *norms_cache, long long cache_head_stride,
                                long long cache_offset, int head_dim, int bits,
                                size_t outlier_blocks, int norm_mode, const void *q, int q_dtype,
                                float *rq, size_t num_q_rows, hipStream_t stream);

/* rq[row] = R q[row] (precompute_query_projections, qjl.rs:488-492; r_q of
 * tq.rs:233-234), q [num_rows][dim] in q_dtype, rq f32. */
int tq_qjl_project(const void *q, int q_dtype, const uint32_t *sign_matrix, float *rq,
                   size_t num_rows, int dim, hipStream_t stream);

/* f32(sqrt(pi/2)) / sqrt(head_dim), the per-norm factor of tq.rs:213-214. */
float tq_qjl_bias_scale(int head_dim);

/* compute_logit_bias (tq.rs:185-253): out [num_q_heads][q_len][kv_len] in
 * out_dtype = (sum_j rq[h][i][j] (2 b_tj - 1)) * (|r_t| * tq_qjl_bias_scale),
 * query head h reading KV head h / (num_q_heads / num_kv_heads);
 * rq [num_q_heads][q_len][head_dim] f32 from tq_qjl_project. */
int tq_qjl_logit_bias(const float *rq, int num_q_heads, int q_len, const uint8_t *signs_cache,
                      const uint16_t *norms_cache, int num_kv_heads, int kv_len,
                      long long cache_head_stride, int head_dim, void *out, int out_dtype,
                      hipStream_t stream);

/* =========================================================================
 * Device-resident KV caches with the CompressedKVCache contract (trait of
 * mistralrs-kv-cache, methods as used in pqo.rs:183-236 and tq.rs:256-324):
 * PqoCache (pqo.rs:21-236; outlier_blocks TQ_OUTLIER_ALL = PQO, 0 = PQ) and
 * TqCache (tq.rs: PQ codes plus the QJL sketch of every key's residual,
 * qjl = 1), over a CompressedStorage (storage.rs:24-203).  The handle owns
 * its device buffers.  K/V inputs are one sequence's
 * [num_kv_heads][tokens][head_dim] (the reference's [1, H, T, D]); queries
 * [num_q_heads][q_len][head_dim] ([1, Hq, q_len, D]).
 * ========================================================================= */

/* PqoCache::new / TqCache::new (CacheConfig{bits, head_dim, num_kv_heads,
 * num_layers, norm_mode, outlier_blocks}). */
int tq_cache_create(int num_layers, int num_kv_heads, int head_dim, int bits, int norm_mode,
                    size_t outlier_blocks, int qjl, void **cache);
/* Frees the handle.  Its device buffers go back to the device's memory pool
 * in the order of the stream of the cache's last call (stream-ordered, no
 * host or device synchronization; work queued on that stream that reads them
 * runs first), as the reference's tensors are released on their device's
 * stream.  That stream must still exist; work on other streams that reads the
 * cache must be ordered before it by the caller. */
void tq_cache_destroy(void *cache);
/* 1 for a TqCache handle. */
int tq_cache_is_tq(void *cache);

/* CompressedKVCache::prefill (pqo.rs:184-200, tq.rs:258-273): stores k, v;
 * on the layer's first call sets *returned_originals = 1 (the caller's k, v
 * are the result), otherwise writes the whole dequantized layer
 * [num_kv_heads][seq_len][head_dim] into k_out, v_out in `dtype`.  A TqCache
 * also writes logit_bias_out [num_q_heads][q_len][seq_len] in q_dtype
 * (compute_logit_bias, tq.rs:185-253); q is unused by a PqoCache. */
int tq_cache_prefill(void *cache, int layer, const void *k, const void *v, int dtype, int tokens,
                     const void *q, int q_dtype, int num_q_heads, int q_len, void *k_out,
                     void *v_out, int *returned_originals, void *logit_bias_out,
                     hipStream_t stream);

/* CompressedKVCache::decode on the fused path (DecodeOutput::Fused): stores
 * k, v, then out [num_q_heads][head_dim] = attention of q [num_q_heads]
 * [head_dim] over the whole layer; a TqCache adds the QJL correction to the
 * logits inline (replacing tq.rs:275-297's dequantize + logit bias). */
int tq_cache_decode(void *cache, int layer, const void *k, const void *v, int kv_dtype, int tokens,
                    const void *q, int q_dtype, int num_q_heads, float softmax_scale, void *out,
                    int out_dtype, hipStream_t stream);

/* CompressedKVCache::decode on the dequantized path (DecodeOutput::
 * Dequantized, pqo.rs:218-221, tq.rs:275-297): stores k, v, writes the whole
 * layer into k_out, v_out and, for a TqCache, logit_bias_out [num_q_heads]
 * [q_len][seq_len] in q_dtype. */
int tq_cache_decode_dequantized(void *cache, int layer, const void *k, const void *v, int dtype,
                                int tokens, const void *q, int q_dtype, int num_q_heads, int q_len,
                                void *k_out, void *v_out, void *logit_bias_out, hipStream_t stream);

/* Multi-query attention of q [num_q_heads][q_len][head_dim] over the whole
 * layer (tq_cache_prefill_attention on the stored records; the queries sit at
 * the layer's last q_len positions), without dequantizing it: the attention a
 * caller runs on prefill's DequantResult (pqo.rs:184-200, tq.rs:258-273),
 * with the QJL correction for a TqCache. */
int tq_cache_attend_prefill(void *cache, int layer, const void *q, int q_dtype, int num_q_heads,
                            int q_len, int causal, float softmax_scale, void *out, int out_dtype,
                            hipStream_t stream);

/* seq_len / reset / memory_usage (pqo.rs:224-236, tq.rs:299-323,
 * storage.rs:175-202).  reset releases every layer's buffers in the order of
 * the cache's last stream, as tq_cache_destroy does (no synchronization); the
 * next append allocates zeroed buffers afresh. */
size_t tq_cache_seq_len(void *cache, int layer);
int tq_cache_reset(void *cache);
size_t tq_cache_memory_usage(void *cache);
/* Records per head allocated for a layer (grows to needed + max(needed/4, 128)). */
size_t tq_cache_capacity(void *cache, int layer);
/* Copies a layer's stored records [num_kv_heads][seq_len] (codes, scales and,
 * for a TqCache, signs and norms when non-null) into contiguous buffers. */
int tq_cache_read_layer(void *cache, int layer, uint8_t *k_indices, uint16_t *k_scales,
                        uint8_t *v_indices, uint16_t *v_scales, uint8_t *qjl_signs,
                        uint16_t *qjl_norms, hipStream_t stream);
/* Device views of a layer's buffers (CompressedStorage::k_indices etc.; the
 * QJL ones null for a PqoCache). */
int tq_cache_buffers(void *cache, int layer, uint8_t **k_indices, uint16_t **k_scales,
                     uint8_t **v_indices, uint16_t **v_scales, uint8_t **qjl_signs,
                     uint16_t **qjl_norms);

/* PqoCache with the PQO config / TqCache with the TQ config (MaxNorm). */
int tq_pqo_cache_create(int num_layers, int num_kv_heads, int head_dim, int bits, void **cache);
int tq_tq_cache_create(int num_layers, int num_kv_heads, int head_dim, int bits, void **cache);
/* The tq_cache_* calls above for PqoCache handles, without the query. */
void tq_pqo_cache_destroy(void *cache);
int tq_pqo_cache_prefill(void *cache, int layer, const void *k, const void *v, int dtype, int tokens,
                         void *k_out, void *v_out, int *returned_originals, hipStream_t stream);
int tq_pqo_cache_decode(void *cache, int layer, const void *k, const void *v, int kv_dtype, int tokens,
                        const void *q, int q_dtype, int num_q_heads, float softmax_scale, void *out,
                        int out_dtype, hipStream_t stream);
size_t tq_pqo_cache_seq_len(void *cache, int layer);
int tq_pqo_cache_reset(void *cache);
size_t tq_pqo_cache_memory_usage(void *cache);
size_t tq_pqo_cache_capacity(void *cache, int layer);
int tq_pqo_cache_read_layer(void *cache, int layer, uint8_t *k_indices, uint16_t *k_scales,
                            uint8_t *v_indices, uint16_t *v_scales, hipStream_t stream);
int tq_pqo_cache_buffers(void *cache, int layer, uint8_t **k_indices, uint16_t **k_scales,
                         uint8_t **v_indices, uint16_t **v_scales);

#ifdef __cplusplus
}
#endif
#endif
