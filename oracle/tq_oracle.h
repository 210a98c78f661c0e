/*
 * tq_oracle.h -- CPU restatement of the TurboQuant reference algorithms.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP
 * kernels are compared against.  Only tests/, __graft_entry__.smoke() and
 * the cpu_baseline leg of bench.py may load it.  The product library
 * (turboquant_amd) never links, loads or calls it.
 *
 * Every function cites the reference file:line it restates.  Arithmetic is
 * IEEE binary32 with no contraction (compile with -ffp-contract=off): the
 * reference is Rust, which never fuses a*b+c.
 *
 * Parity pins (what checks each function independently of this file):
 *   see the per-function comments; functions marked "parity unpinned" have
 *   no independent check beyond self-consistency.
 */
#ifndef TQ_ORACLE_H
#define TQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error codes mirror TurboQuantError (reference src/error.rs:5-29). */
enum {
    TQO_OK = 0,
    TQO_ERR_INVALID_DIMENSION = 1,
    TQO_ERR_UNSUPPORTED_BITS = 2,
    TQO_ERR_DIMENSION_MISMATCH = 3,
    TQO_ERR_LAYER_OUT_OF_RANGE = 4,
    TQO_ERR_RANGE_OUT_OF_BOUNDS = 5,
    TQO_ERR_INVALID_ARGUMENT = 6
};

/* ---- IEEE binary16 (the `half` crate's f16::from_f32 / to_f32) ---- */
uint16_t tqo_f32_to_f16(float x);
float tqo_f16_to_f32(uint16_t h);
/* bf16 round-to-nearest-even (the `half` crate's bf16::from_f32). */
uint16_t tqo_f32_to_bf16(float x);
void tqo_f32_to_f16_batch(const float *x, size_t n, uint16_t *out);
void tqo_f16_to_f32_batch(const uint16_t *h, size_t n, float *out);

/* ---- rotation (src/rotation.rs) ---- */
int tqo_is_valid_dim(size_t dim);
void tqo_generate_sign_pattern(size_t dim, uint64_t seed, float *out);
void tqo_wht_inplace(float *data, size_t n);
int tqo_rotate(float *data, const float *signs, size_t n, size_t sign_len, int inverse);

/* ---- codebooks (src/codebook/mod.rs, tables.rs) ---- */
int tqo_get_codebook(int bits, size_t dim, const double **centroids,
                     const double **boundaries, int *num_centroids);
uint8_t tqo_nearest_centroid(double value, const double *boundaries, int nb);

/* ---- bit packing (src/packed/mod.rs, indices.rs) ---- */
size_t tqo_packed_len(int bits, size_t count);
size_t tqo_pack_indices(int bits, const uint8_t *idx, size_t count, uint8_t *out);
void tqo_unpack_indices(int bits, const uint8_t *packed, size_t packed_len,
                        size_t count, uint8_t *out);

/* ---- core full-vector codec (src/quantize.rs) ---- */
float tqo_l2_norm(const float *x, size_t n);
int tqo_quantize_vec(int bits, size_t dim, uint64_t seed, const float *data,
                     uint8_t *packed_out, uint16_t *scale_out);
int tqo_dequantize_vec(int bits, size_t dim, uint64_t seed, const uint8_t *packed,
                       uint16_t scale, float *out);
int tqo_dequantize_rotated(int bits, size_t dim, const uint8_t *packed,
                           uint16_t scale, float *out);
int tqo_quantize_vec_batch(int bits, size_t dim, uint64_t seed, size_t n,
                           const float *data, uint8_t *packed_out, uint16_t *scales_out);
int tqo_dequantize_vec_batch(int bits, size_t dim, uint64_t seed, size_t n,
                             const uint8_t *packed, const uint16_t *scales, float *out);

/* ---- PQO cache codec (src/cache/precomputed, quantize_tensor.rs, wht_tensor.rs) ---- */
int tqo_pqo_codebook(int bits, float *centroids, float *boundaries, int *num_centroids,
                     float *outer_centroid);
void tqo_pqo_sign32(float *out);
void tqo_pqo_decode_signs(float *out);
void tqo_pqo_rotate_block(const float *x, float *r);
void tqo_pqo_rotate_block_gemm(const float *x, float *r);
void tqo_pqo_rotate_block_fma(const float *x, float *r);
int tqo_pqo_rotate_blocks(int order, size_t n, const float *x, float *r);
int tqo_pqo_quantize_rotated(int bits, size_t num_blocks, const float *rotated,
                             uint8_t *packed_out, uint16_t *scales_out, float scale_sign);
int tqo_pqo_quantize(int bits, size_t n, size_t head_dim, const float *x,
                     uint8_t *packed_out, uint16_t *scales_out);
int tqo_pqo_dequantize(int bits, size_t n, size_t head_dim, const uint8_t *packed,
                       const uint16_t *scales, float *out);

/* polar_quantize / polar_dequantize for the cache modes (outlier_blocks:
 * >= num_blocks PQO, 0 PQ/TQ, else mixed), norm_mode 0 MaxNorm / 1 L2Norm. */
int tqo_polar_quantize(int bits, size_t outlier_blocks, int norm_mode, size_t n, size_t head_dim,
                       const float *x, uint8_t *packed_out, uint16_t *scales_out);
int tqo_polar_dequantize(int bits, size_t outlier_blocks, int norm_mode, size_t n, size_t head_dim,
                         const uint8_t *packed, const uint16_t *scales, float *out);

/* ---- TqCache (src/cache/tq.rs) ---- */
int tqo_tq_signs_norms(size_t n, size_t head_dim, const float *x, const float *xhat, uint8_t *signs,
                       uint16_t *norms);
int tqo_tq_logit_bias(size_t num_q_heads, size_t num_kv_heads, size_t d, size_t q_len, size_t kv_len,
                      const float *q, const uint8_t *signs, const uint16_t *norms, float *out);
int tqo_attention_dense_bias(size_t num_heads, size_t num_kv_heads, size_t head_dim, size_t kv_len,
                             const float *q, const float *k, const float *v, const float *bias,
                             float softmax_scale, float *out);

/* ---- dense attention oracle over dequantized K/V ---- */
int tqo_attention_prefill(size_t num_heads, size_t num_kv_heads, size_t d, size_t q_len,
                          size_t kv_len, const float *q, const float *k, const float *v,
                          const float *bias, float softmax_scale, int causal, float *out);
int tqo_attention_dense(size_t num_heads, size_t num_kv_heads, size_t head_dim,
                        size_t kv_len, const float *q, const float *k, const float *v,
                        float softmax_scale, float *out);

/* ---- QJL (src/qjl.rs) ---- */
uint64_t tqo_qjl_mix_seed(uint64_t seed, size_t row);
float tqo_rademacher_sign(uint64_t row_seed, size_t row, size_t col);
void tqo_generate_rademacher_row(size_t dim, uint64_t seed, size_t row, float *out);
float tqo_rademacher_vector_product(const float *data, size_t dim, uint64_t seed, size_t row);
int tqo_compute_qjl_signs(const float *residual, size_t dim, uint64_t seed, uint8_t *out);
int tqo_quantize_with_qjl(int total_bits, size_t dim, uint64_t rot_seed, uint64_t qjl_seed,
                          const float *data, uint8_t *polar_packed, uint16_t *polar_scale,
                          uint8_t *signs, uint16_t *residual_norm);
void tqo_precompute_query_projections(const float *query, size_t dim, uint64_t seed, float *out);
float tqo_qjl_scaling_constant(float residual_norm, size_t dim);
float tqo_qjl_correction(const float *r_query, const uint8_t *signs, size_t dim);
int tqo_estimate_inner_product(int polar_bits, size_t dim, uint64_t rot_seed,
                               const float *query, const float *r_query,
                               const uint8_t *polar_packed, uint16_t polar_scale,
                               const uint8_t *signs, uint16_t residual_norm, float *out);
int tqo_qjl_quantize_batch(int total_bits, size_t dim, uint64_t rot_seed, uint64_t qjl_seed,
                           size_t n, const float *data, uint8_t *polar_packed,
                           uint16_t *polar_scales, uint8_t *signs, uint16_t *residual_norms);
int tqo_qjl_scores_batch(int polar_bits, size_t dim, uint64_t rot_seed, uint64_t qjl_seed,
                         size_t num_queries, const float *queries, size_t num_keys,
                         const uint8_t *polar_packed, const uint16_t *polar_scales,
                         const uint8_t *signs, const uint16_t *residual_norms, float *scores);
int tqo_weighted_values(int polar_bits, size_t dim, uint64_t rot_seed, size_t num_values,
                        const uint8_t *polar_packed, const uint16_t *polar_scales,
                        const float *weights, float *out);

/* ---- test data generators (reference tests) ---- */
void tqo_pseudo_random_vec(size_t dim, uint64_t seed, float *out);
void tqo_lcg_normal_vecs(uint64_t seed, size_t dim, size_t count, float *out);

#ifdef __cplusplus
}
#endif
#endif
