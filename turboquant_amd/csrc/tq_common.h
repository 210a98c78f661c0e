// tq_common.h -- host-side helpers shared by the C ABI launchers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "turboquant_amd.h"

namespace tqh {

// Records the calling thread's last error message and returns `code`.
int fail(int code, const char *fmt, ...);
// Maps a HIP error after a launch to TQ_ERR_DEVICE with its message.
int check_launch(const char *what);

inline bool valid_dtype(int dt) { return dt == TQ_DTYPE_F32 || dt == TQ_DTYPE_BF16 || dt == TQ_DTYPE_F16; }

// PQO codebook of the reference (src/cache/precomputed/codebooks.rs:51-88)
// evaluated in f32 exactly as there; outer = max centroid (mod.rs:78).
struct PqoCodebook {
  int bits = 0;
  int nc = 0;
  float c[16] = {};
  float b[15] = {};
  float outer = 0.f;
};
PqoCodebook pqo_codebook(int bits);

// Codec of one cache mode (CacheConfig, src/cache/config.rs:50-85;
// GpuPrecomputed, precomputed/mod.rs:45-98).  The outlier codebook has
// `bits` bits, the standard one bits - 1, its codes in bits-wide slots
// (packed_dim = head_dim * bits / 8).  outlier_blocks >= num_blocks (PQO):
// every block on the outlier codebook; 0 (PQ / TQ): every block on the
// standard one; in between, quantize_tensor.rs:118-150 sends the first
// n * outlier_blocks rows of the [n * num_blocks, 32] block matrix to the
// outlier boundaries while the scale sign (negative = outlier, which the
// dequantize dispatches on) marks the first outlier_blocks blocks of each
// vector.  MaxNorm divides by the outlier codebook's largest centroid
// (quantize_tensor.rs:103-108); L2Norm uses the Beta-optimal tables of
// dimension 32 (codebooks.rs:30-47).
struct PolarCodec {
  int bits = 0;         // slot width
  int cb_bits = 0;      // codebook width of uniform modes (bits or bits - 1)
  int norm_mode = 0;
  bool outlier = false; // every block on the outlier codebook
  bool mixed = false;   // 0 < outlier_blocks < num_blocks
  int num_blocks = 0;
  int eo = 0;           // min(outlier_blocks, num_blocks)
  PqoCodebook cb;       // the blocks' codebook in uniform modes
  PqoCodebook ocb, ncb; // outlier (bits) and standard (bits - 1) codebooks
  float outer = 0.f;    // MaxNorm divisor: the outlier codebook's largest centroid
  float scale_sign = 1.f;
};
// Fills `codec` for (bits, norm_mode, outlier_blocks) or returns an error
// status for an invalid mode.
int polar_codec(int bits, int norm_mode, size_t outlier_blocks, int num_blocks, PolarCodec &codec);

// Fused decode attention (tq_cache_decode_attention) with the length given
// by the host: kv_lens null and host_len >= 0 means every sequence holds
// host_len tokens, no length is read on the device; max_kv_len fixes the
// workspace layout (a cache passes its capacity, so the layout stays put as
// the sequence grows).
int decode_attention(const void *q, int q_dtype, const uint8_t *k_indices, const uint16_t *k_scales,
                     const uint8_t *v_indices, const uint16_t *v_scales, const float *rq, const uint8_t *qjl_signs,
                     const uint16_t *qjl_norms, const int *kv_lens, int host_len, int batch, int num_heads,
                     int num_kv_heads, int head_dim, int bits, size_t outlier_blocks, int norm_mode, int max_kv_len,
                     long long kv_head_stride, long long seq_stride, float softmax_scale, void *out, int out_dtype,
                     void *workspace, size_t workspace_bytes, hipStream_t stream, const uint32_t *rmat = nullptr);

// fl(1 / fl(sqrt(dim))): the QJL projection's scale (1 / sqrt(d), qjl.rs),
// each step rounded to f32.
float inv_sqrt_dim(int dim);

// Per-boundary constants of the exact division threshold (see
// tqd::div_threshold): mu = midpoint of b and nextup(b), strict = b even.
struct DivThresholds {
  int nb = 0;
  double mu[15] = {};
  uint32_t strict_mask = 0;
  float mul = 0.f;  // fl(1 / outer), candle's affine(1/rhs) scalar division
};
DivThresholds div_thresholds(const float *b, int nb, float outer);

}  // namespace tqh
