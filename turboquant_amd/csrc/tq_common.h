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
// GpuPrecomputed, precomputed/mod.rs:45-98).  outlier_blocks >= num_blocks
// (PQO): every block on the bits-bit outlier codebook, negative scales.
// outlier_blocks == 0 (PQ / TQ): the standard (bits - 1)-bit codebook, its
// codes in bits-wide slots (packed_dim = head_dim * bits / 8), positive
// scales.  MaxNorm divides by the outlier codebook's largest centroid in both
// (quantize_tensor.rs:103-108).
struct PolarCodec {
  int bits = 0;     // slot width
  int cb_bits = 0;  // codebook width (bits or bits - 1)
  bool outlier = false;
  PqoCodebook cb;   // centroids / boundaries of the blocks' codebook
  float outer = 0.f;
  float scale_sign = 1.f;
};
// Fills `codec` for (bits, norm_mode, outlier_blocks) or returns an error
// status for a mode this library does not implement.
int polar_codec(int bits, int norm_mode, size_t outlier_blocks, int num_blocks, PolarCodec &codec);

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
