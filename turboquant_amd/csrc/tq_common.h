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
