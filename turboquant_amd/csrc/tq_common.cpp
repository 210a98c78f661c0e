// tq_common.cpp -- error reporting and host-side constant tables.
#include "tq_common.h"
#include "tq_codebooks.h"
#include "tq_device.h"

#include <cmath>
#include <cstring>

namespace {
thread_local char g_last_error[512] = "";
}

extern "C" const char *tq_last_error(void) { return g_last_error; }
extern "C" const char *tq_version(void) { return "turboquant_amd 0.1.0 (gfx950)"; }

namespace tqh {

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TQ_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
  return TQ_OK;
}

PqoCodebook pqo_codebook(int bits) {
  // src/cache/precomputed/codebooks.rs:8-88.  3-bit: the llama.cpp table;
  // 4-bit: c4[i] = -R + i * (2R/15), b4[i] = -R + (i + 0.5) * (2R/15), f32.
  // The centroids come from tqd::pqo_centroid, which the decode kernels
  // evaluate on the device, so both sides hold the same values.
  static const float b3[7] = {-1.7455f, -1.0385f, -0.4931f, 0.0f, 0.4931f, 1.0385f, 1.7455f};
  static const float b2[3] = {-1.0385f, 0.0f, 1.0385f};
  PqoCodebook cb;
  cb.bits = bits;
  const float range = 2.1573f;
  if (bits == 3) {
    cb.nc = 8;
    for (int i = 0; i < 8; i++) cb.c[i] = tqd::pqo_centroid<3>(i);
    std::memcpy(cb.b, b3, sizeof b3);
  } else if (bits == 4) {
    cb.nc = 16;
    for (int i = 0; i < 16; i++) cb.c[i] = tqd::pqo_centroid<4>(i);
    volatile float full = 2.0f * range;  // volatile: keep every f32 rounding step
    volatile float step = full / 15.0f;
    for (int i = 0; i < 15; i++) {
      volatile float k = (float)i + 0.5f;
      volatile float t = k * step;
      cb.b[i] = -range + t;
    }
  } else if (bits == 2) {
    cb.nc = 4;
    for (int i = 0; i < 4; i++) cb.c[i] = tqd::pqo_centroid<2>(i);
    std::memcpy(cb.b, b2, sizeof b2);
  } else {
    return cb;
  }
  float m = cb.c[0];
  for (int i = 1; i < cb.nc; i++) m = cb.c[i] > m ? cb.c[i] : m;
  cb.outer = m;
  return cb;
}

// get_codebook(bits, 32) as f32 (build_codebooks_l2, codebooks.rs:30-47)
static PqoCodebook l2_codebook(int bits) {
  PqoCodebook cb;
  const double *c = nullptr, *b = nullptr;
  int nc = 0;
  if (!core_codebook(bits, 32, &c, &b, &nc)) return cb;
  cb.bits = bits;
  cb.nc = nc;
  for (int i = 0; i < nc; i++) cb.c[i] = (float)c[i];
  for (int i = 0; i + 1 < nc; i++) cb.b[i] = (float)b[i];
  float m = cb.c[0];
  for (int i = 1; i < nc; i++) m = cb.c[i] > m ? cb.c[i] : m;
  cb.outer = m;
  return cb;
}

int polar_codec(int bits, int norm_mode, size_t outlier_blocks, int num_blocks, PolarCodec &codec) {
  if (bits != 3 && bits != 4) return fail(TQ_ERR_UNSUPPORTED_BITS, "unsupported bits=%d, expected 3 or 4", bits);
  if (norm_mode != TQ_NORM_MAXNORM && norm_mode != TQ_NORM_L2NORM)
    return fail(TQ_ERR_INVALID_ARGUMENT, "unknown norm mode %d", norm_mode);
  const bool all = outlier_blocks >= (size_t)num_blocks;
  codec.bits = bits;
  codec.norm_mode = norm_mode;
  codec.outlier = all;
  codec.mixed = !all && outlier_blocks != 0;
  codec.num_blocks = num_blocks;
  codec.eo = all ? num_blocks : (int)outlier_blocks;
  codec.cb_bits = all ? bits : bits - 1;
  if (norm_mode == TQ_NORM_MAXNORM) {
    codec.ocb = pqo_codebook(bits);  // outlier = polar_bits + 1 = bits (codebooks.rs:84-88)
    codec.ncb = pqo_codebook(bits - 1);
  } else {
    codec.ocb = l2_codebook(bits);
    codec.ncb = l2_codebook(bits - 1);
  }
  codec.cb = all ? codec.ocb : codec.ncb;
  codec.outer = codec.ocb.outer;
  codec.scale_sign = all ? -1.f : 1.f;  // build_scale_sign_tensor (precomputed/mod.rs:102-114)
  return TQ_OK;
}

static float next_up_host(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) == 0) u = 1u;
  else u = ((int32_t)u >= 0) ? u + 1u : u - 1u;
  float r;
  std::memcpy(&r, &u, 4);
  return r;
}

DivThresholds div_thresholds(const float *b, int nb, float outer) {
  DivThresholds t;
  t.nb = nb;
  for (int k = 0; k < nb; k++) {
    float up = next_up_host(b[k]);
    t.mu[k] = ((double)b[k] + (double)up) * 0.5;  // exact: both fit in 25 bits
    uint32_t u;
    std::memcpy(&u, &b[k], 4);
    if ((u & 1u) == 0) t.strict_mask |= 1u << k;
  }
  t.mul = (float)(1.0 / (double)outer);
  return t;
}

float inv_sqrt_dim(int dim) {
  volatile float fd = (float)dim;  // each step rounded to f32, as the reference's f32 arithmetic
  volatile float sq = sqrtf(fd);
  return 1.0f / sq;
}

}  // namespace tqh
