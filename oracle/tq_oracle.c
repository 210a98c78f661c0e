/*
 * tq_oracle.c -- CPU restatement of the TurboQuant reference algorithms.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels, never the thing
 * measured or shipped.  Loaded by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py through ctypes (oracle/oracle.py).
 *
 * Build: see oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math).
 *
 * Rust semantics restated here:
 *   - every f32 operation rounds once (no a*b+c contraction);
 *   - `iter().sum::<f32>()` is a left fold that starts from -0.0
 *     (core::iter::Sum for f32 in current Rust; a +0.0 start differs only in
 *     the sign of a sum whose every term is -0.0);
 *   - `x as f32` from f64 rounds to nearest-even;
 *   - f16/bf16 conversions are the `half` crate's, which round to
 *     nearest-even.
 */
#include "tq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define SUM_INIT (-0.0f)

/* ------------------------------------------------------------------------
 * IEEE binary16 / bfloat16 conversions
 * Pinned by tests/test_oracle_numerics.py against numpy.float16 over an
 * exhaustive sweep of f16 values and their rounding midpoints.
 * ---------------------------------------------------------------------- */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t tqo_f32_to_f16(float x)
{
    uint32_t u = f2u(x);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t exp = (u >> 23) & 0xffu;
    uint32_t man = u & 0x7fffffu;
    if (exp == 0xffu) {
        /* inf stays inf; NaN keeps its top payload bits and is made quiet */
        if (man == 0) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7c00u | 0x0200u | (man >> 13));
    }
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        /* result is subnormal (or zero): value = full_man * 2^(exp-150),
           f16 subnormal unit is 2^-24, so drop (126 - exp) bits */
        if (exp == 0) return (uint16_t)sign; /* f32 subnormals are < 2^-126 */
        uint32_t full = man | 0x800000u;
        int drop = 126 - (int)exp; /* >= 14 here */
        if (drop > 24) return (uint16_t)sign;
        uint32_t q = full >> drop;
        uint32_t rem = full & ((1u << drop) - 1u);
        uint32_t half = 1u << (drop - 1);
        if (rem > half || (rem == half && (q & 1u))) q += 1u;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1u; /* may carry into exp: correct */
    return (uint16_t)(sign | q);
}

float tqo_f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t man = (uint32_t)h & 0x3ffu;
    if (exp == 0x1fu) return u2f(sign | 0x7f800000u | (man << 13));
    if (exp == 0) {
        if (man == 0) return u2f(sign);
        /* subnormal: man * 2^-24, exact in f32 */
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t tqo_f32_to_bf16(float x)
{
    uint32_t u = f2u(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    uint32_t r = u + 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(r >> 16);
}

void tqo_f32_to_f16_batch(const float *x, size_t n, uint16_t *out)
{
    for (size_t i = 0; i < n; i++) out[i] = tqo_f32_to_f16(x[i]);
}

void tqo_f16_to_f32_batch(const uint16_t *h, size_t n, float *out)
{
    for (size_t i = 0; i < n; i++) out[i] = tqo_f16_to_f32(h[i]);
}

/* ------------------------------------------------------------------------
 * Rotation -- src/rotation.rs
 * ---------------------------------------------------------------------- */

/* src/packed/mod.rs:112-114 */
int tqo_is_valid_dim(size_t dim) { return dim > 0 && (dim & (dim - 1)) == 0; }

/* src/rotation.rs:47-70: s_i = +1 if ((seed+i)*GOLDEN) is even.
   Pin: the multiplier is odd, so s_i = (-1)^(seed+i) (closed form). */
void tqo_generate_sign_pattern(size_t dim, uint64_t seed, float *out)
{
    const uint64_t golden = 0x9E3779B97F4A7C15ull;
    for (size_t i = 0; i < dim; i++) {
        uint64_t h = (seed + (uint64_t)i) * golden;
        out[i] = (h & 1u) == 0 ? 1.0f : -1.0f;
    }
}

/* Unnormalized Sylvester butterflies, h = 1, 2, ..., n/2 (rotation.rs:24-35). */
static void butterfly(float *d, size_t n)
{
    for (size_t h = 1; h < n; h *= 2)
        for (size_t i = 0; i < n; i += 2 * h)
            for (size_t j = i; j < i + h; j++) {
                float x = d[j], y = d[j + h];
                d[j] = x + y;
                d[j + h] = x - y;
            }
}

/* src/rotation.rs:22-40.  Pins: [1,1,1,1] -> [2,0,0,0] (rotation.rs:236-245),
   equality with a from-scratch Hadamard matrix product, self-inverse. */
void tqo_wht_inplace(float *data, size_t n)
{
    butterfly(data, n);
    float norm = 1.0f / sqrtf((float)n);
    for (size_t i = 0; i < n; i++) data[i] *= norm;
}

/* src/rotation.rs:137-150 (Forward = sign then WHT; Inverse = WHT then sign). */
int tqo_rotate(float *data, const float *signs, size_t n, size_t sign_len, int inverse)
{
    if (!tqo_is_valid_dim(n)) return TQO_ERR_INVALID_DIMENSION;
    if (n != sign_len) return TQO_ERR_DIMENSION_MISMATCH;
    if (!inverse) {
        for (size_t i = 0; i < n; i++) data[i] *= signs[i];
        tqo_wht_inplace(data, n);
    } else {
        tqo_wht_inplace(data, n);
        for (size_t i = 0; i < n; i++) data[i] *= signs[i];
    }
    return TQO_OK;
}

/* ------------------------------------------------------------------------
 * Codebooks -- src/codebook/tables.rs:110-377 (data), mod.rs:66-122 (lookup)
 * The tables are the reference's data, restated value for value: the codes
 * produced depend on every bit of them.  Pinned by an independent Lloyd-Max
 * solve of the Beta pdf (tests/test_oracle_codebooks.py, within 1e-6, as the
 * reference's own codebook_tests.rs:256-281 does against its generator).
 * ---------------------------------------------------------------------- */

static const double C2_32[4] = {-0.2633194690486469, -0.07980195923950476, 0.07980195923950384, 0.2633194690486451};
static const double B2_32[3] = {-0.1715607141440758, 0.0, 0.17156071414407448};
static const double C3_32[8] = {-0.3662684197149945, -0.2324607608635176, -0.13175624361004853, -0.042851570066700616,
                                0.04285157006670112, 0.1317562436100487, 0.23246076086351877, 0.36626841971499513};
static const double B3_32[7] = {-0.29936459028925605, -0.18210850223678307, -0.08730390683837458, 0.0,
                                0.08730390683837491, 0.18210850223678374, 0.29936459028925694};
static const double C4_32[16] = {-0.45356484406403885, -0.3500919292405678, -0.276742371576412, -0.2163621312970215,
                                 -0.16307095286109716, -0.11401417528619187, -0.06749924527967034, -0.02235501645565892,
                                 0.022355016455658717, 0.06749924527967022, 0.11401417528619151, 0.16307095286109707,
                                 0.21636213129702167, 0.27674237157641146, 0.35009192924056776, 0.4535648440640396};
static const double B4_32[15] = {-0.40182838665230336, -0.31341715040848994, -0.24655225143671677, -0.18971654207905933,
                                 -0.13854256407364451, -0.09075671028293111, -0.04492713086766463, 0.0,
                                 0.044927130867664464, 0.09075671028293086, 0.1385425640736443, 0.18971654207905936,
                                 0.24655225143671655, 0.3134171504084896, 0.4018283866523037};
static const double C2_64[4] = {-0.18749689292196112, -0.05651489047635318, 0.05651489047635313, 0.18749689292196103};
static const double B2_64[3] = {-0.12200589169915715, 0.0, 0.12200589169915708};
static const double C2_128[4] = {-0.13304154846077318, -0.03999160906335877, 0.03999160906335891, 0.13304154846077348};
static const double B2_128[3] = {-0.08651657876206598, 0.0, 0.0865165787620662};
static const double C2_256[4] = {-0.09423779913129633, -0.02828860721372146, 0.02828860721372166, 0.09423779913129664};
static const double B2_256[3] = {-0.0612632031725089, 0.0, 0.06126320317250915};
static const double C3_64[8] = {-0.26391407457137683, -0.16616801009118487, -0.0938323758441605, -0.03046922045737837,
                                0.03046922045737837, 0.0938323758441605, 0.16616801009118487, 0.26391407457137683};
static const double B3_64[7] = {-0.21504104233128085, -0.13000019296767268, -0.06215079815076943, 0.0,
                                0.06215079815076943, 0.13000019296767268, 0.21504104233128085};
static const double C3_128[8] = {-0.18839728518004373, -0.11813986946554235, -0.06658568378325364, -0.02160433847349997,
                                 0.02160433847349997, 0.06658568378325364, 0.11813986946554235, 0.18839728518004373};
static const double B3_128[7] = {-0.15326857732279303, -0.09236277662439799, -0.0440950111283768, 0.0,
                                 0.0440950111283768, 0.09236277662439799, 0.15326857732279303};
static const double C3_256[8] = {-0.13385436276083063, -0.0837655314597689, -0.04716676527922715, -0.01529750782483941,
                                 0.01529750782483941, 0.04716676527922715, 0.0837655314597689, 0.13385436276083063};
static const double B3_256[7] = {-0.10880994711029976, -0.06546614836949802, -0.03123213655203328, 0.0,
                                 0.03123213655203328, 0.06546614836949802, 0.10880994711029976};
static const double C4_64[16] = {-0.33092994168409773, -0.25307088610074774, -0.19901983361887085, -0.15508179062990365,
                                 -0.11662310388676207, -0.08141753279040376, -0.04815672368589858, -0.0159419303520814,
                                 0.0159419303520814, 0.04815672368589858, 0.08141753279040376, 0.11662310388676207,
                                 0.15508179062990365, 0.19901983361887085, 0.25307088610074774, 0.33092994168409773};
static const double B4_64[15] = {-0.2920004138924227, -0.22604535985980928, -0.17705081212438725, -0.13585244725833287,
                                 -0.09902031833858291, -0.06478712823815116, -0.03204932701898999, 0.0,
                                 0.03204932701898999, 0.06478712823815116, 0.09902031833858291, 0.13585244725833287,
                                 0.17705081212438725, 0.22604535985980928, 0.2920004138924227};
static const double C4_128[16] = {-0.23777655506958537, -0.18096588552769086, -0.14193912272806147, -0.11041538921898804,
                                  -0.08293881469006784, -0.05785765497830671, -0.03420549908335103, -0.01132093590150223,
                                  0.01132093590150223, 0.03420549908335103, 0.05785765497830671, 0.08293881469006784,
                                  0.11041538921898804, 0.14193912272806147, 0.18096588552769086, 0.23777655506958537};
static const double B4_128[15] = {-0.2093712202986381, -0.16145250412787615, -0.12617725597352475, -0.09667710195452794,
                                  -0.07039823483418728, -0.04603157703082887, -0.02276321749242663, 0.0,
                                  0.02276321749242663, 0.04603157703082887, 0.07039823483418728, 0.09667710195452794,
                                  0.12617725597352475, 0.16145250412787615, 0.2093712202986381};
static const double C4_256[16] = {-0.16949853314441155, -0.12868871755030106, -0.10080108457584613, -0.07834675699488723,
                                  -0.05881658417438018, -0.04101444098641885, -0.02424206232116148, -0.00802245010411462,
                                  0.00802245010411462, 0.02424206232116148, 0.04101444098641885, 0.05881658417438018,
                                  0.07834675699488723, 0.10080108457584613, 0.12868871755030106, 0.16949853314441155};
static const double B4_256[15] = {-0.14909362534735632, -0.1147449010630736, -0.08957392078536669, -0.06858167058463371,
                                  -0.04991551258039952, -0.03262825165379016, -0.01613225621263805, 0.0,
                                  0.01613225621263805, 0.03262825165379016, 0.04991551258039952, 0.06858167058463371,
                                  0.08957392078536669, 0.1147449010630736, 0.14909362534735632};

/* src/codebook/mod.rs:118-122 + tables.rs:89-105.  Dimensions outside the
   static tables fall back to the Lloyd-Max generator in the reference
   (codebook/gen.rs), which is outside this path: reported as
   TQO_ERR_INVALID_DIMENSION here. */
int tqo_get_codebook(int bits, size_t dim, const double **c, const double **b, int *nc)
{
    if (bits < 2 || bits > 4) return TQO_ERR_UNSUPPORTED_BITS;
    const double *cc = NULL, *bb = NULL;
#define CB(BI, D) if (bits == BI && dim == D) { cc = C##BI##_##D; bb = B##BI##_##D; }
    CB(2, 32) CB(2, 64) CB(2, 128) CB(2, 256)
    CB(3, 32) CB(3, 64) CB(3, 128) CB(3, 256)
    CB(4, 32) CB(4, 64) CB(4, 128) CB(4, 256)
#undef CB
    if (!cc) return TQO_ERR_INVALID_DIMENSION;
    *c = cc;
    *b = bb;
    *nc = 1 << bits;
    return TQO_OK;
}

/* src/codebook/mod.rs:66-78: lower-bound binary search with strict `>`. */
uint8_t tqo_nearest_centroid(double value, const double *boundaries, int nb)
{
    int lo = 0, hi = nb;
    while (lo < hi) {
        int mid = lo + (hi - lo) / 2;
        if (value > boundaries[mid]) lo = mid + 1;
        else hi = mid;
    }
    return (uint8_t)lo;
}

/* ------------------------------------------------------------------------
 * Bit packing -- src/packed/mod.rs:242-309, indices.rs:152-281
 * LSB-first bitstream: index i occupies bits [i*b, i*b+b).  Tails are
 * zero-padded to whole groups (4 for 2-bit, 8 for 3-bit, 2 for 4-bit).
 * Pins: the reference's exhaustive pack/unpack tests and the closed form.
 * ---------------------------------------------------------------------- */

size_t tqo_packed_len(int bits, size_t count)
{
    switch (bits) {
    case 2: return (count + 3) / 4;
    case 3: return ((count + 7) / 8) * 3;
    case 4: return (count + 1) / 2;
    default: return 0;
    }
}

size_t tqo_pack_indices(int bits, const uint8_t *idx, size_t count, uint8_t *out)
{
    size_t len = tqo_packed_len(bits, count);
    size_t groups = (bits == 3) ? (count + 7) / 8 : 0;
    if (bits == 2) {
        for (size_t byte = 0; byte < len; byte++) {
            uint8_t v = 0;
            for (int k = 0; k < 4; k++) {
                size_t i = byte * 4 + (size_t)k;
                uint8_t x = i < count ? (idx[i] & 3u) : 0;
                v |= (uint8_t)(x << (2 * k));
            }
            out[byte] = v;
        }
    } else if (bits == 3) {
        /* pack_3bit, packed/mod.rs:266-279 */
        for (size_t g = 0; g < groups; g++) {
            uint8_t v[8];
            for (int k = 0; k < 8; k++) {
                size_t i = g * 8 + (size_t)k;
                v[k] = i < count ? idx[i] : 0;
            }
            out[3 * g + 0] = (uint8_t)((v[0] & 7u) | ((v[1] & 7u) << 3) | ((v[2] & 3u) << 6));
            out[3 * g + 1] = (uint8_t)(((v[2] >> 2) & 1u) | ((v[3] & 7u) << 1) | ((v[4] & 7u) << 4) |
                                       ((v[5] & 1u) << 7));
            out[3 * g + 2] = (uint8_t)(((v[5] >> 1) & 3u) | ((v[6] & 7u) << 2) | ((v[7] & 7u) << 5));
        }
    } else if (bits == 4) {
        for (size_t byte = 0; byte < len; byte++) {
            size_t i = byte * 2;
            uint8_t lo = idx[i] & 15u;
            uint8_t hi = (i + 1 < count) ? (idx[i + 1] & 15u) : 0;
            out[byte] = (uint8_t)(lo | (hi << 4));
        }
    }
    return len;
}

void tqo_unpack_indices(int bits, const uint8_t *packed, size_t packed_len, size_t count, uint8_t *out)
{
    size_t produced = 0;
    if (bits == 2) {
        for (size_t b = 0; b < packed_len && produced < count; b++)
            for (int k = 0; k < 4 && produced < count; k++) out[produced++] = (packed[b] >> (2 * k)) & 3u;
    } else if (bits == 3) {
        /* unpack_3bit over whole 3-byte chunks (indices.rs:238-249) */
        for (size_t g = 0; g + 3 <= packed_len && produced < count; g += 3) {
            uint8_t p0 = packed[g], p1 = packed[g + 1], p2 = packed[g + 2];
            uint8_t v[8];
            v[0] = p0 & 7u;
            v[1] = (p0 >> 3) & 7u;
            v[2] = (uint8_t)(((p0 >> 6) & 3u) | ((p1 & 1u) << 2));
            v[3] = (p1 >> 1) & 7u;
            v[4] = (p1 >> 4) & 7u;
            v[5] = (uint8_t)(((p1 >> 7) & 1u) | ((p2 & 3u) << 1));
            v[6] = (p2 >> 2) & 7u;
            v[7] = (p2 >> 5) & 7u;
            for (int k = 0; k < 8 && produced < count; k++) out[produced++] = v[k];
        }
    } else if (bits == 4) {
        for (size_t b = 0; b < packed_len && produced < count; b++)
            for (int k = 0; k < 2 && produced < count; k++) out[produced++] = (packed[b] >> (4 * k)) & 15u;
    }
    /* the reference truncates; a short input leaves the rest untouched */
}

/* ------------------------------------------------------------------------
 * Core full-vector codec -- src/quantize.rs
 * ---------------------------------------------------------------------- */

#define MIN_NORM 1e-10f

/* quantize.rs:51-53: sequential f32 sum of squares, sqrtf. */
float tqo_l2_norm(const float *x, size_t n)
{
    float s = SUM_INIT;
    for (size_t i = 0; i < n; i++) s += x[i] * x[i];
    return sqrtf(s);
}

/* quantize.rs:174-192 (quantize_vec_with_codebook) */
static void quantize_core(int bits, size_t dim, const float *signs, const double *bnd, int nb,
                          const float *data, uint8_t *packed_out, uint16_t *scale_out, float *work,
                          uint8_t *idx)
{
    float norm = tqo_l2_norm(data, dim);
    /* normalize_inplace, quantize.rs:60-71 */
    if (norm < MIN_NORM) {
        for (size_t i = 0; i < dim; i++) work[i] = 0.0f;
    } else {
        float inv = 1.0f / norm;
        for (size_t i = 0; i < dim; i++) work[i] = data[i] * inv;
    }
    tqo_rotate(work, signs, dim, dim, 0);
    for (size_t i = 0; i < dim; i++) idx[i] = tqo_nearest_centroid((double)work[i], bnd, nb);
    /* select_scale, quantize.rs:123-126 */
    *scale_out = tqo_f32_to_f16(norm < MIN_NORM ? 0.0f : norm);
    tqo_pack_indices(bits, idx, dim, packed_out);
}

/* quantize.rs:225-240 (dequantize_vec_with_codebook) */
static void dequantize_core(int bits, size_t dim, const float *signs, const double *cen,
                            const uint8_t *packed, uint16_t scale, float *out, uint8_t *idx)
{
    tqo_unpack_indices(bits, packed, tqo_packed_len(bits, dim), dim, idx);
    for (size_t i = 0; i < dim; i++) out[i] = (float)cen[idx[i]];
    tqo_rotate(out, signs, dim, dim, 1);
    float s = tqo_f16_to_f32(scale);
    for (size_t i = 0; i < dim; i++) out[i] *= s;
}

static int check_cfg(int bits, size_t dim)
{
    if (bits < 2 || bits > 4) return TQO_ERR_UNSUPPORTED_BITS;
    if (!tqo_is_valid_dim(dim)) return TQO_ERR_INVALID_DIMENSION;
    return TQO_OK;
}

int tqo_quantize_vec_batch(int bits, size_t dim, uint64_t seed, size_t n, const float *data,
                           uint8_t *packed_out, uint16_t *scales_out)
{
    int rc = check_cfg(bits, dim);
    if (rc) return rc;
    const double *c, *b;
    int nc;
    rc = tqo_get_codebook(bits, dim, &c, &b, &nc);
    if (rc) return rc;
    float *signs = malloc(dim * sizeof(float));
    float *work = malloc(dim * sizeof(float));
    uint8_t *idx = malloc(dim);
    tqo_generate_sign_pattern(dim, seed, signs);
    size_t plen = tqo_packed_len(bits, dim);
    for (size_t v = 0; v < n; v++)
        quantize_core(bits, dim, signs, b, nc - 1, data + v * dim, packed_out + v * plen, scales_out + v,
                      work, idx);
    free(signs);
    free(work);
    free(idx);
    return TQO_OK;
}

int tqo_dequantize_vec_batch(int bits, size_t dim, uint64_t seed, size_t n, const uint8_t *packed,
                             const uint16_t *scales, float *out)
{
    int rc = check_cfg(bits, dim);
    if (rc) return rc;
    const double *c, *b;
    int nc;
    rc = tqo_get_codebook(bits, dim, &c, &b, &nc);
    if (rc) return rc;
    float *signs = malloc(dim * sizeof(float));
    uint8_t *idx = malloc(dim);
    tqo_generate_sign_pattern(dim, seed, signs);
    size_t plen = tqo_packed_len(bits, dim);
    for (size_t v = 0; v < n; v++)
        dequantize_core(bits, dim, signs, c, packed + v * plen, scales[v], out + v * dim, idx);
    free(signs);
    free(idx);
    return TQO_OK;
}

/* quantize.rs:142-157 */
int tqo_quantize_vec(int bits, size_t dim, uint64_t seed, const float *data, uint8_t *packed_out,
                     uint16_t *scale_out)
{
    return tqo_quantize_vec_batch(bits, dim, seed, 1, data, packed_out, scale_out);
}

/* quantize.rs:207-211 */
int tqo_dequantize_vec(int bits, size_t dim, uint64_t seed, const uint8_t *packed, uint16_t scale,
                       float *out)
{
    return tqo_dequantize_vec_batch(bits, dim, seed, 1, packed, &scale, out);
}

/* quantize.rs:306-316: centroid lookup and scale, no inverse rotation. */
int tqo_dequantize_rotated(int bits, size_t dim, const uint8_t *packed, uint16_t scale, float *out)
{
    int rc = check_cfg(bits, dim);
    if (rc) return rc;
    const double *c, *b;
    int nc;
    rc = tqo_get_codebook(bits, dim, &c, &b, &nc);
    if (rc) return rc;
    uint8_t *idx = malloc(dim);
    tqo_unpack_indices(bits, packed, tqo_packed_len(bits, dim), dim, idx);
    float s = tqo_f16_to_f32(scale);
    for (size_t i = 0; i < dim; i++) out[i] = (float)c[idx[i]] * s;
    free(idx);
    return TQO_OK;
}

/* ------------------------------------------------------------------------
 * PQO cache codec (MaxNorm, all blocks outlier)
 * ---------------------------------------------------------------------- */

#define QBLOCK 32

/* precomputed/codebooks.rs:51-88.  3-bit: literal llama.cpp table.  4-bit:
   f32 arithmetic c4[i] = -R + i*(2R/15), b4[i] = -R + (i+0.5)*(2R/15).
   outer_centroid = max(outlier centroids) (precomputed/mod.rs:78).
   Pins: symmetry/monotonicity and the literal values (tests). */
int tqo_pqo_codebook(int bits, float *c, float *b, int *nc, float *outer)
{
    static const float c3[8] = {-2.1573f, -1.3336f, -0.7434f, -0.2428f, 0.2428f, 0.7434f, 1.3336f, 2.1573f};
    static const float b3[7] = {-1.7455f, -1.0385f, -0.4931f, 0.0f, 0.4931f, 1.0385f, 1.7455f};
    static const float c2[4] = {-2.1573f, -0.7434f, 0.7434f, 2.1573f};
    static const float b2[3] = {-1.0385f, 0.0f, 1.0385f};
    const float range = 2.1573f;
    if (bits == 3) {
        memcpy(c, c3, sizeof c3);
        memcpy(b, b3, sizeof b3);
        *nc = 8;
    } else if (bits == 4) {
        float full = 2.0f * range;
        float step = full / 15.0f;
        for (int i = 0; i < 16; i++) c[i] = -range + (float)i * step;
        for (int i = 0; i < 15; i++) b[i] = -range + ((float)i + 0.5f) * step;
        *nc = 16;
    } else if (bits == 2) {
        memcpy(c, c2, sizeof c2);
        memcpy(b, b2, sizeof b2);
        *nc = 4;
    } else {
        return TQO_ERR_UNSUPPORTED_BITS;
    }
    float m = c[0];
    for (int i = 1; i < *nc; i++) m = c[i] > m ? c[i] : m;
    *outer = m;
    return TQO_OK;
}

/* precomputed/rotation.rs:17-20: the 32-entry sign pattern. */
void tqo_pqo_sign32(float *out)
{
    static const float s[32] = {1, -1, 1, 1, -1, -1, 1, -1, 1, 1, -1, 1, -1, 1, -1, -1,
                                1, -1, -1, 1, 1, -1, 1, -1, -1, 1, 1, 1, -1, -1, 1, -1};
    memcpy(out, s, sizeof s);
}

/* wht_tensor.rs:27-41: the inverse's sign factor is fl(R_fwd[0][j] * sqrt(32))
   with R_fwd[0][j] = fl(1/sqrt(32)) * s_j, i.e. +/-0.99999994. */
void tqo_pqo_decode_signs(float *out)
{
    float s[32];
    tqo_pqo_sign32(s);
    float sq = sqrtf(32.0f);
    float norm = 1.0f / sq;
    for (int j = 0; j < 32; j++) out[j] = (norm * s[j]) * sq;
}

/* Forward block rotation r = x @ R_fwd, R_fwd = H32/sqrt(32) * diag(s)
   (precomputed/rotation.rs:26, quantize_tensor.rs:104).  Evaluated as the
   butterfly of x, one multiply by fl(1/sqrt(32)), then the sign: the same
   value as the matrix product in exact arithmetic.  The reference's own
   f32 rounding here is candle's gemm summation order, which is not pinned
   (not visible from the reference sources); tqo_pqo_rotate_block_gemm is
   the dot-product order for comparison. */
void tqo_pqo_rotate_block(const float *x, float *r)
{
    float s[32];
    tqo_pqo_sign32(s);
    float w[32];
    memcpy(w, x, sizeof w);
    butterfly(w, 32);
    float c = 1.0f / sqrtf(32.0f);
    for (int j = 0; j < 32; j++) r[j] = (w[j] * c) * s[j];
}

void tqo_pqo_rotate_block_gemm(const float *x, float *r)
{
    float s[32];
    tqo_pqo_sign32(s);
    float c = 1.0f / sqrtf(32.0f);
    for (int j = 0; j < 32; j++) {
        float acc = SUM_INIT;
        for (int i = 0; i < 32; i++) {
            /* Sylvester H[i][j] = (-1)^popcount(i&j) */
            float h = (__builtin_popcount((unsigned)(i & j)) & 1) ? -c : c;
            acc += x[i] * (h * s[j]);
        }
        r[j] = acc;
    }
}

/* The same product as one fused multiply-add chain per output, k = 0..31 in
   order from +0: the accumulation a K=32 gemm microkernel on FMA hardware
   most plausibly performs for quantize_tensor.rs:100,104 (candle's CPU
   matmul; its order is not in the reference tree). */
void tqo_pqo_rotate_block_fma(const float *x, float *r)
{
    float s[32];
    tqo_pqo_sign32(s);
    float c = 1.0f / sqrtf(32.0f);
    for (int j = 0; j < 32; j++) {
        float acc = 0.0f;
        for (int i = 0; i < 32; i++) {
            float h = (__builtin_popcount((unsigned)(i & j)) & 1) ? -c : c;
            acc = fmaf(x[i], h * s[j], acc);
        }
        r[j] = acc;
    }
}

/* n blocks of 32 in one of the orders above: 0 butterfly, 1 separately
   rounded dot products, 2 fused multiply-add chains. */
int tqo_pqo_rotate_blocks(int order, size_t n, const float *x, float *r)
{
    if (order < 0 || order > 2) return TQO_ERR_INVALID_ARGUMENT;
    for (size_t b = 0; b < n; b++) {
        if (order == 0) tqo_pqo_rotate_block(x + 32 * b, r + 32 * b);
        else if (order == 1) tqo_pqo_rotate_block_gemm(x + 32 * b, r + 32 * b);
        else tqo_pqo_rotate_block_fma(x + 32 * b, r + 32 * b);
    }
    return TQO_OK;
}

/* quantize_tensor.rs:103-110 (MaxNorm scale), :161-176 (bucketize),
   :68-70 (signed f16 scale), :264-274 (packing); the same contract as the
   reference kernel entry tq_quant_maxnorm_batch (ffi.rs:24-37).
   scale = max(amax * fl(1/outer_c), 1e-10): candle evaluates
   `tensor / f64` as affine(1/rhs, 0), i.e. a multiply by the f32-rounded
   reciprocal (parity unpinned: candle is not in the reference tree). */
static int pqo_quantize_rotated_cb(int bits, size_t num_blocks, const float *rotated, const float *bnd,
                                   int nb, float outer, uint8_t *packed_out, uint16_t *scales_out,
                                   float scale_sign)
{
    const float mul = (float)(1.0 / (double)outer);
    size_t bpb = (size_t)QBLOCK * (size_t)bits / 8;
    uint8_t idx[QBLOCK];
    for (size_t blk = 0; blk < num_blocks; blk++) {
        const float *r = rotated + blk * QBLOCK;
        float amax = 0.0f;
        for (int j = 0; j < QBLOCK; j++) {
            float a = fabsf(r[j]);
            amax = a > amax ? a : amax;
        }
        float s = amax * mul;
        if (s < MIN_NORM) s = MIN_NORM;
        for (int j = 0; j < QBLOCK; j++) {
            float v = r[j] / s;
            int k = 0;
            for (int t = 0; t < nb; t++) k += v > bnd[t];
            idx[j] = (uint8_t)k;
        }
        scales_out[blk] = tqo_f32_to_f16(s * scale_sign);
        tqo_pack_indices(bits, idx, QBLOCK, packed_out + blk * bpb);
    }
    return TQO_OK;
}

int tqo_pqo_quantize_rotated(int bits, size_t num_blocks, const float *rotated, uint8_t *packed_out,
                             uint16_t *scales_out, float scale_sign)
{
    float c[16], b[15], outer;
    int nc;
    int rc = tqo_pqo_codebook(bits, c, b, &nc, &outer);
    if (rc) return rc;
    return pqo_quantize_rotated_cb(bits, num_blocks, rotated, b, nc - 1, outer, packed_out, scales_out,
                                   scale_sign);
}

/* polar_quantize, MaxNorm + PQO (quantize_tensor.rs:40-76). */
int tqo_pqo_quantize(int bits, size_t n, size_t head_dim, const float *x, uint8_t *packed_out,
                     uint16_t *scales_out)
{
    if (head_dim % QBLOCK != 0 || head_dim == 0) return TQO_ERR_INVALID_ARGUMENT;
    if (bits != 3 && bits != 4) return TQO_ERR_UNSUPPORTED_BITS;
    size_t nblk = n * (head_dim / QBLOCK);
    float *rot = malloc(nblk * QBLOCK * sizeof(float));
    for (size_t blk = 0; blk < nblk; blk++) tqo_pqo_rotate_block(x + blk * QBLOCK, rot + blk * QBLOCK);
    int rc = tqo_pqo_quantize_rotated(bits, nblk, rot, packed_out, scales_out, -1.0f);
    free(rot);
    return rc;
}

/* polar_dequantize CPU branch (quantize_tensor.rs:197-219) with
   butterfly_wht_inverse_cpu (wht_tensor.rs:15-68). */
int tqo_pqo_dequantize(int bits, size_t n, size_t head_dim, const uint8_t *packed, const uint16_t *scales,
                       float *out)
{
    if (head_dim % QBLOCK != 0 || head_dim == 0) return TQO_ERR_INVALID_ARGUMENT;
    float c[16], b[15], outer;
    int nc;
    int rc = tqo_pqo_codebook(bits, c, b, &nc, &outer);
    if (rc) return rc;
    float sg[32];
    tqo_pqo_decode_signs(sg);
    const float inv = 1.0f / sqrtf(32.0f);
    size_t bpb = (size_t)QBLOCK * (size_t)bits / 8;
    size_t nblk = n * (head_dim / QBLOCK);
    uint8_t idx[QBLOCK];
    for (size_t blk = 0; blk < nblk; blk++) {
        tqo_unpack_indices(bits, packed + blk * bpb, bpb, QBLOCK, idx);
        float *o = out + blk * QBLOCK;
        for (int j = 0; j < QBLOCK; j++) o[j] = c[idx[j]] * sg[j];
        butterfly(o, QBLOCK);
        float s = fabsf(tqo_f16_to_f32(scales[blk]));
        for (int j = 0; j < QBLOCK; j++) o[j] = (o[j] * inv) * s;
    }
    return TQO_OK;
}

/* polar_quantize for the cache modes (quantize_tensor.rs:40-76): the
   MaxNorm scale divides by the outlier codebook's largest centroid
   (precomputed/mod.rs:78); bucketize_blocks (:118-150) sends the first
   n * min(outlier_blocks, nb) rows of the [n * nb, 32] block matrix to the
   outlier boundaries and the rest to the standard (bits - 1)-bit ones; the
   scale sign is -1 for the first min(outlier_blocks, nb) blocks of every
   vector (build_scale_sign_tensor, precomputed/mod.rs:102-114); codes are
   packed bits-wide (:73).  For outlier_blocks 0 or >= nb the two
   orderings agree.  norm_mode 1 (L2Norm, :90-101): the block's norm
   sqrt(sum x^2) (element order from +0, clamped to 1e-10) divides it before
   the rotation and is its scale; the codebooks are get_codebook(b, 32) in
   f32 (codebooks.rs:30-47). */
static void polar_codebooks(int bits, int norm_mode, float *oc, float *ob, int *onc, float *nc_, float *nb_,
                            int *nnc, float *outer)
{
    float outer_n;
    if (norm_mode == 0) {
        tqo_pqo_codebook(bits, oc, ob, onc, outer);
        tqo_pqo_codebook(bits - 1, nc_, nb_, nnc, &outer_n);
        return;
    }
    const double *c, *b;
    tqo_get_codebook(bits, 32, &c, &b, onc);
    for (int i = 0; i < *onc; i++) oc[i] = (float)c[i];
    for (int i = 0; i + 1 < *onc; i++) ob[i] = (float)b[i];
    tqo_get_codebook(bits - 1, 32, &c, &b, nnc);
    for (int i = 0; i < *nnc; i++) nc_[i] = (float)c[i];
    for (int i = 0; i + 1 < *nnc; i++) nb_[i] = (float)b[i];
    *outer = oc[*onc - 1];
}

int tqo_polar_quantize(int bits, size_t outlier_blocks, int norm_mode, size_t n, size_t head_dim, const float *x,
                       uint8_t *packed_out, uint16_t *scales_out)
{
    if (head_dim % QBLOCK != 0 || head_dim == 0) return TQO_ERR_INVALID_ARGUMENT;
    if (bits != 3 && bits != 4) return TQO_ERR_UNSUPPORTED_BITS;
    if (norm_mode != 0 && norm_mode != 1) return TQO_ERR_INVALID_ARGUMENT;
    float oc[16], ob[15], nc_[16], nb_[15], outer;
    int onc, nnc;
    polar_codebooks(bits, norm_mode, oc, ob, &onc, nc_, nb_, &nnc, &outer);
    const size_t nblk_v = head_dim / QBLOCK;
    const size_t eo = outlier_blocks < nblk_v ? outlier_blocks : nblk_v;
    const size_t rows = n * nblk_v, outlier_rows = n * eo;
    const float mul = (float)(1.0 / (double)outer);
    const size_t bpb = (size_t)QBLOCK * (size_t)bits / 8;
    float r[QBLOCK];
    uint8_t idx[QBLOCK];
    for (size_t row = 0; row < rows; row++) {
        float s;
        if (norm_mode == 1) {
            const float *xb = x + row * QBLOCK;
            float ss = 0.0f;
            for (int j = 0; j < QBLOCK; j++) ss = ss + xb[j] * xb[j];
            s = sqrtf(ss);
            if (s < MIN_NORM) s = MIN_NORM;
            float xn[QBLOCK];
            for (int j = 0; j < QBLOCK; j++) xn[j] = xb[j] / s;
            tqo_pqo_rotate_block(xn, r);
        } else {
            tqo_pqo_rotate_block(x + row * QBLOCK, r);
            float amax = 0.0f;
            for (int j = 0; j < QBLOCK; j++) {
                float a = fabsf(r[j]);
                amax = a > amax ? a : amax;
            }
            s = amax * mul;
            if (s < MIN_NORM) s = MIN_NORM;
        }
        const int outlier_row = row < outlier_rows;
        const float *bnd = outlier_row ? ob : nb_;
        const int nbnd = outlier_row ? onc - 1 : nnc - 1;
        for (int j = 0; j < QBLOCK; j++) {
            float v = norm_mode == 1 ? r[j] : r[j] / s;
            int k = 0;
            for (int t = 0; t < nbnd; t++) k += v > bnd[t];
            idx[j] = (uint8_t)k;
        }
        const float sign = (row % nblk_v) < eo ? -1.0f : 1.0f;
        scales_out[row] = tqo_f32_to_f16(s * sign);
        tqo_pack_indices(bits, idx, QBLOCK, packed_out + row * bpb);
    }
    return TQO_OK;
}

/* polar_dequantize CPU branch (quantize_tensor.rs:197-261): codebook_lookup
   picks the outlier centroids for all-outlier configs, the standard ones
   for outlier_blocks 0, and per block by the scale's sign otherwise (with
   the index clamped into the standard codebook, :242-260). */
int tqo_polar_dequantize(int bits, size_t outlier_blocks, int norm_mode, size_t n, size_t head_dim,
                         const uint8_t *packed, const uint16_t *scales, float *out)
{
    if (head_dim % QBLOCK != 0 || head_dim == 0) return TQO_ERR_INVALID_ARGUMENT;
    if (bits != 3 && bits != 4) return TQO_ERR_UNSUPPORTED_BITS;
    if (norm_mode != 0 && norm_mode != 1) return TQO_ERR_INVALID_ARGUMENT;
    float oc[16], ob[15], ncb[16], nbb[15], outer;
    int onc, nnc;
    polar_codebooks(bits, norm_mode, oc, ob, &onc, ncb, nbb, &nnc, &outer);
    const size_t nblk_v = head_dim / QBLOCK;
    float sg[32];
    tqo_pqo_decode_signs(sg);
    const float inv = 1.0f / sqrtf(32.0f);
    const size_t bpb = (size_t)QBLOCK * (size_t)bits / 8;
    const size_t nblk = n * nblk_v;
    uint8_t idx[QBLOCK];
    for (size_t blk = 0; blk < nblk; blk++) {
        tqo_unpack_indices(bits, packed + blk * bpb, bpb, QBLOCK, idx);
        const float sc = tqo_f16_to_f32(scales[blk]);
        float *o = out + blk * QBLOCK;
        for (int j = 0; j < QBLOCK; j++) {
            float c;
            if (outlier_blocks >= nblk_v) c = oc[idx[j]];
            else if (outlier_blocks == 0) c = ncb[idx[j]];
            else c = sc < 0.0f ? oc[idx[j]] : ncb[idx[j] < nnc ? idx[j] : nnc - 1];
            o[j] = c * sg[j];
        }
        butterfly(o, QBLOCK);
        float s = fabsf(sc);
        for (int j = 0; j < QBLOCK; j++) o[j] = (o[j] * inv) * s;
    }
    return TQO_OK;
}

/* compute_qjl_signs_and_norms (tq.rs:373-412): residual r = x - x_hat,
   norm = f16(sqrt(sum r^2)) (candle sqr, sum_keepdim, sqrt: the sum in
   element order from +0), signs = compute_qjl_signs(r, d, DEFAULT_QJL_SEED
   = 12345). */
int tqo_tq_signs_norms(size_t n, size_t head_dim, const float *x, const float *xhat, uint8_t *signs,
                       uint16_t *norms)
{
    float *r = malloc(head_dim * sizeof(float));
    for (size_t v = 0; v < n; v++) {
        float ss = 0.0f;
        for (size_t e = 0; e < head_dim; e++) {
            r[e] = x[v * head_dim + e] - xhat[v * head_dim + e];
            ss = ss + r[e] * r[e];
        }
        norms[v] = tqo_f32_to_f16(sqrtf(ss));
        int rc = tqo_compute_qjl_signs(r, head_dim, 12345u, signs + v * (head_dim / 8));
        if (rc) {
            free(r);
            return rc;
        }
    }
    free(r);
    return TQO_OK;
}

/* compute_logit_bias (tq.rs:185-253) for one layer: q [num_q_heads][q_len]
   [d]; signs [num_kv_heads][kv_len][d/8], norms [num_kv_heads][kv_len];
   out [num_q_heads][q_len][kv_len] f32.  r_q = q R^T with R[j][c] =
   sign(j, c) * fl(1/sqrt d) (generate_rademacher_row, qjl.rs:179-189),
   raw = r_q s^T, bias = raw * fl(norm * sf), sf = f32(sqrt(pi/2)) / sqrt(d).
   The two products' summation order is candle's matmul order, which is not
   visible in the reference sources: element order here (parity unpinned at
   the last-ulp level). */
int tqo_tq_logit_bias(size_t num_q_heads, size_t num_kv_heads, size_t d, size_t q_len, size_t kv_len,
                      const float *q, const uint8_t *signs, const uint16_t *norms, float *out)
{
    if (num_kv_heads == 0 || num_q_heads % num_kv_heads != 0) return TQO_ERR_INVALID_ARGUMENT;
    const size_t rep = num_q_heads / num_kv_heads;
    float *R = malloc(d * d * sizeof(float));
    for (size_t j = 0; j < d; j++) tqo_generate_rademacher_row(d, 12345u, j, R + j * d);
    const float sp = (float)sqrt(3.14159265358979323846 / 2.0);
    const float sf = sp / sqrtf((float)d);
    float *rq = malloc(d * sizeof(float));
    for (size_t h = 0; h < num_q_heads; h++) {
        const size_t g = h / rep;
        for (size_t i = 0; i < q_len; i++) {
            const float *qv = q + (h * q_len + i) * d;
            for (size_t j = 0; j < d; j++) {
                float acc = 0.0f;
                for (size_t c = 0; c < d; c++) acc += qv[c] * R[j * d + c];
                rq[j] = acc;
            }
            for (size_t t = 0; t < kv_len; t++) {
                const uint8_t *sb = signs + (g * kv_len + t) * (d / 8);
                float raw = 0.0f;
                for (size_t j = 0; j < d; j++) raw += rq[j] * (((sb[j / 8] >> (j % 8)) & 1) ? 1.0f : -1.0f);
                const float c = tqo_f16_to_f32(norms[g * kv_len + t]) * sf;
                out[(h * q_len + i) * kv_len + t] = raw * c;
            }
        }
    }
    free(R);
    free(rq);
    return TQO_OK;
}

/* Decode attention with an additive logit term: o_h = softmax(scale *
   (q_h K^T + bias_h)) V, bias [num_heads][kv_len] -- the TQ logits of the
   QJL branch of tq_attention_kernel.cu:192-231 (score += correction *
   softmax_scale).  Accumulated in double. */
int tqo_attention_dense_bias(size_t num_heads, size_t num_kv_heads, size_t head_dim, size_t kv_len, const float *q,
                             const float *k, const float *v, const float *bias, float softmax_scale, float *out)
{
    if (num_kv_heads == 0 || num_heads % num_kv_heads != 0) return TQO_ERR_INVALID_ARGUMENT;
    size_t rep = num_heads / num_kv_heads;
    double *sc = malloc((kv_len ? kv_len : 1) * sizeof(double));
    double *acc = malloc(head_dim * sizeof(double));
    for (size_t h = 0; h < num_heads; h++) {
        size_t g = h / rep;
        const float *qh = q + h * head_dim;
        const float *kg = k + g * kv_len * head_dim;
        const float *vg = v + g * kv_len * head_dim;
        double mx = -INFINITY;
        for (size_t t = 0; t < kv_len; t++) {
            double s = 0.0;
            for (size_t dd = 0; dd < head_dim; dd++) s += (double)qh[dd] * (double)kg[t * head_dim + dd];
            s = (s + (double)bias[h * kv_len + t]) * (double)softmax_scale;
            sc[t] = s;
            mx = s > mx ? s : mx;
        }
        double l = 0.0;
        for (size_t dd = 0; dd < head_dim; dd++) acc[dd] = 0.0;
        for (size_t t = 0; t < kv_len; t++) {
            double p = exp(sc[t] - mx);
            l += p;
            for (size_t dd = 0; dd < head_dim; dd++) acc[dd] += p * (double)vg[t * head_dim + dd];
        }
        for (size_t dd = 0; dd < head_dim; dd++) out[h * head_dim + dd] = kv_len ? (float)(acc[dd] / l) : 0.0f;
    }
    free(sc);
    free(acc);
    return TQO_OK;
}

/* ------------------------------------------------------------------------
 * Dense decode attention over dequantized K/V: o_h = softmax(scale q_h K^T) V
 * with GQA group g(h) = h / (num_heads / num_kv_heads) (the mapping of
 * tq_attention_kernel.cu:90-93).  Accumulated in double: a reference that is
 * more accurate than the fp32 kernel it checks.
 * k, v: [num_kv_heads][kv_len][head_dim]; q, out: [num_heads][head_dim].
 * ---------------------------------------------------------------------- */
int tqo_attention_dense(size_t num_heads, size_t num_kv_heads, size_t head_dim, size_t kv_len,
                        const float *q, const float *k, const float *v, float softmax_scale, float *out)
{
    if (num_kv_heads == 0 || num_heads % num_kv_heads != 0) return TQO_ERR_INVALID_ARGUMENT;
    size_t rep = num_heads / num_kv_heads;
    double *sc = malloc((kv_len ? kv_len : 1) * sizeof(double));
    double *acc = malloc(head_dim * sizeof(double));
    for (size_t h = 0; h < num_heads; h++) {
        size_t g = h / rep;
        const float *qh = q + h * head_dim;
        const float *kg = k + g * kv_len * head_dim;
        const float *vg = v + g * kv_len * head_dim;
        double mx = -INFINITY;
        for (size_t t = 0; t < kv_len; t++) {
            double s = 0.0;
            for (size_t d = 0; d < head_dim; d++) s += (double)qh[d] * (double)kg[t * head_dim + d];
            s *= (double)softmax_scale;
            sc[t] = s;
            mx = s > mx ? s : mx;
        }
        double l = 0.0;
        for (size_t d = 0; d < head_dim; d++) acc[d] = 0.0;
        for (size_t t = 0; t < kv_len; t++) {
            double p = exp(sc[t] - mx);
            l += p;
            for (size_t d = 0; d < head_dim; d++) acc[d] += p * (double)vg[t * head_dim + d];
        }
        for (size_t d = 0; d < head_dim; d++) out[h * head_dim + d] = kv_len ? (float)(acc[d] / l) : 0.0f;
    }
    free(sc);
    free(acc);
    return TQO_OK;
}

/* Multi-query (prefill) attention over dequantized K/V, accumulated in
   double: out[h][i] = softmax_t(scale * (q[h][i] . k_t + bias[h][i][t]))
   v_t over t < kv_len, and t <= kv_len - q_len + i when causal (the SDPA a
   caller runs on the reference's prefill result); bias may be NULL.
   q, out [num_heads][q_len][d]; k, v [num_kv_heads][kv_len][d];
   bias [num_heads][q_len][kv_len]. */
int tqo_attention_prefill(size_t num_heads, size_t num_kv_heads, size_t d, size_t q_len, size_t kv_len,
                          const float *q, const float *k, const float *v, const float *bias, float softmax_scale,
                          int causal, float *out)
{
    if (num_kv_heads == 0 || num_heads % num_kv_heads != 0) return TQO_ERR_INVALID_ARGUMENT;
    if (causal && q_len > kv_len) return TQO_ERR_INVALID_ARGUMENT;
    const size_t rep = num_heads / num_kv_heads;
    double *sc = malloc((kv_len ? kv_len : 1) * sizeof(double));
    double *acc = malloc(d * sizeof(double));
    for (size_t h = 0; h < num_heads; h++) {
        const size_t g = h / rep;
        const float *kg = k + g * kv_len * d, *vg = v + g * kv_len * d;
        for (size_t i = 0; i < q_len; i++) {
            const float *qv = q + (h * q_len + i) * d;
            const size_t lim = causal ? kv_len - q_len + i + 1 : kv_len;
            double mx = -INFINITY;
            for (size_t t = 0; t < lim; t++) {
                double s = 0.0;
                for (size_t e = 0; e < d; e++) s += (double)qv[e] * (double)kg[t * d + e];
                if (bias) s += (double)bias[(h * q_len + i) * kv_len + t];
                s *= (double)softmax_scale;
                sc[t] = s;
                mx = s > mx ? s : mx;
            }
            double l = 0.0;
            for (size_t e = 0; e < d; e++) acc[e] = 0.0;
            for (size_t t = 0; t < lim; t++) {
                const double p = exp(sc[t] - mx);
                l += p;
                for (size_t e = 0; e < d; e++) acc[e] += p * (double)vg[t * d + e];
            }
            for (size_t e = 0; e < d; e++) out[(h * q_len + i) * d + e] = lim ? (float)(acc[e] / l) : 0.0f;
        }
    }
    free(sc);
    free(acc);
    return TQO_OK;
}

/* ------------------------------------------------------------------------
 * QJL -- src/qjl.rs
 * ---------------------------------------------------------------------- */

/* qjl.rs:143-147 */
uint64_t tqo_qjl_mix_seed(uint64_t seed, size_t row)
{
    uint64_t mixed = seed * 0x517CC1B727220A95ull + (uint64_t)row;
    return mixed ^ (mixed >> 32) ^ 0x6C62272E07BB0142ull;
}

/* qjl.rs:157-171 (SplitMix64 finalizer of seed + row*gamma + col).
   Pin: identical to tq_sign/tq_rademacher_sign in tq_common.h:171-195. */
float tqo_rademacher_sign(uint64_t row_seed, size_t row, size_t col)
{
    uint64_t z = row_seed + (uint64_t)row * 0x9E3779B97F4A7C15ull + (uint64_t)col;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z = z ^ (z >> 31);
    return (z & 1u) == 0 ? 1.0f : -1.0f;
}

/* qjl.rs:179-189 */
void tqo_generate_rademacher_row(size_t dim, uint64_t seed, size_t row, float *out)
{
    uint64_t rs = tqo_qjl_mix_seed(seed, row);
    float inv = 1.0f / sqrtf((float)dim);
    for (size_t c = 0; c < dim; c++) out[c] = tqo_rademacher_sign(rs, row, c) * inv;
}

/* qjl.rs:196-208: (sequential sum of sign*val) * fl(1/sqrt(d)). */
float tqo_rademacher_vector_product(const float *data, size_t dim, uint64_t seed, size_t row)
{
    uint64_t rs = tqo_qjl_mix_seed(seed, row);
    float inv = 1.0f / sqrtf((float)dim);
    float s = SUM_INIT;
    for (size_t c = 0; c < dim; c++) s += tqo_rademacher_sign(rs, row, c) * data[c];
    return s * inv;
}

/* qjl.rs:305-319 + pack_sign_bits :245-256 (bit j of byte j/8 = p_j >= 0). */
int tqo_compute_qjl_signs(const float *residual, size_t dim, uint64_t seed, uint8_t *out)
{
    size_t nbytes = (dim + 7) / 8;
    memset(out, 0, nbytes);
    for (size_t j = 0; j < dim; j++) {
        float p = tqo_rademacher_vector_product(residual, dim, seed, j);
        if (p >= 0.0f) out[j / 8] |= (uint8_t)(1u << (j % 8));
    }
    return TQO_OK;
}

/* qjl.rs:355-377 / 433-466: (bits-1)-bit polar quantize, residual, norm,
   signs, f16 residual norm. */
int tqo_quantize_with_qjl(int total_bits, size_t dim, uint64_t rot_seed, uint64_t qjl_seed, const float *data,
                          uint8_t *polar_packed, uint16_t *polar_scale, uint8_t *signs, uint16_t *residual_norm)
{
    if (total_bits < 3 || total_bits > 4) return TQO_ERR_UNSUPPORTED_BITS;
    int pb = total_bits - 1;
    int rc = tqo_quantize_vec(pb, dim, rot_seed, data, polar_packed, polar_scale);
    if (rc) return rc;
    float *rec = malloc(dim * sizeof(float));
    float *res = malloc(dim * sizeof(float));
    tqo_dequantize_vec(pb, dim, rot_seed, polar_packed, *polar_scale, rec);
    for (size_t i = 0; i < dim; i++) res[i] = data[i] - rec[i];
    float rn = tqo_l2_norm(res, dim);
    tqo_compute_qjl_signs(res, dim, qjl_seed, signs);
    *residual_norm = tqo_f32_to_f16(rn);
    free(rec);
    free(res);
    return TQO_OK;
}

/* qjl.rs:488-492 */
void tqo_precompute_query_projections(const float *query, size_t dim, uint64_t seed, float *out)
{
    for (size_t j = 0; j < dim; j++) out[j] = tqo_rademacher_vector_product(query, dim, seed, j);
}

/* qjl.rs:263-265: (norm * sqrt(pi/2)) / sqrt(d) */
float tqo_qjl_scaling_constant(float residual_norm, size_t dim)
{
    return residual_norm * 1.2533141f / sqrtf((float)dim);
}

/* qjl.rs:512-519 with sign_bit :233-238 (bit*2 - 1). */
float tqo_qjl_correction(const float *r_query, const uint8_t *signs, size_t dim)
{
    float s = SUM_INIT;
    for (size_t i = 0; i < dim; i++) {
        float bit = (float)((signs[i / 8] >> (i % 8)) & 1u);
        s += r_query[i] * (bit * 2.0f + -1.0f);
    }
    return s;
}

/* qjl.rs:585-606 (estimate_inner_product_with_codebook) */
int tqo_estimate_inner_product(int polar_bits, size_t dim, uint64_t rot_seed, const float *query,
                               const float *r_query, const uint8_t *polar_packed, uint16_t polar_scale,
                               const uint8_t *signs, uint16_t residual_norm, float *out)
{
    float *rec = malloc(dim * sizeof(float));
    int rc = tqo_dequantize_vec(polar_bits, dim, rot_seed, polar_packed, polar_scale, rec);
    if (rc) { free(rec); return rc; }
    float base = SUM_INIT;
    for (size_t i = 0; i < dim; i++) base += query[i] * rec[i];
    float c = tqo_qjl_scaling_constant(tqo_f16_to_f32(residual_norm), dim);
    float corr = tqo_qjl_correction(r_query, signs, dim);
    *out = base + c * corr;
    free(rec);
    return TQO_OK;
}

/* QuantizedKVCache::push_batch (attention.rs:274-301) for one stream of vectors. */
int tqo_qjl_quantize_batch(int total_bits, size_t dim, uint64_t rot_seed, uint64_t qjl_seed, size_t n,
                           const float *data, uint8_t *polar_packed, uint16_t *polar_scales, uint8_t *signs,
                           uint16_t *residual_norms)
{
    if (total_bits < 3 || total_bits > 4) return TQO_ERR_UNSUPPORTED_BITS;
    size_t plen = tqo_packed_len(total_bits - 1, dim);
    size_t slen = (dim + 7) / 8;
    for (size_t v = 0; v < n; v++) {
        int rc = tqo_quantize_with_qjl(total_bits, dim, rot_seed, qjl_seed, data + v * dim, polar_packed + v * plen,
                                       polar_scales + v, signs + v * slen, residual_norms + v);
        if (rc) return rc;
    }
    return TQO_OK;
}

/* QuantizedKVCache::attention_scores (attention.rs:319-353) for several
   queries: scores[q][k]. */
int tqo_qjl_scores_batch(int polar_bits, size_t dim, uint64_t rot_seed, uint64_t qjl_seed, size_t num_queries,
                         const float *queries, size_t num_keys, const uint8_t *polar_packed,
                         const uint16_t *polar_scales, const uint8_t *signs, const uint16_t *residual_norms,
                         float *scores)
{
    size_t plen = tqo_packed_len(polar_bits, dim);
    size_t slen = (dim + 7) / 8;
    float *rq = malloc(dim * sizeof(float));
    for (size_t qi = 0; qi < num_queries; qi++) {
        const float *q = queries + qi * dim;
        tqo_precompute_query_projections(q, dim, qjl_seed, rq);
        for (size_t k = 0; k < num_keys; k++) {
            int rc = tqo_estimate_inner_product(polar_bits, dim, rot_seed, q, rq, polar_packed + k * plen,
                                                polar_scales[k], signs + k * slen, residual_norms[k],
                                                scores + qi * num_keys + k);
            if (rc) { free(rq); return rc; }
        }
    }
    free(rq);
    return TQO_OK;
}

/* QuantizedKVCache::weighted_values (attention.rs:371-408) with
   accumulate_weighted (:70-74): out += deq(v_t) * w_t, sequential over t. */
int tqo_weighted_values(int polar_bits, size_t dim, uint64_t rot_seed, size_t num_values,
                        const uint8_t *polar_packed, const uint16_t *polar_scales, const float *weights, float *out)
{
    size_t plen = tqo_packed_len(polar_bits, dim);
    float *rec = malloc(dim * sizeof(float));
    for (size_t i = 0; i < dim; i++) out[i] = 0.0f;
    for (size_t t = 0; t < num_values; t++) {
        int rc = tqo_dequantize_vec(polar_bits, dim, rot_seed, polar_packed + t * plen, polar_scales[t], rec);
        if (rc) { free(rec); return rc; }
        for (size_t i = 0; i < dim; i++) out[i] += rec[i] * weights[t];
    }
    free(rec);
    return TQO_OK;
}

/* ------------------------------------------------------------------------
 * Test-data generators of the reference's tests
 * ---------------------------------------------------------------------- */

/* src/test_utils.rs:11-22 */
void tqo_pseudo_random_vec(size_t dim, uint64_t seed, float *out)
{
    uint64_t state = seed;
    for (size_t i = 0; i < dim; i++) {
        state = state * 6364136223846793005ull + 1ull;
        int32_t bits = (int32_t)(uint32_t)(state >> 33);
        out[i] = (float)bits / (float)2147483647;
    }
}

/* tests/mse_validation.rs:40-79: LCG uniforms + Box-Muller in f64, pairs
   consumed in order; `count` vectors of `dim` written back to back, each
   vector drawing fresh pairs (an odd dim drops the second of the last pair). */
void tqo_lcg_normal_vecs(uint64_t seed, size_t dim, size_t count, float *out)
{
    uint64_t state = seed;
    const double two_pi = 6.283185307179586;
    for (size_t v = 0; v < count; v++) {
        size_t len = 0;
        while (len < dim) {
            state = state * 6364136223846793005ull + 1ull;
            double u1 = ((double)(uint32_t)(state >> 32) + 1.0) / (4294967295.0 + 2.0);
            state = state * 6364136223846793005ull + 1ull;
            double u2 = ((double)(uint32_t)(state >> 32) + 1.0) / (4294967295.0 + 2.0);
            double r = sqrt(-2.0 * log(u1));
            double th = two_pi * u2;
            out[v * dim + len++] = (float)(r * cos(th));
            if (len < dim) out[v * dim + len++] = (float)(r * sin(th));
        }
    }
}
