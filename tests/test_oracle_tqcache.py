"""Pins of the oracle's cache-mode codec and TqCache functions (reference
src/cache/quantize_tensor.rs, precomputed/, tq.rs) against independent
float64 matrix arithmetic: a Sylvester Hadamard built here, numpy
searchsorted for the bucketize, the Rademacher matrix from the already
pinned hash rows, numpy softmax.  A dropped sign, a wrong codebook, a wrong
outer centroid or a transposed product fails one of these."""
import math

import numpy as np
import pytest

from oracle import oracle as orc
from tq_testdata import kv_outlier

SIGN32 = np.array([1, -1, 1, 1, -1, -1, 1, -1, 1, 1, -1, 1, -1, 1, -1, -1,
                   1, -1, -1, 1, 1, -1, 1, -1, -1, 1, 1, 1, -1, -1, 1, -1], np.float64)


def hadamard(n):
    h = np.array([[1.0]])
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


R_FWD = hadamard(32) / math.sqrt(32) * SIGN32[None, :]   # precomputed/rotation.rs: H/sqrt(32) diag(s)

C3 = np.array([-2.1573, -1.3336, -0.7434, -0.2428, 0.2428, 0.7434, 1.3336, 2.1573])
B3 = np.array([-1.7455, -1.0385, -0.4931, 0.0, 0.4931, 1.0385, 1.7455])
C2 = np.array([-2.1573, -0.7434, 0.7434, 2.1573])
B2 = np.array([-1.0385, 0.0, 1.0385])


def unpack(packed, bits, count):
    bitsarr = np.unpackbits(packed, bitorder="little")
    return np.array([int(sum(int(bitsarr[i * bits + b]) << b for b in range(bits))) for i in range(count)])


@pytest.mark.parametrize("bits", [3, 4])
def test_standard_mode_codes_against_float64_textbook(bits):
    """outlier_blocks = 0: codes bucketized against the (bits-1)-bit boundaries,
    in bits-wide slots, after a MaxNorm scale by the bits-bit outer centroid."""
    rng = np.random.default_rng(7 + bits)
    x = kv_outlier(rng, 2, 40).reshape(-1, 128)
    packed, scales = orc.polar_quantize(bits, 0, x, 128)
    if bits == 3:
        bnd, outer = B2, 2.1573
    else:
        bnd, outer = B3, np.float32(-2.1573) + np.float32(15) * (np.float32(2 * 2.1573) / np.float32(15))
    blocks = x.reshape(-1, 32).astype(np.float64)
    r = blocks @ R_FWD
    s = np.maximum(np.abs(r).max(1) / float(outer), 1e-10)
    v = r / s[:, None]
    ref = np.searchsorted(bnd, v, side="left")  # #{k: v > b_k}
    bpb = 4 * bits
    got = np.stack([unpack(packed.reshape(-1, bpb)[i], bits, 32) for i in range(blocks.shape[0])])
    near = np.min(np.abs(v[..., None] - bnd[None, None, :]), axis=-1) < 1e-5
    assert got.max() < 2 ** (bits - 1)             # the slot's top bit stays zero
    assert (got[~near] == ref[~near]).all()
    sc = orc.f16_bits_to_f32(scales.reshape(-1))
    assert (sc > 0).all()                          # standard blocks carry positive scales
    np.testing.assert_allclose(sc, s, rtol=1e-3)   # f16 of the MaxNorm scale


@pytest.mark.parametrize("bits", [3, 4])
def test_standard_mode_dequant_against_matrix_inverse(bits):
    rng = np.random.default_rng(11)
    x = kv_outlier(rng, 1, 30).reshape(-1, 128)
    packed, scales = orc.polar_quantize(bits, 0, x, 128)
    y = orc.polar_dequantize(bits, 0, packed, scales, 128).reshape(-1, 32)
    cb = C2 if bits == 3 else C3
    bpb = 4 * bits
    idx = np.stack([unpack(packed.reshape(-1, bpb)[i], bits, 32) for i in range(y.shape[0])])
    sc = np.abs(orc.f16_bits_to_f32(scales.reshape(-1))).astype(np.float64)
    ref = (cb[idx] @ R_FWD.T) * sc[:, None]        # R_inv = R_fwd^T (precomputed/rotation.rs:29)
    np.testing.assert_allclose(y, ref, rtol=2e-6, atol=2e-6 * np.abs(ref).max())


def test_outlier_mode_equals_pqo():
    x = kv_outlier(np.random.default_rng(3), 2, 25).reshape(-1, 128)
    for bits in (3, 4):
        p0, s0 = orc.pqo_quantize(bits, x, 128)
        p1, s1 = orc.polar_quantize(bits, orc.OUTLIER_ALL, x, 128)
        assert (p0 == p1).all() and (s0 == s1).all()


def rademacher(d, seed=12345):
    return np.stack([orc.rademacher_row(d, seed, j) for j in range(d)]).astype(np.float64)


def test_signs_and_norms_against_matrix_sketch():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((20, 128)).astype(np.float32)
    xhat = (x + rng.standard_normal((20, 128)).astype(np.float32) * np.float32(0.1)).astype(np.float32)
    signs, norms = orc.tq_signs_norms(x, xhat)
    r = (x - xhat).astype(np.float64)
    p = r @ rademacher(128).T
    bits = np.unpackbits(signs, axis=1, bitorder="little").astype(bool)
    clear = np.abs(p) > 1e-5
    assert (bits[clear] == (p >= 0)[clear]).all()
    np.testing.assert_allclose(orc.f16_bits_to_f32(norms), np.linalg.norm(r, axis=1), rtol=1e-3)


def test_logit_bias_against_matrix_products():
    rng = np.random.default_rng(9)
    hq, hkv, ql, t, d = 4, 2, 3, 50, 128
    q = rng.standard_normal((hq, ql, d)).astype(np.float32)
    signs = rng.integers(0, 256, (hkv, t, d // 8), dtype=np.uint8)
    norms = orc.f32_to_f16_bits(rng.uniform(0.1, 2.0, (hkv, t)).astype(np.float32)).reshape(hkv, t)
    got = orc.tq_logit_bias(q, signs, norms)
    R = rademacher(d)
    s = np.unpackbits(signs, axis=2, bitorder="little").astype(np.float64) * 2 - 1   # bit 1 -> +1
    c = orc.f16_bits_to_f32(norms).reshape(hkv, t).astype(np.float64) * math.sqrt(math.pi / 2) / math.sqrt(d)
    for h in range(hq):
        g = h // (hq // hkv)
        ref = (q[h].astype(np.float64) @ R.T) @ s[g].T * c[g][None, :]
        np.testing.assert_allclose(got[h], ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())


def test_dense_bias_attention_against_numpy():
    rng = np.random.default_rng(4)
    h, hkv, t, d = 4, 2, 33, 128
    q = rng.standard_normal((h, d)).astype(np.float32)
    k = rng.standard_normal((hkv, t, d)).astype(np.float32)
    v = rng.standard_normal((hkv, t, d)).astype(np.float32)
    bias = rng.standard_normal((h, t)).astype(np.float32)
    scale = 1 / math.sqrt(d)
    got = orc.attention_dense_bias(q, k, v, bias, scale)
    for hh in range(h):
        g = hh // 2
        lo = (k[g].astype(np.float64) @ q[hh] + bias[hh]) * scale
        p = np.exp(lo - lo.max())
        ref = (p / p.sum()) @ v[g].astype(np.float64)
        np.testing.assert_allclose(got[hh], ref, rtol=1e-5, atol=1e-6)
    # zero bias reduces to the plain dense oracle
    z = orc.attention_dense_bias(q, k, v, np.zeros_like(bias), scale)
    np.testing.assert_allclose(z, orc.attention_dense(q, k, v, scale), rtol=1e-6, atol=1e-7)


def l2_codebook(bits):
    c, b = orc.get_codebook(bits, 32)
    return np.asarray(c, np.float32).astype(np.float64), np.asarray(b, np.float32).astype(np.float64)


@pytest.mark.parametrize("bits,outlier", [(3, 0), (4, 0), (3, orc.OUTLIER_ALL), (4, orc.OUTLIER_ALL)])
def test_l2norm_mode_against_float64_textbook(bits, outlier):
    """L2Norm (quantize_tensor.rs:90-101): x / |x| rotated, bucketized against the
    Beta tables of dimension 32, scale = |x|; dequant = centroids through R_fwd^T."""
    rng = np.random.default_rng(30 + bits)
    x = kv_outlier(rng, 2, 20).reshape(-1, 128)
    packed, scales = orc.polar_quantize(bits, outlier, x, 128, norm_mode=1)
    cb_bits = bits if outlier else bits - 1
    cen, bnd = l2_codebook(cb_bits)
    blocks = x.reshape(-1, 32).astype(np.float64)
    nrm = np.linalg.norm(blocks, axis=1)
    r = (blocks / nrm[:, None]) @ R_FWD
    ref = np.searchsorted(bnd, r, side="left")
    bpb = 4 * bits
    got = np.stack([unpack(packed.reshape(-1, bpb)[i], bits, 32) for i in range(blocks.shape[0])])
    near = np.min(np.abs(r[..., None] - bnd[None, None, :]), axis=-1) < 1e-6
    assert (got[~near] == ref[~near]).all()
    sc = orc.f16_bits_to_f32(scales.reshape(-1)).astype(np.float64)
    np.testing.assert_allclose(np.abs(sc), nrm, rtol=1e-3)
    assert ((sc < 0) == bool(outlier)).all()
    y = orc.polar_dequantize(bits, outlier, packed, scales, 128, norm_mode=1).reshape(-1, 32)
    yref = (cen[got] @ R_FWD.T) * np.abs(sc)[:, None]
    np.testing.assert_allclose(y, yref, rtol=2e-6, atol=2e-6 * np.abs(yref).max())


@pytest.mark.parametrize("eo", [1, 2, 3])
def test_mixed_outlier_blocks_follow_reference_row_order(eo):
    """0 < outlier_blocks < num_blocks: the first n * eo rows of the block matrix
    take the outlier boundaries (bucketize_blocks, quantize_tensor.rs:118-150),
    the scale sign marks blocks j < eo of every vector (precomputed/mod.rs:102-114)
    and the dequantize picks the codebook by that sign, clamping standard codes
    (quantize_tensor.rs:242-260)."""
    bits, n = 3, 5
    rng = np.random.default_rng(eo)
    x = kv_outlier(rng, 1, n).reshape(-1, 128)
    packed, scales = orc.polar_quantize(bits, eo, x, 128)
    blocks = x.reshape(-1, 32).astype(np.float64)
    r = blocks @ R_FWD
    s = np.maximum(np.abs(r).max(1) / 2.1573, 1e-10)
    v = r / s[:, None]
    rows = np.arange(blocks.shape[0])
    out_row = rows < n * eo
    ref = np.where(out_row[:, None], np.searchsorted(B3, v, side="left"), np.searchsorted(B2, v, side="left"))
    got = np.stack([unpack(packed.reshape(-1, 12)[i], bits, 32) for i in range(blocks.shape[0])])
    near = np.min(np.abs(v[..., None] - B3[None, None, :]), axis=-1) < 1e-5
    assert (got[~near] == ref[~near]).all()
    sc = orc.f16_bits_to_f32(scales.reshape(-1))
    assert ((sc < 0) == ((rows % 4) < eo)).all()
    y = orc.polar_dequantize(bits, eo, packed, scales, 128).reshape(-1, 32)
    cen = np.where((sc < 0)[:, None], C3[got], C2[np.minimum(got, 3)])
    yref = (cen @ R_FWD.T) * np.abs(sc)[:, None]
    np.testing.assert_allclose(y, yref, rtol=2e-6, atol=2e-6 * np.abs(yref).max())


def test_prefill_oracle_against_numpy():
    rng = np.random.default_rng(12)
    h, hkv, ql, t, d = 4, 2, 5, 19, 128
    q = rng.standard_normal((h, ql, d)).astype(np.float32)
    k = rng.standard_normal((hkv, t, d)).astype(np.float32)
    v = rng.standard_normal((hkv, t, d)).astype(np.float32)
    bias = rng.standard_normal((h, ql, t)).astype(np.float32)
    scale = 1 / math.sqrt(d)
    for causal in (False, True):
        got = orc.attention_prefill(q, k, v, scale, causal, bias)
        for hh in range(h):
            g = hh // 2
            lo = (q[hh].astype(np.float64) @ k[g].T.astype(np.float64) + bias[hh]) * scale
            if causal:
                lo = np.where(np.arange(t)[None, :] <= (t - ql + np.arange(ql))[:, None], lo, -np.inf)
            p = np.exp(lo - lo.max(1, keepdims=True))
            ref = (p / p.sum(1, keepdims=True)) @ v[g].astype(np.float64)
            np.testing.assert_allclose(got[hh], ref, rtol=1e-5, atol=1e-6)
    # one query at the end with the causal limit is the decode oracle
    one = orc.attention_prefill(q[:, -1:], k, v, scale, True)
    np.testing.assert_allclose(one[:, 0], orc.attention_dense(q[:, -1], k, v, scale), rtol=1e-6, atol=1e-7)
