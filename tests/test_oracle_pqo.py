"""Pins of the oracle's PQO cache codec (reference src/cache/quantize_tensor.rs,
wht_tensor.rs, precomputed/*.rs).

Independent checks:
  * strict bucketing at exact ties: a block whose MaxNorm scale is exactly
    0.5 (found by search) puts r = b_k * 0.5 into bin k and nextup(r) into
    bin k + 1 (quantize.rs:438-452 semantics, cache side);
  * the stored f16 scale is -s (PQO = every block on the outlier codebook);
  * dequantize equals |s| * (c[idx] * d) @ H / sqrt(32) in float64, d the
    decode sign factors (wht_tensor.rs:15-68), to 1e-6 relative;
  * the reference's cosine gates on its closed-form sin/cos K/V
    (cache_pqo_tests.rs:31-43, 151-244): PQO3 > 0.85, PQO4 > 0.92;
  * packed sizes 48 / 64 bytes per 128-vector (cache_storage_tests.rs:80-87).
"""
import numpy as np
import pytest

from oracle import oracle as orc
from test_oracle_rotation import hadamard
from tq_testdata import sincos_kv


def _half_scale_amax(outer):
    m = np.float32(np.float32(1.0) / np.float32(outer))
    a = np.float32(np.float32(0.5) / m)
    for _ in range(64):
        s = np.float32(a * m)
        if s == np.float32(0.5):
            return a
        a = np.nextafter(a, np.float32(np.inf) if s < 0.5 else np.float32(-np.inf))
    raise AssertionError("no amax with an exact 0.5 scale")


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_ties_go_to_the_lower_bin(bits):
    c, b, outer = orc.pqo_codebook(bits)
    amax = _half_scale_amax(outer)
    for k, bk in enumerate(b):
        for up, want in ((False, k), (True, k + 1)):
            r = np.zeros(32, np.float32)
            r[0] = amax
            v = np.float32(bk * np.float32(0.5))
            r[1] = np.nextafter(v, np.float32(np.inf)) if up else v
            packed, scales = orc.pqo_quantize_rotated(bits, r.reshape(1, 32))
            idx = orc.unpack_indices(bits, packed[0], 32)
            assert idx[1] == want, (k, up)
            assert scales[0] == np.float16(-0.5).view(np.uint16)


@pytest.mark.parametrize("bits", [3, 4])
def test_scale_clamp_and_outlier_sign(bits):
    packed, scales = orc.pqo_quantize_rotated(bits, np.zeros((1, 32), np.float32))
    assert scales[0] == np.float16(-1e-10).view(np.uint16)  # max(amax/outer, 1e-10) -> f16(-1e-10) = -0
    rng = np.random.default_rng(bits)
    r = rng.standard_normal((64, 32)).astype(np.float32)
    _, sc = orc.pqo_quantize_rotated(bits, r)
    assert np.all(sc.view(np.float16) < 0)


@pytest.mark.parametrize("bits", [3, 4])
def test_dequantize_matches_textbook_inverse(bits):
    rng = np.random.default_rng(11 + bits)
    x = rng.standard_normal((40, 128)).astype(np.float32) * 3
    packed, scales = orc.pqo_quantize(bits, x, 128)
    out = orc.pqo_dequantize(bits, packed, scales, 128).reshape(-1, 32)
    c, _, _ = orc.pqo_codebook(bits)
    idx = np.stack([orc.unpack_indices(bits, p, 128) for p in packed]).reshape(-1, 32)
    d = orc.pqo_decode_signs().astype(np.float64)
    s = np.abs(scales.reshape(-1).view(np.float16).astype(np.float64))[:, None]
    ref = (c[idx].astype(np.float64) * d) @ hadamard(32) / np.sqrt(32) * s
    assert np.abs(out - ref).max() <= 1e-6 * np.abs(ref).max() * 4


@pytest.mark.parametrize("bits,gate", [(3, 0.85), (4, 0.92)])
def test_cosine_gates_on_reference_inputs(bits, gate):
    k, v = sincos_kv(num_kv_heads=8, seq_len=5, head_dim=128, seed=5.0)
    for t in (k, v):
        x = t.reshape(-1, 128)
        packed, scales = orc.pqo_quantize(bits, x, 128)
        y = orc.pqo_dequantize(bits, packed, scales, 128).reshape(x.shape)
        cos = float((x.astype(np.float64) * y).sum() / np.linalg.norm(x) / np.linalg.norm(y))
        assert cos > gate


@pytest.mark.parametrize("bits,size", [(3, 48), (4, 64)])
def test_packed_dim(bits, size):
    packed, scales = orc.pqo_quantize(bits, np.ones((2, 128), np.float32), 128)
    assert packed.shape == (2, size) and scales.shape == (2, 4)


def _unpack_all(packed, bits):
    b = np.unpackbits(packed, axis=1, bitorder="little").reshape(packed.shape[0], 32, bits)
    return (b * (1 << np.arange(bits))).sum(2)


def _quotients(r, bits):
    """r / s of every element, s = max(amax * fl(1/outer), 1e-10) (quantize_tensor.rs:103-110)."""
    _, _, outer = orc.pqo_codebook(bits)
    mul = np.float32(1.0 / np.float64(outer))
    s = np.maximum((np.abs(r).max(1) * mul).astype(np.float32), np.float32(1e-10))
    return (r / s[:, None]).astype(np.float32)


def rotation_order_mismatches(x, bits, order_a, order_b):
    """Codes of the blocks x [n, 32] under two f32 evaluation orders of x @ R_fwd:
    (mismatch rate, whether every mismatch is one bin apart with the two
    quotients on either side of the boundary between them, within 1e-6)."""
    ra, rb = orc.pqo_rotate(x, order=order_a), orc.pqo_rotate(x, order=order_b)
    ua = _unpack_all(orc.pqo_quantize_rotated(bits, ra)[0], bits)
    ub = _unpack_all(orc.pqo_quantize_rotated(bits, rb)[0], bits)
    va, vb = _quotients(ra, bits), _quotients(rb, bits)
    _, bnd, _ = orc.pqo_codebook(bits)
    ok = True
    for i, j in np.argwhere(ua != ub):
        k = min(ua[i, j], ub[i, j])
        lo, hi = sorted((va[i, j], vb[i, j]))
        ok &= abs(int(ua[i, j]) - int(ub[i, j])) == 1 and lo <= bnd[k] <= hi and abs(va[i, j] - bnd[k]) <= 1e-6
    return float((ua != ub).mean()), bool(ok)


@pytest.mark.parametrize("bits", [3, 4])
def test_rotation_orders_differ_only_across_boundaries(bits):
    """End-to-end code parity against the rotation's unpinned f32 order.  The
    reference rotates with candle's matmul (quantize_tensor.rs:100,104), whose
    summation order is outside the reference tree; the oracle (and the HIP
    kernel, bit-exact to it) uses the butterfly order.  On C2-shaped data
    (bf16 N(0,1) K/V, 4 of 128 channels x8; 65,536 vectors = 8.4 M codes) the
    codes of the butterfly, separately-rounded dot-product and fused
    multiply-add-chain orders differ only where the two quotients r/s fall on
    either side of a codebook boundary (a one-ulp-scale near-tie): about
    4-7e-6 of the codes for every pair of orders, the two gemm orders
    disagreeing with each other as often as with the butterfly."""
    from tq_testdata import kv_outlier
    x = kv_outlier(np.random.default_rng(0), 8, 8192).reshape(-1, 32)
    for a, b in (("butterfly", "dot"), ("butterfly", "fma"), ("dot", "fma")):
        rate, near_ties = rotation_order_mismatches(x, bits, a, b)
        assert near_ties, (a, b)
        assert rate <= 2e-5, (a, b, rate)
