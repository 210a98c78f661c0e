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
