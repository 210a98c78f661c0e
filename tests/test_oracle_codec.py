"""Pins of the oracle's full-vector codec (reference src/quantize.rs:142-316).

Independent checks:
  * composition against textbook float64 math: normalize, x -> H(s * x)/sqrt(d)
    with a Sylvester Hadamard matrix built here, then searchsorted on the f64
    boundaries; codes may differ only where a rotated coordinate sits within
    float32 rounding of a boundary;
  * dequantize against scale * s * (H c[idx]) / sqrt(d) in float64 (1e-6 rel);
  * the reference's statistical windows (mse_validation.rs:83-142, 269-286) on
    its own LCG Box-Muller inputs, and its null / unit / constant vector
    cases (roundtrip_tests.rs:662-750);
  * the f16 scale is numpy's float16 of the float32 norm.
"""
import numpy as np
import pytest

from oracle import oracle as orc
from test_oracle_rotation import hadamard


def _rotated_f64(x, seed):
    d = x.shape[-1]
    s = orc.sign_pattern(d, seed).astype(np.float64)
    n = np.sqrt((x.astype(np.float64) ** 2).sum(axis=-1, keepdims=True))
    return (x / n * s) @ hadamard(d).T / np.sqrt(d)


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("dim", [32, 128, 256])
def test_codes_match_textbook_rotation_and_bucketize(bits, dim):
    rng = np.random.default_rng(bits * 7 + dim)
    x = rng.standard_normal((300, dim)).astype(np.float32)
    packed, scales = orc.quantize_vec_batch(bits, dim, 42, x)
    got = np.stack([orc.unpack_indices(bits, p, dim) for p in packed])
    _, b = orc.get_codebook(bits, dim)
    rot = _rotated_f64(x, 42)
    ref = np.searchsorted(b, rot, side="left")
    mism = got != ref
    assert mism.mean() < 1e-3
    if mism.any():  # only at float32-rounding distance from a boundary
        dist = np.min(np.abs(rot[mism][:, None] - b[None, :]), axis=1)
        assert dist.max() < 1e-5
    norms = np.sqrt((x.astype(np.float32) ** 2).sum(axis=1, dtype=np.float32))
    assert np.array_equal(scales, norms.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("dim", [64, 128])
def test_dequantize_matches_textbook_inverse(bits, dim):
    rng = np.random.default_rng(5 + bits + dim)
    x = rng.standard_normal((50, dim)).astype(np.float32)
    packed, scales = orc.quantize_vec_batch(bits, dim, 7, x)
    out = orc.dequantize_vec_batch(bits, dim, 7, packed, scales)
    c, _ = orc.get_codebook(bits, dim)
    idx = np.stack([orc.unpack_indices(bits, p, dim) for p in packed])
    vals = c[idx].astype(np.float32).astype(np.float64)
    s = orc.sign_pattern(dim, 7).astype(np.float64)
    sc = scales.view(np.float16).astype(np.float64)[:, None]
    ref = (vals @ hadamard(dim).T / np.sqrt(dim)) * s * sc
    assert np.abs(out - ref).max() <= 1e-6 * np.abs(ref).max() * 4


def test_dequantize_rotated_is_scaled_centroids():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((1, 128)).astype(np.float32)
    packed, scales = orc.quantize_vec_batch(3, 128, 42, x)
    c, _ = orc.get_codebook(3, 128)
    idx = orc.unpack_indices(3, packed[0], 128)
    ref = c[idx].astype(np.float32) * scales.view(np.float16).astype(np.float32)[0]
    assert np.array_equal(orc.dequantize_rotated(3, 128, packed[0], int(scales[0])), ref)


def _nmse(bits, dim, n, seed=12345):
    x = orc.lcg_normal_vecs(seed, dim, n).astype(np.float32)
    packed, scales = orc.quantize_vec_batch(bits, dim, 42, x)
    y = orc.dequantize_vec_batch(bits, dim, 42, packed, scales)
    x64 = x.astype(np.float64)
    return float(np.mean(((x64 - y) ** 2).sum(1) / (x64 ** 2).sum(1)))


@pytest.mark.parametrize("bits,dim,n,lo,hi", [(3, 128, 10_000, 0.030, 0.038), (4, 128, 10_000, 0.007, 0.011),
                                              (3, 256, 1_000, 0.025, 0.040), (4, 256, 1_000, 0.005, 0.012)])
def test_nmse_windows(bits, dim, n, lo, hi):
    assert lo <= _nmse(bits, dim, n) <= hi


def test_lcg_normal_generator_moments():
    x = orc.lcg_normal_vecs(12345, 128, 4000).astype(np.float64)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01


@pytest.mark.parametrize("bits", [3, 4])
def test_null_unit_constant_vectors(bits):
    z = np.zeros((1, 128), np.float32)
    p, s = orc.quantize_vec_batch(bits, 128, 99, z)
    assert s[0] == 0
    assert np.abs(orc.dequantize_vec_batch(bits, 128, 99, p, s)).max() == 0.0
    u = np.zeros((1, 128), np.float32)
    u[0, 0] = 1.0
    p, s = orc.quantize_vec_batch(bits, 128, 99, u)
    nrm = np.linalg.norm(orc.dequantize_vec_batch(bits, 128, 99, p, s))
    assert 0.3 < nrm < 2.0
    cst = np.full((1, 128), 0.5, np.float32)
    p, s = orc.quantize_vec_batch(bits, 128, 99, cst)
    ratio = np.linalg.norm(orc.dequantize_vec_batch(bits, 128, 99, p, s)) / np.linalg.norm(cst)
    assert 0.1 < ratio < 3.0


def test_pseudo_random_vec_is_deterministic_and_bounded():
    a = orc.pseudo_random_vec(128, 5)
    assert np.array_equal(a, orc.pseudo_random_vec(128, 5))
    assert not np.array_equal(a, orc.pseudo_random_vec(128, 6))
    assert np.all(np.abs(a) <= 1.0)
