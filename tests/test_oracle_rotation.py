"""Pins of the oracle's rotation (reference src/rotation.rs) and PQO signs."""
import numpy as np
import pytest

from oracle import oracle as orc


def hadamard(n):
    """Sylvester Hadamard matrix built from scratch (H[i][j] = (-1)^popcount(i&j))."""
    i = np.arange(n)
    return np.where(np.vectorize(lambda v: bin(v).count("1") % 2)(i[:, None] & i[None, :]) == 1, -1.0, 1.0)


def test_wht_known_vector():
    # rotation.rs:236-245: WHT([1,1,1,1]) normalized by 1/sqrt(4) -> [2,0,0,0]
    assert np.array_equal(orc.wht(np.ones(4, np.float32)), np.array([2, 0, 0, 0], np.float32))


@pytest.mark.parametrize("n", [2, 8, 32, 128, 256])
def test_wht_equals_hadamard_product_on_integers(n):
    # small integers: every butterfly sum is exact, so the result is exactly
    # fl((H x)_i * fl(1/sqrt(n)))
    rng = np.random.default_rng(n)
    x = rng.integers(-50, 50, size=n).astype(np.float32)
    hx = hadamard(n) @ x.astype(np.float64)
    norm = np.float32(1.0) / np.sqrt(np.float32(n))
    ref = (hx.astype(np.float32) * norm).astype(np.float32)
    assert np.array_equal(orc.wht(x), ref)


@pytest.mark.parametrize("n", [64, 128, 256])
def test_wht_self_inverse_and_norm(n):
    rng = np.random.default_rng(1)
    x = rng.standard_normal(n).astype(np.float32)
    y = orc.wht(x)
    assert abs(np.linalg.norm(y) - np.linalg.norm(x)) < 1e-4 * np.linalg.norm(x)
    assert np.allclose(orc.wht(y), x, atol=1e-5)
    assert np.allclose(y, hadamard(n) @ x / np.sqrt(n), atol=1e-5)


def test_sign_pattern_closed_form():
    # GOLDEN_RATIO is odd, so the parity of (seed+i)*GOLDEN is the parity of seed+i
    for seed in (0, 1, 42, 99, 2**63 + 5):
        s = orc.sign_pattern(64, seed)
        ref = np.where((np.arange(64, dtype=np.uint64) + np.uint64(seed % 2**64)) % 2 == 0, 1.0, -1.0)
        assert np.array_equal(s, ref.astype(np.float32))


def test_rotate_forward_inverse_roundtrip_and_errors():
    x = np.array([1, 2, 3, 4], np.float32)
    s = orc.sign_pattern(4, 42)
    y = orc.rotate(x, s)
    assert np.allclose(orc.rotate(y, s, inverse=True), x, atol=1e-5)
    # forward = WHT(sign * x); inverse = sign * WHT(y)
    assert np.array_equal(y, orc.wht(x * s))
    with pytest.raises(ValueError, match="code 1"):
        orc.rotate(np.ones(3, np.float32), np.ones(3, np.float32))
    with pytest.raises(ValueError, match="code 3"):
        orc.rotate(np.ones(4, np.float32), np.ones(2, np.float32))


def test_pqo_sign_pattern_and_decode_factor():
    s = orc.pqo_sign32()
    ref = np.array([1, -1, 1, 1, -1, -1, 1, -1, 1, 1, -1, 1, -1, 1, -1, -1,
                    1, -1, -1, 1, 1, -1, 1, -1, -1, 1, 1, 1, -1, -1, 1, -1], np.float32)
    assert np.array_equal(s, ref)
    # fl(fl(1/fl(sqrt 32)) * fl(sqrt 32)) = 0.99999994 (wht_tensor.rs:28-41)
    sq = np.sqrt(np.float32(32))
    fac = np.float32(np.float32(1) / sq) * sq
    assert fac == np.float32(0.99999994)
    assert np.array_equal(orc.pqo_decode_signs(), (ref * fac).astype(np.float32))


def test_pqo_rotation_is_matrix_product():
    # r = x @ R_fwd, R_fwd = H32 / sqrt(32) * diag(s) (precomputed/rotation.rs:26)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((64, 32)).astype(np.float32)
    r = orc.pqo_rotate(x)
    R = hadamard(32) / np.sqrt(32) * orc.pqo_sign32()[None, :]
    assert np.allclose(r, x.astype(np.float64) @ R, atol=2e-6)
    # integer inputs: every butterfly sum is exact, so the oracle's order gives
    # exactly fl((H x)_j * fl(1/sqrt 32)) * s_j
    xi = rng.integers(-20, 20, size=(16, 32)).astype(np.float32)
    inv = np.float32(np.float32(1.0) / np.sqrt(np.float32(32)))
    assert inv.view(np.uint32) == 0x3E3504F3
    ref = ((xi.astype(np.float64) @ hadamard(32)).astype(np.float32) * inv) * orc.pqo_sign32()[None, :]
    assert np.array_equal(orc.pqo_rotate(xi), ref.astype(np.float32))
    # the dot-product order (each x_i * R_ij rounded, then summed) agrees to rounding
    assert np.allclose(orc.pqo_rotate(xi, gemm=True), ref, rtol=0, atol=1e-5)


def test_device_sign_mask_matches_pattern():
    # the kernels' compile-time mask (tq_device.h kPqoSignMask) encodes the same pattern
    mask = 0
    for j, v in enumerate(orc.pqo_sign32()):
        if v < 0:
            mask |= 1 << j
    src = open(__file__.replace("tests/test_oracle_rotation.py", "turboquant_amd/csrc/tq_device.h")).read()
    bits = [int(t.split("u <<")[0].strip().lstrip("(")) for t in
            src.split("kPqoSignMask =")[1].split(";")[0].replace("\n", " ").split("|")]
    dev = sum(b << j for j, b in enumerate(bits))
    assert dev == mask
