"""Pins of the oracle's IEEE conversions against library routines (numpy)."""
import numpy as np

from oracle import oracle as orc


def test_f16_from_f32_matches_numpy_exhaustive():
    # every f16 value, the midpoints between neighbours, and +-1 ulp around them
    h = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    f = h.view(np.float16).astype(np.float32)
    f = f[np.isfinite(f)]
    fs = np.sort(f)
    mids = ((fs[:-1].astype(np.float64) + fs[1:].astype(np.float64)) / 2).astype(np.float32)
    cand = np.concatenate([f, mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(-np.inf)),
                           np.array([np.inf, -np.inf, 65520.0, -65520.0, 1e-8, -1e-8, 3e-8, 2.9802322e-08,
                                     1e38, -0.0], np.float32)])
    ref = cand.astype(np.float16).view(np.uint16)
    got = orc.f32_to_f16_bits(cand)
    assert np.array_equal(got, ref)


def test_f16_from_f32_random_bits():
    rng = np.random.default_rng(0)
    u = rng.integers(0, 1 << 32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    f = u.view(np.float32)
    f = f[~np.isnan(f)]
    assert np.array_equal(orc.f32_to_f16_bits(f), f.astype(np.float16).view(np.uint16))


def test_f16_to_f32_exhaustive():
    h = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = orc.f16_bits_to_f32(h)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(ref)]))


def test_bf16_rne():
    rng = np.random.default_rng(1)
    f = rng.standard_normal(100_000).astype(np.float32) * 10
    u = f.view(np.uint32).astype(np.uint64)
    # exact rounding via float64: the nearest bf16 value, ties to even
    hi = (u >> 16) << 16
    lo_v = hi.astype(np.uint32).view(np.float32).astype(np.float64)
    up_v = (hi + (1 << 16)).astype(np.uint32).view(np.float32).astype(np.float64)
    x = f.astype(np.float64)
    d_lo, d_up = np.abs(x - lo_v), np.abs(up_v - x)
    even_lo = ((hi >> 16) & 1) == 0
    pick_up = (d_up < d_lo) | ((d_up == d_lo) & ~even_lo)
    ref = np.where(pick_up, (hi >> 16) + 1, hi >> 16).astype(np.uint16)
    got = np.array([orc.lib.tqo_f32_to_bf16(float(v)) for v in f[:20000]], np.uint16)
    assert np.array_equal(got, ref[:20000])
