"""The Python mirror of the reference's public API (turboquant_amd.api),
written like the reference crate's own tests (roundtrip_tests.rs,
qjl.rs unit tests, attention.rs unit tests) and checked against the oracle."""
import numpy as np
import pytest

from oracle import oracle as orc

torch = pytest.importorskip("torch")
api = pytest.importorskip("turboquant_amd.api")


def test_config_validation_kinds():
    with pytest.raises(api.TurboQuantError) as e:
        api.TurboQuantConfig.new(5, 128)
    assert e.value.code == api.UNSUPPORTED_BITS
    with pytest.raises(api.TurboQuantError) as e:
        api.TurboQuantConfig.new(3, 100)
    assert e.value.code == api.INVALID_DIMENSION
    c = api.TurboQuantConfig.new(3, 128).with_seed(42)
    assert (c.bits, c.dim, c.rotation_seed) == (3, 128, 42)


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("count", [128, 13, 1])
def test_packed_block_matches_reference_packing(bits, count):
    idx = (np.arange(count) * 5 + 1) % (1 << bits)
    b = api.PackedBlock.new(bits, 0x3C00, idx)
    assert b.packed_indices == orc.pack_indices(bits, idx.astype(np.uint8)).tobytes()
    assert b.size_bytes() == 2 + orc.packed_len(bits, count)
    assert b.unpack(count) == idx.tolist()
    assert api.PackedBlock.from_raw(bits, 1, b.packed_indices).unpack(count) == idx.tolist()


@pytest.fixture(scope="module")
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


@pytest.mark.gpu
def test_quantize_dequantize_vec_bit_exact(gpu):
    cfg = api.TurboQuantConfig.new(3, 128).with_seed(42)
    for seed in (1, 2, 3):
        x = orc.pseudo_random_vec(128, seed)
        b = api.quantize_vec(cfg, x)
        rp, rs = orc.quantize_vec_batch(3, 128, 42, x[None])
        assert b.packed_indices == rp[0].tobytes() and b.scale == int(rs[0])
        assert np.array_equal(api.dequantize_vec(cfg, b).cpu().numpy(), orc.dequantize_vec_batch(3, 128, 42, rp, rs)[0])
        assert np.array_equal(api.dequantize_rotated(cfg, b).cpu().numpy(), orc.dequantize_rotated(3, 128, rp[0], rs[0]))
    with pytest.raises(api.TurboQuantError) as e:
        api.quantize_vec(cfg, np.zeros(64, np.float32))
    assert e.value.code == api.DIMENSION_MISMATCH


@pytest.mark.gpu
def test_qjl_block_and_estimates(gpu):
    cfg = api.TurboQuantConfig.new(3, 128).with_seed(42)
    x = orc.pseudo_random_vec(128, 9)
    q = orc.pseudo_random_vec(128, 10)
    b = api.quantize_with_qjl(cfg, x, 12345)
    pp, ps, sg, nm = orc.qjl_quantize_batch(3, 128, 42, 12345, x[None])
    assert b.polar_block.bits == 2 and b.size_bytes() == 52  # qjl.rs:1176
    assert b.polar_block.packed_indices == pp[0].tobytes() and b.polar_block.scale == int(ps[0])
    assert b.qjl_signs == sg[0].tobytes() and b.residual_norm == int(nm[0])
    rq = api.precompute_query_projections(q, 128, 12345).cpu().numpy()
    assert np.array_equal(rq, orc.query_projections(q, 12345))
    est = api.estimate_inner_product_single(q, b, cfg, 12345)
    ref = orc.estimate_inner_product(2, 128, 42, q, rq, pp[0], ps[0], sg[0], nm[0])
    assert abs(est - ref) <= 1e-5 * max(1.0, abs(ref))
    with pytest.raises(api.TurboQuantError) as e:
        api.quantize_with_qjl(api.TurboQuantConfig.new(2, 128), x, 1)
    assert e.value.code == api.UNSUPPORTED_BITS


@pytest.mark.gpu
def test_quantized_kv_cache(gpu):
    cfg = api.TurboQuantConfig.new(3, 64).with_seed(42)
    cache = api.QuantizedKVCache(cfg, 2, 12345)
    keys = np.stack([orc.pseudo_random_vec(64, 100 + i) for i in range(20)])
    values = np.stack([orc.pseudo_random_vec(64, 200 + i) for i in range(20)])
    cache.push_batch(0, keys[:19], values[:19])
    cache.push(0, keys[19], values[19])
    assert cache.entry_count(0) == 20 and cache.entry_count(1) == 0
    assert cache.memory_usage() == 20 * 2 * (2 + 16 + 8 + 2)
    assert cache.fp16_equivalent_memory() == 20 * 64 * 4
    q = orc.pseudo_random_vec(64, 7)
    kp, ks, ksg, knm = orc.qjl_quantize_batch(3, 64, 42, 12345, keys)
    ref = orc.qjl_scores(2, 64, 42, 12345, q[None], kp, ks, ksg, knm)[0]
    got = cache.attention_scores(0, q).cpu().numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())
    w = np.linspace(0.1, 1.0, 20).astype(np.float32)
    vp, vs, _, _ = orc.qjl_quantize_batch(3, 64, 42, 12345, values)
    refw = orc.weighted_values(2, 64, 42, vp, vs, w)
    np.testing.assert_allclose(cache.weighted_values(0, w).cpu().numpy(), refw, rtol=1e-5,
                               atol=1e-5 * np.abs(refw).max())
    kb = cache.key_block(0, 3)
    assert kb.polar_block.packed_indices == kp[3].tobytes() and kb.residual_norm == int(knm[3])
    assert cache.key_block(0, 20) is None
    assert np.array_equal(cache.dequantize_keys_range(0, 2, 5).cpu().numpy(),
                          orc.dequantize_vec_batch(2, 64, 42, kp[2:5], ks[2:5]))
    with pytest.raises(api.TurboQuantError) as e:
        cache.dequantize_values_range(0, 5, 30)
    assert e.value.code == api.RANGE_OUT_OF_BOUNDS
    with pytest.raises(api.TurboQuantError) as e:
        cache.attention_scores(2, q)
    assert e.value.code == api.LAYER_OUT_OF_RANGE
