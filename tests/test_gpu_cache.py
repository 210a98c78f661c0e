"""GPU tests of the device-resident PqoCache (CompressedKVCache contract,
reference src/cache/pqo.rs, storage.rs; cases of cache_pqo_tests.rs and
cache_storage_tests.rs).  Parity: stored codes bit-exact against the oracle's
quantize of the same K/V; prefill/decode semantics; growth policy; decode
output against dense attention over the oracle-dequantized cache (1e-3)."""
import math

import numpy as np
import pytest

from oracle import oracle as orc
from tq_testdata import sincos_kv

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

H, D = 8, 128


@pytest.fixture(scope="module")
def tq():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import turboquant_amd
    return turboquant_amd


def _kv(t, seed):
    k, v = sincos_kv(H, t, D, seed)
    return torch.from_numpy(k[None]).cuda(), torch.from_numpy(v[None]).cuda()


def _cos(a, b):
    a, b = a.double().flatten(), b.double().flatten()
    return float((a @ b) / a.norm() / b.norm())


@pytest.mark.parametrize("bits,gate", [(3, 0.85), (4, 0.92)])
def test_prefill_then_decode_semantics(tq, bits, gate):
    cache = tq.PqoCache(2, H, D, bits)
    k, v = _kv(4, 5.0)
    r = cache.prefill(0, k, v)
    assert r.k is k and r.logit_bias is None  # first prefill returns the originals
    assert cache.seq_len(0) == 4 and cache.seq_len(1) == 0
    k2, v2 = _kv(5, 7.0)
    r2 = cache.prefill(0, k2, v2)
    assert r2.k.shape == (1, H, 9, D)
    full_k = torch.cat([k, k2], 2)
    assert _cos(r2.k, full_k) > gate and _cos(r2.v, torch.cat([v, v2], 2)) > gate
    q = torch.randn((1, 2 * H, 1, D), device="cuda")
    kd, vd = _kv(1, 6.0)
    out = cache.decode(0, kd, vd, q, tq.AttendConfig(1 / math.sqrt(D), 2))
    assert out.shape == (1, 2 * H, 1, D) and cache.seq_len(0) == 10


def test_stored_codes_bit_exact_and_decode_parity(tq):
    bits = 3
    cache = tq.PqoCache(1, H, D, bits)
    rng = np.random.default_rng(0)
    chunks = [rng.standard_normal((1, H, t, D)).astype(np.float32) for t in (37, 1, 200, 1)]
    vchunks = [rng.standard_normal((1, H, t, D)).astype(np.float32) for t in (37, 1, 200, 1)]
    q = rng.standard_normal((2 * H, D)).astype(np.float32) / np.float32(math.sqrt(D))
    for i, (kc, vc) in enumerate(zip(chunks, vchunks)):
        kt, vt = torch.from_numpy(kc).cuda(), torch.from_numpy(vc).cuda()
        if i == 0:
            cache.prefill(0, kt, vt)
        else:
            out = cache.decode(0, kt, vt, torch.from_numpy(q).cuda().reshape(1, 2 * H, 1, D),
                               tq.AttendConfig(1 / math.sqrt(D), 2))
    torch.cuda.synchronize()
    kall = np.concatenate(chunks, 2)[0]
    vall = np.concatenate(vchunks, 2)[0]
    s = kall.shape[1]
    pk, sk = orc.pqo_quantize(bits, kall.reshape(-1, D), D)
    pv, sv = orc.pqo_quantize(bits, vall.reshape(-1, D), D)
    ki, ks, vi, vs = cache.read_layer(0)
    assert np.array_equal(ki.cpu().numpy().reshape(-1, 48), pk)
    assert np.array_equal(ks.cpu().numpy().view(np.uint16).reshape(-1, 4), sk)
    assert np.array_equal(vi.cpu().numpy().reshape(-1, 48), pv)
    assert np.array_equal(vs.cpu().numpy().view(np.uint16).reshape(-1, 4), sv)
    kd = orc.pqo_dequantize(bits, pk, sk, D).reshape(H, s, D)
    vd = orc.pqo_dequantize(bits, pv, sv, D).reshape(H, s, D)
    ref = orc.attention_dense(q, kd, vd, 1 / math.sqrt(D))
    assert np.abs(out.float().cpu().numpy().reshape(2 * H, D) - ref).max() <= 1e-3


def test_growth_policy_memory_usage_and_reset(tq):
    cache = tq.PqoCache(3, H, D, 4)
    k, v = _kv(10, 1.0)
    cache.prefill(1, k, v)
    assert cache.capacity(1) == 10 + 128  # needed + max(needed/4, 128)
    k2, v2 = _kv(600, 2.0)
    cache.prefill(1, k2, v2)
    assert cache.capacity(1) == 610 + 610 // 4
    assert cache.memory_usage() == 2 * H * 610 * 64 + 2 * H * 610 * 4 * 2
    cache.reset()
    assert cache.seq_len(1) == 0 and cache.memory_usage() == 0 and cache.capacity(1) == 0
    r = cache.prefill(1, k, v)
    assert r.k is k


def test_errors(tq):
    with pytest.raises(tq.TurboQuantError, match="QUANT_BLOCK_SIZE"):
        tq.PqoCache(1, H, 100, 3)
    cache = tq.PqoCache(1, H, D, 3)
    k, v = _kv(2, 0.0)
    with pytest.raises(tq.TurboQuantError):
        cache.prefill(3, k, v)


def _pqo_ref(bits, kall, vall, q):
    """Dense attention of q [Hq, D] over the oracle-dequantized PQO records of
    kall, vall [H, S, D]."""
    s = kall.shape[1]
    pk, sk = orc.pqo_quantize(bits, kall.reshape(-1, D), D)
    pv, sv = orc.pqo_quantize(bits, vall.reshape(-1, D), D)
    kd = orc.pqo_dequantize(bits, pk, sk, D).reshape(H, s, D)
    vd = orc.pqo_dequantize(bits, pv, sv, D).reshape(H, s, D)
    return orc.attention_dense(q, kd, vd, 1 / math.sqrt(D))


def test_reset_and_destroy_are_stream_ordered(tq):
    """reset and destroy release the buffers in the order of the cache's
    stream with no synchronization (storage.rs:175-186 touches no device):
    decodes still queued behind a long-running kernel when the cache is reset
    (and refilled with other data), or destroyed (and another cache created on
    the same pool), read the records they were queued against."""
    bits, t = 3, 700
    rng = np.random.default_rng(31)
    k0 = rng.standard_normal((1, H, t, D)).astype(np.float32)
    v0 = rng.standard_normal((1, H, t, D)).astype(np.float32)
    k1 = rng.standard_normal((1, H, t, D)).astype(np.float32)
    v1 = rng.standard_normal((1, H, t, D)).astype(np.float32)
    kn = rng.standard_normal((1, H, 1, D)).astype(np.float32)
    vn = rng.standard_normal((1, H, 1, D)).astype(np.float32)
    q = rng.standard_normal((2 * H, D)).astype(np.float32) / np.float32(math.sqrt(D))
    dev = lambda a: torch.from_numpy(a).cuda()
    k0d, v0d, k1d, v1d, knd, vnd = map(dev, (k0, v0, k1, v1, kn, vn))
    qd = dev(q).reshape(1, 2 * H, 1, D)
    big = torch.randn((4096, 4096), device="cuda")
    cfg = tq.AttendConfig(1 / math.sqrt(D), 2)
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        cache = tq.PqoCache(1, H, D, bits)
        cache.prefill(0, k0d, v0d)
        for _ in range(8):  # the decodes wait behind this on the stream
            big = big @ big
            big = big / big.abs().max()
        outs = [cache.decode(0, knd, vnd, qd, cfg) for _ in range(3)]
        cache.reset()
        assert cache.seq_len(0) == 0 and cache.memory_usage() == 0
        cache.prefill(0, k1d, v1d)
        after = cache.decode(0, knd, vnd, qd, cfg)
        other = tq.PqoCache(1, H, D, bits)
        other.prefill(0, k0d, v0d)
        for _ in range(8):
            big = big @ big
            big = big / big.abs().max()
        queued = other.decode(0, knd, vnd, qd, cfg)
        del other  # destroyed while its decode is still queued
        fresh = tq.PqoCache(1, H, D, bits)
        fresh.prefill(0, k1d, v1d)
        fresh_out = fresh.decode(0, knd, vnd, qd, cfg)
    s.synchronize()
    for i, o in enumerate(outs):
        kall = np.concatenate([k0] + [kn] * (i + 1), 2)[0]
        vall = np.concatenate([v0] + [vn] * (i + 1), 2)[0]
        ref = _pqo_ref(bits, kall, vall, q)
        assert np.abs(o.float().cpu().numpy().reshape(2 * H, D) - ref).max() <= 1e-3, i
    ref1 = _pqo_ref(bits, np.concatenate([k1, kn], 2)[0], np.concatenate([v1, vn], 2)[0], q)
    assert np.abs(after.float().cpu().numpy().reshape(2 * H, D) - ref1).max() <= 1e-3
    assert np.abs(fresh_out.float().cpu().numpy().reshape(2 * H, D) - ref1).max() <= 1e-3
    ref0 = _pqo_ref(bits, np.concatenate([k0, kn], 2)[0], np.concatenate([v0, vn], 2)[0], q)
    assert np.abs(queued.float().cpu().numpy().reshape(2 * H, D) - ref0).max() <= 1e-3
