"""GPU parity of the standard-codebook cache modes (PQ) and of TqCache (PQ
codes plus the QJL sketch of the keys' residuals, reference src/cache/tq.rs)
against the oracle.

Bars: codes, scales, sign bits and residual norms bit-exact given the same
inputs; query projections bit-exact (same column order); logit bias within
1e-5 of its largest magnitude (the reference's matmul order is not pinned);
fused decode (with the QJL correction in the logits) within 1e-3 max-abs of
dense softmax(scale * (q K^T + bias)) V over the oracle-dequantized cache.
"""
import math

import numpy as np
import pytest

from oracle import oracle as orc
from tq_testdata import bf16_bits, bf16_round, kv_outlier

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

D = 128
TOL = 1e-3


@pytest.fixture(scope="module")
def tq():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import turboquant_amd
    return turboquant_amd


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _host(t):
    return t.cpu().numpy()


@pytest.mark.parametrize("bits", [3, 4])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_standard_mode_codec_bit_exact(tq, bits, dtype):
    rng = np.random.default_rng(20 + bits)
    x = kv_outlier(rng, 4, 300).reshape(-1, D)
    xd = _dev(bf16_bits(x)).view(torch.bfloat16) if dtype == "bf16" else _dev(x)
    p, s = tq.polar_quantize(xd, bits, outlier_blocks=0)
    rp, rs = orc.polar_quantize(bits, 0, x, D)
    assert (_host(p) == rp).all()
    assert (_host(s).view(np.uint16) == rs).all()
    y = tq.polar_dequantize(p, s, bits, D, outlier_blocks=0)
    ry = orc.polar_dequantize(bits, 0, rp, rs, D)
    assert (_host(y).view(np.uint32) == ry.view(np.uint32)).all()


def test_sign_matrix_and_projection_bit_exact(tq):
    m = _host(tq.qjl_sign_matrix(D, 12345)).view(np.uint32).reshape(D, D // 32)
    for j in (0, 1, 63, 64, 127):
        row = orc.rademacher_row(D, 12345, j)
        bits = np.array([(m[j, c // 32] >> (c % 32)) & 1 for c in range(D)], bool)
        assert (bits == (row < 0)).all()
    rng = np.random.default_rng(3)
    q = rng.standard_normal((37, D)).astype(np.float32)
    rq = _host(tq.qjl_project(_dev(q), tq.qjl_sign_matrix(D, 12345)))
    ref = np.stack([orc.query_projections(q[i], 12345) for i in range(q.shape[0])])
    assert (rq.view(np.uint32) == ref.view(np.uint32)).all()


def _tq_cache_ref(k_np, bits):
    """Oracle codes, dequantized K and the keys' (signs, norms) for K [H, T, D]."""
    h, t, _ = k_np.shape
    p, s = orc.polar_quantize(bits, 0, k_np.reshape(-1, D), D)
    kd = orc.polar_dequantize(bits, 0, p, s, D)
    sg, nm = orc.tq_signs_norms(k_np.reshape(-1, D), kd)
    return (p.reshape(h, t, -1), s.reshape(h, t, -1), kd.reshape(h, t, D), sg.reshape(h, t, -1),
            nm.reshape(h, t))


@pytest.mark.parametrize("bits", [3, 4])
def test_tq_cache_prefill_records_sketch_and_bias(tq, bits):
    hkv, hq, t = 4, 8, 150
    rng = np.random.default_rng(40 + bits)
    k = kv_outlier(rng, hkv, t)
    v = kv_outlier(rng, hkv, t)
    q = rng.standard_normal((hq, 5, D)).astype(np.float32)
    cache = tq.TqCache(tq.CacheConfig(bits=bits, head_dim=D, num_kv_heads=hkv, num_layers=2, outlier_blocks=0))
    kt, vt = _dev(k[None]), _dev(v[None])
    r = cache.prefill(0, kt, vt, _dev(q[None]))
    assert r.k is kt and r.logit_bias is not None and r.logit_bias.shape == (1, hq, 5, t)
    ki, ks, vi, vs = cache.read_layer(0)
    sg, nm = cache.read_qjl(0)
    rp, rs, kd, rsg, rnm = _tq_cache_ref(k, bits)
    assert (_host(ki) == rp).all() and (_host(ks).view(np.uint16) == rs).all()
    assert (_host(sg) == rsg).all()
    assert (_host(nm).view(np.uint16) == rnm).all()
    pv, sv = orc.polar_quantize(bits, 0, v.reshape(-1, D), D)
    assert (_host(vi).reshape(-1, pv.shape[1]) == pv).all()
    ref_bias = orc.tq_logit_bias(q, rsg, rnm)
    got = _host(r.logit_bias[0])
    np.testing.assert_allclose(got, ref_bias, rtol=0, atol=1e-5 * np.abs(ref_bias).max())
    # second prefill: the whole dequantized layer and a bias over all tokens
    k2 = kv_outlier(rng, hkv, 20)
    v2 = kv_outlier(rng, hkv, 20)
    r2 = cache.prefill(0, _dev(k2[None]), _dev(v2[None]), _dev(q[None, :, :1]))
    kk = np.concatenate([k, k2], 1)
    rp2, rs2, kd2, rsg2, rnm2 = _tq_cache_ref(kk, bits)
    assert (_host(r2.k[0]).view(np.uint32) == kd2.view(np.uint32)).all()
    ref2 = orc.tq_logit_bias(q[:, :1], rsg2, rnm2)
    np.testing.assert_allclose(_host(r2.logit_bias[0]), ref2, rtol=0, atol=1e-5 * np.abs(ref2).max())
    # memory_usage: records of both tensors plus the whole QJL buffers (tq.rs:314-323)
    cap = cache.capacity(0)
    pd = D * bits // 8
    assert cache.memory_usage() == 2 * hkv * 170 * (pd + 8) + hkv * cap * (D // 8 + 2)
    cache.reset()
    assert cache.seq_len(0) == 0 and cache.memory_usage() == 0


@pytest.mark.parametrize("bits,hq,hkv,t", [(3, 16, 8, 1000), (4, 32, 8, 777), (3, 8, 8, 300), (4, 16, 8, 4100),
                                           (3, 32, 8, 2500)])
def test_tq_fused_decode_matches_dense_with_bias(tq, bits, hq, hkv, t):
    rng = np.random.default_rng(60 + t)
    k = kv_outlier(rng, hkv, t)
    v = kv_outlier(rng, hkv, t)
    cache = tq.TqCache(tq.CacheConfig(bits=bits, head_dim=D, num_kv_heads=hkv, num_layers=1, outlier_blocks=0))
    qp = rng.standard_normal((hq, 1, D)).astype(np.float32)
    cache.prefill(0, _dev(k[None, :, :-1]), _dev(v[None, :, :-1]), _dev(qp[None]))
    q = bf16_round(rng.standard_normal((hq, D)).astype(np.float32) / np.float32(math.sqrt(D)))
    qd = _dev(bf16_bits(q)).view(torch.bfloat16).reshape(1, hq, 1, D)
    scale = 1 / math.sqrt(D)
    out = cache.decode(0, _dev(k[None, :, -1:]), _dev(v[None, :, -1:]), qd, tq.AttendConfig(scale, hq // hkv))
    torch.cuda.synchronize()
    _, _, kd, rsg, rnm = _tq_cache_ref(k, bits)
    pv, sv = orc.polar_quantize(bits, 0, v.reshape(-1, D), D)
    vd = orc.polar_dequantize(bits, 0, pv, sv, D).reshape(hkv, t, D)
    bias = orc.tq_logit_bias(q[:, None, :], rsg, rnm)[:, 0, :]
    ref = orc.attention_dense_bias(q, kd, vd, bias, scale)
    got = _host(out.float()).reshape(hq, D)
    err = np.abs(got - ref).max()
    assert err <= TOL, err
    # the correction matters: without it the result moves by more than the tolerance
    plain = orc.attention_dense(q, kd, vd, scale)
    assert np.abs(plain - ref).max() > 10 * err


def test_tq_decode_dequantized_path(tq):
    bits, hkv, hq, t = 3, 4, 8, 64
    rng = np.random.default_rng(77)
    k = kv_outlier(rng, hkv, t)
    v = kv_outlier(rng, hkv, t)
    cache = tq.TqCache(tq.CacheConfig(bits=bits, head_dim=D, num_kv_heads=hkv, num_layers=1, outlier_blocks=0))
    q = rng.standard_normal((hq, 1, D)).astype(np.float32)
    cache.prefill(0, _dev(k[None, :, :-1]), _dev(v[None, :, :-1]), _dev(q[None]))
    r = cache.decode_dequantized(0, _dev(k[None, :, -1:]), _dev(v[None, :, -1:]), _dev(q[None]))
    _, _, kd, rsg, rnm = _tq_cache_ref(k, bits)
    assert (_host(r.k[0]).view(np.uint32) == kd.view(np.uint32)).all()
    ref = orc.tq_logit_bias(q, rsg, rnm)
    np.testing.assert_allclose(_host(r.logit_bias[0]), ref, rtol=0, atol=1e-5 * np.abs(ref).max())


@pytest.mark.parametrize("bits", [3, 4])
def test_pq_cache_decode_matches_dense(tq, bits):
    """PqoCache with outlier_blocks = 0 (PQ): standard codebook, no QJL."""
    hkv, hq, t = 8, 16, 1500
    rng = np.random.default_rng(90 + bits)
    k = kv_outlier(rng, hkv, t)
    v = kv_outlier(rng, hkv, t)
    cache = tq.PqoCache(tq.CacheConfig(bits=bits, head_dim=D, num_kv_heads=hkv, num_layers=1, outlier_blocks=0))
    r = cache.prefill(0, _dev(k[None, :, :-1]), _dev(v[None, :, :-1]))
    assert r.logit_bias is None
    q = bf16_round(rng.standard_normal((hq, D)).astype(np.float32) / np.float32(math.sqrt(D)))
    scale = 1 / math.sqrt(D)
    out = cache.decode(0, _dev(k[None, :, -1:]), _dev(v[None, :, -1:]), _dev(q).reshape(1, hq, 1, D),
                       tq.AttendConfig(scale, 2))
    pk, sk = orc.polar_quantize(bits, 0, k.reshape(-1, D), D)
    pv, sv = orc.polar_quantize(bits, 0, v.reshape(-1, D), D)
    kd = orc.polar_dequantize(bits, 0, pk, sk, D).reshape(hkv, t, D)
    vd = orc.polar_dequantize(bits, 0, pv, sv, D).reshape(hkv, t, D)
    ref = orc.attention_dense(q, kd, vd, scale)
    err = np.abs(_host(out).reshape(hq, D) - ref).max()
    assert err <= TOL, err


def test_reference_abi_qjl_enabled(tq):
    """tq_fused_attention with qjl_enabled = 1 over TQ records (the reference
    kernel's dormant branch, tq_attention_kernel.cu:192-231), given the
    records' codebook (the standard (bits-1)-bit MaxNorm codebook, indexed by
    code as the kernel reads it) and the 32 decode signs."""
    bits, hkv, hq, t = 3, 4, 8, 900
    rng = np.random.default_rng(123)
    k = kv_outlier(rng, hkv, t)
    v = kv_outlier(rng, hkv, t)
    rp, rs, kd, rsg, rnm = _tq_cache_ref(k, bits)
    pv, sv = orc.polar_quantize(bits, 0, v.reshape(-1, D), D)
    vd = orc.polar_dequantize(bits, 0, pv, sv, D).reshape(hkv, t, D)
    q = rng.standard_normal((hq, D)).astype(np.float32) / np.float32(math.sqrt(D))
    rq = np.stack([orc.query_projections(q[i], 12345) for i in range(hq)])
    p = (t + 511) // 512
    dev = lambda a: _dev(np.ascontiguousarray(a))
    out = torch.zeros((hq, D), dtype=torch.float32, device="cuda")
    po = torch.zeros((hq * p, D), dtype=torch.float32, device="cuda")
    pm = torch.zeros((hq * p,), dtype=torch.float32, device="cuda")
    ps = torch.zeros((hq * p,), dtype=torch.float32, device="cuda")
    c_std, _, _ = orc.pqo_codebook(bits - 1)
    cb = dev(np.concatenate([c_std, np.zeros(8 - c_std.size, np.float32)]))
    sgp = dev(orc.pqo_decode_signs())
    ki, ks = dev(rp), dev(rs.view(np.int16))
    vi, vs = dev(pv), dev(sv.view(np.int16))
    sgd, nmd, rqd, qd = dev(rsg), dev(rnm.view(np.int16)), dev(rq), dev(q)
    tq.check(tq.lib.tq_fused_attention(qd.data_ptr(), ki.data_ptr(), ks.data_ptr(), vi.data_ptr(), vs.data_ptr(),
                                       cb.data_ptr(), sgp.data_ptr(), out.data_ptr(), po.data_ptr(), pm.data_ptr(),
                                       ps.data_ptr(), sgd.data_ptr(), nmd.data_ptr(), rqd.data_ptr(), 1, hq, hkv, D, t,
                                       t, D * bits // 8, D // 32, bits, float(1 / math.sqrt(D)), p,
                                       torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    bias = orc.tq_logit_bias(q[:, None, :], rsg, rnm)[:, 0, :]
    ref = orc.attention_dense_bias(q, kd, vd, bias, 1 / math.sqrt(D))
    err = np.abs(_host(out) - ref).max()
    assert err <= TOL, err


def test_tq_cache_rejects_outlier_config(tq):
    with pytest.raises(tq.TurboQuantError):
        tq.TqCache(tq.CacheConfig(bits=3, head_dim=D, num_kv_heads=2, num_layers=1))


@pytest.mark.parametrize("bits,outlier,norm", [(3, 0, 1), (4, 0, 1), (3, orc.OUTLIER_ALL, 1), (4, orc.OUTLIER_ALL, 1),
                                               (3, 1, 0), (4, 2, 0), (3, 3, 1)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_l2norm_and_mixed_codec_bit_exact(tq, bits, outlier, norm, dtype):
    rng = np.random.default_rng(200 + bits + norm)
    x = kv_outlier(rng, 3, 70).reshape(-1, D)
    xd = _dev(bf16_bits(x)).view(torch.bfloat16) if dtype == "bf16" else _dev(x)
    p, s = tq.polar_quantize(xd, bits, outlier_blocks=outlier, norm_mode=norm)
    rp, rs = orc.polar_quantize(bits, outlier, x, D, norm_mode=norm)
    assert (_host(p) == rp).all()
    assert (_host(s).view(np.uint16) == rs).all()
    y = tq.polar_dequantize(p, s, bits, D, outlier_blocks=outlier, norm_mode=norm)
    ry = orc.polar_dequantize(bits, outlier, rp, rs, D, norm_mode=norm)
    assert (_host(y).view(np.uint32) == ry.view(np.uint32)).all()


@pytest.mark.parametrize("kind,bits", [("pqo", 3), ("pq", 4), ("tq", 3), ("tq", 4)])
def test_l2norm_caches_decode(tq, kind, bits):
    hkv, hq, t = 8, 16, 1200
    rng = np.random.default_rng(300 + bits)
    k = kv_outlier(rng, hkv, t)
    v = kv_outlier(rng, hkv, t)
    outlier = orc.OUTLIER_ALL if kind == "pqo" else 0
    cfg = tq.CacheConfig(bits=bits, head_dim=D, num_kv_heads=hkv, num_layers=1,
                         norm_mode=tq.QuantNormMode.L2Norm, outlier_blocks=outlier)
    cache = tq.TqCache(cfg) if kind == "tq" else tq.PqoCache(cfg)
    qp = rng.standard_normal((hq, 1, D)).astype(np.float32)
    if kind == "tq":
        cache.prefill(0, _dev(k[None, :, :-1]), _dev(v[None, :, :-1]), _dev(qp[None]))
    else:
        cache.prefill(0, _dev(k[None, :, :-1]), _dev(v[None, :, :-1]))
    q = bf16_round(rng.standard_normal((hq, D)).astype(np.float32) / np.float32(math.sqrt(D)))
    scale = 1 / math.sqrt(D)
    out = cache.decode(0, _dev(k[None, :, -1:]), _dev(v[None, :, -1:]), _dev(q).reshape(1, hq, 1, D),
                       tq.AttendConfig(scale, 2))
    pk, sk = orc.polar_quantize(bits, outlier, k.reshape(-1, D), D, norm_mode=1)
    pv, sv = orc.polar_quantize(bits, outlier, v.reshape(-1, D), D, norm_mode=1)
    kd = orc.polar_dequantize(bits, outlier, pk, sk, D, norm_mode=1)
    vd = orc.polar_dequantize(bits, outlier, pv, sv, D, norm_mode=1).reshape(hkv, t, D)
    if kind == "tq":
        sg, nm = orc.tq_signs_norms(k.reshape(-1, D), kd)
        bias = orc.tq_logit_bias(q[:, None, :], sg.reshape(hkv, t, -1), nm.reshape(hkv, t))[:, 0, :]
        ref = orc.attention_dense_bias(q, kd.reshape(hkv, t, D), vd, bias, scale)
    else:
        ref = orc.attention_dense(q, kd.reshape(hkv, t, D), vd, scale)
    err = np.abs(_host(out).reshape(hq, D) - ref).max()
    assert err <= TOL, err


def test_mixed_cache_dequantized_paths(tq):
    bits, hkv, eo = 3, 4, 2
    rng = np.random.default_rng(400)
    k1, v1 = kv_outlier(rng, hkv, 30), kv_outlier(rng, hkv, 30)
    k2, v2 = kv_outlier(rng, hkv, 9), kv_outlier(rng, hkv, 9)
    cache = tq.PqoCache(tq.CacheConfig(bits=bits, head_dim=D, num_kv_heads=hkv, num_layers=1, outlier_blocks=eo))
    cache.prefill(0, _dev(k1[None]), _dev(v1[None]))
    r = cache.prefill(0, _dev(k2[None]), _dev(v2[None]))
    # each append quantizes its own [H * T, D] block matrix (quantize_kv_pair per call)
    ref = np.concatenate([orc.polar_dequantize(bits, eo, *orc.polar_quantize(bits, eo, kk.reshape(-1, D), D), D)
                          .reshape(hkv, -1, D) for kk in (k1, k2)], 1)
    assert (_host(r.k[0]).view(np.uint32) == ref.view(np.uint32)).all()
    q = _dev(rng.standard_normal((1, 8, 1, D)).astype(np.float32))
    k3, v3 = kv_outlier(rng, hkv, 1), kv_outlier(rng, hkv, 1)
    with pytest.raises(tq.TurboQuantError):
        cache.decode(0, _dev(k3[None]), _dev(v3[None]), q, tq.AttendConfig(1 / math.sqrt(D), 2))
    out = cache.decode_output(0, _dev(k3[None]), _dev(v3[None]), q, tq.AttendConfig(1 / math.sqrt(D), 2))
    assert isinstance(out, tq.Dequantized) and out.result.k.shape == (1, hkv, 40, D)


def test_tq_cache_decode_without_new_tokens_projects_in_launch(tq):
    """A TqCache decode that appends no token (the append has no sketch
    launch to project q in): the decode launch projects q from the sign
    matrix itself; checked against dense attention with the QJL bias."""
    bits, hq, hkv, t = 3, 16, 8, 900
    rng = np.random.default_rng(91)
    k = kv_outlier(rng, hkv, t)
    v = kv_outlier(rng, hkv, t)
    cache = tq.TqCache(tq.CacheConfig(bits=bits, head_dim=D, num_kv_heads=hkv, num_layers=1, outlier_blocks=0))
    qp = rng.standard_normal((hq, 1, D)).astype(np.float32)
    cache.prefill(0, _dev(k[None]), _dev(v[None]), _dev(qp[None]))
    q = bf16_round(rng.standard_normal((hq, D)).astype(np.float32) / np.float32(math.sqrt(D)))
    qd = _dev(bf16_bits(q)).view(torch.bfloat16).reshape(1, hq, 1, D)
    scale = 1 / math.sqrt(D)
    empty = torch.zeros((1, hkv, 0, D), dtype=torch.float32, device="cuda")
    out = cache.decode(0, empty, empty, qd, tq.AttendConfig(scale, hq // hkv))
    torch.cuda.synchronize()
    assert cache.seq_len(0) == t
    _, _, kd, rsg, rnm = _tq_cache_ref(k, bits)
    pv, sv = orc.polar_quantize(bits, 0, v.reshape(-1, D), D)
    vd = orc.polar_dequantize(bits, 0, pv, sv, D).reshape(hkv, t, D)
    bias = orc.tq_logit_bias(q[:, None, :], rsg, rnm)[:, 0, :]
    ref = orc.attention_dense_bias(q, kd, vd, bias, scale)
    err = np.abs(_host(out.float()).reshape(hq, D) - ref).max()
    assert err <= TOL, err
