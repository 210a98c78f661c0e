"""GPU parity of the multi-query (prefill) attention over compressed records
against the oracle: dequantize with the CPU restatement, then dense
(causal or full) softmax attention in double, with the QJL logit bias for a
TQ cache.  Tolerance: 1e-3 max-abs (fp32 accumulation, f16 two-part
operands)."""
import math

import numpy as np
import pytest

from oracle import oracle as orc
from tq_testdata import bf16_bits, bf16_round, kv_outlier

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

D = 128
TOL = 1e-3
# staged tiles (K inverse-rotated once by the staging pass, the query taken
# unrotated) against tiles decoded in the workgroup (K rotated, the query
# rotated): the same products rounded in two domains
PATHS_TOL = 1e-4


@pytest.fixture(scope="module")
def tq():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import turboquant_amd
    return turboquant_amd


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _records(bits, outlier, x, cap):
    h, t, _ = x.shape
    p, s = orc.polar_quantize(bits, outlier, x.reshape(-1, D), D)
    d = orc.polar_dequantize(bits, outlier, p, s, D).reshape(h, t, D)
    pb = np.zeros((h, cap, p.shape[1]), np.uint8)
    sb = np.zeros((h, cap, 4), np.uint16)
    pb[:, :t] = p.reshape(h, t, -1)
    sb[:, :t] = s.reshape(h, t, 4)
    return _dev(pb), _dev(sb.view(np.int16)), d


@pytest.mark.parametrize("bits,outlier,hq,hkv,ql,t,causal", [
    (3, orc.OUTLIER_ALL, 16, 8, 100, 300, True),
    (4, orc.OUTLIER_ALL, 32, 8, 70, 129, True),
    (3, orc.OUTLIER_ALL, 8, 8, 64, 64, True),
    (3, 0, 16, 8, 33, 200, False),
    (4, 0, 16, 8, 1, 1000, True),
    (3, orc.OUTLIER_ALL, 16, 8, 257, 257, True),
])
def test_prefill_matches_dense_oracle(tq, bits, outlier, hq, hkv, ql, t, causal):
    rng = np.random.default_rng(700 + t + ql)
    k = kv_outlier(rng, hkv, t)
    v = kv_outlier(rng, hkv, t)
    cap = t + 5
    ki, ks, kd = _records(bits, outlier, k, cap)
    vi, vs, vd = _records(bits, outlier, v, cap)
    q = bf16_round(rng.standard_normal((hq, ql, D)).astype(np.float32) / np.float32(math.sqrt(D)))
    qd = _dev(bf16_bits(q)).view(torch.bfloat16)
    scale = 1 / math.sqrt(D)
    out = tq.cache_prefill_attention(qd, ki, ks, vi, vs, hkv, bits, t, cap, scale, outlier, causal=causal)
    torch.cuda.synchronize()
    ref = orc.attention_prefill(q, kd, vd, scale, causal)
    err = np.abs(out.cpu().numpy() - ref).max()
    assert err <= TOL, err


@pytest.mark.parametrize("bits", [3, 4])
def test_tq_cache_attend_prefill_with_qjl(tq, bits):
    hkv, hq, t, ql = 4, 8, 400, 48
    rng = np.random.default_rng(800 + bits)
    k = kv_outlier(rng, hkv, t)
    v = kv_outlier(rng, hkv, t)
    cache = tq.TqCache(tq.CacheConfig(bits=bits, head_dim=D, num_kv_heads=hkv, num_layers=1, outlier_blocks=0))
    q = rng.standard_normal((hq, ql, D)).astype(np.float32) / np.float32(math.sqrt(D))
    r = cache.prefill(0, _dev(k[None]), _dev(v[None]), _dev(q[None]))
    out = cache.attend_prefill(0, _dev(q[None]), 1 / math.sqrt(D))
    torch.cuda.synchronize()
    pk, sk = orc.polar_quantize(bits, 0, k.reshape(-1, D), D)
    pv, sv = orc.polar_quantize(bits, 0, v.reshape(-1, D), D)
    kd = orc.polar_dequantize(bits, 0, pk, sk, D)
    vd = orc.polar_dequantize(bits, 0, pv, sv, D).reshape(hkv, t, D)
    sg, nm = orc.tq_signs_norms(k.reshape(-1, D), kd)
    bias = orc.tq_logit_bias(q, sg.reshape(hkv, t, -1), nm.reshape(hkv, t))
    ref = orc.attention_prefill(q, kd.reshape(hkv, t, D), vd, 1 / math.sqrt(D), True, bias)
    err = np.abs(out[0].cpu().numpy() - ref).max()
    assert err <= TOL, err
    # the caller's alternative: SDPA on the dequantized result plus the returned bias
    np.testing.assert_allclose(r.logit_bias[0].cpu().numpy(), bias, rtol=0, atol=1e-5 * np.abs(bias).max())


def test_pqo_cache_attend_prefill_full_layer(tq):
    hkv, hq, t = 8, 16, 700
    rng = np.random.default_rng(900)
    k = kv_outlier(rng, hkv, t)
    v = kv_outlier(rng, hkv, t)
    cache = tq.PqoCache(2, hkv, D, 3)
    cache.prefill(1, _dev(k[None, :, :500]), _dev(v[None, :, :500]))
    cache.prefill(1, _dev(k[None, :, 500:]), _dev(v[None, :, 500:]))
    q = bf16_round(rng.standard_normal((hq, 200, D)).astype(np.float32) / np.float32(math.sqrt(D)))
    out = cache.attend_prefill(1, _dev(q[None]), 1 / math.sqrt(D), out_dtype=torch.float32)
    pk, sk = orc.pqo_quantize(3, k.reshape(-1, D), D)
    pv, sv = orc.pqo_quantize(3, v.reshape(-1, D), D)
    kd = orc.pqo_dequantize(3, pk, sk, D).reshape(hkv, t, D)
    vd = orc.pqo_dequantize(3, pv, sv, D).reshape(hkv, t, D)
    ref = orc.attention_prefill(q, kd, vd, 1 / math.sqrt(D), True)
    err = np.abs(out[0].cpu().numpy() - ref).max()
    assert err <= TOL, err


def test_prefill_bench_shape_sampled_rows(tq):
    """The bench's prefill shape (16 q-heads over 8 KV heads, 4096 queries
    over 4096 tokens, causal, PQO3, bf16 queries): every workgroup order and
    tile buffer of the full launch runs; sampled query positions (first and
    last query blocks, tile edges) are checked against the oracle.  A causal
    query at position p sees tokens 0..p, which is the oracle's non-causal
    single query over the first p + 1 records; K/V are the oracle's
    dequantization of the GPU's own codes."""
    h, hkv, t, bits = 16, 8, 4096, 3
    gen = torch.Generator(device="cuda").manual_seed(31)
    x = torch.randn((2, hkv * t, D), generator=gen, device="cuda")
    x[:, :, torch.tensor([3, 40, 77, 101], device="cuda")] *= 8.0
    pk, sk = tq.pqo_quantize(x[0].to(torch.bfloat16), bits)
    pv, sv = tq.pqo_quantize(x[1].to(torch.bfloat16), bits)
    q = (torch.randn((h, t, D), generator=gen, device="cuda") / math.sqrt(D)).to(torch.bfloat16)
    scale = 1 / math.sqrt(D)
    out = tq.cache_prefill_attention(q, pk, sk, pv, sv, hkv, bits, t, t, scale, orc.OUTLIER_ALL, causal=True)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    kd = orc.pqo_dequantize(bits, pk.cpu().numpy(), sk.cpu().numpy().view(np.uint16), D).reshape(hkv, t, D)
    vd = orc.pqo_dequantize(bits, pv.cpu().numpy(), sv.cpu().numpy().view(np.uint16), D).reshape(hkv, t, D)
    qf = q.float().cpu().numpy()
    for p in (0, 1, 63, 64, 1000, 2047, 2048 + 37, 4000, 4032, 4095):
        ref = orc.attention_prefill(qf[:, p:p + 1], kd[:, :p + 1], vd[:, :p + 1], scale, False)
        err = np.abs(out[:, p:p + 1] - ref).max()
        assert err <= TOL, (p, err)


@pytest.mark.parametrize("bits,outlier,hq,hkv,ql,t,causal,qdt", [
    (3, orc.OUTLIER_ALL, 16, 8, 300, 300, True, "bf16"),
    (4, orc.OUTLIER_ALL, 32, 8, 270, 333, True, "bf16"),
    (3, 0, 16, 16, 260, 260, False, "f16"),
    (4, 0, 8, 2, 400, 1000, True, "bf16"),
    (3, orc.OUTLIER_ALL, 16, 4, 513, 577, False, "f32"),
    (3, orc.OUTLIER_ALL, 16, 8, 300, 1100, True, "f16"),
])
def test_staged_and_in_workgroup_tiles(tq, monkeypatch, bits, outlier, hq, hkv, ql, t, causal, qdt):
    """Tiles decoded once by the staging pass (K inverse-rotated, the query
    unrotated: two products per key slice for bf16 and f16 queries, three
    for f32) and tiles decoded in every workgroup (TQ_PREFILL_STAGING forces
    either path): both within TOL of the oracle, within PATHS_TOL of each
    other.  Shapes: GQA 1, 2, 4 and 8, 3 and 4 bits, PQ and PQO codes, token
    counts that end inside a tile, queries after earlier tokens."""
    rng = np.random.default_rng(1700 + t + ql)
    k = kv_outlier(rng, hkv, t)
    v = kv_outlier(rng, hkv, t)
    cap = t + 3
    ki, ks, kd = _records(bits, outlier, k, cap)
    vi, vs, vd = _records(bits, outlier, v, cap)
    q = rng.standard_normal((hq, ql, D)).astype(np.float32) / np.float32(math.sqrt(D))
    if qdt == "bf16":
        q = bf16_round(q)
        qd = _dev(bf16_bits(q)).view(torch.bfloat16)
    elif qdt == "f16":
        q = q.astype(np.float16).astype(np.float32)
        qd = _dev(q).to(torch.float16)
    else:
        qd = _dev(q)
    scale = 1 / math.sqrt(D)
    outs = []
    for mode in ("0", "1"):
        monkeypatch.setenv("TQ_PREFILL_STAGING", mode)
        outs.append(tq.cache_prefill_attention(qd, ki, ks, vi, vs, hkv, bits, t, cap, scale, outlier,
                                               causal=causal, out_dtype=torch.float32))
    torch.cuda.synchronize()
    assert float((outs[0] - outs[1]).abs().max()) <= PATHS_TOL
    ref = orc.attention_prefill(q, kd, vd, scale, causal)
    for o in outs:
        err = np.abs(o.cpu().numpy() - ref).max()
        assert err <= TOL, err


@pytest.mark.parametrize("outlier", [orc.OUTLIER_ALL, 0])
def test_l2norm_cache_prefill_staged_and_in_workgroup(tq, monkeypatch, outlier):
    """A PqoCache on the L2Norm codebooks (PQO codes, and PQ codes in 3-bit
    slots): the staging pass and the in-workgroup decode read the caller's
    codebook from the launch arguments; both paths agree within PATHS_TOL
    and match the oracle's L2Norm dequantization within TOL."""
    bits, hkv, hq, t, ql = 3, 4, 8, 700, 300
    rng = np.random.default_rng(1900 + (1 if outlier else 0))
    k = kv_outlier(rng, hkv, t)
    v = kv_outlier(rng, hkv, t)
    cfg = tq.CacheConfig(bits=bits, head_dim=D, num_kv_heads=hkv, num_layers=1,
                         norm_mode=tq.QuantNormMode.L2Norm, outlier_blocks=outlier)
    cache = tq.PqoCache(cfg)
    cache.prefill(0, _dev(k[None]), _dev(v[None]))
    q = bf16_round(rng.standard_normal((hq, ql, D)).astype(np.float32) / np.float32(math.sqrt(D)))
    scale = 1 / math.sqrt(D)
    outs = []
    for mode in ("0", "1"):
        monkeypatch.setenv("TQ_PREFILL_STAGING", mode)
        outs.append(cache.attend_prefill(0, _dev(q[None]), scale, out_dtype=torch.float32))
    torch.cuda.synchronize()
    assert float((outs[0] - outs[1]).abs().max()) <= PATHS_TOL
    pk, sk = orc.polar_quantize(bits, outlier, k.reshape(-1, D), D, norm_mode=1)
    pv, sv = orc.polar_quantize(bits, outlier, v.reshape(-1, D), D, norm_mode=1)
    kd = orc.polar_dequantize(bits, outlier, pk, sk, D, norm_mode=1).reshape(hkv, t, D)
    vd = orc.polar_dequantize(bits, outlier, pv, sv, D, norm_mode=1).reshape(hkv, t, D)
    ref = orc.attention_prefill(q, kd, vd, scale, True)
    for o in outs:
        err = np.abs(o[0].cpu().numpy() - ref).max()
        assert err <= TOL, err


def test_staged_prefill_repeats_across_synchronizations(tq, monkeypatch):
    """The staging buffer comes from the library's own memory pool, which keeps
    its memory across synchronizations: staged launches separated by device
    synchronizations, on the default stream and on a second stream, give the
    same bits as the first."""
    monkeypatch.setenv("TQ_PREFILL_STAGING", "1")
    bits, hkv, hq, t = 3, 4, 8, 1100
    rng = np.random.default_rng(2100)
    k = kv_outlier(rng, hkv, t)
    v = kv_outlier(rng, hkv, t)
    ki, ks, _ = _records(bits, orc.OUTLIER_ALL, k, t)
    vi, vs, _ = _records(bits, orc.OUTLIER_ALL, v, t)
    q = bf16_round(rng.standard_normal((hq, 300, D)).astype(np.float32) / np.float32(math.sqrt(D)))
    qd = _dev(bf16_bits(q)).view(torch.bfloat16)
    scale = 1 / math.sqrt(D)

    def run():
        return tq.cache_prefill_attention(qd, ki, ks, vi, vs, hkv, bits, t, t, scale, orc.OUTLIER_ALL, causal=True)

    first = run()
    torch.cuda.synchronize()
    for _ in range(3):
        again = run()
        torch.cuda.synchronize()
        assert torch.equal(first, again)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        other = run()
    side.synchronize()
    assert torch.equal(first, other)


@pytest.mark.parametrize("bits,hq,hkv,ql,t,causal,qdt", [
    (3, 16, 4, 300, 700, True, "f32"),
    (4, 8, 8, 200, 333, False, "f32"),
    (3, 16, 8, 257, 257, True, "f32"),
    (3, 16, 8, 300, 1100, True, "bf16"),
    (4, 16, 4, 260, 600, False, "bf16"),
])
def test_tq_prefill_several_query_blocks(tq, monkeypatch, bits, hq, hkv, ql, t, causal, qdt):
    """TQ-cache prefill attention (QJL correction inside the key pass) over
    several 128-row workgroups per KV head, GQA 4, 1 and 2, causal and full:
    staged tiles (signs and norms in the image) and in-workgroup decode agree
    within PATHS_TOL and lie within TOL of the oracle's dequantized keys and
    values plus its logit bias."""
    rng = np.random.default_rng(2300 + t + ql)
    k = kv_outlier(rng, hkv, t)
    v = kv_outlier(rng, hkv, t)
    cache = tq.TqCache(tq.CacheConfig(bits=bits, head_dim=D, num_kv_heads=hkv, num_layers=1, outlier_blocks=0))
    q = rng.standard_normal((hq, ql, D)).astype(np.float32) / np.float32(math.sqrt(D))
    if qdt == "bf16":
        # (staged tiles take two products per key slice for a bf16 query)
        q = bf16_round(q)
        qd = _dev(bf16_bits(q)).view(torch.bfloat16)[None]
    else:
        qd = _dev(q[None])
    cache.prefill(0, _dev(k[None]), _dev(v[None]), _dev(q[None]))
    outs = []
    for mode in ("0", "1"):
        monkeypatch.setenv("TQ_PREFILL_STAGING", mode)
        outs.append(cache.attend_prefill(0, qd, 1 / math.sqrt(D), causal=causal, out_dtype=torch.float32))
    torch.cuda.synchronize()
    assert float((outs[0] - outs[1]).abs().max()) <= PATHS_TOL
    pk, sk = orc.polar_quantize(bits, 0, k.reshape(-1, D), D)
    pv, sv = orc.polar_quantize(bits, 0, v.reshape(-1, D), D)
    kd = orc.polar_dequantize(bits, 0, pk, sk, D)
    vd = orc.polar_dequantize(bits, 0, pv, sv, D).reshape(hkv, t, D)
    sg, nm = orc.tq_signs_norms(k.reshape(-1, D), kd)
    bias = orc.tq_logit_bias(q, sg.reshape(hkv, t, -1), nm.reshape(hkv, t))
    ref = orc.attention_prefill(q, kd.reshape(hkv, t, D), vd, 1 / math.sqrt(D), causal, bias)
    for o in outs:
        err = np.abs(o[0].cpu().numpy() - ref).max()
        assert err <= TOL, err


@pytest.mark.parametrize("bits,outlier,hq,hkv,ql,t,causal,splits,odt,staged", [
    (3, orc.OUTLIER_ALL, 16, 8, 64, 4097, True, None, "f32", "1"),
    (3, orc.OUTLIER_ALL, 16, 8, 64, 4097, False, None, "bf16", "1"),
    (4, 0, 16, 4, 1, 2000, True, None, "f32", "1"),
    (3, orc.OUTLIER_ALL, 32, 8, 100, 1500, True, "7", "f16", "1"),
    (3, orc.OUTLIER_ALL, 16, 8, 300, 1000, True, "8", "f32", "1"),
    (4, orc.OUTLIER_ALL, 8, 8, 130, 2500, False, "3", "f32", "1"),
    (3, orc.OUTLIER_ALL, 16, 8, 64, 4097, True, None, "f32", "0"),
    (3, orc.OUTLIER_ALL, 16, 4, 200, 1300, True, "5", "bf16", "0"),
    (4, 0, 16, 8, 1, 700, False, None, "f32", "0"),
])
def test_split_prefill(tq, monkeypatch, bits, outlier, hq, hkv, ql, t, causal, splits, odt, staged):
    """Prefill with its tiles split over several workgroups per query block
    (automatic when the grid would leave compute units idle, or forced with
    TQ_PREFILL_SPLITS, uneven and with empty splits for causal blocks that end
    before a split), on staged tiles and decoding in the workgroups, and the
    splits' merge: within PATHS_TOL of one split and TOL of the oracle, in
    f32, bf16 and f16 outputs."""
    rng = np.random.default_rng(2600 + t + ql)
    k = kv_outlier(rng, hkv, t)
    v = kv_outlier(rng, hkv, t)
    ki, ks, kd = _records(bits, outlier, k, t)
    vi, vs, vd = _records(bits, outlier, v, t)
    q = bf16_round(rng.standard_normal((hq, ql, D)).astype(np.float32) / np.float32(math.sqrt(D)))
    qd = _dev(bf16_bits(q)).view(torch.bfloat16)
    dt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[odt]
    scale = 1 / math.sqrt(D)
    monkeypatch.setenv("TQ_PREFILL_STAGING", staged)
    outs = []
    for sp in ("1", splits):
        if sp is None:
            monkeypatch.delenv("TQ_PREFILL_SPLITS", raising=False)
        else:
            monkeypatch.setenv("TQ_PREFILL_SPLITS", sp)
        outs.append(tq.cache_prefill_attention(qd, ki, ks, vi, vs, hkv, bits, t, t, scale, outlier, causal=causal,
                                               out_dtype=dt).float())
    torch.cuda.synchronize()
    rt = PATHS_TOL if odt == "f32" else 1e-2  # (two roundings of the same value to 16 bits may differ by an ulp)
    assert float((outs[0] - outs[1]).abs().max()) <= rt
    ref = orc.attention_prefill(q, kd, vd, scale, causal)
    tol = TOL if odt == "f32" else 1e-2
    for o in outs:
        err = np.abs(o.cpu().numpy() - ref).max()
        assert err <= tol, err


def test_split_prefill_tq_cache(tq, monkeypatch):
    """A TQ cache (QJL correction in the key pass) with few query blocks over a
    long context: automatic splits against one split and the oracle."""
    bits, hq, hkv, ql, t = 3, 16, 8, 64, 2100
    rng = np.random.default_rng(2700)
    k = kv_outlier(rng, hkv, t)
    v = kv_outlier(rng, hkv, t)
    cache = tq.TqCache(tq.CacheConfig(bits=bits, head_dim=D, num_kv_heads=hkv, num_layers=1, outlier_blocks=0))
    q = rng.standard_normal((hq, ql, D)).astype(np.float32) / np.float32(math.sqrt(D))
    cache.prefill(0, _dev(k[None]), _dev(v[None]), _dev(q[None]))
    outs = []
    for sp in ("1", None):
        if sp is None:
            monkeypatch.delenv("TQ_PREFILL_SPLITS", raising=False)
        else:
            monkeypatch.setenv("TQ_PREFILL_SPLITS", sp)
        outs.append(cache.attend_prefill(0, _dev(q[None]), 1 / math.sqrt(D), causal=True, out_dtype=torch.float32))
    torch.cuda.synchronize()
    assert float((outs[0] - outs[1]).abs().max()) <= PATHS_TOL
    pk, sk = orc.polar_quantize(bits, 0, k.reshape(-1, D), D)
    pv, sv = orc.polar_quantize(bits, 0, v.reshape(-1, D), D)
    kd = orc.polar_dequantize(bits, 0, pk, sk, D)
    vd = orc.polar_dequantize(bits, 0, pv, sv, D).reshape(hkv, t, D)
    sg, nm = orc.tq_signs_norms(k.reshape(-1, D), kd)
    bias = orc.tq_logit_bias(q, sg.reshape(hkv, t, -1), nm.reshape(hkv, t))
    ref = orc.attention_prefill(q, kd.reshape(hkv, t, D), vd, 1 / math.sqrt(D), True, bias)
    for o in outs:
        err = np.abs(o[0].cpu().numpy() - ref).max()
        assert err <= TOL, err
