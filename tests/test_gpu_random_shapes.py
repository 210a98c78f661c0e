"""Seeded random shapes through the library's own dispatch (no forced
paths): batched decode over ragged lengths (one-chunk heads written directly,
64 or 128 tokens per wave, 8- or 4-wave workgroups, ranges of chunks), and
prefill (in-workgroup or staged tiles, split over the tiles or not), each
against dense attention over the oracle's records (with the QJL logit bias
for TQ records).  Tolerance: 1e-3 max-abs."""
import math

import numpy as np
import pytest

from oracle import oracle as orc
from tq_testdata import bf16_bits, bf16_round, kv_outlier

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

TOL = 1e-3


@pytest.fixture(scope="module")
def tq():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import turboquant_amd
    return turboquant_amd


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _decode_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        qjl = bool(rng.random() < 0.3)
        d = int(rng.choice([64, 128, 128, 256]))
        bits = 3 if qjl else int(rng.choice([3, 4]))
        bsz = int(rng.choice([1, 1, 2, 3, 5]))
        hkv = int(rng.choice([1, 2, 4, 8]))
        nr = int(rng.choice([1, 2, 3, 4, 8, 16] if not qjl else [1, 2, 4, 8]))
        cap = int(rng.integers(1, 20001 if bsz == 1 else 6001))
        lens = rng.integers(0, cap + 1, size=bsz)
        if rng.random() < 0.5:
            lens[int(rng.integers(0, bsz))] = cap
        cases.append((i, qjl, d, bits, bsz, hkv, nr, cap, tuple(int(x) for x in lens)))
    return cases


@pytest.mark.parametrize("case", _decode_cases(24, 4242), ids=lambda c: f"dec{c[0]}")
def test_random_decode(tq, case):
    """QJL cases alternate between rq given and R q formed in the launch."""
    _, qjl, d, bits, bsz, hkv, nr, cap, lens = case
    rng = np.random.default_rng(9000 + case[0])
    h = hkv * nr
    pd, nb = d * bits // 8, d // 32
    ob = 0 if qjl else orc.OUTLIER_ALL
    kp = np.zeros((bsz, hkv, cap, pd), np.uint8)
    ks = np.zeros((bsz, hkv, cap, nb), np.int16)
    vp = np.zeros_like(kp)
    vs = np.zeros_like(ks)
    sgb = np.zeros((bsz, hkv, cap, d // 8), np.uint8)
    nmb = np.zeros((bsz, hkv, cap), np.int16)
    q = bf16_round(rng.standard_normal((bsz, h, d)).astype(np.float32) / np.float32(math.sqrt(d)))
    refs = []
    for b in range(bsz):
        t = lens[b]
        if t == 0:
            refs.append(np.zeros((h, d), np.float32))
            continue
        k = kv_outlier(rng, hkv, t, d).reshape(-1, d)
        v = kv_outlier(rng, hkv, t, d).reshape(-1, d)
        pk, sk = orc.polar_quantize(bits, ob, k, d)
        pv, sv = orc.polar_quantize(bits, ob, v, d)
        kd = orc.polar_dequantize(bits, ob, pk, sk, d).reshape(hkv, t, d)
        vd = orc.polar_dequantize(bits, ob, pv, sv, d).reshape(hkv, t, d)
        kp[b, :, :t] = pk.reshape(hkv, t, pd)
        ks[b, :, :t] = sk.view(np.int16).reshape(hkv, t, nb)
        vp[b, :, :t] = pv.reshape(hkv, t, pd)
        vs[b, :, :t] = sv.view(np.int16).reshape(hkv, t, nb)
        if qjl:
            sg, nm = orc.tq_signs_norms(k, kd.reshape(-1, d))
            sgb[b, :, :t] = sg.reshape(hkv, t, -1)
            nmb[b, :, :t] = nm.view(np.int16).reshape(hkv, t)
            bias = orc.tq_logit_bias(q[b][:, None, :], sg.reshape(hkv, t, -1), nm.reshape(hkv, t))[:, 0, :]
            refs.append(orc.attention_dense_bias(q[b], kd, vd, bias, 1 / math.sqrt(d)))
        else:
            refs.append(orc.attention_dense(q[b], kd, vd, 1 / math.sqrt(d)))
    ws = tq.AttentionWorkspace(bsz, h, hkv, d, cap)
    qd = _dev(bf16_bits(q)).view(torch.bfloat16)
    kw = {}
    if qjl:
        kw = dict(qjl_signs=_dev(sgb), qjl_norms=_dev(nmb))
        if case[0] % 2:  # R q formed inside the launch from the sign matrix
            kw["qjl_sign_matrix"] = tq.qjl_sign_matrix(d, 12345)
        else:
            rq = np.stack([[orc.query_projections(q[b, i], 12345) for i in range(h)] for b in range(bsz)])
            kw["rq"] = _dev(rq.astype(np.float32))
    out = tq.cache_decode_attention(qd, _dev(kp), _dev(ks), _dev(vp), _dev(vs), _dev(np.asarray(lens, np.int32)),
                                    hkv, bits, cap, cap, hkv * cap, 1 / math.sqrt(d), ws, ob, **kw)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    for b in range(bsz):
        assert np.abs(out[b] - refs[b]).max() <= TOL, (b, lens[b])


def _prefill_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        bits = int(rng.choice([3, 4]))
        outlier = int(rng.choice([orc.OUTLIER_ALL, 0]))
        hkv = int(rng.choice([2, 4, 8]))
        nr = int(rng.choice([1, 2, 4]))
        causal = bool(rng.random() < 0.7)
        ql = int(rng.integers(1, 321))
        t = int(rng.integers(ql if causal else 1, 3501))
        qdt = str(rng.choice(["bf16", "f32"]))
        cases.append((i, bits, outlier, hkv, nr, causal, ql, t, qdt))
    return cases


@pytest.mark.parametrize("case", _prefill_cases(12, 4343), ids=lambda c: f"pf{c[0]}")
def test_random_prefill(tq, case):
    _, bits, outlier, hkv, nr, causal, ql, t, qdt = case
    d = 128
    rng = np.random.default_rng(9500 + case[0])
    hq = hkv * nr
    k = kv_outlier(rng, hkv, t).reshape(-1, d)
    v = kv_outlier(rng, hkv, t).reshape(-1, d)
    pk, sk = orc.polar_quantize(bits, outlier, k, d)
    pv, sv = orc.polar_quantize(bits, outlier, v, d)
    kd = orc.polar_dequantize(bits, outlier, pk, sk, d).reshape(hkv, t, d)
    vd = orc.polar_dequantize(bits, outlier, pv, sv, d).reshape(hkv, t, d)
    q = rng.standard_normal((hq, ql, d)).astype(np.float32) / np.float32(math.sqrt(d))
    if qdt == "bf16":
        q = bf16_round(q)
        qd = _dev(bf16_bits(q)).view(torch.bfloat16)
    else:
        qd = _dev(q)
    out = tq.cache_prefill_attention(qd, _dev(pk), _dev(sk.view(np.int16)), _dev(pv), _dev(sv.view(np.int16)), hkv,
                                     bits, t, t, 1 / math.sqrt(d), outlier, causal=causal, out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = orc.attention_prefill(q, kd, vd, 1 / math.sqrt(d), causal)
    err = np.abs(out.cpu().numpy() - ref).max()
    assert err <= TOL, err
