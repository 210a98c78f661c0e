"""GPU parity of the fused decode over every head_dim and GQA ratio the cache
takes (the reference kernel handles up to 8 qblocks, head_dim <= 256, and
any ratio kv_head = head / (H / H_kv): tq_attention_kernel.cu:26,92-101):

* head_dim 32, 64, 128, 256 with PQO3 and PQO4 records;
* GQA ratios 1-8 in one pass and 16 (two head groups over the same KV head);
* a Falcon3-1B-like shape (head_dim 64, 8 KV heads; docs/benchmarks.md:55-61)
  and 64 query heads over 8 KV heads;
* TQ records (standard codebook + the keys' QJL sketch, the correction in
  the logits) at head_dim 64, 128 and 256;
* the reference ABI (tq_fused_attention) at head_dim 64 and GQA 8.

Oracle: the CPU restatement's dequantize, then dense softmax attention in
double (with the QJL logit bias for TQ); tolerance 1e-3 max-abs (BASELINE
north_star).
"""
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


def _records(rng, hkv, t, cap, d, bits, outlier_blocks=orc.OUTLIER_ALL):
    k = kv_outlier(rng, hkv, t, d).reshape(-1, d)
    v = kv_outlier(rng, hkv, t, d).reshape(-1, d)
    pk, sk = orc.polar_quantize(bits, outlier_blocks, k, d)
    pv, sv = orc.polar_quantize(bits, outlier_blocks, v, d)
    kd = orc.polar_dequantize(bits, outlier_blocks, pk, sk, d).reshape(hkv, t, d)
    vd = orc.polar_dequantize(bits, outlier_blocks, pv, sv, d).reshape(hkv, t, d)
    pd, nb = d * bits // 8, d // 32

    def lay(a, w, dt):
        buf = np.zeros((hkv, cap, w), dt)
        buf[:, :t] = a.reshape(hkv, t, w)
        return _dev(buf)

    recs = (lay(pk, pd, np.uint8), lay(sk.view(np.int16), nb, np.int16), lay(pv, pd, np.uint8),
            lay(sv.view(np.int16), nb, np.int16))
    return recs, k.reshape(hkv, t, d), kd, vd


def _decode(tq, q, recs, hkv, t, cap, d, bits, outlier_blocks=orc.OUTLIER_ALL, qjl=None):
    h = q.shape[0]
    ws = tq.AttentionWorkspace(1, h, hkv, d, cap)
    qd = _dev(bf16_bits(q)).view(torch.bfloat16).reshape(1, h, d)
    lens = torch.tensor([t], dtype=torch.int32, device="cuda")
    kw = {} if qjl is None else dict(rq=qjl[0], qjl_signs=qjl[1], qjl_norms=qjl[2])
    out = tq.cache_decode_attention(qd, *recs, lens, hkv, bits, cap, cap, 0, 1 / math.sqrt(d), ws,
                                    outlier_blocks, **kw)
    torch.cuda.synchronize()
    return out.cpu().numpy().reshape(h, d)


@pytest.mark.parametrize("d", [32, 64, 128, 256])
@pytest.mark.parametrize("bits", [3, 4])
@pytest.mark.parametrize("nr", [1, 2, 4, 8])
def test_head_dims_and_ratios(tq, d, bits, nr):
    hkv, t = 2, 1300
    rng = np.random.default_rng(d * 10 + bits + nr * 1000)
    recs, _, kd, vd = _records(rng, hkv, t, t + 11, d, bits)
    q = bf16_round(rng.standard_normal((hkv * nr, d)).astype(np.float32) / np.float32(math.sqrt(d)))
    ref = orc.attention_dense(q, kd, vd, 1 / math.sqrt(d))
    out = _decode(tq, q, recs, hkv, t, t + 11, d, bits)
    assert np.abs(out - ref).max() <= TOL


@pytest.mark.parametrize("nr", [3, 5, 6, 7, 16])
def test_any_gqa_ratio(tq, nr):
    """Ratios that leave a head group partly empty (3, 5-7) or need two head
    groups reading the same KV head (16)."""
    hkv, t, d, bits = 2, 2200, 128, 3
    rng = np.random.default_rng(500 + nr)
    recs, _, kd, vd = _records(rng, hkv, t, t, d, bits)
    q = bf16_round(rng.standard_normal((hkv * nr, d)).astype(np.float32) / np.float32(math.sqrt(d)))
    ref = orc.attention_dense(q, kd, vd, 1 / math.sqrt(d))
    assert np.abs(_decode(tq, q, recs, hkv, t, t, d, bits) - ref).max() <= TOL


@pytest.mark.parametrize("shape", [(16, 8, 64, 4100), (64, 8, 128, 3000)], ids=["falcon3-1b", "gqa8-64q"])
def test_model_shapes(tq, shape):
    h, hkv, d, t = shape
    rng = np.random.default_rng(h + d)
    recs, _, kd, vd = _records(rng, hkv, t, t, d, 3)
    q = bf16_round(rng.standard_normal((h, d)).astype(np.float32) / np.float32(math.sqrt(d)))
    ref = orc.attention_dense(q, kd, vd, 1 / math.sqrt(d))
    assert np.abs(_decode(tq, q, recs, hkv, t, t, d, 3) - ref).max() <= TOL


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("nr", [2, 8])
def test_tq_records_with_qjl_correction(tq, d, nr):
    """TQ3 records (2-bit standard codes in 3-bit slots) with the keys' QJL
    sketch; the logits carry softmax_scale * |r| sqrt(pi/2)/sqrt(d) *
    sum_j rq_j (2 b_j - 1) (tq_attention_kernel.cu:192-231, tq.rs:185-253)."""
    hkv, t, bits = 2, 900, 3
    rng = np.random.default_rng(800 + d + nr)
    recs, k, kd, vd = _records(rng, hkv, t, t, d, bits, outlier_blocks=0)
    sg, nm = orc.tq_signs_norms(k.reshape(-1, d), kd.reshape(-1, d))
    h = hkv * nr
    q = bf16_round(rng.standard_normal((h, d)).astype(np.float32) / np.float32(math.sqrt(d)))
    rq = np.stack([orc.query_projections(q[i], 12345) for i in range(h)])
    bias = orc.tq_logit_bias(q[:, None, :], sg.reshape(hkv, t, -1), nm.reshape(hkv, t))[:, 0, :]
    ref = orc.attention_dense_bias(q, kd, vd, bias, 1 / math.sqrt(d))
    qjl = (_dev(rq).reshape(1, h, d), _dev(sg.reshape(hkv, t, -1)), _dev(nm.view(np.int16).reshape(hkv, t)))
    out = _decode(tq, q, recs, hkv, t, t, d, bits, outlier_blocks=0, qjl=qjl)
    assert np.abs(out - ref).max() <= TOL


@pytest.mark.parametrize("d,nr", [(64, 2), (128, 8)])
def test_reference_abi_shapes(tq, d, nr):
    hkv, t, cap, bits = 4, 1500, 1600, 4
    rng = np.random.default_rng(900 + d + nr)
    recs, _, kd, vd = _records(rng, hkv, t, cap, d, bits)
    q = rng.standard_normal((hkv * nr, d)).astype(np.float32) / np.float32(math.sqrt(d))
    ref = orc.attention_dense(q, kd, vd, 1 / math.sqrt(d))
    c, _, _ = orc.pqo_codebook(bits)
    cb, sg = _dev(c), _dev(orc.pqo_decode_signs())
    out = tq.fused_attention(_dev(q), *recs, cb, sg, hkv, t, cap, bits, 1 / math.sqrt(d))
    torch.cuda.synchronize()
    assert np.abs(out.cpu().numpy() - ref).max() <= TOL


@pytest.mark.parametrize("bits,nr", [(3, 2), (4, 4)])
def test_batched_ragged_grid_over_the_compute_units(tq, bits, nr):
    """A batch whose grid of 8-wave workgroups exceeds the compute units runs
    the 4-wave form (twice the chunks per sequence, each merged the same
    way); ragged lengths, one of them empty, one a single token."""
    bsz, hkv, d, cap = 24, 8, 128, 1400
    rng = np.random.default_rng(70 + bits + nr)
    lens = rng.integers(1100, cap + 1, size=bsz)
    lens[3], lens[7] = 0, 1
    h = hkv * nr
    pd, nb = d * bits // 8, d // 32
    kp = np.zeros((bsz, hkv, cap, pd), np.uint8)
    ks = np.zeros((bsz, hkv, cap, nb), np.int16)
    vp = np.zeros_like(kp)
    vs = np.zeros_like(ks)
    q = bf16_round(rng.standard_normal((bsz, h, d)).astype(np.float32) / np.float32(math.sqrt(d)))
    refs = []
    for b in range(bsz):
        t = int(lens[b])
        if t == 0:
            refs.append(np.zeros((h, d), np.float32))
            continue
        k = kv_outlier(rng, hkv, t, d).reshape(-1, d)
        v = kv_outlier(rng, hkv, t, d).reshape(-1, d)
        pk, sk = orc.polar_quantize(bits, orc.OUTLIER_ALL, k, d)
        pv, sv = orc.polar_quantize(bits, orc.OUTLIER_ALL, v, d)
        kd = orc.polar_dequantize(bits, orc.OUTLIER_ALL, pk, sk, d).reshape(hkv, t, d)
        vd = orc.polar_dequantize(bits, orc.OUTLIER_ALL, pv, sv, d).reshape(hkv, t, d)
        kp[b, :, :t] = pk.reshape(hkv, t, pd)
        ks[b, :, :t] = sk.view(np.int16).reshape(hkv, t, nb)
        vp[b, :, :t] = pv.reshape(hkv, t, pd)
        vs[b, :, :t] = sv.view(np.int16).reshape(hkv, t, nb)
        refs.append(orc.attention_dense(q[b], kd, vd, 1 / math.sqrt(d)))
    assert bsz * hkv * -(-cap // 1024) > 256  # the 8-wave grid would exceed 256 compute units
    ws = tq.AttentionWorkspace(bsz, h, hkv, d, cap)
    qd = _dev(bf16_bits(q)).view(torch.bfloat16)
    out = tq.cache_decode_attention(qd, _dev(kp), _dev(ks), _dev(vp), _dev(vs),
                                    _dev(lens.astype(np.int32)), hkv, bits, cap, cap, hkv * cap,
                                    1 / math.sqrt(d), ws, orc.OUTLIER_ALL)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    for b in range(bsz):
        assert np.abs(out[b] - refs[b]).max() <= TOL, b


@pytest.mark.parametrize("bits,nr", [(3, 2), (4, 4)])
def test_batched_ranges_of_chunks(tq, bits, nr):
    """A batch whose single-chunk grid needs several rounds of resident
    workgroups runs ranges of several chunks per workgroup (one online softmax
    over the range, the value sums rescaled as the running max and V-scale
    exponent move); ragged lengths: empty, one token, exactly a chunk
    multiple, the capacity, and ranges left partly or wholly empty."""
    bsz, hkv, d, cap = 12, 8, 128, 9000
    rng = np.random.default_rng(90 + bits + nr)
    lens = rng.integers(1, cap + 1, size=bsz)
    lens[2], lens[5], lens[7], lens[9] = 0, 1, 4096, cap
    h = hkv * nr
    pd, nb = d * bits // 8, d // 32
    kp = np.zeros((bsz, hkv, cap, pd), np.uint8)
    ks = np.zeros((bsz, hkv, cap, nb), np.int16)
    vp = np.zeros_like(kp)
    vs = np.zeros_like(ks)
    q = bf16_round(rng.standard_normal((bsz, h, d)).astype(np.float32) / np.float32(math.sqrt(d)))
    refs = []
    for b in range(bsz):
        t = int(lens[b])
        if t == 0:
            refs.append(np.zeros((h, d), np.float32))
            continue
        k = kv_outlier(rng, hkv, t, d).reshape(-1, d)
        v = kv_outlier(rng, hkv, t, d).reshape(-1, d)
        # a late stretch of keys much larger than the rest: the running max
        # moves up several chunks into a range
        k[-min(t, 700) // 2:] *= 3.0
        pk, sk = orc.polar_quantize(bits, orc.OUTLIER_ALL, k, d)
        pv, sv = orc.polar_quantize(bits, orc.OUTLIER_ALL, v, d)
        kd = orc.polar_dequantize(bits, orc.OUTLIER_ALL, pk, sk, d).reshape(hkv, t, d)
        vd = orc.polar_dequantize(bits, orc.OUTLIER_ALL, pv, sv, d).reshape(hkv, t, d)
        kp[b, :, :t] = pk.reshape(hkv, t, pd)
        ks[b, :, :t] = sk.view(np.int16).reshape(hkv, t, nb)
        vp[b, :, :t] = pv.reshape(hkv, t, pd)
        vs[b, :, :t] = sv.view(np.int16).reshape(hkv, t, nb)
        refs.append(orc.attention_dense(q[b], kd, vd, 1 / math.sqrt(d)))
    # 4-wave chunks of 512 tokens: 18 per (sequence, KV head), 1,728 in all,
    # beyond one round of 768 resident workgroups
    assert bsz * hkv * -(-cap // 512) > 3 * 256
    ws = tq.AttentionWorkspace(bsz, h, hkv, d, cap)
    qd = _dev(bf16_bits(q)).view(torch.bfloat16)
    out = tq.cache_decode_attention(qd, _dev(kp), _dev(ks), _dev(vp), _dev(vs),
                                    _dev(lens.astype(np.int32)), hkv, bits, cap, cap, hkv * cap,
                                    1 / math.sqrt(d), ws, orc.OUTLIER_ALL)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    for b in range(bsz):
        assert np.abs(out[b] - refs[b]).max() <= TOL, (b, int(lens[b]))
    # a second call re-arms every counter it used
    out2 = tq.cache_decode_attention(qd, _dev(kp), _dev(ks), _dev(vp), _dev(vs),
                                     _dev(lens.astype(np.int32)), hkv, bits, cap, cap, hkv * cap,
                                     1 / math.sqrt(d), ws, orc.OUTLIER_ALL)
    torch.cuda.synchronize()
    assert np.array_equal(out2.cpu().numpy(), out)


@pytest.mark.parametrize("kv_len", [1000, 4097])
@pytest.mark.parametrize("d,nr,qjl", [(256, 4, False), (256, 8, False), (128, 8, True), (256, 4, True)],
                         ids=["d256-gqa4", "d256-gqa8", "d128-gqa8-qjl", "d256-gqa4-qjl"])
def test_reference_abi_partition_contract(tq, d, nr, qjl, kv_len):
    """tq_fused_attention with exactly the reference caller's partial buffers,
    ceil(kv_len / 512) partitions (cuda/attention.rs:70-77), at shapes whose
    operands only fit 4-wave workgroups of 64 tokens per wave (256-token
    chunks, taken in 512-token ranges): the output matches the oracle and no
    byte past the caller's partials is written (a NaN guard after each
    buffer)."""
    hkv, bits = 2, 3
    cap = kv_len + 7
    rng = np.random.default_rng(1200 + d + nr + kv_len + 7 * qjl)
    ob = 0 if qjl else orc.OUTLIER_ALL
    recs, k, kd, vd = _records(rng, hkv, kv_len, cap, d, bits, outlier_blocks=ob)
    h = hkv * nr
    q = rng.standard_normal((h, d)).astype(np.float32) / np.float32(math.sqrt(d))
    if qjl:
        sg, nm = orc.tq_signs_norms(k.reshape(-1, d), kd.reshape(-1, d))
        rq = np.stack([orc.query_projections(q[i], 12345) for i in range(h)])
        bias = orc.tq_logit_bias(q[:, None, :], sg.reshape(hkv, kv_len, -1), nm.reshape(hkv, kv_len))[:, 0, :]
        ref = orc.attention_dense_bias(q, kd, vd, bias, 1 / math.sqrt(d))
        sgb = np.zeros((hkv, cap, d // 8), np.uint8)
        sgb[:, :kv_len] = sg.reshape(hkv, kv_len, -1)
        nmb = np.zeros((hkv, cap), np.int16)
        nmb[:, :kv_len] = nm.view(np.int16).reshape(hkv, kv_len)
        c, _, _ = orc.pqo_codebook(bits - 1)
        c = np.concatenate([c, np.zeros((1 << bits) - c.size, np.float32)])
        sgd, nmd, rqd = _dev(sgb), _dev(nmb), _dev(rq)
    else:
        ref = orc.attention_dense(q, kd, vd, 1 / math.sqrt(d))
        c, _, _ = orc.pqo_codebook(bits)
        sgd = nmd = rqd = None
    p = (kv_len + 511) // 512
    guard = 64
    po = torch.full((h * p * d + guard,), float("nan"), dtype=torch.float32, device="cuda")
    pm = torch.full((h * p + guard,), float("nan"), dtype=torch.float32, device="cuda")
    ps = torch.full((h * p + guard,), float("nan"), dtype=torch.float32, device="cuda")
    out = torch.zeros((h * d + guard,), dtype=torch.float32, device="cuda")
    qd, cb, sgp = _dev(q), _dev(c), _dev(orc.pqo_decode_signs())
    ptr = lambda t: None if t is None else t.data_ptr()
    tq.check(tq.lib.tq_fused_attention(qd.data_ptr(), *(r.data_ptr() for r in recs), cb.data_ptr(), sgp.data_ptr(),
                                       out.data_ptr(), po.data_ptr(), pm.data_ptr(), ps.data_ptr(), ptr(sgd),
                                       ptr(nmd), ptr(rqd), int(qjl), h, hkv, d, kv_len, cap, d * bits // 8, d // 32,
                                       bits, float(1 / math.sqrt(d)), p, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    assert np.abs(o[:h * d].reshape(h, d) - ref).max() <= TOL
    assert np.all(o[h * d:] == 0)
    for t, n in ((po, h * p * d), (pm, h * p), (ps, h * p)):
        assert np.isnan(t[n:].cpu().numpy()).all(), "write past the caller's partials"


def _ragged_batch(tq, bsz, hkv, d, cap, bits, nr, lens, seed, qjl=False):
    """Batched decode of ragged sequences through tq_cache_decode_attention,
    each sequence checked against dense attention over the oracle's records
    (with the QJL logit bias for TQ records)."""
    rng = np.random.default_rng(seed)
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
    rq = np.stack([[orc.query_projections(q[b, i], 12345) for i in range(h)] for b in range(bsz)]) if qjl else None
    refs = []
    for b in range(bsz):
        t = int(lens[b])
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
    kw = {} if not qjl else dict(rq=_dev(rq.astype(np.float32)), qjl_signs=_dev(sgb), qjl_norms=_dev(nmb))
    out = tq.cache_decode_attention(qd, _dev(kp), _dev(ks), _dev(vp), _dev(vs),
                                    _dev(np.asarray(lens, np.int32)), hkv, bits, cap, cap, hkv * cap,
                                    1 / math.sqrt(d), ws, ob, **kw)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    for b in range(bsz):
        assert np.abs(out[b] - refs[b]).max() <= TOL, b


@pytest.mark.parametrize("bits,nr,d", [(3, 2, 128), (4, 4, 128), (4, 8, 64), (3, 1, 256), (4, 4, 256)])
def test_balanced_split_ragged_batch(tq, bits, nr, d):
    """A batch whose chunks exceed one round of resident workgroups, at most
    64 sequences and one head group per KV head: the balanced split (each
    sequence's chunks cut into near-equal ranges so that every workgroup
    gets at most the same number), with empty, single-token and near-capacity
    sequences."""
    bsz, hkv, cap = 40, 8, 3000
    rng = np.random.default_rng(300 + bits + nr + d)
    lens = rng.integers(0, cap + 1, size=bsz)
    lens[[2, 9, 17]] = 0
    lens[[5, 23]] = 1
    lens[11] = cap
    assert -(-cap // 512) * hkv * bsz > 3 * 256  # more tasks than one round holds
    _ragged_batch(tq, bsz, hkv, d, cap, bits, nr, lens, 301 + d)


@pytest.mark.parametrize("case", ["batch70", "gqa16", "all_empty", "tq"])
def test_range_split_cases(tq, case):
    """Range launches outside the balanced split (more than 64 sequences; two
    head groups per KV head), a batch of empty sequences under a large
    capacity, and TQ records with the QJL correction under the balanced
    split."""
    if case == "batch70":
        lens = np.random.default_rng(7).integers(0, 2001, size=70)
        _ragged_batch(tq, 70, 4, 64, 2000, 4, 2, lens, 71)
    elif case == "gqa16":
        lens = np.random.default_rng(8).integers(1, 4001, size=12)
        _ragged_batch(tq, 12, 4, 128, 4000, 3, 16, lens, 72)
    elif case == "all_empty":
        _ragged_batch(tq, 30, 8, 128, 5000, 3, 2, np.zeros(30, np.int64), 73)
    else:
        lens = np.random.default_rng(9).integers(0, 2501, size=36)
        lens[4] = 0
        _ragged_batch(tq, 36, 8, 128, 2500, 3, 2, lens, 74, qjl=True)


def _f16_bits(x):
    return np.asarray(x, np.float16).view(np.int16)


@pytest.mark.parametrize("qdt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("d,nr,bsz", [(64, 2, 1), (128, 8, 1), (256, 4, 1), (128, 2, 24), (256, 2, 40)])
def test_in_launch_query_projection(tq, d, nr, bsz, qdt):
    """tq_tq_decode_attention (rq = R q computed inside the decode launch, on
    the matrix cores: +-1 entries times the query cut into exact bf16 parts,
    one part for bf16 queries, two for f16, three for f32) against
    tq_qjl_project (a serial f32 sum per element) + tq_cache_decode_attention:
    every product is exact and only the accumulation order differs, so the
    outputs agree to rounding, 1e-5 here (single sequences and ragged
    batches on the balanced split)."""
    hkv, cap, bits = 4 if bsz == 1 else 8, 1800, 3
    h = hkv * nr
    rng = np.random.default_rng(d * 7 + nr + bsz)
    pd, nb = d * bits // 8, d // 32
    # TQ records: 2-bit codes in 3-bit slots (top bit of every slot zero)
    codes = rng.integers(0, 4, size=(2, bsz, hkv, cap, d))
    packed = []
    for c in codes:
        bitsarr = np.zeros(c.shape[:-1] + (d * bits,), np.uint8)
        for b in range(2):
            bitsarr[..., b::bits] = (c >> b) & 1
        packed.append(np.packbits(bitsarr, axis=-1, bitorder="little"))
    sc = [_f16_bits(np.abs(rng.standard_normal((bsz, hkv, cap, nb))) + 0.05) for _ in range(2)]
    sg = rng.integers(0, 256, size=(bsz, hkv, cap, d // 8), dtype=np.uint8)
    nm = _f16_bits(np.abs(rng.standard_normal((bsz, hkv, cap))) * 0.3)
    lens = rng.integers(0, cap + 1, size=bsz).astype(np.int32) if bsz > 1 else np.array([cap - 5], np.int32)
    q = rng.standard_normal((bsz, h, d)).astype(np.float32) / np.float32(math.sqrt(d))
    if qdt == "bf16":
        qd = _dev(bf16_bits(bf16_round(q))).view(torch.bfloat16)
    elif qdt == "f16":
        qd = _dev(q.astype(np.float16))
    else:
        qd = _dev(q)
    rmat = tq.qjl_sign_matrix(d, 12345)
    rq = tq.qjl_project(qd.reshape(-1, d), rmat).reshape(bsz, h, d)
    ws = tq.AttentionWorkspace(bsz, h, hkv, d, cap)
    args = (qd, _dev(packed[0]), _dev(sc[0]), _dev(packed[1]), _dev(sc[1]), _dev(lens), hkv, bits, cap, cap,
            hkv * cap, 1 / math.sqrt(d), ws, 0)
    a = tq.cache_decode_attention(*args, rq=rq, qjl_signs=_dev(sg), qjl_norms=_dev(nm))
    b = tq.cache_decode_attention(*args, qjl_signs=_dev(sg), qjl_norms=_dev(nm), qjl_sign_matrix=rmat)
    torch.cuda.synchronize()
    a, b = a.cpu().numpy(), b.cpu().numpy()
    assert np.isfinite(a).all() and np.isfinite(b).all()
    assert np.abs(a - b).max() <= 1e-5, np.abs(a - b).max()
