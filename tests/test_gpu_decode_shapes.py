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
