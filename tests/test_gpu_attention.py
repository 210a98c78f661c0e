"""GPU parity of the fused PQO decode attention against the oracle.

Oracle: dequantize the compressed K/V with the CPU restatement, then dense
softmax attention accumulated in double.  Tolerance:
max |out - ref| <= 1e-3, fp32 accumulation, bf16/f16/f32 query I/O.
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


def _make_cache(rng, hkv, t, bits, cap=None):
    """Quantize K/V [hkv, t, 128] with the oracle; returns device cache tensors
    laid out [hkv, cap, ...] plus the oracle's dequantized K/V."""
    cap = cap or t
    k = kv_outlier(rng, hkv, t)
    v = kv_outlier(rng, hkv, t)
    pk, sk = orc.pqo_quantize(bits, k.reshape(-1, 128), 128)
    pv, sv = orc.pqo_quantize(bits, v.reshape(-1, 128), 128)
    kd = orc.pqo_dequantize(bits, pk, sk, 128).reshape(hkv, t, 128)
    vd = orc.pqo_dequantize(bits, pv, sv, 128).reshape(hkv, t, 128)
    pd = 128 * bits // 8

    def lay(a, w, dt):
        buf = np.zeros((hkv, cap, w), dt)
        buf[:, :t] = a.reshape(hkv, t, w)
        return _dev(buf)

    return (lay(pk, pd, np.uint8), lay(sk.view(np.int16), 4, np.int16), lay(pv, pd, np.uint8),
            lay(sv.view(np.int16), 4, np.int16), kd, vd)


def _run_decode(tq, q_np, cache, hkv, t, bits, cap, qdtype=torch.float32, out_dtype=torch.float32, reps=1):
    kidx, ksc, vidx, vsc, _, _ = cache
    h = q_np.shape[0]
    if qdtype == torch.bfloat16:
        q = _dev(bf16_bits(q_np)).view(torch.bfloat16)
    elif qdtype == torch.float16:
        q = _dev(q_np.astype(np.float16))
    else:
        q = _dev(q_np)
    q = q.reshape(1, h, 128)
    lens = torch.tensor([t], dtype=torch.int32, device="cuda")
    ws = tq.AttentionWorkspace(1, h, hkv, 128, t)
    outs = []
    for _ in range(reps):
        outs.append(tq.pqo_decode_attention(q, kidx, ksc, vidx, vsc, lens, hkv, bits, t, cap, 0,
                                            1.0 / math.sqrt(128), ws, out_dtype=out_dtype))
    torch.cuda.synchronize()
    return [o.float().cpu().numpy().reshape(h, 128) for o in outs]


@pytest.mark.parametrize("bits,h,hkv,t", [(3, 16, 8, 1000), (4, 32, 8, 777), (3, 8, 8, 1), (4, 4, 4, 256),
                                          (3, 16, 8, 257), (4, 32, 8, 5000),
                                          (3, 32, 8, 17000),
                                          # more chunks than the merge's first round (32)
                                          (4, 8, 8, 33000)])
def test_decode_matches_dense_oracle(tq, bits, h, hkv, t):
    rng = np.random.default_rng(1000 + t + bits)
    cap = t + 37
    cache = _make_cache(rng, hkv, t, bits, cap)
    q = bf16_round(rng.standard_normal((h, 128)).astype(np.float32) / np.float32(math.sqrt(128)))
    ref = orc.attention_dense(q, cache[4], cache[5], 1.0 / math.sqrt(128))
    for qdt in (torch.float32, torch.bfloat16):
        (out,) = _run_decode(tq, q, cache, hkv, t, bits, cap, qdtype=qdt)
        err = np.abs(out - ref).max()
        assert err <= TOL, (qdt, err)


def test_decode_repeated_calls_rearm_counters(tq):
    rng = np.random.default_rng(5)
    t, hkv, h, bits = 3000, 8, 16, 3
    cache = _make_cache(rng, hkv, t, bits)
    q = bf16_round(rng.standard_normal((h, 128)).astype(np.float32) / np.float32(math.sqrt(128)))
    outs = _run_decode(tq, q, cache, hkv, t, bits, t, reps=4)
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])


def test_decode_graph_replays_match_eager(tq):
    """The decode captured in a HIP graph (as bench.py times it): every replay,
    with eager work and synchronizations between replays, equals the eager
    result bit for bit and the oracle to TOL."""
    rng = np.random.default_rng(6)
    t, hkv, h, bits = 4100, 8, 16, 3
    cache = _make_cache(rng, hkv, t, bits)
    kidx, ksc, vidx, vsc, kd, vd = cache
    qn = bf16_round(rng.standard_normal((h, 128)).astype(np.float32) / np.float32(math.sqrt(128)))
    ref = orc.attention_dense(qn, kd, vd, 1.0 / math.sqrt(128))
    q = _dev(bf16_bits(qn)).view(torch.bfloat16).reshape(1, h, 128)
    lens = torch.tensor([t], dtype=torch.int32, device="cuda")
    ws = tq.AttentionWorkspace(1, h, hkv, 128, t)
    out = torch.empty((1, h, 128), dtype=torch.float32, device="cuda")

    def step():
        tq.pqo_decode_attention(q, kidx, ksc, vidx, vsc, lens, hkv, bits, t, t, 0, 1.0 / math.sqrt(128), ws, out=out)

    step()
    torch.cuda.synchronize()
    eager = out.cpu().numpy().reshape(h, 128).copy()
    assert np.abs(eager - ref).max() <= TOL
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
        step()
    for rep in range(4):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        got = out.cpu().numpy().reshape(h, 128)
        assert np.array_equal(got, eager), rep
        step()  # eager work between replays
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().reshape(h, 128), eager), rep


def test_decode_c3_full_size(tq):
    """BASELINE config 3 at full size: 16 q-heads / 8 KV heads, ctx 32,768, PQO3."""
    rng = np.random.default_rng(3)
    t, hkv, h, bits = 32768, 8, 16, 3
    cache = _make_cache(rng, hkv, t, bits)
    q = bf16_round(rng.standard_normal((h, 128)).astype(np.float32) / np.float32(math.sqrt(128)))
    ref = orc.attention_dense(q, cache[4], cache[5], 1.0 / math.sqrt(128))
    (out,) = _run_decode(tq, q, cache, hkv, t, bits, t, qdtype=torch.bfloat16)
    assert np.abs(out - ref).max() <= TOL


def test_decode_batched_varlen(tq):
    """Config-4 shape at reduced size: batch of sequences with different lengths,
    GQA 4:1, PQO4, each sequence checked against the dense oracle."""
    rng = np.random.default_rng(4)
    bits, h, hkv = 4, 32, 8
    lens = [40, 513, 1, 2048, 777]
    cap = max(lens) + 5
    bsz = len(lens)
    pd = 128 * bits // 8
    kidx = np.zeros((bsz, hkv, cap, pd), np.uint8)
    vidx = np.zeros_like(kidx)
    ksc = np.zeros((bsz, hkv, cap, 4), np.int16)
    vsc = np.zeros_like(ksc)
    refs = []
    qs = bf16_round(rng.standard_normal((bsz, h, 128)).astype(np.float32) / np.float32(math.sqrt(128)))
    for bi, t in enumerate(lens):
        c = _make_cache(rng, hkv, t, bits)
        kidx[bi, :, :t] = c[0].cpu().numpy()
        ksc[bi, :, :t] = c[1].cpu().numpy()
        vidx[bi, :, :t] = c[2].cpu().numpy()
        vsc[bi, :, :t] = c[3].cpu().numpy()
        refs.append(orc.attention_dense(qs[bi], c[4], c[5], 1.0 / math.sqrt(128)))
    ws = tq.AttentionWorkspace(bsz, h, hkv, 128, cap)
    out = tq.pqo_decode_attention(_dev(bf16_bits(qs)).view(torch.bfloat16), _dev(kidx), _dev(ksc), _dev(vidx),
                                  _dev(vsc), torch.tensor(lens, dtype=torch.int32, device="cuda"), hkv, bits, cap,
                                  cap, hkv * cap, 1.0 / math.sqrt(128), ws)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    for bi in range(bsz):
        assert np.abs(out[bi] - refs[bi]).max() <= TOL, bi


def test_decode_c4_full_size(tq):
    """BASELINE config 4 at full size: PQO4, 32 q-heads / 8 KV heads, batch 16
    with contexts drawn uniformly from [4096, 16384] (seeded), bf16 queries,
    split-K over each context; every sequence against the dense oracle."""
    rng = np.random.default_rng(44)
    bits, h, hkv, bsz = 4, 32, 8, 16
    lens = [int(x) for x in rng.integers(4096, 16385, bsz)]
    cap = max(lens)
    pd = 128 * bits // 8
    kidx = np.zeros((bsz, hkv, cap, pd), np.uint8)
    vidx = np.zeros_like(kidx)
    ksc = np.zeros((bsz, hkv, cap, 4), np.int16)
    vsc = np.zeros_like(ksc)
    qs = bf16_round(rng.standard_normal((bsz, h, 128)).astype(np.float32) / np.float32(math.sqrt(128)))
    refs = []
    for bi, t in enumerate(lens):
        k = kv_outlier(rng, hkv, t)
        v = kv_outlier(rng, hkv, t)
        pk, sk = orc.pqo_quantize(bits, k.reshape(-1, 128), 128)
        pv, sv = orc.pqo_quantize(bits, v.reshape(-1, 128), 128)
        kidx[bi, :, :t] = pk.reshape(hkv, t, pd)
        vidx[bi, :, :t] = pv.reshape(hkv, t, pd)
        ksc[bi, :, :t] = sk.view(np.int16).reshape(hkv, t, 4)
        vsc[bi, :, :t] = sv.view(np.int16).reshape(hkv, t, 4)
        kd = orc.pqo_dequantize(bits, pk, sk, 128).reshape(hkv, t, 128)
        vd = orc.pqo_dequantize(bits, pv, sv, 128).reshape(hkv, t, 128)
        refs.append(orc.attention_dense(qs[bi], kd, vd, 1.0 / math.sqrt(128)))
    ws = tq.AttentionWorkspace(bsz, h, hkv, 128, cap)
    out = tq.pqo_decode_attention(_dev(bf16_bits(qs)).view(torch.bfloat16), _dev(kidx), _dev(ksc), _dev(vidx),
                                  _dev(vsc), torch.tensor(lens, dtype=torch.int32, device="cuda"), hkv, bits, cap,
                                  cap, hkv * cap, 1.0 / math.sqrt(128), ws)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    for bi in range(bsz):
        assert np.abs(out[bi] - refs[bi]).max() <= TOL, (bi, lens[bi])


@pytest.mark.parametrize("bits", [3, 4])
def test_fused_attention_reference_abi(tq, bits):
    """tq_fused_attention (reference FFI shape, two launches, 512-token partitions)."""
    rng = np.random.default_rng(6 + bits)
    t, hkv, h = 1500, 8, 16
    cap = 2000
    cache = _make_cache(rng, hkv, t, bits, cap)
    q = rng.standard_normal((h, 128)).astype(np.float32) / np.float32(math.sqrt(128))
    ref = orc.attention_dense(q, cache[4], cache[5], 1.0 / math.sqrt(128))
    c, _, _ = orc.pqo_codebook(bits)
    out = tq.fused_attention(_dev(q), cache[0], cache[1], cache[2], cache[3], _dev(c), _dev(orc.pqo_decode_signs()),
                             hkv, t, cap, bits, 1.0 / math.sqrt(128))
    torch.cuda.synchronize()
    assert np.abs(out.cpu().numpy() - ref).max() <= TOL


def test_decode_peaked_softmax(tq):
    """A query aligned with one key: the softmax is far from uniform."""
    rng = np.random.default_rng(8)
    t, hkv, h, bits = 2000, 2, 4, 4
    cache = _make_cache(rng, hkv, t, bits)
    q = np.stack([cache[4][i // 2, 1234] * 0.5 for i in range(h)]).astype(np.float32)
    ref = orc.attention_dense(q, cache[4], cache[5], 1.0 / math.sqrt(128))
    (out,) = _run_decode(tq, q, cache, hkv, t, bits, t)
    assert np.abs(out - ref).max() <= TOL


def test_host_known_length_matches_device_lengths(tq):
    """kv_lens = null (every sequence holds max_kv_len tokens, known on the host)
    gives the same output as the device length array."""
    bits, h, hkv, t = 3, 16, 8, 3000
    rng = np.random.default_rng(515)
    cache = _make_cache(rng, hkv, t, bits, t)
    kidx, ksc, vidx, vsc, kd, vd = cache
    q = bf16_round(rng.standard_normal((h, 128)).astype(np.float32) / np.float32(math.sqrt(128)))
    qd = _dev(q).reshape(1, h, 128)
    ws = tq.AttentionWorkspace(1, h, hkv, 128, t)
    lens = torch.tensor([t], dtype=torch.int32, device="cuda")
    a = tq.pqo_decode_attention(qd, kidx, ksc, vidx, vsc, lens, hkv, bits, t, t, 0, 1 / math.sqrt(128), ws)
    b = tq.pqo_decode_attention(qd, kidx, ksc, vidx, vsc, None, hkv, bits, t, t, 0, 1 / math.sqrt(128), ws)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    ref = orc.attention_dense(q, kd, vd, 1 / math.sqrt(128))
    assert np.abs(b.cpu().numpy().reshape(h, 128) - ref).max() <= TOL
