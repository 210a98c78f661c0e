"""GPU tests of the decode boundary's edge cases, through the C ABI.

* The split-K workspace: one workspace initialised for the largest batch and
  length serves smaller calls in any order (the counters sit at the
  workspace's end, the partials grow from its start); a launch whose
  counters were not zeroed by the init stores nothing and returns NaN, and
  leaves the workspace usable.
* Empty sequences attend to nothing and produce zeros, as the reference's
  `fused_attention` zero-fills its output (src/cache/cuda/attention.rs:65-68)
  and its reduce writes 0 for a zero sum (tq_attention_kernel.cu:328).
* The reference ABI (`tq_fused_attention`) reads the caller's device
  codebook and sign pattern (tq_attention_kernel.cu:127-130): an L2Norm
  cache brings its Beta tables (pqo.rs:154, precomputed/codebooks.rs:31-48).
* A cache decodes correctly across layers of different capacity and after
  reset() with a shorter context (one workspace shared by all layers).

Oracle: the CPU restatement's dequantize, then dense softmax attention in
double; tolerance 1e-3 max-abs.
"""
import ctypes as C
import math

import numpy as np
import pytest

from oracle import oracle as orc
from tq_testdata import bf16_bits, bf16_round, kv_outlier

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

TOL = 1e-3
D = 128


@pytest.fixture(scope="module")
def tq():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import turboquant_amd
    return turboquant_amd


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _batch_cache(rng, lens, hkv, bits, cap):
    """[B, hkv, cap, ...] records quantized by the oracle, plus the dequantized K/V per sequence."""
    pd = D * bits // 8
    bsz = len(lens)
    kidx = np.zeros((bsz, hkv, cap, pd), np.uint8)
    vidx = np.zeros_like(kidx)
    ksc = np.zeros((bsz, hkv, cap, 4), np.int16)
    vsc = np.zeros_like(ksc)
    deq = []
    for bi, t in enumerate(lens):
        if t == 0:
            deq.append(None)
            continue
        k = kv_outlier(rng, hkv, t)
        v = kv_outlier(rng, hkv, t)
        pk, sk = orc.pqo_quantize(bits, k.reshape(-1, D), D)
        pv, sv = orc.pqo_quantize(bits, v.reshape(-1, D), D)
        kidx[bi, :, :t] = pk.reshape(hkv, t, pd)
        vidx[bi, :, :t] = pv.reshape(hkv, t, pd)
        ksc[bi, :, :t] = sk.view(np.int16).reshape(hkv, t, 4)
        vsc[bi, :, :t] = sv.view(np.int16).reshape(hkv, t, 4)
        deq.append((orc.pqo_dequantize(bits, pk, sk, D).reshape(hkv, t, D),
                    orc.pqo_dequantize(bits, pv, sv, D).reshape(hkv, t, D)))
    return tuple(_dev(x) for x in (kidx, ksc, vidx, vsc)), deq


def _refs(qs, deq):
    out = []
    for bi, kv in enumerate(deq):
        out.append(np.zeros_like(qs[bi]) if kv is None else orc.attention_dense(qs[bi], kv[0], kv[1],
                                                                                 1 / math.sqrt(D)))
    return out


def _decode(tq, qs, recs, lens, hkv, bits, cap, ws, nbytes=None, out_dtype=torch.float32):
    """tq_pqo_decode_attention on the first len(lens) sequences of recs."""
    b = len(lens)
    h = qs.shape[1]
    kidx, ksc, vidx, vsc = recs
    out = torch.full((b, h, D), float("nan"), dtype=out_dtype, device="cuda")
    q = _dev(bf16_bits(qs[:b])).view(torch.bfloat16)
    lens_d = torch.tensor(lens, dtype=torch.int32, device="cuda")
    buf, nb = (ws.buf, ws.nbytes) if nbytes is None else (ws, nbytes)
    rc = tq.lib.tq_pqo_decode_attention(q.data_ptr(), 1, kidx.data_ptr(), ksc.data_ptr(), vidx.data_ptr(),
                                        vsc.data_ptr(), lens_d.data_ptr(), b, h, hkv, D, bits, max(lens + [0]),
                                        cap, hkv * cap, C.c_float(1 / math.sqrt(D)), out.data_ptr(),
                                        {torch.float32: 0, torch.bfloat16: 1}[out_dtype], buf.data_ptr(), nb,
                                        torch.cuda.current_stream().cuda_stream)
    tq.check(rc)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def test_workspace_for_largest_shape_serves_smaller_calls(tq):
    """Init once for (batch 3, length 5000); then calls with fewer sequences and
    shorter contexts, in an order that would put one call's partials where
    another call's counters used to be, all match the oracle."""
    rng = np.random.default_rng(71)
    hkv, h, bits, cap = 8, 16, 3, 5000
    lens_all = [5000, 1200, 2600]
    recs, deq = _batch_cache(rng, lens_all, hkv, bits, cap)
    qs = bf16_round(rng.standard_normal((3, h, D)).astype(np.float32) / np.float32(math.sqrt(D)))
    refs = _refs(qs, deq)
    ws = tq.AttentionWorkspace(3, h, hkv, D, cap)
    for lens in ([5000], [5000, 1200, 2600], [5000, 1200], [1000], [5000, 1200, 2600]):
        sub_deq = [None if t == 0 else (deq[i][0][:, :t], deq[i][1][:, :t]) for i, t in enumerate(lens)]
        sub_refs = _refs(qs, sub_deq)
        out = _decode(tq, qs, recs, lens, hkv, bits, cap, ws)
        for bi in range(len(lens)):
            assert np.abs(out[bi] - sub_refs[bi]).max() <= TOL, (lens, bi)
    assert refs  # the full-length references were exercised above


def test_workspace_with_too_few_zeroed_counters_returns_nan_and_stays_usable(tq):
    """A buffer large enough for batch 3 but initialised for batch 1: a batch-3
    call finds counters the init never zeroed, so it stores nothing and writes
    NaN; the workspace still serves batch-1 calls correctly afterwards."""
    rng = np.random.default_rng(72)
    hkv, h, bits, cap = 4, 8, 4, 3000
    lens = [3000, 2000, 2500]
    recs, deq = _batch_cache(rng, lens, hkv, bits, cap)
    qs = bf16_round(rng.standard_normal((3, h, D)).astype(np.float32) / np.float32(math.sqrt(D)))
    refs = _refs(qs, deq)
    nbytes = tq.lib.tq_attention_workspace_size(3, h, hkv, D, cap)
    buf = torch.empty((nbytes,), dtype=torch.uint8, device="cuda")
    tq.check(tq.lib.tq_attention_workspace_init(buf.data_ptr(), nbytes, 1, h, hkv, D, cap,
                                                torch.cuda.current_stream().cuda_stream))
    out = _decode(tq, qs, recs, lens, hkv, bits, cap, buf, nbytes)
    assert np.isnan(out).all()
    for _ in range(2):
        out1 = _decode(tq, qs, recs, lens[:1], hkv, bits, cap, buf, nbytes)
        assert np.abs(out1[0] - refs[0]).max() <= TOL


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_empty_sequences_produce_zeros(tq, out_dtype):
    rng = np.random.default_rng(73)
    hkv, h, bits = 8, 32, 4
    lens = [700, 0, 2100, 0]
    cap = 2200
    recs, deq = _batch_cache(rng, lens, hkv, bits, cap)
    qs = bf16_round(rng.standard_normal((4, h, D)).astype(np.float32) / np.float32(math.sqrt(D)))
    refs = _refs(qs, deq)
    ws = tq.AttentionWorkspace(4, h, hkv, D, cap)
    tol = TOL if out_dtype == torch.float32 else 2e-2
    for _ in range(2):
        out = _decode(tq, qs, recs, lens, hkv, bits, cap, ws, out_dtype=out_dtype)
        for bi in range(4):
            if lens[bi] == 0:
                assert np.array_equal(out[bi], np.zeros_like(out[bi])), bi
            else:
                assert np.abs(out[bi] - refs[bi]).max() <= tol, bi
    # every sequence empty (max_kv_len 0): no launch over records, zero output
    out = _decode(tq, qs, recs, [0, 0], hkv, bits, cap, ws, out_dtype=out_dtype)
    assert np.array_equal(out, np.zeros_like(out))


def test_reference_abi_zero_length_zeroes_output(tq):
    q = torch.randn((16, D), device="cuda")
    z = torch.zeros((1, 8, 4, 48), dtype=torch.uint8, device="cuda")
    zs = torch.zeros((1, 8, 4, 4), dtype=torch.int16, device="cuda")
    c, _, _ = orc.pqo_codebook(3)
    out = tq.fused_attention(q, z, zs, z, zs, _dev(c), _dev(orc.pqo_decode_signs()), 8, 0, 4, 3,
                             1 / math.sqrt(D))
    torch.cuda.synchronize()
    assert torch.count_nonzero(out).item() == 0


@pytest.mark.parametrize("bits", [3, 4])
def test_reference_abi_uses_callers_l2norm_codebook(tq, bits):
    """L2Norm PQO records (Beta tables of dimension 32 as the outlier codebook,
    precomputed/codebooks.rs:31-48) decoded through tq_fused_attention with the
    codebook the reference's decode_cuda passes (pre.outlier_centroids,
    pqo.rs:154): the output matches the oracle; the MaxNorm constants in its
    place do not."""
    rng = np.random.default_rng(74 + bits)
    hkv, h, t, cap = 4, 8, 1300, 1400
    k = kv_outlier(rng, hkv, t).reshape(-1, D)
    v = kv_outlier(rng, hkv, t).reshape(-1, D)
    pd = D * bits // 8
    pk, sk = orc.polar_quantize(bits, orc.OUTLIER_ALL, k, D, norm_mode=1)
    pv, sv = orc.polar_quantize(bits, orc.OUTLIER_ALL, v, D, norm_mode=1)
    kd = orc.polar_dequantize(bits, orc.OUTLIER_ALL, pk, sk, D, norm_mode=1).reshape(hkv, t, D)
    vd = orc.polar_dequantize(bits, orc.OUTLIER_ALL, pv, sv, D, norm_mode=1).reshape(hkv, t, D)

    def lay(a, w, dt):
        buf = np.zeros((hkv, cap, w), dt)
        buf[:, :t] = a.reshape(hkv, t, w)
        return _dev(buf)

    recs = (lay(pk, pd, np.uint8), lay(sk.view(np.int16), 4, np.int16), lay(pv, pd, np.uint8),
            lay(sv.view(np.int16), 4, np.int16))
    q = rng.standard_normal((h, D)).astype(np.float32) / np.float32(math.sqrt(D))
    ref = orc.attention_dense(q, kd, vd, 1 / math.sqrt(D))
    beta, _ = orc.get_codebook(bits, 32)
    signs = _dev(orc.pqo_decode_signs())
    out = tq.fused_attention(_dev(q), *recs[:2], *recs[2:], _dev(beta.astype(np.float32)), signs, hkv, t, cap,
                             bits, 1 / math.sqrt(D))
    torch.cuda.synchronize()
    assert np.abs(out.cpu().numpy() - ref).max() <= TOL
    c_max, _, _ = orc.pqo_codebook(bits)
    wrong = tq.fused_attention(_dev(q), *recs[:2], *recs[2:], _dev(c_max), signs, hkv, t, cap, bits,
                               1 / math.sqrt(D))
    torch.cuda.synchronize()
    assert np.abs(wrong.cpu().numpy() - ref).max() > 10 * TOL


def test_reference_abi_uses_callers_sign_pattern(tq):
    """The decode signs are the caller's: flipping the sign of element j of
    every block flips element j of the dequantized blocks before the inverse
    WHT, which the oracle reproduces by flipping it in the codes' values."""
    rng = np.random.default_rng(76)
    bits, hkv, h, t = 3, 2, 4, 600
    k = kv_outlier(rng, hkv, t).reshape(-1, D)
    v = kv_outlier(rng, hkv, t).reshape(-1, D)
    pk, sk = orc.pqo_quantize(bits, k, D)
    pv, sv = orc.pqo_quantize(bits, v, D)
    q = rng.standard_normal((h, D)).astype(np.float32) / np.float32(math.sqrt(D))
    c, _, _ = orc.pqo_codebook(bits)
    sg = orc.pqo_decode_signs().copy()
    sg[5] = -sg[5]
    # dequantize by the definition with the altered signs (tq_attention_kernel.cu:33-53):
    # x = H(cb[idx] * sg) * fl(1/sqrt 32) * |s| per block
    idx_k = np.stack([orc.unpack_indices(bits, r.reshape(4, -1)[j], 32) for r in pk for j in range(4)])
    idx_v = np.stack([orc.unpack_indices(bits, r.reshape(4, -1)[j], 32) for r in pv for j in range(4)])
    hmat = np.array([[(-1) ** bin(i & j).count("1") for j in range(32)] for i in range(32)], np.float64)

    def deq(idx, s):
        sc = np.abs(orc.f16_bits_to_f32(s.reshape(-1))).astype(np.float64)
        blocks = (c[idx].astype(np.float64) * sg.astype(np.float64)) @ hmat.T
        return (blocks * (1 / math.sqrt(32)) * sc[:, None]).reshape(hkv, t, D)

    ref = orc.attention_dense(q, deq(idx_k, sk), deq(idx_v, sv), 1 / math.sqrt(D))
    rec = lambda a, w, dt: _dev(a.reshape(hkv, t, w).astype(dt))  # noqa: E731
    out = tq.fused_attention(_dev(q), rec(pk, 48, np.uint8), rec(sk.view(np.int16), 4, np.int16),
                             rec(pv, 48, np.uint8), rec(sv.view(np.int16), 4, np.int16), _dev(c), _dev(sg), hkv, t,
                             t, bits, 1 / math.sqrt(D))
    torch.cuda.synchronize()
    assert np.abs(out.cpu().numpy() - ref).max() <= TOL


def test_cache_decode_across_layer_capacities_and_reset(tq):
    """One cache, one shared decode workspace: decode a long layer, then a short
    one, then reset() and decode a shorter context; each against the oracle."""
    rng = np.random.default_rng(77)
    hkv, h, bits = 8, 16, 3
    cache = tq.PqoCache(2, hkv, D, bits)
    cfg = tq.AttendConfig(1 / math.sqrt(D), h // hkv)
    stored = {}

    def step(layer, t_prefill):
        k = rng.standard_normal((1, hkv, t_prefill, D)).astype(np.float32)
        v = rng.standard_normal((1, hkv, t_prefill, D)).astype(np.float32)
        cache.prefill(layer, _dev(k), _dev(v))
        k1 = rng.standard_normal((1, hkv, 1, D)).astype(np.float32)
        v1 = rng.standard_normal((1, hkv, 1, D)).astype(np.float32)
        q = rng.standard_normal((h, D)).astype(np.float32) / np.float32(math.sqrt(D))
        out = cache.decode(layer, _dev(k1), _dev(v1), _dev(q).reshape(1, h, 1, D), cfg)
        torch.cuda.synchronize()
        kall = np.concatenate([k, k1], 2)[0].reshape(-1, D)
        vall = np.concatenate([v, v1], 2)[0].reshape(-1, D)
        pk, sk = orc.pqo_quantize(bits, kall, D)
        pv, sv = orc.pqo_quantize(bits, vall, D)
        s = t_prefill + 1
        kd = orc.pqo_dequantize(bits, pk, sk, D).reshape(hkv, s, D)
        vd = orc.pqo_dequantize(bits, pv, sv, D).reshape(hkv, s, D)
        ref = orc.attention_dense(q, kd, vd, 1 / math.sqrt(D))
        o = (out.out if hasattr(out, "out") else out).float().cpu().numpy().reshape(h, D)
        stored[(layer, s)] = np.abs(o - ref).max()

    step(0, 3000)   # long layer: 3 chunks per head
    step(1, 100)    # short layer: the workspace layout of the long one
    cache.reset()
    step(0, 40)     # after reset, a shorter context on the same workspace
    step(1, 2100)
    for key, err in stored.items():
        assert err <= TOL, (key, err)
