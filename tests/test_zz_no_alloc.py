"""The decode entry point that allocates nothing (tq_pqo_decode_attention_noalloc):
its split-K partials and counters live in the library's per-device static
scratch array.  Checked through the C ABI against tq_pqo_decode_attention
(the same kernels over a caller workspace): bit-identical outputs on two
calls in a row, the second with a smaller input, both also within 1e-3 of
the dense oracle; a shape beyond the scratch array's limit is rejected with
an error; a HIP graph capture of the call replays to the eager result.
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


def _fn(tq):
    return tq.lib.tq_pqo_decode_attention_noalloc  # prototype from turboquant_amd/_lib.py


def _case(rng, lens, hkv, h, bits):
    """Records [B, hkv, cap, ...] of PQO-quantized K/V (oracle) and the dense references."""
    cap = max(lens)
    pd = D * bits // 8
    bsz = len(lens)
    kidx = np.zeros((bsz, hkv, cap, pd), np.uint8)
    vidx = np.zeros_like(kidx)
    ksc = np.zeros((bsz, hkv, cap, 4), np.int16)
    vsc = np.zeros_like(ksc)
    qs = bf16_round(rng.standard_normal((bsz, h, D)).astype(np.float32) / np.float32(math.sqrt(D)))
    refs = []
    for bi, t in enumerate(lens):
        k = kv_outlier(rng, hkv, t).reshape(-1, D)
        v = kv_outlier(rng, hkv, t).reshape(-1, D)
        pk, sk = orc.pqo_quantize(bits, k, D)
        pv, sv = orc.pqo_quantize(bits, v, D)
        kidx[bi, :, :t] = pk.reshape(hkv, t, pd)
        vidx[bi, :, :t] = pv.reshape(hkv, t, pd)
        ksc[bi, :, :t] = sk.view(np.int16).reshape(hkv, t, 4)
        vsc[bi, :, :t] = sv.view(np.int16).reshape(hkv, t, 4)
        kd = orc.pqo_dequantize(bits, pk, sk, D).reshape(hkv, t, D)
        vd = orc.pqo_dequantize(bits, pv, sv, D).reshape(hkv, t, D)
        refs.append(orc.attention_dense(qs[bi], kd, vd, 1 / math.sqrt(D)))
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    return dict(q=dev(bf16_bits(qs)).view(torch.bfloat16), kidx=dev(kidx), ksc=dev(ksc), vidx=dev(vidx),
                vsc=dev(vsc), lens=torch.tensor(lens, dtype=torch.int32, device="cuda"), cap=cap, hkv=hkv, h=h,
                bits=bits, refs=refs)


def _noalloc(tq, c, out):
    b = len(c["refs"])
    return _fn(tq)(c["q"].data_ptr(), 1, c["kidx"].data_ptr(), c["ksc"].data_ptr(), c["vidx"].data_ptr(),
                   c["vsc"].data_ptr(), c["lens"].data_ptr(), b, c["h"], c["hkv"], D, c["bits"], c["cap"], c["cap"],
                   c["hkv"] * c["cap"], 1 / math.sqrt(D), out.data_ptr(), 0,
                   torch.cuda.current_stream().cuda_stream)


def _with_workspace(tq, c):
    b = len(c["refs"])
    ws = tq.AttentionWorkspace(b, c["h"], c["hkv"], D, c["cap"])
    return tq.pqo_decode_attention(c["q"], c["kidx"], c["ksc"], c["vidx"], c["vsc"], c["lens"], c["hkv"], c["bits"],
                                   c["cap"], c["cap"], c["hkv"] * c["cap"], 1 / math.sqrt(D), ws)


def test_noalloc_matches_workspace_entry_on_two_calls(tq):
    rng = np.random.default_rng(90)
    big = _case(rng, [9000, 4100], 8, 16, 3)       # C3 head shape, two sequences
    small = _case(rng, [1500], 8, 32, 4)           # then fewer sequences, shorter, another GQA ratio
    for c in (big, small):
        out = torch.full((len(c["refs"]), c["h"], D), float("nan"), device="cuda")
        tq.check(_noalloc(tq, c, out))
        want = _with_workspace(tq, c)
        torch.cuda.synchronize()
        assert torch.equal(out, want)
        got = out.cpu().numpy()
        for bi, ref in enumerate(c["refs"]):
            assert np.abs(got[bi] - ref).max() <= TOL, bi


def test_noalloc_rejects_shapes_beyond_the_scratch(tq):
    c = _case(np.random.default_rng(91), [64], 8, 16, 3)
    out = torch.empty((1, 16, D), device="cuda")
    f = _fn(tq)
    # 64 sequences x 32 heads x 16 chunks of 128 f32 partials = 16 MiB > 8 MiB
    rc = f(c["q"].data_ptr(), 1, c["kidx"].data_ptr(), c["ksc"].data_ptr(), c["vidx"].data_ptr(), c["vsc"].data_ptr(),
           None, 64, 32, 8, D, 3, 16384, 16384, 8 * 16384, 1 / math.sqrt(D), out.data_ptr(), 0,
           torch.cuda.current_stream().cuda_stream)
    assert rc != 0 and b"scratch" in tq.lib.tq_last_error()
    # more (sequence, KV head) pairs than counters
    rc = f(c["q"].data_ptr(), 1, c["kidx"].data_ptr(), c["ksc"].data_ptr(), c["vidx"].data_ptr(), c["vsc"].data_ptr(),
           None, 200, 8, 8, D, 3, 64, 64, 8 * 64, 1 / math.sqrt(D), out.data_ptr(), 0,
           torch.cuda.current_stream().cuda_stream)
    assert rc != 0 and b"counters" in tq.lib.tq_last_error()


def test_noalloc_graph_replays_match_eager(tq):
    c = _case(np.random.default_rng(92), [5000], 8, 16, 3)
    out = torch.empty((1, 16, D), device="cuda")
    tq.check(_noalloc(tq, c, out))
    torch.cuda.synchronize()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        tq.check(_noalloc(tq, c, out))
    for rep in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), rep
        tq.check(_noalloc(tq, c, out))  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(out, eager), rep
