"""GPU parity of the PQO codec kernels against the CPU restatement (oracle).

Bar: packed codes and f16 scales bit-exact; dequantized values bit-exact
(f32) and bf16 outputs the round-to-nearest-even of those values.
"""
import numpy as np
import pytest

from oracle import oracle as orc
from tq_testdata import bf16_bits, bf16_round, kv_outlier, sincos_kv

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def tq():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import turboquant_amd
    return turboquant_amd


def _dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


def _u16(t):
    return t.cpu().numpy().view(np.uint16)


def _edge_blocks(rng):
    """Rotated blocks hitting the corners of the MaxNorm bucketize."""
    blocks = []
    c3, b3, outer = orc.pqo_codebook(3)
    blocks.append(np.zeros(32, np.float32))                      # amax 0 -> scale clamp 1e-10
    blocks.append(np.tile(c3, 4).astype(np.float32))              # exact centroids
    blocks.append(np.tile(np.concatenate([b3, [0.0]]), 4).astype(np.float32))  # exact boundaries
    blocks.append(np.full(32, 1e-38, np.float32))                 # tiny normals
    blocks.append((rng.standard_normal(32) * 1e-42).astype(np.float32))  # denormals
    blocks.append((rng.standard_normal(32) * 1e30).astype(np.float32))   # huge
    x = rng.standard_normal(32).astype(np.float32)
    x[5] = -x[5] * 100
    blocks.append(x)                                              # one dominant outlier
    blocks.append(np.array([(-1) ** j * (j + 1) for j in range(32)], np.float32))
    return np.stack(blocks)


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_quant_maxnorm_batch_bit_exact(tq, bits):
    """Reference ABI (already-rotated f32 input): codes and scales bit-exact."""
    rng = np.random.default_rng(100 + bits)
    rot = np.concatenate([_edge_blocks(rng), rng.standard_normal((4096, 32)).astype(np.float32) * 3])
    c, b, outer = orc.pqo_codebook(bits)
    p_ref, s_ref = orc.pqo_quantize_rotated(bits, rot, -1.0)
    p, s = tq.quant_maxnorm_batch(_dev(rot), _dev(b), bits, float(outer), -1.0)
    torch.cuda.synchronize()
    assert np.array_equal(p.cpu().numpy(), p_ref)
    assert np.array_equal(_u16(s), s_ref)


def test_quant_maxnorm_near_ties(tq):
    """Values placed one ulp around every threshold v = b_k * scale."""
    bits = 3
    rng = np.random.default_rng(7)
    c, b, outer = orc.pqo_codebook(bits)
    blocks = []
    for _ in range(512):
        amax = np.float32(rng.uniform(0.5, 50.0))
        s = np.float32(amax * np.float32(1.0 / np.float64(outer)))
        blk = np.empty(32, np.float32)
        blk[0] = amax
        for j in range(1, 32):
            t = np.float32(b[rng.integers(len(b))] * s)
            blk[j] = np.nextafter(t, np.float32(np.inf * rng.choice([-1, 1])), dtype=np.float32) \
                if rng.random() < 0.7 else t
        blocks.append(blk)
    rot = np.stack(blocks)
    p_ref, s_ref = orc.pqo_quantize_rotated(bits, rot, -1.0)
    p, s = tq.quant_maxnorm_batch(_dev(rot), _dev(b), bits, float(outer), -1.0)
    torch.cuda.synchronize()
    assert np.array_equal(p.cpu().numpy(), p_ref)
    assert np.array_equal(_u16(s), s_ref)


@pytest.mark.parametrize("bits", [3, 4])
@pytest.mark.parametrize("dtype", ["bf16", "f32", "f16"])
def test_pqo_quantize_fused_bit_exact(tq, bits, dtype):
    """Fused rotation + quantize from activations: bit-exact vs the oracle."""
    rng = np.random.default_rng(11)
    x = kv_outlier(rng, 2, 700, 128).reshape(-1, 128)
    x = np.concatenate([x, np.zeros((3, 128), np.float32)])
    if dtype == "bf16":
        xin = _dev(bf16_bits(x)).view(torch.bfloat16)
    elif dtype == "f16":
        x = x.astype(np.float16).astype(np.float32)
        xin = _dev(x.astype(np.float16))
    else:
        x = (x + rng.standard_normal(x.shape).astype(np.float32) * 1e-3).astype(np.float32)
        xin = _dev(x)
    p_ref, s_ref = orc.pqo_quantize(bits, x, 128)
    p, s = tq.pqo_quantize(xin, bits)
    torch.cuda.synchronize()
    assert np.array_equal(p.cpu().numpy(), p_ref)
    assert np.array_equal(_u16(s), s_ref)


@pytest.mark.parametrize("bits", [3, 4])
def test_pqo_quantize_fused_boundary_ties(tq, bits):
    """Fused quantize on blocks whose rotated values land on, and one or a
    few ulps either side of, every boundary b_k: a block (1, beta, 0, ...)
    rotates to +-(1 + beta) / sqrt(32) and +-(1 - beta) / sqrt(32), so
    v = (1 - beta) / (1 + beta) * outer up to rounding; beta is stepped by
    ulps around each tie point.  Bit-exact vs the oracle; some v equal a
    boundary exactly (the ties that the 4-bit grid path must hand to the
    exact thresholds)."""
    c, b, outer = orc.pqo_codebook(bits)[:3]
    rows = []
    for bk in b:
        if bk <= 0:
            continue
        beta0 = np.float32((outer - bk) / (outer + bk))
        for n in range(-48, 49):
            beta = np.float32(beta0 + np.float32(n) * np.spacing(beta0))
            blk = np.zeros(32, np.float32)
            blk[0], blk[1] = 1.0, beta
            rows.append(blk)
    x = np.stack(rows).reshape(-1, 32)
    x = np.concatenate([x, np.zeros((len(x) % 4 and 4 - len(x) % 4, 32), np.float32)]).reshape(-1, 128)
    # the reference arithmetic: r = fl(x f), s = fl(max |r| * fl(1 / outer)), v = fl(r / s)
    f = np.float32(float.fromhex("0x1.6a09e6p-3"))
    blocks = x.reshape(-1, 32)
    r = np.stack([blocks[:, 0] + blocks[:, 1], blocks[:, 0] - blocks[:, 1]], 1).astype(np.float32) * f
    s = np.maximum((np.abs(r).max(1) * np.float32(1.0 / float(outer))).astype(np.float32), np.float32(1e-10))
    v = (r / s[:, None]).astype(np.float32)
    assert np.isin(v, b).sum() >= 3
    p_ref, s_ref = orc.pqo_quantize(bits, x, 128)
    p, sc = tq.pqo_quantize(_dev(x), bits)
    torch.cuda.synchronize()
    assert np.array_equal(p.cpu().numpy(), p_ref)
    assert np.array_equal(_u16(sc), s_ref)


@pytest.mark.parametrize("bits", [3, 4])
def test_pqo_dequantize_bit_exact(tq, bits):
    rng = np.random.default_rng(12)
    x = kv_outlier(rng, 2, 500, 128).reshape(-1, 128)
    p_ref, s_ref = orc.pqo_quantize(bits, x, 128)
    d_ref = orc.pqo_dequantize(bits, p_ref, s_ref, 128)
    d32 = tq.pqo_dequantize(_dev(p_ref), _dev(s_ref.view(np.int16)), bits, 128, torch.float32)
    dbf = tq.pqo_dequantize(_dev(p_ref), _dev(s_ref.view(np.int16)), bits, 128, torch.bfloat16)
    torch.cuda.synchronize()
    assert np.array_equal(d32.cpu().numpy().view(np.uint32), d_ref.view(np.uint32))
    assert np.array_equal(dbf.view(torch.int16).cpu().numpy().view(np.uint16), bf16_bits(d_ref))


@pytest.mark.parametrize("bits", [3, 4])
def test_dequant_batch_reference_abi(tq, bits):
    """tq_dequant_batch with the reference's device codebook and sign pattern
    (R_fwd[0] * sqrt(32), pqo.rs:134-138): bit-exact vs polar_dequantize."""
    rng = np.random.default_rng(13)
    x = kv_outlier(rng, 1, 300, 128).reshape(-1, 128)
    p_ref, s_ref = orc.pqo_quantize(bits, x, 128)
    d_ref = orc.pqo_dequantize(bits, p_ref, s_ref, 128).reshape(-1, 32)
    c, _, _ = orc.pqo_codebook(bits)
    out = tq.dequant_batch(_dev(p_ref.reshape(-1, 4 * bits)), _dev(s_ref.reshape(-1).view(np.int16)), _dev(c),
                           _dev(orc.pqo_decode_signs()), bits)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), d_ref.view(np.uint32))


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_pack_indices(tq, bits):
    rng = np.random.default_rng(14)
    for bs in (32, 8, 5):
        idx = rng.integers(0, 1 << bits, size=(37, bs), dtype=np.uint8)
        ref = np.stack([orc.pack_indices(bits, row) for row in idx])
        out = tq.pack_indices(_dev(idx), bits)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), ref)


def test_pqo_roundtrip_cosine_reference_gates(tq):
    """cache_pqo_tests.rs:151-244 gates on the reference's sin/cos K/V."""
    k, _ = sincos_kv(8, 5, 128, 5.0)
    k = k.reshape(-1, 128)
    for bits, gate in ((3, 0.85), (4, 0.92)):
        p, s = tq.pqo_quantize(_dev(k), bits)
        d = tq.pqo_dequantize(p, s, bits, 128).cpu().numpy().astype(np.float64)
        cos = (d * k).sum() / np.sqrt((d * d).sum() * (k * k).sum())
        assert cos > gate, (bits, cos)


def test_pqo_full_size_c2_properties(tq):
    """Config 2 at full size (28 x 8 x 4096 x 128, K and V): every vector
    round-trips with the codec's error bound, scales are negative, and a
    seeded sample of vectors is bit-exact with the oracle."""
    rng = np.random.default_rng(2)
    layers, heads, toks = 28, 8, 4096
    gen = torch.Generator(device="cuda").manual_seed(2)
    n = layers * heads * toks * 2
    x = torch.randn((n, 128), generator=gen, device="cuda", dtype=torch.float32)
    ch = torch.from_numpy(rng.choice(128, size=4, replace=False)).cuda()
    x[:, ch] *= 8.0
    xb = x.to(torch.bfloat16)
    for bits in (3, 4):
        p, s = tq.pqo_quantize(xb, bits)
        d = tq.pqo_dequantize(p, s, bits, 128, torch.float32)
        xf = xb.float()
        rel = ((d - xf).norm(dim=1) / xf.norm(dim=1)).max().item()
        assert rel < (0.4 if bits == 3 else 0.25), rel
        assert bool((s < 0).all())
        idx = torch.from_numpy(rng.choice(n, size=2048, replace=False)).cuda()
        xs = xf[idx].cpu().numpy()
        p_ref, s_ref = orc.pqo_quantize(bits, xs, 128)
        assert np.array_equal(p[idx].cpu().numpy(), p_ref)
        assert np.array_equal(_u16(s[idx]), s_ref)
        del p, s, d


@pytest.mark.parametrize("bits", [3, 4])
def test_end_to_end_codes_against_gemm_rotation_orders(tq, bits):
    """End-to-end code parity on C2-shaped data (bf16 N(0,1) K/V with 4 of 128
    channels x8; 65,536 vectors): the HIP quantize (butterfly rotation) against
    the codes of the rotation evaluated as separately rounded dot products and
    as fused multiply-add chains (the reference rotates with candle's matmul,
    quantize_tensor.rs:100,104, whose f32 order is not in the reference tree).
    Every differing code is one bin away, with the two quotients r/s on either
    side of the boundary between (within 1e-6 of it); at most 2e-5 of the
    codes differ (about 4-7e-6 measured)."""
    x = kv_outlier(np.random.default_rng(0), 8, 8192).reshape(-1, 128)
    p, s = tq.pqo_quantize(_dev(bf16_bits(x)).view(torch.bfloat16), bits)
    u_hip = np.unpackbits(p.cpu().numpy().reshape(-1, 4 * bits), axis=1, bitorder="little")
    u_hip = (u_hip.reshape(-1, 32, bits) * (1 << np.arange(bits))).sum(2)
    c, bnd, outer = orc.pqo_codebook(bits)
    mul = np.float32(1.0 / np.float64(outer))
    blocks = x.reshape(-1, 32)
    for order in ("dot", "fma"):
        r = orc.pqo_rotate(blocks, order=order)
        pr, _ = orc.pqo_quantize_rotated(bits, r)
        u_ref = (np.unpackbits(pr, axis=1, bitorder="little").reshape(-1, 32, bits) * (1 << np.arange(bits))).sum(2)
        sc = np.maximum((np.abs(r).max(1) * mul).astype(np.float32), np.float32(1e-10))
        v_ref = (r / sc[:, None]).astype(np.float32)
        rb = orc.pqo_rotate(blocks, order="butterfly")
        scb = np.maximum((np.abs(rb).max(1) * mul).astype(np.float32), np.float32(1e-10))
        v_hip = (rb / scb[:, None]).astype(np.float32)
        diff = np.argwhere(u_hip != u_ref)
        rate = len(diff) / u_ref.size
        assert rate <= 2e-5, (order, rate)
        for i, j in diff:
            k = min(u_hip[i, j], u_ref[i, j])
            lo, hi = sorted((v_hip[i, j], v_ref[i, j]))
            assert abs(int(u_hip[i, j]) - int(u_ref[i, j])) == 1 and lo <= bnd[k] <= hi, (order, i, j)
            assert abs(v_hip[i, j] - bnd[k]) <= 1e-6, (order, i, j)
        print(f"PQO{bits} HIP vs {order}-order rotation: {len(diff)} of {u_ref.size} codes differ ({rate:.2e})")
