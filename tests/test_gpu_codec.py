"""GPU parity of the core full-vector codec (quantize_vec / dequantize_vec /
dequantize_rotated, reference src/quantize.rs:142-316) against the oracle.

Bar: codes and f16 scales bit-exact on the same f32 inputs (the kernel keeps
the reference's sequential norm and butterfly order and compares against
exact f32 images of the f64 boundaries); dequantized values bit-exact.
At the full C1 size (10,000 LCG vectors, d=128, seed 42) also the nMSE
window of mse_validation.rs:125-142.
"""
import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def tq():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import turboquant_amd
    return turboquant_amd


def _inputs(rng, n, dim):
    x = rng.standard_normal((n, dim)).astype(np.float32)
    x[0] = 0.0                      # null vector: scale 0, zero output
    x[1] = 0.0
    x[1, 3] = 1.0                   # unit vector
    x[2] = 0.5                      # constant vector
    x[3] *= 1e-12                   # norm below MIN_NORM
    x[4] *= 7e4                     # f16 scale overflow -> inf
    return x


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("dim", [32, 64, 128, 256])
@pytest.mark.parametrize("seed", [42, 7])
def test_quantize_matches_oracle_bit_exact(tq, bits, dim, seed):
    rng = np.random.default_rng(bits * 1000 + dim + seed)
    x = _inputs(rng, 1000, dim)
    p_ref, s_ref = orc.quantize_vec_batch(bits, dim, seed, x)
    p, s = tq.quantize_vec_batch(torch.from_numpy(x).cuda(), bits, seed)
    assert np.array_equal(s.cpu().numpy().view(np.uint16), s_ref)
    assert np.array_equal(p.cpu().numpy(), p_ref)


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("dim", [32, 64, 128, 256])
def test_dequantize_matches_oracle_bit_exact(tq, bits, dim):
    rng = np.random.default_rng(bits + dim)
    x = _inputs(rng, 500, dim)
    x[4] = rng.standard_normal(dim).astype(np.float32)
    p_ref, s_ref = orc.quantize_vec_batch(bits, dim, 42, x)
    ref = orc.dequantize_vec_batch(bits, dim, 42, p_ref, s_ref)
    out = tq.dequantize_vec_batch(torch.from_numpy(p_ref).cuda(), torch.from_numpy(s_ref.view(np.int16)).cuda(),
                                  bits, dim, 42).cpu().numpy()
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    rot = tq.dequantize_rotated_batch(torch.from_numpy(p_ref).cuda(), torch.from_numpy(s_ref.view(np.int16)).cuda(),
                                      bits, dim).cpu().numpy()
    for i in (5, 17, 499):
        assert np.array_equal(rot[i], orc.dequantize_rotated(bits, dim, p_ref[i], int(s_ref[i])))


def test_c1_full_size_nmse_and_parity(tq):
    """BASELINE config 1 at its size on the GPU: 10,000 LCG N(0,1) vectors, d=128,
    TQ3 seed 42; codes bit-exact and nMSE in the reference window."""
    x = orc.lcg_normal_vecs(12345, 128, 10_000).astype(np.float32)
    p, s = tq.quantize_vec_batch(torch.from_numpy(x).cuda(), 3, 42)
    y = tq.dequantize_vec_batch(p, s, 3, 128, 42).cpu().numpy()
    p_ref, s_ref = orc.quantize_vec_batch(3, 128, 42, x)
    assert np.array_equal(p.cpu().numpy(), p_ref)
    x64 = x.astype(np.float64)
    nmse = float(np.mean(((x64 - y) ** 2).sum(1) / (x64 ** 2).sum(1)))
    assert 0.030 <= nmse <= 0.038


def test_rejects_bad_config(tq):
    x = torch.zeros((4, 48), dtype=torch.float32, device="cuda")
    with pytest.raises(tq.TurboQuantError):
        tq.quantize_vec_batch(x, 3)
    x = torch.zeros((4, 512), dtype=torch.float32, device="cuda")
    with pytest.raises(tq.TurboQuantError):
        tq.quantize_vec_batch(x, 3)
    x = torch.zeros((4, 128), dtype=torch.float32, device="cuda")
    with pytest.raises(tq.TurboQuantError):
        tq.quantize_vec_batch(x, 5)
