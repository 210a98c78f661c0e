"""The C++ host API (include/turboquant_amd.hpp), which mirrors the reference
crate's Rust types, checked against the oracle through tests/cpp/api_test:
TurboQuantConfig validation kinds and PackedBlock packing on the host (CPU
test); quantize_vec / dequantize_vec, QjlBlock, query projections,
estimates, QuantizedKVCache and the two CompressedKVCache implementations
on the device (GPU test)."""
import json
import math
import os
import subprocess
import tempfile

import numpy as np
import pytest

from oracle import oracle as orc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "api_test")
needs_bin = pytest.mark.skipif(not os.path.exists(BIN), reason="api_test not built (run __graft_entry__.build())")


def run(*args):
    res = subprocess.run([BIN, *args], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    return [json.loads(line) for line in res.stdout.splitlines() if line.strip()]


@needs_bin
def test_config_validation_and_packed_block():
    out = run("host")
    cfg = out[0]["config"]
    # TurboQuantError kinds (error.rs:5-29): UnsupportedBits = 2, InvalidDimension = 1
    assert cfg == {"unsupported_bits": 2, "invalid_dim": 1, "zero_dim": 1, "bits": 4, "dim": 64, "seed": 42}
    packs = [o["pack"] for o in out[1:]]
    assert len(packs) == 9
    for p in packs:
        idx = np.array(p["indices"], np.uint8)
        ref = orc.pack_indices(p["bits"], idx)
        assert p["packed"] == ref.tolist(), (p["bits"], p["count"])
        assert p["size_bytes"] == 2 + orc.packed_len(p["bits"], p["count"])
        assert p["round_trip"]


@pytest.mark.gpu
@needs_bin
def test_device_api_against_oracle():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    n, dim = 8, 128
    vecs = np.stack([orc.pseudo_random_vec(dim, 1000 + i) for i in range(n)]).astype(np.float32)
    query = orc.pseudo_random_vec(dim, 77).astype(np.float32)
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "in.bin")
        with open(path, "wb") as f:
            f.write(np.array([n, dim], np.uint32).tobytes() + vecs.tobytes() + query.tobytes())
        out = run("gpu", path)
    recs = {}
    for o in out:
        for k, v in o.items():
            recs.setdefault(k, []).append(v)

    # quantize_vec / dequantize_vec / dequantize_rotated: bit-exact
    rp, rs = orc.quantize_vec_batch(3, dim, 42, vecs[:3])
    rd = orc.dequantize_vec_batch(3, dim, 42, rp, rs)
    for q in recs["quantize_vec"]:
        i = q["i"]
        assert q["packed"] == rp[i].tolist() and q["scale"] == int(rs[i])
        assert np.array_equal(np.array(q["dequant"], np.float32), rd[i])
        assert np.array_equal(np.array(q["rotated"], np.float32), orc.dequantize_rotated(3, dim, rp[i], rs[i]))
    assert recs["dimension_mismatch"] == [3]

    # QjlBlock and estimates
    pp, ps, sg, nm = orc.qjl_quantize_batch(3, dim, 42, 12345, vecs)
    qb = recs["qjl_block"][0]
    assert qb["polar_bits"] == 2 and qb["size_bytes"] == 2 + 32 + 16 + 2
    assert qb["polar"] == pp[0].tolist() and qb["scale"] == int(ps[0])
    assert qb["signs"] == sg[0].tolist() and qb["norm"] == int(nm[0])
    rq = orc.query_projections(query, 12345)
    assert np.array_equal(np.array(recs["rq"][0], np.float32), rq)
    est = orc.estimate_inner_product(2, dim, 42, query, rq, pp[0], ps[0], sg[0], nm[0])
    assert abs(qb["single"] - est) <= 1e-5 * max(1.0, abs(est))

    # QuantizedKVCache: keys = vecs[:4] + vecs[0], values = vecs[4:] + vecs[1]
    kv = recs["kv_cache"][0]
    keys = np.concatenate([vecs[:4], vecs[:1]])
    values = np.concatenate([vecs[4:], vecs[1:2]])
    assert kv["entries"] == 5 and kv["empty_layer"] == 0 and kv["layer_error"] == 4
    assert kv["memory"] == 5 * 2 * 52 and kv["fp16"] == 5 * dim * 4
    kp, ks, ksg, knm = orc.qjl_quantize_batch(3, dim, 42, 12345, keys)
    ref_scores = orc.qjl_scores(2, dim, 42, 12345, query[None], kp, ks, ksg, knm)[0]
    np.testing.assert_allclose(kv["scores"], ref_scores, rtol=1e-5, atol=1e-5 * np.abs(ref_scores).max())
    assert kv["key2_scale"] == int(ks[2])
    vp, vs, _, _ = orc.qjl_quantize_batch(3, dim, 42, 12345, values)
    ref_w = orc.weighted_values(2, dim, 42, vp, vs, np.array(kv["weights"], np.float32))
    np.testing.assert_allclose(kv["weighted"], ref_w, rtol=1e-5, atol=1e-5 * np.abs(ref_w).max())
    key1 = orc.dequantize_vec_batch(2, dim, 42, kp[1:2], ks[1:2])[0]
    assert np.array_equal(np.array(kv["key1"], np.float32), key1)

    # PqoCache / TqCache through the trait: 2 KV heads x 9 tokens, bits 3
    caches = {c["kind"]: c for c in recs["cache"]}
    for kind, c in caches.items():
        assert c["originals"] and c["seq"] == 9
        out_v = np.array(c["out"], np.float32)
        assert out_v.shape == (4 * dim,) and np.isfinite(out_v).all()
    rec = 2 * 2 * 9 * (48 + 8)
    assert caches["pqo"]["memory"] == rec
    # QJL buffers counted whole: capacity 8 + max(8 / 4, 128) records from the prefill
    assert caches["tq"]["memory"] == rec + 2 * (8 + 128) * (16 + 2)
