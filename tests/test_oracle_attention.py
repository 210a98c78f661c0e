"""Pin of the dense attention oracle (the semantic reference for the fused
decode, SURVEY row C5r: dequantize then softmax(scale q K^T) V with GQA head
h reading KV head h // (H / H_kv), as tq_attention_kernel.cu:92-93 maps it),
against a textbook numpy float64 softmax."""
import numpy as np
import pytest

from oracle import oracle as orc


def softmax_attention(q, k, v, scale):
    h, hkv = q.shape[0], k.shape[0]
    rep = h // hkv
    out = np.zeros((h, q.shape[1]))
    for i in range(h):
        s = scale * (k[i // rep].astype(np.float64) @ q[i].astype(np.float64))
        p = np.exp(s - s.max())
        out[i] = p @ v[i // rep].astype(np.float64) / p.sum()
    return out


@pytest.mark.parametrize("h,hkv,t", [(16, 8, 300), (32, 8, 77), (4, 4, 1), (8, 2, 1025)])
def test_attention_dense_is_softmax_attention(h, hkv, t):
    rng = np.random.default_rng(h * 100 + t)
    q = rng.standard_normal((h, 128)).astype(np.float32)
    k = rng.standard_normal((hkv, t, 128)).astype(np.float32)
    v = rng.standard_normal((hkv, t, 128)).astype(np.float32)
    got = orc.attention_dense(q, k, v, 1 / np.sqrt(128))
    assert np.abs(got - softmax_attention(q, k, v, 1 / np.sqrt(128))).max() < 1e-6


def test_attention_dense_single_token_returns_value():
    q = np.ones((2, 128), np.float32)
    k = np.zeros((1, 1, 128), np.float32)
    v = np.arange(128, dtype=np.float32).reshape(1, 1, 128)
    assert np.array_equal(orc.attention_dense(q, k, v, 0.1), np.stack([v[0, 0], v[0, 0]]))
