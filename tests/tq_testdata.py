"""Seeded synthetic inputs shared by tests and bench."""
from __future__ import annotations

import numpy as np


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round f32 to bf16 (nearest-even) and return the f32 values."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    r = (u >> 16) & np.uint32(1)   # ties to even
    r += u
    r += np.uint32(0x7FFF)           # wraps mod 2^32 like the truncating 64-bit form
    r &= np.uint32(0xFFFF0000)
    return r.view(np.float32)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def kv_outlier(rng: np.random.Generator, heads: int, tokens: int, head_dim: int = 128, n_outlier: int = 4,
               factor: float = 8.0) -> np.ndarray:
    """N(0,1) values [heads, tokens, head_dim] with n_outlier channels per head
    scaled by `factor`, rounded to bf16."""
    x = rng.standard_normal((heads, tokens, head_dim), dtype=np.float32)
    for h in range(heads):
        ch = rng.choice(head_dim, size=n_outlier, replace=False)
        x[h, :, ch] *= np.float32(factor)
    return bf16_round(x)


def sincos_kv(num_kv_heads: int, seq_len: int, head_dim: int, seed: float):
    """The closed-form K/V of the reference's cache tests (cache_pqo_tests.rs:31-43)."""
    n = num_kv_heads * seq_len * head_dim
    i = np.arange(n, dtype=np.float32)
    k = np.sin((i + np.float32(seed)) * np.float32(0.0137)).astype(np.float32) * np.float32(2.0)
    v = np.cos((i + np.float32(seed) + np.float32(1000.0)) * np.float32(0.0213)).astype(np.float32) * np.float32(1.5)
    return k.reshape(num_kv_heads, seq_len, head_dim), v.reshape(num_kv_heads, seq_len, head_dim)
