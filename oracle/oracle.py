"""ctypes loader for the CPU restatement (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker.  The product package
(turboquant_amd) never imports this module.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_sz = C.c_size_t
_u64 = C.c_uint64


def _load():
    if not os.path.exists(_LIB_PATH):
        raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run `make -C oracle`)")
    lib = C.CDLL(_LIB_PATH)
    sig = {
        "tqo_f32_to_f16": (C.c_uint16, [C.c_float]),
        "tqo_f16_to_f32": (C.c_float, [C.c_uint16]),
        "tqo_f32_to_bf16": (C.c_uint16, [C.c_float]),
        "tqo_f32_to_f16_batch": (None, [_f32p, _sz, _u16p]),
        "tqo_f16_to_f32_batch": (None, [_u16p, _sz, _f32p]),
        "tqo_generate_sign_pattern": (None, [_sz, _u64, _f32p]),
        "tqo_wht_inplace": (None, [_f32p, _sz]),
        "tqo_rotate": (C.c_int, [_f32p, _f32p, _sz, _sz, C.c_int]),
        "tqo_nearest_centroid": (C.c_uint8, [C.c_double, C.POINTER(C.c_double), C.c_int]),
        "tqo_get_codebook": (C.c_int, [C.c_int, _sz, C.POINTER(C.POINTER(C.c_double)),
                                       C.POINTER(C.POINTER(C.c_double)), C.POINTER(C.c_int)]),
        "tqo_packed_len": (_sz, [C.c_int, _sz]),
        "tqo_pack_indices": (_sz, [C.c_int, _u8p, _sz, _u8p]),
        "tqo_unpack_indices": (None, [C.c_int, _u8p, _sz, _sz, _u8p]),
        "tqo_l2_norm": (C.c_float, [_f32p, _sz]),
        "tqo_quantize_vec_batch": (C.c_int, [C.c_int, _sz, _u64, _sz, _f32p, _u8p, _u16p]),
        "tqo_dequantize_vec_batch": (C.c_int, [C.c_int, _sz, _u64, _sz, _u8p, _u16p, _f32p]),
        "tqo_dequantize_rotated": (C.c_int, [C.c_int, _sz, _u8p, C.c_uint16, _f32p]),
        "tqo_pqo_codebook": (C.c_int, [C.c_int, _f32p, _f32p, C.POINTER(C.c_int), C.POINTER(C.c_float)]),
        "tqo_pqo_sign32": (None, [_f32p]),
        "tqo_pqo_decode_signs": (None, [_f32p]),
        "tqo_pqo_rotate_block": (None, [_f32p, _f32p]),
        "tqo_pqo_rotate_block_gemm": (None, [_f32p, _f32p]),
        "tqo_pqo_rotate_block_fma": (None, [_f32p, _f32p]),
        "tqo_pqo_rotate_blocks": (C.c_int, [C.c_int, _sz, _f32p, _f32p]),
        "tqo_pqo_quantize_rotated": (C.c_int, [C.c_int, _sz, _f32p, _u8p, _u16p, C.c_float]),
        "tqo_pqo_quantize": (C.c_int, [C.c_int, _sz, _sz, _f32p, _u8p, _u16p]),
        "tqo_pqo_dequantize": (C.c_int, [C.c_int, _sz, _sz, _u8p, _u16p, _f32p]),
        "tqo_attention_dense": (C.c_int, [_sz, _sz, _sz, _sz, _f32p, _f32p, _f32p, C.c_float, _f32p]),
        "tqo_attention_prefill": (C.c_int, [_sz, _sz, _sz, _sz, _sz, _f32p, _f32p, _f32p, C.c_void_p, C.c_float,
                                            C.c_int, _f32p]),
        "tqo_polar_quantize": (C.c_int, [C.c_int, _sz, C.c_int, _sz, _sz, _f32p, _u8p, _u16p]),
        "tqo_polar_dequantize": (C.c_int, [C.c_int, _sz, C.c_int, _sz, _sz, _u8p, _u16p, _f32p]),
        "tqo_tq_signs_norms": (C.c_int, [_sz, _sz, _f32p, _f32p, _u8p, _u16p]),
        "tqo_tq_logit_bias": (C.c_int, [_sz, _sz, _sz, _sz, _sz, _f32p, _u8p, _u16p, _f32p]),
        "tqo_attention_dense_bias": (C.c_int, [_sz, _sz, _sz, _sz, _f32p, _f32p, _f32p, _f32p, C.c_float,
                                               _f32p]),
        "tqo_qjl_mix_seed": (_u64, [_u64, _sz]),
        "tqo_rademacher_sign": (C.c_float, [_u64, _sz, _sz]),
        "tqo_generate_rademacher_row": (None, [_sz, _u64, _sz, _f32p]),
        "tqo_rademacher_vector_product": (C.c_float, [_f32p, _sz, _u64, _sz]),
        "tqo_compute_qjl_signs": (C.c_int, [_f32p, _sz, _u64, _u8p]),
        "tqo_precompute_query_projections": (None, [_f32p, _sz, _u64, _f32p]),
        "tqo_qjl_scaling_constant": (C.c_float, [C.c_float, _sz]),
        "tqo_qjl_correction": (C.c_float, [_f32p, _u8p, _sz]),
        "tqo_estimate_inner_product": (C.c_int, [C.c_int, _sz, _u64, _f32p, _f32p, _u8p, C.c_uint16,
                                                 _u8p, C.c_uint16, C.POINTER(C.c_float)]),
        "tqo_qjl_quantize_batch": (C.c_int, [C.c_int, _sz, _u64, _u64, _sz, _f32p, _u8p, _u16p, _u8p, _u16p]),
        "tqo_qjl_scores_batch": (C.c_int, [C.c_int, _sz, _u64, _u64, _sz, _f32p, _sz, _u8p, _u16p, _u8p,
                                           _u16p, _f32p]),
        "tqo_weighted_values": (C.c_int, [C.c_int, _sz, _u64, _sz, _u8p, _u16p, _f32p, _f32p]),
        "tqo_pseudo_random_vec": (None, [_sz, _u64, _f32p]),
        "tqo_lcg_normal_vecs": (None, [_u64, _sz, _sz, _f32p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def _check(rc):
    if rc != 0:
        raise ValueError(f"oracle error code {rc}")


# ---- numerics -------------------------------------------------------------

def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32).ravel()
    out = np.zeros(x.size, np.uint16)
    if x.size:
        lib.tqo_f32_to_f16_batch(x, x.size, out)
    return out


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = _c(h, np.uint16).ravel()
    out = np.zeros(h.size, np.float32)
    if h.size:
        lib.tqo_f16_to_f32_batch(h, h.size, out)
    return out


# ---- rotation / codebook / packing ----------------------------------------

def sign_pattern(dim: int, seed: int) -> np.ndarray:
    out = np.empty(dim, np.float32)
    lib.tqo_generate_sign_pattern(dim, seed, out)
    return out


def wht(x: np.ndarray) -> np.ndarray:
    d = _c(x, np.float32).copy()
    lib.tqo_wht_inplace(d, d.size)
    return d


def rotate(x: np.ndarray, signs: np.ndarray, inverse: bool = False) -> np.ndarray:
    d = _c(x, np.float32).copy()
    s = _c(signs, np.float32)
    _check(lib.tqo_rotate(d, s, d.size, s.size, int(inverse)))
    return d


def get_codebook(bits: int, dim: int):
    c = C.POINTER(C.c_double)()
    b = C.POINTER(C.c_double)()
    n = C.c_int()
    _check(lib.tqo_get_codebook(bits, dim, C.byref(c), C.byref(b), C.byref(n)))
    k = n.value
    return np.array(c[:k], np.float64), np.array(b[:k - 1], np.float64)


def nearest_centroid(value: float, boundaries: np.ndarray) -> int:
    b = _c(boundaries, np.float64)
    return lib.tqo_nearest_centroid(float(value), b.ctypes.data_as(C.POINTER(C.c_double)), b.size)


def packed_len(bits: int, count: int) -> int:
    return lib.tqo_packed_len(bits, count)


def pack_indices(bits: int, idx: np.ndarray) -> np.ndarray:
    idx = _c(idx, np.uint8)
    out = np.zeros(max(1, packed_len(bits, idx.size)), np.uint8)
    n = lib.tqo_pack_indices(bits, idx, idx.size, out)
    return out[:n]


def unpack_indices(bits: int, packed: np.ndarray, count: int) -> np.ndarray:
    packed = _c(packed, np.uint8)
    out = np.zeros(max(1, count), np.uint8)
    lib.tqo_unpack_indices(bits, packed if packed.size else np.zeros(1, np.uint8), packed.size, count, out)
    return out[:count]


# ---- core codec -------------------------------------------------------------

def quantize_vec_batch(bits: int, dim: int, seed: int, data: np.ndarray):
    data = _c(data, np.float32).reshape(-1, dim)
    n = data.shape[0]
    plen = packed_len(bits, dim)
    packed = np.zeros((n, plen), np.uint8)
    scales = np.zeros(n, np.uint16)
    _check(lib.tqo_quantize_vec_batch(bits, dim, seed, n, data, packed, scales))
    return packed, scales


def dequantize_vec_batch(bits: int, dim: int, seed: int, packed: np.ndarray, scales: np.ndarray):
    packed = _c(packed, np.uint8)
    scales = _c(scales, np.uint16).ravel()
    n = scales.size
    out = np.zeros((n, dim), np.float32)
    _check(lib.tqo_dequantize_vec_batch(bits, dim, seed, n, packed, scales, out))
    return out


def dequantize_rotated(bits: int, dim: int, packed: np.ndarray, scale: int):
    out = np.zeros(dim, np.float32)
    _check(lib.tqo_dequantize_rotated(bits, dim, _c(packed, np.uint8), int(scale), out))
    return out


def l2_norm(x: np.ndarray) -> float:
    x = _c(x, np.float32)
    return float(lib.tqo_l2_norm(x, x.size))


# ---- PQO codec --------------------------------------------------------------

def pqo_codebook(bits: int):
    c = np.zeros(16, np.float32)
    b = np.zeros(15, np.float32)
    n = C.c_int()
    o = C.c_float()
    _check(lib.tqo_pqo_codebook(bits, c, b, C.byref(n), C.byref(o)))
    k = n.value
    return c[:k].copy(), b[:k - 1].copy(), np.float32(o.value)


def pqo_sign32() -> np.ndarray:
    out = np.zeros(32, np.float32)
    lib.tqo_pqo_sign32(out)
    return out


def pqo_decode_signs() -> np.ndarray:
    out = np.zeros(32, np.float32)
    lib.tqo_pqo_decode_signs(out)
    return out


ROTATE_ORDERS = {"butterfly": 0, "dot": 1, "fma": 2}


def pqo_rotate(x: np.ndarray, gemm: bool = False, order: str | None = None) -> np.ndarray:
    """Forward block rotation x @ R_fwd of [n, 32] blocks in one f32 evaluation
    order: "butterfly" (the oracle's), "dot" (separately rounded products
    summed in k order; gemm=True) or "fma" (one fused multiply-add chain)."""
    x = _c(x, np.float32).reshape(-1, 32)
    out = np.zeros_like(x)
    o = ROTATE_ORDERS[order or ("dot" if gemm else "butterfly")]
    _check(lib.tqo_pqo_rotate_blocks(o, x.shape[0], x, out))
    return out


def pqo_quantize_rotated(bits: int, rotated: np.ndarray, scale_sign: float = -1.0):
    r = _c(rotated, np.float32).reshape(-1, 32)
    nb = r.shape[0]
    packed = np.zeros((nb, 32 * bits // 8), np.uint8)
    scales = np.zeros(nb, np.uint16)
    _check(lib.tqo_pqo_quantize_rotated(bits, nb, r, packed, scales, scale_sign))
    return packed, scales


def pqo_quantize(bits: int, x: np.ndarray, head_dim: int):
    x = _c(x, np.float32).reshape(-1, head_dim)
    n = x.shape[0]
    packed = np.zeros((n, head_dim * bits // 8), np.uint8)
    scales = np.zeros((n, head_dim // 32), np.uint16)
    _check(lib.tqo_pqo_quantize(bits, n, head_dim, x, packed, scales))
    return packed, scales


def pqo_dequantize(bits: int, packed: np.ndarray, scales: np.ndarray, head_dim: int):
    packed = _c(packed, np.uint8)
    scales = _c(scales, np.uint16)
    n = packed.size // (head_dim * bits // 8)
    out = np.zeros((n, head_dim), np.float32)
    _check(lib.tqo_pqo_dequantize(bits, n, head_dim, packed, scales, out))
    return out


OUTLIER_ALL = (1 << 64) - 1


def polar_quantize(bits: int, outlier_blocks: int, x: np.ndarray, head_dim: int, norm_mode: int = 0):
    x = _c(x, np.float32).reshape(-1, head_dim)
    n = x.shape[0]
    packed = np.zeros((n, head_dim * bits // 8), np.uint8)
    scales = np.zeros((n, head_dim // 32), np.uint16)
    _check(lib.tqo_polar_quantize(bits, outlier_blocks, norm_mode, n, head_dim, x, packed, scales))
    return packed, scales


def polar_dequantize(bits: int, outlier_blocks: int, packed: np.ndarray, scales: np.ndarray, head_dim: int,
                     norm_mode: int = 0):
    packed = _c(packed, np.uint8)
    scales = _c(scales, np.uint16)
    n = packed.size // (head_dim * bits // 8)
    out = np.zeros((n, head_dim), np.float32)
    _check(lib.tqo_polar_dequantize(bits, outlier_blocks, norm_mode, n, head_dim, packed, scales, out))
    return out


def tq_signs_norms(x: np.ndarray, xhat: np.ndarray):
    """(signs [N, D/8] u8, norms [N] f16 bits) of the residuals x - xhat (tq.rs:373-412)."""
    x = _c(x, np.float32)
    xhat = _c(xhat, np.float32)
    n, d = x.shape
    signs = np.zeros((n, d // 8), np.uint8)
    norms = np.zeros(n, np.uint16)
    _check(lib.tqo_tq_signs_norms(n, d, x, xhat, signs, norms))
    return signs, norms


def tq_logit_bias(q: np.ndarray, signs: np.ndarray, norms: np.ndarray) -> np.ndarray:
    """q [Hq, q_len, D]; signs [Hkv, T, D/8]; norms [Hkv, T] f16 bits -> [Hq, q_len, T] f32."""
    q = _c(q, np.float32)
    signs = _c(signs, np.uint8)
    norms = _c(norms, np.uint16)
    hq, ql, d = q.shape
    hkv, t = norms.shape
    out = np.zeros((hq, ql, t), np.float32)
    _check(lib.tqo_tq_logit_bias(hq, hkv, d, ql, t, q, signs, norms, out))
    return out


def attention_dense_bias(q, k, v, bias, softmax_scale: float) -> np.ndarray:
    """softmax(scale * (q K^T + bias)) V; q [H, D]; k, v [Hkv, T, D]; bias [H, T]."""
    q, k, v, bias = (_c(a, np.float32) for a in (q, k, v, bias))
    h, d = q.shape
    hkv, t, _ = k.shape
    out = np.zeros((h, d), np.float32)
    _check(lib.tqo_attention_dense_bias(h, hkv, d, t, q, k, v, bias, softmax_scale, out))
    return out


def attention_prefill(q, k, v, softmax_scale: float, causal: bool, bias=None) -> np.ndarray:
    """q [H, L, D]; k, v [Hkv, S, D]; bias [H, L, S] or None -> out [H, L, D]."""
    q, k, v = (_c(a, np.float32) for a in (q, k, v))
    h, ql, d = q.shape
    hkv, t, _ = k.shape
    out = np.zeros((h, ql, d), np.float32)
    b = None
    if bias is not None:
        bias = _c(bias, np.float32)
        b = bias.ctypes.data_as(C.c_void_p)
    _check(lib.tqo_attention_prefill(h, hkv, d, ql, t, q, k, v, b, softmax_scale, 1 if causal else 0, out))
    return out


def attention_dense(q: np.ndarray, k: np.ndarray, v: np.ndarray, softmax_scale: float) -> np.ndarray:
    """q [H, D]; k, v [Hkv, T, D] (dequantized) -> out [H, D] (f32)."""
    q = _c(q, np.float32)
    k = _c(k, np.float32)
    v = _c(v, np.float32)
    h, d = q.shape
    hkv, t, _ = k.shape
    out = np.zeros((h, d), np.float32)
    _check(lib.tqo_attention_dense(h, hkv, d, t, q, k, v, softmax_scale, out))
    return out


# ---- QJL ---------------------------------------------------------------------

def rademacher_row(dim: int, seed: int, row: int) -> np.ndarray:
    out = np.zeros(dim, np.float32)
    lib.tqo_generate_rademacher_row(dim, seed, row, out)
    return out


def compute_qjl_signs(residual: np.ndarray, seed: int) -> np.ndarray:
    r = _c(residual, np.float32)
    out = np.zeros((r.size + 7) // 8, np.uint8)
    _check(lib.tqo_compute_qjl_signs(r, r.size, seed, out))
    return out


def query_projections(q: np.ndarray, seed: int) -> np.ndarray:
    q = _c(q, np.float32)
    out = np.zeros(q.size, np.float32)
    lib.tqo_precompute_query_projections(q, q.size, seed, out)
    return out


def qjl_quantize_batch(total_bits: int, dim: int, rot_seed: int, qjl_seed: int, data: np.ndarray):
    data = _c(data, np.float32).reshape(-1, dim)
    n = data.shape[0]
    pb = total_bits - 1
    packed = np.zeros((n, packed_len(pb, dim)), np.uint8)
    scales = np.zeros(n, np.uint16)
    signs = np.zeros((n, (dim + 7) // 8), np.uint8)
    norms = np.zeros(n, np.uint16)
    _check(lib.tqo_qjl_quantize_batch(total_bits, dim, rot_seed, qjl_seed, n, data, packed, scales, signs, norms))
    return packed, scales, signs, norms


def qjl_scores(polar_bits: int, dim: int, rot_seed: int, qjl_seed: int, queries: np.ndarray, packed, scales,
               signs, norms) -> np.ndarray:
    queries = _c(queries, np.float32).reshape(-1, dim)
    nq = queries.shape[0]
    nk = _c(scales, np.uint16).size
    out = np.zeros((nq, nk), np.float32)
    _check(lib.tqo_qjl_scores_batch(polar_bits, dim, rot_seed, qjl_seed, nq, queries, nk, _c(packed, np.uint8),
                                    _c(scales, np.uint16), _c(signs, np.uint8), _c(norms, np.uint16), out))
    return out


def estimate_inner_product(polar_bits, dim, rot_seed, query, r_query, packed, scale, signs, norm) -> float:
    out = C.c_float()
    _check(lib.tqo_estimate_inner_product(polar_bits, dim, rot_seed, _c(query, np.float32),
                                          _c(r_query, np.float32), _c(packed, np.uint8), int(scale),
                                          _c(signs, np.uint8), int(norm), C.byref(out)))
    return out.value


def weighted_values(polar_bits, dim, rot_seed, packed, scales, weights) -> np.ndarray:
    w = _c(weights, np.float32)
    out = np.zeros(dim, np.float32)
    _check(lib.tqo_weighted_values(polar_bits, dim, rot_seed, w.size, _c(packed, np.uint8),
                                   _c(scales, np.uint16), w, out))
    return out


# ---- generators ----------------------------------------------------------------

def pseudo_random_vec(dim: int, seed: int) -> np.ndarray:
    out = np.zeros(dim, np.float32)
    lib.tqo_pseudo_random_vec(dim, seed, out)
    return out


def lcg_normal_vecs(seed: int, dim: int, count: int) -> np.ndarray:
    out = np.zeros((count, dim), np.float32)
    lib.tqo_lcg_normal_vecs(seed, dim, count, out)
    return out
