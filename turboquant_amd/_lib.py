"""ctypes binding of libturboquant_amd.so (the C ABI in include/turboquant_amd.h).

Loading fails loudly if the library is missing: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libturboquant_amd.so")

TQ_DTYPE_F32, TQ_DTYPE_BF16, TQ_DTYPE_F16 = 0, 1, 2
TQ_NORM_MAXNORM, TQ_NORM_L2NORM = 0, 1
TQ_OUTLIER_ALL = (1 << 64) - 1  # CacheConfig::outlier_blocks = usize::MAX (PQO)

ERRORS = {
    1: "InvalidDimension",
    2: "UnsupportedBits",
    3: "DimensionMismatch",
    4: "LayerOutOfRange",
    5: "RangeOutOfBounds",
    6: "InvalidArgument",
    7: "DeviceError",
}

_p = C.c_void_p
_i = C.c_int
_f = C.c_float
_sz = C.c_size_t
_ll = C.c_longlong
_u64 = C.c_uint64

# name -> (restype, argtypes); every symbol declared in include/turboquant_amd.h
SIGNATURES = {
    "tq_last_error": (C.c_char_p, []),
    "tq_version": (C.c_char_p, []),
    "tq_dequant_batch": (_i, [_p, _p, _p, _p, _p, _i, _i, _i, _i, _p]),
    "tq_quant_maxnorm_batch": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _i, _f, _f, _p]),
    "tq_pack_indices": (_i, [_p, _p, _i, _i, _i, _i, _p]),
    "tq_fused_attention": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i,
                                _i, _i, _i, _f, _i, _p]),
    "tq_pqo_quantize": (_i, [_p, _i, _p, _p, _sz, _i, _i, _p]),
    "tq_pqo_dequantize": (_i, [_p, _p, _p, _i, _sz, _i, _i, _p]),
    "tq_attention_workspace_size": (_sz, [_i, _i, _i, _i, _i]),
    "tq_attention_workspace_init": (_i, [_p, _sz, _i, _i, _i, _i, _i, _p]),
    "tq_pqo_decode_attention": (_i, [_p, _i, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _ll, _ll, _f, _p, _i,
                                     _p, _sz, _p]),
    "tq_pqo_decode_attention_noalloc": (_i, [_p, _i, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _ll, _ll, _f, _p,
                                             _i, _p]),
    "tq_quantize_vec_batch": (_i, [_p, _p, _p, _sz, _i, _i, _u64, _p]),
    "tq_dequantize_vec_batch": (_i, [_p, _p, _p, _sz, _i, _i, _u64, _p]),
    "tq_dequantize_rotated_batch": (_i, [_p, _p, _p, _sz, _i, _i, _p]),
    "tq_qjl_quantize_batch": (_i, [_p, _p, _p, _p, _p, _sz, _i, _i, _u64, _u64, _p]),
    "tq_qjl_query_context": (_i, [_p, _p, _sz, _i, _u64, _u64, _p]),
    "tq_qjl_scores": (_i, [_p, _sz, _p, _p, _p, _p, _sz, _i, _i, _u64, _p, _p]),
    "tq_softmax_rows": (_i, [_p, _p, _sz, _sz, _f, _p]),
    "tq_qjl_weighted_values_workspace_size": (_sz, [_sz, _sz, _i]),
    "tq_qjl_weighted_values": (_i, [_p, _p, _sz, _p, _sz, _i, _i, _u64, _p, _p, _sz, _p]),
    "tq_pqo_quantize_to_cache": (_i, [_p, _i, _i, _i, _p, _p, _ll, _ll, _i, _i, _p]),
    "tq_pqo_dequantize_from_cache": (_i, [_p, _p, _ll, _i, _i, _p, _i, _i, _i, _p]),
    "tq_polar_quantize": (_i, [_p, _i, _p, _p, _sz, _i, _i, _sz, _i, _p]),
    "tq_polar_dequantize": (_i, [_p, _p, _p, _i, _sz, _i, _i, _sz, _i, _p]),
    "tq_polar_quantize_to_cache": (_i, [_p, _i, _i, _i, _p, _p, _ll, _ll, _i, _i, _sz, _i, _p]),
    "tq_polar_dequantize_from_cache": (_i, [_p, _p, _ll, _i, _i, _p, _i, _i, _i, _sz, _i, _p]),
    "tq_cache_decode_attention": (_i, [_p, _i, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _sz, _i, _i,
                                       _ll, _ll, _f, _p, _i, _p, _sz, _p]),
    "tq_tq_decode_attention": (_i, [_p, _i, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i, _ll, _ll,
                                    _f, _p, _i, _p, _sz, _p]),
    "tq_qjl_sign_matrix": (_i, [_p, _i, _u64, _p]),
    "tq_cache_prefill_attention": (_i, [_p, _i, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _sz, _i, _i, _ll, _i,
                                        _f, _p, _i, _p]),
    "tq_cache_attend_prefill": (_i, [_p, _i, _p, _i, _i, _i, _i, _f, _p, _i, _p]),
    "tq_qjl_cache_sketch": (_i, [_p, _i, _i, _i, _p, _p, _p, _p, _p, _ll, _ll, _i, _i, _sz, _i, _p]),
    "tq_qjl_project": (_i, [_p, _i, _p, _p, _sz, _i, _p]),
    "tq_qjl_cache_sketch_project": (_i, [_p, _i, _i, _i, _p, _p, _p, _p, _p, _ll, _ll, _i, _i, _sz, _i, _p, _i, _p,
                                         _sz, _p]),
    "tq_qjl_bias_scale": (_f, [_i]),
    "tq_qjl_logit_bias": (_i, [_p, _i, _i, _p, _p, _i, _i, _ll, _i, _p, _i, _p]),
    "tq_cache_create": (_i, [_i, _i, _i, _i, _i, _sz, _i, C.POINTER(C.c_void_p)]),
    "tq_cache_destroy": (None, [_p]),
    "tq_cache_is_tq": (_i, [_p]),
    "tq_cache_prefill": (_i, [_p, _i, _p, _p, _i, _i, _p, _i, _i, _i, _p, _p, C.POINTER(C.c_int), _p, _p]),
    "tq_cache_decode": (_i, [_p, _i, _p, _p, _i, _i, _p, _i, _i, _f, _p, _i, _p]),
    "tq_cache_decode_dequantized": (_i, [_p, _i, _p, _p, _i, _i, _p, _i, _i, _i, _p, _p, _p, _p]),
    "tq_cache_seq_len": (_sz, [_p, _i]),
    "tq_cache_reset": (_i, [_p]),
    "tq_cache_memory_usage": (_sz, [_p]),
    "tq_cache_capacity": (_sz, [_p, _i]),
    "tq_cache_read_layer": (_i, [_p, _i, _p, _p, _p, _p, _p, _p, _p]),
    "tq_cache_buffers": (_i, [_p, _i] + [C.POINTER(C.c_void_p)] * 6),
    "tq_tq_cache_create": (_i, [_i, _i, _i, _i, C.POINTER(C.c_void_p)]),
    "tq_pqo_cache_create": (_i, [_i, _i, _i, _i, C.POINTER(C.c_void_p)]),
    "tq_pqo_cache_destroy": (None, [_p]),
    "tq_pqo_cache_prefill": (_i, [_p, _i, _p, _p, _i, _i, _p, _p, C.POINTER(C.c_int), _p]),
    "tq_pqo_cache_decode": (_i, [_p, _i, _p, _p, _i, _i, _p, _i, _i, _f, _p, _i, _p]),
    "tq_pqo_cache_seq_len": (_sz, [_p, _i]),
    "tq_pqo_cache_reset": (_i, [_p]),
    "tq_pqo_cache_memory_usage": (_sz, [_p]),
    "tq_pqo_cache_capacity": (_sz, [_p, _i]),
    "tq_pqo_cache_read_layer": (_i, [_p, _i, _p, _p, _p, _p, _p]),
    "tq_pqo_cache_buffers": (_i, [_p, _i, C.POINTER(C.c_void_p), C.POINTER(C.c_void_p), C.POINTER(C.c_void_p),
                                  C.POINTER(C.c_void_p)]),
}


class TurboQuantError(RuntimeError):
    """Raised when a C ABI call returns a non-zero status."""

    def __init__(self, code: int, message: str):
        super().__init__(f"{ERRORS.get(code, code)}: {message}")
        self.code = code


def _load() -> C.CDLL:
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"turboquant_amd native library not built: {LIB_PATH} "
            "(run `python -m turboquant_amd.build`)")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def check(rc: int) -> None:
    if rc != 0:
        raise TurboQuantError(rc, lib.tq_last_error().decode())
