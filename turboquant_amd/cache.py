"""Device-resident compressed KV caches with the CompressedKVCache contract of
the reference: PqoCache (src/cache/pqo.rs:21-236; PQO and PQ modes) and
TqCache (src/cache/tq.rs: PQ codes plus the QJL sketch of the keys'
residuals, logit bias on prefill, fused decode with the QJL correction
inline).  The caches live in HBM behind the C ABI (tq_cache_*); tensors here
are PyTorch views for I/O only.  Trait methods as used by the reference's
tests (cache_pqo_tests.rs, cache_type_correctness.rs): prefill, decode,
seq_len, reset, memory_usage.
"""
from __future__ import annotations

import ctypes as C
import enum
from typing import NamedTuple, Optional, Union

import torch

from ._lib import (TQ_DTYPE_BF16, TQ_DTYPE_F16, TQ_DTYPE_F32, TQ_NORM_L2NORM, TQ_NORM_MAXNORM, TQ_OUTLIER_ALL,
                   check, lib)

_DT = {torch.float32: TQ_DTYPE_F32, torch.bfloat16: TQ_DTYPE_BF16, torch.float16: TQ_DTYPE_F16}

QUANT_BLOCK_SIZE = 32        # config.rs:9
DEFAULT_ROTATION_SEED = 42   # config.rs:14
DEFAULT_QJL_SEED = 12345     # config.rs:17
OUTLIER_ALL = TQ_OUTLIER_ALL  # usize::MAX: every block on the outlier codebook (PQO)


class QuantNormMode(enum.IntEnum):
    """config.rs:20-31 (MaxNorm is the default)."""
    L2Norm = TQ_NORM_L2NORM
    MaxNorm = TQ_NORM_MAXNORM


class CacheConfig(NamedTuple):
    """config.rs:50-85: outlier_blocks = OUTLIER_ALL for PQO, 0 for PQ / TQ."""
    bits: int
    head_dim: int
    num_kv_heads: int
    num_layers: int
    norm_mode: QuantNormMode = QuantNormMode.MaxNorm
    outlier_blocks: int = OUTLIER_ALL

    def qjl_enabled(self) -> bool:
        return self.outlier_blocks == 0

    def num_blocks(self) -> int:
        return self.head_dim // QUANT_BLOCK_SIZE

    def packed_dim(self) -> int:
        return self.head_dim * self.bits // 8


class DequantResult(NamedTuple):
    """common.rs:115-121: full K/V of a layer [1, H, S, D]; logit_bias [1, Hq,
    q_len, S] for TQ, None for PQ / PQO."""
    k: torch.Tensor
    v: torch.Tensor
    logit_bias: Optional[torch.Tensor] = None


class AttendConfig(NamedTuple):
    """cache_pqo_tests.rs:130-133."""
    softmax_scale: float
    n_kv_groups: int


class Fused(NamedTuple):
    """DecodeOutput::Fused: the attention output [1, Hq, 1, D]."""
    out: torch.Tensor


class Dequantized(NamedTuple):
    """DecodeOutput::Dequantized: the whole layer plus the logit bias."""
    result: DequantResult


DecodeOutput = Union[Fused, Dequantized]


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_cur_device = getattr(torch._C, "_cuda_getDevice", None)


def _stream() -> int:
    """The current HIP stream of the current device as an integer handle
    (the stream a `torch.cuda.stream(...)` context selects).  torch's raw
    getters return it without building a Stream object, which costs about
    2.5 us of host time per call against 13-14 us for a whole decode step;
    the public API is the fallback."""
    if _raw_stream is not None and _cur_device is not None:
        return _raw_stream(_cur_device())
    return torch.cuda.current_stream().cuda_stream


def _check_kv(k: torch.Tensor, v: torch.Tensor, heads: int, head_dim: int):
    if k.shape != v.shape or k.dim() != 4 or k.shape[0] != 1 or k.shape[1] != heads or k.shape[3] != head_dim:
        raise ValueError(f"k/v must be [1, {heads}, T, {head_dim}], got {tuple(k.shape)} / {tuple(v.shape)}")
    if k.dtype not in _DT or v.dtype != k.dtype:
        raise ValueError("k/v must share one of f32/bf16/f16")
    return k.contiguous(), v.contiguous()


def _check_q(q: torch.Tensor, num_kv_heads: int, head_dim: int) -> torch.Tensor:
    if q.dim() != 4 or q.shape[0] != 1 or q.shape[3] != head_dim or q.shape[1] % num_kv_heads != 0:
        raise ValueError(f"q must be [1, Hq, q_len, {head_dim}] with Hq a multiple of {num_kv_heads}")
    if q.dtype not in _DT:
        raise ValueError("q must be f32/bf16/f16")
    return q.contiguous()


class _DeviceCache:
    """Shared handle logic of PqoCache and TqCache."""

    _qjl = 0

    def __init__(self, config: CacheConfig):
        h = C.c_void_p()
        check(lib.tq_cache_create(config.num_layers, config.num_kv_heads, config.head_dim, config.bits,
                                  int(config.norm_mode), int(config.outlier_blocks), self._qjl, C.byref(h)))
        self._h = h
        self.config = config
        self.num_layers, self.num_kv_heads, self.head_dim, self.bits = (config.num_layers, config.num_kv_heads,
                                                                        config.head_dim, config.bits)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            lib.tq_cache_destroy(h)  # stream-ordered release: no synchronization
            self._h = None

    def _layer_out(self, k: torch.Tensor, s: int):
        k_out = torch.empty((1, self.num_kv_heads, s, self.head_dim), dtype=k.dtype, device=k.device)
        return k_out, torch.empty_like(k_out)

    def seq_len(self, layer: int) -> int:
        return int(lib.tq_cache_seq_len(self._h, layer))

    def capacity(self, layer: int) -> int:
        return int(lib.tq_cache_capacity(self._h, layer))

    def reset(self) -> None:
        check(lib.tq_cache_reset(self._h))

    def memory_usage(self) -> int:
        return int(lib.tq_cache_memory_usage(self._h))

    def read_layer(self, layer: int):
        """(k_idx [H, S, pd] u8, k_sc [H, S, nb] int16, v_idx, v_sc): copies of the stored records."""
        s = self.seq_len(layer)
        pd, nb = self.head_dim * self.bits // 8, self.head_dim // 32
        dev = torch.device("cuda")
        ki = torch.empty((self.num_kv_heads, s, pd), dtype=torch.uint8, device=dev)
        vi = torch.empty_like(ki)
        ks = torch.empty((self.num_kv_heads, s, nb), dtype=torch.int16, device=dev)
        vs = torch.empty_like(ks)
        check(lib.tq_cache_read_layer(self._h, layer, ki.data_ptr(), ks.data_ptr(), vi.data_ptr(), vs.data_ptr(),
                                      None, None, _stream()))
        return ki, ks, vi, vs

    def buffers(self, layer: int):
        """Raw device pointers (k_idx, k_sc, v_idx, v_sc, qjl_signs, qjl_norms) of a layer."""
        ptrs = [C.c_void_p() for _ in range(6)]
        check(lib.tq_cache_buffers(self._h, layer, *[C.byref(p) for p in ptrs]))
        return [p.value for p in ptrs]

    def attend_prefill(self, layer: int, q: torch.Tensor, softmax_scale: float, causal: bool = True,
                       out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        """Multi-query attention of q [1, Hq, q_len, D] over the whole layer (the
        queries at its last q_len positions) straight from the compressed
        records; a TqCache includes the QJL correction.  Returns [1, Hq, q_len, D]."""
        qc = _check_q(q, self.num_kv_heads, self.head_dim)
        hq, ql = qc.shape[1], qc.shape[2]
        out = torch.empty((1, hq, ql, self.head_dim), dtype=out_dtype or qc.dtype, device=qc.device)
        check(lib.tq_cache_attend_prefill(self._h, layer, qc.data_ptr(), _DT[qc.dtype], hq, ql, 1 if causal else 0,
                                          float(softmax_scale), out.data_ptr(), _DT[out.dtype], _stream()))
        return out

    def _prefill(self, layer, k, v, q):
        k, v = _check_kv(k, v, self.num_kv_heads, self.head_dim)
        t = k.shape[2]
        s = self.seq_len(layer) + t
        k_out, v_out = self._layer_out(k, s)
        bias = None
        qc, hq, ql = None, 0, 0
        if self._qjl:
            qc = _check_q(q, self.num_kv_heads, self.head_dim)
            hq, ql = qc.shape[1], qc.shape[2]
            bias = torch.empty((1, hq, ql, s), dtype=qc.dtype, device=k.device)
        orig = C.c_int(0)
        check(lib.tq_cache_prefill(self._h, layer, k.data_ptr(), v.data_ptr(), _DT[k.dtype], t,
                                   qc.data_ptr() if qc is not None else None, _DT[qc.dtype] if qc is not None else 0,
                                   hq, ql, k_out.data_ptr(), v_out.data_ptr(), C.byref(orig),
                                   bias.data_ptr() if bias is not None else None, _stream()))
        if orig.value:
            return DequantResult(k, v, bias)
        return DequantResult(k_out, v_out, bias)

    def _decode_fused(self, layer, k, v, q, config: AttendConfig) -> torch.Tensor:
        k, v = _check_kv(k, v, self.num_kv_heads, self.head_dim)
        qc = _check_q(q, self.num_kv_heads, self.head_dim)
        if qc.shape[2] != 1:
            raise ValueError("decode takes one query position: q [1, Hq, 1, head_dim]")
        hq = qc.shape[1]
        out = torch.empty((1, hq, 1, self.head_dim), dtype=k.dtype, device=k.device)
        check(lib.tq_cache_decode(self._h, layer, k.data_ptr(), v.data_ptr(), _DT[k.dtype], k.shape[2],
                                  qc.data_ptr(), _DT[qc.dtype], hq, float(config.softmax_scale), out.data_ptr(),
                                  _DT[out.dtype], _stream()))
        return out

    def _decode_dequantized(self, layer, k, v, q) -> DequantResult:
        k, v = _check_kv(k, v, self.num_kv_heads, self.head_dim)
        t = k.shape[2]
        s = self.seq_len(layer) + t
        k_out, v_out = self._layer_out(k, s)
        bias = None
        qc, hq, ql = None, 0, 0
        if self._qjl:
            qc = _check_q(q, self.num_kv_heads, self.head_dim)
            hq, ql = qc.shape[1], qc.shape[2]
            bias = torch.empty((1, hq, ql, s), dtype=qc.dtype, device=k.device)
        check(lib.tq_cache_decode_dequantized(self._h, layer, k.data_ptr(), v.data_ptr(), _DT[k.dtype], t,
                                              qc.data_ptr() if qc is not None else None,
                                              _DT[qc.dtype] if qc is not None else 0, hq, ql, k_out.data_ptr(),
                                              v_out.data_ptr(), bias.data_ptr() if bias is not None else None,
                                              _stream()))
        return DequantResult(k_out, v_out, bias)


class PqoCache(_DeviceCache):
    """PqoCache::new(CacheConfig) (pqo.rs:21-51).  `PqoCache(config)` or the
    earlier `PqoCache(num_layers, num_kv_heads, head_dim, bits)` (PQO)."""

    _qjl = 0

    def __init__(self, config_or_layers, num_kv_heads: int = None, head_dim: int = None, bits: int = None):
        if isinstance(config_or_layers, CacheConfig):
            config = config_or_layers
        else:
            config = CacheConfig(bits=bits, head_dim=head_dim, num_kv_heads=num_kv_heads,
                                 num_layers=config_or_layers)
        super().__init__(config)

    def prefill(self, layer: int, k: torch.Tensor, v: torch.Tensor, q: Optional[torch.Tensor] = None) -> DequantResult:
        """Stores k, v; returns them unchanged on the layer's first call, else the
        whole dequantized layer in k's dtype (pqo.rs:184-200).  No logit bias."""
        return self._prefill(layer, k, v, None)

    def decode(self, layer: int, k: torch.Tensor, v: torch.Tensor, q: torch.Tensor,
               config: AttendConfig) -> torch.Tensor:
        """Stores k, v and returns the fused attention output [1, Hq, 1, D] in k's
        dtype (DecodeOutput::Fused, pqo.rs:202-222 on the device path)."""
        return self._decode_fused(layer, k, v, q, config)

    def decode_dequantized(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> DequantResult:
        """Stores k, v and returns the whole dequantized layer (the reference's
        CPU decode path, pqo.rs:218-221)."""
        return self._decode_dequantized(layer, k, v, None)

    def decode_output(self, layer: int, k, v, q, config: AttendConfig) -> DecodeOutput:
        """DecodeOutput as the trait returns it: Fused for PQO and PQ configs;
        Dequantized for mixed outlier configs, which the fused kernel does not
        take (the reference's CUDA path would read them with the outlier
        codebook only, pqo.rs:152)."""
        ob = self.config.outlier_blocks
        if 0 < ob < self.config.num_blocks():
            return Dequantized(self.decode_dequantized(layer, k, v))
        return Fused(self.decode(layer, k, v, q, config))


class TqCache(_DeviceCache):
    """TqCache::new(CacheConfig) (tq.rs:20-57): the standard (bits-1)-bit
    codebook in bits-wide slots plus a 1-bit QJL sketch of every key's
    residual (DEFAULT_QJL_SEED).  Requires outlier_blocks == 0."""

    _qjl = 1

    def __init__(self, config: CacheConfig):
        super().__init__(config)

    def prefill(self, layer: int, k: torch.Tensor, v: torch.Tensor, q: torch.Tensor) -> DequantResult:
        """tq.rs:258-273: stores k, v (and the keys' signs and residual norms);
        K/V as PqoCache.prefill, logit_bias [1, Hq, q_len, seq_len] in q's dtype."""
        return self._prefill(layer, k, v, q)

    def decode(self, layer: int, k: torch.Tensor, v: torch.Tensor, q: torch.Tensor,
               config: AttendConfig) -> torch.Tensor:
        """Stores k, v and returns the fused attention output [1, Hq, 1, D] with
        the QJL correction in the logits (the Fused variant; the reference's
        CUDA kernel carries this branch dormant, tq_attention_kernel.cu:192-231)."""
        return self._decode_fused(layer, k, v, q, config)

    def decode_dequantized(self, layer: int, k: torch.Tensor, v: torch.Tensor, q: torch.Tensor) -> DequantResult:
        """The reference's TqCache::decode (tq.rs:275-297): whole dequantized layer
        plus the logit bias for q."""
        return self._decode_dequantized(layer, k, v, q)

    def decode_output(self, layer: int, k, v, q, config: AttendConfig) -> DecodeOutput:
        return Fused(self.decode(layer, k, v, q, config))

    def read_qjl(self, layer: int):
        """(signs [H, S, D/8] u8, norms [H, S] int16 f16 bits) of the stored keys."""
        s = self.seq_len(layer)
        dev = torch.device("cuda")
        ki = torch.empty((self.num_kv_heads, s, self.head_dim * self.bits // 8), dtype=torch.uint8, device=dev)
        ks = torch.empty((self.num_kv_heads, s, self.head_dim // 32), dtype=torch.int16, device=dev)
        vi, vs = torch.empty_like(ki), torch.empty_like(ks)
        sg = torch.empty((self.num_kv_heads, s, self.head_dim // 8), dtype=torch.uint8, device=dev)
        nm = torch.empty((self.num_kv_heads, s), dtype=torch.int16, device=dev)
        check(lib.tq_cache_read_layer(self._h, layer, ki.data_ptr(), ks.data_ptr(), vi.data_ptr(), vs.data_ptr(),
                                      sg.data_ptr(), nm.data_ptr(), _stream()))
        return sg, nm
