"""PqoCache: device-resident PQO KV cache with the CompressedKVCache contract
of the reference (src/cache/pqo.rs:183-236; trait from mistralrs-kv-cache,
methods as used by cache_pqo_tests.rs).  The cache lives in HBM behind the C
ABI (tq_pqo_cache_*); tensors here are PyTorch views for I/O only.
"""
from __future__ import annotations

import ctypes as C
from typing import NamedTuple, Optional

import torch

from ._lib import TQ_DTYPE_BF16, TQ_DTYPE_F16, TQ_DTYPE_F32, check, lib

_DT = {torch.float32: TQ_DTYPE_F32, torch.bfloat16: TQ_DTYPE_BF16, torch.float16: TQ_DTYPE_F16}


class DequantResult(NamedTuple):
    """common.rs:115-121: full K/V of a layer [1, H, S, D]; PQO has no logit bias."""
    k: torch.Tensor
    v: torch.Tensor
    logit_bias: Optional[torch.Tensor] = None


class AttendConfig(NamedTuple):
    """cache_pqo_tests.rs:130-133."""
    softmax_scale: float
    n_kv_groups: int


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _check_kv(k: torch.Tensor, v: torch.Tensor, heads: int, head_dim: int):
    if k.shape != v.shape or k.dim() != 4 or k.shape[0] != 1 or k.shape[1] != heads or k.shape[3] != head_dim:
        raise ValueError(f"k/v must be [1, {heads}, T, {head_dim}], got {tuple(k.shape)} / {tuple(v.shape)}")
    if k.dtype not in _DT or v.dtype != k.dtype:
        raise ValueError("k/v must share one of f32/bf16/f16")
    return k.contiguous(), v.contiguous()


class PqoCache:
    """PqoCache::new(CacheConfig{bits, head_dim, num_kv_heads, num_layers, PQO})."""

    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, bits: int):
        h = C.c_void_p()
        check(lib.tq_pqo_cache_create(num_layers, num_kv_heads, head_dim, bits, C.byref(h)))
        self._h = h
        self.num_layers, self.num_kv_heads, self.head_dim, self.bits = num_layers, num_kv_heads, head_dim, bits

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            torch.cuda.synchronize()
            lib.tq_pqo_cache_destroy(h)
            self._h = None

    def prefill(self, layer: int, k: torch.Tensor, v: torch.Tensor, q: Optional[torch.Tensor] = None) -> DequantResult:
        """Stores k, v; returns them unchanged on the layer's first call, else the
        whole dequantized layer in k's dtype (pqo.rs:184-200)."""
        k, v = _check_kv(k, v, self.num_kv_heads, self.head_dim)
        t = k.shape[2]
        s = self.seq_len(layer) + t
        k_out = torch.empty((1, self.num_kv_heads, s, self.head_dim), dtype=k.dtype, device=k.device)
        v_out = torch.empty_like(k_out)
        orig = C.c_int(0)
        check(lib.tq_pqo_cache_prefill(self._h, layer, k.data_ptr(), v.data_ptr(), _DT[k.dtype], t, k_out.data_ptr(),
                                       v_out.data_ptr(), C.byref(orig), _stream()))
        return DequantResult(k, v) if orig.value else DequantResult(k_out, v_out)

    def decode(self, layer: int, k: torch.Tensor, v: torch.Tensor, q: torch.Tensor,
               config: AttendConfig) -> torch.Tensor:
        """Stores k, v and returns the fused attention output [1, Hq, 1, D] in k's
        dtype (DecodeOutput::Fused, pqo.rs:202-222 on the device path)."""
        k, v = _check_kv(k, v, self.num_kv_heads, self.head_dim)
        if q.dim() != 4 or q.shape[0] != 1 or q.shape[2] != 1 or q.shape[3] != self.head_dim:
            raise ValueError("q must be [1, Hq, 1, head_dim]")
        hq = q.shape[1]
        qc = q.contiguous()
        out = torch.empty((1, hq, 1, self.head_dim), dtype=k.dtype, device=k.device)
        check(lib.tq_pqo_cache_decode(self._h, layer, k.data_ptr(), v.data_ptr(), _DT[k.dtype], k.shape[2],
                                      qc.data_ptr(), _DT[qc.dtype], hq, float(config.softmax_scale),
                                      out.data_ptr(), _DT[out.dtype], _stream()))
        return out

    def seq_len(self, layer: int) -> int:
        return int(lib.tq_pqo_cache_seq_len(self._h, layer))

    def capacity(self, layer: int) -> int:
        return int(lib.tq_pqo_cache_capacity(self._h, layer))

    def reset(self) -> None:
        check(lib.tq_pqo_cache_reset(self._h))

    def memory_usage(self) -> int:
        return int(lib.tq_pqo_cache_memory_usage(self._h))

    def read_layer(self, layer: int):
        """(k_idx [H, S, pd] u8, k_sc [H, S, nb] int16, v_idx, v_sc): copies of the stored records."""
        s = self.seq_len(layer)
        pd, nb = self.head_dim * self.bits // 8, self.head_dim // 32
        dev = torch.device("cuda")
        ki = torch.empty((self.num_kv_heads, s, pd), dtype=torch.uint8, device=dev)
        vi = torch.empty_like(ki)
        ks = torch.empty((self.num_kv_heads, s, nb), dtype=torch.int16, device=dev)
        vs = torch.empty_like(ks)
        check(lib.tq_pqo_cache_read_layer(self._h, layer, ki.data_ptr(), ks.data_ptr(), vi.data_ptr(), vs.data_ptr(),
                                          _stream()))
        return ki, ks, vi, vs

    def buffers(self, layer: int):
        """Raw device pointers (k_idx, k_sc, v_idx, v_sc) of a layer."""
        ptrs = [C.c_void_p() for _ in range(4)]
        check(lib.tq_pqo_cache_buffers(self._h, layer, *[C.byref(p) for p in ptrs]))
        return [p.value for p in ptrs]
