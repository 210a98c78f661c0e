"""turboquant_amd -- MI355X-native TurboQuant KV-cache hot path.

Thin Python surface over the C ABI (include/turboquant_amd.h) for tests and
benchmarks.  Device memory and streams come from PyTorch (ROCm); every
compute call goes to the hand-written gfx950 kernels in
libturboquant_amd.so.  There is no CPU fallback: importing this package
without the built library raises.
"""
from __future__ import annotations

import math

import torch

from ._lib import (TQ_DTYPE_BF16, TQ_DTYPE_F16, TQ_DTYPE_F32, TQ_NORM_MAXNORM, TQ_OUTLIER_ALL, TurboQuantError,
                   check, lib)
from .cache import (AttendConfig, CacheConfig, DecodeOutput, Dequantized, DequantResult, Fused, PqoCache,
                    QuantNormMode, TqCache)

__all__ = [
    "TurboQuantError", "lib", "pqo_quantize", "pqo_dequantize", "quant_maxnorm_batch", "dequant_batch",
    "pack_indices", "fused_attention", "AttentionWorkspace", "pqo_decode_attention", "pqo_codebook_values",
    "quantize_vec_batch", "dequantize_vec_batch", "dequantize_rotated_batch", "qjl_quantize_batch",
    "qjl_query_context", "qjl_scores", "softmax_rows", "qjl_weighted_values", "PqoCache", "AttendConfig",
    "DequantResult", "TqCache", "CacheConfig", "QuantNormMode", "DecodeOutput", "Fused", "Dequantized",
    "polar_quantize", "polar_dequantize", "cache_decode_attention", "qjl_sign_matrix", "qjl_project",
    "qjl_cache_sketch", "qjl_logit_bias", "cache_prefill_attention",
]

_DT = {torch.float32: TQ_DTYPE_F32, torch.bfloat16: TQ_DTYPE_BF16, torch.float16: TQ_DTYPE_F16}


from .cache import _stream  # noqa: E402  (the current HIP stream's handle)


def _ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("expected a device tensor")
    if not t.is_contiguous():
        raise ValueError("expected a contiguous tensor")
    return t.data_ptr()


def pqo_quantize(x: torch.Tensor, bits: int):
    """PQO quantize [N, head_dim] (f32/bf16/f16) with the fused block rotation.

    Returns (packed u8 [N, head_dim*bits/8], scales int16 [N, head_dim/32]
    holding f16 bits, negative = outlier block)."""
    if x.dim() != 2:
        raise ValueError("x must be [N, head_dim]")
    n, hd = x.shape
    packed = torch.empty((n, hd * bits // 8), dtype=torch.uint8, device=x.device)
    scales = torch.empty((n, max(hd // 32, 1)), dtype=torch.int16, device=x.device)
    check(lib.tq_pqo_quantize(_ptr(x), _DT[x.dtype], _ptr(packed), _ptr(scales), n, hd, bits, _stream()))
    return packed, scales


def polar_quantize(x: torch.Tensor, bits: int, outlier_blocks: int = TQ_OUTLIER_ALL,
                   norm_mode: int = TQ_NORM_MAXNORM):
    """polar_quantize (quantize_tensor.rs:40-76) of [N, head_dim] for a cache mode:
    outlier_blocks TQ_OUTLIER_ALL (PQO) or 0 (PQ / TQ: (bits-1)-bit codes in
    bits-wide slots, positive scales)."""
    if x.dim() != 2:
        raise ValueError("x must be [N, head_dim]")
    n, hd = x.shape
    packed = torch.empty((n, hd * bits // 8), dtype=torch.uint8, device=x.device)
    scales = torch.empty((n, max(hd // 32, 1)), dtype=torch.int16, device=x.device)
    check(lib.tq_polar_quantize(_ptr(x), _DT[x.dtype], _ptr(packed), _ptr(scales), n, hd, bits, int(outlier_blocks),
                                int(norm_mode), _stream()))
    return packed, scales


def polar_dequantize(packed: torch.Tensor, scales: torch.Tensor, bits: int, head_dim: int,
                     outlier_blocks: int = TQ_OUTLIER_ALL, norm_mode: int = TQ_NORM_MAXNORM,
                     out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    n = packed.shape[0]
    out = torch.empty((n, head_dim), dtype=out_dtype, device=packed.device)
    check(lib.tq_polar_dequantize(_ptr(packed), _ptr(scales), _ptr(out), _DT[out_dtype], n, head_dim, bits,
                                  int(outlier_blocks), int(norm_mode), _stream()))
    return out


def pqo_dequantize(packed: torch.Tensor, scales: torch.Tensor, bits: int, head_dim: int,
                   out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    n = packed.shape[0]
    out = torch.empty((n, head_dim), dtype=out_dtype, device=packed.device)
    check(lib.tq_pqo_dequantize(_ptr(packed), _ptr(scales), _ptr(out), _DT[out_dtype], n, head_dim, bits,
                                _stream()))
    return out


def quant_maxnorm_batch(rotated: torch.Tensor, boundaries: torch.Tensor, bits: int, outer_centroid: float,
                        scale_sign: float = -1.0):
    """Reference-ABI quantize of already-rotated f32 blocks [num_blocks, 32]."""
    nb = rotated.numel() // 32
    bpb = 32 * bits // 8
    packed = torch.empty((nb, bpb), dtype=torch.uint8, device=rotated.device)
    scales = torch.empty((nb,), dtype=torch.int16, device=rotated.device)
    check(lib.tq_quant_maxnorm_batch(_ptr(rotated), _ptr(boundaries), _ptr(packed), _ptr(scales), nb, 32, bits,
                                     boundaries.numel(), bpb, float(outer_centroid), float(scale_sign), _stream()))
    return packed, scales


def dequant_batch(packed: torch.Tensor, scales: torch.Tensor, codebook: torch.Tensor, sign_pattern: torch.Tensor,
                  bits: int) -> torch.Tensor:
    """Reference-ABI dequantize: [num_blocks, 32] f32."""
    nb = scales.numel()
    out = torch.empty((nb, 32), dtype=torch.float32, device=packed.device)
    check(lib.tq_dequant_batch(_ptr(packed), _ptr(scales), _ptr(codebook), _ptr(sign_pattern), _ptr(out), nb, 32,
                               bits, 32 * bits // 8, _stream()))
    return out


def pack_indices(indices: torch.Tensor, bits: int, bytes_per_block: int | None = None) -> torch.Tensor:
    """Reference-ABI packing of [num_vectors, block_size] u8 codes.  The default
    bytes_per_block follows the reference packers' zero-padded tails
    (whole 3-byte groups for 3-bit, packed/indices.rs:72-78)."""
    nv, bs = indices.shape
    if bytes_per_block is None:
        bytes_per_block = {2: (bs + 3) // 4, 3: ((bs + 7) // 8) * 3, 4: (bs + 1) // 2}[bits]
    bpb = bytes_per_block
    out = torch.empty((nv, bpb), dtype=torch.uint8, device=indices.device)
    check(lib.tq_pack_indices(_ptr(indices), _ptr(out), nv, bs, bits, bpb, _stream()))
    return out


def fused_attention(q, k_idx, k_sc, v_idx, v_sc, codebook, sign_pattern, num_kv_heads, kv_len, kv_stride, bits,
                    softmax_scale, qjl=None):
    """Reference-ABI fused decode attention (single sequence, f32 q/out), with
    the caller's partials sized as cuda/attention.rs:70-77 sizes them:
    ceil(kv_len / 512) partitions.  qjl = (rq, signs, residual_norms) attends
    TQ records with the QJL correction (qjl_enabled = 1)."""
    h, hd = q.shape
    p = (kv_len + 511) // 512
    dev = q.device
    out = torch.zeros((h, hd), dtype=torch.float32, device=dev)
    po = torch.zeros((h * max(p, 1), hd), dtype=torch.float32, device=dev)
    pm = torch.zeros((h * max(p, 1),), dtype=torch.float32, device=dev)
    ps = torch.zeros((h * max(p, 1),), dtype=torch.float32, device=dev)
    rq, sg, nm = qjl if qjl is not None else (None, None, None)
    check(lib.tq_fused_attention(_ptr(q), _ptr(k_idx), _ptr(k_sc), _ptr(v_idx), _ptr(v_sc), _ptr(codebook),
                                 _ptr(sign_pattern), _ptr(out), _ptr(po), _ptr(pm), _ptr(ps),
                                 _ptr(sg), _ptr(nm), _ptr(rq), int(qjl is not None),
                                 h, num_kv_heads, hd, kv_len, kv_stride, hd * bits // 8, hd // 32, bits,
                                 float(softmax_scale), p, _stream()))
    return out


class AttentionWorkspace:
    """Device workspace for pqo_decode_attention (split-K partials + counters)."""

    def __init__(self, batch: int, num_heads: int, num_kv_heads: int, head_dim: int, max_kv_len: int,
                 device="cuda"):
        self.shape = (batch, num_heads, num_kv_heads, head_dim, max_kv_len)
        self.nbytes = lib.tq_attention_workspace_size(batch, num_heads, num_kv_heads, head_dim, max_kv_len)
        if self.nbytes == 0:
            raise ValueError("invalid workspace shape")
        self.buf = torch.empty((self.nbytes,), dtype=torch.uint8, device=device)
        check(lib.tq_attention_workspace_init(_ptr(self.buf), self.nbytes, batch, num_heads, num_kv_heads, head_dim,
                                              max_kv_len, _stream()))


def pqo_decode_attention(q, k_idx, k_sc, v_idx, v_sc, kv_lens, num_kv_heads, bits, max_kv_len, kv_head_stride,
                         seq_stride, softmax_scale, workspace: AttentionWorkspace,
                         out_dtype: torch.dtype = torch.float32, out: torch.Tensor | None = None):
    """Batched fused decode attention.  q [B, H, D]; kv_lens int32 [B] (device)."""
    b, h, hd = q.shape
    if out is None:
        out = torch.empty((b, h, hd), dtype=out_dtype, device=q.device)
    check(lib.tq_pqo_decode_attention(_ptr(q), _DT[q.dtype], _ptr(k_idx), _ptr(k_sc), _ptr(v_idx), _ptr(v_sc),
                                      _ptr(kv_lens), b, h, num_kv_heads, hd, bits, max_kv_len, kv_head_stride,
                                      seq_stride, float(softmax_scale), _ptr(out), _DT[out.dtype],
                                      _ptr(workspace.buf), workspace.nbytes, _stream()))
    return out


def cache_decode_attention(q, k_idx, k_sc, v_idx, v_sc, kv_lens, num_kv_heads, bits, max_kv_len, kv_head_stride,
                           seq_stride, softmax_scale, workspace: AttentionWorkspace, outlier_blocks: int,
                           rq: torch.Tensor | None = None, qjl_signs: torch.Tensor | None = None,
                           qjl_norms: torch.Tensor | None = None, out_dtype: torch.dtype = torch.float32,
                           qjl_sign_matrix: torch.Tensor | None = None):
    """Fused decode attention over PQO / PQ records, or TQ records with the QJL
    correction when qjl_signs is given (rq [B, H, D] f32 = R q; or rq None and
    qjl_sign_matrix given: the decode launch projects the query itself)."""
    b, h, hd = q.shape
    out = torch.empty((b, h, hd), dtype=out_dtype, device=q.device)
    if rq is None and qjl_sign_matrix is not None:
        check(lib.tq_tq_decode_attention(_ptr(q), _DT[q.dtype], _ptr(k_idx), _ptr(k_sc), _ptr(v_idx), _ptr(v_sc),
                                         _ptr(qjl_signs), _ptr(qjl_norms), _ptr(qjl_sign_matrix), _ptr(kv_lens), b,
                                         h, num_kv_heads, hd, bits, TQ_NORM_MAXNORM, max_kv_len, kv_head_stride,
                                         seq_stride, float(softmax_scale), _ptr(out), _DT[out.dtype],
                                         _ptr(workspace.buf), workspace.nbytes, _stream()))
        return out
    check(lib.tq_cache_decode_attention(_ptr(q), _DT[q.dtype], _ptr(k_idx), _ptr(k_sc), _ptr(v_idx), _ptr(v_sc),
                                        _ptr(rq), _ptr(qjl_signs), _ptr(qjl_norms), _ptr(kv_lens), b, h,
                                        num_kv_heads, hd, bits, int(outlier_blocks), TQ_NORM_MAXNORM, max_kv_len,
                                        kv_head_stride, seq_stride, float(softmax_scale), _ptr(out), _DT[out.dtype],
                                        _ptr(workspace.buf), workspace.nbytes, _stream()))
    return out


def cache_prefill_attention(q, k_idx, k_sc, v_idx, v_sc, num_kv_heads, bits, kv_len, kv_head_stride, softmax_scale,
                            outlier_blocks: int, causal: bool = True, rq=None, qjl_signs=None, qjl_norms=None,
                            out_dtype: torch.dtype = torch.float32):
    """Multi-query attention over compressed records: q [H, L, D] -> [H, L, D];
    query i at position kv_len - L + i (causal: sees tokens up to it)."""
    h, ql, hd = q.shape
    out = torch.empty((h, ql, hd), dtype=out_dtype, device=q.device)
    check(lib.tq_cache_prefill_attention(_ptr(q), _DT[q.dtype], _ptr(k_idx), _ptr(k_sc), _ptr(v_idx), _ptr(v_sc),
                                         _ptr(rq), _ptr(qjl_signs), _ptr(qjl_norms), h, ql, num_kv_heads, hd, bits,
                                         int(outlier_blocks), TQ_NORM_MAXNORM, kv_len, kv_head_stride,
                                         1 if causal else 0, float(softmax_scale), _ptr(out), _DT[out.dtype],
                                         _stream()))
    return out


def qjl_sign_matrix(dim: int, qjl_seed: int, device="cuda") -> torch.Tensor:
    """Sign bits of R: int32 [dim * dim / 32], bit b of word j*dim/32 + w set <=> R[j][32w+b] < 0."""
    out = torch.empty((dim * dim // 32,), dtype=torch.int32, device=device)
    check(lib.tq_qjl_sign_matrix(_ptr(out), dim, qjl_seed, _stream()))
    return out


def qjl_project(q: torch.Tensor, sign_matrix: torch.Tensor) -> torch.Tensor:
    """rq = R q per row of q [N, dim] (f32 out)."""
    n, d = q.shape
    rq = torch.empty((n, d), dtype=torch.float32, device=q.device)
    check(lib.tq_qjl_project(_ptr(q), _DT[q.dtype], _ptr(sign_matrix), _ptr(rq), n, d, _stream()))
    return rq


def qjl_cache_sketch(k: torch.Tensor, packed_cache, scales_cache, sign_matrix, signs_cache, norms_cache,
                     head_stride: int, offset: int, bits: int, outlier_blocks: int = 0):
    """Signs and residual norms of keys k [H, T, D] already stored at records h*head_stride + offset + t."""
    h, t, d = k.shape
    check(lib.tq_qjl_cache_sketch(_ptr(k), _DT[k.dtype], h, t, _ptr(packed_cache), _ptr(scales_cache),
                                  _ptr(sign_matrix), _ptr(signs_cache), _ptr(norms_cache), head_stride, offset, d,
                                  bits, int(outlier_blocks), TQ_NORM_MAXNORM, _stream()))


def qjl_logit_bias(rq: torch.Tensor, signs_cache, norms_cache, num_kv_heads: int, kv_len: int, head_stride: int,
                   out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """compute_logit_bias: rq [Hq, q_len, D] f32 -> bias [Hq, q_len, kv_len]."""
    hq, ql, d = rq.shape
    out = torch.empty((hq, ql, kv_len), dtype=out_dtype, device=rq.device)
    check(lib.tq_qjl_logit_bias(_ptr(rq), hq, ql, _ptr(signs_cache), _ptr(norms_cache), num_kv_heads, kv_len,
                                head_stride, d, _ptr(out), _DT[out_dtype], _stream()))
    return out


def pqo_codebook_values(bits: int):
    """(centroids, boundaries, outer) of the PQO MaxNorm codebook, f32 arithmetic as in
    src/cache/precomputed/codebooks.rs:51-88 (host-side constants)."""
    import numpy as np
    r = np.float32(2.1573)
    if bits == 3:
        c = np.array([-2.1573, -1.3336, -0.7434, -0.2428, 0.2428, 0.7434, 1.3336, 2.1573], np.float32)
        b = np.array([-1.7455, -1.0385, -0.4931, 0.0, 0.4931, 1.0385, 1.7455], np.float32)
    elif bits == 4:
        step = np.float32(np.float32(2.0) * r) / np.float32(15.0)
        c = np.array([-r + np.float32(i) * step for i in range(16)], np.float32)
        b = np.array([-r + (np.float32(i) + np.float32(0.5)) * step for i in range(15)], np.float32)
    else:
        raise ValueError("bits must be 3 or 4")
    return c, b, np.float32(c.max())


def quantize_vec_batch(x: torch.Tensor, bits: int, rotation_seed: int = 0):
    """Core codec quantize_vec over the rows of x [N, dim] f32 (dim 32..256).
    Returns (packed u8 [N, dim*bits/8], scales int16 [N] holding f16 bits)."""
    if x.dim() != 2 or x.dtype != torch.float32:
        raise ValueError("x must be f32 [N, dim]")
    n, d = x.shape
    packed = torch.empty((n, d * bits // 8), dtype=torch.uint8, device=x.device)
    scales = torch.empty((n,), dtype=torch.int16, device=x.device)
    check(lib.tq_quantize_vec_batch(_ptr(x), _ptr(packed), _ptr(scales), n, bits, d, rotation_seed, _stream()))
    return packed, scales


def dequantize_vec_batch(packed: torch.Tensor, scales: torch.Tensor, bits: int, dim: int, rotation_seed: int = 0):
    n = scales.numel()
    out = torch.empty((n, dim), dtype=torch.float32, device=packed.device)
    check(lib.tq_dequantize_vec_batch(_ptr(packed), _ptr(scales), _ptr(out), n, bits, dim, rotation_seed,
                                      _stream()))
    return out


def dequantize_rotated_batch(packed: torch.Tensor, scales: torch.Tensor, bits: int, dim: int):
    n = scales.numel()
    out = torch.empty((n, dim), dtype=torch.float32, device=packed.device)
    check(lib.tq_dequantize_rotated_batch(_ptr(packed), _ptr(scales), _ptr(out), n, bits, dim, _stream()))
    return out


def qjl_quantize_batch(x: torch.Tensor, total_bits: int, rotation_seed: int, qjl_seed: int):
    """quantize_with_qjl over the rows of x [N, dim] f32.  Returns (polar packed
    u8 [N, dim*(total_bits-1)/8], polar scales int16 [N], signs u8 [N, dim/8],
    residual norms int16 [N]); f16 values as raw bits."""
    if x.dim() != 2 or x.dtype != torch.float32:
        raise ValueError("x must be f32 [N, dim]")
    n, d = x.shape
    dev = x.device
    polar = torch.empty((n, d * (total_bits - 1) // 8), dtype=torch.uint8, device=dev)
    scales = torch.empty((n,), dtype=torch.int16, device=dev)
    signs = torch.empty((n, d // 8), dtype=torch.uint8, device=dev)
    norms = torch.empty((n,), dtype=torch.int16, device=dev)
    check(lib.tq_qjl_quantize_batch(_ptr(x), _ptr(polar), _ptr(scales), _ptr(signs), _ptr(norms), n, total_bits, d,
                                    rotation_seed, qjl_seed, _stream()))
    return polar, scales, signs, norms


def qjl_query_context(queries: torch.Tensor, rotation_seed: int, qjl_seed: int) -> torch.Tensor:
    """[nq, 2*dim] f32: forward-rotated query, then its Rademacher projections."""
    nq, d = queries.shape
    ctx = torch.empty((nq, 2 * d), dtype=torch.float32, device=queries.device)
    check(lib.tq_qjl_query_context(_ptr(queries), _ptr(ctx), nq, d, rotation_seed, qjl_seed, _stream()))
    return ctx


def qjl_scores(ctx: torch.Tensor, polar, scales, signs, norms, polar_bits: int, rotation_seed: int) -> torch.Tensor:
    nq, d2 = ctx.shape
    nk = scales.numel()
    out = torch.empty((nq, nk), dtype=torch.float32, device=ctx.device)
    check(lib.tq_qjl_scores(_ptr(ctx), nq, _ptr(polar), _ptr(scales), _ptr(signs), _ptr(norms), nk, polar_bits,
                            d2 // 2, rotation_seed, _ptr(out), _stream()))
    return out


def softmax_rows(scores: torch.Tensor, scale: float) -> torch.Tensor:
    rows, cols = scores.shape
    out = torch.empty_like(scores)
    check(lib.tq_softmax_rows(_ptr(scores), _ptr(out), rows, cols, float(scale), _stream()))
    return out


def qjl_weighted_values(polar, scales, weights: torch.Tensor, polar_bits: int, dim: int, rotation_seed: int):
    nq, nv = weights.shape
    out = torch.empty((nq, dim), dtype=torch.float32, device=weights.device)
    nbytes = lib.tq_qjl_weighted_values_workspace_size(nq, nv, dim)
    ws = torch.empty((max(nbytes, 1),), dtype=torch.uint8, device=weights.device)
    check(lib.tq_qjl_weighted_values(_ptr(polar), _ptr(scales), nv, _ptr(weights), nq, polar_bits, dim, rotation_seed,
                                     _ptr(out), _ptr(ws), nbytes, _stream()))
    return out


def default_softmax_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)
