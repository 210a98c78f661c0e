"""Python mirror of the reference crate's public API (the Rust types of
src/packed, src/quantize.rs, src/qjl.rs and src/attention.rs), over the
batched gfx950 kernels.  Same names, argument meaning and error kinds
(TurboQuantError, error.rs:5-29); vectors are torch tensors on the device
(or anything torch.as_tensor accepts, moved there).  The per-vector calls
are conveniences over the batch kernels; batch work uses the batch forms.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np
import torch

from . import (dequantize_rotated_batch, dequantize_vec_batch, qjl_quantize_batch, qjl_query_context, qjl_scores,
               qjl_weighted_values, quantize_vec_batch)
from ._lib import TurboQuantError

INVALID_DIMENSION, UNSUPPORTED_BITS, DIMENSION_MISMATCH, LAYER_OUT_OF_RANGE, RANGE_OUT_OF_BOUNDS = 1, 2, 3, 4, 5


def _require(cond: bool, code: int, msg: str) -> None:
    if not cond:
        raise TurboQuantError(code, msg)


def _check_len(actual: int, expected: int) -> None:
    _require(actual == expected, DIMENSION_MISMATCH, f"expected vector of length {expected}, got {actual}")


def _dev(x) -> torch.Tensor:
    return torch.as_tensor(x, dtype=torch.float32).to("cuda").contiguous()


@dataclass(frozen=True)
class TurboQuantConfig:
    """packed/mod.rs:92-139: bits in {2, 3, 4}, dim a power of two."""
    bits: int
    dim: int
    rotation_seed: int = 0

    @staticmethod
    def new(bits: int, dim: int) -> "TurboQuantConfig":
        _require(bits in (2, 3, 4), UNSUPPORTED_BITS, f"unsupported bit width {bits}, expected 2, 3, or 4")
        _require(dim > 0 and dim & (dim - 1) == 0, INVALID_DIMENSION, f"dimension {dim} is not a power of two")
        return TurboQuantConfig(bits, dim, 0)

    def with_seed(self, seed: int) -> "TurboQuantConfig":
        return TurboQuantConfig(self.bits, self.dim, seed)


def packed_len(bits: int, count: int) -> int:
    """Byte length of the reference packers' output (zero-padded tails)."""
    return {2: (count + 3) // 4, 3: (count + 7) // 8 * 3, 4: (count + 1) // 2}[bits]


@dataclass
class PackedBlock:
    """packed/mod.rs:149-233: f16 scale bits plus an LSB-first bitstream."""
    bits: int
    scale: int  # f16 bits
    packed_indices: bytes

    @staticmethod
    def new(bits: int, scale: int, indices: Sequence[int]) -> "PackedBlock":
        idx = np.asarray(indices, np.uint8) & ((1 << bits) - 1)
        bitarr = ((idx[:, None] >> np.arange(bits)) & 1).astype(np.uint8).reshape(-1)
        out = np.zeros(packed_len(bits, len(idx)) * 8, np.uint8)
        out[:bitarr.size] = bitarr
        return PackedBlock(bits, scale, np.packbits(out, bitorder="little").tobytes())

    @staticmethod
    def from_raw(bits: int, scale: int, packed: bytes) -> "PackedBlock":
        return PackedBlock(bits, scale, bytes(packed))

    def size_bytes(self) -> int:
        return 2 + len(self.packed_indices)

    def unpack(self, count: int) -> List[int]:
        bitarr = np.unpackbits(np.frombuffer(self.packed_indices, np.uint8), bitorder="little")
        bitarr = bitarr[:count * self.bits].reshape(count, self.bits)
        return (bitarr.astype(np.uint32) << np.arange(self.bits)).sum(1).astype(int).tolist()


def quantize_vec(config: TurboQuantConfig, data) -> PackedBlock:
    """quantize.rs:142-157."""
    x = _dev(data).reshape(-1)
    _check_len(x.numel(), config.dim)
    p, s = quantize_vec_batch(x[None], config.bits, config.rotation_seed)
    return PackedBlock(config.bits, int(s.cpu().numpy().view(np.uint16)[0]), p[0].cpu().numpy().tobytes())


def _block_tensors(blocks: Sequence[PackedBlock]):
    p = torch.from_numpy(np.frombuffer(b"".join(b.packed_indices for b in blocks), np.uint8).copy()).cuda()
    s = torch.from_numpy(np.array([b.scale for b in blocks], np.uint16).view(np.int16)).cuda()
    return p.reshape(len(blocks), -1), s


def dequantize_vec(config: TurboQuantConfig, block: PackedBlock) -> torch.Tensor:
    """quantize.rs:207-240."""
    p, s = _block_tensors([block])
    return dequantize_vec_batch(p, s, block.bits, config.dim, config.rotation_seed)[0]


def dequantize_rotated(config: TurboQuantConfig, block: PackedBlock) -> torch.Tensor:
    """quantize.rs:306-316."""
    p, s = _block_tensors([block])
    return dequantize_rotated_batch(p, s, block.bits, config.dim)[0]


@dataclass
class QjlBlock:
    """qjl.rs:111-134: (bits-1)-bit polar block, packed signs, f16 residual norm."""
    polar_block: PackedBlock
    qjl_signs: bytes
    residual_norm: int  # f16 bits

    @staticmethod
    def from_parts(polar_block: PackedBlock, qjl_signs: bytes, residual_norm: int) -> "QjlBlock":
        return QjlBlock(polar_block, bytes(qjl_signs), residual_norm)

    def size_bytes(self) -> int:
        return self.polar_block.size_bytes() + len(self.qjl_signs) + 2


def _validate_qjl(bits: int) -> None:
    _require(bits in (3, 4), UNSUPPORTED_BITS, f"unsupported bit width {bits}, expected 2, 3, or 4")


def quantize_with_qjl(config: TurboQuantConfig, data, qjl_seed: int) -> QjlBlock:
    """qjl.rs:355-377."""
    _validate_qjl(config.bits)
    x = _dev(data).reshape(-1)
    _check_len(x.numel(), config.dim)
    p, s, g, n = qjl_quantize_batch(x[None], config.bits, config.rotation_seed, qjl_seed)
    pb = PackedBlock(config.bits - 1, int(s.cpu().numpy().view(np.uint16)[0]), p[0].cpu().numpy().tobytes())
    return QjlBlock(pb, g[0].cpu().numpy().tobytes(), int(n.cpu().numpy().view(np.uint16)[0]))


def precompute_query_projections(query, dim: int, qjl_seed: int) -> torch.Tensor:
    """qjl.rs:488-492: R q."""
    q = _dev(query).reshape(1, -1)
    _check_len(q.shape[1], dim)
    return qjl_query_context(q, 0, qjl_seed)[0, dim:]


class EstimationContext:
    """qjl.rs:561-572: what is fetched once per query -- its rotated form and R q."""

    def __init__(self, config: TurboQuantConfig, query, qjl_seed: int):
        _validate_qjl(config.bits)
        q = _dev(query).reshape(1, -1)
        _check_len(q.shape[1], config.dim)
        self.polar_config = TurboQuantConfig.new(config.bits - 1, config.dim).with_seed(config.rotation_seed)
        self.dim = config.dim
        self.ctx = qjl_query_context(q, config.rotation_seed, qjl_seed)

    def estimate(self, keys: Sequence[QjlBlock]) -> torch.Tensor:
        """estimate_inner_product_with_codebook (qjl.rs:585-606) for each key."""
        p, s = _block_tensors([k.polar_block for k in keys])
        g = torch.from_numpy(np.frombuffer(b"".join(k.qjl_signs for k in keys), np.uint8).copy()).cuda()
        n = torch.from_numpy(np.array([k.residual_norm for k in keys], np.uint16).view(np.int16)).cuda()
        return qjl_scores(self.ctx, p, s, g.reshape(len(keys), -1), n, self.polar_config.bits,
                          self.polar_config.rotation_seed)[0]


def estimate_inner_product_single(query, block: QjlBlock, config: TurboQuantConfig, qjl_seed: int) -> float:
    """qjl.rs:619-627."""
    return float(EstimationContext(config, query, qjl_seed).estimate([block])[0])


class QuantizedKVCache:
    """attention.rs:45-700: QJL-quantized keys and values per layer, kept on the
    device as flat tensors (polar codes, scales, signs, residual norms)."""

    def __init__(self, config: TurboQuantConfig, num_layers: int, qjl_seed: int):
        self.config, self.qjl_seed = config, qjl_seed
        self._k = [None] * num_layers
        self._v = [None] * num_layers

    def num_layers(self) -> int:
        return len(self._k)

    def _check_layer(self, layer: int) -> None:
        _require(0 <= layer < self.num_layers(), LAYER_OUT_OF_RANGE,
                 f"layer index {layer} out of range (num_layers = {self.num_layers()})")

    def entry_count(self, layer: int) -> int:
        return 0 if self._k[layer] is None else self._k[layer][0].shape[0]

    def push(self, layer: int, key, value) -> None:
        self.push_batch(layer, [key], [value])

    def push_batch(self, layer: int, keys, values) -> None:
        """attention.rs:274-301."""
        self._check_layer(layer)
        _check_len(len(keys), len(values))
        kx = torch.stack([_dev(k).reshape(-1) for k in keys]) if len(keys) else None
        vx = torch.stack([_dev(v).reshape(-1) for v in values]) if len(values) else None
        if kx is None:
            return
        _check_len(kx.shape[1], self.config.dim)
        _check_len(vx.shape[1], self.config.dim)
        _validate_qjl(self.config.bits)
        for store, x in ((self._k, kx), (self._v, vx)):
            new = qjl_quantize_batch(x, self.config.bits, self.config.rotation_seed, self.qjl_seed)
            store[layer] = new if store[layer] is None else tuple(torch.cat([a, b]) for a, b in zip(store[layer], new))

    def attention_scores(self, layer: int, query) -> torch.Tensor:
        """attention.rs:319-353."""
        self._check_layer(layer)
        if self._k[layer] is None:
            return torch.empty(0, device="cuda")
        ctx = EstimationContext(self.config, query, self.qjl_seed)
        p, s, g, n = self._k[layer]
        return qjl_scores(ctx.ctx, p, s, g, n, self.config.bits - 1, self.config.rotation_seed)[0]

    def weighted_values(self, layer: int, weights) -> torch.Tensor:
        """attention.rs:371-408."""
        self._check_layer(layer)
        w = _dev(weights).reshape(1, -1)
        _check_len(w.shape[1], self.entry_count(layer))
        if self._v[layer] is None:
            return torch.zeros(self.config.dim, device="cuda")
        p, s, _, _ = self._v[layer]
        return qjl_weighted_values(p, s, w, self.config.bits - 1, self.config.dim, self.config.rotation_seed)[0]

    def memory_usage(self) -> int:
        """attention.rs:414-430: every block's bytes."""
        per = 2 + self.config.dim * (self.config.bits - 1) // 8 + self.config.dim // 8 + 2
        return sum(2 * self.entry_count(layer) * per for layer in range(self.num_layers()))

    def fp16_equivalent_memory(self) -> int:
        return sum(self.entry_count(layer) for layer in range(self.num_layers())) * self.config.dim * 2 * 2

    def key_block(self, layer: int, index: int) -> Optional[QjlBlock]:
        if not (0 <= layer < self.num_layers()) or not (0 <= index < self.entry_count(layer)):
            return None
        p, s, g, n = (t[index].cpu().numpy() for t in self._k[layer])
        return QjlBlock(PackedBlock(self.config.bits - 1, int(s.view(np.uint16)), p.tobytes()), g.tobytes(),
                        int(n.view(np.uint16)))

    def _dequant(self, store, layer: int, start: int, end: int) -> torch.Tensor:
        self._check_layer(layer)
        count = self.entry_count(layer)
        _require(0 <= start <= end <= count, RANGE_OUT_OF_BOUNDS,
                 f"range [{start}..{end}) out of bounds for entry_count = {count}")
        if end == start:
            return torch.empty((0, self.config.dim), device="cuda")
        p, s, _, _ = store[layer]
        return dequantize_vec_batch(p[start:end].contiguous(), s[start:end].contiguous(), self.config.bits - 1,
                                    self.config.dim, self.config.rotation_seed)

    def dequantize_all_keys(self, layer: int) -> torch.Tensor:
        return self._dequant(self._k, layer, 0, self.entry_count(layer) if 0 <= layer < self.num_layers() else 0)

    def dequantize_all_values(self, layer: int) -> torch.Tensor:
        return self._dequant(self._v, layer, 0, self.entry_count(layer) if 0 <= layer < self.num_layers() else 0)

    def dequantize_keys_range(self, layer: int, start: int, end: int) -> torch.Tensor:
        return self._dequant(self._k, layer, start, end)

    def dequantize_values_range(self, layer: int, start: int, end: int) -> torch.Tensor:
        return self._dequant(self._v, layer, start, end)
