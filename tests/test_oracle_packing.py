"""Pins of the oracle's index packing (reference src/packed/mod.rs:242-309,
src/packed/indices.rs:152-281).

The layout is a little-endian LSB-first bitstream: index i occupies bits
[i*b, i*b + b) of the packed byte string, with the tail zero-padded to a whole
group (4 indices for 2-bit, 8 for 3-bit, 2 for 4-bit).  The expected bytes
are built here from that definition with Python integers, independently of
the oracle's shift-and-mask code, plus the reference's own round-trip and
size cases (roundtrip_tests.rs:305-400, packed/mod.rs:483-567).
"""
import numpy as np
import pytest

from oracle import oracle as orc

GROUP = {2: 4, 3: 8, 4: 2}


def bitstream(bits, idx):
    n = len(idx)
    padded = -(-n // GROUP[bits]) * GROUP[bits]
    v = 0
    for i, x in enumerate(idx):
        v |= int(x) << (i * bits)
    return np.frombuffer(v.to_bytes(padded * bits // 8, "little"), np.uint8)


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("count", [1, 2, 3, 7, 8, 9, 13, 31, 32, 33, 128, 256])
def test_pack_is_lsb_first_bitstream(bits, count):
    rng = np.random.default_rng(bits * 1000 + count)
    idx = rng.integers(0, 1 << bits, size=count).astype(np.uint8)
    got = orc.pack_indices(bits, idx)
    assert np.array_equal(got, bitstream(bits, idx))
    assert orc.packed_len(bits, count) == len(got)
    assert np.array_equal(orc.unpack_indices(bits, got, count), idx)


def test_3bit_group_known_answer():
    # values 0..7 -> 24-bit word sum(v_i << 3i) = 0b111110101100011010001000 -> bytes 88 C6 FA
    got = orc.pack_indices(3, np.arange(8, dtype=np.uint8))
    assert list(got) == [0x88, 0xC6, 0xFA]


def test_4bit_low_nibble_first():
    assert list(orc.pack_indices(4, np.array([3, 12], np.uint8))) == [0xC3]


def test_2bit_known_answer():
    assert list(orc.pack_indices(2, np.array([1, 2, 3, 0, 3], np.uint8))) == [0x39, 0x03]


def test_reference_roundtrip_cases():
    # roundtrip_tests.rs:305-345: every (a, b) in the first two 3-bit slots
    for a in range(8):
        for b in range(8):
            v = np.array([a, b, 0, 7, 3, 5, 1, 6], np.uint8)
            assert np.array_equal(orc.unpack_indices(3, orc.pack_indices(3, v), 8), v)
    for a in range(16):
        for b in range(16):
            v = np.array([a, b], np.uint8)
            assert np.array_equal(orc.unpack_indices(4, orc.pack_indices(4, v), 2), v)


@pytest.mark.parametrize("bits,dim,size", [(3, 32, 12), (3, 128, 48), (4, 32, 16), (4, 128, 64), (2, 128, 32)])
def test_packed_block_sizes(bits, dim, size):
    # roundtrip_tests.rs:347-389 (size_bytes = 2 + packed)
    assert orc.packed_len(bits, dim) == size
