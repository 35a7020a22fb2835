"""The W3A16 / W2A16 formats on the CPU: the oracle's low-bit GEMV
(orc_gemv_lowbit, restating gemvLowBitReference, ref_gemv.cpp:98-106, which is
what gemvW3A16Neon / gemvW2A16Neon call) and the bitstream layout it reads.

Pins:
* hand-packed bitstreams (LSB first, codes crossing byte boundaries, rows not
  padded to bytes) read back code by code through one-hot activations;
* the 4-bit bitstream is the nibble layout, so at bits 4 the low-bit GEMV must
  agree with the textbook W4 form on the same bytes;
* with the compiled reference present: orc_gemv_lowbit is bit-identical to the
  reference's own gemvW3A16Neon / gemvW2A16Neon, and the oracle quantiser's
  3- and 2-bit bitstreams are byte-identical to quantizeLowBit's.
"""
import numpy as np
import pytest

import oracle_bind as ob

needs_ref = pytest.mark.skipif(not ob.ref_available(), reason="compiled reference not built (oracle/_ref)")


def pack_bits(codes, bits):
    """Independent packer: integer sum of code_i << (bits * i), little-endian bytes."""
    v = 0
    for i, c in enumerate(np.asarray(codes).reshape(-1)):
        v |= int(c) << (bits * i)
    n = (len(np.asarray(codes).reshape(-1)) * bits + 7) // 8
    return np.frombuffer(v.to_bytes(n, "little"), np.uint8).copy()


def read_back(packed, rows, cols, bits, group=8):
    g = (cols + group - 1) // group
    q = ob.Quantized(packed, np.ones(rows * g, np.float32), np.zeros(rows * g, np.float32), rows, cols, group)
    out = np.empty((rows, cols), np.float32)
    for c in range(cols):
        x = np.zeros(cols, np.float32)
        x[c] = 1.0
        out[:, c] = ob.gemv_lowbit(q, bits, x)
    return out


def test_three_bit_known_answer():
    codes = [5, 3, 7, 1, 0, 6, 2, 4]
    packed = np.array([0xDD, 0x03, 0x8B], np.uint8)  # 0x8B03DD = sum code_i << 3i, worked by hand
    assert np.array_equal(pack_bits(codes, 3), packed)
    assert read_back(packed, 1, 8, 3).reshape(-1).tolist() == codes


def test_two_bit_known_answer():
    codes = [1, 2, 3, 0, 3, 3, 1, 2]
    packed = np.array([0x39, 0x9F], np.uint8)  # 0x9F39
    assert np.array_equal(pack_bits(codes, 2), packed)
    assert read_back(packed, 1, 8, 2).reshape(-1).tolist() == codes


@pytest.mark.parametrize("bits", [2, 3])
def test_rows_are_not_byte_padded(bits):
    rng = np.random.default_rng(bits)
    codes = rng.integers(0, 1 << bits, (3, 5))  # 5 * bits bits per row: rows start mid-byte
    got = read_back(pack_bits(codes, bits), 3, 5, bits)
    assert np.array_equal(got, codes.astype(np.float32))


def test_four_bit_bitstream_is_the_nibble_layout():
    rng = np.random.default_rng(4)
    rows, cols = 9, 128
    codes = rng.integers(0, 16, (rows, cols))
    packed = pack_bits(codes, 4)
    assert np.array_equal(packed & 15, codes[:, 0::2].reshape(-1)) and np.array_equal(packed >> 4, codes[:, 1::2].reshape(-1))
    g = cols // 64
    q = ob.Quantized(packed, rng.uniform(0.01, 0.03, rows * g), rng.integers(0, 16, rows * g), rows, cols)
    x = rng.normal(0, 1, cols).astype(np.float32)
    want = ob.gemv(q, x, fn="orc_gemv_textbook")
    assert np.array_equal(ob.gemv_lowbit(q, 4, x), want)


@needs_ref
@pytest.mark.parametrize("bits", [2, 3])
@pytest.mark.parametrize("rows,cols,group,affine", [(7, 24, 8, 0), (33, 100, 10, 1), (64, 4096, 64, 0),
                                                    (5, 130, 64, 1), (16, 1024, 128, 0)])
def test_oracle_matches_reference_lowbit_kernels(bits, rows, cols, group, affine):
    rng = np.random.default_rng(rows * cols + bits)
    g = (cols + group - 1) // group
    packed = rng.integers(0, 256, (rows * cols * bits + 7) // 8, dtype=np.uint8)
    scales = rng.uniform(0.005, 0.05, rows * g).astype(np.float32)
    zeros = (rng.normal(0, 0.1, rows * g) if affine else rng.integers(0, 1 << bits, rows * g)).astype(np.float32)
    q = ob.Quantized(packed, scales, zeros, rows, cols, group, affine)
    x = rng.normal(0, 1, cols).astype(np.float32)
    want = ob.gemv_lowbit(q, bits, x, lib=ob.ref(), fn="ref_gemv_lowbit")
    assert np.array_equal(ob.gemv_lowbit(q, bits, x), want)


@needs_ref
@pytest.mark.parametrize("bits", [2, 3])
def test_quantiser_bitstreams_match_reference(bits):
    rows, cols = 12, 200
    w = (np.sin(np.arange(rows * cols, dtype=np.float32) * np.float32(0.37)) * np.float32(0.5)).astype(np.float32)
    a = ob.quantize_lowbit(w, rows, cols, bits, 64)
    b = ob.quantize_lowbit(w, rows, cols, bits, 64, lib=ob.ref(), fn="ref_quantize_lowbit")
    assert np.array_equal(a.packed, b.packed)
    assert np.array_equal(a.scales, b.scales) and np.array_equal(a.zeros, b.zeros)
    # the codes respect the width
    got = read_back(a.packed, rows, cols, bits, group=64)
    assert got.max() <= (1 << bits) - 1
