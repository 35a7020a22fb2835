"""Seeded synthetic inputs with the distributions of the benchmark workloads:
unsigned 4-bit codes uniform in 0..15 packed two per byte (even column in the
low nibble), fp16-representable scales ~|N(0, 0.02)|, zero 8, fp16 activations
~N(0, 1)."""
import numpy as np

from oracle_bind import Quantized


def w4_matrix(rows, cols, seed, group=64, zero=8.0, scale_std=0.02, affine=0):
    rng = np.random.default_rng(seed)
    assert cols % 2 == 0
    packed = rng.integers(0, 256, size=rows * cols // 2, dtype=np.uint8)
    g = (cols + group - 1) // group
    scales = np.abs(rng.normal(0.0, scale_std, rows * g)).astype(np.float16).astype(np.float32)
    if affine:
        zeros = rng.normal(0.0, 0.1, rows * g).astype(np.float16).astype(np.float32)
    else:
        zeros = np.full(rows * g, zero, np.float32)
    return Quantized(packed, scales, zeros, rows, cols, group, affine)


def f16_vector(n, seed, std=1.0):
    rng = np.random.default_rng(seed)
    return rng.normal(0.0, std, n).astype(np.float16)


def unpack_codes(q):
    """All codes of a reference-layout matrix as [rows, cols] uint8 (even column = low nibble)."""
    rb = (q.cols + 1) // 2
    b = q.packed[: q.rows * rb].reshape(q.rows, rb)
    codes = np.empty((q.rows, rb * 2), np.uint8)
    codes[:, 0::2] = b & 0x0F
    codes[:, 1::2] = b >> 4
    return codes[:, : q.cols]


def dense_f64(q):
    """Dequantized weights in float64 (for error-bound checks)."""
    codes = unpack_codes(q).astype(np.float64)
    g = (q.cols + q.group - 1) // q.group
    s = np.repeat(q.scales.reshape(q.rows, g).astype(np.float64), q.group, axis=1)[:, : q.cols]
    z = np.repeat(q.zeros.reshape(q.rows, g).astype(np.float64), q.group, axis=1)[:, : q.cols]
    return codes * s + z if q.affine else (codes - z) * s
