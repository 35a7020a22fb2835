"""GPU parity for matrices whose group scales or zeros fp16 cannot hold, and
for prefill activations beyond the fp16 range.

The reference keeps every scale and zero in fp32 (QuantizedMatrix,
customlib/kernels/kernels.hpp:18-19); its default asymmetric packer writes
scale = (max - min) / 15 (pack_qwen35_xq4_numpy.py:218-247), which fp16 rounds
by up to 2^-11 and flushes below 6e-5.  Such matrices upload in the
TILED64_F32META layout and the GEMV and the prefill GEMM use the fp32 values.
Checked against the oracle's gemvW4A16Neon restatement with the tolerance of
the other GEMV tests (1e-2 abs + 1e-3 rel) on scales that fp16 would round
badly (a 1e-3 relative scale error of the fp16 path would fail it, see the
control below).

Prefill activations: silu(gate) * up of a large residual stream reaches 1e5,
past fp16's 65504; the GEMM's x preparation scales each token row by a power
of two, so the down projection of such rows still matches the oracle.
"""
import ctypes

import numpy as np
import pytest

import oracle_bind as ob
import xqbind as xb
from test_decode_ops_gpu import close, dev
from test_prefill_gpu import oracle_rows, run_gemm

pytestmark = pytest.mark.gpu


def fp32_meta_matrix(rows, cols, seed, affine=0, tiny=False):
    """Scales that are not fp16 values (|N(0, 0.02)| in fp32, optionally down at
    1e-6 where fp16 flushes), zeros from the asymmetric quantiser's range."""
    rng = np.random.default_rng(seed)
    packed = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
    g = rows * (cols // 64)
    scales = np.abs(rng.normal(0.0, 0.02, g)).astype(np.float32) + np.float32(1e-4)
    if tiny:
        scales[::3] = np.float32(1e-6) * (1 + rng.random(scales[::3].size, np.float32))
    zeros = (rng.normal(0.0, 0.05, g) if affine else rng.uniform(0.0, 15.0, g)).astype(np.float32)
    return ob.Quantized(packed, scales, zeros, rows, cols, 64, affine)


def run_gemv(q, x, epi=xb.EPI_STORE):
    w = xb.DeviceW4(q.packed, q.scales, q.zeros, q.rows, q.cols, q.group, q.affine)
    xd = xb.DeviceBuffer.from_array(x)
    n = q.rows // 2 if epi == xb.EPI_SILU_PAIR else q.rows
    yd = xb.DeviceBuffer(n * 4)
    xb.ck(xb.hip().xqhip_gemv_w4a16(w.ref, xd.ptr, xb.F32, None, yd.ptr, xb.F32, epi, None))
    xb.ck(xb.hip().xqhip_device_synchronize())
    return yd.download(np.float32, n), w


@pytest.mark.parametrize("rows,cols,affine,tiny", [(4096, 4096, 0, False), (1000, 12288, 0, True),
                                                   (2048, 4096, 1, False), (300, 8256, 0, False)])
def test_gemv_fp32_metadata_matches_oracle(rows, cols, affine, tiny):
    q = fp32_meta_matrix(rows, cols, rows + cols + affine, affine, tiny)
    x = np.random.default_rng(7).normal(0, 1, cols).astype(np.float32)
    want = ob.gemv(q, x)
    got, w = run_gemv(q, x)
    assert w.w.layout == xb.LAYOUT_TILED64_F32META and w.w.inexact_meta > 0
    assert w.weight_bytes() == rows * cols // 2 + rows * (cols // 64) * 8
    close(got, want, f"fp32-metadata gemv {rows}x{cols} affine={affine}")
    # control: the same matrix with its metadata rounded to fp16 misses the oracle
    # by far more than the tolerance, so the check above pins the fp32 path
    q16 = ob.Quantized(q.packed, q.scales.astype(np.float16).astype(np.float32),
                       q.zeros.astype(np.float16).astype(np.float32), rows, cols, 64, affine)
    err16 = np.abs(ob.gemv(q16, x).astype(np.float64) - want)
    err32 = np.abs(got.astype(np.float64) - want)
    assert err16.max() > 4 * err32.max()


def test_gemv_fp32_metadata_argmax_and_lowbit():
    rows, cols = 30000, 4096
    q = fp32_meta_matrix(rows, cols, 31)
    x = np.random.default_rng(32).normal(0, 1, cols).astype(np.float32)
    want_idx, want_val = ob.gemv_argmax(q, x)
    w = xb.DeviceW4(q.packed, q.scales, q.zeros, rows, cols)
    xd = xb.DeviceBuffer.from_array(x)
    ws = xb.DeviceBuffer(xb.hip().xqhip_argmax_workspace_bytes(rows))
    idx, val = xb.DeviceBuffer(4), xb.DeviceBuffer(4)
    xb.ck(xb.hip().xqhip_gemv_w4a16_argmax(w.ref, xd.ptr, xb.F32, None, ws.ptr, idx.ptr, val.ptr, None))
    gv = float(val.download(np.float32, 1)[0])
    assert abs(gv - want_val) <= 1e-2 + 1e-3 * abs(want_val)
    logits = np.sort(ob.gemv(q, x).astype(np.float64))
    if logits[-1] - logits[-2] > 1e-2:
        assert int(idx.download(np.int32, 1)[0]) == want_idx
    # 3- and 2-bit matrices from the reference quantiser (fp32 scales (max - min) / levels)
    for bits in (3, 2):
        wv = np.sin(np.arange(512 * 4096, dtype=np.float32) * np.float32(0.013)) * np.float32(0.3)
        ql = ob.quantize_lowbit(wv, 512, 4096, bits, 64)
        dl = xb.DeviceW4(ql.packed, ql.scales, ql.zeros, 512, 4096, 64, 0, bits=bits)
        assert dl.w.layout == xb.LAYOUT_TILED64_F32META
        yd = xb.DeviceBuffer(512 * 4)
        xb.ck(xb.hip().xqhip_gemv_w4a16(dl.ref, xd.ptr, xb.F32, None, yd.ptr, xb.F32, xb.EPI_STORE, None))
        close(yd.download(np.float32, 512), ob.gemv_lowbit(ql, bits, x), f"W{bits} fp32-metadata gemv")


@pytest.mark.parametrize("epi", [xb.EPI_STORE, xb.EPI_ADD, xb.EPI_SILU_PAIR])
def test_gemm_fp32_metadata_matches_per_token_gemv(epi):
    rows, cols, m = 512, 4096, 40
    q = fp32_meta_matrix(rows, cols, 41 + epi)
    rng = np.random.default_rng(42)
    X = rng.normal(0, 1, (m, cols)).astype(np.float32)
    gamma = rng.normal(1, 0.1, cols).astype(np.float32)
    want = oracle_rows(q, X, "rms", gamma)
    if epi == xb.EPI_STORE:
        close(run_gemm(q, X, epi, "rms", gamma), want, "fp32-metadata gemm")
    elif epi == xb.EPI_ADD:
        y0 = rng.normal(0, 1, (m, rows)).astype(np.float32)
        close(run_gemm(q, X, epi, "rms", gamma, y0=y0), y0 + want, "fp32-metadata gemm add")
    else:
        g, u = want[:, 0::2].astype(np.float64), want[:, 1::2].astype(np.float64)
        close(run_gemm(q, X, epi, "rms", gamma), g / (1 + np.exp(-g)) * u, "fp32-metadata gemm silu")


@pytest.mark.parametrize("scale", [1e5, 3e-6])
def test_gemm_activations_outside_fp16_range(scale):
    """down_proj inputs around 1e5 (past fp16's maximum) and around 3e-6
    (fp16 subnormals), no prologue, against the per-token oracle GEMV."""
    rows, cols, m = 256, 12288, 24
    from synth import w4_matrix
    q = w4_matrix(rows, cols, 51)
    rng = np.random.default_rng(52)
    X = (rng.normal(0, 1, (m, cols)) * scale).astype(np.float32)
    X[3, 17] = np.float32(2.5e5 if scale > 1 else 1e-7)
    want = oracle_rows(q, X)
    got = run_gemm(q, X, xb.EPI_STORE)
    assert np.isfinite(got).all()
    tol = 1e-2 * scale  # the 1e-2 absolute bound of unit-scale inputs, scaled with them
    err = np.abs(got.astype(np.float64) - want)
    assert (err <= tol + 1e-3 * np.abs(want)).all(), err.max()
