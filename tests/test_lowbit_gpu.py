"""GPU parity of the W3A16 / W2A16 GEMV (xqhip_wlb_upload + xqhip_gemv_w4a16 /
_argmax) against the oracle's gemvLowBitReference restatement (orc_gemv_lowbit;
gemvW3A16Neon / gemvW2A16Neon call exactly that, arm64_neon/xq_gemv_w{3,2}a16_neon.cpp:6-8).

Random bitstreams with fp16-exact scales, both layouts (TILED64 bit planes for
group 64, the GENERIC bitstream kernel otherwise), the fused RMS prologue, the
residual-add and SiLU-pair epilogues and the argmax.
Tolerance: |gpu - oracle| <= 1e-2 + 1e-3 * |oracle|; greedy ids bit-exact where
the oracle's top-2 margin exceeds 1e-2.
"""
import ctypes

import numpy as np
import pytest

import oracle_bind as ob
import xqbind as xb
from test_gemv_gpu import assert_close, top2_margin

pytestmark = pytest.mark.gpu


def lowbit_matrix(rows, cols, bits, seed, group=64, affine=0):
    rng = np.random.default_rng(seed)
    g = (cols + group - 1) // group
    packed = rng.integers(0, 256, (rows * cols * bits + 7) // 8, dtype=np.uint8)
    scales = np.abs(rng.normal(0.0, 0.05, rows * g)).astype(np.float16).astype(np.float32)
    if affine:
        zeros = rng.normal(0.0, 0.1, rows * g).astype(np.float16).astype(np.float32)
    else:
        zeros = rng.integers(0, 1 << bits, rows * g).astype(np.float32)
    return ob.Quantized(packed, scales, zeros, rows, cols, group, affine)


def upload(q, bits):
    return xb.DeviceW4(q.packed, q.scales, q.zeros, q.rows, q.cols, q.group, q.affine, bits=bits)


def run(q, bits, x, epi=xb.EPI_STORE, norm_w=None, y_init=None):
    w = upload(q, bits)
    xd = xb.DeviceBuffer.from_array(x.astype(np.float32))
    nd = xb.DeviceBuffer.from_array(norm_w.astype(np.float32)) if norm_w is not None else None
    n = q.rows // 2 if epi == xb.EPI_SILU_PAIR else q.rows
    yd = xb.DeviceBuffer(n * 4)
    if y_init is not None:
        yd.upload(y_init.astype(np.float32))
    pro = xb.prologue(xb.PRO_RMS, nd, eps=1e-6) if nd else None
    xb.ck(xb.hip().xqhip_gemv_w4a16(w.ref, xd.ptr, xb.F32, ctypes.byref(pro) if pro else None, yd.ptr, xb.F32, epi,
                                    None))
    xb.ck(xb.hip().xqhip_device_synchronize())
    return yd.download(np.float32, n), w


@pytest.mark.parametrize("bits", [3, 2])
@pytest.mark.parametrize("rows,cols,seed", [(4096, 4096, 0), (12288, 4096, 1), (4096, 12288, 2), (1000, 1024, 3),
                                            (130, 4160, 4), (8, 64, 5), (3, 16384, 6)])
def test_tiled_lowbit_matches_oracle(bits, rows, cols, seed):
    q = lowbit_matrix(rows, cols, bits, seed)
    x = np.random.default_rng(seed + 50).normal(0, 1, cols).astype(np.float32)
    got, w = run(q, bits, x)
    assert (w.w.layout, w.w.bits, w.w.inexact_meta) == (xb.LAYOUT_TILED64, bits, 0)
    assert w.weight_bytes() == rows * cols * bits // 8 + rows * (cols // 64) * 4
    assert_close(got, ob.gemv_lowbit(q, bits, x), f"w{bits} {rows}x{cols}")


@pytest.mark.parametrize("bits", [3, 2])
def test_tiled_lowbit_affine_rms_add_silu(bits):
    rows, cols = 2048, 4096
    rng = np.random.default_rng(bits + 10)
    q = lowbit_matrix(rows, cols, bits, 20 + bits, affine=1)
    h = rng.normal(0, 1, cols).astype(np.float32)
    nw = rng.normal(1.0, 0.1, cols).astype(np.float32)
    normed = np.empty(cols, np.float32)
    ob.oracle().orc_rmsnorm(ob.p(h), ob.p(nw), cols, 1e-6, ob.p(normed))
    want = ob.gemv_lowbit(q, bits, normed)
    got, _ = run(q, bits, h, norm_w=nw)
    assert_close(got, want, "rms prologue, affine")
    resid = rng.normal(0, 1, rows).astype(np.float32)
    got, _ = run(q, bits, normed, epi=xb.EPI_ADD, y_init=resid)
    assert_close(got, resid + want, "residual add")
    got, _ = run(q, bits, normed, epi=xb.EPI_SILU_PAIR)
    silu = np.array([ob.oracle().orc_silu(float(a)) for a in want[0::2]], np.float32)
    assert_close(got, silu * want[1::2], "silu pair")


@pytest.mark.parametrize("bits", [3, 2])
@pytest.mark.parametrize("rows,cols,group,affine", [(7, 24, 8, 0), (33, 100, 10, 1), (64, 4096, 128, 0),
                                                    (5, 130, 64, 1)])
def test_generic_lowbit_matches_oracle(bits, rows, cols, group, affine):
    q = lowbit_matrix(rows, cols, bits, rows + cols, group=group, affine=affine)
    x = np.random.default_rng(7).normal(0, 1, cols).astype(np.float32)
    got, w = run(q, bits, x)
    assert w.w.layout == xb.LAYOUT_GENERIC and w.w.bits == bits
    # fp32 activations and metadata: only the summation order differs from the oracle
    np.testing.assert_allclose(got, ob.gemv_lowbit(q, bits, x), rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("bits", [3, 2])
def test_lowbit_argmax(bits):
    rows, cols = 50000, 4096
    q = lowbit_matrix(rows, cols, bits, 30 + bits)
    x = np.random.default_rng(31).normal(0, 1, cols).astype(np.float32)
    logits = ob.gemv_lowbit(q, bits, x)
    w = upload(q, bits)
    xd = xb.DeviceBuffer.from_array(x)
    ws = xb.DeviceBuffer(xb.hip().xqhip_argmax_workspace_bytes(rows))
    idx, val = xb.DeviceBuffer(4), xb.DeviceBuffer(4)
    xb.ck(xb.hip().xqhip_gemv_w4a16_argmax(w.ref, xd.ptr, xb.F32, None, ws.ptr, idx.ptr, val.ptr, None))
    xb.ck(xb.hip().xqhip_device_synchronize())
    got_idx, got_val = int(idx.download(np.int32, 1)[0]), float(val.download(np.float32, 1)[0])
    want_idx = int(np.argmax(logits))
    assert abs(got_val - logits[want_idx]) <= 1e-2 + 1e-3 * abs(logits[want_idx])
    if top2_margin(logits) > 1e-2:
        assert got_idx == want_idx


def test_lowbit_rejected_by_prefill_gemm_and_bad_widths():
    q = lowbit_matrix(64, 256, 3, 40)
    w = upload(q, 3)
    x = xb.DeviceBuffer(4 * 256 * 4)
    y = xb.DeviceBuffer(4 * 64 * 4)
    ws = xb.DeviceBuffer(xb.hip().xqhip_gemm_workspace_bytes(4, 256, 64))
    rc = xb.hip().xqhip_gemm_w4a16(w.ref, x.ptr, 4, 256, None, 0, y.ptr, 64, xb.EPI_STORE, ws.ptr, ws.nbytes, None)
    assert rc != 0 and b"4-bit" in xb.hip().xqhip_last_error()
    bad = xb.W4()
    rc = xb.hip().xqhip_wlb_upload(ob.p(q.packed), ob.p(q.scales), ob.p(q.zeros), 64, 256, 64, 5, 0,
                                   ctypes.byref(bad))
    assert rc != 0
