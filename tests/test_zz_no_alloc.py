"""The no-allocation greedy lm_head entry point (xqhip_gemv_w4a16_argmax_static)
against the workspace entry point it shares its kernels with
(xqhip_gemv_w4a16_argmax): identical token index and value, bit for bit, on
two calls in a row, the second with a smaller matrix, both through the C ABI
of libxqhip.so; and the index against the oracle's gemvW4A16ArgmaxNeon
restatement wherever the top-2 logit margin exceeds 1e-2."""
import ctypes

import numpy as np
import pytest

import oracle_bind as ob
import xqbind as xb
from synth import w4_matrix

pytestmark = pytest.mark.gpu


def argmax_both(q, h, nw):
    hip = xb.hip()
    w = xb.DeviceW4(q.packed, q.scales, q.zeros, q.rows, q.cols)
    hd, nd = xb.DeviceBuffer.from_array(h), xb.DeviceBuffer.from_array(nw)
    pro = xb.prologue(xb.PRO_RMS, nd, eps=1e-6)
    ws = xb.DeviceBuffer(hip.xqhip_argmax_workspace_bytes(q.rows))
    idx_a, val_a, idx_b, val_b = (xb.DeviceBuffer(4) for _ in range(4))
    xb.ck(hip.xqhip_gemv_w4a16_argmax(w.ref, hd.ptr, xb.F32, ctypes.byref(pro), ws.ptr, idx_a.ptr, val_a.ptr, None))
    xb.ck(hip.xqhip_gemv_w4a16_argmax_static(w.ref, hd.ptr, xb.F32, ctypes.byref(pro), idx_b.ptr, val_b.ptr, None))
    xb.ck(hip.xqhip_device_synchronize())
    return ((int(idx_a.download(np.int32, 1)[0]), idx_b.download(np.int32, 1)[0].item()),
            (val_a.download(np.uint32, 1)[0].item(), val_b.download(np.uint32, 1)[0].item()))


def test_static_argmax_matches_workspace_argmax_twice():
    xb.ck(xb.hip().xqhip_set_device(0))
    for rows, cols, seed in ((248320, 4096, 501), (3001, 1024, 502)):  # the second call is smaller
        q = w4_matrix(rows, cols, seed)
        rng = np.random.default_rng(seed + 1)
        h = rng.normal(0, 1, cols).astype(np.float32)
        nw = rng.normal(1.0, 0.1, cols).astype(np.float32)
        (ia, ib), (va, vb) = argmax_both(q, h, nw)
        assert ia == ib and va == vb, (rows, ia, ib, hex(va), hex(vb))
        normed = np.empty(cols, np.float32)
        ob.oracle().orc_rmsnorm(ob.p(h), ob.p(nw), cols, 1e-6, ob.p(normed))
        want_idx, want_val = ob.gemv_argmax(q, normed)
        got_val = float(np.array([vb], np.uint32).view(np.float32)[0])
        assert abs(got_val - want_val) <= 1e-2 + 1e-3 * abs(want_val)
        logits = np.sort(ob.gemv(q, normed).astype(np.float64))
        if logits[-1] - logits[-2] > 1e-2:
            assert ib == want_idx
