"""GPU parity of the TILED64_F32S_Z4 layout: 4-bit format-v1 matrices whose
zeros are integers 0..15 and whose scales fp16 cannot hold, the metadata of
the reference packer's asymmetric quantiser (scale = (max - min) / 15 in fp32,
zero = round(-min / scale) clamped to 0..15, pack_qwen35_xq4_numpy.py:218-247;
w = (q - z) s, customlib/kernels/kernels.hpp:18-19).  Each group keeps the
fp32 scale and a 4-bit zero code (4.5 bytes instead of the 8 of the fp32 pair).

Checks:
* GEMV (store, add, SiLU pair, argmax) and prefill GEMM against the oracle's
  gemvW4A16Neon restatement, 1e-2 abs + 1e-3 rel, on shapes whose group count
  is not a multiple of 8 (partial zero words) and on scales fp16 would flush;
* the same values through the fp32-pair layout give bit-identical rows: the
  two layouts differ only in where the zero is read from, so a wrong nibble,
  word or row of the zero array shows as a mismatch (the fp32-pair upload is
  forced by one non-integer zero in row 0, which is left out of the compare);
* a control: the fp16-rounded scales miss the oracle by far more than the
  tolerance, so the check pins the fp32 scales;
* a small asymmetric synthetic model end to end against the oracle model.
"""
import ctypes

import numpy as np
import pytest

import oracle_bind as ob
import xqbind as xb
from test_decode_ops_gpu import close, dev
from test_prefill_gpu import oracle_rows, run_gemm

pytestmark = pytest.mark.gpu


def z4_matrix(rows, cols, seed, tiny=False):
    """Uniform codes, fp32 scales that fp16 does not hold, integer zeros 0..15."""
    rng = np.random.default_rng(seed)
    packed = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
    g = rows * (cols // 64)
    scales = np.abs(rng.normal(0.0, 0.02, g)).astype(np.float32) + np.float32(1e-4)
    if tiny:
        scales[::3] = np.float32(1e-6) * (1 + rng.random(scales[::3].size, np.float32))
    zeros = rng.integers(0, 16, g).astype(np.float32)
    return ob.Quantized(packed, scales, zeros, rows, cols, 64, 0)


def with_pair_layout(q):
    """The same matrix with zero (row 0, group 0) moved off the integers: the
    upload then keeps the fp32 pair for every group."""
    zeros = q.zeros.copy()
    zeros[0] += np.float32(0.5)
    return ob.Quantized(q.packed, q.scales, zeros, q.rows, q.cols, q.group, q.affine)


def gemv(w, x, epi, n, y0=None):
    xd = xb.DeviceBuffer.from_array(x)
    yd = xb.DeviceBuffer.from_array(y0) if y0 is not None else xb.DeviceBuffer(n * 4)
    xb.ck(xb.hip().xqhip_gemv_w4a16(w.ref, xd.ptr, xb.F32, None, yd.ptr, xb.F32, epi, None))
    xb.ck(xb.hip().xqhip_device_synchronize())
    return yd.download(np.float32, n)


def upload(q):
    return xb.DeviceW4(q.packed, q.scales, q.zeros, q.rows, q.cols, q.group, q.affine)


@pytest.mark.parametrize("rows,cols,tiny", [(4096, 4096, False), (1000, 12288, True), (300, 8256, False),
                                            (24576, 4096, False), (77, 640, False)])
def test_gemv_z4_matches_oracle_and_pair_layout(rows, cols, tiny):
    print(f"z4 gemv {rows}x{cols} tiny={tiny}", flush=True)
    q = z4_matrix(rows, cols, rows + cols, tiny)
    x = np.random.default_rng(9).normal(0, 1, cols).astype(np.float32)
    w = upload(q)
    G = cols // 64
    assert w.w.layout == xb.LAYOUT_TILED64_F32S_Z4 and w.w.inexact_meta > 0
    assert w.weight_bytes() == rows * cols // 2 + rows * G * 4 + rows * ((G + 7) // 8) * 4
    want = ob.gemv(q, x)
    got = gemv(w, x, xb.EPI_STORE, rows)
    close(got, want, f"z4 gemv {rows}x{cols}")
    # bit-identical to the fp32-pair layout on every row but row 0
    p = upload(with_pair_layout(q))
    assert p.w.layout == xb.LAYOUT_TILED64_F32META
    pair = gemv(p, x, xb.EPI_STORE, rows)
    assert np.array_equal(got[1:].view(np.uint32), pair[1:].view(np.uint32))
    # control: the metadata rounded to fp16 misses the oracle by far more
    q16 = ob.Quantized(q.packed, q.scales.astype(np.float16).astype(np.float32), q.zeros, rows, cols, 64, 0)
    err16 = np.abs(ob.gemv(q16, x).astype(np.float64) - want)
    assert err16.max() > 4 * np.abs(got.astype(np.float64) - want).max()
    w.free()
    p.free()


def test_gemv_z4_epilogues():
    rows, cols = 2048, 4096
    q = z4_matrix(rows, cols, 5)
    x = np.random.default_rng(6).normal(0, 1, cols).astype(np.float32)
    w, p = upload(q), upload(with_pair_layout(q))
    want = ob.gemv(q, x).astype(np.float64)
    y0 = np.random.default_rng(7).normal(0, 1, rows).astype(np.float32)
    got = gemv(w, x, xb.EPI_ADD, rows, y0)
    close(got, y0 + want, "z4 gemv add")
    assert np.array_equal(got[1:].view(np.uint32), gemv(p, x, xb.EPI_ADD, rows, y0)[1:].view(np.uint32))
    got = gemv(w, x, xb.EPI_SILU_PAIR, rows // 2)
    g, u = want[0::2], want[1::2]
    close(got, g / (1 + np.exp(-g)) * u, "z4 gemv silu pair")
    assert np.array_equal(got[1:].view(np.uint32), gemv(p, x, xb.EPI_SILU_PAIR, rows // 2)[1:].view(np.uint32))


def test_gemv_z4_argmax():
    rows, cols = 30000, 4096
    q = z4_matrix(rows, cols, 11)
    x = np.random.default_rng(12).normal(0, 1, cols).astype(np.float32)
    want_idx, want_val = ob.gemv_argmax(q, x)
    w = upload(q)
    assert w.w.layout == xb.LAYOUT_TILED64_F32S_Z4
    xd = xb.DeviceBuffer.from_array(x)
    ws = xb.DeviceBuffer(xb.hip().xqhip_argmax_workspace_bytes(rows))
    idx, val = xb.DeviceBuffer(4), xb.DeviceBuffer(4)
    xb.ck(xb.hip().xqhip_gemv_w4a16_argmax(w.ref, xd.ptr, xb.F32, None, ws.ptr, idx.ptr, val.ptr, None))
    gv = float(val.download(np.float32, 1)[0])
    assert abs(gv - want_val) <= 1e-2 + 1e-3 * abs(want_val)
    logits = np.sort(ob.gemv(q, x).astype(np.float64))
    if logits[-1] - logits[-2] > 1e-2:
        assert int(idx.download(np.int32, 1)[0]) == want_idx


def test_gemv_z4_rms_prologue():
    rows, cols = 4096, 4096
    q = z4_matrix(rows, cols, 21)
    rng = np.random.default_rng(22)
    x = rng.normal(0, 1, cols).astype(np.float32)
    gamma = rng.normal(1, 0.1, cols).astype(np.float32)
    w = upload(q)
    xd, gd, yd = xb.DeviceBuffer.from_array(x), xb.DeviceBuffer.from_array(gamma), xb.DeviceBuffer(rows * 4)
    pro = xb.prologue(xb.PRO_RMS, gd, eps=1e-6)
    xb.ck(xb.hip().xqhip_gemv_w4a16(w.ref, xd.ptr, xb.F32, ctypes.byref(pro), yd.ptr, xb.F32, xb.EPI_STORE, None))
    xb.ck(xb.hip().xqhip_device_synchronize())
    close(yd.download(np.float32, rows), oracle_rows(q, x[None, :], "rms", gamma)[0], "z4 gemv rms prologue")


@pytest.mark.parametrize("rows,cols,m,epi", [(512, 4096, 40, xb.EPI_STORE), (256, 12288, 70, xb.EPI_ADD),
                                             (512, 4096, 33, xb.EPI_SILU_PAIR), (200, 8256, 17, xb.EPI_STORE)])
def test_gemm_z4_matches_oracle_and_pair_layout(rows, cols, m, epi):
    """The prefill GEMM's zero-point pass reads the 4-bit zeros (12288 and
    8256 columns are split over K: G = 129 in splits of 33 groups, which
    start inside a zero word)."""
    print(f"z4 gemm {rows}x{cols} m={m} epi={epi}", flush=True)
    q = z4_matrix(rows, cols, rows + m + epi)
    rng = np.random.default_rng(m)
    X = rng.normal(0, 1, (m, cols)).astype(np.float32)
    gamma = rng.normal(1, 0.1, cols).astype(np.float32)
    pro = "rms" if cols == 4096 else None
    want = oracle_rows(q, X, pro, gamma if pro else None)
    y0 = rng.normal(0, 1, (m, rows)).astype(np.float32) if epi == xb.EPI_ADD else None
    got = run_gemm(q, X, epi, pro, gamma if pro else None, y0=y0)
    pair = run_gemm(with_pair_layout(q), X, epi, pro, gamma if pro else None, y0=y0)
    if epi == xb.EPI_STORE:
        close(got, want, "z4 gemm")
    elif epi == xb.EPI_ADD:
        close(got, y0 + want, "z4 gemm add")
    else:
        g, u = want[:, 0::2].astype(np.float64), want[:, 1::2].astype(np.float64)
        close(got, g / (1 + np.exp(-g)) * u, "z4 gemm silu")
    # output column 0 holds row 0 (the SiLU pair: rows 0 and 1), the row whose zero differs
    assert np.array_equal(got[:, 1:].view(np.uint32), pair[:, 1:].view(np.uint32))


def test_chain_refuses_z4_layout():
    q = z4_matrix(256, 4096, 3)
    w = upload(q)
    x = dev(np.ones(4096, np.float32))
    ops = (xb.ChainOp * 1)()
    ops[0].w, ops[0].epi, ops[0].x = ctypes.pointer(w.w), xb.EPI_STORE, xb.ChainSrc(x.ptr, 0, 0)
    ch = ctypes.c_void_p()
    assert xb.hip().xqhip_chain_create(ops, 1, ctypes.byref(ch)) == -1
    assert b"layout 4" in xb.hip().xqhip_last_error()


@pytest.fixture(scope="module")
def asym_dir(tmp_path_factory):
    from tiny_model import SMALL
    d = str(tmp_path_factory.mktemp("asym"))
    xb.write_synth_model(d, **SMALL, asymmetric=1)
    return d


def test_asymmetric_model_matches_oracle(asym_dir):
    """Every projection of the model in the 4-bit-zero layout: batched prefill
    and greedy decode against the oracle model on the same files."""
    from test_model_gpu import close as mclose, compare_tokens, oracle_run
    prompt = [int(t) for t in np.random.default_rng(77).integers(0, 4096, 70)]
    n_new = 8
    want, margins, hiddens = oracle_run(asym_dir, prompt, n_new)
    s = xb.Session(asym_dir, xb.options())
    assert s.status == xb.XQ_OK
    st, info = s.json("xq_get_backend_info")
    assert "f32s_z4:0" not in info and "f32meta:0" in info, info
    st, m = s.prefill(prompt)
    assert st == 0
    mclose(s.hidden()[1], hiddens[0], "asymmetric model hidden after prefill")
    got = []
    for i in range(n_new):
        st, tok, m = s.decode_one()
        assert st == 0
        got.append(tok)
        if got == want[: i + 1]:
            mclose(s.hidden()[1], hiddens[i + 1], f"asymmetric model hidden after decode step {i}")
    steps = compare_tokens(got, want, margins)
    assert steps >= 4 or min(margins[:4]) <= 1e-2
    s.close()
