"""GPU parity of xqhip_linear_attn_step_outproj, the linear-attention decode
step and the output projection that consumes it as one launch.

Reference semantics: conv1d + SiLU, q / k L2 norm and the gated delta rule
(custom_model.cpp:961-1096), then applyGatedHeadRms over the step's output
with the SiLU'd z gate (custom_model.cpp:329-349, 1123-1133), the out_proj
GEMV (gemvW4A16Neon) and addResidual into the hidden state (:1135, 1179).

Checks:
* against the two separate calls (xqhip_linear_attn_step_act, then
  xqhip_gemv_w4a16 with PRO_GATED_HEAD_ACT and the ADD epilogue) bit for bit
  on every output the pair writes (step output, activated gate, recurrent
  state, both conv history copies, residual), over three consecutive
  positions (both history parities, and the hand-off counters reused by
  consecutive launches), on the 9B shape in all four metadata forms and on
  shapes whose projection has fewer rows than a grid's worth, more rows than
  the two weight batches requested before the wait, and a step with fewer
  blocks than the projection;
* the residual against the oracle's step + gated norm + GEMV + residual add;
* the error word stays 0, and unsupported combinations are refused.
"""
import ctypes

import numpy as np
import pytest

import oracle_bind as ob
import xqbind as xb
from test_decode_ops_gpu import O, close, dev, linear_inputs, oracle_linear_step

pytestmark = pytest.mark.gpu


def proj_matrix(rows, cols, kind, seed):
    """A 4-bit format-v1 matrix whose metadata selects one upload layout:
    s16 (zeros 8, fp16 scales), f16pair (integer zeros, fp16 scales), f32pair
    (fp32 scales, non-integer zeros), z4 (fp32 scales, integer zeros)."""
    rng = np.random.default_rng(seed)
    packed = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
    g = rows * (cols // 64)
    s32 = (np.abs(rng.normal(0.0, 0.02, g)) + 1e-4).astype(np.float32)
    s16 = s32.astype(np.float16).astype(np.float32)
    zi = rng.integers(0, 16, g).astype(np.float32)
    scales, zeros = {"s16": (s16, np.full(g, 8.0, np.float32)), "f16pair": (s16, zi),
                     "f32pair": (s32, (zi + 0.25).astype(np.float32)), "z4": (s32, zi)}[kind]
    return ob.Quantized(packed, scales, zeros, rows, cols, 64, 0)


LAYOUT = {"s16": xb.LAYOUT_TILED64_SCALE16, "f16pair": xb.LAYOUT_TILED64, "f32pair": xb.LAYOUT_TILED64_F32META,
          "z4": xb.LAYOUT_TILED64_F32S_Z4}


def step_inputs(shape, seed):
    lk_n, lv_n, lk_hd, lv_hd, ks = shape
    rng = np.random.default_rng(seed)
    mixed, cstate, cw = linear_inputs(lk_n, lv_n, lk_hd, lv_hd, ks, seed=seed + 1)
    a = rng.normal(0, 1, lv_n).astype(np.float32)
    b = rng.normal(0, 1, lv_n).astype(np.float32)
    a_log = rng.normal(-1, 0.5, lv_n).astype(np.float32)
    dt = rng.normal(0, 0.5, lv_n).astype(np.float32)
    S0 = rng.normal(0, 0.1, lv_n * lk_hd * lv_hd).astype(np.float32)
    mixes = [mixed] + [rng.normal(0, 1, mixed.size).astype(np.float32) for _ in range(2)]
    zs = [rng.normal(0, 2, lv_n * lv_hd).astype(np.float32) for _ in range(3)]
    return mixes, zs, cstate, cw, a, b, a_log, dt, S0


class Run:
    """Device state of one path (its own copies of every buffer the pair writes)."""

    def __init__(self, shape, cstate, S0, y0):
        lk_n, lv_n, lk_hd, lv_hd, ks = shape
        hist = cstate.size
        self.hist = hist
        self.sd = dev(np.concatenate([cstate, np.full(hist, 3.0, np.float32)]))
        self.Sd = dev(S0)
        self.yd = dev(y0)
        self.od = xb.DeviceBuffer(lv_n * lv_hd * 4)

    def snapshot(self, zd, n_out, n_state, n_y):
        return (self.od.download(np.float32, n_out), zd.download(np.float32, n_out),
                self.Sd.download(np.float32, n_state), self.sd.download(np.float32, 2 * self.hist),
                self.yd.download(np.float32, n_y))


CASES = [((16, 32, 128, 128, 4), 4096, "s16"), ((16, 32, 128, 128, 4), 4096, "f16pair"),
         ((16, 32, 128, 128, 4), 4096, "f32pair"), ((16, 32, 128, 128, 4), 4096, "z4"),
         ((2, 4, 64, 64, 4), 300, "s16"),       # 25 projection blocks, 16 step blocks
         ((4, 8, 128, 128, 4), 8000, "z4"),     # 3 row batches per wave: one streamed after the wait
         ((2, 2, 256, 96, 4), 1000, "f32pair")]  # head_dim 96 is not a gated-prologue shape: refused


@pytest.mark.parametrize("shape,rows,kind", CASES)
def test_step_outproj_matches_separate_calls_and_oracle(shape, rows, kind):
    lk_n, lv_n, lk_hd, lv_hd, ks = shape
    cols = lv_n * lv_hd
    print(f"step+outproj shape {shape} rows {rows} kind {kind}", flush=True)
    hip = xb.hip()
    q = proj_matrix(rows, cols, kind, rows + cols)
    w = xb.DeviceW4(q.packed, q.scales, q.zeros, q.rows, q.cols, q.group, q.affine)
    assert w.w.layout == LAYOUT[kind]
    if lv_hd % 8 or (lv_hd // 8) & (lv_hd // 8 - 1):
        assert hip.xqhip_step_outproj_supported(w.ref, lk_n, lk_hd, lv_n, lv_hd, ks) == 0
        return
    assert hip.xqhip_step_outproj_supported(w.ref, lk_n, lk_hd, lv_n, lv_hd, ks) == 1
    mixes, zs, cstate, cw, a, b, a_log, dt, S0 = step_inputs(shape, rows + 7)
    rng = np.random.default_rng(rows)
    y0 = rng.normal(0, 1, rows).astype(np.float32)
    nw = rng.normal(1, 0.1, lv_hd).astype(np.float32)
    wd, ad, bd, ald, dtd, nwd = dev(cw), dev(a), dev(b), dev(a_log), dev(dt), dev(nw)
    sync = xb.DeviceBuffer(hip.xqhip_step_outproj_sync_bytes())
    sync.zero()
    sep, fus = Run(shape, cstate, S0, y0), Run(shape, cstate, S0, y0)
    st_o, S_o, y_o = cstate.copy(), S0.copy(), y0.astype(np.float64)
    pos0 = 6
    for step in range(3):
        md, pd = dev(mixes[step]), dev(np.array([pos0 + step], np.int32))
        z_sep, z_fus = dev(zs[step]), dev(zs[step])
        # the two separate calls
        args = (md.ptr, sep.sd.ptr, wd.ptr, ad.ptr, bd.ptr, ald.ptr, dtd.ptr, sep.Sd.ptr, lk_n, lk_hd, lv_n, lv_hd, ks,
                pd.ptr, sep.od.ptr, z_sep.ptr)
        xb.ck(hip.xqhip_linear_attn_step_act(*args, None))
        pro = xb.prologue(xb.PRO_GATED_HEAD_ACT, nwd, z_sep, head_dim=lv_hd, eps=1e-6)
        xb.ck(hip.xqhip_gemv_w4a16(w.ref, sep.od.ptr, xb.F32, ctypes.byref(pro), sep.yd.ptr, xb.F32, xb.EPI_ADD,
                                   None))
        # one launch
        xb.ck(hip.xqhip_linear_attn_step_outproj(md.ptr, fus.sd.ptr, wd.ptr, ad.ptr, bd.ptr, ald.ptr, dtd.ptr,
                                                 fus.Sd.ptr, lk_n, lk_hd, lv_n, lv_hd, ks, pd.ptr, fus.od.ptr,
                                                 z_fus.ptr, w.ref, nwd.ptr, 1e-6, fus.yd.ptr, sync.ptr, None))
        xb.ck(hip.xqhip_device_synchronize())
        got_s = sep.snapshot(z_sep, cols, S0.size, rows)
        got_f = fus.snapshot(z_fus, cols, S0.size, rows)
        for what, s_arr, f_arr in zip(("step output", "activated gate", "state", "conv history", "residual"),
                                      got_s, got_f):
            assert np.array_equal(s_arr.view(np.uint32), f_arr.view(np.uint32)), f"{what}, step {step}"
        # oracle: step, gated norm over the silu'd gate, GEMV, residual add
        out_o = oracle_linear_step(mixes[step], st_o, cw, a, b, a_log, dt, S_o, shape)
        normed = np.empty_like(out_o)
        O().orc_gated_head_rms(ob.p(out_o), ob.p(nw), ob.p(zs[step]), lv_n, lv_hd, 1e-6, ob.p(normed))
        y_o = y_o + ob.gemv(q, normed).astype(np.float64)
        close(got_f[4], y_o, f"step+outproj residual vs oracle, step {step}")
    bad = ctypes.c_int(-1)
    xb.ck(hip.xqhip_step_outproj_error(sync.ptr, ctypes.byref(bad)))
    assert bad.value == 0
    assert not np.any(sync.download(np.uint32, sync.nbytes // 4))  # every launch leaves the counters at zero
    w.free()


def test_step_outproj_refusals():
    hip = xb.hip()
    lk_n, lv_n, lk_hd, lv_hd = 16, 32, 128, 128
    q = proj_matrix(256, 4096, "s16", 5)
    w = xb.DeviceW4(q.packed, q.scales, q.zeros, q.rows, q.cols, q.group, q.affine)
    assert hip.xqhip_step_outproj_supported(w.ref, lk_n, lk_hd, lv_n, lv_hd, 4) == 1
    assert hip.xqhip_step_outproj_supported(w.ref, lk_n, lk_hd, lv_n, lv_hd, 3) == 0  # conv width 4 only
    assert hip.xqhip_step_outproj_supported(w.ref, lk_n, lk_hd, 16, lv_hd, 4) == 0    # columns != lv_n * lv_hd
    buf = xb.DeviceBuffer(1 << 20)
    sync = xb.DeviceBuffer(hip.xqhip_step_outproj_sync_bytes())
    sync.zero()
    p = buf.ptr
    args = [p] * 8 + [lk_n, lk_hd, lv_n, lv_hd, 3, p, p, p, w.ref, p, 1e-6, p, sync.ptr, None]
    assert hip.xqhip_linear_attn_step_outproj(*args) == -4  # XQHIP_ENOTSUP
    args[12] = 4
    args[20] = ctypes.c_void_p(sync.ptr.value + 4)  # sync must be 128-byte aligned
    assert hip.xqhip_linear_attn_step_outproj(*args) == -1
    assert b"128-byte" in hip.xqhip_last_error()
    w.free()
