"""GPU parity of the prompt-chunk (prefill) kernels.  The reference prefills
token by token (customlib/runtime/custom_model.cpp:610-640), so every batched
kernel is checked against its per-token form:
  GEMM            against the oracle's per-token RMSNorm / gated head norm +
                  fused GEMV (xq_gemv_w4a16_neon.cpp:259-291), all epilogues;
  embed / qk prep against T single-token calls of the decode kernels (exact);
  attention       against the oracle's attention (custom_model.cpp:840-928)
                  over the causal prefix of every token, then the output gate;
  linear scan     against T consecutive xqhip_linear_attn_step calls.
Tolerance for fp32 outputs: 1e-2 abs + 1e-3 rel (the GEMM carries weights and
activations as fp16 hi + lo pairs, about 22 significant bits each)."""
import ctypes

import numpy as np
import pytest

import oracle_bind as ob
import xqbind as xb
from synth import w4_matrix
from test_decode_ops_gpu import close, dev, linear_inputs

pytestmark = pytest.mark.gpu
O = ob.oracle


def at(buf, byte_off):
    """Device pointer byte_off bytes into buf."""
    return ctypes.c_void_p(buf.ptr.value + byte_off)


def oracle_rows(q, X, pro=None, gamma=None, z=None, head_dim=0):
    """Per token: prologue (RMS with gamma, or gated head norm with gamma, z), then the oracle GEMV."""
    out = []
    for t in range(X.shape[0]):
        x = X[t].astype(np.float32).copy()
        if pro == "rms":
            y = np.empty_like(x)
            O().orc_rmsnorm(ob.p(x), ob.p(gamma), x.size, 1e-6, ob.p(y))
            x = y
        elif pro == "gated":
            y = np.empty_like(x)
            zz = np.ascontiguousarray(z[t], np.float32)
            O().orc_gated_head_rms(ob.p(x), ob.p(gamma), ob.p(zz), x.size // head_dim, head_dim, 1e-6, ob.p(y))
            x = y
        out.append(ob.gemv(q, x))
    return np.stack(out)


def run_gemm(q, X, epi, pro=None, gamma=None, z=None, head_dim=0, y0=None):
    m, cols = X.shape
    w = xb.DeviceW4(q.packed, q.scales, q.zeros, q.rows, q.cols, group=q.group, affine=q.affine)
    out_cols = q.rows // 2 if epi == xb.EPI_SILU_PAIR else q.rows
    ydev = dev(y0 if y0 is not None else np.zeros((m, out_cols), np.float32))
    ws = xb.DeviceBuffer(xb.hip().xqhip_gemm_workspace_bytes(m, cols, q.rows))
    pr, ld_gate = None, 0
    if pro == "rms":
        pr = xb.prologue(xb.PRO_RMS, dev(gamma), eps=1e-6)
    elif pro == "gated":
        zd = dev(z)
        pr = xb.prologue(xb.PRO_GATED_HEAD, dev(gamma), gate=zd, head_dim=head_dim, eps=1e-6)
        ld_gate = z.shape[1]
    xb.ck(xb.hip().xqhip_gemm_w4a16(w.ref, dev(X).ptr, m, cols, ctypes.byref(pr) if pr else None, ld_gate,
                                    ydev.ptr, out_cols, epi, ws.ptr, ws.nbytes, None))
    return ydev.download(np.float32, m * out_cols).reshape(m, out_cols)


@pytest.mark.parametrize("rows,cols,m,pro,affine,zero", [(4096, 4096, 64, "rms", 0, 8.0), (200, 4096, 5, "rms", 0, 8.0),
                                                         (96, 12288, 70, None, 0, 8.0), (130, 640, 130, "rms", 1, 8.0),
                                                         (64, 4096, 33, "gated", 0, 8.0),
                                                         (256, 4096, 40, "rms", 0, 6.0)])
def test_gemm_store_vs_per_token_gemv(rows, cols, m, pro, affine, zero):
    """Zero 8 (format v1): the scale-only layout, no zero-point pass; zero 6
    and the affine format: fp16 (scale, zero) pairs and the zero-point pass."""
    q = w4_matrix(rows, cols, rows + cols + m, affine=affine, zero=zero)
    rng = np.random.default_rng(m)
    X = rng.normal(0, 1, (m, cols)).astype(np.float32)
    gamma = z = None
    if pro == "rms":
        gamma = rng.normal(1, 0.1, cols).astype(np.float32)
    elif pro == "gated":
        gamma = rng.normal(1, 0.1, 128).astype(np.float32)
        z = rng.normal(0, 1, (m, cols)).astype(np.float32)
    want = oracle_rows(q, X, pro, gamma, z, 128)
    got = run_gemm(q, X, xb.EPI_STORE, pro, gamma, z, 128)
    close(got, want, f"gemm {rows}x{cols} m={m} {pro} affine={affine}")


def test_gemm_add_and_silu_pair_epilogues():
    rows, cols, m = 512, 4096, 48
    q = w4_matrix(rows, cols, 77)
    rng = np.random.default_rng(5)
    X = rng.normal(0, 1, (m, cols)).astype(np.float32)
    gamma = rng.normal(1, 0.1, cols).astype(np.float32)
    want = oracle_rows(q, X, "rms", gamma)
    y0 = rng.normal(0, 1, (m, rows)).astype(np.float32)
    close(run_gemm(q, X, xb.EPI_ADD, "rms", gamma, y0=y0), y0 + want, "gemm add epilogue")
    g, u = want[:, 0::2].astype(np.float64), want[:, 1::2].astype(np.float64)
    close(run_gemm(q, X, xb.EPI_SILU_PAIR, "rms", gamma), g / (1 + np.exp(-g)) * u, "gemm silu pair epilogue")


def test_embed_batch_matches_single_rows():
    vocab, hidden, n = 1000, 512, 9
    rng = np.random.default_rng(1)
    table = (rng.normal(0, 1, vocab * hidden).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    ids = np.array([0, 5, 999, -3, 1000, 17, 17, 250, -1001], np.int32)
    out = xb.DeviceBuffer(n * hidden * 4)
    xb.ck(xb.hip().xqhip_embed_bf16_batch(dev(table).ptr, vocab, hidden, dev(ids).ptr, n, out.ptr, None))
    got = out.download(np.float32, n * hidden).reshape(n, hidden)
    for t, tok in enumerate(ids):
        row = tok if 0 <= tok < vocab else abs(int(tok)) % vocab
        assert np.array_equal(got[t], (table[row * hidden:(row + 1) * hidden].astype(np.uint32) << 16).view(np.float32))


def test_attn_prep_batch_matches_single_token_calls():
    nq, nkv, hd, rot, T, pos0 = 4, 2, 64, 16, 7, 20
    rng = np.random.default_rng(3)
    stride = 2 * nq * hd + 2 * nkv * hd + 5
    proj = rng.normal(0, 1, (T, stride)).astype(np.float32)
    qn, kn = rng.normal(1, 0.1, hd).astype(np.float32), rng.normal(1, 0.1, hd).astype(np.float32)
    cap = 64
    tab = np.empty(cap * (rot // 2) * 2, np.float32)
    xb.hip().xqhip_rope_table(1e7, rot, cap, tab.ctypes.data_as(ctypes.c_void_p))
    cs = dev(tab)
    pd, qnd, knd = dev(np.array([pos0], np.int32)), dev(qn), dev(kn)
    pjd = dev(proj)
    ko = nq * 2 * hd
    vo = ko + nkv * hd
    kc_b, vc_b = xb.DeviceBuffer(cap * nkv * hd * 2), xb.DeviceBuffer(cap * nkv * hd * 2)
    kc_b.zero(), vc_b.zero()
    qo_b, go_b = xb.DeviceBuffer(T * nq * hd * 4), xb.DeviceBuffer(T * nq * hd * 4)
    xb.ck(xb.hip().xqhip_attn_prep_batch(pjd.ptr, at(pjd, ko * 4), at(pjd, vo * 4), 1, nq, nkv, hd, rot, qnd.ptr,
                                         knd.ptr, 1e-6, cs.ptr, pd.ptr, T, stride, nq * hd, qo_b.ptr, go_b.ptr,
                                         kc_b.ptr, vc_b.ptr, None))
    kc_s, vc_s = xb.DeviceBuffer(cap * nkv * hd * 2), xb.DeviceBuffer(cap * nkv * hd * 2)
    kc_s.zero(), vc_s.zero()
    qo_s, go_s = xb.DeviceBuffer(nq * hd * 4), xb.DeviceBuffer(nq * hd * 4)
    for t in range(T):
        row = dev(proj[t])
        xb.ck(xb.hip().xqhip_attn_prep(row.ptr, at(row, ko * 4), at(row, vo * 4), 1, nq, nkv, hd, rot, qnd.ptr,
                                       knd.ptr, 1e-6, cs.ptr, dev(np.array([pos0 + t], np.int32)).ptr, qo_s.ptr,
                                       go_s.ptr, kc_s.ptr, vc_s.ptr, None))
        qb = qo_b.download(np.float32, T * nq * hd).reshape(T, -1)
        gb = go_b.download(np.float32, T * nq * hd).reshape(T, -1)
        assert np.array_equal(qb[t], qo_s.download(np.float32, nq * hd))
        assert np.array_equal(gb[t], go_s.download(np.float32, nq * hd))
    assert np.array_equal(kc_b.download(np.float16, cap * nkv * hd), kc_s.download(np.float16, cap * nkv * hd))
    assert np.array_equal(vc_b.download(np.float16, cap * nkv * hd), vc_s.download(np.float16, cap * nkv * hd))


@pytest.mark.parametrize("nq,nkv,hd,T,pos0", [(32, 8, 128, 70, 0), (32, 8, 128, 9, 500), (32, 8, 128, 33, 130),
                                              (4, 2, 8, 5, 3)])
def test_prefill_attention_vs_causal_oracle(nq, nkv, hd, T, pos0):
    rng = np.random.default_rng(T + pos0)
    ctx = pos0 + T
    kc = rng.normal(0, 1, (ctx, nkv, hd)).astype(np.float16)
    vc = rng.normal(0, 1, (ctx, nkv, hd)).astype(np.float16)
    q = rng.normal(0, 1, (T, nq * hd)).astype(np.float32)
    gate = rng.normal(0, 1, (T, nq * hd)).astype(np.float32)
    out = xb.DeviceBuffer(T * nq * hd * 4)
    xb.ck(xb.hip().xqhip_prefill_attention(dev(q).ptr, dev(gate).ptr, dev(kc).ptr, dev(vc).ptr, nq, nkv, hd, T,
                                           nq * hd, dev(np.array([pos0], np.int32)).ptr, out.ptr, nq * hd, None))
    got = out.download(np.float32, T * nq * hd).reshape(T, -1)
    kf, vf = kc.astype(np.float32), vc.astype(np.float32)
    for t in range(T):
        n = pos0 + t + 1
        att = np.empty(nq * hd, np.float32)
        kk, vv = np.ascontiguousarray(kf[:n]).reshape(-1), np.ascontiguousarray(vf[:n]).reshape(-1)
        O().orc_attention_model(ob.p(q[t]), ob.p(kk), ob.p(vv), n, nkv, nq, hd, ob.p(att))
        want = att * np.array([O().orc_sigmoid(float(g)) for g in gate[t]], np.float32)
        close(got[t], want, f"prefill attention token {t} (ctx {n})")


@pytest.mark.parametrize("with_ws", [False, True])
@pytest.mark.parametrize("shape,T,pos0", [((16, 32, 128, 128, 4), 12, 0), ((16, 32, 128, 128, 4), 7, 5),
                                          ((16, 32, 128, 128, 4), 37, 3), ((3, 6, 64, 32, 3), 9, 2),
                                          ((2, 2, 256, 40, 4), 4, 1), ((2, 4, 128, 24, 2), 2, 0),
                                          ((16, 32, 128, 128, 4), 64, 0), ((16, 32, 128, 128, 4), 130, 7),
                                          ((2, 4, 128, 24, 2), 100, 1)])
def test_linear_scan_matches_consecutive_steps(shape, T, pos0, with_ws):
    """The prefill scan (fused per-token kernel, or with a workspace the
    token-parallel conv pass + the chunked recurrence for 128-dim key heads)
    against consecutive decode steps; 37 tokens cross the 16-token staging
    groups, 64 fill one 64-token chunk exactly, 130 and 100 span several
    chunks with a short last one (100 with value heads of 24 columns)."""
    lk_n, lv_n, lk_hd, lv_hd, ks = shape
    rng = np.random.default_rng(T * 7 + pos0)
    _, cstate, cw = linear_inputs(lk_n, lv_n, lk_hd, lv_hd, ks, seed=41)
    conv_dim = 2 * lk_n * lk_hd + lv_n * lv_hd
    stride = conv_dim + 2 * lv_n + 3
    rows = rng.normal(0, 1, (T, stride)).astype(np.float32)
    a_log = rng.normal(-1, 0.5, lv_n).astype(np.float32)
    dt = rng.normal(0, 0.5, lv_n).astype(np.float32)
    S0 = rng.normal(0, 0.1, lv_n * lk_hd * lv_hd).astype(np.float32)
    hist = cstate.size
    two = np.zeros(2 * hist, np.float32)
    two[(pos0 & 1) * hist:((pos0 & 1) + 1) * hist] = cstate
    # batched
    sd_b, Sd_b, rd = dev(two), dev(S0), dev(rows)
    out_b = xb.DeviceBuffer(T * lv_n * lv_hd * 4)
    args = (rd.ptr, at(rd, conv_dim * 4), at(rd, (conv_dim + lv_n) * 4), stride, sd_b.ptr, pos0, dev(cw).ptr,
            dev(a_log).ptr, dev(dt).ptr, Sd_b.ptr, lk_n, lk_hd, lv_n, lv_hd, ks, T, out_b.ptr, lv_n * lv_hd)
    if with_ws:
        wsd = xb.DeviceBuffer(xb.hip().xqhip_linear_scan_workspace_bytes(T, lk_n, lk_hd, lv_n, lv_hd))
        xb.ck(xb.hip().xqhip_linear_attn_scan_ws(*args, wsd.ptr, None))
    else:
        xb.ck(xb.hip().xqhip_linear_attn_scan(*args, None))
    # consecutive single steps
    sd_s, Sd_s = dev(two), dev(S0)
    cwd, ald, dtd = dev(cw), dev(a_log), dev(dt)
    outs = []
    for t in range(T):
        row = dev(rows[t])
        od = xb.DeviceBuffer(lv_n * lv_hd * 4)
        xb.ck(xb.hip().xqhip_linear_attn_step(row.ptr, sd_s.ptr, cwd.ptr, at(row, conv_dim * 4),
                                              at(row, (conv_dim + lv_n) * 4), ald.ptr, dtd.ptr, Sd_s.ptr, lk_n, lk_hd,
                                              lv_n, lv_hd, ks, dev(np.array([pos0 + t], np.int32)).ptr, od.ptr, None))
        outs.append(od.download(np.float32, lv_n * lv_hd))
    got = out_b.download(np.float32, T * lv_n * lv_hd).reshape(T, -1)
    close(got, np.stack(outs), "linear scan outputs", atol=1e-5, rtol=1e-5)
    close(Sd_b.download(np.float32, S0.size), Sd_s.download(np.float32, S0.size), "linear scan state",
          atol=1e-6, rtol=1e-5)
    nxt = (pos0 + T) & 1  # the copy the next decode position reads
    hb = sd_b.download(np.float32, 2 * hist)[nxt * hist:(nxt + 1) * hist]
    hs = sd_s.download(np.float32, 2 * hist)[nxt * hist:(nxt + 1) * hist]
    assert np.array_equal(hb, hs)


def test_linear_scan_130_tokens_matches_oracle():
    """The chunked prefill recurrence (token-parallel conv pass, then 64-token
    chunks: three chunks, the last one short) at the 9B shape (16 key heads,
    32 value heads of 128 x 128, 4 taps) directly against the oracle's
    per-token restatement: orc_conv1d_step + orc_l2norm_heads + the gate /
    beta formulas + orc_gated_delta for each of 130 tokens
    (custom_model.cpp:961-1096, ref_delta.cpp:8-41).  Outputs and the final
    state within 1e-6 (outputs) or 5e-6 (state) abs + 1e-5 rel (measured 6e-8 and
    7e-7; the chunked form sums in another fp32
    order); the conv history the next decode position reads bit-exact."""
    from test_decode_ops_gpu import oracle_linear_step
    shape = lk_n, lv_n, lk_hd, lv_hd, ks = (16, 32, 128, 128, 4)
    T, pos0 = 130, 7
    rng = np.random.default_rng(130)
    _, cstate, cw = linear_inputs(lk_n, lv_n, lk_hd, lv_hd, ks, seed=43)
    conv_dim = 2 * lk_n * lk_hd + lv_n * lv_hd
    stride = conv_dim + 2 * lv_n + 3
    rows = rng.normal(0, 1, (T, stride)).astype(np.float32)
    a_log = rng.normal(-1, 0.5, lv_n).astype(np.float32)
    dt = rng.normal(0, 0.5, lv_n).astype(np.float32)
    S0 = rng.normal(0, 0.1, lv_n * lk_hd * lv_hd).astype(np.float32)
    hist = cstate.size
    two = np.zeros(2 * hist, np.float32)
    two[(pos0 & 1) * hist:((pos0 & 1) + 1) * hist] = cstate
    sd, Sd, rd = dev(two), dev(S0), dev(rows)
    out = xb.DeviceBuffer(T * lv_n * lv_hd * 4)
    wsd = xb.DeviceBuffer(xb.hip().xqhip_linear_scan_workspace_bytes(T, lk_n, lk_hd, lv_n, lv_hd))
    xb.ck(xb.hip().xqhip_linear_attn_scan_ws(rd.ptr, at(rd, conv_dim * 4), at(rd, (conv_dim + lv_n) * 4), stride,
                                             sd.ptr, pos0, dev(cw).ptr, dev(a_log).ptr, dev(dt).ptr, Sd.ptr, lk_n,
                                             lk_hd, lv_n, lv_hd, ks, T, out.ptr, lv_n * lv_hd, wsd.ptr, None))
    got = out.download(np.float32, T * lv_n * lv_hd).reshape(T, -1)
    st, S = cstate.copy(), S0.copy()
    want = np.empty_like(got)
    for t in range(T):
        r = rows[t]
        want[t] = oracle_linear_step(r[:conv_dim].copy(), st, cw, r[conv_dim:conv_dim + lv_n],
                                     r[conv_dim + lv_n:conv_dim + 2 * lv_n], a_log, dt, S, shape)
    print(f"scan vs oracle: max output err {np.abs(got - want).max():.3g}, "
          f"max state err {np.abs(Sd.download(np.float32, S.size) - S).max():.3g}", flush=True)
    close(got, want, "chunked scan vs oracle outputs", atol=1e-6, rtol=1e-5)
    close(Sd.download(np.float32, S.size), S, "chunked scan vs oracle state", atol=5e-6, rtol=1e-5)
    nxt = (pos0 + T) & 1
    assert np.array_equal(sd.download(np.float32, 2 * hist)[nxt * hist:(nxt + 1) * hist], st)


def test_gemm_rejects_a_short_workspace():
    """The workspace holds the staged x and, for launches split over the columns,
    the partial products of every row: one sized for fewer rows is refused
    (XQHIP_EINVAL) instead of being written past its end."""
    rows, cols, m = 4096, 4096, 64
    q = w4_matrix(rows, cols, 3)
    w = xb.DeviceW4(q.packed, q.scales, q.zeros, rows, cols)
    x, y = dev(np.zeros((m, cols), np.float32)), xb.DeviceBuffer(m * rows * 4)
    need = xb.hip().xqhip_gemm_workspace_bytes(m, cols, rows)
    short = xb.hip().xqhip_gemm_workspace_bytes(m, cols, 0)
    ws = xb.DeviceBuffer(need)
    if short < need:  # a split launch: the partial products need room
        assert xb.hip().xqhip_gemm_w4a16(w.ref, x.ptr, m, cols, None, 0, y.ptr, rows, xb.EPI_STORE, ws.ptr, short,
                                         None) == -1
        assert b"workspace" in xb.hip().xqhip_last_error()
    xb.ck(xb.hip().xqhip_gemm_w4a16(w.ref, x.ptr, m, cols, None, 0, y.ptr, rows, xb.EPI_STORE, ws.ptr, need, None))
