"""GPU parity of the non-GEMV decode kernels against the oracle restatements of
customlib/runtime/custom_model.cpp (embedding :569-608, q/gate split :740-753,
head RMSNorm :301-313, partial RoPE :351-370, KV append :673-733, GQA decode
:840-928, output gate :929-951, conv1d :961-1010, L2 norm :315-327, gated delta
:1074-1096 / ref_delta.cpp:8-41).

Shapes follow the one-layer decode workloads at position 511: 32 query heads,
8 KV heads, head_dim 128, rotary 32, theta 1e7, a seeded fp16 KV cache of 511
tokens ~N(0,1) plus the appended one; linear attention with 16 key heads and
32 value heads of 128, fp32 state ~N(0, 0.1), decay in (0,1), beta ~U(0,1).
Tolerance for fp32/fp16 outputs: |gpu - oracle| <= 1e-2 + 1e-3 |oracle|;
index and layout checks are exact.
"""
import ctypes

import numpy as np
import pytest

import oracle_bind as ob
import xqbind as xb
from synth import w4_matrix

pytestmark = pytest.mark.gpu
O = ob.oracle
ATOL, RTOL = 1e-2, 1e-3


def close(got, want, what, atol=ATOL, rtol=RTOL):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    err = np.abs(got - want)
    bad = ~(err <= atol + rtol * np.abs(want))  # a NaN anywhere counts as bad
    assert not bad.any(), f"{what}: {bad.sum()} / {bad.size} bad, max err {np.nanmax(err):.3g}"


_keep = []  # device buffers stay alive until the module ends (no free before the kernel ran)


def dev(a):
    b = xb.DeviceBuffer.from_array(np.ascontiguousarray(a))
    _keep.append(b)
    return b


def bf16_bits(x):
    return (np.asarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def test_embedding_rows_and_wrap():
    vocab, hidden = 1000, 4096
    rng = np.random.default_rng(0)
    table = bf16_bits(rng.normal(0, 1, vocab * hidden).astype(np.float32))
    td = dev(table)
    out = xb.DeviceBuffer(hidden * 4)
    tok = xb.DeviceBuffer(4)
    for t in (0, 17, 999, -5, 1003, -2000):
        tok.upload(np.array([t], np.int32))
        xb.ck(xb.hip().xqhip_embed_bf16(td.ptr, vocab, hidden, tok.ptr, out.ptr, None))
        got = out.download(np.float32, hidden)
        row = t if 0 <= t < vocab else abs(t) % vocab
        want = (table[row * hidden:(row + 1) * hidden].astype(np.uint32) << 16).view(np.float32)
        assert np.array_equal(got, want), t


def test_rope_table_matches_oracle_libm():
    rd, theta, npos = 32, 1e7, 600
    tab = np.empty(npos * rd, np.float32)
    xb.ck(xb.hip().xqhip_rope_table(theta, rd, npos, xb.ptr(tab)))
    tab = tab.reshape(npos, rd // 2, 2)
    # rotate unit vectors with the oracle: (1,0) -> (cos, sin)
    for pos in (0, 1, 511, 599):
        x = np.zeros(rd, np.float32)
        x[: rd // 2] = 1.0
        O().orc_rope_partial(ob.p(x), 1, rd, rd, pos, theta)
        assert np.array_equal(x[: rd // 2], tab[pos, :, 0]) and np.array_equal(x[rd // 2:], tab[pos, :, 1])


def attn_layer_inputs(nq=32, nkv=8, hd=128, ctx_before=511, seed=5, gated=True):
    rng = np.random.default_rng(seed)
    qsrc = rng.normal(0, 1, nq * hd * (2 if gated else 1)).astype(np.float32)
    k = rng.normal(0, 1, nkv * hd).astype(np.float32)
    v = rng.normal(0, 1, nkv * hd).astype(np.float32)
    qn = rng.normal(1, 0.1, hd).astype(np.float32)
    kn = rng.normal(1, 0.1, hd).astype(np.float32)
    kc = rng.normal(0, 1, (ctx_before, nkv, hd)).astype(np.float16)
    vc = rng.normal(0, 1, (ctx_before, nkv, hd)).astype(np.float16)
    return qsrc, k, v, qn, kn, kc, vc


@pytest.mark.parametrize("gated", [True, False])
def test_attention_prep_and_gqa_decode_pos511(gated):
    nq, nkv, hd, rd, theta, pos, eps = 32, 8, 128, 32, 1e7, 511, 1e-6
    max_ctx = 1024
    qsrc, k, v, qn, kn, kc, vc = attn_layer_inputs(gated=gated)
    # ---- oracle (custom_model.cpp:740-951 order) ----
    if gated:
        qq = qsrc.reshape(nq, 2, hd)[:, 0].reshape(-1).copy()
        gate = qsrc.reshape(nq, 2, hd)[:, 1].reshape(-1).copy()
    else:
        qq, gate = qsrc.copy(), np.zeros(nq * hd, np.float32)
    kk = k.copy()
    O().orc_head_rms(ob.p(qq), ob.p(qn), nq, hd, eps)
    O().orc_head_rms(ob.p(kk), ob.p(kn), nkv, hd, eps)
    O().orc_rope_partial(ob.p(qq), nq, hd, rd, pos, theta)
    O().orc_rope_partial(ob.p(kk), nkv, hd, rd, pos, theta)
    # ---- device ----
    tab = np.empty(max_ctx * rd, np.float32)
    xb.ck(xb.hip().xqhip_rope_table(theta, rd, max_ctx, xb.ptr(tab)))
    kcache = np.zeros((max_ctx, nkv, hd), np.float16)
    vcache = np.zeros((max_ctx, nkv, hd), np.float16)
    kcache[:pos], vcache[:pos] = kc, vc
    kd, vd = dev(kcache), dev(vcache)
    qs_d, k_d, v_d = dev(qsrc), dev(k), dev(v)
    qn_d, kn_d, tab_d = dev(qn), dev(kn), dev(tab)
    pos_d = dev(np.array([pos], np.int32))
    qo, go = xb.DeviceBuffer(nq * hd * 4), xb.DeviceBuffer(nq * hd * 4)
    xb.ck(xb.hip().xqhip_attn_prep(qs_d.ptr, k_d.ptr, v_d.ptr, int(gated), nq, nkv, hd, rd, qn_d.ptr, kn_d.ptr, eps,
                                   tab_d.ptr, pos_d.ptr, qo.ptr, go.ptr, kd.ptr, vd.ptr, None))
    q_got = qo.download(np.float32, nq * hd)
    close(q_got, qq, "q after norm+rope", atol=1e-5, rtol=1e-5)
    assert np.array_equal(go.download(np.float32, nq * hd), gate)
    kc_got = kd.download(np.float16, max_ctx * nkv * hd).reshape(max_ctx, nkv, hd)
    vc_got = vd.download(np.float16, max_ctx * nkv * hd).reshape(max_ctx, nkv, hd)
    assert np.array_equal(kc_got[:pos], kc) and np.array_equal(vc_got[:pos], vc)  # earlier slots untouched
    assert np.array_equal(vc_got[pos].reshape(-1), v.astype(np.float16))          # slot layout [t][kvh][d]
    close(kc_got[pos].reshape(-1).astype(np.float32), kk, "appended k", atol=2e-3, rtol=1e-3)
    # ---- attention over the fp16 cache (the oracle sees the same fp16 values) ----
    ctx = pos + 1
    kf = kc_got[:ctx].astype(np.float32).reshape(-1)
    vf = vc_got[:ctx].astype(np.float32).reshape(-1)
    att = np.empty(nq * hd, np.float32)
    O().orc_attention_model(ob.p(qq), ob.p(kf), ob.p(vf), ctx, nkv, nq, hd, ob.p(att))
    sig = np.array([O().orc_sigmoid(float(g)) for g in gate], np.float32)
    want = att * sig
    ws = xb.DeviceBuffer(xb.hip().xqhip_gqa_workspace_bytes(nq, nkv, hd))
    ws.zero()
    out = xb.DeviceBuffer(nq * hd * 4)
    for _ in range(2):  # a second call on the same workspace gives the same result
        xb.ck(xb.hip().xqhip_gqa_decode(qo.ptr, kd.ptr, vd.ptr, go.ptr, nq, nkv, hd, max_ctx, pos_d.ptr, out.ptr,
                                        ws.ptr, None))
        close(out.download(np.float32, nq * hd), want, "gqa decode + gate")


def oracle_attention_step(qsrc, k, gated, qn, kn, nq, nkv, hd, rd, pos, theta, eps, kcache_f16, vcache_f16):
    """Oracle of one decode attention step over caches that already hold slot pos."""
    if gated:
        qq = qsrc.reshape(nq, 2, hd)[:, 0].reshape(-1).copy()
        gate = qsrc.reshape(nq, 2, hd)[:, 1].reshape(-1).copy()
    else:
        qq, gate = qsrc.copy(), np.zeros(nq * hd, np.float32)
    kk = k.copy()
    O().orc_head_rms(ob.p(qq), ob.p(qn), nq, hd, eps)
    O().orc_head_rms(ob.p(kk), ob.p(kn), nkv, hd, eps)
    O().orc_rope_partial(ob.p(qq), nq, hd, rd, pos, theta)
    O().orc_rope_partial(ob.p(kk), nkv, hd, rd, pos, theta)
    ctx = pos + 1
    kf = kcache_f16[:ctx].astype(np.float32).reshape(-1)
    vf = vcache_f16[:ctx].astype(np.float32).reshape(-1)
    att = np.empty(nq * hd, np.float32)
    O().orc_attention_model(ob.p(qq), ob.p(kf), ob.p(vf), ctx, nkv, nq, hd, ob.p(att))
    sig = np.array([O().orc_sigmoid(float(g)) for g in gate], np.float32)
    return kk, att * sig


# (nq, nkv, head_dim, rotary, pos, max_ctx, gated).  The chunk kernel spreads
# the context over 256 / nkv slots per kv head (at most 64) in chunks of
# 16, 32 or 64 tokens, a slot taking several chunks past 64 per slot.  Cases:
# the Qwen3.5-9B head layout (16-token chunks of head_dim 256); the config-3
# point (32q/8kv d128 at position 511: 16-token chunks, one per slot); the
# first position; 32-token chunks; 64-token chunks, several per slot; a
# head_dim without a specialised kernel; group 8 at the end of the first
# chunk; and a context past 16384 tokens (one kv head, 64 slots of 5 chunks).
FUSED_CASES = [(16, 4, 256, 64, 700, 1024, True), (32, 8, 128, 32, 511, 1024, True), (32, 8, 128, 32, 0, 64, False),
               (32, 8, 128, 32, 700, 1024, True), (8, 2, 64, 64, 4160, 8192, True), (32, 8, 128, 32, 9000, 9216, True),
               (4, 2, 96, 32, 130, 256, True), (16, 2, 128, 32, 63, 128, False), (4, 1, 128, 32, 20000, 20480, False)]


@pytest.mark.parametrize("case", FUSED_CASES, ids=lambda c: "nq%d_nkv%d_hd%d_rd%d_pos%d" % c[:5])
def test_fused_attention_decode(case):
    """xqhip_attn_decode (prep folded into the chunk kernel) against the oracle
    and against xqhip_attn_prep + xqhip_gqa_decode, for two consecutive positions
    (the second reads the slot the first appended)."""
    nq, nkv, hd, rd, pos, max_ctx, gated = case
    theta, eps = 1e7, 1e-6
    print(f"fused attention case {case}", flush=True)
    assert pos + 2 <= max_ctx
    qsrc, k, v, qn, kn, kc, vc = attn_layer_inputs(nq, nkv, hd, pos, seed=pos + hd, gated=gated)
    tab = np.empty(max_ctx * rd, np.float32)
    xb.ck(xb.hip().xqhip_rope_table(theta, rd, max_ctx, xb.ptr(tab)))
    kcache = np.zeros((max_ctx, nkv, hd), np.float16)
    vcache = np.zeros((max_ctx, nkv, hd), np.float16)
    kcache[:pos], vcache[:pos] = kc, vc
    kd, vd = dev(kcache), dev(vcache)    # fused path
    kd2, vd2 = dev(kcache), dev(vcache)  # two-launch path
    qn_d, kn_d, tab_d = dev(qn), dev(kn), dev(tab)
    ws = dev(np.zeros(xb.hip().xqhip_gqa_workspace_bytes(nq, nkv, hd), np.uint8))
    out, out2 = xb.DeviceBuffer(nq * hd * 4), xb.DeviceBuffer(nq * hd * 4)
    qo, go = xb.DeviceBuffer(nq * hd * 4), xb.DeviceBuffer(nq * hd * 4)
    rng = np.random.default_rng(pos)
    for step in range(2):
        p = pos + step
        if step:
            qsrc = rng.normal(0, 1, qsrc.size).astype(np.float32)
            k = rng.normal(0, 1, k.size).astype(np.float32)
            v = rng.normal(0, 1, v.size).astype(np.float32)
        qs_d, k_d, v_d = dev(qsrc), dev(k), dev(v)
        pos_d = dev(np.array([p], np.int32))
        xb.ck(xb.hip().xqhip_attn_decode(qs_d.ptr, k_d.ptr, v_d.ptr, int(gated), nq, nkv, hd, rd, qn_d.ptr, kn_d.ptr,
                                         eps, tab_d.ptr, pos_d.ptr, kd.ptr, vd.ptr, max_ctx, out.ptr, ws.ptr, None))
        xb.ck(xb.hip().xqhip_attn_prep(qs_d.ptr, k_d.ptr, v_d.ptr, int(gated), nq, nkv, hd, rd, qn_d.ptr, kn_d.ptr,
                                       eps, tab_d.ptr, pos_d.ptr, qo.ptr, go.ptr, kd2.ptr, vd2.ptr, None))
        xb.ck(xb.hip().xqhip_gqa_decode(qo.ptr, kd2.ptr, vd2.ptr, go.ptr, nq, nkv, hd, max_ctx, pos_d.ptr, out2.ptr,
                                        ws.ptr, None))
        kc_got = kd.download(np.float16, max_ctx * nkv * hd).reshape(max_ctx, nkv, hd)
        vc_got = vd.download(np.float16, max_ctx * nkv * hd).reshape(max_ctx, nkv, hd)
        assert np.array_equal(kc_got[:pos], kc) and np.array_equal(vc_got[:pos], vc)  # earlier slots untouched
        assert not kc_got[p + 1:].any() and not vc_got[p + 1:].any()                  # later slots untouched
        assert np.array_equal(vc_got[p].reshape(-1), v.astype(np.float16))
        kk, want = oracle_attention_step(qsrc, k, gated, qn, kn, nq, nkv, hd, rd, p, theta, eps, kc_got, vc_got)
        close(kc_got[p].reshape(-1).astype(np.float32), kk, f"appended k pos {p}", atol=2e-3, rtol=1e-3)
        got = out.download(np.float32, nq * hd)
        close(got, want, f"fused attention pos {p}")
        close(got, out2.download(np.float32, nq * hd), f"fused vs two-launch pos {p}", atol=1e-5, rtol=1e-4)


# head_dim 128 shapes for the one-block-per-query-head kernel: contexts inside
# one 1024-token pass (first slot, mid, last slot of the pass), exactly at and
# across pass boundaries (1023 -> 1024, 2047 -> 2048), several passes, group
# sizes 1, 4 and 8, gated and not.
HEAD_CASES = [(32, 8, 128, 32, 0, 64, True), (32, 8, 128, 32, 511, 1024, True), (32, 8, 128, 64, 540, 1024, False),
              (32, 8, 128, 32, 1022, 1040, True), (16, 2, 128, 32, 1023, 2048, True), (8, 8, 128, 128, 2046, 2048, True),
              (32, 8, 128, 32, 3000, 3072, True), (4, 1, 128, 32, 9000, 9216, False)]


@pytest.mark.parametrize("case", HEAD_CASES, ids=lambda c: "nq%d_nkv%d_hd%d_rd%d_pos%d" % c[:5])
def test_head_attention_decode(case):
    """xqhip_attn_decode_head (one block per query head, no merge kernel)
    against the oracle and against xqhip_attn_decode on its own copy of the
    caches, for two consecutive positions."""
    nq, nkv, hd, rd, pos, max_ctx, gated = case
    theta, eps = 1e7, 1e-6
    print(f"head attention case {case}", flush=True)
    assert pos + 2 <= max_ctx
    qsrc, k, v, qn, kn, kc, vc = attn_layer_inputs(nq, nkv, hd, pos, seed=pos + 3, gated=gated)
    tab = np.empty(max_ctx * rd, np.float32)
    xb.ck(xb.hip().xqhip_rope_table(theta, rd, max_ctx, xb.ptr(tab)))
    kcache = np.zeros((max_ctx, nkv, hd), np.float16)
    vcache = np.zeros((max_ctx, nkv, hd), np.float16)
    kcache[:pos], vcache[:pos] = kc, vc
    kd, vd = dev(kcache), dev(vcache)    # per-head kernel
    kd2, vd2 = dev(kcache), dev(vcache)  # slot kernel + merge
    qn_d, kn_d, tab_d = dev(qn), dev(kn), dev(tab)
    ws = dev(np.zeros(xb.hip().xqhip_gqa_workspace_bytes(nq, nkv, hd), np.uint8))
    out, out2 = xb.DeviceBuffer(nq * hd * 4), xb.DeviceBuffer(nq * hd * 4)
    rng = np.random.default_rng(pos + 1)
    for step in range(2):
        p = pos + step
        if step:
            qsrc = rng.normal(0, 1, qsrc.size).astype(np.float32)
            k = rng.normal(0, 1, k.size).astype(np.float32)
            v = rng.normal(0, 1, v.size).astype(np.float32)
        qs_d, k_d, v_d = dev(qsrc), dev(k), dev(v)
        pos_d = dev(np.array([p], np.int32))
        xb.ck(xb.hip().xqhip_attn_decode_head(qs_d.ptr, k_d.ptr, v_d.ptr, int(gated), nq, nkv, hd, rd, qn_d.ptr,
                                              kn_d.ptr, eps, tab_d.ptr, pos_d.ptr, kd.ptr, vd.ptr, out.ptr, None))
        xb.ck(xb.hip().xqhip_attn_decode(qs_d.ptr, k_d.ptr, v_d.ptr, int(gated), nq, nkv, hd, rd, qn_d.ptr, kn_d.ptr,
                                         eps, tab_d.ptr, pos_d.ptr, kd2.ptr, vd2.ptr, max_ctx, out2.ptr, ws.ptr, None))
        kc_got = kd.download(np.float16, max_ctx * nkv * hd).reshape(max_ctx, nkv, hd)
        vc_got = vd.download(np.float16, max_ctx * nkv * hd).reshape(max_ctx, nkv, hd)
        assert np.array_equal(kc_got[:pos], kc) and np.array_equal(vc_got[:pos], vc)  # earlier slots untouched
        assert not kc_got[p + 1:].any() and not vc_got[p + 1:].any()                  # later slots untouched
        assert np.array_equal(vc_got[p].reshape(-1), v.astype(np.float16))
        kc2 = kd2.download(np.float16, max_ctx * nkv * hd).reshape(max_ctx, nkv, hd)
        assert np.array_equal(kc_got, kc2)  # the same fp16 append as the slot kernel
        kk, want = oracle_attention_step(qsrc, k, gated, qn, kn, nq, nkv, hd, rd, p, theta, eps, kc_got, vc_got)
        close(kc_got[p].reshape(-1).astype(np.float32), kk, f"appended k pos {p}", atol=2e-3, rtol=1e-3)
        got = out.download(np.float32, nq * hd)
        close(got, want, f"head attention pos {p}")
        close(got, out2.download(np.float32, nq * hd), f"head vs slot kernel pos {p}", atol=1e-5, rtol=1e-4)


def test_head_attention_rejects_other_head_sizes():
    z = dev(np.zeros(64, np.float32))
    rc = xb.hip().xqhip_attn_decode_head(z.ptr, z.ptr, z.ptr, 1, 8, 2, 64, 32, z.ptr, z.ptr, 1e-6, z.ptr, z.ptr,
                                         z.ptr, z.ptr, z.ptr, None)
    assert rc == -1 and b"head_dim 128" in xb.hip().xqhip_last_error()  # XQHIP_EINVAL


# The per-head attention split over 1, 2 or 4 context ranges per query head
# and merged by the last block of each head: the new token alone, fewer cached
# positions than splits (empty ranges), the 512-token point, a range of exactly
# one 1024-token pass and ranges past it (up to 20000 cached positions), group
# sizes 1, 4 and 8, gated and not.
PART_CASES = [(32, 8, 128, 32, 0, 64, True), (32, 8, 128, 32, 2, 64, True), (32, 8, 128, 32, 511, 1024, True),
              (32, 8, 128, 64, 540, 1024, False), (16, 2, 128, 32, 1023, 2048, True),
              (8, 8, 128, 128, 4095, 4160, True), (4, 1, 128, 32, 9000, 9216, False),
              (4, 1, 128, 32, 20000, 20480, True)]


@pytest.mark.parametrize("splits", [1, 2, 4, 8])
@pytest.mark.parametrize("case", PART_CASES, ids=lambda c: "nq%d_nkv%d_hd%d_rd%d_pos%d" % c[:5])
def test_split_attention_merged_in_kernel(case, splits):
    """xqhip_attn_decode_split (partials merged by the last block of each query
    head) against the oracle and against xqhip_attn_decode_head on its own copy
    of the caches: bit-identical with one split while the context fits one
    pass of both kernels (the split kernel's passes are 512 positions, the
    per-head kernel's 1024: past 512 the running maximum is merged at
    another point), within 1e-5 otherwise; three consecutive positions on
    one workspace, zero-filled once (each call must leave its counters at
    zero)."""
    nq, nkv, hd, rd, pos, max_ctx, gated = case
    theta, eps = 1e7, 1e-6
    print(f"split attention case {case} splits {splits}", flush=True)
    assert pos + 3 <= max_ctx
    qsrc, k, v, qn, kn, kc, vc = attn_layer_inputs(nq, nkv, hd, pos, seed=pos + 13, gated=gated)
    tab = np.empty(max_ctx * rd, np.float32)
    xb.ck(xb.hip().xqhip_rope_table(theta, rd, max_ctx, xb.ptr(tab)))
    kcache = np.zeros((max_ctx, nkv, hd), np.float16)
    vcache = np.zeros((max_ctx, nkv, hd), np.float16)
    kcache[:pos], vcache[:pos] = kc, vc
    kd, vd = dev(kcache), dev(vcache)    # split kernel
    kd2, vd2 = dev(kcache), dev(vcache)  # single-block kernel
    qn_d, kn_d, tab_d = dev(qn), dev(kn), dev(tab)
    nbytes = xb.hip().xqhip_attn_split_workspace_bytes(nq)
    ws = dev(np.zeros(nbytes, np.uint8))
    out, out2 = xb.DeviceBuffer(nq * hd * 4), xb.DeviceBuffer(nq * hd * 4)
    rng = np.random.default_rng(pos + 4)
    for step in range(3):
        p = pos + step
        if step:
            qsrc = rng.normal(0, 1, qsrc.size).astype(np.float32)
            k = rng.normal(0, 1, k.size).astype(np.float32)
            v = rng.normal(0, 1, v.size).astype(np.float32)
        qs_d, k_d, v_d = dev(qsrc), dev(k), dev(v)
        pos_d = dev(np.array([p], np.int32))
        xb.ck(xb.hip().xqhip_attn_decode_split(qs_d.ptr, k_d.ptr, v_d.ptr, int(gated), nq, nkv, hd, rd, qn_d.ptr,
                                               kn_d.ptr, eps, tab_d.ptr, pos_d.ptr, kd.ptr, vd.ptr, splits, ws.ptr,
                                               out.ptr, None))
        xb.ck(xb.hip().xqhip_attn_decode_head(qs_d.ptr, k_d.ptr, v_d.ptr, int(gated), nq, nkv, hd, rd, qn_d.ptr,
                                              kn_d.ptr, eps, tab_d.ptr, pos_d.ptr, kd2.ptr, vd2.ptr, out2.ptr, None))
        kc_got = kd.download(np.float16, max_ctx * nkv * hd).reshape(max_ctx, nkv, hd)
        vc_got = vd.download(np.float16, max_ctx * nkv * hd).reshape(max_ctx, nkv, hd)
        assert np.array_equal(kc_got, kd2.download(np.float16, max_ctx * nkv * hd).reshape(max_ctx, nkv, hd))
        assert np.array_equal(vc_got, vd2.download(np.float16, max_ctx * nkv * hd).reshape(max_ctx, nkv, hd))
        assert np.array_equal(vc_got[p].reshape(-1), v.astype(np.float16))
        assert not kc_got[p + 1:].any() and not vc_got[p + 1:].any()  # later slots untouched
        _, want = oracle_attention_step(qsrc, k, gated, qn, kn, nq, nkv, hd, rd, p, theta, eps, kc_got, vc_got)
        got, ref = out.download(np.float32, nq * hd), out2.download(np.float32, nq * hd)
        close(got, want, f"split attention pos {p}")
        if splits == 1 and p < 512:
            assert np.array_equal(got, ref), "one split must match the single-block kernel bit for bit"
        else:
            close(got, ref, f"split vs single-block pos {p}", atol=1e-5, rtol=1e-5)
    cnt = ws.download(np.uint32, nbytes // 4)[xb.ATTN_MAX_SPLITS * nq * xb.ATTN_PART_STRIDE:]
    assert not cnt.any()  # the counters are back at zero


def test_split_attention_rejections():
    z = dev(np.zeros(64, np.float32))
    assert xb.hip().xqhip_attn_split_workspace_bytes(0) == 0
    ws = dev(np.zeros(xb.hip().xqhip_attn_split_workspace_bytes(32), np.uint8))
    for splits, hd in ((0, 128), (9, 128), (2, 64)):
        rc = xb.hip().xqhip_attn_decode_split(z.ptr, z.ptr, z.ptr, 1, 32, 8, hd, 32, z.ptr, z.ptr, 1e-6, z.ptr, z.ptr,
                                              z.ptr, z.ptr, splits, ws.ptr, z.ptr, None)
        assert rc == -1  # XQHIP_EINVAL
    assert b"head_dim 128" in xb.hip().xqhip_last_error()


@pytest.mark.parametrize("ctx", [1, 2, 15, 16, 17, 100])
def test_gqa_short_contexts(ctx):
    nq, nkv, hd = 4, 2, 8
    rng = np.random.default_rng(ctx)
    q = rng.normal(0, 1, nq * hd).astype(np.float32)
    kc = rng.normal(0, 1, (ctx, nkv, hd)).astype(np.float16)
    vc = rng.normal(0, 1, (ctx, nkv, hd)).astype(np.float16)
    gate = rng.normal(0, 1, nq * hd).astype(np.float32)
    att = np.empty(nq * hd, np.float32)
    kf, vf = kc.astype(np.float32).reshape(-1), vc.astype(np.float32).reshape(-1)
    O().orc_attention_model(ob.p(q), ob.p(kf), ob.p(vf), ctx, nkv, nq, hd, ob.p(att))
    want = att * np.array([O().orc_sigmoid(float(g)) for g in gate], np.float32)
    ws = xb.DeviceBuffer(xb.hip().xqhip_gqa_workspace_bytes(nq, nkv, hd))
    ws.zero()
    out = xb.DeviceBuffer(nq * hd * 4)
    xb.ck(xb.hip().xqhip_gqa_decode(dev(q).ptr, dev(kc).ptr, dev(vc).ptr, dev(gate).ptr, nq, nkv, hd, 128,
                                    dev(np.array([ctx - 1], np.int32)).ptr, out.ptr, ws.ptr, None))
    close(out.download(np.float32, nq * hd), want, f"gqa ctx={ctx}")


def linear_inputs(lk_n=16, lv_n=32, lk_hd=128, lv_hd=128, ks=4, seed=9):
    rng = np.random.default_rng(seed)
    conv_dim = 2 * lk_n * lk_hd + lv_n * lv_hd
    mixed = rng.normal(0, 1, conv_dim).astype(np.float32)
    state = rng.normal(0, 0.5, conv_dim * (ks - 1)).astype(np.float32)
    w = rng.normal(0, 0.5, conv_dim * ks).astype(np.float32)
    return mixed, state, w


@pytest.mark.parametrize("shape", [(16, 32, 128, 128, 4), (1, 2, 2, 2, 2), (3, 6, 64, 32, 3)])
def test_linear_conv_and_gated_delta(shape):
    lk_n, lv_n, lk_hd, lv_hd, ks = shape
    mixed, cstate, cw = linear_inputs(lk_n, lv_n, lk_hd, lv_hd, ks)
    conv_dim = mixed.size
    # oracle conv + l2 norm (custom_model.cpp:986-1047)
    st_o = cstate.copy()
    conv_o = np.empty(conv_dim, np.float32)
    O().orc_conv1d_step(ob.p(mixed), ob.p(st_o), ob.p(cw), conv_dim, ks, ob.p(conv_o))
    qv = conv_o[: lk_n * lk_hd].copy()
    kv = conv_o[lk_n * lk_hd: 2 * lk_n * lk_hd].copy()
    O().orc_l2norm_heads(ob.p(qv), lk_n, lk_hd)
    O().orc_l2norm_heads(ob.p(kv), lk_n, lk_hd)
    conv_o[: lk_n * lk_hd] = qv
    conv_o[lk_n * lk_hd: 2 * lk_n * lk_hd] = kv
    # device conv
    md, sd, wd = dev(mixed), dev(cstate), dev(cw)
    cout = xb.DeviceBuffer(conv_dim * 4)
    xb.ck(xb.hip().xqhip_linear_conv(md.ptr, sd.ptr, wd.ptr, lk_n, lk_hd, lv_n, lv_hd, ks, cout.ptr, None))
    conv_g = cout.download(np.float32, conv_dim)
    close(conv_g, conv_o, "conv1d+silu+l2norm", atol=1e-5, rtol=1e-5)
    assert np.array_equal(sd.download(np.float32, cstate.size), st_o)  # history shift is exact
    # gated delta: decay in (0,1), beta ~U(0,1)
    rng = np.random.default_rng(11)
    beta_t = rng.uniform(0, 1, lv_n)
    b = np.log(beta_t / (1 - beta_t)).astype(np.float32)
    a = rng.normal(0, 1, lv_n).astype(np.float32)
    a_log = rng.normal(-1, 0.5, lv_n).astype(np.float32)
    dt = rng.normal(0, 0.5, lv_n).astype(np.float32)
    S0 = rng.normal(0, 0.1, lv_n * lk_hd * lv_hd).astype(np.float32)
    S_o = S0.copy()
    out_o = np.zeros(lv_n * lv_hd, np.float32)
    factor = max(1, lv_n // max(1, lk_n))
    for vh in range(lv_n):
        kh = min(lk_n - 1, vh // factor)
        beta = O().orc_sigmoid(float(b[vh]))
        gate = np.float32(-np.exp(np.float32(a_log[vh]))) * np.float32(O().orc_softplus(float(a[vh] + dt[vh])))
        qh = np.ascontiguousarray(conv_o[kh * lk_hd:(kh + 1) * lk_hd])
        khv = np.ascontiguousarray(conv_o[lk_n * lk_hd + kh * lk_hd: lk_n * lk_hd + (kh + 1) * lk_hd])
        vv = np.ascontiguousarray(conv_o[2 * lk_n * lk_hd + vh * lv_hd: 2 * lk_n * lk_hd + (vh + 1) * lv_hd])
        Sv = S_o[vh * lk_hd * lv_hd:(vh + 1) * lk_hd * lv_hd]
        ov = np.zeros(lv_hd, np.float32)
        O().orc_gated_delta(ob.p(qh), ob.p(khv), ob.p(vv), beta, float(gate), lk_hd, lv_hd, ob.p(Sv), ob.p(ov))
        S_o[vh * lk_hd * lv_hd:(vh + 1) * lk_hd * lv_hd] = Sv
        out_o[vh * lv_hd:(vh + 1) * lv_hd] = ov
    Sd = dev(S0)
    od = xb.DeviceBuffer(lv_n * lv_hd * 4)
    xb.ck(xb.hip().xqhip_gated_delta(dev(conv_o).ptr, dev(a).ptr, dev(b).ptr, dev(a_log).ptr, dev(dt).ptr, Sd.ptr,
                                     lk_n, lv_n, lk_hd, lv_hd, od.ptr, None))
    close(od.download(np.float32, lv_n * lv_hd), out_o, "gated delta out", atol=1e-4, rtol=1e-4)
    close(Sd.download(np.float32, S0.size), S_o, "gated delta state", atol=1e-5, rtol=1e-4)


def oracle_linear_step(mixed, st, cw, a, b, a_log, dt, S, shape):
    """conv1d + SiLU + q/k L2 norm + gated delta for one position, in place on st and S."""
    lk_n, lv_n, lk_hd, lv_hd, ks = shape
    conv_dim = mixed.size
    conv_o = np.empty(conv_dim, np.float32)
    O().orc_conv1d_step(ob.p(mixed), ob.p(st), ob.p(cw), conv_dim, ks, ob.p(conv_o))
    qv = conv_o[: lk_n * lk_hd].copy()
    kv = conv_o[lk_n * lk_hd: 2 * lk_n * lk_hd].copy()
    O().orc_l2norm_heads(ob.p(qv), lk_n, lk_hd)
    O().orc_l2norm_heads(ob.p(kv), lk_n, lk_hd)
    out = np.zeros(lv_n * lv_hd, np.float32)
    factor = max(1, lv_n // max(1, lk_n))
    for vh in range(lv_n):
        kh = min(lk_n - 1, vh // factor)
        beta = O().orc_sigmoid(float(b[vh]))
        gate = np.float32(-np.exp(np.float32(a_log[vh]))) * np.float32(O().orc_softplus(float(a[vh] + dt[vh])))
        qh = np.ascontiguousarray(qv[kh * lk_hd:(kh + 1) * lk_hd])
        kh_v = np.ascontiguousarray(kv[kh * lk_hd:(kh + 1) * lk_hd])
        vv = np.ascontiguousarray(conv_o[2 * lk_n * lk_hd + vh * lv_hd: 2 * lk_n * lk_hd + (vh + 1) * lv_hd])
        Sv = np.ascontiguousarray(S[vh * lk_hd * lv_hd:(vh + 1) * lk_hd * lv_hd])
        ov = np.zeros(lv_hd, np.float32)
        O().orc_gated_delta(ob.p(qh), ob.p(kh_v), ob.p(vv), beta, float(gate), lk_hd, lv_hd, ob.p(Sv), ob.p(ov))
        S[vh * lk_hd * lv_hd:(vh + 1) * lk_hd * lv_hd] = Sv
        out[vh * lv_hd:(vh + 1) * lv_hd] = ov
    return out


@pytest.mark.parametrize("shape", [(16, 32, 128, 128, 4), (1, 2, 2, 2, 2), (3, 6, 64, 32, 3), (2, 2, 256, 40, 4),
                                   (2, 4, 64, 64, 5), (2, 4, 32, 32, 8)])
def test_fused_linear_attn_step_two_positions(shape):
    """xqhip_linear_attn_step against the oracle's conv + L2 norm + gated delta on
    two consecutive positions, which exercises both halves of the parity-
    double-buffered conv history."""
    lk_n, lv_n, lk_hd, lv_hd, ks = shape
    rng = np.random.default_rng(21)
    mixed0, cstate, cw = linear_inputs(lk_n, lv_n, lk_hd, lv_hd, ks, seed=31)
    mixed1 = rng.normal(0, 1, mixed0.size).astype(np.float32)
    hist = cstate.size
    beta_t = rng.uniform(0, 1, lv_n)
    b = np.log(beta_t / (1 - beta_t)).astype(np.float32)
    a = rng.normal(0, 1, lv_n).astype(np.float32)
    a_log = rng.normal(-1, 0.5, lv_n).astype(np.float32)
    dt = rng.normal(0, 0.5, lv_n).astype(np.float32)
    S0 = rng.normal(0, 0.1, lv_n * lk_hd * lv_hd).astype(np.float32)
    st_o, S_o = cstate.copy(), S0.copy()
    want0 = oracle_linear_step(mixed0, st_o, cw, a, b, a_log, dt, S_o, shape)
    want1 = oracle_linear_step(mixed1, st_o, cw, a, b, a_log, dt, S_o, shape)
    pos = 5  # odd: the first step reads copy 1
    two = np.concatenate([np.full(hist, 777.0, np.float32), cstate])
    sd, Sd, wd = dev(two), dev(S0), dev(cw)
    ad, bd, ald, dtd = dev(a), dev(b), dev(a_log), dev(dt)
    outs = []
    for step, mixed in enumerate([mixed0, mixed1]):
        md, pd = dev(mixed), dev(np.array([pos + step], np.int32))
        od = xb.DeviceBuffer(lv_n * lv_hd * 4)
        xb.ck(xb.hip().xqhip_linear_attn_step(md.ptr, sd.ptr, wd.ptr, ad.ptr, bd.ptr, ald.ptr, dtd.ptr, Sd.ptr, lk_n,
                                              lk_hd, lv_n, lv_hd, ks, pd.ptr, od.ptr, None))
        outs.append(od.download(np.float32, lv_n * lv_hd))
    close(outs[0], want0, "fused linear step, first position", atol=1e-4, rtol=1e-4)
    close(outs[1], want1, "fused linear step, second position", atol=1e-4, rtol=1e-4)
    close(Sd.download(np.float32, S0.size), S_o, "fused linear step state", atol=1e-5, rtol=1e-4)
    got_hist = sd.download(np.float32, 2 * hist)
    assert np.array_equal(got_hist[hist:], st_o)  # the second step wrote copy 1 again; shifts are exact


@pytest.mark.parametrize("shape", [(16, 32, 128, 128, 4), (3, 6, 64, 32, 3), (2, 2, 256, 40, 4)])
def test_linear_step_act_matches_step_and_activates_gate(shape):
    """xqhip_linear_attn_step_act: bit-identical outputs, state and conv history
    to xqhip_linear_attn_step, and the gate vector replaced by silu(gate); the
    gated-norm GEMV on that activated gate (XQHIP_PRO_GATED_HEAD_ACT) gives the
    XQHIP_PRO_GATED_HEAD result on the raw gate bit for bit, and both match the
    oracle's applyGatedHeadRms + GEMV (custom_model.cpp:329-349)."""
    lk_n, lv_n, lk_hd, lv_hd, ks = shape
    rng = np.random.default_rng(41)
    mixed, cstate, cw = linear_inputs(lk_n, lv_n, lk_hd, lv_hd, ks, seed=43)
    hist = cstate.size
    a = rng.normal(0, 1, lv_n).astype(np.float32)
    b = rng.normal(0, 1, lv_n).astype(np.float32)
    a_log = rng.normal(-1, 0.5, lv_n).astype(np.float32)
    dt = rng.normal(0, 0.5, lv_n).astype(np.float32)
    S0 = rng.normal(0, 0.1, lv_n * lk_hd * lv_hd).astype(np.float32)
    z = rng.normal(0, 2, lv_n * lv_hd).astype(np.float32)
    two = np.concatenate([cstate, np.full(hist, 5.0, np.float32)])
    md, wd, ad, bd, ald, dtd = dev(mixed), dev(cw), dev(a), dev(b), dev(a_log), dev(dt)
    pd = dev(np.array([8], np.int32))
    res = []
    for act in (False, True):
        sd, Sd, zd = dev(two), dev(S0), dev(z)
        od = xb.DeviceBuffer(lv_n * lv_hd * 4)
        args = (md.ptr, sd.ptr, wd.ptr, ad.ptr, bd.ptr, ald.ptr, dtd.ptr, Sd.ptr, lk_n, lk_hd, lv_n, lv_hd, ks, pd.ptr,
                od.ptr)
        if act:
            xb.ck(xb.hip().xqhip_linear_attn_step_act(*args, zd.ptr, None))
        else:
            xb.ck(xb.hip().xqhip_linear_attn_step(*args, None))
        res.append((od.download(np.float32, lv_n * lv_hd), Sd.download(np.float32, S0.size),
                    sd.download(np.float32, 2 * hist), zd))
    (o0, s0, h0, z_raw), (o1, s1, h1, z_act) = res
    assert np.array_equal(o0, o1) and np.array_equal(s0, s1) and np.array_equal(h0, h1)
    assert np.array_equal(z_raw.download(np.float32, z.size), z)  # the plain step leaves the gate alone
    zz = z.astype(np.float64)
    close(z_act.download(np.float32, z.size), zz / (1 + np.exp(-zz)), "activated gate", atol=1e-6, rtol=1e-6)
    # the output projection of the step output, gate raw (silu in the prologue) or activated
    if lv_hd % 8 or (lv_hd // 8) & (lv_hd // 8 - 1):
        return  # the tiled GEMV's gated prologue needs head_dim / 8 a power of two
    hidden = 256
    q = w4_matrix(hidden, lv_n * lv_hd, 17)
    w4 = xb.DeviceW4(q.packed, q.scales, q.zeros, q.rows, q.cols)
    nw = dev(rng.normal(1, 0.1, lv_hd).astype(np.float32))
    xo = dev(o0)
    ys = []
    for mode, gate in ((xb.PRO_GATED_HEAD, z_raw), (xb.PRO_GATED_HEAD_ACT, z_act)):
        y = xb.DeviceBuffer(hidden * 4)
        pro = xb.prologue(mode, nw, gate, head_dim=lv_hd, eps=1e-6)
        xb.ck(xb.hip().xqhip_gemv_w4a16(w4.ref, xo.ptr, xb.F32, ctypes.byref(pro), y.ptr, xb.F32, xb.EPI_STORE, None))
        ys.append(y.download(np.float32, hidden))
    assert np.array_equal(ys[0], ys[1])
    normed = np.empty_like(o0)
    O().orc_gated_head_rms(ob.p(o0), ob.p(nw.download(np.float32, lv_hd)), ob.p(z), lv_n, lv_hd, 1e-6, ob.p(normed))
    close(ys[1], ob.gemv(q, normed), "gated-norm GEMV on the activated gate")
    # the prefill GEMM prepares its own gate: the activated form is refused there
    ws = xb.DeviceBuffer(xb.hip().xqhip_gemm_workspace_bytes(4, lv_n * lv_hd, hidden))
    pro = xb.prologue(xb.PRO_GATED_HEAD_ACT, nw, z_act, head_dim=lv_hd, eps=1e-6)
    assert xb.hip().xqhip_gemm_w4a16(w4.ref, xo.ptr, 1, lv_n * lv_hd, ctypes.byref(pro), lv_n * lv_hd, y.ptr,
                                     hidden, xb.EPI_STORE, ws.ptr, ws.nbytes, None) == -1


def test_rmsnorm_kernel():
    rng = np.random.default_rng(3)
    x = rng.normal(0, 5, 4096).astype(np.float32)
    w = rng.normal(1, 0.1, 4096).astype(np.float32)
    want = np.empty_like(x)
    O().orc_rmsnorm(ob.p(x), ob.p(w), 4096, 1e-6, ob.p(want))
    y = xb.DeviceBuffer(4096 * 4)
    xb.ck(xb.hip().xqhip_rmsnorm(dev(x).ptr, dev(w).ptr, 4096, 1e-6, y.ptr, None))
    close(y.download(np.float32, 4096), want, "rmsnorm", atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("fill", [1.0e30, -1.0e30])
@pytest.mark.parametrize("kernel,pos", [("head", 511), ("head", 540), ("split", 511), ("split", 1100)])
def test_attention_ignores_stale_lds(kernel, pos, fill):
    """Regression guard for a fixed race: the per-head / split decode attention
    must read no LDS word before its own block wrote it (the new token's score
    once entered the pass maximum before the barrier that publishes it).  The
    LDS of every CU is filled with a huge value right before the launch
    (xqhip_lds_fill; LDS keeps its contents between kernels), then the output
    is compared with the oracle (custom_model.cpp:840-951) at 32q/8kv d128."""
    nq, nkv, hd, rd, gated = 32, 8, 128, 32, True
    theta, eps, max_ctx = 1e7, 1e-6, 2048
    print(f"stale-LDS attention case {kernel} pos {pos} fill {fill:g}", flush=True)
    qsrc, k, v, qn, kn, kc, vc = attn_layer_inputs(nq, nkv, hd, pos, seed=pos + 29, gated=gated)
    tab = np.empty(max_ctx * rd, np.float32)
    xb.ck(xb.hip().xqhip_rope_table(theta, rd, max_ctx, xb.ptr(tab)))
    kcache = np.zeros((max_ctx, nkv, hd), np.float16)
    vcache = np.zeros((max_ctx, nkv, hd), np.float16)
    kcache[:pos], vcache[:pos] = kc, vc
    kd, vd = dev(kcache), dev(vcache)
    qs_d, k_d, v_d, qn_d, kn_d, tab_d = dev(qsrc), dev(k), dev(v), dev(qn), dev(kn), dev(tab)
    pos_d = dev(np.array([pos], np.int32))
    out = xb.DeviceBuffer(nq * hd * 4)
    ws = dev(np.zeros(xb.hip().xqhip_attn_split_workspace_bytes(nq), np.uint8))
    xb.ck(xb.hip().xqhip_device_synchronize())
    xb.ck(xb.hip().xqhip_lds_fill(fill, None))
    if kernel == "head":
        xb.ck(xb.hip().xqhip_attn_decode_head(qs_d.ptr, k_d.ptr, v_d.ptr, int(gated), nq, nkv, hd, rd, qn_d.ptr,
                                              kn_d.ptr, eps, tab_d.ptr, pos_d.ptr, kd.ptr, vd.ptr, out.ptr, None))
    else:
        xb.ck(xb.hip().xqhip_attn_decode_split(qs_d.ptr, k_d.ptr, v_d.ptr, int(gated), nq, nkv, hd, rd, qn_d.ptr,
                                               kn_d.ptr, eps, tab_d.ptr, pos_d.ptr, kd.ptr, vd.ptr, 8, ws.ptr,
                                               out.ptr, None))
    kc_got = kd.download(np.float16, max_ctx * nkv * hd).reshape(max_ctx, nkv, hd)
    vc_got = vd.download(np.float16, max_ctx * nkv * hd).reshape(max_ctx, nkv, hd)
    _, want = oracle_attention_step(qsrc, k, gated, qn, kn, nq, nkv, hd, rd, pos, theta, eps, kc_got, vc_got)
    close(out.download(np.float32, nq * hd), want, f"{kernel} attention after an LDS fill, pos {pos}")
