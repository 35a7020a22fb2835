"""Decode chains (xqhip_chain_*): the projections between two non-GEMV ops of
runLayer (customlib/runtime/custom_model.cpp:1138-1256) in one persistent
launch with in-kernel hand-offs.  The chain's arithmetic is that of the
one-launch-per-GEMV path, so its outputs must equal xqhip_gemv_w4a16's on the
same operands bit for bit; those are pinned against the oracle by
test_gemv_gpu.py / test_configs_gpu.py, and one case here checks the oracle
directly too."""
import ctypes

import numpy as np
import pytest

import oracle_bind as ob
import xqbind as xb

pytestmark = pytest.mark.gpu
H = xb.hip()


def rand_matrix(rng, rows, cols, meta):
    """meta 2: zero 8 and fp16 scales (scale-only layout), 0: fp16 (scale, zero),
    1: fp32 (scale, zero) values fp16 cannot hold."""
    packed = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
    scales = np.abs(rng.normal(0, 0.02, rows * cols // 64)).astype(np.float32)
    zeros = np.full_like(scales, 8.0)
    if meta in (0, 2):
        scales = scales.astype(np.float16).astype(np.float32)
    if meta == 0:
        zeros = rng.integers(0, 16, scales.size).astype(np.float32)
    if meta == 1:
        zeros = rng.uniform(0, 15, scales.size).astype(np.float32)
    return packed, scales, zeros


def dev(a):
    return xb.DeviceBuffer.from_array(np.ascontiguousarray(a, np.float32))


class ChainCase:
    """A linear-attention layer's chain (out_proj with the gated head norm, gate/up
    with RMSNorm and SiLU*up, down with the residual add, the next input
    projection with RMSNorm) or a full-attention layer's (o_proj without a
    prologue).  `sep` runs the same ops as four GEMV launches."""

    def __init__(self, rng, hidden, inter, proj, gated, meta=2):
        self.hidden, self.inter, self.proj, self.gated = hidden, inter, proj, gated
        shapes = dict(out=(hidden, hidden), gu=(2 * inter, hidden), down=(hidden, inter), inp=(proj, hidden))
        self.m = {k: xb.DeviceW4(*rand_matrix(rng, r, c, meta), r, c) for k, (r, c) in shapes.items()}
        self.attn = rng.normal(0, 1, hidden).astype(np.float32)
        self.z = (rng.normal(0, 1, hidden) * 0.5).astype(np.float32)
        self.lin_norm = rng.normal(1, 0.1, 128).astype(np.float32)
        self.post_norm = rng.normal(1, 0.1, hidden).astype(np.float32)
        self.in_norm = rng.normal(1, 0.1, hidden).astype(np.float32)
        self.resid0 = rng.normal(0, 1, hidden).astype(np.float32)
        self.d = {k: dev(getattr(self, k)) for k in ("attn", "z", "lin_norm", "post_norm", "in_norm")}

    def ops(self, resid, proj):
        ops = (xb.ChainOp * 4)()
        for i, (k, epi, pro) in enumerate([("out", xb.EPI_ADD, xb.PRO_GATED_HEAD_ACT if self.gated else xb.PRO_NONE),
                                           ("gu", xb.EPI_SILU_PAIR, xb.PRO_RMS), ("down", xb.EPI_ADD, xb.PRO_NONE),
                                           ("inp", xb.EPI_STORE, xb.PRO_RMS)]):
            ops[i].w = ctypes.pointer(self.m[k].w)
            ops[i].epi, ops[i].pro, ops[i].eps = epi, pro, 1e-6
        if self.gated:
            ops[0].pro_w, ops[0].head_dim = self.d["lin_norm"].ptr, 128
            ops[0].gate = xb.ChainSrc(self.d["z"].ptr, 0, 0)
        ops[0].x = xb.ChainSrc(self.d["attn"].ptr, 0, 0)
        ops[0].res = xb.ChainSrc(resid.ptr, 0, 0)
        ops[1].pro_w, ops[1].x = self.d["post_norm"].ptr, xb.ChainSrc(None, 0, 0)
        ops[2].x, ops[2].res, ops[2].y_plain = xb.ChainSrc(None, 1, 0), xb.ChainSrc(None, 0, 0), resid.ptr
        ops[3].pro_w, ops[3].x, ops[3].y_plain = self.d["in_norm"].ptr, xb.ChainSrc(None, 2, 0), proj.ptr
        return ops

    def sep(self, resid, proj):
        ffn = xb.DeviceBuffer(self.inter * 4)
        g = xb.prologue(xb.PRO_GATED_HEAD_ACT, self.d["lin_norm"], self.d["z"], 128)
        xb.ck(H.xqhip_gemv_w4a16(self.m["out"].ref, self.d["attn"].ptr, xb.F32,
                                 ctypes.byref(g) if self.gated else None, resid.ptr, xb.F32, xb.EPI_ADD, None))
        r = xb.prologue(xb.PRO_RMS, self.d["post_norm"])
        xb.ck(H.xqhip_gemv_w4a16(self.m["gu"].ref, resid.ptr, xb.F32, ctypes.byref(r), ffn.ptr, xb.F32,
                                 xb.EPI_SILU_PAIR, None))
        xb.ck(H.xqhip_gemv_w4a16(self.m["down"].ref, ffn.ptr, xb.F32, None, resid.ptr, xb.F32, xb.EPI_ADD, None))
        r2 = xb.prologue(xb.PRO_RMS, self.d["in_norm"])
        xb.ck(H.xqhip_gemv_w4a16(self.m["inp"].ref, resid.ptr, xb.F32, ctypes.byref(r2), proj.ptr, xb.F32,
                                 xb.EPI_STORE, None))
        xb.ck(H.xqhip_device_synchronize())
        return resid.download(np.float32, self.hidden), proj.download(np.float32, self.proj)


def make_chain(ops, n):
    c = ctypes.c_void_p()
    xb.ck(H.xqhip_chain_create(ops, n, ctypes.byref(c)))
    return c


def run_chain(c, arena, sync, resid, proj, case):
    xb.ck(H.xqhip_chain_launch(c, arena.ptr, sync.ptr, None))
    xb.ck(H.xqhip_device_synchronize())
    err = ctypes.c_int()
    xb.ck(H.xqhip_chain_error(sync.ptr, ctypes.byref(err)))
    assert err.value == 0, "a hand-off wait gave up"
    return resid.download(np.float32, case.hidden), proj.download(np.float32, case.proj)


@pytest.mark.parametrize("gated,hidden,inter,proj", [(True, 4096, 12288, 12352), (False, 4096, 12288, 10240),
                                                     (True, 512, 960, 1344)])
def test_chain_equals_separate_gemvs(gated, hidden, inter, proj):
    """The 9B linear-attention and full-attention chains (hidden 4096, MLP 12288,
    input projections 12352 / 10240 rows) and a small one; three launches in a
    row on the same arena and sync block (each launch's records carry its own
    number, so stale records of the previous launch are never taken), every
    one bit-identical to the four GEMV launches."""
    rng = np.random.default_rng(hidden + proj)
    case = ChainCase(rng, hidden, inter, proj, gated)
    resid, proj_b = dev(case.resid0), xb.DeviceBuffer(proj * 4)
    c = make_chain(case.ops(resid, proj_b), 4)
    try:
        arena = xb.DeviceBuffer(H.xqhip_chain_arena_records(c) * 8)
        arena.zero()
        sync = xb.DeviceBuffer(H.xqhip_chain_sync_bytes())
        sync.zero()
        resid_s, proj_s = dev(case.resid0), xb.DeviceBuffer(proj * 4)
        for launch in range(3):
            want_r, want_p = case.sep(resid_s, proj_s)
            got_r, got_p = run_chain(c, arena, sync, resid, proj_b, case)
            assert np.array_equal(got_r, want_r), (launch, np.abs(got_r - want_r).max())
            assert np.array_equal(got_p, want_p), (launch, np.abs(got_p - want_p).max())
    finally:
        H.xqhip_chain_destroy(c)


@pytest.mark.parametrize("meta", [0, 1])
def test_chain_metadata_layouts(meta):
    """fp16 (scale, zero) and fp32 (scale, zero) matrices run through the same
    chain kernel (its metadata template), bit-identical to the GEMV launches."""
    rng = np.random.default_rng(40 + meta)
    case = ChainCase(rng, 512, 960, 1344, True, meta=meta)
    assert all(case.m[k].w.layout == (xb.LAYOUT_TILED64 if meta == 0 else xb.LAYOUT_TILED64_F32META)
               for k in case.m)
    resid, proj_b = dev(case.resid0), xb.DeviceBuffer(case.proj * 4)
    c = make_chain(case.ops(resid, proj_b), 4)
    try:
        arena = xb.DeviceBuffer(H.xqhip_chain_arena_records(c) * 8)
        arena.zero()
        sync = xb.DeviceBuffer(H.xqhip_chain_sync_bytes())
        sync.zero()
        want_r, want_p = case.sep(dev(case.resid0), xb.DeviceBuffer(case.proj * 4))
        got_r, got_p = run_chain(c, arena, sync, resid, proj_b, case)
        assert np.array_equal(got_r, want_r) and np.array_equal(got_p, want_p)
    finally:
        H.xqhip_chain_destroy(c)


def test_chain_single_gemv_matches_oracle():
    """One-op chain (RMSNorm prologue, store) against the oracle's GEMV
    (gemvW4A16Neon restated, xq_gemv_w4a16_neon.cpp:259-291) on the RMS-normed
    input (ref_rmsnorm.cpp:8-17), 1e-3 rel / 1e-2 abs."""
    rng = np.random.default_rng(5)
    rows, cols = 3000, 4096
    packed, scales, zeros = rand_matrix(rng, rows, cols, 2)
    w = xb.DeviceW4(packed, scales, zeros, rows, cols)
    x = rng.normal(0, 1, cols).astype(np.float32)
    nw = rng.normal(1, 0.1, cols).astype(np.float32)
    xd, nwd, y = dev(x), dev(nw), xb.DeviceBuffer(rows * 4)
    ops = (xb.ChainOp * 1)()
    ops[0].w = ctypes.pointer(w.w)
    ops[0].epi, ops[0].pro, ops[0].pro_w, ops[0].eps = xb.EPI_STORE, xb.PRO_RMS, nwd.ptr, 1e-6
    ops[0].x, ops[0].y_plain = xb.ChainSrc(xd.ptr, 0, 0), y.ptr
    c = make_chain(ops, 1)
    try:
        arena = xb.DeviceBuffer(H.xqhip_chain_arena_records(c) * 8)
        arena.zero()
        sync = xb.DeviceBuffer(H.xqhip_chain_sync_bytes())
        sync.zero()
        xb.ck(H.xqhip_chain_launch(c, arena.ptr, sync.ptr, None))
        got = y.download(np.float32, rows)
    finally:
        H.xqhip_chain_destroy(c)
    normed = np.empty(cols, np.float32)
    ob.oracle().orc_rmsnorm(ob.p(x), ob.p(nw), cols, 1e-6, ob.p(normed))
    want = ob.gemv(ob.Quantized(packed, scales, zeros, rows, cols), normed)
    err = np.abs(got.astype(np.float64) - want)
    assert (err <= 1e-2 + 1e-3 * np.abs(want)).all(), err.max()


def test_chain_create_rejects_unsupported():
    rng = np.random.default_rng(9)
    ok = xb.DeviceW4(*rand_matrix(rng, 128, 512, 2), 128, 512)
    generic = xb.DeviceW4(*rand_matrix(rng, 64, 512, 2), 64, 512, group=128)  # group 128: GENERIC layout
    fp16z = xb.DeviceW4(*rand_matrix(rng, 128, 512, 0), 128, 512)
    x = dev(np.ones(512, np.float32))
    c = ctypes.c_void_p()

    def one(w, src=None, epi=xb.EPI_STORE):
        ops = (xb.ChainOp * 2)()
        ops[0].w, ops[0].epi, ops[0].x = ctypes.pointer(ok.w), xb.EPI_STORE, xb.ChainSrc(x.ptr, 0, 0)
        ops[1].w, ops[1].epi = ctypes.pointer(w.w), epi
        ops[1].x = src if src is not None else xb.ChainSrc(x.ptr, 0, 0)
        return ops

    assert H.xqhip_chain_create(one(generic), 2, ctypes.byref(c)) == -1          # not TILED64
    assert H.xqhip_chain_create(one(fp16z), 2, ctypes.byref(c)) == -1            # metadata differs from op 0
    assert H.xqhip_chain_create(one(ok, xb.ChainSrc(None, 1, 0)), 2, ctypes.byref(c)) == -1  # source is not earlier
    assert H.xqhip_chain_create(one(ok, xb.ChainSrc(None, 0, 64)), 2, ctypes.byref(c)) == -1  # 64 + 512 > 128 rows
    assert H.xqhip_chain_create(one(ok, epi=7), 2, ctypes.byref(c)) == -1       # unknown epilogue
    assert H.xqhip_chain_create(None, 0, ctypes.byref(c)) == -1
