"""Pins the oracle against the compiled reference (oracle/_ref/libxqref.so, built
from the reference's own customlib sources by oracle/Makefile): every kernel
and the whole model forward must agree bit-for-bit on the same host.  Skipped
where the reference checkout was not available to build _ref (the committed
golden fixtures in tests/golden/ cover the same cases then).  CPU only."""
import ctypes

import numpy as np
import pytest

import oracle_bind as ob
import xqbind as xb
from synth import w4_matrix
from tiny_model import SMALL, write_tiny_model

pytestmark = pytest.mark.skipif(not ob.ref_available(), reason="oracle/_ref not built (reference checkout absent)")


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def reference_pool_safe(rows, min_rows):
    """The reference WorkerPool wakes every worker for each task; when a call
    uses fewer threads than the pool, its completion counter can run past zero
    and the caller never returns (xq_gemv_w4a16_neon.cpp:146-207).  Calls with
    one thread or with the whole pool are safe."""
    import os
    pool = min(8, os.cpu_count() or 1)
    want = min(pool, max(1, -(-rows // min_rows)))
    return want == 1 or want == pool


@pytest.mark.parametrize("rows,cols,group,affine", [(4096, 4096, 64, 0), (12288, 4096, 64, 0), (300, 12288, 64, 0),
                                                    (7, 24, 8, 0), (33, 100, 10, 1), (40000, 256, 64, 1)])
def test_gemv_bit_exact(rows, cols, group, affine):
    q = w4_matrix(rows, cols, rows + cols, group=group, affine=affine)
    x = np.random.default_rng(1).normal(0, 1, cols).astype(np.float32)
    min_rows = 128 if cols >= 2048 else 512
    if rows < 2 * min_rows or reference_pool_safe(rows, min_rows):
        assert np.array_equal(bits(ob.gemv(q, x)), bits(ob.gemv(q, x, ob.ref(), "ref_gemv_w4a16")))
    assert np.array_equal(bits(ob.gemv(q, x, fn="orc_gemv_textbook")),
                          bits(ob.gemv(q, x, ob.ref(), "ref_gemv_textbook")))
    if rows < 8192 or reference_pool_safe(rows, 4096):
        assert ob.gemv_argmax(q, x) == ob.gemv_argmax(q, x, ob.ref(), "ref_gemv_w4a16_argmax")


def test_quantizer_bit_exact():
    w = (np.sin(np.arange(64 * 200, dtype=np.float32) * np.float32(0.37)) * np.float32(0.9)).astype(np.float32)
    a = ob.quantize_lowbit(w, 64, 200, 4, 64)
    b = ob.quantize_lowbit(w, 64, 200, 4, 64, ob.ref(), "ref_quantize_lowbit")
    assert np.array_equal(a.packed, b.packed) and np.array_equal(bits(a.scales), bits(b.scales))
    assert np.array_equal(bits(a.zeros), bits(b.zeros))


def test_vector_kernels_bit_exact():
    rng = np.random.default_rng(2)
    o, r = ob.oracle(), ob.ref()
    x = rng.normal(0, 3, 4096).astype(np.float32)
    w = rng.normal(1, 0.1, 4096).astype(np.float32)
    y1, y2 = np.empty_like(x), np.empty_like(x)
    o.orc_rmsnorm(ob.p(x), ob.p(w), 4096, 1e-6, ob.p(y1))
    r.ref_rmsnorm(ob.p(x), ob.p(w), 4096, 1e-6, ob.p(y2))
    assert np.array_equal(bits(y1), bits(y2))
    q = rng.normal(0, 1, 16 * 256).astype(np.float32)
    k = rng.normal(0, 1, 16 * 256).astype(np.float32)
    q1, k1, q2, k2 = q.copy(), k.copy(), q.copy(), k.copy()
    o.orc_rope_full(ob.p(q1), ob.p(k1), 16, 256, 512, 1e7)
    r.ref_rope(ob.p(q2), ob.p(k2), 16, 256, 512, 1e7)
    assert np.array_equal(bits(q1), bits(q2)) and np.array_equal(bits(k1), bits(k2))
    ctx, kvh, qh, hd = 64, 4, 16, 64
    qq = rng.normal(0, 1, qh * hd).astype(np.float32)
    kc = rng.normal(0, 1, ctx * kvh * hd).astype(np.float32)
    vc = rng.normal(0, 1, ctx * kvh * hd).astype(np.float32)
    a1, a2 = np.empty(qh * hd, np.float32), np.empty(qh * hd, np.float32)
    o.orc_attention_ref(ob.p(qq), ob.p(kc), ob.p(vc), ctx, kvh, qh, hd, ob.p(a1))
    r.ref_attention(ob.p(qq), ob.p(kc), ob.p(vc), ctx, kvh, qh, hd, ob.p(a2))
    assert np.array_equal(bits(a1), bits(a2))
    S = rng.normal(0, 0.1, 128 * 128).astype(np.float32)
    s1, s2 = S.copy(), S.copy()
    v = rng.normal(0, 1, 128).astype(np.float32)
    d1, d2 = np.empty(128, np.float32), np.empty(128, np.float32)
    o.orc_gated_delta(ob.p(qq), ob.p(kc), ob.p(v), 0.3, -0.2, 128, 128, ob.p(s1), ob.p(d1))
    r.ref_gated_delta(ob.p(qq), ob.p(kc), ob.p(v), 0.3, -0.2, 128, 128, ob.p(s2), ob.p(d2))
    assert np.array_equal(bits(s1), bits(s2)) and np.array_equal(bits(d1), bits(d2))


def reference_session(model_dir):
    ref_abi = xb.bind_xq_abi(ctypes.CDLL(ob.REF_SO))
    s = xb.Session(model_dir, xb.options(backend=b"cpu"), lib=ref_abi)
    assert s.status == 0
    return s


@pytest.mark.parametrize("which", ["tiny_runtime_model", "small_synthetic"])
def test_model_forward_bit_exact(tmp_path, which):
    d = str(tmp_path / which)
    if which == "tiny_runtime_model":
        write_tiny_model(d)
        prompt, n_new = [1, 2, 3], 6
    else:
        xb.write_synth_model(d, **SMALL)
        prompt, n_new = [11, 4000, 7, 250, 3, 3, 99], 10
    om = ob.OracleModel(d)
    om.prefill(prompt)
    toks = [om.decode_one(len(prompt) + i) for i in range(n_new)]
    s = reference_session(d)
    st, out, m = s.generate(prompt, n_new)
    assert st == 0 and out.tolist() == toks
    st, h, n = s.hidden()
    assert np.array_equal(bits(om.hidden_state()), bits(h))
