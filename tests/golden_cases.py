"""Input recipes shared by tests/golden/make_golden.py (which records the
compiled reference's outputs) and tests/test_golden.py (which checks the
oracle against them).  Every input is regenerated from a seed, so the fixture
holds outputs only."""
import ctypes
import tempfile

import numpy as np

import oracle_bind as ob
from synth import w4_matrix
from tiny_model import SMALL, write_tiny_model


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32).copy()


def gemv_cases():
    """Shapes the reference runs single-threaded (clear of its worker-pool race)."""
    cases = {}
    for name, rows, cols, group, affine in [("7x24_g8", 7, 24, 8, 0), ("33x100_g10_affine", 33, 100, 10, 1),
                                            ("200x4096_g64", 200, 4096, 64, 0), ("96x12288_g64", 96, 12288, 64, 0),
                                            ("64x640_g64_affine", 64, 640, 64, 1)]:
        q = w4_matrix(rows, cols, rows * 31 + cols, group=group, affine=affine)
        x = np.random.default_rng(rows + 7 * cols).normal(0, 1, cols).astype(np.float32)
        cases[name] = (q, x)
    return cases


def _rmsnorm(lib, prefix):
    rng = np.random.default_rng(11)
    x = rng.normal(0, 3, 4096).astype(np.float32)
    w = rng.normal(1, 0.1, 4096).astype(np.float32)
    y = np.empty_like(x)
    getattr(lib, prefix + "_rmsnorm")(ob.p(x), ob.p(w), 4096, ctypes.c_float(1e-6), ob.p(y))
    return bits(y)


def _rope(lib, prefix):
    rng = np.random.default_rng(12)
    q = rng.normal(0, 1, 4 * 128).astype(np.float32)
    k = rng.normal(0, 1, 4 * 128).astype(np.float32)
    fn = getattr(lib, "orc_rope_full" if prefix == "orc" else "ref_rope")
    qq, kk = q.copy(), k.copy()
    fn(ob.p(qq), ob.p(kk), 4, 128, 511, ctypes.c_float(1e7))  # (q, k, heads, head_dim, pos, theta)
    return np.concatenate([bits(qq), bits(kk)])


def _attention(lib, prefix):
    rng = np.random.default_rng(13)
    ctx, kvh, qh, hd = 48, 2, 8, 64
    q = rng.normal(0, 1, qh * hd).astype(np.float32)
    kc = rng.normal(0, 1, ctx * kvh * hd).astype(np.float32)
    vc = rng.normal(0, 1, ctx * kvh * hd).astype(np.float32)
    out = np.empty(qh * hd, np.float32)
    fn = getattr(lib, "orc_attention_ref" if prefix == "orc" else "ref_attention")
    fn(ob.p(q), ob.p(kc), ob.p(vc), ctx, kvh, qh, hd, ob.p(out))
    return bits(out)


def _delta(lib, prefix):
    rng = np.random.default_rng(14)
    q = rng.normal(0, 1, 128).astype(np.float32)
    k = rng.normal(0, 1, 128).astype(np.float32)
    v = rng.normal(0, 1, 128).astype(np.float32)
    S = rng.normal(0, 0.1, 128 * 128).astype(np.float32)
    out = np.empty(128, np.float32)
    getattr(lib, prefix + "_gated_delta")(ob.p(q), ob.p(k), ob.p(v), ctypes.c_float(0.7), ctypes.c_float(-0.3),
                                         128, 128, ob.p(S), ob.p(out))
    return np.concatenate([bits(out), bits(S)])


VECTOR_CASES = {"rmsnorm4096": _rmsnorm, "rope_pos511": _rope, "attention_ctx48": _attention,
                "gated_delta128": _delta}

MODEL_CASES = {"tiny_runtime_model": ([1, 2, 3], 6), "small_synthetic": ([11, 4000, 7, 250, 3, 3, 99], 10)}


def _write_model(name, d):
    if name == "tiny_runtime_model":
        write_tiny_model(d)
    else:
        import xqbind as xb
        xb.write_synth_model(d, **SMALL)


def run_reference_model(name):
    import xqbind as xb
    prompt, n_new = MODEL_CASES[name]
    with tempfile.TemporaryDirectory() as d:
        _write_model(name, d)
        lib = xb.bind_xq_abi(ctypes.CDLL(ob.REF_SO))
        s = xb.Session(d, xb.options(backend=b"cpu"), lib=lib)
        assert s.status == 0
        st, out, _ = s.generate(prompt, n_new)
        assert st == 0
        _, h, _ = s.hidden()
        return out.tolist(), np.asarray(h, np.float32)


def run_oracle_model(name):
    prompt, n_new = MODEL_CASES[name]
    with tempfile.TemporaryDirectory() as d:
        _write_model(name, d)
        om = ob.OracleModel(d)
        om.prefill(prompt)
        toks = [om.decode_one(len(prompt) + i) for i in range(n_new)]
        return toks, np.asarray(om.hidden_state(), np.float32)
