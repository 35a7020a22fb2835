"""Greedy decode of the 9B-shaped model at full size against the compiled
reference (customlib/runtime/session.cpp:385-421, custom_model.cpp:1281-1356).

The fixture tests/golden/full_9b_reference.npz (tests/golden/make_full_9b.py)
holds the reference's own run through its C ABI on the seeded synthetic model
(xqsynth_default_config: 32 layers 3 linear : 1 full, hidden 4096, MLP 12288,
vocab 248320, W4A16 g64) with a 512-token seeded prompt: the greedy id of each
of 16 decode steps, the final-normed hidden state after the prefill and after
every step, the lm_head top-10 of each of those states, and sha256 digests of
six model files.  Here the same model is written where the test runs (checked
against the digests) and run through libxqwen35.so: batched MFMA prefill of
the 512 tokens, then 16 decode steps.

Checks, at every state:
* greedy ids bit-exact where the reference's top-2 margin exceeds 1e-2 (here
  every margin is about 4.28);
* hidden within 1e-2 abs + 1e-3 rel;
* the prompt-dependent part of the hidden: the residual direction h / w (w the
  final-norm weights) is about -1 everywhere plus a deviation d of std ~0.02
  that carries the prompt; d must match the reference's to DEV_RTOL = 1e-4
  relative (in norm; measured 7e-6).  From one state to the next d changes by
  2.2 % (step 1) down to 3.7e-4 (step 16) relative (computed from the
  fixture), every one of them above DEV_RTOL, and d of state i must also lie
  nearer the reference's state i than any other reference state, so a run
  that drops, repeats or reorders a step, or loses the context, fails;
* the top-10 logits within 1e-2 abs + 1e-3 rel of the reference's, same ids
  where their gaps exceed 1e-2.
"""
import hashlib
import json
import os

import numpy as np
import pytest

import xqbind as xb

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "golden", "full_9b_reference.npz")
MODEL_DIR = os.environ.get("XQ_BENCH_MODEL_DIR", "/tmp/xq_synth_9b_w4a16_g64")
ATOL, RTOL, MARGIN = 1e-2, 1e-3, 1e-2
DEV_RTOL = 1e-4


def file_digest(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for block in iter(lambda: f.read(1 << 24), b""):
            h.update(block)
    return h.digest()


@pytest.fixture(scope="module")
def model():
    ref = np.load(FIXTURE)
    if not os.path.exists(os.path.join(MODEL_DIR, ".complete")):
        xb.write_synth_model(MODEL_DIR, threads=min(16, os.cpu_count() or 1))
        open(os.path.join(MODEL_DIR, ".complete"), "w").write("ok")
    for key in ref.files:
        if key.startswith("digest_"):
            name = key[len("digest_"):]
            stem, ext = name.rsplit("_", 1)
            path = os.path.join(MODEL_DIR, stem + "." + ext)
            assert file_digest(path) == ref[key].tobytes(), f"{path} differs from the fixture's model"
    return ref


def topk(sess):
    st, txt = sess.json("xq_get_debug_json", 1 << 16)
    assert st == 0
    rows = json.loads(txt)["lm_head_topk"]
    return np.array([r["token"] for r in rows]), np.array([r["logit"] for r in rows], np.float64)


def deviation(h, w):
    r = h.astype(np.float64) / w
    return r - r.mean()


def test_full_9b_greedy_decode_matches_reference(model):
    ref = model
    w = np.fromfile(os.path.join(MODEL_DIR, "norm_weight.f32"), np.float32).astype(np.float64) + 1.0
    sess = xb.Session(MODEL_DIR, xb.options(backend=b"hip", max_context=8192))
    assert sess.ok(), sess.status
    st, m = sess.prefill(ref["prompt"])
    assert st == 0, m.error
    n_steps = ref["ids"].size
    ref_devs = [deviation(ref["hidden"][j].astype(np.float64), w) for j in range(n_steps + 1)]
    report = []
    for i in range(n_steps + 1):
        st, h, _ = sess.hidden()
        assert st == 0
        want = ref["hidden"][i].astype(np.float64)
        err = np.abs(h - want)
        bad = ~(err <= ATOL + RTOL * np.abs(want))  # a NaN anywhere counts as bad
        dev_got, dev_want = deviation(h, w), deviation(want, w)
        dev_rel = float(np.linalg.norm(dev_got - dev_want) / np.linalg.norm(dev_want))
        tk_tok, tk_val = topk(sess)
        want_tok, want_val = ref["topk_tokens"][i], ref["topk_logits"][i].astype(np.float64)
        logit_err = float(np.max(np.abs(tk_val - want_val)))
        report.append(f"state {i}: hidden max err {err.max():.3g}, deviation rel err {dev_rel:.3g}, "
                      f"top-10 logit max err {logit_err:.3g}")
        print(report[-1], flush=True)
        assert not bad.any(), f"state {i}: {bad.sum()} hidden values outside tolerance (max err {err.max():.3g})"
        assert dev_rel <= DEV_RTOL, f"state {i}: prompt-dependent hidden deviation off by {dev_rel:.3g}"
        dists = [np.linalg.norm(dev_got - d) for d in ref_devs]
        assert int(np.argmin(dists)) == i, f"state {i}: deviation nearest to the reference's state {np.argmin(dists)}"
        assert np.all(np.abs(tk_val - want_val) <= ATOL + RTOL * np.abs(want_val)), (i, tk_val, want_val)
        gaps = np.diff(-want_val)
        for j in range(len(want_tok)):
            # rank j is pinned when it is separated from both neighbours by more than the margin
            if (j == 0 or gaps[j - 1] > MARGIN) and (j == len(gaps) or gaps[j] > MARGIN):
                assert tk_tok[j] == want_tok[j], (i, j, tk_tok, want_tok)
        if i == n_steps:
            break
        margin = want_val[0] - want_val[1]
        st, tok, m = sess.decode_one()
        assert st == 0, m.error
        if margin > MARGIN:
            assert tok == ref["ids"][i], f"step {i}: gpu id {tok} vs reference {ref['ids'][i]} (margin {margin:.4g})"
    sess.close()
