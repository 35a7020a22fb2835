"""Writes tests/golden/full_9b_reference.npz: the compiled reference
(oracle/_ref/libxqref.so, built by `make -C oracle ref` from the reference's
own customlib sources) run through its own C ABI (xq_create / xq_prefill /
xq_decode_one / xq_get_hidden_state / xq_get_debug_json) on the seeded
9B-shaped synthetic model (xqsynth_default_config: 32 layers 3 linear : 1
full, hidden 4096, MLP 12288, vocab 248320, W4A16 g64) with a 512-token
seeded random prompt, then N_STEPS greedy decode steps.

Stored per run:
  prompt            the 512 prompt ids (numpy default_rng(4), as bench.py)
  ids               the reference's greedy ids, one per decode step
  hidden            [1 + N_STEPS, 4096] f32: the final-normed hidden after the
                    prefill and after every decode step (xq_get_hidden_state)
  topk_tokens/logits [1 + N_STEPS, k]: the reference's lm_head top-k on each of
                    those hidden states (xq_get_debug_json), so top-2 margins
  digest_*          sha256 of a few model files, so a test that rewrites the
                    model elsewhere can show it holds the same bytes

The reference takes about 1 s of 8 host threads per token at this size, so
this is run once, offline, in a container holding the reference checkout:

    python tests/golden/make_full_9b.py [model_dir]
"""
import ctypes
import hashlib
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import conftest  # noqa: F401,E402  (sets up the import paths)
import oracle_bind as ob  # noqa: E402
import xqbind as xb  # noqa: E402

N_PROMPT = 512
N_STEPS = 16
PROMPT_SEED = 4
VOCAB = 248320
# files whose digests pin the model bytes: the manifest, one matrix of each
# layer kind, the final norm and the lm_head
DIGEST_FILES = (
    "xqwen35_manifest.json",
    "layers_0_linear_attn_in_proj_qkv_weight.xq4",
    "layers_3_self_attn_q_proj_weight.xq4",
    "layers_31_mlp_down_proj_weight.xq4",
    "norm_weight.f32",
    "lm_head_weight.xq4",
)


def prompt_ids():
    return np.random.default_rng(PROMPT_SEED).integers(0, VOCAB, N_PROMPT, dtype=np.int32)


def file_digest(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for block in iter(lambda: f.read(1 << 24), b""):
            h.update(block)
    return h.hexdigest()


def topk(sess):
    st, txt = sess.json("xq_get_debug_json", 1 << 16)
    if st != 0:
        raise RuntimeError(f"xq_get_debug_json: status {st}")
    rows = json.loads(txt)["lm_head_topk"]
    return [r["token"] for r in rows], [r["logit"] for r in rows]


def main():
    if not ob.ref_available():
        raise SystemExit("oracle/_ref/libxqref.so is not built (make -C oracle ref)")
    model_dir = sys.argv[1] if len(sys.argv) > 1 else "/tmp/xq_synth_9b_w4a16_g64"
    if not os.path.exists(os.path.join(model_dir, ".complete")):
        t0 = time.perf_counter()
        xb.write_synth_model(model_dir, threads=min(16, os.cpu_count() or 1))
        open(os.path.join(model_dir, ".complete"), "w").write("ok")
        print(f"model written in {time.perf_counter() - t0:.1f} s", flush=True)
    out = {"digest_" + f.replace(".", "_"): np.frombuffer(bytes.fromhex(file_digest(os.path.join(model_dir, f))),
                                                          np.uint8) for f in DIGEST_FILES}
    ref = xb.bind_xq_abi(ctypes.CDLL(ob.REF_SO))
    sess = xb.Session(model_dir, xb.options(backend=b"cpu", threads=8), lib=ref)
    if not sess.ok():
        raise SystemExit(f"reference xq_create failed: {sess.status}")
    prompt = prompt_ids()
    t0 = time.perf_counter()
    st, m = sess.prefill(prompt)
    assert st == 0, m.error
    print(f"prefill {N_PROMPT} tokens in {time.perf_counter() - t0:.0f} s", flush=True)
    hidden, tk_tok, tk_val, ids = [], [], [], []

    def record():
        st, h, _ = sess.hidden()
        assert st == 0
        hidden.append(h)
        t, v = topk(sess)
        tk_tok.append(t)
        tk_val.append(v)

    record()
    for i in range(N_STEPS):
        st, tok, m = sess.decode_one()
        assert st == 0, m.error
        ids.append(tok)
        record()
        print(f"step {i}: id {tok}, top-2 {tk_val[i][:2]}", flush=True)
    sess.close()
    out.update(prompt=prompt, ids=np.asarray(ids, np.int32), hidden=np.stack(hidden).astype(np.float32),
               topk_tokens=np.asarray(tk_tok, np.int32), topk_logits=np.asarray(tk_val, np.float32))
    path = os.path.join(HERE, "full_9b_reference.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
