"""Writes tests/golden/reference_vectors.npz: outputs of the compiled reference
(oracle/_ref/libxqref.so, built by `make -C oracle ref` from the reference's
own customlib sources) on seeded inputs that tests/test_golden.py regenerates
from the same recipes.  The fixture pins the oracle where the reference
checkout (and so _ref) is absent.  Run from the repo root:

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import conftest  # noqa: F401,E402  (sets up the import paths)
import golden_cases as gc  # noqa: E402
import oracle_bind as ob  # noqa: E402


def main():
    if not ob.ref_available():
        raise SystemExit("oracle/_ref/libxqref.so is not built (make -C oracle ref)")
    out = {}
    for name, (q, x) in gc.gemv_cases().items():
        out["gemv_" + name] = gc.bits(ob.gemv(q, x, ob.ref(), "ref_gemv_w4a16"))
        out["textbook_" + name] = gc.bits(ob.gemv(q, x, ob.ref(), "ref_gemv_textbook"))
        idx, val = ob.gemv_argmax(q, x, ob.ref(), "ref_gemv_w4a16_argmax")
        out["argmax_" + name] = np.array([idx, int(gc.bits(np.float32(val))[0])], np.int64)
    for name, fn in gc.VECTOR_CASES.items():
        out["vec_" + name] = fn(ob.ref(), "ref")
    for name in gc.MODEL_CASES:
        toks, hidden = gc.run_reference_model(name)
        out["model_tokens_" + name] = np.asarray(toks, np.int64)
        out["model_hidden_" + name] = gc.bits(hidden)
    path = os.path.join(HERE, "reference_vectors.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {len(out)} arrays, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
