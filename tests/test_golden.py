"""The oracle against committed outputs of the compiled reference
(tests/golden/reference_vectors.npz, written by tests/golden/make_golden.py
from oracle/_ref): GEMV (fused and textbook), argmax, RMSNorm, RoPE,
attention, gated delta and two whole-model forwards, bit for bit.  Runs
without the reference checkout.  CPU only."""
import os

import numpy as np
import pytest

import golden_cases as gc
import oracle_bind as ob

FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.npz")


@pytest.fixture(scope="module")
def golden():
    with np.load(FIXTURE, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("name", list(gc.gemv_cases().keys()))
def test_gemv_and_argmax_vs_reference_fixture(golden, name):
    q, x = gc.gemv_cases()[name]
    assert np.array_equal(gc.bits(ob.gemv(q, x)), golden["gemv_" + name])
    assert np.array_equal(gc.bits(ob.gemv(q, x, fn="orc_gemv_textbook")), golden["textbook_" + name])
    idx, val = ob.gemv_argmax(q, x)
    assert [idx, int(gc.bits(np.float32(val))[0])] == golden["argmax_" + name].tolist()


@pytest.mark.parametrize("name", list(gc.VECTOR_CASES.keys()))
def test_vector_kernels_vs_reference_fixture(golden, name):
    assert np.array_equal(gc.VECTOR_CASES[name](ob.oracle(), "orc"), golden["vec_" + name])


@pytest.mark.parametrize("name", list(gc.MODEL_CASES.keys()))
def test_model_forward_vs_reference_fixture(golden, name):
    toks, hidden = gc.run_oracle_model(name)
    assert toks == golden["model_tokens_" + name].tolist()
    assert np.array_equal(gc.bits(hidden), golden["model_hidden_" + name])
