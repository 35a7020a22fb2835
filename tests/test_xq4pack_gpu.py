"""A packed checkpoint end to end on the GPU: the quantiser on the GPU (torch
device cuda) writes the same bytes as the numpy path, and the library
generating from the package matches the oracle's CustomModel restatement on
the same files (greedy ids bit-exact while the oracle's top-2 margin exceeds
1e-2, hidden state within 1e-2 abs + 1e-3 rel), for the three quantisation
schemes, including the affine (XQ4 version 2) form.  The GPU packing runs as
its command line in a child process: torch brings its own HIP runtime, which
does not initialise in a process where the library's runtime already did."""
import filecmp
import os
import subprocess
import sys

import numpy as np
import pytest

import xq4pack as xp
import xqbind as xb
from ckpt import make_checkpoint
from test_model_gpu import close, compare_tokens, oracle_run

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def checkpoint(tmp_path_factory):
    d = str(tmp_path_factory.mktemp("ckpt"))
    make_checkpoint(d, seed=5)
    return d


@pytest.mark.parametrize("scheme,alpha", [("asymmetric", False), ("symmetric", False), ("affine", True)])
def test_packed_checkpoint_generates_like_the_oracle(checkpoint, tmp_path, scheme, alpha):
    cpu, gpu = str(tmp_path / "cpu"), str(tmp_path / "gpu")
    xp.pack_checkpoint(checkpoint, cpu, 64, scheme, alpha)
    flags = {"asymmetric": [], "symmetric": ["--symmetric"], "affine": ["--mnn-affine-asym"]}[scheme]
    flags += ["--mnn-alpha-fp16"] if alpha else []
    subprocess.run([sys.executable, xp.__file__, "--model-dir", checkpoint, "--out-dir", gpu, "--device", "cuda"] +
                   flags, check=True, timeout=300, stdout=subprocess.DEVNULL)
    names = sorted(os.listdir(cpu))
    assert names == sorted(os.listdir(gpu))
    for n in names:
        if n.endswith(".xq4"):
            assert filecmp.cmp(os.path.join(cpu, n), os.path.join(gpu, n), shallow=False), n
    prompt = [11, 400, 7, 250, 3, 3, 99, 1024]
    n_new = 12
    want, margins, hiddens = oracle_run(cpu, prompt, n_new)
    s = xb.Session(cpu, xb.options())
    assert s.status == xb.XQ_OK
    st, m = s.prefill(prompt)
    assert st == 0
    close(s.hidden()[1], hiddens[0], "hidden after prefill")
    got = []
    for i in range(n_new):
        st, tok, m = s.decode_one()
        assert st == 0
        got.append(tok)
    steps = compare_tokens(got, want, margins)
    assert steps >= 4 or min(margins[:4]) <= 1e-2
    assert np.all(np.array(got) >= 0)
