"""The caller-side harness programs on the HIP library (MI355X).

* xq_host_quality_runner on libxqwen35.so: the report has the reference
  runner's structure and verdicts, and its greedy ids match the reference
  runner driving the compiled reference library (oracle/_ref, a CPU run) on
  the same model: bit-exact while the reference's top-2 logit margin at a step
  exceeds 1e-2 (read from the reference's prefill_debug dumps); after the first
  step at or below it the sequences may legitimately part.
* xq_benchmark: the benchmark mode passes the instrumentation test's checks on
  the HIP path, its kernel microbench reproduces the reference microbench's
  published checksums on the HIP kernels (GEMV 4096x4096 / 12288x4096 /
  4096x12288: 320.586 / 13.1145 / 207.929, RMSNorm 9.94688, GQA -0.00442318
  with keys and values in the fp16 cache, gated delta -0.0171842 after four
  calls), and the self-test mode passes.
"""
import os

import pytest

import xqbind as xb
from harness_util import (BENCH, QUALITY, REF_LIB, REF_QUALITY, normalised_quality, reference_lib_dir, run_json,
                          step_margins)
from tiny_model import SMALL

pytestmark = pytest.mark.gpu
MARGIN = 1e-2


@pytest.fixture(scope="module")
def small_dir(tmp_path_factory):
    d = str(tmp_path_factory.mktemp("small"))
    xb.write_synth_model(d, **SMALL)
    return d


@pytest.mark.skipif(not (os.path.exists(REF_LIB) and os.path.exists(REF_QUALITY)),
                    reason="the compiled reference (oracle/_ref) is not present")
def test_quality_runner_on_hip_matches_reference_runner(small_dir, tmp_path):
    n_new = "12"
    rc_ref, want, _ = run_json([REF_QUALITY, small_dir, n_new, "8", "", "prefill_debug"],
                               lib_dir=reference_lib_dir(tmp_path), timeout=300)
    rc, got, err = run_json([QUALITY, small_dir, n_new, "8"], timeout=300)
    assert got["custom_backend_actual"] == "hip", err
    assert got["validation"]["validation_dump_intermediate"] is False
    compared = 0
    for g, w in zip(got["prompts"], want["prompts"]):
        assert g["id"] == w["id"] and g["status_code"] == 0
        margins = step_margins(w)
        for i, (a, b) in enumerate(zip(g["generated_token_ids"], w["generated_token_ids"])):
            if a != b:
                assert margins[i] <= MARGIN, f"{g['id']} step {i}: hip {a} vs reference {b}, margin {margins[i]:.4g}"
                break
            compared += 1
        else:
            assert g["generated_token_ids"] == w["generated_token_ids"]
            # identical ids give identical verdicts and repetition statistics
            ng = normalised_quality({"prompts": [g]}, keep_backend=False)["prompts"][0]
            nw = normalised_quality({"prompts": [w]}, keep_backend=False)["prompts"][0]
            assert ng == nw
    assert compared >= 20
    # the report's frame matches the reference runner's
    a, b = normalised_quality(got, keep_backend=False), normalised_quality(want, keep_backend=False)
    for k in ("prompts", "validation"):
        a.pop(k), b.pop(k)
    assert a.pop("status") is not None and b.pop("status") is not None
    a.pop("quality_gate_passed"), b.pop("quality_gate_passed")
    assert a == b
    assert (rc == 0) == got["quality_gate_passed"]


def test_benchmark_on_hip_passes_checks_and_microbench_checksums(small_dir, tmp_path):
    rc, d, err = run_json([BENCH, "--custom-backend", "hip", "--prompt-tokens", "64", "--max-new-tokens", "16",
                           "--warmup-iterations", "1", "--measured-iterations", "2", "--artifact-dir", str(tmp_path),
                           small_dir], timeout=300)
    assert rc == 0, err[-3000:]
    assert d["custom_backend_actual"] == "hip" and d["custom_backend_requested"] == "hip"
    assert [r["generated_tokens"] for r in d["runs"]] == [16, 16, 16]
    assert d["tokens_per_second"]["decode"]["min"] > 0
    fam = d["runtime"]["selected_kernels"]["op_family_backends"]
    assert fam["q_proj"] == fam["lm_head"] == fam["sampling"] == fam["attention"] == "hip"
    mb = d["custom_kernel_microbench"]
    assert mb["status"] == "ok", mb
    rows = {r["name"]: r for r in mb["rows"]}
    tol = {"gemv_w4a16_attn_4096x4096": (1e-3, 1e-3), "gemv_w4a16_mlp_up_12288x4096": (1e-3, 1e-3),
           "gemv_w4a16_mlp_down_4096x12288": (1e-3, 1e-3), "rmsnorm_hidden4096": (1e-5, 1e-5),
           "gqa_decode_ctx512_q16_kv4_dim256": (1e-4, 0.0), "gated_delta_decode_k128_v128": (1e-5, 1e-3)}
    for name, (atol, rtol) in tol.items():
        r = rows[name]
        assert r["backend"] == "hip" and r["wall_ms"]["min"] > 0
        assert abs(r["checksum"] - r["published_checksum"]) <= atol + rtol * abs(r["published_checksum"]), r
    assert rows["rope_q_heads16_dim256_pos512"]["wall_ms"]["min"] > 0


def test_benchmark_selftest_mode_on_hip():
    rc, s, err = run_json([BENCH, "--run-vulkan-selftest"], timeout=300)
    bad = [r for r in s.get("results", []) + s.get("vector_results", []) if not r["pass"]]
    assert rc == 0 and not bad, (err, bad)
    assert s["pass"] is True and s["custom_backend_actual"] == "hip"
