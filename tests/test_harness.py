"""The caller-side harness programs (csrc/tools) on the CPU.

Both talk to the library only through xqwen35.h, so with the compiled reference
library (oracle/_ref/libxqref.so) put behind them they can be checked against
the reference's own harness on the same library:

* xq_host_quality_runner: its report equals the one the reference's
  customlib/tools/xq_host_quality_runner.cpp (compiled from its source into
  oracle/_ref) prints for the same model and arguments, timings aside, in
  plain and prefill_debug modes, and the exit codes and error report agree.
* xq_benchmark: the benchmark, quality-validation and self-test modes produce
  the JSON the Android harness would (benchmark_jni.cpp:957-1098, :1128-1268)
  and apply BenchmarkInstrumentationTest.java's checks.  Its statistics are
  recomputed here from the per-run records it reports.
"""
import json
import os

import numpy as np
import pytest

import xqbind as xb
from harness_util import (BENCH, QUALITY, REF_LIB, REF_QUALITY, normalised_quality, reference_lib_dir, run,
                          run_json)
from tiny_model import SMALL

needs_ref = pytest.mark.skipif(not (os.path.exists(REF_LIB) and os.path.exists(REF_QUALITY)),
                               reason="the compiled reference (oracle/_ref) is built only where its sources are mounted")
needs_tools = pytest.mark.skipif(not (os.path.exists(QUALITY) and os.path.exists(BENCH)),
                                 reason="harness programs not built (build.py)")


@pytest.fixture(scope="module")
def small_dir(tmp_path_factory):
    d = str(tmp_path_factory.mktemp("small"))
    xb.write_synth_model(d, **SMALL)
    return d


@pytest.fixture(scope="module")
def reflib(tmp_path_factory):
    return reference_lib_dir(tmp_path_factory.mktemp("lib"))


@needs_ref
@needs_tools
@pytest.mark.parametrize("args", [["8", "8"], ["4", "2", "code_like", "prefill_debug"],
                                  ["3", "1", "long_512_token_style"]])
def test_quality_runner_report_equals_reference_runner(small_dir, reflib, args):
    rc_ref, want, _ = run_json([REF_QUALITY, small_dir, *args], timeout=300)
    rc, got, _ = run_json([QUALITY, small_dir, *args], lib_dir=reflib, timeout=300)
    assert rc == rc_ref
    assert normalised_quality(got) == normalised_quality(want)
    assert got["custom_backend_actual"] == "cpu"  # what the reference library's trace rows report


@needs_ref
@needs_tools
def test_quality_runner_error_paths_match(small_dir, reflib, tmp_path):
    rc_ref, out_ref, err_ref = run([REF_QUALITY, small_dir, "4", "8", "no_such_prompt"])
    rc, out, err = run([QUALITY, small_dir, "4", "8", "no_such_prompt"], lib_dir=reflib)
    assert (rc, out, err) == (rc_ref, out_ref, err_ref) and rc == 2
    missing = str(tmp_path / "missing")
    rc_ref, out_ref, _ = run([REF_QUALITY, missing])
    rc, out, _ = run([QUALITY, missing], lib_dir=reflib)
    assert (rc, out) == (rc_ref, out_ref) and rc == 1
    rc, out, err = run([QUALITY])
    assert rc == 2 and out == "" and "usage" in err


def check_benchmark_report(d, prompt_tokens, max_new, warmup, measured):
    assert d["schema_version"] == 4 and d["status"] == "ok"
    assert d["generation"]["prompt_tokens_requested"] == prompt_tokens
    assert d["generation"]["prompt_token_id"] == 16
    assert d["iterations"] == {"warmup": warmup, "measured": measured, "target_measured": measured}
    runs = d["runs"]
    assert [r["index"] for r in runs] == list(range(warmup + measured))
    assert [r["warmup"] for r in runs] == [True] * warmup + [False] * measured
    timed = [r for r in runs if not r["warmup"]]
    for r in runs:
        assert r["status_code"] == 0 and r["prompt_tokens"] == prompt_tokens and r["generated_tokens"] == max_new
        assert r["prefill_tokens_per_second"] == pytest.approx(1000 * prompt_tokens / r["prefill_ms"], rel=1e-4)
    dec = np.array([r["decode_tokens_per_second"] for r in timed])
    tps = d["tokens_per_second"]["decode"]
    assert tps["mean"] == pytest.approx(dec.mean(), rel=1e-4)
    assert tps["median"] == pytest.approx(np.median(dec), rel=1e-4)
    assert tps["stdev"] == pytest.approx(dec.std(), rel=1e-3, abs=1e-3)  # population stdev
    assert (tps["min"], tps["max"]) == (pytest.approx(dec.min(), rel=1e-4), pytest.approx(dec.max(), rel=1e-4))
    tpot = d["time_per_output_token_ms"]["decode"]
    assert tpot["min"] == pytest.approx(1000 / dec.max(), rel=1e-4)
    assert tpot["median"] == pytest.approx(1000 / np.median(dec), rel=1e-4)
    names = {r["name"] for r in d["per_kernel_wall_clock"]["rows"]}
    assert any(n.startswith("lm_head_custom") for n in names) and "sampling_greedy_custom" in names
    sk = d["runtime"]["selected_kernels"]
    assert sk["hotpath_replaced"] and sk["full_custom_decode"] and sk["fallback_op_families"] == []
    assert d["custom_path"]["calls_mnn_llm_response_for_measured_generation"] is False


@needs_ref
@needs_tools
def test_benchmark_modes_on_reference_library(small_dir, reflib, tmp_path):
    art = str(tmp_path / "art")
    rc, d, err = run_json([BENCH, "--prompt-tokens", "48", "--max-new-tokens", "6", "--warmup-iterations", "1",
                           "--measured-iterations", "3", "--no-microbench", "--artifact-dir", art, small_dir],
                          lib_dir=reflib)
    assert rc == 0, err
    check_benchmark_report(d, 48, 6, 1, 3)
    assert d["custom_backend_requested"] == "cpu" and d["custom_backend_actual"] == "cpu"
    assert d["runtime"]["selected_kernels"]["op_family_backends"]["lm_head"] == "cpu"
    assert d["custom_kernel_microbench"]["status"] == "skipped"
    assert "BENCH_ITER" in err
    with open(os.path.join(art, "bench_artifacts", "customlib_cpu_benchmark.json")) as f:
        assert json.load(f) == d
    # quality validation: the same greedy ids as the reference runner on the same library
    rc, q, err = run_json([BENCH, "--run-quality-validation", "--validation-max-new-tokens", "6", small_dir],
                          lib_dir=reflib)
    _, want, _ = run_json([REF_QUALITY, small_dir, "6", "8"])
    assert [p["generated_token_ids"] for p in q["prompts"]] == [p["generated_token_ids"] for p in want["prompts"]]
    assert (rc == 0) == q["quality_gate_passed"]
    # the reference library has no GPU self-test off-Android: the checks must fail
    rc, s, err = run_json([BENCH, "--run-vulkan-selftest"], lib_dir=reflib)
    assert rc == 1 and s["pass"] is False and "CHECK FAILED" in err


@needs_tools
def test_benchmark_rejects_bad_command_lines():
    assert run([BENCH])[0] == 2
    assert run([BENCH, "--prompt-tokens"])[0] == 2
    assert run([BENCH, "--bogus", "x"])[0] == 2
