"""Builds the two shared libraries of the MI355X decode path, in-tree.

  lib/libxqhip.so    hand-written gfx950 HIP kernels + the thin C ABI of include/xqhip.h
  lib/libxqwen35.so  C++ host runtime (Session / model / XQ4 reader) exporting the
                     reference C ABI of include/xqwen35.h; links libxqhip.so
  bin/xq_host_quality_runner, bin/xq_benchmark
                     the caller-side harness programs (csrc/tools), linked against
                     lib/libxqwen35.so through the xqwen35.h ABI only (RUNPATH
                     $ORIGIN/../lib, so LD_LIBRARY_PATH can put another build of
                     that ABI behind them)

Usage: python build.py [--jobs N] [--only hip|host|tools] [--sanitize]
Compiles every time it is called (hipcc cross-compiles for gfx950 without a GPU).

--sanitize builds the host library and the harness programs again with
AddressSanitizer and UndefinedBehaviorSanitizer (host code only; the kernels
are lib/libxqhip.so, copied beside them) into sanitize/lib and sanitize/bin,
for running the harness programs, which link the sanitizer runtime
themselves, over the whole HIP path.
"""
import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
INCLUDE = os.path.join(ROOT, "include")
HIP_SRC = os.path.join(HERE, "csrc", "hip")
HOST_SRC = os.path.join(HERE, "csrc", "host")
TOOL_SRC = os.path.join(HERE, "csrc", "tools")
LIB = os.path.join(HERE, "lib")
BIN = os.path.join(HERE, "bin")
OBJ = os.path.join(HERE, "_build")
SAN = os.path.join(HERE, "sanitize")
SAN_FLAGS = ["-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined"]
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # packed fp32 VALU ops are disabled for all device code on this target
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics", "-Wall", "-Wno-unused-function",
    "-I", INCLUDE, "-I", HIP_SRC,
]
# per-source additions: the prefill GEMM scales every MFMA result with VALU ops, so its
# MFMAs write VGPRs directly instead of accumulation registers that need copying out
HIP_FILE_FLAGS = {"prefill_ops.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}
HOST_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter",
              "-fvisibility=hidden", "-I", INCLUDE, "-I", HOST_SRC, "-DXQWEN35_BUILD=1"]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError("build step failed:\n" + " ".join(cmd) + "\n" + r.stdout)
    return r.stdout


def _compile_many(jobs, tasks):
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for out in ex.map(_run, tasks):
            if out.strip():
                sys.stderr.write(out)


def build_hip(jobs):
    srcs = sorted(f for f in os.listdir(HIP_SRC) if f.endswith(".hip"))
    objs, tasks = [], []
    for f in srcs:
        o = os.path.join(OBJ, "hip", f[:-4] + ".o")
        objs.append(o)
        tasks.append([HIPCC, *HIP_FLAGS, *HIP_FILE_FLAGS.get(f, []), "-c", os.path.join(HIP_SRC, f), "-o", o])
    os.makedirs(os.path.join(OBJ, "hip"), exist_ok=True)
    _compile_many(jobs, tasks)
    out = os.path.join(LIB, "libxqhip.so")
    tmp = out + ".tmp"
    _run([HIPCC, "-shared", f"--offload-arch={ARCH}", "-fPIC", "-o", tmp, *objs,
          "-Wl,-soname,libxqhip.so"])
    os.replace(tmp, out)
    return out


def build_host(jobs, lib=LIB, extra=()):
    if not os.path.isdir(HOST_SRC):
        return None
    srcs = sorted(f for f in os.listdir(HOST_SRC) if f.endswith(".cpp"))
    if not srcs:
        return None
    objs, tasks = [], []
    for f in srcs:
        o = os.path.join(OBJ, "host", f[:-4] + ".o")
        objs.append(o)
        tasks.append(["g++", *HOST_FLAGS, *extra, "-c", os.path.join(HOST_SRC, f), "-o", o])
    os.makedirs(os.path.join(OBJ, "host"), exist_ok=True)
    _compile_many(jobs, tasks)
    out = os.path.join(lib, "libxqwen35.so")
    tmp = out + ".tmp"
    _run(["g++", "-shared", *extra, "-o", tmp, *objs, "-L", lib, "-lxqhip", "-Wl,-rpath,$ORIGIN",
          "-Wl,-soname,libxqwen35.so", "-lpthread"])
    os.replace(tmp, out)
    return out


# tool -> the libraries it links besides libxqwen35.so
TOOLS = {"xq_host_quality_runner": [], "xq_benchmark": ["-lxqhip"]}


def build_tools(jobs, lib=LIB, bin_dir=BIN, flags=()):
    os.makedirs(bin_dir, exist_ok=True)
    tasks, outs = [], []
    for name, extra in TOOLS.items():
        out = os.path.join(bin_dir, name)
        outs.append(out)
        tasks.append(["g++", "-O2", "-std=c++17", "-Wall", "-Wextra", *flags, "-I", INCLUDE, "-I", TOOL_SRC,
                      os.path.join(TOOL_SRC, name + ".cpp"), "-o", out, "-L", lib, "-lxqwen35", *extra,
                      "-Wl,--enable-new-dtags,-rpath,$ORIGIN/../lib"])
    _compile_many(jobs, tasks)
    return outs


def build(jobs=None, only=None):
    jobs = jobs or min(8, os.cpu_count() or 1)
    os.makedirs(LIB, exist_ok=True)
    built = []
    if only in (None, "hip"):
        built.append(build_hip(jobs))
    if only in (None, "host"):
        h = build_host(jobs)
        if h:
            built.append(h)
    if only in (None, "tools"):
        built.extend(build_tools(jobs))
    shutil.rmtree(OBJ, ignore_errors=True)
    return built


def build_sanitized(jobs=None):
    """The host library and harness programs with ASan + UBSan, beside a copy of
    the kernel library (built first if it is missing)."""
    jobs = jobs or min(8, os.cpu_count() or 1)
    if not os.path.exists(os.path.join(LIB, "libxqhip.so")):
        build(jobs, "hip")
    lib, bin_dir = os.path.join(SAN, "lib"), os.path.join(SAN, "bin")
    os.makedirs(lib, exist_ok=True)
    shutil.copy2(os.path.join(LIB, "libxqhip.so"), os.path.join(lib, "libxqhip.so"))
    built = [build_host(jobs, lib, SAN_FLAGS)]
    built.extend(build_tools(jobs, lib, bin_dir, SAN_FLAGS))
    shutil.rmtree(OBJ, ignore_errors=True)
    return built


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--only", choices=["hip", "host", "tools"], default=None)
    ap.add_argument("--sanitize", action="store_true", help="ASan + UBSan host build into sanitize/")
    a = ap.parse_args()
    for p in (build_sanitized(a.jobs) if a.sanitize else build(a.jobs, a.only)):
        print(p)
