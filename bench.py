#!/usr/bin/env python3
"""Benchmark of the MI355X batch-1 W4A16 decode path (one GPU).

Prints ONE JSON line.  Workloads (--workload):
  decode (default) random-init 9B-shaped hybrid model (32 layers, 3 linear : 1
         full attention, hidden 4096, MLP 12288, vocab 248320, W4A16 g64) run
         through the xqwen35.h ABI: a 512-token prefill of random token ids,
         then K greedy decode steps.  value = decode tokens/s (generated tokens
         / decode wall time, as xq_metrics reports it).  A second run on the
         same shape written with the asymmetric quantiser's metadata (fp32
         scales, integer zeros; --no-asymmetric skips it) is reported under
         "asymmetric_metadata", and the prefill's gate/up GEMM over 512 tokens
         against the fp16 MFMA peak under "prefill_gemm".
  mlp    decode MLP block, hidden 4096 -> 12288 -> 4096, W4A16 g64: fused
         RMSNorm + gate/up GEMV + SiLU*up, then down GEMV + residual add.
         value = algorithmic HBM GB/s of the block (the GEMV bandwidth metric).
  decode-asym
         the second run of the decode workload alone (the model written with
         the asymmetric quantiser's metadata).
  gemv-sweep
         every decode-step projection shape of the 9B-shaped model (with the
         prologue and epilogue it runs with in the model) for 4-, 3- and 2-bit
         codes (--bits), n back-to-back launches each on rotated weight copies;
         value = algorithmic HBM GB/s of the gate/up launch at the first width.
A step is one pass of the workload over inputs already resident in HBM.  Weight
copies are rotated so the working set (> 2x the 256 MB Infinity Cache) is
streamed from HBM on every step.
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "yingjie-work-trial-mnn-custom-inference-library_amd")
sys.path.insert(0, os.path.join(PKG, "python"))

import xqbind as xb  # noqa: E402

HBM_PEAK_GBS = 8000.0
MFMA_FP16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
METRIC = "batch-1 decode tokens/s; W4A16 GEMV achieved HBM GB/s (% of peak)"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Events:
    def __init__(self):
        self.a, self.b = ctypes.c_void_p(), ctypes.c_void_p()
        xb.ck(xb.hip().xqhip_event_create(ctypes.byref(self.a)))
        xb.ck(xb.hip().xqhip_event_create(ctypes.byref(self.b)))

    def start(self):
        xb.ck(xb.hip().xqhip_event_record(self.a, None))

    def stop_ms(self):
        xb.ck(xb.hip().xqhip_event_record(self.b, None))
        ms = ctypes.c_float()
        xb.ck(xb.hip().xqhip_event_elapsed_ms(self.a, self.b, ctypes.byref(ms)))
        return ms.value


def w4_bytes(rows, cols, meta=2):
    """Device bytes of a W4 g64 matrix: the codes plus `meta` bytes of group
    metadata (2: the fp16 scale the upload keeps when every zero point is 8, as
    in these synthetic weights; 4: fp16 scale and zero)."""
    return rows * cols // 2 + rows * (cols // 64) * meta


# ---------------------------------------------------------------------------
# workload: decode MLP block
# ---------------------------------------------------------------------------
def mlp_inputs(hidden, inter, seed=1234):
    rng = np.random.default_rng(seed)
    gu_packed = rng.integers(0, 256, size=2 * inter * hidden // 2, dtype=np.uint8)
    gu_scales = np.abs(rng.normal(0, 0.02, 2 * inter * hidden // 64)).astype(np.float16).astype(np.float32)
    dn_packed = rng.integers(0, 256, size=hidden * inter // 2, dtype=np.uint8)
    dn_scales = np.abs(rng.normal(0, 0.02, hidden * inter // 64)).astype(np.float16).astype(np.float32)
    norm_w = rng.normal(1.0, 0.1, hidden).astype(np.float16).astype(np.float32)
    h = rng.normal(0, 1, hidden).astype(np.float16).astype(np.float32)
    return dict(gu=(gu_packed, gu_scales, np.full_like(gu_scales, 8.0)),
                dn=(dn_packed, dn_scales, np.full_like(dn_scales, 8.0)), norm_w=norm_w, h=h)


def bench_mlp(args):
    hidden, inter = 4096, 12288
    inp = mlp_inputs(hidden, inter)
    gu_rows = 2 * inter
    bytes_gu = w4_bytes(gu_rows, hidden) + hidden * 4 + inter * 4
    bytes_dn = w4_bytes(hidden, inter) + inter * 4 + 2 * hidden * 4
    step_bytes = bytes_gu + bytes_dn
    ncopy = max(2, int(np.ceil(640e6 / step_bytes)))
    log(f"[bench] mlp: uploading {ncopy} weight copies ({ncopy * step_bytes / 1e6:.0f} MB)")
    copies = []
    for _ in range(ncopy):
        gu = xb.DeviceW4(*inp["gu"], gu_rows, hidden)
        dn = xb.DeviceW4(*inp["dn"], hidden, inter)
        copies.append((gu, dn))
    nw = xb.DeviceBuffer.from_array(inp["norm_w"])
    h = xb.DeviceBuffer.from_array(inp["h"])
    ffn = xb.DeviceBuffer(inter * 4)
    hip = xb.hip()
    pro = xb.prologue(xb.PRO_RMS, nw, eps=1e-6)
    pro_ref = ctypes.byref(pro)

    def step(i):
        gu, dn = copies[i % ncopy]
        xb.ck(hip.xqhip_gemv_w4a16(gu.ref, h.ptr, xb.F32, pro_ref, ffn.ptr, xb.F32, xb.EPI_SILU_PAIR, None))
        xb.ck(hip.xqhip_gemv_w4a16(dn.ref, ffn.ptr, xb.F32, None, h.ptr, xb.F32, xb.EPI_ADD, None))

    for i in range(args.warmup):
        step(i)
    xb.ck(hip.xqhip_device_synchronize())
    ev = Events()
    ev.start()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    ms = ev.stop_ms()
    wall = (time.perf_counter() - t0) * 1e3
    ms_per_step = ms / args.steps
    gbs = step_bytes / (ms_per_step * 1e-3) / 1e9

    # per-kernel average durations (same stream, rotating copies)
    def time_kernel(fn, n=200):
        for i in range(10):
            fn(i)
        ev.start()
        for i in range(n):
            fn(i)
        return ev.stop_ms() / n

    t_gu = time_kernel(lambda i: xb.ck(hip.xqhip_gemv_w4a16(copies[i % ncopy][0].ref, h.ptr, xb.F32, pro_ref,
                                                            ffn.ptr, xb.F32, xb.EPI_SILU_PAIR, None)))
    t_dn = time_kernel(lambda i: xb.ck(hip.xqhip_gemv_w4a16(copies[i % ncopy][1].ref, ffn.ptr, xb.F32, None,
                                                            h.ptr, xb.F32, xb.EPI_ADD, None)))
    log(f"[bench] mlp step {ms_per_step * 1e3:.1f} us (wall {wall / args.steps * 1e3:.1f} us); "
        f"gate/up {t_gu * 1e3:.1f} us = {bytes_gu / t_gu / 1e6:.0f} GB/s; down {t_dn * 1e3:.1f} us = "
        f"{bytes_dn / t_dn / 1e6:.0f} GB/s")
    ach = bytes_gu / (t_gu * 1e-3) / 1e9
    result = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u4xf16->f32", "data": "synthetic",
        "config": {"workload": "decode MLP block, hidden 4096, intermediate 12288, W4A16 g64, batch 1",
                   "bytes_per_step": step_bytes, "weight_copies_rotated": ncopy},
        "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "gemv_w4_tiled gate/up 24576x4096 + RMSNorm prologue + SiLU epilogue",
                     "bytes_per_launch": bytes_gu, "avg_launch_us": round(t_gu * 1e3, 2),
                     "down_proj": {"bytes_per_launch": bytes_dn, "avg_launch_us": round(t_dn * 1e3, 2),
                                   "achieved": round(bytes_dn / (t_dn * 1e-3) / 1e9, 1)}},
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline_mlp(inp, hidden, inter, step_bytes, args.cpu_seconds)
    return result


def cpu_baseline_mlp(inp, hidden, inter, step_bytes, seconds):
    """Reference CPU path on the host cores: the compiled reference kernels
    (oracle/_ref) when present, else the oracle restatement."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle_bind as ob
    kind = "reference" if ob.ref_available() else "port"
    lib = ob.ref() if kind == "reference" else ob.oracle()
    pre = "ref_" if kind == "reference" else "orc_"
    gu_packed, gu_scales, gu_zeros = inp["gu"]
    rb, gpr = hidden // 2, hidden // 64
    gate = ob.Quantized(gu_packed.reshape(inter, 2, rb)[:, 0].copy(), gu_scales.reshape(inter, 2, gpr)[:, 0].copy(),
                        gu_zeros.reshape(inter, 2, gpr)[:, 0].copy(), inter, hidden)
    up = ob.Quantized(gu_packed.reshape(inter, 2, rb)[:, 1].copy(), gu_scales.reshape(inter, 2, gpr)[:, 1].copy(),
                      gu_zeros.reshape(inter, 2, gpr)[:, 1].copy(), inter, hidden)
    down = ob.Quantized(*inp["dn"], hidden, inter)
    h = inp["h"].copy()
    nw = inp["norm_w"]
    normed = np.empty(hidden, np.float32)

    def step():
        getattr(lib, pre + "rmsnorm")(ob.p(h), ob.p(nw), hidden, 1e-6, ob.p(normed))
        g = ob.gemv(gate, normed, lib, pre + "gemv_w4a16")
        u = ob.gemv(up, normed, lib, pre + "gemv_w4a16")
        f = (g / (1.0 + np.exp(-g.astype(np.float64)))).astype(np.float32) * u
        h[:] += ob.gemv(down, f, lib, pre + "gemv_w4a16")

    step()
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        step()
        n += 1
    dt = (time.perf_counter() - t0) / n
    threads = min(8, os.cpu_count() or 1)
    return {"value": round(step_bytes / dt / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": kind,
            "sample": f"{n} MLP-block steps ({dt * 1e3:.1f} ms each): RMSNorm + gate/up/down gemvW4A16 "
                      f"(reference worker pool, {threads} threads of {os.cpu_count()} host cores) + SiLU/residual"}


# ---------------------------------------------------------------------------
# per-projection GEMV timing: the decode step's matrices at their real shapes,
# each with the prologue and epilogue it runs with in the model
# ---------------------------------------------------------------------------
# (name, rows, cols, prologue, epilogue); rows of gate/up are the interleaved
# (gate_i, up_i) pairs, in_proj the fused projections of each layer kind
PROJECTIONS = [
    ("gate_up", 24576, 4096, "rms", "silu"),
    ("down", 4096, 12288, "none", "add"),
    ("in_proj_linear", 12352, 4096, "rms", "store"),   # qkv 8192 | a 32 | b 32 | z 4096
    ("in_proj_full", 10240, 4096, "rms", "store"),     # q 8192 (gated) | k 1024 | v 1024
    ("out_proj_linear", 4096, 4096, "gated", "add"),   # gated head RMSNorm prologue (gate activated by the step)
    ("o_proj_full", 4096, 4096, "none", "add"),
    ("lm_head", 248320, 4096, "rms", "argmax"),
]
# launches of each projection per decode step of the 9B-shaped model (24 linear + 8 full layers)
PROJ_PER_STEP = {"gate_up": 32, "down": 32, "in_proj_linear": 24, "in_proj_full": 8, "out_proj_linear": 24,
                 "o_proj_full": 8, "lm_head": 1}


# group metadata of the synthetic matrices (time_projection):
#   sym   fp16 scales, every zero point 2^(bits-1) (8 for 4-bit codes): the
#         upload keeps the fp16 scale alone (2 B per group; 3 and 2 bits: the
#         fp16 (scale, zero) pair, 4 B)
#   asym  the asymmetric packer's metadata: fp32 scales, integer zeros 0..15:
#         the fp32 scale and a 4-bit zero code (4.5 B per group)
#   pair  fp32 scales, non-integer zeros: the fp32 (scale, zero) pair (8 B)
META_KINDS = ("sym", "asym", "pair")


def time_projection(name, rows, cols, pro_kind, epi, bits=4, n=200, budget=640e6, meta="sym"):
    """Average duration of n back-to-back launches of one projection (HIP events
    on the default stream around the loop), weights rotated over enough copies
    (> 2x the 256 MB last-level cache) that every launch streams from HBM.
    Algorithmic bytes = the uploaded matrix (codes + group metadata in the
    layout the upload picks for `meta`) + x + y."""
    hip = xb.hip()
    rng = np.random.default_rng(rows + cols + bits)
    g = cols // 64
    packed = rng.integers(0, 256, (rows * cols * bits + 7) // 8, dtype=np.uint8)
    scales32 = np.abs(rng.normal(0.0, 0.02, rows * g)).astype(np.float32)
    if meta == "sym":
        scales = scales32.astype(np.float16).astype(np.float32)
        zeros = np.full(rows * g, float(1 << (bits - 1)), np.float32)
    elif meta == "asym":
        scales = scales32
        zeros = np.clip(np.rint(7.5 + rng.normal(0.0, 1.0, rows * g)), 0, 15).astype(np.float32)
    else:
        scales = scales32
        zeros = (7.5 + rng.normal(0.0, 1.0, rows * g)).astype(np.float32)
    meta_bytes = {"sym": rows * g * (2 if bits == 4 else 4), "asym": rows * g * 4 + rows * ((g + 7) // 8) * 4,
                  "pair": rows * g * 8}[meta]
    one = rows * cols * bits // 8 + meta_bytes
    ncopy = max(2, min(64, int(np.ceil(budget / one))))
    copies = [xb.DeviceW4(packed, scales, zeros, rows, cols, 64, 0, bits=bits) for _ in range(ncopy)]
    assert copies[0].weight_bytes() == one, (name, meta, copies[0].weight_bytes(), one)
    layout = int(copies[0].w.layout)
    x = xb.DeviceBuffer.from_array(rng.normal(0, 1, cols).astype(np.float32))
    nw = xb.DeviceBuffer.from_array(rng.normal(1.0, 0.1, cols).astype(np.float32))
    hw = xb.DeviceBuffer.from_array(rng.normal(1.0, 0.1, 128).astype(np.float32))
    z = xb.DeviceBuffer.from_array(rng.normal(0, 1, cols).astype(np.float32))
    out_n = rows // 2 if epi == "silu" else rows
    y = xb.DeviceBuffer(out_n * 4)
    y.zero()
    ws = xb.DeviceBuffer(hip.xqhip_argmax_workspace_bytes(rows))
    idx, val = xb.DeviceBuffer(4), xb.DeviceBuffer(4)
    pro = {"none": None, "rms": xb.prologue(xb.PRO_RMS, nw, eps=1e-6),
           "gated": xb.prologue(xb.PRO_GATED_HEAD_ACT, hw, z, head_dim=128, eps=1e-6)}[pro_kind]
    pro_ref = ctypes.byref(pro) if pro is not None else None
    epi_code = {"store": xb.EPI_STORE, "add": xb.EPI_ADD, "silu": xb.EPI_SILU_PAIR}.get(epi)

    def launch(i):
        w = copies[i % ncopy].ref
        if epi == "argmax":
            xb.ck(hip.xqhip_gemv_w4a16_argmax(w, x.ptr, xb.F32, pro_ref, ws.ptr, idx.ptr, val.ptr, None))
        else:
            xb.ck(hip.xqhip_gemv_w4a16(w, x.ptr, xb.F32, pro_ref, y.ptr, xb.F32, epi_code, None))

    if name == "lm_head":
        n = min(n, 50)
    for i in range(max(10, 2 * ncopy)):
        launch(i)
    ev = Events()
    ev.start()
    for i in range(n):
        launch(i)
    us = ev.stop_ms() * 1e3 / n
    algo = copies[0].weight_bytes() + cols * 4 + (rows // 2 if epi == "silu" else rows) * 4 * (2 if epi == "add" else 1)
    if epi == "argmax":
        algo = copies[0].weight_bytes() + cols * 4
    for c in copies:
        c.free()
    return {"name": name, "bits": bits, "rows": rows, "cols": cols, "prologue": pro_kind, "epilogue": epi,
            "meta": meta, "layout": layout,
            "launches": n, "weight_copies": ncopy, "avg_us": round(us, 2), "bytes": int(algo),
            "GBps": round(algo / us / 1e3, 1), "frac": round(algo / (us * 1e-6) / (HBM_PEAK_GBS * 1e9), 4)}


def time_prefill_gemm(rows=24576, cols=4096, m=512, n=20):
    """The prefill's largest GEMM, gate/up (RMSNorm prologue, SiLU pair
    epilogue) over a 512-token chunk through xqhip_gemm_w4a16: the average of n
    back-to-back calls (each the activation preparation kernel and the MFMA
    GEMM), HIP events on the launch stream.  Algorithmic work 2 m rows cols
    FLOP against the dense fp16 MFMA peak; the kernel issues two fp16 MFMA
    passes per product (x as fp16 hi + lo), so its MFMA work is twice that."""
    hip = xb.hip()
    rng = np.random.default_rng(rows + cols + m)
    g = rows * (cols // 64)
    packed = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
    scales = np.abs(rng.normal(0.0, 0.02, g)).astype(np.float16).astype(np.float32)
    w = xb.DeviceW4(packed, scales, np.full(g, 8.0, np.float32), rows, cols)
    X = xb.DeviceBuffer.from_array(rng.normal(0, 1, (m, cols)).astype(np.float32))
    gam = xb.DeviceBuffer.from_array(rng.normal(1.0, 0.1, cols).astype(np.float32))
    y = xb.DeviceBuffer(m * (rows // 2) * 4)
    ws = xb.DeviceBuffer(hip.xqhip_gemm_workspace_bytes(m, cols, rows))
    pro = xb.prologue(xb.PRO_RMS, gam, eps=1e-6)

    def launch():
        xb.ck(hip.xqhip_gemm_w4a16(w.ref, X.ptr, m, cols, ctypes.byref(pro), 0, y.ptr, rows // 2,
                                   xb.EPI_SILU_PAIR, ws.ptr, ws.nbytes, None))

    for _ in range(3):
        launch()
    ev = Events()
    ev.start()
    for _ in range(n):
        launch()
    us = ev.stop_ms() * 1e3 / n
    w.free()
    flop = 2.0 * m * rows * cols
    tflops = flop / (us * 1e-6) / 1e12
    return {"bound": "mfma", "kernel": "prep_x_vec_kernel + gemm_w4_mfma_kernel<4, 1, 2, 4, 2, 2>: prefill gate/up "
                                       f"{rows}x{cols} W4A16 g64 over {m} tokens, RMSNorm prologue, SiLU*up epilogue",
            "method": f"HIP events around {n} back-to-back calls of xqhip_gemm_w4a16 (preparation + GEMM); "
                      "algorithmic FLOP = 2 m rows cols",
            "avg_us": round(us, 1), "flop": flop, "achieved": round(tflops, 1), "peak": MFMA_FP16_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": round(tflops / MFMA_FP16_PEAK_TFLOPS, 4), "mfma_passes": 2,
            "mfma_work_frac": round(2 * tflops / MFMA_FP16_PEAK_TFLOPS, 4)}


def projection_table(bits=4, n=200, meta="sym", names=None):
    rows = []
    for name, r, c, pro, epi in PROJECTIONS:
        if names is not None and name not in names:
            continue
        rows.append(time_projection(name, r, c, pro, epi, bits=bits, n=n, meta=meta))
        t = rows[-1]
        log(f"[bench] W{bits} {meta:4s} {name:16s} {r}x{c} {t['avg_us']:8.2f} us {t['bytes'] / 1e6:8.2f} MB "
            f"{t['GBps']:7.1f} GB/s frac {t['frac']:.3f}")
    return rows


def bench_gemv_sweep(args):
    table = []
    for bits in args.bits:
        table.extend(projection_table(bits, n=args.steps))
    first = table[0]
    return {"metric": METRIC, "value": first["GBps"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
            "warmup": 0, "ms_per_step": round(first["avg_us"] / 1e3, 5), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "u4xf16->f32", "data": "synthetic",
            "config": {"workload": "decode-step projection GEMVs of the 9B-shaped model, batch 1, g64, "
                                   f"{args.steps} back-to-back launches per shape on rotated weights",
                       "bits": args.bits},
            "projections": table}


# ---------------------------------------------------------------------------
# workload: end-to-end batch-1 decode of the 9B-shaped model
# ---------------------------------------------------------------------------
MODEL_DIR = os.environ.get("XQ_BENCH_MODEL_DIR", "/tmp/xq_synth_9b_w4a16_g64")


# ---------------------------------------------------------------------------
# HBM traffic of the roofline kernel from rocprofv3 counters (two passes:
# FETCH_SIZE, then WRITE_SIZE, each in KiB per dispatch), each scaled by what
# the same counter reads for a plain device-to-device copy of known size.
# ---------------------------------------------------------------------------
PMC_COPY_BYTES = 64 << 20
GATE_UP_KERNEL = "gemv_w4_tiled<1, 12, 2, 2, 4, 2>"  # NCH=1, 12 row groups, 2 rows per wave, SiLU pair, 4-bit codes, fp16 scale (zero 8)


def pmc_probe(args):
    """Child workload run under rocprofv3 --pmc: 5 copies of PMC_COPY_BYTES,
    then 6 gate/up GEMVs (24576x4096, RMSNorm prologue, SiLU*up) on rotated
    weight copies."""
    hidden, inter = 4096, 12288
    hip = xb.hip()
    src, dst = xb.DeviceBuffer(PMC_COPY_BYTES), xb.DeviceBuffer(PMC_COPY_BYTES)
    src.zero()
    for _ in range(5):
        xb.ck(hip.xqhip_copy(dst.ptr, src.ptr, PMC_COPY_BYTES, None))
    inp = mlp_inputs(hidden, inter)
    copies = [xb.DeviceW4(*inp["gu"], 2 * inter, hidden) for _ in range(6)]
    nw = xb.DeviceBuffer.from_array(inp["norm_w"])
    h = xb.DeviceBuffer.from_array(inp["h"])
    ffn = xb.DeviceBuffer(inter * 4)
    pro = xb.prologue(xb.PRO_RMS, nw, eps=1e-6)
    for w in copies:
        xb.ck(hip.xqhip_gemv_w4a16(w.ref, h.ptr, xb.F32, ctypes.byref(pro), ffn.ptr, xb.F32, xb.EPI_SILU_PAIR, None))
    xb.ck(hip.xqhip_device_synchronize())
    return {"pmc_probe": "done"}


def _pmc_pass(counter, workdir):
    import csv
    import glob
    import shutil
    import subprocess
    rocprof = shutil.which("rocprofv3")
    if not rocprof:
        return None
    out = os.path.join(workdir, counter)
    cmd = ["timeout", "-s", "KILL", "120", rocprof, "--pmc", counter, "--output-format", "csv", "-d", out, "-o", "pmc",
           "--", sys.executable, os.path.join(ROOT, "bench.py"), "--workload", "pmc-probe"]
    env = dict(os.environ, TMPDIR="/tmp")
    log(f"[bench] traffic: {' '.join(cmd[4:8])} pass")
    r = subprocess.run(cmd, cwd="/tmp", env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    files = glob.glob(os.path.join(out, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        log(f"[bench] traffic: rocprofv3 {counter} pass produced no counters (rc {r.returncode})")
        return None
    vals = {"copy": [], "gemv": []}
    for f in files:
        for row in csv.DictReader(open(f)):
            name = row.get("Kernel_Name", "")
            v = float(row.get("Counter_Value", "nan"))
            if "copy_u32x4_kernel" in name:
                vals["copy"].append(v)
            elif GATE_UP_KERNEL in name:
                vals["gemv"].append(v)
    if not vals["copy"] or not vals["gemv"]:
        return None
    return sum(vals["copy"]) / len(vals["copy"]), sum(vals["gemv"]) / len(vals["gemv"]), len(vals["gemv"])


def measure_traffic():
    """HBM bytes per launch of the gate/up GEMV: FETCH_SIZE and WRITE_SIZE,
    each calibrated on a device-to-device copy of PMC_COPY_BYTES."""
    import tempfile
    with tempfile.TemporaryDirectory(dir="/tmp") as d:
        f = _pmc_pass("FETCH_SIZE", d)
        w = _pmc_pass("WRITE_SIZE", d)
    if not f or not w:
        return None
    fetch_scale, write_scale = PMC_COPY_BYTES / f[0], PMC_COPY_BYTES / w[0]  # bytes per counted KiB
    fetch, write = f[1] * fetch_scale, w[1] * write_scale
    return {"bytes": round(fetch + write), "fetch_bytes": round(fetch), "write_bytes": round(write),
            "fetch_scale_bytes_per_kib": round(fetch_scale, 2), "write_scale_bytes_per_kib": round(write_scale, 2),
            "dispatches": f[2], "method": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes over a child run of "
            "bench.py --workload pmc-probe, calibrated on a 64 MiB one-dispatch device copy (xqhip_copy)"}


def ensure_model(path, **overrides):
    marker = os.path.join(path, ".complete")
    if os.path.exists(marker):
        return 0.0
    t0 = time.perf_counter()
    log(f"[bench] writing the synthetic 9B-shaped model to {path} ({overrides or 'default metadata'}) ...")
    xb.write_synth_model(path, threads=min(16, os.cpu_count() or 1), **overrides)
    open(marker, "w").write("ok")
    dt = time.perf_counter() - t0
    log(f"[bench] model written in {dt:.1f} s")
    return dt


def trace_rows(sess):
    st, txt = sess.json("xq_get_kernel_trace_json", 1 << 22)
    return {r["name"]: r for r in json.loads(txt)["rows"]} if st == 0 else {}


def backend_field(info, key):
    return info.split(key + "=")[1].split(";")[0] if key + "=" in info else None


def timed_decode(sess, prompt, args):
    """Warmup (one prefill + W decode steps, which capture the step graphs),
    then the timed run: a fresh prefill and the first decode step after it
    (untimed: that step replays the traced copy of the step graph, timestamps
    between its ops for the kernel trace), then exactly K decode steps, each
    one graph launch (every 128th the traced copy)."""
    st, m = sess.prefill(prompt)
    assert st == 0, m.error
    for _ in range(args.warmup):
        st, tok, m = sess.decode_one()
        assert st == 0
    assert sess.lib.xq_reset(sess.h) == 0
    st, m = sess.prefill(prompt)
    assert st == 0, m.error
    prefill_ms = m.prefill_ms
    st, tok, m = sess.decode_one()
    assert st == 0, m.error
    xb.ck(xb.hip().xqhip_device_synchronize())
    toks = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        st, tok, m = sess.decode_one()
        assert st == 0, m.error
        toks.append(tok)
    xb.ck(xb.hip().xqhip_device_synchronize())
    wall = time.perf_counter() - t0
    return {"wall_s": wall, "ms_per_step": wall * 1e3 / args.steps, "tps": args.steps / wall,
            "prefill_ms": prefill_ms, "decode_ms": m.decode_total_ms, "tokens": toks}


def bench_decode(args):
    prompt_len, hidden, inter = 512, 4096, 12288
    gen_s = ensure_model(MODEL_DIR)
    rng = np.random.default_rng(4)
    prompt = rng.integers(0, 248320, prompt_len, dtype=np.int32)
    t0 = time.perf_counter()
    sess = xb.Session(MODEL_DIR, xb.options(backend=b"hip", max_context=8192))
    if not sess.ok():
        raise RuntimeError(f"xq_create failed: {sess.status}")
    load_s = time.perf_counter() - t0
    log(f"[bench] model loaded in {load_s:.1f} s: {sess.json('xq_get_backend_info')[1][:300]}")
    run = timed_decode(sess, prompt, args)
    prefill_ms, decode_ms, ms_per_step, tps = run["prefill_ms"], run["decode_ms"], run["ms_per_step"], run["tps"]
    rows = trace_rows(sess)
    gu = next((r for n, r in rows.items() if n.startswith("linear_gate_proj")), None)
    dn = next((r for n, r in rows.items() if n.startswith("linear_down_proj")), None)
    lm = next((r for n, r in rows.items() if n.startswith("lm_head_custom")), None)
    step = rows.get("decode_step_graph_custom")
    traced = rows.get("decode_step_graph_traced_custom")
    st_tr, txt_tr = sess.json("xq_get_kernel_trace_json", 1 << 22)
    trace_counts = {k: v for k, v in json.loads(txt_tr).items() if k != "rows"} if st_tr == 0 else {}
    bytes_gu = w4_bytes(2 * inter, hidden) + hidden * 4 + inter * 4
    bytes_dn = w4_bytes(hidden, inter) + inter * 4 + 2 * hidden * 4
    bytes_lm = w4_bytes(248320, hidden) + hidden * 4
    info = sess.json("xq_get_backend_info")[1]
    wbytes = int(backend_field(info, "weight_bytes_per_token") or 0)
    # --no-projections (profiling runs: only the decode path's own kernels in
    # the trace) leaves the roofline fields null
    proj = [] if args.no_projections else projection_table(4, n=200)
    t_gu = next((p["avg_us"] for p in proj if p["name"] == "gate_up"), None)
    ach = bytes_gu / (t_gu * 1e-6) / 1e9 if t_gu else None
    gemv_us = sum(p["avg_us"] * PROJ_PER_STEP[p["name"]] for p in proj)
    gemv_bytes = sum(p["bytes"] * PROJ_PER_STEP[p["name"]] for p in proj)
    step_ms = step["mean_ms"] if step else ms_per_step
    log(f"[bench] decode {args.steps} steps: {ms_per_step:.3f} ms/token wall ({tps:.1f} tok/s), graph step "
        f"{step_ms:.3f} ms, weights {wbytes / 1e9:.3f} GB/token -> {wbytes / (step_ms * 1e-3) / 1e9:.0f} GB/s; "
        f"prefill {prefill_ms:.1f} ms ({prompt_len / prefill_ms * 1e3:.0f} tok/s)")
    result = {
        "metric": METRIC, "value": round(tps, 2), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u4xf16->f32", "data": "synthetic",
        "config": {"workload": "batch-1 greedy decode, random-init 9B-shaped hybrid model (32 layers 3:1 linear:full, "
                               "hidden 4096, MLP 12288, vocab 248320, 32q/8kv heads d128, W4A16 g64), "
                               f"{prompt_len}-token prefill and one untimed decode step, then {args.steps} timed "
                               "decode steps",
                   "prompt_tokens": prompt_len, "weight_bytes_per_token": wbytes,
                   "graph_step_ms": round(step_ms, 4), "decode_total_ms_from_xq_metrics": round(decode_ms, 3),
                   "traced_graph_step_ms": round(traced["mean_ms"], 4) if traced else None,
                   "kernel_trace_sampling": trace_counts,
                   "weight_stream_GBps": round(wbytes / (step_ms * 1e-3) / 1e9, 1),
                   "prefill_ms": round(prefill_ms, 2), "prefill_tokens_per_s": round(prompt_len / prefill_ms * 1e3, 1),
                   "model_write_s": round(gen_s, 1), "load_s": round(load_s, 1)},
        "roofline": {"bound": "hbm", "achieved": round(ach, 1) if ach else None, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4) if ach else None, "traffic": None,
                     "kernel": f"{GATE_UP_KERNEL}: gate/up 24576x4096 W4A16 g64 + RMSNorm prologue + SiLU*up "
                               "epilogue",
                     "method": "HIP events on the launch stream around 200 back-to-back launches on rotated weight "
                               "copies (> 2x the last-level cache); algorithmic bytes = codes + fp16 scale per group "
                               "(every zero point is 8: the layout keeps the scale alone) + x + y",
                     "bytes_per_launch": bytes_gu, "avg_launch_us": t_gu, "launches_timed": 200 if proj else 0,
                     "per_projection": [{k: p[k] for k in ("name", "rows", "cols", "prologue", "epilogue", "avg_us",
                                                           "bytes", "GBps", "frac")} for p in proj],
                     "projections_per_step": {"launches": sum(PROJ_PER_STEP.values()), "bytes": gemv_bytes,
                                              "sum_avg_us": round(gemv_us, 1),
                                              "frac": round(gemv_bytes / (gemv_us * 1e-6) / (HBM_PEAK_GBS * 1e9), 4)
                                              if gemv_us else None},
                     "in_model_avg_us": {"gate_up": round(gu["mean_ms"] * 1e3, 2) if gu else None,
                                         "down_proj": round(dn["mean_ms"] * 1e3, 2) if dn else None,
                                         "lm_head_argmax": round(lm["mean_ms"] * 1e3, 2) if lm else None},
                     "bytes_per_launch_down_proj": bytes_dn, "bytes_per_launch_lm_head": bytes_lm},
    }
    if not args.no_projections:
        pg = time_prefill_gemm()
        result["prefill_gemm"] = pg
        log(f"[bench] prefill gate/up GEMM (512 tokens): {pg['avg_us']:.1f} us, {pg['achieved']:.0f} TFLOP/s "
            f"algorithmic = {pg['frac']:.3f} of the fp16 MFMA peak ({pg['mfma_work_frac']:.3f} counting both passes)")
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline_decode(prompt, sess)
    sess.close()
    if not args.no_asymmetric:
        result["asymmetric_metadata"] = bench_decode_asymmetric(args, prompt, tps, proj)
    if not args.no_traffic:
        t = measure_traffic()
        if t:
            result["roofline"]["traffic"] = t["bytes"]
            result["roofline"]["traffic_detail"] = t
            log(f"[bench] gate/up traffic {t['bytes']} B per launch (algorithmic {bytes_gu})")
    return result


ASYM_DIR = MODEL_DIR.rstrip("/") + "_asym"


def bench_decode_asymmetric(args, prompt, sym_tps, sym_proj):
    """The same decode workload on the same 9B shape written with the metadata
    of the reference packer's asymmetric quantiser (fp32 scales, integer zeros
    0..15, pack_qwen35_xq4_numpy.py:218-247): every matrix uploads in the
    fp32-scale + 4-bit-zero layout (4.5 B per group).  Reports decode tok/s,
    the weight bytes per token and the per-projection GEMV table of that
    layout, and gate/up in the fp32-pair layout (8 B per group, what these
    matrices would need without the 4-bit zero) for comparison."""
    gen_s = ensure_model(ASYM_DIR, asymmetric=1)
    t0 = time.perf_counter()
    sess = xb.Session(ASYM_DIR, xb.options(backend=b"hip", max_context=8192))
    if not sess.ok():
        raise RuntimeError(f"xq_create failed (asymmetric model): {sess.status}")
    load_s = time.perf_counter() - t0
    info = sess.json("xq_get_backend_info")[1]
    wbytes = int(backend_field(info, "weight_bytes_per_token") or 0)
    run = timed_decode(sess, prompt, args)
    rows = trace_rows(sess)
    sess.close()
    step = rows.get("decode_step_graph_custom")
    step_ms = step["mean_ms"] if step else run["ms_per_step"]
    log(f"[bench] asymmetric metadata: {run['ms_per_step']:.3f} ms/token wall ({run['tps']:.1f} tok/s), graph step "
        f"{step_ms:.3f} ms, weights {wbytes / 1e9:.3f} GB/token; layouts {backend_field(info, 'weight_layouts')}")
    out = {"model": "the same 9B shape and seed, XQ4 v1 files with fp32 scales |N(0, 0.02)| and integer zeros "
                    "clamp(round(7.5 + N(0, 1)), 0, 15) per group (xqsynth asymmetric=1)",
           "tokens_per_s": round(run["tps"], 2), "ms_per_step": round(run["ms_per_step"], 4),
           "graph_step_ms": round(step_ms, 4), "vs_symmetric": round(run["tps"] / sym_tps, 4) if sym_tps else None,
           "weight_bytes_per_token": wbytes, "weight_layouts": backend_field(info, "weight_layouts"),
           "prefill_ms": round(run["prefill_ms"], 2), "model_write_s": round(gen_s, 1), "load_s": round(load_s, 1),
           "layout": "TILED64_F32S_Z4: fp32 scale + 4-bit zero code per group (4.5 B), exact for these values"}
    if not args.no_projections:
        proj = projection_table(4, n=200, meta="asym")
        pair = projection_table(4, n=200, meta="pair", names=("gate_up",))
        gemv_us = sum(p["avg_us"] * PROJ_PER_STEP[p["name"]] for p in proj)
        gemv_bytes = sum(p["bytes"] * PROJ_PER_STEP[p["name"]] for p in proj)
        keys = ("name", "rows", "cols", "prologue", "epilogue", "layout", "avg_us", "bytes", "GBps", "frac")
        out["per_projection"] = [{k: p[k] for k in keys} for p in proj]
        out["projections_per_step"] = {"bytes": gemv_bytes, "sum_avg_us": round(gemv_us, 1),
                                       "frac": round(gemv_bytes / (gemv_us * 1e-6) / (HBM_PEAK_GBS * 1e9), 4)}
        out["gate_up_f32_pair_layout"] = {k: pair[0][k] for k in keys}
        sym_gu = next((p for p in sym_proj if p["name"] == "gate_up"), None)
        if sym_gu:
            out["gate_up_fp16_scale_layout_us"] = sym_gu["avg_us"]
    return out


def bench_decode_asym_only(args):
    """--workload decode-asym: only the asymmetric-metadata run of the decode
    workload (for profiling that model on its own)."""
    prompt = np.random.default_rng(4).integers(0, 248320, 512, dtype=np.int32)
    a = bench_decode_asymmetric(args, prompt, None, [])
    return {"metric": METRIC, "value": a["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": a["ms_per_step"], "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "u4xf16->f32", "data": "synthetic",
            "config": {"workload": "batch-1 greedy decode of the 9B-shaped model written with the asymmetric "
                                   "quantiser's metadata, 512-token prefill and one untimed decode step, then "
                                   f"{args.steps} timed decode steps", **a}}


def cpu_baseline_decode(prompt, gpu_sess, runs=3):
    """The compiled reference customlib (oracle/_ref) on the same model files and
    host cores, timed by its own xq_metrics (decode tokens / decode ms,
    session.cpp:595-602); falls back to the oracle port.  Bounded sample: an
    8-token prompt and 4 greedy steps, one warmup run and `runs` measured runs
    (each xq_reset + xq_generate, as the reference harness,
    benchmark_jni.cpp:1324-1357).  The GPU session runs the same sample so the
    greedy ids, and the GPU's top-2 logit margin at each step, can be compared
    at full size."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle_bind as ob
    n_prompt, n_new = 8, 4
    sample = prompt[:n_prompt]
    threads = min(8, os.cpu_count() or 1)
    # GPU ids and margins, step by step (xq_get_debug_json top-k before each step)
    assert gpu_sess.prefill(sample)[0] == 0
    gpu_toks, margins = [], []
    for _ in range(n_new):
        st, txt = gpu_sess.json("xq_get_debug_json", 1 << 16)
        top = json.loads(txt)["lm_head_topk"] if st == 0 else []
        margins.append(round(top[0]["logit"] - top[1]["logit"], 5) if len(top) > 1 else None)
        st, tok, _ = gpu_sess.decode_one()
        gpu_toks.append(tok)
    h_gpu = gpu_sess.hidden()[1].astype(np.float64)
    if ob.ref_available():
        ref = xb.bind_xq_abi(ctypes.CDLL(ob.REF_SO))
        t0 = time.perf_counter()
        rs = xb.Session(MODEL_DIR, xb.options(backend=b"cpu", threads=threads), lib=ref)
        load_s = time.perf_counter() - t0
        tps, pre = [], []
        for r in range(1 + runs):
            assert ref.xq_reset(rs.h) == 0
            st, toks, m = rs.generate(sample, n_new)
            assert st == 0, m.error
            if r > 0:
                tps.append(m.decode_tokens_per_second)
                pre.append(m.prefill_tokens_per_second)
        h_cpu = rs.hidden()[1].astype(np.float64)
        rs.close()
        kind = "reference"
    else:
        t0 = time.perf_counter()
        om = ob.OracleModel(MODEL_DIR)
        load_s = time.perf_counter() - t0
        tps, pre = [], []
        for r in range(1 + runs):
            t1 = time.perf_counter()
            om.prefill(sample)
            t2 = time.perf_counter()
            toks = np.array([om.decode_one(n_prompt + i) for i in range(n_new)])
            t3 = time.perf_counter()
            if r > 0:
                tps.append(n_new / (t3 - t2))
                pre.append(n_prompt / (t2 - t1))
        h_cpu = np.asarray(om.hidden_state(), np.float64)
        kind = "port"
    match = [int(a) == int(b) for a, b in zip(gpu_toks, toks)]
    # the final-normed hidden after the sample's last step, GPU against CPU: ids
    # alone repeat one token on this random-init model (see the full-size
    # parity test for the per-state comparison)
    herr = np.abs(h_gpu - h_cpu)
    h_ok = bool(h_gpu.shape == h_cpu.shape and np.all(herr <= 1e-2 + 1e-3 * np.abs(h_cpu)))
    return {"value": round(float(np.mean(tps)), 4), "unit": "tokens/s", "cores": threads, "kind": kind,
            "sample": f"{n_prompt}-token prompt + {n_new} greedy decode steps on the same 9B-shaped model files, "
                      f"1 warmup + {runs} measured runs (reset + generate each), mean decode tok/s "
                      f"{', '.join(f'{t:.3f}' for t in tps)}; reference worker pool {threads} threads of "
                      f"{os.cpu_count()} host cores; load {load_s:.1f} s; prefill {np.mean(pre):.3f} tok/s",
            "runs_decode_tps": [round(t, 4) for t in tps],
            "greedy_ids_gpu": [int(t) for t in gpu_toks], "greedy_ids_cpu": [int(t) for t in toks],
            "greedy_ids_match": all(match), "gpu_top2_margins": margins,
            "hidden_max_abs_err": float(herr.max()) if herr.size else None,
            "hidden_within_1e-2_abs_1e-3_rel": h_ok}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--workload", default="decode",
                    choices=["decode", "decode-asym", "mlp", "gemv-sweep", "pmc-probe"])
    ap.add_argument("--bits", type=int, nargs="+", default=[4, 3, 2], help="gemv-sweep code widths")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 counter passes")
    ap.add_argument("--no-projections", action="store_true",
                    help="decode: skip the per-projection GEMV table (roofline fields null; for kernel traces)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-asymmetric", action="store_true",
                    help="decode: skip the second run on the model written with asymmetric-quantiser metadata")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); multi-GPU runs are not part of "
              f"this build", file=sys.stderr)
        sys.exit(2)
    if xb.hip().xqhip_device_count() < 1:
        print("no GPU visible to libxqhip", file=sys.stderr)
        sys.exit(1)
    xb.ck(xb.hip().xqhip_set_device(0))
    name = ctypes.create_string_buffer(256)
    xb.hip().xqhip_device_name(name, 256)
    log(f"[bench] device: {name.value.decode()}")
    res = {"decode": bench_decode, "decode-asym": bench_decode_asym_only, "mlp": bench_mlp,
           "gemv-sweep": bench_gemv_sweep, "pmc-probe": pmc_probe}[args.workload](args)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
