"""W4A16 / W3A16 / W2A16 GEMV throughput against the HBM roofline.

For each code width and each decode-step matrix shape of the 9B-shaped model
(attention/output 4096x4096, interleaved gate/up 24576x4096, down 4096x12288,
lm_head 248320x4096) a random group-64 matrix is uploaded in several copies
(together more than twice the 256 MB last-level cache, so every launch streams
from HBM), n launches of xqhip_gemv_w4a16 (fp32 in and out, store epilogue) run
back to back on the default stream between two HIP events, and the report gives
the average duration and the algorithmic bytes per launch (codes + fp16 group
metadata + x + y) over it, as GB/s and as a fraction of the 8 TB/s HBM peak.

    python gemv_sweep.py [--bits 4 3 2] [--n 200] [--json]
"""
import argparse
import ctypes
import json
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import xqbind as xb  # noqa: E402

HBM_PEAK = 8.0e12
SHAPES = [("attention_4096x4096", 4096, 4096), ("gate_up_24576x4096", 24576, 4096),
          ("down_4096x12288", 4096, 12288), ("lm_head_248320x4096", 248320, 4096)]


def matrix(rows, cols, bits, seed):
    rng = np.random.default_rng(seed)
    g = cols // 64
    packed = rng.integers(0, 256, (rows * cols * bits + 7) // 8, dtype=np.uint8)
    scales = np.abs(rng.normal(0.0, 0.02, rows * g)).astype(np.float16).astype(np.float32)
    zeros = rng.integers(0, 1 << bits, rows * g).astype(np.float32)
    return packed, scales, zeros


def time_shape(rows, cols, bits, n):
    hip = xb.hip()
    packed, scales, zeros = matrix(rows, cols, bits, rows + bits)
    one = rows * cols * bits // 8
    ncopy = max(2, min(16, -(-(600 << 20) // one)))
    copies = [xb.DeviceW4(packed, scales, zeros, rows, cols, 64, 0, bits=bits) for _ in range(ncopy)]
    x = xb.DeviceBuffer.from_array(np.random.default_rng(1).normal(0, 1, cols).astype(np.float32))
    y = xb.DeviceBuffer(rows * 4)

    def launch(i):
        xb.ck(hip.xqhip_gemv_w4a16(copies[i % ncopy].ref, x.ptr, xb.F32, None, y.ptr, xb.F32, xb.EPI_STORE, None))

    for i in range(2 * ncopy):
        launch(i)
    a, b = ctypes.c_void_p(), ctypes.c_void_p()
    xb.ck(hip.xqhip_event_create(ctypes.byref(a)))
    xb.ck(hip.xqhip_event_create(ctypes.byref(b)))
    xb.ck(hip.xqhip_event_record(a, None))
    for i in range(n):
        launch(i)
    xb.ck(hip.xqhip_event_record(b, None))
    xb.ck(hip.xqhip_stream_synchronize(None))
    ms = ctypes.c_float()
    xb.ck(hip.xqhip_event_elapsed_ms(a, b, ctypes.byref(ms)))
    hip.xqhip_event_destroy(a)
    hip.xqhip_event_destroy(b)
    us = ms.value * 1e3 / n
    algo = copies[0].weight_bytes() + cols * 4 + rows * 4
    del copies
    return {"bits": bits, "rows": rows, "cols": cols, "us": round(us, 2), "bytes": algo,
            "gbps": round(algo / us / 1e3, 1), "frac": round(algo / (us * 1e-6) / HBM_PEAK, 3)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--bits", type=int, nargs="+", default=[4, 3, 2])
    ap.add_argument("--n", type=int, default=200)
    ap.add_argument("--json", action="store_true")
    a = ap.parse_args()
    xb.ck(xb.hip().xqhip_set_device(0))
    for bits in a.bits:
        for name, rows, cols in SHAPES:
            r = time_shape(rows, cols, bits, a.n)
            r["shape"] = name
            if a.json:
                print(json.dumps(r), flush=True)
            else:
                print(f"W{bits}A16 {name:22s} {r['us']:8.2f} us  {r['bytes'] / 1e6:8.2f} MB  "
                      f"{r['gbps']:7.1f} GB/s  frac {r['frac']:.3f}", flush=True)


if __name__ == "__main__":
    main()
