"""ctypes bindings for the two product libraries (no torch: the HIP runtime in
the process is the one libxqhip.so links, never a second copy).

  hip()   -> libxqhip.so    thin C ABI over the gfx950 kernels (include/xqhip.h)
  xq()    -> libxqwen35.so  the reference C ABI (include/xqwen35.h)

Both raise RuntimeError when the library is missing: there is no fallback path.
"""
import ctypes
import os

import numpy as np

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_DIR = os.path.join(PKG, "lib")

c_int, c_float, c_size_t, c_void_p, c_char_p = ctypes.c_int, ctypes.c_float, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_char_p
c_uint64, c_int32, c_uint8 = ctypes.c_uint64, ctypes.c_int32, ctypes.c_uint8

F32, F16 = 0, 1
EPI_STORE, EPI_ADD, EPI_SILU_PAIR = 0, 1, 2
LAYOUT_TILED64, LAYOUT_GENERIC = 0, 1


class W4(ctypes.Structure):
    """Mirror of xqhip_w4 (include/xqhip.h)."""
    _fields_ = [("rows", ctypes.c_int32), ("cols", ctypes.c_int32), ("group", ctypes.c_int32),
                ("affine", ctypes.c_int32), ("layout", ctypes.c_int32), ("inexact_meta", ctypes.c_int32),
                ("nib", c_void_p), ("meta", c_void_p), ("nib_bytes", c_uint64), ("meta_bytes", c_uint64)]


_HIP_SIGS = {
    "xqhip_last_error": (c_char_p, []),
    "xqhip_device_count": (c_int, []),
    "xqhip_set_device": (c_int, [c_int]),
    "xqhip_device_name": (c_int, [c_char_p, c_size_t]),
    "xqhip_malloc": (c_int, [ctypes.POINTER(c_void_p), c_size_t]),
    "xqhip_free": (c_int, [c_void_p]),
    "xqhip_memcpy_h2d": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "xqhip_memcpy_d2h": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "xqhip_memcpy_d2d": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "xqhip_fill_u8": (c_int, [c_void_p, c_uint8, c_size_t, c_void_p]),
    "xqhip_stream_synchronize": (c_int, [c_void_p]),
    "xqhip_device_synchronize": (c_int, []),
    "xqhip_event_create": (c_int, [ctypes.POINTER(c_void_p)]),
    "xqhip_event_destroy": (c_int, [c_void_p]),
    "xqhip_event_record": (c_int, [c_void_p, c_void_p]),
    "xqhip_event_elapsed_ms": (c_int, [c_void_p, c_void_p, ctypes.POINTER(c_float)]),
    "xqhip_w4_upload": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, ctypes.POINTER(W4)]),
    "xqhip_w4_free": (c_int, [ctypes.POINTER(W4)]),
    "xqhip_w4_weight_bytes": (c_uint64, [ctypes.POINTER(W4)]),
    "xqhip_gemv_w4a16": (c_int, [ctypes.POINTER(W4), c_void_p, c_int, c_void_p, c_float, c_void_p, c_int, c_int,
                                 c_void_p]),
    "xqhip_argmax_workspace_bytes": (c_size_t, [c_int]),
    "xqhip_gemv_w4a16_argmax": (c_int, [ctypes.POINTER(W4), c_void_p, c_int, c_void_p, c_float, c_void_p, c_void_p,
                                        c_void_p, c_void_p]),
}

_cache = {}


def _load(name, sigs):
    if name in _cache:
        return _cache[name]
    path = os.path.join(LIB_DIR, name)
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built (run build.py); there is no CPU fallback")
    lib = ctypes.CDLL(path)
    for fn, (res, args) in sigs.items():
        f = getattr(lib, fn)
        f.restype = res
        f.argtypes = args
    _cache[name] = lib
    return lib


def hip():
    return _load("libxqhip.so", _HIP_SIGS)


def hip_path():
    return os.path.join(LIB_DIR, "libxqhip.so")


class HipError(RuntimeError):
    pass


def ck(rc):
    if rc != 0:
        raise HipError(f"xqhip error {rc}: {hip().xqhip_last_error().decode(errors='replace')}")
    return rc


def ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


class DeviceBuffer:
    """Owned device allocation made through libxqhip (hipMalloc)."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = c_void_p()
        ck(hip().xqhip_malloc(ctypes.byref(p), max(self.nbytes, 1)))
        self.ptr = p

    @classmethod
    def from_array(cls, a):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        ck(hip().xqhip_memcpy_h2d(b.ptr, ptr(a), a.nbytes, None))
        return b

    def upload(self, a):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        ck(hip().xqhip_memcpy_h2d(self.ptr, ptr(a), a.nbytes, None))

    def download(self, dtype, count):
        out = np.empty(count, dtype=dtype)
        assert out.nbytes <= self.nbytes
        ck(hip().xqhip_memcpy_d2h(ptr(out), self.ptr, out.nbytes, None))
        return out

    def zero(self):
        ck(hip().xqhip_fill_u8(self.ptr, 0, self.nbytes, None))

    def free(self):
        if self.ptr:
            hip().xqhip_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class DeviceW4:
    """A W4A16 matrix uploaded into the device layout (xqhip_w4_upload)."""

    def __init__(self, packed, scales, zeros, rows, cols, group=64, affine=0):
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        scales = np.ascontiguousarray(scales, dtype=np.float32)
        zeros = np.ascontiguousarray(zeros, dtype=np.float32)
        self.w = W4()
        ck(hip().xqhip_w4_upload(ptr(packed), ptr(scales), ptr(zeros), rows, cols, group, affine,
                                 ctypes.byref(self.w)))

    @property
    def ref(self):
        return ctypes.byref(self.w)

    def weight_bytes(self):
        return int(hip().xqhip_w4_weight_bytes(self.ref))

    def free(self):
        if self.w.nib:
            hip().xqhip_w4_free(self.ref)

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
