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
PRO_NONE, PRO_RMS, PRO_GATED_HEAD, PRO_GATED_HEAD_ACT = 0, 1, 2, 3
ATTN_PART_STRIDE, ATTN_MAX_SPLITS = 160, 8  # split attention workspace: partials, then counters
EPI_STORE, EPI_ADD, EPI_SILU_PAIR = 0, 1, 2
LAYOUT_TILED64, LAYOUT_GENERIC, LAYOUT_TILED64_F32META, LAYOUT_TILED64_SCALE16, LAYOUT_TILED64_F32S_Z4 = 0, 1, 2, 3, 4


class W4(ctypes.Structure):
    """Mirror of xqhip_w4 (include/xqhip.h)."""
    _fields_ = [("rows", ctypes.c_int32), ("cols", ctypes.c_int32), ("group", ctypes.c_int32),
                ("affine", ctypes.c_int32), ("layout", ctypes.c_int32), ("inexact_meta", ctypes.c_int32),
                ("bits", ctypes.c_int32), ("zero_is_8", ctypes.c_int32), ("nib", c_void_p), ("meta", c_void_p), ("nib_bytes", c_uint64), ("meta_bytes", c_uint64)]


class Prologue(ctypes.Structure):
    """Mirror of xqhip_prologue (include/xqhip.h)."""
    _fields_ = [("mode", ctypes.c_int32), ("head_dim", ctypes.c_int32), ("weight", c_void_p), ("gate", c_void_p),
                ("eps", c_float)]


class ChainSrc(ctypes.Structure):
    """Mirror of xqhip_chain_src (include/xqhip.h): a plain device vector, or
    (plain NULL) element `offset` on of op `op`'s output in the same chain."""
    _fields_ = [("plain", c_void_p), ("op", ctypes.c_int32), ("offset", ctypes.c_int32)]


class ChainOp(ctypes.Structure):
    """Mirror of xqhip_chain_op (include/xqhip.h)."""
    _fields_ = [("w", ctypes.POINTER(W4)), ("epi", ctypes.c_int32), ("pro", ctypes.c_int32), ("pro_w", c_void_p),
                ("head_dim", ctypes.c_int32), ("eps", c_float), ("x", ChainSrc), ("gate", ChainSrc),
                ("res", ChainSrc), ("y_plain", c_void_p)]


_P = ctypes.POINTER

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
    "xqhip_copy": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "xqhip_stream_synchronize": (c_int, [c_void_p]),
    "xqhip_device_synchronize": (c_int, []),
    "xqhip_event_create": (c_int, [ctypes.POINTER(c_void_p)]),
    "xqhip_event_destroy": (c_int, [c_void_p]),
    "xqhip_event_record": (c_int, [c_void_p, c_void_p]),
    "xqhip_event_synchronize": (c_int, [c_void_p]),
    "xqhip_event_elapsed_ms": (c_int, [c_void_p, c_void_p, ctypes.POINTER(c_float)]),
    "xqhip_event_query": (c_int, [c_void_p]),
    "xqhip_host_alloc_coherent": (c_int, [ctypes.POINTER(c_void_p), c_size_t]),
    "xqhip_host_free": (c_int, [c_void_p]),
    "xqhip_w4_upload": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, ctypes.POINTER(W4)]),
    "xqhip_wlb_upload": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                 ctypes.POINTER(W4)]),
    "xqhip_w4_free": (c_int, [ctypes.POINTER(W4)]),
    "xqhip_w4_weight_bytes": (c_uint64, [ctypes.POINTER(W4)]),
    "xqhip_gemv_w4a16": (c_int, [_P(W4), c_void_p, c_int, _P(Prologue), c_void_p, c_int, c_int, c_void_p]),
    "xqhip_argmax_workspace_bytes": (c_size_t, [c_int]),
    "xqhip_gemv_w4a16_argmax": (c_int, [_P(W4), c_void_p, c_int, _P(Prologue), c_void_p, c_void_p, c_void_p,
                                        c_void_p]),
    "xqhip_gemv_w4a16_argmax_publish": (c_int, [_P(W4), c_void_p, c_int, _P(Prologue), c_void_p, c_void_p, c_void_p,
                                                c_void_p, c_void_p, c_void_p]),
    "xqhip_gemv_w4a16_argmax_publish_embed": (c_int, [_P(W4), c_void_p, c_int, _P(Prologue), c_void_p, c_void_p,
                                                      c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p,
                                                      c_void_p]),
    "xqhip_gemv_w4a16_argmax_static": (c_int, [_P(W4), c_void_p, c_int, _P(Prologue), c_void_p, c_void_p,
                                               c_void_p]),
    "xqhip_embed_bf16": (c_int, [c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p]),
    "xqhip_rope_table": (c_int, [c_float, c_int, c_int, c_void_p]),
    "xqhip_attn_prep": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p,
                                c_float, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "xqhip_gqa_workspace_bytes": (c_size_t, [c_int, c_int, c_int]),
    "xqhip_gqa_decode": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p,
                                 c_void_p, c_void_p, c_void_p]),
    "xqhip_attn_decode": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p,
                                  c_void_p, c_float, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p,
                                  c_void_p, c_void_p]),
    "xqhip_attn_decode_head": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p,
                                       c_void_p, c_float, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_void_p]),
    "xqhip_attn_split_workspace_bytes": (c_size_t, [c_int]),
    "xqhip_attn_decode_split": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p,
                                        c_void_p, c_float, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p,
                                        c_void_p, c_void_p]),
    "xqhip_linear_conv": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p,
                                  c_void_p]),
    "xqhip_gated_delta": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int,
                                  c_int, c_void_p, c_void_p]),
    "xqhip_linear_attn_step": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p]),
    "xqhip_linear_attn_step_act": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                           c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p,
                                           c_void_p]),
    "xqhip_step_outproj_sync_bytes": (c_size_t, []),
    "xqhip_step_outproj_supported": (c_int, [_P(W4), c_int, c_int, c_int, c_int, c_int]),
    "xqhip_linear_attn_step_outproj": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                               c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p,
                                               c_void_p, _P(W4), c_void_p, c_float, c_void_p, c_void_p, c_void_p]),
    "xqhip_step_outproj_error": (c_int, [c_void_p, _P(c_int)]),
    "xqhip_gemm_workspace_bytes": (c_size_t, [c_int, c_int, c_int]),
    "xqhip_gemm_w4a16": (c_int, [_P(W4), c_void_p, c_int, c_int, _P(Prologue), c_int, c_void_p, c_int, c_int,
                                 c_void_p, c_size_t, c_void_p]),
    "xqhip_embed_bf16_batch": (c_int, [c_void_p, c_int, c_int, c_void_p, c_int, c_void_p, c_void_p]),
    "xqhip_attn_prep_batch": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p,
                                      c_void_p, c_float, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p, c_void_p,
                                      c_void_p, c_void_p, c_void_p]),
    "xqhip_prefill_attention": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                        c_void_p, c_void_p, c_int, c_void_p]),
    "xqhip_linear_attn_scan": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_int, c_void_p, c_void_p,
                                       c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_void_p, c_int,
                                       c_void_p]),
    "xqhip_linear_scan_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "xqhip_linear_attn_scan_ws": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_int, c_void_p, c_void_p,
                                          c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_void_p,
                                          c_int, c_void_p, c_void_p]),
    "xqhip_rmsnorm": (c_int, [c_void_p, c_void_p, c_int, c_float, c_void_p, c_void_p]),
    "xqhip_lds_fill": (c_int, [c_float, c_void_p]),
    "xqhip_timestamp": (c_int, [c_void_p, c_void_p]),
    "xqhip_chain_create": (c_int, [_P(ChainOp), c_int, _P(c_void_p)]),
    "xqhip_chain_destroy": (c_int, [c_void_p]),
    "xqhip_chain_arena_records": (c_size_t, [c_void_p]),
    "xqhip_chain_sync_bytes": (c_size_t, []),
    "xqhip_chain_launch": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p]),
    "xqhip_chain_launch_stamped": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "xqhip_chain_grid": (c_int, [c_void_p]),
    "xqhip_chain_error": (c_int, [c_void_p, _P(c_int)]),
    "xqhip_stream_create": (c_int, [_P(c_void_p)]),
    "xqhip_stream_destroy": (c_int, [c_void_p]),
    "xqhip_graph_begin": (c_int, [c_void_p]),
    "xqhip_graph_end": (c_int, [c_void_p, _P(c_void_p)]),
    "xqhip_graph_launch": (c_int, [c_void_p, c_void_p]),
    "xqhip_graph_destroy": (c_int, [c_void_p]),
}


def prologue(mode=PRO_NONE, weight=None, gate=None, head_dim=0, eps=1e-6):
    """Build an xqhip_prologue; weight/gate are DeviceBuffers (or None)."""
    return Prologue(mode, head_dim, weight.ptr if weight is not None else None,
                    gate.ptr if gate is not None else None, eps)

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
    """A W4A16 matrix uploaded into the device layout (xqhip_w4_upload), or with
    bits 3 / 2 a W3A16 / W2A16 bitstream matrix (xqhip_wlb_upload)."""

    def __init__(self, packed, scales, zeros, rows, cols, group=64, affine=0, bits=4):
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        scales = np.ascontiguousarray(scales, dtype=np.float32)
        zeros = np.ascontiguousarray(zeros, dtype=np.float32)
        self.w = W4()
        if bits == 4:
            ck(hip().xqhip_w4_upload(ptr(packed), ptr(scales), ptr(zeros), rows, cols, group, affine,
                                     ctypes.byref(self.w)))
        else:
            ck(hip().xqhip_wlb_upload(ptr(packed), ptr(scales), ptr(zeros), rows, cols, group, bits, affine,
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


# ---------------------------------------------------------------------------
# libxqwen35.so: the reference C ABI (include/xqwen35.h) + synthetic writer
# ---------------------------------------------------------------------------
XQ_OK, XQ_ERR_INVALID_ARGUMENT, XQ_ERR_NOT_READY, XQ_ERR_MODEL, XQ_ERR_RUNTIME, XQ_ERR_BUFFER_TOO_SMALL = \
    0, -1, -2, -3, -4, -5


class XqOptions(ctypes.Structure):
    _fields_ = [("struct_size", c_size_t), ("backend", c_char_p), ("threads", c_int), ("quant_bits", c_int),
                ("group_size", c_int), ("max_context_tokens", c_int), ("enable_autotune", c_int),
                ("use_mnn_fallback", c_int), ("telemetry_path", c_char_p)]


class XqMetrics(ctypes.Structure):
    _fields_ = [("struct_size", c_size_t), ("prompt_tokens", c_uint64), ("generated_tokens", c_uint64),
                ("load_ms", ctypes.c_double), ("prefill_ms", ctypes.c_double), ("first_token_ms", ctypes.c_double),
                ("decode_total_ms", ctypes.c_double), ("total_generate_ms", ctypes.c_double),
                ("prefill_tokens_per_second", ctypes.c_double), ("decode_tokens_per_second", ctypes.c_double),
                ("rss_kb", c_uint64), ("pss_kb", c_uint64), ("backend", ctypes.c_char * 64),
                ("selected_kernels", ctypes.c_char * 512), ("error", ctypes.c_char * 256)]


class SynthConfig(ctypes.Structure):
    """Mirror of xqsynth_config (include/xqsynth.h)."""
    _fields_ = [("seed", c_uint64), ("hidden_size", c_int32), ("intermediate_size", c_int32),
                ("vocab_size", c_int32), ("num_layers", c_int32), ("full_attention_interval", c_int32),
                ("num_attention_heads", c_int32), ("num_key_value_heads", c_int32), ("head_dim", c_int32),
                ("partial_rotary_factor", c_float), ("gated_q_proj", c_int32), ("linear_key_head_dim", c_int32),
                ("linear_value_head_dim", c_int32), ("linear_num_key_heads", c_int32),
                ("linear_num_value_heads", c_int32), ("linear_conv_kernel_dim", c_int32), ("group_size", c_int32),
                ("rms_norm_eps", c_float), ("rope_theta", c_float), ("scale_std", c_float), ("zero", c_float),
                ("embed_std", c_float), ("norm_std", c_float), ("threads", c_int32),
                ("asymmetric", c_int32)]


_S = c_void_p
XQ_SIGS = {
    "xq_create": (c_int, [c_char_p, _P(XqOptions), _P(_S)]),
    "xq_destroy": (None, [_S]),
    "xq_prefill": (c_int, [_S, c_void_p, c_size_t, _P(XqMetrics)]),
    "xq_decode_one": (c_int, [_S, _P(c_int32), _P(XqMetrics)]),
    "xq_generate": (c_int, [_S, c_void_p, c_size_t, c_size_t, c_void_p, c_size_t, _P(XqMetrics)]),
    "xq_reset": (c_int, [_S]),
    "xq_get_last_metrics": (c_int, [_S, _P(XqMetrics)]),
    "xq_get_backend_info": (c_int, [_S, c_char_p, c_size_t]),
    "xq_get_kernel_trace_json": (c_int, [_S, c_char_p, c_size_t]),
    "xq_get_debug_json": (c_int, [_S, c_char_p, c_size_t]),
    "xq_get_hidden_state": (c_int, [_S, c_void_p, c_size_t, _P(c_size_t)]),
    "xq_run_vulkan_w4a16_selftest": (c_int, [c_char_p, c_size_t]),
}
SYNTH_SIGS = {
    "xqsynth_default_config": (None, [_P(SynthConfig)]),
    "xqsynth_write_model": (c_int, [c_char_p, _P(SynthConfig), c_char_p, c_size_t]),
}


def xq():
    return _load("libxqwen35.so", {**XQ_SIGS, **SYNTH_SIGS})


def xq_path():
    return os.path.join(LIB_DIR, "libxqwen35.so")


def bind_xq_abi(lib):
    """Apply the xqwen35.h signatures to another library exporting the same ABI."""
    for fn, (res, args) in XQ_SIGS.items():
        f = getattr(lib, fn)
        f.restype = res
        f.argtypes = args
    return lib


def synth_config(**overrides):
    c = SynthConfig()
    xq().xqsynth_default_config(ctypes.byref(c))
    for k, v in overrides.items():
        setattr(c, k, v)
    return c


def write_synth_model(path, **overrides):
    cfg = synth_config(**overrides)
    err = ctypes.create_string_buffer(512)
    if xq().xqsynth_write_model(path.encode(), ctypes.byref(cfg), err, 512) != 0:
        raise RuntimeError("xqsynth_write_model: " + err.value.decode())
    return cfg


def options(backend=b"hip", max_context=8192, fallback=0, threads=8, group=64):
    o = XqOptions()
    o.struct_size = ctypes.sizeof(XqOptions)
    o.backend = backend
    o.threads = threads
    o.quant_bits = 4
    o.group_size = group
    o.max_context_tokens = max_context
    o.enable_autotune = 0
    o.use_mnn_fallback = fallback
    return o


class Session:
    """Thin wrapper over an xq_session of `lib` (this library or another with the same ABI)."""

    def __init__(self, model_dir, opts=None, lib=None):
        self.lib = lib or xq()
        self.h = c_void_p()
        self.status = self.lib.xq_create(model_dir.encode(), ctypes.byref(opts) if opts is not None else None,
                                         ctypes.byref(self.h))

    def ok(self):
        return self.status == XQ_OK and bool(self.h)

    def metrics(self):
        m = XqMetrics()
        m.struct_size = ctypes.sizeof(XqMetrics)
        self.lib.xq_get_last_metrics(self.h, ctypes.byref(m))
        return m

    def prefill(self, tokens):
        t = np.ascontiguousarray(tokens, np.int32)
        m = XqMetrics()
        m.struct_size = ctypes.sizeof(XqMetrics)
        return self.lib.xq_prefill(self.h, ptr(t), t.size, ctypes.byref(m)), m

    def decode_one(self):
        tok = c_int32()
        m = XqMetrics()
        m.struct_size = ctypes.sizeof(XqMetrics)
        st = self.lib.xq_decode_one(self.h, ctypes.byref(tok), ctypes.byref(m))
        return st, tok.value, m

    def generate(self, tokens, max_new):
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.zeros(max(1, max_new), np.int32)
        m = XqMetrics()
        m.struct_size = ctypes.sizeof(XqMetrics)
        st = self.lib.xq_generate(self.h, ptr(t), t.size, max_new, ptr(out), max_new, ctypes.byref(m))
        return st, out[:max_new].copy(), m

    def json(self, fn, cap=1 << 20):
        buf = ctypes.create_string_buffer(cap)
        st = getattr(self.lib, fn)(self.h, buf, cap)
        return st, buf.value.decode(errors="replace")

    def hidden(self, cap=None):
        n = c_size_t()
        if cap is None:
            self.lib.xq_get_hidden_state(self.h, None, 0, ctypes.byref(n))
            cap = n.value
        out = np.zeros(max(1, cap), np.float32)
        st = self.lib.xq_get_hidden_state(self.h, ptr(out), cap, ctypes.byref(n))
        return st, out[: n.value].copy() if st == XQ_OK else None, n.value

    def close(self):
        if self.h:
            self.lib.xq_destroy(self.h)
            self.h = c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
