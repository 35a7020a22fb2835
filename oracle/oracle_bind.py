"""ctypes bindings for the oracle (liboracle.so) and the compiled reference
(_ref/libxqref.so).  TEST INFRASTRUCTURE ONLY: imported by tests/,
__graft_entry__.smoke() and the cpu_baseline leg of bench.py, never by the
product path.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libxqref.so")

_vp, _i, _f, _sz, _u64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t, ctypes.c_uint64

_GEMV = [_vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp]

_ORACLE_SIGS = {
    "orc_set_threads": (None, [_i]),
    "orc_threads": (_i, []),
    "orc_det_value": (_f, [_u64, _f]),
    "orc_det_fill": (None, [_vp, _u64, _f]),
    "orc_checksum": (_f, [_vp, _u64]),
    "orc_quantize_lowbit": (None, [_vp, _i, _i, _i, _i, _vp, _vp, _vp]),
    "orc_gemv_w4a16": (None, _GEMV),
    "orc_gemv_w4a16_argmax": (_i, _GEMV),
    "orc_gemv_textbook": (None, _GEMV),
    "orc_dequantize": (None, [_vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "orc_gemv_lowbit": (None, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _vp]),
    "orc_rmsnorm": (None, [_vp, _vp, _i, _f, _vp]),
    "orc_head_rms": (None, [_vp, _vp, _i, _i, _f]),
    "orc_l2norm_heads": (None, [_vp, _i, _i]),
    "orc_gated_head_rms": (None, [_vp, _vp, _vp, _i, _i, _f, _vp]),
    "orc_rope_partial": (None, [_vp, _i, _i, _i, _i, _f]),
    "orc_rope_full": (None, [_vp, _vp, _i, _i, _i, _f]),
    "orc_attention_ref": (None, [_vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "orc_attention_model": (None, [_vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "orc_gated_delta": (None, [_vp, _vp, _vp, _f, _f, _i, _i, _vp, _vp]),
    "orc_conv1d_step": (None, [_vp, _vp, _vp, _i, _i, _vp]),
    "orc_silu": (_f, [_f]),
    "orc_sigmoid": (_f, [_f]),
    "orc_softplus": (_f, [_f]),
    "orc_bf16_to_f32": (_f, [ctypes.c_uint16]),
    "orc_model_load": (_vp, [ctypes.c_char_p, ctypes.c_char_p, _sz]),
    "orc_model_free": (None, [_vp]),
    "orc_model_reset": (None, [_vp]),
    "orc_model_prefill": (_i, [_vp, _vp, _sz]),
    "orc_model_decode_one": (_i, [_vp, _vp, _sz]),
    "orc_model_dims": (_i, [_vp, _vp]),
    "orc_model_layer_is_full": (_i, [_vp, _i]),
    "orc_model_get_hidden": (None, [_vp, _vp]),
    "orc_model_set_hidden": (None, [_vp, _vp]),
    "orc_model_logits": (None, [_vp, _vp]),
    "orc_model_embed": (_i, [_vp, ctypes.c_int32]),
    "orc_model_run_layer": (None, [_vp, _i, _sz]),
    "orc_model_final_norm": (None, [_vp]),
    "orc_model_kv_len": (_sz, [_vp, _i]),
    "orc_model_get_kv": (None, [_vp, _i, _vp, _vp]),
    "orc_model_set_kv": (None, [_vp, _i, _vp, _vp, _sz]),
    "orc_model_get_linear_state": (None, [_vp, _i, _vp, _vp]),
    "orc_model_set_linear_state": (None, [_vp, _i, _vp, _vp]),
}

_REF_SIGS = {
    "ref_gemv_w4a16": (None, _GEMV),
    "ref_gemv_w4a16_argmax": (_i, _GEMV),
    "ref_gemv_textbook": (None, _GEMV),
    "ref_quantize_lowbit": (None, [_vp, _i, _i, _i, _i, _vp, _vp, _vp]),
    "ref_gemv_lowbit": (None, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _vp]),
    "ref_rmsnorm": (None, [_vp, _vp, _i, _f, _vp]),
    "ref_rope": (None, [_vp, _vp, _i, _i, _i, _f]),
    "ref_attention": (None, [_vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "ref_gated_delta": (None, [_vp, _vp, _vp, _f, _f, _i, _i, _vp, _vp]),
}


def _bind(path, sigs):
    lib = ctypes.CDLL(path)
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_libs = {}


def oracle():
    if "o" not in _libs:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"{ORACLE_SO} missing: run `make -C oracle`")
        _libs["o"] = _bind(ORACLE_SO, _ORACLE_SIGS)
    return _libs["o"]


def ref_available():
    return os.path.exists(REF_SO)


def ref():
    if "r" not in _libs:
        _libs["r"] = _bind(REF_SO, _REF_SIGS)
        _libs["r_abi"] = ctypes.CDLL(REF_SO)
    return _libs["r"]


def p(a):
    return ctypes.c_void_p(a.ctypes.data)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class Quantized:
    """A matrix in the reference QuantizedMatrix format (kernels.hpp:11-21)."""

    def __init__(self, packed, scales, zeros, rows, cols, group=64, affine=0):
        self.packed = np.ascontiguousarray(packed, dtype=np.uint8)
        self.scales = f32(scales)
        self.zeros = f32(zeros)
        self.rows, self.cols, self.group, self.affine = int(rows), int(cols), int(group), int(affine)

    def args(self):
        return (p(self.packed), p(self.scales), p(self.zeros), self.rows, self.cols, self.group, self.affine)


def gemv(q, x, lib=None, fn="orc_gemv_w4a16"):
    lib = lib or oracle()
    x = f32(x)
    y = np.empty(q.rows, np.float32)
    getattr(lib, fn)(*q.args(), p(x), p(y))
    return y


def gemv_argmax(q, x, lib=None, fn="orc_gemv_w4a16_argmax"):
    lib = lib or oracle()
    x = f32(x)
    best = np.zeros(1, np.float32)
    idx = getattr(lib, fn)(*q.args(), p(x), p(best))
    return int(idx), float(best[0])


def quantize_lowbit(w, rows, cols, bits=4, group=64, lib=None, fn="orc_quantize_lowbit"):
    lib = lib or oracle()
    w = f32(w)
    g = (cols + group - 1) // group
    packed = np.zeros((rows * cols * bits + 7) // 8, np.uint8)
    scales = np.empty(rows * g, np.float32)
    zeros = np.empty(rows * g, np.float32)
    getattr(lib, fn)(p(w), rows, cols, bits, group, p(packed), p(scales), p(zeros))
    return Quantized(packed, scales, zeros, rows, cols, group, 0)


def gemv_lowbit(q, bits, x, lib=None, fn="orc_gemv_lowbit"):
    """y = W x for a bitstream matrix of `bits`-bit codes (gemvLowBitReference)."""
    lib = lib or oracle()
    x = f32(x)
    y = np.empty(q.rows, np.float32)
    getattr(lib, fn)(p(q.packed), p(q.scales), p(q.zeros), q.rows, q.cols, q.group, bits, q.affine, p(x), p(y))
    return y


def det_fill(n, scale):
    a = np.empty(n, np.float32)
    oracle().orc_det_fill(p(a), n, scale)
    return a


def checksum(a):
    a = f32(a)
    return float(oracle().orc_checksum(p(a), a.size))


class OracleModel:
    """The oracle's restatement of CustomModel over a model directory."""

    def __init__(self, model_dir):
        err = ctypes.create_string_buffer(512)
        self.h = oracle().orc_model_load(model_dir.encode(), err, 512)
        if not self.h:
            raise RuntimeError("oracle model load failed: " + err.value.decode())
        d = np.zeros(16, np.int32)
        oracle().orc_model_dims(self.h, p(d))
        (self.hidden, self.inter, self.vocab, self.nq, self.nkv, self.hd, self.rot, self.lk_hd, self.lv_hd,
         self.lk_n, self.lv_n, self.ksz, self.n_layers) = [int(v) for v in d[:13]]

    def close(self):
        if self.h:
            oracle().orc_model_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def prefill(self, tokens):
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        if oracle().orc_model_prefill(self.h, p(t), t.size) != 0:
            raise RuntimeError("oracle prefill failed")

    def decode_one(self, pos):
        tok = np.zeros(1, np.int32)
        if oracle().orc_model_decode_one(self.h, p(tok), pos) != 0:
            raise RuntimeError("oracle decode failed")
        return int(tok[0])

    def hidden_state(self):
        out = np.empty(self.hidden, np.float32)
        oracle().orc_model_get_hidden(self.h, p(out))
        return out

    def set_hidden(self, h):
        h = f32(h)
        oracle().orc_model_set_hidden(self.h, p(h))

    def logits(self):
        out = np.empty(self.vocab, np.float32)
        oracle().orc_model_logits(self.h, p(out))
        return out

    def layer_is_full(self, i):
        return bool(oracle().orc_model_layer_is_full(self.h, i))

    def embed(self, tok):
        oracle().orc_model_embed(self.h, tok)

    def run_layer(self, i, pos):
        oracle().orc_model_run_layer(self.h, i, pos)

    def final_norm(self):
        oracle().orc_model_final_norm(self.h)

    def kv(self, i):
        n = oracle().orc_model_kv_len(self.h, i)
        k = np.empty(n * self.nkv * self.hd, np.float32)
        v = np.empty_like(k)
        oracle().orc_model_get_kv(self.h, i, p(k), p(v))
        return k.reshape(n, self.nkv, self.hd), v.reshape(n, self.nkv, self.hd)

    def set_kv(self, i, k, v):
        k, v = f32(k), f32(v)
        n = k.size // (self.nkv * self.hd)
        oracle().orc_model_set_kv(self.h, i, p(k), p(v), n)

    def linear_state(self, i):
        conv_dim = 2 * self.lk_hd * self.lk_n + self.lv_hd * self.lv_n
        conv = np.empty(conv_dim * (self.ksz - 1), np.float32)
        rec = np.empty(self.lv_n * self.lk_hd * self.lv_hd, np.float32)
        oracle().orc_model_get_linear_state(self.h, i, p(conv), p(rec))
        return conv, rec

    def set_linear_state(self, i, conv, rec):
        conv, rec = f32(conv), f32(rec)
        oracle().orc_model_set_linear_state(self.h, i, p(conv), p(rec))
