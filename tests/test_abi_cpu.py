"""C-ABI checks that need no GPU: both product libraries load and export every
symbol their headers declare; struct layouts match the reference header; the
session state machine, error codes and JSON getters behave like
customlib/runtime/session.cpp (compared against the compiled reference where
it is built)."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle_bind as ob
import xqbind as xb

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header, macro):
    text = open(os.path.join(ROOT, "include", header)).read()
    return sorted(set(re.findall(macro + r"[^;{]*?\b(x\w+)\s*\(", text)))


@pytest.mark.parametrize("header,macro,lib", [("xqhip.h", r"XQHIP_API", "hip"), ("xqwen35.h", r"XQ_API", "xq"),
                                              ("xqsynth.h", r"visibility\(\"default\"\)\)\)", "xq")])
def test_library_exports_every_declared_symbol(header, macro, lib):
    names = declared(header, macro)
    assert len(names) >= 2
    so = xb.hip() if lib == "hip" else xb.xq()
    missing = [n for n in names if not hasattr(so, n)]
    assert not missing, missing


def test_xqwen35_abi_has_the_reference_entry_points():
    """The twelve functions of customlib/include/xqwen35.h:60-77."""
    names = declared("xqwen35.h", r"XQ_API")
    assert names == sorted(["xq_create", "xq_destroy", "xq_prefill", "xq_decode_one", "xq_generate", "xq_reset",
                            "xq_get_last_metrics", "xq_get_backend_info", "xq_get_kernel_trace_json",
                            "xq_get_debug_json", "xq_get_hidden_state", "xq_run_vulkan_w4a16_selftest"])


def test_struct_layouts_match_reference_header():
    # size_t + 2 u64 + 7 double + 2 u64 + char[64] + char[512] + char[256]
    assert ctypes.sizeof(xb.XqMetrics) == 8 + 16 + 56 + 16 + 64 + 512 + 256
    assert ctypes.sizeof(xb.XqOptions) == 8 + 8 + 4 * 6 + 8


def test_null_arguments():
    lib = xb.xq()
    h = ctypes.c_void_p()
    assert lib.xq_create(None, None, ctypes.byref(h)) == xb.XQ_ERR_INVALID_ARGUMENT
    assert lib.xq_create(b"/nonexistent", None, None) == xb.XQ_ERR_INVALID_ARGUMENT
    assert lib.xq_prefill(None, None, 0, None) == xb.XQ_ERR_INVALID_ARGUMENT
    assert lib.xq_decode_one(None, None, None) == xb.XQ_ERR_INVALID_ARGUMENT
    assert lib.xq_reset(None) == xb.XQ_ERR_INVALID_ARGUMENT
    n = ctypes.c_size_t()
    assert lib.xq_get_hidden_state(None, None, 0, ctypes.byref(n)) == xb.XQ_ERR_INVALID_ARGUMENT


def libs_to_compare():
    out = [("product", xb.xq())]
    if ob.ref_available():
        out.append(("reference", xb.bind_xq_abi(ctypes.CDLL(ob.REF_SO))))
    return out


def run_dummy_session(lib, d):
    """NULL options -> the reference's model-less session (session.cpp:297-301, 364-367)."""
    s = xb.Session(d, None, lib=lib)
    assert s.ok()
    rec = []
    st, tok, m = s.decode_one()
    rec.append(("decode_before_prefill", st, m.error))
    st, m = s.prefill([])
    rec.append(("empty_prefill", st, m.error))
    st, m = s.prefill([5, 9, 2])
    rec.append(("prefill", st, m.prompt_tokens, m.generated_tokens))
    for _ in range(3):
        st, tok, m = s.decode_one()
        rec.append(("decode", st, tok, m.generated_tokens))
    st, out, m = s.generate([1, 2], 4)
    rec.append(("generate", st, out.tolist(), m.prompt_tokens, m.generated_tokens))
    t = np.zeros(1, np.int32)
    small = s.lib.xq_generate(s.h, xb.ptr(np.array([1], np.int32)), 1, 3, xb.ptr(t), 1, None)
    rec.append(("small_buffer", small))
    buf = ctypes.create_string_buffer(4)
    rec.append(("trace_too_small", s.lib.xq_get_kernel_trace_json(s.h, buf, 4)))
    rec.append(("trace_zero_cap", s.lib.xq_get_kernel_trace_json(s.h, buf, 0)))
    rec.append(("debug", s.json("xq_get_debug_json")))
    n = ctypes.c_size_t()
    rec.append(("hidden_no_model", s.lib.xq_get_hidden_state(s.h, None, 0, ctypes.byref(n))))
    # metrics honour a smaller struct_size (session.cpp:182-191)
    m = xb.XqMetrics()
    m.struct_size = 24
    m.load_ms = 123.0
    s.lib.xq_get_last_metrics(s.h, ctypes.byref(m))
    rec.append(("metrics_prefix", m.struct_size, m.load_ms))
    rec.append(("reset", s.lib.xq_reset(s.h), s.decode_one()[0]))
    s.close()
    return rec


def test_dummy_session_matches_reference(tmp_path):
    d = str(tmp_path / "m")
    os.makedirs(d)
    open(os.path.join(d, "xqwen35_manifest.json"), "w").write('{"vocab_size": 50, "hidden_size": 8}')
    results = {name: run_dummy_session(lib, d) for name, lib in libs_to_compare()}
    prod = results["product"]
    assert ("decode", 0, (2 + 1 + 3) % 50, 1) in prod
    if "reference" in results:
        assert prod == results["reference"]


def test_missing_model_is_a_model_error(tmp_path):
    for name, lib in libs_to_compare():
        s = xb.Session(str(tmp_path / "missing"), xb.options(backend=b"cpu"), lib=lib)
        assert s.status == xb.XQ_ERR_MODEL and not s.h, name


def test_library_without_gpu_refuses_to_load_a_model(tmp_path):
    """No CPU fallback: with no HIP device the real model path fails loudly."""
    if xb.hip().xqhip_device_count() > 0:
        pytest.skip("a GPU is visible")
    d = str(tmp_path / "m")
    xb.write_synth_model(d, hidden_size=128, intermediate_size=256, vocab_size=64, num_layers=1,
                         full_attention_interval=0, linear_num_key_heads=1, linear_num_value_heads=1,
                         linear_key_head_dim=64, linear_value_head_dim=64)
    s = xb.Session(d, xb.options())
    assert s.status == xb.XQ_ERR_MODEL


def test_synthetic_writer_is_deterministic(tmp_path):
    a, b = str(tmp_path / "a"), str(tmp_path / "b")
    kw = dict(hidden_size=128, intermediate_size=256, vocab_size=64, num_layers=2, num_attention_heads=2,
              num_key_value_heads=1, head_dim=64, linear_key_head_dim=64, linear_value_head_dim=64,
              linear_num_key_heads=1, linear_num_value_heads=2, full_attention_interval=2)
    xb.write_synth_model(a, **kw)
    xb.write_synth_model(b, **kw)
    files = sorted(os.listdir(a))
    assert files == sorted(os.listdir(b)) and "layers_1_self_attn_q_proj_weight.xq4" in files
    for f in files:
        assert open(os.path.join(a, f), "rb").read() == open(os.path.join(b, f), "rb").read(), f
    # distributions: codes uniform, zero 8, scales fp16-representable |N(0,0.02)|
    raw = open(os.path.join(a, "lm_head_weight.xq4"), "rb").read()
    rows, cols, group = np.frombuffer(raw[12:24], np.uint32)
    packed = np.frombuffer(raw[52:52 + rows * cols // 2], np.uint8)
    g = rows * cols // group
    scales = np.frombuffer(raw[52 + packed.size:52 + packed.size + 4 * g], np.float32)
    zeros = np.frombuffer(raw[52 + packed.size + 4 * g:], np.float32)
    assert np.all(zeros == 8.0) and np.array_equal(scales, scales.astype(np.float16).astype(np.float32))
    assert 0.01 < scales.mean() < 0.025 and np.all(scales >= 0)
    codes = np.concatenate([packed & 15, packed >> 4])
    assert abs(codes.mean() - 7.5) < 0.3


def read_xq4(path):
    """Header fields, codes, scales and zeros of an XQ4 file (custom_model.cpp:218-262)."""
    raw = open(path, "rb").read()
    assert raw[:7] == b"XQW4A16"
    version, rows, cols, group, bits = np.frombuffer(raw, np.uint32, 5, 8)
    n_packed, n_scales, n_zeros = np.frombuffer(raw, np.uint64, 3, 28)
    off = 52 + int(n_packed)
    scales = np.frombuffer(raw, np.float32, int(n_scales), off)
    zeros = np.frombuffer(raw, np.float32, int(n_zeros), off + 4 * int(n_scales))
    return int(version), int(rows), int(cols), scales, zeros


@pytest.mark.parametrize("asymmetric", [0, 1])
def test_synth_writer_metadata(tmp_path, asymmetric):
    """Default: fp16 scales, every zero 8.  asymmetric=1: the metadata of the
    asymmetric packer (fp32 scales, integer zeros 0..15 centred near 7.5)."""
    from tiny_model import SMALL
    xb.write_synth_model(str(tmp_path), **SMALL, asymmetric=asymmetric)
    files = sorted(p for p in os.listdir(tmp_path) if p.endswith(".xq4"))
    assert files
    for name in files[:6]:
        version, rows, cols, scales, zeros = read_xq4(os.path.join(tmp_path, name))
        assert version == 1 and scales.size == zeros.size == rows * ((cols + 63) // 64)
        f16_exact = scales.astype(np.float16).astype(np.float32) == scales
        if asymmetric:
            assert np.all(zeros == np.floor(zeros)) and zeros.min() >= 0 and zeros.max() <= 15
            assert 7.0 <= zeros.mean() <= 8.0 and np.unique(zeros).size >= 4
            assert f16_exact.mean() < 0.01
        else:
            assert np.all(zeros == 8.0) and f16_exact.all()
