"""The checkpoint packer (python/xq4pack.py; reference:
customlib/packer/pack_qwen35_xq4_numpy.py).  The reference packer is not run
here, so its quantisers are pinned by hand-computed cases on exactly
representable values (half-to-even rounding at exact .5 steps, zero-point
clipping, constant groups, the fp16 alpha round trip), by the reconstruction
error bounds the schemes guarantee, and by the XQ4 reader of the oracle
(read_xq4, restating custom_model.cpp:218-262) loading the packed model."""
import json
import os
import struct

import numpy as np
import pytest

import oracle_bind as ob
import xq4pack as xp
from ckpt import CFG, make_checkpoint


def q1(values, scheme, alpha_fp16=False):
    w = np.asarray([values], np.float32)
    q, s, z = xp.quantize_w4(w, group=len(values), scheme=scheme, alpha_fp16=alpha_fp16)
    return q[0].tolist(), float(s[0, 0]), float(z[0, 0])


def test_asymmetric_known_answers():
    # s = 3.75 / 15 = 0.25 exactly, z = 0; 0.375 / 0.25 = 1.5 -> 2 and 0.625 / 0.25 = 2.5 -> 2 (half to even)
    assert q1([0.0, 0.375, 0.625, 3.75], "asymmetric") == ([0, 2, 2, 15], 0.25, 0.0)
    # min -1.25: z = rint(5.0) = 5; codes w / s + 5
    assert q1([-1.25, 0.0, 1.125, 2.5], "asymmetric") == ([0, 5, 10, 15], 0.25, 5.0)
    # all-positive group: -min / s = -4 clips to z = 0, so codes saturate at 15
    assert q1([1.0, 1.25, 2.5, 4.75], "asymmetric") == ([4, 5, 10, 15], 0.25, 0.0)
    # constant group: scale 1, z = rint(-2) clipped to 0, code rint(2) = 2
    assert q1([2.0, 2.0, 2.0, 2.0], "asymmetric") == ([2, 2, 2, 2], 1.0, 0.0)


def test_symmetric_known_answers():
    # max|w| = 3.5 -> s = 0.5, z = 8; 1.25 / 0.5 + 8 = 10.5 -> 10 (half to even)
    assert q1([-3.5, 0.0, 1.25, 3.5], "symmetric") == ([1, 8, 10, 15], 0.5, 8.0)
    assert q1([0.0, 0.0, 0.0, 0.0], "symmetric") == ([8, 8, 8, 8], 1.0, 8.0)


def test_affine_known_answers():
    # z = min = 1, s = 0.25; (1.625 - 1) / 0.25 = 2.5 -> 2
    assert q1([1.0, 1.625, 2.0, 4.75], "affine") == ([0, 2, 4, 15], 0.25, 1.0)


def test_affine_alpha_fp16_round_trip():
    rng = np.random.default_rng(3)
    w = rng.normal(0.3, 0.05, (16, 256)).astype(np.float32)
    q, s, z = xp.quantize_w4(w, 64, "affine", alpha_fp16=True)
    # the scale and the zero bias z + 8 s are the fp16-rounded pair of the exact path
    _, s0, z0 = xp.quantize_w4(w, 64, "affine")
    assert np.array_equal(s, s0.astype(np.float16).astype(np.float32))
    assert not np.array_equal(s, s0)  # the rounding happened
    # z + 8 s is the fp16-rounded zero bias of the exact path, up to the fp32 rounding of z
    zb, zb0 = (z + np.float32(8.0) * s).astype(np.float64), (z0 + np.float32(8.0) * s0).astype(np.float64)
    zb16 = zb0.astype(np.float16).astype(np.float64)
    assert np.allclose(zb, zb16, rtol=0, atol=1e-7)
    assert (np.abs(zb16 - zb0) <= np.abs(zb0) * 2.0 ** -11 * 1.0001).all()  # within half an fp16 ulp
    assert (np.abs(zb - zb0) > 1e-7).any()


@pytest.mark.parametrize("scheme", ["asymmetric", "symmetric", "affine"])
def test_reconstruction_error_bounds(scheme):
    rng = np.random.default_rng(1)
    w = rng.normal(0, 0.02, (64, 512)).astype(np.float32)
    q, s, z = xp.quantize_w4(w, 64, scheme)
    g = q.reshape(64, 8, 64).astype(np.float32)
    deq = (g * s[..., None] + z[..., None]) if scheme == "affine" else (g - z[..., None]) * s[..., None]
    err = np.abs(deq.reshape(64, 512) - w).reshape(64, 8, 64).max(axis=2)
    # symmetric and affine round once (half a step); asymmetric also rounds the zero point
    bound = (0.5 if scheme != "asymmetric" else 1.0) * s * (1 + 1e-5)
    assert (err <= bound).all()
    assert q.min() >= 0 and q.max() <= 15


@pytest.mark.parametrize("scheme,alpha", [("asymmetric", False), ("symmetric", False), ("affine", False),
                                          ("affine", True)])
def test_numpy_and_torch_quantisers_agree(scheme, alpha):
    rng = np.random.default_rng(2)
    w = rng.normal(0, 0.02, (96, 640)).astype(np.float32)
    w[3, :64] = 0.0  # constant group
    w[5, 64:128] = np.abs(w[5, 64:128]) + 0.01  # all-positive group
    a = xp.quantize_w4(w, 64, scheme, alpha)
    b = xp.quantize_w4(w, 64, scheme, alpha, device="cpu")
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


def test_xq4_header_and_nibble_order(tmp_path):
    codes = np.array([[1, 2, 3, 4, 5, 6, 7, 8]], np.uint8)
    assert xp.pack_nibbles(codes).tolist() == [[0x21, 0x43, 0x65, 0x87]]  # even column in the low nibble
    h = xp.xq4_header(3, 128, 64, 2)
    assert len(h) == 52 and h[:8] == b"XQW4A16\0"
    assert struct.unpack("<IIIII", h[8:28]) == (2, 3, 128, 64, 4)
    assert struct.unpack("<QQQ", h[28:52]) == (3 * 64, 6, 6)


@pytest.fixture(scope="module")
def packed(tmp_path_factory):
    src = str(tmp_path_factory.mktemp("ckpt"))
    tensors = make_checkpoint(src)
    out = str(tmp_path_factory.mktemp("pkg"))
    manifest = xp.pack_checkpoint(src, out, group_size=64)
    return src, out, tensors, manifest


def read_xq4(path):
    with open(path, "rb") as f:
        h = f.read(52)
        ver, rows, cols, group, bits = struct.unpack("<IIIII", h[8:28])
        nb, ns, nz = struct.unpack("<QQQ", h[28:52])
        packed = np.frombuffer(f.read(nb), np.uint8).reshape(rows, cols // 2)
        s = np.frombuffer(f.read(ns * 4), np.float32).reshape(rows, cols // group)
        z = np.frombuffer(f.read(nz * 4), np.float32).reshape(rows, cols // group)
        assert f.read() == b""
    codes = np.empty((rows, cols), np.uint8)
    codes[:, 0::2], codes[:, 1::2] = packed & 15, packed >> 4
    return ver, codes, s, z


def test_packed_package_layout(packed):
    src, out, tensors, manifest = packed
    c = CFG
    m = json.load(open(os.path.join(out, "xqwen35_manifest.json")))
    for k in ("hidden_size", "intermediate_size", "vocab_size", "num_attention_heads", "num_key_value_heads",
              "head_dim", "linear_key_head_dim", "linear_value_head_dim", "linear_num_key_heads",
              "linear_num_value_heads", "linear_conv_kernel_dim", "num_hidden_layers"):
        assert m[k] == c[k], k
    assert m["rope_theta"] == 1e7 and m["partial_rotary_factor"] == 0.25
    emb = np.fromfile(os.path.join(out, "embeddings_bf16.bin"), np.uint16).reshape(c["vocab_size"], -1)
    want = tensors["model.language_model.embed_tokens.weight"]
    assert np.array_equal((emb.astype(np.uint32) << 16).view(np.float32), want)  # bf16 copied bit for bit
    conv = np.fromfile(os.path.join(out, "layers_0_linear_attn_conv1d_weight.f32"), np.float32)
    assert np.array_equal(conv, tensors["model.language_model.layers.0.linear_attn.conv1d.weight"].reshape(-1))
    for name, path in [("lm_head.weight", "lm_head_weight.xq4"),
                       ("model.language_model.layers.3.self_attn.q_proj.weight", "layers_3_self_attn_q_proj_weight.xq4"),
                       ("model.language_model.layers.0.mlp.down_proj.weight", "layers_0_mlp_down_proj_weight.xq4")]:
        ver, codes, s, z = read_xq4(os.path.join(out, path))
        w = tensors[name]
        assert ver == 1 and codes.shape == w.shape
        deq = (codes.reshape(*s.shape, 64) - z[..., None]) * s[..., None]
        assert (np.abs(deq.reshape(w.shape) - w).reshape(*s.shape, 64).max(axis=2) <= s * 1.00001).all()


def test_oracle_model_runs_the_packed_checkpoint(packed):
    _, out, _, _ = packed
    om = ob.OracleModel(out)
    assert (om.hidden, om.vocab, om.n_layers, om.nq, om.hd) == (512, 4096, 4, 2, 128)
    om.prefill([3, 17, 400, 9])
    toks = [om.decode_one(4 + i) for i in range(3)]
    assert all(0 <= t < 4096 for t in toks)
    assert np.isfinite(om.hidden_state()).all()
