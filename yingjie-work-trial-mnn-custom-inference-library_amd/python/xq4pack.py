#!/usr/bin/env python3
"""xq4pack.py - a Qwen3.5 safetensors checkpoint -> the XQ4 model package that
the decode library loads (xqwen35_manifest.json, embeddings_bf16.bin, *.f32
vectors, *.xq4 matrices; the layout read by customlib/runtime/custom_model.cpp
:185-262, 423-553).

It follows the reference packer customlib/packer/pack_qwen35_xq4_numpy.py:
the tensor list per layer type (:40-78), the file names (`model.language_model.`
dropped, dots -> underscores, :28-29), the 52-byte XQ4 header (:166-188) and
the three group quantisers of pack_matrix_w4 (:191-247):

  asymmetric (default)  s = (max - min) / 15 (1 if 0), z = rint(-min / s)
                        clipped to [0, 15], q = clip(rint(w / s + z)); XQ4 v1,
                        w ~ (q - z) s
  symmetric             s = max|w| / 7 (1 if 0), z = 8, q = clip(rint(w / s + 8));
                        XQ4 v1
  affine (MNN)          s as asymmetric, z = min, q = clip(rint((w - z) / s));
                        XQ4 v2, w ~ q s + z.  With alpha_fp16 the pair
                        (min + 8 s, s) is rounded through fp16 first and
                        z = fp16(min + 8 s) - 8 fp16(s).

All arithmetic is elementwise float32 with round-half-to-even (np.rint), so
the numpy path and the optional torch path (device "cuda" runs the quantiser
on the GPU) give the same bytes.  Beyond the reference packer it also writes
embeddings_bf16.bin (the reference copies it from an MNN export) and takes
lm_head from the embedding table when the checkpoint ties them.  Default
group size 64, the layout of the GPU's fast kernels (the reference's default
is 128, which the library runs through its generic kernels).
"""
import argparse
import json
import os
import pathlib
import struct
import sys

import numpy as np

MAGIC = b"XQW4A16\0"
SCHEMES = ("asymmetric", "symmetric", "affine")
_ITEM = {"BF16": 2, "F16": 2, "F32": 4}


def file_name(tensor, prefix="model.language_model."):
    """Package file stem of a checkpoint tensor name: the model prefix dropped,
    dots -> underscores (pack_qwen35_xq4_numpy.py:28-29)."""
    if tensor.startswith(prefix):
        tensor = tensor[len(prefix):]
    return tensor.replace(".", "_")


def bf16_bits_to_f32(u16):
    return (np.asarray(u16, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x):
    """Round to nearest even (the embedding table of an fp32 / fp16 checkpoint)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


class Checkpoint:
    """The tensors of a Hugging Face safetensors checkpoint directory: shards
    listed by model.safetensors.index.json, or one model.safetensors.  Reads
    are memory-mapped and converted to float32 a row range at a time."""

    def __init__(self, model_dir):
        self.dir = pathlib.Path(model_dir)
        index = self.dir / "model.safetensors.index.json"
        if index.exists():
            self.weight_map = json.loads(index.read_text(encoding="utf-8"))["weight_map"]
        else:
            single = self.dir / "model.safetensors"
            if not single.exists():
                raise FileNotFoundError(f"{self.dir}: no model.safetensors(.index.json)")
            header, _ = self._read_header(single)
            self.weight_map = {k: single.name for k in header if k != "__metadata__"}
        self._shards = {}

    @staticmethod
    def _read_header(path):
        with open(path, "rb") as f:
            n = struct.unpack("<Q", f.read(8))[0]
            header = json.loads(f.read(n).decode("utf-8"))
        return header, 8 + n

    def _shard(self, name):
        shard = self.weight_map[name]
        if shard not in self._shards:
            path = self.dir / shard
            header, base = self._read_header(path)
            self._shards[shard] = (header, base, np.memmap(path, dtype=np.uint8, mode="r"))
        return self._shards[shard]

    def has(self, name):
        return name in self.weight_map

    def meta(self, name):
        header, _, _ = self._shard(name)
        item = header[name]
        if item["dtype"] not in _ITEM:
            raise ValueError(f"{name}: unsupported dtype {item['dtype']}")
        return item["dtype"], [int(d) for d in item["shape"]]

    def _raw(self, name, first, count):
        """`count` elements from element `first` of the tensor, as stored."""
        header, base, mm = self._shard(name)
        item = header[name]
        dtype = item["dtype"]
        size = _ITEM[dtype]
        start = base + int(item["data_offsets"][0]) + first * size
        raw = mm[start:start + count * size]
        if raw.size != count * size:
            raise IOError(f"{name}: short read")
        return raw.view({"BF16": "<u2", "F16": "<f2", "F32": "<f4"}[dtype]), dtype

    def rows(self, name, r0, n):
        """float32 [n][cols] of rows r0..r0+n-1 of a 2-D tensor (a 1-D tensor is one column)."""
        _, shape = self.meta(name)
        cols = int(np.prod(shape[1:])) if len(shape) > 1 else 1
        raw, dtype = self._raw(name, r0 * cols, n * cols)
        if dtype == "BF16":
            out = bf16_bits_to_f32(raw)
        else:
            out = raw.astype(np.float32)
        return np.array(out, np.float32).reshape(n, cols)

    def tensor(self, name):
        _, shape = self.meta(name)
        n = shape[0] if shape else 1
        return self.rows(name, 0, n).reshape(shape)

    def bf16_rows(self, name, r0, n):
        """Rows as bf16 bits: copied for a bf16 tensor, rounded otherwise."""
        dtype, shape = self.meta(name)
        cols = int(np.prod(shape[1:]))
        if dtype == "BF16":
            raw, _ = self._raw(name, r0 * cols, n * cols)
            return np.array(raw, np.uint16).reshape(n, cols)
        return f32_to_bf16_bits(self.rows(name, r0, n)).reshape(n, cols)


# ---------------------------------------------------------------------------
# group quantisers (pack_qwen35_xq4_numpy.py:213-244)
# ---------------------------------------------------------------------------
def _np_quant(w, group, scheme, alpha_fp16):
    rows, cols = w.shape
    g = w.reshape(rows, cols // group, group)
    lo, hi = g.min(axis=2), g.max(axis=2)
    if scheme == "symmetric":
        s = (np.abs(g).max(axis=2) / np.float32(7.0)).astype(np.float32)
        s = np.where(s > 0, s, np.float32(1.0)).astype(np.float32)
        z = np.full_like(s, np.float32(8.0))
        t = g / s[..., None] + np.float32(8.0)
    else:
        s = ((hi - lo) / np.float32(15.0)).astype(np.float32)
        s = np.where(s > 0, s, np.float32(1.0)).astype(np.float32)
        if scheme == "affine":
            if alpha_fp16:
                s16 = s.astype(np.float16).astype(np.float32)
                zb16 = (lo + np.float32(8.0) * s).astype(np.float16).astype(np.float32)
                s, z = s16, (zb16 - np.float32(8.0) * s16).astype(np.float32)
            else:
                z = lo.astype(np.float32)
            t = (g - z[..., None]) / s[..., None]
        else:
            # (+ 0: a zero point of -0.0, from a group minimum of +0.0, is stored as +0.0)
            z = (np.clip(np.rint(-lo / s), np.float32(0.0), np.float32(15.0)) + np.float32(0.0)).astype(np.float32)
            t = g / s[..., None] + z[..., None]
    q = np.clip(np.rint(t), 0, 15).astype(np.uint8).reshape(rows, cols)
    return q, s.astype(np.float32), z.astype(np.float32)


def _torch_quant(w, group, scheme, alpha_fp16, device):
    import torch
    g = torch.from_numpy(np.ascontiguousarray(w)).to(device).reshape(w.shape[0], -1, group)
    one, eight, fifteen, seven = (torch.tensor(v, dtype=torch.float32, device=device) for v in (1.0, 8.0, 15.0, 7.0))
    lo, hi = g.amin(dim=2), g.amax(dim=2)
    if scheme == "symmetric":
        s = g.abs().amax(dim=2) / seven
        s = torch.where(s > 0, s, one)
        z = torch.full_like(s, 8.0)
        t = g / s[..., None] + eight
    else:
        s = (hi - lo) / fifteen
        s = torch.where(s > 0, s, one)
        if scheme == "affine":
            if alpha_fp16:
                s16 = s.half().float()
                zb16 = (lo + eight * s).half().float()
                s, z = s16, zb16 - eight * s16
            else:
                z = lo
            t = (g - z[..., None]) / s[..., None]
        else:
            z = torch.clamp(torch.round(-lo / s), 0.0, 15.0) + 0.0
            t = g / s[..., None] + z[..., None]
    q = torch.clamp(torch.round(t), 0, 15).to(torch.uint8).reshape(w.shape)
    return q.cpu().numpy(), s.cpu().numpy().astype(np.float32), z.cpu().numpy().astype(np.float32)


def quantize_w4(w, group=64, scheme="asymmetric", alpha_fp16=False, device=None):
    """Codes [rows][cols] u8 in 0..15, scales and zeros [rows][cols/group] f32."""
    w = np.ascontiguousarray(w, np.float32)
    if scheme not in SCHEMES:
        raise ValueError(f"unknown scheme {scheme}")
    if alpha_fp16 and scheme != "affine":
        raise ValueError("alpha_fp16 needs the affine scheme")
    if w.ndim != 2 or w.shape[1] % group != 0:
        raise ValueError(f"shape {w.shape} is not [rows][k*{group}]")
    if device and device != "numpy":
        return _torch_quant(w, group, scheme, alpha_fp16, device)
    return _np_quant(w, group, scheme, alpha_fp16)


def pack_nibbles(codes):
    """Two codes per byte, the even column in the low nibble (custom_model.cpp:218-262)."""
    codes = np.asarray(codes, np.uint8)
    return (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)


def xq4_header(rows, cols, group, version):
    packed = rows * cols // 2
    meta = rows * (cols // group)
    return struct.pack("<8sIIIIIQQQ", MAGIC, version, rows, cols, group, 4, packed, meta, meta)


def write_xq4_matrix(path, rows_fn, rows, cols, group, scheme, alpha_fp16, device, chunk_rows):
    """Streams the matrix through the quantiser `chunk_rows` rows at a time."""
    version = 2 if scheme == "affine" else 1
    scales = np.empty((rows, cols // group), np.float32)
    zeros = np.empty_like(scales)
    with open(path, "wb") as f:
        f.write(xq4_header(rows, cols, group, version))
        for r0 in range(0, rows, chunk_rows):
            n = min(chunk_rows, rows - r0)
            q, s, z = quantize_w4(rows_fn(r0, n), group, scheme, alpha_fp16, device)
            f.write(pack_nibbles(q).tobytes())
            scales[r0:r0 + n], zeros[r0:r0 + n] = s, z
        f.write(scales.tobytes())
        f.write(zeros.tobytes())
    return {"file": os.path.basename(path), "rows": rows, "cols": cols, "bits": 4, "group_size": group,
            "format_version": version, "scheme": scheme, "alpha_fp16": bool(alpha_fp16)}


def read_config(model_dir):
    cfg = json.loads((pathlib.Path(model_dir) / "config.json").read_text(encoding="utf-8"))
    return cfg.get("text_config", cfg)


def tensor_plan(ck, cfg, limit_layers=0):
    """(prefix, matrices, vectors) in the reference's order; prefix is the
    checkpoint's layer-tensor prefix (`model.language_model.` or `model.`)."""
    prefix = "model.language_model." if ck.has("model.language_model.embed_tokens.weight") else "model."
    n_layers = int(cfg["num_hidden_layers"])
    if limit_layers > 0:
        n_layers = min(n_layers, limit_layers)
    types = cfg.get("layer_types") or ["full_attention" if i % 4 == 3 else "linear_attention" for i in range(n_layers)]
    mats, vecs = [], [prefix + "norm.weight"]
    for i in range(n_layers):
        p = f"{prefix}layers.{i}."
        vecs += [p + "input_layernorm.weight", p + "post_attention_layernorm.weight"]
        mats += [p + "mlp.gate_proj.weight", p + "mlp.up_proj.weight", p + "mlp.down_proj.weight"]
        if types[i] == "full_attention":
            mats += [p + f"self_attn.{n}_proj.weight" for n in ("q", "k", "v", "o")]
            vecs += [p + "self_attn.q_norm.weight", p + "self_attn.k_norm.weight"]
        else:
            mats += [p + f"linear_attn.{n}.weight" for n in ("in_proj_qkv", "in_proj_a", "in_proj_b", "in_proj_z",
                                                              "out_proj")]
            vecs += [p + "linear_attn.norm.weight", p + "linear_attn.conv1d.weight", p + "linear_attn.A_log",
                     p + "linear_attn.dt_bias"]
    return prefix, n_layers, types[:n_layers], mats, vecs


def pack_checkpoint(model_dir, out_dir, group_size=64, scheme="asymmetric", alpha_fp16=False, limit_layers=0,
                    device=None, chunk_rows=1024, log=None):
    """Writes the package; returns the manifest dict."""
    ck = Checkpoint(model_dir)
    cfg = read_config(model_dir)
    out = pathlib.Path(out_dir)
    out.mkdir(parents=True, exist_ok=True)
    prefix, n_layers, types, mats, vecs = tensor_plan(ck, cfg, limit_layers)
    say = log or (lambda m: None)
    embed = prefix + "embed_tokens.weight"
    _, (vocab, hidden) = ck.meta(embed)
    with open(out / "embeddings_bf16.bin", "wb") as f:
        for r0 in range(0, vocab, chunk_rows):
            f.write(ck.bf16_rows(embed, r0, min(chunk_rows, vocab - r0)).tobytes())
    say(f"embeddings {vocab}x{hidden} -> embeddings_bf16.bin")
    matrices, vectors = {}, {}
    head = "lm_head.weight" if ck.has("lm_head.weight") else embed  # tied embeddings
    for name in [head] + mats:
        dst = "lm_head_weight.xq4" if name == head else file_name(name, prefix) + ".xq4"
        _, shape = ck.meta(name)
        if len(shape) != 2:
            raise ValueError(f"{name}: matrix expected, shape {shape}")
        rows, cols = shape
        matrices[name] = write_xq4_matrix(out / dst, lambda r0, n, nm=name: ck.rows(nm, r0, n), rows, cols,
                                          group_size, scheme, alpha_fp16, device, chunk_rows)
        say(f"{name} {rows}x{cols} -> {dst}")
    for name in vecs:
        if not ck.has(name):
            continue
        arr = ck.tensor(name).astype(np.float32).reshape(-1)
        dst = file_name(name, prefix) + ".f32"
        arr.tofile(out / dst)
        vectors[name] = {"file": dst, "elements": int(arr.size), "dtype": "float32"}
        say(f"{name} -> {dst}")
    rope = cfg.get("rope_parameters") or {}
    manifest = {
        "format": "xqwen35_custom_w4a16",
        "hf_repo": cfg.get("_name_or_path", "local-checkpoint"),
        "quantization": {"bits": 4, "group_size": group_size, "scheme": "w4a16_groupwise_" + scheme,
                         "alpha_fp16": bool(alpha_fp16)},
        "hidden_size": int(cfg["hidden_size"]),
        "intermediate_size": int(cfg["intermediate_size"]),
        "num_hidden_layers": n_layers,
        "num_attention_heads": int(cfg["num_attention_heads"]),
        "num_key_value_heads": int(cfg["num_key_value_heads"]),
        "head_dim": int(cfg.get("head_dim", int(cfg["hidden_size"]) // int(cfg["num_attention_heads"]))),
        "linear_key_head_dim": int(cfg.get("linear_key_head_dim", 128)),
        "linear_value_head_dim": int(cfg.get("linear_value_head_dim", 128)),
        "linear_num_key_heads": int(cfg.get("linear_num_key_heads", 16)),
        "linear_num_value_heads": int(cfg.get("linear_num_value_heads", 32)),
        "linear_conv_kernel_dim": int(cfg.get("linear_conv_kernel_dim", 4)),
        "vocab_size": int(cfg.get("vocab_size", vocab)),
        "layer_types": types,
        "rms_norm_eps": float(cfg.get("rms_norm_eps", 1e-6)),
        "rope_theta": float(rope.get("rope_theta", cfg.get("rope_theta", 1e7))),
        "partial_rotary_factor": float(rope.get("partial_rotary_factor", cfg.get("partial_rotary_factor", 0.25))),
        "matrices": matrices,
        "vectors": vectors,
    }
    (out / "xqwen35_manifest.json").write_text(json.dumps(manifest, indent=2), encoding="utf-8")
    return manifest


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--model-dir", required=True, help="safetensors checkpoint directory with config.json")
    ap.add_argument("--out-dir", required=True)
    ap.add_argument("--group-size", type=int, default=64)
    ap.add_argument("--symmetric", action="store_true", help="signed symmetric codes, zero 8")
    ap.add_argument("--mnn-affine-asym", action="store_true", help="XQ4 v2: w = q * scale + min")
    ap.add_argument("--mnn-alpha-fp16", action="store_true", help="round the affine (min + 8 scale, scale) via fp16")
    ap.add_argument("--limit-layers", type=int, default=0)
    ap.add_argument("--chunk-rows", type=int, default=1024)
    ap.add_argument("--device", default=None, help="torch device for the quantiser, e.g. cuda (default numpy)")
    a = ap.parse_args(argv)
    if a.symmetric and a.mnn_affine_asym:
        ap.error("--symmetric and --mnn-affine-asym are mutually exclusive")
    if a.mnn_alpha_fp16 and not a.mnn_affine_asym:
        ap.error("--mnn-alpha-fp16 needs --mnn-affine-asym")
    scheme = "symmetric" if a.symmetric else ("affine" if a.mnn_affine_asym else "asymmetric")
    m = pack_checkpoint(a.model_dir, a.out_dir, a.group_size, scheme, a.mnn_alpha_fp16, a.limit_layers, a.device,
                        a.chunk_rows, log=lambda s: print(s, flush=True))
    print(json.dumps({"out_dir": a.out_dir, "matrices": len(m["matrices"]), "vectors": len(m["vectors"])}))
    return 0


if __name__ == "__main__":
    sys.exit(main())
