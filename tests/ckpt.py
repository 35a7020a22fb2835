"""A small random Qwen3.5-layout safetensors checkpoint for the packer tests
(tensor names and shapes as pack_qwen35_xq4_numpy.py:40-78 reads them; bf16
payloads written directly in the safetensors format: u64 header length,
JSON header, raw little-endian data)."""
import json
import os
import struct

import numpy as np

# the SMALL synthetic model's shapes (tiny_model.SMALL): 3 linear-attention layers + 1 full
CFG = dict(hidden_size=512, intermediate_size=960, vocab_size=4096, num_hidden_layers=4, num_attention_heads=2,
           num_key_value_heads=1, head_dim=128, linear_key_head_dim=128, linear_value_head_dim=128,
           linear_num_key_heads=1, linear_num_value_heads=2, linear_conv_kernel_dim=4,
           layer_types=["linear_attention"] * 3 + ["full_attention"], rms_norm_eps=1e-6,
           rope_parameters={"rope_theta": 10000000.0, "partial_rotary_factor": 0.25}, tie_word_embeddings=False)


def to_bf16_bits(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def write_safetensors(path, tensors):
    """tensors: name -> float32 array, stored as bf16."""
    header, blobs, off = {}, [], 0
    for name in sorted(tensors):
        a = np.asarray(tensors[name], np.float32)
        raw = to_bf16_bits(a).tobytes()
        header[name] = {"dtype": "BF16", "shape": list(a.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    hj = json.dumps(header).encode()
    hj += b" " * ((8 - len(hj) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hj)))
        f.write(hj)
        for b in blobs:
            f.write(b)


def make_checkpoint(d, seed=11, shards=2):
    """Writes config.json, model-0000k-of-0000n.safetensors and the index; returns the float32 tensors."""
    os.makedirs(d, exist_ok=True)
    c = CFG
    rng = np.random.default_rng(seed)
    H, I, V = c["hidden_size"], c["intermediate_size"], c["vocab_size"]
    nq, nkv, hd = c["num_attention_heads"], c["num_key_value_heads"], c["head_dim"]
    lk = c["linear_key_head_dim"] * c["linear_num_key_heads"]
    lv = c["linear_value_head_dim"] * c["linear_num_value_heads"]
    conv = 2 * lk + lv
    n = lambda *s, std=0.02, mean=0.0: (mean + std * rng.standard_normal(s)).astype(np.float32)
    pre = "model.language_model."
    t = {pre + "embed_tokens.weight": n(V, H, std=1.0), "lm_head.weight": n(V, H), pre + "norm.weight": n(H, std=0.1)}
    for i, kind in enumerate(c["layer_types"]):
        p = f"{pre}layers.{i}."
        t[p + "input_layernorm.weight"] = n(H, std=0.1)
        t[p + "post_attention_layernorm.weight"] = n(H, std=0.1)
        t[p + "mlp.gate_proj.weight"] = n(I, H)
        t[p + "mlp.up_proj.weight"] = n(I, H)
        t[p + "mlp.down_proj.weight"] = n(H, I)
        if kind == "full_attention":
            t[p + "self_attn.q_proj.weight"] = n(2 * nq * hd, H)  # gated: [q | gate] per head
            t[p + "self_attn.k_proj.weight"] = n(nkv * hd, H)
            t[p + "self_attn.v_proj.weight"] = n(nkv * hd, H)
            t[p + "self_attn.o_proj.weight"] = n(H, nq * hd)
            t[p + "self_attn.q_norm.weight"] = n(hd, std=0.1)
            t[p + "self_attn.k_norm.weight"] = n(hd, std=0.1)
        else:
            t[p + "linear_attn.in_proj_qkv.weight"] = n(conv, H)
            t[p + "linear_attn.in_proj_a.weight"] = n(c["linear_num_value_heads"], H)
            t[p + "linear_attn.in_proj_b.weight"] = n(c["linear_num_value_heads"], H)
            t[p + "linear_attn.in_proj_z.weight"] = n(lv, H)
            t[p + "linear_attn.out_proj.weight"] = n(H, lv)
            t[p + "linear_attn.norm.weight"] = n(c["linear_value_head_dim"], std=0.1, mean=1.0)
            t[p + "linear_attn.conv1d.weight"] = n(conv, 1, c["linear_conv_kernel_dim"], std=0.3)
            t[p + "linear_attn.A_log"] = n(c["linear_num_value_heads"], std=0.5)
            t[p + "linear_attn.dt_bias"] = n(c["linear_num_value_heads"], std=0.5)
    names = sorted(t)
    parts = [names[k::shards] for k in range(shards)]
    weight_map = {}
    for k, part in enumerate(parts):
        fn = f"model-{k + 1:05d}-of-{shards:05d}.safetensors"
        write_safetensors(os.path.join(d, fn), {nm: t[nm] for nm in part})
        weight_map.update({nm: fn for nm in part})
    with open(os.path.join(d, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": weight_map}, f)
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump({"architectures": ["Qwen3_5ForConditionalGeneration"], "text_config": c}, f)
    # the checkpoint holds bf16: the values the packer sees
    return {k: (to_bf16_bits(v).astype(np.uint32) << 16).view(np.float32).reshape(v.shape) for k, v in t.items()}
