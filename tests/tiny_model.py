"""The reference runtime test's tiny model package
(customlib/tests/runtime_correctness/test_runtime.cpp:60-144): hidden 4, two
layers (layer 0 linear attention, layer 1 full attention), vocab 8, group 4,
`patternedMatrix` weights quantised with the reference min/max quantiser
(restated by the oracle, bit-exact), bf16 embeddings by truncation."""
import json
import os
import shutil

import numpy as np

import oracle_bind as ob

MANIFEST = {"format": "xqwen35_custom_w4a16", "hidden_size": 4, "intermediate_size": 8, "vocab_size": 8,
            "num_hidden_layers": 2, "num_attention_heads": 2, "num_key_value_heads": 1, "head_dim": 2,
            "linear_key_head_dim": 2, "linear_value_head_dim": 2, "linear_num_key_heads": 1,
            "linear_num_value_heads": 2, "linear_conv_kernel_dim": 2, "rms_norm_eps": 0.000001, "rope_theta": 10000,
            "partial_rotary_factor": 1.0}


def patterned(rows, cols, scale):
    r = np.arange(rows)[:, None]
    c = np.arange(cols)[None, :]
    sign = np.where((r + c) % 2 == 0, np.float32(1.0), np.float32(-1.0))
    return (sign * np.float32(scale) * (np.float32(1.0) + ((r * 3 + c * 5) % 7).astype(np.float32))).astype(np.float32)


def write_xq4(path, rows, cols, values, group=4):
    q = ob.quantize_lowbit(values.reshape(-1), rows, cols, 4, group)
    with open(path, "wb") as f:
        f.write(b"XQW4A16\0")
        f.write(np.array([1, rows, cols, group, 4], np.uint32).tobytes())
        f.write(np.array([q.packed.size, q.scales.size, q.zeros.size], np.uint64).tobytes())
        f.write(q.packed.tobytes())
        f.write(q.scales.tobytes())
        f.write(q.zeros.tobytes())


def write_f32(path, values):
    np.asarray(values, np.float32).tofile(path)


def write_tiny_model(d):
    shutil.rmtree(d, ignore_errors=True)
    os.makedirs(d)
    with open(os.path.join(d, "xqwen35_manifest.json"), "w") as f:
        f.write(json.dumps(MANIFEST, separators=(",", ":")))
    emb = np.zeros((8, 4), np.float32)
    for t in range(8):
        for dd in range(4):
            emb[t, dd] = np.float32(0.05) * np.float32(t + 1) + (np.float32(1.0) if t == dd else np.float32(0.0))
    (emb.view(np.uint32) >> 16).astype(np.uint16).tofile(os.path.join(d, "embeddings_bf16.bin"))
    j = lambda n: os.path.join(d, n)
    write_f32(j("norm_weight.f32"), np.ones(4))
    for layer in range(2):
        p = f"layers_{layer}_"
        write_f32(j(p + "input_layernorm_weight.f32"), np.ones(4))
        write_f32(j(p + "post_attention_layernorm_weight.f32"), np.ones(4))
        write_xq4(j(p + "mlp_gate_proj_weight.xq4"), 8, 4, patterned(8, 4, 0.02))
        write_xq4(j(p + "mlp_up_proj_weight.xq4"), 8, 4, patterned(8, 4, 0.015))
        write_xq4(j(p + "mlp_down_proj_weight.xq4"), 4, 8, patterned(4, 8, 0.01))
    write_xq4(j("layers_0_linear_attn_in_proj_qkv_weight.xq4"), 8, 4, patterned(8, 4, 0.03))
    write_xq4(j("layers_0_linear_attn_in_proj_a_weight.xq4"), 2, 4, patterned(2, 4, 0.02))
    write_xq4(j("layers_0_linear_attn_in_proj_b_weight.xq4"), 2, 4, patterned(2, 4, 0.025))
    write_xq4(j("layers_0_linear_attn_in_proj_z_weight.xq4"), 4, 4, patterned(4, 4, 0.03))
    write_xq4(j("layers_0_linear_attn_out_proj_weight.xq4"), 4, 4, patterned(4, 4, 0.02))
    write_f32(j("layers_0_linear_attn_norm_weight.f32"), np.ones(2))
    conv = np.zeros(16, np.float32)
    conv[0::2], conv[1::2] = 0.25, 1.0
    write_f32(j("layers_0_linear_attn_conv1d_weight.f32"), conv)
    write_f32(j("layers_0_linear_attn_A_log.f32"), [-2.0, -2.2])
    write_f32(j("layers_0_linear_attn_dt_bias.f32"), [0.0, 0.1])
    write_xq4(j("layers_1_self_attn_q_proj_weight.xq4"), 8, 4, patterned(8, 4, 0.025))
    write_xq4(j("layers_1_self_attn_k_proj_weight.xq4"), 2, 4, patterned(2, 4, 0.02))
    write_xq4(j("layers_1_self_attn_v_proj_weight.xq4"), 2, 4, patterned(2, 4, 0.03))
    write_xq4(j("layers_1_self_attn_o_proj_weight.xq4"), 4, 4, patterned(4, 4, 0.02))
    write_f32(j("layers_1_self_attn_q_norm_weight.f32"), np.ones(2))
    write_f32(j("layers_1_self_attn_k_norm_weight.f32"), np.ones(2))
    write_xq4(j("lm_head_weight.xq4"), 8, 4, patterned(8, 4, 0.04))
    return d


# Small synthetic shape exercising the group-64 fast paths (3 linear + 1 full layer,
# partial 4096-column chunks).  Every reference GEMV of this shape runs on one
# thread (rows < 2x the pool's minimum chunk), which keeps the compiled reference
# clear of its worker-pool completion race (xq_gemv_w4a16_neon.cpp:146-207).
SMALL = dict(hidden_size=512, intermediate_size=960, vocab_size=4096, num_layers=4, num_attention_heads=2,
             num_key_value_heads=1, head_dim=128, linear_key_head_dim=128, linear_value_head_dim=128,
             linear_num_key_heads=1, linear_num_value_heads=2, seed=7)


# The head layout of Qwen3.5-9B (custom_model.hpp:101-104: 16 query heads, 4
# kv heads, head_dim 256, gated q_proj; partial rotary 0.25 -> 64 dims;
# linear attention 16 key heads and 32 value heads of 128,
# docs/model_facts.md:17-21) with its hidden size 4096 (the reference sizes
# its attention buffers by the hidden size, custom_model.cpp:481-486) and a
# small MLP and vocabulary, so the oracle runs it in seconds.
QWEN35_9B_HEADS = dict(hidden_size=4096, intermediate_size=1024, vocab_size=4096, num_layers=4,
                       num_attention_heads=16, num_key_value_heads=4, head_dim=256, partial_rotary_factor=0.25,
                       gated_q_proj=1, linear_key_head_dim=128, linear_value_head_dim=128, linear_num_key_heads=16,
                       linear_num_value_heads=32, seed=31)
