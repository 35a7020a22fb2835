/* xqsynth.h - seeded synthetic model packages in the on-disk format the decode
 * library reads (xqwen35_manifest.json, embeddings_bf16.bin, *.f32, *.xq4; see
 * customlib/runtime/custom_model.cpp:185-262, 423-553 and the tiny-model writer
 * of customlib/tests/runtime_correctness/test_runtime.cpp:38-144).  There is no
 * counterpart in the reference (it converts real checkpoints); this writer makes
 * random-init models of any shape so that the library, the oracle and the
 * compiled reference can all be run on identical files.
 *
 * Values (counter-based generator, one stream per tensor name):
 *   4-bit codes uniform in 0..15, two per byte, even column in the low nibble;
 *   scales |N(0, scale_std)| rounded to fp16 and stored as fp32; zeros = `zero`
 *   (XQ4 version 1, w = (q - zero) * scale);
 *   with `asymmetric` set, the metadata of the reference packer's asymmetric
 *   quantiser (pack_qwen35_xq4_numpy.py:218-247: fp32 scales, integer zeros
 *   0..15) instead: scales |N(0, scale_std)| in fp32, not rounded, and zeros
 *   clamp(round(7.5 + N(0, 1)), 0, 15) per group (`zero` unused);
 *   embeddings N(0, embed_std) as bf16;
 *   norm weights with effective value N(1, norm_std) rounded to fp16 (stored
 *   minus one where the reader adds one);
 *   conv1d weights N(0, 0.3), A_log N(0, 0.5), dt_bias N(0, 0.5).
 * Layer i is full attention iff full_attention_interval > 0 and
 * i % full_attention_interval == full_attention_interval - 1. */
#ifndef XQSYNTH_H_
#define XQSYNTH_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct xqsynth_config {
    uint64_t seed;
    int32_t hidden_size;
    int32_t intermediate_size;
    int32_t vocab_size;
    int32_t num_layers;
    int32_t full_attention_interval;
    int32_t num_attention_heads;
    int32_t num_key_value_heads;
    int32_t head_dim;
    float partial_rotary_factor;
    int32_t gated_q_proj;
    int32_t linear_key_head_dim;
    int32_t linear_value_head_dim;
    int32_t linear_num_key_heads;
    int32_t linear_num_value_heads;
    int32_t linear_conv_kernel_dim;
    int32_t group_size;
    float rms_norm_eps;
    float rope_theta;
    float scale_std;
    float zero;
    float embed_std;
    float norm_std;
    int32_t threads;
    int32_t asymmetric;
} xqsynth_config;

/* Fills `cfg` with the 9B-shaped hybrid model of the benchmark workload:
 * 32 layers (3 linear : 1 full), hidden 4096, MLP 12288, vocab 248320,
 * 32 query / 8 KV heads of 128 (gated q_proj), rotary 0.25, theta 1e7,
 * linear attention 16 key / 32 value heads of 128, conv 4, group 64. */
__attribute__((visibility("default"))) void xqsynth_default_config(xqsynth_config* cfg);
/* Writes the package into `dir` (created if missing).  Returns 0 or -1 with
 * the reason in `err`. */
__attribute__((visibility("default"))) int xqsynth_write_model(const char* dir, const xqsynth_config* cfg, char* err,
                                                               size_t err_capacity);

#ifdef __cplusplus
}
#endif

#endif /* XQSYNTH_H_ */
