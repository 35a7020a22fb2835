/* xqhip.h - thin C ABI between the C++ host runtime (libxqwen35.so) and the
 * hand-written gfx950 HIP kernels (libxqhip.so).
 *
 * Everything here is plain C: device pointers are `void*`, streams are `void*`
 * (a hipStream_t; NULL means the library's own stream on the current device),
 * every call returns 0 on success or a negative XQHIP_E* code, with the message
 * available from xqhip_last_error().  No torch or HIP types appear in the
 * signatures.
 *
 * This layer is the MI355X replacement of the reference's per-op GPU seam
 * (customlib/runtime/vulkan_backend.hpp:21-121, `bool op(..., timing, error)`),
 * re-designed so that weights, KV cache, recurrent state and activations stay
 * resident in HBM and no op uploads or downloads per call.  The CPU kernel each
 * entry point replaces is cited beside it.
 */
#ifndef XQHIP_H_
#define XQHIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define XQHIP_API __attribute__((visibility("default")))

enum {
    XQHIP_OK = 0,
    XQHIP_EINVAL = -1,   /* bad argument or unsupported shape */
    XQHIP_EDEVICE = -2,  /* HIP runtime error (message in xqhip_last_error) */
    XQHIP_ENOMEM = -3,
    XQHIP_ENOTSUP = -4   /* valid arguments this entry point cannot run on this
                            matrix or device (the caller uses the separate calls) */
};

/* Element types of activation vectors. */
enum { XQHIP_F32 = 0, XQHIP_F16 = 1 };

/* Epilogues fused into the GEMV store. */
enum {
    XQHIP_EPI_STORE = 0,     /* y[r] = acc                                           */
    XQHIP_EPI_ADD = 1,       /* y[r] += acc (fp32 residual add, custom_model.cpp:294) */
    XQHIP_EPI_SILU_PAIR = 2  /* rows interleaved (gate_i, up_i): y[i] = silu(g)*u    */
};

/* Device layouts of a W4A16 matrix. */
enum {
    XQHIP_LAYOUT_TILED64 = 0, /* group 64, cols % 64 == 0: 16-byte chunks of each row
                                 permuted so a wave's loads are contiguous; per-group
                                 (fp16 scale, fp16 zero) packed in one u32          */
    XQHIP_LAYOUT_GENERIC = 1, /* any group size: reference row-major nibbles, fp32
                                 scales and zeros (used only for tiny shapes)        */
    XQHIP_LAYOUT_TILED64_F32META = 2, /* TILED64 codes with the reference's fp32
                                 (scale, zero) per group (8 bytes): chosen when a
                                 value is not exact in fp16 (e.g. asymmetric scales
                                 (max - min) / 15)                                  */
    XQHIP_LAYOUT_TILED64_SCALE16 = 3, /* TILED64 codes with one fp16 scale per group
                                 (2 bytes): chosen for 4-bit format-v1 matrices whose
                                 zeros are all 8 (the symmetric quantiser, the
                                 synthetic weights) and whose scales fp16 holds; the
                                 zero point is implied                              */
    XQHIP_LAYOUT_TILED64_F32S_Z4 = 4 /* TILED64 codes with the fp32 scale and a 4-bit
                                 zero code per group (4.5 bytes: fp32 scales
                                 [rows][G], then per row ceil(G/8) u32 words, nibble
                                 k of word j = zero of group 8j+k): chosen for 4-bit
                                 format-v1 matrices whose zeros are integers 0..15
                                 and whose scales fp16 cannot hold (the reference
                                 packer's asymmetric quantiser,
                                 pack_qwen35_xq4_numpy.py:218-247)                  */
};

/* A W4A16 matrix resident in HBM.  Semantics of the reference QuantizedMatrix
 * (customlib/kernels/kernels.hpp:11-21): rows x cols unsigned 4-bit codes, even
 * column in the low nibble, one (scale, zero) per `group` columns of a row;
 * affine == 0: w = (q - zero) * scale (XQ4 version 1), affine == 1:
 * w = q * scale + zero (version 2). */
typedef struct xqhip_w4 {
    int32_t rows;
    int32_t cols;
    int32_t group;
    int32_t affine;
    int32_t layout;
    int32_t inexact_meta; /* scales/zeros fp16 cannot hold exactly: kept in fp32
                             (layouts TILED64_F32META, TILED64_F32S_Z4)          */
    int32_t bits;         /* code width: 4 (xqhip_w4_upload), 3 or 2 (xqhip_wlb_upload) */
    int32_t zero_is_8;    /* affine == 0 and every zero is 8: w = (q - 8) s, so the
                             zero-point term of the prefill GEMM vanishes          */
    void* nib;            /* device codes                                         */
    void* meta;           /* device per-group metadata                            */
    uint64_t nib_bytes;
    uint64_t meta_bytes;
} xqhip_w4;

/* ---- device, memory, streams, events ---------------------------------- */
XQHIP_API const char* xqhip_last_error(void);
XQHIP_API int xqhip_device_count(void);
XQHIP_API int xqhip_set_device(int device);
XQHIP_API int xqhip_device_name(char* out, size_t capacity);
XQHIP_API int xqhip_malloc(void** ptr, size_t bytes);
XQHIP_API int xqhip_free(void* ptr);
XQHIP_API int xqhip_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
XQHIP_API int xqhip_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
XQHIP_API int xqhip_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
/* Asynchronous copies (no synchronisation); host memory should be pinned. */
XQHIP_API int xqhip_memcpy_h2d_async(void* dst, const void* src, size_t bytes, void* stream);
XQHIP_API int xqhip_memcpy_d2h_async(void* dst, const void* src, size_t bytes, void* stream);
/* Pinned host memory (hipHostMalloc). */
XQHIP_API int xqhip_host_alloc(void** ptr, size_t bytes);
XQHIP_API int xqhip_host_free(void* ptr);
/* Pinned host memory that kernels may store to directly (hipHostMalloc,
 * mapped and coherent): a kernel's system-scope store reaches the host
 * without a copy on the stream. */
XQHIP_API int xqhip_host_alloc_coherent(void** ptr, size_t bytes);
/* Byte fill done by a kernel (safe inside captured graphs). */
XQHIP_API int xqhip_fill_u8(void* dst, uint8_t value, size_t bytes, void* stream);
/* Device-to-device copy as one plain kernel dispatch (graph-capturable; also
 * the known-size copy that HBM byte counters are calibrated on).  16-byte
 * aligned pointers. */
XQHIP_API int xqhip_copy(void* dst, const void* src, size_t bytes, void* stream);
XQHIP_API int xqhip_stream_synchronize(void* stream);
/* 1 once all work enqueued on `stream` has finished, 0 while some is pending,
 * a negative XQHIP_E* code on a device error.  Does not block. */
XQHIP_API int xqhip_stream_query(void* stream);
XQHIP_API int xqhip_device_synchronize(void);
XQHIP_API int xqhip_event_create(void** ev);
XQHIP_API int xqhip_event_destroy(void* ev);
XQHIP_API int xqhip_event_record(void* ev, void* stream);
/* Blocks the host until the work recorded before `ev` has finished. */
XQHIP_API int xqhip_event_synchronize(void* ev);
XQHIP_API int xqhip_event_elapsed_ms(void* start, void* stop, float* ms);
/* 1 once the work recorded before `ev` has finished, 0 while it is pending,
 * a negative XQHIP_E* code on a device error.  Does not block. */
XQHIP_API int xqhip_event_query(void* ev);

/* ---- W4A16 weights ----------------------------------------------------- */
/* Repack a reference-format matrix (packed[rows][ceil(cols/2)], fp32
 * scales/zeros[rows][ceil(cols/group)], as read by custom_model.cpp:218-262)
 * into the device layout and upload it.  group == 64 and cols % 64 == 0 give a
 * TILED64 layout, with the smallest metadata that holds every scale and zero
 * exactly: SCALE16 (format v1, zeros all 8, fp16 scales), TILED64 (fp16 scale
 * and zero), F32S_Z4 (format v1, integer zeros 0..15, fp32 scales) or
 * F32META (fp32 pair); anything else gives GENERIC. */
XQHIP_API int xqhip_w4_upload(const uint8_t* packed, const float* scales, const float* zeros, int rows, int cols,
                              int group, int affine, xqhip_w4* out);
/* 3- and 2-bit matrices (W3A16 / W2A16): the reference's low-bit format
 * (QuantizedMatrix with bits 3 or 2, kernels/kernels.hpp:11-21; packed by
 * quantizeLowBit, read by readBits / dequantizeValue, ref_gemv.cpp:10-30,
 * 38-87): one LSB-first bitstream, code of (r, c) at bit (r * cols + c) * bits,
 * no row padding; scales/zeros as for 4 bits.  Replaces the matrix side of
 * gemvW3A16Neon / gemvW2A16Neon (arm64_neon/xq_gemv_w{3,2}a16_neon.cpp:6-8);
 * the result works with xqhip_gemv_w4a16 and xqhip_gemv_w4a16_argmax (not
 * with xqhip_gemm_w4a16).  group 64 with cols % 64 == 0 gives the TILED64
 * layout (codes split into bit planes, fp16 metadata), anything else the
 * GENERIC one (the bitstream as given, fp32 metadata).  The reference's
 * per-row bias is always zero (quantizeLowBit, and no file format sets it)
 * and is not carried. */
XQHIP_API int xqhip_wlb_upload(const uint8_t* bitstream, const float* scales, const float* zeros, int rows, int cols,
                               int group, int bits, int affine, xqhip_w4* out);
XQHIP_API int xqhip_w4_free(xqhip_w4* w);
/* Bytes the GEMV must read per call for this matrix (nibbles + metadata). */
XQHIP_API uint64_t xqhip_w4_weight_bytes(const xqhip_w4* w);

/* ---- fused dequant GEMV ------------------------------------------------ */
/* Normalisation applied to the GEMV input inside the kernel prologue. */
enum {
    XQHIP_PRO_NONE = 0,
    XQHIP_PRO_RMS = 1,        /* x * inv * weight[c], inv = 1/sqrt(mean(x^2) + eps)
                                 (rmsnormReference, ref_rmsnorm.cpp:8-17)          */
    XQHIP_PRO_GATED_HEAD = 2, /* per head of head_dim values:
                                 x * inv_h * weight[c % head_dim] * silu(gate[c])
                                 (applyGatedHeadRms, custom_model.cpp:329-349)     */
    XQHIP_PRO_GATED_HEAD_ACT = 3 /* GATED_HEAD with gate[c] already holding
                                 silu(gate[c]) (as xqhip_linear_attn_step_act
                                 leaves it): the GEMV entry points only        */
};
typedef struct xqhip_prologue {
    int32_t mode;
    int32_t head_dim;     /* GATED_HEAD only                                      */
    const float* weight;  /* device: RMS [cols], GATED_HEAD [head_dim]             */
    const float* gate;    /* device: GATED_HEAD [cols]                             */
    float eps;
} xqhip_prologue;

/* y = W x, replacing gemvW4A16Neon
 * (customlib/kernels/generated/arm64_neon/xq_gemv_w4a16_neon.cpp:259-291), and
 * gemvW3A16Neon / gemvW2A16Neon for matrices from xqhip_wlb_upload.
 * x: `cols` values of x_type, optionally normalised by `pro` (NULL = none).
 * y: `rows` values of y_type (EPI_SILU_PAIR: rows/2 values).  Inputs must not
 * alias outputs. */
XQHIP_API int xqhip_gemv_w4a16(const xqhip_w4* w, const void* x, int x_type, const xqhip_prologue* pro, void* y,
                               int y_type, int epilogue, void* stream);

/* Workspace bytes xqhip_gemv_w4a16_argmax needs for a matrix of `rows` rows. */
XQHIP_API size_t xqhip_argmax_workspace_bytes(int rows);
/* Greedy lm_head: argmax_r (W x)[r] without materialising logits, ties to the
 * lowest row, replacing gemvW4A16ArgmaxNeon (xq_gemv_w4a16_neon.cpp:293-348)
 * and sampleGreedy (custom_model.cpp:1281-1338).  Every GEMV block stores its
 * best (value, row) key in the workspace, then a one-block kernel reduces them.
 * workspace: device memory of xqhip_argmax_workspace_bytes(rows), no
 * initialisation needed.  out_index / out_value: device. */
XQHIP_API int xqhip_gemv_w4a16_argmax(const xqhip_w4* w, const void* x, int x_type, const xqhip_prologue* pro,
                                      void* workspace, int32_t* out_index, float* out_value, void* stream);

/* xqhip_gemv_w4a16_argmax that also advances a device position and hands the
 * result to the host without a copy: no counterpart in the reference, whose
 * decodeOne samples on the calling thread (custom_model.cpp:1281-1356).  After
 * the argmax, the finishing kernel adds 1 to *position (device int32) and
 * stores ((uint64_t)(uint32_t)new_position << 32) | (uint32_t)index to
 * *host_slot (8-byte aligned memory from xqhip_host_alloc_coherent) in one
 * system-scope store.  A host thread polls the slot for the position it
 * expects, so sampling, the next token's position and its forward pass can be
 * one captured graph with no copies between them. */
XQHIP_API int xqhip_gemv_w4a16_argmax_publish(const xqhip_w4* w, const void* x, int x_type, const xqhip_prologue* pro,
                                              void* workspace, int32_t* out_index, float* out_value,
                                              int32_t* position, uint64_t* host_slot, void* stream);

/* xqhip_gemv_w4a16_argmax_publish whose finishing kernel also writes the
 * winner's embedding row, the next position's input: sampleGreedy followed by
 * loadEmbeddingRow (custom_model.cpp:1281-1338, 569-608) in the same two
 * launches instead of three.  embed_out[0 .. hidden) = the bf16 row
 * table[index] widened to fp32, bit for bit what xqhip_embed_bf16 writes for
 * *out_index (ids past the table wrap to index % vocab).  table: device
 * [vocab][hidden] bf16; embed_out: device, may be the buffer x points to (the
 * GEMV has finished reading x when the row is written). */
XQHIP_API int xqhip_gemv_w4a16_argmax_publish_embed(const xqhip_w4* w, const void* x, int x_type,
                                                    const xqhip_prologue* pro, void* workspace, int32_t* out_index,
                                                    float* out_value, int32_t* position, uint64_t* host_slot,
                                                    const uint16_t* table, int vocab, int hidden, float* embed_out,
                                                    void* stream);

/* xqhip_gemv_w4a16_argmax without a workspace argument and without any
 * allocation: no counterpart in the reference.  For callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops or
 * harnesses that forbid hipMalloc).  The per-block keys go to a 16 KiB array
 * of the library's own device memory (one per GPU, held until the process
 * ends; any matrix size fits, the launch caps its blocks), which keeps the last
 * call's contents and needs no clearing.  Calls that overlap on one GPU (other
 * streams, other threads) race on that array: serialise them.  The array used
 * is the current device's: a non-NULL `stream` must belong to that device
 * (XQHIP_EINVAL otherwise).  Same results as xqhip_gemv_w4a16_argmax. */
XQHIP_API int xqhip_gemv_w4a16_argmax_static(const xqhip_w4* w, const void* x, int x_type, const xqhip_prologue* pro,
                                             int32_t* out_index, float* out_value, void* stream);

/* ---- decode-step ops (all device pointers; `pos` is a device int32) ----- */
/* out[hidden] = bf16 table row of *token as fp32; ids outside [0, vocab) wrap
 * to |id| % vocab (loadEmbeddingRow, custom_model.cpp:569-608). */
XQHIP_API int xqhip_embed_bf16(const uint16_t* table, int vocab, int hidden, const int32_t* token, float* out,
                               void* stream);

/* Host helper: the RoPE (cos, sin) table [max_pos][rotary_dim/2] for
 * applyRopeVector (custom_model.cpp:351-370), computed with the host libm in
 * the reference's float operation order: inv_freq = powf(theta, -2i/rd),
 * angle = pos * inv_freq, (cosf(angle), sinf(angle)).  out: host floats,
 * 2 * max_pos * (rotary_dim/2) of them. */
XQHIP_API int xqhip_rope_table(float theta, int rotary_dim, int max_pos, float* out);

/* Full-attention head preparation for position *pos: per query head, split
 * the gated q_proj output into (q, gate) (custom_model.cpp:740-753), per-head
 * RMSNorm of q and k (custom_model.cpp:301-313, weights already +1), partial
 * RoPE from rope_cs (device copy of xqhip_rope_table), then k and v appended
 * as fp16 at cache slot *pos of the [t][kv_head][head_dim] caches
 * (appendKv, custom_model.cpp:673-733).  q_out, gate_out: nq*head_dim fp32
 * (gate_out is 0 when gated == 0, matching custom_model.cpp:750-753). */
XQHIP_API int xqhip_attn_prep(const float* q_src, const float* k_src, const float* v_src, int gated, int nq, int nkv,
                              int head_dim, int rotary_dim, const float* q_norm, const float* k_norm, float eps,
                              const float* rope_cs, const int32_t* pos, float* q_out, float* gate_out, void* k_cache,
                              void* v_cache, void* stream);

/* GQA decode over the fp16 caches for context *pos + 1 (scores, softmax and
 * V reduction of custom_model.cpp:840-928) followed by the sigmoid output gate
 * (custom_model.cpp:929-951): out = softmax(q k^T / sqrt(d)) v * sigmoid(gate).
 * Two kernels: per-(kv head, 64-token chunk) partial softmax-attention into the
 * workspace, then a per-query-head merge.  max_ctx <= 16384.
 * workspace: xqhip_gqa_workspace_bytes() (sized for 16384 tokens), no
 * initialisation needed. */
XQHIP_API size_t xqhip_gqa_workspace_bytes(int nq, int nkv, int head_dim);
XQHIP_API int xqhip_gqa_decode(const float* q, const void* k_cache, const void* v_cache, const float* gate, int nq,
                               int nkv, int head_dim, int max_ctx, const int32_t* pos, float* out, void* workspace,
                               void* stream);

/* xqhip_attn_prep followed by xqhip_gqa_decode in two launches: the q/k
 * RMSNorm + RoPE, the fp16 append of the new key/value at slot *pos and the
 * gated GQA of custom_model.cpp:740-951 (the decode half of
 * CustomModel::forwardAttention).  q_src is the q_proj output ([q | gate] per
 * head when gated, gate 0 otherwise); same caches, limits and workspace as
 * xqhip_gqa_decode. */
XQHIP_API int xqhip_attn_decode(const float* q_src, const float* k_src, const float* v_src, int gated, int nq,
                                int nkv, int head_dim, int rotary_dim, const float* q_norm, const float* k_norm,
                                float eps, const float* rope_cs, const int32_t* pos, void* k_cache, void* v_cache,
                                int max_ctx, float* out, void* workspace, void* stream);
/* The same step in one launch and no workspace: one block per query head
 * reads its kv head's whole context (in passes of 1024 tokens merged with a
 * running max) and writes the gated output.  head_dim 128 only; any context
 * the caches hold.  Same cache layout, append and numerics as
 * xqhip_attn_decode; faster where the context is short (the slot kernel
 * spreads long contexts over more CUs).  Replaces the same reference code
 * (custom_model.cpp:740-951). */
XQHIP_API int xqhip_attn_decode_head(const float* q_src, const float* k_src, const float* v_src, int gated, int nq,
                                     int nkv, int head_dim, int rotary_dim, const float* q_norm, const float* k_norm,
                                     float eps, const float* rope_cs, const int32_t* pos, void* k_cache,
                                     void* v_cache, float* out, void* stream);
/* The same step with the cached context split over `splits` (1..8) blocks per
 * query head: split s takes the positions [s per, (s + 1) per), per =
 * ceil(pos / splits), the last split also the new token (appended as above).
 * Each block writes its partial (running max, exp sum, exp-weighted value
 * sums) to the workspace and counts itself on its head's counter; the block
 * completing the count merges the head's partials and writes the gated output
 * to `out` (no block waits for another, no merge kernel).  One split gives
 * xqhip_attn_decode_head's result bit for bit.  workspace:
 * xqhip_attn_split_workspace_bytes(nq) bytes, 16-byte aligned, zero-filled
 * once before the first call: partials [XQHIP_ATTN_MAX_SPLITS][nq]
 * [XQHIP_ATTN_PART_STRIDE] floats, then one counter per head 128 bytes apart;
 * every call leaves the counters at zero again, and calls that overlap on one
 * device race on them.  Replaces the same reference code as
 * xqhip_attn_decode_head (custom_model.cpp:740-951). */
#define XQHIP_ATTN_PART_STRIDE 160 /* floats per (split, head): m, l, 2 pad, o[128], pad to
                                      five 128-byte lines (no line holds two records) */
#define XQHIP_ATTN_MAX_SPLITS 8
XQHIP_API size_t xqhip_attn_split_workspace_bytes(int nq);
XQHIP_API int xqhip_attn_decode_split(const float* q_src, const float* k_src, const float* v_src, int gated, int nq,
                                      int nkv, int head_dim, int rotary_dim, const float* q_norm, const float* k_norm,
                                      float eps, const float* rope_cs, const int32_t* pos, void* k_cache,
                                      void* v_cache, int splits, void* workspace, float* out, void* stream);

/* Linear attention: conv1d + SiLU over the mixed q|k|v channels with the
 * [channels][ksize-1] history updated in place, then L2-normalised q and k
 * heads (custom_model.cpp:961-1047).  out: conv_dim fp32. */
XQHIP_API int xqhip_linear_conv(const float* mixed, float* conv_state, const float* conv_w, int lk_n, int lk_hd,
                                int lv_n, int lv_hd, int ksize, float* out, void* stream);
/* Gated delta rule per value head on the fp32 state [lv_n][lk_hd][lv_hd]
 * (custom_model.cpp:1074-1096, gatedDeltaDecodeReference ref_delta.cpp:8-41),
 * with beta = sigmoid(b), g = -exp(a_log) * softplus(a + dt_bias).
 * conv: output of xqhip_linear_conv; out: lv_n * lv_hd fp32. */
XQHIP_API int xqhip_gated_delta(const float* conv, const float* a, const float* b, const float* a_log,
                                const float* dt_bias, float* state, int lk_n, int lv_n, int lk_hd, int lv_hd,
                                float* out, void* stream);
/* One decode step of the linear-attention state update in a single kernel:
 * conv1d + SiLU with L2-normalised q/k heads (as xqhip_linear_conv) feeding the
 * gated delta rule (as xqhip_gated_delta), custom_model.cpp:961-1096.
 * conv_state holds TWO copies of the [conv_dim][ksize-1] history: copy
 * (*pos & 1) is read and copy ((*pos + 1) & 1) written, so consecutive
 * positions alternate (zero both copies to reset).  mixed: conv_dim channels
 * (q | k | v); a, b: lv_n gate inputs; out: lv_n * lv_hd. */
XQHIP_API int xqhip_linear_attn_step(const float* mixed, float* conv_state, const float* conv_w, const float* a,
                                     const float* b, const float* a_log, const float* dt_bias, float* state, int lk_n,
                                     int lk_hd, int lv_n, int lv_hd, int ksize, const int32_t* pos, float* out,
                                     void* stream);
/* The same step that also replaces `gate` (lv_n * lv_hd, the gated output
 * norm's z) by silu(gate) in place, once per step, so that the output
 * projection's XQHIP_PRO_GATED_HEAD_ACT prologue reads it instead of every one
 * of its blocks evaluating the 4096 SiLUs (custom_model.cpp:329-349). */
XQHIP_API int xqhip_linear_attn_step_act(const float* mixed, float* conv_state, const float* conv_w, const float* a,
                                         const float* b, const float* a_log, const float* dt_bias, float* state,
                                         int lk_n, int lk_hd, int lv_n, int lv_hd, int ksize, const int32_t* pos,
                                         float* out, float* gate, void* stream);

/* The linear-attention decode step and the output projection that consumes
 * it, as one launch: the same results, bit for bit, as
 *   xqhip_linear_attn_step_act(mixed, ..., pos, out, gate, stream);
 *   xqhip_prologue pro = {XQHIP_PRO_GATED_HEAD_ACT, lv_hd, norm_weight, gate, eps};
 *   xqhip_gemv_w4a16(w, out, XQHIP_F32, &pro, y, XQHIP_F32, XQHIP_EPI_ADD, stream);
 * (the step, applyGatedHeadRms, out_proj and addResidual of a linear-attention
 * layer, customlib/runtime/custom_model.cpp:1074-1135, 1179), with the
 * projection's weights requested while the step runs instead of after a
 * kernel boundary.  One 1024-thread block per CU (every block must be resident
 * at once: each waits, boundedly, for the step's output of all of them).
 * w: a 4-bit TILED64 matrix (any of its metadata forms) with lv_n * lv_hd <=
 * 4096 columns; ksize 4.  sync: xqhip_step_outproj_sync_bytes() bytes of
 * device memory, 128-byte aligned, zero-filled once before the first launch;
 * every launch leaves it zeroed, launches sharing it must be ordered (one
 * stream).  Graph-capturable.  Returns XQHIP_ENOTSUP when the matrix or the
 * device does not allow the combination (xqhip_step_outproj_supported says so
 * beforehand).  No counterpart in the reference, which runs the two ops one
 * after the other.  Measured on MI355X (9B shapes) slower than the two calls,
 * 15.9 against 11.0 us: the hand-off between CUs of different XCDs inside one
 * launch costs more than a kernel boundary. */
XQHIP_API size_t xqhip_step_outproj_sync_bytes(void);
XQHIP_API int xqhip_step_outproj_supported(const xqhip_w4* w, int lk_n, int lk_hd, int lv_n, int lv_hd, int ksize);
XQHIP_API int xqhip_linear_attn_step_outproj(const float* mixed, float* conv_state, const float* conv_w,
                                             const float* a, const float* b, const float* a_log,
                                             const float* dt_bias, float* state, int lk_n, int lk_hd, int lv_n,
                                             int lv_hd, int ksize, const int32_t* pos, float* out, float* gate,
                                             const xqhip_w4* w, const float* norm_weight, float eps, float* y,
                                             void* sync, void* stream);
/* Reads the sync block's error word (synchronous copy): 0, or nonzero after a
 * launch whose wait gave up (its results are then invalid; zero-fill the block
 * again before the next launch). */
XQHIP_API int xqhip_step_outproj_error(const void* sync, int* error);
/* y = x * inv * w (rmsnormReference, ref_rmsnorm.cpp:8-17). */
XQHIP_API int xqhip_rmsnorm(const float* x, const float* w, int n, float eps, float* y, void* stream);

/* ---- prefill: a prompt chunk of m tokens at once ------------------------- */
/* The reference prefills token by token (CustomModel::prefill,
 * custom_model.cpp:610-640, each token through runLayer :1138-1256); these run
 * the same per-token arithmetic for a chunk: the projections as GEMMs on the
 * matrix cores, attention and the linear-attention recurrence as batched
 * kernels.  Row-major [token][...] activations with explicit row strides. */

/* Workspace bytes xqhip_gemm_w4a16 needs for m tokens of `cols` columns and a
 * matrix of `rows` rows (the staged x, plus the partial products of a launch
 * whose columns are split over several blocks when it has too few blocks to
 * fill the device; a workspace sized for the largest rows of a set of
 * matrices serves them all). */
XQHIP_API size_t xqhip_gemm_workspace_bytes(int m, int cols, int rows);
/* y[t] (op)= W prologue(x[t]) for t < m: every token as xqhip_gemv_w4a16 does it
 * (same epilogues; EPI_SILU_PAIR writes rows/2 values per token), on a TILED64
 * matrix.  Per 64-column group the codes q - 8 (exact in fp16) multiply x held
 * as fp16 hi + lo halves on fp16 MFMA with fp32 accumulation, the group sum is
 * scaled by the group scale, and the zero-point term is added as the product of
 * the per-group offsets with the per-token group sums of x.  GATED_HEAD reads the gate
 * of token t at pro->gate + t * ld_gate.  workspace: 16-byte aligned, of
 * workspace_bytes >= xqhip_gemm_workspace_bytes(m, cols, rows of w) (checked:
 * XQHIP_EINVAL when smaller). */
XQHIP_API int xqhip_gemm_w4a16(const xqhip_w4* w, const float* x, int m, int ldx, const xqhip_prologue* pro,
                               int ld_gate, float* y, int ldy, int epilogue, void* workspace, size_t workspace_bytes,
                               void* stream);
/* xqhip_embed_bf16 for n tokens (device ids) into out[n][hidden]. */
XQHIP_API int xqhip_embed_bf16_batch(const uint16_t* table, int vocab, int hidden, const int32_t* tokens, int n,
                                     float* out, void* stream);
/* xqhip_attn_prep for tokens consecutive positions *pos0 .. *pos0 + tokens - 1:
 * token t reads its projections at q_src/k_src/v_src + t * src_stride and writes
 * q and gate at t * out_stride; k and v are appended at cache slot *pos0 + t. */
XQHIP_API int xqhip_attn_prep_batch(const float* q_src, const float* k_src, const float* v_src, int gated, int nq,
                                    int nkv, int head_dim, int rotary_dim, const float* q_norm, const float* k_norm,
                                    float eps, const float* rope_cs, const int32_t* pos0, int tokens, int src_stride,
                                    int out_stride, float* q_out, float* gate_out, void* k_cache, void* v_cache,
                                    void* stream);
/* Causal GQA for the chunk: token t (position *pos0 + t) attends to cache slots
 * 0 .. *pos0 + t, then the sigmoid output gate (custom_model.cpp:840-951 per
 * token).  q, gate: [tokens][q_stride]; out: [tokens][out_stride]. */
XQHIP_API int xqhip_prefill_attention(const float* q, const float* gate, const void* k_cache, const void* v_cache,
                                      int nq, int nkv, int head_dim, int tokens, int q_stride, const int32_t* pos0,
                                      float* out, int out_stride, void* stream);
/* xqhip_linear_attn_step for tokens consecutive positions pos0 .. pos0+tokens-1
 * (pos0 given on the host) in one kernel: mixed, a, b rows of token t at
 * t * stride; conv_state holds the two parity copies of xqhip_linear_attn_step
 * and is left as that step expects for position pos0 + tokens. */
XQHIP_API int xqhip_linear_attn_scan(const float* mixed, const float* a, const float* b, int stride,
                                     float* conv_state, int pos0, const float* conv_w, const float* a_log,
                                     const float* dt_bias, float* state, int lk_n, int lk_hd, int lv_n, int lv_hd,
                                     int ksize, int tokens, float* out, int out_stride, void* stream);
/* xqhip_linear_attn_scan with a workspace of xqhip_linear_scan_workspace_bytes()
 * (16-byte aligned): the conv1d + SiLU, q/k L2 norms and gates of all tokens
 * run first as one token-parallel pass; for key heads of 128 dims the state
 * recurrence then runs in 64-token chunks (the per-token update unrolled over a
 * chunk into products with a triangular solve, parallel over chunks except one
 * pass per value head and 16 columns).  Same mathematics as the per-token scan,
 * a different fp32 summation order.  No counterpart in the reference (which
 * prefills token by token, custom_model.cpp:610-640); same contract as
 * xqhip_linear_attn_scan. */
XQHIP_API size_t xqhip_linear_scan_workspace_bytes(int tokens, int lk_n, int lk_hd, int lv_n, int lv_hd);
XQHIP_API int xqhip_linear_attn_scan_ws(const float* mixed, const float* a, const float* b, int stride,
                                        float* conv_state, int pos0, const float* conv_w, const float* a_log,
                                        const float* dt_bias, float* state, int lk_n, int lk_hd, int lv_n, int lv_hd,
                                        int ksize, int tokens, float* out, int out_stride, void* workspace,
                                        void* stream);

/* One kernel of one thread that stores the device's 100 MHz realtime counter
 * (s_memrealtime) to *slot with a system-scope store; slot may be device or
 * coherent host memory (xqhip_host_alloc_coherent).  Between two kernels on a
 * stream it marks the end of the first; graph-capturable.  Times the ops of
 * traced decode-step graphs (the kernel trace's per-op rows, after
 * custom_model.cpp:374-417). */
XQHIP_API int xqhip_timestamp(uint64_t* slot, void* stream);
/* Test diagnostic, no counterpart in the reference: fills the LDS of every CU
 * with `value` (blocks holding a CU's whole 160 KiB), so that a kernel
 * launched next on the same stream finds that value wherever it reads LDS it
 * has not written itself (LDS keeps its contents between kernels).  The
 * attention tests run the decode attention right after it. */
XQHIP_API int xqhip_lds_fill(float value, void* stream);

/* ---- decode chains: consecutive projections in one persistent launch --- */
/* A chain runs a sequence of decode-step GEMVs (the projections between two
 * non-GEMV ops of the reference's runLayer, customlib/runtime/custom_model.cpp
 * :1138-1256: o/out_proj -> gate/up -> down -> the next layer's input
 * projection) as one launch of one block per CU.  Each CU keeps streaming
 * weights across the op boundaries (the next op's first weights are requested
 * before the current op's output is complete), and an op reads its input
 * vector from the previous op through a hand-off arena of 8-byte records
 * (value, launch sequence number) stored write-through, polled with bounded
 * waits: no kernel boundary and no grid barrier between the ops.  Results are
 * those of xqhip_gemv_w4a16 on the same operands, bit for bit.
 *
 * Every matrix of a chain must be a 4-bit TILED64 matrix with fp16, fp32-pair
 * or fp16-scale metadata (layouts TILED64, TILED64_F32META, TILED64_SCALE16,
 * not TILED64_F32S_Z4), all in one of them; cols <= 16384. */
typedef struct xqhip_chain_src {
    const float* plain; /* a device fp32 vector complete before the launch, or */
    int32_t op;         /* (plain == NULL) the output of op `op` of the chain */
    int32_t offset;     /* first element taken from that output */
} xqhip_chain_src;

typedef struct xqhip_chain_op {
    const xqhip_w4* w;
    int32_t epi;          /* XQHIP_EPI_STORE / ADD / SILU_PAIR                  */
    int32_t pro;          /* XQHIP_PRO_NONE / RMS / GATED_HEAD_ACT              */
    const float* pro_w;   /* RMS: [cols]; GATED_HEAD_ACT: [head_dim]            */
    int32_t head_dim;     /* GATED_HEAD_ACT                                     */
    float eps;
    xqhip_chain_src x;    /* input, cols values                                */
    xqhip_chain_src gate; /* GATED_HEAD_ACT: silu(gate), cols values            */
    xqhip_chain_src res;  /* ADD: the residual added to                         */
    float* y_plain;       /* also store the output here (NULL: later ops only)  */
} xqhip_chain_op;

/* Validates the ops and uploads a device description; *chain receives an
 * opaque handle.  XQHIP_EINVAL when a matrix or shape is not supported. */
XQHIP_API int xqhip_chain_create(const xqhip_chain_op* ops, int n_ops, void** chain);
XQHIP_API int xqhip_chain_destroy(void* chain);
/* Hand-off records a launch of this chain needs (8 bytes each). */
XQHIP_API size_t xqhip_chain_arena_records(const void* chain);
/* Bytes of the synchronisation block shared by the chains of one stream
 * (zero-filled once before the first launch, then left alone). */
XQHIP_API size_t xqhip_chain_sync_bytes(void);
/* One launch: arena of at least xqhip_chain_arena_records records (zero-filled
 * once before first use), sync block as above.  Graph-capturable.  Launches
 * sharing an arena or sync block must be ordered (one stream). */
XQHIP_API int xqhip_chain_launch(const void* chain, void* arena, void* sync, void* stream);
/* The same launch recording per op and block the device's 100 MHz realtime
 * counter when the op's input is staged and when its last output is stored:
 * stamps[(op * grid + block) * 2 + {0, 1}] (uint64), grid = xqhip_chain_grid. */
XQHIP_API int xqhip_chain_launch_stamped(const void* chain, void* arena, void* sync, void* stamps, void* stream);
XQHIP_API int xqhip_chain_grid(const void* chain);
/* Reads the sync block's error word (synchronous copy): 0, or nonzero after a
 * launch whose hand-off wait gave up (its results are then invalid). */
XQHIP_API int xqhip_chain_error(const void* sync, int* error);

/* ---- streams and graphs ------------------------------------------------ */
XQHIP_API int xqhip_stream_create(void** stream);
XQHIP_API int xqhip_stream_destroy(void* stream);
XQHIP_API int xqhip_graph_begin(void* stream);
XQHIP_API int xqhip_graph_end(void* stream, void** graph_exec);
XQHIP_API int xqhip_graph_launch(void* graph_exec, void* stream);
XQHIP_API int xqhip_graph_destroy(void* graph_exec);

#ifdef __cplusplus
}
#endif

#endif /* XQHIP_H_ */
