// xqhip_kernels.hpp - launch interfaces shared between the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace xqhip {

// PRO_GATED_ACT: PRO_GATED whose gate vector already holds silu(gate)
enum { PRO_NONE = 0, PRO_RMS = 1, PRO_GATED = 2, PRO_GATED_ACT = 3 };
constexpr int kMaxNormHeads = 256;
// Split decode attention partials (attn_decode_part_kernel): per split and
// query head, the running max at 0, the exp sum at 1 and the head_dim (128)
// exp-weighted value sums from kAttnPartO (16-byte aligned rows).
constexpr int kAttnPartO = 4, kAttnPartStride = 160, kAttnMaxSplits = 8;  // a record fills five 128-byte lines

// Normalisation applied to the GEMV input inside the kernel prologue.
struct Prologue {
    int mode;          // PRO_*
    const float* w;    // PRO_RMS: [cols]; PRO_GATED: [head_dim]
    const float* z;    // PRO_GATED: gate [cols]
    int head_dim;      // PRO_GATED
    float eps;
};

// One fused-dequant GEMV launch (gemv_w4a16.hip).
struct GemvLaunch {
    const uint8_t* nib;
    const void* meta;
    int rows, cols, group, affine, layout;
    int bits;            // 4, 3 or 2
    uint64_t nib_bytes;  // code bytes (the GENERIC bitstream's bound)
    const void* x;
    int x_f16;
    Prologue pro;
    void* y;
    int y_f16;
    int epi;  // 0 store, 1 add, 2 silu pair, 3 argmax
    uint64_t* partial;  // argmax: one key per block
    int32_t* out_idx;
    float* out_val;
    int32_t* position;    // argmax: advanced by one after the argmax (nullptr: untouched)
    uint64_t* host_slot;  // argmax with position: receives (new position << 32) | index
    // argmax: when embed_out is set, the winner's bf16 row of embed_table
    // ([embed_vocab][embed_hidden]) is also written to embed_out as fp32
    const uint16_t* embed_table;
    int embed_vocab, embed_hidden;
    float* embed_out;
    int max_blocks;  // <= 0: as many blocks as are resident on the device at once
};

// Argmax partial keys the workspace holds (one per block).
constexpr int kArgmaxMaxBlocks = 2048;

hipError_t launch_gemv(const GemvLaunch& p, hipStream_t s);

// decode_ops.hip
struct EmbedLaunch {
    const uint16_t* table;
    int vocab, hidden;
    const int32_t* tok;  // [tokens]
    float* out;          // [tokens][hidden]
    int tokens;
};
hipError_t launch_embed(const EmbedLaunch& p, hipStream_t s);

struct QkPrepLaunch {
    const float* q_src;  // q_proj output (gated: per head [q | gate])
    const float* k_src;
    const float* v_src;
    int gated, nq, nkv, head_dim, rotary_dim, rope_pairs;
    const float* q_norm;
    const float* k_norm;
    float eps;
    const float* rope_cs;  // [max_ctx][rope_pairs] (cos, sin)
    const int32_t* pos;
    float* q_out;
    float* gate_out;
    _Float16* k_cache;
    _Float16* v_cache;
    int tokens;      // batch of consecutive positions *pos .. *pos + tokens - 1
    int src_stride;  // floats between consecutive tokens' projection rows
    int out_stride;  // floats between consecutive tokens' q / gate rows
};
hipError_t launch_qk_prep(const QkPrepLaunch& p, hipStream_t s);

struct GqaLaunch {
    const float* q;
    const _Float16* k_cache;
    const _Float16* v_cache;
    const float* gate;
    int nq, nkv, head_dim, max_ctx;
    const int32_t* pos;
    float* out;
    float* part_m;  // workspace: [nq][max chunks] chunk max
    float* part_l;  //            [nq][max chunks] chunk sum of exp
    float* part_o;  //            [nq][max chunks][head_dim] unnormalised output
    int gate_stride;  // floats between the gates of consecutive query heads (gate == nullptr: none)
};

// Decode attention with the q/k preparation and KV append folded in
// (attn_decode_kernel + gqa_combine_kernel).
struct AttnDecodeLaunch {
    GqaLaunch g;  // g.q unused; g.gate = q projection + head_dim (gated) or nullptr
    const float* q_src;  // q projection output (gated: per head [q | gate])
    const float* k_src;
    const float* v_src;
    int gated, rotary_dim, rope_pairs;
    const float* q_norm;
    const float* k_norm;
    float eps;
    const float* rope_cs;
    _Float16* k_cache;
    _Float16* v_cache;
};
hipError_t launch_attn_decode(const AttnDecodeLaunch& a, hipStream_t s);
// one block per query head, no merge kernel (head_dim 128)
bool attn_head_supported(int nq, int nkv, int head_dim);
hipError_t launch_attn_decode_head(const AttnDecodeLaunch& a, hipStream_t s);
// the same over `splits` context ranges per query head, merged by the last
// block of each head (cnt: a zeroed counter per head, 128 bytes apart, left
// zeroed) into the gated output a.g.out
hipError_t launch_attn_decode_part(const AttnDecodeLaunch& a, int splits, float* part, uint32_t* cnt, hipStream_t s);
size_t gqa_workspace_bytes(int nq, int nkv, int head_dim);
bool gqa_supported(int nq, int nkv, int head_dim, int max_ctx);
hipError_t launch_gqa(const GqaLaunch& p, hipStream_t s);

struct ConvLaunch {
    const float* mixed;
    float* state;
    const float* conv_w;
    int lk_n, lk_hd, lv_n, lv_hd, ksize;
    float* out;
};
bool conv_supported(int lk_hd, int lv_hd);
hipError_t launch_conv(const ConvLaunch& p, hipStream_t s);

struct DeltaLaunch {
    const float* conv;  // normalised q | k | v
    const float* a;
    const float* b;
    const float* a_log;
    const float* dt_bias;
    float* state;
    int lk_n, lv_n, lk_hd, lv_hd;
    float* out;
};
bool delta_supported(int lk_hd);
hipError_t launch_delta(const DeltaLaunch& p, hipStream_t s);

// Fused linear-attention step (conv1d + SiLU + q/k L2 norm + gated delta) for
// the decode graph.  The conv history is double-buffered by position parity:
// copy (pos & 1) is read and copy ((pos + 1) & 1) written, so the blocks that
// recompute a key head's q/k channels never race with the one that stores them.
struct LinearStepLaunch {
    const float* mixed;   // conv input: q | k | v channels
    float* conv_state;    // [2][conv_dim][ksize - 1]
    const float* conv_w;  // [conv_dim][ksize]
    const float* a;
    const float* b;
    const float* a_log;
    const float* dt_bias;
    float* state;  // [lv_n][lk_hd][lv_hd]
    int lk_n, lk_hd, lv_n, lv_hd, ksize;
    const int32_t* pos;
    float* out;    // lv_n * lv_hd
    float* z_act;  // optional: the gated norm's gate (lv_n * lv_hd), replaced by silu(gate) in place
};
bool linear_step_supported(int lk_n, int lk_hd, int lv_n, int lv_hd, int ksize);
hipError_t launch_linear_step(const LinearStepLaunch& p, hipStream_t s);

// decode_fused.hip: the step and the output projection g (ADD epilogue, x =
// p.out) as one launch; sync: step_outproj_sync_bytes(), zeroed before the
// first launch and left zeroed by every launch.
size_t step_outproj_sync_bytes();
int step_outproj_error_word();  // index of the error word (uint32) in sync
bool step_outproj_shape_ok(const LinearStepLaunch& p, const GemvLaunch& g);
int step_outproj_grid(const LinearStepLaunch& p, const GemvLaunch& g);  // 0: not runnable on this device
hipError_t launch_step_outproj(const LinearStepLaunch& p, const GemvLaunch& g, uint32_t* sync, hipStream_t s);

hipError_t launch_rmsnorm(const float* x, const float* w, int n, float eps, float* y, hipStream_t s);
hipError_t launch_lds_fill(float value, hipStream_t s);
hipError_t launch_timestamp(uint64_t* slot, hipStream_t s);

// prefill_ops.hip: multi-token kernels of a prompt chunk.
struct GemmLaunch {
    const uint8_t* nib;  // TILED64 matrix
    const void* meta;
    int rows, cols, affine;
    int layout;      // 0 TILED64 (fp16 metadata), 2 TILED64_F32META, 3 TILED64_SCALE16
    int zero_is_8;   // w = (q - 8) s everywhere: no zero-point term
    const float* x;  // [m][ldx]
    int ldx, m;
    Prologue pro;  // per token; PRO_GATED reads pro.z + t * ldz
    int ldz;
    float* y;  // [m][ldy]
    int ldy;
    int epi;          // 0 store, 1 add, 2 silu pair
    void* workspace;  // gemm_workspace_bytes(m, cols, rows)
};
size_t gemm_workspace_bytes(int m, int cols, int rows);
bool gemm_supported(int rows, int cols, int group, int layout, const Prologue& pro);
hipError_t launch_gemm(const GemmLaunch& p, hipStream_t s);

struct PrefillAttnLaunch {
    const float* q;     // [tokens][q_stride], heads [nq][hd]
    const float* gate;  // same layout as q
    const _Float16* k_cache;
    const _Float16* v_cache;
    int nq, nkv, head_dim, tokens, q_stride, out_stride;
    const int32_t* pos0;  // device: position of token 0
    float* out;           // [tokens][out_stride]
};
bool prefill_attn_supported(int nq, int nkv, int head_dim);
hipError_t launch_prefill_attn(const PrefillAttnLaunch& p, hipStream_t s);

struct LinearScanLaunch {
    const float* mixed;  // [tokens][mixed_stride]: conv input channels q | k | v
    const float* a;      // [tokens][mixed_stride] rows, lv_n values each
    const float* b;
    int mixed_stride;
    const float* hist_in;  // [conv_dim][ksize - 1] history before token 0
    float* hist_out;       // [conv_dim][ksize - 1] history after the last token (not hist_in)
    const float* conv_w;
    const float* a_log;
    const float* dt_bias;
    float* state;  // [lv_n][lk_hd][lv_hd]
    int lk_n, lk_hd, lv_n, lv_hd, ksize, tokens;
    float* out;  // [tokens][out_stride]
    int out_stride;
    float* ws;  // optional workspace (linear_scan_workspace_bytes): conv in a token-parallel pass first
};
size_t linear_scan_workspace_bytes(int tokens, int lk_n, int lk_hd, int lv_n, int lv_hd);
bool linear_scan_supported(int lk_n, int lk_hd, int lv_n, int lv_hd, int ksize);
hipError_t launch_linear_scan(const LinearScanLaunch& p, hipStream_t s);

}  // namespace xqhip
