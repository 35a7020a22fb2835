// device_model.hpp - the decode model resident on one MI355X.
//
// Replaces CustomModel (customlib/runtime/custom_model.hpp:38-146,
// custom_model.cpp:423-1447) with the same load / prefill / decodeOne /
// resetState / coverageSummary / debugJson / copyHidden behaviour.  All weights,
// the fp16 KV cache, the fp32 recurrent state and every activation live in HBM;
// the host only feeds (position, token) and reads back the sampled token.
// A decode step is two captured HIP graphs: the lm_head argmax that samples the
// token, then the forward pass of that token through every layer (about six
// kernels per layer).  decode_one returns as soon as the token is known and
// leaves the forward pass running on the stream, so the host's work between
// steps overlaps the device's; every call that reads device state first waits
// for it (sync).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "kernel_trace.hpp"
#include "model_files.hpp"
#include "xqhip.h"

namespace xqh {

class DeviceModel {
public:
    DeviceModel() = default;
    ~DeviceModel();
    DeviceModel(const DeviceModel&) = delete;
    DeviceModel& operator=(const DeviceModel&) = delete;

    bool load(const std::string& model_dir, const std::string& backend_request, int max_context, std::string* error);
    bool prefill(const int32_t* token_ids, size_t n_tokens, KernelTrace* trace, std::string* error);
    bool decode_one(int32_t* token_id, size_t position, KernelTrace* trace, std::string* error);
    // Waits for every enqueued step and credits the last graph step's time to
    // `trace` (dropped when null).  false on a device error.
    bool sync(KernelTrace* trace, std::string* error);
    void reset_state();

    int hidden_size() const { return hidden_; }
    int vocab_size() const { return vocab_; }
    int layers() const { return static_cast<int>(layers_.size()); }
    std::string coverage_summary() const;
    std::string debug_json(int top_k);
    bool copy_hidden(float* out_values, size_t value_capacity, size_t* out_size);
    uint64_t weight_bytes_per_token() const { return weight_bytes_; }
    const std::string& device_name() const { return device_name_; }

private:
    struct Layer {
        bool full = false;
        // norms (reference +1 already applied where the reference applies it)
        float* in_norm = nullptr;
        float* post_norm = nullptr;
        float* q_norm = nullptr;
        float* k_norm = nullptr;
        float* lin_norm = nullptr;
        float* conv_w = nullptr;
        float* a_log = nullptr;
        float* dt_bias = nullptr;
        // weights: fused input projection, output projection, gate/up (interleaved), down
        xqhip_w4 in_proj{};
        xqhip_w4 out_proj{};
        xqhip_w4 gate_up{};
        xqhip_w4 down{};
        bool q_gated = false;
        // state
        void* k_cache = nullptr;  // fp16 [max_ctx][nkv][hd]
        void* v_cache = nullptr;
        float* conv_state = nullptr;  // [conv_dim][ksize-1]
        float* rec_state = nullptr;   // [lv_n][lk_hd][lv_hd]
    };

    struct TimedOp {
        std::string name;
        std::vector<std::string> extra_names;  // rows that share this op's time
        int split = 1;                         // time divided over extra rows (fused attention)
        void* ev0 = nullptr;
        void* ev1 = nullptr;
        int ts0 = -1, ts1 = -1;  // traced graph: slots of h_ts_ (timestamp kernels) instead of events
    };

    bool upload_matrix(const HostMatrix& m, xqhip_w4* out, std::string* error);
    bool upload_vec(const std::vector<float>& v, float** out, std::string* error);
    template <typename T>
    bool alloc(T** p, size_t count, std::string* error);
    bool load_layer(int index, Layer* L, std::string* error);
    bool build_rope_table(std::string* error);
    bool ensure_capacity(size_t positions, std::string* error);
    bool select_attention(size_t ctx, KernelTrace* trace, std::string* error);
    void release(void* p);

    // enqueue one token through all layers (reads pos from d_ctrl_[0])
    bool enqueue_layers(bool timed, std::string* error);
    bool enqueue_embed(const int32_t* token_dev, bool timed, std::string* error);
    bool enqueue_lm_head(bool timed, std::string* error);
    bool read_slot(long long want, int32_t* token_id, std::string* error) const;
    // credits the first n enqueued graph steps (complete by then) to `trace`
    void credit_steps(KernelTrace* trace, size_t n);
    void* next_step_event();
    bool op_begin(bool timed, const std::string& name, std::vector<std::string> extra = {}, int split = 1);
    void op_end(bool timed);
    void flush_timed(KernelTrace* trace);
    bool ensure_graphs(std::string* error);
    void drop_graphs();
    // decode chains: the projections between two non-GEMV ops as one launch
    bool build_chains(std::string* error);
    bool setup_step_fusion(std::string* error);
    bool enqueue_chain(size_t k, bool timed, std::string* error);
    // batched prefill of prompt chunks (GEMMs on the matrix cores)
    bool prefill_chunk(const int32_t* h_tokens, const int32_t* h_pos, int n, int pos0, bool timed,
                       std::string* error);
    bool alloc_prefill_buffers(std::string* error);
    bool fail_hip(std::string* error, const char* what);

    // dimensions (defaults of custom_model.hpp:98-114)
    int hidden_ = 4096, inter_ = 12288, vocab_ = 248320, nq_ = 16, nkv_ = 4, hd_ = 256, rot_ = 64;
    int lk_hd_ = 128, lv_hd_ = 128, lk_n_ = 16, lv_n_ = 32, ksize_ = 4, lk_dim_ = 2048, lv_dim_ = 4096;
    int conv_dim_ = 8192;
    float eps_ = 1.0e-6f, theta_ = 10000000.0f;
    static constexpr int kMaxContext = 1 << 20;  // the attention kernels' limit
    int max_ctx_ = 8192;                          // KV capacity (positions), grows on demand
    // Decode attention of the full-attention layers at head_dim 128, by
    // context (attention + o_proj GEMV per layer, 32q/8kv, measured in step
    // graphs): one block per query head below kSplitMinCtx (9.9 against 10.8
    // us at 256 tokens, 10.7 / 10.9 at 384); kAttnSplits context splits per
    // query head merged by each head's last block from there on (10.9 / 11.0
    // / 11.8 / 19.7 / 53.1 us at 512 / 1024 / 2048 / 8191 / 32767 tokens
    // against 11.6 / 15.3 / 22.5 / 80.1 / 314.6 for one block per head and
    // 16.4 / 17.1 / 18.8 / 38.0 / 109.1 for the slot kernel + merge, which
    // serves other head sizes).  The step graphs hold one of them and are
    // captured again on a switch.
    enum class AttnMode { kSlot, kHead, kSplit };
    static constexpr int kSplitMinCtx = 400, kAttnSplits = 8;
    static constexpr int kHeadAttnMaxCtx = 1024;  // without splits (XQ_ATTN_SPLITS=0): one block per head up to here
    AttnMode attn_mode_ = AttnMode::kSlot;
    std::string model_dir_, backend_request_, device_name_;
    uint64_t weight_bytes_ = 0;
    int inexact_meta_ = 0;
    static constexpr int kLayouts = 5;  // matrices uploaded per XQHIP_LAYOUT_* value
    int layout_count_[kLayouts] = {};

    std::vector<Layer> layers_;
    xqhip_w4 lm_head_{};
    float* final_norm_ = nullptr;
    uint16_t* embed_ = nullptr;
    float* rope_cs_ = nullptr;

    // activations / workspaces
    float* resid_ = nullptr;     // fp32 residual stream (pre final-norm)
    float* normed_ = nullptr;    // final-normed hidden (exposed hidden state)
    float* proj_ = nullptr;      // fused input projection output
    float* attn_ = nullptr;      // attention / delta output
    void* attn_split_ws_ = nullptr;  // split attention partials + per-head counters (zeroed once)
    float* ffn_ = nullptr;
    float* logits_ = nullptr;    // debug_json only
    float* best_val_ = nullptr;
    void* argmax_ws_ = nullptr;
    void* gqa_ws_ = nullptr;
    int32_t* d_ctrl_ = nullptr;  // [0] position, [1] input token, [2] sampled token
    int32_t* h_ctrl_ = nullptr;  // pinned staging, 2 ints per queued token
    size_t h_ctrl_cap_ = 0;
    int32_t* h_tok_ = nullptr;   // pinned control staging of the decode step
    uint64_t* h_slot_ = nullptr; // coherent pinned: (position << 32) | sampled token, stored by the sampling kernel
    static constexpr long long kPosUnknown = -(1LL << 40);
    long long dev_pos_ = kPosUnknown;  // d_ctrl_[0] once the queued work has run, if known
    void* stream_ = nullptr;
    void* g_prefill_ = nullptr;  // graph: embed(input token) + layers
    // graph: lm_head argmax -> sampled token (d_ctrl_[2]), d_ctrl_[0] + 1 and the
    // published slot, then embed(sampled token) + layers at the new position
    void* g_step_ = nullptr;
    // Decode-step timing: every graph step records an end event, and a step
    // that follows the previous one is timed from that step's end event (one
    // event per step between the graphs); steps are credited once a later
    // step has started (its sampling ran after them) or at a sync.
    static constexpr int kStepEvents = 8;  // ring: at most two steps (four events) are ever pending
    void* step_ev_[kStepEvents] = {};
    int step_ev_next_ = 0;
    void* last_end_ = nullptr;  // end event of the last graph step
    struct PendingStep {
        void* start;
        void* end;
        bool traced;
    };
    std::vector<PendingStep> pending_;
    // The traced step graph: the same kernels with a timestamp after every op,
    // replayed instead of g_step_ on the first step after each prefill and on
    // every trace_every_-th graph step (XQ_TRACE_EVERY; 0: only after a
    // prefill), so the trace has per-op rows of graph steps all along.
    void* g_step_traced_ = nullptr;
    std::vector<TimedOp> traced_ops_;
    // timestamps of the traced graph (xqhip_timestamp kernels between its ops,
    // 100 MHz counter) in coherent host memory; ts_mode_ while it is captured
    static constexpr int kMaxTimestamps = 1024;
    uint64_t* h_ts_ = nullptr;
    int ts_next_ = 0;
    bool ts_mode_ = false;
    int trace_every_ = 128;
    uint64_t graph_steps_ = 0, traced_steps_ = 0;
    bool trace_next_ = true;
    std::string trace_note_ = "per_op_every_128_graph_steps";
    KernelTrace* trace_ = nullptr;  // the trace passed with the last prefill / decode / sync
    bool chained_ = false;          // the last work enqueued is a graph step
    bool detail_prefill_ = true, detail_decode_ = true;
    // prompt-chunk buffers, [token][...] rows (allocated when every matrix is TILED64)
    bool batched_prefill_ = false;
    int chunk_ = 512;
    int max_proj_ = 1, attn_n_ = 1;
    float* x_all_ = nullptr;     // [chunk][hidden] residual stream
    float* proj_all_ = nullptr;  // [chunk][max_proj] fused input projections
    float* q_all_ = nullptr;     // [chunk][nq * hd]
    float* gate_all_ = nullptr;  // [chunk][nq * hd]
    float* attn_all_ = nullptr;  // [chunk][attn_n] attention / delta output
    float* ffn_all_ = nullptr;   // [chunk][inter]
    void* gemm_ws_ = nullptr;
    size_t gemm_ws_bytes_ = 0;
    void* scan_ws_ = nullptr;  // linear-attention scan workspace (token-parallel conv pass)
    int32_t* tok_dev_ = nullptr;  // [chunk]
    std::vector<TimedOp> ops_;
    std::vector<void*> event_pool_;
    size_t event_next_ = 0;
    bool op_chained_ = false;  // the last event recorded on the stream ended the last timed op
    std::vector<void*> allocations_;
    std::vector<xqhip_w4*> matrices_;
    // Decode chains (xqhip_chain_*): chain 0 = layer 0's input projection,
    // chain k (1 <= k < layers) = layer k-1's output projection, gate/up and
    // down and layer k's input projection, the last = the last layer's output
    // projection, gate/up and down.  Between chains k and k+1 runs layer k's
    // attention or linear-attention step.  Empty when a matrix does not fit
    // (then every projection is its own GEMV launch).
    std::vector<void*> chains_;
    std::vector<std::string> chain_names_;
    void* chain_arena_ = nullptr;
    void* chain_sync_ = nullptr;
    std::string chain_note_ = "off";  // why the chains are not used, or "on"
    // the linear-attention step and its output projection as one launch
    // (xqhip_linear_attn_step_outproj) in the per-op decode path
    bool fuse_step_ = false;
    void* fuse_sync_ = nullptr;
    std::string fuse_note_ = "off";
};

}  // namespace xqh
