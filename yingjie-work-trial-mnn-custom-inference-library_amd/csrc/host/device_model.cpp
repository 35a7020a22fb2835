// device_model.cpp - see device_model.hpp.
//
// Op order per layer follows CustomModel::runLayer (custom_model.cpp:1138-1256);
// fused kernels are named after every reference op they absorb, so the kernel
// trace keeps the reference's row vocabulary.
#include "device_model.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <mutex>
#include <sstream>

namespace xqh {
namespace {

using Clock = std::chrono::steady_clock;
const char* kTraceBackend = "hip";

// One stream for every model of the process: the decode chains need all CUs
// at once, so two models' steps must never run side by side (xq_decode_one
// returns while the step's forward pass still runs).  Shared and counted;
// destroyed with the last model.
std::mutex g_stream_mu;
void* g_stream = nullptr;
int g_stream_users = 0;

void* acquire_stream() {
    std::lock_guard<std::mutex> lock(g_stream_mu);
    if (!g_stream && xqhip_stream_create(&g_stream) != 0) return nullptr;
    ++g_stream_users;
    return g_stream;
}

void release_stream() {
    std::lock_guard<std::mutex> lock(g_stream_mu);
    if (--g_stream_users == 0 && g_stream) {
        xqhip_stream_destroy(g_stream);
        g_stream = nullptr;
    }
}

double elapsed_ms(void* a, void* b) {
    float ms = 0.0f;
    if (xqhip_event_elapsed_ms(a, b, &ms) != 0) return 0.0;
    return static_cast<double>(ms);
}

}  // namespace

#define XQ_CALL(expr, what) \
    if ((expr) != 0) return fail_hip(error, what)

DeviceModel::~DeviceModel() {
    if (stream_) xqhip_stream_synchronize(stream_);
    if (g_prefill_) xqhip_graph_destroy(g_prefill_);
    if (g_step_) xqhip_graph_destroy(g_step_);
    for (void* c : chains_) xqhip_chain_destroy(c);
    if (g_step_traced_) xqhip_graph_destroy(g_step_traced_);
    for (void* e : step_ev_)
        if (e) xqhip_event_destroy(e);
    for (xqhip_w4* m : matrices_) xqhip_w4_free(m);
    for (void* p : allocations_) xqhip_free(p);
    for (void* e : event_pool_) xqhip_event_destroy(e);
    if (h_ctrl_) xqhip_host_free(h_ctrl_);
    if (h_tok_) xqhip_host_free(h_tok_);
    if (h_slot_) xqhip_host_free(h_slot_);
    if (h_ts_) xqhip_host_free(h_ts_);
    if (stream_) release_stream();
}

bool DeviceModel::fail_hip(std::string* error, const char* what) {
    *error = std::string(what) + ": " + xqhip_last_error();
    return false;
}

template <typename T>
bool DeviceModel::alloc(T** p, size_t count, std::string* error) {
    void* q = nullptr;
    if (xqhip_malloc(&q, std::max<size_t>(1, count * sizeof(T))) != 0) return fail_hip(error, "device allocation");
    allocations_.push_back(q);
    *p = static_cast<T*>(q);
    return true;
}

bool DeviceModel::upload_vec(const std::vector<float>& v, float** out, std::string* error) {
    if (!alloc(out, v.size(), error)) return false;
    if (xqhip_memcpy_h2d(*out, v.data(), v.size() * sizeof(float), nullptr) != 0) return fail_hip(error, "upload");
    return true;
}

bool DeviceModel::upload_matrix(const HostMatrix& m, xqhip_w4* out, std::string* error) {
    if (xqhip_w4_upload(m.packed.data(), m.scales.data(), m.zeros.data(), m.rows, m.cols, m.group, m.affine ? 1 : 0,
                        out) != 0)
        return fail_hip(error, "weight upload");
    matrices_.push_back(out);
    weight_bytes_ += xqhip_w4_weight_bytes(out);
    inexact_meta_ += out->inexact_meta;
    if (out->layout >= 0 && out->layout < kLayouts) ++layout_count_[out->layout];
    return true;
}

static void add_one(std::vector<float>* v) {
    for (float& x : *v) x += 1.0f;
}

bool DeviceModel::load_layer(int index, Layer* L, std::string* error) {
    const std::string p = model_dir_ + "/layers_" + std::to_string(index) + "_";
    std::vector<float> in_norm, post_norm;
    HostMatrix gate, up, down;
    if (!read_f32_file(p + "input_layernorm_weight.f32", hidden_, &in_norm, error) ||
        !read_f32_file(p + "post_attention_layernorm_weight.f32", hidden_, &post_norm, error) ||
        !read_xq4_file(p + "mlp_gate_proj_weight.xq4", &gate, error) ||
        !read_xq4_file(p + "mlp_up_proj_weight.xq4", &up, error) ||
        !read_xq4_file(p + "mlp_down_proj_weight.xq4", &down, error))
        return false;
    add_one(&in_norm);  // custom_model.cpp:524-525
    add_one(&post_norm);
    if (gate.rows != inter_ || up.rows != inter_ || gate.cols != hidden_ || down.cols != inter_ ||
        down.rows != hidden_) {
        *error = "layer " + std::to_string(index) + ": MLP shapes disagree with the manifest";
        return false;
    }
    HostMatrix gu;
    if (!interleave_rows(gate, up, &gu, error) || !upload_matrix(gu, &L->gate_up, error) ||
        !upload_matrix(down, &L->down, error) || !upload_vec(in_norm, &L->in_norm, error) ||
        !upload_vec(post_norm, &L->post_norm, error))
        return false;

    if (file_exists(p + "self_attn_q_proj_weight.xq4")) {  // custom_model.cpp:526
        L->full = true;
        HostMatrix q, k, v, o;
        std::vector<float> qn, kn;
        if (!read_xq4_file(p + "self_attn_q_proj_weight.xq4", &q, error) ||
            !read_xq4_file(p + "self_attn_k_proj_weight.xq4", &k, error) ||
            !read_xq4_file(p + "self_attn_v_proj_weight.xq4", &v, error) ||
            !read_xq4_file(p + "self_attn_o_proj_weight.xq4", &o, error) ||
            !read_f32_file(p + "self_attn_q_norm_weight.f32", hd_, &qn, error) ||
            !read_f32_file(p + "self_attn_k_norm_weight.f32", hd_, &kn, error))
            return false;
        add_one(&qn);  // custom_model.cpp:536-537
        add_one(&kn);
        L->q_gated = q.rows >= nq_ * 2 * hd_;  // custom_model.cpp:742
        const int q_rows = nq_ * hd_ * (L->q_gated ? 2 : 1);
        if (q.rows != q_rows || k.rows != nkv_ * hd_ || v.rows != nkv_ * hd_ || q.cols != hidden_ ||
            o.cols != nq_ * hd_ || o.rows != hidden_ || nq_ * hd_ > std::max(hidden_, lv_dim_)) {
            *error = "layer " + std::to_string(index) + ": attention shapes disagree with the manifest";
            return false;
        }
        HostMatrix qkv;
        if (!concat_rows({&q, &k, &v}, &qkv, error) || !upload_matrix(qkv, &L->in_proj, error) ||
            !upload_matrix(o, &L->out_proj, error) || !upload_vec(qn, &L->q_norm, error) ||
            !upload_vec(kn, &L->k_norm, error))
            return false;
        const size_t kv = static_cast<size_t>(max_ctx_) * nkv_ * hd_;
        uint16_t *kc = nullptr, *vc = nullptr;
        if (!alloc(&kc, kv, error) || !alloc(&vc, kv, error)) return false;
        L->k_cache = kc;
        L->v_cache = vc;
        return true;
    }
    L->full = false;
    HostMatrix qkv, a, b, z, out;
    std::vector<float> lin_norm, conv_w, a_log, dt_bias;
    if (!read_xq4_file(p + "linear_attn_in_proj_qkv_weight.xq4", &qkv, error) ||
        !read_xq4_file(p + "linear_attn_in_proj_a_weight.xq4", &a, error) ||
        !read_xq4_file(p + "linear_attn_in_proj_b_weight.xq4", &b, error) ||
        !read_xq4_file(p + "linear_attn_in_proj_z_weight.xq4", &z, error) ||
        !read_xq4_file(p + "linear_attn_out_proj_weight.xq4", &out, error) ||
        !read_f32_file(p + "linear_attn_norm_weight.f32", lv_hd_, &lin_norm, error) ||
        !read_f32_file(p + "linear_attn_conv1d_weight.f32", conv_dim_ * ksize_, &conv_w, error) ||
        !read_f32_file(p + "linear_attn_A_log.f32", lv_n_, &a_log, error) ||
        !read_f32_file(p + "linear_attn_dt_bias.f32", lv_n_, &dt_bias, error))
        return false;
    if (qkv.rows != conv_dim_ || a.rows != lv_n_ || b.rows != lv_n_ || z.rows != lv_dim_ || qkv.cols != hidden_ ||
        out.cols != lv_dim_ || out.rows != hidden_) {
        *error = "layer " + std::to_string(index) + ": linear-attention shapes disagree with the manifest";
        return false;
    }
    HostMatrix fused;
    if (!concat_rows({&qkv, &a, &b, &z}, &fused, error) || !upload_matrix(fused, &L->in_proj, error) ||
        !upload_matrix(out, &L->out_proj, error) || !upload_vec(lin_norm, &L->lin_norm, error) ||
        !upload_vec(conv_w, &L->conv_w, error) || !upload_vec(a_log, &L->a_log, error) ||
        !upload_vec(dt_bias, &L->dt_bias, error))
        return false;
    return alloc(&L->conv_state, 2 * static_cast<size_t>(conv_dim_) * std::max(0, ksize_ - 1), error) &&
           alloc(&L->rec_state, static_cast<size_t>(lv_n_) * lk_hd_ * lv_hd_, error);
}

bool DeviceModel::load(const std::string& model_dir, const std::string& backend_request, int max_context,
                       std::string* error) {
    model_dir_ = model_dir;
    backend_request_ = backend_request.empty() ? "cpu" : backend_request;
    if (xqhip_device_count() < 1) {
        *error = "no HIP device visible: this library runs the decode path on an MI355X and has no CPU path";
        return false;
    }
    if (xqhip_set_device(0) != 0) return fail_hip(error, "select device");
    char name[256] = {};
    xqhip_device_name(name, sizeof(name));
    device_name_ = name;

    const std::string js = read_text(model_dir + "/xqwen35_manifest.json");  // custom_model.cpp:431-453
    hidden_ = manifest_int(js, "hidden_size", hidden_);
    inter_ = manifest_int(js, "intermediate_size", inter_);
    vocab_ = manifest_int(js, "vocab_size", vocab_);
    nq_ = manifest_int(js, "num_attention_heads", nq_);
    nkv_ = manifest_int(js, "num_key_value_heads", nkv_);
    hd_ = manifest_int(js, "head_dim", hd_);
    const float prf = manifest_float(js, "partial_rotary_factor", 0.25f);
    rot_ = std::max(2, static_cast<int>(std::round(static_cast<float>(hd_) * prf)));
    if (rot_ & 1) --rot_;
    lk_hd_ = manifest_int(js, "linear_key_head_dim", lk_hd_);
    lv_hd_ = manifest_int(js, "linear_value_head_dim", lv_hd_);
    lk_n_ = manifest_int(js, "linear_num_key_heads", lk_n_);
    lv_n_ = manifest_int(js, "linear_num_value_heads", lv_n_);
    ksize_ = manifest_int(js, "linear_conv_kernel_dim", ksize_);
    lk_dim_ = lk_hd_ * lk_n_;
    lv_dim_ = lv_hd_ * lv_n_;
    conv_dim_ = 2 * lk_dim_ + lv_dim_;
    eps_ = manifest_float(js, "rms_norm_eps", eps_);
    theta_ = manifest_float(js, "rope_theta", theta_);
    const int n_layers = manifest_int(js, "num_hidden_layers", 32);
    // KV capacity: the reference grows its caches as tokens arrive
    // (custom_model.cpp:616-622, 673-733); here they start at
    // max(8192, max_context_tokens) positions and double when a prompt or a
    // decode position needs more (ensure_capacity), up to kMaxContext.
    if (max_context > kMaxContext) {
        *error = "max_context_tokens " + std::to_string(max_context) + " exceeds the supported " +
                 std::to_string(kMaxContext);
        return false;
    }
    max_ctx_ = std::max(8192, max_context);
    if (hidden_ <= 0 || vocab_ <= 0 || n_layers < 0 || nq_ <= 0 || nkv_ <= 0 || hd_ <= 0 || nq_ % nkv_ != 0) {
        *error = "invalid model dimensions in xqwen35_manifest.json";
        return false;
    }

    // embeddings (custom_model.cpp:454-464): whole table resident in HBM
    {
        std::ifstream f(model_dir + "/embeddings_bf16.bin", std::ios::binary | std::ios::ate);
        if (!f) {
            *error = "missing embeddings_bf16.bin";
            return false;
        }
        const uint64_t want = static_cast<uint64_t>(vocab_) * hidden_ * 2;
        if (static_cast<uint64_t>(f.tellg()) < want) {
            *error = "short embeddings_bf16.bin";
            return false;
        }
        std::vector<uint16_t> host(static_cast<size_t>(want / 2));
        f.seekg(0);
        f.read(reinterpret_cast<char*>(host.data()), static_cast<std::streamsize>(want));
        if (!alloc(&embed_, host.size(), error)) return false;
        if (xqhip_memcpy_h2d(embed_, host.data(), want, nullptr) != 0) return fail_hip(error, "embedding upload");
    }
    std::vector<float> fn;
    if (!read_f32_file(model_dir + "/norm_weight.f32", hidden_, &fn, error)) return false;
    add_one(&fn);  // custom_model.cpp:468
    HostMatrix lm;
    if (!upload_vec(fn, &final_norm_, error) || !read_xq4_file(model_dir + "/lm_head_weight.xq4", &lm, error) ||
        !upload_matrix(lm, &lm_head_, error))
        return false;
    layers_.assign(static_cast<size_t>(n_layers), Layer());  // sized once: matrices_ keeps pointers into it
    for (int i = 0; i < n_layers; ++i)
        if (!load_layer(i, &layers_[i], error)) return false;
    bool any_full = false, any_linear = false;
    int max_proj = 1;
    for (const Layer& L : layers_) {
        any_full |= L.full;
        any_linear |= !L.full;
        max_proj = std::max(max_proj, L.in_proj.rows);
    }
    if (any_full && xqhip_gqa_workspace_bytes(nq_, nkv_, hd_) == 0) {
        *error = "attention workspace";
        return false;
    }
    const int attn_n = std::max({nq_ * hd_, lv_dim_, hidden_});
    size_t ws_argmax = xqhip_argmax_workspace_bytes(lm_head_.rows);
    size_t ws_gqa = any_full ? xqhip_gqa_workspace_bytes(nq_, nkv_, hd_) : 1;
    size_t ws_split = any_full ? std::max<size_t>(1, xqhip_attn_split_workspace_bytes(nq_)) : 1;
    uint8_t *wa = nullptr, *wg = nullptr, *wsp = nullptr;
    if (!alloc(&resid_, hidden_, error) || !alloc(&normed_, hidden_, error) || !alloc(&proj_, max_proj, error) ||
        !alloc(&attn_, attn_n, error) ||

        !alloc(&ffn_, inter_, error) || !alloc(&best_val_, 1, error) || !alloc(&d_ctrl_, 4, error) ||
        !alloc(&wa, ws_argmax, error) || !alloc(&wg, ws_gqa, error) || !alloc(&wsp, ws_split, error))
        return false;
    argmax_ws_ = wa;
    gqa_ws_ = wg;
    attn_split_ws_ = wsp;
    stream_ = acquire_stream();
    if (!stream_) return fail_hip(error, "stream");
    xqhip_fill_u8(resid_, 0, sizeof(float) * hidden_, stream_);  // hidden_ starts at zero (custom_model.cpp:478)
    xqhip_fill_u8(argmax_ws_, 0, ws_argmax, stream_);
    xqhip_fill_u8(gqa_ws_, 0, ws_gqa, stream_);
    xqhip_fill_u8(attn_split_ws_, 0, ws_split, stream_);  // the split attention's counters start (and stay) at 0
    xqhip_fill_u8(d_ctrl_, 0, 16, stream_);
    if (any_full && !build_rope_table(error)) return false;
    (void)any_linear;
    max_proj_ = max_proj;
    attn_n_ = attn_n;
    if (!alloc_prefill_buffers(error)) return false;
    void* pinned = nullptr;
    if (xqhip_host_alloc(&pinned, 4 * sizeof(int32_t)) != 0) return fail_hip(error, "pinned memory");
    h_tok_ = static_cast<int32_t*>(pinned);
    if (xqhip_host_alloc_coherent(&pinned, sizeof(uint64_t)) != 0) return fail_hip(error, "coherent host memory");
    h_slot_ = static_cast<uint64_t*>(pinned);
    *h_slot_ = ~0ull;
    if (xqhip_host_alloc_coherent(&pinned, sizeof(uint64_t) * kMaxTimestamps) != 0)
        return fail_hip(error, "coherent host memory");
    h_ts_ = static_cast<uint64_t*>(pinned);
    for (void*& e : step_ev_)
        if (xqhip_event_create(&e) != 0) return fail_hip(error, "event");
    if (const char* v = std::getenv("XQ_TRACE_EVERY")) trace_every_ = std::max(0, std::atoi(v));
    trace_note_ = trace_every_ > 0 ? "per_op_every_" + std::to_string(trace_every_) + "_graph_steps"
                                   : std::string("per_op_first_step_after_prefill");
    if (!build_chains(error) || !setup_step_fusion(error)) return false;
    reset_state();
    return xqhip_stream_synchronize(stream_) == 0 || fail_hip(error, "load sync");
}

// The linear-attention layers' step and output projection as one launch
// (xqhip_linear_attn_step_outproj, bit-identical to the two) is opt-in,
// XQ_FUSE_STEP=1: measured on the 9B shapes it takes 15.9 us against 11.0 us
// for the two kernels, because its in-kernel hand-off between CUs of
// different XCDs (write-through stores, then polls that bypass the L2) costs
// 4-5 us where the kernel boundary costs 1.6 us.
bool DeviceModel::setup_step_fusion(std::string* error) {
    const char* v = std::getenv("XQ_FUSE_STEP");
    if (!v || v[0] != '1') {
        fuse_note_ = "off";
        return true;
    }
    bool any = false;
    for (const Layer& L : layers_) {
        if (L.full) continue;
        any = true;
        if (!xqhip_step_outproj_supported(&L.out_proj, lk_n_, lk_hd_, lv_n_, lv_hd_, ksize_)) {
            fuse_note_ = "off(unsupported)";
            return true;
        }
    }
    if (!any) {
        fuse_note_ = "off(no_linear_layers)";
        return true;
    }
    uint8_t* sync = nullptr;
    if (!alloc(&sync, xqhip_step_outproj_sync_bytes(), error)) return false;
    if (xqhip_fill_u8(sync, 0, xqhip_step_outproj_sync_bytes(), stream_) != 0) return fail_hip(error, "fill");
    fuse_sync_ = sync;
    fuse_step_ = true;
    fuse_note_ = "on";
    return true;
}

// Decode chains are opt-in (XQ_DECODE_CHAIN=1): measured on the 9B shapes a
// chain of out_proj, gate/up, down and the next in_proj takes 39.2 us against
// 33.5 us for the four GEMV launches (every in-kernel hand-off costs 2-4 us,
// as much as the kernel boundary it replaces), so the step graphs keep one
// launch per projection by default.
static bool chains_enabled() {
    const char* v = std::getenv("XQ_DECODE_CHAIN");
    return v && v[0] == '1';
}

bool DeviceModel::build_chains(std::string* error) {
    if (!chains_enabled()) {
        chain_note_ = "off";
        return true;
    }
    const size_t n = layers_.size();
    if (n == 0) return true;
    std::vector<std::vector<xqhip_chain_op>> specs(n + 1);
    std::vector<std::string> names(n + 1);
    auto plain = [](const float* p) {
        xqhip_chain_src s{};
        s.plain = p;
        return s;
    };
    auto from = [](int op, int offset) {
        xqhip_chain_src s{};
        s.plain = nullptr;
        s.op = op;
        s.offset = offset;
        return s;
    };
    for (size_t k = 0; k <= n; ++k) {
        std::vector<xqhip_chain_op>& ops = specs[k];
        std::string& nm = names[k];
        int down_op = -1;
        if (k > 0) {  // layer k-1: output projection, gate/up, down
            Layer& L = layers_[k - 1];
            xqhip_chain_op o{};
            o.w = &L.out_proj;
            o.epi = XQHIP_EPI_ADD;
            o.x = plain(attn_);
            o.res = plain(resid_);
            if (!L.full) {  // linear attention: gated head norm of the step output (gate already silu)
                o.pro = XQHIP_PRO_GATED_HEAD_ACT;
                o.pro_w = L.lin_norm;
                o.head_dim = lv_hd_;
                o.eps = eps_;
                o.gate = plain(proj_ + conv_dim_ + 2 * lv_n_);
            }
            ops.push_back(o);
            xqhip_chain_op g{};
            g.w = &L.gate_up;
            g.epi = XQHIP_EPI_SILU_PAIR;
            g.pro = XQHIP_PRO_RMS;
            g.pro_w = L.post_norm;
            g.eps = eps_;
            g.x = from(0, 0);
            ops.push_back(g);
            xqhip_chain_op dn{};
            dn.w = &L.down;
            dn.epi = XQHIP_EPI_ADD;
            dn.x = from(1, 0);
            dn.res = from(0, 0);
            dn.y_plain = resid_;
            ops.push_back(dn);
            down_op = 2;
            nm = L.full ? "decode_chain_w4a16(o_proj,residual_add_attention,gate_proj,up_proj,rmsnorm_post_attention,"
                          "silu_gate_mul,down_proj,residual_add_mlp"
                        : "decode_chain_w4a16(linear_attn_out_proj,linear_attention_gated_rmsnorm,residual_add_attention,"
                          "gate_proj,up_proj,rmsnorm_post_attention,silu_gate_mul,down_proj,residual_add_mlp";
        }
        if (k < n) {  // layer k's input projection
            Layer& L = layers_[k];
            xqhip_chain_op q{};
            q.w = &L.in_proj;
            q.epi = XQHIP_EPI_STORE;
            q.pro = XQHIP_PRO_RMS;
            q.pro_w = L.in_norm;
            q.eps = eps_;
            q.x = down_op >= 0 ? from(down_op, 0) : plain(resid_);
            q.y_plain = proj_;
            ops.push_back(q);
            nm += nm.empty() ? "decode_chain_w4a16(" : ",";
            nm += L.full ? "q_proj,k_proj,v_proj,rmsnorm_input" : "in_proj_qkv,in_proj_a,in_proj_b,in_proj_z,rmsnorm_input";
        }
        nm += ")";
    }
    std::vector<void*> made;
    size_t records = 0;
    for (size_t k = 0; k <= n; ++k) {
        void* c = nullptr;
        if (xqhip_chain_create(specs[k].data(), static_cast<int>(specs[k].size()), &c) != 0) {
            for (void* m : made) xqhip_chain_destroy(m);
            std::string why = xqhip_last_error();
            for (char& ch : why)
                if (ch == ';' || ch == '=') ch = ' ';  // the summary is a ;-separated key=value list
            chain_note_ = "off(" + why + ")";
            return true;  // the per-op launches serve this model
        }
        made.push_back(c);
        records = std::max(records, xqhip_chain_arena_records(c));
    }
    uint8_t *arena = nullptr, *sync = nullptr;
    if (!alloc(&arena, records * 8, error) || !alloc(&sync, xqhip_chain_sync_bytes(), error)) {
        for (void* m : made) xqhip_chain_destroy(m);
        return false;
    }
    xqhip_fill_u8(arena, 0, records * 8, stream_);
    xqhip_fill_u8(sync, 0, xqhip_chain_sync_bytes(), stream_);
    chain_arena_ = arena;
    chain_sync_ = sync;
    chains_ = std::move(made);
    chain_names_ = std::move(names);
    chain_note_ = "on";
    return true;
}

bool DeviceModel::enqueue_chain(size_t k, bool timed, std::string* error) {
    op_begin(timed, chain_names_[k]);
    XQ_CALL(xqhip_chain_launch(chains_[k], chain_arena_, chain_sync_, stream_), "decode chain");
    op_end(timed);
    return true;
}

bool DeviceModel::build_rope_table(std::string* error) {
    const int rot_active = std::max(0, std::min(hd_, rot_));
    if (rot_active <= 0) return true;
    if (rope_cs_) release(rope_cs_);
    rope_cs_ = nullptr;
    std::vector<float> tab(static_cast<size_t>(max_ctx_) * (rot_active / 2) * 2);
    xqhip_rope_table(theta_, rot_active, max_ctx_, tab.data());
    return upload_vec(tab, &rope_cs_, error);
}

void DeviceModel::release(void* p) {
    auto it = std::find(allocations_.begin(), allocations_.end(), p);
    if (it != allocations_.end()) allocations_.erase(it);
    xqhip_free(p);
}

// Grows the KV caches (and the RoPE table) to hold `positions` positions:
// capacity doubles, the cached prefix is copied, and the step graphs, which
// hold the old addresses, are captured again on their next use.
bool DeviceModel::ensure_capacity(size_t positions, std::string* error) {
    if (positions <= static_cast<size_t>(max_ctx_)) return true;
    if (positions > static_cast<size_t>(kMaxContext)) {
        *error = "context of " + std::to_string(positions) + " tokens exceeds the supported " +
                 std::to_string(kMaxContext);
        return false;
    }
    if (!sync(nullptr, error)) return false;
    const int old_ctx = max_ctx_;
    const int new_ctx = static_cast<int>(std::min<size_t>(kMaxContext, std::max<size_t>(positions, 2 * static_cast<size_t>(old_ctx))));
    const size_t row = static_cast<size_t>(nkv_) * hd_;
    for (Layer& L : layers_) {
        if (!L.full) continue;
        for (void** cache : {&L.k_cache, &L.v_cache}) {
            uint16_t* grown = nullptr;
            if (!alloc(&grown, static_cast<size_t>(new_ctx) * row, error)) return false;
            XQ_CALL(xqhip_memcpy_d2d(grown, *cache, sizeof(uint16_t) * static_cast<size_t>(old_ctx) * row, stream_),
                    "KV cache copy");
            release(*cache);
            *cache = grown;
        }
    }
    max_ctx_ = new_ctx;
    if (!build_rope_table(error)) return false;
    drop_graphs();
    return xqhip_stream_synchronize(stream_) == 0 || fail_hip(error, "KV cache growth");
}

static bool head_attention_enabled() {
    const char* v = std::getenv("XQ_HEAD_ATTENTION");
    return !(v && v[0] == '0');
}

// Context splits of the split attention; XQ_ATTN_SPLITS overrides the default
// (0: no split attention, for measurements).
static int attn_splits(int dflt) {
    const char* v = std::getenv("XQ_ATTN_SPLITS");
    if (!v || !*v) return dflt;
    const int n = std::atoi(v);
    return n < 0 ? 0 : (n > XQHIP_ATTN_MAX_SPLITS ? XQHIP_ATTN_MAX_SPLITS : n);
}

// Picks the attention kernel of the full-attention layers for a step whose
// context is `ctx` tokens.  The kernels give the same results within fp32
// rounding; the graphs that hold another one are dropped after the queued
// steps have finished.
bool DeviceModel::select_attention(size_t ctx, KernelTrace* trace, std::string* error) {
    const bool per_head = head_attention_enabled() && hd_ == 128 && nq_ % nkv_ == 0;
    const bool split = per_head && attn_splits(kAttnSplits) > 0;
    AttnMode want = AttnMode::kSlot;
    if (split && ctx >= static_cast<size_t>(kSplitMinCtx))
        want = AttnMode::kSplit;
    else if (per_head && ctx <= static_cast<size_t>(split ? kSplitMinCtx : kHeadAttnMaxCtx))
        want = AttnMode::kHead;
    if (want == attn_mode_) return true;
    if (!sync(trace, error)) return false;
    attn_mode_ = want;
    drop_graphs();
    return true;
}

void DeviceModel::reset_state() {  // custom_model.cpp:555-567 (KV slots past the position are never read)
    std::string ignored;
    sync(nullptr, &ignored);  // the trace of the steps being discarded is dropped with them
    for (Layer& L : layers_) {
        if (L.full) continue;
        xqhip_fill_u8(L.conv_state, 0, 2 * sizeof(float) * conv_dim_ * std::max(0, ksize_ - 1), stream_);
        xqhip_fill_u8(L.rec_state, 0, sizeof(float) * lv_n_ * lk_hd_ * lv_hd_, stream_);
    }
    detail_prefill_ = detail_decode_ = true;
    dev_pos_ = kPosUnknown;
    chained_ = false;
}

bool DeviceModel::op_begin(bool timed, const std::string& name, std::vector<std::string> extra, int split) {
    if (!timed) return true;
    TimedOp op;
    op.name = name;
    op.extra_names = std::move(extra);
    op.split = split;
    if (ts_mode_) {  // traced graph: a timestamp kernel before the op (unless the previous op's end marks it)
        if (op_chained_ && !ops_.empty()) {
            op.ts0 = ops_.back().ts1;
        } else {
            if (ts_next_ >= kMaxTimestamps || xqhip_timestamp(h_ts_ + ts_next_, stream_) != 0) return false;
            op.ts0 = ts_next_++;
        }
        op_chained_ = false;
        ops_.push_back(std::move(op));
        return true;
    }
    while (event_pool_.size() < event_next_ + 2) {
        void* e = nullptr;
        if (xqhip_event_create(&e) != 0) return false;
        event_pool_.push_back(e);
    }
    op.ev0 = event_pool_[event_next_++];
    op.ev1 = event_pool_[event_next_++];
    // an op that directly follows the previous one starts at its end event:
    // one event recorded on the stream per op instead of two
    if (op_chained_ && !ops_.empty())
        op.ev0 = ops_.back().ev1;
    else
        xqhip_event_record(op.ev0, stream_);
    op_chained_ = false;
    ops_.push_back(std::move(op));
    return true;
}

void DeviceModel::op_end(bool timed) {
    if (!timed || ops_.empty()) return;
    if (ts_mode_) {
        if (ts_next_ < kMaxTimestamps && xqhip_timestamp(h_ts_ + ts_next_, stream_) == 0) ops_.back().ts1 = ts_next_++;
    } else {
        xqhip_event_record(ops_.back().ev1, stream_);
    }
    op_chained_ = true;
}

void DeviceModel::flush_timed(KernelTrace* trace) {
    for (const TimedOp& op : ops_) {
        const double ms = elapsed_ms(op.ev0, op.ev1);
        if (trace) {
            trace->add(op.name, ms, kTraceBackend);
            for (const std::string& e : op.extra_names) trace->add(e, ms / op.split, kTraceBackend);
        }
    }
    ops_.clear();
    event_next_ = 0;
    op_chained_ = false;
}


bool DeviceModel::enqueue_embed(const int32_t* token_dev, bool timed, std::string* error) {
    op_begin(timed, "embedding_bf16_row_read");
    XQ_CALL(xqhip_embed_bf16(embed_, vocab_, hidden_, token_dev, resid_, stream_), "embedding");
    op_end(timed);
    return true;
}

bool DeviceModel::enqueue_lm_head(bool timed, std::string* error) {
    xqhip_prologue fin{XQHIP_PRO_RMS, 0, final_norm_, nullptr, eps_};
    op_begin(timed, "lm_head_custom(fused:rmsnorm_final,argmax,embedding)",
             {"sampling_greedy_custom", "embedding_bf16_row_read"});
    // the sampled token is the input of the next position: the finishing
    // kernel advances d_ctrl_[0], publishes (position, token) to h_slot_ and
    // writes the token's embedding row to resid_ (loadEmbeddingRow,
    // custom_model.cpp:569-608), which the next layers read
    XQ_CALL(xqhip_gemv_w4a16_argmax_publish_embed(&lm_head_, resid_, XQHIP_F32, &fin, argmax_ws_, d_ctrl_ + 2,
                                                  best_val_, d_ctrl_, h_slot_, static_cast<const uint16_t*>(embed_),
                                                  vocab_, hidden_, resid_, stream_),
            "lm_head argmax");
    op_end(timed);
    return true;
}

bool DeviceModel::enqueue_layers(bool timed, std::string* error) {
    const int32_t* pos = d_ctrl_;
    const bool chain = !chains_.empty();
    if (chain && !enqueue_chain(0, timed, error)) return false;
    for (size_t li = 0; li < layers_.size(); ++li) {
        Layer& L = layers_[li];
        xqhip_prologue rms_in{XQHIP_PRO_RMS, 0, L.in_norm, nullptr, eps_};
        if (chain) {  // the layer's attention or linear-attention step between two chains
            if (L.full) {
                const float* k_src = proj_ + static_cast<size_t>(nq_) * hd_ * (L.q_gated ? 2 : 1);
                const float* v_src = k_src + static_cast<size_t>(nkv_) * hd_;
                op_begin(timed, "attention_gqa_decode_custom(fused:q_norm,k_norm,rope_qk,kv_append,output_gate)",
                         {"prefill_kv_build_custom", "attention_score_custom", "attention_softmax_custom",
                          "attention_v_reduce_custom"},
                         4);
                if (attn_mode_ == AttnMode::kSplit) {
                    XQ_CALL(xqhip_attn_decode_split(proj_, k_src, v_src, L.q_gated ? 1 : 0, nq_, nkv_, hd_, rot_,
                                                    L.q_norm, L.k_norm, eps_, rope_cs_, pos, L.k_cache, L.v_cache,
                                                    attn_splits(kAttnSplits), attn_split_ws_, attn_, stream_),
                            "attention decode");
                } else if (attn_mode_ == AttnMode::kHead) {
                    XQ_CALL(xqhip_attn_decode_head(proj_, k_src, v_src, L.q_gated ? 1 : 0, nq_, nkv_, hd_, rot_,
                                                   L.q_norm, L.k_norm, eps_, rope_cs_, pos, L.k_cache, L.v_cache, attn_,
                                                   stream_),
                            "attention decode");
                } else {
                    XQ_CALL(xqhip_attn_decode(proj_, k_src, v_src, L.q_gated ? 1 : 0, nq_, nkv_, hd_, rot_, L.q_norm,
                                              L.k_norm, eps_, rope_cs_, pos, L.k_cache, L.v_cache, max_ctx_, attn_,
                                              gqa_ws_, stream_),
                            "attention decode");
                }
                op_end(timed);
            } else {
                const float* a = proj_ + conv_dim_;
                const float* b = a + lv_n_;
                float* z = proj_ + conv_dim_ + 2 * lv_n_;
                op_begin(timed, "linear_attention_state_update_custom(fused:conv1d,qk_l2norm,gated_delta)",
                         {"linear_attention_conv1d_custom"}, 2);
                XQ_CALL(xqhip_linear_attn_step_act(proj_, L.conv_state, L.conv_w, a, b, L.a_log, L.dt_bias,
                                                   L.rec_state, lk_n_, lk_hd_, lv_n_, lv_hd_, ksize_, pos, attn_, z,
                                                   stream_),
                        "linear-attention step");
                op_end(timed);
            }
            if (!enqueue_chain(li + 1, timed, error)) return false;
            continue;
        }
        if (L.full) {
            op_begin(timed, "linear_q_proj_w4a16(fused:k_proj,v_proj,rmsnorm_input)");
            XQ_CALL(xqhip_gemv_w4a16(&L.in_proj, resid_, XQHIP_F32, &rms_in, proj_, XQHIP_F32, XQHIP_EPI_STORE, stream_),
                    "qkv projection");
            op_end(timed);
            const float* k_src = proj_ + static_cast<size_t>(nq_) * hd_ * (L.q_gated ? 2 : 1);
            const float* v_src = k_src + static_cast<size_t>(nkv_) * hd_;
            op_begin(timed, "attention_gqa_decode_custom(fused:q_norm,k_norm,rope_qk,kv_append,output_gate)",
                     {"prefill_kv_build_custom", "attention_score_custom", "attention_softmax_custom",
                      "attention_v_reduce_custom"},
                     4);
            if (attn_mode_ == AttnMode::kSplit) {
                XQ_CALL(xqhip_attn_decode_split(proj_, k_src, v_src, L.q_gated ? 1 : 0, nq_, nkv_, hd_, rot_, L.q_norm,
                                                L.k_norm, eps_, rope_cs_, pos, L.k_cache, L.v_cache,
                                                attn_splits(kAttnSplits), attn_split_ws_, attn_, stream_),
                        "attention decode");
            } else if (attn_mode_ == AttnMode::kHead) {
                XQ_CALL(xqhip_attn_decode_head(proj_, k_src, v_src, L.q_gated ? 1 : 0, nq_, nkv_, hd_, rot_, L.q_norm,
                                               L.k_norm, eps_, rope_cs_, pos, L.k_cache, L.v_cache, attn_, stream_),
                        "attention decode");
            } else {
                XQ_CALL(xqhip_attn_decode(proj_, k_src, v_src, L.q_gated ? 1 : 0, nq_, nkv_, hd_, rot_, L.q_norm,
                                          L.k_norm, eps_, rope_cs_, pos, L.k_cache, L.v_cache, max_ctx_, attn_, gqa_ws_,
                                          stream_),
                        "attention decode");
            }
            op_end(timed);
            op_begin(timed, "linear_o_proj_w4a16(fused:residual_add_attention)");
            XQ_CALL(xqhip_gemv_w4a16(&L.out_proj, attn_, XQHIP_F32, nullptr, resid_, XQHIP_F32, XQHIP_EPI_ADD, stream_),
                    "o projection");
            op_end(timed);
        } else {
            op_begin(timed, "linear_attn_in_proj_qkv_w4a16(fused:in_proj_a,in_proj_b,in_proj_z,rmsnorm_input)");
            XQ_CALL(xqhip_gemv_w4a16(&L.in_proj, resid_, XQHIP_F32, &rms_in, proj_, XQHIP_F32, XQHIP_EPI_STORE, stream_),
                    "linear-attention in projection");
            op_end(timed);
            const float* a = proj_ + conv_dim_;
            const float* b = a + lv_n_;
            float* z = proj_ + conv_dim_ + 2 * lv_n_;
            if (fuse_step_) {  // one launch: the step, then the projection of its output
                op_begin(timed,
                         "linear_attention_state_update_custom+linear_attn_out_proj_w4a16(fused:conv1d,qk_l2norm,"
                         "gated_delta,linear_attention_gated_rmsnorm,residual_add_attention)",
                         {"linear_attention_conv1d_custom"}, 2);
                XQ_CALL(xqhip_linear_attn_step_outproj(proj_, L.conv_state, L.conv_w, a, b, L.a_log, L.dt_bias,
                                                       L.rec_state, lk_n_, lk_hd_, lv_n_, lv_hd_, ksize_, pos, attn_,
                                                       z, &L.out_proj, L.lin_norm, eps_, resid_, fuse_sync_, stream_),
                        "linear-attention step + out projection");
                op_end(timed);
            } else {
                // the step also replaces z by silu(z) once, for the output norm's prologue
                op_begin(timed, "linear_attention_state_update_custom(fused:conv1d,qk_l2norm,gated_delta)",
                         {"linear_attention_conv1d_custom"}, 2);
                XQ_CALL(xqhip_linear_attn_step_act(proj_, L.conv_state, L.conv_w, a, b, L.a_log, L.dt_bias,
                                                   L.rec_state, lk_n_, lk_hd_, lv_n_, lv_hd_, ksize_, pos, attn_, z,
                                                   stream_),
                        "linear-attention step");
                op_end(timed);
                xqhip_prologue gated{XQHIP_PRO_GATED_HEAD_ACT, lv_hd_, L.lin_norm, z, eps_};
                op_begin(timed,
                         "linear_attn_out_proj_w4a16(fused:linear_attention_gated_rmsnorm,residual_add_attention)");
                XQ_CALL(xqhip_gemv_w4a16(&L.out_proj, attn_, XQHIP_F32, &gated, resid_, XQHIP_F32, XQHIP_EPI_ADD,
                                         stream_),
                        "out projection");
                op_end(timed);
            }
        }
        xqhip_prologue rms_post{XQHIP_PRO_RMS, 0, L.post_norm, nullptr, eps_};
        op_begin(timed, "linear_gate_proj_w4a16(fused:up_proj,rmsnorm_post_attention,silu_gate_mul)");
        XQ_CALL(xqhip_gemv_w4a16(&L.gate_up, resid_, XQHIP_F32, &rms_post, ffn_, XQHIP_F32, XQHIP_EPI_SILU_PAIR, stream_),
                "gate/up projection");
        op_end(timed);
        op_begin(timed, "linear_down_proj_w4a16(fused:residual_add_mlp)");
        XQ_CALL(xqhip_gemv_w4a16(&L.down, ffn_, XQHIP_F32, nullptr, resid_, XQHIP_F32, XQHIP_EPI_ADD, stream_),
                "down projection");
        op_end(timed);
    }
    return true;
}

static bool graphs_enabled() {
    const char* v = std::getenv("XQ_DECODE_GRAPHS");
    return !(v && v[0] == '0');
}

void DeviceModel::drop_graphs() {
    for (void** g : {&g_prefill_, &g_step_, &g_step_traced_}) {
        if (*g) xqhip_graph_destroy(*g);
        *g = nullptr;
    }
    traced_ops_.clear();
}

bool DeviceModel::ensure_graphs(std::string* error) {
    if (!graphs_enabled()) return true;  // eager launches of the same kernels
    if (g_prefill_ && g_step_) return true;
    auto capture = [&](void** out, auto&& enqueue) {
        XQ_CALL(xqhip_graph_begin(stream_), "graph capture");
        const bool ok = enqueue();
        void* g = nullptr;
        if (xqhip_graph_end(stream_, &g) != 0 || !ok) return ok ? fail_hip(error, "graph instantiate") : false;
        *out = g;
        return true;
    };
    if (!capture(&g_prefill_, [&] { return enqueue_embed(d_ctrl_ + 1, false, error) && enqueue_layers(false, error); }) ||
        !capture(&g_step_, [&] {
            return enqueue_lm_head(false, error) && enqueue_layers(false, error);
        }))
        return false;
    // the traced step: the same launches with a timestamp kernel after every
    // op (event-record nodes of a graph give no timings here).  XQ_TRACE_EVERY=0
    // leaves it out: the first step after a prefill then runs eagerly with
    // per-op events, and graph steps are only timed as a whole
    if (trace_every_ <= 0) return true;
    ops_.clear();
    event_next_ = 0;
    op_chained_ = false;
    ts_next_ = 0;
    ts_mode_ = true;
    void* g = nullptr;
    std::string ignored;
    bool ok = xqhip_graph_begin(stream_) == 0;
    if (ok) {
        const bool enq = enqueue_lm_head(true, &ignored) && enqueue_layers(true, &ignored);
        ok = xqhip_graph_end(stream_, &g) == 0 && enq;
    }
    ts_mode_ = false;
    for (const TimedOp& op : ops_) ok = ok && op.ts0 >= 0 && op.ts1 >= 0;
    if (ok) {
        g_step_traced_ = g;
        traced_ops_ = std::move(ops_);
    } else {
        if (g) xqhip_graph_destroy(g);
        trace_note_ = "per_op_first_eager_step_after_prefill(traced_graph_unavailable)";
    }
    ops_.clear();
    event_next_ = 0;
    op_chained_ = false;
    return true;
}

// Batched prefill needs every matrix in the TILED64 layout (group 64) and the
// shapes of the chunk kernels; tiny models prefill token by token through the
// decode-step kernels.  XQ_PREFILL_BATCH=0 forces the token-by-token path.
bool DeviceModel::alloc_prefill_buffers(std::string* error) {
    const char* env = std::getenv("XQ_PREFILL_BATCH");
    if (env && env[0] == '0') return true;
    bool ok = hidden_ % 4 == 0 && inter_ % 4 == 0 && attn_n_ % 4 == 0 && max_proj_ % 4 == 0;
    for (const Layer& L : layers_) {
        for (const xqhip_w4* w : {&L.in_proj, &L.out_proj, &L.gate_up, &L.down})
            ok = ok && w->layout != XQHIP_LAYOUT_GENERIC;
        if (!L.full) ok = ok && lk_hd_ <= 256 && lv_n_ % lk_n_ == 0 && ksize_ >= 1 && ksize_ <= 8 && lv_hd_ % 8 == 0;
    }
    ok = ok && (nq_ / nkv_) <= 8;
    if (!ok) return true;
    const size_t c = static_cast<size_t>(chunk_);
    size_t ws_bytes = 0;  // the largest need over the layers' matrices
    for (const Layer& L : layers_)
        for (const xqhip_w4* w : {&L.in_proj, &L.out_proj, &L.gate_up, &L.down})
            ws_bytes = std::max(ws_bytes, xqhip_gemm_workspace_bytes(chunk_, w->cols, w->rows));
    uint8_t* ws = nullptr;
    if (!alloc(&x_all_, c * hidden_, error) || !alloc(&proj_all_, c * max_proj_, error) ||
        !alloc(&q_all_, c * nq_ * hd_, error) || !alloc(&gate_all_, c * nq_ * hd_, error) ||
        !alloc(&attn_all_, c * attn_n_, error) || !alloc(&ffn_all_, c * inter_, error) ||
        !alloc(&ws, ws_bytes, error) || !alloc(&tok_dev_, c, error))
        return false;
    gemm_ws_ = ws;
    gemm_ws_bytes_ = ws_bytes;
    bool any_linear = false;
    for (const Layer& L : layers_) any_linear |= !L.full;
    if (any_linear) {
        uint8_t* sw = nullptr;
        if (!alloc(&sw, xqhip_linear_scan_workspace_bytes(chunk_, lk_n_, lk_hd_, lv_n_, lv_hd_), error)) return false;
        scan_ws_ = sw;
    }
    batched_prefill_ = true;
    return true;
}

// One prompt chunk of n tokens at positions pos0 .. pos0+n-1 through every
// layer; the last token's residual stream ends in resid_.
// h_tokens / h_pos: pinned host copies that stay untouched until the chunk ran.
bool DeviceModel::prefill_chunk(const int32_t* h_tokens, const int32_t* h_pos, int n, int pos0, bool timed,
                                std::string* error) {
    XQ_CALL(xqhip_memcpy_h2d_async(tok_dev_, h_tokens, sizeof(int32_t) * n, stream_), "prompt upload");
    XQ_CALL(xqhip_memcpy_h2d_async(d_ctrl_, h_pos, sizeof(int32_t), stream_), "position upload");
    const int32_t* pos = d_ctrl_;
    op_begin(timed, "prefill_embedding_bf16_rows");
    XQ_CALL(xqhip_embed_bf16_batch(embed_, vocab_, hidden_, tok_dev_, n, x_all_, stream_), "prefill embedding");
    op_end(timed);
    const int qd = nq_ * hd_;
    for (Layer& L : layers_) {
        xqhip_prologue rms_in{XQHIP_PRO_RMS, 0, L.in_norm, nullptr, eps_};
        op_begin(timed, L.full ? "prefill_gemm_w4a16_mfma(q_proj,k_proj,v_proj,rmsnorm_input)"
                               : "prefill_gemm_w4a16_mfma(in_proj_qkv,in_proj_a,in_proj_b,in_proj_z,rmsnorm_input)");
        XQ_CALL(xqhip_gemm_w4a16(&L.in_proj, x_all_, n, hidden_, &rms_in, 0, proj_all_, max_proj_, XQHIP_EPI_STORE,
                                 gemm_ws_, gemm_ws_bytes_, stream_),
                "prefill input projection");
        op_end(timed);
        if (L.full) {
            const float* k_src = proj_all_ + static_cast<size_t>(qd) * (L.q_gated ? 2 : 1);
            const float* v_src = k_src + static_cast<size_t>(nkv_) * hd_;
            op_begin(timed, "prefill_kv_build_custom(fused:q_norm,k_norm,rope,kv_append)");
            XQ_CALL(xqhip_attn_prep_batch(proj_all_, k_src, v_src, L.q_gated ? 1 : 0, nq_, nkv_, hd_, rot_, L.q_norm,
                                          L.k_norm, eps_, rope_cs_, pos, n, max_proj_, qd, q_all_, gate_all_,
                                          L.k_cache, L.v_cache, stream_),
                    "prefill attention prep");
            op_end(timed);
            op_begin(timed, "prefill_attention_gqa_causal_custom(fused:output_gate)");
            XQ_CALL(xqhip_prefill_attention(q_all_, gate_all_, L.k_cache, L.v_cache, nq_, nkv_, hd_, n, qd, pos,
                                            attn_all_, attn_n_, stream_),
                    "prefill attention");
            op_end(timed);
            op_begin(timed, "prefill_gemm_w4a16_mfma(o_proj,residual_add)");
            XQ_CALL(xqhip_gemm_w4a16(&L.out_proj, attn_all_, n, attn_n_, nullptr, 0, x_all_, hidden_, XQHIP_EPI_ADD,
                                     gemm_ws_, gemm_ws_bytes_, stream_),
                    "prefill o projection");
            op_end(timed);
        } else {
            const float* a = proj_all_ + conv_dim_;
            const float* b = a + lv_n_;
            const float* z = b + lv_n_;
            op_begin(timed, "linear_attention_state_update_custom(prefill_scan:conv1d,qk_l2norm,gated_delta)");
            XQ_CALL(xqhip_linear_attn_scan_ws(proj_all_, a, b, max_proj_, L.conv_state, pos0, L.conv_w, L.a_log,
                                              L.dt_bias, L.rec_state, lk_n_, lk_hd_, lv_n_, lv_hd_, ksize_, n,
                                              attn_all_, attn_n_, scan_ws_, stream_),
                    "prefill linear-attention scan");
            op_end(timed);
            xqhip_prologue gated{XQHIP_PRO_GATED_HEAD, lv_hd_, L.lin_norm, z, eps_};
            op_begin(timed, "prefill_gemm_w4a16_mfma(out_proj,gated_rmsnorm,residual_add)");
            XQ_CALL(xqhip_gemm_w4a16(&L.out_proj, attn_all_, n, attn_n_, &gated, max_proj_, x_all_, hidden_,
                                     XQHIP_EPI_ADD, gemm_ws_, gemm_ws_bytes_, stream_),
                    "prefill out projection");
            op_end(timed);
        }
        xqhip_prologue rms_post{XQHIP_PRO_RMS, 0, L.post_norm, nullptr, eps_};
        op_begin(timed, "prefill_gemm_w4a16_mfma(gate_proj,up_proj,rmsnorm_post_attention,silu_gate_mul)");
        XQ_CALL(xqhip_gemm_w4a16(&L.gate_up, x_all_, n, hidden_, &rms_post, 0, ffn_all_, inter_, XQHIP_EPI_SILU_PAIR,
                                 gemm_ws_, gemm_ws_bytes_, stream_),
                "prefill gate/up projection");
        op_end(timed);
        op_begin(timed, "prefill_gemm_w4a16_mfma(down_proj,residual_add)");
        XQ_CALL(xqhip_gemm_w4a16(&L.down, ffn_all_, n, inter_, nullptr, 0, x_all_, hidden_, XQHIP_EPI_ADD, gemm_ws_,
                                 gemm_ws_bytes_, stream_),
                "prefill down projection");
        op_end(timed);
    }
    XQ_CALL(xqhip_copy(resid_, x_all_ + static_cast<size_t>(n - 1) * hidden_, sizeof(float) * hidden_, stream_),
            "last hidden");
    return true;
}

bool DeviceModel::prefill(const int32_t* token_ids, size_t n_tokens, KernelTrace* trace, std::string* error) {
    if (!token_ids || n_tokens == 0) {  // custom_model.cpp:611-614
        *error = "custom prefill requires prompt tokens";
        return false;
    }
    if (!ensure_capacity(n_tokens, error)) return false;
    if (!select_attention(n_tokens, trace, error)) return false;
    for (size_t i = 0; i < n_tokens; ++i) {
        // std::abs(INT_MIN) has no positive value: the reference's row offset
        // turns negative and its read fails (custom_model.cpp:573-597)
        if (token_ids[i] == INT32_MIN) {
            *error = "short embeddings_bf16.bin row read (token id " + std::to_string(token_ids[i]) + " at prompt index " +
                     std::to_string(i) + " has no row)";
            return false;
        }
    }
    if (!sync(trace, error)) return false;
    reset_state();
    if (!ensure_graphs(error)) return false;
    if (h_ctrl_cap_ < 2 * n_tokens) {
        if (h_ctrl_) xqhip_host_free(h_ctrl_);
        h_ctrl_ = nullptr;
        void* p = nullptr;
        XQ_CALL(xqhip_host_alloc(&p, sizeof(int32_t) * 2 * n_tokens), "pinned memory");
        h_ctrl_ = static_cast<int32_t*>(p);
        h_ctrl_cap_ = 2 * n_tokens;
    }
    const size_t op_events = 2 * (6 * layers_.size() + 4);
    while (event_pool_.size() < n_tokens + 1 + op_events) {
        void* e = nullptr;
        XQ_CALL(xqhip_event_create(&e), "event");
        event_pool_.push_back(e);
    }
    // per-token boundary events live at the top of the pool, op events at the bottom
    auto tok_ev = [&](size_t i) { return event_pool_[event_pool_.size() - 1 - i]; };
    if (batched_prefill_ && n_tokens > 1) {
        // chunks of up to chunk_ tokens; every token of a chunk is credited the
        // chunk's time / its size in the prefill_token_custom rows
        const size_t n_chunks = (n_tokens + chunk_ - 1) / chunk_;
        for (size_t i = 0; i < n_tokens; ++i) h_ctrl_[i] = token_ids[i];  // pinned: [tokens][chunk positions]
        xqhip_event_record(tok_ev(0), stream_);
        for (size_t c = 0; c < n_chunks; ++c) {
            const size_t p0 = c * chunk_;
            const int n = static_cast<int>(std::min<size_t>(chunk_, n_tokens - p0));
            h_ctrl_[n_tokens + c] = static_cast<int32_t>(p0);
            if (!prefill_chunk(h_ctrl_ + p0, h_ctrl_ + n_tokens + c, n, static_cast<int>(p0), c == 0 && detail_prefill_,
                               error))
                return false;
            xqhip_event_record(tok_ev(c + 1), stream_);
        }
        XQ_CALL(xqhip_stream_synchronize(stream_), "prefill");
        detail_prefill_ = false;
        if (trace) {
            for (size_t c = 0; c < n_chunks; ++c) {
                const size_t n = std::min<size_t>(chunk_, n_tokens - c * chunk_);
                const double ms = elapsed_ms(tok_ev(c), tok_ev(c + 1));
                for (size_t i = 0; i < n; ++i) trace->add("prefill_token_custom", ms / n, kTraceBackend);
            }
        }
        flush_timed(trace);
        detail_decode_ = true;
        return true;
    }
    xqhip_event_record(tok_ev(0), stream_);
    for (size_t i = 0; i < n_tokens; ++i) {
        h_ctrl_[2 * i] = static_cast<int32_t>(i);
        h_ctrl_[2 * i + 1] = token_ids[i];
        XQ_CALL(xqhip_memcpy_h2d_async(d_ctrl_, h_ctrl_ + 2 * i, 2 * sizeof(int32_t), stream_), "control upload");
        if ((i == 0 && detail_prefill_) || !g_prefill_) {
            const bool timed = i == 0 && detail_prefill_;
            if (!enqueue_embed(d_ctrl_ + 1, timed, error) || !enqueue_layers(timed, error)) return false;
        } else {
            XQ_CALL(xqhip_graph_launch(g_prefill_, stream_), "prefill graph");
        }
        xqhip_event_record(tok_ev(i + 1), stream_);
    }
    XQ_CALL(xqhip_stream_synchronize(stream_), "prefill");
    detail_prefill_ = false;
    if (trace) {
        for (size_t i = 0; i < n_tokens; ++i)
            trace->add("prefill_token_custom", elapsed_ms(tok_ev(i), tok_ev(i + 1)), kTraceBackend);
    }
    flush_timed(trace);
    detail_decode_ = true;
    return true;
}

bool DeviceModel::decode_one(int32_t* token_id, size_t position, KernelTrace* trace, std::string* error) {
    if (!token_id) {
        *error = "decodeOne token output is null";
        return false;
    }
    if (lm_head_.rows <= 0 || lm_head_.cols != hidden_) {  // custom_model.cpp:1282-1285
        *error = "lm_head matrix is not loaded";
        return false;
    }
    if (!ensure_capacity(position + 1, error)) return false;
    if (!select_attention(position + 1, trace, error)) return false;
    if (!ensure_graphs(error)) return false;
    // The sampling kernel adds 1 to d_ctrl_[0] before the forward pass reads
    // it, so the device must hold position - 1: after a step at position - 1
    // it does, otherwise it is uploaded.  The previous step's forward pass may
    // still be running: h_tok_[0..1] are free again because their upload
    // preceded that step's sampling, which the previous call waited for, and
    // so is h_slot_, which only sampling kernels store to.
    const long long want = static_cast<long long>(position);
    const bool upload = dev_pos_ != want - 1;
    dev_pos_ = kPosUnknown;
    *h_slot_ = ~0ull;
    if (upload) {
        h_tok_[0] = static_cast<int32_t>(want - 1);
        h_tok_[1] = 0;
        XQ_CALL(xqhip_memcpy_h2d_async(d_ctrl_, h_tok_, 2 * sizeof(int32_t), stream_), "control upload");
    }
    if (trace) trace_ = trace;
    if (!g_step_ || (detail_decode_ && !g_step_traced_)) {
        // eager launches (graphs off, or no traced graph for the first step
        // after a prefill): per-op events, the whole step waited for
        chained_ = false;
        const bool timed = detail_decode_;
        if (!sync(trace, error)) return false;
        if (!enqueue_lm_head(timed, error) || !enqueue_layers(timed, error)) return false;
        XQ_CALL(xqhip_stream_synchronize(stream_), "decode");
        if (!read_slot(want, token_id, error)) return false;
        dev_pos_ = want;
        detail_decode_ = false;
        flush_timed(trace);
        return true;
    }
    // One graph samples, publishes the token, advances the position and runs
    // the forward pass; the call returns once the token is published.  The
    // step is timed from the previous graph step's end event (or an event of
    // its own when it does not follow one) to its own end event; the traced
    // graph (an event after every op) replaces it on the first step after a
    // prefill and on every trace_every_-th graph step.
    ++graph_steps_;
    const bool traced = g_step_traced_ &&
                        (detail_decode_ || (trace_every_ > 0 && graph_steps_ % static_cast<uint64_t>(trace_every_) == 0));
    if (traced) {
        // every traced step stamps the same host array: a traced step not yet
        // credited is waited for and credited before the next one overwrites it
        bool earlier_traced = false;
        for (const PendingStep& st : pending_) earlier_traced = earlier_traced || st.traced;
        if (earlier_traced) {
            XQ_CALL(xqhip_event_synchronize(pending_.back().end), "step event");
            credit_steps(trace, pending_.size());
        }
    }
    void* start = last_end_;
    if (!chained_ || upload || !start) {
        start = next_step_event();
        XQ_CALL(xqhip_event_record(start, stream_), "step event");
    }
    chained_ = false;
    XQ_CALL(xqhip_graph_launch(traced ? g_step_traced_ : g_step_, stream_), "decode step graph");
    void* end = next_step_event();
    XQ_CALL(xqhip_event_record(end, stream_), "step event");
    pending_.push_back(PendingStep{start, end, traced});
    detail_decode_ = false;
    for (uint32_t spin = 1;; ++spin) {
        if (static_cast<uint32_t>(__atomic_load_n(h_slot_, __ATOMIC_ACQUIRE) >> 32) == static_cast<uint32_t>(want))
            break;
#if defined(__x86_64__) || defined(__i386__)
        __builtin_ia32_pause();  // spin-wait hint: yields the core's pipeline to its sibling thread
#endif
        if ((spin & 1023u) == 0) {  // the stream drained (or failed) without publishing: report it
            const int q = xqhip_stream_query(stream_);
            if (q < 0) return fail_hip(error, "decode step");
            if (q == 1 && static_cast<uint32_t>(__atomic_load_n(h_slot_, __ATOMIC_ACQUIRE) >> 32) !=
                              static_cast<uint32_t>(want)) {
                *error = "decode step ended without publishing the sampled token";
                return false;
            }
        }
    }
    if (!read_slot(want, token_id, error)) return false;
    dev_pos_ = want;
    // this step's sampling ran after every earlier step had finished
    credit_steps(trace, pending_.size() - 1);
    last_end_ = end;
    chained_ = true;
    return true;
}

void* DeviceModel::next_step_event() {
    void* e = step_ev_[step_ev_next_];
    step_ev_next_ = (step_ev_next_ + 1) % kStepEvents;
    return e;
}

// One row per graph step (decode_step_graph_custom; a traced step under
// decode_step_graph_traced_custom, its time including its events), and the
// traced steps' per-op rows.
void DeviceModel::credit_steps(KernelTrace* trace, size_t n) {
    n = std::min(n, pending_.size());
    for (size_t i = 0; i < n && trace; ++i) {
        const PendingStep& st = pending_[i];
        trace->add(st.traced ? "decode_step_graph_traced_custom" : "decode_step_graph_custom",
                   elapsed_ms(st.start, st.end), kTraceBackend);
        if (st.traced) {
            ++traced_steps_;
            for (const TimedOp& op : traced_ops_) {
                // 100 MHz counter: 1e5 ticks per ms
                const double ms = static_cast<double>(static_cast<int64_t>(h_ts_[op.ts1] - h_ts_[op.ts0])) * 1e-5;
                trace->add(op.name, ms, kTraceBackend);
                for (const std::string& e : op.extra_names) trace->add(e, ms / op.split, kTraceBackend);
            }
        }
    }
    if (trace) {
        trace->set_count("decode_graph_steps", static_cast<int64_t>(graph_steps_));
        trace->set_count("decode_op_traced_graph_steps", static_cast<int64_t>(traced_steps_));
        trace->set_count("decode_op_trace_every", trace_every_);
    }
    pending_.erase(pending_.begin(), pending_.begin() + static_cast<std::ptrdiff_t>(n));
}

// The slot the sampling kernel published: (position << 32) | token.
bool DeviceModel::read_slot(long long want, int32_t* token_id, std::string* error) const {
    const uint64_t v = __atomic_load_n(h_slot_, __ATOMIC_ACQUIRE);
    if (static_cast<uint32_t>(v >> 32) != static_cast<uint32_t>(want)) {
        *error = "sampled token published for another position";
        return false;
    }
    *token_id = static_cast<int32_t>(static_cast<uint32_t>(v));
    return true;
}

bool DeviceModel::sync(KernelTrace* trace, std::string* error) {
    chained_ = false;  // whatever the caller enqueues next runs between the steps
    if (!stream_) return true;
    if (trace) trace_ = trace;
    if (xqhip_stream_synchronize(stream_) != 0) return fail_hip(error, "decode step");
    if (chain_sync_) {
        int bad = 0;
        if (xqhip_chain_error(chain_sync_, &bad) != 0) return fail_hip(error, "decode chain status");
        if (bad) {
            *error = "decode chain: a hand-off wait gave up (not every block of the chain launch was resident); "
                     "results since the last check are invalid";
            return false;
        }
    }
    if (fuse_sync_) {
        int bad = 0;
        if (xqhip_step_outproj_error(fuse_sync_, &bad) != 0) return fail_hip(error, "step + projection status");
        if (bad) {
            xqhip_fill_u8(fuse_sync_, 0, xqhip_step_outproj_sync_bytes(), stream_);
            xqhip_stream_synchronize(stream_);
            *error = "linear-attention step + out projection: a hand-off wait gave up; results since the last check "
                     "are invalid";
            return false;
        }
    }
    credit_steps(trace, pending_.size());
    return true;
}

std::string DeviceModel::coverage_summary() const {  // fields of custom_model.cpp:1358-1380
    std::ostringstream o;
    o << "custom_decode_loop;hotpath_replaced=true;full_custom_decode=true;"
      << "backend_request=" << backend_request_ << ";device=hip:" << device_name_ << ";"
      << "linear_backend=hip_gfx950_w4a16_int4_digit_gemv_sdot8;"
      << "linear=q_proj,k_proj,v_proj,o_proj,gate_proj,up_proj,down_proj,linear_attn_qkv_a_b_z_out,lm_head;"
      << "rmsnorm=hip_fused_gemv_prologue;rope=hip_table_libm;attention=hip_gqa_decode_split_fp16_kv;"
      << "attention_output_gate=hip_fused;linear_attention_state=hip_gated_delta_fp32_state;"
      << "linear_attention_qk_norm=hip_fused_conv1d;linear_attention_gated_rmsnorm=hip_fused_gemv_prologue;"
      << "sampling=hip_fused_lm_head_argmax;prefill_kv_build=hip_fp16_append;decode_step=hip_graph;"
      << "weight_bytes_per_token=" << weight_bytes_ << ";fp16_meta_inexact=" << inexact_meta_
      << ";weight_layouts=tiled64:" << layout_count_[XQHIP_LAYOUT_TILED64]
      << ",generic:" << layout_count_[XQHIP_LAYOUT_GENERIC] << ",f32meta:" << layout_count_[XQHIP_LAYOUT_TILED64_F32META]
      << ",scale16:" << layout_count_[XQHIP_LAYOUT_TILED64_SCALE16]
      << ",f32s_z4:" << layout_count_[XQHIP_LAYOUT_TILED64_F32S_Z4]
      << ";kv_capacity=" << max_ctx_ << ";decode_chain=" << chain_note_ << ";linear_step_outproj=" << fuse_note_ << ";kernel_trace=" << trace_note_
      << ";fallback_ops=none";
    return o.str();
}

bool DeviceModel::copy_hidden(float* out_values, size_t value_capacity, size_t* out_size) {
    if (out_size) *out_size = static_cast<size_t>(hidden_);
    if (!out_values || value_capacity < static_cast<size_t>(hidden_)) return false;
    // the queued steps are credited to the trace first: this work runs between them
    std::string err;
    if (!sync(trace_, &err)) return false;
    if (xqhip_rmsnorm(resid_, final_norm_, hidden_, eps_, normed_, stream_) != 0) return false;
    return xqhip_memcpy_d2h(out_values, normed_, sizeof(float) * hidden_, stream_) == 0;
}

std::string DeviceModel::debug_json(int top_k) {  // custom_model.cpp:1382-1436
    const int k = std::max(1, std::min(top_k, 16));
    {
        std::string err;
        sync(trace_, &err);  // (copy_hidden below waits too; the steps are credited first)
    }
    std::vector<float> h(static_cast<size_t>(hidden_), 0.0f);
    size_t n_h = 0;
    copy_hidden(h.data(), h.size(), &n_h);
    double sum = 0.0, sum_sq = 0.0;
    float mn = h.empty() ? 0.0f : h[0], mx = mn;
    int nonfinite = 0;
    for (float v : h) {
        if (!std::isfinite(v)) {
            ++nonfinite;
            continue;
        }
        sum += v;
        sum_sq += static_cast<double>(v) * v;
        mn = std::min(mn, v);
        mx = std::max(mx, v);
    }
    const double n = static_cast<double>(h.size());
    const double mean = n > 0 ? sum / n : 0.0;
    const double var = n > 0 ? std::max(0.0, sum_sq / n - mean * mean) : 0.0;
    std::vector<float> logits(static_cast<size_t>(std::max(0, lm_head_.rows)), 0.0f);
    if (lm_head_.rows > 0 && lm_head_.cols == hidden_) {
        std::string err;
        if (!logits_) alloc(&logits_, lm_head_.rows, &err);
        if (logits_ &&
            xqhip_gemv_w4a16(&lm_head_, normed_, XQHIP_F32, nullptr, logits_, XQHIP_F32, XQHIP_EPI_STORE, stream_) == 0)
            xqhip_memcpy_d2h(logits.data(), logits_, sizeof(float) * logits.size(), stream_);
    }
    std::vector<int> best;
    for (int i = 0; i < static_cast<int>(logits.size()); ++i) {
        size_t at = 0;
        while (at < best.size() && logits[best[at]] >= logits[i]) ++at;
        if (at < static_cast<size_t>(k)) {
            best.insert(best.begin() + static_cast<std::ptrdiff_t>(at), i);
            if (best.size() > static_cast<size_t>(k)) best.pop_back();
        }
    }
    std::ostringstream o;
    o << "{\"hidden\":{\"size\":" << h.size() << ",\"mean\":" << mean << ",\"std\":" << std::sqrt(var)
      << ",\"min\":" << mn << ",\"max\":" << mx << ",\"l2\":" << std::sqrt(sum_sq) << ",\"nonfinite\":" << nonfinite
      << "},\"lm_head_topk\":[";
    for (size_t i = 0; i < best.size(); ++i)
        o << (i ? "," : "") << "{\"token\":" << best[i] << ",\"logit\":" << logits[best[i]] << "}";
    o << "]}";
    return o.str();
}

}  // namespace xqh
