// session.cpp - the xqwen35.h C ABI over a device-resident model.
//
// Behaviour follows customlib/runtime/session.{hpp,cpp}: options normalisation
// (session.cpp:154-180), metrics publication honouring struct_size (:182-191),
// the prefill / decode / generate / reset state machine (:304-525), the JSON
// getters that copy whole or return XQ_ERR_BUFFER_TOO_SMALL (:532-585) and the
// extern "C" shims (:618-712).  A NULL options pointer selects the reference's
// model-less fallback session, which emits (last + 1 + position) % vocab.
#include <algorithm>
#include <chrono>
#include <cstring>
#include <memory>
#include <sstream>
#include <string>
#include <vector>

#include "device_model.hpp"
#include "kernel_trace.hpp"
#include "model_files.hpp"
#include "xqwen35.h"

namespace xqh {
namespace {

using Clock = std::chrono::steady_clock;

double ms_between(Clock::time_point a, Clock::time_point b) {
    return std::chrono::duration<double, std::milli>(b - a).count();
}

void copy_cstr(char* dst, size_t cap, const std::string& src) {
    if (cap == 0) return;
    const size_t n = std::min(cap - 1, src.size());
    std::memcpy(dst, src.data(), n);
    dst[n] = '\0';
}

xq_status copy_json(const std::string& json, char* out, size_t cap) {
    if (!out || cap == 0) return XQ_ERR_INVALID_ARGUMENT;
    if (json.size() + 1 > cap) return XQ_ERR_BUFFER_TOO_SMALL;
    std::memcpy(out, json.c_str(), json.size() + 1);
    return XQ_OK;
}

struct Options {  // session.hpp:36-45 defaults
    std::string backend = "cpu";
    int threads = 4;
    int quant_bits = 4;
    int group_size = 64;
    int max_context_tokens = 8192;
    bool enable_autotune = true;
    bool use_mnn_fallback = true;
    std::string telemetry_path;
};

Options normalize(const xq_options* o) {
    Options out;
    if (!o) return out;
    if (o->backend && o->backend[0] != '\0') out.backend = o->backend;
    if (o->threads > 0) out.threads = o->threads;
    if (o->quant_bits == 2 || o->quant_bits == 3 || o->quant_bits == 4) out.quant_bits = o->quant_bits;
    if (o->group_size > 0) out.group_size = o->group_size;
    if (o->max_context_tokens > 0) out.max_context_tokens = o->max_context_tokens;
    out.enable_autotune = o->enable_autotune != 0;
    out.use_mnn_fallback = o->use_mnn_fallback != 0;
    if (o->telemetry_path) out.telemetry_path = o->telemetry_path;
    return out;
}

void publish(const xq_metrics& src, xq_metrics* dst) {
    if (!dst) return;
    const size_t want = dst->struct_size ? dst->struct_size : sizeof(xq_metrics);
    const size_t n = std::min(want, sizeof(xq_metrics));
    std::memset(dst, 0, n);
    std::memcpy(dst, &src, n);
    dst->struct_size = sizeof(xq_metrics);
}

class Session {
public:
    Session(std::string dir, Options opt) : dir_(std::move(dir)), opt_(std::move(opt)) {
        m_.struct_size = sizeof(xq_metrics);
        copy_cstr(m_.backend, sizeof(m_.backend), opt_.backend);
        copy_cstr(m_.selected_kernels, sizeof(m_.selected_kernels), kernel_summary());
    }

    xq_status load() {
        const auto t0 = Clock::now();
        const std::string js = read_text(dir_ + "/xqwen35_manifest.json");
        if (!js.empty()) {
            hf_repo_ = manifest_string(js, "hf_repo", hf_repo_);
            hf_revision_ = manifest_string(js, "hf_revision", hf_revision_);
            vocab_ = manifest_int(js, "vocab_size", vocab_);
        }
        if (!opt_.use_mnn_fallback) {
            model_ = std::make_unique<DeviceModel>();
            std::string err;
            if (!model_->load(dir_, opt_.backend, opt_.max_context_tokens, &err)) {
                model_.reset();
                set_error(err);
                return XQ_ERR_MODEL;
            }
            loaded_ = true;
            m_.load_ms = ms_between(t0, Clock::now());
            copy_cstr(m_.backend, sizeof(m_.backend), "xq_custom_decode_hip_gfx950");
            copy_cstr(m_.selected_kernels, sizeof(m_.selected_kernels), kernel_summary());
            set_error("");
            return XQ_OK;
        }
        loaded_ = true;  // model-less fallback session (session.cpp:297-301)
        m_.load_ms = ms_between(t0, Clock::now());
        set_error("");
        return XQ_OK;
    }

    xq_status prefill(const int32_t* toks, size_t n, xq_metrics* out) {
        if (!loaded_) return fail(XQ_ERR_NOT_READY, "session is not loaded", out);
        if (!toks || n == 0) return fail(XQ_ERR_INVALID_ARGUMENT, "prefill requires at least one token", out);
        const auto t0 = Clock::now();
        last_token_ = toks[n - 1];
        position_ = n;
        if (model_) {
            std::string err;
            if (!model_->prefill(toks, n, &trace_, &err)) return fail(XQ_ERR_MODEL, err, out);
        }
        has_prefill_ = true;
        m_.prompt_tokens = n;
        m_.generated_tokens = 0;
        m_.prefill_ms = ms_between(t0, Clock::now());
        m_.first_token_ms = 0.0;
        m_.decode_total_ms = 0.0;
        m_.total_generate_ms = m_.prefill_ms;
        rates();
        copy_cstr(m_.selected_kernels, sizeof(m_.selected_kernels), kernel_summary());
        set_error("");
        publish(m_, out);
        return XQ_OK;
    }

    xq_status decode_one(int32_t* out_tok, xq_metrics* out) {
        if (!loaded_ || !has_prefill_)
            return fail(XQ_ERR_NOT_READY, "decode requires a loaded session and completed prefill", out);
        if (!out_tok) return fail(XQ_ERR_INVALID_ARGUMENT, "decode output pointer is null", out);
        const auto t0 = Clock::now();
        if (model_) {
            std::string err;
            if (!model_->decode_one(&last_token_, position_, &trace_, &err)) return fail(XQ_ERR_RUNTIME, err, out);
        } else {
            last_token_ = static_cast<int32_t>((static_cast<int64_t>(last_token_) + 1 + static_cast<int64_t>(position_)) %
                                               std::max(2, vocab_));
        }
        ++position_;
        *out_tok = last_token_;
        const double ms = ms_between(t0, Clock::now());
        if (m_.generated_tokens == 0) m_.first_token_ms = ms;
        m_.generated_tokens += 1;
        m_.decode_total_ms += ms;
        m_.total_generate_ms = m_.prefill_ms + m_.decode_total_ms;
        rates();
        copy_cstr(m_.selected_kernels, sizeof(m_.selected_kernels), kernel_summary());
        set_error("");
        publish(m_, out);
        return XQ_OK;
    }

    xq_status generate(const int32_t* toks, size_t n, size_t max_new, int32_t* buf, size_t cap, xq_metrics* out) {
        if (!buf || cap < max_new) return fail(XQ_ERR_BUFFER_TOO_SMALL, "output buffer is too small", out);
        const auto t0 = Clock::now();
        xq_status st = prefill(toks, n, nullptr);
        if (st != XQ_OK) {
            publish(m_, out);
            return st;
        }
        for (size_t i = 0; i < max_new; ++i) {
            st = decode_one(&buf[i], nullptr);
            if (st != XQ_OK) {
                publish(m_, out);
                return st;
            }
        }
        if (model_ && max_new > 0) {
            // the last token's forward pass is still on the device: wait for it
            // and count it as decode time, so the rates cover all the work
            const auto t1 = Clock::now();
            std::string err;
            if (!model_->sync(&trace_, &err)) return fail(XQ_ERR_RUNTIME, err, out);
            m_.decode_total_ms += ms_between(t1, Clock::now());
        }
        m_.total_generate_ms = ms_between(t0, Clock::now());
        rates();
        copy_cstr(m_.selected_kernels, sizeof(m_.selected_kernels), kernel_summary());
        publish(m_, out);
        return XQ_OK;
    }

    xq_status reset() {
        has_prefill_ = false;
        last_token_ = 0;
        position_ = 0;
        m_ = xq_metrics{};
        m_.struct_size = sizeof(xq_metrics);
        trace_.reset();
        if (model_) model_->reset_state();
        copy_cstr(m_.backend, sizeof(m_.backend), opt_.backend);
        copy_cstr(m_.selected_kernels, sizeof(m_.selected_kernels), kernel_summary());
        return XQ_OK;
    }

    xq_status last_metrics(xq_metrics* out) const {
        publish(m_, out);
        return XQ_OK;
    }

    xq_status backend_info(char* out, size_t cap) const {
        if (!out || cap == 0) return XQ_ERR_INVALID_ARGUMENT;
        std::ostringstream o;
        o << "{\"backend\":\"" << json_escape(opt_.backend) << "\",\"mnn_substrate\":\"not_used\",\"mnn_commit\":\"\","
          << "\"hf_repo\":\"" << json_escape(hf_repo_) << "\",\"hf_revision\":\"" << json_escape(hf_revision_) << "\","
          << "\"quant_bits\":" << opt_.quant_bits << ",\"group_size\":" << opt_.group_size << ","
          << "\"threads\":" << opt_.threads << ",\"device\":\"" << json_escape(model_ ? model_->device_name() : "")
          << "\",\"selected_kernels\":\"" << json_escape(kernel_summary()) << "\"}";
        return copy_json(o.str(), out, cap);
    }

    xq_status trace_json(char* out, size_t cap) {
        if (model_) {
            std::string err;
            if (!model_->sync(&trace_, &err)) return fail(XQ_ERR_RUNTIME, err, nullptr);
        }
        return copy_json(trace_.to_json(), out, cap);
    }

    xq_status debug_json(char* out, size_t cap) {
        if (!out || cap == 0) return XQ_ERR_INVALID_ARGUMENT;
        return copy_json(model_ ? model_->debug_json(10) : std::string("{\"debug\":\"unavailable\"}"), out, cap);
    }

    xq_status hidden(float* out, size_t cap, size_t* out_size) {
        if (!model_) return XQ_ERR_NOT_READY;
        return model_->copy_hidden(out, cap, out_size) ? XQ_OK : XQ_ERR_BUFFER_TOO_SMALL;
    }

private:
    std::string kernel_summary() const {
        if (model_) return model_->coverage_summary();
        std::ostringstream o;  // shape of kernels::selectKernelSummary (generated_dispatch.cpp:24-39)
        o << "linear=w" << opt_.quant_bits << "a16_" << (opt_.quant_bits == 4 ? "hip_gfx950_dequant_gemv" : "unsupported")
          << ";rmsnorm=hip_fused;rope=hip_table;attention=hip_gqa_decode;delta=hip_gated_delta";
        return o.str();
    }

    void set_error(const std::string& msg) { copy_cstr(m_.error, sizeof(m_.error), msg); }

    xq_status fail(xq_status st, const std::string& msg, xq_metrics* out) {
        set_error(msg);
        publish(m_, out);
        return st;
    }

    void rates() {  // session.cpp:595-602
        m_.prefill_tokens_per_second = m_.prefill_ms > 0.0 ? m_.prompt_tokens * 1000.0 / m_.prefill_ms : 0.0;
        m_.decode_tokens_per_second = m_.decode_total_ms > 0.0 ? m_.generated_tokens * 1000.0 / m_.decode_total_ms : 0.0;
    }

    std::string dir_;
    Options opt_;
    xq_metrics m_{};
    bool loaded_ = false, has_prefill_ = false;
    int32_t last_token_ = 0;
    size_t position_ = 0;
    int vocab_ = 248320;
    std::string hf_repo_ = "Qwen/Qwen3.5-9B";
    std::string hf_revision_ = "c202236235762e1c871ad0ccb60c8ee5ba337b9a";
    std::unique_ptr<DeviceModel> model_;
    KernelTrace trace_;
};

Session* S(xq_session* s) { return reinterpret_cast<Session*>(s); }

}  // namespace
}  // namespace xqh

extern "C" {

XQ_API xq_status xq_create(const char* model_dir, const xq_options* options, xq_session** out_session) {
    if (!model_dir || !out_session) return XQ_ERR_INVALID_ARGUMENT;
    *out_session = nullptr;
    std::unique_ptr<xqh::Session> s(new xqh::Session(model_dir, xqh::normalize(options)));
    const xq_status st = s->load();
    if (st != XQ_OK) return st;
    *out_session = reinterpret_cast<xq_session*>(s.release());
    return XQ_OK;
}

XQ_API void xq_destroy(xq_session* session) { delete xqh::S(session); }

XQ_API xq_status xq_prefill(xq_session* s, const int32_t* token_ids, size_t n_tokens, xq_metrics* out_metrics) {
    return s ? xqh::S(s)->prefill(token_ids, n_tokens, out_metrics) : XQ_ERR_INVALID_ARGUMENT;
}

XQ_API xq_status xq_decode_one(xq_session* s, int32_t* out_token_id, xq_metrics* out_metrics) {
    return s ? xqh::S(s)->decode_one(out_token_id, out_metrics) : XQ_ERR_INVALID_ARGUMENT;
}

XQ_API xq_status xq_generate(xq_session* s, const int32_t* token_ids, size_t n_tokens, size_t max_new_tokens,
                             int32_t* output_buffer, size_t output_capacity, xq_metrics* out_metrics) {
    return s ? xqh::S(s)->generate(token_ids, n_tokens, max_new_tokens, output_buffer, output_capacity, out_metrics)
             : XQ_ERR_INVALID_ARGUMENT;
}

XQ_API xq_status xq_reset(xq_session* s) { return s ? xqh::S(s)->reset() : XQ_ERR_INVALID_ARGUMENT; }

XQ_API xq_status xq_get_last_metrics(xq_session* s, xq_metrics* out_metrics) {
    return s ? xqh::S(s)->last_metrics(out_metrics) : XQ_ERR_INVALID_ARGUMENT;
}

XQ_API xq_status xq_get_backend_info(xq_session* s, char* json_out, size_t json_capacity) {
    return s ? xqh::S(s)->backend_info(json_out, json_capacity) : XQ_ERR_INVALID_ARGUMENT;
}

XQ_API xq_status xq_get_kernel_trace_json(xq_session* s, char* json_out, size_t json_capacity) {
    if (!s) return XQ_ERR_INVALID_ARGUMENT;
    if (!json_out || json_capacity == 0) return XQ_ERR_INVALID_ARGUMENT;
    return xqh::S(s)->trace_json(json_out, json_capacity);
}

XQ_API xq_status xq_get_debug_json(xq_session* s, char* json_out, size_t json_capacity) {
    return s ? xqh::S(s)->debug_json(json_out, json_capacity) : XQ_ERR_INVALID_ARGUMENT;
}

XQ_API xq_status xq_get_hidden_state(xq_session* s, float* out_values, size_t value_capacity, size_t* out_size) {
    if (!s || !out_size) return XQ_ERR_INVALID_ARGUMENT;
    return xqh::S(s)->hidden(out_values, value_capacity, out_size);
}

}  // extern "C"
