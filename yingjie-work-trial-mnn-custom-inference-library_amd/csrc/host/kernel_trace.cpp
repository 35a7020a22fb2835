// kernel_trace.cpp - see kernel_trace.hpp.
#include "kernel_trace.hpp"

#include <algorithm>
#include <sstream>
#include <utility>
#include <vector>

namespace xqh {

void KernelTrace::add(const std::string& name, double ms, const std::string& backend) {
    TraceStat& s = rows_[name];
    if (s.calls == 0) {
        s.min_ms = s.max_ms = ms;
        s.backend = backend;
    } else {
        s.min_ms = std::min(s.min_ms, ms);
        s.max_ms = std::max(s.max_ms, ms);
        if (s.backend != backend) s.backend = "mixed";
    }
    s.calls += 1;
    s.total_ms += ms;
}

std::string json_escape(const std::string& s) {
    std::string o;
    o.reserve(s.size() + 8);
    for (char c : s) {
        switch (c) {
            case '\\': o += "\\\\"; break;
            case '"': o += "\\\""; break;
            case '\n': o += "\\n"; break;
            case '\r': o += "\\r"; break;
            case '\t': o += "\\t"; break;
            default: o += c;
        }
    }
    return o;
}

std::string op_family(const std::string& n) {
    // first matching substring wins, in the reference's order
    static const std::vector<std::pair<std::vector<const char*>, const char*>> table = {
        {{"linear_q_proj"}, "q_proj"},
        {{"linear_k_proj"}, "k_proj"},
        {{"linear_v_proj"}, "v_proj"},
        {{"linear_o_proj"}, "o_proj"},
        {{"linear_gate_proj"}, "gate_proj"},
        {{"linear_up_proj"}, "up_proj"},
        {{"linear_down_proj"}, "down_proj"},
        {{"linear_attn"}, "linear_attention_projection"},
        {{"linear_attention_state", "linear_attention_conv", "linear_attention_qk", "linear_attention_gated"},
         "linear_attention_state"},
        {{"rmsnorm"}, "rmsnorm"},
        {{"rope"}, "rope"},
        {{"attention_score"}, "attention_score"},
        {{"attention_softmax"}, "attention_softmax"},
        {{"attention_v_reduce"}, "attention_v_reduce"},
        {{"attention"}, "attention"},
        {{"lm_head"}, "lm_head"},
        {{"sampling"}, "sampling"},
        {{"prefill_kv_build", "kv_append", "kv_cache", "embedding_load"}, "prefill_kv_build"},
        {{"silu"}, "activation"},
    };
    for (const auto& row : table)
        for (const char* key : row.first)
            if (n.find(key) != std::string::npos) return row.second;
    return "other";
}

std::string KernelTrace::to_json() const {
    std::ostringstream o;
    o << "{\"rows\":[";
    bool first = true;
    for (const auto& kv : rows_) {
        const TraceStat& s = kv.second;
        o << (first ? "" : ",") << "{\"name\":\"" << json_escape(kv.first) << "\",\"op_family\":\""
          << op_family(kv.first) << "\",\"backend\":\"" << json_escape(s.backend) << "\",\"calls\":" << s.calls
          << ",\"total_ms\":" << s.total_ms << ",\"mean_ms\":" << (s.calls ? s.total_ms / s.calls : 0.0)
          << ",\"min_ms\":" << s.min_ms << ",\"max_ms\":" << s.max_ms << "}";
        first = false;
    }
    o << "]";
    for (const auto& kv : counts_) o << ",\"" << json_escape(kv.first) << "\":" << kv.second;
    o << "}";
    return o.str();
}

}  // namespace xqh
