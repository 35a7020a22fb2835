// xq_host_quality_runner - greedy generation over the fixed token-id prompt set,
// one JSON report on stdout (the quality_validation artifact, schema 1).
//
// Command line and report of customlib/tools/xq_host_quality_runner.cpp:200-402:
//   xq_host_quality_runner <model_dir> [max_new_tokens=32] [threads=8] [prompt_id] [prefill_debug]
// exit 0 = every prompt passed the gate, 3 = some prompt failed it, 2 = usage /
// unknown prompt id, 1 = xq_create failed.  With "prefill_debug" each prompt is
// run as xq_prefill + xq_decode_one steps and the xq_get_debug_json snapshot
// after the prefill and before every later step is embedded in the report.
//
// The requested backend is "cpu" (the reference runner's request) unless the
// XQ_BACKEND environment variable names another; the backend reported as
// actual is the one the kernel-trace rows ran on.
#include <cstdlib>
#include <iostream>

#include "harness.hpp"

using namespace xqtool;

namespace {

struct PromptResult {
    xq_status status = XQ_OK;
    std::vector<int32_t> ids;
    xq_metrics m{};
    std::string prefill_debug = "{}";
    std::vector<std::string> step_debug;
};

PromptResult run_prompt(xq_session* s, const PromptCase& p, int max_new, bool debug) {
    PromptResult r;
    r.m.struct_size = sizeof(r.m);
    r.ids.assign(static_cast<size_t>(max_new), 0);
    xq_reset(s);
    if (!debug) {
        r.status = xq_generate(s, p.ids.data(), p.ids.size(), r.ids.size(), r.ids.data(), r.ids.size(), &r.m);
    } else {
        r.status = xq_prefill(s, p.ids.data(), p.ids.size(), &r.m);
        if (r.status != XQ_OK) {
            r.ids.clear();
        } else {
            r.prefill_debug = session_json(xq_get_debug_json, s, "{}");
            r.step_debug.push_back(r.prefill_debug);
            for (size_t t = 0; t < r.ids.size(); ++t) {
                if (t > 0) r.step_debug.push_back(session_json(xq_get_debug_json, s, "{}"));
                xq_metrics sm{};
                sm.struct_size = sizeof(sm);
                r.status = xq_decode_one(s, &r.ids[t], &sm);
                r.m = sm;
                if (r.status != XQ_OK) {
                    r.ids.resize(t);
                    break;
                }
            }
        }
    }
    r.ids.resize(std::min<size_t>(r.ids.size(), r.m.generated_tokens));
    return r;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 2) {
        std::cerr << "usage: " << argv[0] << " <model_dir> [max_new_tokens] [threads] [prompt_id]\n";
        return 2;
    }
    const std::string model_dir = argv[1];
    const int max_new = argc > 2 ? std::max(1, std::atoi(argv[2])) : 32;
    const int threads = argc > 3 ? std::max(1, std::atoi(argv[3])) : 8;
    const std::string only = argc > 4 ? argv[4] : "";
    const bool debug = argc > 5 && std::string(argv[5]) == "prefill_debug";
    const char* env_backend = std::getenv("XQ_BACKEND");
    const std::string requested = env_backend && *env_backend ? env_backend : "cpu";

    const xq_options opt = harness_options(requested.c_str(), threads);
    xq_session* s = nullptr;
    const xq_status cs = xq_create(model_dir.c_str(), &opt, &s);
    if (cs != XQ_OK || !s) {
        std::cout << "{\"schema_version\":1,\"artifact_type\":\"quality_validation\",\"engine\":\"customlib\","
                  << "\"status\":\"error\",\"quality_gate_passed\":false,\"error\":\"xq_create failed\","
                  << "\"status_code\":" << cs << "}\n";
        return 1;
    }
    xq_metrics initial{};
    initial.struct_size = sizeof(initial);
    xq_get_last_metrics(s, &initial);

    std::vector<PromptCase> cases;
    for (const PromptCase& p : validation_prompts())
        if (only.empty() || only == p.id) cases.push_back(p);
    if (cases.empty()) {
        std::cerr << "unknown prompt_id: " << only << "\n";
        xq_destroy(s);
        return 2;
    }

    bool all_ok = true;
    std::ostringstream pj;
    pj << '[';
    for (size_t i = 0; i < cases.size(); ++i) {
        const PromptCase& p = cases[i];
        const PromptResult r = run_prompt(s, p, max_new, debug);
        const SeqStats st = sequence_stats(r.ids);
        const bool ok = r.status == XQ_OK && st.invalid == 0 && !st.empty && !st.degenerate;
        all_ok = all_ok && ok;
        pj << (i ? "," : "") << "{\"id\":\"" << esc(p.id) << "\",\"prompt_kind\":\"" << esc(p.kind)
           << "\",\"prompt_text_hint\":\"" << esc(p.hint) << "\",\"raw_text_prompt_available\":false,"
           << "\"prompt_token_count\":" << p.ids.size() << ",\"prompt_token_ids\":";
        put_ids(pj, p.ids);
        pj << ",\"generated_token_count\":" << r.ids.size() << ",\"generated_token_ids\":";
        put_ids(pj, r.ids);
        pj << ",\"decoded_text_available\":false,\"decoded_generated_text\":\"\",\"status_code\":" << r.status
           << ",\"status\":\"" << (ok ? "ok" : "error") << "\",\"invalid_token_count\":" << st.invalid
           << ",\"empty_output\":" << tf(st.empty) << ",\"longest_repeated_run\":" << st.longest_run
           << ",\"longest_repeated_run_token\":" << st.longest_run_token << ",\"most_repeated_token\":" << st.most_token
           << ",\"most_repeated_token_count\":" << st.most_count
           << ",\"repeated_token_220_longest_run\":" << st.space_run
           << ",\"repeated_token_220_failure\":" << tf(st.space_run >= 8) << ",\"unique_token_count\":" << st.unique
           << ",\"obvious_degenerate_output\":" << tf(st.degenerate) << ",\"prefill_ms\":" << r.m.prefill_ms
           << ",\"decode_total_ms\":" << r.m.decode_total_ms << ",\"prefill_debug\":" << r.prefill_debug
           << ",\"decode_step_debug\":[";
        for (size_t d = 0; d < r.step_debug.size(); ++d) pj << (d ? "," : "") << r.step_debug[d];
        pj << "]}";
    }
    pj << ']';
    const std::string trace = session_json(xq_get_kernel_trace_json, s, "{\"rows\":[]}");
    xq_destroy(s);
    const std::string actual = trace_backend_all(trace, requested);

    std::cout << "{\"schema_version\":1,\"artifact_type\":\"quality_validation\",\"engine\":\"customlib\","
              << "\"status\":\"" << (all_ok ? "ok" : "error") << "\",\"quality_gate_passed\":" << tf(all_ok)
              << ",\"model\":{\"hf_repo\":\"Qwen/Qwen3.5-9B\",\"hf_revision\":\"c202236235762e1c871ad0ccb60c8ee5ba337b9a\","
              << "\"format\":\"xqwen35_custom_w4a16\",\"vocab_size_assumed\":" << kQwen35Vocab << "},"
              << "\"artifact\":{\"model_dir\":\"" << esc(model_dir) << "\"},\"runtime\":{\"threads\":" << threads
              << ",\"selected_kernels\":{\"summary\":\"" << esc(initial.selected_kernels)
              << "\",\"hotpath_replaced\":true,\"full_custom_decode\":true,\"replaced_op_families\":[\"q_proj\","
              << "\"k_proj\",\"v_proj\",\"o_proj\",\"gate_proj\",\"up_proj\",\"down_proj\",\"rmsnorm\",\"rope\","
              << "\"attention\",\"linear_attention_state\",\"lm_head\",\"sampling\",\"prefill_kv_build\"],"
              << "\"fallback_op_families\":[]}},\"custom_path\":{\"calls_mnn_llm_response_for_measured_generation\":false,"
              << "\"use_mnn_fallback\":0,\"full_custom_decode\":true,\"fallback_op_families\":[]},"
              << "\"custom_backend_requested\":\"" << esc(requested) << "\",\"custom_backend_actual\":\"" << esc(actual)
              << "\",\"validation\":{\"prompt_set\":\"small_english_tokenizer_ids\",\"validation_compare_to_stock\":true,"
              << "\"tokenizer_decode_available\":false,\"validation_dump_tokens\":true,\"validation_dump_text\":false,"
              << "\"validation_dump_intermediate\":" << tf(debug) << ",\"max_new_tokens\":" << max_new
              << ",\"temperature\":0,\"top_k\":1,\"top_p\":1},\"prompts\":" << pj.str()
              << ",\"per_kernel_wall_clock\":" << trace << "}\n";
    return all_ok ? 0 : 3;
}
