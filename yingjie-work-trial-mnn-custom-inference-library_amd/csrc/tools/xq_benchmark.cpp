// xq_benchmark - the benchmark harness as a host program: the three entry points
// the reference's Android benchmark exposes through JNI, and the acceptance checks
// its instrumentation test applies to their JSON.
//
//   benchmark (default)   android/benchmark_app/src/main/cpp/benchmark_jni.cpp:1271-1396
//                         (runBenchmark: warmup + measured xq_generate runs of a
//                         prompt of token 16, per-run metrics, run statistics, the
//                         kernel trace, a kernel microbench); JSON of makeJson
//                         (:957-1098, schema 4)
//   --run-quality-validation   runCustomQualityValidationJson (:1128-1268)
//   --run-vulkan-selftest      runVulkanSelfTest (:1425-1437)
//   checks                BenchmarkInstrumentationTest.java:17-137
//
//   xq_benchmark [--prompt-tokens 512] [--max-new-tokens 256] [--warmup-iterations 1]
//                [--measured-iterations 5] [--validation-max-new-tokens 32]
//                [--custom-backend cpu] [--run-quality-validation] [--run-vulkan-selftest]
//                [--no-microbench] [--artifact-dir DIR] <model_dir>
//
// The JSON goes to stdout (and to DIR/bench_artifacts/ under the instrumentation
// test's file names); progress lines to stderr.  Exit 0 when every check passes.
//
// The kernel microbench runs this library's HIP kernels (include/xqhip.h) on the
// reference microbench's deterministic inputs and shapes (:177-196, :495-646), timed
// with HIP events per call, and reports each row's checksum beside the published one.
#include <cctype>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <functional>
#include <iostream>
#include <stdexcept>
#include <sys/stat.h>

#include "harness.hpp"
#include "xqhip.h"

using namespace xqtool;

namespace {

constexpr int32_t kPromptToken = 16;
constexpr int kThreads = 8;
constexpr int kKernelWarmup = 1;
constexpr int kKernelMeasured = 3;

struct Args {
    std::string model_dir, backend = "cpu", artifact_dir;
    int prompt_tokens = 512, max_new = 256, warmup = 1, measured = 5, validation_max_new = 32;
    bool quality = false, selftest = false, microbench = true;
};

std::string lower(std::string s) {
    for (char& c : s) c = static_cast<char>(std::tolower(static_cast<unsigned char>(c)));
    return s;
}

// The instrumentation test's backend names, plus "hip".
std::string sanitize_backend(const std::string& v) {
    const std::string n = lower(v);
    return (n == "cpu" || n == "vulkan" || n == "cpu_vulkan_hybrid" || n == "hip") ? n : "cpu";
}

// ---- kernel microbench ---------------------------------------------------------

// Inputs of the reference microbench: an LCG index hash mapped to [-scale, scale).
float det_value(size_t i, float scale) {
    uint32_t x = static_cast<uint32_t>(i) * 1664525u + 1013904223u;
    x ^= x >> 16;
    return (static_cast<float>(x & 0xffffu) / 32768.0f - 1.0f) * scale;
}
std::vector<float> det_vector(size_t n, float scale) {
    std::vector<float> v(n);
    for (size_t i = 0; i < n; ++i) v[i] = det_value(i, scale);
    return v;
}
// Float sum of about 257 evenly strided samples.
float sampled_sum(const std::vector<float>& v) {
    const size_t stride = std::max<size_t>(1, v.size() / 257);
    float s = 0.0f;
    for (size_t i = 0; i < v.size(); i += stride) s += v[i];
    return s;
}

uint16_t f32_to_f16(float f) {  // round to nearest even; finite inputs of modest range
    uint32_t u;
    std::memcpy(&u, &f, 4);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const int32_t exp = static_cast<int32_t>((u >> 23) & 0xff) - 127 + 15;
    uint32_t man = u & 0x7fffffu;
    if (exp >= 31) return static_cast<uint16_t>(sign | 0x7c00u);
    if (exp <= 0) {  // subnormal half
        if (exp < -10) return static_cast<uint16_t>(sign);
        man |= 0x800000u;
        const int shift = 14 - exp;
        uint32_t h = man >> shift;
        const uint32_t rem = man & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1))) ++h;
        return static_cast<uint16_t>(sign | h);
    }
    uint32_t h = (static_cast<uint32_t>(exp) << 10) | (man >> 13);
    const uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) ++h;
    return static_cast<uint16_t>(sign | h);
}
float f16_to_f32(uint16_t h) {
    const uint32_t sign = (h & 0x8000u) << 16, e = (h >> 10) & 31, m = h & 1023u;
    float v;
    if (e == 0) {
        v = std::ldexp(static_cast<float>(m), -24);
    } else if (e == 31) {
        v = m ? NAN : INFINITY;
    } else {
        v = std::ldexp(static_cast<float>(m | 1024u), static_cast<int>(e) - 25);
    }
    return sign ? -v : v;
}

// Min/max 4-bit group quantisation, zero point rounded (kernels/reference/ref_gemv.cpp:38-75).
void quantize_w4(const std::vector<float>& w, int rows, int cols, int group, std::vector<uint8_t>* packed,
                 std::vector<float>* scales, std::vector<float>* zeros) {
    const int gpr = (cols + group - 1) / group;
    packed->assign((static_cast<size_t>(rows) * cols + 1) / 2, 0);
    scales->assign(static_cast<size_t>(rows) * gpr, 1.0f);
    zeros->assign(static_cast<size_t>(rows) * gpr, 0.0f);
    for (int r = 0; r < rows; ++r) {
        const float* row = w.data() + static_cast<size_t>(r) * cols;
        for (int g = 0; g < gpr; ++g) {
            const int c0 = g * group, c1 = std::min(cols, c0 + group);
            const auto mm = std::minmax_element(row + c0, row + c1);
            const float lo = *mm.first, hi = *mm.second;
            const float s = hi > lo ? (hi - lo) / 15.0f : 1.0f;
            const float z = hi > lo ? std::round(-lo / s) : 0.0f;
            (*scales)[static_cast<size_t>(r) * gpr + g] = s;
            (*zeros)[static_cast<size_t>(r) * gpr + g] = z;
            for (int c = c0; c < c1; ++c) {
                const int q = std::max(0, std::min(15, static_cast<int>(std::round(row[c] / s + z))));
                const size_t i = static_cast<size_t>(r) * cols + c;
                (*packed)[i >> 1] |= static_cast<uint8_t>((i & 1) ? q << 4 : q);
            }
        }
    }
}

struct Dev {  // one device allocation, freed on scope exit
    void* p = nullptr;
    explicit Dev(size_t bytes) {
        if (xqhip_malloc(&p, bytes) != 0) throw std::runtime_error(xqhip_last_error());
    }
    ~Dev() { xqhip_free(p); }
    template <typename T>
    T* as() const { return static_cast<T*>(p); }
};
void hip_ok(int rc) {
    if (rc != 0) throw std::runtime_error(xqhip_last_error());
}
template <typename T>
void upload(const Dev& d, const std::vector<T>& v) { hip_ok(xqhip_memcpy_h2d(d.p, v.data(), v.size() * sizeof(T), nullptr)); }
template <typename T>
std::vector<T> download(const Dev& d, size_t n) {
    std::vector<T> v(n);
    hip_ok(xqhip_memcpy_d2h(v.data(), d.p, n * sizeof(T), nullptr));
    return v;
}

// Runs `launch` kKernelWarmup + kKernelMeasured times on the null stream and
// returns the HIP-event durations of the measured calls.
RunStats time_kernel(const std::function<void()>& launch) {
    void *e0 = nullptr, *e1 = nullptr;
    hip_ok(xqhip_event_create(&e0));
    hip_ok(xqhip_event_create(&e1));
    std::vector<double> ms;
    for (int i = 0; i < kKernelWarmup + kKernelMeasured; ++i) {
        hip_ok(xqhip_event_record(e0, nullptr));
        launch();
        hip_ok(xqhip_event_record(e1, nullptr));
        hip_ok(xqhip_stream_synchronize(nullptr));
        float t = 0.0f;
        hip_ok(xqhip_event_elapsed_ms(e0, e1, &t));
        if (i >= kKernelWarmup) ms.push_back(t);
    }
    xqhip_event_destroy(e0);
    xqhip_event_destroy(e1);
    return run_stats(ms);
}

struct KernelRow {
    std::string name, family, implementation, shape, dims;
    RunStats ms;
    float checksum = 0.0f;
    double published = NAN;  // the reference microbench's published checksum, when it has one
    std::string note;
};

void put_row(std::ostream& o, const KernelRow& r) {
    o << "{\"name\":\"" << r.name << "\",\"family\":\"" << r.family << "\",\"op_family\":\"" << r.family
      << "\",\"backend\":\"hip\",\"implementation\":\"" << r.implementation << "\",\"qwen35_shape\":\"" << r.shape
      << "\",\"dims\":" << r.dims << ",\"timing\":\"hip_events_per_call\",\"wall_ms\":";
    put_stats(o, r.ms);
    o << ",\"checksum\":" << r.checksum;
    if (!std::isnan(r.published)) o << ",\"published_checksum\":" << r.published;
    if (!r.note.empty()) o << ",\"note\":\"" << esc(r.note) << "\"";
    o << '}';
}

KernelRow gemv_row(const char* name, int rows, int cols, double published) {
    std::vector<uint8_t> packed;
    std::vector<float> scales, zeros;
    {
        const std::vector<float> w = det_vector(static_cast<size_t>(rows) * cols, 0.04f);
        quantize_w4(w, rows, cols, 64, &packed, &scales, &zeros);
    }
    const std::vector<float> x = det_vector(static_cast<size_t>(cols), 0.25f);
    xqhip_w4 w{};
    hip_ok(xqhip_w4_upload(packed.data(), scales.data(), zeros.data(), rows, cols, 64, 0, &w));
    Dev xd(x.size() * 4), yd(static_cast<size_t>(rows) * 4);
    upload(xd, x);
    KernelRow r;
    try {
        r.ms = time_kernel([&] { hip_ok(xqhip_gemv_w4a16(&w, xd.p, XQHIP_F32, nullptr, yd.p, XQHIP_F32, XQHIP_EPI_STORE, nullptr)); });
    } catch (...) {
        xqhip_w4_free(&w);
        throw;
    }
    xqhip_w4_free(&w);
    r.name = name;
    r.family = "linear_w4a16_gemv";
    r.implementation = "hip_gfx950_fused_dequant_gemv_w4a16";
    r.shape = rows == 12288 ? "mlp_gate_or_up_projection"
                            : (cols == 12288 ? "mlp_down_projection" : "attention_or_output_projection");
    std::ostringstream d;
    d << "{\"rows\":" << rows << ",\"cols\":" << cols << ",\"bits\":4,\"group_size\":64,\"input_dtype\":\"fp32\"}";
    r.dims = d.str();
    r.checksum = sampled_sum(download<float>(yd, static_cast<size_t>(rows)));
    r.published = published;
    return r;
}

std::vector<KernelRow> vector_rows() {
    std::vector<KernelRow> rows;
    {  // RMSNorm of 4096 values, unit weights
        const int n = 4096;
        const std::vector<float> x = det_vector(n, 0.2f), w(n, 1.0f);
        Dev xd(n * 4), wd(n * 4), yd(n * 4);
        upload(xd, x);
        upload(wd, w);
        KernelRow r;
        r.ms = time_kernel([&] { hip_ok(xqhip_rmsnorm(xd.as<float>(), wd.as<float>(), n, 1.0e-6f, yd.as<float>(), nullptr)); });
        r.name = "rmsnorm_hidden4096";
        r.family = "rmsnorm";
        r.implementation = "hip_rmsnorm";
        r.shape = "hidden_size";
        r.dims = "{\"n\":4096,\"eps\":0.000001,\"dtype\":\"fp32\"}";
        r.checksum = sampled_sum(download<float>(yd, n));
        r.published = 9.94688;
        rows.push_back(r);
    }
    {  // RoPE of 16 query and 16 key heads of 256 at position 512 (the path's fused
       // per-head RMSNorm + RoPE + fp16 key append, norm weights 1)
        const int heads = 16, hd = 256, pos = 512;
        const std::vector<float> q = det_vector(heads * hd, 0.2f), k = det_vector(heads * hd, 0.2f);
        std::vector<float> cs(2 * static_cast<size_t>(pos + 1) * (hd / 2));
        hip_ok(xqhip_rope_table(1.0e7f, hd, pos + 1, cs.data()));
        const std::vector<float> ones(hd, 1.0f);
        const std::vector<int32_t> p{pos};
        const size_t cache = static_cast<size_t>(pos + 1) * heads * hd * 2;
        Dev qd(q.size() * 4), kd(k.size() * 4), vd(k.size() * 4), csd(cs.size() * 4), nd(hd * 4), pd(4),
            qo(q.size() * 4), go(q.size() * 4), kc(cache), vc(cache);
        upload(qd, q);
        upload(kd, k);
        upload(vd, k);
        upload(csd, cs);
        upload(nd, ones);
        upload(pd, p);
        KernelRow r;
        r.ms = time_kernel([&] {
            hip_ok(xqhip_attn_prep(qd.as<float>(), kd.as<float>(), vd.as<float>(), 0, heads, heads, hd, hd,
                                   nd.as<float>(), nd.as<float>(), 1.0e-6f, csd.as<float>(), pd.as<int32_t>(),
                                   qo.as<float>(), go.as<float>(), kc.p, vc.p, nullptr));
        });
        const std::vector<uint16_t> kh = download<uint16_t>(kc, cache / 2);
        std::vector<float> kr(static_cast<size_t>(heads) * hd);
        for (size_t i = 0; i < kr.size(); ++i) kr[i] = f16_to_f32(kh[static_cast<size_t>(pos) * heads * hd + i]);
        r.name = "rope_q_heads16_dim256_pos512";
        r.family = "rope";
        r.implementation = "hip_fused_qk_norm_rope_kv_append";
        r.shape = "q_heads_x_head_dim";
        r.dims = "{\"heads\":16,\"head_dim\":256,\"position\":512,\"theta\":10000000}";
        r.checksum = sampled_sum(download<float>(qo, q.size())) + sampled_sum(kr);
        r.note = "checksum of q plus the fp16-appended k after one call; the path fuses a per-head RMSNorm "
                 "(unit weights here) ahead of RoPE";
        rows.push_back(r);
    }
    {  // GQA decode, 512 cached tokens, 16 query / 4 kv heads of 256 (fp16 cache)
        const int ctx = 512, nkv = 4, nq = 16, hd = 256;
        const std::vector<float> q = det_vector(nq * hd, 0.1f), kv = det_vector(static_cast<size_t>(ctx) * nkv * hd, 0.1f);
        std::vector<uint16_t> kvh(kv.size());
        for (size_t i = 0; i < kv.size(); ++i) kvh[i] = f32_to_f16(kv[i]);
        const std::vector<float> open_gate(static_cast<size_t>(nq) * hd, 40.0f);  // sigmoid(40) == 1 in fp32
        const std::vector<int32_t> p{ctx - 1};
        Dev qd(q.size() * 4), kc(kvh.size() * 2), vc(kvh.size() * 2), gd(open_gate.size() * 4), pd(4),
            od(q.size() * 4), ws(xqhip_gqa_workspace_bytes(nq, nkv, hd));
        upload(qd, q);
        upload(kc, kvh);
        upload(vc, kvh);
        upload(gd, open_gate);
        upload(pd, p);
        KernelRow r;
        r.ms = time_kernel([&] {
            hip_ok(xqhip_gqa_decode(qd.as<float>(), kc.p, vc.p, gd.as<float>(), nq, nkv, hd, ctx, pd.as<int32_t>(),
                                    od.as<float>(), ws.p, nullptr));
        });
        r.name = "gqa_decode_ctx512_q16_kv4_dim256";
        r.family = "attention_decode";
        r.implementation = "hip_gqa_decode_split_fp16_kv";
        r.shape = "full_attention_layer_decode";
        r.dims = "{\"context\":512,\"kv_heads\":4,\"q_heads\":16,\"head_dim\":256,\"kv_cache\":\"fp16\"}";
        r.checksum = sampled_sum(download<float>(od, q.size()));
        r.published = -0.00442318;
        r.note = "output gate held open (gate 40); keys and values rounded to the fp16 cache";
        rows.push_back(r);
    }
    {  // gated delta rule, key and value dims 128, beta 0.5, log decay -0.1; the state
       // carries over, so the checksum is the one after all four calls
        const int dk = 128, dv = 128;
        std::vector<float> conv = det_vector(dk, 0.1f);
        const std::vector<float> k = det_vector(dk, 0.1f), v = det_vector(dv, 0.1f);
        conv.insert(conv.end(), k.begin(), k.end());
        conv.insert(conv.end(), v.begin(), v.end());
        const std::vector<float> state = det_vector(static_cast<size_t>(dk) * dv, 0.01f);
        // g = -exp(a_log) softplus(a + dt_bias) = -0.1 with a_log = dt_bias = 0, a = log(e^0.1 - 1);
        // beta = sigmoid(b) = 0.5 with b = 0
        const std::vector<float> a{std::log(std::expm1(0.1f))}, zero{0.0f};
        Dev cd(conv.size() * 4), sd(state.size() * 4), ad(4), bd(4), ld(4), dd(4), od(dv * 4);
        upload(cd, conv);
        upload(sd, state);
        upload(ad, a);
        upload(bd, zero);
        upload(ld, zero);
        upload(dd, zero);
        KernelRow r;
        r.ms = time_kernel([&] {
            hip_ok(xqhip_gated_delta(cd.as<float>(), ad.as<float>(), bd.as<float>(), ld.as<float>(), dd.as<float>(),
                                     sd.as<float>(), 1, 1, dk, dv, od.as<float>(), nullptr));
        });
        r.name = "gated_delta_decode_k128_v128";
        r.family = "linear_attention_delta";
        r.implementation = "hip_gated_delta_fp32_state";
        r.shape = "linear_attention_layer_decode";
        r.dims = "{\"key_dim\":128,\"value_dim\":128,\"state_elements\":16384}";
        r.checksum = sampled_sum(download<float>(od, dv));
        r.published = -0.0171842;
        rows.push_back(r);
    }
    return rows;
}

std::string microbench_json() {
    try {
        if (xqhip_device_count() <= 0 || xqhip_set_device(0) != 0)
            return "{\"status\":\"error\",\"error\":\"no HIP device visible\"}";
        std::vector<KernelRow> rows;
        rows.push_back(gemv_row("gemv_w4a16_attn_4096x4096", 4096, 4096, 320.586));
        rows.push_back(gemv_row("gemv_w4a16_mlp_up_12288x4096", 12288, 4096, 13.1145));
        rows.push_back(gemv_row("gemv_w4a16_mlp_down_4096x12288", 4096, 12288, 207.929));
        for (const KernelRow& r : vector_rows()) rows.push_back(r);
        std::ostringstream o;
        o << "{\"status\":\"ok\",\"measurement\":\"on_device_microbench\",\"implementation\":\"hip_gfx950\","
          << "\"iterations\":{\"warmup\":" << kKernelWarmup << ",\"measured\":" << kKernelMeasured << "},"
          << "\"qwen35_shapes\":{\"hidden_size\":4096,\"intermediate_size\":12288,\"num_attention_heads\":16,"
          << "\"num_key_value_heads\":4,\"head_dim\":256,\"linear_key_head_dim\":128,\"linear_value_head_dim\":128},"
          << "\"rows\":[";
        for (size_t i = 0; i < rows.size(); ++i) {
            o << (i ? "," : "");
            put_row(o, rows[i]);
        }
        o << "]}";
        return o.str();
    } catch (const std::exception& e) {
        return "{\"status\":\"error\",\"error\":\"" + esc(e.what()) + "\"}";
    }
}

// ---- the three harness entry points --------------------------------------------

struct Run {
    int index = 0;
    bool warmup = false;
    xq_status status = XQ_OK;
    xq_metrics m{};
};

const char* kReplaced =
    "[\"q_proj\",\"k_proj\",\"v_proj\",\"o_proj\",\"gate_proj\",\"up_proj\",\"down_proj\",\"rmsnorm\",\"rope\","
    "\"attention\",\"linear_attention_state\",\"lm_head\",\"sampling\",\"prefill_kv_build\"]";
const char* kModel =
    "\"model\":{\"hf_repo\":\"Qwen/Qwen3.5-9B\",\"hf_revision\":\"c202236235762e1c871ad0ccb60c8ee5ba337b9a\","
    "\"format\":\"xqwen35_custom_w4a16\"";

std::string backend_fields(const std::string& requested, const std::string& actual) {
    std::ostringstream o;
    o << "\"backend\":\"" << esc(actual) << "\",\"backend_requested\":\"" << esc(requested)
      << "\",\"backend_actual\":\"" << esc(actual) << "\",\"custom_backend_requested\":\"" << esc(requested)
      << "\",\"custom_backend_actual\":\"" << esc(actual) << "\",";
    return o.str();
}

std::string vulkan_attempt(const std::string& requested) {
    const bool asked = requested == "vulkan" || requested == "cpu_vulkan_hybrid";
    return std::string("{\"status\":\"skipped\",\"requested_backend\":\"") + esc(requested) + "\",\"reason\":\"" +
           (asked ? "no_vulkan_on_this_build_hip_serves_the_request" : "vulkan_not_requested") + "\"}";
}

std::string run_benchmark(const Args& a) {
    const xq_options opt = harness_options(a.backend.c_str(), kThreads);
    xq_session* s = nullptr;
    const xq_status cs = xq_create(a.model_dir.c_str(), &opt, &s);
    if (cs != XQ_OK || !s) {
        std::ostringstream o;
        o << "{\"schema_version\":4,\"engine\":\"customlib\"," << backend_fields(a.backend, a.backend)
          << "\"status\":\"error\",\"error_code\":" << cs << ",\"error\":\"xq_create failed\","
          << "\"custom_path\":{\"calls_mnn_llm_response_for_measured_generation\":false,\"use_mnn_fallback\":0,"
          << "\"vulkan_generation_kernels_used\":false},\"vulkan_attempt\":" << vulkan_attempt(a.backend)
          << ",\"artifact\":{\"model_dir\":\"" << esc(a.model_dir) << "\"}}";
        return o.str();
    }
    xq_metrics initial{};
    initial.struct_size = sizeof(initial);
    xq_get_last_metrics(s, &initial);
    const int warmups = std::max(0, a.warmup), measured = std::max(1, a.measured);
    const std::vector<int32_t> prompt(static_cast<size_t>(std::max(0, a.prompt_tokens)), kPromptToken);
    std::vector<int32_t> out(static_cast<size_t>(std::max(0, a.max_new)));
    std::vector<Run> runs;
    std::vector<double> prefill_tps, decode_tps, total_ms;
    xq_status terminal = XQ_OK;
    std::string terminal_error;
    for (int i = 0; i < warmups + measured; ++i) {
        xq_reset(s);
        Run r;
        r.index = i;
        r.warmup = i < warmups;
        r.m.struct_size = sizeof(r.m);
        std::fill(out.begin(), out.end(), 0);
        r.status = xq_generate(s, prompt.data(), prompt.size(), out.size(), out.data(), out.size(), &r.m);
        std::cerr << "BENCH_ITER engine=customlib warmup=" << r.warmup << " prompt=" << r.m.prompt_tokens
                  << " generated=" << r.m.generated_tokens << " prefill_ms=" << r.m.prefill_ms
                  << " decode_ms=" << r.m.decode_total_ms << " status=" << r.status << std::endl;
        runs.push_back(r);
        if (r.status != XQ_OK) {
            terminal = r.status;
            terminal_error = r.m.error;
            break;
        }
        if (!r.warmup) {
            prefill_tps.push_back(per_second(r.m.prompt_tokens, r.m.prefill_ms));
            decode_tps.push_back(per_second(r.m.generated_tokens, r.m.decode_total_ms));
            total_ms.push_back(r.m.total_generate_ms);
        }
    }
    const std::string trace = session_json(xq_get_kernel_trace_json, s, "{\"rows\":[]}");
    xq_destroy(s);
    const std::string micro = a.microbench ? microbench_json()
                                           : std::string("{\"status\":\"skipped\",\"reason\":\"--no-microbench\"}");
    const std::string actual = trace_backend_all(trace, a.backend);
    const bool ok = terminal == XQ_OK && prefill_tps.size() == static_cast<size_t>(measured);
    const RunStats ps = run_stats(prefill_tps), ds = run_stats(decode_tps), ts = run_stats(total_ms);

    std::ostringstream o;
    o << "{\"schema_version\":4,\"engine\":\"customlib\"," << backend_fields(a.backend, actual) << "\"status\":\""
      << (ok ? "ok" : "error") << "\",";
    if (!ok)
        o << "\"error_code\":" << terminal << ",\"error\":\""
          << esc(terminal_error.empty() ? "not all measurement iterations completed" : terminal_error) << "\",";
    // families with no row of their own (fused into another kernel, or inside the
    // decode graph) report the session's backend
    auto fam = [&](std::vector<std::string> f) { return trace_backend(trace, f, actual); };
    o << kModel << ",\"quantization\":{\"bits\":4,\"group_size\":64,\"scheme\":\"w4a16_groupwise\"}},"
      << "\"artifact\":{\"model_dir\":\"" << esc(a.model_dir) << "\"},\"runtime\":{\"threads\":" << kThreads
      << ",\"backend_actual_verified\":true,\"precision\":\"low\",\"memory\":\"low\",\"power\":\"normal\","
      << "\"use_mmap\":true,\"reuse_kv\":false,\"selected_kernels\":{\"summary\":\""
      << esc(runs.empty() ? initial.selected_kernels : runs.back().m.selected_kernels)
      << "\",\"hotpath_replaced\":true,\"full_custom_decode\":true,\"replaced_op_families\":" << kReplaced
      << ",\"fallback_op_families\":[],\"op_family_backends\":{\"q_proj\":\"" << fam({"q_proj"})
      << "\",\"k_proj\":\"" << fam({"k_proj"}) << "\",\"v_proj\":\"" << fam({"v_proj"}) << "\",\"o_proj\":\""
      << fam({"o_proj"}) << "\",\"gate_proj\":\"" << fam({"gate_proj"}) << "\",\"up_proj\":\"" << fam({"up_proj"})
      << "\",\"down_proj\":\"" << fam({"down_proj"}) << "\",\"linear_attention_projections\":\""
      << fam({"linear_attention_projection"}) << "\",\"rmsnorm\":\"" << fam({"rmsnorm"}) << "\",\"rope\":\""
      << fam({"rope"}) << "\",\"attention\":\""
      << fam({"attention", "attention_score", "attention_softmax", "attention_v_reduce"})
      << "\",\"linear_attention_state\":\"" << fam({"linear_attention_state"}) << "\",\"activation\":\""
      << fam({"activation", "silu"}) << "\",\"lm_head\":\"" << fam({"lm_head"}) << "\",\"sampling\":\""
      << fam({"sampling"}) << "\",\"prefill_kv_build\":\"" << fam({"prefill_kv_build"}) << "\"}}},"
      << "\"custom_path\":{\"calls_mnn_llm_response_for_measured_generation\":false,\"use_mnn_fallback\":0,"
      << "\"vulkan_generation_kernels_used\":false,\"decode_loop\":\"xq_session::generate -> xq_prefill/xq_decode_one"
      << " -> device model prefill/decode graph\",\"weight_format\":\"xq4_groupwise_w4a16\"},"
      << "\"vulkan_attempt\":" << vulkan_attempt(a.backend) << ",\"generation\":{\"prompt_tokens_requested\":"
      << a.prompt_tokens << ",\"max_new_tokens\":" << a.max_new << ",\"prompt_token_id\":" << kPromptToken
      << ",\"temperature\":0,\"top_k\":1,\"top_p\":1,\"batch_size\":1},\"iterations\":{\"warmup\":" << warmups
      << ",\"measured\":" << prefill_tps.size() << ",\"target_measured\":" << measured << "},"
      << "\"timing\":{\"load_ms\":" << initial.load_ms << ",\"total_generate_ms\":";
    put_stats(o, ts);
    o << "},\"tokens_per_second\":{\"prefill\":";
    put_stats(o, ps);
    o << ",\"decode\":";
    put_stats(o, ds);
    // time per output token from the decode rate statistics (min time <- max rate)
    RunStats tpot;
    auto inv = [](double tps) { return tps > 0 ? 1000.0 / tps : 0.0; };
    tpot.mean = inv(ds.mean);
    tpot.median = inv(ds.median);
    tpot.min = inv(ds.max);
    tpot.max = inv(ds.min);
    o << "},\"time_per_output_token_ms\":{\"decode\":";
    put_stats(o, tpot, false);
    o << "},\"runs\":[";
    for (size_t i = 0; i < runs.size(); ++i) {
        const Run& r = runs[i];
        o << (i ? "," : "") << "{\"index\":" << r.index << ",\"warmup\":" << tf(r.warmup)
          << ",\"status_code\":" << r.status << ",\"prompt_tokens\":" << r.m.prompt_tokens
          << ",\"generated_tokens\":" << r.m.generated_tokens << ",\"prefill_ms\":" << r.m.prefill_ms
          << ",\"first_token_ms\":" << r.m.first_token_ms << ",\"decode_total_ms\":" << r.m.decode_total_ms
          << ",\"total_generate_ms\":" << r.m.total_generate_ms
          << ",\"prefill_tokens_per_second\":" << per_second(r.m.prompt_tokens, r.m.prefill_ms)
          << ",\"decode_tokens_per_second\":" << per_second(r.m.generated_tokens, r.m.decode_total_ms)
          << ",\"error\":\"" << esc(r.m.error) << "\"}";
    }
    o << "],\"per_kernel_wall_clock\":" << trace << ",\"custom_kernel_microbench\":" << micro
      << ",\"mnn_hotpath_op_trace\":{\"status\":\"error\",\"error\":\"built without MNN\"}}";
    return o.str();
}

std::string run_quality(const Args& a) {
    const int max_new = std::max(1, std::min(64, a.validation_max_new));
    const xq_options opt = harness_options(a.backend.c_str(), kThreads);
    xq_session* s = nullptr;
    xq_status st = xq_create(a.model_dir.c_str(), &opt, &s);
    if (st != XQ_OK || !s) {
        std::ostringstream o;
        o << "{\"schema_version\":1,\"artifact_type\":\"quality_validation\",\"engine\":\"customlib\","
          << "\"status\":\"error\",\"quality_gate_passed\":false,\"error_code\":" << st
          << ",\"error\":\"xq_create failed\",\"custom_backend_requested\":\"" << esc(a.backend)
          << "\",\"custom_backend_actual\":\"" << esc(a.backend) << "\",\"custom_path\":{"
          << "\"calls_mnn_llm_response_for_measured_generation\":false,\"use_mnn_fallback\":0,"
          << "\"full_custom_decode\":true,\"fallback_op_families\":[]},\"validation\":{\"prompt_set\":"
          << "\"small_english_tokenizer_ids\",\"validation_compare_to_stock\":true,\"tokenizer_decode_available\":false,"
          << "\"max_new_tokens\":" << max_new << ",\"temperature\":0,\"top_k\":1,\"top_p\":1},"
          << "\"artifact\":{\"model_dir\":\"" << esc(a.model_dir) << "\"}}";
        return o.str();
    }
    xq_metrics initial{};
    initial.struct_size = sizeof(initial);
    xq_get_last_metrics(s, &initial);
    xq_metrics last = initial;
    bool all_ok = true;
    std::ostringstream pj;
    pj << '[';
    const std::vector<PromptCase> cases = validation_prompts();
    for (size_t i = 0; i < cases.size(); ++i) {
        const PromptCase& p = cases[i];
        xq_reset(s);
        std::vector<int32_t> out(static_cast<size_t>(max_new));
        xq_metrics m{};
        m.struct_size = sizeof(m);
        st = xq_generate(s, p.ids.data(), p.ids.size(), out.size(), out.data(), out.size(), &m);
        last = m;
        out.resize(st == XQ_OK ? std::min<size_t>(out.size(), m.generated_tokens) : 0);
        const SeqStats ss = sequence_stats(out);
        const bool ok = st == XQ_OK && ss.invalid == 0 && !ss.empty && !ss.degenerate;
        all_ok = all_ok && ok;
        pj << (i ? "," : "") << "{\"id\":\"" << esc(p.id) << "\",\"prompt_kind\":\"" << esc(p.kind)
           << "\",\"prompt_text_hint\":\"" << esc(p.hint) << "\",\"raw_text_prompt_available\":false,"
           << "\"prompt_token_count\":" << p.ids.size() << ",\"prompt_token_ids\":";
        put_ids(pj, p.ids);
        pj << ",\"generated_token_count\":" << out.size() << ",\"generated_token_ids\":";
        put_ids(pj, out);
        pj << ",\"decoded_text_available\":false,\"decoded_generated_text\":\"\",\"status_code\":" << st
           << ",\"status\":\"" << (ok ? "ok" : "error") << "\",\"invalid_token_count\":" << ss.invalid
           << ",\"empty_output\":" << tf(ss.empty) << ",\"longest_repeated_run\":" << ss.longest_run
           << ",\"longest_repeated_run_token\":" << ss.longest_run_token << ",\"most_repeated_token\":" << ss.most_token
           << ",\"most_repeated_token_count\":" << ss.most_count
           << ",\"repeated_token_220_longest_run\":" << ss.space_run
           << ",\"repeated_token_220_failure\":" << tf(ss.space_run >= 8) << ",\"unique_token_count\":" << ss.unique
           << ",\"obvious_degenerate_output\":" << tf(ss.degenerate) << ",\"prefill_ms\":" << m.prefill_ms
           << ",\"decode_total_ms\":" << m.decode_total_ms << "}";
    }
    pj << ']';
    const std::string trace = session_json(xq_get_kernel_trace_json, s, "{\"rows\":[]}");
    xq_destroy(s);
    const std::string actual = trace_backend_all(trace, a.backend);
    std::ostringstream o;
    o << "{\"schema_version\":1,\"artifact_type\":\"quality_validation\",\"engine\":\"customlib\",\"status\":\""
      << (all_ok ? "ok" : "error") << "\",\"quality_gate_passed\":" << tf(all_ok) << "," << kModel
      << ",\"vocab_size_assumed\":" << kQwen35Vocab << "},\"artifact\":{\"model_dir\":\"" << esc(a.model_dir)
      << "\"},\"runtime\":{\"threads\":" << kThreads << ",\"selected_kernels\":{\"summary\":\""
      << esc(last.selected_kernels[0] ? last.selected_kernels : initial.selected_kernels)
      << "\",\"hotpath_replaced\":true,\"full_custom_decode\":true,\"replaced_op_families\":" << kReplaced
      << ",\"fallback_op_families\":[]}},\"custom_path\":{\"calls_mnn_llm_response_for_measured_generation\":false,"
      << "\"use_mnn_fallback\":0,\"full_custom_decode\":true,\"fallback_op_families\":[],\"decode_loop\":"
      << "\"xq_session::generate -> xq_prefill/xq_decode_one -> device model prefill/decode graph\"},"
      << "\"custom_backend_requested\":\"" << esc(a.backend) << "\",\"custom_backend_actual\":\"" << esc(actual)
      << "\",\"validation\":{\"prompt_set\":\"small_english_tokenizer_ids\",\"validation_compare_to_stock\":true,"
      << "\"tokenizer_decode_available\":false,\"validation_dump_tokens\":true,\"validation_dump_text\":false,"
      << "\"max_new_tokens\":" << max_new << ",\"temperature\":0,\"top_k\":1,\"top_p\":1,\"note\":\"Fixed token-ID "
      << "prompts are used so stock MNN and customlib receive identical prompt IDs.\"},\"prompts\":" << pj.str()
      << ",\"per_kernel_wall_clock\":" << trace << "}";
    return o.str();
}

std::string run_selftest() {
    std::vector<char> buf(1 << 20);
    const xq_status st = xq_run_vulkan_w4a16_selftest(buf.data(), buf.size());
    std::string js = buf.data();
    if (js.empty())
        js = "{\"engine\":\"customlib\",\"test\":\"vulkan_w4a16_gemv_correctness\",\"status\":\"error\","
             "\"pass\":false,\"error\":\"empty selftest JSON\"}";
    std::cerr << "BENCH_VULKAN_SELFTEST_STATUS " << st << std::endl;
    return js;
}

bool has(const std::string& js, const std::string& s) { return js.find(s) != std::string::npos; }

// The instrumentation test's checks for each mode; returns the failed ones.
std::vector<std::string> check(const Args& a, const std::string& js) {
    std::vector<std::string> bad;
    auto need = [&](const std::string& s, const char* what) {
        if (!has(js, s)) bad.push_back(what);
    };
    if (a.selftest) {
        need("\"status\":\"ok\"", "selftest status not ok");
        need("\"pass\":true", "selftest did not pass");
        need("\"custom_backend_actual\":\"hip\"", "selftest did not run on the HIP device");
        need("\"hip_runtime_initialized\":true", "HIP runtime evidence missing");
    } else if (a.quality) {
        need("\"status\":\"ok\"", "quality validation returned non-ok JSON");
        need("\"quality_gate_passed\":true", "quality sanity gate failed");
        need("\"full_custom_decode\":true", "custom quality path evidence missing");
        need("\"fallback_op_families\":[]", "custom quality path evidence missing");
        need("\"calls_mnn_llm_response_for_measured_generation\":false", "custom quality path evidence missing");
    } else {
        need("\"status\":\"ok\"", "benchmark returned non-ok JSON");
        need("\"hotpath_replaced\":true", "hotpath replacement evidence missing");
        need("\"full_custom_decode\":true", "full custom decode evidence missing");
        need("\"fallback_op_families\":[]", "fallback list is not empty");
        need("\"calls_mnn_llm_response_for_measured_generation\":false", "MNN-response evidence missing");
        need("\"custom_backend_requested\":\"" + a.backend + "\"", "backend request evidence missing");
        need("\"custom_backend_actual\"", "backend actual evidence missing");
        need("\"lm_head_custom", "lm_head trace evidence missing");
        need("\"sampling_greedy_custom\"", "sampling trace evidence missing");
    }
    return bad;
}

void write_artifact(const Args& a, const std::string& file, const std::string& js) {
    if (a.artifact_dir.empty()) return;
    const std::string dir = a.artifact_dir + "/bench_artifacts";
    mkdir(a.artifact_dir.c_str(), 0755);
    mkdir(dir.c_str(), 0755);
    std::ofstream(dir + "/" + file) << js;
}

int usage(const char* argv0) {
    std::cerr << "usage: " << argv0
              << " [--prompt-tokens N] [--max-new-tokens N] [--warmup-iterations N] [--measured-iterations N]"
                 " [--validation-max-new-tokens N] [--custom-backend B] [--run-quality-validation]"
                 " [--run-vulkan-selftest] [--no-microbench] [--artifact-dir DIR] <model_dir>\n";
    return 2;
}

}  // namespace

int main(int argc, char** argv) {
    Args a;
    for (int i = 1; i < argc; ++i) {
        const std::string k = argv[i];
        auto num = [&](int* dst) {
            if (i + 1 >= argc) return false;
            *dst = std::atoi(argv[++i]);
            return true;
        };
        bool ok = true;
        if (k == "--prompt-tokens") ok = num(&a.prompt_tokens);
        else if (k == "--max-new-tokens") ok = num(&a.max_new);
        else if (k == "--warmup-iterations") ok = num(&a.warmup);
        else if (k == "--measured-iterations") ok = num(&a.measured);
        else if (k == "--validation-max-new-tokens") ok = num(&a.validation_max_new);
        else if (k == "--custom-backend" && i + 1 < argc) a.backend = sanitize_backend(argv[++i]);
        else if (k == "--artifact-dir" && i + 1 < argc) a.artifact_dir = argv[++i];
        else if (k == "--run-quality-validation") a.quality = true;
        else if (k == "--run-vulkan-selftest") a.selftest = true;
        else if (k == "--no-microbench") a.microbench = false;
        else if (!k.empty() && k[0] != '-' && a.model_dir.empty()) a.model_dir = k;
        else ok = false;
        if (!ok) return usage(argv[0]);
    }
    if (a.model_dir.empty() && !a.selftest) return usage(argv[0]);
    std::string js, file;
    if (a.selftest) {
        js = run_selftest();
        file = "vulkan_w4a16_selftest.json";
    } else if (a.quality) {
        js = run_quality(a);
        file = "quality_validation_custom.json";
    } else {
        std::cerr << "BENCH_START engine=customlib model_dir=" << a.model_dir << " requested_backend=" << a.backend
                  << std::endl;
        js = run_benchmark(a);
        file = "customlib_" + a.backend + "_benchmark.json";
    }
    std::cout << js << std::endl;
    write_artifact(a, file, js);
    const std::vector<std::string> bad = check(a, js);
    for (const std::string& b : bad) std::cerr << "CHECK FAILED: " << b << std::endl;
    return bad.empty() ? 0 : 1;
}
