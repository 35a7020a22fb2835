// harness.hpp - pieces shared by the two caller-side tools (xq_host_quality_runner,
// xq_benchmark): the fixed token-id prompt set, degeneracy statistics of a
// generated sequence, run statistics and JSON text helpers.  The tools talk to
// the library only through include/xqwen35.h, so either build of the library
// (this HIP one or the reference CPU one) can sit behind them.
//
// Prompt set and statistics follow the reference harnesses:
//   prompts              customlib/tools/xq_host_quality_runner.cpp:26-70,
//                        android/benchmark_app/src/main/cpp/benchmark_jni.cpp:228-264
//   run statistics       xq_host_quality_runner.cpp:128-199
//   mean/median/stdev    benchmark_jni.cpp:111-176 (population stdev)
#pragma once

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <map>
#include <sstream>
#include <string>
#include <vector>

#include "xqwen35.h"

namespace xqtool {

constexpr int kQwen35Vocab = 248320;
constexpr int32_t kSpaceToken = 220;  // the token whose runs the quality gate watches

struct PromptCase {
    std::string id, kind, hint;
    std::vector<int32_t> ids;
};

// The five validation prompts: tokenizer-derived ids of four short English /
// code / arithmetic prompts and a 512-token benchmark-style prompt (a 12-token
// sentence, then a 12-token variant repeated until 512 ids).
inline std::vector<PromptCase> validation_prompts() {
    std::vector<PromptCase> p;
    p.push_back({"english_factual", "short_english_factual",
                 "Tokenizer-derived IDs for: What is the capital of France? Answer in one short sentence.",
                 {3710, 369, 279, 6511, 314, 9338, 30, 21134, 303, 799, 2716, 11316, 13}});
    p.push_back({"english_explain", "short_english_explain",
                 "Tokenizer-derived IDs for: Explain in one sentence why the sky looks blue.",
                 {814, 20139, 303, 799, 11316, 3069, 279, 12515, 5686, 6105, 13}});
    p.push_back({"code_like", "code_like",
                 "Tokenizer-derived IDs for: Write a Python function add(a, b) that returns their sum.",
                 {7734, 264, 12654, 709, 884, 2784, 11, 292, 8, 421, 4523, 836, 2542, 13}});
    p.push_back({"math_reasoning", "math_reasoning", "Tokenizer-derived IDs for a short arithmetic reasoning prompt.",
                 {2592, 1017, 513, 220, 18, 39332, 321, 488, 3569, 220, 17, 777, 11, 1204, 1599, 39332, 635, 488, 599,
                  30, 21134, 1132, 279, 1324, 13}});
    static const int32_t head[12] = {8917, 5437, 537, 279, 2614, 27502, 8129, 303, 1330, 61446, 31969, 13};
    std::vector<int32_t> longp(head, head + 12);
    for (size_t i = 0; longp.size() < 512; ++i) longp.push_back(i % 12 == 0 ? 7860 : head[i % 12]);
    p.push_back({"long_512_token_style", "long_512_token_style", "Tokenizer-derived 512-token benchmark-style prompt.",
                 longp});
    return p;
}

// Repetition statistics of one generated sequence.
struct SeqStats {
    int invalid = 0;           // ids outside [0, vocab)
    int longest_run = 0;       // longest run of one repeated id
    int32_t longest_run_token = -1;
    int32_t most_token = -1;   // the id that first reaches the highest count
    int most_count = 0;
    int space_run = 0;         // longest run of kSpaceToken
    int unique = 0;
    bool empty = true;
    bool degenerate = true;    // empty, a run of 16, or 8 spaces in a row
};

inline SeqStats sequence_stats(const std::vector<int32_t>& ids, int vocab = kQwen35Vocab) {
    SeqStats s;
    s.empty = ids.empty();
    std::map<int32_t, int> count;
    int run = 0, srun = 0;
    for (size_t i = 0; i < ids.size(); ++i) {
        const int32_t t = ids[i];
        if (t < 0 || t >= vocab) ++s.invalid;
        run = (i > 0 && t == ids[i - 1]) ? run + 1 : 1;
        if (run > s.longest_run) {  // strict: ties keep the earlier run
            s.longest_run = run;
            s.longest_run_token = t;
        }
        srun = t == kSpaceToken ? srun + 1 : 0;
        s.space_run = std::max(s.space_run, srun);
        const int c = ++count[t];
        if (c > s.most_count) {
            s.most_count = c;
            s.most_token = t;
        }
    }
    s.unique = static_cast<int>(count.size());
    s.degenerate = s.empty || s.longest_run >= 16 || s.space_run >= 8;
    return s;
}

struct RunStats {
    double mean = 0, median = 0, min = 0, max = 0, stdev = 0;
};

inline RunStats run_stats(std::vector<double> v) {
    RunStats r;
    if (v.empty()) return r;
    std::sort(v.begin(), v.end());
    const size_t n = v.size();
    r.min = v.front();
    r.max = v.back();
    r.median = n % 2 ? v[n / 2] : 0.5 * (v[n / 2 - 1] + v[n / 2]);
    double sum = 0;
    for (double x : v) sum += x;
    r.mean = sum / static_cast<double>(n);
    double sq = 0;
    for (double x : v) sq += (x - r.mean) * (x - r.mean);
    r.stdev = std::sqrt(sq / static_cast<double>(n));
    return r;
}

inline double per_second(uint64_t n, double ms) { return n == 0 || ms <= 0 ? 0.0 : static_cast<double>(n) * 1000.0 / ms; }

inline std::string esc(const std::string& in) {
    static const char* hex = "0123456789abcdef";
    std::string o;
    for (char c : in) {
        switch (c) {
            case '"': o += "\\\""; break;
            case '\\': o += "\\\\"; break;
            case '\b': o += "\\b"; break;
            case '\f': o += "\\f"; break;
            case '\n': o += "\\n"; break;
            case '\r': o += "\\r"; break;
            case '\t': o += "\\t"; break;
            default:
                if (static_cast<unsigned char>(c) < 0x20) {
                    o += "\\u00";
                    o += hex[(c >> 4) & 15];
                    o += hex[c & 15];
                } else {
                    o += c;
                }
        }
    }
    return o;
}

inline void put_ids(std::ostream& o, const std::vector<int32_t>& ids) {
    o << '[';
    for (size_t i = 0; i < ids.size(); ++i) o << (i ? "," : "") << ids[i];
    o << ']';
}

inline void put_stats(std::ostream& o, const RunStats& s, bool with_stdev = true) {
    o << "{\"mean\":" << s.mean << ",\"median\":" << s.median << ",\"min\":" << s.min << ",\"max\":" << s.max;
    if (with_stdev) o << ",\"stdev\":" << s.stdev;
    o << '}';
}

inline const char* tf(bool b) { return b ? "true" : "false"; }

// One of the session's JSON getters into a 1 MiB buffer; `fallback` on failure.
template <typename Getter>
std::string session_json(Getter get, xq_session* s, const char* fallback) {
    std::vector<char> buf(1 << 20);
    return get(s, buf.data(), buf.size()) == XQ_OK ? std::string(buf.data()) : std::string(fallback);
}

// The backends the kernel-trace rows of the given op families ran on: one
// name, "mixed" for several, `none` when no row of those families exists.
// A family also matches rows that list it among their fused ops ("fused:k_proj").
inline std::string trace_backend(const std::string& trace, const std::vector<std::string>& families,
                                 const std::string& none) {
    std::vector<std::string> seen;
    size_t pos = 0;
    while ((pos = trace.find("{\"name\":\"", pos)) != std::string::npos) {
        const size_t end = trace.find('}', pos);
        if (end == std::string::npos) break;
        const std::string row = trace.substr(pos, end - pos);
        pos = end;
        auto field = [&](const char* key) {
            const std::string k = std::string("\"") + key + "\":\"";
            const size_t b = row.find(k);
            if (b == std::string::npos) return std::string();
            const size_t e = row.find('"', b + k.size());
            return row.substr(b + k.size(), e - b - k.size());
        };
        const std::string name = field("name"), fam = field("op_family"), be = field("backend");
        bool hit = false;
        for (const std::string& f : families) {
            const size_t fz = name.find("fused:");
            hit = hit || fam == f || (fz != std::string::npos && name.find(f, fz) != std::string::npos);
        }
        if (hit && std::find(seen.begin(), seen.end(), be) == seen.end()) seen.push_back(be);
    }
    if (seen.empty()) return none;
    return seen.size() == 1 ? seen[0] : "mixed";
}

// The backend every trace row reports ("mixed" when they differ), else `none`.
inline std::string trace_backend_all(const std::string& trace, const std::string& none) {
    std::vector<std::string> seen;
    const std::string k = "\"backend\":\"";
    size_t pos = 0;
    while ((pos = trace.find(k, pos)) != std::string::npos) {
        const size_t b = pos + k.size(), e = trace.find('"', b);
        if (e == std::string::npos) break;
        const std::string be = trace.substr(b, e - b);
        if (std::find(seen.begin(), seen.end(), be) == seen.end()) seen.push_back(be);
        pos = e;
    }
    if (seen.empty()) return none;
    return seen.size() == 1 ? seen[0] : "mixed";
}

inline xq_options harness_options(const char* backend, int threads) {
    xq_options o{};
    o.struct_size = sizeof(o);
    o.backend = backend;
    o.threads = threads;
    o.quant_bits = 4;
    o.group_size = 64;
    o.max_context_tokens = 8192;
    o.enable_autotune = 1;
    o.use_mnn_fallback = 0;
    return o;
}

}  // namespace xqtool
