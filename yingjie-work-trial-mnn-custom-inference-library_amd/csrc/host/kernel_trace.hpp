// kernel_trace.hpp - per-op timing table exported as JSON by
// xq_get_kernel_trace_json, with the reference's row layout
// (customlib/runtime/custom_model.hpp:19-36, custom_model.cpp:374-417):
// {"rows":[{"name","op_family","backend","calls","total_ms","mean_ms","min_ms","max_ms"}]}, plus
// integer fields beside "rows" that say how the rows were sampled
#pragma once

#include <cstdint>
#include <map>
#include <string>

namespace xqh {

struct TraceStat {
    uint64_t calls = 0;
    double total_ms = 0.0, min_ms = 0.0, max_ms = 0.0;
    std::string backend;
};

class KernelTrace {
public:
    void add(const std::string& name, double ms, const std::string& backend);
    // a top-level integer field of the JSON beside "rows" (e.g. how many decode
    // steps the per-op rows were sampled from)
    void set_count(const std::string& key, int64_t value) { counts_[key] = value; }
    void reset() {
        rows_.clear();
        counts_.clear();
    }
    std::string to_json() const;
    bool empty() const { return rows_.empty(); }

private:
    std::map<std::string, TraceStat> rows_;
    std::map<std::string, int64_t> counts_;
};

std::string json_escape(const std::string& s);
// Op family of a trace row name (the reference's classification,
// custom_model.cpp:116-179; the same substrings map to the same families).
std::string op_family(const std::string& name);

}  // namespace xqh
