// selftest.cpp - xq_run_vulkan_w4a16_selftest on the HIP device.
//
// Same deterministic workload as the reference's GPU self-test
// (customlib/runtime/vulkan_backend.cpp:65-84 generators, :1638-1720 shapes and
// tolerances): dense weights 0.20 sin(((17r+13c) mod 997) 0.013) +
// 0.05 cos(((7r+19c) mod 769) 0.017), min/max 4-bit quantisation with group 64
// (kernels/reference/ref_gemv.cpp:38-75), input 0.15 sin((c mod 1021) 0.011) +
// 0.03 cos((c mod 577) 0.019); the device GEMV is compared with a float64
// dequantised dot product computed here on the host.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <sstream>
#include <string>
#include <vector>

#include "kernel_trace.hpp"
#include "xqhip.h"
#include "xqwen35.h"

namespace {

struct QM {
    int rows, cols, group;
    std::vector<uint8_t> packed;
    std::vector<float> scales, zeros;
};

QM quantize_minmax(const std::vector<float>& w, int rows, int cols, int group) {
    QM q{rows, cols, group, {}, {}, {}};
    const int gpr = (cols + group - 1) / group;
    q.packed.assign((static_cast<size_t>(rows) * cols + 1) / 2, 0);
    q.scales.assign(static_cast<size_t>(rows) * gpr, 1.0f);
    q.zeros.assign(static_cast<size_t>(rows) * gpr, 0.0f);
    for (int r = 0; r < rows; ++r)
        for (int g = 0; g < gpr; ++g) {
            const int c0 = g * group, c1 = std::min(cols, c0 + group);
            float lo = w[static_cast<size_t>(r) * cols + c0], hi = lo;
            for (int c = c0; c < c1; ++c) {
                lo = std::min(lo, w[static_cast<size_t>(r) * cols + c]);
                hi = std::max(hi, w[static_cast<size_t>(r) * cols + c]);
            }
            const float s = hi > lo ? (hi - lo) / 15.0f : 1.0f;
            const float z = hi > lo ? std::round(-lo / s) : 0.0f;
            q.scales[static_cast<size_t>(r) * gpr + g] = s;
            q.zeros[static_cast<size_t>(r) * gpr + g] = z;
            for (int c = c0; c < c1; ++c) {
                int code = static_cast<int>(std::round(w[static_cast<size_t>(r) * cols + c] / s + z));
                code = std::max(0, std::min(15, code));
                const size_t i = static_cast<size_t>(r) * cols + c;
                q.packed[i >> 1] |= static_cast<uint8_t>((i & 1) ? (code << 4) : code);
            }
        }
    return q;
}

}  // namespace

extern "C" XQ_API xq_status xq_run_vulkan_w4a16_selftest(char* json_out, size_t json_capacity) {
    using Clock = std::chrono::steady_clock;
    std::ostringstream js;
    const bool have_gpu = xqhip_device_count() > 0 && xqhip_set_device(0) == 0;
    char name[256] = {};
    if (have_gpu) xqhip_device_name(name, sizeof(name));
    js << "{\"engine\":\"customlib\",\"test\":\"vulkan_w4a16_gemv_correctness\",\"custom_backend_requested\":\"vulkan\","
       << "\"custom_backend_actual\":\"" << (have_gpu ? "hip" : "unavailable") << "\",\"vulkan_runtime_initialized\":false,"
       << "\"hip_runtime_initialized\":" << (have_gpu ? "true" : "false") << ",\"device_name\":\""
       << xqh::json_escape(name) << "\"";
    if (!have_gpu) {
        js << ",\"status\":\"error\",\"pass\":false,\"error\":\"no HIP device visible\"}";
        const std::string s = js.str();
        if (json_out && json_capacity) {
            const size_t n = std::min(json_capacity - 1, s.size());
            std::memcpy(json_out, s.data(), n);
            json_out[n] = '\0';
        }
        return XQ_ERR_RUNTIME;
    }
    struct Shape {
        int rows, cols;
        const char* name;
        double tol;
    };
    const Shape shapes[] = {{256, 256, "small_correctness", 1.0e-3}, {4096, 4096, "qwen_4096x4096", 2.0e-2}};
    bool all_pass = true;
    js << ",\"results\":[";
    for (size_t si = 0; si < 2; ++si) {
        const Shape& sh = shapes[si];
        std::vector<float> dense(static_cast<size_t>(sh.rows) * sh.cols), x(static_cast<size_t>(sh.cols));
        for (int r = 0; r < sh.rows; ++r)
            for (int c = 0; c < sh.cols; ++c) {
                const float a = std::sin(static_cast<float>((r * 17 + c * 13) % 997) * 0.013f);
                const float b = std::cos(static_cast<float>((r * 7 + c * 19) % 769) * 0.017f);
                dense[static_cast<size_t>(r) * sh.cols + c] = 0.20f * a + 0.05f * b;
            }
        for (int c = 0; c < sh.cols; ++c)
            x[c] = 0.15f * std::sin(static_cast<float>(c % 1021) * 0.011f) +
                   0.03f * std::cos(static_cast<float>(c % 577) * 0.019f);
        const QM q = quantize_minmax(dense, sh.rows, sh.cols, 64);
        const auto c0 = Clock::now();
        std::vector<double> ref(static_cast<size_t>(sh.rows));
        const int gpr = sh.cols / 64;
        for (int r = 0; r < sh.rows; ++r) {
            double acc = 0.0;
            for (int c = 0; c < sh.cols; ++c) {
                const size_t i = static_cast<size_t>(r) * sh.cols + c;
                const int code = (i & 1) ? (q.packed[i >> 1] >> 4) : (q.packed[i >> 1] & 15);
                const size_t m = static_cast<size_t>(r) * gpr + c / 64;
                acc += (code - static_cast<double>(q.zeros[m])) * q.scales[m] * x[c];
            }
            ref[r] = acc;
        }
        const double cpu_ms = std::chrono::duration<double, std::milli>(Clock::now() - c0).count();
        xqhip_w4 w{};
        void *xd = nullptr, *yd = nullptr;
        std::vector<float> y(static_cast<size_t>(sh.rows));
        const auto t0 = Clock::now();
        bool ok = xqhip_w4_upload(q.packed.data(), q.scales.data(), q.zeros.data(), sh.rows, sh.cols, 64, 0, &w) == 0 &&
                  xqhip_malloc(&xd, x.size() * 4) == 0 && xqhip_malloc(&yd, y.size() * 4) == 0 &&
                  xqhip_memcpy_h2d(xd, x.data(), x.size() * 4, nullptr) == 0;
        const auto t1 = Clock::now();
        ok = ok && xqhip_gemv_w4a16(&w, xd, XQHIP_F32, nullptr, yd, XQHIP_F32, XQHIP_EPI_STORE, nullptr) == 0 &&
             xqhip_device_synchronize() == 0;
        const auto t2 = Clock::now();
        ok = ok && xqhip_memcpy_d2h(y.data(), yd, y.size() * 4, nullptr) == 0;
        const auto t3 = Clock::now();
        std::string err = ok ? "" : xqhip_last_error();
        xqhip_w4_free(&w);
        xqhip_free(xd);
        xqhip_free(yd);
        double max_abs = 0.0, sum = 0.0;
        for (int r = 0; r < sh.rows && ok; ++r) {
            const double d = std::fabs(ref[r] - y[r]);
            max_abs = std::max(max_abs, d);
            sum += d;
        }
        const bool pass = ok && max_abs <= sh.tol && std::isfinite(max_abs);
        all_pass = all_pass && pass;
        auto ms = [](Clock::time_point a, Clock::time_point b) {
            return std::chrono::duration<double, std::milli>(b - a).count();
        };
        js << (si ? "," : "") << "{\"name\":\"" << sh.name << "\",\"shape\":\"" << sh.rows << "x" << sh.cols
           << "\",\"backend\":\"hip\",\"rows\":" << sh.rows << ",\"cols\":" << sh.cols
           << ",\"group_size\":64,\"cpu_reference_ms\":" << cpu_ms << ",\"upload_ms\":" << ms(t0, t1)
           << ",\"dispatch_ms\":" << ms(t1, t2) << ",\"download_ms\":" << ms(t2, t3) << ",\"total_ms\":" << ms(t0, t3)
           << ",\"max_abs_error\":" << max_abs << ",\"mean_abs_error\":" << (ok ? sum / sh.rows : 0.0)
           << ",\"tolerance\":" << sh.tol << ",\"pass\":" << (pass ? "true" : "false");
        if (!ok) js << ",\"error\":\"" << xqh::json_escape(err) << "\"";
        js << "}";
    }
    js << "],\"status\":\"" << (all_pass ? "ok" : "error") << "\",\"pass\":" << (all_pass ? "true" : "false") << "}";
    const std::string s = js.str();
    if (!json_out || json_capacity == 0) return XQ_ERR_INVALID_ARGUMENT;
    if (s.size() + 1 > json_capacity) return XQ_ERR_BUFFER_TOO_SMALL;
    std::memcpy(json_out, s.c_str(), s.size() + 1);
    return all_pass ? XQ_OK : XQ_ERR_RUNTIME;
}
