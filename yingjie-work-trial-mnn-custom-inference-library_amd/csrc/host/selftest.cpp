// selftest.cpp - xq_run_vulkan_w4a16_selftest on the HIP device.
//
// Same deterministic workload, shapes, tolerances and JSON layout as the
// reference's GPU self-test (customlib/runtime/vulkan_backend.cpp:1638-2029):
//   results         W4A16 GEMV 256x256 (tol 1e-3) and 4096x4096 (tol 2e-2) on
//                   dense weights 0.20 sin(((17r+13c) mod 997) 0.013) +
//                   0.05 cos(((7r+19c) mod 769) 0.017), min/max 4-bit group-64
//                   quantisation (kernels/reference/ref_gemv.cpp:38-75), input
//                   0.15 sin((c mod 1021) 0.011) + 0.03 cos((c mod 577) 0.019)
//                   (vulkan_backend.cpp:65-86); expected = float64 dequantised dot
//   vector_results  the element-wise ops (:1723-2022), each run through the kernel
//                   this library uses for it.  The decode path fuses several of
//                   them into a neighbour, so those are checked in that form:
//                   SiLU*up and the residual add as GEMV epilogues (against the
//                   plain GEMV output), RoPE behind the per-head RMSNorm of the
//                   q/k preparation kernel (norm weights 0.01, so the fp16 key
//                   cache holds the result well inside the tolerance), the
//                   conv1d with the L2 norm of its q/k heads, greedy argmax as
//                   the lm_head GEMV + argmax, GQA over the fp16 KV cache
//                   (expected values computed from the fp16-rounded cache).
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <functional>
#include <limits>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "kernel_trace.hpp"
#include "xqhip.h"
#include "xqwen35.h"

namespace {

using Clock = std::chrono::steady_clock;
double ms_between(Clock::time_point a, Clock::time_point b) {
    return std::chrono::duration<double, std::milli>(b - a).count();
}

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

QM det_matrix(int rows, int cols) {
    std::vector<float> dense(static_cast<size_t>(rows) * cols);
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) {
            const float a = std::sin(static_cast<float>((r * 17 + c * 13) % 997) * 0.013f);
            const float b = std::cos(static_cast<float>((r * 7 + c * 19) % 769) * 0.017f);
            dense[static_cast<size_t>(r) * cols + c] = 0.20f * a + 0.05f * b;
        }
    return quantize_minmax(dense, rows, cols, 64);
}

std::vector<float> det_input(int n) {
    std::vector<float> x(static_cast<size_t>(n));
    for (int c = 0; c < n; ++c)
        x[c] = 0.15f * std::sin(static_cast<float>(c % 1021) * 0.011f) +
               0.03f * std::cos(static_cast<float>(c % 577) * 0.019f);
    return x;
}

// fp32 <-> fp16 bit conversions (round to nearest even) for the KV-cache checks.
uint16_t to_half(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const int32_t e = static_cast<int32_t>((u >> 23) & 0xff) - 112;
    uint32_t m = u & 0x7fffffu;
    if (e >= 31) return static_cast<uint16_t>(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return static_cast<uint16_t>(sign);
        m |= 0x800000u;
        const int sh = 14 - e;
        uint32_t h = m >> sh;
        const uint32_t rem = m & ((1u << sh) - 1), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (h & 1))) ++h;
        return static_cast<uint16_t>(sign | h);
    }
    uint32_t h = (static_cast<uint32_t>(e) << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) ++h;
    return static_cast<uint16_t>(sign | h);
}
float from_half(uint16_t h) {
    const uint32_t e = (h >> 10) & 31, m = h & 1023u;
    const float v = e == 0 ? std::ldexp(static_cast<float>(m), -24)
                           : (e == 31 ? (m ? NAN : INFINITY) : std::ldexp(static_cast<float>(m | 1024u), int(e) - 25));
    return (h & 0x8000u) ? -v : v;
}

struct Diff {
    double max_abs = 0.0, mean_abs = 0.0;
};
Diff compare(const std::vector<float>& want, const std::vector<float>& got) {
    Diff d;
    const size_t n = std::min(want.size(), got.size());
    double sum = 0.0;
    for (size_t i = 0; i < n; ++i) {
        const double e = std::fabs(static_cast<double>(want[i]) - static_cast<double>(got[i]));
        d.max_abs = std::max(d.max_abs, e);
        sum += e;
    }
    d.mean_abs = n ? sum / static_cast<double>(n) : 0.0;
    return d;
}

// ---- device plumbing: failures throw with the library's error text ----------
void ck(int rc) {
    if (rc != 0) throw std::runtime_error(xqhip_last_error());
}
struct Buf {
    void* p = nullptr;
    explicit Buf(size_t bytes) { ck(xqhip_malloc(&p, std::max<size_t>(bytes, 4))); }
    ~Buf() { xqhip_free(p); }
    Buf(const Buf&) = delete;
    Buf& operator=(const Buf&) = delete;
    float* f() const { return static_cast<float*>(p); }
};
template <typename T>
void put(const Buf& b, const std::vector<T>& v) {
    ck(xqhip_memcpy_h2d(b.p, v.data(), v.size() * sizeof(T), nullptr));
}
template <typename T>
std::vector<T> get(const Buf& b, size_t n) {
    std::vector<T> v(n);
    ck(xqhip_memcpy_d2h(v.data(), b.p, n * sizeof(T), nullptr));
    return v;
}
struct W4 {
    xqhip_w4 w{};
    explicit W4(const QM& q) { ck(xqhip_w4_upload(q.packed.data(), q.scales.data(), q.zeros.data(), q.rows, q.cols, 64, 0, &w)); }
    ~W4() { xqhip_w4_free(&w); }
};

struct Timing {
    double upload = 0, dispatch = 0, download = 0;
};
// Times the three phases of one check: host->device, kernels (synchronised), device->host.
struct Phases {
    Timing t;
    Clock::time_point mark = Clock::now();
    void lap(double* into) {
        const auto now = Clock::now();
        *into += ms_between(mark, now);
        mark = now;
    }
    void uploaded() { lap(&t.upload); }
    void dispatched() {
        ck(xqhip_device_synchronize());
        lap(&t.dispatch);
    }
    void downloaded() { lap(&t.download); }
};

struct VecResult {
    std::string name, kernel;
    Diff diff;
    double tol;
    Timing t;
    std::string error;
};

// ---- the vector checks ------------------------------------------------------

VecResult rmsnorm_check() {
    const int n = 1024;
    const std::vector<float> x = det_input(n);
    std::vector<float> w(n), want(n);
    for (int i = 0; i < n; ++i) w[i] = 0.8f + 0.001f * static_cast<float>(i % 17);
    double ss = 0.0;
    for (float v : x) ss += static_cast<double>(v) * v;
    const float inv = 1.0f / std::sqrt(static_cast<float>(ss / n) + 1.0e-6f);
    for (int i = 0; i < n; ++i) want[i] = x[i] * inv * w[i];
    Phases ph;
    Buf xd(n * 4), wd(n * 4), yd(n * 4);
    put(xd, x);
    put(wd, w);
    ph.uploaded();
    ck(xqhip_rmsnorm(xd.f(), wd.f(), n, 1.0e-6f, yd.f(), nullptr));
    ph.dispatched();
    const std::vector<float> got = get<float>(yd, n);
    ph.downloaded();
    return {"rmsnorm_vector", "rmsnorm", compare(want, got), 1.0e-4, ph.t, ""};
}

VecResult rope_check() {
    const int nq = 2, nkv = 1, hd = 16, rd = 8, pos = 7;
    const float theta = 1.0e7f, eps = 1.0e-6f, nw = 0.01f;
    const std::vector<float> q = det_input(nq * hd), k = det_input(nkv * hd), v = det_input(nkv * hd);
    // expected: per-head RMSNorm (weights nw) then RoPE on the first rd dims, pairs (i, rd/2 + i)
    auto prep = [&](std::vector<float> x, int heads) {
        for (int h = 0; h < heads; ++h) {
            float* b = x.data() + h * hd;
            double ss = 0.0;
            for (int d = 0; d < hd; ++d) ss += static_cast<double>(b[d]) * b[d];
            const float inv = 1.0f / std::sqrt(static_cast<float>(ss / hd) + eps);
            for (int d = 0; d < hd; ++d) b[d] = b[d] * inv * nw;
            const int half = rd / 2;
            for (int i = 0; i < half; ++i) {
                const float ang = static_cast<float>(pos) * std::pow(theta, -static_cast<float>(2 * i) / rd);
                const float c = std::cos(ang), s = std::sin(ang), x0 = b[i], x1 = b[half + i];
                b[i] = x0 * c - x1 * s;
                b[half + i] = x1 * c + x0 * s;
            }
        }
        return x;
    };
    std::vector<float> want = prep(q, nq);
    const std::vector<float> kw = prep(k, nkv);
    want.insert(want.end(), kw.begin(), kw.end());
    std::vector<float> cs(2 * static_cast<size_t>(pos + 1) * (rd / 2));
    ck(xqhip_rope_table(theta, rd, pos + 1, cs.data()));
    const std::vector<float> norm(hd, nw);
    const std::vector<int32_t> p{pos};
    const size_t cache = static_cast<size_t>(pos + 1) * nkv * hd;
    Phases ph;
    Buf qd(q.size() * 4), kd(k.size() * 4), vd(v.size() * 4), csd(cs.size() * 4), nd(hd * 4), pd(4), qo(q.size() * 4),
        go(q.size() * 4), kc(cache * 2), vc(cache * 2);
    put(qd, q);
    put(kd, k);
    put(vd, v);
    put(csd, cs);
    put(nd, norm);
    put(pd, p);
    ph.uploaded();
    ck(xqhip_attn_prep(qd.f(), kd.f(), vd.f(), 0, nq, nkv, hd, rd, nd.f(), nd.f(), eps, csd.f(),
                       static_cast<const int32_t*>(pd.p), qo.f(), go.f(), kc.p, vc.p, nullptr));
    ph.dispatched();
    std::vector<float> got = get<float>(qo, q.size());
    const std::vector<uint16_t> kh = get<uint16_t>(kc, cache);
    ph.downloaded();
    for (int d = 0; d < nkv * hd; ++d) got.push_back(from_half(kh[static_cast<size_t>(pos) * nkv * hd + d]));
    return {"rope_qk_vector", "qk_norm_rope_kv_append", compare(want, got), 1.0e-4, ph.t, ""};
}

// gate/up interleaved rows, plain GEMV vs the SiLU-pair epilogue
VecResult silu_mul_check() {
    const int n = 2048, cols = 256;
    const QM q = det_matrix(2 * n, cols);
    const std::vector<float> x = det_input(cols);
    Phases ph;
    W4 w(q);
    Buf xd(cols * 4), yd(2 * n * 4), zd(n * 4);
    put(xd, x);
    ph.uploaded();
    ck(xqhip_gemv_w4a16(&w.w, xd.p, XQHIP_F32, nullptr, yd.p, XQHIP_F32, XQHIP_EPI_STORE, nullptr));
    ck(xqhip_gemv_w4a16(&w.w, xd.p, XQHIP_F32, nullptr, zd.p, XQHIP_F32, XQHIP_EPI_SILU_PAIR, nullptr));
    ph.dispatched();
    const std::vector<float> y = get<float>(yd, 2 * n), got = get<float>(zd, n);
    ph.downloaded();
    std::vector<float> want(n);
    for (int i = 0; i < n; ++i) {
        const float g = y[2 * i], u = y[2 * i + 1];
        want[i] = g / (1.0f + std::exp(-g)) * u;
    }
    return {"silu_gate_mul_vector", "gemv_w4a16_epilogue_silu_pair", compare(want, got), 1.0e-5, ph.t, ""};
}

// plain GEMV vs the residual-add epilogue onto a hidden vector
VecResult residual_check() {
    const int n = 2048, cols = 256;
    const QM q = det_matrix(n, cols);
    const std::vector<float> x = det_input(cols), hidden = det_input(n);
    Phases ph;
    W4 w(q);
    Buf xd(cols * 4), yd(n * 4), hd(n * 4);
    put(xd, x);
    put(hd, hidden);
    ph.uploaded();
    ck(xqhip_gemv_w4a16(&w.w, xd.p, XQHIP_F32, nullptr, yd.p, XQHIP_F32, XQHIP_EPI_STORE, nullptr));
    ck(xqhip_gemv_w4a16(&w.w, xd.p, XQHIP_F32, nullptr, hd.p, XQHIP_F32, XQHIP_EPI_ADD, nullptr));
    ph.dispatched();
    const std::vector<float> y = get<float>(yd, n), got = get<float>(hd, n);
    ph.downloaded();
    std::vector<float> want = hidden;
    for (int i = 0; i < n; ++i) want[i] += y[i];
    return {"residual_add_vector", "gemv_w4a16_epilogue_add", compare(want, got), 1.0e-6, ph.t, ""};
}

VecResult gqa_check() {
    const int ctx = 5, nq = 4, nkv = 2, hd = 8;
    const std::vector<float> q = det_input(nq * hd), kv = det_input(ctx * nkv * hd);
    std::vector<uint16_t> kvh(kv.size());
    std::vector<float> kvr(kv.size());  // what the fp16 cache holds
    for (size_t i = 0; i < kv.size(); ++i) {
        kvh[i] = to_half(kv[i]);
        kvr[i] = from_half(kvh[i]);
    }
    std::vector<float> want(static_cast<size_t>(nq) * hd, 0.0f), sc(ctx);
    const int group = std::max(1, nq / nkv);
    const float scale = 1.0f / std::sqrt(static_cast<float>(hd));
    for (int h = 0; h < nq; ++h) {
        const int kh = std::min(nkv - 1, h / group);
        float mx = -std::numeric_limits<float>::infinity();
        for (int t = 0; t < ctx; ++t) {
            float dot = 0.0f;
            for (int d = 0; d < hd; ++d) dot += q[h * hd + d] * kvr[(t * nkv + kh) * hd + d];
            sc[t] = dot * scale;
            mx = std::max(mx, sc[t]);
        }
        float den = 0.0f;
        for (int t = 0; t < ctx; ++t) den += (sc[t] = std::exp(sc[t] - mx));
        for (int t = 0; t < ctx; ++t)
            for (int d = 0; d < hd; ++d) want[h * hd + d] += sc[t] / den * kvr[(t * nkv + kh) * hd + d];
    }
    const std::vector<float> open_gate(static_cast<size_t>(nq) * hd, 40.0f);  // sigmoid(40) == 1 in fp32
    const std::vector<int32_t> p{ctx - 1};
    Phases ph;
    Buf qd(q.size() * 4), kc(kvh.size() * 2), vc(kvh.size() * 2), gd(open_gate.size() * 4), pd(4),
        od(q.size() * 4), ws(xqhip_gqa_workspace_bytes(nq, nkv, hd));
    put(qd, q);
    put(kc, kvh);
    put(vc, kvh);
    put(gd, open_gate);
    put(pd, p);
    ph.uploaded();
    ck(xqhip_gqa_decode(qd.f(), kc.p, vc.p, gd.f(), nq, nkv, hd, ctx, static_cast<const int32_t*>(pd.p), od.f(), ws.p,
                        nullptr));
    ph.dispatched();
    const std::vector<float> got = get<float>(od, q.size());
    ph.downloaded();
    return {"gqa_decode_vector", "gqa_decode_fp16_kv", compare(want, got), 1.0e-4, ph.t, ""};
}

// conv1d + SiLU with the cache shift; channels 0-15 / 16-31 are one q / k head, L2-normalised
VecResult conv_check() {
    const int lk_n = 1, lk_hd = 16, lv_n = 4, lv_hd = 16, ks = 4, hist = ks - 1;
    const int conv = 2 * lk_n * lk_hd + lv_n * lv_hd;  // 96 channels
    const std::vector<float> in = det_input(conv), state = det_input(conv * hist), w = det_input(conv * ks);
    std::vector<float> out(conv), st = state;
    for (int c = 0; c < conv; ++c) {
        float acc = 0.0f;
        for (int k = 0; k < hist; ++k) acc += state[c * hist + k] * w[c * ks + k];
        acc += in[c] * w[c * ks + hist];
        out[c] = acc / (1.0f + std::exp(-acc));
        for (int k = 0; k < hist; ++k) st[c * hist + k] = k + 1 < hist ? state[c * hist + k + 1] : in[c];
    }
    for (int h = 0; h < 2 * lk_n; ++h) {
        float ss = 0.0f;
        for (int d = 0; d < lk_hd; ++d) ss += out[h * lk_hd + d] * out[h * lk_hd + d];
        const float inv = 1.0f / std::sqrt(ss + 1.0e-6f);
        for (int d = 0; d < lk_hd; ++d) out[h * lk_hd + d] *= inv;
    }
    std::vector<float> want = out;
    want.insert(want.end(), st.begin(), st.end());
    Phases ph;
    Buf id(conv * 4), sd(state.size() * 4), wd(w.size() * 4), od(conv * 4);
    put(id, in);
    put(sd, state);
    put(wd, w);
    ph.uploaded();
    ck(xqhip_linear_conv(id.f(), sd.f(), wd.f(), lk_n, lk_hd, lv_n, lv_hd, ks, od.f(), nullptr));
    ph.dispatched();
    std::vector<float> got = get<float>(od, conv);
    const std::vector<float> gst = get<float>(sd, state.size());
    ph.downloaded();
    got.insert(got.end(), gst.begin(), gst.end());
    return {"linear_attention_conv1d_vector", "linear_conv_l2norm", compare(want, got), 1.0e-5, ph.t, ""};
}

VecResult delta_check() {
    const int lk_n = 2, lv_n = 4, dk = 8, dv = 8;
    const std::vector<float> conv = det_input(2 * lk_n * dk + lv_n * dv), a = det_input(lv_n), b = det_input(lv_n);
    std::vector<float> a_log(lv_n), dt(lv_n);
    for (int i = 0; i < lv_n; ++i) {
        a_log[i] = -0.7f + 0.02f * static_cast<float>(i);
        dt[i] = 0.03f * static_cast<float>(i - 1);
    }
    const std::vector<float> state = det_input(lv_n * dk * dv);
    std::vector<float> st = state, out(static_cast<size_t>(lv_n) * dv);
    const int factor = std::max(1, lv_n / lk_n);
    for (int vh = 0; vh < lv_n; ++vh) {  // gated delta rule (kernels/reference/ref_delta.cpp:8-41)
        const int kh = std::min(lk_n - 1, vh / factor);
        const float* qv = conv.data() + kh * dk;
        const float* kv = conv.data() + lk_n * dk + kh * dk;
        const float* vv = conv.data() + 2 * lk_n * dk + vh * dv;
        const float beta = 1.0f / (1.0f + std::exp(-b[vh]));
        const float decay = std::exp(-std::exp(a_log[vh]) * std::log(1.0f + std::exp(a[vh] + dt[vh])));
        float* S = st.data() + static_cast<size_t>(vh) * dk * dv;
        for (int i = 0; i < dk * dv; ++i) S[i] *= decay;
        for (int j = 0; j < dv; ++j) {
            float pred = 0.0f;
            for (int i = 0; i < dk; ++i) pred += S[i * dv + j] * kv[i];
            const float delta = beta * (vv[j] - pred);
            for (int i = 0; i < dk; ++i) S[i * dv + j] += kv[i] * delta;
        }
        const float scale = 1.0f / std::sqrt(static_cast<float>(dk));
        for (int j = 0; j < dv; ++j) {
            float acc = 0.0f;
            for (int i = 0; i < dk; ++i) acc += S[i * dv + j] * qv[i] * scale;
            out[vh * dv + j] = acc;
        }
    }
    std::vector<float> want = out;
    want.insert(want.end(), st.begin(), st.end());
    Phases ph;
    Buf cd(conv.size() * 4), ad(lv_n * 4), bd(lv_n * 4), ld(lv_n * 4), dd(lv_n * 4), sd(state.size() * 4),
        od(out.size() * 4);
    put(cd, conv);
    put(ad, a);
    put(bd, b);
    put(ld, a_log);
    put(dd, dt);
    put(sd, state);
    ph.uploaded();
    ck(xqhip_gated_delta(cd.f(), ad.f(), bd.f(), ld.f(), dd.f(), sd.f(), lk_n, lv_n, dk, dv, od.f(), nullptr));
    ph.dispatched();
    std::vector<float> got = get<float>(od, out.size());
    const std::vector<float> gst = get<float>(sd, state.size());
    ph.downloaded();
    got.insert(got.end(), gst.begin(), gst.end());
    return {"linear_attention_state_update_vector", "gated_delta", compare(want, got), 1.0e-4, ph.t, ""};
}

VecResult append_check() {
    const std::vector<float> old_v = det_input(17), add = det_input(9);
    std::vector<float> want = old_v;
    want.insert(want.end(), add.begin(), add.end());
    Phases ph;
    Buf od(old_v.size() * 4), ad(add.size() * 4), dst(want.size() * 4);
    put(od, old_v);
    put(ad, add);
    ph.uploaded();
    // the appended part lands at a 68-byte offset: a runtime copy, not the 16-byte copy kernel
    ck(xqhip_memcpy_d2d(dst.p, od.p, old_v.size() * 4, nullptr));
    ck(xqhip_memcpy_d2d(static_cast<char*>(dst.p) + old_v.size() * 4, ad.p, add.size() * 4, nullptr));
    ph.dispatched();
    const std::vector<float> got = get<float>(dst, want.size());
    ph.downloaded();
    return {"append_vector", "device_copy", compare(want, got), 1.0e-6, ph.t, ""};
}

// greedy argmax as the lm_head runs it: GEMV + argmax over 2048 rows, one row
// (1337) boosted to the top; checked against the plain GEMV output's first maximum
VecResult argmax_check() {
    const int n = 2048, cols = 256;
    QM q = det_matrix(n, cols);
    for (int g = 0; g < cols / 64; ++g) q.scales[1337 * (cols / 64) + g] *= 8.0f;
    const std::vector<float> x = det_input(cols);
    Phases ph;
    W4 w(q);
    Buf xd(cols * 4), yd(n * 4), ws(xqhip_argmax_workspace_bytes(n)), idx(4), val(4);
    put(xd, x);
    ph.uploaded();
    ck(xqhip_gemv_w4a16(&w.w, xd.p, XQHIP_F32, nullptr, yd.p, XQHIP_F32, XQHIP_EPI_STORE, nullptr));
    ck(xqhip_gemv_w4a16_argmax(&w.w, xd.p, XQHIP_F32, nullptr, ws.p, static_cast<int32_t*>(idx.p), val.f(), nullptr));
    ph.dispatched();
    const std::vector<float> y = get<float>(yd, n);
    const int32_t gi = get<int32_t>(idx, 1)[0];
    const float gv = get<float>(val, 1)[0];
    ph.downloaded();
    int best = 0;
    for (int i = 1; i < n; ++i)
        if (y[i] > y[best]) best = i;
    Diff d;
    d.max_abs = d.mean_abs = (gi == best && best == 1337) ? std::fabs(static_cast<double>(gv) - y[best]) : 1.0e9;
    return {"argmax_vector", "gemv_w4a16_argmax", d, 1.0e-5, ph.t, ""};
}

VecResult guarded(const char* name, const std::function<VecResult()>& f) {
    try {
        return f();
    } catch (const std::exception& e) {
        return {name, "", Diff{}, 0.0, Timing{}, e.what()};
    }
}

}  // namespace

extern "C" XQ_API xq_status xq_run_vulkan_w4a16_selftest(char* json_out, size_t json_capacity) {
    const auto start = Clock::now();
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
        const QM q = det_matrix(sh.rows, sh.cols);
        const std::vector<float> x = det_input(sh.cols);
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
        const double cpu_ms = ms_between(c0, Clock::now());
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
        js << (si ? "," : "") << "{\"name\":\"" << sh.name << "\",\"shape\":\"" << sh.rows << "x" << sh.cols
           << "\",\"backend\":\"hip\",\"rows\":" << sh.rows << ",\"cols\":" << sh.cols
           << ",\"group_size\":64,\"cpu_reference_ms\":" << cpu_ms << ",\"upload_ms\":" << ms_between(t0, t1)
           << ",\"dispatch_ms\":" << ms_between(t1, t2) << ",\"download_ms\":" << ms_between(t2, t3)
           << ",\"total_ms\":" << ms_between(t0, t3) << ",\"max_abs_error\":" << max_abs
           << ",\"mean_abs_error\":" << (ok ? sum / sh.rows : 0.0) << ",\"tolerance\":" << sh.tol
           << ",\"pass\":" << (pass ? "true" : "false");
        if (!ok) js << ",\"error\":\"" << xqh::json_escape(err) << "\"";
        js << "}";
    }
    js << "],\"vector_results\":[";
    const std::vector<VecResult> vec = {
        guarded("rmsnorm_vector", rmsnorm_check),
        guarded("rope_qk_vector", rope_check),
        guarded("silu_gate_mul_vector", silu_mul_check),
        guarded("residual_add_vector", residual_check),
        guarded("gqa_decode_vector", gqa_check),
        guarded("linear_attention_conv1d_vector", conv_check),
        guarded("linear_attention_state_update_vector", delta_check),
        guarded("append_vector", append_check),
        guarded("argmax_vector", argmax_check),
    };
    for (size_t i = 0; i < vec.size(); ++i) {
        const VecResult& r = vec[i];
        const bool ok = r.error.empty();
        const bool pass = ok && r.diff.max_abs <= r.tol && std::isfinite(r.diff.max_abs);
        all_pass = all_pass && pass;
        js << (i ? "," : "") << "{\"name\":\"" << r.name << "\",\"backend\":\"hip\",\"kernel\":\"" << r.kernel
           << "\",\"upload_ms\":" << r.t.upload << ",\"dispatch_ms\":" << r.t.dispatch
           << ",\"download_ms\":" << r.t.download << ",\"total_ms\":" << r.t.upload + r.t.dispatch + r.t.download
           << ",\"max_abs_error\":" << r.diff.max_abs << ",\"mean_abs_error\":" << r.diff.mean_abs
           << ",\"tolerance\":" << r.tol << ",\"pass\":" << (pass ? "true" : "false");
        if (!ok) js << ",\"error\":\"" << xqh::json_escape(r.error) << "\"";
        js << "}";
    }
    js << "],\"wall_clock_ms\":" << ms_between(start, Clock::now()) << ",\"status\":\"" << (all_pass ? "ok" : "error")
       << "\",\"pass\":" << (all_pass ? "true" : "false") << "}";
    const std::string s = js.str();
    if (!json_out || json_capacity == 0) return XQ_ERR_INVALID_ARGUMENT;
    if (s.size() + 1 > json_capacity) return XQ_ERR_BUFFER_TOO_SMALL;
    std::memcpy(json_out, s.c_str(), s.size() + 1);
    return all_pass ? XQ_OK : XQ_ERR_RUNTIME;
}
