// oracle.cpp - CPU restatement of the reference's W4A16 group-64 batch-1 decode path.
//
// TEST INFRASTRUCTURE ONLY.  This file is the checker: it is loaded by tests/,
// by __graft_entry__.smoke() and by the cpu_baseline leg of bench.py, and by
// nothing else.  The product library never links it and has no CPU fallback.
//
// Every function restates the arithmetic of the reference file:line it cites,
// in the same operation order, so that when it is compiled like the reference
// (-std=c++17 -O3, baseline x86-64, -ffp-contract=off, no fast-math) its float
// results are bit-identical to the compiled reference on the same host libm.
// Reference paths are relative to the reference checkout root.
//
// Pins (see tests/test_oracle_*.py):
//   gemv / rmsnorm / gqa / gated-delta : published microbench checksums
//       (results/reports/evidence/customlib_cpu_vulkan_hybrid_benchmark_v27.json)
//       and bit-exact agreement with the compiled reference (oracle/_ref).
//   nibble unpack : hand-packed KAT + brute force against the bit-level reader.
//   model forward : bit-exact token ids and hidden state against the compiled
//       reference session on the same synthetic model files.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <functional>
#include <limits>
#include <memory>
#include <mutex>
#include <sstream>
#include <string>
#include <thread>
#include <vector>

namespace orc {

// ---------------------------------------------------------------------------
// scalar helpers: customlib/runtime/custom_model.cpp:264-292
// ---------------------------------------------------------------------------
static float bf16_to_f32(uint16_t v) {  // custom_model.cpp:264-269
    uint32_t bits = static_cast<uint32_t>(v) << 16;
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

static float silu_f(float x) { return x / (1.0f + std::exp(-x)); }  // custom_model.cpp:271-273

static float sigmoid_f(float x) {  // custom_model.cpp:275-282 (two-branch, overflow safe)
    if (x >= 0.0f) {
        const float e = std::exp(-x);
        return 1.0f / (1.0f + e);
    }
    const float e = std::exp(x);
    return e / (1.0f + e);
}

static float softplus_f(float x) {  // custom_model.cpp:284-292
    if (x > 20.0f) return x;
    if (x < -20.0f) return std::exp(x);
    return std::log1p(std::exp(x));
}

// ---------------------------------------------------------------------------
// Quantized matrix: customlib/kernels/kernels.hpp:11-21
// packed[rows][ceil(cols/2)] with the even column in the low nibble,
// scales/zeros[rows][groups] fp32.  version 1 (symmetric form, w=(q-z)*s),
// version 2 (affine, w=q*s+z).
// ---------------------------------------------------------------------------
struct QMat {
    int rows = 0, cols = 0, group = 64, bits = 4;
    bool affine = false;
    std::vector<uint8_t> packed;
    std::vector<float> scales, zeros;
    int groups() const { return (cols + group - 1) / group; }
    size_t row_bytes() const { return (static_cast<size_t>(cols) + 1) / 2; }
};

// Bit-level reader: customlib/kernels/reference/ref_gemv.cpp:10-18 (LSB first).
static uint32_t read_code_bits(const uint8_t* bytes, size_t bit_off, int bits) {
    uint32_t v = 0;
    for (int i = 0; i < bits; ++i) {
        const size_t p = bit_off + static_cast<size_t>(i);
        v |= static_cast<uint32_t>((bytes[p >> 3] >> (p & 7)) & 1u) << i;
    }
    return v;
}

// ref_gemv.cpp:77-87
static float dequant_one(const QMat& m, int r, int c) {
    const size_t bit_off = (static_cast<size_t>(r) * m.cols + c) * m.bits;
    const uint32_t code = read_code_bits(m.packed.data(), bit_off, m.bits);
    const size_t meta = static_cast<size_t>(r) * m.groups() + c / m.group;
    if (m.affine) return static_cast<float>(code) * m.scales[meta] + m.zeros[meta];
    return (static_cast<float>(code) - m.zeros[meta]) * m.scales[meta];
}

// ref_gemv.cpp:38-75 (min/max asymmetric quantizer used by the reference's
// tests and microbench generators; writes version-1 form).
static void quantize_lowbit(const float* w, int rows, int cols, int bits, int group, QMat* q) {
    q->rows = rows;
    q->cols = cols;
    q->bits = bits;
    q->group = group;
    q->affine = false;
    const int qmax = (1 << bits) - 1;
    const int g_n = (cols + group - 1) / group;
    q->scales.assign(static_cast<size_t>(rows) * g_n, 1.0f);
    q->zeros.assign(static_cast<size_t>(rows) * g_n, 0.0f);
    q->packed.assign((static_cast<size_t>(rows) * cols * bits + 7) / 8, 0);
    for (int r = 0; r < rows; ++r) {
        const float* wr = w + static_cast<size_t>(r) * cols;
        for (int g = 0; g < g_n; ++g) {
            const int c0 = g * group, c1 = std::min(cols, c0 + group);
            float lo = wr[c0], hi = wr[c0];
            for (int c = c0; c < c1; ++c) {
                lo = std::min(lo, wr[c]);
                hi = std::max(hi, wr[c]);
            }
            const float s = hi > lo ? (hi - lo) / static_cast<float>(qmax) : 1.0f;
            const float z = hi > lo ? std::round(-lo / s) : 0.0f;
            q->scales[static_cast<size_t>(r) * g_n + g] = s;
            q->zeros[static_cast<size_t>(r) * g_n + g] = z;
            for (int c = c0; c < c1; ++c) {
                const float t = wr[c] / s + z;
                int code = static_cast<int>(std::round(t));
                code = std::max(0, std::min(qmax, code));
                const size_t bit_off = (static_cast<size_t>(r) * cols + c) * bits;
                for (int i = 0; i < bits; ++i) {
                    const size_t p = bit_off + i;
                    const uint8_t mask = static_cast<uint8_t>(1u << (p & 7));
                    if ((static_cast<uint32_t>(code) >> i) & 1u)
                        q->packed[p >> 3] = static_cast<uint8_t>(q->packed[p >> 3] | mask);
                    else
                        q->packed[p >> 3] = static_cast<uint8_t>(q->packed[p >> 3] & ~mask);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Row-parallel pool with the reference's partition rules
// (customlib/kernels/generated/arm64_neon/xq_gemv_w4a16_neon.cpp:117-222):
// min(8, hardware_concurrency) threads, chunked dynamic row ranges.  Row
// results do not depend on the partition; it only matters for timing.
// ---------------------------------------------------------------------------
class RowPool {
public:
    explicit RowPool(int n) {
        for (int i = 1; i < n; ++i) threads_.emplace_back([this] { loop(); });
    }
    ~RowPool() {
        {
            std::lock_guard<std::mutex> g(mu_);
            stop_ = true;
            ++epoch_;
        }
        cv_.notify_all();
        for (auto& t : threads_) t.join();
    }
    int size() const { return static_cast<int>(threads_.size()) + 1; }
    void run(int begin, int end, int min_rows, const std::function<void(int, int)>& body) {
        const int count = end - begin;
        if (count <= 0) return;
        const int want = std::min(size(), std::max(1, (count + min_rows - 1) / min_rows));
        if (want <= 1) {
            body(begin, end);
            return;
        }
        std::atomic<int> cursor{begin};
        const int chunk = std::max(min_rows, (count + want * 4 - 1) / (want * 4));
        std::function<void()> job = [&] {
            for (;;) {
                const int r0 = cursor.fetch_add(chunk);
                if (r0 >= end) break;
                body(r0, std::min(end, r0 + chunk));
            }
        };
        {
            std::lock_guard<std::mutex> g(mu_);
            job_ = &job;
            pending_ = want - 1;
            helpers_ = want - 1;
            ++epoch_;
        }
        cv_.notify_all();
        job();
        std::unique_lock<std::mutex> lk(mu_);
        done_.wait(lk, [&] { return pending_ == 0; });
        job_ = nullptr;
    }

private:
    void loop() {
        uint64_t seen = 0;
        for (;;) {
            std::function<void()>* j = nullptr;
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [&] { return stop_ || (epoch_ != seen && helpers_ > 0); });
                if (stop_) return;
                seen = epoch_;
                --helpers_;
                j = job_;
            }
            (*j)();
            std::lock_guard<std::mutex> g(mu_);
            if (--pending_ == 0) done_.notify_one();
        }
    }
    std::vector<std::thread> threads_;
    std::mutex mu_;
    std::condition_variable cv_, done_;
    std::function<void()>* job_ = nullptr;
    int pending_ = 0, helpers_ = 0;
    uint64_t epoch_ = 0;
    bool stop_ = false;
};

static int g_pool_threads = -1;  // <0: reference default min(8, hw)
static std::unique_ptr<RowPool> g_pool;
static std::mutex g_pool_mu;

static RowPool& pool() {
    std::lock_guard<std::mutex> g(g_pool_mu);
    if (!g_pool) {
        int n = g_pool_threads;
        if (n <= 0) {
            const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
            n = static_cast<int>(std::min(8u, hw));
        }
        g_pool.reset(new RowPool(n));
    }
    return *g_pool;
}

// ---------------------------------------------------------------------------
// Fused W4A16 GEMV, scalar branch of
// customlib/kernels/generated/arm64_neon/xq_gemv_w4a16_neon.cpp:
//   per-group x sums (:224-232, :25-31), per-row accumulation (:234-255) with the
//   codes-only nibble dot (:61-71): low nibble first, then high nibble.
// ---------------------------------------------------------------------------
static void group_sums(const QMat& m, const float* x, std::vector<float>* sums) {
    const int g_n = m.groups();
    sums->resize(g_n);
    for (int g = 0; g < g_n; ++g) {
        const int c0 = g * m.group;
        const int n = std::min(m.group, m.cols - c0);
        float s = 0.0f;
        for (int c = 0; c < n; ++c) s += x[c0 + c];
        (*sums)[g] = s;
    }
}

static float row_dot(const QMat& m, const float* x, const float* sums, int r) {
    const int g_n = m.groups();
    const uint8_t* row = m.packed.data() + static_cast<size_t>(r) * m.row_bytes();
    float acc = 0.0f;  // bias is all-zero in every reference loader (custom_model.cpp:251)
    for (int g = 0; g < g_n; ++g) {
        const int c0 = g * m.group;
        const int n = std::min(m.group, m.cols - c0);
        const uint8_t* p = row + (c0 >> 1);
        const float* xs = x + c0;
        float cd = 0.0f;
        for (int c = 0; c < n; c += 2) {
            const uint8_t b = p[c >> 1];
            cd += static_cast<float>(b & 0x0fu) * xs[c];
            if (c + 1 < n) cd += static_cast<float>(b >> 4) * xs[c + 1];
        }
        const size_t mi = static_cast<size_t>(r) * g_n + g;
        if (m.affine) {
            acc += m.scales[mi] * cd + m.zeros[mi] * sums[g];
        } else {
            acc += m.scales[mi] * (cd - m.zeros[mi] * sums[g]);
        }
    }
    return acc;
}

// xq_gemv_w4a16_neon.cpp:259-291
static void gemv(const QMat& m, const float* x, float* y) {
    if (m.bits != 4 || m.rows <= 0 || m.cols <= 0 || m.group <= 0) {
        for (int r = 0; r < m.rows; ++r) y[r] = 0.0f;
        return;
    }
    std::vector<float> sums;
    group_sums(m, x, &sums);
    const float* s = sums.data();
    auto body = [&](int r0, int r1) {
        for (int r = r0; r < r1; ++r) y[r] = row_dot(m, x, s, r);
    };
    const int min_rows = m.cols >= 2048 ? 128 : 512;
    if (m.rows < 2 * min_rows)
        body(0, m.rows);
    else
        pool().run(0, m.rows, min_rows, body);
}

// xq_gemv_w4a16_neon.cpp:293-348: streaming argmax, ties resolve to the lowest row.
static int gemv_argmax(const QMat& m, const float* x, float* best_out) {
    const float ninf = -std::numeric_limits<float>::infinity();
    if (m.bits != 4 || m.rows <= 0 || m.cols <= 0 || m.group <= 0) {
        if (best_out) *best_out = ninf;
        return 0;
    }
    std::vector<float> sums;
    group_sums(m, x, &sums);
    std::mutex mu;
    int best_i = 0;
    float best_v = ninf;
    auto body = [&](int r0, int r1) {
        int li = r0;
        float lv = ninf;
        for (int r = r0; r < r1; ++r) {
            const float v = row_dot(m, x, sums.data(), r);
            if (v > lv || (v == lv && r < li)) {
                lv = v;
                li = r;
            }
        }
        std::lock_guard<std::mutex> g(mu);
        if (lv > best_v || (lv == best_v && li < best_i)) {
            best_v = lv;
            best_i = li;
        }
    };
    if (m.rows < 8192)
        body(0, m.rows);
    else
        pool().run(0, m.rows, 4096, body);
    if (best_out) *best_out = best_v;
    return best_i;
}

// ---------------------------------------------------------------------------
// vector ops
// ---------------------------------------------------------------------------
// customlib/kernels/reference/ref_rmsnorm.cpp:8-17
static void rmsnorm(const float* x, const float* w, int n, float eps, float* y) {
    float ss = 0.0f;
    for (int i = 0; i < n; ++i) ss += x[i] * x[i];
    const float inv = 1.0f / std::sqrt(ss / static_cast<float>(n) + eps);
    for (int i = 0; i < n; ++i) y[i] = x[i] * inv * w[i];
}

// custom_model.cpp:301-313 (note: scales by (inv * w), a different association)
static void head_rms(float* x, const float* w, int heads, int hd, float eps) {
    for (int h = 0; h < heads; ++h) {
        float* v = x + static_cast<size_t>(h) * hd;
        float ss = 0.0f;
        for (int d = 0; d < hd; ++d) ss += v[d] * v[d];
        const float inv = 1.0f / std::sqrt(ss / static_cast<float>(hd) + eps);
        for (int d = 0; d < hd; ++d) v[d] *= inv * w[d];
    }
}

// custom_model.cpp:315-327
static void l2norm_heads(float* x, int heads, int hd) {
    for (int h = 0; h < heads; ++h) {
        float* v = x + static_cast<size_t>(h) * hd;
        float ss = 0.0f;
        for (int d = 0; d < hd; ++d) ss += v[d] * v[d];
        const float inv = 1.0f / std::sqrt(ss + 1.0e-6f);
        for (int d = 0; d < hd; ++d) v[d] *= inv;
    }
}

// custom_model.cpp:329-349 (weight applied as stored, no +1)
static void gated_head_rms(const float* in, const float* w, const float* z, int heads, int hd, float eps,
                           float* out) {
    for (int h = 0; h < heads; ++h) {
        const float* a = in + static_cast<size_t>(h) * hd;
        const float* g = z + static_cast<size_t>(h) * hd;
        float* o = out + static_cast<size_t>(h) * hd;
        float ss = 0.0f;
        for (int d = 0; d < hd; ++d) ss += a[d] * a[d];
        const float inv = 1.0f / std::sqrt(ss / static_cast<float>(hd) + eps);
        for (int d = 0; d < hd; ++d) o[d] = a[d] * inv * w[d] * silu_f(g[d]);
    }
}

// custom_model.cpp:351-370: partial rotary over the first rotary_dim values,
// pairs (i, rd/2+i), the rest of the head passes through.
static void rope_partial(float* x, int heads, int hd, int rotary_dim, int pos, float theta) {
    const int active = std::max(0, std::min(hd, rotary_dim));
    const int half = active / 2;
    for (int h = 0; h < heads; ++h) {
        float* v = x + static_cast<size_t>(h) * hd;
        for (int i = 0; i < half; ++i) {
            const float inv_freq = std::pow(theta, -static_cast<float>(2 * i) / static_cast<float>(active));
            const float ang = static_cast<float>(pos) * inv_freq;
            const float c = std::cos(ang), s = std::sin(ang);
            const float a = v[i], b = v[half + i];
            v[i] = a * c - b * s;
            v[half + i] = b * c + a * s;
        }
    }
}

// customlib/kernels/reference/ref_rope.cpp:8-28 (full-width rotary, test only)
static void rope_full(float* q, float* k, int heads, int hd, int pos, float theta) {
    const int half = hd / 2;
    for (int h = 0; h < heads; ++h) {
        float* qh = q + static_cast<size_t>(h) * hd;
        float* kh = k + static_cast<size_t>(h) * hd;
        for (int i = 0; i < half; ++i) {
            const float inv_freq = std::pow(theta, -static_cast<float>(2 * i) / static_cast<float>(hd));
            const float ang = static_cast<float>(pos) * inv_freq;
            const float c = std::cos(ang), s = std::sin(ang);
            const float q0 = qh[i], q1 = qh[half + i], k0 = kh[i], k1 = kh[half + i];
            qh[i] = q0 * c - q1 * s;
            qh[half + i] = q1 * c + q0 * s;
            kh[i] = k0 * c - k1 * s;
            kh[half + i] = k1 * c + k0 * s;
        }
    }
}

// customlib/kernels/reference/ref_attention.cpp:10-50 (divides by the denominator)
static void attention_ref(const float* q, const float* kc, const float* vc, int ctx, int kvh, int qh_n, int hd,
                          float* out) {
    const int grp = std::max(1, qh_n / std::max(1, kvh));
    std::vector<float> sc(static_cast<size_t>(ctx));
    for (int qh = 0; qh < qh_n; ++qh) {
        const int kh = std::min(kvh - 1, qh / grp);
        const float* qv = q + static_cast<size_t>(qh) * hd;
        float mx = -1.0e30f;
        for (int t = 0; t < ctx; ++t) {
            const float* kv = kc + (static_cast<size_t>(t) * kvh + kh) * hd;
            float dot = 0.0f;
            for (int d = 0; d < hd; ++d) dot += qv[d] * kv[d];
            sc[t] = dot / std::sqrt(static_cast<float>(hd));
            mx = std::max(mx, sc[t]);
        }
        float den = 0.0f;
        for (int t = 0; t < ctx; ++t) {
            sc[t] = std::exp(sc[t] - mx);
            den += sc[t];
        }
        float* o = out + static_cast<size_t>(qh) * hd;
        for (int d = 0; d < hd; ++d) o[d] = 0.0f;
        for (int t = 0; t < ctx; ++t) {
            const float p = sc[t] / den;
            const float* vv = vc + (static_cast<size_t>(t) * kvh + kh) * hd;
            for (int d = 0; d < hd; ++d) o[d] += p * vv[d];
        }
    }
}

// custom_model.cpp:840-928: the in-model decode attention (multiplies by 1/denominator).
static void attention_model(const float* q, const float* kc, const float* vc, int ctx, int kvh, int qh_n, int hd,
                            float* out) {
    const int grp = std::max(1, qh_n / std::max(1, kvh));
    std::vector<float> sc(static_cast<size_t>(std::max(1, ctx * qh_n)));
    std::vector<float> mx(static_cast<size_t>(qh_n), -1.0e30f);
    for (int qh = 0; qh < qh_n; ++qh) {
        const int kh = std::min(kvh - 1, qh / grp);
        const float* qv = q + static_cast<size_t>(qh) * hd;
        for (int t = 0; t < ctx; ++t) {
            const float* kv = kc + (static_cast<size_t>(t) * kvh + kh) * hd;
            float dot = 0.0f;
            for (int d = 0; d < hd; ++d) dot += qv[d] * kv[d];
            const float s = dot / std::sqrt(static_cast<float>(hd));
            sc[static_cast<size_t>(qh) * ctx + t] = s;
            mx[qh] = std::max(mx[qh], s);
        }
    }
    for (int qh = 0; qh < qh_n; ++qh) {
        float den = 0.0f;
        float* row = sc.data() + static_cast<size_t>(qh) * ctx;
        for (int t = 0; t < ctx; ++t) {
            row[t] = std::exp(row[t] - mx[qh]);
            den += row[t];
        }
        const float inv = den > 0.0f ? 1.0f / den : 0.0f;
        for (int t = 0; t < ctx; ++t) row[t] *= inv;
    }
    for (int i = 0; i < qh_n * hd; ++i) out[i] = 0.0f;
    for (int qh = 0; qh < qh_n; ++qh) {
        const int kh = std::min(kvh - 1, qh / grp);
        float* o = out + static_cast<size_t>(qh) * hd;
        const float* row = sc.data() + static_cast<size_t>(qh) * ctx;
        for (int t = 0; t < ctx; ++t) {
            const float p = row[t];
            const float* vv = vc + (static_cast<size_t>(t) * kvh + kh) * hd;
            for (int d = 0; d < hd; ++d) o[d] += p * vv[d];
        }
    }
}

// customlib/kernels/reference/ref_delta.cpp:8-41; state is [key i][value j].
static void gated_delta(const float* q, const float* k, const float* v, float beta, float gate, int dk, int dv,
                        float* S, float* out) {
    const float decay = std::exp(gate);
    for (int i = 0; i < dk * dv; ++i) S[i] *= decay;
    for (int j = 0; j < dv; ++j) {
        float pred = 0.0f;
        for (int i = 0; i < dk; ++i) pred += S[static_cast<size_t>(i) * dv + j] * k[i];
        const float delta = beta * (v[j] - pred);
        for (int i = 0; i < dk; ++i) S[static_cast<size_t>(i) * dv + j] += k[i] * delta;
    }
    const float scale = 1.0f / std::sqrt(static_cast<float>(dk));
    for (int j = 0; j < dv; ++j) {
        float acc = 0.0f;
        for (int i = 0; i < dk; ++i) acc += S[static_cast<size_t>(i) * dv + j] * q[i] * scale;
        out[j] = acc;
    }
}

// custom_model.cpp:986-1005: causal depthwise conv step + SiLU, then shift the history.
static void conv1d_step(const float* x, float* state, const float* w, int channels, int ksize, float* out) {
    const int hist = std::max(0, ksize - 1);
    for (int c = 0; c < channels; ++c) {
        float acc = 0.0f;
        for (int t = 0; t < hist; ++t)
            acc += state[static_cast<size_t>(c) * hist + t] * w[static_cast<size_t>(c) * ksize + t];
        acc += x[c] * w[static_cast<size_t>(c) * ksize + hist];
        out[c] = silu_f(acc);
    }
    for (int c = 0; c < channels; ++c) {
        float* st = state + static_cast<size_t>(c) * hist;
        for (int t = 0; t + 1 < hist; ++t) st[t] = st[t + 1];
        if (hist > 0) st[hist - 1] = x[c];
    }
}

// ---------------------------------------------------------------------------
// On-disk format: custom_model.cpp:185-262, manifest scan :38-87
// ---------------------------------------------------------------------------
static std::string slurp(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return std::string();
    std::ostringstream ss;
    ss << f.rdbuf();
    return ss.str();
}

static bool value_start(const std::string& js, const std::string& key, size_t* at) {
    const std::string pat = "\"" + key + "\"";
    const size_t k = js.find(pat);
    if (k == std::string::npos) return false;
    const size_t colon = js.find(':', k + pat.size());
    if (colon == std::string::npos) return false;
    const size_t s = js.find_first_of("-0123456789", colon + 1);
    if (s == std::string::npos) return false;
    *at = s;
    return true;
}

static int json_int(const std::string& js, const std::string& key, int dflt) {
    size_t s;
    if (!value_start(js, key, &s)) return dflt;
    size_t e = s + 1;
    while (e < js.size() && js[e] >= '0' && js[e] <= '9') ++e;
    try {
        return std::stoi(js.substr(s, e - s));
    } catch (...) {
        return dflt;
    }
}

static float json_float(const std::string& js, const std::string& key, float dflt) {
    size_t s;
    if (!value_start(js, key, &s)) return dflt;
    size_t e = s + 1;
    while (e < js.size() && (std::isdigit(static_cast<unsigned char>(js[e])) || js[e] == '.' || js[e] == 'e' ||
                             js[e] == 'E' || js[e] == '-' || js[e] == '+'))
        ++e;
    try {
        return std::stof(js.substr(s, e - s));
    } catch (...) {
        return dflt;
    }
}

static bool read_f32(const std::string& path, int n, std::vector<float>* out, std::string* err) {
    std::ifstream f(path, std::ios::binary);
    if (!f) {
        *err = "missing vector file: " + path;
        return false;
    }
    out->assign(static_cast<size_t>(n), 0.0f);
    f.read(reinterpret_cast<char*>(out->data()), static_cast<std::streamsize>(n) * 4);
    if (f.gcount() != static_cast<std::streamsize>(n) * 4) {
        *err = "short vector file: " + path;
        return false;
    }
    return true;
}

static bool read_xq4(const std::string& path, QMat* m, std::string* err) {
    std::ifstream f(path, std::ios::binary);
    if (!f) {
        *err = "missing xq4 matrix: " + path;
        return false;
    }
    char magic[8] = {};
    uint32_t h32[5] = {};
    uint64_t h64[3] = {};
    f.read(magic, 8);
    if (std::memcmp(magic, "XQW4A16", 7) != 0) {
        *err = "bad xq4 magic: " + path;
        return false;
    }
    f.read(reinterpret_cast<char*>(h32), sizeof(h32));
    f.read(reinterpret_cast<char*>(h64), sizeof(h64));
    const uint32_t version = h32[0], rows = h32[1], cols = h32[2], group = h32[3], bits = h32[4];
    if (!f || (version != 1 && version != 2) || bits != 4 || rows == 0 || cols == 0 || group == 0 ||
        h64[1] != h64[2]) {
        *err = "invalid xq4 header: " + path;
        return false;
    }
    m->rows = static_cast<int>(rows);
    m->cols = static_cast<int>(cols);
    m->group = static_cast<int>(group);
    m->bits = 4;
    m->affine = version == 2;
    m->packed.assign(static_cast<size_t>(h64[0]), 0);
    m->scales.assign(static_cast<size_t>(h64[1]), 1.0f);
    m->zeros.assign(static_cast<size_t>(h64[2]), 0.0f);
    f.read(reinterpret_cast<char*>(m->packed.data()), static_cast<std::streamsize>(m->packed.size()));
    f.read(reinterpret_cast<char*>(m->scales.data()), static_cast<std::streamsize>(m->scales.size() * 4));
    f.read(reinterpret_cast<char*>(m->zeros.data()), static_cast<std::streamsize>(m->zeros.size() * 4));
    if (!f) {
        *err = "short xq4 payload: " + path;
        return false;
    }
    return true;
}

static void plus_one(std::vector<float>* v) {
    for (float& x : *v) x += 1.0f;
}

// ---------------------------------------------------------------------------
// Model: customlib/runtime/custom_model.cpp (load :423-553, reset :555-567,
// prefill :610-640, layer :1138-1256, final norm :1258-1279, sample :1281-1338,
// decode :1340-1356).
// ---------------------------------------------------------------------------
struct Layer {
    bool full = false;
    std::vector<float> in_norm, post_norm, q_norm, k_norm, lin_norm, conv_w, a_log, dt_bias;
    QMat q, k, v, o, qkv, a, b, z, out, gate, up, down;
    std::vector<float> kc, vc;  // [t][kv_head][head_dim]
    size_t kv_len = 0;
    std::vector<float> conv_state, rec_state;
};

struct Model {
    std::string dir;
    int hidden = 4096, inter = 12288, vocab = 248320, nq = 16, nkv = 4, hd = 256, rot = 64;
    int lk_hd = 128, lv_hd = 128, lk_n = 16, lv_n = 32, ksz = 4, lk_dim = 2048, lv_dim = 4096, conv_dim = 8192;
    float eps = 1.0e-6f, theta = 10000000.0f;
    std::vector<Layer> layers;
    QMat lm_head;
    std::vector<float> final_norm;
    std::vector<uint16_t> emb;  // whole table (vocab x hidden bf16); identical values to a file row read
    // activations (custom_model.cpp:478-498)
    std::vector<float> h, scratch, normed, qbuf, qq, qgate, kb, vb, attn, mixed, la, lb, lz, conv, gbuf, ubuf, ffn;
    std::string err;
};

static bool load_layer(Model& M, int idx, Layer* L) {
    const std::string p = M.dir + "/layers_" + std::to_string(idx) + "_";
    std::string& e = M.err;
    if (!read_f32(p + "input_layernorm_weight.f32", M.hidden, &L->in_norm, &e) ||
        !read_f32(p + "post_attention_layernorm_weight.f32", M.hidden, &L->post_norm, &e) ||
        !read_xq4(p + "mlp_gate_proj_weight.xq4", &L->gate, &e) ||
        !read_xq4(p + "mlp_up_proj_weight.xq4", &L->up, &e) ||
        !read_xq4(p + "mlp_down_proj_weight.xq4", &L->down, &e))
        return false;
    plus_one(&L->in_norm);
    plus_one(&L->post_norm);
    std::ifstream probe(p + "self_attn_q_proj_weight.xq4", std::ios::binary);
    if (probe.good()) {  // a layer is full attention iff its q_proj file exists (custom_model.cpp:526)
        L->full = true;
        if (!read_xq4(p + "self_attn_q_proj_weight.xq4", &L->q, &e) ||
            !read_xq4(p + "self_attn_k_proj_weight.xq4", &L->k, &e) ||
            !read_xq4(p + "self_attn_v_proj_weight.xq4", &L->v, &e) ||
            !read_xq4(p + "self_attn_o_proj_weight.xq4", &L->o, &e) ||
            !read_f32(p + "self_attn_q_norm_weight.f32", M.hd, &L->q_norm, &e) ||
            !read_f32(p + "self_attn_k_norm_weight.f32", M.hd, &L->k_norm, &e))
            return false;
        plus_one(&L->q_norm);
        plus_one(&L->k_norm);
        return true;
    }
    L->full = false;
    return read_xq4(p + "linear_attn_in_proj_qkv_weight.xq4", &L->qkv, &e) &&
           read_xq4(p + "linear_attn_in_proj_a_weight.xq4", &L->a, &e) &&
           read_xq4(p + "linear_attn_in_proj_b_weight.xq4", &L->b, &e) &&
           read_xq4(p + "linear_attn_in_proj_z_weight.xq4", &L->z, &e) &&
           read_xq4(p + "linear_attn_out_proj_weight.xq4", &L->out, &e) &&
           read_f32(p + "linear_attn_norm_weight.f32", M.lv_hd, &L->lin_norm, &e) &&
           read_f32(p + "linear_attn_conv1d_weight.f32", M.conv_dim * M.ksz, &L->conv_w, &e) &&
           read_f32(p + "linear_attn_A_log.f32", M.lv_n, &L->a_log, &e) &&
           read_f32(p + "linear_attn_dt_bias.f32", M.lv_n, &L->dt_bias, &e);
}

static void reset_state(Model& M) {
    for (Layer& L : M.layers) {
        L.kc.clear();
        L.vc.clear();
        L.kv_len = 0;
        if (!L.full) {
            L.conv_state.assign(static_cast<size_t>(M.conv_dim) * std::max(0, M.ksz - 1), 0.0f);
            L.rec_state.assign(static_cast<size_t>(M.lv_n) * M.lk_hd * M.lv_hd, 0.0f);
        }
    }
}

static bool load_model(Model& M, const std::string& dir) {
    M.dir = dir;
    const std::string js = slurp(dir + "/xqwen35_manifest.json");
    M.hidden = json_int(js, "hidden_size", M.hidden);
    M.inter = json_int(js, "intermediate_size", M.inter);
    M.vocab = json_int(js, "vocab_size", M.vocab);
    M.nq = json_int(js, "num_attention_heads", M.nq);
    M.nkv = json_int(js, "num_key_value_heads", M.nkv);
    M.hd = json_int(js, "head_dim", M.hd);
    const float prf = json_float(js, "partial_rotary_factor", 0.25f);
    M.rot = std::max(2, static_cast<int>(std::round(static_cast<float>(M.hd) * prf)));
    if (M.rot & 1) --M.rot;
    M.lk_hd = json_int(js, "linear_key_head_dim", M.lk_hd);
    M.lv_hd = json_int(js, "linear_value_head_dim", M.lv_hd);
    M.lk_n = json_int(js, "linear_num_key_heads", M.lk_n);
    M.lv_n = json_int(js, "linear_num_value_heads", M.lv_n);
    M.ksz = json_int(js, "linear_conv_kernel_dim", M.ksz);
    M.lk_dim = M.lk_hd * M.lk_n;
    M.lv_dim = M.lv_hd * M.lv_n;
    M.conv_dim = 2 * M.lk_dim + M.lv_dim;
    // The reference sizes its query, gate and attention-output buffers by the
    // hidden size (custom_model.cpp:481-486), so a wider attention or linear
    // value dimension overruns them there; refuse such a model instead.
    if (M.nq * M.hd > M.hidden || M.lv_dim > M.hidden) {
        M.err = "attention width " + std::to_string(M.nq * M.hd) + " / linear value width " +
                std::to_string(M.lv_dim) + " exceeds hidden_size " + std::to_string(M.hidden) +
                " (the reference's buffers are sized by hidden_size)";
        return false;
    }
    M.eps = json_float(js, "rms_norm_eps", M.eps);
    M.theta = json_float(js, "rope_theta", M.theta);
    const int n_layers = json_int(js, "num_hidden_layers", 32);
    {
        std::ifstream f(dir + "/embeddings_bf16.bin", std::ios::binary | std::ios::ate);
        if (!f) {
            M.err = "missing embeddings_bf16.bin";
            return false;
        }
        const std::streamoff bytes = f.tellg();
        const std::streamoff want = static_cast<std::streamoff>(M.vocab) * M.hidden * 2;
        M.emb.assign(static_cast<size_t>(std::min(bytes, want) / 2), 0);
        f.seekg(0);
        f.read(reinterpret_cast<char*>(M.emb.data()), static_cast<std::streamsize>(M.emb.size() * 2));
    }
    if (!read_f32(dir + "/norm_weight.f32", M.hidden, &M.final_norm, &M.err)) return false;
    plus_one(&M.final_norm);
    if (!read_xq4(dir + "/lm_head_weight.xq4", &M.lm_head, &M.err)) return false;
    M.layers.resize(static_cast<size_t>(n_layers));
    for (int i = 0; i < n_layers; ++i)
        if (!load_layer(M, i, &M.layers[i])) return false;
    const size_t H = static_cast<size_t>(M.hidden);
    M.h.assign(H, 0.0f);
    M.scratch.assign(H, 0.0f);
    M.normed.assign(H, 0.0f);
    M.qbuf.assign(static_cast<size_t>(std::max(M.hidden * 2, M.conv_dim)), 0.0f);
    M.qq.assign(H, 0.0f);
    M.qgate.assign(H, 0.0f);
    M.kb.assign(static_cast<size_t>(std::max(M.nkv * M.hd, 1)), 0.0f);
    M.vb.assign(static_cast<size_t>(std::max(M.nkv * M.hd, 1)), 0.0f);
    M.attn.assign(H, 0.0f);
    M.mixed.assign(static_cast<size_t>(M.conv_dim), 0.0f);
    M.la.assign(static_cast<size_t>(M.lv_n), 0.0f);
    M.lb.assign(static_cast<size_t>(M.lv_n), 0.0f);
    M.lz.assign(static_cast<size_t>(M.lv_dim), 0.0f);
    M.conv.assign(static_cast<size_t>(M.conv_dim), 0.0f);
    M.gbuf.assign(static_cast<size_t>(M.inter), 0.0f);
    M.ubuf.assign(static_cast<size_t>(M.inter), 0.0f);
    M.ffn.assign(static_cast<size_t>(M.inter), 0.0f);
    reset_state(M);
    return true;
}

// custom_model.cpp:642-671: output is resized to the matrix row count.
static void linear(const QMat& m, const std::vector<float>& x, std::vector<float>* y) {
    if (y->size() != static_cast<size_t>(m.rows)) y->resize(static_cast<size_t>(m.rows));
    gemv(m, x.data(), y->data());
}

// custom_model.cpp:569-608 (out-of-range ids wrap to |id| % vocab)
static bool embed(Model& M, int32_t tok, std::vector<float>* out) {
    if (tok < 0 || tok >= M.vocab) tok = std::abs(tok) % std::max(1, M.vocab);
    const size_t off = static_cast<size_t>(tok) * M.hidden;
    if (off + M.hidden > M.emb.size()) {
        M.err = "short embeddings_bf16.bin row read";
        return false;
    }
    out->resize(static_cast<size_t>(M.hidden));
    for (int i = 0; i < M.hidden; ++i) (*out)[i] = bf16_to_f32(M.emb[off + i]);
    return true;
}

// custom_model.cpp:673-733 (append after norm+RoPE, before attention)
static void append_kv(Model& M, Layer& L) {
    const size_t per = static_cast<size_t>(M.nkv) * M.hd;
    const size_t old = L.kc.size();
    L.kc.resize(old + per, 0.0f);
    L.vc.resize(old + per, 0.0f);
    std::copy_n(M.kb.data(), std::min(M.kb.size(), per), L.kc.data() + old);
    std::copy_n(M.vb.data(), std::min(M.vb.size(), per), L.vc.data() + old);
    L.kv_len += 1;
}

// custom_model.cpp:735-953
static void full_attention(Model& M, Layer& L, size_t pos) {
    linear(L.q, M.normed, &M.qbuf);
    linear(L.k, M.normed, &M.kb);
    linear(L.v, M.normed, &M.vb);
    const int q_dim = M.nq * M.hd;
    const int ghd = 2 * M.hd;
    if (static_cast<int>(M.qbuf.size()) >= M.nq * ghd) {  // gated q_proj: [q_h | gate_h] per head
        for (int h = 0; h < M.nq; ++h) {
            const float* src = M.qbuf.data() + static_cast<size_t>(h) * ghd;
            std::copy(src, src + M.hd, M.qq.data() + static_cast<size_t>(h) * M.hd);
            std::copy(src + M.hd, src + ghd, M.qgate.data() + static_cast<size_t>(h) * M.hd);
        }
    } else {
        std::copy(M.qbuf.begin(), M.qbuf.begin() + std::min<int>(q_dim, static_cast<int>(M.qbuf.size())),
                  M.qq.begin());
        std::fill(M.qgate.begin(), M.qgate.end(), 0.0f);
    }
    head_rms(M.qq.data(), L.q_norm.data(), M.nq, M.hd, M.eps);
    head_rms(M.kb.data(), L.k_norm.data(), M.nkv, M.hd, M.eps);
    rope_partial(M.qq.data(), M.nq, M.hd, M.rot, static_cast<int>(pos), M.theta);
    rope_partial(M.kb.data(), M.nkv, M.hd, M.rot, static_cast<int>(pos), M.theta);
    append_kv(M, L);
    const int ctx = static_cast<int>(L.kv_len);
    attention_model(M.qq.data(), L.kc.data(), L.vc.data(), ctx, M.nkv, M.nq, M.hd, M.attn.data());
    for (int i = 0; i < q_dim; ++i) M.attn[i] *= sigmoid_f(M.qgate[i]);
    linear(L.o, M.attn, &M.scratch);
}

// custom_model.cpp:955-1136
static void linear_attention(Model& M, Layer& L) {
    linear(L.qkv, M.normed, &M.mixed);
    linear(L.a, M.normed, &M.la);
    linear(L.b, M.normed, &M.lb);
    linear(L.z, M.normed, &M.lz);
    conv1d_step(M.mixed.data(), L.conv_state.data(), L.conv_w.data(), M.conv_dim, M.ksz, M.conv.data());
    float* qv = M.conv.data();
    float* kv = M.conv.data() + M.lk_dim;
    float* vv = M.conv.data() + 2 * M.lk_dim;
    l2norm_heads(qv, M.lk_n, M.lk_hd);
    l2norm_heads(kv, M.lk_n, M.lk_hd);
    const int factor = std::max(1, M.lv_n / std::max(1, M.lk_n));
    std::fill(M.attn.begin(), M.attn.end(), 0.0f);
    for (int vh = 0; vh < M.lv_n; ++vh) {
        const int kh = std::min(M.lk_n - 1, vh / factor);
        const float beta = sigmoid_f(M.lb[vh]);
        const float gate = -std::exp(L.a_log[vh]) * softplus_f(M.la[vh] + L.dt_bias[vh]);
        float* S = L.rec_state.data() + static_cast<size_t>(vh) * M.lk_hd * M.lv_hd;
        gated_delta(qv + static_cast<size_t>(kh) * M.lk_hd, kv + static_cast<size_t>(kh) * M.lk_hd,
                    vv + static_cast<size_t>(vh) * M.lv_hd, beta, gate, M.lk_hd, M.lv_hd, S,
                    M.attn.data() + static_cast<size_t>(vh) * M.lv_hd);
    }
    gated_head_rms(M.attn.data(), L.lin_norm.data(), M.lz.data(), M.lv_n, M.lv_hd, M.eps, M.attn.data());
    linear(L.out, M.attn, &M.scratch);
}

static void add_into(std::vector<float>* h, const std::vector<float>& d) {  // custom_model.cpp:294-299
    const size_t n = std::min(h->size(), d.size());
    for (size_t i = 0; i < n; ++i) (*h)[i] += d[i];
}

// custom_model.cpp:1138-1256
static void run_layer(Model& M, Layer& L, size_t pos) {
    rmsnorm(M.h.data(), L.in_norm.data(), M.hidden, M.eps, M.normed.data());
    if (L.full)
        full_attention(M, L, pos);
    else
        linear_attention(M, L);
    add_into(&M.h, M.scratch);
    rmsnorm(M.h.data(), L.post_norm.data(), M.hidden, M.eps, M.normed.data());
    linear(L.gate, M.normed, &M.gbuf);
    linear(L.up, M.normed, &M.ubuf);
    M.ffn.resize(static_cast<size_t>(M.inter));
    for (int i = 0; i < M.inter; ++i) M.ffn[i] = silu_f(M.gbuf[i]) * M.ubuf[i];
    linear(L.down, M.ffn, &M.scratch);
    add_into(&M.h, M.scratch);
}

static void final_norm(Model& M) {  // custom_model.cpp:1258-1279 (result replaces the hidden)
    rmsnorm(M.h.data(), M.final_norm.data(), M.hidden, M.eps, M.scratch.data());
    M.h.swap(M.scratch);
}

static bool prefill(Model& M, const int32_t* toks, size_t n) {
    if (!toks || n == 0) {
        M.err = "custom prefill requires prompt tokens";
        return false;
    }
    reset_state(M);
    for (size_t i = 0; i < n; ++i) {
        if (!embed(M, toks[i], &M.h)) return false;
        for (Layer& L : M.layers) run_layer(M, L, i);
        final_norm(M);
    }
    return true;
}

// custom_model.cpp:1340-1356: sample from the current (already normed) hidden first,
// then run the sampled token forward at `pos`.
static bool decode_one(Model& M, int32_t* tok, size_t pos) {
    if (M.lm_head.rows <= 0 || M.lm_head.cols != M.hidden) {
        M.err = "lm_head matrix is not loaded";
        return false;
    }
    float best = 0.0f;
    *tok = gemv_argmax(M.lm_head, M.h.data(), &best);
    if (!embed(M, *tok, &M.h)) return false;
    for (Layer& L : M.layers) run_layer(M, L, pos);
    final_norm(M);
    return true;
}

}  // namespace orc

// ===========================================================================
// C ABI used by tests (ctypes) and by bench.py's cpu_baseline leg.
// ===========================================================================
using namespace orc;

static QMat make_qmat(const uint8_t* packed, const float* scales, const float* zeros, int rows, int cols,
                      int group, int affine) {
    QMat m;
    m.rows = rows;
    m.cols = cols;
    m.group = group;
    m.affine = affine != 0;
    m.packed.assign(packed, packed + m.row_bytes() * rows);
    const size_t nm = static_cast<size_t>(rows) * m.groups();
    m.scales.assign(scales, scales + nm);
    m.zeros.assign(zeros, zeros + nm);
    return m;
}

extern "C" {

void orc_set_threads(int n) {
    std::lock_guard<std::mutex> g(g_pool_mu);
    g_pool_threads = n;
    g_pool.reset();
}

int orc_threads(void) { return pool().size(); }

// Generators of android/benchmark_app/src/main/cpp/benchmark_jni.cpp:177-196
float orc_det_value(uint64_t index, float scale) {
    uint32_t x = static_cast<uint32_t>(index) * 1664525u + 1013904223u;
    x ^= x >> 16;
    const float unit = static_cast<float>(x & 0xffffu) / 32768.0f - 1.0f;
    return unit * scale;
}

void orc_det_fill(float* v, uint64_t n, float scale) {
    for (uint64_t i = 0; i < n; ++i) v[i] = orc_det_value(i, scale);
}

float orc_checksum(const float* v, uint64_t n) {
    float s = 0.0f;
    const uint64_t stride = std::max<uint64_t>(1, n / 257);
    for (uint64_t i = 0; i < n; i += stride) s += v[i];
    return s;
}

void orc_quantize_lowbit(const float* w, int rows, int cols, int bits, int group, uint8_t* packed_out,
                         float* scales_out, float* zeros_out) {
    QMat q;
    quantize_lowbit(w, rows, cols, bits, group, &q);
    std::memcpy(packed_out, q.packed.data(), q.packed.size());
    std::memcpy(scales_out, q.scales.data(), q.scales.size() * 4);
    std::memcpy(zeros_out, q.zeros.data(), q.zeros.size() * 4);
}

void orc_gemv_w4a16(const uint8_t* packed, const float* scales, const float* zeros, int rows, int cols, int group,
                    int affine, const float* x, float* y) {
    const QMat m = make_qmat(packed, scales, zeros, rows, cols, group, affine);
    gemv(m, x, y);
}

int orc_gemv_w4a16_argmax(const uint8_t* packed, const float* scales, const float* zeros, int rows, int cols,
                          int group, int affine, const float* x, float* best) {
    const QMat m = make_qmat(packed, scales, zeros, rows, cols, group, affine);
    return gemv_argmax(m, x, best);
}

// Textbook per-element form (ref_gemv.cpp:98-106): used to pin the fused GEMV.
void orc_gemv_textbook(const uint8_t* packed, const float* scales, const float* zeros, int rows, int cols, int group,
                       int affine, const float* x, float* y) {
    const QMat m = make_qmat(packed, scales, zeros, rows, cols, group, affine);
    for (int r = 0; r < rows; ++r) {
        float acc = 0.0f;
        for (int c = 0; c < cols; ++c) acc += dequant_one(m, r, c) * x[c];
        y[r] = acc;
    }
}

// W3A16 / W2A16 (and the 4-bit bitstream): gemvW3A16Neon / gemvW2A16Neon
// (arm64_neon/xq_gemv_w{3,2}a16_neon.cpp:6-8) are gemvLowBitReference
// (ref_gemv.cpp:98-106): per row, bias (zero) then per column in order
// acc += dequantizeValue(r, c) * x[c], with the LSB-first bitstream reader.
void orc_gemv_lowbit(const uint8_t* packed, const float* scales, const float* zeros, int rows, int cols, int group,
                     int bits, int affine, const float* x, float* y) {
    QMat m;
    m.rows = rows;
    m.cols = cols;
    m.group = group;
    m.bits = bits;
    m.affine = affine != 0;
    const size_t g_n = static_cast<size_t>(m.groups()) * rows;
    m.packed.assign(packed, packed + (static_cast<size_t>(rows) * cols * bits + 7) / 8);
    m.scales.assign(scales, scales + g_n);
    m.zeros.assign(zeros, zeros + g_n);
    for (int r = 0; r < rows; ++r) {
        float acc = 0.0f;
        for (int c = 0; c < cols; ++c) acc += dequant_one(m, r, c) * x[c];
        y[r] = acc;
    }
}

void orc_dequantize(const uint8_t* packed, const float* scales, const float* zeros, int rows, int cols, int group,
                    int affine, float* out) {
    const QMat m = make_qmat(packed, scales, zeros, rows, cols, group, affine);
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) out[static_cast<size_t>(r) * cols + c] = dequant_one(m, r, c);
}

void orc_rmsnorm(const float* x, const float* w, int n, float eps, float* y) { rmsnorm(x, w, n, eps, y); }
void orc_head_rms(float* x, const float* w, int heads, int hd, float eps) { head_rms(x, w, heads, hd, eps); }
void orc_l2norm_heads(float* x, int heads, int hd) { l2norm_heads(x, heads, hd); }
void orc_gated_head_rms(const float* in, const float* w, const float* z, int heads, int hd, float eps, float* out) {
    gated_head_rms(in, w, z, heads, hd, eps, out);
}
void orc_rope_partial(float* x, int heads, int hd, int rotary_dim, int pos, float theta) {
    rope_partial(x, heads, hd, rotary_dim, pos, theta);
}
void orc_rope_full(float* q, float* k, int heads, int hd, int pos, float theta) {
    rope_full(q, k, heads, hd, pos, theta);
}
void orc_attention_ref(const float* q, const float* kc, const float* vc, int ctx, int kvh, int qh, int hd,
                       float* out) {
    attention_ref(q, kc, vc, ctx, kvh, qh, hd, out);
}
void orc_attention_model(const float* q, const float* kc, const float* vc, int ctx, int kvh, int qh, int hd,
                         float* out) {
    attention_model(q, kc, vc, ctx, kvh, qh, hd, out);
}
void orc_gated_delta(const float* q, const float* k, const float* v, float beta, float gate, int dk, int dv, float* S,
                     float* out) {
    gated_delta(q, k, v, beta, gate, dk, dv, S, out);
}
void orc_conv1d_step(const float* x, float* state, const float* w, int channels, int ksize, float* out) {
    conv1d_step(x, state, w, channels, ksize, out);
}
float orc_silu(float x) { return silu_f(x); }
float orc_sigmoid(float x) { return sigmoid_f(x); }
float orc_softplus(float x) { return softplus_f(x); }
float orc_bf16_to_f32(uint16_t v) { return bf16_to_f32(v); }

// ---- model ----
void* orc_model_load(const char* dir, char* err, size_t err_cap) {
    std::unique_ptr<Model> M(new Model());
    if (!load_model(*M, dir)) {
        if (err && err_cap) std::snprintf(err, err_cap, "%s", M->err.c_str());
        return nullptr;
    }
    return M.release();
}
void orc_model_free(void* h) { delete static_cast<Model*>(h); }
void orc_model_reset(void* h) { reset_state(*static_cast<Model*>(h)); }
int orc_model_prefill(void* h, const int32_t* toks, size_t n) { return prefill(*static_cast<Model*>(h), toks, n) ? 0 : -1; }
int orc_model_decode_one(void* h, int32_t* tok, size_t pos) {
    return decode_one(*static_cast<Model*>(h), tok, pos) ? 0 : -1;
}
int orc_model_dims(void* h, int* out16) {
    const Model& M = *static_cast<Model*>(h);
    const int v[16] = {M.hidden, M.inter, M.vocab, M.nq, M.nkv, M.hd, M.rot, M.lk_hd,
                       M.lv_hd, M.lk_n, M.lv_n, M.ksz, static_cast<int>(M.layers.size()), 0, 0, 0};
    std::memcpy(out16, v, sizeof(v));
    return 0;
}
int orc_model_layer_is_full(void* h, int i) { return static_cast<Model*>(h)->layers[i].full ? 1 : 0; }
void orc_model_get_hidden(void* h, float* out) {
    const Model& M = *static_cast<Model*>(h);
    std::copy(M.h.begin(), M.h.end(), out);
}
void orc_model_set_hidden(void* h, const float* in) {
    Model& M = *static_cast<Model*>(h);
    std::copy(in, in + M.hidden, M.h.begin());
}
// Logits of the current hidden (what the next decode step's lm_head would see).
void orc_model_logits(void* h, float* out) {
    Model& M = *static_cast<Model*>(h);
    gemv(M.lm_head, M.h.data(), out);
}
int orc_model_embed(void* h, int32_t tok) {
    Model& M = *static_cast<Model*>(h);
    return embed(M, tok, &M.h) ? 0 : -1;
}
void orc_model_run_layer(void* h, int i, size_t pos) {
    Model& M = *static_cast<Model*>(h);
    run_layer(M, M.layers[i], pos);
}
void orc_model_final_norm(void* h) { final_norm(*static_cast<Model*>(h)); }
// KV cache of a full-attention layer, [len][kv_heads][head_dim] fp32.
size_t orc_model_kv_len(void* h, int i) { return static_cast<Model*>(h)->layers[i].kv_len; }
void orc_model_get_kv(void* h, int i, float* k, float* v) {
    const Layer& L = static_cast<Model*>(h)->layers[i];
    std::copy(L.kc.begin(), L.kc.end(), k);
    std::copy(L.vc.begin(), L.vc.end(), v);
}
void orc_model_set_kv(void* h, int i, const float* k, const float* v, size_t len) {
    Model& M = *static_cast<Model*>(h);
    Layer& L = M.layers[i];
    const size_t n = len * M.nkv * M.hd;
    L.kc.assign(k, k + n);
    L.vc.assign(v, v + n);
    L.kv_len = len;
}
// Linear-attention state: conv [conv_dim][ksize-1], recurrent [v_heads][key][value].
void orc_model_get_linear_state(void* h, int i, float* conv, float* rec) {
    const Layer& L = static_cast<Model*>(h)->layers[i];
    std::copy(L.conv_state.begin(), L.conv_state.end(), conv);
    std::copy(L.rec_state.begin(), L.rec_state.end(), rec);
}
void orc_model_set_linear_state(void* h, int i, const float* conv, const float* rec) {
    Layer& L = static_cast<Model*>(h)->layers[i];
    std::copy(conv, conv + L.conv_state.size(), L.conv_state.begin());
    std::copy(rec, rec + L.rec_state.size(), L.rec_state.begin());
}

}  // extern "C"
