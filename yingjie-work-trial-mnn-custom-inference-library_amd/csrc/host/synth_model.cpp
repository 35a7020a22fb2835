// synth_model.cpp - seeded synthetic model packages (see include/xqsynth.h).
#include "xqsynth.h"

#include <sys/stat.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <functional>
#include <sstream>
#include <string>
#include <thread>
#include <vector>

namespace {

uint64_t mix64(uint64_t z) {  // splitmix64 finaliser
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

struct Stream {  // counter-based: value i depends only on (seed, name, i)
    uint64_t key;
    Stream(uint64_t seed, const std::string& name) {
        uint64_t h = 1469598103934665603ull;
        for (unsigned char c : name) h = (h ^ c) * 1099511628211ull;
        key = mix64(h ^ mix64(seed));
    }
    uint64_t u64(uint64_t i) const { return mix64(key + i * 0xD1B54A32D192ED03ull); }
    double normal(uint64_t i) const {
        const uint64_t u = u64(i);
        const double a = (static_cast<double>(u & 0xffffffffull) + 0.5) * (1.0 / 4294967296.0);
        const double b = (static_cast<double>(u >> 32) + 0.5) * (1.0 / 4294967296.0);
        return std::sqrt(-2.0 * std::log(a)) * std::cos(6.283185307179586 * b);
    }
};

// Round to the nearest IEEE binary16 value (ties to even), returned as float.
float round_f16(float v) {
    if (!std::isfinite(v) || v == 0.0f) return v;
    int ex = 0;
    std::frexp(v, &ex);
    const int e = std::max(ex - 1, -14);  // binary16 subnormals share the 2^-24 quantum
    const double q = std::ldexp(1.0, e - 10);
    const double r = std::nearbyint(static_cast<double>(v) / q) * q;
    if (std::fabs(r) > 65504.0) return std::copysign(INFINITY, v);
    return static_cast<float>(r);
}

uint16_t to_bf16(float v) {  // round to nearest even
    uint32_t b;
    std::memcpy(&b, &v, 4);
    if ((b & 0x7f800000u) == 0x7f800000u) return static_cast<uint16_t>(b >> 16);
    b += 0x7fffu + ((b >> 16) & 1u);
    return static_cast<uint16_t>(b >> 16);
}

void parallel_for(size_t n, int threads, const std::function<void(size_t, size_t)>& fn) {
    threads = std::max(1, std::min<int>(threads, static_cast<int>((n + 65535) / 65536)));
    if (threads <= 1) {
        fn(0, n);
        return;
    }
    std::vector<std::thread> ts;
    const size_t chunk = (n + threads - 1) / threads;
    for (int t = 0; t < threads; ++t) {
        const size_t a = t * chunk, b = std::min(n, a + chunk);
        if (a < b) ts.emplace_back(fn, a, b);
    }
    for (auto& t : ts) t.join();
}

struct Writer {
    std::string dir;
    xqsynth_config c;
    std::string err;

    bool put(const std::string& name, const void* data, size_t bytes) {
        std::ofstream f(dir + "/" + name, std::ios::binary);
        if (!f) {
            err = "cannot create " + dir + "/" + name;
            return false;
        }
        f.write(static_cast<const char*>(data), static_cast<std::streamsize>(bytes));
        if (!f) {
            err = "short write " + name;
            return false;
        }
        return true;
    }

    bool xq4(const std::string& name, int rows, int cols) {
        const int g = c.group_size;
        const size_t rb = (static_cast<size_t>(cols) + 1) / 2;
        const size_t gpr = static_cast<size_t>((cols + g - 1) / g);
        std::vector<uint8_t> packed(rb * rows);
        std::vector<float> scales(gpr * rows), zeros(gpr * rows, c.zero);
        const Stream sp(c.seed, name + ":codes"), ss(c.seed, name + ":scales"), sz(c.seed, name + ":zeros");
        parallel_for(packed.size() / 8 + 1, c.threads, [&](size_t a, size_t b) {
            for (size_t i = a; i < b; ++i) {
                const uint64_t v = sp.u64(i);
                for (int k = 0; k < 8 && i * 8 + k < packed.size(); ++k)
                    packed[i * 8 + k] = static_cast<uint8_t>(v >> (8 * k));
            }
        });
        if (cols & 1)  // keep the unused high nibble of odd-width rows zero
            for (int r = 0; r < rows; ++r) packed[rb * r + rb - 1] &= 0x0f;
        parallel_for(scales.size(), c.threads, [&](size_t a, size_t b) {
            for (size_t i = a; i < b; ++i) {
                const float s = static_cast<float>(std::fabs(ss.normal(i)) * c.scale_std);
                if (c.asymmetric) {
                    scales[i] = s;
                    zeros[i] = static_cast<float>(std::min(15.0, std::max(0.0, std::nearbyint(7.5 + sz.normal(i)))));
                } else {
                    scales[i] = round_f16(s);
                }
            }
        });
        char hdr[52] = {};
        std::memcpy(hdr, "XQW4A16", 8);
        const uint32_t h32[5] = {1u, static_cast<uint32_t>(rows), static_cast<uint32_t>(cols), static_cast<uint32_t>(g),
                                 4u};
        const uint64_t h64[3] = {packed.size(), scales.size(), zeros.size()};
        std::memcpy(hdr + 8, h32, sizeof(h32));
        std::memcpy(hdr + 28, h64, sizeof(h64));
        std::ofstream f(dir + "/" + name, std::ios::binary);
        if (!f) {
            err = "cannot create " + name;
            return false;
        }
        f.write(hdr, 52);
        f.write(reinterpret_cast<const char*>(packed.data()), static_cast<std::streamsize>(packed.size()));
        f.write(reinterpret_cast<const char*>(scales.data()), static_cast<std::streamsize>(scales.size() * 4));
        f.write(reinterpret_cast<const char*>(zeros.data()), static_cast<std::streamsize>(zeros.size() * 4));
        if (!f) {
            err = "short write " + name;
            return false;
        }
        return true;
    }

    // plus_one: the reader adds 1 (input/post/final/q/k norms), so store eff - 1
    bool norm(const std::string& name, int n, bool plus_one) {
        std::vector<float> v(static_cast<size_t>(n));
        const Stream s(c.seed, name);
        for (int i = 0; i < n; ++i) {
            const float eff = round_f16(static_cast<float>(1.0 + c.norm_std * s.normal(i)));
            v[i] = plus_one ? eff - 1.0f : eff;
        }
        return put(name, v.data(), v.size() * 4);
    }

    bool normal_f32(const std::string& name, size_t n, double std, double mean = 0.0) {
        std::vector<float> v(n);
        const Stream s(c.seed, name);
        for (size_t i = 0; i < n; ++i) v[i] = static_cast<float>(mean + std * s.normal(i));
        return put(name, v.data(), v.size() * 4);
    }
};

}  // namespace

extern "C" {

void xqsynth_default_config(xqsynth_config* c) {
    std::memset(c, 0, sizeof(*c));
    c->seed = 20261201;
    c->hidden_size = 4096;
    c->intermediate_size = 12288;
    c->vocab_size = 248320;
    c->num_layers = 32;
    c->full_attention_interval = 4;
    c->num_attention_heads = 32;
    c->num_key_value_heads = 8;
    c->head_dim = 128;
    c->partial_rotary_factor = 0.25f;
    c->gated_q_proj = 1;
    c->linear_key_head_dim = 128;
    c->linear_value_head_dim = 128;
    c->linear_num_key_heads = 16;
    c->linear_num_value_heads = 32;
    c->linear_conv_kernel_dim = 4;
    c->group_size = 64;
    c->rms_norm_eps = 1.0e-6f;
    c->rope_theta = 1.0e7f;
    c->scale_std = 0.02f;
    c->zero = 8.0f;
    c->embed_std = 1.0f;
    c->norm_std = 0.1f;
    c->threads = 16;
}

int xqsynth_write_model(const char* dir, const xqsynth_config* cfg, char* err, size_t err_capacity) {
    auto fail = [&](const std::string& m) {
        if (err && err_capacity) std::snprintf(err, err_capacity, "%s", m.c_str());
        return -1;
    };
    if (!dir || !cfg) return fail("null argument");
    mkdir(dir, 0775);
    Writer w{dir, *cfg, {}};
    xqsynth_config& c = w.c;
    if (c.threads <= 0) c.threads = static_cast<int>(std::max(1u, std::thread::hardware_concurrency()));
    const int H = c.hidden_size, nq = c.num_attention_heads, nkv = c.num_key_value_heads, hd = c.head_dim;
    const int lk = c.linear_key_head_dim * c.linear_num_key_heads;
    const int lv = c.linear_value_head_dim * c.linear_num_value_heads;
    const int conv_dim = 2 * lk + lv;
    {
        std::ostringstream m;
        m.precision(9);
        m << "{\"format\":\"xqwen35_custom_w4a16\",\"hf_repo\":\"synthetic/random-init\",\"hf_revision\":\"seed-"
          << c.seed << "\",\"hidden_size\":" << H << ",\"intermediate_size\":" << c.intermediate_size
          << ",\"vocab_size\":" << c.vocab_size << ",\"num_hidden_layers\":" << c.num_layers
          << ",\"num_attention_heads\":" << nq << ",\"num_key_value_heads\":" << nkv << ",\"head_dim\":" << hd
          << ",\"linear_key_head_dim\":" << c.linear_key_head_dim
          << ",\"linear_value_head_dim\":" << c.linear_value_head_dim
          << ",\"linear_num_key_heads\":" << c.linear_num_key_heads
          << ",\"linear_num_value_heads\":" << c.linear_num_value_heads
          << ",\"linear_conv_kernel_dim\":" << c.linear_conv_kernel_dim << ",\"rms_norm_eps\":" << c.rms_norm_eps
          << ",\"rope_theta\":" << c.rope_theta << ",\"partial_rotary_factor\":" << c.partial_rotary_factor
          << ",\"quant_bits\":4,\"group_size\":" << c.group_size << "}";
        const std::string s = m.str();
        if (!w.put("xqwen35_manifest.json", s.data(), s.size())) return fail(w.err);
    }
    {
        std::vector<uint16_t> emb(static_cast<size_t>(c.vocab_size) * H);
        const Stream s(c.seed, "embeddings");
        parallel_for(emb.size(), c.threads, [&](size_t a, size_t b) {
            for (size_t i = a; i < b; ++i) emb[i] = to_bf16(static_cast<float>(c.embed_std * s.normal(i)));
        });
        if (!w.put("embeddings_bf16.bin", emb.data(), emb.size() * 2)) return fail(w.err);
    }
    if (!w.norm("norm_weight.f32", H, true) || !w.xq4("lm_head_weight.xq4", c.vocab_size, H)) return fail(w.err);
    for (int i = 0; i < c.num_layers; ++i) {
        const std::string p = "layers_" + std::to_string(i) + "_";
        const bool full = c.full_attention_interval > 0 && i % c.full_attention_interval == c.full_attention_interval - 1;
        bool ok = w.norm(p + "input_layernorm_weight.f32", H, true) &&
                  w.norm(p + "post_attention_layernorm_weight.f32", H, true) &&
                  w.xq4(p + "mlp_gate_proj_weight.xq4", c.intermediate_size, H) &&
                  w.xq4(p + "mlp_up_proj_weight.xq4", c.intermediate_size, H) &&
                  w.xq4(p + "mlp_down_proj_weight.xq4", H, c.intermediate_size);
        if (ok && full) {
            ok = w.xq4(p + "self_attn_q_proj_weight.xq4", nq * hd * (c.gated_q_proj ? 2 : 1), H) &&
                 w.xq4(p + "self_attn_k_proj_weight.xq4", nkv * hd, H) &&
                 w.xq4(p + "self_attn_v_proj_weight.xq4", nkv * hd, H) &&
                 w.xq4(p + "self_attn_o_proj_weight.xq4", H, nq * hd) &&
                 w.norm(p + "self_attn_q_norm_weight.f32", hd, true) &&
                 w.norm(p + "self_attn_k_norm_weight.f32", hd, true);
        } else if (ok) {
            ok = w.xq4(p + "linear_attn_in_proj_qkv_weight.xq4", conv_dim, H) &&
                 w.xq4(p + "linear_attn_in_proj_a_weight.xq4", c.linear_num_value_heads, H) &&
                 w.xq4(p + "linear_attn_in_proj_b_weight.xq4", c.linear_num_value_heads, H) &&
                 w.xq4(p + "linear_attn_in_proj_z_weight.xq4", lv, H) &&
                 w.xq4(p + "linear_attn_out_proj_weight.xq4", H, lv) &&
                 w.norm(p + "linear_attn_norm_weight.f32", c.linear_value_head_dim, false) &&
                 w.normal_f32(p + "linear_attn_conv1d_weight.f32",
                              static_cast<size_t>(conv_dim) * c.linear_conv_kernel_dim, 0.3) &&
                 w.normal_f32(p + "linear_attn_A_log.f32", c.linear_num_value_heads, 0.5) &&
                 w.normal_f32(p + "linear_attn_dt_bias.f32", c.linear_num_value_heads, 0.5);
        }
        if (!ok) return fail(w.err);
    }
    return 0;
}

}  // extern "C"
