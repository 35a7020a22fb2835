// decode_ops.hip - the non-GEMV kernels of one batch-1 decode step on gfx950.
//
// Every kernel reads the token position from device memory (`pos`), so a whole
// decode step can be captured once into a HIP graph and replayed per token.
// Reference functions restated here (paths relative to the reference checkout):
//   embedding row           customlib/runtime/custom_model.cpp:569-608
//   q/gate split            custom_model.cpp:740-753
//   per-head RMSNorm        custom_model.cpp:301-313
//   partial RoPE            custom_model.cpp:351-370 (cos/sin table built on the host with libm)
//   KV append [t][h][d]     custom_model.cpp:673-733
//   GQA decode + out gate   custom_model.cpp:840-951
//   conv1d + SiLU           custom_model.cpp:961-1010
//   L2-normalised heads     custom_model.cpp:315-327
//   gated delta rule        custom_model.cpp:1074-1096, kernels/reference/ref_delta.cpp:8-41
#include "xqhip_common.hpp"
#include "xqhip_kernels.hpp"

namespace xqhip {

// ---------------------------------------------------------------------------
// embedding: bf16 row -> fp32 hidden (exact), token read from device memory.
// ---------------------------------------------------------------------------
// Token t = blockIdx.y reads id tok_ptr[t] and writes row t of out.
__global__ void embed_bf16_kernel(const uint16_t* __restrict__ table, int vocab, int hidden,
                                  const int32_t* __restrict__ tok_ptr, float* __restrict__ out) {
    int tok = tok_ptr[blockIdx.y];
    if (tok < 0 || tok >= vocab) {
        // |id| % vocab as loadEmbeddingRow (custom_model.cpp:573-575), with the
        // magnitude taken in uint32 so even INT_MIN maps to a row in range (the
        // host rejects that id before a prompt reaches the device)
        const uint32_t mag = tok < 0 ? 0u - static_cast<uint32_t>(tok) : static_cast<uint32_t>(tok);
        tok = static_cast<int>(mag % static_cast<uint32_t>(max(1, vocab)));
    }
    const uint16_t* row = table + static_cast<size_t>(tok) * hidden;
    float* o = out + static_cast<size_t>(blockIdx.y) * hidden;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x)
        o[i] = __uint_as_float(static_cast<uint32_t>(row[i]) << 16);
}

hipError_t launch_embed(const EmbedLaunch& p, hipStream_t s) {
    const int blocks = min(16, (p.hidden + 255) / 256);
    hipLaunchKernelGGL(embed_bf16_kernel, dim3(blocks, max(1, p.tokens)), dim3(256), 0, s, p.table, p.vocab,
                       p.hidden, p.tok, p.out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Full-attention head preparation.  Block b < nq: query head b (split from the
// gated q_proj output, per-head RMSNorm, RoPE) -> q_out, gate -> gate_out.
// Block nq + h: kv head h: key RMSNorm + RoPE, key and value stored as fp16 at
// cache slot `pos` ([t][kv_head][head_dim]).
// ---------------------------------------------------------------------------
// Batched form (prefill): token t = blockIdx.y at position *pos + t reads its
// projections at t * src_stride and writes q/gate at t * out_stride.
__global__ void qk_norm_rope_append_kernel(QkPrepLaunch p) {
    extern __shared__ float vals[];  // head_dim
    __shared__ float red[32];
    const int b = blockIdx.x;
    const int t = blockIdx.y;
    const int hd = p.head_dim;
    const int pos = *p.pos + t;
    const bool is_q = b < p.nq;
    const int h = is_q ? b : b - p.nq;
    const size_t src_off = static_cast<size_t>(t) * p.src_stride;
    const float* src;
    const float* w;
    if (is_q) {
        src = p.q_src + src_off + static_cast<size_t>(h) * (p.gated ? 2 * hd : hd);
        w = p.q_norm;
    } else {
        src = p.k_src + src_off + static_cast<size_t>(h) * hd;
        w = p.k_norm;
    }
    float ss = 0.0f;
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        const float v = src[d];
        vals[d] = v;
        ss += v * v;
    }
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(hd) + p.eps);
    for (int d = threadIdx.x; d < hd; d += blockDim.x) vals[d] = vals[d] * (inv * w[d]);
    __syncthreads();
    const int active = max(0, min(hd, p.rotary_dim));
    const int half = active / 2;
    const float2* cs = reinterpret_cast<const float2*>(p.rope_cs) + static_cast<size_t>(pos) * p.rope_pairs;
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        float v = vals[d];
        if (d < half) {
            const float2 c = cs[d];
            v = vals[d] * c.x - vals[half + d] * c.y;
        } else if (d < 2 * half) {
            const float2 c = cs[d - half];
            v = vals[d] * c.x + vals[d - half] * c.y;
        }
        if (is_q) {
            const size_t o = static_cast<size_t>(t) * p.out_stride + static_cast<size_t>(h) * hd + d;
            p.q_out[o] = v;
            p.gate_out[o] = p.gated ? src[hd + d] : 0.0f;
        } else {
            const size_t slot = (static_cast<size_t>(pos) * p.nkv + h) * hd + d;
            p.k_cache[slot] = static_cast<_Float16>(v);
            p.v_cache[slot] = static_cast<_Float16>(p.v_src[src_off + static_cast<size_t>(h) * hd + d]);
        }
    }
}

hipError_t launch_qk_prep(const QkPrepLaunch& p, hipStream_t s) {
    const int threads = p.head_dim >= 256 ? 256 : (p.head_dim > 64 ? 128 : 64);
    hipLaunchKernelGGL(qk_norm_rope_append_kernel, dim3(p.nq + p.nkv, max(1, p.tokens)), dim3(threads),
                       static_cast<size_t>(p.head_dim) * sizeof(float), s, p);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// GQA decode attention in two kernels.
//
// gqa_chunk_kernel: block (kh, j) takes the `group` query heads of kv head kh
// over the 64-token chunks j, j + gridDim.y, ... of the context: scores
// q.k/sqrt(d), the chunk's max m and sum l of exp(s - m), and the unnormalised
// sum of exp(s - m) v, written to the workspace per (head, chunk).
// gqa_combine_kernel: one block per query head merges the chunks of the
// context (weights exp(m_c - M)), normalises, applies the sigmoid output gate.
// The kernel boundary orders the two, so no block waits on another and no
// grid-wide fence is needed.
// ---------------------------------------------------------------------------
constexpr int kAttnChunk = 64;
constexpr int kAttnMaxGroup = 8;
constexpr int kAttnMaxCtx = 16384;
constexpr int kAttnMaxChunks = kAttnMaxCtx / kAttnChunk;
constexpr int kAttnGridChunks = 64;  // chunk slots per kv head in the grid
constexpr int kAttnThreads = 256;

// A chunk's K and V as this thread consumes them (HD > 0): K for the scores
// (4 lanes per token, HD/4 dims each), V for the weighted sum (HD/8 lanes per
// token, 8 dims each, tokens ts, ts + TPP, ...).  Loaded by load_kv before the
// query is ready so the cache latency overlaps the q preparation; token
// indices past the chunk are clamped to its last token (in bounds, unused).
template <int HD>
struct KvRegs {
    static constexpr int kK = HD / 32;             // uint4 of K per thread
    static constexpr int kV = kAttnChunk * HD / 2048;  // tokens of V per thread
    uint4 k[kK > 0 ? kK : 1];
    uint4 v[kV > 0 ? kV : 1];
};

template <int HD>
__device__ __forceinline__ void load_kv(const GqaLaunch& p, int kh, int t0, int n, KvRegs<HD>& r) {
    if constexpr (HD > 0) {
        constexpr int DL = HD / 4, LPT = HD / 8, TPP = kAttnThreads / LPT;
        const int sub = threadIdx.x & 3, tt = threadIdx.x >> 2;
        const _Float16* krow = p.k_cache + (static_cast<size_t>(t0 + min(tt, n - 1)) * p.nkv + kh) * HD + sub * DL;
#pragma unroll
        for (int u = 0; u < KvRegs<HD>::kK; ++u) r.k[u] = *reinterpret_cast<const uint4*>(krow + 8 * u);
        const int dsl = threadIdx.x % LPT, ts = threadIdx.x / LPT;
#pragma unroll
        for (int u = 0; u < KvRegs<HD>::kV; ++u) {
            const int t = min(ts + u * TPP, n - 1);
            r.v[u] = *reinterpret_cast<const uint4*>(p.v_cache + (static_cast<size_t>(t0 + t) * p.nkv + kh) * HD + dsl * 8);
        }
    }
}

// pos_new >= 0: key/value of position pos_new come from kn / vn (LDS, the
// values the same launch appends to the cache) instead of the cache.
template <int HD>
__device__ __forceinline__ void gqa_chunk(const GqaLaunch& p, int kh, int ch, int t0, int n, int group, int hd,
                                          const float* qs, float* sc, float* vred, const KvRegs<HD>& kvr,
                                          int pos_new = -1, const float* kn = nullptr, const float* vn = nullptr) {
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    const float rscale = 1.0f / sqrtf(static_cast<float>(hd));
    const int qh0 = kh * group;
    // scores: 4 lanes per token, each lane HD/4 consecutive dims (16-byte loads)
    if constexpr (HD > 0) {
        constexpr int DL = HD / 4;
        const int sub = threadIdx.x & 3, tt = threadIdx.x >> 2;
        const bool valid = tt < n;
        float kv[DL];
#pragma unroll
        for (int u = 0; u < DL / 8; ++u) {
            const uint4 w = kvr.k[u];
            const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                kv[8 * u + 2 * e] = half_lo(ww[e]);
                kv[8 * u + 2 * e + 1] = half_hi(ww[e]);
            }
        }
        if (valid && t0 + tt == pos_new) {
#pragma unroll
            for (int d = 0; d < DL; ++d) kv[d] = kn[sub * DL + d];
        }
        for (int g = 0; g < group; ++g) {
            const float* qv = qs + g * HD + sub * DL;
            float dot = 0.0f;
#pragma unroll
            for (int d = 0; d < DL; ++d) dot += qv[d] * kv[d];
            dot = lanes_sum<4>(dot);
            if (valid && sub == 0) sc[g * kAttnChunk + tt] = dot * rscale;
        }
    } else {
        for (int pr = threadIdx.x; pr < n * group; pr += kAttnThreads) {
            const int t = pr / group, g = pr % group;
            const _Float16* krow = p.k_cache + (static_cast<size_t>(t0 + t) * p.nkv + kh) * hd;
            const bool is_new = t0 + t == pos_new;
            float dot = 0.0f;
            for (int d = 0; d < hd; ++d) dot += qs[g * hd + d] * (is_new ? kn[d] : static_cast<float>(krow[d]));
            sc[g * kAttnChunk + t] = dot * rscale;
        }
    }
    __syncthreads();
    // chunk softmax statistics: one wave per head, one lane per token
    for (int g = wid; g < group; g += kAttnThreads / kWave) {
        const float sv = lane < n ? sc[g * kAttnChunk + lane] : -INFINITY;
        const float m = wave_max(sv);
        const float e = lane < n ? expf(sv - m) : 0.0f;
        const float l = wave_sum(e);
        sc[g * kAttnChunk + lane] = e;
        if (lane == 0) {
            p.part_m[(qh0 + g) * kAttnMaxChunks + ch] = m;
            p.part_l[(qh0 + g) * kAttnMaxChunks + ch] = l;
        }
    }
    __syncthreads();
    // sum_t e_t v_t: 16-byte loads of v, HD/8 lanes per token
    if constexpr (HD > 0) {
        constexpr int LPT = HD / 8;
        static_assert(LPT >= 8 && LPT <= 32, "pair sums below cover lane distances 8..32");
        constexpr int TPP = kAttnThreads / LPT;
        const int dsl = threadIdx.x % LPT, ts = threadIdx.x / LPT;
        float o[kAttnMaxGroup][8];
#pragma unroll
        for (int g = 0; g < kAttnMaxGroup; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e) o[g][e] = 0.0f;
#pragma unroll
        for (int u = 0; u < KvRegs<HD>::kV; ++u) {
            const int t = ts + u * TPP;
            if (t >= n) break;
            const uint4 w = kvr.v[u];
            float vv[8] = {half_lo(w.x), half_hi(w.x), half_lo(w.y), half_hi(w.y),
                           half_lo(w.z), half_hi(w.z), half_lo(w.w), half_hi(w.w)};
            if (t0 + t == pos_new) {
#pragma unroll
                for (int e = 0; e < 8; ++e) vv[e] = vn[dsl * 8 + e];
            }
#pragma unroll
            for (int g = 0; g < kAttnMaxGroup; ++g) {
                if (g < group) {
                    const float pr = sc[g * kAttnChunk + t];
#pragma unroll
                    for (int e = 0; e < 8; ++e) o[g][e] += pr * vv[e];
                }
            }
        }
#pragma unroll
        for (int g = 0; g < kAttnMaxGroup; ++g) {
            if (g < group) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    if constexpr (LPT <= 8) o[g][e] = xor_pair_sum<8>(o[g][e]);
                    if constexpr (LPT <= 16) o[g][e] = xor_pair_sum<16>(o[g][e]);
                    o[g][e] = xor_pair_sum<32>(o[g][e]);
                }
            }
        }
        if (lane < LPT) {
#pragma unroll
            for (int g = 0; g < kAttnMaxGroup; ++g)
                if (g < group)
#pragma unroll
                    for (int e = 0; e < 8; ++e) vred[(wid * group + g) * HD + dsl * 8 + e] = o[g][e];
        }
        __syncthreads();
        for (int i = threadIdx.x; i < group * HD; i += kAttnThreads) {
            const int g = i / HD, d = i % HD;
            float acc = 0.0f;
#pragma unroll
            for (int w = 0; w < kAttnThreads / kWave; ++w) acc += vred[(w * group + g) * HD + d];
            p.part_o[(static_cast<size_t>(qh0 + g) * kAttnMaxChunks + ch) * HD + d] = acc;
        }
    } else {
        for (int i = threadIdx.x; i < group * hd; i += kAttnThreads) {
            const int g = i / hd, d = i % hd;
            float acc = 0.0f;
            for (int t = 0; t < n; ++t)
                acc += sc[g * kAttnChunk + t] *
                       (t0 + t == pos_new ? vn[d]
                                          : static_cast<float>(p.v_cache[(static_cast<size_t>(t0 + t) * p.nkv + kh) * hd + d]));
            p.part_o[(static_cast<size_t>(qh0 + g) * kAttnMaxChunks + ch) * hd + d] = acc;
        }
    }
    __syncthreads();  // sc and vred are reused by the block's next chunk
}

template <int HD>
__global__ void __launch_bounds__(kAttnThreads) gqa_chunk_kernel(GqaLaunch p) {
    extern __shared__ float smem[];
    const int hd = HD > 0 ? HD : p.head_dim;
    const int group = p.nq / p.nkv;
    const int kh = blockIdx.x;
    const int ctx = *p.pos + 1;
    if (static_cast<int>(blockIdx.y) * kAttnChunk >= ctx) return;  // whole block: nothing to do
    float* qs = smem;                       // [group][hd]
    float* sc = qs + group * hd;            // [group][64]
    float* vred = sc + group * kAttnChunk;  // [4 waves][group][hd]
    const int nch = (ctx + kAttnChunk - 1) / kAttnChunk;
    KvRegs<HD> kvr;
    load_kv<HD>(p, kh, blockIdx.y * kAttnChunk, min(kAttnChunk, ctx - static_cast<int>(blockIdx.y) * kAttnChunk), kvr);
    for (int i = threadIdx.x; i < group * hd; i += kAttnThreads) qs[i] = p.q[static_cast<size_t>(kh) * group * hd + i];
    __syncthreads();
    for (int ch = blockIdx.y; ch < nch; ch += gridDim.y) {
        const int t0 = ch * kAttnChunk;
        const int n = min(kAttnChunk, ctx - t0);
        if (ch != static_cast<int>(blockIdx.y)) load_kv<HD>(p, kh, t0, n, kvr);
        gqa_chunk<HD>(p, kh, ch, t0, n, group, hd, qs, sc, vred, kvr);
    }
}

// Decode attention with the q/k preparation folded in: every block normalises
// and rotates the q heads of its kv head (cheap), and the block whose chunks
// include position pos also prepares that position's key and value, appends
// them to the fp16 caches and uses them (rounded to fp16, like every cached
// position) from LDS; the slot this launch writes is never taken from memory.
template <int HD>
__global__ void __launch_bounds__(kAttnThreads) attn_decode_kernel(AttnDecodeLaunch a) {
    extern __shared__ float smem[];
    const GqaLaunch& p = a.g;
    const int hd = HD > 0 ? HD : p.head_dim;
    const int group = p.nq / p.nkv;
    const int kh = blockIdx.x;
    const int pos = *p.pos;
    const int ctx = pos + 1;
    if (static_cast<int>(blockIdx.y) * kAttnChunk >= ctx) return;  // whole block: nothing to do
    float* qs = smem;                       // [group][hd]
    float* sc = qs + group * hd;            // [group][64]
    float* vred = sc + group * kAttnChunk;  // [4 waves][group][hd]
    float* kn = vred + (kAttnThreads / kWave) * group * hd;  // [hd]
    float* vn = kn + hd;                                     // [hd]
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    const int half = a.rotary_dim / 2;
    const float2* cs = reinterpret_cast<const float2*>(a.rope_cs) + static_cast<size_t>(pos) * a.rope_pairs;
    const int nch = (ctx + kAttnChunk - 1) / kAttnChunk;
    const bool owns_new = (pos / kAttnChunk) % static_cast<int>(gridDim.y) == static_cast<int>(blockIdx.y);
    // K/V of the block's first chunk are requested before the q preparation
    // (the slot of `pos` is read too but replaced by kn / vn below)
    KvRegs<HD> kvr;
    load_kv<HD>(p, kh, blockIdx.y * kAttnChunk, min(kAttnChunk, ctx - static_cast<int>(blockIdx.y) * kAttnChunk), kvr);
    // per-head RMSNorm (custom_model.cpp:301-313): one wave per head; heads
    // 0..group-1 are q, head `group` (owner only) is the new key
    const int nheads = group + (owns_new ? 1 : 0);
    for (int h = wid; h < nheads; h += kAttnThreads / kWave) {
        const bool is_k = h == group;
        const float* src = is_k ? a.k_src + static_cast<size_t>(kh) * hd
                                : a.q_src + static_cast<size_t>(kh * group + h) * (a.gated ? 2 * hd : hd);
        const float* w = is_k ? a.k_norm : a.q_norm;
        float* dst = is_k ? kn : qs + h * hd;
        float ss = 0.0f;
        for (int d = lane; d < hd; d += kWave) {
            const float v = src[d];
            dst[d] = v;
            ss += v * v;
        }
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss / static_cast<float>(hd) + a.eps);
        for (int d = lane; d < hd; d += kWave) dst[d] = dst[d] * (inv * w[d]);
    }
    if (owns_new)
        for (int d = threadIdx.x; d < hd; d += kAttnThreads) vn[d] = a.v_src[static_cast<size_t>(kh) * hd + d];
    __syncthreads();
    // partial RoPE (custom_model.cpp:351-370) on the first rotary_dim dims, pairs (i, half + i)
    for (int i = threadIdx.x; i < nheads * half; i += kAttnThreads) {
        const int h = i / half, d = i % half;
        float* v = h == group ? kn : qs + h * hd;
        const float2 c = cs[d];
        const float x0 = v[d], x1 = v[half + d];
        v[d] = x0 * c.x - x1 * c.y;
        v[half + d] = x1 * c.x + x0 * c.y;
    }
    __syncthreads();
    if (owns_new) {  // append at slot pos, and use the fp16-rounded values like every other slot
        for (int d = threadIdx.x; d < hd; d += kAttnThreads) {
            const size_t slot = (static_cast<size_t>(pos) * p.nkv + kh) * hd + d;
            const _Float16 kq = static_cast<_Float16>(kn[d]), vq = static_cast<_Float16>(vn[d]);
            a.k_cache[slot] = kq;
            a.v_cache[slot] = vq;
            kn[d] = static_cast<float>(kq);
            vn[d] = static_cast<float>(vq);
        }
        __syncthreads();
    }
    for (int ch = blockIdx.y; ch < nch; ch += gridDim.y) {
        const int t0 = ch * kAttnChunk;
        const int n = min(kAttnChunk, ctx - t0);
        if (ch != static_cast<int>(blockIdx.y)) load_kv<HD>(p, kh, t0, n, kvr);
        gqa_chunk<HD>(p, kh, ch, t0, n, group, hd, qs, sc, vred, kvr, pos, kn, vn);
    }
}

__global__ void __launch_bounds__(256) gqa_combine_kernel(GqaLaunch p) {
    __shared__ float wgt[kAttnMaxChunks];
    __shared__ float red[32];
    const int qh = blockIdx.x;
    const int hd = p.head_dim;
    const int ctx = *p.pos + 1;
    const int nch = (ctx + kAttnChunk - 1) / kAttnChunk;
    const float* pm = p.part_m + static_cast<size_t>(qh) * kAttnMaxChunks;
    const float* pl = p.part_l + static_cast<size_t>(qh) * kAttnMaxChunks;
    float m = -INFINITY;
    for (int c = threadIdx.x; c < nch; c += blockDim.x) m = fmaxf(m, pm[c]);
    m = wave_max(m);
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    if (lane == 0) red[wid] = m;
    __syncthreads();
    float mm = -INFINITY;
    for (int i = 0; i < static_cast<int>(blockDim.x) / kWave; ++i) mm = fmaxf(mm, red[i]);
    __syncthreads();
    float l = 0.0f;
    for (int c = threadIdx.x; c < nch; c += blockDim.x) {
        const float f = expf(pm[c] - mm);
        wgt[c] = f;
        l += pl[c] * f;
    }
    l = block_sum(l, red);  // also orders the wgt writes before the reads below
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    const float* po = p.part_o + static_cast<size_t>(qh) * kAttnMaxChunks * hd;
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        float o = 0.0f;
        for (int c = 0; c < nch; ++c) o += po[static_cast<size_t>(c) * hd + d] * wgt[c];
        const size_t oi = static_cast<size_t>(qh) * hd + d;
        // no gate projection: the reference's zero gate, sigmoid(0) (custom_model.cpp:750-753)
        const float gv = p.gate ? p.gate[static_cast<size_t>(qh) * p.gate_stride + d] : 0.0f;
        p.out[oi] = (o * inv) * sigmoid_dev(gv);
    }
}

size_t gqa_workspace_bytes(int nq, int nkv, int head_dim) {
    (void)nkv;
    return sizeof(float) * static_cast<size_t>(nq) * kAttnMaxChunks * (head_dim + 2);
}

static size_t gqa_lds_bytes(int group, int head_dim) {
    return sizeof(float) * (static_cast<size_t>(group) * head_dim + static_cast<size_t>(group) * kAttnChunk +
                            (kAttnThreads / kWave) * static_cast<size_t>(group) * head_dim);
}

hipError_t launch_attn_decode(const AttnDecodeLaunch& a, hipStream_t s) {
    const GqaLaunch& p = a.g;
    const int group = p.nq / p.nkv;
    const size_t lds = gqa_lds_bytes(group, p.head_dim) + 2 * sizeof(float) * p.head_dim;
    const int slots = min(kAttnGridChunks, (p.max_ctx + kAttnChunk - 1) / kAttnChunk);
    const dim3 grid(p.nkv, slots);
    switch (p.head_dim) {
        case 64: hipLaunchKernelGGL(attn_decode_kernel<64>, grid, dim3(kAttnThreads), lds, s, a); break;
        case 128: hipLaunchKernelGGL(attn_decode_kernel<128>, grid, dim3(kAttnThreads), lds, s, a); break;
        case 256: hipLaunchKernelGGL(attn_decode_kernel<256>, grid, dim3(kAttnThreads), lds, s, a); break;
        default: hipLaunchKernelGGL(attn_decode_kernel<0>, grid, dim3(kAttnThreads), lds, s, a); break;
    }
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    hipLaunchKernelGGL(gqa_combine_kernel, dim3(p.nq), dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_gqa(const GqaLaunch& p, hipStream_t s) {
    const int group = p.nq / p.nkv;
    const size_t lds = gqa_lds_bytes(group, p.head_dim);
    const int slots = min(kAttnGridChunks, (p.max_ctx + kAttnChunk - 1) / kAttnChunk);
    const dim3 grid(p.nkv, slots);
    switch (p.head_dim) {
        case 64: hipLaunchKernelGGL(gqa_chunk_kernel<64>, grid, dim3(kAttnThreads), lds, s, p); break;
        case 128: hipLaunchKernelGGL(gqa_chunk_kernel<128>, grid, dim3(kAttnThreads), lds, s, p); break;
        case 256: hipLaunchKernelGGL(gqa_chunk_kernel<256>, grid, dim3(kAttnThreads), lds, s, p); break;
        default: hipLaunchKernelGGL(gqa_chunk_kernel<0>, grid, dim3(kAttnThreads), lds, s, p); break;
    }
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    hipLaunchKernelGGL(gqa_combine_kernel, dim3(p.nq), dim3(256), 0, s, p);
    return hipGetLastError();
}

bool gqa_supported(int nq, int nkv, int head_dim, int max_ctx) {
    if (nkv <= 0 || nq % nkv != 0 || nq / nkv > kAttnMaxGroup || head_dim <= 0) return false;
    if (max_ctx < 1 || max_ctx > kAttnMaxCtx) return false;
    return gqa_lds_bytes(nq / nkv, head_dim) + 2 * sizeof(float) * head_dim <= 64 * 1024;
}

// ---------------------------------------------------------------------------
// Linear attention, step 1: causal depthwise conv1d + SiLU over the mixed
// q|k|v channels (state [channel][ksize-1], shifted in the same thread that
// reads it), then L2 normalisation of each query and key head.
// Blocks: [0, lk_n) query heads, [lk_n, 2 lk_n) key heads, then value heads.
// ---------------------------------------------------------------------------
__global__ void conv_l2norm_kernel(ConvLaunch p) {
    __shared__ float red[32];
    const int b = blockIdx.x;
    int c0, width;
    bool norm;
    if (b < p.lk_n) {
        c0 = b * p.lk_hd;
        width = p.lk_hd;
        norm = true;
    } else if (b < 2 * p.lk_n) {
        c0 = p.lk_n * p.lk_hd + (b - p.lk_n) * p.lk_hd;
        width = p.lk_hd;
        norm = true;
    } else {
        c0 = 2 * p.lk_n * p.lk_hd + (b - 2 * p.lk_n) * p.lv_hd;
        width = p.lv_hd;
        norm = false;
    }
    const int hist = max(0, p.ksize - 1);
    const int j = threadIdx.x;  // one channel per thread (width <= blockDim.x)
    float y = 0.0f;
    if (j < width) {
        const int c = c0 + j;
        float* st = p.state + static_cast<size_t>(c) * hist;
        const float* w = p.conv_w + static_cast<size_t>(c) * p.ksize;
        float acc = 0.0f;
        for (int t = 0; t < hist; ++t) acc += st[t] * w[t];
        const float xv = p.mixed[c];
        acc += xv * w[hist];
        for (int t = 0; t + 1 < hist; ++t) st[t] = st[t + 1];
        if (hist > 0) st[hist - 1] = xv;
        y = silu_dev(acc);
        if (!norm) p.out[c] = y;
    }
    if (!norm) return;  // uniform per block
    const float ss = block_sum(y * y, red);
    const float inv = 1.0f / sqrtf(ss + 1.0e-6f);
    if (j < width) p.out[c0 + j] = y * inv;
}

hipError_t launch_conv(const ConvLaunch& p, hipStream_t s) {
    const int width = max(p.lk_hd, p.lv_hd);
    const int threads = ((width + 63) / 64) * 64;
    hipLaunchKernelGGL(conv_l2norm_kernel, dim3(2 * p.lk_n + p.lv_n), dim3(threads), 0, s, p);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Linear attention, step 2: gated delta rule for one value head and a slice of
// kDeltaCols value columns.  S[i][j] (key i, value j) fp32 stays in HBM between
// tokens; each column is owned by exactly one thread column of one block.
//   decay = exp(g), g = -exp(A_log) * softplus(a + dt_bias), beta = sigmoid(b)
//   S *= decay; pred_j = sum_i S[i][j] k_i; S[i][j] += k_i * beta (v_j - pred_j)
//   out_j = sum_i S[i][j] q_i / sqrt(dk)
// ---------------------------------------------------------------------------
constexpr int kDeltaCols = 16;
constexpr int kDeltaIGroups = 16;   // threads per column
constexpr int kDeltaMaxKPerThread = 16;  // key dim <= 256
constexpr int kStepMaxTaps = 8;          // conv kernel size of the fused step

__global__ void __launch_bounds__(256) gated_delta_kernel(DeltaLaunch p) {
    __shared__ float qk[2 * 256];
    __shared__ float colsum[4][kDeltaCols];
    const int vh = blockIdx.x;
    const int j0 = blockIdx.y * kDeltaCols;
    const int factor = max(1, p.lv_n / max(1, p.lk_n));
    const int kh = min(p.lk_n - 1, vh / factor);
    const int dk = p.lk_hd, dv = p.lv_hd;
    const float* q = p.conv + static_cast<size_t>(kh) * dk;
    const float* k = p.conv + static_cast<size_t>(p.lk_n) * dk + static_cast<size_t>(kh) * dk;
    const float* v = p.conv + 2 * static_cast<size_t>(p.lk_n) * dk + static_cast<size_t>(vh) * dv;
    const int jl = threadIdx.x % kDeltaCols;
    const int ig = threadIdx.x / kDeltaCols;
    const int j = j0 + jl;
    const bool active = j < dv;
    float* S = p.state + static_cast<size_t>(vh) * dk * dv;
    float sreg[kDeltaMaxKPerThread];
#pragma unroll
    for (int r = 0; r < kDeltaMaxKPerThread; ++r) {  // state loads first: they do not depend on q, k
        const int i = ig + r * kDeltaIGroups;
        sreg[r] = (active && i < dk) ? S[static_cast<size_t>(i) * dv + j] : 0.0f;
    }
    for (int i = threadIdx.x; i < dk; i += blockDim.x) {
        qk[i] = q[i];
        qk[256 + i] = k[i];
    }
    const float vj = active ? v[j] : 0.0f;
    const float beta = sigmoid_dev(p.b[vh]);
    const float gate = -expf(p.a_log[vh]) * softplus_dev(p.a[vh] + p.dt_bias[vh]);
    const float decay = expf(gate);
    __syncthreads();
    float pred = 0.0f;
#pragma unroll
    for (int r = 0; r < kDeltaMaxKPerThread; ++r) {
        const int i = ig + r * kDeltaIGroups;
        if (active && i < dk) {
            sreg[r] *= decay;
            pred += sreg[r] * qk[256 + i];
        }
    }
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    // threads of one column inside a wave are 16 lanes apart
    pred = xor_pair_sum<32>(xor_pair_sum<16>(pred));
    if (lane < kDeltaCols) colsum[wid][lane] = pred;
    __syncthreads();
    pred = colsum[0][jl] + colsum[1][jl] + colsum[2][jl] + colsum[3][jl];
    __syncthreads();
    const float delta = active ? beta * (vj - pred) : 0.0f;
    float o = 0.0f;
#pragma unroll
    for (int r = 0; r < kDeltaMaxKPerThread; ++r) {
        const int i = ig + r * kDeltaIGroups;
        if (active && i < dk) {
            sreg[r] += qk[256 + i] * delta;
            S[static_cast<size_t>(i) * dv + j] = sreg[r];
            o += sreg[r] * qk[i];
        }
    }
    o = xor_pair_sum<32>(xor_pair_sum<16>(o));
    if (lane < kDeltaCols) colsum[wid][lane] = o;
    __syncthreads();
    if (threadIdx.x < kDeltaCols && active) {
        const float tot = colsum[0][jl] + colsum[1][jl] + colsum[2][jl] + colsum[3][jl];
        p.out[static_cast<size_t>(vh) * dv + j] = tot * (1.0f / sqrtf(static_cast<float>(dk)));
    }
}

hipError_t launch_delta(const DeltaLaunch& p, hipStream_t s) {
    hipLaunchKernelGGL(gated_delta_kernel, dim3(p.lv_n, (p.lv_hd + kDeltaCols - 1) / kDeltaCols), dim3(256), 0, s, p);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Fused linear-attention step: block (vh, column slice) recomputes the conv1d +
// SiLU + L2 norm of its key head's q and k channels (cheap: 2 * lk_hd channels
// of ksize taps), the conv of its own kDeltaCols value channels, then runs the
// gated delta update of gated_delta_kernel on those columns.  Conv history is
// double-buffered by position parity (read copy pos & 1, write the other): the
// q/k history is written by one block per key head (vh % factor == 0, first
// slice), the value history by the block that owns the channel.
// ---------------------------------------------------------------------------
// KS > 0: the conv kernel size as a compile-time constant (the tap loops then
// issue exactly the loads they need); KS == 0: runtime p.ksize <= kStepMaxTaps.
template <int KS>
__global__ void __launch_bounds__(256) linear_step_kernel(LinearStepLaunch p) {
    constexpr int kTaps = KS > 0 ? KS : kStepMaxTaps;
    __shared__ float qk[2 * 256];
    __shared__ float vsh[kDeltaCols];
    __shared__ float colsum[4][kDeltaCols];
    __shared__ float red[2][4];
    const int vh = blockIdx.x;
    const int j0 = blockIdx.y * kDeltaCols;
    const int factor = max(1, p.lv_n / max(1, p.lk_n));
    const int kh = min(p.lk_n - 1, vh / factor);
    const int dk = p.lk_hd, dv = p.lv_hd;
    const int hist = KS > 0 ? KS - 1 : max(0, p.ksize - 1);
    const int conv_dim = 2 * p.lk_n * dk + p.lv_n * dv;
    const bool qk_writer = (vh % factor == 0) && blockIdx.y == 0;
    const int jl = threadIdx.x % kDeltaCols;
    const int ig = threadIdx.x / kDeltaCols;
    const int j = j0 + jl;
    const bool active = j < dv;
    float* S = p.state + static_cast<size_t>(vh) * dk * dv;
    // Loads in the order their data is needed: the conv inputs (filter taps,
    // history, the in_proj output: cache-resident) first, the state (HBM)
    // after them, so the conv arithmetic runs while the state streams in
    // (a wave's loads return in issue order).  Thread t owns q/k channel t
    // and t + 256 (dk <= 256), threads < kDeltaCols one value channel.
    struct Taps {
        float h[kTaps > 1 ? kTaps - 1 : 1], h_other[kTaps > 1 ? kTaps - 1 : 1], w[kTaps], x;
    };
    // Unconditional range-checked loads (c < 0: an unused channel, reads 0).
    // Both history copies are read, so no load waits for the position; the
    // copy of this position's parity is selected afterwards.
    const uint32_t hist_bytes = static_cast<uint32_t>(conv_dim * hist) * 4u;
    const __amdgpu_buffer_rsrc_t r_hist = buf_rsrc(p.conv_state, 2u * hist_bytes);
    const __amdgpu_buffer_rsrc_t r_w = buf_rsrc(p.conv_w, static_cast<uint32_t>(conv_dim * p.ksize) * 4u);
    const __amdgpu_buffer_rsrc_t r_x = buf_rsrc(p.mixed, static_cast<uint32_t>(conv_dim) * 4u);
    auto load_taps = [&](int c, Taps& tp) {
        const bool ok = c >= 0;
        const uint32_t ho = static_cast<uint32_t>(c * hist) * 4u, wo = static_cast<uint32_t>(c * p.ksize) * 4u;
#pragma unroll
        for (int t = 0; t < kTaps - 1; ++t) {
            tp.h[t] = buf_load_f32(r_hist, ok && t < hist ? ho + 4u * t : kBufOOB);
            tp.h_other[t] = buf_load_f32(r_hist, ok && t < hist ? hist_bytes + ho + 4u * t : kBufOOB);
        }
#pragma unroll
        for (int t = 0; t < kTaps; ++t) tp.w[t] = buf_load_f32(r_w, ok && t <= hist ? wo + 4u * t : kBufOOB);
        tp.x = buf_load_f32(r_x, ok ? static_cast<uint32_t>(c) * 4u : kBufOOB);
    };
    // per-head gate inputs first (4 uniform loads; read as scalars they would
    // be fetched only when first used, after the conv)
    const uint32_t ho4 = static_cast<uint32_t>(vh) * 4u, hbytes = static_cast<uint32_t>(p.lv_n) * 4u;
    const float gb = buf_load_f32(buf_rsrc(p.b, hbytes), ho4);
    const float ga = buf_load_f32(buf_rsrc(p.a, hbytes), ho4);
    const float galog = buf_load_f32(buf_rsrc(p.a_log, hbytes), ho4);
    const float gdtb = buf_load_f32(buf_rsrc(p.dt_bias, hbytes), ho4);
    auto select_parity = [&](Taps& tp, int odd) {
#pragma unroll
        for (int t = 0; t < kTaps - 1; ++t) tp.h[t] = odd ? tp.h_other[t] : tp.h[t];
    };
    // (register arrays indexed by unrolled constants only: a runtime index would
    // move them to scratch memory)
    auto conv = [&](const Taps& tp) {
        float acc = 0.0f;
#pragma unroll
        for (int t = 0; t < kTaps - 1; ++t) acc += tp.h[t] * tp.w[t];  // taps past hist are 0
#pragma unroll
        for (int t = 0; t < kTaps; ++t)
            if (t == hist) acc += tp.x * tp.w[t];
        return silu_dev(acc);
    };
    // the shifted history goes out at the end of the kernel: a store issued
    // before the state is consumed would make every later wait a full drain
    auto write_history = [&](float* st_out, int c, const Taps& tp) {
        if (hist == 0) return;
        float* so = st_out + static_cast<size_t>(c) * hist;
#pragma unroll
        for (int t = 0; t + 1 < kTaps - 1; ++t)
            if (t + 1 < hist) so[t] = tp.h[t + 1];
        so[hist - 1] = tp.x;
    };
    constexpr int kThreads = 256;  // the launch's block size
    const int nqk = (2 * dk + kThreads - 1) / kThreads;  // <= 2
    Taps tq[2], tv;
    auto qk_channel = [&](int t, int& d, bool& is_k) {
        is_k = t >= dk;
        d = is_k ? t - dk : t;
        return (is_k ? p.lk_n * dk : 0) + kh * dk + d;
    };
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int t = threadIdx.x + u * kThreads;
        int d; bool is_k;
        const int c = qk_channel(t, d, is_k);
        load_taps(u < nqk && t < 2 * dk ? c : -1, tq[u]);
    }
    const bool has_v = threadIdx.x < kDeltaCols && j0 + static_cast<int>(threadIdx.x) < dv;
    load_taps(has_v ? 2 * p.lk_n * dk + vh * dv + j0 + static_cast<int>(threadIdx.x) : -1, tv);
    const __amdgpu_buffer_rsrc_t r_state = buf_rsrc(S, static_cast<uint32_t>(dk * dv) * 4u);
    float sreg[kDeltaMaxKPerThread];
#pragma unroll
    for (int r = 0; r < kDeltaMaxKPerThread; ++r) {
        const int i = ig + r * kDeltaIGroups;
        sreg[r] = buf_load_f32(r_state, active && i < dk ? static_cast<uint32_t>(i * dv + j) * 4u : kBufOOB);
    }
    // the position is read after every load is issued (its parity picks the
    // history copy read above and the one written at the end)
    const int par = __builtin_nontemporal_load(p.pos) & 1;
    float* st_out = p.conv_state + static_cast<size_t>(par ^ 1) * conv_dim * hist;
    select_parity(tq[0], par);
    select_parity(tq[1], par);
    select_parity(tv, par);
    // q and k channels of key head kh: thread t < dk -> q[t], dk <= t < 2 dk -> k[t - dk]
    float ssq = 0.0f, ssk = 0.0f;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int t = threadIdx.x + u * kThreads;
        if (u < nqk && t < 2 * dk) {
            int d; bool is_k;
            qk_channel(t, d, is_k);
            const float y = conv(tq[u]);
            qk[(is_k ? 256 : 0) + d] = y;
            if (is_k) ssk += y * y; else ssq += y * y;
        }
    }
    if (has_v) vsh[threadIdx.x] = conv(tv);
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    ssq = wave_sum(ssq);
    ssk = wave_sum(ssk);
    if (lane == 0) {
        red[0][wid] = ssq;
        red[1][wid] = ssk;
    }
    const float beta = sigmoid_dev(gb);
    const float gate = -expf(galog) * softplus_dev(ga + gdtb);
    const float decay = expf(gate);
    __syncthreads();
    // l2NormalizeHeads: x * 1/sqrt(sum x^2 + 1e-6)
    const float invq = 1.0f / sqrtf(red[0][0] + red[0][1] + red[0][2] + red[0][3] + 1.0e-6f);
    const float invk = 1.0f / sqrtf(red[1][0] + red[1][1] + red[1][2] + red[1][3] + 1.0e-6f);
    const float vj = active ? vsh[jl] : 0.0f;
    float pred = 0.0f;
#pragma unroll
    for (int r = 0; r < kDeltaMaxKPerThread; ++r) {
        const int i = ig + r * kDeltaIGroups;
        if (active && i < dk) {
            sreg[r] *= decay;
            pred += sreg[r] * (qk[256 + i] * invk);
        }
    }
    pred = xor_pair_sum<32>(xor_pair_sum<16>(pred));
    if (lane < kDeltaCols) colsum[wid][lane] = pred;
    __syncthreads();
    pred = colsum[0][jl] + colsum[1][jl] + colsum[2][jl] + colsum[3][jl];
    __syncthreads();
    const float delta = active ? beta * (vj - pred) : 0.0f;
    float o = 0.0f;
#pragma unroll
    for (int r = 0; r < kDeltaMaxKPerThread; ++r) {
        const int i = ig + r * kDeltaIGroups;
        if (active && i < dk) {
            sreg[r] += (qk[256 + i] * invk) * delta;
            S[static_cast<size_t>(i) * dv + j] = sreg[r];
            o += sreg[r] * (qk[i] * invq);
        }
    }
    o = xor_pair_sum<32>(xor_pair_sum<16>(o));
    if (lane < kDeltaCols) colsum[wid][lane] = o;
    __syncthreads();
    if (threadIdx.x < kDeltaCols && active) {
        const float tot = colsum[0][jl] + colsum[1][jl] + colsum[2][jl] + colsum[3][jl];
        p.out[static_cast<size_t>(vh) * dv + j] = tot * (1.0f / sqrtf(static_cast<float>(dk)));
    }
    if (qk_writer) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int t = threadIdx.x + u * kThreads;
            if (u < nqk && t < 2 * dk) {
                int d; bool is_k;
                write_history(st_out, qk_channel(t, d, is_k), tq[u]);
            }
        }
    }
    if (has_v) write_history(st_out, 2 * p.lk_n * dk + vh * dv + j0 + threadIdx.x, tv);
}

bool linear_step_supported(int lk_n, int lk_hd, int lv_n, int lv_hd, int ksize) {
    return lk_n > 0 && lv_n > 0 && lv_n % lk_n == 0 && lk_hd > 0 && lk_hd <= 256 && lv_hd > 0 && ksize >= 1 &&
           ksize <= kStepMaxTaps && lk_hd <= kDeltaIGroups * kDeltaMaxKPerThread;
}

hipError_t launch_linear_step(const LinearStepLaunch& p, hipStream_t s) {
    const dim3 grid(p.lv_n, (p.lv_hd + kDeltaCols - 1) / kDeltaCols);
    if (p.ksize == 4)
        hipLaunchKernelGGL(linear_step_kernel<4>, grid, dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL(linear_step_kernel<0>, grid, dim3(256), 0, s, p);
    return hipGetLastError();
}

bool conv_supported(int lk_hd, int lv_hd) { return lk_hd > 0 && lv_hd > 0 && lk_hd <= 1024 && lv_hd <= 1024; }

bool delta_supported(int lk_hd) { return lk_hd > 0 && lk_hd <= kDeltaIGroups * kDeltaMaxKPerThread; }

// ---------------------------------------------------------------------------
// standalone RMSNorm (ref_rmsnorm.cpp:8-17), used for the exposed final hidden.
// ---------------------------------------------------------------------------
__global__ void rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w, int n, float eps,
                               float* __restrict__ y) {
    __shared__ float red[32];
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) ss += x[i] * x[i];
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(n) + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) y[i] = x[i] * inv * w[i];
}

hipError_t launch_rmsnorm(const float* x, const float* w, int n, float eps, float* y, hipStream_t s) {
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(1024), 0, s, x, w, n, eps, y);
    return hipGetLastError();
}

}  // namespace xqhip
