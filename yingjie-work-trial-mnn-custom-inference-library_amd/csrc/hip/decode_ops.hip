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
#include "linear_step.hpp"

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
// Chunk kernel: grid (kv head kh, slot s), S = gridDim.y slots per kv head
// (about one block per CU in all).  The context of ctx tokens is cut into
// chunks of C tokens, C = attn_chunk_len(ctx, S): a power of two in [16, 64]
// large enough that the S slots cover the context in one chunk each where
// they can (ctx <= 64 S), so every slot has work at decode contexts; longer
// contexts give each slot chunks s, s + S, ...  For each chunk the block
// takes the `group` query heads of kv head kh: scores q.k/sqrt(d), the chunk's
// max m and sum l of exp(s - m), and sum exp(s - m) v; its chunks are merged
// in registers (rescaling by exp(m_old - m_new)), and the block writes one
// partial (m, l, o) per query head.
// Merge kernel: one block per query head combines the slots' partials
// (weights exp(m_s - M)), multiplies by 1/l (custom_model.cpp:901-904) and
// applies the sigmoid output gate.  The kernel boundary orders the two, so no
// block waits on another and no grid-wide fence is needed.
// ---------------------------------------------------------------------------
constexpr int kAttnChunk = 64;     // most tokens in one chunk
constexpr int kAttnMaxGroup = 8;
constexpr int kAttnMaxSlots = 64;  // slots per kv head = partials per query head
constexpr int kAttnMaxCtx = 1 << 20;
constexpr int kAttnThreads = 256;

// The head sizes with a compiled chunk kernel; others run the generic one (0).
__host__ __device__ inline int attn_hd_class(int head_dim) {
    return (head_dim == 64 || head_dim == 128 || head_dim == 256) ? head_dim : 0;
}
// Shortest chunk of a head size: the score phase splits a key over
// kAttnThreads / C lanes of at least 8 dims (one 16-byte load) each.
__host__ __device__ constexpr int attn_min_chunk(int hd_class) {
    return hd_class == 0 ? kAttnChunk : (2048 / hd_class > 16 ? 2048 / hd_class : 16);
}
__host__ __device__ inline int attn_chunk_len(int ctx, int slots, int hd_class) {
    const int want = (ctx + slots - 1) / slots;
    int c = attn_min_chunk(hd_class);
    while (c < want && c < kAttnChunk) c <<= 1;
    return c;
}
__host__ __device__ inline int attn_slots(int nkv) {
    const int s = 256 / (nkv > 0 ? nkv : 1);
    return s < 1 ? 1 : (s > kAttnMaxSlots ? kAttnMaxSlots : s);
}

// K and V of one chunk as this thread consumes them: K for the scores (LPK =
// 256 / C lanes per token, DL = HD / LPK consecutive dims each), V for the
// weighted sum (HD / 8 lanes per token, 8 dims each, tokens ts, ts + TPP, ...).
// Token indices past the chunk are clamped to its last token (in bounds, unused).
template <int HD, int C>
struct KvRegs {
    static constexpr int kLPK = kAttnThreads / C;
    static constexpr int kDL = HD / kLPK;
    static constexpr int kK = kDL / 8;                  // uint4 of K per thread
    static constexpr int kLPT = HD / 8;                 // lanes per token of V
    static constexpr int kTPP = kAttnThreads / kLPT;    // tokens per V pass
    static constexpr int kV = (C + kTPP - 1) / kTPP;    // V passes
    static_assert(kDL >= 8 && kDL % 8 == 0, "a score lane reads whole 16-byte pieces of K");
    uint4 k[kK];
    uint4 v[kV];
};

template <int HD, int C>
__device__ __forceinline__ void load_kv(const GqaLaunch& p, int kh, int t0, int n, KvRegs<HD, C>& r) {
    using R = KvRegs<HD, C>;
    const int sub = threadIdx.x % R::kLPK, tt = threadIdx.x / R::kLPK;
    const _Float16* krow = p.k_cache + (static_cast<size_t>(t0 + min(tt, n - 1)) * p.nkv + kh) * HD + sub * R::kDL;
#pragma unroll
    for (int u = 0; u < R::kK; ++u) r.k[u] = *reinterpret_cast<const uint4*>(krow + 8 * u);
    const int dsl = threadIdx.x % R::kLPT, ts = threadIdx.x / R::kLPT;
#pragma unroll
    for (int u = 0; u < R::kV; ++u) {
        const int t = min(ts + u * R::kTPP, n - 1);
        r.v[u] = *reinterpret_cast<const uint4*>(p.v_cache + (static_cast<size_t>(t0 + t) * p.nkv + kh) * HD + dsl * 8);
    }
}

// Per-thread running state of a block's chunks: items i = threadIdx.x + k *
// kAttnThreads of the group x HD outputs (head g = i / HD).
template <int HD>
struct AttnRun {
    static constexpr int kItems = (kAttnMaxGroup * (HD > 0 ? HD : 256) + kAttnThreads - 1) / kAttnThreads;
    float m[kItems], l[kItems], o[kItems];
};

// Merges a chunk (stats cm / cl per head in LDS, output `acc` of item k) into
// the running state.  The first chunk gives exactly (cm, cl, acc).
template <int HD>
__device__ __forceinline__ void run_merge(AttnRun<HD>& run, int k, float cm, float cl, float acc) {
    const float mn = fmaxf(run.m[k], cm);
    const float a = expf(run.m[k] - mn), b = expf(cm - mn);
    run.o[k] = run.o[k] * a + acc * b;
    run.l[k] = run.l[k] * a + cl * b;
    run.m[k] = mn;
}

// One chunk of C tokens (t0 .. t0 + n - 1, n <= C) for the query heads of kv
// head kh.  pos_new >= 0: the key/value of position pos_new come from kn / vn
// (LDS: the values the same launch appends to the cache) instead of the cache.
// LDS: qs [group][hd], sc [group][64] scores / weights, cst [2][8] chunk stats,
// vred [4 waves][group][hd].
template <int HD, int C>
__device__ __forceinline__ void gqa_chunk(const GqaLaunch& p, int kh, int t0, int n, int group, const float* qs,
                                          float* sc, float* cst, float* vred, const KvRegs<HD, C>& kvr,
                                          AttnRun<HD>& run, int pos_new, const float* kn, const float* vn) {
    using R = KvRegs<HD, C>;
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    const float rscale = 1.0f / sqrtf(static_cast<float>(HD));
    {  // scores
        const int sub = threadIdx.x % R::kLPK, tt = threadIdx.x / R::kLPK;
        const bool valid = tt < n;
        float kv[R::kDL];
#pragma unroll
        for (int u = 0; u < R::kK; ++u) {
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
            for (int d = 0; d < R::kDL; ++d) kv[d] = kn[sub * R::kDL + d];
        }
        for (int g = 0; g < group; ++g) {
            const float* qv = qs + g * HD + sub * R::kDL;
            float dot = 0.0f;
#pragma unroll
            for (int d = 0; d < R::kDL; ++d) dot += qv[d] * kv[d];
            dot = lanes_sum<R::kLPK>(dot);
            if (valid && sub == 0) sc[g * kAttnChunk + tt] = dot * rscale;
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
            cst[g] = m;
            cst[kAttnMaxGroup + g] = l;
        }
    }
    __syncthreads();
    {  // sum_t e_t v_t: 16-byte loads of v, HD/8 lanes per token
        static_assert(R::kLPT >= 8 && R::kLPT <= 32, "pair sums below cover lane distances 8..32");
        const int dsl = threadIdx.x % R::kLPT, ts = threadIdx.x / R::kLPT;
        float o[kAttnMaxGroup][8];
#pragma unroll
        for (int g = 0; g < kAttnMaxGroup; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e) o[g][e] = 0.0f;
#pragma unroll
        for (int u = 0; u < R::kV; ++u) {
            const int t = ts + u * R::kTPP;
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
                    if constexpr (R::kLPT <= 8) o[g][e] = xor_pair_sum<8>(o[g][e]);
                    if constexpr (R::kLPT <= 16) o[g][e] = xor_pair_sum<16>(o[g][e]);
                    o[g][e] = xor_pair_sum<32>(o[g][e]);
                }
            }
        }
        if (lane < R::kLPT) {
#pragma unroll
            for (int g = 0; g < kAttnMaxGroup; ++g)
                if (g < group)
#pragma unroll
                    for (int e = 0; e < 8; ++e) vred[(wid * group + g) * HD + dsl * 8 + e] = o[g][e];
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < AttnRun<HD>::kItems; ++k) {
        const int i = threadIdx.x + k * kAttnThreads;
        if (i < group * HD) {
            const int g = i / HD, d = i % HD;
            float acc = 0.0f;
#pragma unroll
            for (int w = 0; w < kAttnThreads / kWave; ++w) acc += vred[(w * group + g) * HD + d];
            run_merge<HD>(run, k, cst[g], cst[kAttnMaxGroup + g], acc);
        }
    }
    __syncthreads();  // sc, cst and vred are reused by the block's next chunk
}

// Generic head size (HD == 0, C == 64): the same steps with plain loops.
__device__ void gqa_chunk_generic(const GqaLaunch& p, int kh, int t0, int n, int group, int hd, const float* qs,
                                  float* sc, float* cst, AttnRun<0>& run, int pos_new, const float* kn,
                                  const float* vn) {
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    const float rscale = 1.0f / sqrtf(static_cast<float>(hd));
    for (int pr = threadIdx.x; pr < n * group; pr += kAttnThreads) {
        const int t = pr / group, g = pr % group;
        const _Float16* krow = p.k_cache + (static_cast<size_t>(t0 + t) * p.nkv + kh) * hd;
        const bool is_new = t0 + t == pos_new;
        float dot = 0.0f;
        for (int d = 0; d < hd; ++d) dot += qs[g * hd + d] * (is_new ? kn[d] : static_cast<float>(krow[d]));
        sc[g * kAttnChunk + t] = dot * rscale;
    }
    __syncthreads();
    for (int g = wid; g < group; g += kAttnThreads / kWave) {
        const float sv = lane < n ? sc[g * kAttnChunk + lane] : -INFINITY;
        const float m = wave_max(sv);
        const float e = lane < n ? expf(sv - m) : 0.0f;
        const float l = wave_sum(e);
        sc[g * kAttnChunk + lane] = e;
        if (lane == 0) {
            cst[g] = m;
            cst[kAttnMaxGroup + g] = l;
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < AttnRun<0>::kItems; ++k) {
        const int i = threadIdx.x + k * kAttnThreads;
        if (i < group * hd) {
            const int g = i / hd, d = i % hd;
            float acc = 0.0f;
            for (int t = 0; t < n; ++t)
                acc += sc[g * kAttnChunk + t] *
                       (t0 + t == pos_new ? vn[d]
                                          : static_cast<float>(p.v_cache[(static_cast<size_t>(t0 + t) * p.nkv + kh) * hd + d]));
            run_merge<0>(run, k, cst[g], cst[kAttnMaxGroup + g], acc);
        }
    }
    __syncthreads();
}

template <int HD>
__device__ __forceinline__ void run_init(AttnRun<HD>& run) {
#pragma unroll
    for (int k = 0; k < AttnRun<HD>::kItems; ++k) {
        run.m[k] = -INFINITY;
        run.l[k] = 0.0f;
        run.o[k] = 0.0f;
    }
}

// The block's partial (m, l, o) per query head of kv head kh, slot s.
template <int HD>
__device__ __forceinline__ void store_partial(const GqaLaunch& p, int kh, int s, int group, int hd,
                                              const AttnRun<HD>& run) {
#pragma unroll
    for (int k = 0; k < AttnRun<HD>::kItems; ++k) {
        const int i = threadIdx.x + k * kAttnThreads;
        if (i < group * hd) {
            const int g = i / hd, d = i % hd;
            const size_t ps = static_cast<size_t>(kh * group + g) * kAttnMaxSlots + s;
            p.part_o[ps * hd + d] = run.o[k];
            if (d == 0) {
                p.part_m[ps] = run.m[k];
                p.part_l[ps] = run.l[k];
            }
        }
    }
}

// The chunks of slot s (s, s + S, ...) given the prepared query heads in qs;
// the first chunk's K/V are already in kvr.
template <int HD, int C>
__device__ __forceinline__ void attn_slot(const GqaLaunch& p, int kh, int ctx, int group, const float* qs, float* sc,
                                          float* cst, float* vred, KvRegs<HD, C>& kvr, int pos_new, const float* kn,
                                          const float* vn) {
    const int s = blockIdx.y, S = gridDim.y;
    const int nch = (ctx + C - 1) / C;
    AttnRun<HD> run;
    run_init<HD>(run);
    for (int ch = s; ch < nch; ch += S) {
        const int t0 = ch * C;
        const int n = min(C, ctx - t0);
        if (ch != s) load_kv<HD, C>(p, kh, t0, n, kvr);
        gqa_chunk<HD, C>(p, kh, t0, n, group, qs, sc, cst, vred, kvr, run, pos_new, kn, vn);
    }
    store_partial<HD>(p, kh, s, group, HD, run);
}

// The kernel-level GQA (query heads already normalised and rotated in p.q).
template <int HD, int C>
__device__ __forceinline__ void gqa_block(const GqaLaunch& p, int kh, int ctx, int group, float* smem) {
    float* qs = smem;                       // [group][HD]
    float* sc = qs + group * HD;            // [group][64]
    float* cst = sc + group * kAttnChunk;   // [2][8]
    float* vred = cst + 2 * kAttnMaxGroup;  // [4 waves][group][HD]
    const int s = blockIdx.y;
    KvRegs<HD, C> kvr;
    load_kv<HD, C>(p, kh, s * C, min(C, ctx - s * C), kvr);
    for (int i = threadIdx.x; i < group * HD; i += kAttnThreads) qs[i] = p.q[static_cast<size_t>(kh) * group * HD + i];
    __syncthreads();
    attn_slot<HD, C>(p, kh, ctx, group, qs, sc, cst, vred, kvr, -1, nullptr, nullptr);
}

template <int HD>
__global__ void __launch_bounds__(kAttnThreads) gqa_chunk_kernel(GqaLaunch p) {
    extern __shared__ float smem[];
    const int group = p.nq / p.nkv;
    const int kh = blockIdx.x;
    const int ctx = *p.pos + 1;
    const int C = attn_chunk_len(ctx, gridDim.y, HD);
    if (static_cast<int>(blockIdx.y) * C >= ctx) return;  // no chunk for this slot: the merge skips it
    if constexpr (HD == 0) {
        const int hd = p.head_dim;
        float* qs = smem;
        float* sc = qs + group * hd;
        float* cst = sc + group * kAttnChunk;
        for (int i = threadIdx.x; i < group * hd; i += kAttnThreads) qs[i] = p.q[static_cast<size_t>(kh) * group * hd + i];
        __syncthreads();
        AttnRun<0> run;
        run_init<0>(run);
        const int nch = (ctx + C - 1) / C;
        for (int ch = blockIdx.y; ch < nch; ch += gridDim.y)
            gqa_chunk_generic(p, kh, ch * C, min(C, ctx - ch * C), group, hd, qs, sc, cst, run, -1, nullptr, nullptr);
        store_partial<0>(p, kh, blockIdx.y, group, hd, run);
    } else {
        if (C == 16 && attn_min_chunk(HD) <= 16) {
            if constexpr (attn_min_chunk(HD) <= 16) gqa_block<HD, 16>(p, kh, ctx, group, smem);
        } else if (C == 32) {
            gqa_block<HD, 32>(p, kh, ctx, group, smem);
        } else {
            gqa_block<HD, 64>(p, kh, ctx, group, smem);
        }
    }
}

// Decode attention with the q/k preparation folded in: every block normalises
// and rotates the q heads of its kv head (cheap), and the block whose chunks
// include position pos also prepares that position's key and value, appends
// them to the fp16 caches and uses them (rounded to fp16, like every cached
// position) from LDS; the slot this launch writes is never taken from memory.
template <int HD, int C>
__device__ __forceinline__ void attn_decode_block(const AttnDecodeLaunch& a, int kh, int pos, float* smem) {
    const GqaLaunch& p = a.g;
    const int group = p.nq / p.nkv;
    const int ctx = pos + 1;
    const int s = blockIdx.y, S = gridDim.y;
    float* qs = smem;                                        // [group][HD]
    float* sc = qs + group * HD;                             // [group][64]
    float* cst = sc + group * kAttnChunk;                    // [2][8]
    float* vred = cst + 2 * kAttnMaxGroup;                   // [4 waves][group][HD]
    float* kn = vred + (kAttnThreads / kWave) * group * HD;  // [HD]
    float* vn = kn + HD;                                     // [HD]
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    const int half = a.rotary_dim / 2;
    const bool owns_new = (pos / C) % S == s;
    // per-head RMSNorm (custom_model.cpp:301-313): heads 0..group-1 are q,
    // head `group` (owner only) is the new key; wave w takes heads w, w + 4, ...
    // The query loads are issued first, then the chunk's K/V, so the q
    // preparation runs while the cache streams in.
    constexpr int kPer = HD / kWave;  // values per lane of one head
    constexpr int kMaxHeadsPerWave = (kAttnMaxGroup + 1 + 3) / 4;
    const int nheads = group + (owns_new ? 1 : 0);
    float qr[kMaxHeadsPerWave][kPer];
#pragma unroll
    for (int j = 0; j < kMaxHeadsPerWave; ++j) {
        const int h = wid + 4 * j;
        if (h < nheads) {
            const bool is_k = h == group;
            const float* src = is_k ? a.k_src + static_cast<size_t>(kh) * HD
                                    : a.q_src + static_cast<size_t>(kh * group + h) * (a.gated ? 2 * HD : HD);
#pragma unroll
            for (int e = 0; e < kPer; ++e) qr[j][e] = src[lane + e * kWave];
        }
    }
    float vr[kPer > 0 ? (HD + kAttnThreads - 1) / kAttnThreads : 1];
    if (owns_new) {
#pragma unroll
        for (int e = 0; e < (HD + kAttnThreads - 1) / kAttnThreads; ++e) {
            const int d = threadIdx.x + e * kAttnThreads;
            vr[e] = d < HD ? a.v_src[static_cast<size_t>(kh) * HD + d] : 0.0f;
        }
    }
    KvRegs<HD, C> kvr;
    load_kv<HD, C>(p, kh, s * C, min(C, ctx - s * C), kvr);
#pragma unroll
    for (int j = 0; j < kMaxHeadsPerWave; ++j) {
        const int h = wid + 4 * j;
        if (h < nheads) {
            const bool is_k = h == group;
            const float* w = is_k ? a.k_norm : a.q_norm;
            float* dst = is_k ? kn : qs + h * HD;
            float ss = 0.0f;
#pragma unroll
            for (int e = 0; e < kPer; ++e) ss += qr[j][e] * qr[j][e];
            ss = wave_sum(ss);
            const float inv = 1.0f / sqrtf(ss / static_cast<float>(HD) + a.eps);
#pragma unroll
            for (int e = 0; e < kPer; ++e) {
                const int d = lane + e * kWave;
                dst[d] = qr[j][e] * (inv * w[d]);
            }
        }
    }
    if (owns_new) {
#pragma unroll
        for (int e = 0; e < (HD + kAttnThreads - 1) / kAttnThreads; ++e) {
            const int d = threadIdx.x + e * kAttnThreads;
            if (d < HD) vn[d] = vr[e];
        }
    }
    __syncthreads();
    // partial RoPE (custom_model.cpp:351-370) on the first rotary_dim dims, pairs (i, half + i)
    const float2* cs = reinterpret_cast<const float2*>(a.rope_cs) + static_cast<size_t>(pos) * a.rope_pairs;
    for (int i = threadIdx.x; i < nheads * half; i += kAttnThreads) {
        const int h = i / half, d = i % half;
        float* v = h == group ? kn : qs + h * HD;
        const float2 c = cs[d];
        const float x0 = v[d], x1 = v[half + d];
        v[d] = x0 * c.x - x1 * c.y;
        v[half + d] = x1 * c.x + x0 * c.y;
    }
    __syncthreads();
    if (owns_new) {  // append at slot pos, and use the fp16-rounded values like every other slot
        for (int d = threadIdx.x; d < HD; d += kAttnThreads) {
            const size_t slot = (static_cast<size_t>(pos) * p.nkv + kh) * HD + d;
            const _Float16 kq = static_cast<_Float16>(kn[d]), vq = static_cast<_Float16>(vn[d]);
            a.k_cache[slot] = kq;
            a.v_cache[slot] = vq;
            kn[d] = static_cast<float>(kq);
            vn[d] = static_cast<float>(vq);
        }
        __syncthreads();
    }
    attn_slot<HD, C>(p, kh, ctx, group, qs, sc, cst, vred, kvr, pos, kn, vn);
}

// Generic head size: the same steps with plain loops (C = 64).
__device__ void attn_decode_generic(const AttnDecodeLaunch& a, int kh, int pos, float* smem) {
    const GqaLaunch& p = a.g;
    const int hd = p.head_dim;
    const int group = p.nq / p.nkv;
    const int ctx = pos + 1;
    const int C = kAttnChunk;
    float* qs = smem;
    float* sc = qs + group * hd;
    float* cst = sc + group * kAttnChunk;
    float* kn = cst + 2 * kAttnMaxGroup;
    float* vn = kn + hd;
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    const int half = a.rotary_dim / 2;
    const bool owns_new = (pos / C) % static_cast<int>(gridDim.y) == static_cast<int>(blockIdx.y);
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
    const float2* cs = reinterpret_cast<const float2*>(a.rope_cs) + static_cast<size_t>(pos) * a.rope_pairs;
    for (int i = threadIdx.x; i < nheads * half; i += kAttnThreads) {
        const int h = i / half, d = i % half;
        float* v = h == group ? kn : qs + h * hd;
        const float2 c = cs[d];
        const float x0 = v[d], x1 = v[half + d];
        v[d] = x0 * c.x - x1 * c.y;
        v[half + d] = x1 * c.x + x0 * c.y;
    }
    __syncthreads();
    if (owns_new) {
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
    AttnRun<0> run;
    run_init<0>(run);
    const int nch = (ctx + C - 1) / C;
    for (int ch = blockIdx.y; ch < nch; ch += gridDim.y)
        gqa_chunk_generic(p, kh, ch * C, min(C, ctx - ch * C), group, hd, qs, sc, cst, run, pos, kn, vn);
    store_partial<0>(p, kh, blockIdx.y, group, hd, run);
}

template <int HD>
__global__ void __launch_bounds__(kAttnThreads) attn_decode_kernel(AttnDecodeLaunch a) {
    extern __shared__ float smem[];
    const int kh = blockIdx.x;
    const int pos = *a.g.pos;
    const int ctx = pos + 1;
    const int C = attn_chunk_len(ctx, gridDim.y, HD);
    if (static_cast<int>(blockIdx.y) * C >= ctx) return;  // no chunk for this slot: the merge skips it
    if constexpr (HD == 0) {
        attn_decode_generic(a, kh, pos, smem);
    } else {
        if (C == 16 && attn_min_chunk(HD) <= 16) {
            if constexpr (attn_min_chunk(HD) <= 16) attn_decode_block<HD, 16>(a, kh, pos, smem);
        } else if (C == 32) {
            attn_decode_block<HD, 32>(a, kh, pos, smem);
        } else {
            attn_decode_block<HD, 64>(a, kh, pos, smem);
        }
    }
}

// One block per query head: merge the partials of the slots that had chunks,
// normalise by multiplying with 1/l (custom_model.cpp:901-904), apply the gate.
// The first wave takes one slot per lane (max, weights exp(m_s - M), l), the
// block then sums the slots' outputs with those weights.
__global__ void __launch_bounds__(256) gqa_combine_kernel(GqaLaunch p, int slots) {
    static_assert(kAttnMaxSlots <= kWave, "one slot per lane of the first wave");
    __shared__ float wgt[kAttnMaxSlots];
    __shared__ float inv_l;
    const int qh = blockIdx.x;
    const int hd = p.head_dim;
    const int ctx = *p.pos + 1;
    const int C = attn_chunk_len(ctx, slots, attn_hd_class(hd));
    const int nact = min(slots, (ctx + C - 1) / C);
    if (threadIdx.x < kWave) {
        const int sl = threadIdx.x;
        const size_t ps = static_cast<size_t>(qh) * kAttnMaxSlots + sl;
        const float m = sl < nact ? p.part_m[ps] : -INFINITY;
        const float l = sl < nact ? p.part_l[ps] : 0.0f;
        const float M = wave_max(m);
        const float w = sl < nact ? expf(m - M) : 0.0f;
        const float tot = wave_sum(l * w);
        wgt[sl] = w;
        if (sl == 0) inv_l = tot > 0.0f ? 1.0f / tot : 0.0f;
    }
    __syncthreads();
    const float inv = inv_l;
    const float* po = p.part_o + static_cast<size_t>(qh) * kAttnMaxSlots * hd;
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        float o = 0.0f;
        for (int s0 = 0; s0 < nact; s0 += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = s0 + u < nact ? po[static_cast<size_t>(s0 + u) * hd + d] : 0.0f;
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (s0 + u < nact) o += v[u] * wgt[s0 + u];
        }
        const size_t oi = static_cast<size_t>(qh) * hd + d;
        // no gate projection: the reference's zero gate, sigmoid(0) (custom_model.cpp:750-753)
        const float gv = p.gate ? p.gate[static_cast<size_t>(qh) * p.gate_stride + d] : 0.0f;
        p.out[oi] = (o * inv) * sigmoid_dev(gv);
    }
}

size_t gqa_workspace_bytes(int nq, int nkv, int head_dim) {
    (void)nkv;
    return sizeof(float) * static_cast<size_t>(nq) * kAttnMaxSlots * (head_dim + 2);
}

static size_t gqa_lds_bytes(int group, int head_dim) {
    return sizeof(float) * (static_cast<size_t>(group) * head_dim + static_cast<size_t>(group) * kAttnChunk +
                            2 * kAttnMaxGroup + (kAttnThreads / kWave) * static_cast<size_t>(group) * head_dim);
}

static int combine_threads(int head_dim) { return min(256, max(64, ((head_dim + 63) / 64) * 64)); }

hipError_t launch_attn_decode(const AttnDecodeLaunch& a, hipStream_t s) {
    const GqaLaunch& p = a.g;
    const int group = p.nq / p.nkv;
    const size_t lds = gqa_lds_bytes(group, p.head_dim) + 2 * sizeof(float) * p.head_dim;
    const int slots = attn_slots(p.nkv);
    const dim3 grid(p.nkv, slots);
    switch (attn_hd_class(p.head_dim)) {
        case 64: hipLaunchKernelGGL(attn_decode_kernel<64>, grid, dim3(kAttnThreads), lds, s, a); break;
        case 128: hipLaunchKernelGGL(attn_decode_kernel<128>, grid, dim3(kAttnThreads), lds, s, a); break;
        case 256: hipLaunchKernelGGL(attn_decode_kernel<256>, grid, dim3(kAttnThreads), lds, s, a); break;
        default: hipLaunchKernelGGL(attn_decode_kernel<0>, grid, dim3(kAttnThreads), lds, s, a); break;
    }
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    hipLaunchKernelGGL(gqa_combine_kernel, dim3(p.nq), dim3(combine_threads(p.head_dim)), 0, s, p, slots);
    return hipGetLastError();
}

hipError_t launch_gqa(const GqaLaunch& p, hipStream_t s) {
    const int group = p.nq / p.nkv;
    const size_t lds = gqa_lds_bytes(group, p.head_dim);
    const int slots = attn_slots(p.nkv);
    const dim3 grid(p.nkv, slots);
    switch (attn_hd_class(p.head_dim)) {
        case 64: hipLaunchKernelGGL(gqa_chunk_kernel<64>, grid, dim3(kAttnThreads), lds, s, p); break;
        case 128: hipLaunchKernelGGL(gqa_chunk_kernel<128>, grid, dim3(kAttnThreads), lds, s, p); break;
        case 256: hipLaunchKernelGGL(gqa_chunk_kernel<256>, grid, dim3(kAttnThreads), lds, s, p); break;
        default: hipLaunchKernelGGL(gqa_chunk_kernel<0>, grid, dim3(kAttnThreads), lds, s, p); break;
    }
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    hipLaunchKernelGGL(gqa_combine_kernel, dim3(p.nq), dim3(combine_threads(p.head_dim)), 0, s, p, slots);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Decode attention with one block per query head, no merge kernel: the block
// reads its kv head's cached context in passes of up to kHeadPass tokens with
// the whole pass in flight, so at decode contexts a full-attention layer is
// one launch.  Same per-head preparation as attn_decode_kernel (q and the new
// key normalised and rotated, the new key / value used fp16-rounded from LDS;
// the first query head of each kv head appends them to the caches), then
// scores, one softmax (max subtracted, 1/l multiplied as
// custom_model.cpp:901-904) and the gated output.  Passes are merged with a
// running max (exp(m_old - m_new) rescale).
// HD = 128: 4 lanes per token for the scores (32 dims, four 16-byte K loads),
// 16 lanes per token for the value sum (8 dims, one 16-byte V load).  The
// value loads of each 128-token score sub-pass are issued as soon as its keys
// are consumed (they take over the key registers).  The new token's score and
// value come from LDS: cache rows are read only for the positions before it.
// Every load is straight-line code (range-checked buffer loads read 0 past
// the cached positions): a load under a branch makes the compiler's wait for
// any earlier load a wait for all of them.  The kernel picks, from the
// position, a body whose first pass has just enough 128-token sub-passes.
// ---------------------------------------------------------------------------
constexpr int kHeadThreads = 512;
constexpr int kHeadPass = 1024;                    // tokens per pass
constexpr int kHeadKSub = kHeadThreads / 4;        // tokens per K sub-pass (128)
constexpr int kHeadKSubs = kHeadPass / kHeadKSub;  // 8
constexpr int kHeadVTok = kHeadThreads / 16;       // tokens per V sub-pass (32)
constexpr int kHeadVPerK = kHeadKSub / kHeadVTok;  // V sub-passes per K sub-pass (4)

template <int HD>
struct HeadSmem {
    float qs[HD], kn[HD], vn[HD], gate[HD];
    float sc[kHeadPass];
    float red[kHeadThreads / kWave];
    float fresh_s;
    float ored[kHeadThreads / kWave][HD + 1];
};

__device__ __forceinline__ uint4 buf_load_u4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}

// Orders one wave's LDS accesses: a wave's LDS instructions execute in issue
// order, so after this point its lanes see each other's earlier LDS writes
// (the fences keep the compiler from moving LDS accesses across it); no block
// barrier is involved.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One query head over the cached positions [c0, c1) and, when `fresh`, the new
// token at `pos` (appended to the caches by the first query head of each kv
// head), with first-pass sub-passes KS (later passes, for ranges past one
// pass, use all the pass's sub-passes).  PART: the unnormalised result goes to
// part_out (running max, exp sum, sum of exp-weighted values; the consumer
// merges the ranges and applies 1/l and the gate); otherwise the gated output.
// A pass is kHeadPass tokens for the per-head kernel and half that for the
// split kernel (whose ranges are an eighth of the context), which keeps the
// split kernel's longest body within the register file.
// kPassSubs(PART): 128-token sub-passes per pass
template <bool PART>
constexpr int kPassSubs = PART ? kHeadKSubs / 2 : kHeadKSubs;

template <int HD, int KS, bool PART>
__device__ __forceinline__ void head_attention(const AttnDecodeLaunch& a, HeadSmem<HD>& sm, int pos, int c0, int c1,
                                               bool fresh, float* part_out) {
    static_assert(HD == 128, "4 score lanes x 32 dims, 16 value lanes x 8 dims");
    constexpr int kWaves = kHeadThreads / kWave;
    constexpr int kSubs = kPassSubs<PART>;
    constexpr int kPass = kSubs * kHeadKSub;  // tokens per pass
    static_assert(KS >= 1 && KS <= kSubs, "first-pass sub-passes");
    // the first pass's values are requested with its keys when both fit the
    // register budget beside each other (up to 512 tokens)
    constexpr bool kVPre = KS <= 4;
    const GqaLaunch& p = a.g;
    const int group = p.nq / p.nkv;
    // blocks b, b + nkv, b + 2 nkv, ... take the query heads of one kv head:
    // blocks are dealt to the 8 XCDs round robin, so with nkv a multiple of 8
    // a kv head's blocks share one XCD's L2 and its K / V come from memory once
    const int kh = static_cast<int>(blockIdx.x) % p.nkv;
    const int qh = kh * group + static_cast<int>(blockIdx.x) / p.nkv;
    const bool owner = fresh && qh % group == 0;  // appends the new key / value of kv head kh
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wid = tid / kWave;
    const int sub = tid & 3, tt = tid >> 2;   // score lanes: dims 32 u + 8 sub + e of token tt
    const int dsl = tid & 15, ts = tid >> 4;  // value lanes: dims 8 dsl + e of token ts
    const float rscale = 1.0f / sqrtf(static_cast<float>(HD));
    const size_t kv_stride = static_cast<size_t>(p.nkv) * HD;
    const uint32_t row_bytes = static_cast<uint32_t>(kv_stride) * 2u;  // one position of a cache
    // query (wave 0), new key (wave 1), new value (wave 2, and the idle waves),
    // their norm weights, the RoPE pair and the gate
    const float* src = wid == 0 ? a.q_src + static_cast<size_t>(qh) * (a.gated ? 2 * HD : HD)
                                : (wid == 1 ? a.k_src : a.v_src) + static_cast<size_t>(kh) * HD;
    const float* nw = wid == 0 ? a.q_norm : a.k_norm;
    const float hv0 = src[lane], hv1 = src[lane + kWave];
    const float w0 = nw[lane], w1 = nw[lane + kWave];
    const int half = a.rotary_dim / 2;  // <= HD / 2 = kWave: one rotary pair per lane of waves 0 and 1
    const __amdgpu_buffer_rsrc_t r_cs =
        buf_rsrc(a.rope_cs, half > 0 ? static_cast<uint32_t>(pos + 1) * a.rope_pairs * 8u : 0u);
    const uint32_t cs_off =
        wid < 2 && lane < half ? (static_cast<uint32_t>(pos) * a.rope_pairs + lane) * 8u : kBufOOB;
    const auto csw = __builtin_amdgcn_raw_buffer_load_b64(r_cs, cs_off, 0, 0);
    // no gate projection: the reference's zero gate, sigmoid(0) (custom_model.cpp:750-753)
    const __amdgpu_buffer_rsrc_t r_gate =
        buf_rsrc(p.gate, p.gate ? static_cast<uint32_t>(p.nq) * p.gate_stride * 4u : 0u);
    const float gv = buf_load_f32(
        r_gate, !PART && tid < HD ? (static_cast<uint32_t>(qh) * p.gate_stride + tid) * 4u : kBufOOB);
    // the keys of a pass: cached positions [t0, t0 + nc), rows past nc read 0
    auto load_k = [&](int t0, int nc, auto& kr) {
        constexpr int J = sizeof(kr) / sizeof(kr[0]);
        const __amdgpu_buffer_rsrc_t r = buf_rsrc(p.k_cache + static_cast<size_t>(t0) * kv_stride + kh * HD,
                                                  static_cast<uint32_t>(nc) * row_bytes);
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
            for (int u = 0; u < 4; ++u)
                kr[j][u] = buf_load_u4(r, static_cast<uint32_t>(tt + kHeadKSub * j) * row_bytes + sub * 16u + u * 64u);
    };
    // the values of cached positions [t0, t0 + nc), rows past nc read 0: value
    // sub-pass jj (32 tokens) of this thread is token ts + 32 jj
    auto load_v = [&](int t0, int nc, auto& vr) {
        constexpr int JV = sizeof(vr) / sizeof(vr[0]);
        const __amdgpu_buffer_rsrc_t r = buf_rsrc(p.v_cache + static_cast<size_t>(t0) * kv_stride + kh * HD,
                                                  static_cast<uint32_t>(nc) * row_bytes);
#pragma unroll
        for (int jj = 0; jj < JV; ++jj)
            vr[jj] = buf_load_u4(r, static_cast<uint32_t>(ts + kHeadVTok * jj) * row_bytes + dsl * 16u);
    };
    uint4 kr[KS][4];
    uint4 vpre[kVPre ? KS * kHeadVPerK : 1];
    load_k(c0, min(kPass, c1 - c0), kr);
    if constexpr (kVPre) load_v(c0, min(kPass, c1 - c0), vpre);
    // per-head RMSNorm (custom_model.cpp:301-313) of q (wave 0) and k (wave 1),
    // then their partial RoPE (custom_model.cpp:351-370), pairs (i, half + i),
    // each wave on its own LDS row (wave_lds_sync, no block barrier); the new
    // key (wave 1) and value (wave 2) enter the cache in fp16 and are used
    // rounded, like every slot, appended by the kv head's first query head
    const size_t slot = static_cast<size_t>(pos) * kv_stride + static_cast<size_t>(kh) * HD;
    if (wid < 2) {
        float ss = hv0 * hv0 + hv1 * hv1;
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss / static_cast<float>(HD) + a.eps);
        float* dst = wid == 0 ? sm.qs : sm.kn;
        dst[lane] = hv0 * (inv * w0);
        dst[lane + kWave] = hv1 * (inv * w1);
        wave_lds_sync();
        if (lane < half) {
            const float cx = __uint_as_float(csw[0]), cy = __uint_as_float(csw[1]);
            const float x0 = dst[lane], x1 = dst[half + lane];
            dst[lane] = x0 * cx - x1 * cy;
            dst[half + lane] = x1 * cx + x0 * cy;
        }
        if (wid == 1) {
            wave_lds_sync();
            const _Float16 k0 = static_cast<_Float16>(sm.kn[lane]), k1 = static_cast<_Float16>(sm.kn[lane + kWave]);
            if (owner) {
                a.k_cache[slot + lane] = k0;
                a.k_cache[slot + lane + kWave] = k1;
            }
            sm.kn[lane] = static_cast<float>(k0);
            sm.kn[lane + kWave] = static_cast<float>(k1);
        }
    } else if (wid == 2) {
        const _Float16 v0 = static_cast<_Float16>(hv0), v1 = static_cast<_Float16>(hv1);
        if (owner) {
            a.v_cache[slot + lane] = v0;
            a.v_cache[slot + lane + kWave] = v1;
        }
        sm.vn[lane] = static_cast<float>(v0);
        sm.vn[lane + kWave] = static_cast<float>(v1);
    }
    if (tid < HD) sm.gate[tid] = gv;
    __syncthreads();
    // q in registers, in the score lanes' dim order
    float qreg[32];
#pragma unroll
    for (int d = 0; d < 32; ++d) qreg[d] = sm.qs[(d >> 3) * 32 + sub * 8 + (d & 7)];
    // the new token's score (the last wave; pos lies in the last pass)
    if (wid == kWaves - 1) {
        float s = sm.qs[lane] * sm.kn[lane] + sm.qs[lane + kWave] * sm.kn[lane + kWave];
        s = wave_sum(s);
        if (lane == 0) sm.fresh_s = s * rscale;
    }
    float run_m = -INFINITY, l = 0.0f, o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = 0.0f;
    // one pass over cached positions [t0, t0 + nc) with their keys in kp (and
    // the new token when it falls in this pass)
    // (vr: the pass's values, already requested when VLOADED, else requested
    // sub-pass by sub-pass as the keys are consumed)
    auto pass = [&](int t0, const auto& kp, auto& vr, auto vloaded) {
        constexpr int J = sizeof(kp) / sizeof(kp[0]);
        constexpr bool kLoaded = decltype(vloaded)::value;
        const int nc = min(kPass, c1 - t0);
        const bool last = fresh && c1 - t0 < kPass;
        const __amdgpu_buffer_rsrc_t r_v = buf_rsrc(p.v_cache + static_cast<size_t>(t0) * kv_stride + kh * HD,
                                                    static_cast<uint32_t>(nc) * row_bytes);
        float m = -INFINITY;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int tl = tt + kHeadKSub * j;
            float dot = 0.0f;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t ww[4] = {kp[j][u].x, kp[j][u].y, kp[j][u].z, kp[j][u].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    dot += qreg[8 * u + 2 * e] * half_lo(ww[e]);
                    dot += qreg[8 * u + 2 * e + 1] * half_hi(ww[e]);
                }
            }
            dot = lanes_sum<4>(dot) * rscale;
            if (tl < nc) {
                if (sub == 0) sm.sc[tl] = dot;
                m = fmaxf(m, dot);
            }
            // the values of these 128 tokens, into the registers the keys held
            if constexpr (!kLoaded) {
#pragma unroll
                for (int r = 0; r < kHeadVPerK; ++r) {
                    const int jj = kHeadVPerK * j + r;
                    vr[jj] = buf_load_u4(r_v, static_cast<uint32_t>(ts + kHeadVTok * jj) * row_bytes + dsl * 16u);
                }
            }
        }
        m = wave_max(m);
        if (lane == 0) sm.red[wid] = m;
        __syncthreads();  // also orders the last wave's fresh_s before it is read
        m = last ? sm.fresh_s : -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) m = fmaxf(m, sm.red[w]);
        const float mn = fmaxf(run_m, m);
        const float f_old = expf(run_m - mn);
        l *= f_old;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] *= f_old;
        run_m = mn;
        // sum_t exp(s_t - m) v_t over this thread's tokens ts, ts + 32, ...
#pragma unroll
        for (int jj = 0; jj < J * kHeadVPerK; ++jj) {
            const int tl = ts + kHeadVTok * jj;
            if (tl < nc) {
                const float pr = expf(sm.sc[tl] - mn);
                l += pr;
                o[0] += pr * half_lo(vr[jj].x);
                o[1] += pr * half_hi(vr[jj].x);
                o[2] += pr * half_lo(vr[jj].y);
                o[3] += pr * half_hi(vr[jj].y);
                o[4] += pr * half_lo(vr[jj].z);
                o[5] += pr * half_hi(vr[jj].z);
                o[6] += pr * half_lo(vr[jj].w);
                o[7] += pr * half_hi(vr[jj].w);
            }
        }
        if (last && ts == 0) {  // the new token, once per dim slice
            const float pr = expf(sm.fresh_s - mn);
            l += pr;
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] += pr * sm.vn[dsl * 8 + e];
        }
        __syncthreads();  // sc and red are rewritten by the next pass
    };
    if constexpr (kVPre) {
        pass(c0, kr, vpre, std::true_type{});
    } else {
        uint4 vr[KS * kHeadVPerK];
        pass(c0, kr, vr, std::false_type{});
    }
    // longer ranges: further passes of kSubs sub-passes, each loading its
    // keys first (kept apart from the first pass so that no key register lives
    // across a value phase); the new token may open a pass of its own
    for (int t0 = c0 + kPass; fresh ? t0 <= c1 : t0 < c1; t0 += kPass) {
        uint4 kr2[kSubs][4];
        uint4 vr2[kSubs * kHeadVPerK];
        load_k(t0, min(kPass, c1 - t0), kr2);
        pass(t0, kr2, vr2, std::false_type{});
    }
    // lanes with the same dsl: 4 per wave (16 apart), then the waves through LDS;
    // l is the same in every dsl lane of a token group and reduces alongside
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = xor_pair_sum<32>(xor_pair_sum<16>(o[e]));
    l = xor_pair_sum<32>(xor_pair_sum<16>(l));
    if (lane < 16) {
#pragma unroll
        for (int e = 0; e < 8; ++e) sm.ored[wid][dsl * 8 + e] = o[e];
        if (lane == 0) sm.ored[wid][HD] = l;
    }
    __syncthreads();
    if (tid < HD) {
        float acc = 0.0f, lt = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            acc += sm.ored[w][tid];
            lt += sm.ored[w][HD];
        }
        if constexpr (PART) {  // written through to memory: the merging block may run on another XCD
            __hip_atomic_store(part_out + kAttnPartO + tid, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (tid == 0) {
                __hip_atomic_store(part_out, run_m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(part_out + 1, lt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        } else {
            p.out[static_cast<size_t>(qh) * HD + tid] = (acc * (1.0f / lt)) * sigmoid_dev(sm.gate[tid]);
        }
    }
}

template <int HD>
__global__ void __launch_bounds__(kHeadThreads) attn_decode_head_kernel(AttnDecodeLaunch a) {
    __shared__ HeadSmem<HD> sm;
    const int pos = *a.g.pos;
    // 128-token sub-passes holding the first pass's cached positions
    const int ks = max(1, (min(pos, kHeadPass) + kHeadKSub - 1) / kHeadKSub);
    switch (ks) {
        case 1: head_attention<HD, 1, false>(a, sm, pos, 0, pos, true, nullptr); break;
        case 2: head_attention<HD, 2, false>(a, sm, pos, 0, pos, true, nullptr); break;
        case 3: head_attention<HD, 3, false>(a, sm, pos, 0, pos, true, nullptr); break;
        case 4: head_attention<HD, 4, false>(a, sm, pos, 0, pos, true, nullptr); break;
        case 5: head_attention<HD, 5, false>(a, sm, pos, 0, pos, true, nullptr); break;
        case 6: head_attention<HD, 6, false>(a, sm, pos, 0, pos, true, nullptr); break;
        case 7: head_attention<HD, 7, false>(a, sm, pos, 0, pos, true, nullptr); break;
        default: head_attention<HD, 8, false>(a, sm, pos, 0, pos, true, nullptr); break;
    }
}

// The context split over gridDim.y blocks per query head: split s takes the
// cached positions [s per, (s + 1) per) (per = ceil(pos / splits)), the last
// split also the new token, and each writes its partial to
// part[s][query head][kAttnPartStride] with write-through stores.  Once they
// are complete the block counts itself on the query head's counter
// (cnt[head * 32], zero before the launch), and the block that completes the
// count merges the head's partials (loads that bypass the per-XCD L2: the
// splits may run on other XCDs), weights exp(m_s - max m), multiplies by 1 / l
// (custom_model.cpp:901-904) and the sigmoid gate, writes a.g.out and sets the
// counter back to 0; no block waits for another.  With one split the result is
// the single-block kernel's, bit for bit, up to 512 cached positions (one pass
// of this kernel; the single-block kernel's passes are twice as long).
template <int HD>
__global__ void __launch_bounds__(kHeadThreads) attn_decode_part_kernel(AttnDecodeLaunch a, float* part,
                                                                        uint32_t* cnt) {
    __shared__ HeadSmem<HD> sm;
    const int pos = *a.g.pos;
    const int splits = static_cast<int>(gridDim.y), sp = static_cast<int>(blockIdx.y);
    const int per = (pos + splits - 1) / splits;
    const int c0 = min(pos, sp * per), c1 = min(pos, c0 + per);
    const bool fresh = sp == splits - 1;
    const int kh = static_cast<int>(blockIdx.x) % a.g.nkv;
    const int qh = kh * (a.g.nq / a.g.nkv) + static_cast<int>(blockIdx.x) / a.g.nkv;
    float* out = part + (static_cast<size_t>(sp) * a.g.nq + qh) * kAttnPartStride;
    if (!fresh && c0 == c1) {  // nothing cached in this range (block-uniform): an empty partial
        if (threadIdx.x < HD)
            __hip_atomic_store(out + kAttnPartO + threadIdx.x, 0.0f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (threadIdx.x == 0) {
            __hip_atomic_store(out, -INFINITY, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(out + 1, 0.0f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    } else {
        constexpr int kSubs = kPassSubs<true>;
        const int ks = max(1, (min(c1 - c0, kSubs * kHeadKSub) + kHeadKSub - 1) / kHeadKSub);
        switch (ks) {
            case 1: head_attention<HD, 1, true>(a, sm, pos, c0, c1, fresh, out); break;
            case 2: head_attention<HD, 2, true>(a, sm, pos, c0, c1, fresh, out); break;
            case 3: head_attention<HD, 3, true>(a, sm, pos, c0, c1, fresh, out); break;
            default: head_attention<HD, kSubs, true>(a, sm, pos, c0, c1, fresh, out); break;
        }
    }
    // Ordering without fences: every partial store above is an agent-scope
    // store (written through the L2) and this wait completes them, so they
    // are visible device-wide before the counter's atomic is issued; the
    // merging block reads them with agent-scope loads (which bypass the L2)
    // after its atomic has returned the final count.  That is the release /
    // acquire sequence of the target's memory model minus its L2 write-back
    // and invalidate, which only non-agent-scope accesses would need (and
    // which cost 22-32 us per launch when measured).  Records are padded to
    // whole 128-byte lines.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partial stores are complete
    __syncthreads();
    __shared__ int last;
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(cnt + qh * 32, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               static_cast<uint32_t>(splits - 1);
    __syncthreads();
    if (!last) return;  // block-uniform
    if (threadIdx.x < HD) {
        const int tid = threadIdx.x;
        // no gate projection: the reference's zero gate, sigmoid(0) (custom_model.cpp:750-753)
        const float g = a.g.gate ? a.g.gate[static_cast<size_t>(qh) * a.g.gate_stride + tid] : 0.0f;
        float mv[kAttnMaxSplits], lv[kAttnMaxSplits], ov[kAttnMaxSplits];
        float M = -INFINITY;
#pragma unroll
        for (int s2 = 0; s2 < kAttnMaxSplits; ++s2) {
            const float* q2 = part + (static_cast<size_t>(min(s2, splits - 1)) * a.g.nq + qh) * kAttnPartStride;
            mv[s2] = __hip_atomic_load(q2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            lv[s2] = __hip_atomic_load(q2 + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ov[s2] = __hip_atomic_load(q2 + kAttnPartO + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (int s2 = 0; s2 < kAttnMaxSplits; ++s2) {
            if (s2 >= splits) mv[s2] = -INFINITY;  // re-read of the last split: weight 0
            M = fmaxf(M, mv[s2]);
        }
        float L = 0.0f, acc = 0.0f;
#pragma unroll
        for (int s2 = 0; s2 < kAttnMaxSplits; ++s2) {
            const float wgt = expf(mv[s2] - M);  // an empty range (m = -inf): 0
            L += wgt * lv[s2];
            acc += wgt * ov[s2];
        }
        a.g.out[static_cast<size_t>(qh) * HD + tid] = (acc * (1.0f / L)) * sigmoid_dev(g);
    }
    if (threadIdx.x == 0) __hip_atomic_store(cnt + qh * 32, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

bool attn_head_supported(int nq, int nkv, int head_dim) {
    return head_dim == 128 && nkv > 0 && nq >= nkv && nq % nkv == 0;
}

hipError_t launch_attn_decode_head(const AttnDecodeLaunch& a, hipStream_t s) {
    hipLaunchKernelGGL(attn_decode_head_kernel<128>, dim3(a.g.nq), dim3(kHeadThreads), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_attn_decode_part(const AttnDecodeLaunch& a, int splits, float* part, uint32_t* cnt, hipStream_t s) {
    hipLaunchKernelGGL(attn_decode_part_kernel<128>, dim3(a.g.nq, splits), dim3(kHeadThreads), 0, s, a, part, cnt);
    return hipGetLastError();
}

bool gqa_supported(int nq, int nkv, int head_dim, int max_ctx) {
    if (nkv <= 0 || nq % nkv != 0 || nq / nkv > kAttnMaxGroup || head_dim <= 0) return false;
    if (max_ctx < 1 || max_ctx > kAttnMaxCtx) return false;
    if (attn_hd_class(head_dim) == 0 && head_dim > 256) return false;  // items per thread of AttnRun<0>
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

// Fused linear-attention step: the block body is linear_step_body
// (linear_step.hpp); one 256-thread block per (value head, 16-column slice).
template <int KS>
__global__ void __launch_bounds__(256) linear_step_kernel(LinearStepLaunch p) {
    __shared__ StepSmem sm;
    linear_step_body<KS, false>(p, static_cast<int>(blockIdx.x), static_cast<int>(blockIdx.y),
                                threadIdx.x, sm, StepHandOff{nullptr, nullptr});
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

// ---------------------------------------------------------------------------
// Timestamp: one thread stores the device's 100 MHz realtime counter to *slot
// with a system-scope store (a slot in coherent host memory is read by the
// host without a copy).  Between two kernels of a stream it marks the end of
// the first and the start of the second; used to time the ops of a traced
// decode-step graph, where event-record nodes give no timings.
// ---------------------------------------------------------------------------
__global__ void timestamp_kernel(uint64_t* slot) {
    __hip_atomic_store(slot, static_cast<uint64_t>(__builtin_amdgcn_s_memrealtime()), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_SYSTEM);
}

hipError_t launch_timestamp(uint64_t* slot, hipStream_t s) {
    hipLaunchKernelGGL(timestamp_kernel, dim3(1), dim3(1), 0, s, slot);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// LDS fill (a diagnostic for tests): every block writes `value` over the whole
// LDS a block may hold, so a kernel launched next on the same stream finds it
// wherever it reads LDS it has not written itself (LDS keeps its contents
// between kernels).
// ---------------------------------------------------------------------------
constexpr int kLdsFillBytes = 160 * 1024;
__global__ void __launch_bounds__(1024) lds_fill_kernel(float value) {
    extern __shared__ float lds_all[];
    volatile float* l = lds_all;  // stores nothing reads in this kernel stay
    for (int i = threadIdx.x; i < kLdsFillBytes / 4; i += 1024) l[i] = value;
}

hipError_t launch_lds_fill(float value, hipStream_t s) {
    const auto fn = reinterpret_cast<const void*>(&lds_fill_kernel);
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsFillBytes);
    if (e != hipSuccess) return e;
    int dev = 0, cus = 0;
    if ((e = hipGetDevice(&dev)) != hipSuccess) return e;
    if ((e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
    // one block fills a CU's whole LDS, so no two run on one CU at once; twice
    // the CU count reaches every CU
    hipLaunchKernelGGL(lds_fill_kernel, dim3(2 * cus), dim3(1024), kLdsFillBytes, s, value);
    return hipGetLastError();
}

hipError_t launch_rmsnorm(const float* x, const float* w, int n, float eps, float* y, hipStream_t s) {
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(1024), 0, s, x, w, n, eps, y);
    return hipGetLastError();
}

}  // namespace xqhip
