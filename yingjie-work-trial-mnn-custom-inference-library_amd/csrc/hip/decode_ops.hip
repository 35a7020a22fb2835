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

constexpr int kAttnSplits = 16;
constexpr int kAttnMaxGroup = 8;
constexpr int kAttnMaxSlice = 1024;  // tokens per split: context <= 16384

// ---------------------------------------------------------------------------
// embedding: bf16 row -> fp32 hidden (exact), token read from device memory.
// ---------------------------------------------------------------------------
__global__ void embed_bf16_kernel(const uint16_t* __restrict__ table, int vocab, int hidden,
                                  const int32_t* __restrict__ tok_ptr, float* __restrict__ out) {
    int tok = *tok_ptr;
    if (tok < 0 || tok >= vocab) tok = abs(tok) % max(1, vocab);
    const uint16_t* row = table + static_cast<size_t>(tok) * hidden;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x)
        out[i] = __uint_as_float(static_cast<uint32_t>(row[i]) << 16);
}

hipError_t launch_embed(const EmbedLaunch& p, hipStream_t s) {
    const int blocks = min(16, (p.hidden + 255) / 256);
    hipLaunchKernelGGL(embed_bf16_kernel, dim3(blocks), dim3(256), 0, s, p.table, p.vocab, p.hidden, p.tok, p.out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Full-attention head preparation.  Block b < nq: query head b (split from the
// gated q_proj output, per-head RMSNorm, RoPE) -> q_out, gate -> gate_out.
// Block nq + h: kv head h: key RMSNorm + RoPE, key and value stored as fp16 at
// cache slot `pos` ([t][kv_head][head_dim]).
// ---------------------------------------------------------------------------
__global__ void qk_norm_rope_append_kernel(QkPrepLaunch p) {
    extern __shared__ float vals[];  // head_dim
    __shared__ float red[32];
    const int b = blockIdx.x;
    const int hd = p.head_dim;
    const int pos = *p.pos;
    const bool is_q = b < p.nq;
    const int h = is_q ? b : b - p.nq;
    const float* src;
    const float* w;
    if (is_q) {
        src = p.q_src + static_cast<size_t>(h) * (p.gated ? 2 * hd : hd);
        w = p.q_norm;
    } else {
        src = p.k_src + static_cast<size_t>(h) * hd;
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
            p.q_out[static_cast<size_t>(h) * hd + d] = v;
            p.gate_out[static_cast<size_t>(h) * hd + d] = p.gated ? src[hd + d] : 0.0f;
        } else {
            const size_t slot = (static_cast<size_t>(pos) * p.nkv + h) * hd + d;
            p.k_cache[slot] = static_cast<_Float16>(v);
            p.v_cache[slot] = static_cast<_Float16>(p.v_src[static_cast<size_t>(h) * hd + d]);
        }
    }
}

hipError_t launch_qk_prep(const QkPrepLaunch& p, hipStream_t s) {
    const int threads = p.head_dim >= 256 ? 256 : (p.head_dim > 64 ? 128 : 64);
    hipLaunchKernelGGL(qk_norm_rope_append_kernel, dim3(p.nq + p.nkv), dim3(threads),
                       static_cast<size_t>(p.head_dim) * sizeof(float), s, p);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// GQA decode attention, split over the context.  Block (kh, split) takes the
// `group` query heads of kv head kh over a slice of the context: scores
// q.k/sqrt(d), a local max/sum softmax and the partial sum p*v.  The last split
// of each kv head to finish merges the partials (rescaling by exp(m_s - m)),
// applies the sigmoid output gate and writes the head outputs.
// ---------------------------------------------------------------------------

// Partial softmax-attention of `group` query heads over tokens [t0, t0+n) of one
// kv head.  Scores: 8 lanes per token, each lane owning HD/8 consecutive dims
// (16-byte loads); the 8 partial dots of every query head are summed across the
// 8 lanes.  V: each lane owns HD/64 dims of all heads for a quarter of the
// tokens; the quarters are summed through LDS.  HD == 0: any head_dim
// (scalar loads, tiny shapes).
template <int HD>
__device__ void gqa_slice(const GqaLaunch& p, int kh, int t0, int n, int group, int hd, float* qs, float* sc, float* ml,
                          float* vpart) {
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    const float rscale = 1.0f / sqrtf(static_cast<float>(hd));
    const int per_stride = blockDim.x / 8;  // tokens per pass
    if constexpr (HD > 0) {
        constexpr int DL = HD / 8;  // dims per lane
        const int sub = threadIdx.x & 7;
        for (int tt = threadIdx.x / 8; tt < ((n + per_stride - 1) / per_stride) * per_stride; tt += per_stride) {
            const bool valid = tt < n;
            float kv[DL];
            if (valid) {
                const _Float16* krow = p.k_cache + (static_cast<size_t>(t0 + tt) * p.nkv + kh) * HD + sub * DL;
#pragma unroll
                for (int u = 0; u < DL / 8; ++u) {
                    const uint4 w = *reinterpret_cast<const uint4*>(krow + 8 * u);
                    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        kv[8 * u + 2 * e] = half_lo(ww[e]);
                        kv[8 * u + 2 * e + 1] = half_hi(ww[e]);
                    }
                }
            } else {
#pragma unroll
                for (int d = 0; d < DL; ++d) kv[d] = 0.0f;
            }
            for (int g = 0; g < group; ++g) {
                const float* qv = qs + g * HD + sub * DL;
                float dot = 0.0f;
#pragma unroll
                for (int d = 0; d < DL; ++d) dot += qv[d] * kv[d];
                dot += __shfl_xor(dot, 1, kWave);
                dot += __shfl_xor(dot, 2, kWave);
                dot += __shfl_xor(dot, 4, kWave);
                if (valid && sub == 0) sc[g * p.slice + tt] = dot * rscale;
            }
        }
    } else {
        for (int pr = threadIdx.x; pr < n * group; pr += blockDim.x) {
            const int t = pr / group, g = pr % group;
            const _Float16* krow = p.k_cache + (static_cast<size_t>(t0 + t) * p.nkv + kh) * hd;
            float dot = 0.0f;
            for (int d = 0; d < hd; ++d) dot += qs[g * hd + d] * static_cast<float>(krow[d]);
            sc[g * p.slice + t] = dot * rscale;
        }
    }
    __syncthreads();
    for (int g = wid; g < group; g += blockDim.x / kWave) {
        float m = -INFINITY;
        for (int t = lane; t < n; t += kWave) m = fmaxf(m, sc[g * p.slice + t]);
        m = wave_max(m);
        float l = 0.0f;
        for (int t = lane; t < n; t += kWave) {
            const float e = expf(sc[g * p.slice + t] - m);
            sc[g * p.slice + t] = e;
            l += e;
        }
        l = wave_sum(l);
        if (lane == 0) {
            ml[2 * g] = m;
            ml[2 * g + 1] = l;
        }
    }
    __syncthreads();
    const int quarters = blockDim.x / kWave;  // token groups
    for (int d0 = lane; d0 < hd; d0 += kWave) {  // this lane's dims: d0, d0 + 64, ...
        float o[kAttnMaxGroup];
#pragma unroll
        for (int g = 0; g < kAttnMaxGroup; ++g) o[g] = 0.0f;
        for (int t = wid; t < n; t += quarters) {
            const float vv = static_cast<float>(p.v_cache[(static_cast<size_t>(t0 + t) * p.nkv + kh) * hd + d0]);
#pragma unroll
            for (int g = 0; g < kAttnMaxGroup; ++g)
                if (g < group) o[g] += sc[g * p.slice + t] * vv;
        }
#pragma unroll
        for (int g = 0; g < kAttnMaxGroup; ++g)
            if (g < group) vpart[(wid * group + g) * hd + d0] = o[g];
    }
    __syncthreads();
}

__global__ void __launch_bounds__(256) gqa_decode_kernel(GqaLaunch p) {
    extern __shared__ float smem[];
    const int hd = p.head_dim;
    const int group = p.nq / p.nkv;
    const int kh = blockIdx.x;
    const int split = blockIdx.y;
    const int ctx = *p.pos + 1;
    const int per = (ctx + kAttnSplits - 1) / kAttnSplits;
    const int t0 = split * per;
    const int n = max(0, min(ctx, t0 + per) - t0);
    float* qs = smem;                              // [group][hd]
    float* sc = qs + group * hd;                   // [group][slice]
    float* ml = sc + group * p.slice;              // [group][2]
    float* vpart = ml + 2 * group;                 // [4][group][hd]
    __shared__ int is_last;

    for (int i = threadIdx.x; i < group * hd; i += blockDim.x)
        qs[i] = p.q[static_cast<size_t>(kh * group + i / hd) * hd + (i % hd)];
    __syncthreads();
    if (hd == 128)
        gqa_slice<128>(p, kh, t0, n, group, hd, qs, sc, ml, vpart);
    else if (hd == 256)
        gqa_slice<256>(p, kh, t0, n, group, hd, qs, sc, ml, vpart);
    else if (hd == 64)
        gqa_slice<64>(p, kh, t0, n, group, hd, qs, sc, ml, vpart);
    else
        gqa_slice<0>(p, kh, t0, n, group, hd, qs, sc, ml, vpart);
    const int qh0 = kh * group;
    const int quarters = blockDim.x / kWave;
    for (int i = threadIdx.x; i < group * hd; i += blockDim.x) {
        const int g = i / hd, d = i % hd;
        float o = 0.0f;
        for (int w = 0; w < quarters; ++w) o += vpart[(w * group + g) * hd + d];
        p.part_o[(static_cast<size_t>(qh0 + g) * kAttnSplits + split) * hd + d] = o;
    }
    for (int g = threadIdx.x; g < group; g += blockDim.x) {
        p.part_ml[(static_cast<size_t>(qh0 + g) * kAttnSplits + split) * 2] = ml[2 * g];
        p.part_ml[(static_cast<size_t>(qh0 + g) * kAttnSplits + split) * 2 + 1] = (n > 0) ? ml[2 * g + 1] : 0.0f;
    }
    // every wave's partial stores have completed at L2 before wave 0 releases
    // them (one agent-scope fence per block: it writes back the XCD's L2)
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    if (threadIdx.x == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        const uint32_t ticket = atomicAdd(&p.counters[kh], 1u);
        is_last = ticket == kAttnSplits - 1;
        if (is_last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    __syncthreads();
    if (!is_last) return;
    for (int i = threadIdx.x; i < group * hd; i += blockDim.x) {
        const int g = i / hd, d = i % hd;
        const size_t base = static_cast<size_t>(qh0 + g) * kAttnSplits;
        float mm = -INFINITY;
        for (int s2 = 0; s2 < kAttnSplits; ++s2)
            mm = fmaxf(mm, __hip_atomic_load(&p.part_ml[(base + s2) * 2], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        float l = 0.0f, o = 0.0f;
        for (int s2 = 0; s2 < kAttnSplits; ++s2) {
            const float ms = __hip_atomic_load(&p.part_ml[(base + s2) * 2], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const float ls =
                __hip_atomic_load(&p.part_ml[(base + s2) * 2 + 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (ls == 0.0f) continue;
            const float f = expf(ms - mm);
            l += ls * f;
            o += __hip_atomic_load(&p.part_o[(base + s2) * hd + d], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) * f;
        }
        const size_t oi = static_cast<size_t>(qh0 + g) * hd + d;
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        p.out[oi] = (o * inv) * sigmoid_dev(p.gate[oi]);
    }
    if (threadIdx.x == 0) p.counters[kh] = 0u;
}

size_t gqa_workspace_bytes(int nq, int nkv, int head_dim) {
    return 256 + sizeof(uint32_t) * static_cast<size_t>(nkv) +
           sizeof(float) * static_cast<size_t>(nq) * kAttnSplits * (head_dim + 2);
}

static size_t gqa_lds_bytes(int group, int head_dim, int slice) {
    return sizeof(float) * (static_cast<size_t>(group) * head_dim + static_cast<size_t>(group) * slice + 2 * group +
                            4 * static_cast<size_t>(group) * head_dim);
}

hipError_t launch_gqa(const GqaLaunch& p0, hipStream_t s) {
    GqaLaunch p = p0;
    const int group = p.nq / p.nkv;
    p.slice = (p.max_ctx + kAttnSplits - 1) / kAttnSplits;
    const size_t lds = gqa_lds_bytes(group, p.head_dim, p.slice);
    if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gqa_decode_kernel),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(gqa_decode_kernel, dim3(p.nkv, kAttnSplits), dim3(256), lds, s, p);
    return hipGetLastError();
}

bool gqa_supported(int nq, int nkv, int head_dim, int max_ctx) {
    if (nkv <= 0 || nq % nkv != 0 || nq / nkv > kAttnMaxGroup || head_dim <= 0) return false;
    const int per_max = (max_ctx + kAttnSplits - 1) / kAttnSplits;
    if (per_max > kAttnMaxSlice) return false;
    return gqa_lds_bytes(nq / nkv, head_dim, per_max) <= 160 * 1024;
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
    pred += __shfl_xor(pred, 16, kWave);
    pred += __shfl_xor(pred, 32, kWave);
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
    o += __shfl_xor(o, 16, kWave);
    o += __shfl_xor(o, 32, kWave);
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
