// gemv_w4a16.hip - batch-1 W4A16 group-64 GEMV for gfx950 (CDNA4, wave64).
//
// Replaces gemvW4A16Neon / gemvW4A16ArgmaxNeon
// (customlib/kernels/generated/arm64_neon/xq_gemv_w4a16_neon.cpp:259-348).
// The reference factorises each group g of a row as
//     acc += s_g * (sum_c q_c x_c  -  z_g * sum_c x_c)          (version 1)
//     acc += s_g * sum_c q_c x_c  +  z_g * sum_c x_c            (version 2)
// and so do these kernels: the per-group sums of x are computed once per block
// and the inner loop is a pure code-times-activation integer dot product.
//
// Inner loop (TILED64 layout).  One lane owns one 64-column group of a row per
// 4096-column chunk: it streams the group's 32 bytes of nibbles with two 16-byte
// loads (a wave's load instruction covers 1 KiB contiguous) and one u32 of
// (fp16 scale, fp16 zero).  The device copy of every nibble is q ^ 8, which read
// as a signed 4-bit integer is q - 8, so a u32 of 8 codes feeds v_dot8_i32_i4
// directly (no unpacking).
//
// Activations are staged once per block as integers: each 64-column group is
// scaled by e = max|x| / 2^21 and rounded, X = rint(x / e) (|X| <= 2^21), and X
// is written as six signed hex digits, X = sum_d t_d 16^d with t_d in [-8, 7]
// (t_d = hex digit d of X + 0x888888, minus 8).  Digit d of eight consecutive
// columns is one u32 of signed nibbles, so per word of weights the lane issues
// six v_dot8_i32_i4 into six integer accumulators; per group they combine
// exactly into D = sum_c (q_c - 8) X_c (|D| < 2^30) and, with G = sum_c X_c,
//     sum_c q_c x_c = e (D + 8 G),   sum_c x_c = e G.
// The only rounding besides the final fp32 accumulation over groups is that of
// x to 22 significant bits relative to its group maximum.  Per 8 weights this
// is 6 VALU ops (the fp16 magic-number path it replaces needed 13).
//
// Columns beyond 4096 are split over the waves of a block (one 4096-column chunk
// per wave), whose partial row sums are combined through LDS in a fixed order.
//
// 3- and 2-bit codes (the reference's W3A16 / W2A16 bitstreams,
// customlib/kernels/reference/ref_gemv.cpp:10-30, 77-106) run through the same
// kernel: the upload splits each group's codes into bit planes laid out so that
// one or two shift-and-mask steps rebuild exactly the eight signed-nibble words
// (q | 8, i.e. q - 8 in signed 4-bit) the W4 layout stores, so staging,
// metadata, epilogues and argmax are shared; only the bytes streamed per group
// shrink (32 -> 24 -> 16).
#include "xqhip_common.hpp"
#include "gemv_tiled.hpp"

namespace xqhip {

__device__ __forceinline__ float load_act(const void* x, int x_f16, int i) {
    if (x_f16) return static_cast<float>(static_cast<const _Float16*>(x)[i]);
    return static_cast<const float*>(x)[i];
}

// Normalisation prologues fused into the GEMV (computed by every block from x):
//   PRO_RMS   x * inv * w[c], inv = 1/sqrt(mean(x^2)+eps)        (ref_rmsnorm.cpp:8-17)
//   PRO_GATED per head h of head_dim values: x * inv_h * w[c % head_dim] * silu(z[c])
//             (applyGatedHeadRms, custom_model.cpp:329-349); PRO_GATED_ACT the same
//             with z holding silu(z) already
// inv_lds receives inv (PRO_RMS) or inv_h for every head (PRO_GATED).
__device__ void prologue_factors(const void* x, int x_f16, int n, const Prologue& pro, float* inv_lds, float* red) {
    if (pro.mode == PRO_RMS) {
        float ss = 0.0f;
        for (int c = threadIdx.x; c < n; c += blockDim.x) {
            const float v = load_act(x, x_f16, c);
            ss += v * v;
        }
        ss = block_sum(ss, red);
        if (threadIdx.x == 0) inv_lds[0] = 1.0f / sqrtf(ss / static_cast<float>(n) + pro.eps);
    } else if (pro.mode == PRO_GATED || pro.mode == PRO_GATED_ACT) {
        const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave, nw = blockDim.x / kWave;
        const int heads = n / pro.head_dim;
        for (int h = wid; h < heads; h += nw) {
            float ss = 0.0f;
            for (int d = lane; d < pro.head_dim; d += kWave) {
                const float v = load_act(x, x_f16, h * pro.head_dim + d);
                ss += v * v;
            }
            ss = wave_sum(ss);
            if (lane == 0) inv_lds[h] = 1.0f / sqrtf(ss / static_cast<float>(pro.head_dim) + pro.eps);
        }
    }
    __syncthreads();
}

__device__ __forceinline__ float prologue_apply(float v, int c, const Prologue& pro, const float* inv_lds) {
    if (pro.mode == PRO_RMS) return v * inv_lds[0] * pro.w[c];
    if (pro.mode == PRO_GATED || pro.mode == PRO_GATED_ACT) {
        const int h = c / pro.head_dim;
        const float g = pro.mode == PRO_GATED_ACT ? pro.z[c] : silu_dev(pro.z[c]);
        return v * inv_lds[h] * pro.w[c - h * pro.head_dim] * g;
    }
    return v;
}

// position != nullptr: also advances *position by one and publishes
// (new position << 32 | index) to host_slot (coherent pinned host memory) in
// one system-scope store, which a host thread polls for.
// embed_out != nullptr: also writes the bf16 embedding row of the winner as
// fp32 (the next position's input, as embed_bf16_kernel would from out_idx:
// the same wrap of ids past the table and the same exact widening).
__global__ void __launch_bounds__(256) argmax_finish_kernel(const uint64_t* __restrict__ partial, int n,
                                                            int32_t* __restrict__ out_idx,
                                                            float* __restrict__ out_val, int32_t* position,
                                                            uint64_t* host_slot, const uint16_t* __restrict__ table,
                                                            int vocab, int hidden, float* __restrict__ embed_out) {
    __shared__ uint64_t keys[4];
    // every key of this thread requested at once (range-checked: past n, 0)
    constexpr int kPer = kArgmaxMaxBlocks / 256;
    const __amdgpu_buffer_rsrc_t pr = buf_rsrc(partial, static_cast<uint32_t>(n) * 8u);
    uint64_t best = 0;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(pr, (threadIdx.x + 256u * k) * 8u, 0, 0);
        best = u64_max(best, (static_cast<uint64_t>(w.y) << 32) | w.x);
    }
    best = wave_max_u64(best);
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    if (lane == 0) keys[wid] = best;
    __syncthreads();
    const uint64_t b = u64_max(u64_max(keys[0], keys[1]), u64_max(keys[2], keys[3]));
    const uint32_t idx = 0xffffffffu - static_cast<uint32_t>(b);
    if (threadIdx.x == 0) {
        *out_idx = static_cast<int32_t>(idx);
        *out_val = float_from_order_key(static_cast<uint32_t>(b >> 32));
        if (position) {
            const int32_t np = *position + 1;
            *position = np;
            __hip_atomic_store(host_slot, (static_cast<uint64_t>(static_cast<uint32_t>(np)) << 32) | idx,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
    if (embed_out == nullptr) return;
    // idx is below 2^31 (a row of the matrix), so as an id it is non-negative
    const uint32_t tok = idx < static_cast<uint32_t>(vocab) ? idx : idx % static_cast<uint32_t>(max(1, vocab));
    const uint16_t* row = table + static_cast<size_t>(tok) * hidden;
    const bool vec = (hidden & 7) == 0 && ((reinterpret_cast<uintptr_t>(row) | reinterpret_cast<uintptr_t>(embed_out)) & 15) == 0;
    if (vec) {  // 8 values per 16-byte load (uniform branch)
        for (int i = threadIdx.x * 8; i < hidden; i += 256 * 8) {
            const uint4 w = *reinterpret_cast<const uint4*>(row + i);
            const uint32_t h[4] = {w.x, w.y, w.z, w.w};
            float4 lo, hi;
            lo.x = __uint_as_float(h[0] << 16); lo.y = __uint_as_float(h[0] & 0xffff0000u);
            lo.z = __uint_as_float(h[1] << 16); lo.w = __uint_as_float(h[1] & 0xffff0000u);
            hi.x = __uint_as_float(h[2] << 16); hi.y = __uint_as_float(h[2] & 0xffff0000u);
            hi.z = __uint_as_float(h[3] << 16); hi.w = __uint_as_float(h[3] & 0xffff0000u);
            *reinterpret_cast<float4*>(embed_out + i) = lo;
            *reinterpret_cast<float4*>(embed_out + i + 4) = hi;
        }
    } else {
        for (int i = threadIdx.x; i < hidden; i += 256) embed_out[i] = __uint_as_float(static_cast<uint32_t>(row[i]) << 16);
    }
}

hipError_t launch_argmax_finish(const GemvLaunch& p, int blocks, hipStream_t s) {
    hipLaunchKernelGGL(argmax_finish_kernel, dim3(1), dim3(256), 0, s, p.partial, blocks, p.out_idx, p.out_val,
                       p.position, p.host_slot, p.embed_table, p.embed_vocab, p.embed_hidden, p.embed_out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// GENERIC kernel: any group size, reference row-major layout, fp32 metadata.
// One wave per unit (a row, or a (gate, up) row pair for EPI_SILU); it follows
// the reference's per-group factorisation directly.  Used for tiny shapes only.
// ---------------------------------------------------------------------------
template <int EPI>
__global__ void __launch_bounds__(256) gemv_w4_generic(const uint8_t* __restrict__ nib,
                                                       const float* __restrict__ scales,
                                                       const float* __restrict__ zeros, int rows, int cols,
                                                       int group, int affine, int bits, uint64_t nib_bytes,
                                                       const void* __restrict__ x, int x_f16,
                                                       Prologue pro, void* __restrict__ y, int y_f16,
                                                       uint64_t* __restrict__ partial) {
    __shared__ float red[32];
    __shared__ uint64_t lds_keys[16];
    __shared__ float inv_lds[kMaxNormHeads];
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = threadIdx.x / kWave;
    const int nw = blockDim.x / kWave;
    prologue_factors(x, x_f16, cols, pro, inv_lds, red);
    const int G = (cols + group - 1) / group;
    const size_t row_bytes = (static_cast<size_t>(cols) + 1) >> 1;
    const int per_unit = (EPI == EPI_SILU) ? 2 : 1;
    const int units = (rows + per_unit - 1) / per_unit;
    uint64_t best = 0;
    for (int u = blockIdx.x * nw + wid; u < units; u += gridDim.x * nw) {
        float res[2] = {0.0f, 0.0f};
        for (int k = 0; k < per_unit; ++k) {
            const int row = u * per_unit + k;
            if (row >= rows) break;
            float a = 0.0f;
            for (int g = lane; g < G; g += kWave) {
                const int c0 = g * group;
                const int n = min(group, cols - c0);
                float cd = 0.0f, gs = 0.0f;
                for (int c = c0; c < c0 + n; ++c) {
                    uint32_t code;
                    if (bits == 4) {
                        const uint8_t b = nib[static_cast<size_t>(row) * row_bytes + (c >> 1)];
                        code = (c & 1) ? (b >> 4) : (b & 0x0f);
                    } else {
                        // LSB-first bitstream without row padding (ref_gemv.cpp:10-18, 77-81)
                        const uint64_t bit = (static_cast<uint64_t>(row) * cols + c) * bits;
                        const uint64_t byte = bit >> 3;
                        const uint32_t lo = nib[byte], hi = byte + 1 < nib_bytes ? nib[byte + 1] : 0u;
                        code = ((lo | (hi << 8)) >> (bit & 7)) & ((1u << bits) - 1u);
                    }
                    const float q = static_cast<float>(code);
                    const float xv = prologue_apply(load_act(x, x_f16, c), c, pro, inv_lds);
                    cd += q * xv;
                    gs += xv;
                }
                const size_t mi = static_cast<size_t>(row) * G + g;
                if (affine)
                    a += scales[mi] * cd + zeros[mi] * gs;
                else
                    a += scales[mi] * (cd - zeros[mi] * gs);
            }
            res[k] = wave_sum(a);
        }
        if (lane == 0) {
            if constexpr (EPI == EPI_ARGMAX) {
                best = u64_max(best, argmax_key(res[0], static_cast<uint32_t>(u)));
            } else if constexpr (EPI == EPI_SILU) {
                static_cast<float*>(y)[u] = silu_dev(res[0]) * res[1];
            } else if constexpr (EPI == EPI_ADD) {
                static_cast<float*>(y)[u] += res[0];
            } else {
                if (y_f16)
                    static_cast<_Float16*>(y)[u] = static_cast<_Float16>(res[0]);
                else
                    static_cast<float*>(y)[u] = res[0];
            }
        }
    }
    if constexpr (EPI == EPI_ARGMAX) {
        if (lane == 0) lds_keys[wid] = best;
        __syncthreads();
        uint64_t b = 0;
        if (threadIdx.x == 0)
            for (int i = 0; i < nw; ++i) b = u64_max(b, lds_keys[i]);
        __syncthreads();
        store_block_key(b, partial, threadIdx.x, blockIdx.x);
    }
}

template <int EPI>
static hipError_t launch_generic_t(const GemvLaunch& p, hipStream_t s) {
    const int per_unit = (EPI == EPI_SILU) ? 2 : 1;
    const int units = (p.rows + per_unit - 1) / per_unit;
    const int nw = kThreads / kWave;
    int blocks = (units + nw - 1) / nw;
    const int cap = p.max_blocks > 0 ? p.max_blocks : 1024;
    if (blocks > cap) blocks = cap;
    if (EPI == EPI_ARGMAX && blocks > kArgmaxMaxBlocks) blocks = kArgmaxMaxBlocks;
    if (blocks < 1) blocks = 1;
    const float* sc = static_cast<const float*>(p.meta);
    const int G = (p.cols + p.group - 1) / p.group;
    const float* zr = sc + static_cast<size_t>(p.rows) * G;
    hipLaunchKernelGGL((gemv_w4_generic<EPI>), dim3(blocks), dim3(kThreads), 0, s, p.nib, sc, zr, p.rows, p.cols,
                       p.group, p.affine, p.bits, p.nib_bytes, p.x, p.x_f16, p.pro, p.y, p.y_f16, p.partial);
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    return EPI == EPI_ARGMAX ? launch_argmax_finish(p, blocks, s) : hipSuccess;
}

hipError_t launch_gemv(const GemvLaunch& p, hipStream_t s) {
    if (p.layout == 2) return launch_gemv_tiled_m32(p, s);
    if (p.layout == 3) return launch_gemv_tiled_s16(p, s);
    if (p.layout == 4) return launch_gemv_tiled_z4(p, s);
    if (p.layout == 0) {
        switch (p.bits) {
            case 4: return launch_tiled_bits<4, 0>(p, s);
            case 3: return launch_tiled_bits<3, 0>(p, s);
            case 2: return launch_tiled_bits<2, 0>(p, s);
            default: return hipErrorInvalidValue;
        }
    }
    switch (p.epi) {
        case EPI_STORE: return launch_generic_t<EPI_STORE>(p, s);
        case EPI_ADD: return launch_generic_t<EPI_ADD>(p, s);
        case EPI_SILU: return launch_generic_t<EPI_SILU>(p, s);
        case EPI_ARGMAX: return launch_generic_t<EPI_ARGMAX>(p, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace xqhip
