// prefill_ops.hip - the multi-token (prefill) kernels of the decode path on gfx950.
//
// The reference prefills token by token (CustomModel::prefill,
// customlib/runtime/custom_model.cpp:610-640); the arithmetic per token is the
// same as decode.  Here the dense contractions of a prompt chunk (the
// q/k/v/o, gate/up and down projections of every layer for up to
// kPrefillChunk tokens) run as one W4A16 GEMM each on the matrix cores, and
// the sequential parts run as batched kernels:
//   prep_x_kernel        per-token RMSNorm / gated head norm, x -> fp16 hi + lo
//                        and per-group sums of x
//   gemm_w4_mfma_kernel  per 64-column group: codes q - 8 (exact in fp16) times
//                        x hi / lo on v_mfma_f32_16x16x32_f16, group sums scaled
//                        by the group scale; the zero-point term as a K = G
//                        MFMA contraction after the group loop
//   prefill_attn_mfma_kernel / prefill_attn_kernel   causal GQA over the cache
//   linear_conv_prefill_tg_kernel + scan_chunk_prep_kernel + scan_chunk_state_kernel   conv1d + norms +
//                        gates for all tokens, then the gated-delta recurrence
//                        with the state in registers (one-pass kernels
//                        linear_scan_wave_kernel / linear_scan_kernel otherwise)
#include <algorithm>

#include "xqhip_common.hpp"
#include "xqhip_kernels.hpp"

namespace xqhip {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
// register arrays of native vectors (arrays of HIP's uint4 / uint2 structs are kept in scratch)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_h2(_Float16 lo, _Float16 hi) {
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, lo)) |
           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, hi)) << 16);
}

// ---------------------------------------------------------------------------
// B operand preparation: token t = blockIdx.x of x (row stride ldx) with the
// prologue applied (RMS over the row, or per-head gated norm with the gate
// row at t * ldz) -> v, stored as xh = fp16(v) and xl = fp16(v - xh) (about
// 22 significant bits together) with every aligned run of 8 columns in the
// order [0 4 1 5 2 6 3 7], the order in which the GEMM unpacks a word of 8
// weight codes; xs[t][g] = fp32 sum of v over column group g (64 columns).
// Each row is first scaled by a power of two, ts[t] = 2^k, that brings its
// largest magnitude into [2^12, 2^13): fp16 then holds any fp32 activation
// (silu(gate) * up of a large residual stream can exceed 65504) without
// overflow or subnormal loss, and the GEMM multiplies its results by ts[t]
// (exact).  Rows m..m_pad-1 are zero-filled (ts 1).
// ---------------------------------------------------------------------------
constexpr int kPrepMaxHeads = 256;

__global__ void __launch_bounds__(256) prep_x_kernel(const float* __restrict__ x, int ldx, int m, int cols,
                                                     Prologue pro, int ldz, _Float16* __restrict__ xh,
                                                     _Float16* __restrict__ xl, float* __restrict__ xs,
                                                     float* __restrict__ ts) {
    __shared__ float red[32];
    __shared__ float head_inv[kPrepMaxHeads];
    const int t = blockIdx.x;
    const int G = cols >> 6, nch = cols >> 3;
    uint4* oh = reinterpret_cast<uint4*>(xh + static_cast<size_t>(t) * cols);
    uint4* ol = reinterpret_cast<uint4*>(xl + static_cast<size_t>(t) * cols);
    float* os = xs + static_cast<size_t>(t) * G;
    if (t >= m) {
        for (int c = threadIdx.x; c < nch; c += blockDim.x) oh[c] = ol[c] = make_uint4(0u, 0u, 0u, 0u);
        for (int g = threadIdx.x; g < G; g += blockDim.x) os[g] = 0.0f;
        if (threadIdx.x == 0) ts[t] = 1.0f;
        return;
    }
    const float* xr = x + static_cast<size_t>(t) * ldx;
    const float* zr = pro.mode == PRO_GATED ? pro.z + static_cast<size_t>(t) * ldz : nullptr;
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave, nw = blockDim.x / kWave;
    float inv = 1.0f;
    if (pro.mode == PRO_RMS) {
        float ss = 0.0f;
        for (int c = threadIdx.x; c < cols; c += blockDim.x) ss += xr[c] * xr[c];
        ss = block_sum(ss, red);
        inv = 1.0f / sqrtf(ss / static_cast<float>(cols) + pro.eps);
    } else if (pro.mode == PRO_GATED) {
        const int heads = cols / pro.head_dim;
        for (int h = wid; h < heads; h += nw) {  // one wave per head
            const float* xv = xr + h * pro.head_dim;
            float ss = 0.0f;
            for (int d = lane; d < pro.head_dim; d += kWave) ss += xv[d] * xv[d];
            ss = wave_sum(ss);
            if (lane == 0) head_inv[h] = 1.0f / sqrtf(ss / static_cast<float>(pro.head_dim) + pro.eps);
        }
        __syncthreads();
    }
    // one thread per 8 columns; the 8 threads of a group are consecutive lanes (nch % 8 == 0)
    auto load8 = [&](int c, float (&v)[8]) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = xr[c + e];
        if (pro.mode == PRO_RMS) {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = v[e] * inv * pro.w[c + e];
        } else if (pro.mode == PRO_GATED) {
            const int h = c / pro.head_dim, d = c - h * pro.head_dim;  // head_dim % 8 == 0
            const float ih = head_inv[h];
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = v[e] * ih * pro.w[d + e] * silu_dev(zr[c + e]);
        }
    };
    // the row's power-of-two scale from its largest magnitude
    float mx = 0.0f;
    for (int c8 = threadIdx.x; c8 < nch; c8 += blockDim.x) {
        float v[8];
        load8(c8 * 8, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(v[e]));
    }
    mx = wave_max(mx);
    __syncthreads();  // red may still be read by the norm's block_sum
    if (lane == 0) red[wid] = mx;
    __syncthreads();
    for (int i = 0; i < nw; ++i) mx = fmaxf(mx, red[i]);
    int ex = 0;
    frexpf(mx, &ex);                                       // mx = f 2^ex, f in [0.5, 1)
    const float down = mx > 0.0f ? ldexpf(1.0f, 13 - ex) : 1.0f;  // mx * down in [2^12, 2^13)
    if (threadIdx.x == 0) ts[t] = mx > 0.0f ? ldexpf(1.0f, ex - 13) : 1.0f;
    for (int c8 = threadIdx.x; c8 < nch; c8 += blockDim.x) {
        const int c = c8 * 8;
        float v[8];
        load8(c, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] *= down;
        uint32_t ph[4], pl[4];
        float sum = 0.0f;
#pragma unroll
        for (int p = 0; p < 4; ++p) {  // positions 2p, 2p + 1 <- columns p, p + 4
            const float va = v[p], vb = v[p + 4];
            const _Float16 ha = static_cast<_Float16>(va), hb = static_cast<_Float16>(vb);
            ph[p] = pack_h2(ha, hb);
            pl[p] = pack_h2(static_cast<_Float16>(va - static_cast<float>(ha)),
                            static_cast<_Float16>(vb - static_cast<float>(hb)));
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) sum += v[e];
        oh[c8] = make_uint4(ph[0], ph[1], ph[2], ph[3]);
        ol[c8] = make_uint4(pl[0], pl[1], pl[2], pl[3]);
        sum = lanes_sum<8>(sum);
        if ((c8 & 7) == 0) os[c8 >> 3] = sum;
    }
}

// The same for rows of NK * 2048 columns with 16-byte aligned rows, weights and
// gates, the prologue mode a template argument: thread i owns the 8-column
// pieces i, i + 256, ... of its token's row and loads each once, as 16-byte
// loads with no branch around them (the generic kernel reads the row three
// times, one float per load); the gated norm's per-head sums stay inside the
// 16 lanes that own a 128-column head.
template <int NK, int MODE>
__global__ void __launch_bounds__(256) prep_x_vec_kernel(const float* __restrict__ x, int ldx, int m, Prologue pro,
                                                         int ldz, _Float16* __restrict__ xh, _Float16* __restrict__ xl,
                                                         float* __restrict__ xs, float* __restrict__ ts) {
    constexpr int kCols = NK * 2048, kG = kCols / 64;
    __shared__ float red_s[4], red_m[4];
    const int t = blockIdx.x;
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    uint4* oh = reinterpret_cast<uint4*>(xh + static_cast<size_t>(t) * kCols);
    uint4* ol = reinterpret_cast<uint4*>(xl + static_cast<size_t>(t) * kCols);
    float* os = xs + static_cast<size_t>(t) * kG;
    if (t >= m) {  // block-uniform
#pragma unroll
        for (int k = 0; k < NK; ++k) oh[threadIdx.x + 256 * k] = ol[threadIdx.x + 256 * k] = make_uint4(0u, 0u, 0u, 0u);
        for (int g = threadIdx.x; g < kG; g += 256) os[g] = 0.0f;
        if (threadIdx.x == 0) ts[t] = 1.0f;
        return;
    }
    const float4* xr = reinterpret_cast<const float4*>(x + static_cast<size_t>(t) * ldx);
    float4 xv[NK][2], wv[NK][2], zv[NK][2];
#pragma unroll
    for (int k = 0; k < NK; ++k) {
        const int c4 = 2 * (threadIdx.x + 256 * k);  // float4 index of the piece
        xv[k][0] = xr[c4];
        xv[k][1] = xr[c4 + 1];
        if constexpr (MODE == PRO_RMS) {
            wv[k][0] = reinterpret_cast<const float4*>(pro.w)[c4];
            wv[k][1] = reinterpret_cast<const float4*>(pro.w)[c4 + 1];
        } else if constexpr (MODE == PRO_GATED) {
            // head_dim 128: the piece's offset in its head is 8 (i mod 16)
            const int d4 = 2 * (threadIdx.x & 15);
            wv[k][0] = reinterpret_cast<const float4*>(pro.w)[d4];
            wv[k][1] = reinterpret_cast<const float4*>(pro.w)[d4 + 1];
            const float4* zr = reinterpret_cast<const float4*>(pro.z + static_cast<size_t>(t) * ldz);
            zv[k][0] = zr[c4];
            zv[k][1] = zr[c4 + 1];
        }
    }
    float v[NK][8];
#pragma unroll
    for (int k = 0; k < NK; ++k) {
        const float4 a = xv[k][0], b = xv[k][1];
        v[k][0] = a.x; v[k][1] = a.y; v[k][2] = a.z; v[k][3] = a.w;
        v[k][4] = b.x; v[k][5] = b.y; v[k][6] = b.z; v[k][7] = b.w;
    }
    if constexpr (MODE == PRO_RMS) {
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < NK; ++k)
#pragma unroll
            for (int e = 0; e < 8; ++e) ss += v[k][e] * v[k][e];
        ss = wave_sum(ss);
        if (lane == 0) red_s[wid] = ss;
        __syncthreads();
        ss = (red_s[0] + red_s[1]) + (red_s[2] + red_s[3]);
        const float inv = 1.0f / sqrtf(ss / static_cast<float>(kCols) + pro.eps);
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            const float w8[8] = {wv[k][0].x, wv[k][0].y, wv[k][0].z, wv[k][0].w,
                                 wv[k][1].x, wv[k][1].y, wv[k][1].z, wv[k][1].w};
#pragma unroll
            for (int e = 0; e < 8; ++e) v[k][e] = v[k][e] * inv * w8[e];
        }
    } else if constexpr (MODE == PRO_GATED) {
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            float ss = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) ss += v[k][e] * v[k][e];
            ss = lanes_sum<16>(ss);  // the head's 16 pieces
            const float ih = 1.0f / sqrtf(ss / 128.0f + pro.eps);
            const float w8[8] = {wv[k][0].x, wv[k][0].y, wv[k][0].z, wv[k][0].w,
                                 wv[k][1].x, wv[k][1].y, wv[k][1].z, wv[k][1].w};
            const float z8[8] = {zv[k][0].x, zv[k][0].y, zv[k][0].z, zv[k][0].w,
                                 zv[k][1].x, zv[k][1].y, zv[k][1].z, zv[k][1].w};
#pragma unroll
            for (int e = 0; e < 8; ++e) v[k][e] = v[k][e] * ih * w8[e] * silu_dev(z8[e]);
        }
    }
    // the row's power-of-two scale from its largest magnitude
    float mx = 0.0f;
#pragma unroll
    for (int k = 0; k < NK; ++k)
#pragma unroll
        for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(v[k][e]));
    mx = wave_max(mx);
    if (lane == 0) red_m[wid] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red_m[0], red_m[1]), fmaxf(red_m[2], red_m[3]));
    int ex = 0;
    frexpf(mx, &ex);
    const float down = mx > 0.0f ? ldexpf(1.0f, 13 - ex) : 1.0f;
    if (threadIdx.x == 0) ts[t] = mx > 0.0f ? ldexpf(1.0f, ex - 13) : 1.0f;
#pragma unroll
    for (int k = 0; k < NK; ++k) {
        const int c8 = threadIdx.x + 256 * k;
        uint32_t ph[4], pl[4];
        float sum = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[k][e] *= down;
#pragma unroll
        for (int q = 0; q < 4; ++q) {  // positions 2q, 2q + 1 <- columns q, q + 4
            const float va = v[k][q], vb = v[k][q + 4];
            const _Float16 ha = static_cast<_Float16>(va), hb = static_cast<_Float16>(vb);
            ph[q] = pack_h2(ha, hb);
            pl[q] = pack_h2(static_cast<_Float16>(va - static_cast<float>(ha)),
                            static_cast<_Float16>(vb - static_cast<float>(hb)));
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) sum += v[k][e];
        oh[c8] = make_uint4(ph[0], ph[1], ph[2], ph[3]);
        ol[c8] = make_uint4(pl[0], pl[1], pl[2], pl[3]);
        sum = lanes_sum<8>(sum);
        if ((c8 & 7) == 0) os[c8 >> 3] = sum;
    }
}

// the vectorised form's launch, or false when the shape or alignment needs the generic kernel
template <int NK>
static bool launch_prep_vec(const GemmLaunch& p, int m_pad, _Float16* xh, _Float16* xl, float* xs, float* ts,
                            hipStream_t s) {
    if (p.pro.mode == PRO_RMS)
        hipLaunchKernelGGL((prep_x_vec_kernel<NK, PRO_RMS>), dim3(m_pad), dim3(256), 0, s, p.x, p.ldx, p.m, p.pro,
                           p.ldz, xh, xl, xs, ts);
    else if (p.pro.mode == PRO_GATED)
        hipLaunchKernelGGL((prep_x_vec_kernel<NK, PRO_GATED>), dim3(m_pad), dim3(256), 0, s, p.x, p.ldx, p.m, p.pro,
                           p.ldz, xh, xl, xs, ts);
    else
        hipLaunchKernelGGL((prep_x_vec_kernel<NK, PRO_NONE>), dim3(m_pad), dim3(256), 0, s, p.x, p.ldx, p.m, p.pro,
                           p.ldz, xh, xl, xs, ts);
    return true;
}

static bool prep_vec_ok(const GemmLaunch& p) {
    auto al16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; };
    if (p.cols % 2048 != 0 || !al16(p.x) || p.ldx % 4 != 0) return false;
    if (p.pro.mode == PRO_RMS) return al16(p.pro.w);
    if (p.pro.mode == PRO_GATED) return p.pro.head_dim == 128 && al16(p.pro.w) && al16(p.pro.z) && p.ldz % 4 == 0;
    return p.pro.mode == PRO_NONE;
}

// ---------------------------------------------------------------------------
// W4A16 GEMM, y[t][r] (op)= sum_k w[r][k] x[t][k] for a prompt chunk.
//
// In column group g (64 columns) a row's weights are w = sn s + c0 with
// sn = q - 8 the signed code, s the group scale and c0 = (8 - z) s for
// w = (q - z) s, or 8 s + z for w = q s + z.  Hence
//     y[t][r] = sum_g s[r][g] A[r][t][g] + sum_g c0[r][g] xs[t][g],
//     A[r][t][g] = sum_{k in g} sn[r][k] x[t][k],  xs[t][g] = sum_{k in g} x[t][k].
// sn is exact in fp16, so A takes two v_mfma_f32_16x16x32_f16 passes per 32
// columns (sn x_hi + sn x_lo, x = x_hi + x_lo to about 22 bits) into a
// per-group accumulator, which is scaled by s into the fp32 result.  The c0
// term is a K = G contraction done after the group loop in three fp16 hi/lo
// passes (c0 scaled by 64 and xs by 1/64, both exact, to stay in fp16 range).
//
// Block: WGR x WGT waves, each owning TI x TJ tiles of 16 rows x 16 tokens.
// A operand: each lane loads its 8 bytes of a tile row's group straight from
// the TILED64 matrix into registers, in a four-group ring ahead of the MFMAs:
// lane l takes row l & 15 and words 2 (q & 1), 2 (q & 1) + 1 of half q >> 1,
// q = l >> 4 (columns 32 (q >> 1) + 16 (q & 1) + 0..15), and unpacks a word
// of 8 codes to fp16 q - 8 with integer ops ((u >> 4j) & 0x000F000F | 0x64006400
// is fp16 1024 + q for codes j and j + 4) and one packed fp16 subtraction.
// B operand: the block's BT tokens x 64 columns of x_hi and x_lo go through a
// register ring two groups ahead into double-buffered LDS, one barrier per
// group, with the scales of the block's rows.
// MFMA operand layout (16x16x32): lane l supplies row/column (l & 15) and 8
// consecutive k at 8 (l >> 4); lane l receives D[4 (l >> 4) + v][l & 15].
// Here the k of an MFMA is a permutation of the group's columns, the same for
// both operands.  Token tiles are the fastest grid dimension, so the blocks
// that share a weight tile run together and it is fetched from HBM about once.
// ---------------------------------------------------------------------------
constexpr int kGemmPad = 128;  // xh / xl / xs rows are padded to a multiple of this

struct GemmArgs {
    const uint8_t* nib;
    const uint32_t* meta;
    int rows, cols, affine;
    int zero_is_8;       // c0 = (8 - z) s is 0 for every group: the c0 pass is skipped
    const _Float16* xh;  // [m_pad][cols], followed by xl [m_pad][cols]
    const float* xs;     // [m_pad][cols / 64]
    const float* ts;     // [m_pad] per-token power-of-two scale of xh / xl / xs
    int gps;             // column groups per K split (blockIdx.z); the whole row when unsplit
    float* part;         // split K: [gridDim.z][m][rows] partial products (the reduce applies EPI)
    int m, m_pad;
    float* y;
    int ldy;
};

constexpr int kGemmXLd = 136;  // LDS x row in halves: x_hi[64] | x_lo[64] | 8 padding

template <int WGR, int WGT, int TI, int TJ>
struct GemmTile {
    static constexpr int kWaves = WGR * WGT, kThreads = kWave * kWaves;
    static constexpr int kWR = 16 * TI, kWT = 16 * TJ, kBR = WGR * kWR, kBT = WGT * kWT;
    static constexpr int kXU = kBT * 16 / kThreads;  // 16-byte pieces of x per thread per group
    static constexpr int kXStage = kBT * kGemmXLd;   // halves per stage
    static constexpr size_t kLds = 2 * (static_cast<size_t>(kXStage) * sizeof(_Float16) + kBR * sizeof(float));
    static_assert(kXU * kThreads == kBT * 16, "x staging");
    static_assert(kBR <= kThreads, "scale staging");
};

// 8 stored codes (q ^ 8; column n of the word in bits 4n..4n+3) -> fp16 q - 8
// in the column order [0 4 1 5 2 6 3 7]: ((w >> 4j) & 0x000F000F) ^ 0x64086408
// is fp16 (1024 + q) for the codes j and j + 4 (one shift and one three-input
// bit op), less 1032 in one packed fp16 subtraction.
__device__ __forceinline__ half8 codes_to_h8(uint32_t w) {
    typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
    const half2_t bias = {static_cast<_Float16>(1032.0f), static_cast<_Float16>(1032.0f)};
    uint32_t p[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const half2_t h = __builtin_bit_cast(half2_t, ((w >> (4 * j)) & 0x000F000Fu) ^ 0x64086408u) - bias;
        p[j] = __builtin_bit_cast(uint32_t, h);
    }
    return __builtin_bit_cast(half8, make_uint4(p[0], p[1], p[2], p[3]));
}

// two waves per SIMD (at most 256 registers per lane), so one block's barrier wait overlaps another's work
template <int WGR, int WGT, int TI, int TJ, int EPI, int META>
__global__ void __launch_bounds__(kWave * WGR * WGT) __attribute__((amdgpu_waves_per_eu(2)))
gemm_w4_mfma_kernel(GemmArgs a) {
    // fp16 (scale, zero) in a u32, the fp32 pair (the scale is its first word), the fp16 scale alone,
    // or the fp32 scale (its zero in the separate array of 4-bit codes)
    constexpr uint32_t kMetaBytes = kMetaGroupBytes<META>;
    using T = GemmTile<WGR, WGT, TI, TJ>;
    constexpr int BR = T::kBR, BT = T::kBT, XU = T::kXU, NT = T::kThreads;
    constexpr int kTokStep = NT / 16;  // tokens between a thread's x pieces
    extern __shared__ uint4 gemm_lds[];
    _Float16* xlds = reinterpret_cast<_Float16*>(gemm_lds);         // [2 stages][BT][kGemmXLd]
    float* slds = reinterpret_cast<float*>(xlds + 2 * T::kXStage);  // [2 stages][BR] scales
    // Tile of this block.  Blocks are dealt to the 8 XCDs round robin in
    // launch order; a weight slab (128 rows of one K split, a "unit") is read
    // by every token tile, so the token tiles of a unit are given launch
    // indices b = 8 k + (unit mod 8) and share one XCD's L2: the weights come
    // from memory once instead of once per XCD.  Units past the last multiple
    // of 8 keep the plain order.
    int tt, unit;
    {
        const int nt = gridDim.x;
        const int b = blockIdx.x + nt * (blockIdx.y + gridDim.y * blockIdx.z);
        const int units8 = (gridDim.y * gridDim.z) & ~7;
        if (b < units8 * nt) {
            const int k = b >> 3;
            unit = (k / nt) * 8 + (b & 7);
            tt = k % nt;
        } else {
            const int b2 = b - units8 * nt;
            unit = units8 + b2 / nt;
            tt = b2 % nt;
        }
    }
    const int split = unit / static_cast<int>(gridDim.y);
    const int t0 = tt * BT, r0 = (unit - split * static_cast<int>(gridDim.y)) * BR;
    const int G = a.cols >> 6, gl = G - 1;
    // this block's column groups: [g0, g1) of K split `split`
    const int g0 = split * a.gps, g1 = min(G, g0 + a.gps), glast = g1 - 1;
    const uint32_t row_bytes = static_cast<uint32_t>(a.cols) >> 1;
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    const int q = lane >> 4, lr = lane & 15;
    const int wr = (wid / WGT) * T::kWR, wt = (wid % WGT) * T::kWT;
    // A operand: byte offsets of this lane's 8 bytes in each tile row (rows past the end read the
    // last row); the half-1 offset depends on the chunk's group count, full or the last chunk's
    const __amdgpu_buffer_rsrc_t nib_r = buf_rsrc(a.nib, static_cast<uint32_t>(a.rows) * row_bytes);
    const int lastc = gl >> 6;
    const uint32_t gc_full = static_cast<uint32_t>(min(64, G)), gc_last = static_cast<uint32_t>(G - (lastc << 6));
    uint32_t aoff_full[TI], aoff_last[TI];
#pragma unroll
    for (int i = 0; i < TI; ++i) {
        const uint32_t base =
            static_cast<uint32_t>(min(r0 + wr + 16 * i + lr, a.rows - 1)) * row_bytes + (q & 1) * 8u;
        aoff_full[i] = base + static_cast<uint32_t>(q >> 1) * gc_full * 16u;
        aoff_last[i] = base + static_cast<uint32_t>(q >> 1) * gc_last * 16u;
    }
    // x staging: piece j of this thread is token (tid >> 4) + kTokStep j, 16 bytes at (tid & 15) of
    // the token's 256-byte LDS row (x_hi columns 0..63, then x_lo)
    const __amdgpu_buffer_rsrc_t x_r = buf_rsrc(a.xh, static_cast<uint32_t>(a.m_pad) * a.cols * 4u);
    const int xtok = threadIdx.x >> 4, c16 = threadIdx.x & 15;
    uint32_t xoff[XU];
#pragma unroll
    for (int j = 0; j < XU; ++j)
        xoff[j] = (static_cast<uint32_t>((c16 >> 3) * a.m_pad + t0 + xtok + j * kTokStep) * a.cols +
                   (c16 & 7) * 8u) * 2u;
    const int xdst = xtok * kGemmXLd + c16 * 8;
    // scales: thread < BR stages row r0 + tid (the others load out of range: zero, no branch)
    const __amdgpu_buffer_rsrc_t meta_r =
        buf_rsrc(a.meta, meta_total_bytes<META>(static_cast<uint32_t>(a.rows), static_cast<uint32_t>(G)));
    const bool s_thread = threadIdx.x < BR;
    const uint32_t moff =
        s_thread ? static_cast<uint32_t>(min(r0 + static_cast<int>(threadIdx.x), a.rows - 1)) * G * kMetaBytes : kBufOOB;

#define GEMM_LOAD_A(W, gg)                                                                                   \
    {                                                                                                        \
        const int g_ = (gg), c_ = g_ >> 6;                                                                   \
        const uint32_t so_ = static_cast<uint32_t>(c_) * 2048u + static_cast<uint32_t>(g_ & 63) * 16u;       \
        const bool last_ = c_ == lastc;                                                                      \
        _Pragma("unroll") for (int i_ = 0; i_ < TI; ++i_) W[i_] = __builtin_amdgcn_raw_buffer_load_b64(      \
            nib_r, last_ ? aoff_last[i_] : aoff_full[i_], so_, 0);                                            \
    }
#define GEMM_LOAD_X(X, M, gg)                                                                                \
    {                                                                                                        \
        const uint32_t g_ = static_cast<uint32_t>(gg);                                                       \
        _Pragma("unroll") for (int j_ = 0; j_ < XU; ++j_) X[j_] =                                            \
            __builtin_amdgcn_raw_buffer_load_b128(x_r, xoff[j_], g_ * 128u, 0);                              \
        M = META == 2 ? static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b16(meta_r, moff, g_ * kMetaBytes, 0)) \
                      : __builtin_amdgcn_raw_buffer_load_b32(meta_r, moff, g_ * kMetaBytes, 0);                \
    }
#define GEMM_STORE_X(X, M, st)                                                                               \
    {                                                                                                        \
        _Float16* d_ = xlds + (st) * T::kXStage + xdst;                                                      \
        _Pragma("unroll") for (int j_ = 0; j_ < XU; ++j_) *reinterpret_cast<u32x4*>(d_ + j_ * kTokStep * kGemmXLd) = \
            X[j_];                                                                                           \
        if (s_thread) slds[(st) * BR + threadIdx.x] = META == 1 || META == 3 ? __uint_as_float(M) : half_lo(M); \
    }
// MFMAs of one group, each tile's four chained into a per-group sum that is scaled into acc
#define GEMM_COMPUTE(st, W)                                                                                  \
    {                                                                                                        \
        const _Float16* xs_ = xlds + (st) * T::kXStage;                                                      \
        half8 bh_[TJ][2], bl_[TJ][2];                                                                        \
        _Pragma("unroll") for (int j_ = 0; j_ < TJ; ++j_) {                                                  \
            _Pragma("unroll") for (int k_ = 0; k_ < 2; ++k_) {                                               \
                const int o_ = (wt + 16 * j_ + lr) * kGemmXLd + (2 * q + k_) * 8;                            \
                bh_[j_][k_] = *reinterpret_cast<const half8*>(xs_ + o_);                                     \
                bl_[j_][k_] = *reinterpret_cast<const half8*>(xs_ + o_ + 64);                                \
            }                                                                                                \
        }                                                                                                    \
        _Pragma("unroll") for (int i_ = 0; i_ < TI; ++i_) {                                                  \
            const floatx4 sv_ = *reinterpret_cast<const floatx4*>(slds + (st) * BR + wr + 16 * i_ + 4 * q);  \
            const half8 a0_ = codes_to_h8(W[i_].x), a1_ = codes_to_h8(W[i_].y);                              \
            _Pragma("unroll") for (int j_ = 0; j_ < TJ; ++j_) {                                              \
                floatx4 t_ = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0_, bh_[j_][0], zero4, 0, 0, 0);        \
                t_ = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0_, bl_[j_][0], t_, 0, 0, 0);                   \
                t_ = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1_, bh_[j_][1], t_, 0, 0, 0);                   \
                t_ = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1_, bl_[j_][1], t_, 0, 0, 0);                   \
                _Pragma("unroll") for (int v_ = 0; v_ < 4; ++v_) acc[i_][j_][v_] =                           \
                    fmaf(sv_[v_], t_[v_], acc[i_][j_][v_]);                                                  \
            }                                                                                                \
        }                                                                                                    \
    }
// step U of four: MFMAs of group g + U (LDS stage U & 1, A ring slot W), refill W with
// group g + U + 4, store the x piece X (group g + U + 1) to the other stage, refill X
// with group g + U + 3.  Loads past the last group re-read it, so every step issues the
// same loads and the wait counts stay exact.
#define GEMM_STEP(U, W, X, M)                                                                                \
    {                                                                                                        \
        const int gg_ = g + (U);                                                                             \
        if (gg_ < g1) GEMM_COMPUTE((U) & 1, W);                                                              \
        GEMM_LOAD_A(W, min(gg_ + 4, glast));                                                                 \
        GEMM_STORE_X(X, M, ((U) + 1) & 1);                                                                   \
        GEMM_LOAD_X(X, M, min(gg_ + 3, glast));                                                              \
        __syncthreads();                                                                                     \
    }

    const floatx4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
    floatx4 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = zero4;
    u32x2 wa0[TI], wa1[TI], wa2[TI], wa3[TI];
    u32x4 xa[XU], xb[XU];  // x pieces of the even / odd groups
    uint32_t ma = 0, mb = 0;
    GEMM_LOAD_A(wa0, g0);
    GEMM_LOAD_A(wa1, min(g0 + 1, glast));
    GEMM_LOAD_A(wa2, min(g0 + 2, glast));
    GEMM_LOAD_A(wa3, min(g0 + 3, glast));
    GEMM_LOAD_X(xa, ma, g0);
    GEMM_LOAD_X(xb, mb, min(g0 + 1, glast));
    GEMM_STORE_X(xa, ma, 0);
    GEMM_LOAD_X(xa, ma, min(g0 + 2, glast));
    __syncthreads();
    for (int g = g0; g < g1; g += 4) {
        GEMM_STEP(0, wa0, xb, mb);
        GEMM_STEP(1, wa1, xa, ma);
        GEMM_STEP(2, wa2, xb, mb);
        GEMM_STEP(3, wa3, xa, ma);
    }
#undef GEMM_STEP
#undef GEMM_COMPUTE
#undef GEMM_STORE_X
#undef GEMM_LOAD_X
#undef GEMM_LOAD_A
    // c0 term: K = G, lane group q takes groups gb + 8 q + 0..7 of its row / token.  All loads of a
    // chunk are issued before any use; groups past G read out of range (zero), so c0 and xs are 0.
    const __amdgpu_buffer_rsrc_t xs_r = buf_rsrc(a.xs, static_cast<uint32_t>(a.m_pad) * G * 4u);
    for (int gb = g0; gb < (a.zero_is_8 ? g0 : g1); gb += 32) {
        const int g8 = gb + 8 * q;
        MetaWord<META> mw[TI][8];
        uint32_t xw[TJ][8];
#pragma unroll
        for (int i = 0; i < TI; ++i) {
            const uint32_t row = static_cast<uint32_t>(min(r0 + wr + 16 * i + lr, a.rows - 1));
            const uint32_t off = (row * G + static_cast<uint32_t>(g8)) * kMetaBytes;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const bool in = g8 + e < g1;
                const uint32_t o = in ? off + kMetaBytes * e : kBufOOB;
                const uint32_t zo =
                    META == 3 && in ? z4_offset(static_cast<uint32_t>(a.rows), static_cast<uint32_t>(G), row,
                                                static_cast<uint32_t>(g8 + e))
                                    : kBufOOB;
                mw[i][e] = load_meta<META, 0>(meta_r, o, zo);
            }
        }
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const uint32_t off = (static_cast<uint32_t>(t0 + wt + 16 * j + lr) * G + static_cast<uint32_t>(g8)) * 4u;
#pragma unroll
            for (int e = 0; e < 8; ++e)
                xw[j][e] = __builtin_amdgcn_raw_buffer_load_b32(xs_r, g8 + e < g1 ? off + 4u * e : kBufOOB, 0, 0);
        }
        half8 ch[TI], cl[TI], sh[TJ], sl[TJ];
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float sc = meta_scale(mw[i][e]);
                const float z = meta_zero_at(mw[i][e], static_cast<uint32_t>((g8 + e) & 7) * 4u);
                const float c0 = 64.0f * (a.affine ? fmaf(8.0f, sc, z) : (8.0f - z) * sc);
                ch[i][e] = static_cast<_Float16>(c0);
                cl[i][e] = static_cast<_Float16>(c0 - static_cast<float>(ch[i][e]));
            }
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float v = __builtin_bit_cast(float, xw[j][e]) * 0.015625f;
                sh[j][e] = static_cast<_Float16>(v);
                sl[j][e] = static_cast<_Float16>(v - static_cast<float>(sh[j][e]));
            }
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(cl[i], sh[j], acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ch[i], sl[j], acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ch[i], sh[j], acc[i][j], 0, 0, 0);
            }
    }

    // epilogue: lane holds rows 4 (lane >> 4) + v of tile i, token (lane & 15) of tile j
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int t = t0 + wt + j * 16 + lr;
            const int rb = r0 + wr + i * 16 + 4 * q;
            if (t >= a.m) continue;
            const float tsc = a.ts[t];
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[i][j][v] *= tsc;
            if (a.part) {  // K split: this split's partial products, the reduce applies the epilogue
                float* pr = a.part + (static_cast<size_t>(split) * a.m + t) * a.rows;
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    if (rb + v < a.rows) pr[rb + v] = acc[i][j][v];
                continue;
            }
            float* yr = a.y + static_cast<size_t>(t) * a.ldy;
            if constexpr (EPI == 2) {  // interleaved (gate, up) rows -> silu(gate) * up
#pragma unroll
                for (int v = 0; v < 4; v += 2)
                    if (rb + v + 1 < a.rows) yr[(rb + v) >> 1] = silu_dev(acc[i][j][v]) * acc[i][j][v + 1];
            } else {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    if (rb + v >= a.rows) continue;
                    if constexpr (EPI == 1)
                        yr[rb + v] += acc[i][j][v];
                    else
                        yr[rb + v] = acc[i][j][v];
                }
            }
        }
}

// The launch's tile (gemm_w4_mfma_kernel<4, 1, 2, 4, ...>): 128 rows x 64 tokens.
constexpr int kGemmBR = 128, kGemmBT = 64;
constexpr int kGemmMaxSplits = 4;

// K splits of a launch: with fewer than two blocks per CU (the 4096-row
// projections of a 512-token chunk: 256 blocks) the column groups are split
// over blockIdx.z, each split keeping at least 16 groups, and a second kernel
// adds the splits' partial products in a fixed order (deterministic).  The
// SiLU-pair epilogue (gate/up, 1536 blocks) is never split.
static int gemm_splits(int rows, int m, int cols, int epi) {
    if (epi == 2) return 1;
    const int blocks = ((m + kGemmBT - 1) / kGemmBT) * ((rows + kGemmBR - 1) / kGemmBR);
    const int G = cols / 64;
    int splits = 1;
    while (splits < kGemmMaxSplits && blocks * splits < 2 * 256 && G / (2 * splits) >= 16) splits *= 2;
    return splits;
}

static size_t gemm_prep_bytes(int m, int cols) {
    const size_t m_pad = static_cast<size_t>((m + kGemmPad - 1) / kGemmPad) * kGemmPad;
    return m_pad * static_cast<size_t>(cols) * (2 * sizeof(_Float16)) +
           m_pad * static_cast<size_t>(cols / 64) * sizeof(float) + m_pad * sizeof(float);
}

size_t gemm_workspace_bytes(int m, int cols, int rows) {
    const int splits = rows > 0 ? gemm_splits(rows, m, cols, 0) : 1;
    const size_t part = splits > 1 ? static_cast<size_t>(splits) * m * rows * sizeof(float) : 0;
    return gemm_prep_bytes(m, cols) + (part + 255) / 256 * 256;
}

// y[t][r] (op)= sum over splits z (in order) of part[z][t][r]; op: store, add
__global__ void __launch_bounds__(256) gemm_splitk_reduce_kernel(const float* __restrict__ part, int splits, int m,
                                                                 int rows, float* __restrict__ y, int ldy, int add) {
    const size_t n = static_cast<size_t>(m) * rows;
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        float v = part[i];
        for (int z = 1; z < splits; ++z) v += part[static_cast<size_t>(z) * n + i];
        const size_t t = i / rows, r = i - t * rows;
        float* yp = y + t * ldy + r;
        *yp = add ? *yp + v : v;
    }
}

bool gemm_supported(int rows, int cols, int group, int layout, const Prologue& pro) {
    if ((layout != 0 && layout != 2 && layout != 3 && layout != 4) || group != 64 || cols % 64 != 0 || cols / 64 > 256 ||
        rows <= 0)
        return false;
    if (pro.mode == PRO_GATED)
        return pro.head_dim > 0 && pro.head_dim % 8 == 0 && cols % pro.head_dim == 0 &&
               cols / pro.head_dim <= kPrepMaxHeads;
    return true;
}

template <int WGR, int WGT, int TI, int TJ, int EPI, int META>
static hipError_t launch_gemm_cfg(const GemmArgs& a, int splits, hipStream_t s) {
    using T = GemmTile<WGR, WGT, TI, TJ>;
    const auto fn = reinterpret_cast<const void*>(&gemm_w4_mfma_kernel<WGR, WGT, TI, TJ, EPI, META>);
    if constexpr (T::kLds > 64 * 1024) {  // beyond the default dynamic-LDS limit (gfx950 has 160 KiB per CU)
        if (hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(T::kLds));
            e != hipSuccess)
            return e;
    }
    static_assert(T::kBR == kGemmBR && T::kBT == kGemmBT, "split choice assumes this tile");
    const dim3 grid((a.m + T::kBT - 1) / T::kBT, (a.rows + T::kBR - 1) / T::kBR, splits);
    hipLaunchKernelGGL((gemm_w4_mfma_kernel<WGR, WGT, TI, TJ, EPI, META>), grid, dim3(T::kThreads), T::kLds, s, a);
    return hipGetLastError();
}

hipError_t launch_gemm(const GemmLaunch& p, hipStream_t s) {
    const int m_pad = (p.m + kGemmPad - 1) / kGemmPad * kGemmPad;
    _Float16* xh = static_cast<_Float16*>(p.workspace);
    _Float16* xl = xh + static_cast<size_t>(m_pad) * p.cols;
    float* xs = reinterpret_cast<float*>(xl + static_cast<size_t>(m_pad) * p.cols);
    float* ts = xs + static_cast<size_t>(m_pad) * (p.cols / 64);
    const int nk = p.cols / 2048;
    const bool vec = prep_vec_ok(p) && (nk == 1 || nk == 2 || nk == 6) &&
                     (nk == 1 ? launch_prep_vec<1>(p, m_pad, xh, xl, xs, ts, s)
                              : nk == 2 ? launch_prep_vec<2>(p, m_pad, xh, xl, xs, ts, s)
                                        : launch_prep_vec<6>(p, m_pad, xh, xl, xs, ts, s));
    if (!vec)
        hipLaunchKernelGGL(prep_x_kernel, dim3(m_pad), dim3(256), 0, s, p.x, p.ldx, p.m, p.cols, p.pro, p.ldz, xh, xl,
                           xs, ts);
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    const int splits = gemm_splits(p.rows, p.m, p.cols, p.epi);
    const int G = p.cols / 64;
    float* part = splits > 1 ? reinterpret_cast<float*>(static_cast<uint8_t*>(p.workspace) +
                                                        gemm_prep_bytes(m_pad, p.cols)) : nullptr;
    GemmArgs a{p.nib, static_cast<const uint32_t*>(p.meta), p.rows, p.cols, p.affine, p.zero_is_8, xh, xs, ts,
               (G + splits - 1) / splits, part, p.m, m_pad, p.y, p.ldy};
    // 128 rows x 64 tokens per block: four waves of 32 rows x 64 tokens
    // metadata form: 0 fp16 (scale, zero), 1 fp32 pair (layout 2), 2 fp16 scale, zero 8 (layout 3),
    // 3 fp32 scale and 4-bit zero (layout 4)
    const int meta = p.layout == 2 ? 1 : (p.layout == 3 ? 2 : (p.layout == 4 ? 3 : 0));
    hipError_t e = hipErrorInvalidValue;
    switch (p.epi * 4 + meta) {
        case 0: e = launch_gemm_cfg<4, 1, 2, 4, 0, 0>(a, splits, s); break;
        case 1: e = launch_gemm_cfg<4, 1, 2, 4, 0, 1>(a, splits, s); break;
        case 2: e = launch_gemm_cfg<4, 1, 2, 4, 0, 2>(a, splits, s); break;
        case 3: e = launch_gemm_cfg<4, 1, 2, 4, 0, 3>(a, splits, s); break;
        case 4: e = launch_gemm_cfg<4, 1, 2, 4, 1, 0>(a, splits, s); break;
        case 5: e = launch_gemm_cfg<4, 1, 2, 4, 1, 1>(a, splits, s); break;
        case 6: e = launch_gemm_cfg<4, 1, 2, 4, 1, 2>(a, splits, s); break;
        case 7: e = launch_gemm_cfg<4, 1, 2, 4, 1, 3>(a, splits, s); break;
        case 8: e = launch_gemm_cfg<4, 1, 2, 4, 2, 0>(a, splits, s); break;
        case 9: e = launch_gemm_cfg<4, 1, 2, 4, 2, 1>(a, splits, s); break;
        case 10: e = launch_gemm_cfg<4, 1, 2, 4, 2, 2>(a, splits, s); break;
        case 11: e = launch_gemm_cfg<4, 1, 2, 4, 2, 3>(a, splits, s); break;
        default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess || splits == 1) return e;
    const size_t n = static_cast<size_t>(p.m) * p.rows;
    const int blocks = static_cast<int>(std::min<size_t>((n + 255) / 256, 2048));
    hipLaunchKernelGGL(gemm_splitk_reduce_kernel, dim3(blocks), dim3(256), 0, s, part, splits, p.m, p.rows, p.y,
                       p.ldy, p.epi == 1 ? 1 : 0);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Causal GQA for a prompt chunk: block (t, kh) takes query token t (position
// pos0 + t) and the `group` query heads of kv head kh over keys 0..pos0+t in
// 64-token chunks with a running max / sum (rescaled by exp(m_old - m_new)),
// then normalises by multiplying with 1/l and applies the sigmoid gate
// (custom_model.cpp:840-951 per token).
// ---------------------------------------------------------------------------
constexpr int kPAttnChunk = 64;
constexpr int kPAttnMaxGroup = 8;

__global__ void __launch_bounds__(256) prefill_attn_kernel(PrefillAttnLaunch p) {
    extern __shared__ float smem[];
    const int t = blockIdx.x, kh = blockIdx.y;
    const int hd = p.head_dim, group = p.nq / p.nkv;
    const int ctx = *p.pos0 + t + 1;
    float* qs = smem;                        // [group][hd]
    float* sc = qs + group * hd;             // [group][64]
    float* osum = sc + group * kPAttnChunk;  // [group][hd] running output
    float* ml = osum + group * hd;           // [group][2] running max, sum
    float* fac = ml + 2 * group;             // [group] rescale of this chunk
    const float* qrow = p.q + static_cast<size_t>(t) * p.q_stride + static_cast<size_t>(kh) * group * hd;
    for (int i = threadIdx.x; i < group * hd; i += blockDim.x) {
        qs[i] = qrow[i];
        osum[i] = 0.0f;
    }
    if (threadIdx.x < group) {
        ml[2 * threadIdx.x] = -INFINITY;
        ml[2 * threadIdx.x + 1] = 0.0f;
    }
    __syncthreads();
    const float rscale = 1.0f / sqrtf(static_cast<float>(hd));
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    for (int c0 = 0; c0 < ctx; c0 += kPAttnChunk) {
        const int n = min(kPAttnChunk, ctx - c0);
        // scores: 4 threads per key, each a quarter of the dims
        {
            const int sub = threadIdx.x & 3, tt = threadIdx.x >> 2;
            const int dq = (hd + 3) / 4, d0 = sub * dq, d1 = min(hd, d0 + dq);
            const bool valid = tt < n;
            const _Float16* krow = p.k_cache + (static_cast<size_t>(c0 + (valid ? tt : 0)) * p.nkv + kh) * hd;
            for (int g = 0; g < group; ++g) {
                float dot = 0.0f;
                for (int d = d0; d < d1; ++d) dot += qs[g * hd + d] * static_cast<float>(krow[d]);
                dot = lanes_sum<4>(dot);
                if (valid && sub == 0) sc[g * kPAttnChunk + tt] = dot * rscale;
            }
        }
        __syncthreads();
        // online softmax update per head (one wave per head)
        for (int g = wid; g < group; g += blockDim.x / kWave) {
            const float sv = lane < n ? sc[g * kPAttnChunk + lane] : -INFINITY;
            const float mc = wave_max(sv);
            const float m_old = ml[2 * g];
            const float m_new = fmaxf(m_old, mc);
            const float e = lane < n ? expf(sv - m_new) : 0.0f;
            const float lsum = wave_sum(e);
            sc[g * kPAttnChunk + lane] = e;
            if (lane == 0) {
                const float f = expf(m_old - m_new);  // 0 for the first chunk
                fac[g] = f;
                ml[2 * g] = m_new;
                ml[2 * g + 1] = ml[2 * g + 1] * f + lsum;
            }
        }
        __syncthreads();
        for (int i = threadIdx.x; i < group * hd; i += blockDim.x) {
            const int g = i / hd, d = i % hd;
            float o = osum[i] * fac[g];
            for (int j = 0; j < n; ++j)
                o += sc[g * kPAttnChunk + j] *
                     static_cast<float>(p.v_cache[(static_cast<size_t>(c0 + j) * p.nkv + kh) * hd + d]);
            osum[i] = o;
        }
        __syncthreads();
    }
    for (int i = threadIdx.x; i < group * hd; i += blockDim.x) {
        const int g = i / hd;
        const float l = ml[2 * g + 1];
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        const size_t oi = static_cast<size_t>(t) * p.out_stride + static_cast<size_t>(kh) * group * hd + i;
        const size_t gi = static_cast<size_t>(t) * p.q_stride + static_cast<size_t>(kh) * group * hd + i;
        p.out[oi] = (osum[i] * inv) * sigmoid_dev(p.gate[gi]);
    }
}

// Matrix-core form for head_dim 128 and 4 query heads per kv head (the 9B
// shape): block (16-token tile, kv head), wave h = query head h of the kv head,
// keys in 64-key chunks with a running max / sum (rescaled by
// exp(m_old - m_new)), then 1/l and the sigmoid gate, as prefill_attn_kernel.
// Scores are formed transposed, S^T = K Q^T (keys are the MFMA rows), so a
// lane holds 16 keys of one token: the token's max and sum are over the lane's
// own values and the lanes 16 and 32 away, and its probabilities are already
// the B operand of O^T = V^T P^T.  q and p are split into fp16 hi + lo (about
// 22 bits together; k and v are fp16 in the cache), two
// v_mfma_f32_16x16x32_f16 per product, fp32 accumulation.  The k index of an
// MFMA may be any permutation of the keys as long as both operands use it:
// lane group g (lanes 16g..16g+15) feeds keys 32s + 4g + 0..3 and
// 32s + 16 + 4g + 0..3 of step s, the keys its score tiles hold.  A chunk's K
// (rows of 128 dims) and V (transposed: rows of 64 keys) go through LDS; the
// next chunk is loaded into registers while the current one is used.
constexpr int kFT = 16;        // tokens per tile
constexpr int kFLdk = 136;     // halves per K row in LDS
constexpr int kFLdv = 72;      // halves per V^T row in LDS
constexpr int kFHd = 128, kFGroup = 4;

template <int M>
__device__ __forceinline__ float xor_pair_max(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    if constexpr (M == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        return fmaxf(__builtin_bit_cast(float, static_cast<uint32_t>(r[0])),
                     __builtin_bit_cast(float, static_cast<uint32_t>(r[1])));
    } else {
        static_assert(M == 32, "pair distance");
        const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        return fmaxf(__builtin_bit_cast(float, static_cast<uint32_t>(r[0])),
                     __builtin_bit_cast(float, static_cast<uint32_t>(r[1])));
    }
}

// fp32 -> fp16 hi + fp16 lo (x - hi) of 8 values
__device__ __forceinline__ void split_h8(const float (&x)[8], half8& hi, half8& lo) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const _Float16 h = static_cast<_Float16>(x[e]);
        hi[e] = h;
        lo[e] = static_cast<_Float16>(x[e] - static_cast<float>(h));
    }
}

__global__ void __launch_bounds__(256) prefill_attn_mfma_kernel(PrefillAttnLaunch p) {
    __shared__ _Float16 Ks[kPAttnChunk * kFLdk];
    __shared__ _Float16 Vt[kFHd * kFLdv];
    const int t0 = blockIdx.x * kFT, kh = blockIdx.y;
    const int lane = threadIdx.x & (kWave - 1), h = threadIdx.x / kWave;
    const int tl = lane & 15, g = lane >> 4;
    // block-uniform values computed with vector ops are made scalar with
    // readfirstlane: a buffer descriptor built from a vector register becomes a
    // loop over the distinct values of the wave
    const int pos0 = *p.pos0;
    const int ntok = __builtin_amdgcn_readfirstlane(min(kFT, p.tokens - t0));
    const int qpos = pos0 + t0 + tl;        // this lane's token
    const int last = pos0 + t0 + ntok - 1;  // last key any token of the tile sees
    const int qh = kh * kFGroup + h;
    const float rscale = 1.0f / sqrtf(static_cast<float>(kFHd));
    // q fragments: lane supplies Q[token tl][dims 32 s + 8 g .. + 7] (tokens past ntok read 0)
    const uint32_t qrow = static_cast<uint32_t>(p.q_stride) * 4u;
    const __amdgpu_buffer_rsrc_t r_q = buf_rsrc(p.q + static_cast<size_t>(t0) * p.q_stride, ntok * qrow);
    half8 qhi[4], qlo[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const uint32_t off = static_cast<uint32_t>(tl) * qrow + (static_cast<uint32_t>(qh) * kFHd + 32 * s + 8 * g) * 4u;
        const auto a = __builtin_amdgcn_raw_buffer_load_b128(r_q, off, 0, 0);
        const auto b = __builtin_amdgcn_raw_buffer_load_b128(r_q, off + 16u, 0, 0);
        const float x[8] = {__uint_as_float(a[0]), __uint_as_float(a[1]), __uint_as_float(a[2]), __uint_as_float(a[3]),
                            __uint_as_float(b[0]), __uint_as_float(b[1]), __uint_as_float(b[2]), __uint_as_float(b[3])};
        split_h8(x, qhi[s], qlo[s]);
    }
    // chunk loads: piece i = threadIdx + 256 u is key i & 63, dims 8 (i >> 6) .. + 7
    const uint32_t krow = static_cast<uint32_t>(p.nkv) * kFHd * 2u;  // bytes per cache position
    u32x4 kr[4], vr[4];
    auto load_chunk = [&](int c0) {
        const uint32_t range =
            static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(max(0, min(kPAttnChunk, last - c0 + 1)))) * krow;
        const size_t base = static_cast<size_t>(__builtin_amdgcn_readfirstlane(max(0, min(c0, last)))) * p.nkv * kFHd +
                            static_cast<size_t>(kh) * kFHd;
        const __amdgpu_buffer_rsrc_t rk = buf_rsrc(p.k_cache + base, range), rv = buf_rsrc(p.v_cache + base, range);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = static_cast<int>(threadIdx.x) + 256 * u;
            const uint32_t off = static_cast<uint32_t>(i & 63) * krow + static_cast<uint32_t>(i >> 6) * 16u;
            kr[u] = __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0);
            vr[u] = __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0);
        }
    };
    float m = -INFINITY, l = 0.0f;
    floatx4 o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    const floatx4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
    load_chunk(0);
    for (int c0 = 0; c0 <= last; c0 += kPAttnChunk) {  // block-uniform
        __syncthreads();  // the previous chunk's K and V have been read
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = static_cast<int>(threadIdx.x) + 256 * u, key = i & 63, d8 = i >> 6;
            *reinterpret_cast<u32x4*>(Ks + key * kFLdk + 8 * d8) = kr[u];
            const uint32_t w[4] = {vr[u][0], vr[u][1], vr[u][2], vr[u][3]};
#pragma unroll
            for (int e = 0; e < 8; ++e)
                Vt[(8 * d8 + e) * kFLdv + key] = __builtin_bit_cast(_Float16, static_cast<uint16_t>(w[e >> 1] >> (16 * (e & 1))));
        }
        __syncthreads();
        load_chunk(c0 + kPAttnChunk);  // past `last`: reads 0, never stored as data
        // S^T tiles c: keys c0 + 16 c + 4 g + v of token tl
        floatx4 sc[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            sc[c] = zero4;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const half8 a = *reinterpret_cast<const half8*>(Ks + (16 * c + tl) * kFLdk + 32 * s + 8 * g);
                sc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qhi[s], sc[c], 0, 0, 0);
                sc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qlo[s], sc[c], 0, 0, 0);
            }
        }
        // causal mask, the token's chunk max and sum, online rescale
        float mc = -INFINITY;
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const bool ok = c0 + 16 * c + 4 * g + v <= qpos;
                sc[c][v] = ok ? sc[c][v] * rscale : -INFINITY;
                mc = fmaxf(mc, sc[c][v]);
            }
        mc = xor_pair_max<32>(xor_pair_max<16>(mc));
        const float m_new = fmaxf(m, mc);
        float ls = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float e = sc[c][v] == -INFINITY ? 0.0f : expf(sc[c][v] - m_new);
                sc[c][v] = e;
                ls += e;
            }
        ls = xor_pair_sum<32>(xor_pair_sum<16>(ls));
        const float f = m == -INFINITY ? 0.0f : expf(m - m_new);
        m = m_new;
        l = l * f + ls;
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] *= f;
        // P^T fragments of key steps s2 (keys 32 s2 + 4 g + v, then 32 s2 + 16 + 4 g + v)
        half8 phi[2], plo[2];
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
            const float x[8] = {sc[2 * s2][0], sc[2 * s2][1], sc[2 * s2][2], sc[2 * s2][3],
                                sc[2 * s2 + 1][0], sc[2 * s2 + 1][1], sc[2 * s2 + 1][2], sc[2 * s2 + 1][3]};
            split_h8(x, phi[s2], plo[s2]);
        }
        // O^T tiles j: dims 16 j + 4 g + v of token tl
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
                const _Float16* vrow = Vt + (16 * j + tl) * kFLdv + 32 * s2 + 4 * g;
                const u32x2 lo4 = *reinterpret_cast<const u32x2*>(vrow);
                const u32x2 hi4 = *reinterpret_cast<const u32x2*>(vrow + 16);
                const half8 a = __builtin_bit_cast(half8, u32x4{lo4[0], lo4[1], hi4[0], hi4[1]});
                o[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, phi[s2], o[j], 0, 0, 0);
                o[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, plo[s2], o[j], 0, 0, 0);
            }
    }
    if (tl >= ntok) return;
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    const size_t head = static_cast<size_t>(qh) * kFHd + 4 * g;
    const float* gr = p.gate + static_cast<size_t>(t0 + tl) * p.q_stride + head;
    float* orow = p.out + static_cast<size_t>(t0 + tl) * p.out_stride + head;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float4 gv = *reinterpret_cast<const float4*>(gr + 16 * j);
        *reinterpret_cast<float4*>(orow + 16 * j) =
            make_float4((o[j][0] * inv) * sigmoid_dev(gv.x), (o[j][1] * inv) * sigmoid_dev(gv.y),
                        (o[j][2] * inv) * sigmoid_dev(gv.z), (o[j][3] * inv) * sigmoid_dev(gv.w));
    }
}

bool prefill_attn_supported(int nq, int nkv, int head_dim) {
    return nkv > 0 && nq % nkv == 0 && nq / nkv <= kPAttnMaxGroup && head_dim > 0 &&
           sizeof(float) * (2 * (nq / nkv) * head_dim + (nq / nkv) * (kPAttnChunk + 3)) <= 64 * 1024;
}

hipError_t launch_prefill_attn(const PrefillAttnLaunch& p, hipStream_t s) {
    const int group = p.nq / p.nkv;
    // the matrix-core kernel reads q, the gate and the output as 16-byte pieces
    const bool al16 = ((reinterpret_cast<uintptr_t>(p.q) | reinterpret_cast<uintptr_t>(p.gate) |
                        reinterpret_cast<uintptr_t>(p.out)) & 15u) == 0 && p.q_stride % 4 == 0 && p.out_stride % 4 == 0;
    if (p.head_dim == kFHd && group == kFGroup && al16) {
        hipLaunchKernelGGL(prefill_attn_mfma_kernel, dim3((p.tokens + kFT - 1) / kFT, p.nkv), dim3(256), 0, s, p);
        return hipGetLastError();
    }
    const size_t lds = sizeof(float) * (2 * static_cast<size_t>(group) * p.head_dim + group * (kPAttnChunk + 3));
    hipLaunchKernelGGL(prefill_attn_kernel, dim3(p.tokens, p.nkv), dim3(256), lds, s, p);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Linear attention over a prompt chunk: block (vh, 16-column slice) runs the
// decode step of linear_step_kernel for tokens 0..tokens-1 in order, with its
// recurrent-state columns and the conv history of the channels it computes
// held in registers for the whole chunk.  The history is read from hist_in
// and the final one written to hist_out (distinct buffers: the caller picks
// the parity copies); the q/k history is written by one block per key head,
// the value history by the block that owns the channel.
// ---------------------------------------------------------------------------
constexpr int kScanCols = 16;
constexpr int kScanIGroups = 16;
constexpr int kScanMaxK = 16;     // key dim <= 256
constexpr int kScanMaxHist = 7;   // conv kernel <= 8
constexpr int kScanMaxQkPerThread = 2;
constexpr int kScanAhead = 4;       // tokens per load group

__global__ void __launch_bounds__(256) linear_scan_kernel(LinearScanLaunch p) {
    __shared__ float qk[2 * 256];
    __shared__ float vsh[kScanCols];
    __shared__ float colsum[4][kScanCols];
    __shared__ float red[2][4];
    const int vh = blockIdx.x;
    const int j0 = blockIdx.y * kScanCols;
    const int factor = max(1, p.lv_n / max(1, p.lk_n));
    const int kh = min(p.lk_n - 1, vh / factor);
    const int dk = p.lk_hd, dv = p.lv_hd;
    const int hist = max(0, p.ksize - 1);
    const bool qk_writer = (vh % factor == 0) && blockIdx.y == 0;
    const int jl = threadIdx.x % kScanCols;
    const int ig = threadIdx.x / kScanCols;
    const int j = j0 + jl;
    const bool active = j < dv;
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    float* S = p.state + static_cast<size_t>(vh) * dk * dv;
    float sreg[kScanMaxK];
#pragma unroll
    for (int r = 0; r < kScanMaxK; ++r) {
        const int i = ig + r * kScanIGroups;
        sreg[r] = (active && i < dk) ? S[static_cast<size_t>(i) * dv + j] : 0.0f;
    }
    // channels this thread convolves: q/k channels tid and tid + 256 (< 2 dk),
    // and (threads < 16) the value channel of column j0 + tid
    int ch[kScanMaxQkPerThread + 1];
    float hreg[kScanMaxQkPerThread + 1][kScanMaxHist];
    float wreg[kScanMaxQkPerThread + 1][kScanMaxHist];
    float wx[kScanMaxQkPerThread + 1];
#pragma unroll
    for (int u = 0; u <= kScanMaxQkPerThread; ++u) {
        int c = -1;
        if (u < kScanMaxQkPerThread) {
            const int tq = threadIdx.x + u * 256;
            if (tq < 2 * dk) c = (tq >= dk ? p.lk_n * dk : 0) + kh * dk + (tq >= dk ? tq - dk : tq);
        } else if (threadIdx.x < kScanCols && j0 + static_cast<int>(threadIdx.x) < dv) {
            c = 2 * p.lk_n * dk + vh * dv + j0 + threadIdx.x;
        }
        ch[u] = c;
#pragma unroll
        for (int i = 0; i < kScanMaxHist; ++i) {
            hreg[u][i] = (c >= 0 && i < hist) ? p.hist_in[static_cast<size_t>(c) * hist + i] : 0.0f;
            wreg[u][i] = (c >= 0 && i < hist) ? p.conv_w[static_cast<size_t>(c) * p.ksize + i] : 0.0f;
        }
        wx[u] = c >= 0 ? p.conv_w[static_cast<size_t>(c) * p.ksize + hist] : 0.0f;
    }
    const float rdk = 1.0f / sqrtf(static_cast<float>(dk));
    const float neg_exp_alog = -expf(p.a_log[vh]);
    const float dtb = p.dt_bias[vh];
    // Token inputs are loaded kScanAhead tokens at a time, one group ahead of
    // the group being computed (a token's compute is shorter than a load's
    // latency), with range-checked buffer loads: rows past the last token
    // read as 0 without a memory access, so every load is unconditional.
    const uint32_t stride4 = static_cast<uint32_t>(p.mixed_stride) * 4u;
    const __amdgpu_buffer_rsrc_t r_mixed = buf_rsrc(p.mixed, static_cast<uint32_t>(p.tokens) * stride4);
    const uint32_t ab_bytes = static_cast<uint32_t>(p.tokens - 1) * stride4 + static_cast<uint32_t>(p.lv_n) * 4u;
    const __amdgpu_buffer_rsrc_t r_a = buf_rsrc(p.a, ab_bytes), r_b = buf_rsrc(p.b, ab_bytes);
    float xg[2][kScanAhead][kScanMaxQkPerThread + 1], ag[2][kScanAhead], bg[2][kScanAhead];
    auto load_group = [&](int t0, int buf) {
#pragma unroll
        for (int k = 0; k < kScanAhead; ++k) {
            const uint32_t row = static_cast<uint32_t>(t0 + k) * stride4;
#pragma unroll
            for (int u = 0; u <= kScanMaxQkPerThread; ++u)
                xg[buf][k][u] = buf_load_f32(r_mixed, ch[u] >= 0 ? row + static_cast<uint32_t>(ch[u]) * 4u : kBufOOB);
            ag[buf][k] = buf_load_f32(r_a, row + static_cast<uint32_t>(vh) * 4u);
            bg[buf][k] = buf_load_f32(r_b, row + static_cast<uint32_t>(vh) * 4u);
        }
    };
    load_group(0, 0);
    for (int t0 = 0; t0 < p.tokens; t0 += kScanAhead) {
        load_group(t0 + kScanAhead, 1);
#pragma unroll
        for (int k = 0; k < kScanAhead; ++k) {
        const int t = t0 + k;
        if (t >= p.tokens) break;  // block-uniform
        float xcur[kScanMaxQkPerThread + 1];
#pragma unroll
        for (int u = 0; u <= kScanMaxQkPerThread; ++u) xcur[u] = xg[0][k][u];
        const float a_cur = ag[0][k], b_cur = bg[0][k];
        float ssq = 0.0f, ssk = 0.0f;
#pragma unroll
        for (int u = 0; u <= kScanMaxQkPerThread; ++u) {
            const int c = ch[u];
            if (c < 0) continue;
            const float xv = xcur[u];
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < kScanMaxHist; ++i)
                if (i < hist) acc += hreg[u][i] * wreg[u][i];
            acc += xv * wx[u];
#pragma unroll
            for (int i = 0; i < kScanMaxHist; ++i) {
                if (i + 1 < hist) hreg[u][i] = hreg[u][i + 1];
                else if (i + 1 == hist) hreg[u][i] = xv;
            }
            const float yv = silu_dev(acc);
            if (u < kScanMaxQkPerThread) {
                const int tq = threadIdx.x + u * 256;
                const bool is_k = tq >= dk;
                qk[(is_k ? 256 : 0) + (is_k ? tq - dk : tq)] = yv;
                if (is_k)
                    ssk += yv * yv;
                else
                    ssq += yv * yv;
            } else {
                vsh[threadIdx.x] = yv;
            }
        }
        ssq = wave_sum(ssq);
        ssk = wave_sum(ssk);
        if (lane == 0) {
            red[0][wid] = ssq;
            red[1][wid] = ssk;
        }
        const float beta = sigmoid_dev(b_cur);
        const float gate = neg_exp_alog * softplus_dev(a_cur + dtb);
        const float decay = expf(gate);
        __syncthreads();
        const float invq = 1.0f / sqrtf(red[0][0] + red[0][1] + red[0][2] + red[0][3] + 1.0e-6f);
        const float invk = 1.0f / sqrtf(red[1][0] + red[1][1] + red[1][2] + red[1][3] + 1.0e-6f);
        const float vj = active ? vsh[jl] : 0.0f;
        float pred = 0.0f;
#pragma unroll
        for (int r = 0; r < kScanMaxK; ++r) {
            const int i = ig + r * kScanIGroups;
            if (active && i < dk) {
                sreg[r] *= decay;
                pred += sreg[r] * (qk[256 + i] * invk);
            }
        }
        pred = xor_pair_sum<32>(xor_pair_sum<16>(pred));
        if (lane < kScanCols) colsum[wid][lane] = pred;
        __syncthreads();
        pred = colsum[0][jl] + colsum[1][jl] + colsum[2][jl] + colsum[3][jl];
        __syncthreads();
        const float delta = active ? beta * (vj - pred) : 0.0f;
        float o = 0.0f;
#pragma unroll
        for (int r = 0; r < kScanMaxK; ++r) {
            const int i = ig + r * kScanIGroups;
            if (active && i < dk) {
                sreg[r] += (qk[256 + i] * invk) * delta;
                o += sreg[r] * (qk[i] * invq);
            }
        }
        o = xor_pair_sum<32>(xor_pair_sum<16>(o));
        if (lane < kScanCols) colsum[wid][lane] = o;
        __syncthreads();
        if (threadIdx.x < kScanCols && active) {
            const float tot = colsum[0][jl] + colsum[1][jl] + colsum[2][jl] + colsum[3][jl];
            p.out[static_cast<size_t>(t) * p.out_stride + static_cast<size_t>(vh) * dv + j] = tot * rdk;
        }
        __syncthreads();  // qk, vsh, red and colsum are rewritten by the next token
        }
#pragma unroll
        for (int k = 0; k < kScanAhead; ++k) {
#pragma unroll
            for (int u = 0; u <= kScanMaxQkPerThread; ++u) xg[0][k][u] = xg[1][k][u];
            ag[0][k] = ag[1][k];
            bg[0][k] = bg[1][k];
        }
    }
#pragma unroll
    for (int r = 0; r < kScanMaxK; ++r) {
        const int i = ig + r * kScanIGroups;
        if (active && i < dk) S[static_cast<size_t>(i) * dv + j] = sreg[r];
    }
#pragma unroll
    for (int u = 0; u <= kScanMaxQkPerThread; ++u) {
        const int c = ch[u];
        if (c < 0 || (u < kScanMaxQkPerThread && !qk_writer)) continue;
#pragma unroll
        for (int i = 0; i < kScanMaxHist; ++i)
            if (i < hist) p.hist_out[static_cast<size_t>(c) * hist + i] = hreg[u][i];
    }
}

// Wave-independent form for key dim DK and conv size KS (the 9B shape: 128, 4).
// Wave w of block (vh, y) owns CPW value columns of head vh; lane l owns
// column l / (64/CPW) and key rows i = l % (64/CPW) + (64/CPW) r, so both sums
// over the key dimension (the prediction and the output) are reductions over
// the 16 lanes of a DPP row (CPW = 4) or two rows (CPW = 2, one permlane swap).  Every wave convolves the whole q/k head itself (cheap) and
// exchanges the convolved channels through its own LDS slice, so a token
// needs no block barrier at all.
template <int DK, int KS, int CPW>
__global__ void __launch_bounds__(256) linear_scan_wave_kernel(LinearScanLaunch p) {
    constexpr int CH = 2 * DK / kWave;  // q/k channels per lane
    constexpr int LPC = kWave / CPW;    // lanes per value column
    constexpr int RS = DK / LPC;        // state rows per lane
    constexpr int BC = 4 * CPW;         // value columns per block
    constexpr int H = KS - 1;
    static_assert(CH >= 1 && CH % 2 == 0 && RS >= 1, "key dim");
    __shared__ float qk_lds[4][2 * DK];
    const int vh = blockIdx.x;
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    const int factor = max(1, p.lv_n / max(1, p.lk_n));
    const int kh = min(p.lk_n - 1, vh / factor);
    const int dv = p.lv_hd;
    const int ig = lane % LPC;
    const int j = blockIdx.y * BC + wid * CPW + lane / LPC;
    const bool active = j < dv;
    float* qk_w = qk_lds[wid];
    auto qk_channel = [&](int t) { return (t >= DK ? p.lk_n * DK : 0) + kh * DK + (t % DK); };
    const int vch = 2 * p.lk_n * DK + vh * dv + j;
    // filter taps and history (history in registers across the tokens)
    float hq[CH][H > 0 ? H : 1], wq[CH][KS], hv[H > 0 ? H : 1], wvv[KS];
#pragma unroll
    for (int u = 0; u < CH; ++u) {
        const int c = qk_channel(lane + u * kWave);
#pragma unroll
        for (int t = 0; t < H; ++t) hq[u][t] = p.hist_in[static_cast<size_t>(c) * H + t];
#pragma unroll
        for (int t = 0; t < KS; ++t) wq[u][t] = p.conv_w[static_cast<size_t>(c) * KS + t];
    }
#pragma unroll
    for (int t = 0; t < H; ++t) hv[t] = active ? p.hist_in[static_cast<size_t>(vch) * H + t] : 0.0f;
#pragma unroll
    for (int t = 0; t < KS; ++t) wvv[t] = active ? p.conv_w[static_cast<size_t>(vch) * KS + t] : 0.0f;
    float* S = p.state + static_cast<size_t>(vh) * DK * dv;
    float sreg[RS];
#pragma unroll
    for (int r = 0; r < RS; ++r) sreg[r] = active ? S[static_cast<size_t>(ig + LPC * r) * dv + j] : 0.0f;
    const float rdk = 1.0f / sqrtf(static_cast<float>(DK));
    const float neg_exp_alog = -expf(p.a_log[vh]);
    const float dtb = p.dt_bias[vh];
    // token inputs, a group of kScanAhead tokens ahead (range-checked: rows past
    // the last token read 0 without a memory access)
    const uint32_t stride4 = static_cast<uint32_t>(p.mixed_stride) * 4u;
    const __amdgpu_buffer_rsrc_t r_mixed = buf_rsrc(p.mixed, static_cast<uint32_t>(p.tokens) * stride4);
    const uint32_t ab_bytes = static_cast<uint32_t>(p.tokens - 1) * stride4 + static_cast<uint32_t>(p.lv_n) * 4u;
    const __amdgpu_buffer_rsrc_t r_a = buf_rsrc(p.a, ab_bytes), r_b = buf_rsrc(p.b, ab_bytes);
    float xg[2][kScanAhead][CH + 1], ag[2][kScanAhead], bg[2][kScanAhead];
    auto load_group = [&](int t0, int buf) {
#pragma unroll
        for (int k = 0; k < kScanAhead; ++k) {
            const uint32_t row = static_cast<uint32_t>(t0 + k) * stride4;
#pragma unroll
            for (int u = 0; u < CH; ++u)
                xg[buf][k][u] = buf_load_f32(r_mixed, row + static_cast<uint32_t>(qk_channel(lane + u * kWave)) * 4u);
            xg[buf][k][CH] = buf_load_f32(r_mixed, active ? row + static_cast<uint32_t>(vch) * 4u : kBufOOB);
            ag[buf][k] = buf_load_f32(r_a, row + static_cast<uint32_t>(vh) * 4u);
            bg[buf][k] = buf_load_f32(r_b, row + static_cast<uint32_t>(vh) * 4u);
        }
    };
    auto conv_step = [&](float (&h)[H > 0 ? H : 1], const float (&w)[KS], float x) {
        float acc = 0.0f;
#pragma unroll
        for (int t = 0; t < H; ++t) acc += h[t] * w[t];
        acc += x * w[H];
#pragma unroll
        for (int t = 0; t + 1 < H; ++t) h[t] = h[t + 1];
        if constexpr (H > 0) h[H - 1] = x;
        return silu_dev(acc);
    };
    load_group(0, 0);
    for (int t0 = 0; t0 < p.tokens; t0 += kScanAhead) {
        load_group(t0 + kScanAhead, 1);
#pragma unroll
        for (int k = 0; k < kScanAhead; ++k) {
            const int t = t0 + k;
            if (t >= p.tokens) break;  // grid-uniform
            float ssq = 0.0f, ssk = 0.0f;
#pragma unroll
            for (int u = 0; u < CH; ++u) {
                const float y = conv_step(hq[u], wq[u], xg[0][k][u]);
                qk_w[lane + u * kWave] = y;
                if (u < CH / 2) ssq += y * y; else ssk += y * y;
            }
            const float vj = conv_step(hv, wvv, xg[0][k][CH]);
            ssq = wave_sum(ssq);
            ssk = wave_sum(ssk);
            const float invq = 1.0f / sqrtf(ssq + 1.0e-6f);
            const float invk = 1.0f / sqrtf(ssk + 1.0e-6f);
            const float beta = sigmoid_dev(bg[0][k]);
            const float decay = expf(neg_exp_alog * softplus_dev(ag[0][k] + dtb));
            // the wave's own LDS writes above complete before these reads (LDS
            // operations of a wave are performed in order): no barrier
            float kr[RS], qr[RS];
#pragma unroll
            for (int r = 0; r < RS; ++r) {
                kr[r] = qk_w[DK + ig + LPC * r] * invk;
                qr[r] = qk_w[ig + LPC * r] * invq;
            }
            float pred = 0.0f;
#pragma unroll
            for (int r = 0; r < RS; ++r) {
                sreg[r] *= decay;
                pred += sreg[r] * kr[r];
            }
            pred = lanes_sum<16>(pred);
            if constexpr (LPC == 32) pred = xor_pair_sum<16>(pred);
            const float delta = beta * (vj - pred);
            float o = 0.0f;
#pragma unroll
            for (int r = 0; r < RS; ++r) {
                sreg[r] += kr[r] * delta;
                o += sreg[r] * qr[r];
            }
            o = lanes_sum<16>(o);
            if constexpr (LPC == 32) o = xor_pair_sum<16>(o);
            if (ig == 0 && active) p.out[static_cast<size_t>(t) * p.out_stride + static_cast<size_t>(vh) * dv + j] = o * rdk;
        }
#pragma unroll
        for (int k = 0; k < kScanAhead; ++k) {
#pragma unroll
            for (int u = 0; u <= CH; ++u) xg[0][k][u] = xg[1][k][u];
            ag[0][k] = ag[1][k];
            bg[0][k] = bg[1][k];
        }
    }
#pragma unroll
    for (int r = 0; r < RS; ++r)
        if (active) S[static_cast<size_t>(ig + LPC * r) * dv + j] = sreg[r];
    const bool qk_writer = (vh % factor == 0) && blockIdx.y == 0 && wid == 0;
    if (qk_writer) {
#pragma unroll
        for (int u = 0; u < CH; ++u) {
            const int c = qk_channel(lane + u * kWave);
#pragma unroll
            for (int t = 0; t < H; ++t) p.hist_out[static_cast<size_t>(c) * H + t] = hq[u][t];
        }
    }
    if (ig == 0 && active) {
#pragma unroll
        for (int t = 0; t < H; ++t) p.hist_out[static_cast<size_t>(vch) * H + t] = hv[t];
    }
}

// ---------------------------------------------------------------------------
// Two-pass form of the prefill linear-attention scan (with a workspace, key
// heads of 128 dims):
// 1. linear_conv_prefill_tg_kernel / linear_conv_prefill_kernel, parallel over
//    tokens and heads: the causal conv1d + SiLU of every channel for every
//    token of the chunk (inputs of earlier tokens from the chunk, before the
//    chunk from hist_in), the L2 norm of the q and k heads, the per-(token,
//    value head) beta = sigmoid(b) and log decay g = -exp(A_log) softplus(a +
//    dt_bias), and the final history.
// 2. the chunked recurrence (scan_chunk_prep_kernel, scan_chunk_state_kernel,
//    below): parallel over 64-token chunks except for one pass over the chunks
//    per (value head, 16 columns).
// Workspace: conv output [tokens][conv_dim], (beta, g) [tokens][lv_n][2], then
// per (chunk, value head) the record T [64][64], Wq [64][64], gamma [64],
// gamma_last / gamma [64].
// ---------------------------------------------------------------------------
constexpr int kChunkTokens = 64;
constexpr int kChunkRecord = 2 * kChunkTokens * kChunkTokens + 2 * kChunkTokens;

size_t linear_scan_workspace_bytes(int tokens, int lk_n, int lk_hd, int lv_n, int lv_hd) {
    const size_t conv_dim = 2 * static_cast<size_t>(lk_n) * lk_hd + static_cast<size_t>(lv_n) * lv_hd;
    const size_t chunks = (static_cast<size_t>(tokens) + kChunkTokens - 1) / kChunkTokens;
    return sizeof(float) * (static_cast<size_t>(tokens) * (conv_dim + 2 * static_cast<size_t>(lv_n)) +
                            chunks * lv_n * kChunkRecord);
}

__global__ void __launch_bounds__(256) linear_conv_prefill_kernel(LinearScanLaunch p) {
    __shared__ float red[4];
    const int t = blockIdx.x, hb = blockIdx.y;
    const int dk = p.lk_hd, dv = p.lv_hd, H = p.ksize - 1;
    const int conv_dim = 2 * p.lk_n * dk + p.lv_n * dv;
    const bool is_qk = hb < 2 * p.lk_n;
    const int width = is_qk ? dk : dv;
    const int c = (is_qk ? hb * dk : 2 * p.lk_n * dk + (hb - 2 * p.lk_n) * dv) + static_cast<int>(threadIdx.x);
    const bool ok = static_cast<int>(threadIdx.x) < width;
    // input of token tau of the chunk (tau < 0: the history before it)
    auto xin = [&](int tau) {
        return tau >= 0 ? p.mixed[static_cast<size_t>(tau) * p.mixed_stride + c]
                        : p.hist_in[static_cast<size_t>(c) * H + (H + tau)];
    };
    float y = 0.0f;
    if (ok) {
        const float* w = p.conv_w + static_cast<size_t>(c) * p.ksize;
        float acc = 0.0f;
        for (int i = 0; i < H; ++i) acc += xin(t - H + i) * w[i];
        acc += xin(t) * w[H];
        y = silu_dev(acc);
        if (t == p.tokens - 1)
            for (int i = 0; i < H; ++i) p.hist_out[static_cast<size_t>(c) * H + i] = xin(p.tokens - H + i);
    }
    if (is_qk) {  // l2NormalizeHeads: x / sqrt(sum x^2 + 1e-6)
        float ss = wave_sum(y * y);
        const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
        if (lane == 0) red[wid] = ss;
        __syncthreads();
        ss = 0.0f;
        for (int i = 0; i < (width + kWave - 1) / kWave; ++i) ss += red[i];
        y *= 1.0f / sqrtf(ss + 1.0e-6f);
    } else if (threadIdx.x == 0) {
        const int vh = hb - 2 * p.lk_n;
        const size_t row = static_cast<size_t>(t) * p.mixed_stride + vh;
        float* aux = p.ws + static_cast<size_t>(p.tokens) * conv_dim + (static_cast<size_t>(t) * p.lv_n + vh) * 2;
        aux[0] = sigmoid_dev(p.b[row]);
        aux[1] = -expf(p.a_log[vh]) * softplus_dev(p.a[row] + p.dt_bias[vh]);  // log of the decay
    }
    if (ok) p.ws[static_cast<size_t>(t) * conv_dim + c] = y;
}

// The same pass for 128-channel heads and a conv kernel of KS taps, one block
// per (head, kConvTokens tokens): each thread keeps its channel's inputs for
// the tokens and the KS - 1 before them in registers (every input read once,
// range-checked buffer loads with no branch around them), and the q / k norms
// of the block's tokens share one barrier.  Same arithmetic and order as
// linear_conv_prefill_kernel.
constexpr int kConvTokens = 16;

template <int KS>
__global__ void __launch_bounds__(128) linear_conv_prefill_tg_kernel(LinearScanLaunch p) {
    constexpr int H = KS - 1, TG = kConvTokens, W = TG + H;
    __shared__ float red[2][TG];
    const int hb = blockIdx.x, g0 = blockIdx.y * TG;
    const int conv_dim = 2 * p.lk_n * 128 + p.lv_n * 128;
    const bool is_qk = hb < 2 * p.lk_n;
    const int c = (is_qk ? hb * 128 : 2 * p.lk_n * 128 + (hb - 2 * p.lk_n) * 128) + static_cast<int>(threadIdx.x);
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    // window slot i holds the input of token g0 - H + i: rows [r0, r1) of the
    // chunk, the history before token 0 (only the first group reaches it)
    const int r0 = max(0, g0 - H), r1 = min(p.tokens, g0 + TG);
    const uint32_t stride4 = static_cast<uint32_t>(p.mixed_stride) * 4u;
    const __amdgpu_buffer_rsrc_t r_x =
        buf_rsrc(p.mixed + static_cast<size_t>(r0) * p.mixed_stride, static_cast<uint32_t>(r1 - r0) * stride4);
    const __amdgpu_buffer_rsrc_t r_h = buf_rsrc(p.hist_in, static_cast<uint32_t>(conv_dim * H) * 4u);
    float xw[W], w[KS];
#pragma unroll
    for (int i = 0; i < W; ++i) {
        const int tau = g0 - H + i;
        float v = buf_load_f32(r_x, tau >= r0 ? static_cast<uint32_t>(tau - r0) * stride4 + c * 4u : kBufOOB);
        if (i < H) v += buf_load_f32(r_h, tau < 0 ? static_cast<uint32_t>(c * H + H + tau) * 4u : kBufOOB);
        xw[i] = v;
    }
#pragma unroll
    for (int i = 0; i < KS; ++i) w[i] = p.conv_w[static_cast<size_t>(c) * KS + i];
    float y[TG];
#pragma unroll
    for (int k = 0; k < TG; ++k) {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < H; ++i) acc += xw[k + i] * w[i];
        acc += xw[k + H] * w[H];
        y[k] = silu_dev(acc);
    }
    if (is_qk) {  // block-uniform; l2NormalizeHeads: x / sqrt(sum x^2 + 1e-6)
#pragma unroll
        for (int k = 0; k < TG; ++k) {
            const float ss = wave_sum(y[k] * y[k]);
            if (lane == 0) red[wid][k] = ss;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < TG; ++k) {
            float ss = 0.0f;
            ss += red[0][k];
            ss += red[1][k];
            y[k] *= 1.0f / sqrtf(ss + 1.0e-6f);
        }
    } else if (threadIdx.x < TG && g0 + static_cast<int>(threadIdx.x) < p.tokens) {
        const int t = g0 + threadIdx.x, vh = hb - 2 * p.lk_n;
        const size_t row = static_cast<size_t>(t) * p.mixed_stride + vh;
        float* aux = p.ws + static_cast<size_t>(p.tokens) * conv_dim + (static_cast<size_t>(t) * p.lv_n + vh) * 2;
        aux[0] = sigmoid_dev(p.b[row]);
        aux[1] = -expf(p.a_log[vh]) * softplus_dev(p.a[row] + p.dt_bias[vh]);  // log of the decay
    }
#pragma unroll
    for (int k = 0; k < TG; ++k)
        if (g0 + k < p.tokens) p.ws[static_cast<size_t>(g0 + k) * conv_dim + c] = y[k];
    // the history after the chunk: inputs of tokens tokens - H .. tokens - 1, slots
    // tokens - g0 + i of the group that holds the last token
    if (g0 <= p.tokens - 1 && p.tokens - 1 < g0 + TG) {
        const int base = p.tokens - g0;
#pragma unroll
        for (int i = 0; i < H; ++i) {
            float v = 0.0f;
#pragma unroll
            for (int j = 0; j < W; ++j)
                if (j == base + i) v = xw[j];
            p.hist_out[static_cast<size_t>(c) * H + i] = v;
        }
    }
}

// Chunked (parallel-in-time) form of the gated-delta recurrence over a prompt
// chunk, for key heads of 128 dims.  Within a chunk of C = 64 tokens
// (local i, decay a_i = exp(g_i), cumulative log decay G_i = g_0 + .. + g_i,
// gamma_i = exp(G_i)), the per-token update
//     S_i = a_i (I - b_i k_i k_i^T) S_{i-1} + b_i k_i v_i^T,   o_i = S_i^T q_i
// unrolls (by induction on i) to S_i = gamma_i S_0 + sum_{j<=i} exp(G_i - G_j) k_j u_j^T
// with the rows u_j^T of U solving the unit lower-triangular system
//     (I + A) U = R,   A_ij = b_i exp(G_i - G_j) (k_i . k_j) (j < i),
//     R_i = b_i (v_i - gamma_i S_0^T k_i),
// so that
//     o_i = gamma_i S_0^T q_i + sum_{j<=i} exp(G_i - G_j) (q_i . k_j) u_j,
//     S_C = gamma_{C-1} S_0 + sum_j exp(G_{C-1} - G_j) k_j u_j^T.
// scan_chunk_prep_kernel, parallel over (value head, chunk): the Gram products
// K K^T and Q K^T, T = (I + A)^{-1} (forward substitution, row by row) and
// Wq_ij = exp(G_i - G_j) (q_i . k_j) (j <= i); scan_chunk_state_kernel, one block
// per (value head, 16 value columns), walks the chunks in order with the state
// slice in LDS and the products on v_mfma_f32_16x16x4_f32 (fp32 operands, fp32
// accumulation).  Same mathematics as the per-token recurrence
// (custom_model.cpp:1074-1096), a different fp32 summation order.
constexpr int kChunk = kChunkTokens;  // tokens per chunk
constexpr int kChLd = 132;   // floats per 128-dim row in LDS (16-byte aligned rows)
constexpr int kChLdT = 68;   // floats per 64-wide row in LDS
constexpr int kChRec = kChunkRecord;  // floats per (value head, chunk) record

static size_t scan_chunk_prep_lds() {
    return sizeof(float) * (2 * static_cast<size_t>(kChunk) * kChLd + 2 * kChunk * kChLdT + 4 * 16 * 17 + 3 * kChunk);
}
static size_t scan_chunk_state_lds() {
    return sizeof(float) * (2 * static_cast<size_t>(kChunk) * kChLd + 2 * kChunk * kChLdT + 2 * 16 * kChLdT +
                            16 * kChLd + kChunk * 16 + 3 * kChunk);
}

// q and k rows of key head kh for the chunk's tokens [t0, t0 + n) -> LDS rows of
// kChLd floats (rows past n are 0)
__device__ __forceinline__ void stage_qk_rows(const LinearScanLaunch& p, int conv_dim, int kh, int t0, int n,
                                              float* Ks, float* Qs) {
    const __amdgpu_buffer_rsrc_t r = buf_rsrc(p.ws + static_cast<size_t>(t0) * conv_dim,
                                              static_cast<uint32_t>(max(0, n)) * conv_dim * 4u);
    const uint32_t kc = static_cast<uint32_t>(p.lk_n * 128 + kh * 128), qc = static_cast<uint32_t>(kh * 128);
    u32x4 kv[8], qv[8];  // all loads in flight before the first store
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int e = static_cast<int>(threadIdx.x) + 256 * u, row = e >> 5, d4 = e & 31;
        const uint32_t base = static_cast<uint32_t>(row) * conv_dim + 4u * d4;
        kv[u] = __builtin_amdgcn_raw_buffer_load_b128(r, (base + kc) * 4u, 0, 0);
        qv[u] = __builtin_amdgcn_raw_buffer_load_b128(r, (base + qc) * 4u, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int e = static_cast<int>(threadIdx.x) + 256 * u, row = e >> 5, d4 = e & 31;
        *reinterpret_cast<u32x4*>(Ks + row * kChLd + 4 * d4) = kv[u];
        *reinterpret_cast<u32x4*>(Qs + row * kChLd + 4 * d4) = qv[u];
    }
}

__global__ void __launch_bounds__(256) scan_chunk_prep_kernel(LinearScanLaunch p) {
    extern __shared__ float4 scan_lds[];
    float* Ks = reinterpret_cast<float*>(scan_lds);  // [64][kChLd]
    float* Qs = Ks + kChunk * kChLd;                 // [64][kChLd]
    float* Am = Qs + kChunk * kChLd;                 // [64][kChLdT] A (strictly lower)
    float* Tm = Am + kChunk * kChLdT;                // [64][kChLdT] T = (I + A)^{-1}, by 16 x 16 blocks
    float* Mw = Tm + kChunk * kChLdT;                // [4 waves][16][17] block products
    float* Gc = Mw + 4 * 16 * 17;                    // [64] cumulative log decay
    float* Bt = Gc + kChunk;                         // [64] beta
    float* gl = Bt + kChunk;                         // [64] log decay
    const int vh = blockIdx.x, ch = blockIdx.y, t0 = ch * kChunk;
    const int n = __builtin_amdgcn_readfirstlane(min(kChunk, p.tokens - t0));  // scalar: buffer descriptors use it
    const int factor = max(1, p.lv_n / max(1, p.lk_n));
    const int kh = __builtin_amdgcn_readfirstlane(min(p.lk_n - 1, vh / factor));
    const int conv_dim = 2 * p.lk_n * 128 + p.lv_n * p.lv_hd;
    const int tid = threadIdx.x;
    stage_qk_rows(p, conv_dim, kh, t0, n, Ks, Qs);
    if (tid < kChunk) {  // tokens past n: beta 0, log decay 0 (the state passes unchanged)
        const float* aux = p.ws + static_cast<size_t>(p.tokens) * conv_dim;
        const size_t ai = (static_cast<size_t>(t0 + tid) * p.lv_n + vh) * 2;
        Bt[tid] = tid < n ? aux[ai] : 0.0f;
        gl[tid] = tid < n ? aux[ai + 1] : 0.0f;
    }
    __syncthreads();
    if (tid < kChunk) {
        float acc = 0.0f;
        for (int l = 0; l <= tid; ++l) acc += gl[l];
        Gc[tid] = acc;
    }
    // K K^T and Q K^T on v_mfma_f32_16x16x4_f32: wave w takes rows 16 w .. 16 w + 15
    // against the four 16-key column tiles; lane (li, lq) feeds dims 32 lq + s at
    // step s (the same permutation of the contraction for both operands)
    const int lane = tid & (kWave - 1), w = tid / kWave, li = lane & 15, lq = lane >> 4;
    float ka[32], qa[32];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const float4 kv = *reinterpret_cast<const float4*>(Ks + (16 * w + li) * kChLd + 32 * lq + 4 * u);
        const float4 qv = *reinterpret_cast<const float4*>(Qs + (16 * w + li) * kChLd + 32 * lq + 4 * u);
        ka[4 * u] = kv.x; ka[4 * u + 1] = kv.y; ka[4 * u + 2] = kv.z; ka[4 * u + 3] = kv.w;
        qa[4 * u] = qv.x; qa[4 * u + 1] = qv.y; qa[4 * u + 2] = qv.z; qa[4 * u + 3] = qv.w;
    }
    floatx4 kk[4], qk[4];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) kk[ct] = qk[ct] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    // eight independent accumulation chains, four dims of every column tile per round
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        float kb[4][4];
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
            const float4 v = *reinterpret_cast<const float4*>(Ks + (16 * ct + li) * kChLd + 32 * lq + 4 * u);
            kb[ct][0] = v.x; kb[ct][1] = v.y; kb[ct][2] = v.z; kb[ct][3] = v.w;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) {
                kk[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[4 * u + e], kb[ct][e], kk[ct], 0, 0, 0);
                qk[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[4 * u + e], kb[ct][e], qk[ct], 0, 0, 0);
            }
    }
    __syncthreads();  // Gc is complete
    float* rec = p.ws + static_cast<size_t>(p.tokens) * (conv_dim + 2 * p.lv_n) +
                 (static_cast<size_t>(ch) * p.lv_n + vh) * kChRec;
    float* Wq = rec + kChunk * kChunk;
    // lane holds rows 16 w + 4 lq + v, column 16 ct + li of each product
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int i = 16 * w + 4 * lq + v, j = 16 * ct + li;
            const float dec = j <= i ? expf(Gc[i] - Gc[j]) : 0.0f;
            Am[i * kChLdT + j] = j < i ? Bt[i] * dec * kk[ct][v] : 0.0f;
            Wq[i * kChunk + j] = dec * qk[ct][v];
        }
    __syncthreads();
    // T = (I + A)^{-1} by 16 x 16 blocks (A is strictly lower, so T is unit lower
    // triangular).  Diagonal blocks D_k = (I + A_kk)^{-1}, wave k: lane column c
    // keeps column c of D_k in registers, row r = e_r - sum_{j<r} A_rj D_j.
    const int c16 = lane & 15;
    {
        float dc[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < r; ++j) acc += Am[(16 * w + r) * kChLdT + 16 * w + j] * dc[j];
            dc[r] = (c16 == r ? 1.0f : 0.0f) - acc;
        }
        if (lane < 16)
#pragma unroll
            for (int r = 0; r < 16; ++r) Tm[(16 * w + r) * kChLdT + 16 * w + c16] = dc[r];
    }
    __syncthreads();
    // off-diagonal blocks by distance: T_ij = -D_i sum_{k=j}^{i-1} A_ik T_kj (wave j
    // takes block (j + dist, j)); lane: row lane / 4, columns 4 (lane % 4) .. + 3
    const int br = lane >> 2, bc = 4 * (lane & 3);
    for (int dist = 1; dist < 4; ++dist) {  // block-uniform
        const int bi = w + dist, bj = w;
        const bool task = bi < 4;
        float m4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (task)
            for (int k = bj; k < bi; ++k)
#pragma unroll
                for (int mm = 0; mm < 16; ++mm) {
                    const float a = Am[(16 * bi + br) * kChLdT + 16 * k + mm];
#pragma unroll
                    for (int e = 0; e < 4; ++e) m4[e] += a * Tm[(16 * k + mm) * kChLdT + 16 * bj + bc + e];
                }
        float* mw = Mw + w * 16 * 17;
        if (task)
#pragma unroll
            for (int e = 0; e < 4; ++e) mw[br * 17 + bc + e] = m4[e];
        __syncthreads();
        if (task) {
            float t4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int mm = 0; mm < 16; ++mm) {
                const float d = Tm[(16 * bi + br) * kChLdT + 16 * bi + mm];
#pragma unroll
                for (int e = 0; e < 4; ++e) t4[e] += d * mw[mm * 17 + bc + e];
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) Tm[(16 * bi + br) * kChLdT + 16 * bj + bc + e] = -t4[e];
        }
        __syncthreads();
    }
    for (int e = tid; e < kChunk * kChunk; e += 256) {
        const int i = e >> 6, j = e & 63;
        rec[e] = (j >> 4) <= (i >> 4) ? Tm[i * kChLdT + j] : 0.0f;  // blocks above the diagonal are 0
    }
    if (tid < kChunk) {
        rec[2 * kChunk * kChunk + tid] = expf(Gc[tid]);                          // gamma_i
        rec[2 * kChunk * kChunk + kChunk + tid] = expf(Gc[kChunk - 1] - Gc[tid]);  // gamma_last / gamma_j
    }
}

// a chunk's inputs in registers: q / k rows, T, Wq, the value slice, beta and
// the decay factors (loaded for chunk c + 1 while chunk c is computed)
struct ChunkRegs {
    u32x4 k[8], q[8], t[4], wq[4];
    float v[4], bet, gam, del;
};

__global__ void __launch_bounds__(256) scan_chunk_state_kernel(LinearScanLaunch p) {
    extern __shared__ float4 scan_lds[];
    float* Kc = reinterpret_cast<float*>(scan_lds);  // [64][kChLd]
    float* Qc = Kc + kChunk * kChLd;                 // [64][kChLd]
    float* Tc = Qc + kChunk * kChLd;                 // [64][kChLdT]
    float* Wc = Tc + kChunk * kChLdT;                // [64][kChLdT]
    // R, U and the state slice are kept transposed (column-major in the value
    // column): the MFMA operand a lane needs is then a contiguous run
    float* Rt = Wc + kChunk * kChLdT;                // [16][kChLdT] R^T
    float* Ut = Rt + 16 * kChLdT;                    // [16][kChLdT] U^T
    float* St = Ut + 16 * kChLdT;                    // [16][kChLd] the state slice, transposed
    float* Vc = St + 16 * kChLd;                     // [64][16]
    float* gam = Vc + kChunk * 16;                   // [64]
    float* del = gam + kChunk;                       // [64]
    float* bet = del + kChunk;                       // [64]
    const int vh = blockIdx.x, j0 = blockIdx.y * 16;
    const int factor = max(1, p.lv_n / max(1, p.lk_n));
    const int kh = __builtin_amdgcn_readfirstlane(min(p.lk_n - 1, vh / factor));
    const int dv = p.lv_hd;
    const int conv_dim = 2 * p.lk_n * 128 + p.lv_n * dv;
    const int chunks = __builtin_amdgcn_readfirstlane((p.tokens + kChunk - 1) / kChunk);
    const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
    const int li = lane & 15, lq = lane >> 4;  // MFMA operand row / column li, k slot lq
    const bool cact = j0 + li < dv;
    const float rdk = 1.0f / sqrtf(128.0f);
    float* S = p.state + static_cast<size_t>(vh) * 128 * dv;
    const float* aux = p.ws + static_cast<size_t>(p.tokens) * conv_dim;
    const float* recs = aux + static_cast<size_t>(p.tokens) * p.lv_n * 2;
    const uint32_t kcol = static_cast<uint32_t>(p.lk_n * 128 + kh * 128), qcol = static_cast<uint32_t>(kh * 128);
    const uint32_t vcol = static_cast<uint32_t>(2 * p.lk_n * 128 + vh * dv + j0);
    // every load is a range-checked buffer load issued back to back: tokens past
    // the prompt and chunks past the last read 0
    // (sizes and bases through readfirstlane: scalar buffer descriptors)
    auto load_chunk = [&](int ch, ChunkRegs& r) {
        const int t0 = __builtin_amdgcn_readfirstlane(min(ch * kChunk, p.tokens));
        const int n = __builtin_amdgcn_readfirstlane(max(0, min(kChunk, p.tokens - t0)));
        const int cr = __builtin_amdgcn_readfirstlane(min(ch, chunks - 1));
        const uint32_t rbytes = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(ch < chunks ? kChRec * 4 : 0));
        const __amdgpu_buffer_rsrc_t rc =
            buf_rsrc(p.ws + static_cast<size_t>(t0) * conv_dim, static_cast<uint32_t>(n) * conv_dim * 4u);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int e = tid + 256 * u, row = e >> 5, d4 = e & 31;
            const uint32_t base = static_cast<uint32_t>(row) * conv_dim + 4u * d4;
            r.k[u] = __builtin_amdgcn_raw_buffer_load_b128(rc, (base + kcol) * 4u, 0, 0);
            r.q[u] = __builtin_amdgcn_raw_buffer_load_b128(rc, (base + qcol) * 4u, 0, 0);
        }
        const __amdgpu_buffer_rsrc_t rr = buf_rsrc(recs + static_cast<size_t>(cr * p.lv_n + vh) * kChRec, rbytes);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t e4 = static_cast<uint32_t>(tid + 256 * u);
            r.t[u] = __builtin_amdgcn_raw_buffer_load_b128(rr, e4 * 16u, 0, 0);
            r.wq[u] = __builtin_amdgcn_raw_buffer_load_b128(rr, kChunk * kChunk * 4u + e4 * 16u, 0, 0);
        }
        const int vi = tid >> 2, vc = 4 * (tid & 3);  // value rows x 4 columns
#pragma unroll
        for (int e = 0; e < 4; ++e)
            r.v[e] = buf_load_f32(rc, j0 + vc + e < dv ? (static_cast<uint32_t>(vi) * conv_dim + vcol + vc + e) * 4u : kBufOOB);
        const __amdgpu_buffer_rsrc_t ra =
            buf_rsrc(aux + static_cast<size_t>(t0) * p.lv_n * 2, static_cast<uint32_t>(n) * p.lv_n * 8u);
        r.bet = buf_load_f32(ra, tid < kChunk ? (static_cast<uint32_t>(tid) * p.lv_n * 2 + vh * 2) * 4u : kBufOOB);
        r.gam = buf_load_f32(rr, tid < kChunk ? (2 * kChunk * kChunk + tid) * 4u : kBufOOB);
        r.del = buf_load_f32(rr, tid < kChunk ? (2 * kChunk * kChunk + kChunk + tid) * 4u : kBufOOB);
    };
    auto store_chunk = [&](const ChunkRegs& r) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int e = tid + 256 * u, row = e >> 5, d4 = e & 31;
            *reinterpret_cast<u32x4*>(Kc + row * kChLd + 4 * d4) = r.k[u];
            *reinterpret_cast<u32x4*>(Qc + row * kChLd + 4 * d4) = r.q[u];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e4 = tid + 256 * u, i = e4 >> 4, j4 = e4 & 15;
            *reinterpret_cast<u32x4*>(Tc + i * kChLdT + 4 * j4) = r.t[u];
            *reinterpret_cast<u32x4*>(Wc + i * kChLdT + 4 * j4) = r.wq[u];
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) Vc[(tid >> 2) * 16 + 4 * (tid & 3) + e] = r.v[e];
        if (tid < kChunk) {
            bet[tid] = r.bet;
            gam[tid] = r.gam;
            del[tid] = r.del;
        }
    };
    for (int e = tid; e < 128 * 16; e += 256) {
        const int d = e >> 4, cc = e & 15;
        St[cc * kChLd + d] = j0 + cc < dv ? S[static_cast<size_t>(d) * dv + j0 + cc] : 0.0f;
    }
    // a float4 of LDS into four registers
    auto ld4 = [](const float* q, float* d) {
        const float4 v = *reinterpret_cast<const float4*>(q);
        d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
    };
    ChunkRegs nx;
    load_chunk(0, nx);
    const floatx4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int ch = 0; ch < chunks; ++ch) {  // block-uniform
        const int t0 = ch * kChunk, n = min(kChunk, p.tokens - t0);
        __syncthreads();  // the previous chunk's LDS data have been read
        store_chunk(nx);
        __syncthreads();
        load_chunk(ch + 1, nx);  // in flight during this chunk's products
        // The contraction index of every product below is a permutation shared by
        // both operands: lane (li, lq) feeds dims 32 lq + s (K S, Q S) or tokens
        // 16 lq + s (T R, Wq U, K^T U) at step s, so its operands are contiguous.
        // X = K S_0, Y = Q S_0 for the wave's 16 tokens
        floatx4 X = zero4, Y = zero4;
        {
            float ka[32], qa[32], sp[32];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                ld4(Kc + (16 * w + li) * kChLd + 32 * lq + 4 * u, ka + 4 * u);
                ld4(Qc + (16 * w + li) * kChLd + 32 * lq + 4 * u, qa + 4 * u);
                ld4(St + li * kChLd + 32 * lq + 4 * u, sp + 4 * u);
            }
            floatx4 X1 = zero4, Y1 = zero4;  // two chains each (even / odd steps)
#pragma unroll
            for (int st = 0; st < 32; st += 2) {
                X = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[st], sp[st], X, 0, 0, 0);
                Y = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[st], sp[st], Y, 0, 0, 0);
                X1 = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[st + 1], sp[st + 1], X1, 0, 0, 0);
                Y1 = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[st + 1], sp[st + 1], Y1, 0, 0, 0);
            }
            X += X1;
            Y += Y1;
        }
        // R_i = b_i (v_i - gamma_i X_i) (rows 16 w + 4 lq + v, column li), stored transposed
        {
            float r4[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int i = 16 * w + 4 * lq + v;
                r4[v] = bet[i] * (Vc[i * 16 + li] - gam[i] * X[v]);
            }
            *reinterpret_cast<float4*>(Rt + li * kChLdT + 16 * w + 4 * lq) = make_float4(r4[0], r4[1], r4[2], r4[3]);
        }
        __syncthreads();
        // U = T R for the wave's 16 tokens
        floatx4 U = zero4;
        {
            float ta[16], rb[16];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                ld4(Tc + (16 * w + li) * kChLdT + 16 * lq + 4 * u, ta + 4 * u);
                ld4(Rt + li * kChLdT + 16 * lq + 4 * u, rb + 4 * u);
            }
            floatx4 U1 = zero4;
#pragma unroll
            for (int st = 0; st < 16; st += 2) {
                U = __builtin_amdgcn_mfma_f32_16x16x4f32(ta[st], rb[st], U, 0, 0, 0);
                U1 = __builtin_amdgcn_mfma_f32_16x16x4f32(ta[st + 1], rb[st + 1], U1, 0, 0, 0);
            }
            U += U1;
        }
        *reinterpret_cast<float4*>(Ut + li * kChLdT + 16 * w + 4 * lq) = make_float4(U[0], U[1], U[2], U[3]);
        __syncthreads();
        // O = diag(gamma) Y + Wq U; the state update's U operand, scaled by del
        floatx4 O = zero4;
        float ub[16];
        {
            float wa[16], dl[16];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                ld4(Wc + (16 * w + li) * kChLdT + 16 * lq + 4 * u, wa + 4 * u);
                ld4(Ut + li * kChLdT + 16 * lq + 4 * u, ub + 4 * u);
                ld4(del + 16 * lq + 4 * u, dl + 4 * u);
            }
            floatx4 O1 = zero4;
#pragma unroll
            for (int st = 0; st < 16; st += 2) {
                O = __builtin_amdgcn_mfma_f32_16x16x4f32(wa[st], ub[st], O, 0, 0, 0);
                O1 = __builtin_amdgcn_mfma_f32_16x16x4f32(wa[st + 1], ub[st + 1], O1, 0, 0, 0);
            }
            O += O1;
#pragma unroll
            for (int st = 0; st < 16; ++st) ub[st] *= dl[st];
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int i = 16 * w + 4 * lq + v;
            if (i < n && cact)
                p.out[static_cast<size_t>(t0 + i) * p.out_stride + static_cast<size_t>(vh) * dv + j0 + li] =
                    (gam[i] * Y[v] + O[v]) * rdk;
        }
        // S_C = gamma_last S_0 + K^T diag(del) U: the wave's state rows 32 w .. 32 w + 31
        floatx4 Sn[2];
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
            const int rt = 2 * w + rr;
            float s4[4], kt[16];
            ld4(St + li * kChLd + 16 * rt + 4 * lq, s4);
#pragma unroll
            for (int v = 0; v < 4; ++v) Sn[rr][v] = gam[kChunk - 1] * s4[v];
#pragma unroll
            for (int st = 0; st < 16; ++st) kt[st] = Kc[(16 * lq + st) * kChLd + 16 * rt + li];
#pragma unroll
            for (int st = 0; st < 16; ++st) Sn[rr] = __builtin_amdgcn_mfma_f32_16x16x4f32(kt[st], ub[st], Sn[rr], 0, 0, 0);
        }
        __syncthreads();  // every wave has read the old state
#pragma unroll
        for (int rr = 0; rr < 2; ++rr)
            *reinterpret_cast<float4*>(St + li * kChLd + 16 * (2 * w + rr) + 4 * lq) =
                make_float4(Sn[rr][0], Sn[rr][1], Sn[rr][2], Sn[rr][3]);
    }
    __syncthreads();
    for (int e = tid; e < 128 * 16; e += 256) {
        const int d = e >> 4, cc = e & 15;
        if (j0 + cc < dv) S[static_cast<size_t>(d) * dv + j0 + cc] = St[cc * kChLd + d];
    }
}

bool linear_scan_supported(int lk_n, int lk_hd, int lv_n, int lv_hd, int ksize) {
    return lk_n > 0 && lv_n > 0 && lv_n % lk_n == 0 && lk_hd > 0 && lk_hd <= 256 && lv_hd > 0 && ksize >= 1 &&
           ksize - 1 <= kScanMaxHist && lk_hd <= kScanIGroups * kScanMaxK;
}

hipError_t launch_linear_scan(const LinearScanLaunch& p, hipStream_t s) {
    if (p.ws && p.lk_hd == 128 && p.lv_hd <= 256) {
        if (p.lv_hd == 128 && p.ksize == 4) {
            hipLaunchKernelGGL(linear_conv_prefill_tg_kernel<4>,
                               dim3(2 * p.lk_n + p.lv_n, (p.tokens + kConvTokens - 1) / kConvTokens), dim3(128), 0, s, p);
        } else {
            const int width = max(p.lk_hd, p.lv_hd);
            hipLaunchKernelGGL(linear_conv_prefill_kernel, dim3(p.tokens, 2 * p.lk_n + p.lv_n),
                               dim3((width + kWave - 1) / kWave * kWave), 0, s, p);
        }
        if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
        static bool attr_set = false;
        if (!attr_set) {
            if (hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&scan_chunk_prep_kernel),
                                                   hipFuncAttributeMaxDynamicSharedMemorySize,
                                                   static_cast<int>(scan_chunk_prep_lds()));
                e != hipSuccess)
                return e;
            if (hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&scan_chunk_state_kernel),
                                                   hipFuncAttributeMaxDynamicSharedMemorySize,
                                                   static_cast<int>(scan_chunk_state_lds()));
                e != hipSuccess)
                return e;
            attr_set = true;
        }
        const int chunks = (p.tokens + kChunk - 1) / kChunk;
        hipLaunchKernelGGL(scan_chunk_prep_kernel, dim3(p.lv_n, chunks), dim3(256), scan_chunk_prep_lds(), s, p);
        if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
        hipLaunchKernelGGL(scan_chunk_state_kernel, dim3(p.lv_n, (p.lv_hd + 15) / 16), dim3(256), scan_chunk_state_lds(),
                           s, p);
        return hipGetLastError();
    }
    const dim3 grid(p.lv_n, (p.lv_hd + kScanCols - 1) / kScanCols);
    if (p.lk_hd == 128 && p.ksize == 4) {
        // four value columns per wave (two per wave, i.e. twice the blocks, measured
        // slower: every wave convolves the whole q/k head)
        const dim3 grid4(p.lv_n, (p.lv_hd + 15) / 16);
        hipLaunchKernelGGL((linear_scan_wave_kernel<128, 4, 4>), grid4, dim3(256), 0, s, p);
    }
    else
        hipLaunchKernelGGL(linear_scan_kernel, grid, dim3(256), 0, s, p);
    return hipGetLastError();
}

}  // namespace xqhip
