// gemv_tiled.hpp - the TILED64 W4A16 GEMV kernel template and its launchers,
// shared by gemv_w4a16.hip (fp16 group metadata, the layout of matrices whose
// scales and zeros fp16 holds exactly) and gemv_w4a16_m32.hip (fp32 group
// metadata), so the two sets of instantiations compile in parallel.  The
// design of the kernel is described at the top of gemv_w4a16.hip.
#pragma once

#include "xqhip_common.hpp"
#include "xqhip_kernels.hpp"

namespace xqhip {

enum { EPI_STORE = 0, EPI_ADD = 1, EPI_SILU = 2, EPI_ARGMAX = 3 };

// ---------------------------------------------------------------------------
// Activation staging into LDS, done by every GEMV block while its first
// weight batches are in flight.  Record of group g (kStageRecord uint4 = 52
// words): words [8 d + j] hold digit d of columns 8j..8j+7 (nibble i = column
// 8j+i, matching the nibble order of a weight word), then e and G (as floats).
// ---------------------------------------------------------------------------
constexpr int kDigits = 6;
constexpr int kXMax = 1 << (4 * kDigits - 3);  // 2^21: |X| <= kXMax keeps |D| < 2^30
constexpr uint32_t kDigitBias = 0x888888u;     // 8 in every hex digit of the 6
constexpr float kRoundMagic = 12582912.0f;     // 1.5 * 2^23: x + it rounds x to an integer in the low bits
constexpr uint32_t kRoundMagicBits = 0x4B400000u;
constexpr int kStageRecord = (8 * kDigits + 2 + 3) / 4;
constexpr int kMaxStageCols = 16384;

// Nibble transpose: W[d] nibble i = hex digit d of U[i] (i < 8, d < 6).
// Bytes are gathered with v_perm_b32 (A_k: byte k of U0, U2, U4, U6; B_k:
// byte k of U1, U3, U5, U7), then each byte's two digits are split with one
// bit-field insert each, so nibble 2j / 2j+1 of a word come from U_2j / U_2j+1.
__device__ __forceinline__ void digit_words(const uint32_t (&U)[8], uint32_t (&W)[kDigits]) {
    static_assert(kDigits == 6, "three bytes of digits");
    const uint32_t p02 = __builtin_amdgcn_perm(U[2], U[0], 0x05010400u);  // U0.b0 U2.b0 U0.b1 U2.b1
    const uint32_t q02 = __builtin_amdgcn_perm(U[2], U[0], 0x07030602u);  // U0.b2 U2.b2 U0.b3 U2.b3
    const uint32_t p46 = __builtin_amdgcn_perm(U[6], U[4], 0x05010400u);
    const uint32_t q46 = __builtin_amdgcn_perm(U[6], U[4], 0x07030602u);
    const uint32_t p13 = __builtin_amdgcn_perm(U[3], U[1], 0x05010400u);
    const uint32_t q13 = __builtin_amdgcn_perm(U[3], U[1], 0x07030602u);
    const uint32_t p57 = __builtin_amdgcn_perm(U[7], U[5], 0x05010400u);
    const uint32_t q57 = __builtin_amdgcn_perm(U[7], U[5], 0x07030602u);
    const uint32_t A[3] = {__builtin_amdgcn_perm(p46, p02, 0x05040100u), __builtin_amdgcn_perm(p46, p02, 0x07060302u),
                           __builtin_amdgcn_perm(q46, q02, 0x05040100u)};
    const uint32_t B[3] = {__builtin_amdgcn_perm(p57, p13, 0x05040100u), __builtin_amdgcn_perm(p57, p13, 0x07060302u),
                           __builtin_amdgcn_perm(q57, q13, 0x05040100u)};
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        W[2 * k] = (A[k] & 0x0F0F0F0Fu) | ((B[k] << 4) & 0xF0F0F0F0u);
        W[2 * k + 1] = ((A[k] >> 4) & 0x0F0F0F0Fu) | (B[k] & 0xF0F0F0F0u);
    }
}

constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw 32-bit buffer, gfx9-family format
constexpr int kLoadNT = 2;                    // non-temporal (streamed once)
constexpr uint32_t kOutOfRange = 0x80000000u; // beyond every range (matrices < 2 GiB)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t vec_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, kRsrcWord3);
}
template <int AUX = 0>
__device__ __forceinline__ u32x4 load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX);
}
__device__ __forceinline__ void as_floats8(const u32x4& a, const u32x4& b, float* v) {
    v[0] = __uint_as_float(a.x); v[1] = __uint_as_float(a.y); v[2] = __uint_as_float(a.z); v[3] = __uint_as_float(a.w);
    v[4] = __uint_as_float(b.x); v[5] = __uint_as_float(b.y); v[6] = __uint_as_float(b.z); v[7] = __uint_as_float(b.w);
}
// 8 activations from two 16-byte loads: fp32 (a, b) or fp16 (a only), chosen
// by a select rather than a branch
__device__ __forceinline__ void decode_act8(const u32x4& a, const u32x4& b, int x_f16, float* v) {
    const uint32_t h[4] = {a.x, a.y, a.z, a.w};
    float f[8];
    as_floats8(a, b, f);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = x_f16 ? ((i & 1) ? half_hi(h[i >> 1]) : half_lo(h[i >> 1])) : f[i];
}

// The block stages the whole vector: thread t (tid, 0 .. THREADS - 1) owns the
// (group, word) items t, t + THREADS, ... (8 consecutive columns each).  Every wave first issues
// the 16-byte loads of x and of the prologue vectors, the block then passes a
// barrier that waits for none of them, and only then calls `prefetch`, which
// issues the block's first weight loads; the activations thus return first and
// the staging arithmetic below overlaps the weight stream.  The norm factors
// come from the same registers: for PRO_RMS each wave's sum of squares (the
// factor itself is applied to the group scales after the barrier, see
// rms_factor), for PRO_GATED the per-head factors by a lane reduction over the
// head's consecutive items.  ITEMS * THREADS * 8 must cover `cols`; the caller
// synchronises the block before reading xs.  Prologue vectors are preloaded
// only for <= 2 items per thread (the 4096-column launches): wider blocks load
// them after the prefetch, to keep the register budget of the main loop.
// XAUX: cache policy of the loads of x and of the gate vector (kAuxAgent when
// other blocks of the same launch wrote them).
template <int THREADS, int ITEMS, int XAUX = 0, typename Prefetch>
__device__ __forceinline__ void stage_x_lds(const void* x, int x_f16, const Prologue& pro, int cols,
                                            uint4* __restrict__ xs, float* red, int tid, Prefetch&& prefetch) {
    __builtin_assume(tid >= 0 && tid < THREADS);
    constexpr bool kPre = ITEMS <= 2;
    constexpr int kW = kPre ? ITEMS : 1;
    const int G = cols >> 6;
    const int n_items = G * 8;
    // All activation and prologue loads are unconditional range-checked buffer
    // loads (an unused vector has range 0 and reads as zeros without a memory
    // access): straight-line code, so no wait is forced before the barrier.
    const bool gated = pro.mode == PRO_GATED || pro.mode == PRO_GATED_ACT;
    const __amdgpu_buffer_rsrc_t xr = vec_rsrc(x, static_cast<uint32_t>(cols) * (x_f16 ? 2u : 4u));
    const __amdgpu_buffer_rsrc_t wr =
        vec_rsrc(pro.w, pro.mode == PRO_RMS ? cols * 4u : (gated ? static_cast<uint32_t>(pro.head_dim) * 4u : 0u));
    const __amdgpu_buffer_rsrc_t zr = vec_rsrc(pro.z, gated ? cols * 4u : 0u);
    const int hmask = gated ? pro.head_dim - 1 : -1;  // head_dim is a power of two for PRO_GATED
    u32x4 xa[ITEMS], xb[ITEMS], wa[kW], wb[kW], za[kW], zb[kW];
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
        const uint32_t item = static_cast<uint32_t>(min(tid + k * THREADS, n_items - 1));
        xa[k] = load16<XAUX>(xr, x_f16 ? item * 16u : item * 32u);
        xb[k] = load16<XAUX>(xr, x_f16 ? kOutOfRange : item * 32u + 16u);
        if constexpr (kPre) {
            const uint32_t woff = static_cast<uint32_t>(static_cast<int>(item * 8u) & hmask) * 4u;
            wa[k] = load16(wr, woff);
            wb[k] = load16(wr, woff + 16u);
            za[k] = load16<XAUX>(zr, item * 32u);
            zb[k] = load16<XAUX>(zr, item * 32u + 16u);
        }
    }
    // Every wave's activation loads are issued before any wave's weight loads:
    // a CU's vector-memory requests are served in issue order, so without this
    // barrier (which waits for no load) the activations of late waves queue
    // behind the weight stream of early ones and the staging, which needs all
    // of them, finishes only after most of the prefetched weights.
    // (an asm barrier with a memory clobber: the compiler moves no load across it)
    asm volatile("s_barrier" ::: "memory");
    prefetch();
    float v[ITEMS][8], wv[kW][8], zv[kW][8];
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
        decode_act8(xa[k], xb[k], x_f16, v[k]);
        if constexpr (kPre) {
            as_floats8(wa[k], wb[k], wv[k]);
            as_floats8(za[k], zb[k], zv[k]);
        }
    }
    if (pro.mode == PRO_RMS) {
        // The RMS factor is one scalar for the whole vector and the digits are
        // relative to each group's maximum, so the groups are staged from x * w
        // and the factor multiplies the group scales after the caller's barrier
        // (rms_factor): here each wave only leaves its sum of squares in red.
        // explicit fused multiply-adds on selected operands: the rounding of
        // the sum of squares does not depend on how the compiler contracts or
        // if-converts it (the decode chains stage with the same sequence)
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < ITEMS; ++k) {
            const bool in = tid + k * THREADS < n_items;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float a = in ? v[k][i] : 0.0f;
                ss = fmaf(a, a, ss);
            }
        }
        ss = wave_sum(ss);
        if ((tid & (kWave - 1)) == 0) red[tid / kWave] = ss;
#pragma unroll
        for (int k = 0; k < ITEMS; ++k) {
            float wl[8];
            if constexpr (kPre) {
#pragma unroll
                for (int i = 0; i < 8; ++i) wl[i] = wv[k][i];
            } else {
                const uint32_t item = static_cast<uint32_t>(min(tid + k * THREADS, n_items - 1));
                as_floats8(load16(wr, item * 32u), load16(wr, item * 32u + 16u), wl);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) v[k][i] = v[k][i] * wl[i];
        }
    } else if (gated) {
        // head_dim % 8 == 0 and head_dim / 8 a power of two <= 64: the items of a
        // head are head_dim/8 consecutive lanes of one wave
        const int per_head = pro.head_dim >> 3;
#pragma unroll
        for (int k = 0; k < ITEMS; ++k) {
            float hs = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) hs = fmaf(v[k][i], v[k][i], hs);
            if (per_head >= 2) hs += dpp_f32<kDppXor1>(hs);
            if (per_head >= 4) hs += dpp_f32<kDppXor2>(hs);
            if (per_head >= 8) hs += dpp_f32<kDppHalfMirror>(hs);
            if (per_head >= 16) hs += dpp_f32<kDppMirror>(hs);
            if (per_head >= 32) hs = xor_pair_sum<16>(hs);
            if (per_head >= 64) hs = xor_pair_sum<32>(hs);
            const float inv = 1.0f / sqrtf(hs / static_cast<float>(pro.head_dim) + pro.eps);
            float wl[8], zl[8];
            if constexpr (kPre) {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    wl[i] = wv[k][i];
                    zl[i] = zv[k][i];
                }
            } else {
                const uint32_t item = static_cast<uint32_t>(min(tid + k * THREADS, n_items - 1));
                const uint32_t woff = static_cast<uint32_t>(static_cast<int>(item * 8u) & hmask) * 4u;
                as_floats8(load16(wr, woff), load16(wr, woff + 16u), wl);
                as_floats8(load16<XAUX>(zr, item * 32u), load16<XAUX>(zr, item * 32u + 16u), zl);
            }
            if (pro.mode == PRO_GATED_ACT) {  // the gate holds silu(gate) already (uniform branch)
#pragma unroll
                for (int i = 0; i < 8; ++i) v[k][i] = v[k][i] * inv * wl[i] * zl[i];
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) v[k][i] = v[k][i] * inv * wl[i] * silu_dev(zl[i]);
            }
        }
    }
    uint32_t* xw = reinterpret_cast<uint32_t*>(xs);
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
        const int item = tid + k * THREADS;
        const int g = item >> 3, w = item & 7;
        // group maximum over the 8 items of the group (8 consecutive lanes)
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(v[k][i]));
        mx = lanes_max<8>(mx);
        // X = rint(x * 2^21 / mx) is the low mantissa of fma(x, inv, 1.5 * 2^23) (|x inv| <= 2^21 + 1/4,
        // inv from v_rcp_f32 within an ulp), so U = X + kDigitBias is that float's bits minus a constant
        const float inv = mx > 0.0f ? static_cast<float>(kXMax) * __builtin_amdgcn_rcpf(mx) : 0.0f;
        uint32_t U[8];
        uint32_t us = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            U[i] = __float_as_uint(fmaf(v[k][i], inv, kRoundMagic)) - (kRoundMagicBits - kDigitBias);
            us += U[i];
        }
        const int gs = lanes_sum_i<8>(static_cast<int>(us)) - 64 * static_cast<int>(kDigitBias);
        if (item < n_items) {
            uint32_t W[kDigits];
            digit_words(U, W);
#pragma unroll
            for (int d = 0; d < kDigits; ++d) xw[g * (4 * kStageRecord) + d * 8 + w] = W[d] ^ 0x88888888u;
            if (w == 0) {
                xw[g * (4 * kStageRecord) + 8 * kDigits] = __float_as_uint(mx * (1.0f / static_cast<float>(kXMax)));
                xw[g * (4 * kStageRecord) + 8 * kDigits + 1] = __float_as_uint(static_cast<float>(gs));
            }
        }
    }
}

// PRO_RMS factor 1/sqrt(mean(x^2) + eps) from the per-wave sums of squares
// stage_x_lds left in red (read after the block barrier that follows it)
template <int NW>
__device__ __forceinline__ float rms_factor(const float* red, int cols, float eps) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NW; ++i) ss += red[i];
    return 1.0f / sqrtf(ss / static_cast<float>(cols) + eps);
}

inline bool stage_supported(int cols, const Prologue& pro) {
    if (cols % 64 != 0 || cols > kMaxStageCols) return false;
    if (pro.mode == PRO_GATED || pro.mode == PRO_GATED_ACT) {
        const int per = pro.head_dim / 8;
        return pro.head_dim % 8 == 0 && per >= 1 && per <= 64 && (per & (per - 1)) == 0;
    }
    return true;
}

// Greedy argmax in two kernels: every GEMV block stores its best (value, row)
// key, then argmax_finish_kernel reduces the keys.  The kernel boundary orders
// the two (no grid-wide fence, no completion counter).
__device__ __forceinline__ void store_block_key(uint64_t block_best, uint64_t* partial, int tid, int block) {
    if (tid == 0) partial[block] = block_best;
}

hipError_t launch_argmax_finish(const GemvLaunch& p, int blocks, hipStream_t s);  // gemv_w4a16.hip

// ---------------------------------------------------------------------------
// TILED64 kernel.  NCH = number of 4096-column chunks (the last may be partial);
// a block has RG row groups x NCH waves, wave (rg, c) owns chunk c for the rows
// of row group rg; R = rows per wave iteration.  Two register buffers of
// weights: a buffer is refilled with the batch two trips ahead as soon as it
// is reduced, and the first two batches are requested before the activations
// are staged.
//
// Weights are read through buffer resources: a load past the end of the
// matrix (a row beyond `rows`, a lane beyond the last group of a partial
// chunk) is dropped by the hardware range check and returns zeros, so every
// load is issued unconditionally.  That keeps the number of loads in flight
// the same on every path, which lets each wait cover exactly the buffer it
// consumes (vector loads complete in issue order) instead of draining both.
// ---------------------------------------------------------------------------
// Partial row sums of column-split launches (NCH > 1) are kept in LDS,
// [slot][row group][chunk][R] floats, and combined for kDeferredSlots batches
// at a time (in practice once, after the loop), one barrier per combine
// instead of two per batch.
constexpr int kMaxDeferredPartials = 4096;
template <int RG, int NCH, int R>
constexpr int kDeferredSlots = kMaxDeferredPartials / (RG * NCH * R) > 0 ? kMaxDeferredPartials / (RG * NCH * R) : 1;
__host__ __device__ inline int batches_of(int trips) { return 2 * ((trips + 1) / 2); }

template <int R, int META>
struct WBatch {
    uint4 a[R], b[R];
    MetaWord<META> m[R];
};


struct WSrc {
    __amdgpu_buffer_rsrc_t nib, meta;
};

// Bytes of one TILED64 row: cols * BITS / 8 (cols % 64 == 0).
template <int BITS>
__host__ __device__ constexpr uint32_t tiled_row_bytes(int cols) {
    return static_cast<uint32_t>(cols >> 3) * BITS;
}

template <int BITS, int META>
__device__ __forceinline__ WSrc make_wsrc(const uint8_t* nib, const uint32_t* meta, int rows, int cols) {
    const uint32_t nib_bytes = static_cast<uint32_t>(rows) * tiled_row_bytes<BITS>(cols);
    const uint32_t meta_bytes = meta_total_bytes<META>(static_cast<uint32_t>(rows), static_cast<uint32_t>(cols >> 6));
    WSrc s;
    s.nib = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(nib), 0, nib_bytes, kRsrcWord3);
    s.meta = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(meta), 0, meta_bytes, kRsrcWord3);
    return s;
}

__device__ __forceinline__ uint4 as_uint4(u32x4 v) { return make_uint4(v.x, v.y, v.z, v.w); }

// Row layout per 4096-column chunk c (64 groups, gcnt of them present), at
// c * 512 * BITS bytes into the row:
//   BITS 4: [gcnt x 16 B: bytes 0-15 of each group][gcnt x 16 B: bytes 16-31]
//   BITS 3: [gcnt x 16 B: low-two-bit plane][gcnt x 8 B: high-bit plane]
//   BITS 2: [gcnt x 16 B: two-bit plane]
// so each load instruction of a wave reads one contiguous run.
template <int R, int BITS, int META>
__device__ __forceinline__ void load_batch(WBatch<R, META>& wb, const WSrc& src, int r0, int rows, uint32_t row_bytes,
                                           int G, int c, int lane, int gcnt, bool has_group) {
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int row = r0 + i;
        const bool ok = has_group && row < rows;
        // 24-bit multiplies (rows, row bytes and groups per row are below 2^24):
        // the 64-bit multiply-add the compiler otherwise picks reads an unused
        // high half that can alias a pending load, and the wait for that load
        // would hold back this batch
        const uint32_t base = __umul24(static_cast<uint32_t>(row), row_bytes) + static_cast<uint32_t>(c * 512 * BITS);
        const uint32_t off = base + static_cast<uint32_t>(lane * 16);
        const uint32_t moff = (__umul24(static_cast<uint32_t>(row), static_cast<uint32_t>(G)) + c * 64 + lane) *
                              kMetaGroupBytes<META>;
        wb.a[i] = as_uint4(__builtin_amdgcn_raw_buffer_load_b128(src.nib, ok ? off : kOutOfRange, 0, kLoadNT));
        if constexpr (BITS == 4) {
            wb.b[i] = as_uint4(
                __builtin_amdgcn_raw_buffer_load_b128(src.nib, ok ? off + gcnt * 16 : kOutOfRange, 0, kLoadNT));
        } else if constexpr (BITS == 3) {
            const uint32_t hoff = base + static_cast<uint32_t>(gcnt * 16 + lane * 8);
            const u32x2 h = __builtin_amdgcn_raw_buffer_load_b64(src.nib, ok ? hoff : kOutOfRange, 0, kLoadNT);
            wb.b[i] = make_uint4(h.x, h.y, 0u, 0u);
        }
        uint32_t zoff = 0;
        if constexpr (META == 3)
            zoff = ok ? z4_offset(static_cast<uint32_t>(rows), static_cast<uint32_t>(G), static_cast<uint32_t>(row),
                                  static_cast<uint32_t>(c * 64 + lane))
                      : kOutOfRange;
        wb.m[i] = load_meta<META, kLoadNT>(src.meta, ok ? moff : kOutOfRange, zoff);
    }
}

// The eight signed-nibble words (column 8j + i in nibble i of word j, code q as
// q | 8) of one group from its loaded bytes.
//   BITS 2: plane word m holds columns 16m..16m+15: nibble i bits 0-1 = q(16m + i),
//           bits 2-3 = q(16m + 8 + i)
//   BITS 3: the low two bits as BITS 2; high-bit word k holds, at bit 4i + r,
//           bit 2 of q(8 (4k + r) + i)
template <int BITS>
__device__ __forceinline__ void group_words(const uint4& a, const uint4& b, uint32_t (&wd)[8]) {
    if constexpr (BITS == 4) {
        wd[0] = a.x; wd[1] = a.y; wd[2] = a.z; wd[3] = a.w;
        wd[4] = b.x; wd[5] = b.y; wd[6] = b.z; wd[7] = b.w;
    } else {
        const uint32_t v[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            wd[2 * m] = (v[m] & 0x33333333u) | 0x88888888u;
            wd[2 * m + 1] = ((v[m] >> 2) & 0x33333333u) | 0x88888888u;
        }
        if constexpr (BITS == 3) {
            const uint32_t h[2] = {b.x, b.y};
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t hk = h[j >> 2];
                const int r = j & 3;
                const uint32_t hb = r <= 2 ? (hk << (2 - r)) : (hk >> 1);
                wd[j] |= hb & 0x44444444u;
            }
        }
    }
}

// The kernel body, for the 64 * NCH * RG threads tid = 0 .. of block `block`
// out of `grid`; xs / red / lds_keys are the block's LDS areas.
// EARLY = false (the plain GEMV): the activations are requested first, then
// the first weight batches, then the staging arithmetic runs while the weights
// stream in; pre() and wait() are not called.
// EARLY = true (a GEMV whose input another part of the same launch produces):
// pre() first, then the first two weight batches (with trips <= 2 every weight
// the block reads), then wait(), which returns once the input is complete, and
// only then the activation loads, with cache policy XAUX.
template <int NCH, int RG, int R, int EPI, int BITS, int META, bool EARLY = false, int XAUX = 0,
          typename Pre = void (*)(), typename Wait = void (*)()>
__device__ __forceinline__ void gemv_tiled_run(const uint8_t* __restrict__ nib, const uint32_t* __restrict__ meta,
                                               int rows, int cols, int affine, const void* x, int x_f16,
                                               const Prologue& pro, void* __restrict__ y, int y_f16,
                                               uint64_t* __restrict__ partial, int grid, int tid, int block,
                                               uint4* xs, float* red, uint64_t* lds_keys, Pre&& pre, Wait&& wait) {
    __builtin_assume(tid >= 0 && tid < 64 * NCH * RG);
    __builtin_assume(block >= 0 && block < grid);
    const int G = cols >> 6;
    const int lane = tid & (kWave - 1);
    const int wid = tid / kWave;
    const int c = wid % NCH;
    const int rg = wid / NCH;
    const int g = c * 64 + lane;
    const bool has_group = g < G;
    const int gcnt = min(64, G - c * 64);
    const uint32_t row_bytes = tiled_row_bytes<BITS>(cols);
    const int stride = grid * RG;
    const WSrc src = make_wsrc<BITS, META>(nib, meta, rows, cols);
    // First row of this wave's batch (R rows) in trip t (b: block * RG +
    // t * stride, kept incrementally).  Full trips deal the batches block by
    // block (block b's waves take batches t stride + b RG + rg).  For the
    // one-row-batch, one-chunk launches (the 4096-, 10240- and 12352-row
    // projections, whose rows leave a partial last trip) that trip deals its
    // batches wave by wave across the blocks (batch t stride + rg grid + b), so
    // every CU streams within one row of every other instead of a few blocks
    // taking the whole remainder with all their waves; measured 0.25-0.4 us
    // off those launches.  (The other instantiations keep the plain mapping:
    // the extra select cost gate/up and down 0.2-0.3 us.)  Which wave computes
    // a row does not change its arithmetic.
    constexpr bool kSpreadTail = R == 1 && NCH == 1 && EPI != EPI_ARGMAX;
    const int full_trips = ((rows + R - 1) / R) / stride;
    auto row0 = [&](int t, int b) {
        if constexpr (kSpreadTail) return (t < full_trips ? b + rg : t * stride + rg * grid + block) * R;
        return (b + rg) * R;
    };

    // The residual-add epilogue of a one-chunk launch reads y[row] when it
    // finishes the row: that load is issued with the batch's weights (lane i <
    // R: row r0 + i), so it returns with them instead of costing a memory
    // round trip, and a wait for it, after the batch's dot products.  Only the
    // wave finishing a row writes it, once, so the early read sees the value
    // the launch started with.
    constexpr bool kPrefetchY = EPI == EPI_ADD && NCH == 1;
    const __amdgpu_buffer_rsrc_t y_r = buf_rsrc(y, kPrefetchY ? static_cast<uint32_t>(rows) * 4u : 0u);
    auto load_b = [&](WBatch<R, META>& wb, float& yv, int r0) {
        load_batch<R, BITS, META>(wb, src, r0, rows, row_bytes, G, c, lane, gcnt, has_group);
        if constexpr (kPrefetchY)
            yv = buf_load_f32(y_r, lane < R && r0 + lane < rows ? static_cast<uint32_t>(r0 + lane) * 4u : kBufOOB);
    };

    // activations first, then the first weight batches, then the staging
    // arithmetic while the weights stream in
    WBatch<R, META> buf0, buf1;
    float yv0 = 0.0f, yv1 = 0.0f;
    int base = block * RG;
    if constexpr (EARLY) {
        pre();
        load_b(buf0, yv0, row0(0, base));
        load_b(buf1, yv1, row0(1, base + stride));
        wait();
        stage_x_lds<64 * NCH * RG, (8 + RG - 1) / RG, XAUX>(x, x_f16, pro, cols, xs, red, tid, []() {});
    } else {
        // With R >= 2 only the first batch is issued before the staging: a second
        // one would stall its issue on the CU's in-flight memory requests, and the
        // staging waits behind it.
        stage_x_lds<64 * NCH * RG, (8 + RG - 1) / RG>(x, x_f16, pro, cols, xs, red, tid, [&]() {
            load_b(buf0, yv0, row0(0, base));
            if constexpr (R == 1) load_b(buf1, yv1, row0(1, base + stride));
        });
        if constexpr (R > 1) load_b(buf1, yv1, row0(1, base + stride));
    }
    __syncthreads();
    // this lane's group: kDigits x 8 words of digits, then e and G
    uint32_t xd[kDigits][8];
    float ge = 0.0f, gg = 0.0f;
    {
        const uint4* rec = xs + (has_group ? g : 0) * kStageRecord;
#pragma unroll
        for (int d = 0; d < kDigits; ++d) {
            const uint4 lo4 = rec[2 * d], hi4 = rec[2 * d + 1];
            xd[d][0] = lo4.x; xd[d][1] = lo4.y; xd[d][2] = lo4.z; xd[d][3] = lo4.w;
            xd[d][4] = hi4.x; xd[d][5] = hi4.y; xd[d][6] = hi4.z; xd[d][7] = hi4.w;
        }
        const uint4 kk = rec[2 * kDigits];
        ge = has_group ? __uint_as_float(kk.x) : 0.0f;
        gg = has_group ? __uint_as_float(kk.y) : 0.0f;
    }
    if (pro.mode == PRO_RMS) ge *= rms_factor<NCH * RG>(red, cols, pro.eps);

    uint64_t best = 0;
    const int units = (rows + R * RG - 1) / (R * RG);
    const int trips = (units + grid - 1) / grid;
    float* partial_all = reinterpret_cast<float*>(xs + G * kStageRecord);
    constexpr int kSlots = kDeferredSlots<RG, NCH, R>;

    // epilogue of rows r0 .. r0 + R - 1 (chunk-0 waves; every lane holds the sums)
    auto finish_rows = [&](const float (&acc)[R], int r0, float yv) {
        if constexpr (EPI == EPI_ARGMAX) {
#pragma unroll
            for (int i = 0; i < R; ++i)
                if (r0 + i < rows) best = u64_max(best, argmax_key(acc[i], static_cast<uint32_t>(r0 + i)));
        } else if constexpr (EPI == EPI_SILU) {
            float gv = acc[0], uv = acc[1];
#pragma unroll
            for (int i = 1; i < R / 2; ++i)
                if (lane == i) {
                    gv = acc[2 * i];
                    uv = acc[2 * i + 1];
                }
            const int orow = (r0 >> 1) + lane;
            if (lane < R / 2 && 2 * orow < rows) static_cast<float*>(y)[orow] = silu_dev(gv) * uv;
        } else {
            float v = acc[0];
#pragma unroll
            for (int i = 1; i < R; ++i)
                if (lane == i) v = acc[i];
            const int row = r0 + lane;
            if (lane < R && row < rows) {
                if constexpr (EPI == EPI_ADD) {
                    static_cast<float*>(y)[row] = (kPrefetchY ? yv : static_cast<float*>(y)[row]) + v;
                } else {
                    if (y_f16)
                        static_cast<_Float16*>(y)[row] = static_cast<_Float16>(v);
                    else
                        static_cast<float*>(y)[row] = v;
                }
            }
        }
    };

    // sums the chunk partials of batches b0 .. b0 + n - 1 and finishes their rows
    auto combine = [&](int b0, int n) {
        __syncthreads();
        if (c == 0) {
            if constexpr (EPI == EPI_STORE || EPI == EPI_ADD) {
                // one (batch, row) per lane, so the residual reads of all the
                // rows are in flight together
                for (int k = lane; k < n * R; k += kWave) {
                    const int bi = b0 + k / R, i = k % R;
                    const int row = row0(bi, block * RG + bi * stride) + i;
                    if (row >= rows) continue;
                    float t = 0.0f;
#pragma unroll
                    for (int cc = 0; cc < NCH; ++cc) t += partial_all[(((bi % kSlots) * RG + rg) * NCH + cc) * R + i];
                    if constexpr (EPI == EPI_ADD)
                        static_cast<float*>(y)[row] += t;
                    else if (y_f16)
                        static_cast<_Float16*>(y)[row] = static_cast<_Float16>(t);
                    else
                        static_cast<float*>(y)[row] = t;
                }
            } else {
                for (int bi = b0; bi < b0 + n; ++bi) {
                    const int r0 = row0(bi, block * RG + bi * stride);
                    if (r0 >= rows) continue;
                    float acc[R];
#pragma unroll
                    for (int i = 0; i < R; ++i) {
                        float t = 0.0f;
#pragma unroll
                        for (int cc = 0; cc < NCH; ++cc)
                            t += partial_all[(((bi % kSlots) * RG + rg) * NCH + cc) * R + i];
                        acc[i] = t;
                    }
                    finish_rows(acc, r0, 0.0f);
                }
            }
        }
        __syncthreads();  // the slots are reused by the next batches
    };

    auto process = [&](WBatch<R, META>& cur, float yv, int bbase, int bidx) {
        const int r0 = row0(bidx, bbase);
        float acc[R];
#pragma unroll
        for (int i = 0; i < R; ++i) acc[i] = 0.0f;
        if (r0 < rows) {
#pragma unroll
            for (int i = 0; i < R; ++i) {
                uint32_t wd[8];
                group_words<BITS>(cur.a[i], cur.b[i], wd);
                int A[kDigits];
#pragma unroll
                for (int d = 0; d < kDigits; ++d) A[d] = 0;
#pragma unroll
                for (int j = 0; j < 8; ++j)
#pragma unroll
                    for (int d = 0; d < kDigits; ++d)
                        A[d] = __builtin_amdgcn_sdot8(static_cast<int>(wd[j]), static_cast<int>(xd[d][j]), A[d], false);
                // D = sum_d A_d 16^d, exact in int32 (|D| < 2^30, partial sums smaller)
                int Dg = A[kDigits - 1];
#pragma unroll
                for (int d = kDigits - 2; d >= 0; --d) Dg = (Dg << 4) + A[d];
                // sum_c q_c x_c = e (D + 8 G), sum_c x_c = e G, so
                //   v1: s (sum qx - z sum x) = s e (D + (8 - z) G)   (exact cancellation for z = 8)
                //   v2: s sum qx + z sum x   = e (s D + (8 s + z) G)
                // (the group's term is rounded on its own before the row sum, mul_rn,
                // so every metadata form and the decode chains round alike)
                const float df = static_cast<float>(Dg);
                const float sc = meta_scale(cur.m[i]);
                if constexpr (META == 2) {  // zero 8, format v1: s e D (the v1 form with 8 - z = 0)
                    acc[i] = mul_rn(sc * ge, df);
                } else if constexpr (META == 3) {  // format v1, integer zero (group g = 64 c + lane: nibble lane % 8)
                    const float z = meta_zero_at(cur.m[i], static_cast<uint32_t>(lane & 7) * 4u);
                    acc[i] = mul_rn(sc * ge, fmaf(8.0f - z, gg, df));
                } else {
                    const float z = meta_zero(cur.m[i]);
                    acc[i] = affine ? mul_rn(ge, fmaf(sc, df, fmaf(8.0f, sc, z) * gg))
                                    : mul_rn(sc * ge, fmaf(8.0f - z, gg, df));
                }
                acc[i] = wave_sum(acc[i]);
            }
        }
        if constexpr (NCH > 1) {
            float v = acc[0];
#pragma unroll
            for (int i = 1; i < R; ++i)
                if (lane == i) v = acc[i];
            if (lane < R) partial_all[(((bidx % kSlots) * RG + rg) * NCH + c) * R + lane] = v;
            if ((bidx + 1) % kSlots == 0) combine(bidx + 1 - kSlots, kSlots);  // block-uniform
            return;
        }
        if (r0 >= rows) return;
        finish_rows(acc, r0, yv);
    };

    // two batches per trip so each register buffer has a fixed name; a buffer
    // is refilled with the batch two trips ahead as soon as it is reduced
    // The trip count is the grid-wide maximum (uniform, so the loop has no
    // early exit between the two buffers): batches past the end load nothing
    // and are skipped by process().
    for (int t = 0; t < trips; t += 2) {
        process(buf0, yv0, base, t);
        load_b(buf0, yv0, row0(t + 2, base + 2 * stride));
        process(buf1, yv1, base + stride, t + 1);
        load_b(buf1, yv1, row0(t + 3, base + 3 * stride));
        base += 2 * stride;
    }
    if constexpr (NCH > 1) {
        const int nb = batches_of(trips);
        const int done = (nb / kSlots) * kSlots;
        if (nb > done) combine(done, nb - done);
    }

    if constexpr (EPI == EPI_ARGMAX) {
        if (lane == 0) lds_keys[wid] = (c == 0) ? best : 0;
        __syncthreads();
        uint64_t b = 0;
        if (tid == 0)
            for (int i = 0; i < NCH * RG; ++i) b = u64_max(b, lds_keys[i]);
        __syncthreads();
        store_block_key(b, partial, tid, block);
    }
}

template <int NCH, int RG, int R, int EPI, int BITS, int META>
__global__ void __launch_bounds__(64 * NCH * RG) gemv_w4_tiled(
    // x is not __restrict__: with it the compiler may move the staging loads of
    // x across the asm barrier of stage_x_lds (it would assume no aliasing)
    const uint8_t* __restrict__ nib, const uint32_t* __restrict__ meta, int rows, int cols, int affine,
    const void* x, int x_f16, Prologue pro, void* __restrict__ y, int y_f16,
    uint64_t* __restrict__ partial, int grid) {  // grid == gridDim.x (an argument: no late kernarg fetch)
    extern __shared__ uint4 xs[];  // staged activations, kStageRecord uint4 per group
    __shared__ float red[32];
    __shared__ uint64_t lds_keys[16];
    gemv_tiled_run<NCH, RG, R, EPI, BITS, META>(nib, meta, rows, cols, affine, x, x_f16, pro, y, y_f16, partial, grid,
                                                static_cast<int>(threadIdx.x), static_cast<int>(blockIdx.x), xs, red,
                                                lds_keys, []() {}, []() {});
}

// ---------------------------------------------------------------------------
// host-side launch
// ---------------------------------------------------------------------------

constexpr int kThreads = 256;

// Blocks of `fn` resident on the current device at once (occupancy x CUs),
// cached per kernel and device.
static int resident_blocks(const void* fn, int threads, size_t lds, int* cache) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) return 0;
    if (cache[dev] > 0) return cache[dev];
    int cus = 0, per = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, fn, threads, lds) != hipSuccess) return 0;
    cache[dev] = (per > 0 ? per : 1) * cus;
    return cache[dev];
}

// One block per CU: 12 waves (NCH chunks x 12/NCH row groups), so the
// activation staging is done once per CU rather than once per small block.
template <int NCH>
constexpr int kRowGroups = 12 / NCH;

static int device_cus() {
    static int cache[16] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) return 256;
    if (cache[dev] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 256;
        cache[dev] = cus;
    }
    return cache[dev];
}

template <int NCH, int R, int EPI, int BITS, int META>
static hipError_t launch_tiled_t(const GemvLaunch& p, hipStream_t s) {
    constexpr int RG = kRowGroups<NCH>;
    const int G = p.cols >> 6;
    const size_t stage_lds = static_cast<size_t>(G) * kStageRecord * sizeof(uint4);
    // occupancy and the LDS limit are set for the largest partial-sum area
    const size_t lds_max = stage_lds + (NCH > 1 ? sizeof(float) * kMaxDeferredPartials : 0);
    const auto fn = reinterpret_cast<const void*>(&gemv_w4_tiled<NCH, RG, R, EPI, BITS, META>);
    if (lds_max > 64 * 1024) {  // beyond the default dynamic-LDS limit (gfx950 has 160 KiB per CU)
        const hipError_t e =
            hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds_max));
        if (e != hipSuccess) return e;
    }
    // No more blocks than are resident at once (each stages x once); trips are
    // grid-uniform, blocks whose later rows fall past the end skip them.
    static int resident_cache[16] = {};
    int cap = p.max_blocks > 0 ? p.max_blocks : resident_blocks(fn, 64 * NCH * RG, lds_max, resident_cache);
    if (cap < 1) cap = device_cus();
    if (EPI == EPI_ARGMAX && cap > kArgmaxMaxBlocks) cap = kArgmaxMaxBlocks;
    const int units = (p.rows + R * RG - 1) / (R * RG);
    const int blocks = units < cap ? units : cap;
    const int trips = (units + blocks - 1) / blocks;
    size_t lds = stage_lds;
    if (NCH > 1)
    {
        constexpr int kSlots = kDeferredSlots<RG, NCH, R>;
        const int slots = batches_of(trips) < kSlots ? batches_of(trips) : kSlots;
        lds += sizeof(float) * static_cast<size_t>(slots) * RG * NCH * R;
    }
    hipLaunchKernelGGL((gemv_w4_tiled<NCH, RG, R, EPI, BITS, META>), dim3(blocks), dim3(64 * NCH * RG), lds, s, p.nib,
                       static_cast<const uint32_t*>(p.meta), p.rows, p.cols, p.affine, p.x, p.x_f16, p.pro, p.y,
                       p.y_f16, p.partial, blocks);
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    return EPI == EPI_ARGMAX ? launch_argmax_finish(p, blocks, s) : hipSuccess;
}

// Rows per wave batch: the R in {1, 2, 4} that minimises the rows one wave
// streams on the critical path, ceil(units_R / blocks) * R (ties: the smaller
// R, i.e. more trips and a deeper load pipeline per wave); SILU pairs need R
// even.
template <int NCH>
static int choose_rows_per_wave(const GemvLaunch& p) {
    constexpr int RG = kRowGroups<NCH>;
    const int cap = p.max_blocks > 0 ? p.max_blocks : device_cus();
    int best_r = 2, best_cost = 1 << 30;
    for (int r : {1, 2, 4}) {
        if ((p.epi == EPI_SILU && r == 1) || (p.epi == EPI_ARGMAX && r == 4)) continue;  // pairs; VGPR budget
        const int units = (p.rows + r * RG - 1) / (r * RG);
        const int cost = ((units + cap - 1) / cap) * r;
        if (cost < best_cost) {
            best_cost = cost;
            best_r = r;
        }
    }
    // 3- and 2-bit rows are shorter: when two rows per wave still give every
    // block work and cost at most 5 % more, they stream faster (measured on the
    // 4096x12288, 24576x4096 and 248320x4096 shapes)
    if (p.bits != 4 && best_r == 1) {
        const int units2 = (p.rows + 2 * RG - 1) / (2 * RG);
        if (units2 >= cap && ((units2 + cap - 1) / cap) * 2 * 20 <= best_cost * 21) best_r = 2;
    }
    return best_r;
}

template <int NCH, int EPI, int BITS, int META>
static hipError_t launch_tiled_epi(const GemvLaunch& p, hipStream_t s) {
    switch (choose_rows_per_wave<NCH>(p)) {
        case 1:
            if constexpr (EPI != EPI_SILU) return launch_tiled_t<NCH, 1, EPI, BITS, META>(p, s);
            return hipErrorInvalidValue;
        case 2: return launch_tiled_t<NCH, 2, EPI, BITS, META>(p, s);
        default:
            if constexpr (EPI != EPI_ARGMAX) return launch_tiled_t<NCH, 4, EPI, BITS, META>(p, s);
            return hipErrorInvalidValue;
    }
}

template <int NCH, int BITS, int META>
static hipError_t launch_tiled_nch(const GemvLaunch& p, hipStream_t s) {
    if (!stage_supported(p.cols, p.pro)) return hipErrorInvalidValue;
    // buffer-resource offsets are 32-bit and kOutOfRange must lie past the end
    if (static_cast<uint64_t>(p.rows) * tiled_row_bytes<BITS>(p.cols) >= kOutOfRange) return hipErrorInvalidValue;
    switch (p.epi) {
        case EPI_STORE: return launch_tiled_epi<NCH, EPI_STORE, BITS, META>(p, s);
        case EPI_ADD: return launch_tiled_epi<NCH, EPI_ADD, BITS, META>(p, s);
        case EPI_SILU: return launch_tiled_epi<NCH, EPI_SILU, BITS, META>(p, s);
        case EPI_ARGMAX: return launch_tiled_epi<NCH, EPI_ARGMAX, BITS, META>(p, s);
    }
    return hipErrorInvalidValue;
}

template <int BITS, int META>
static hipError_t launch_tiled_bits(const GemvLaunch& p, hipStream_t s) {
    switch (((p.cols >> 6) + 63) / 64) {
        case 1: return launch_tiled_nch<1, BITS, META>(p, s);
        case 2: return launch_tiled_nch<2, BITS, META>(p, s);
        case 3: return launch_tiled_nch<3, BITS, META>(p, s);
        case 4: return launch_tiled_nch<4, BITS, META>(p, s);
        default: return hipErrorInvalidValue;
    }
}

// TILED64 launches with fp32 metadata (gemv_w4a16_m32.hip), with the fp16
// scale alone, zero 8 (gemv_w4a16_s16.hip), and with the fp32 scale and a
// 4-bit zero (gemv_w4a16_z4.hip).
hipError_t launch_gemv_tiled_m32(const GemvLaunch& p, hipStream_t s);
hipError_t launch_gemv_tiled_s16(const GemvLaunch& p, hipStream_t s);
hipError_t launch_gemv_tiled_z4(const GemvLaunch& p, hipStream_t s);

}  // namespace xqhip
