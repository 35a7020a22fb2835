// decode_chain.hip - consecutive decode-step projections as one persistent
// launch (the xqhip_chain_* entry points of include/xqhip.h).
//
// The projections of a decode step form a dependent chain (each GEMV reads the
// whole vector the previous one wrote, custom_model.cpp:1138-1256), and with
// one kernel per GEMV every boundary costs a dispatch, the next kernel's ramp
// and the previous one's drain while HBM idles.  Here one block per CU runs
// the ops of a chain in order:
//   * each wave streams its weight units (one row x one 4096-column chunk:
//     32 bytes of codes + the group metadata per lane, the TILED64 layout of
//     gemv_tiled.hpp) through P register buffers; a buffer is refilled
//     with the wave's next unit as soon as it is consumed, and the next unit
//     after an op's last one is the first of the op after it, so at an op
//     boundary the next op's weights are already in flight;
//   * an op's outputs go to a hand-off arena as 8-byte records (value bits,
//     launch sequence number) written through to memory (one store each, so a
//     record is never seen half written), and the next op's blocks poll their
//     whole input vector until every record carries this launch's number
//     (bounded: a wait that gives up sets the error word and the block goes
//     on, so every block always exits);
//   * the arithmetic of every op is that of gemv_w4_tiled with one row per
//     wave batch: the same digit staging of x, the same integer dot products
//     and factorisation, the same order of the chunk sums and of the residual
//     add, so results are bit-identical to the one-kernel-per-op path.
// All blocks of the grid must be resident at once (one per CU: the grid is the
// CU count and the LDS request admits one block per CU); the launch sequence
// number comes from the sync block and is advanced by the last block to finish.
#include "xqhip.h"
#include "gemv_tiled.hpp"

#include <cstdlib>
#include <string>
#include <vector>

namespace xqhip {
void set_last_error(const std::string& msg);  // xqhip_api.hip

namespace {

constexpr int kChainThreads = 768;
constexpr int kChainWaves = kChainThreads / kWave;  // 12
constexpr int kChainPDefault = 2;                    // weight units in flight per wave (2 or 4)
constexpr int kChainMaxCols = 16384;
constexpr int kChainPartMax = 4096;                  // chunk partial sums of an op per block
constexpr uint32_t kSpinLimit = 1u << 16;            // polls before a wait gives up (~0.1 s)
constexpr int kAuxSc1 = 16;                          // cache policy: agent-coherent (write-through / L2 bypass)
constexpr size_t kChainLds = 96 * 1024;              // > half of the CU's LDS: one block per CU
// sync block words (128-byte lines apart)
constexpr int kSyncSeq = 0, kSyncDone = 32, kSyncErr = 64, kSyncWords = 96;

// Device description of one op (built by xqhip_chain_create).
struct ChainOp {
    const uint8_t* nib;
    const void* meta;
    const float* pro_w;
    const float* x_plain;
    const float* z_plain;
    const float* h_plain;
    float* y_plain;
    int rows, cols, affine, epi, pro, head_dim;
    float eps;
    int nch, rgs, trips, trips_pad;
    int x_ll, z_ll, h_ll, y_ll;  // record offsets (-1: none)
    int silu;
};

template <int META>
struct Unit {
    uint4 a, b;
    MetaWord<META> m;
};

// Row of unit u of a wave in row group rg of block b: rows are dealt to the
// blocks' row groups in turn; SILU ops take the two rows of a pair (gate, up)
// as consecutive units of one wave.
__device__ __forceinline__ int unit_row(int u, int b, int grid, int rgs, int rg, int silu) {
    if (silu) return 2 * (((u >> 1) * grid + b) * rgs + rg) + (u & 1);
    return (u * grid + b) * rgs + rg;
}

// The weight stream of one wave: the op of its next unit and that op's
// load parameters.
template <int META>
struct Cursor {
    int op, u;
    __amdgpu_buffer_rsrc_t nib, meta;
    uint32_t row_bytes;
    int G, rows, rgs, rg, c, silu, trips_pad, gcnt;
    bool has_group;

    __device__ __forceinline__ void load_op(const ChainOp* __restrict__ ops, int n_ops, int i, int wid, int lane) {
        op = i;
        u = 0;
        if (i >= n_ops) {
            rows = 0;
            trips_pad = 1 << 30;
            nib = buf_rsrc(nullptr, 0u);
            meta = buf_rsrc(nullptr, 0u);
            row_bytes = 0;
            G = 1; rgs = 1; rg = 0; c = 0; silu = 0; gcnt = 0; has_group = false;
            return;
        }
        const ChainOp& d = ops[i];
        rows = d.rows;
        G = d.cols >> 6;
        row_bytes = tiled_row_bytes<4>(d.cols);
        const int nch = d.nch;
        rgs = d.rgs;
        c = wid % nch;
        rg = wid / nch;
        silu = d.silu;
        trips_pad = d.trips_pad;
        gcnt = min(64, G - c * 64);
        has_group = c * 64 + lane < G && rg < rgs;
        nib = buf_rsrc(d.nib, static_cast<uint32_t>(rows) * row_bytes);
        meta = buf_rsrc(d.meta, static_cast<uint32_t>(rows) * static_cast<uint32_t>(G) * kMetaGroupBytes<META>);
    }

    // issues the loads of the next unit into w and advances
    __device__ __forceinline__ void next(Unit<META>& w, const ChainOp* __restrict__ ops, int n_ops, int b, int grid,
                                         int wid, int lane) {
        const int row = unit_row(u, b, grid, rgs, rg, silu);
        const bool ok = has_group && row < rows;
        const uint32_t base = __umul24(static_cast<uint32_t>(row), row_bytes) + static_cast<uint32_t>(c * 2048);
        const uint32_t off = base + static_cast<uint32_t>(lane * 16);
        const uint32_t moff =
            (__umul24(static_cast<uint32_t>(row), static_cast<uint32_t>(G)) + c * 64 + lane) * kMetaGroupBytes<META>;
        w.a = as_uint4(__builtin_amdgcn_raw_buffer_load_b128(nib, ok ? off : kOutOfRange, 0, kLoadNT));
        w.b = as_uint4(__builtin_amdgcn_raw_buffer_load_b128(nib, ok ? off + gcnt * 16 : kOutOfRange, 0, kLoadNT));
        w.m = load_meta<META, kLoadNT>(meta, ok ? moff : kOutOfRange);
        if (++u == trips_pad) load_op(ops, n_ops, op + 1, wid, lane);
    }
};

// Row sum of one unit against the lane's staged group (gemv_w4_tiled's
// process() with one row).
template <int META>
__device__ __forceinline__ float unit_dot(const Unit<META>& w, const uint32_t (&xd)[kDigits][8], float ge, float gg,
                                          int affine) {
    uint32_t wd[8];
    group_words<4>(w.a, w.b, wd);
    int A[kDigits];
#pragma unroll
    for (int d = 0; d < kDigits; ++d) A[d] = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int d = 0; d < kDigits; ++d)
            A[d] = __builtin_amdgcn_sdot8(static_cast<int>(wd[j]), static_cast<int>(xd[d][j]), A[d], false);
    int Dg = A[kDigits - 1];
#pragma unroll
    for (int d = kDigits - 2; d >= 0; --d) Dg = (Dg << 4) + A[d];
    const float df = static_cast<float>(Dg);
    const float sc = meta_scale(w.m);
    float acc;
    if constexpr (META == 2) {
        acc = mul_rn(sc * ge, df);
    } else {
        const float z = meta_zero(w.m);
        acc = affine ? mul_rn(ge, fmaf(sc, df, fmaf(8.0f, sc, z) * gg)) : mul_rn(sc * ge, fmaf(8.0f - z, gg, df));
    }
    return wave_sum(acc);
}

// Load of 8 consecutive values (item `item`) of a source: a plain fp32 vector
// (two 16-byte loads) or hand-off records (four 16-byte loads of two records).
struct SrcRegs {
    u32x4 r[4];
};
__device__ __forceinline__ void issue_item(__amdgpu_buffer_rsrc_t rs, bool is_ll, bool want, int item, SrcRegs& s) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t off = kOutOfRange;
        if (want) off = is_ll ? static_cast<uint32_t>(item) * 64u + i * 16u
                              : (i < 2 ? static_cast<uint32_t>(item) * 32u + i * 16u : kOutOfRange);
        s.r[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, opaque_offset(off), 0, kAuxSc1);
    }
}
// true (and v filled) when every value of the item is present
__device__ __forceinline__ bool take_item(const SrcRegs& s, bool is_ll, uint32_t seq, float* v) {
    if (!is_ll) {
        v[0] = __uint_as_float(s.r[0].x); v[1] = __uint_as_float(s.r[0].y);
        v[2] = __uint_as_float(s.r[0].z); v[3] = __uint_as_float(s.r[0].w);
        v[4] = __uint_as_float(s.r[1].x); v[5] = __uint_as_float(s.r[1].y);
        v[6] = __uint_as_float(s.r[1].z); v[7] = __uint_as_float(s.r[1].w);
        return true;
    }
    bool ok = true;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        ok = ok && s.r[i].y == seq && s.r[i].w == seq;
        v[2 * i] = __uint_as_float(s.r[i].x);
        v[2 * i + 1] = __uint_as_float(s.r[i].z);
    }
    return ok;
}

__device__ __forceinline__ void chain_fail(uint32_t* sync, bool& failed) {
    failed = true;
    __hip_atomic_store(sync + kSyncErr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Prologue weights of item `item`: RMS w[8 item ..], gated w[(8 item) % head_dim ..]
__device__ __forceinline__ void issue_w(const ChainOp& d, __amdgpu_buffer_rsrc_t wr, bool want, int item, int n_items,
                                        u32x4& a, u32x4& b) {
    const uint32_t it = static_cast<uint32_t>(min(item, n_items - 1));
    const uint32_t off = d.pro == PRO_RMS ? it * 32u : static_cast<uint32_t>(static_cast<int>(it * 8u) & (d.head_dim - 1)) * 4u;
    a = __builtin_amdgcn_raw_buffer_load_b128(wr, opaque_offset(want ? off : kOutOfRange), 0, 0);
    b = __builtin_amdgcn_raw_buffer_load_b128(wr, opaque_offset(want ? off + 16u : kOutOfRange), 0, 0);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t pro_rsrc(const ChainOp& d, int cols) {
    const uint32_t bytes = d.pro == PRO_RMS ? cols * 4u
                           : (d.pro == PRO_GATED_ACT ? static_cast<uint32_t>(d.head_dim) * 4u : 0u);
    return buf_rsrc(d.pro_w, bytes);
}

// Prologue and digit staging of the acquired input (v, gate zv, prologue
// weights wl when WPRE, else loaded here): the arithmetic of stage_x_lds, the
// per-wave sums of squares left in red.
template <int ITEMS, bool GATED, bool WPRE>
__device__ __forceinline__ void stage_digits(const ChainOp& d, float (&v)[ITEMS][8], const float (&zv)[ITEMS][8],
                                             const float (&wl_pre)[ITEMS][8], uint4* xs, float* red) {
    const int cols = d.cols;
    const int n_items = cols >> 3;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const __amdgpu_buffer_rsrc_t wr = pro_rsrc(d, cols);
    auto weights = [&](int k, float (&wl)[8]) {
        if constexpr (WPRE) {
#pragma unroll
            for (int i = 0; i < 8; ++i) wl[i] = wl_pre[k][i];
        } else {
            u32x4 a, b;
            issue_w(d, wr, true, tid + k * kChainThreads, n_items, a, b);
            as_floats8(a, b, wl);
        }
    };
    if (d.pro == PRO_RMS) {
        // the sequence of stage_x_lds: explicit fused multiply-adds on selected operands
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < ITEMS; ++k) {
            const bool in = tid + k * kChainThreads < n_items;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float a = in ? v[k][i] : 0.0f;
                ss = fmaf(a, a, ss);
            }
        }
        ss = wave_sum(ss);
        if (lane == 0) red[tid / kWave] = ss;
#pragma unroll
        for (int k = 0; k < ITEMS; ++k) {
            float wl[8];
            weights(k, wl);
#pragma unroll
            for (int i = 0; i < 8; ++i) v[k][i] = v[k][i] * wl[i];
        }
    } else if (GATED) {
        // head_dim / 8 consecutive lanes of one wave hold a head (a power of two <= 64)
        const int per_head = d.head_dim >> 3;
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
            const float inv = 1.0f / sqrtf(hs / static_cast<float>(d.head_dim) + d.eps);
            float wl[8];
            weights(k, wl);
#pragma unroll
            for (int i = 0; i < 8; ++i) v[k][i] = v[k][i] * inv * wl[i] * zv[k][i];
        }
    }
    uint32_t* xw = reinterpret_cast<uint32_t*>(xs);
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
        const int item = tid + k * kChainThreads;
        const int g = item >> 3, w = item & 7;
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(v[k][i]));
        mx = lanes_max<8>(mx);
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
            for (int dg = 0; dg < kDigits; ++dg) xw[g * (4 * kStageRecord) + dg * 8 + w] = W[dg] ^ 0x88888888u;
            if (w == 0) {
                xw[g * (4 * kStageRecord) + 8 * kDigits] = __float_as_uint(mx * (1.0f / static_cast<float>(kXMax)));
                xw[g * (4 * kStageRecord) + 8 * kDigits + 1] = __float_as_uint(static_cast<float>(gs));
            }
        }
    }
    if (d.pro != PRO_RMS && lane == 0) red[tid / kWave] = 0.0f;
}

// Input of a chain's first op (every source plain, complete before the
// launch): the activation, gate, residual and prologue-weight loads are issued
// first, then `prefetch` requests the first weight units, so the activations
// return ahead of the weight stream (a CU's vector loads return in issue
// order) and the staging arithmetic overlaps it.  Returns the residual value
// of the epilogue rows (hr / h_off: plain fp32).
template <int ITEMS, bool GATED, typename Prefetch>
__device__ float chain_stage_first(const ChainOp& d, uint4* xs, float* red, __amdgpu_buffer_rsrc_t hr, uint32_t h_off,
                                   Prefetch&& prefetch) {
    const int cols = d.cols;
    const int n_items = cols >> 3;
    const int tid = threadIdx.x;
    const __amdgpu_buffer_rsrc_t xr = buf_rsrc(d.x_plain, cols * 4u);
    const __amdgpu_buffer_rsrc_t zr = buf_rsrc(GATED ? d.z_plain : nullptr, GATED ? cols * 4u : 0u);
    const __amdgpu_buffer_rsrc_t wr = pro_rsrc(d, cols);
    constexpr bool kPre = ITEMS == 1;
    SrcRegs xq[ITEMS], zq[ITEMS];
    u32x4 wa[ITEMS], wb[ITEMS];
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
        const int item = tid + k * kChainThreads;
        const bool want = item < n_items;
        issue_item(xr, false, want, item, xq[k]);
        if constexpr (GATED) issue_item(zr, false, want, item, zq[k]);
        if constexpr (kPre) issue_w(d, wr, want && d.pro != PRO_NONE, item, n_items, wa[k], wb[k]);
    }
    const float hold = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(hr, opaque_offset(h_off), 0, kAuxSc1));
    // (an asm barrier with a memory clobber: no load moves across it)
    asm volatile("" ::: "memory");
    prefetch();
    float v[ITEMS][8], zv[ITEMS][8], wl[ITEMS][8];
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
        take_item(xq[k], false, 0u, v[k]);
        if constexpr (GATED) take_item(zq[k], false, 0u, zv[k]);
        else
#pragma unroll
            for (int i = 0; i < 8; ++i) zv[k][i] = 0.0f;
        if constexpr (kPre) as_floats8(wa[k], wb[k], wl[k]);
    }
    stage_digits<ITEMS, GATED, kPre>(d, v, zv, wl, xs, red);
    return hold;
}

// Input of a later op: hand-off records (or plain vectors) polled until every
// value carries this launch's number, bounded; the residual value of the
// epilogue rows and (one item per thread) the prologue weights are requested
// with the first poll, so both are complete when it returns (loads issued
// after it would wait behind the weight stream queued meanwhile).
template <int ITEMS, bool GATED>
__device__ float chain_stage(const ChainOp& d, const uint64_t* ll, uint32_t seq, uint4* xs, float* red,
                             uint32_t* sync, bool& failed, __amdgpu_buffer_rsrc_t hr, uint32_t h_off, bool h_ll) {
    const int cols = d.cols;
    const int n_items = cols >> 3;
    const int tid = threadIdx.x;
    const bool x_ll = d.x_plain == nullptr;
    const __amdgpu_buffer_rsrc_t xr =
        x_ll ? buf_rsrc(ll + d.x_ll, static_cast<uint32_t>(cols) * 8u) : buf_rsrc(d.x_plain, cols * 4u);
    const bool z_ll = d.z_plain == nullptr;
    const __amdgpu_buffer_rsrc_t zr = !GATED ? buf_rsrc(nullptr, 0u)
                                      : (z_ll ? buf_rsrc(ll + d.z_ll, static_cast<uint32_t>(cols) * 8u)
                                              : buf_rsrc(d.z_plain, cols * 4u));
    const __amdgpu_buffer_rsrc_t wr = pro_rsrc(d, cols);
    constexpr bool kPre = ITEMS == 1;
    float v[ITEMS][8], zv[ITEMS][8], wl[ITEMS][8];
    uint32_t pending = 0;
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
        if (tid + k * kChainThreads < n_items) pending |= 1u << k;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[k][i] = zv[k][i] = wl[k][i] = 0.0f;
    }
    float hold = 0.0f;
    uint32_t hseq = seq;
    for (uint32_t spin = 0;; ++spin) {
        SrcRegs xq[ITEMS], zq[ITEMS];
        u32x4 wa[ITEMS], wb[ITEMS];
        const uint32_t h_now = spin == 0 ? h_off : kOutOfRange;
        const u32x2 hv = __builtin_amdgcn_raw_buffer_load_b64(hr, opaque_offset(h_ll ? h_now : kOutOfRange), 0, kAuxSc1);
        const uint32_t hp = __builtin_amdgcn_raw_buffer_load_b32(hr, opaque_offset(h_ll ? kOutOfRange : h_now), 0, kAuxSc1);
#pragma unroll
        for (int k = 0; k < ITEMS; ++k) {
            const bool want = (pending >> k) & 1u;
            issue_item(xr, x_ll, want, tid + k * kChainThreads, xq[k]);
            if constexpr (GATED) issue_item(zr, z_ll, want, tid + k * kChainThreads, zq[k]);
            if constexpr (kPre)
                issue_w(d, wr, spin == 0 && d.pro != PRO_NONE, tid + k * kChainThreads, n_items, wa[k], wb[k]);
        }
        if (spin == 0) {
            hold = __uint_as_float(h_ll ? hv.x : hp);
            hseq = h_ll ? hv.y : seq;
            if constexpr (kPre)
#pragma unroll
                for (int k = 0; k < ITEMS; ++k) as_floats8(wa[k], wb[k], wl[k]);
        }
#pragma unroll
        for (int k = 0; k < ITEMS; ++k) {
            if ((pending >> k) & 1u) {
                float a[8], g[8];
                bool ok = take_item(xq[k], x_ll, seq, a);
                if constexpr (GATED) ok = take_item(zq[k], z_ll, seq, g) && ok;
                if (ok) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        v[k][i] = a[i];
                        if constexpr (GATED) zv[k][i] = g[i];
                    }
                    pending &= ~(1u << k);
                }
            }
        }
        if (pending == 0 || failed) break;
        if (spin >= kSpinLimit) {
            chain_fail(sync, failed);
            break;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    if (h_off != kOutOfRange && hseq != seq && !failed) chain_fail(sync, failed);
    stage_digits<ITEMS, GATED, kPre>(d, v, zv, wl, xs, red);
    return hold;
}

// Stores one output value: a hand-off record and/or the plain copy, lane 0
// only (the other lanes' offsets are out of range: the stores stay
// unconditional, so the compiler's load-count waits stay exact).
__device__ __forceinline__ void store_out(__amdgpu_buffer_rsrc_t yl, __amdgpu_buffer_rsrc_t yp, int idx, bool valid,
                                          float val, uint32_t seq, int lane) {
    const bool st = valid && lane == 0;
    const u32x2 rec = {__float_as_uint(val), seq};
    __builtin_amdgcn_raw_buffer_store_b64(rec, yl, st ? static_cast<uint32_t>(idx) * 8u : kOutOfRange, 0, kAuxSc1);
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(val), yp, st ? static_cast<uint32_t>(idx) * 4u : kOutOfRange,
                                          0, 0);
}

// stamps (optional): per op and block the realtime counter (100 MHz) when the
// op's input is staged and when its last output is stored, [op][block][2]
__device__ __forceinline__ void chain_stamp(uint64_t* stamps, int op, int which, int grid) {
    if (stamps && threadIdx.x == 0)
        stamps[(static_cast<size_t>(op) * grid + blockIdx.x) * 2 + which] = __builtin_amdgcn_s_memrealtime();
}

template <int META, int P>
__global__ void __launch_bounds__(kChainThreads) chain_kernel(const ChainOp* __restrict__ ops, int n_ops,
                                                              uint64_t* __restrict__ ll, uint32_t* sync, int grid,
                                                              uint64_t* stamps) {
    extern __shared__ uint4 xs[];
    __shared__ float red[kChainWaves];
    __shared__ float part[kChainPartMax];
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wid = tid / kWave;
    const int b = blockIdx.x;
    // the launch number, requested first and waited for only after the first
    // weight units are in flight
    const uint32_t seq_raw = __hip_atomic_load(sync + kSyncSeq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // after a launch whose wait gave up, later launches wait for nothing (their
    // results are invalid anyway) until the host has seen the error word
    const uint32_t err_raw = __hip_atomic_load(sync + kSyncErr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    Cursor<META> cur;
    cur.load_op(ops, n_ops, 0, wid, lane);
    Unit<META> buf[P];
    // the first P weight units, requested after the first op's activations
    auto prefetch = [&]() {
#pragma unroll
        for (int p = 0; p < P; ++p) cur.next(buf[p], ops, n_ops, b, grid, wid, lane);
    };
    uint32_t seq = 0;
    bool failed = false;

    for (int op = 0; op < n_ops; ++op) {
        const ChainOp& d = ops[op];
        const int cols = d.cols, G = cols >> 6, nch = d.nch, rgs = d.rgs;
        const int c = wid % nch, rg = wid / nch;
        const int trips = d.trips, trips_pad = d.trips_pad, epi = d.epi, silu = d.silu, affine = d.affine;
        const bool gated = d.pro == PRO_GATED_ACT;
        // residual of the rows this wave finishes (lane t: unit t's row); it is
        // complete (an earlier op of the dependency chain read all of it)
        __amdgpu_buffer_rsrc_t hr = buf_rsrc(nullptr, 0u);
        uint32_t h_off = kOutOfRange;
        const bool h_ll = d.h_plain == nullptr;
        if (epi == EPI_ADD) {
            hr = h_ll ? buf_rsrc(ll + d.h_ll, static_cast<uint32_t>(d.rows) * 8u) : buf_rsrc(d.h_plain, d.rows * 4u);
            const int row = unit_row(lane, b, grid, rgs, rg, 0);
            if (lane < trips && row < d.rows && c == 0 && rg < rgs)
                h_off = static_cast<uint32_t>(row) * (h_ll ? 8u : 4u);
        }
        // input: poll, prologue, digits (the first op's sources are plain)
        const int items = (cols / 8 + kChainThreads - 1) / kChainThreads;
        float hold;
        if (op == 0 && items <= 1) {  // (wider first inputs: weights first, then the plain input)
            if (gated)
                hold = chain_stage_first<1, true>(d, xs, red, hr, h_off, prefetch);
            else
                hold = chain_stage_first<1, false>(d, xs, red, hr, h_off, prefetch);
            seq = __builtin_amdgcn_readfirstlane(seq_raw) + 1u;
            failed = __builtin_amdgcn_readfirstlane(err_raw) != 0u;
        } else if (op == 0) {
            prefetch();
            seq = __builtin_amdgcn_readfirstlane(seq_raw) + 1u;
            failed = __builtin_amdgcn_readfirstlane(err_raw) != 0u;
            hold = items == 2 ? chain_stage<2, false>(d, ll, seq, xs, red, sync, failed, hr, h_off, h_ll)
                              : chain_stage<3, false>(d, ll, seq, xs, red, sync, failed, hr, h_off, h_ll);
        } else if (gated) {
            hold = chain_stage<1, true>(d, ll, seq, xs, red, sync, failed, hr, h_off, h_ll);
        } else if (items <= 1) {
            hold = chain_stage<1, false>(d, ll, seq, xs, red, sync, failed, hr, h_off, h_ll);
        } else if (items == 2) {
            hold = chain_stage<2, false>(d, ll, seq, xs, red, sync, failed, hr, h_off, h_ll);
        } else {
            hold = chain_stage<3, false>(d, ll, seq, xs, red, sync, failed, hr, h_off, h_ll);
        }
        __syncthreads();
        const int g = c * 64 + lane;
        const bool has_group = g < G && rg < rgs;
        uint32_t xd[kDigits][8];
        float ge, gg;
        {
            const uint4* rec = xs + (has_group ? g : 0) * kStageRecord;
#pragma unroll
            for (int dg = 0; dg < kDigits; ++dg) {
                const uint4 lo4 = rec[2 * dg], hi4 = rec[2 * dg + 1];
                xd[dg][0] = lo4.x; xd[dg][1] = lo4.y; xd[dg][2] = lo4.z; xd[dg][3] = lo4.w;
                xd[dg][4] = hi4.x; xd[dg][5] = hi4.y; xd[dg][6] = hi4.z; xd[dg][7] = hi4.w;
            }
            const uint4 kk = rec[2 * kDigits];
            ge = has_group ? __uint_as_float(kk.x) : 0.0f;
            gg = has_group ? __uint_as_float(kk.y) : 0.0f;
        }
        if (d.pro == PRO_RMS) ge *= rms_factor<kChainWaves>(red, cols, d.eps);
        chain_stamp(stamps, op, 0, grid);
        const int out_n = silu ? d.rows / 2 : d.rows;
        const __amdgpu_buffer_rsrc_t yl = buf_rsrc(d.y_ll >= 0 ? ll + d.y_ll : nullptr, d.y_ll >= 0 ? out_n * 8u : 0u);
        const __amdgpu_buffer_rsrc_t yp = buf_rsrc(d.y_plain, d.y_plain ? out_n * 4u : 0u);
        float gate_keep = 0.0f;
        // the op's units; buffers past its last unit already hold the next op's
        for (int u0 = 0; u0 < trips_pad; u0 += P) {
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const int u = u0 + p;
                float val = 0.0f;
                int idx = 0;
                bool valid = false;
                if (u < trips) {
                    const float acc = unit_dot<META>(buf[p], xd, ge, gg, affine);
                    const int row = unit_row(u, b, grid, rgs, rg, silu);
                    if (nch > 1) {
                        if (lane == 0 && rg < rgs) part[(u * rgs + rg) * nch + c] = acc;
                    } else if (silu) {
                        if (u & 1) {
                            val = silu_dev(gate_keep) * acc;
                            idx = row >> 1;
                            valid = row < d.rows && rg < rgs;
                        } else {
                            gate_keep = acc;
                        }
                    } else {
                        val = epi == EPI_ADD ? readlane_f32(hold, u) + acc : acc;
                        idx = row;
                        valid = row < d.rows && rg < rgs;
                    }
                }
                store_out(yl, yp, idx, valid, val, seq, lane);
                cur.next(buf[p], ops, n_ops, b, grid, wid, lane);
            }
        }
        if (nch > 1) {  // chunk sums in chunk order, then the epilogue (chunk-0 waves)
            __syncthreads();
            if (c == 0 && rg < rgs) {
                for (int u = 0; u < trips; ++u) {
                    const int row = unit_row(u, b, grid, rgs, rg, 0);
                    float t = 0.0f;
                    for (int cc = 0; cc < nch; ++cc) t += part[(u * rgs + rg) * nch + cc];
                    const float val = epi == EPI_ADD ? readlane_f32(hold, u) + t : t;
                    store_out(yl, yp, row, row < d.rows, val, seq, lane);
                }
            }
        }
        chain_stamp(stamps, op, 1, grid);
        __syncthreads();  // xs, red and part are rewritten by the next op
    }
    if (tid == 0) {
        const uint32_t old = __hip_atomic_fetch_add(sync + kSyncDone, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == static_cast<uint32_t>(grid - 1)) {
            __hip_atomic_store(sync + kSyncDone, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(sync + kSyncSeq, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
struct Chain {
    ChainOp* dev = nullptr;  // device copy of ops
    int n_ops = 0;
    int meta = 0;
    int p = kChainPDefault;
    int grid = 0;
    size_t records = 0;
    int device = 0;
};

int chain_fail_host(int code, const std::string& msg) {
    set_last_error(msg);
    return code;
}

int meta_of(int layout) {
    switch (layout) {
        case XQHIP_LAYOUT_TILED64: return 0;
        case XQHIP_LAYOUT_TILED64_F32META: return 1;
        case XQHIP_LAYOUT_TILED64_SCALE16: return 2;
        default: return -1;
    }
}

template <int META, int P>
hipError_t launch_chain_t(const Chain& ch, uint64_t* ll, uint32_t* sync, uint64_t* stamps, hipStream_t s) {
    // (the LDS limit was raised by xqhip_chain_create)
    hipLaunchKernelGGL((chain_kernel<META, P>), dim3(ch.grid), dim3(kChainThreads), kChainLds, s, ch.dev, ch.n_ops, ll,
                       sync, ch.grid, stamps);
    return hipGetLastError();
}

template <int META>
hipError_t launch_chain_m(const Chain& ch, uint64_t* ll, uint32_t* sync, uint64_t* stamps, hipStream_t s) {
    return ch.p == 2 ? launch_chain_t<META, 2>(ch, ll, sync, stamps, s) : launch_chain_t<META, 4>(ch, ll, sync, stamps, s);
}

const void* chain_fn(int meta, int p) {
    switch (meta * 2 + (p == 2 ? 0 : 1)) {
        case 0: return reinterpret_cast<const void*>(&chain_kernel<0, 2>);
        case 1: return reinterpret_cast<const void*>(&chain_kernel<0, 4>);
        case 2: return reinterpret_cast<const void*>(&chain_kernel<1, 2>);
        case 3: return reinterpret_cast<const void*>(&chain_kernel<1, 4>);
        case 4: return reinterpret_cast<const void*>(&chain_kernel<2, 2>);
        default: return reinterpret_cast<const void*>(&chain_kernel<2, 4>);
    }
}

// Weight units in flight per wave: XQHIP_CHAIN_UNITS (2 or 4) overrides the default.
int chain_units() {
    const char* v = std::getenv("XQHIP_CHAIN_UNITS");
    if (v && std::atoi(v) == 2) return 2;
    if (v && std::atoi(v) == 4) return 4;
    return kChainPDefault;
}

}  // namespace
}  // namespace xqhip

using xqhip::Chain;
using xqhip::ChainOp;

extern "C" {

XQHIP_API size_t xqhip_chain_sync_bytes(void) { return xqhip::kSyncWords * sizeof(uint32_t); }

XQHIP_API int xqhip_chain_create(const xqhip_chain_op* ops, int n_ops, void** chain) {
    using namespace xqhip;
    if (!ops || n_ops <= 0 || !chain) return chain_fail_host(XQHIP_EINVAL, "xqhip_chain_create: no ops");
    *chain = nullptr;
    int dev = 0, cus = 0, per = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
        return chain_fail_host(XQHIP_EDEVICE, "xqhip_chain_create: device query failed");
    const int P = chain_units();
    std::vector<ChainOp> d(static_cast<size_t>(n_ops));
    std::vector<int> out_n(static_cast<size_t>(n_ops)), y_ll(static_cast<size_t>(n_ops));
    int meta = -1;
    size_t records = 0;
    for (int i = 0; i < n_ops; ++i) {
        const xqhip_chain_op& o = ops[i];
        const std::string at = "xqhip_chain_create op " + std::to_string(i) + ": ";
        if (!o.w || o.w->bits != 4) return chain_fail_host(XQHIP_EINVAL, at + "needs a 4-bit matrix");
        const int m = meta_of(o.w->layout);
        if (m < 0)
            return chain_fail_host(XQHIP_EINVAL, at + "needs a TILED64 matrix with fp16, fp32-pair or fp16-scale "
                                                      "metadata (layout " + std::to_string(o.w->layout) + ")");
        if (meta >= 0 && m != meta) return chain_fail_host(XQHIP_EINVAL, at + "metadata layout differs from op 0");
        meta = m;
        const int rows = o.w->rows, cols = o.w->cols;
        if (cols % 64 != 0 || cols > kChainMaxCols || rows < 1)
            return chain_fail_host(XQHIP_EINVAL, at + "unsupported shape");
        if (static_cast<uint64_t>(rows) * (cols / 2) >= kOutOfRange)
            return chain_fail_host(XQHIP_EINVAL, at + "matrix too large");
        ChainOp& c = d[static_cast<size_t>(i)];
        c = ChainOp{};
        c.nib = static_cast<const uint8_t*>(o.w->nib);
        c.meta = o.w->meta;
        c.rows = rows;
        c.cols = cols;
        c.affine = o.w->affine;
        c.epi = o.epi;
        c.pro = o.pro;
        c.pro_w = o.pro_w;
        c.head_dim = o.head_dim;
        c.eps = o.eps;
        c.y_plain = o.y_plain;
        c.silu = o.epi == XQHIP_EPI_SILU_PAIR ? 1 : 0;
        if (o.epi != XQHIP_EPI_STORE && o.epi != XQHIP_EPI_ADD && o.epi != XQHIP_EPI_SILU_PAIR)
            return chain_fail_host(XQHIP_EINVAL, at + "unknown epilogue");
        if (o.pro != XQHIP_PRO_NONE && o.pro != XQHIP_PRO_RMS && o.pro != XQHIP_PRO_GATED_HEAD_ACT)
            return chain_fail_host(XQHIP_EINVAL, at + "unsupported prologue");
        if ((o.pro != XQHIP_PRO_NONE) && !o.pro_w) return chain_fail_host(XQHIP_EINVAL, at + "prologue weight missing");
        if (o.pro == XQHIP_PRO_GATED_HEAD_ACT) {
            const int per = o.head_dim / 8;
            if (o.head_dim % 8 != 0 || per < 1 || per > 64 || (per & (per - 1)) != 0 || cols > 4096)
                return chain_fail_host(XQHIP_EINVAL, at + "gated prologue shape");
        }
        c.nch = (cols / 64 + 63) / 64;
        c.rgs = kChainWaves / c.nch;
        if (c.silu && (c.nch != 1 || rows % 2 != 0))
            return chain_fail_host(XQHIP_EINVAL, at + "SiLU pairs need one chunk and an even row count");
        const int per_trip = cus * c.rgs;
        c.trips = c.silu ? 2 * ((rows / 2 + per_trip - 1) / per_trip) : (rows + per_trip - 1) / per_trip;
        c.trips_pad = (c.trips + P - 1) / P * P;
        if (c.trips > kWave) return chain_fail_host(XQHIP_EINVAL, at + "too many rows per wave");
        if (c.nch > 1 && c.trips * c.rgs * c.nch > kChainPartMax)
            return chain_fail_host(XQHIP_EINVAL, at + "too many chunk partials");
        if (static_cast<size_t>(cols / 64) * kStageRecord * sizeof(uint4) > kChainLds)
            return chain_fail_host(XQHIP_EINVAL, at + "input too wide");
        out_n[static_cast<size_t>(i)] = c.silu ? rows / 2 : rows;
        records = (records + 15) / 16 * 16;  // each output starts on a 128-byte line
        y_ll[static_cast<size_t>(i)] = static_cast<int>(records);
        c.y_ll = static_cast<int>(records);
        records += static_cast<size_t>(out_n[static_cast<size_t>(i)]);
        // sources
        auto src = [&](const xqhip_chain_src& s, int n, const float** plain, int* ll_off, const char* what) -> bool {
            *plain = s.plain;
            *ll_off = -1;
            if (s.plain) return true;
            if (s.op < 0 || s.op >= i || s.offset < 0 || s.offset % 2 != 0 ||
                s.offset + n > out_n[static_cast<size_t>(s.op)]) {
                set_last_error(at + what + " source out of range");
                return false;
            }
            *ll_off = y_ll[static_cast<size_t>(s.op)] + s.offset;
            return true;
        };
        if (!src(o.x, cols, &c.x_plain, &c.x_ll, "input")) return XQHIP_EINVAL;
        c.z_plain = nullptr;
        c.z_ll = -1;
        if (o.pro == XQHIP_PRO_GATED_HEAD_ACT && !src(o.gate, cols, &c.z_plain, &c.z_ll, "gate")) return XQHIP_EINVAL;
        c.h_plain = nullptr;
        c.h_ll = -1;
        if (o.epi == XQHIP_EPI_ADD && !src(o.res, rows, &c.h_plain, &c.h_ll, "residual")) return XQHIP_EINVAL;
    }
    if (records >= (1u << 28)) return chain_fail_host(XQHIP_EINVAL, "xqhip_chain_create: arena too large");
    const void* fn = chain_fn(meta, P);
    if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kChainLds)) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, fn, kChainThreads, kChainLds) != hipSuccess || per < 1)
        return chain_fail_host(XQHIP_EDEVICE, "xqhip_chain_create: the chain kernel does not fit a CU");
    auto* ch = new Chain();
    ch->n_ops = n_ops;
    ch->meta = meta;
    ch->p = P;
    ch->grid = cus;  // one block per CU, all resident at once
    ch->records = records;
    ch->device = dev;
    if (hipMalloc(&ch->dev, sizeof(ChainOp) * d.size()) != hipSuccess ||
        hipMemcpy(ch->dev, d.data(), sizeof(ChainOp) * d.size(), hipMemcpyHostToDevice) != hipSuccess) {
        if (ch->dev) (void)hipFree(ch->dev);
        delete ch;
        return chain_fail_host(XQHIP_ENOMEM, "xqhip_chain_create: device op table");
    }
    *chain = ch;
    return XQHIP_OK;
}

XQHIP_API int xqhip_chain_destroy(void* chain) {
    auto* ch = static_cast<Chain*>(chain);
    if (!ch) return XQHIP_OK;
    if (ch->dev) (void)hipFree(ch->dev);
    delete ch;
    return XQHIP_OK;
}

XQHIP_API size_t xqhip_chain_arena_records(const void* chain) {
    const auto* ch = static_cast<const Chain*>(chain);
    return ch ? ch->records : 0;
}

XQHIP_API int xqhip_chain_launch(const void* chain, void* arena, void* sync, void* stream) {
    return xqhip_chain_launch_stamped(chain, arena, sync, nullptr, stream);
}

XQHIP_API int xqhip_chain_grid(const void* chain) {
    const auto* ch = static_cast<const Chain*>(chain);
    return ch ? ch->grid : 0;
}

XQHIP_API int xqhip_chain_launch_stamped(const void* chain, void* arena, void* sync, void* stamps, void* stream) {
    using namespace xqhip;
    const auto* ch = static_cast<const Chain*>(chain);
    if (!ch || !arena || !sync) return chain_fail_host(XQHIP_EINVAL, "xqhip_chain_launch: null argument");
    auto* ll = static_cast<uint64_t*>(arena);
    auto* sy = static_cast<uint32_t*>(sync);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e;
    switch (ch->meta) {
        case 0: e = launch_chain_m<0>(*ch, ll, sy, static_cast<uint64_t*>(stamps), s); break;
        case 1: e = launch_chain_m<1>(*ch, ll, sy, static_cast<uint64_t*>(stamps), s); break;
        default: e = launch_chain_m<2>(*ch, ll, sy, static_cast<uint64_t*>(stamps), s); break;
    }
    if (e != hipSuccess) return chain_fail_host(XQHIP_EDEVICE, std::string("xqhip_chain_launch: ") + hipGetErrorString(e));
    return XQHIP_OK;
}

XQHIP_API int xqhip_chain_error(const void* sync, int* error) {
    using namespace xqhip;
    if (!sync || !error) return chain_fail_host(XQHIP_EINVAL, "xqhip_chain_error: null argument");
    uint32_t w = 0;
    if (hipMemcpy(&w, static_cast<const uint32_t*>(sync) + kSyncErr, sizeof(w), hipMemcpyDeviceToHost) != hipSuccess)
        return chain_fail_host(XQHIP_EDEVICE, "xqhip_chain_error: copy failed");
    *error = w != 0;
    return XQHIP_OK;
}

}  // extern "C"
