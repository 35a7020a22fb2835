// linear_step.hpp - the fused linear-attention decode step (conv1d + SiLU,
// q / k L2 norm, gated delta rule) as the body of one 256-thread block, shared
// by linear_step_kernel (decode_ops.hip) and the launch that runs the step and
// the output projection that consumes it (decode_fused.hip).
#pragma once

#include "xqhip_common.hpp"
#include "xqhip_kernels.hpp"

namespace xqhip {

constexpr int kDeltaCols = 16;
constexpr int kDeltaIGroups = 16;   // threads per column
constexpr int kDeltaMaxKPerThread = 16;  // key dim <= 256
constexpr int kStepMaxTaps = 8;          // conv kernel size of the fused step

// The block's LDS, and the hand-off words of the FUSED form (below).
struct StepSmem {
    float qk[2 * 256];
    float vsh[kDeltaCols];
    float red[2][4];
};
struct StepHandOff {
    uint32_t* arrive;
    uint32_t* lds_cnt;
};

// ---------------------------------------------------------------------------
// Fused linear-attention step, the body of one block of 256 threads (tid
// 0 .. 255) for value head vh and column slice `slice`: the block recomputes
// the conv1d + SiLU + L2 norm of its key head's q and k channels (cheap:
// 2 * lk_hd channels of ksize taps), the conv of its own kDeltaCols value
// channels, then runs the gated delta update of gated_delta_kernel on those
// columns.  Conv history is double-buffered by position parity (read copy
// pos & 1, write the other): the q/k history is written by one block per key
// head (vh % factor == 0, first slice), the value history by the block that
// owns the channel.
// KS > 0: the conv kernel size as a compile-time constant (the tap loops then
// issue exactly the loads they need); KS == 0: runtime p.ksize <= kStepMaxTaps.
// FUSED: the block's four waves run inside a launch whose other waves read
// the step's output (decode_fused.hip).  The output and the activated gate
// are then stored through to memory (agent scope: the readers may run on
// another XCD), the other waves of the block pass two barriers with these
// four (one right after the step has issued its loads, so their own loads
// queue behind the step's, and the step's own barrier), and once every store
// of the four waves is complete the last of them to finish adds 1 to the
// hand-off counter ho.arrive (ho.lds_cnt: a zeroed LDS word of the block).
// ---------------------------------------------------------------------------
template <int KS, bool FUSED>
__device__ __forceinline__ void linear_step_body(const LinearStepLaunch& p, int vh, int slice, uint32_t tid,
                                                 StepSmem& sm, StepHandOff ho) {
    constexpr int kTaps = KS > 0 ? KS : kStepMaxTaps;
    float* qk = sm.qk;
    float* vsh = sm.vsh;
    float (*red)[4] = sm.red;
    const int j0 = slice * kDeltaCols;
    const int factor = max(1, p.lv_n / max(1, p.lk_n));
    const int kh = min(p.lk_n - 1, vh / factor);
    const int dk = p.lk_hd, dv = p.lv_hd;
    const int hist = KS > 0 ? KS - 1 : max(0, p.ksize - 1);
    const int conv_dim = 2 * p.lk_n * dk + p.lv_n * dv;
    const bool qk_writer = (vh % factor == 0) && slice == 0;
    // the delta rule is wave-local: wave w owns columns 4w .. 4w + 3 of the
    // slice, 16 lanes per column (lane l: column l / 16, rows l % 16 + 16 r),
    // so its row sums are DPP reductions inside the wave, with no LDS or
    // barrier after the conv
    static_assert(kDeltaCols == 4 * 4 && kDeltaIGroups == 16, "4 waves x 4 columns x 16 lanes");
    const int jl = 4 * (static_cast<int>(tid) / kWave) + (static_cast<int>(tid) & (kWave - 1)) / 16;
    const int ig = tid & 15;
    const int j = j0 + jl;
    const bool active = j < dv;
    float* S = p.state + static_cast<size_t>(vh) * dk * dv;
    const int pos_s = *p.pos;
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
            tp.h[t] = buf_load_f32(r_hist, opaque_offset(ok && t < hist ? ho + 4u * t : kBufOOB));
            tp.h_other[t] = buf_load_f32(r_hist, opaque_offset(ok && t < hist ? hist_bytes + ho + 4u * t : kBufOOB));
        }
#pragma unroll
        for (int t = 0; t < kTaps; ++t)
            tp.w[t] = buf_load_f32(r_w, opaque_offset(ok && t <= hist ? wo + 4u * t : kBufOOB));
        tp.x = buf_load_f32(r_x, opaque_offset(ok ? static_cast<uint32_t>(c) * 4u : kBufOOB));
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
        const int t = tid + u * kThreads;
        int d; bool is_k;
        const int c = qk_channel(t, d, is_k);
        load_taps(u < nqk && t < 2 * dk ? c : -1, tq[u]);
    }
    const bool has_v = tid < kDeltaCols && j0 + static_cast<int>(tid) < dv;
    load_taps(has_v ? 2 * p.lk_n * dk + vh * dv + j0 + static_cast<int>(tid) : -1, tv);
    // the gated norm's gate of this block's columns, activated here once instead
    // of in every block of the output projection (read now, written at the end)
    const bool has_z = p.z_act != nullptr && has_v;
    const float zraw = buf_load_f32(buf_rsrc(p.z_act, p.z_act ? static_cast<uint32_t>(p.lv_n * dv) * 4u : 0u),
                                    has_z ? static_cast<uint32_t>(vh * dv + j0 + static_cast<int>(tid)) * 4u
                                          : kBufOOB);
    const __amdgpu_buffer_rsrc_t r_state = buf_rsrc(S, static_cast<uint32_t>(dk * dv) * 4u);
    float sreg[kDeltaMaxKPerThread];
#pragma unroll
    for (int r = 0; r < kDeltaMaxKPerThread; ++r) {
        const int i = ig + r * kDeltaIGroups;
        // (a 24-bit multiply: the 64-bit multiply-add the compiler picks for
        // i * dv + j reads an unused high half that can alias a pending load)
        sreg[r] = buf_load_f32(r_state, active && i < dk ? (__umul24(i, dv) + j) * 4u : kBufOOB);
    }
    // every load above is issued before any arithmetic that waits for one
    __builtin_amdgcn_sched_barrier(0);
    // (an asm barrier with a memory clobber: it waits for none of the loads)
    if constexpr (FUSED) asm volatile("s_barrier" ::: "memory");
    // the position's parity picks the history copy read above and the one
    // written at the end (a scalar load, requested at the top with the kernel
    // arguments: waiting for it drains none of the vector loads)
    const int par = pos_s & 1;
    float* st_out = p.conv_state + static_cast<size_t>(par ^ 1) * conv_dim * hist;
    select_parity(tq[0], par);
    select_parity(tq[1], par);
    select_parity(tv, par);
    // q and k channels of key head kh: thread t < dk -> q[t], dk <= t < 2 dk -> k[t - dk]
    float ssq = 0.0f, ssk = 0.0f;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int t = tid + u * kThreads;
        if (u < nqk && t < 2 * dk) {
            int d; bool is_k;
            qk_channel(t, d, is_k);
            const float y = conv(tq[u]);
            qk[(is_k ? 256 : 0) + d] = y;
            if (is_k) ssk += y * y; else ssq += y * y;
        }
    }
    if (has_v) vsh[tid] = conv(tv);
    const int lane = tid & (kWave - 1), wid = tid / kWave;
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
    // The lane's rows i = ig + 16 r, as straight-line code: every LDS read of
    // the normalised k_i and q_i issued before the first use (rows past dk
    // select 0: their state words were read as 0 and are never stored), the
    // state stores range-checked (kBufOOB for rows past dk and inactive
    // columns).  Per-row branches had made each row a block of its own with a
    // full wait for its LDS read.  The second half of the rows exists only for
    // dk > 128 (a uniform branch).
    constexpr int kHalf = kDeltaMaxKPerThread / 2;
    const bool upper = dk > kHalf * kDeltaIGroups;
    float kn[kDeltaMaxKPerThread], qn[kDeltaMaxKPerThread];
    auto read_rows = [&](int r0) {
        // all reads first, unconditionally (i <= 255: both stay inside qk);
        // the empty asm after them keeps the compiler from moving a read under
        // the select's branch
        float kv[kHalf], qv[kHalf];
#pragma unroll
        for (int r = 0; r < kHalf; ++r) {
            const int i = ig + (r0 + r) * kDeltaIGroups;
            kv[r] = qk[256 + i];
            qv[r] = qk[i];
        }
#pragma unroll
        for (int r = 0; r < kHalf; ++r) asm volatile("" : "+v"(kv[r]), "+v"(qv[r]));
#pragma unroll
        for (int r = 0; r < kHalf; ++r) {
            const bool in = ig + (r0 + r) * kDeltaIGroups < dk;
            kn[r0 + r] = in ? kv[r] * invk : 0.0f;
            qn[r0 + r] = in ? qv[r] * invq : 0.0f;
        }
    };
    read_rows(0);
    if (upper) read_rows(kHalf);
    float pred = 0.0f;
    auto decay_rows = [&](int r0) {
#pragma unroll
        for (int r = r0; r < r0 + kHalf; ++r) {
            sreg[r] *= decay;
            pred += sreg[r] * kn[r];
        }
    };
    decay_rows(0);
    if (upper) decay_rows(kHalf);
    pred = lanes_sum<16>(pred);
    const float delta = active ? beta * (vj - pred) : 0.0f;
    float o = 0.0f;
    auto update_rows = [&](int r0) {
#pragma unroll
        for (int r = r0; r < r0 + kHalf; ++r) {
            const int i = ig + r * kDeltaIGroups;
            sreg[r] += kn[r] * delta;
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, sreg[r]), r_state,
                                                  active && i < dk ? (__umul24(i, dv) + j) * 4u : kBufOOB, 0, 0);
            o += sreg[r] * qn[r];
        }
    };
    update_rows(0);
    if (upper) update_rows(kHalf);
    o = lanes_sum<16>(o);
    if (ig == 0 && active) {
        const float ov = o * (1.0f / sqrtf(static_cast<float>(dk)));
        if constexpr (FUSED)
            __hip_atomic_store(p.out + static_cast<size_t>(vh) * dv + j, ov, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
            p.out[static_cast<size_t>(vh) * dv + j] = ov;
    }
    if (qk_writer) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int t = tid + u * kThreads;
            if (u < nqk && t < 2 * dk) {
                int d; bool is_k;
                write_history(st_out, qk_channel(t, d, is_k), tq[u]);
            }
        }
    }
    if (has_v) write_history(st_out, 2 * p.lk_n * dk + vh * dv + j0 + tid, tv);
    if (has_z) {
        if constexpr (FUSED)
            __hip_atomic_store(p.z_act + vh * dv + j0 + tid, silu_dev(zraw), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
            p.z_act[vh * dv + j0 + tid] = silu_dev(zraw);
    }
    if constexpr (FUSED) {
        // this wave's stores are complete (the agent-scope ones written through
        // to memory); the block's fourth wave to get here counts the block
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if ((tid & (kWave - 1)) == 0 &&
            __hip_atomic_fetch_add(ho.lds_cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) == 3u)
            __hip_atomic_fetch_add(ho.arrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}


}  // namespace xqhip
