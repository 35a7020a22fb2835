// decode_fused.hip - the linear-attention decode step and the output projection
// that consumes it, as one launch.
//
// In the decode graph the step (linear_step_kernel: conv1d + SiLU, q / k L2
// norm, gated delta rule, custom_model.cpp:961-1096) is latency-bound: its
// blocks spend ~3.6 us on a dependent chain over 5 MB.  The output projection
// after it (out_proj 4096 x 4096 W4A16 with the gated head norm prologue and
// the residual add, custom_model.cpp:1123-1135, 1179) then pays a kernel boundary
// and the first weights' memory latency before it can do anything.  Here one
// block per CU runs both:
//   * waves 0-3: one block of the step (linear_step_body<KS, true>), its output
//     and activated gate written through to memory, the block counted on a
//     hand-off counter once those stores are complete;
//   * waves 4-15: a block of the projection (gemv_tiled_run<..., EARLY>): its
//     weights (at 4096 rows, all of them: two rows per wave) are requested as
//     soon as the step's own loads are, so they arrive while the step
//     computes; one wave then waits until every step block is counted, and the
//     block stages the step's output and finishes the projection from
//     registers.
// The arithmetic of both parts is that of the two separate kernels, so the
// results are bit-identical to linear_step_kernel followed by gemv_w4_tiled.
//
// Hand-off.  The step blocks count themselves on kHandOffLines counters
// (block b on counter b % kHandOffLines, each in its own 128-byte line, so no
// line takes more than a few atomics); the waiting wave reads all of them with
// one load per poll (lane i reads counter i) and sums them.  Ordering without
// fences, as in the split attention: the output stores are agent-scope
// (written through the L2), a wave's `s_waitcnt vmcnt(0)` completes them
// before the block's count is issued, and the waiting wave reads the counters
// and then the output with agent-scope loads, which bypass the per-XCD L2.
// Every block then counts itself on a departure counter, and the block that
// completes it (all waits are over) sets the counters back to zero, so every
// launch starts from zeros.  The wait is bounded: a wait that gives up sets
// the error word and the block carries on (its results are invalid), so every
// wave always exits.  Every block waits for every step block, so the launch
// needs all its blocks resident at once (one 1024-thread block per CU): the
// host checks that with the occupancy API and otherwise reports the
// combination unsupported (the caller then launches the two kernels).
//
// Measured on the 9B shapes (out_proj 4096 x 4096, 32 value heads): 15.9 us
// per launch against 11.0 us for the two kernels back to back.  Per-block
// stamps: the step's last block counts itself 5.3 us after the first block
// starts (~1 us later than alone, its memory operations now sharing the CU
// with the projection's weight stream), the waiting waves see the complete
// count 3-5 us after that, and staging + the rest of the projection take
// 2.3 us.  The hand-off is the loss: with L2-resident (MTYPE RW) device
// memory, data written on one XCD reaches another only through memory, and
// each such hop (a write-through store, a poll that bypasses the L2) is a
// ~1.3 us round trip, where a kernel boundary costs 1.6 us in all.  The
// decode graph therefore keeps the two kernels unless asked (XQ_FUSE_STEP=1).
#include "gemv_tiled.hpp"
#include "linear_step.hpp"

namespace xqhip {

constexpr int kFusedThreads = 1024;
constexpr int kStepWaves = 4;                       // one 256-thread step block
constexpr int kProjWaves = kFusedThreads / kWave - kStepWaves;  // 12: the GEMV's row groups
constexpr int kHandOffLines = 32;
constexpr int kLineWords = 32;                      // 128 bytes
constexpr int kSyncDepart = kHandOffLines * kLineWords;
constexpr int kSyncError = kSyncDepart + kLineWords;
constexpr int kSyncWords = kSyncError + kLineWords;
constexpr uint32_t kHandOffSpin = 1u << 16;         // polls before a wait gives up (~0.1 s)
constexpr int kAuxAgent = 16;                       // buffer cache policy: agent-coherent (L2 bypass / write-through)
static_assert(kProjWaves == 12, "the projection part is the 12-wave GEMV block");

// One wave (all 64 lanes, uniform control flow): waits until the step blocks
// have all counted themselves, then counts this block as departed; the block
// that completes the departures zeroes every counter for the next launch.
__device__ __forceinline__ void hand_off_wait(uint32_t* sync, uint32_t step_blocks, int lane, int grid) {
    const __amdgpu_buffer_rsrc_t r = buf_rsrc(sync, kSyncWords * 4u);
    const uint32_t off = lane < kHandOffLines ? static_cast<uint32_t>(lane * kLineWords) * 4u : kBufOOB;
    bool ok = false;
    for (uint32_t spin = 0; spin < kHandOffSpin; ++spin) {
        const uint32_t v = __builtin_amdgcn_raw_buffer_load_b32(r, opaque_offset(off), 0, kAuxAgent);
        // (counts below 2^24: the float sum is exact; lanes past the counters read 0)
        const float total = wave_sum(static_cast<float>(v));
        if (__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(total)) >= step_blocks) {
            ok = true;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    if (lane == 0) {
        if (!ok) __hip_atomic_store(sync + kSyncError, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t d = __hip_atomic_fetch_add(sync + kSyncDepart, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (d == static_cast<uint32_t>(grid - 1)) {
            for (int i = 0; i < kHandOffLines; ++i)
                __hip_atomic_store(sync + i * kLineWords, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(sync + kSyncDepart, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// grid blocks of kFusedThreads; blocks 0 .. step_blocks - 1 run a step block
// each (value head b % lv_n, column slice b / lv_n: the order of the separate
// kernel's grid), every block a GEMV block of a grid-block launch.
template <int KS, int META>
__global__ void __launch_bounds__(kFusedThreads) step_outproj_kernel(LinearStepLaunch sp, int step_blocks,
                                                                     const uint8_t* __restrict__ nib,
                                                                     const uint32_t* __restrict__ meta, int rows,
                                                                     int cols, int affine, Prologue pro, float* y,
                                                                     uint32_t* sync, int grid) {
    extern __shared__ uint4 xs[];  // the GEMV's staged activations
    __shared__ StepSmem ssm;
    __shared__ float red[32];
    __shared__ uint64_t lds_keys[16];
    __shared__ uint32_t lds_cnt;
    const int b = static_cast<int>(blockIdx.x);
    // the wave index as a scalar: the branches below are wave-uniform, so the
    // waves that do not take one skip it (its barriers included)
    const int wid = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    if (threadIdx.x == 0) lds_cnt = 0u;  // complete before the step's own barrier (a full __syncthreads)
    if (wid < kStepWaves) {
        if (b < step_blocks) {
            linear_step_body<KS, true>(sp, b % sp.lv_n, b / sp.lv_n, threadIdx.x, ssm,
                                       StepHandOff{sync + (b % kHandOffLines) * kLineWords, &lds_cnt});
        } else {  // the two barriers of the step body
            asm volatile("s_barrier" ::: "memory");
            __syncthreads();
        }
        return;  // exited waves no longer take part in the block's barriers
    }
    const int tid = static_cast<int>(threadIdx.x) - kStepWaves * kWave;
    gemv_tiled_run<1, kProjWaves, 1, EPI_ADD, 4, META, true, kAuxAgent>(
        nib, meta, rows, cols, affine, sp.out, 0, pro, y, 0, nullptr, grid, tid, b, xs, red, lds_keys,
        []() { asm volatile("s_barrier" ::: "memory"); },  // the step has issued its loads
        [&]() {
            asm volatile("s_barrier" ::: "memory");  // the step's own barrier
            if (wid == kStepWaves) hand_off_wait(sync, static_cast<uint32_t>(step_blocks), tid, grid);
            asm volatile("s_barrier" ::: "memory");  // the wait is over
        });
}

size_t step_outproj_sync_bytes() { return kSyncWords * sizeof(uint32_t); }
int step_outproj_error_word() { return kSyncError; }

bool step_outproj_shape_ok(const LinearStepLaunch& sp, const GemvLaunch& g) {
    const bool meta_ok = g.layout == 0 || g.layout == 2 || g.layout == 3 || g.layout == 4;
    return sp.ksize == 4 && linear_step_supported(sp.lk_n, sp.lk_hd, sp.lv_n, sp.lv_hd, sp.ksize) && meta_ok &&
           g.bits == 4 && g.cols % 64 == 0 && g.cols <= 4096 && g.cols == sp.lv_n * sp.lv_hd && g.rows > 0 &&
           g.epi == EPI_ADD && !g.x_f16 && !g.y_f16 && stage_supported(g.cols, g.pro);
}

// The launch's block count, or 0 when its blocks cannot all be resident at once.
template <int KS, int META>
static int step_outproj_grid_t(const LinearStepLaunch& sp, const GemvLaunch& g) {
    const int step_blocks = sp.lv_n * ((sp.lv_hd + kDeltaCols - 1) / kDeltaCols);
    const size_t lds = static_cast<size_t>(g.cols >> 6) * kStageRecord * sizeof(uint4);
    static int resident_cache[16] = {};
    const int resident = resident_blocks(reinterpret_cast<const void*>(&step_outproj_kernel<KS, META>), kFusedThreads,
                                         lds, resident_cache);
    const int units = (g.rows + kProjWaves - 1) / kProjWaves;  // one row per wave batch
    int grid = units < resident ? units : resident;
    if (grid < step_blocks) grid = step_blocks;
    return resident >= 1 && grid <= resident ? grid : 0;
}

template <int KS, int META>
static hipError_t launch_step_outproj_t(const LinearStepLaunch& sp, const GemvLaunch& g, uint32_t* sync,
                                        hipStream_t s) {
    const int grid = step_outproj_grid_t<KS, META>(sp, g);
    if (grid == 0) return hipErrorNotSupported;
    const int step_blocks = sp.lv_n * ((sp.lv_hd + kDeltaCols - 1) / kDeltaCols);
    const size_t lds = static_cast<size_t>(g.cols >> 6) * kStageRecord * sizeof(uint4);
    hipLaunchKernelGGL((step_outproj_kernel<KS, META>), dim3(grid), dim3(kFusedThreads), lds, s, sp, step_blocks,
                       g.nib, static_cast<const uint32_t*>(g.meta), g.rows, g.cols, g.affine, g.pro,
                       static_cast<float*>(g.y), sync, grid);
    return hipGetLastError();
}

int step_outproj_grid(const LinearStepLaunch& sp, const GemvLaunch& g) {
    if (!step_outproj_shape_ok(sp, g)) return 0;
    switch (g.layout) {
        case 0: return step_outproj_grid_t<4, 0>(sp, g);
        case 2: return step_outproj_grid_t<4, 1>(sp, g);
        case 3: return step_outproj_grid_t<4, 2>(sp, g);
        case 4: return step_outproj_grid_t<4, 3>(sp, g);
    }
    return 0;
}

hipError_t launch_step_outproj(const LinearStepLaunch& sp, const GemvLaunch& g, uint32_t* sync, hipStream_t s) {
    if (!step_outproj_shape_ok(sp, g)) return hipErrorNotSupported;
    switch (g.layout) {
        case 0: return launch_step_outproj_t<4, 0>(sp, g, sync, s);
        case 2: return launch_step_outproj_t<4, 1>(sp, g, sync, s);
        case 3: return launch_step_outproj_t<4, 2>(sp, g, sync, s);
        case 4: return launch_step_outproj_t<4, 3>(sp, g, sync, s);
    }
    return hipErrorNotSupported;
}

}  // namespace xqhip
