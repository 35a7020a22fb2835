// xqhip_kernels.hpp - launch interfaces shared between the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace xqhip {

// One fused-dequant GEMV launch (gemv_w4a16.hip).
struct GemvLaunch {
    const uint8_t* nib;
    const void* meta;
    int rows, cols, group, affine, layout;
    const void* x;
    int x_f16;
    const float* norm_w;  // fused RMSNorm of x when non-null
    float eps;
    void* y;
    int y_f16;
    int epi;  // 0 store, 1 add, 2 silu pair, 3 argmax
    uint64_t* partial;
    uint32_t* counter;
    int32_t* out_idx;
    float* out_val;
    int max_blocks;
};

hipError_t launch_gemv(const GemvLaunch& p, hipStream_t s);

}  // namespace xqhip
