// gemv_w4a16_s16.hip - the TILED64 GEMV for 4-bit format-v1 matrices whose
// zero points are all 8 (the symmetric quantiser, the synthetic weights): the
// metadata is the fp16 group scale alone, 2 bytes per group instead of 4, and
// the zero point is implied (w = (q - 8) s, kernels.hpp:18-19 with zero 8).
// Same kernel as gemv_w4a16.hip.
#include "gemv_tiled.hpp"

namespace xqhip {

hipError_t launch_gemv_tiled_s16(const GemvLaunch& p, hipStream_t s) {
    if (p.bits != 4 || p.affine) return hipErrorInvalidValue;
    return launch_tiled_bits<4, 2>(p, s);
}

}  // namespace xqhip
