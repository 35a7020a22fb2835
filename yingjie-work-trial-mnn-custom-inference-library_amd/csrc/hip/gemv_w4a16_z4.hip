// gemv_w4a16_z4.hip - the TILED64 GEMV for 4-bit format-v1 matrices whose
// zero points are integers 0..15 but whose scales fp16 cannot hold (the
// reference packer's asymmetric quantiser: scale = (max - min) / 15 in fp32,
// zero = round(-min / scale) clamped to 0..15, pack_qwen35_xq4_numpy.py:218-247).
// Each group keeps its fp32 scale and a 4-bit zero code, 4.5 bytes instead of
// the 8 of the fp32 (scale, zero) pair, with the reference's values exactly
// (w = (q - z) s, kernels.hpp:18-19).  Same kernel as gemv_w4a16.hip.
#include "gemv_tiled.hpp"

namespace xqhip {

hipError_t launch_gemv_tiled_z4(const GemvLaunch& p, hipStream_t s) {
    if (p.bits != 4 || p.affine) return hipErrorInvalidValue;
    return launch_tiled_bits<4, 3>(p, s);
}

}  // namespace xqhip
