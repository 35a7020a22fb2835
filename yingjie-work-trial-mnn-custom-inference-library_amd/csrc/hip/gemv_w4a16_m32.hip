// gemv_w4a16_m32.hip - the TILED64 GEMV with fp32 group metadata: matrices
// whose scales or zeros fp16 cannot hold exactly (e.g. the reference packer's
// asymmetric scales (max - min) / 15) keep the reference's fp32 values
// (QuantizedMatrix, customlib/kernels/kernels.hpp:18-19); each lane then reads
// 8 bytes of metadata per group instead of 4.  Same kernel as gemv_w4a16.hip.
#include "gemv_tiled.hpp"

namespace xqhip {

hipError_t launch_gemv_tiled_m32(const GemvLaunch& p, hipStream_t s) {
    switch (p.bits) {
        case 4: return launch_tiled_bits<4, 1>(p, s);
        case 3: return launch_tiled_bits<3, 1>(p, s);
        case 2: return launch_tiled_bits<2, 1>(p, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace xqhip
