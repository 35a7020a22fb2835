// ref_shim.cpp - extern "C" adapters over the compiled reference kernels.
//
// TEST INFRASTRUCTURE ONLY.  Linked with the reference's own sources (compiled
// where they lie under the reference checkout, see oracle/Makefile) into
// oracle/_ref/libxqref.so, so that tests can call the reference's C++ kernel
// functions through ctypes and pin the oracle restatement bit-for-bit.  The
// reference's xq_* C ABI is exported by its own session.cpp in the same library.
#include "kernels.hpp"

#include <cstdint>
#include <cstring>
#include <vector>

namespace {
xq::kernels::QuantizedMatrix wrap(const uint8_t* packed, const float* scales, const float* zeros, int rows, int cols,
                                  int group, int affine) {
    xq::kernels::QuantizedMatrix m;
    m.rows = rows;
    m.cols = cols;
    m.bits = 4;
    m.group_size = group;
    m.affine_asymmetric = affine != 0;
    const size_t row_bytes = (static_cast<size_t>(cols) + 1) / 2;
    const size_t groups = static_cast<size_t>((cols + group - 1) / group);
    m.packed.assign(packed, packed + row_bytes * rows);
    m.scales.assign(scales, scales + groups * rows);
    m.zeros.assign(zeros, zeros + groups * rows);
    m.bias.assign(static_cast<size_t>(rows), 0.0f);
    return m;
}
}  // namespace

extern "C" {

void ref_gemv_w4a16(const uint8_t* packed, const float* scales, const float* zeros, int rows, int cols, int group,
                    int affine, const float* x, float* y) {
    const auto m = wrap(packed, scales, zeros, rows, cols, group, affine);
    xq::kernels::gemvW4A16Neon(m, x, y);
}

int ref_gemv_w4a16_argmax(const uint8_t* packed, const float* scales, const float* zeros, int rows, int cols,
                          int group, int affine, const float* x, float* best) {
    const auto m = wrap(packed, scales, zeros, rows, cols, group, affine);
    return xq::kernels::gemvW4A16ArgmaxNeon(m, x, best);
}

void ref_gemv_textbook(const uint8_t* packed, const float* scales, const float* zeros, int rows, int cols, int group,
                       int affine, const float* x, float* y) {
    const auto m = wrap(packed, scales, zeros, rows, cols, group, affine);
    xq::kernels::gemvLowBitReference(m, x, y);
}

// The reference's W3A16 / W2A16 kernels (and gemvLowBitReference for other widths)
// on a bitstream matrix.
void ref_gemv_lowbit(const uint8_t* packed, const float* scales, const float* zeros, int rows, int cols, int group,
                     int bits, int affine, const float* x, float* y) {
    xq::kernels::QuantizedMatrix m;
    m.rows = rows;
    m.cols = cols;
    m.bits = bits;
    m.group_size = group;
    m.affine_asymmetric = affine != 0;
    const size_t groups = static_cast<size_t>((cols + group - 1) / group) * rows;
    m.packed.assign(packed, packed + (static_cast<size_t>(rows) * cols * bits + 7) / 8);
    m.scales.assign(scales, scales + groups);
    m.zeros.assign(zeros, zeros + groups);
    m.bias.assign(static_cast<size_t>(rows), 0.0f);
    if (bits == 3)
        xq::kernels::gemvW3A16Neon(m, x, y);
    else if (bits == 2)
        xq::kernels::gemvW2A16Neon(m, x, y);
    else
        xq::kernels::gemvLowBitReference(m, x, y);
}

void ref_quantize_lowbit(const float* w, int rows, int cols, int bits, int group, uint8_t* packed_out,
                         float* scales_out, float* zeros_out) {
    const auto q = xq::kernels::quantizeLowBit(w, rows, cols, bits, group);
    std::memcpy(packed_out, q.packed.data(), q.packed.size());
    std::memcpy(scales_out, q.scales.data(), q.scales.size() * sizeof(float));
    std::memcpy(zeros_out, q.zeros.data(), q.zeros.size() * sizeof(float));
}

void ref_rmsnorm(const float* x, const float* w, int n, float eps, float* y) {
    xq::kernels::rmsnormReference(x, w, n, eps, y);
}

void ref_rope(float* q, float* k, int heads, int hd, int pos, float theta) {
    xq::kernels::ropeReference(q, k, heads, hd, pos, theta);
}

void ref_attention(const float* q, const float* kc, const float* vc, int ctx, int kvh, int qh, int hd, float* out) {
    xq::kernels::attentionDecodeReference(q, kc, vc, ctx, kvh, qh, hd, out);
}

void ref_gated_delta(const float* q, const float* k, const float* v, float beta, float gate, int dk, int dv, float* S,
                     float* out) {
    xq::kernels::gatedDeltaDecodeReference(q, k, v, beta, gate, dk, dv, S, out);
}

}  // extern "C"
