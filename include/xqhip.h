/* xqhip.h - thin C ABI between the C++ host runtime (libxqwen35.so) and the
 * hand-written gfx950 HIP kernels (libxqhip.so).
 *
 * Everything here is plain C: device pointers are `void*`, streams are `void*`
 * (a hipStream_t; NULL means the library's own stream on the current device),
 * every call returns 0 on success or a negative XQHIP_E* code, with the message
 * available from xqhip_last_error().  No torch or HIP types appear in the
 * signatures.
 *
 * This layer is the MI355X replacement of the reference's per-op GPU seam
 * (customlib/runtime/vulkan_backend.hpp:21-121, `bool op(..., timing, error)`),
 * re-designed so that weights, KV cache, recurrent state and activations stay
 * resident in HBM and no op uploads or downloads per call.  The CPU kernel each
 * entry point replaces is cited beside it.
 */
#ifndef XQHIP_H_
#define XQHIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define XQHIP_API __attribute__((visibility("default")))

enum {
    XQHIP_OK = 0,
    XQHIP_EINVAL = -1,   /* bad argument or unsupported shape */
    XQHIP_EDEVICE = -2,  /* HIP runtime error (message in xqhip_last_error) */
    XQHIP_ENOMEM = -3
};

/* Element types of activation vectors. */
enum { XQHIP_F32 = 0, XQHIP_F16 = 1 };

/* Epilogues fused into the GEMV store. */
enum {
    XQHIP_EPI_STORE = 0,     /* y[r] = acc                                           */
    XQHIP_EPI_ADD = 1,       /* y[r] += acc (fp32 residual add, custom_model.cpp:294) */
    XQHIP_EPI_SILU_PAIR = 2  /* rows interleaved (gate_i, up_i): y[i] = silu(g)*u    */
};

/* Device layouts of a W4A16 matrix. */
enum {
    XQHIP_LAYOUT_TILED64 = 0, /* group 64, cols % 64 == 0: 16-byte chunks of each row
                                 permuted so a wave's loads are contiguous; per-group
                                 (fp16 scale, fp16 zero) packed in one u32          */
    XQHIP_LAYOUT_GENERIC = 1  /* any group size: reference row-major nibbles, fp32
                                 scales and zeros (used only for tiny shapes)        */
};

/* A W4A16 matrix resident in HBM.  Semantics of the reference QuantizedMatrix
 * (customlib/kernels/kernels.hpp:11-21): rows x cols unsigned 4-bit codes, even
 * column in the low nibble, one (scale, zero) per `group` columns of a row;
 * affine == 0: w = (q - zero) * scale (XQ4 version 1), affine == 1:
 * w = q * scale + zero (version 2). */
typedef struct xqhip_w4 {
    int32_t rows;
    int32_t cols;
    int32_t group;
    int32_t affine;
    int32_t layout;
    int32_t inexact_meta; /* scales/zeros not exactly representable in fp16 (TILED64) */
    void* nib;            /* device nibbles                                       */
    void* meta;           /* device per-group metadata                            */
    uint64_t nib_bytes;
    uint64_t meta_bytes;
} xqhip_w4;

/* ---- device, memory, streams, events ---------------------------------- */
XQHIP_API const char* xqhip_last_error(void);
XQHIP_API int xqhip_device_count(void);
XQHIP_API int xqhip_set_device(int device);
XQHIP_API int xqhip_device_name(char* out, size_t capacity);
XQHIP_API int xqhip_malloc(void** ptr, size_t bytes);
XQHIP_API int xqhip_free(void* ptr);
XQHIP_API int xqhip_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
XQHIP_API int xqhip_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
XQHIP_API int xqhip_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
/* Byte fill done by a kernel (safe inside captured graphs). */
XQHIP_API int xqhip_fill_u8(void* dst, uint8_t value, size_t bytes, void* stream);
XQHIP_API int xqhip_stream_synchronize(void* stream);
XQHIP_API int xqhip_device_synchronize(void);
XQHIP_API int xqhip_event_create(void** ev);
XQHIP_API int xqhip_event_destroy(void* ev);
XQHIP_API int xqhip_event_record(void* ev, void* stream);
XQHIP_API int xqhip_event_elapsed_ms(void* start, void* stop, float* ms);

/* ---- W4A16 weights ----------------------------------------------------- */
/* Repack a reference-format matrix (packed[rows][ceil(cols/2)], fp32
 * scales/zeros[rows][ceil(cols/group)], as read by custom_model.cpp:218-262)
 * into the device layout and upload it.  Chooses TILED64 when group == 64 and
 * cols % 64 == 0, else GENERIC. */
XQHIP_API int xqhip_w4_upload(const uint8_t* packed, const float* scales, const float* zeros, int rows, int cols,
                              int group, int affine, xqhip_w4* out);
XQHIP_API int xqhip_w4_free(xqhip_w4* w);
/* Bytes the GEMV must read per call for this matrix (nibbles + metadata). */
XQHIP_API uint64_t xqhip_w4_weight_bytes(const xqhip_w4* w);

/* ---- fused dequant GEMV ------------------------------------------------ */
/* y = W x, replacing gemvW4A16Neon
 * (customlib/kernels/generated/arm64_neon/xq_gemv_w4a16_neon.cpp:259-291).
 * x: `cols` values of x_type.  If norm_w != NULL the kernel first applies the
 * RMSNorm of ref_rmsnorm.cpp:8-17 to x (x * inv * norm_w, eps) in its prologue.
 * y: `rows` values of y_type (EPI_SILU_PAIR: rows/2 values).  Inputs must not
 * alias outputs. */
XQHIP_API int xqhip_gemv_w4a16(const xqhip_w4* w, const void* x, int x_type, const float* norm_w, float eps,
                               void* y, int y_type, int epilogue, void* stream);

/* Workspace bytes xqhip_gemv_w4a16_argmax needs for a matrix of `rows` rows. */
XQHIP_API size_t xqhip_argmax_workspace_bytes(int rows);
/* Greedy lm_head: argmax_r (W x)[r] without materialising logits, ties to the
 * lowest row, replacing gemvW4A16ArgmaxNeon (xq_gemv_w4a16_neon.cpp:293-348).
 * Block-level argmax, then the last block to finish reduces the partials.
 * workspace: device memory of xqhip_argmax_workspace_bytes(rows), zeroed once
 * before first use (the kernel leaves it ready for the next call).
 * out_index / out_value: device int32 / float. */
XQHIP_API int xqhip_gemv_w4a16_argmax(const xqhip_w4* w, const void* x, int x_type, const float* norm_w, float eps,
                                      void* workspace, int32_t* out_index, float* out_value, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* XQHIP_H_ */
