// xqhip_api.hip - the thin C ABI of libxqhip.so (declared in include/xqhip.h):
// device and memory management, weight repacking/upload and kernel launchers.
#include "xqhip.h"
#include "xqhip_common.hpp"
#include "xqhip_kernels.hpp"

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>


namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int check(hipError_t e, const char* what) {
    if (e == hipSuccess) return XQHIP_OK;
    return fail(XQHIP_EDEVICE, "%s: %s", what, hipGetErrorString(e));
}

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

int env_int(const char* name, int dflt) {
    const char* v = std::getenv(name);
    if (!v || !*v) return dflt;
    return std::atoi(v);
}

// Blocks per GEMV launch: enough waves to cover HBM latency while each wave
// handles several row batches, so the per-block activation staging is amortised.
int gemv_block_cap() {
    static const int cap = env_int("XQHIP_GEMV_MAX_BLOCKS", 1024);
    return cap > 0 ? cap : 1024;
}

constexpr int kArgmaxMaxBlocks = 2048;

uint16_t f32_to_f16_bits(float f, bool* exact) {
    const _Float16 h = static_cast<_Float16>(f);
    *exact = static_cast<float>(h) == f;
    return __builtin_bit_cast(uint16_t, h);
}

__global__ void fill_u8_kernel(uint8_t* p, uint8_t v, size_t n) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = v;
}

}  // namespace

extern "C" {

const char* xqhip_last_error(void) { return g_err.c_str(); }

int xqhip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

int xqhip_set_device(int device) { return check(hipSetDevice(device), "hipSetDevice"); }

int xqhip_device_name(char* out, size_t capacity) {
    int dev = 0;
    hipDeviceProp_t prop;
    if (int rc = check(hipGetDevice(&dev), "hipGetDevice")) return rc;
    if (int rc = check(hipGetDeviceProperties(&prop, dev), "hipGetDeviceProperties")) return rc;
    std::snprintf(out, capacity, "%s (%s, %d CUs)", prop.name, prop.gcnArchName, prop.multiProcessorCount);
    return XQHIP_OK;
}

int xqhip_malloc(void** ptr, size_t bytes) {
    if (!ptr) return fail(XQHIP_EINVAL, "xqhip_malloc: null out pointer");
    *ptr = nullptr;
    if (bytes == 0) return XQHIP_OK;
    hipError_t e = hipMalloc(ptr, bytes);
    if (e == hipErrorOutOfMemory) return fail(XQHIP_ENOMEM, "hipMalloc(%zu): out of memory", bytes);
    return check(e, "hipMalloc");
}

int xqhip_free(void* ptr) { return ptr ? check(hipFree(ptr), "hipFree") : XQHIP_OK; }

int xqhip_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return XQHIP_OK;
    if (int rc = check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)), "memcpy h2d"))
        return rc;
    return check(hipStreamSynchronize(as_stream(stream)), "memcpy h2d sync");
}

int xqhip_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return XQHIP_OK;
    if (int rc = check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream)), "memcpy d2h"))
        return rc;
    return check(hipStreamSynchronize(as_stream(stream)), "memcpy d2h sync");
}

int xqhip_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return XQHIP_OK;
    return check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)), "memcpy d2d");
}

int xqhip_fill_u8(void* dst, uint8_t value, size_t bytes, void* stream) {
    if (bytes == 0) return XQHIP_OK;
    const size_t blocks = std::min<size_t>((bytes + 255) / 256, 4096);
    hipLaunchKernelGGL(fill_u8_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, as_stream(stream),
                       static_cast<uint8_t*>(dst), value, bytes);
    return check(hipGetLastError(), "fill_u8");
}

int xqhip_stream_synchronize(void* stream) { return check(hipStreamSynchronize(as_stream(stream)), "stream sync"); }
int xqhip_device_synchronize(void) { return check(hipDeviceSynchronize(), "device sync"); }

int xqhip_event_create(void** ev) {
    hipEvent_t e;
    if (int rc = check(hipEventCreate(&e), "hipEventCreate")) return rc;
    *ev = e;
    return XQHIP_OK;
}
int xqhip_event_destroy(void* ev) { return check(hipEventDestroy(static_cast<hipEvent_t>(ev)), "hipEventDestroy"); }
int xqhip_event_record(void* ev, void* stream) {
    return check(hipEventRecord(static_cast<hipEvent_t>(ev), as_stream(stream)), "hipEventRecord");
}
int xqhip_event_elapsed_ms(void* start, void* stop, float* ms) {
    if (int rc = check(hipEventSynchronize(static_cast<hipEvent_t>(stop)), "hipEventSynchronize")) return rc;
    return check(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)),
                 "hipEventElapsedTime");
}

// Reference layout (custom_model.cpp:218-262) -> device layout.
// TILED64: within each row the 16-byte half-groups are reordered so that, for
// chunk c of up to 64 groups (gc of them), half h of group c*64+l lands at
// c*2048 + h*gc*16 + l*16: one wave-wide 16-byte load per half is 1 KiB
// contiguous.  Nibble order inside each 16 bytes is unchanged (even column in
// the low nibble).  Metadata becomes one u32 per group: fp16 scale | fp16 zero<<16.
int xqhip_w4_upload(const uint8_t* packed, const float* scales, const float* zeros, int rows, int cols, int group,
                    int affine, xqhip_w4* out) {
    if (!packed || !scales || !zeros || !out || rows <= 0 || cols <= 0 || group <= 0)
        return fail(XQHIP_EINVAL, "xqhip_w4_upload: bad arguments (rows=%d cols=%d group=%d)", rows, cols, group);
    std::memset(out, 0, sizeof(*out));
    out->rows = rows;
    out->cols = cols;
    out->group = group;
    out->affine = affine ? 1 : 0;
    const size_t row_bytes = (static_cast<size_t>(cols) + 1) / 2;
    const int G = (cols + group - 1) / group;
    const bool tiled = group == 64 && cols % 64 == 0 && G <= 256;
    out->layout = tiled ? XQHIP_LAYOUT_TILED64 : XQHIP_LAYOUT_GENERIC;
    out->nib_bytes = row_bytes * rows;
    std::vector<uint8_t> nib_host;
    std::vector<uint32_t> meta_u32;
    std::vector<float> meta_f32;
    const void* nib_src = packed;
    const void* meta_src = nullptr;
    if (tiled) {
        nib_host.resize(out->nib_bytes);
        for (int r = 0; r < rows; ++r) {
            const uint8_t* src = packed + static_cast<size_t>(r) * row_bytes;
            uint8_t* dst = nib_host.data() + static_cast<size_t>(r) * row_bytes;
            for (int g = 0; g < G; ++g) {
                const int c = g / 64, l = g % 64;
                const int gcnt = std::min(64, G - c * 64);
                for (int h = 0; h < 2; ++h)
                    std::memcpy(dst + c * 2048 + h * gcnt * 16 + l * 16, src + g * 32 + h * 16, 16);
            }
        }
        nib_src = nib_host.data();
        meta_u32.resize(static_cast<size_t>(rows) * G);
        int inexact = 0;
        for (size_t i = 0; i < meta_u32.size(); ++i) {
            bool e1, e2;
            const uint16_t s = f32_to_f16_bits(scales[i], &e1);
            const uint16_t z = f32_to_f16_bits(zeros[i], &e2);
            inexact += (!e1) + (!e2);
            meta_u32[i] = static_cast<uint32_t>(s) | (static_cast<uint32_t>(z) << 16);
        }
        out->inexact_meta = inexact;
        out->meta_bytes = meta_u32.size() * 4;
        meta_src = meta_u32.data();
    } else {
        meta_f32.resize(static_cast<size_t>(rows) * G * 2);
        std::memcpy(meta_f32.data(), scales, static_cast<size_t>(rows) * G * 4);
        std::memcpy(meta_f32.data() + static_cast<size_t>(rows) * G, zeros, static_cast<size_t>(rows) * G * 4);
        out->meta_bytes = meta_f32.size() * 4;
        meta_src = meta_f32.data();
    }
    if (int rc = xqhip_malloc(&out->nib, out->nib_bytes)) return rc;
    if (int rc = xqhip_malloc(&out->meta, out->meta_bytes)) {
        xqhip_free(out->nib);
        out->nib = nullptr;
        return rc;
    }
    if (int rc = check(hipMemcpy(out->nib, nib_src, out->nib_bytes, hipMemcpyHostToDevice), "upload nibbles"))
        return rc;
    return check(hipMemcpy(out->meta, meta_src, out->meta_bytes, hipMemcpyHostToDevice), "upload metadata");
}

int xqhip_w4_free(xqhip_w4* w) {
    if (!w) return XQHIP_OK;
    int rc = xqhip_free(w->nib);
    int rc2 = xqhip_free(w->meta);
    w->nib = w->meta = nullptr;
    return rc ? rc : rc2;
}

uint64_t xqhip_w4_weight_bytes(const xqhip_w4* w) { return w ? w->nib_bytes + w->meta_bytes : 0; }

static int validate_w4(const xqhip_w4* w, const char* who) {
    if (!w || !w->nib || !w->meta || w->rows <= 0 || w->cols <= 0)
        return fail(XQHIP_EINVAL, "%s: matrix is not uploaded", who);
    if (w->layout == XQHIP_LAYOUT_TILED64 && (w->group != 64 || w->cols % 64 != 0 || w->cols / 64 > 256))
        return fail(XQHIP_EINVAL, "%s: inconsistent TILED64 matrix %dx%d g%d", who, w->rows, w->cols, w->group);
    return XQHIP_OK;
}

int xqhip_gemv_w4a16(const xqhip_w4* w, const void* x, int x_type, const float* norm_w, float eps, void* y,
                     int y_type, int epilogue, void* stream) {
    if (int rc = validate_w4(w, "xqhip_gemv_w4a16")) return rc;
    if (!x || !y) return fail(XQHIP_EINVAL, "xqhip_gemv_w4a16: null vector");
    if (epilogue < XQHIP_EPI_STORE || epilogue > XQHIP_EPI_SILU_PAIR)
        return fail(XQHIP_EINVAL, "xqhip_gemv_w4a16: unknown epilogue %d", epilogue);
    if (epilogue == XQHIP_EPI_SILU_PAIR && (w->rows % 2 != 0))
        return fail(XQHIP_EINVAL, "xqhip_gemv_w4a16: SILU_PAIR needs an even row count");
    if (epilogue != XQHIP_EPI_STORE && y_type != XQHIP_F32)
        return fail(XQHIP_EINVAL, "xqhip_gemv_w4a16: ADD/SILU_PAIR write fp32");
    xqhip::GemvLaunch p{};
    p.nib = static_cast<const uint8_t*>(w->nib);
    p.meta = w->meta;
    p.rows = w->rows;
    p.cols = w->cols;
    p.group = w->group;
    p.affine = w->affine;
    p.layout = w->layout;
    p.x = x;
    p.x_f16 = x_type == XQHIP_F16;
    p.norm_w = norm_w;
    p.eps = eps;
    p.y = y;
    p.y_f16 = y_type == XQHIP_F16;
    p.epi = epilogue;
    p.max_blocks = gemv_block_cap();
    return check(xqhip::launch_gemv(p, as_stream(stream)), "gemv_w4a16 launch");
}

size_t xqhip_argmax_workspace_bytes(int rows) {
    (void)rows;
    return 256 + sizeof(uint64_t) * kArgmaxMaxBlocks;
}

int xqhip_gemv_w4a16_argmax(const xqhip_w4* w, const void* x, int x_type, const float* norm_w, float eps,
                            void* workspace, int32_t* out_index, float* out_value, void* stream) {
    if (int rc = validate_w4(w, "xqhip_gemv_w4a16_argmax")) return rc;
    if (!x || !workspace || !out_index || !out_value)
        return fail(XQHIP_EINVAL, "xqhip_gemv_w4a16_argmax: null argument");
    xqhip::GemvLaunch p{};
    p.nib = static_cast<const uint8_t*>(w->nib);
    p.meta = w->meta;
    p.rows = w->rows;
    p.cols = w->cols;
    p.group = w->group;
    p.affine = w->affine;
    p.layout = w->layout;
    p.x = x;
    p.x_f16 = x_type == XQHIP_F16;
    p.norm_w = norm_w;
    p.eps = eps;
    p.epi = 3;
    p.counter = static_cast<uint32_t*>(workspace);
    p.partial = reinterpret_cast<uint64_t*>(static_cast<uint8_t*>(workspace) + 256);
    p.out_idx = out_index;
    p.out_val = out_value;
    p.max_blocks = kArgmaxMaxBlocks;
    return check(xqhip::launch_gemv(p, as_stream(stream)), "gemv_w4a16_argmax launch");
}

}  // extern "C"
