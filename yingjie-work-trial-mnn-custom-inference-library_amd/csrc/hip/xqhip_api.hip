// xqhip_api.hip - the thin C ABI of libxqhip.so (declared in include/xqhip.h):
// device and memory management, weight repacking/upload and kernel launchers.
#include "xqhip.h"
#include "xqhip_common.hpp"
#include "xqhip_kernels.hpp"

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

// Device memory of the library itself for xqhip_gemv_w4a16_argmax_static: the
// per-block argmax keys (uint64 each, at most kArgmaxMaxBlocks blocks), 16 KiB
// on every device the library runs on, held until the process ends.  Host code
// never uses this name as an address: it reads each device's copy's address
// once with hipGetSymbolAddress (static_scratch below) and passes that.
static __device__ __align__(256) uint64_t scratch[xqhip::kArgmaxMaxBlocks];

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

// Blocks per tiled GEMV launch: 0 lets the launcher use the device's resident
// block count; XQHIP_GEMV_MAX_BLOCKS overrides it (launch-shape sweeps).
int gemv_block_cap() {
    static const int cap = env_int("XQHIP_GEMV_MAX_BLOCKS", 0);
    return cap > 0 ? cap : 0;
}

using xqhip::kArgmaxMaxBlocks;

}  // namespace

// Error text of entry points defined in other files of the library.
namespace xqhip {
void set_last_error(const std::string& msg) { g_err = msg; }
}  // namespace xqhip

namespace {

uint16_t f32_to_f16_bits(float f, bool* exact) {
    const _Float16 h = static_cast<_Float16>(f);
    *exact = static_cast<float>(h) == f;
    return __builtin_bit_cast(uint16_t, h);
}

__global__ void fill_u8_kernel(uint8_t* p, uint8_t v, size_t n) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = v;
}

// Plain device copy in one dispatch: 16-byte elements over a grid-stride
// loop, then the tail bytes.
__global__ void copy_u32x4_kernel(uint4* __restrict__ dst, const uint4* __restrict__ src, size_t n16,
                                  uint8_t* __restrict__ dst_tail, const uint8_t* __restrict__ src_tail, size_t tail) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    const size_t t = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    for (size_t i = t; i < n16; i += stride) dst[i] = src[i];
    if (t < tail) dst_tail[t] = src_tail[t];
}

// Address of `scratch` on the current device, resolved once per device with
// that device current.  A launch stream must belong to that device (its
// kernels would otherwise write another device's copy).  nullptr (and the
// error set) on failure.
constexpr int kMaxDevices = 64;
void* static_scratch(hipStream_t stream = nullptr) {
    static std::mutex mu;
    static void* addr[kMaxDevices] = {};
    int dev = 0;
    if (check(hipGetDevice(&dev), "hipGetDevice")) return nullptr;
    if (stream) {
        int sdev = 0;
        if (check(hipStreamGetDevice(stream, &sdev), "hipStreamGetDevice")) return nullptr;
        if (sdev != dev) {
            fail(XQHIP_EINVAL, "the stream belongs to device %d, the current device is %d", sdev, dev);
            return nullptr;
        }
    }
    if (dev < 0 || dev >= kMaxDevices) {
        fail(XQHIP_EDEVICE, "device %d beyond the %d devices the static scratch covers", dev, kMaxDevices);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void* ptr = nullptr;
        if (check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)")) return nullptr;
        addr[dev] = ptr;
    }
    return addr[dev];
}

}  // namespace

extern "C" {

const char* xqhip_last_error(void) { return g_err.c_str(); }

int xqhip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

int xqhip_set_device(int device) {
    if (int rc = check(hipSetDevice(device), "hipSetDevice")) return rc;
    return static_scratch() ? XQHIP_OK : XQHIP_EDEVICE;  // set-up of the no-allocation entry point
}

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

int xqhip_memcpy_h2d_async(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return XQHIP_OK;
    return check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)), "memcpy h2d async");
}

int xqhip_memcpy_d2h_async(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return XQHIP_OK;
    return check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream)), "memcpy d2h async");
}

int xqhip_host_alloc(void** ptr, size_t bytes) {
    if (!ptr) return fail(XQHIP_EINVAL, "xqhip_host_alloc: null out pointer");
    return check(hipHostMalloc(ptr, bytes == 0 ? 1 : bytes, hipHostMallocDefault), "hipHostMalloc");
}

int xqhip_host_alloc_coherent(void** ptr, size_t bytes) {
    if (!ptr) return fail(XQHIP_EINVAL, "xqhip_host_alloc_coherent: null out pointer");
    return check(hipHostMalloc(ptr, bytes == 0 ? 1 : bytes, hipHostMallocMapped | hipHostMallocCoherent),
                 "hipHostMalloc(coherent)");
}

int xqhip_host_free(void* ptr) { return ptr ? check(hipHostFree(ptr), "hipHostFree") : XQHIP_OK; }

int xqhip_fill_u8(void* dst, uint8_t value, size_t bytes, void* stream) {
    if (bytes == 0) return XQHIP_OK;
    const size_t blocks = std::min<size_t>((bytes + 255) / 256, 4096);
    hipLaunchKernelGGL(fill_u8_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, as_stream(stream),
                       static_cast<uint8_t*>(dst), value, bytes);
    return check(hipGetLastError(), "fill_u8");
}

int xqhip_copy(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return XQHIP_OK;
    if (!dst || !src) return fail(XQHIP_EINVAL, "xqhip_copy: null pointer");
    if ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) & 15u)
        return fail(XQHIP_EINVAL, "xqhip_copy: pointers must be 16-byte aligned");
    const size_t n16 = bytes / 16, tail = bytes % 16;
    const size_t blocks = std::max<size_t>(1, std::min<size_t>((n16 + 255) / 256, 4096));
    hipLaunchKernelGGL(copy_u32x4_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, as_stream(stream),
                       static_cast<uint4*>(dst), static_cast<const uint4*>(src), n16,
                       static_cast<uint8_t*>(dst) + n16 * 16, static_cast<const uint8_t*>(src) + n16 * 16, tail);
    return check(hipGetLastError(), "copy");
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
int xqhip_event_synchronize(void* ev) {
    return check(hipEventSynchronize(static_cast<hipEvent_t>(ev)), "hipEventSynchronize");
}

int xqhip_stream_query(void* stream) {
    const hipError_t e = hipStreamQuery(as_stream(stream));
    if (e == hipSuccess) return 1;
    if (e == hipErrorNotReady) return 0;
    return check(e, "hipStreamQuery");
}

int xqhip_event_query(void* ev) {
    const hipError_t e = hipEventQuery(static_cast<hipEvent_t>(ev));
    if (e == hipSuccess) return 1;
    if (e == hipErrorNotReady) return 0;
    return check(e, "hipEventQuery");
}

int xqhip_event_elapsed_ms(void* start, void* stop, float* ms) {
    if (int rc = check(hipEventSynchronize(static_cast<hipEvent_t>(stop)), "hipEventSynchronize")) return rc;
    const hipError_t e = hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop));
    if (e != hipSuccess) (void)hipGetLastError();  // not left behind for the next launch's error check
    return check(e, "hipEventElapsedTime");
}

int xqhip_timestamp(uint64_t* slot, void* stream) {
    if (!slot) return fail(XQHIP_EINVAL, "xqhip_timestamp: null slot");
    return check(xqhip::launch_timestamp(slot, as_stream(stream)), "timestamp launch");
}

// fp16 (scale, zero) pairs of the TILED64 layout; returns the count of inexact values.
static int pack_meta_f16(const float* scales, const float* zeros, size_t n, std::vector<uint32_t>* out) {
    out->resize(n);
    int inexact = 0;
    for (size_t i = 0; i < n; ++i) {
        bool e1, e2;
        const uint16_t s = f32_to_f16_bits(scales[i], &e1);
        const uint16_t z = f32_to_f16_bits(zeros[i], &e2);
        inexact += (!e1) + (!e2);
        (*out)[i] = static_cast<uint32_t>(s) | (static_cast<uint32_t>(z) << 16);
    }
    return inexact;
}

// 1 when w = (q - 8) s for every group (format v1 with zero 8): the GEMM's
// zero-point term (8 - z) s x-sum is then identically 0.
static int32_t zero_is_8(const float* zeros, size_t n, int affine) {
    if (affine) return 0;
    for (size_t i = 0; i < n; ++i)
        if (zeros[i] != 8.0f) return 0;
    return 1;
}

// 1 when every zero is an integer 0..15 in format v1 (the reference packer's
// asymmetric quantiser, pack_qwen35_xq4_numpy.py:218-247): the zero then fits
// a 4-bit code exactly.
static bool zeros_are_codes(const float* zeros, size_t n, int affine) {
    if (affine) return false;
    for (size_t i = 0; i < n; ++i)
        if (!(zeros[i] >= 0.0f && zeros[i] <= 15.0f && zeros[i] == std::floor(zeros[i]))) return false;
    return true;
}

// TILED64_F32S_Z4 metadata: the fp32 scales [rows][G], then per row
// ceil(G / 8) u32 words of 4-bit zero codes (nibble k of word j = group 8 j + k).
static void pack_meta_z4(const float* scales, const float* zeros, int rows, int G, std::vector<uint32_t>* out) {
    const size_t n = static_cast<size_t>(rows) * G, zw = (static_cast<size_t>(G) + 7) / 8;
    out->assign(n + static_cast<size_t>(rows) * zw, 0u);
    std::memcpy(out->data(), scales, n * 4);
    for (int r = 0; r < rows; ++r)
        for (int g = 0; g < G; ++g) {
            const uint32_t z = static_cast<uint32_t>(zeros[static_cast<size_t>(r) * G + g]);
            (*out)[n + r * zw + g / 8] |= z << (4 * (g % 8));
        }
}

// fp32 (scale, zero) pairs of the TILED64_F32META layout, two words per group.
static void pack_meta_f32(const float* scales, const float* zeros, size_t n, std::vector<uint32_t>* out) {
    out->resize(2 * n);
    for (size_t i = 0; i < n; ++i) {
        std::memcpy(&(*out)[2 * i], &scales[i], 4);
        std::memcpy(&(*out)[2 * i + 1], &zeros[i], 4);
    }
}

// Reference layout (custom_model.cpp:218-262) -> device layout.
// TILED64: within each row the 16-byte half-groups are reordered so that, for
// chunk c of up to 64 groups (gc of them), half h of group c*64+l lands at
// c*2048 + h*gc*16 + l*16: one wave-wide 16-byte load per half is 1 KiB
// contiguous.  Nibble order inside each 16 bytes is unchanged (even column in
// the low nibble); every code q is stored as q ^ 8.  Metadata becomes one u32
// per group: fp16 scale | fp16 zero<<16; the fp16 scale alone (u16) when every
// zero is 8 (format v1); when fp16 cannot hold a value, the fp32 scale with a
// 4-bit zero code if every zero is an integer 0..15 (format v1), else the fp32
// pair.
int xqhip_w4_upload(const uint8_t* packed, const float* scales, const float* zeros, int rows, int cols, int group,
                    int affine, xqhip_w4* out) {
    if (!packed || !scales || !zeros || !out || rows <= 0 || cols <= 0 || group <= 0)
        return fail(XQHIP_EINVAL, "xqhip_w4_upload: bad arguments (rows=%d cols=%d group=%d)", rows, cols, group);
    std::memset(out, 0, sizeof(*out));
    out->rows = rows;
    out->cols = cols;
    out->group = group;
    out->affine = affine ? 1 : 0;
    out->bits = 4;
    const size_t row_bytes = (static_cast<size_t>(cols) + 1) / 2;
    const int G = (cols + group - 1) / group;
    out->zero_is_8 = zero_is_8(zeros, static_cast<size_t>(rows) * G, out->affine);
    const bool tiled = group == 64 && cols % 64 == 0 && G <= 256;
    out->layout = tiled ? XQHIP_LAYOUT_TILED64 : XQHIP_LAYOUT_GENERIC;
    out->nib_bytes = row_bytes * rows;
    std::vector<uint8_t> nib_host;
    std::vector<uint32_t> meta_u32;
    std::vector<uint16_t> meta_u16;
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
                for (int h = 0; h < 2; ++h) {
                    // each code q stored as q ^ 8 = (q - 8) in signed 4-bit, the operand of v_dot8_i32_i4
                    uint8_t* d16 = dst + c * 2048 + h * gcnt * 16 + l * 16;
                    const uint8_t* s16 = src + g * 32 + h * 16;
                    for (int i = 0; i < 16; ++i) d16[i] = static_cast<uint8_t>(s16[i] ^ 0x88u);
                }
            }
        }
        nib_src = nib_host.data();
        const size_t n_meta = static_cast<size_t>(rows) * G;
        out->inexact_meta = pack_meta_f16(scales, zeros, n_meta, &meta_u32);
        if (out->inexact_meta > 0 && zeros_are_codes(zeros, n_meta, out->affine)) {
            // the reference's fp32 scales, the integer zeros as 4-bit codes
            pack_meta_z4(scales, zeros, rows, G, &meta_u32);
            out->layout = XQHIP_LAYOUT_TILED64_F32S_Z4;
            out->meta_bytes = meta_u32.size() * 4;
        } else if (out->inexact_meta > 0) {  // keep the reference's fp32 values
            pack_meta_f32(scales, zeros, n_meta, &meta_u32);
            out->layout = XQHIP_LAYOUT_TILED64_F32META;
            out->meta_bytes = meta_u32.size() * 4;
        } else if (out->zero_is_8) {  // the zero point is implied: the fp16 scales alone
            meta_u16.resize(n_meta);
            for (size_t i = 0; i < n_meta; ++i) meta_u16[i] = static_cast<uint16_t>(meta_u32[i] & 0xFFFFu);
            out->layout = XQHIP_LAYOUT_TILED64_SCALE16;
            out->meta_bytes = meta_u16.size() * 2;
        } else {
            out->meta_bytes = meta_u32.size() * 4;
        }
        meta_src = out->layout == XQHIP_LAYOUT_TILED64_SCALE16 ? static_cast<const void*>(meta_u16.data())
                                                                : static_cast<const void*>(meta_u32.data());
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

static int upload_pair(xqhip_w4* out, const void* nib, const void* meta) {
    if (int rc = xqhip_malloc(&out->nib, out->nib_bytes)) return rc;
    if (int rc = xqhip_malloc(&out->meta, out->meta_bytes)) {
        xqhip_free(out->nib);
        out->nib = nullptr;
        return rc;
    }
    if (int rc = check(hipMemcpy(out->nib, nib, out->nib_bytes, hipMemcpyHostToDevice), "upload codes")) return rc;
    return check(hipMemcpy(out->meta, meta, out->meta_bytes, hipMemcpyHostToDevice), "upload metadata");
}

int xqhip_wlb_upload(const uint8_t* bitstream, const float* scales, const float* zeros, int rows, int cols, int group,
                     int bits, int affine, xqhip_w4* out) {
    if (!bitstream || !scales || !zeros || !out || rows <= 0 || cols <= 0 || group <= 0 || (bits != 2 && bits != 3))
        return fail(XQHIP_EINVAL, "xqhip_wlb_upload: bad arguments (rows=%d cols=%d group=%d bits=%d)", rows, cols,
                    group, bits);
    std::memset(out, 0, sizeof(*out));
    out->rows = rows;
    out->cols = cols;
    out->group = group;
    out->affine = affine ? 1 : 0;
    out->bits = bits;
    const int G = (cols + group - 1) / group;
    const size_t n_meta = static_cast<size_t>(rows) * G;
    const size_t total_bytes = (static_cast<size_t>(rows) * cols * bits + 7) / 8;
    out->zero_is_8 = zero_is_8(zeros, n_meta, out->affine);
    if (!(group == 64 && cols % 64 == 0 && G <= 256)) {
        // GENERIC: the bitstream as it is, fp32 scales then zeros
        out->layout = XQHIP_LAYOUT_GENERIC;
        out->nib_bytes = total_bytes;
        std::vector<float> meta(2 * n_meta);
        std::memcpy(meta.data(), scales, n_meta * 4);
        std::memcpy(meta.data() + n_meta, zeros, n_meta * 4);
        out->meta_bytes = meta.size() * 4;
        return upload_pair(out, bitstream, meta.data());
    }
    // TILED64: per 4096-column chunk, the groups' 16-byte two-bit planes, then (3 bits)
    // their 8-byte high-bit planes; the word layout is the one group_words() expands
    out->layout = XQHIP_LAYOUT_TILED64;
    const size_t row_bytes = static_cast<size_t>(cols / 8) * bits;
    out->nib_bytes = row_bytes * rows;
    std::vector<uint8_t> dev(out->nib_bytes, 0);
    auto code = [&](int r, int c) {
        const size_t bit = (static_cast<size_t>(r) * cols + c) * bits;
        const uint32_t lo = bitstream[bit >> 3], hi = (bit >> 3) + 1 < total_bytes ? bitstream[(bit >> 3) + 1] : 0u;
        return ((lo | (hi << 8)) >> (bit & 7)) & ((1u << bits) - 1u);
    };
    for (int r = 0; r < rows; ++r) {
        uint8_t* row = dev.data() + static_cast<size_t>(r) * row_bytes;
        for (int g = 0; g < G; ++g) {
            const int ch = g / 64, l = g % 64, gcnt = std::min(64, G - ch * 64);
            uint8_t* chunk = row + static_cast<size_t>(ch) * 512 * bits;
            uint32_t plane[4] = {0, 0, 0, 0}, high[2] = {0, 0};
            for (int j = 0; j < 8; ++j)      // word j: columns 8j .. 8j+7 of the group
                for (int i = 0; i < 8; ++i) {
                    const uint32_t q = code(r, g * 64 + 8 * j + i);
                    plane[j >> 1] |= (q & 3u) << (4 * i + 2 * (j & 1));
                    high[j >> 2] |= ((q >> 2) & 1u) << (4 * i + (j & 3));
                }
            std::memcpy(chunk + l * 16, plane, 16);
            if (bits == 3) std::memcpy(chunk + gcnt * 16 + l * 8, high, 8);
        }
    }
    std::vector<uint32_t> meta;
    out->inexact_meta = pack_meta_f16(scales, zeros, n_meta, &meta);
    if (out->inexact_meta > 0) {  // keep the reference's fp32 values
        pack_meta_f32(scales, zeros, n_meta, &meta);
        out->layout = XQHIP_LAYOUT_TILED64_F32META;
    }
    out->meta_bytes = meta.size() * 4;
    return upload_pair(out, dev.data(), meta.data());
}

uint64_t xqhip_w4_weight_bytes(const xqhip_w4* w) { return w ? w->nib_bytes + w->meta_bytes : 0; }

static int validate_w4(const xqhip_w4* w, const char* who) {
    if (!w || !w->nib || !w->meta || w->rows <= 0 || w->cols <= 0)
        return fail(XQHIP_EINVAL, "%s: matrix is not uploaded", who);
    if (w->layout != XQHIP_LAYOUT_TILED64 && w->layout != XQHIP_LAYOUT_GENERIC &&
        w->layout != XQHIP_LAYOUT_TILED64_F32META && w->layout != XQHIP_LAYOUT_TILED64_SCALE16 &&
        w->layout != XQHIP_LAYOUT_TILED64_F32S_Z4)
        return fail(XQHIP_EINVAL, "%s: unknown layout %d", who, w->layout);
    if (w->layout == XQHIP_LAYOUT_TILED64_SCALE16 && (w->bits != 4 || w->affine || !w->zero_is_8))
        return fail(XQHIP_EINVAL, "%s: the scale-only layout holds 4-bit format-v1 matrices with zero 8", who);
    if (w->layout == XQHIP_LAYOUT_TILED64_F32S_Z4 && (w->bits != 4 || w->affine))
        return fail(XQHIP_EINVAL, "%s: the 4-bit-zero layout holds 4-bit format-v1 matrices", who);
    if (w->layout != XQHIP_LAYOUT_GENERIC && (w->group != 64 || w->cols % 64 != 0 || w->cols / 64 > 256))
        return fail(XQHIP_EINVAL, "%s: inconsistent TILED64 matrix %dx%d g%d", who, w->rows, w->cols, w->group);
    if (w->bits != 4 && w->bits != 3 && w->bits != 2)
        return fail(XQHIP_EINVAL, "%s: unsupported code width %d", who, w->bits);
    return XQHIP_OK;
}

static xqhip::Prologue make_prologue(const xqhip_prologue* pro) {
    xqhip::Prologue p{};
    if (pro) {
        p.mode = pro->mode;
        p.w = pro->weight;
        p.z = pro->gate;
        p.head_dim = pro->head_dim;
        p.eps = pro->eps;
    }
    return p;
}

static_assert(XQHIP_PRO_GATED_HEAD_ACT == xqhip::PRO_GATED_ACT && XQHIP_PRO_GATED_HEAD == xqhip::PRO_GATED,
              "prologue modes");

// gated_act: whether the entry point takes XQHIP_PRO_GATED_HEAD_ACT (the GEMVs; the
// prefill GEMM prepares its activations with the reference's own silu)
static int validate_prologue(const xqhip_prologue* pro, int cols, const char* who, bool gated_act = true) {
    if (!pro || pro->mode == XQHIP_PRO_NONE) return XQHIP_OK;
    if (pro->mode == XQHIP_PRO_RMS && pro->weight) return XQHIP_OK;
    if ((pro->mode == XQHIP_PRO_GATED_HEAD || (gated_act && pro->mode == XQHIP_PRO_GATED_HEAD_ACT)) && pro->weight &&
        pro->gate && pro->head_dim > 0 && cols % pro->head_dim == 0 && cols / pro->head_dim <= xqhip::kMaxNormHeads)
        return XQHIP_OK;
    return fail(XQHIP_EINVAL, "%s: bad prologue (mode %d)", who, pro->mode);
}

// The TILED64 kernels read x and the prologue vectors with 16-byte loads.
static int validate_alignment(const xqhip_w4* w, const void* x, const xqhip_prologue* pro, const char* who) {
    if (w->layout == XQHIP_LAYOUT_GENERIC) return XQHIP_OK;
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (!a16(x)) return fail(XQHIP_EINVAL, "%s: x must be 16-byte aligned", who);
    if (pro && pro->mode != XQHIP_PRO_NONE && !a16(pro->weight))
        return fail(XQHIP_EINVAL, "%s: prologue weight must be 16-byte aligned", who);
    if (pro && (pro->mode == XQHIP_PRO_GATED_HEAD || pro->mode == XQHIP_PRO_GATED_HEAD_ACT) && !a16(pro->gate))
        return fail(XQHIP_EINVAL, "%s: prologue gate must be 16-byte aligned", who);
    return XQHIP_OK;
}

static xqhip::GemvLaunch base_launch(const xqhip_w4* w, const void* x, int x_type, const xqhip_prologue* pro) {
    xqhip::GemvLaunch p{};
    p.nib = static_cast<const uint8_t*>(w->nib);
    p.meta = w->meta;
    p.rows = w->rows;
    p.cols = w->cols;
    p.group = w->group;
    p.affine = w->affine;
    p.layout = w->layout;
    p.bits = w->bits;
    p.nib_bytes = w->nib_bytes;
    p.x = x;
    p.x_f16 = x_type == XQHIP_F16;
    p.pro = make_prologue(pro);
    return p;
}

int xqhip_gemv_w4a16(const xqhip_w4* w, const void* x, int x_type, const xqhip_prologue* pro, void* y, int y_type,
                     int epilogue, void* stream) {
    if (int rc = validate_w4(w, "xqhip_gemv_w4a16")) return rc;
    if (int rc = validate_prologue(pro, w->cols, "xqhip_gemv_w4a16")) return rc;
    if (!x || !y) return fail(XQHIP_EINVAL, "xqhip_gemv_w4a16: null vector");
    if (int rc = validate_alignment(w, x, pro, "xqhip_gemv_w4a16")) return rc;
    if (epilogue < XQHIP_EPI_STORE || epilogue > XQHIP_EPI_SILU_PAIR)
        return fail(XQHIP_EINVAL, "xqhip_gemv_w4a16: unknown epilogue %d", epilogue);
    if (epilogue == XQHIP_EPI_SILU_PAIR && (w->rows % 2 != 0))
        return fail(XQHIP_EINVAL, "xqhip_gemv_w4a16: SILU_PAIR needs an even row count");
    if (epilogue != XQHIP_EPI_STORE && y_type != XQHIP_F32)
        return fail(XQHIP_EINVAL, "xqhip_gemv_w4a16: ADD/SILU_PAIR write fp32");
    xqhip::GemvLaunch p = base_launch(w, x, x_type, pro);
    p.y = y;
    p.y_f16 = y_type == XQHIP_F16;
    p.epi = epilogue;
    p.max_blocks = gemv_block_cap();
    return check(xqhip::launch_gemv(p, as_stream(stream)), "gemv_w4a16 launch");
}

size_t xqhip_argmax_workspace_bytes(int rows) {
    (void)rows;
    return sizeof(uint64_t) * kArgmaxMaxBlocks;
}

int xqhip_gemv_w4a16_argmax(const xqhip_w4* w, const void* x, int x_type, const xqhip_prologue* pro, void* workspace,
                            int32_t* out_index, float* out_value, void* stream) {
    if (int rc = validate_w4(w, "xqhip_gemv_w4a16_argmax")) return rc;
    if (int rc = validate_prologue(pro, w->cols, "xqhip_gemv_w4a16_argmax")) return rc;
    if (!x || !workspace || !out_index || !out_value)
        return fail(XQHIP_EINVAL, "xqhip_gemv_w4a16_argmax: null argument");
    if (int rc = validate_alignment(w, x, pro, "xqhip_gemv_w4a16_argmax")) return rc;
    xqhip::GemvLaunch p = base_launch(w, x, x_type, pro);
    p.epi = 3;
    p.partial = static_cast<uint64_t*>(workspace);
    p.out_idx = out_index;
    p.out_val = out_value;
    p.max_blocks = gemv_block_cap() > 0 ? std::min(kArgmaxMaxBlocks, gemv_block_cap()) : 0;
    return check(xqhip::launch_gemv(p, as_stream(stream)), "gemv_w4a16_argmax launch");
}

int xqhip_gemv_w4a16_argmax_publish(const xqhip_w4* w, const void* x, int x_type, const xqhip_prologue* pro,
                                    void* workspace, int32_t* out_index, float* out_value, int32_t* position,
                                    uint64_t* host_slot, void* stream) {
    if (!position || !host_slot) return fail(XQHIP_EINVAL, "xqhip_gemv_w4a16_argmax_publish: null argument");
    if (reinterpret_cast<uintptr_t>(host_slot) % alignof(uint64_t) != 0)
        return fail(XQHIP_EINVAL, "xqhip_gemv_w4a16_argmax_publish: host_slot is not 8-byte aligned");
    if (int rc = validate_w4(w, "xqhip_gemv_w4a16_argmax_publish")) return rc;
    if (int rc = validate_prologue(pro, w->cols, "xqhip_gemv_w4a16_argmax_publish")) return rc;
    if (!x || !workspace || !out_index || !out_value)
        return fail(XQHIP_EINVAL, "xqhip_gemv_w4a16_argmax_publish: null argument");
    if (int rc = validate_alignment(w, x, pro, "xqhip_gemv_w4a16_argmax_publish")) return rc;
    xqhip::GemvLaunch p = base_launch(w, x, x_type, pro);
    p.epi = 3;
    p.partial = static_cast<uint64_t*>(workspace);
    p.out_idx = out_index;
    p.out_val = out_value;
    p.position = position;
    p.host_slot = host_slot;
    p.max_blocks = gemv_block_cap() > 0 ? std::min(kArgmaxMaxBlocks, gemv_block_cap()) : 0;
    return check(xqhip::launch_gemv(p, as_stream(stream)), "gemv_w4a16_argmax_publish launch");
}

int xqhip_gemv_w4a16_argmax_publish_embed(const xqhip_w4* w, const void* x, int x_type, const xqhip_prologue* pro,
                                          void* workspace, int32_t* out_index, float* out_value, int32_t* position,
                                          uint64_t* host_slot, const uint16_t* table, int vocab, int hidden,
                                          float* embed_out, void* stream) {
    const char* fn = "xqhip_gemv_w4a16_argmax_publish_embed";
    if (!position || !host_slot || !table || !embed_out) return fail(XQHIP_EINVAL, "%s: null argument", fn);
    if (vocab <= 0 || hidden <= 0) return fail(XQHIP_EINVAL, "%s: vocab and hidden must be positive", fn);
    if (reinterpret_cast<uintptr_t>(host_slot) % alignof(uint64_t) != 0)
        return fail(XQHIP_EINVAL, "%s: host_slot is not 8-byte aligned", fn);
    if (int rc = validate_w4(w, fn)) return rc;
    if (int rc = validate_prologue(pro, w->cols, fn)) return rc;
    if (!x || !workspace || !out_index || !out_value) return fail(XQHIP_EINVAL, "%s: null argument", fn);
    if (int rc = validate_alignment(w, x, pro, fn)) return rc;
    xqhip::GemvLaunch p = base_launch(w, x, x_type, pro);
    p.epi = 3;
    p.partial = static_cast<uint64_t*>(workspace);
    p.out_idx = out_index;
    p.out_val = out_value;
    p.position = position;
    p.host_slot = host_slot;
    p.embed_table = table;
    p.embed_vocab = vocab;
    p.embed_hidden = hidden;
    p.embed_out = embed_out;
    p.max_blocks = gemv_block_cap() > 0 ? std::min(kArgmaxMaxBlocks, gemv_block_cap()) : 0;
    return check(xqhip::launch_gemv(p, as_stream(stream)), "gemv_w4a16_argmax_publish_embed launch");
}

int xqhip_gemv_w4a16_argmax_static(const xqhip_w4* w, const void* x, int x_type, const xqhip_prologue* pro,
                                   int32_t* out_index, float* out_value, void* stream) {
    const size_t need = xqhip_argmax_workspace_bytes(w ? w->rows : 0);
    if (need > sizeof(scratch))
        return fail(XQHIP_EINVAL, "xqhip_gemv_w4a16_argmax_static: needs %zu bytes of scratch, the library holds %zu",
                    need, sizeof(scratch));
    void* ptr = static_scratch(as_stream(stream));
    if (!ptr) return std::strstr(g_err.c_str(), "the stream belongs") ? XQHIP_EINVAL : XQHIP_EDEVICE;
    // the keys need no clearing: every block of the launch writes its own
    // before the finishing kernel reads exactly those
    return xqhip_gemv_w4a16_argmax(w, x, x_type, pro, ptr, out_index, out_value, stream);
}

int xqhip_embed_bf16(const uint16_t* table, int vocab, int hidden, const int32_t* token, float* out, void* stream) {
    if (!table || !token || !out || vocab <= 0 || hidden <= 0) return fail(XQHIP_EINVAL, "xqhip_embed_bf16: bad args");
    xqhip::EmbedLaunch p{table, vocab, hidden, token, out};
    return check(xqhip::launch_embed(p, as_stream(stream)), "embed launch");
}

int xqhip_rope_table(float theta, int rotary_dim, int max_pos, float* out) {
    if (!out || rotary_dim < 0 || max_pos <= 0) return fail(XQHIP_EINVAL, "xqhip_rope_table: bad args");
    const int half = rotary_dim / 2;
    for (int pos = 0; pos < max_pos; ++pos) {
        for (int i = 0; i < half; ++i) {
            const float inv_freq = std::pow(theta, -static_cast<float>(2 * i) / static_cast<float>(rotary_dim));
            const float angle = static_cast<float>(pos) * inv_freq;
            out[(static_cast<size_t>(pos) * half + i) * 2] = std::cos(angle);
            out[(static_cast<size_t>(pos) * half + i) * 2 + 1] = std::sin(angle);
        }
    }
    return XQHIP_OK;
}

int xqhip_attn_prep(const float* q_src, const float* k_src, const float* v_src, int gated, int nq, int nkv,
                    int head_dim, int rotary_dim, const float* q_norm, const float* k_norm, float eps,
                    const float* rope_cs, const int32_t* pos, float* q_out, float* gate_out, void* k_cache,
                    void* v_cache, void* stream) {
    if (!q_src || !k_src || !v_src || !q_norm || !k_norm || !pos || !q_out || !gate_out || !k_cache || !v_cache ||
        nq <= 0 || nkv <= 0 || head_dim <= 0 || head_dim > 1024 || (rotary_dim > 0 && !rope_cs))
        return fail(XQHIP_EINVAL, "xqhip_attn_prep: bad args");
    const int active = std::max(0, std::min(head_dim, rotary_dim));
    xqhip::QkPrepLaunch p{};
    p.q_src = q_src;
    p.k_src = k_src;
    p.v_src = v_src;
    p.gated = gated;
    p.nq = nq;
    p.nkv = nkv;
    p.head_dim = head_dim;
    p.rotary_dim = active;
    p.rope_pairs = active / 2;
    p.q_norm = q_norm;
    p.k_norm = k_norm;
    p.eps = eps;
    p.rope_cs = rope_cs;
    p.pos = pos;
    p.q_out = q_out;
    p.gate_out = gate_out;
    p.k_cache = static_cast<_Float16*>(k_cache);
    p.v_cache = static_cast<_Float16*>(v_cache);
    return check(xqhip::launch_qk_prep(p, as_stream(stream)), "attn_prep launch");
}

size_t xqhip_gqa_workspace_bytes(int nq, int nkv, int head_dim) { return xqhip::gqa_workspace_bytes(nq, nkv, head_dim); }

int xqhip_gqa_decode(const float* q, const void* k_cache, const void* v_cache, const float* gate, int nq, int nkv,
                     int head_dim, int max_ctx, const int32_t* pos, float* out, void* workspace, void* stream) {
    if (!q || !k_cache || !v_cache || !gate || !pos || !out || !workspace)
        return fail(XQHIP_EINVAL, "xqhip_gqa_decode: null argument");
    if (!xqhip::gqa_supported(nq, nkv, head_dim, max_ctx))
        return fail(XQHIP_EINVAL, "xqhip_gqa_decode: unsupported shape nq=%d nkv=%d hd=%d ctx=%d", nq, nkv, head_dim,
                    max_ctx);
    xqhip::GqaLaunch p{};
    p.q = q;
    p.k_cache = static_cast<const _Float16*>(k_cache);
    p.v_cache = static_cast<const _Float16*>(v_cache);
    p.gate = gate;
    p.gate_stride = head_dim;
    p.nq = nq;
    p.nkv = nkv;
    p.head_dim = head_dim;
    p.max_ctx = max_ctx;
    p.pos = pos;
    p.out = out;
    // workspace: part_m [nq][slots], part_l [nq][slots], part_o [nq][slots][head_dim]
    float* f = static_cast<float*>(workspace);
    const size_t per = xqhip::gqa_workspace_bytes(nq, nkv, head_dim) / sizeof(float) / (head_dim + 2);
    p.part_m = f;
    p.part_l = f + per;
    p.part_o = f + 2 * per;
    return check(xqhip::launch_gqa(p, as_stream(stream)), "gqa launch");
}

// The launch arguments shared by the two decode attention entry points
// (workspace: the slot kernel's partials, nullptr for the per-head kernel).
static xqhip::AttnDecodeLaunch attn_decode_args(const float* q_src, const float* k_src, const float* v_src, int gated,
                                                int nq, int nkv, int head_dim, int rotary_dim, const float* q_norm,
                                                const float* k_norm, float eps, const float* rope_cs,
                                                const int32_t* pos, void* k_cache, void* v_cache, int max_ctx,
                                                float* out, void* workspace) {
    xqhip::AttnDecodeLaunch a{};
    xqhip::GqaLaunch& p = a.g;
    p.k_cache = static_cast<const _Float16*>(k_cache);
    p.v_cache = static_cast<const _Float16*>(v_cache);
    p.gate = gated ? q_src + head_dim : nullptr;
    p.gate_stride = 2 * head_dim;
    p.nq = nq;
    p.nkv = nkv;
    p.head_dim = head_dim;
    p.max_ctx = max_ctx;
    p.pos = pos;
    p.out = out;
    if (workspace) {
        float* f = static_cast<float*>(workspace);
        const size_t per = xqhip::gqa_workspace_bytes(nq, nkv, head_dim) / sizeof(float) / (head_dim + 2);
        p.part_m = f;
        p.part_l = f + per;
        p.part_o = f + 2 * per;
    }
    a.q_src = q_src;
    a.k_src = k_src;
    a.v_src = v_src;
    a.gated = gated;
    a.rotary_dim = std::max(0, std::min(head_dim, rotary_dim)) / 2 * 2;
    a.rope_pairs = std::max(0, std::min(head_dim, rotary_dim)) / 2;
    a.q_norm = q_norm;
    a.k_norm = k_norm;
    a.eps = eps;
    a.rope_cs = rope_cs;
    a.k_cache = static_cast<_Float16*>(k_cache);
    a.v_cache = static_cast<_Float16*>(v_cache);
    return a;
}

int xqhip_attn_decode(const float* q_src, const float* k_src, const float* v_src, int gated, int nq, int nkv,
                      int head_dim, int rotary_dim, const float* q_norm, const float* k_norm, float eps,
                      const float* rope_cs, const int32_t* pos, void* k_cache, void* v_cache, int max_ctx, float* out,
                      void* workspace, void* stream) {
    if (!q_src || !k_src || !v_src || !q_norm || !k_norm || !pos || !k_cache || !v_cache || !out || !workspace ||
        (rotary_dim > 0 && !rope_cs))
        return fail(XQHIP_EINVAL, "xqhip_attn_decode: null argument");
    if (!xqhip::gqa_supported(nq, nkv, head_dim, max_ctx))
        return fail(XQHIP_EINVAL, "xqhip_attn_decode: unsupported shape nq=%d nkv=%d hd=%d ctx=%d", nq, nkv,
                    head_dim, max_ctx);
    const xqhip::AttnDecodeLaunch a = attn_decode_args(q_src, k_src, v_src, gated, nq, nkv, head_dim, rotary_dim,
                                                       q_norm, k_norm, eps, rope_cs, pos, k_cache, v_cache, max_ctx,
                                                       out, workspace);
    return check(xqhip::launch_attn_decode(a, as_stream(stream)), "attn_decode launch");
}

int xqhip_attn_decode_head(const float* q_src, const float* k_src, const float* v_src, int gated, int nq, int nkv,
                           int head_dim, int rotary_dim, const float* q_norm, const float* k_norm, float eps,
                           const float* rope_cs, const int32_t* pos, void* k_cache, void* v_cache, float* out,
                           void* stream) {
    if (!q_src || !k_src || !v_src || !q_norm || !k_norm || !pos || !k_cache || !v_cache || !out ||
        (rotary_dim > 0 && !rope_cs))
        return fail(XQHIP_EINVAL, "xqhip_attn_decode_head: null argument");
    if (!xqhip::attn_head_supported(nq, nkv, head_dim))
        return fail(XQHIP_EINVAL, "xqhip_attn_decode_head: unsupported shape nq=%d nkv=%d hd=%d (head_dim 128 only)",
                    nq, nkv, head_dim);
    const xqhip::AttnDecodeLaunch a = attn_decode_args(q_src, k_src, v_src, gated, nq, nkv, head_dim, rotary_dim,
                                                       q_norm, k_norm, eps, rope_cs, pos, k_cache, v_cache, 0, out,
                                                       nullptr);
    return check(xqhip::launch_attn_decode_head(a, as_stream(stream)), "attn_decode_head launch");
}

static_assert(XQHIP_ATTN_PART_STRIDE == xqhip::kAttnPartStride && XQHIP_ATTN_MAX_SPLITS == xqhip::kAttnMaxSplits,
              "split attention workspace layout");

size_t xqhip_attn_split_workspace_bytes(int nq) {
    if (nq <= 0) return 0;
    // partials [XQHIP_ATTN_MAX_SPLITS][nq][stride] floats, then one counter per head, 128 bytes apart
    return sizeof(float) * static_cast<size_t>(XQHIP_ATTN_MAX_SPLITS) * nq * XQHIP_ATTN_PART_STRIDE +
           static_cast<size_t>(nq) * 128;
}

int xqhip_attn_decode_split(const float* q_src, const float* k_src, const float* v_src, int gated, int nq, int nkv,
                            int head_dim, int rotary_dim, const float* q_norm, const float* k_norm, float eps,
                            const float* rope_cs, const int32_t* pos, void* k_cache, void* v_cache, int splits,
                            void* workspace, float* out, void* stream) {
    if (!q_src || !k_src || !v_src || !q_norm || !k_norm || !pos || !k_cache || !v_cache || !workspace || !out ||
        (rotary_dim > 0 && !rope_cs))
        return fail(XQHIP_EINVAL, "xqhip_attn_decode_split: null argument");
    if (!xqhip::attn_head_supported(nq, nkv, head_dim))
        return fail(XQHIP_EINVAL, "xqhip_attn_decode_split: unsupported shape nq=%d nkv=%d hd=%d (head_dim 128 only)",
                    nq, nkv, head_dim);
    if (splits < 1 || splits > XQHIP_ATTN_MAX_SPLITS)
        return fail(XQHIP_EINVAL, "xqhip_attn_decode_split: splits %d outside 1..%d", splits, XQHIP_ATTN_MAX_SPLITS);
    if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0)
        return fail(XQHIP_EINVAL, "xqhip_attn_decode_split: workspace not 16-byte aligned");
    float* part = static_cast<float*>(workspace);
    uint32_t* cnt = reinterpret_cast<uint32_t*>(part + static_cast<size_t>(XQHIP_ATTN_MAX_SPLITS) * nq *
                                                           XQHIP_ATTN_PART_STRIDE);
    const xqhip::AttnDecodeLaunch a = attn_decode_args(q_src, k_src, v_src, gated, nq, nkv, head_dim, rotary_dim,
                                                       q_norm, k_norm, eps, rope_cs, pos, k_cache, v_cache, 0, out,
                                                       nullptr);
    return check(xqhip::launch_attn_decode_part(a, splits, part, cnt, as_stream(stream)),
                 "attn_decode_split launch");
}

int xqhip_linear_conv(const float* mixed, float* conv_state, const float* conv_w, int lk_n, int lk_hd, int lv_n,
                      int lv_hd, int ksize, float* out, void* stream) {
    if (!mixed || !conv_state || !conv_w || !out || lk_n <= 0 || lv_n <= 0 || ksize < 1 ||
        !xqhip::conv_supported(lk_hd, lv_hd))
        return fail(XQHIP_EINVAL, "xqhip_linear_conv: bad args");
    xqhip::ConvLaunch p{mixed, conv_state, conv_w, lk_n, lk_hd, lv_n, lv_hd, ksize, out};
    return check(xqhip::launch_conv(p, as_stream(stream)), "conv launch");
}

int xqhip_gated_delta(const float* conv, const float* a, const float* b, const float* a_log, const float* dt_bias,
                      float* state, int lk_n, int lv_n, int lk_hd, int lv_hd, float* out, void* stream) {
    if (!conv || !a || !b || !a_log || !dt_bias || !state || !out || lk_n <= 0 || lv_n <= 0 || lv_hd <= 0 ||
        !xqhip::delta_supported(lk_hd))
        return fail(XQHIP_EINVAL, "xqhip_gated_delta: bad args");
    xqhip::DeltaLaunch p{conv, a, b, a_log, dt_bias, state, lk_n, lv_n, lk_hd, lv_hd, out};
    return check(xqhip::launch_delta(p, as_stream(stream)), "delta launch");
}

int xqhip_linear_attn_step(const float* mixed, float* conv_state, const float* conv_w, const float* a, const float* b,
                           const float* a_log, const float* dt_bias, float* state, int lk_n, int lk_hd, int lv_n,
                           int lv_hd, int ksize, const int32_t* pos, float* out, void* stream) {
    if (!mixed || !conv_state || !conv_w || !a || !b || !a_log || !dt_bias || !state || !pos || !out)
        return fail(XQHIP_EINVAL, "xqhip_linear_attn_step: null argument");
    if (!xqhip::linear_step_supported(lk_n, lk_hd, lv_n, lv_hd, ksize))
        return fail(XQHIP_EINVAL, "xqhip_linear_attn_step: unsupported shape lk=%dx%d lv=%dx%d k=%d", lk_n, lk_hd, lv_n,
                    lv_hd, ksize);
    xqhip::LinearStepLaunch p{mixed, conv_state, conv_w, a, b, a_log, dt_bias, state,
                              lk_n, lk_hd, lv_n, lv_hd, ksize, pos, out, nullptr};
    return check(xqhip::launch_linear_step(p, as_stream(stream)), "linear step launch");
}

int xqhip_linear_attn_step_act(const float* mixed, float* conv_state, const float* conv_w, const float* a,
                               const float* b, const float* a_log, const float* dt_bias, float* state, int lk_n,
                               int lk_hd, int lv_n, int lv_hd, int ksize, const int32_t* pos, float* out,
                               float* gate, void* stream) {
    if (!gate) return fail(XQHIP_EINVAL, "xqhip_linear_attn_step_act: null gate");
    if (!mixed || !conv_state || !conv_w || !a || !b || !a_log || !dt_bias || !state || !pos || !out)
        return fail(XQHIP_EINVAL, "xqhip_linear_attn_step_act: null argument");
    if (!xqhip::linear_step_supported(lk_n, lk_hd, lv_n, lv_hd, ksize))
        return fail(XQHIP_EINVAL, "xqhip_linear_attn_step_act: unsupported shape lk=%dx%d lv=%dx%d k=%d", lk_n, lk_hd,
                    lv_n, lv_hd, ksize);
    xqhip::LinearStepLaunch p{mixed, conv_state, conv_w, a, b, a_log, dt_bias, state,
                              lk_n, lk_hd, lv_n, lv_hd, ksize, pos, out, gate};
    return check(xqhip::launch_linear_step(p, as_stream(stream)), "linear step launch");
}

size_t xqhip_step_outproj_sync_bytes(void) { return xqhip::step_outproj_sync_bytes(); }

// The launch descriptors of xqhip_linear_attn_step_outproj, validated as the
// two separate entry points validate them.
static int step_outproj_args(const float* mixed, float* conv_state, const float* conv_w, const float* a,
                             const float* b, const float* a_log, const float* dt_bias, float* state, int lk_n,
                             int lk_hd, int lv_n, int lv_hd, int ksize, const int32_t* pos, float* out, float* gate,
                             const xqhip_w4* w, const float* norm_weight, float eps, float* y,
                             xqhip::LinearStepLaunch* sp, xqhip::GemvLaunch* g, const char* who) {
    if (!mixed || !conv_state || !conv_w || !a || !b || !a_log || !dt_bias || !state || !pos || !out || !gate ||
        !norm_weight || !y)
        return fail(XQHIP_EINVAL, "%s: null argument", who);
    if (!xqhip::linear_step_supported(lk_n, lk_hd, lv_n, lv_hd, ksize))
        return fail(XQHIP_EINVAL, "%s: unsupported step shape lk=%dx%d lv=%dx%d k=%d", who, lk_n, lk_hd, lv_n, lv_hd,
                    ksize);
    if (int rc = validate_w4(w, who)) return rc;
    const xqhip_prologue pro{XQHIP_PRO_GATED_HEAD_ACT, lv_hd, norm_weight, gate, eps};
    if (int rc = validate_prologue(&pro, w->cols, who)) return rc;
    if (int rc = validate_alignment(w, out, &pro, who)) return rc;
    if (w->cols != lv_n * lv_hd)
        return fail(XQHIP_EINVAL, "%s: the projection has %d columns, the step writes %d", who, w->cols, lv_n * lv_hd);
    *sp = xqhip::LinearStepLaunch{mixed, conv_state, conv_w, a, b, a_log, dt_bias, state,
                                  lk_n, lk_hd, lv_n, lv_hd, ksize, pos, out, gate};
    *g = base_launch(w, out, XQHIP_F32, &pro);
    g->y = y;
    g->epi = XQHIP_EPI_ADD;
    return XQHIP_OK;
}

int xqhip_step_outproj_supported(const xqhip_w4* w, int lk_n, int lk_hd, int lv_n, int lv_hd, int ksize) {
    if (!w || !w->nib || !w->meta) return 0;
    // placeholder vectors: only the shapes and the device's residency are checked
    alignas(16) static float f[4] = {};
    static int32_t i = 0;
    xqhip::LinearStepLaunch sp{};
    xqhip::GemvLaunch g{};
    if (step_outproj_args(f, f, f, f, f, f, f, f, lk_n, lk_hd, lv_n, lv_hd, ksize, &i, f, f, w, f, 1e-6f, f, &sp, &g,
                          "xqhip_step_outproj_supported") != XQHIP_OK)
        return 0;
    return xqhip::step_outproj_grid(sp, g) > 0 ? 1 : 0;
}

int xqhip_linear_attn_step_outproj(const float* mixed, float* conv_state, const float* conv_w, const float* a,
                                   const float* b, const float* a_log, const float* dt_bias, float* state, int lk_n,
                                   int lk_hd, int lv_n, int lv_hd, int ksize, const int32_t* pos, float* out,
                                   float* gate, const xqhip_w4* w, const float* norm_weight, float eps, float* y,
                                   void* sync, void* stream) {
    static const char* who = "xqhip_linear_attn_step_outproj";
    xqhip::LinearStepLaunch sp{};
    xqhip::GemvLaunch g{};
    if (int rc = step_outproj_args(mixed, conv_state, conv_w, a, b, a_log, dt_bias, state, lk_n, lk_hd, lv_n, lv_hd,
                                   ksize, pos, out, gate, w, norm_weight, eps, y, &sp, &g, who))
        return rc;
    if (!sync || (reinterpret_cast<uintptr_t>(sync) & 127u) != 0)
        return fail(XQHIP_EINVAL, "%s: sync must be a 128-byte aligned block of xqhip_step_outproj_sync_bytes()", who);
    if (!xqhip::step_outproj_shape_ok(sp, g) || xqhip::step_outproj_grid(sp, g) == 0)
        return fail(XQHIP_ENOTSUP, "%s: not available for this matrix (%dx%d layout %d) or device", who, w->rows,
                    w->cols, w->layout);
    return check(xqhip::launch_step_outproj(sp, g, static_cast<uint32_t*>(sync), as_stream(stream)),
                 "step + output projection launch");
}

int xqhip_step_outproj_error(const void* sync, int* error) {
    if (!sync || !error) return fail(XQHIP_EINVAL, "xqhip_step_outproj_error: null argument");
    const size_t words = xqhip::step_outproj_sync_bytes() / sizeof(uint32_t);
    std::vector<uint32_t> host(words);
    if (int rc = check(hipMemcpy(host.data(), sync, words * sizeof(uint32_t), hipMemcpyDeviceToHost),
                       "xqhip_step_outproj_error copy"))
        return rc;
    *error = host[xqhip::step_outproj_error_word()] != 0;
    return XQHIP_OK;
}

// ---- prefill (multi-token) ---------------------------------------------------

size_t xqhip_gemm_workspace_bytes(int m, int cols, int rows) {
    return m > 0 && cols > 0 && rows >= 0 ? xqhip::gemm_workspace_bytes(m, cols, rows) : 0;
}

int xqhip_gemm_w4a16(const xqhip_w4* w, const float* x, int m, int ldx, const xqhip_prologue* pro, int ld_gate,
                     float* y, int ldy, int epilogue, void* workspace, size_t workspace_bytes, void* stream) {
    if (int rc = validate_w4(w, "xqhip_gemm_w4a16")) return rc;
    if (w->bits != 4) return fail(XQHIP_EINVAL, "xqhip_gemm_w4a16: 4-bit matrices only (got %d bits)", w->bits);
    if (int rc = validate_prologue(pro, w->cols, "xqhip_gemm_w4a16", false)) return rc;
    if (!x || !y || !workspace || m <= 0 || ldx < w->cols)
        return fail(XQHIP_EINVAL, "xqhip_gemm_w4a16: bad vectors (m=%d ldx=%d)", m, ldx);
    if (epilogue < XQHIP_EPI_STORE || epilogue > XQHIP_EPI_SILU_PAIR)
        return fail(XQHIP_EINVAL, "xqhip_gemm_w4a16: unknown epilogue %d", epilogue);
    const int out_cols = epilogue == XQHIP_EPI_SILU_PAIR ? w->rows / 2 : w->rows;
    if ((epilogue == XQHIP_EPI_SILU_PAIR && w->rows % 2 != 0) || ldy < out_cols)
        return fail(XQHIP_EINVAL, "xqhip_gemm_w4a16: bad output layout (rows=%d ldy=%d)", w->rows, ldy);
    const xqhip::Prologue pr = make_prologue(pro);
    if (pr.mode == xqhip::PRO_GATED && ld_gate < w->cols)
        return fail(XQHIP_EINVAL, "xqhip_gemm_w4a16: gate row stride %d < cols", ld_gate);
    if (!xqhip::gemm_supported(w->rows, w->cols, w->group, w->layout, pr))
        return fail(XQHIP_EINVAL, "xqhip_gemm_w4a16: needs a TILED64 matrix (%dx%d g%d)", w->rows, w->cols, w->group);
    if ((reinterpret_cast<uintptr_t>(workspace) & 15u) != 0)
        return fail(XQHIP_EINVAL, "xqhip_gemm_w4a16: workspace must be 16-byte aligned");
    // the staged x and, for launches split over the columns, the partial products
    if (const size_t need = xqhip::gemm_workspace_bytes(m, w->cols, w->rows); workspace_bytes < need)
        return fail(XQHIP_EINVAL, "xqhip_gemm_w4a16: workspace of %zu bytes, %zu needed", workspace_bytes, need);
    // the kernels address the staged x (hi and lo halves) with 32-bit buffer offsets
    if (xqhip::gemm_workspace_bytes(m, w->cols, 0) >= (size_t{1} << 31))
        return fail(XQHIP_EINVAL, "xqhip_gemm_w4a16: %d tokens of %d columns exceed one call (2 GiB of staged x)", m,
                    w->cols);
    xqhip::GemmLaunch p{};
    p.nib = static_cast<const uint8_t*>(w->nib);
    p.meta = w->meta;
    p.rows = w->rows;
    p.cols = w->cols;
    p.affine = w->affine;
    p.layout = w->layout;
    p.zero_is_8 = w->zero_is_8;
    p.x = x;
    p.ldx = ldx;
    p.m = m;
    p.pro = pr;
    p.ldz = ld_gate;
    p.y = y;
    p.ldy = ldy;
    p.epi = epilogue;
    p.workspace = workspace;
    return check(xqhip::launch_gemm(p, as_stream(stream)), "gemm launch");
}

int xqhip_embed_bf16_batch(const uint16_t* table, int vocab, int hidden, const int32_t* tokens, int n, float* out,
                           void* stream) {
    if (!table || !tokens || !out || vocab <= 0 || hidden <= 0 || n <= 0 || n > 65535)
        return fail(XQHIP_EINVAL, "xqhip_embed_bf16_batch: bad args");
    xqhip::EmbedLaunch p{table, vocab, hidden, tokens, out, n};
    return check(xqhip::launch_embed(p, as_stream(stream)), "embed batch launch");
}

int xqhip_attn_prep_batch(const float* q_src, const float* k_src, const float* v_src, int gated, int nq, int nkv,
                          int head_dim, int rotary_dim, const float* q_norm, const float* k_norm, float eps,
                          const float* rope_cs, const int32_t* pos0, int tokens, int src_stride, int out_stride,
                          float* q_out, float* gate_out, void* k_cache, void* v_cache, void* stream) {
    if (!q_src || !k_src || !v_src || !q_norm || !k_norm || !pos0 || !q_out || !gate_out || !k_cache || !v_cache ||
        nq <= 0 || nkv <= 0 || head_dim <= 0 || head_dim > 1024 || (rotary_dim > 0 && !rope_cs) || tokens <= 0 ||
        tokens > 65535 || out_stride < nq * head_dim)
        return fail(XQHIP_EINVAL, "xqhip_attn_prep_batch: bad args");
    const int active = std::max(0, std::min(head_dim, rotary_dim));
    xqhip::QkPrepLaunch p{};
    p.q_src = q_src;
    p.k_src = k_src;
    p.v_src = v_src;
    p.gated = gated;
    p.nq = nq;
    p.nkv = nkv;
    p.head_dim = head_dim;
    p.rotary_dim = active;
    p.rope_pairs = active / 2;
    p.q_norm = q_norm;
    p.k_norm = k_norm;
    p.eps = eps;
    p.rope_cs = rope_cs;
    p.pos = pos0;
    p.q_out = q_out;
    p.gate_out = gate_out;
    p.k_cache = static_cast<_Float16*>(k_cache);
    p.v_cache = static_cast<_Float16*>(v_cache);
    p.tokens = tokens;
    p.src_stride = src_stride;
    p.out_stride = out_stride;
    return check(xqhip::launch_qk_prep(p, as_stream(stream)), "attn_prep batch launch");
}

int xqhip_prefill_attention(const float* q, const float* gate, const void* k_cache, const void* v_cache, int nq,
                            int nkv, int head_dim, int tokens, int q_stride, const int32_t* pos0, float* out,
                            int out_stride, void* stream) {
    if (!q || !gate || !k_cache || !v_cache || !pos0 || !out || tokens <= 0 || tokens > 65535 ||
        q_stride < nq * head_dim || out_stride < nq * head_dim || !xqhip::prefill_attn_supported(nq, nkv, head_dim))
        return fail(XQHIP_EINVAL, "xqhip_prefill_attention: bad args (nq=%d nkv=%d hd=%d)", nq, nkv, head_dim);
    xqhip::PrefillAttnLaunch p{q, gate, static_cast<const _Float16*>(k_cache), static_cast<const _Float16*>(v_cache),
                               nq, nkv, head_dim, tokens, q_stride, out_stride, pos0, out};
    return check(xqhip::launch_prefill_attn(p, as_stream(stream)), "prefill attention launch");
}

size_t xqhip_linear_scan_workspace_bytes(int tokens, int lk_n, int lk_hd, int lv_n, int lv_hd) {
    if (tokens <= 0 || lk_n <= 0 || lk_hd <= 0 || lv_n <= 0 || lv_hd <= 0) return 0;
    return xqhip::linear_scan_workspace_bytes(tokens, lk_n, lk_hd, lv_n, lv_hd);
}

static int linear_attn_scan_impl(const float* mixed, const float* a, const float* b, int stride, float* conv_state,
                                 int pos0, const float* conv_w, const float* a_log, const float* dt_bias, float* state,
                                 int lk_n, int lk_hd, int lv_n, int lv_hd, int ksize, int tokens, float* out,
                                 int out_stride, void* workspace, void* stream) {
    if (!mixed || !a || !b || !conv_state || !conv_w || !a_log || !dt_bias || !state || !out || tokens <= 0 ||
        pos0 < 0 || !xqhip::linear_scan_supported(lk_n, lk_hd, lv_n, lv_hd, ksize) || out_stride < lv_n * lv_hd)
        return fail(XQHIP_EINVAL, "xqhip_linear_attn_scan: bad args");
    const int conv_dim = 2 * lk_n * lk_hd + lv_n * lv_hd;
    const size_t hist_floats = static_cast<size_t>(conv_dim) * std::max(0, ksize - 1);
    float* copy_in = conv_state + static_cast<size_t>(pos0 & 1) * hist_floats;
    float* copy_next = conv_state + static_cast<size_t>((pos0 + tokens) & 1) * hist_floats;
    float* other = conv_state + static_cast<size_t>((pos0 & 1) ^ 1) * hist_floats;
    xqhip::LinearScanLaunch p{mixed, a, b, stride, copy_in, other, conv_w, a_log, dt_bias, state,
                              lk_n, lk_hd, lv_n, lv_hd, ksize, tokens, out, out_stride,
                              static_cast<float*>(workspace)};
    if (int rc = check(xqhip::launch_linear_scan(p, as_stream(stream)), "linear scan launch")) return rc;
    // the next position reads copy (pos0 + tokens) & 1: when that is the input
    // copy (even token count), move the new history there
    if (copy_next != other && hist_floats > 0) return xqhip_copy(copy_next, other, hist_floats * sizeof(float), stream);
    return XQHIP_OK;
}

int xqhip_linear_attn_scan(const float* mixed, const float* a, const float* b, int stride, float* conv_state,
                           int pos0, const float* conv_w, const float* a_log, const float* dt_bias, float* state,
                           int lk_n, int lk_hd, int lv_n, int lv_hd, int ksize, int tokens, float* out,
                           int out_stride, void* stream) {
    return linear_attn_scan_impl(mixed, a, b, stride, conv_state, pos0, conv_w, a_log, dt_bias, state, lk_n, lk_hd,
                                 lv_n, lv_hd, ksize, tokens, out, out_stride, nullptr, stream);
}

int xqhip_linear_attn_scan_ws(const float* mixed, const float* a, const float* b, int stride, float* conv_state,
                              int pos0, const float* conv_w, const float* a_log, const float* dt_bias, float* state,
                              int lk_n, int lk_hd, int lv_n, int lv_hd, int ksize, int tokens, float* out,
                              int out_stride, void* workspace, void* stream) {
    if (!workspace || (reinterpret_cast<uintptr_t>(workspace) & 15u) != 0)
        return fail(XQHIP_EINVAL, "xqhip_linear_attn_scan_ws: workspace must be non-null and 16-byte aligned");
    return linear_attn_scan_impl(mixed, a, b, stride, conv_state, pos0, conv_w, a_log, dt_bias, state, lk_n, lk_hd,
                                 lv_n, lv_hd, ksize, tokens, out, out_stride, workspace, stream);
}

int xqhip_rmsnorm(const float* x, const float* w, int n, float eps, float* y, void* stream) {
    if (!x || !w || !y || n <= 0) return fail(XQHIP_EINVAL, "xqhip_rmsnorm: bad args");
    return check(xqhip::launch_rmsnorm(x, w, n, eps, y, as_stream(stream)), "rmsnorm launch");
}

int xqhip_lds_fill(float value, void* stream) {
    return check(xqhip::launch_lds_fill(value, as_stream(stream)), "lds fill launch");
}

int xqhip_stream_create(void** stream) {
    hipStream_t s;
    if (int rc = check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate")) return rc;
    *stream = s;
    return XQHIP_OK;
}
int xqhip_stream_destroy(void* stream) { return check(hipStreamDestroy(as_stream(stream)), "hipStreamDestroy"); }

int xqhip_graph_begin(void* stream) {
    return check(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
}
int xqhip_graph_end(void* stream, void** graph_exec) {
    hipGraph_t g;
    if (int rc = check(hipStreamEndCapture(as_stream(stream), &g), "hipStreamEndCapture")) return rc;
    hipGraphExec_t e;
    const int rc = check(hipGraphInstantiate(&e, g, nullptr, nullptr, 0), "hipGraphInstantiate");
    (void)hipGraphDestroy(g);
    if (rc) return rc;
    *graph_exec = e;
    return XQHIP_OK;
}
int xqhip_graph_launch(void* graph_exec, void* stream) {
    return check(hipGraphLaunch(static_cast<hipGraphExec_t>(graph_exec), as_stream(stream)), "hipGraphLaunch");
}
int xqhip_graph_destroy(void* graph_exec) {
    return check(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph_exec)), "hipGraphExecDestroy");
}

}  // extern "C"
