// xqhip_common.hpp - shared device helpers for the gfx950 (CDNA4, wave64) kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace xqhip {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// Streaming (non-temporal) 16-byte load: weights are read once per token and
// should not displace activations or the KV cache from the caches.
__device__ __forceinline__ uint4 load_nt16(const void* p) {
    const u32x4 v = __builtin_nontemporal_load(static_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// fp16 bit pattern 0x6400 is 1024.0; OR-ing a 4-bit code into mantissa bits
// 0-3 gives 1024+q exactly, into bits 4-7 gives 1024+16q exactly.
constexpr uint32_t kMagic2 = 0x64006400u;

// (a & mask) | bits in one v_and_or_b32.  Written as inline asm because VOP3
// cannot encode literal constants on gfx9-family targets and the compiler would
// otherwise split it into v_and_b32 + v_or_b32 with literals; with the two
// constants held in VGPRs (hoisted out of the loop) it is one instruction.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t bits) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(mask), "v"(bits));
    return r;
}

__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
__device__ __forceinline__ uint32_t as_u32(h2 v) { return __builtin_bit_cast(uint32_t, v); }

// v_dot2_f32_f16: a.x*b.x + a.y*b.y + c with fp32 accumulation (products of two
// fp16 values are exact in fp32).
__device__ __forceinline__ float dot2(h2 a, h2 b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }

__device__ __forceinline__ float half_lo(uint32_t u) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(u & 0xffffu)));
}
__device__ __forceinline__ float half_hi(uint32_t u) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(u >> 16)));
}

// a * b rounded to fp32 on its own: never contracted into a later add (the
// first step of a row sum), so a product's rounding does not depend on how
// the compiler schedules the code that consumes it
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
    return a * b;
}

// Group metadata word of a TILED64 matrix: fp16 (scale, zero) in one u32
// (META 0), the fp32 (scale, zero) pair in two (META 1, matrices whose values
// fp16 cannot hold exactly), the fp16 scale alone with the zero point 8
// implied (META 2, format-v1 matrices whose zeros are all 8), or the fp32
// scale with the zero as a 4-bit code (META 3, format-v1 matrices whose zeros
// are integers 0..15 and whose scales fp16 cannot hold: the reference packer's
// asymmetric quantiser).  META 3 keeps two arrays in one allocation: the fp32
// scales [rows][G], then u32 zero words [rows][ceil(G / 8)], nibble k of word
// j holding the zero of group 8 j + k; a group's word is (scale bits, the zero
// word that holds its nibble), and meta_zero_at takes the nibble's bit offset.
struct Scale16 {
    uint32_t v;  // fp16 scale in the low half
};
struct ScaleZ4 {
    uint32_t s;   // fp32 scale bits
    uint32_t zw;  // zero word of 8 consecutive groups
};
template <int META>
using MetaWord = typename std::conditional<
    META == 1, u32x2,
    typename std::conditional<META == 2, Scale16,
                              typename std::conditional<META == 3, ScaleZ4, uint32_t>::type>::type>::type;
// bytes per group of the (first) metadata array: the offset stride of a group's word
template <int META>
constexpr uint32_t kMetaGroupBytes = META == 1 ? 8u : (META == 2 ? 2u : 4u);
// META 3: zero words per row, and the bytes of both arrays of a rows x G matrix
__host__ __device__ constexpr uint32_t z4_words(uint32_t G) { return (G + 7u) / 8u; }
template <int META>
__host__ __device__ constexpr uint32_t meta_total_bytes(uint32_t rows, uint32_t G) {
    return META == 3 ? rows * G * 4u + rows * z4_words(G) * 4u : rows * G * kMetaGroupBytes<META>;
}
__device__ __forceinline__ float meta_scale(uint32_t m) { return half_lo(m); }
__device__ __forceinline__ float meta_zero(uint32_t m) { return half_hi(m); }
__device__ __forceinline__ float meta_scale(u32x2 m) { return __uint_as_float(m.x); }
__device__ __forceinline__ float meta_zero(u32x2 m) { return __uint_as_float(m.y); }
__device__ __forceinline__ float meta_scale(Scale16 m) { return half_lo(m.v); }
__device__ __forceinline__ float meta_zero(Scale16) { return 8.0f; }
__device__ __forceinline__ float meta_scale(ScaleZ4 m) { return __uint_as_float(m.s); }
// The zero of a group; zsh = 4 (g mod 8), the bit offset of group g's nibble
// in its META 3 zero word (ignored by the other forms).
template <typename M>
__device__ __forceinline__ float meta_zero_at(const M& m, uint32_t) { return meta_zero(m); }
__device__ __forceinline__ float meta_zero_at(const ScaleZ4& m, uint32_t zsh) {
    return static_cast<float>(__builtin_amdgcn_ubfe(m.zw, zsh, 4));
}
// A group's metadata from a buffer resource at byte offset off (META 3: the
// scale at off, the zero word at zoff).
// (AUX: the load's cache-policy bits)
template <int META, int AUX>
__device__ __forceinline__ MetaWord<META> load_meta(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t zoff = 0) {
    if constexpr (META == 1) {
        return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, AUX);
    } else if constexpr (META == 2) {
        return Scale16{static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, AUX))};
    } else if constexpr (META == 3) {
        return ScaleZ4{__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, AUX),
                       __builtin_amdgcn_raw_buffer_load_b32(r, zoff, 0, AUX)};
    } else {
        return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, AUX);
    }
}
// Byte offset of the zero word of group g of `row` (META 3): past the rows x G
// scales.  Out-of-range inputs give an offset past the buffer (reads zero).
__device__ __forceinline__ uint32_t z4_offset(uint32_t rows, uint32_t G, uint32_t row, uint32_t g) {
    return rows * G * 4u + (__umul24(row, z4_words(G)) + (g >> 3)) * 4u;
}

// Range-checked buffer loads: an offset at or past the resource's byte range
// returns 0 without a memory access, so a load can be issued unconditionally
// (straight-line code keeps the compiler's load-count waits exact).
constexpr uint32_t kBufWord3 = 0x00020000u;  // raw 32-bit buffer, gfx9-family format
constexpr uint32_t kBufOOB = 0x80000000u;    // an offset past every range used here
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, kBufWord3);
}
__device__ __forceinline__ float buf_load_f32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
// A per-lane offset the compiler cannot see through: loads whose offsets are
// selected between a real one and kBufOOB then stay straight-line code (left
// visible, identical out-of-range loads get merged under a branch whose join
// waits for every outstanding load).
__device__ __forceinline__ uint32_t opaque_offset(uint32_t off) {
    asm volatile("" : "+v"(off));
    return off;
}

// Cross-lane reductions by DPP lane moves inside the VALU (no LDS round trip,
// unlike ds_bpermute): quad_perm [1,0,3,2] and [2,3,0,1] exchange lanes i^1
// and i^2, row_half_mirror maps lane i to 7-i within each 8, row_mirror maps
// lane i to 15-i within each 16.  After the quad steps every lane of a quad
// holds the quad's value, so each mirror step pairs it with the neighbouring
// quad / half-row: the result is the reduction over the aligned group of N
// lanes, identical in every lane of the group.
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, dpp_i32<CTRL>(__builtin_bit_cast(int, v)));
}

// Reduction over each aligned group of N in {2, 4, 8, 16} consecutive lanes.
template <int N>
__device__ __forceinline__ float lanes_sum(float v) {
    static_assert(N == 2 || N == 4 || N == 8 || N == 16, "lane group");
    v += dpp_f32<kDppXor1>(v);
    if constexpr (N >= 4) v += dpp_f32<kDppXor2>(v);
    if constexpr (N >= 8) v += dpp_f32<kDppHalfMirror>(v);
    if constexpr (N >= 16) v += dpp_f32<kDppMirror>(v);
    return v;
}
template <int N>
__device__ __forceinline__ int lanes_sum_i(int v) {
    static_assert(N == 2 || N == 4 || N == 8 || N == 16, "lane group");
    v += dpp_i32<kDppXor1>(v);
    if constexpr (N >= 4) v += dpp_i32<kDppXor2>(v);
    if constexpr (N >= 8) v += dpp_i32<kDppHalfMirror>(v);
    if constexpr (N >= 16) v += dpp_i32<kDppMirror>(v);
    return v;
}
template <int N>
__device__ __forceinline__ float lanes_max(float v) {
    static_assert(N == 2 || N == 4 || N == 8 || N == 16, "lane group");
    v = fmaxf(v, dpp_f32<kDppXor1>(v));
    if constexpr (N >= 4) v = fmaxf(v, dpp_f32<kDppXor2>(v));
    if constexpr (N >= 8) v = fmaxf(v, dpp_f32<kDppHalfMirror>(v));
    if constexpr (N >= 16) v = fmaxf(v, dpp_f32<kDppMirror>(v));
    return v;
}

// v[l] + v[l ^ M] in every lane l, for M = 8 (DPP row_ror:8 within a row of
// 16), 16 and 32 (gfx950 v_permlane16_swap / v_permlane32_swap: both
// outputs of the swap together hold the two halves of every pair).
template <int M>
__device__ __forceinline__ float xor_pair_sum(float v) {
    static_assert(M == 8 || M == 16 || M == 32, "pair distance");
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    if constexpr (M == 8) {
        return v + dpp_f32<0x128>(v);
    } else if constexpr (M == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        return __builtin_bit_cast(float, static_cast<uint32_t>(r[0])) + __builtin_bit_cast(float, static_cast<uint32_t>(r[1]));
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        return __builtin_bit_cast(float, static_cast<uint32_t>(r[0])) + __builtin_bit_cast(float, static_cast<uint32_t>(r[1]));
    }
}

__device__ __forceinline__ float readlane_f32(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Sum over the 64 lanes of a wave (rows of 16 by DPP, then the four row sums
// read as scalars); every lane gets the total.  Must be called by the whole
// wave (all lanes active).
__device__ __forceinline__ float wave_sum(float v) {
    v = lanes_sum<16>(v);
    return (readlane_f32(v, 0) + readlane_f32(v, 16)) + (readlane_f32(v, 32) + readlane_f32(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
    v = lanes_max<16>(v);
    return fmaxf(fmaxf(readlane_f32(v, 0), readlane_f32(v, 16)), fmaxf(readlane_f32(v, 32), readlane_f32(v, 48)));
}

// Sum over all threads of a block (blockDim.x a multiple of 64, <= 1024).
// `red` is __shared__ scratch of at least 16 floats.  Every thread gets the total.
__device__ __forceinline__ float block_sum(float v, float* red) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = threadIdx.x / kWave;
    const int nw = (blockDim.x + kWave - 1) / kWave;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) red[wid] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < nw; ++i) t += red[i];
    return t;
}

// block_sum for a block of NW waves known at compile time (no blockDim read,
// which is a vector-memory load of the dispatch packet on this target).
template <int NW>
__device__ __forceinline__ float block_sum_t(float v, float* red) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = threadIdx.x / kWave;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) red[wid] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < NW; ++i) t += red[i];
    return t;
}

__device__ __forceinline__ float silu_dev(float x) { return x / (1.0f + expf(-x)); }

__device__ __forceinline__ float sigmoid_dev(float x) {
    if (x >= 0.0f) {
        const float e = expf(-x);
        return 1.0f / (1.0f + e);
    }
    const float e = expf(x);
    return e / (1.0f + e);
}

__device__ __forceinline__ float softplus_dev(float x) {
    if (x > 20.0f) return x;
    if (x < -20.0f) return expf(x);
    return log1pf(expf(x));
}

// Order-preserving map of a float to uint32 (larger float -> larger key);
// NaN maps below -inf so it never wins an argmax.
__device__ __forceinline__ uint32_t float_order_key(float v) {
    if (v != v) return 0u;
    const uint32_t b = v == 0.0f ? 0u : __float_as_uint(v);  // -0 ties with +0, as in a float compare
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float float_from_order_key(uint32_t k) {
    const uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __uint_as_float(b);
}

// (value, index) packed so that the numeric max of the key is the largest value
// and, among equal values, the lowest index.
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t idx) {
    return (static_cast<uint64_t>(float_order_key(v)) << 32) | static_cast<uint64_t>(0xffffffffu - idx);
}

__device__ __forceinline__ uint64_t u64_max(uint64_t a, uint64_t b) { return a > b ? a : b; }

template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
    const uint32_t lo = static_cast<uint32_t>(dpp_i32<CTRL>(static_cast<int>(static_cast<uint32_t>(v))));
    const uint32_t hi = static_cast<uint32_t>(dpp_i32<CTRL>(static_cast<int>(static_cast<uint32_t>(v >> 32))));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}
// maximum over the wave, in every lane: DPP steps inside each row of 16
// lanes (as the float reductions above), then two lane swaps across rows
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    v = u64_max(v, dpp_u64<kDppXor1>(v));
    v = u64_max(v, dpp_u64<kDppXor2>(v));
    v = u64_max(v, dpp_u64<kDppHalfMirror>(v));
    v = u64_max(v, dpp_u64<kDppMirror>(v));
#pragma unroll
    for (int off = 16; off <= 32; off <<= 1) {
        const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), off, kWave);
        const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), off, kWave);
        v = u64_max(v, (static_cast<uint64_t>(hi) << 32) | lo);
    }
    return v;
}

}  // namespace xqhip
