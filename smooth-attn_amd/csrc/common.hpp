// Shared device helpers for the gfx950 smooth-attn kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "smooth_attn_amd.h"

namespace sa {

using bf16 = __bf16;
using f16 = _Float16;

// Epsilon added to every row sum (reference kernels.py:57, :529, :1584).
constexpr float kEps = 1e-12f;

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(f16 x) { return static_cast<float>(x); }
__device__ __forceinline__ float to_f32(bf16 x) { return static_cast<float>(x); }

template <typename T>
__device__ __forceinline__ T from_f32(float x) { return static_cast<T>(x); }

// v_sqrt_f32.  Every argument on this path is a^2 + 4 >= 4, so the denormal
// pre-scaling of the correctly rounded sqrtf sequence is never needed.
__device__ __forceinline__ float fast_sqrt(float x) { return __builtin_amdgcn_sqrtf(x); }
__device__ __forceinline__ float fast_rsqrt(float x) { return __builtin_amdgcn_rsqf(x); }

// Lane-to-lane moves inside a 16-lane DPP row.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

// Sum over the 64 lanes of a wavefront; every lane receives the total.
// quad_perm xor1 / xor2, then half-row and row mirrors give each 16-lane row
// its own sum in all of its lanes; the four row sums are combined with
// v_readlane in a fixed order, so the result is deterministic.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_mov<0x141>(v);  // row_half_mirror
    v += dpp_mov<0x140>(v);  // row_mirror
    const int b = __float_as_int(v);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(b, 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(b, 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(b, 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(b, 48));
    return (r0 + r1) + (r2 + r3);
}

// Maximum over the 64 lanes of a wavefront (same pattern as wave_sum).
__device__ __forceinline__ float wave_max(float v) {
    v = __builtin_fmaxf(v, dpp_mov<0xB1>(v));
    v = __builtin_fmaxf(v, dpp_mov<0x4E>(v));
    v = __builtin_fmaxf(v, dpp_mov<0x141>(v));
    v = __builtin_fmaxf(v, dpp_mov<0x140>(v));
    const int b = __float_as_int(v);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(b, 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(b, 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(b, 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(b, 48));
    return __builtin_fmaxf(__builtin_fmaxf(r0, r1), __builtin_fmaxf(r2, r3));
}

// 16-byte vector type used for coalesced global traffic.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ u32x4 load16(const T* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

template <typename T>
__device__ __forceinline__ void store16(T* p, u32x4 v) {
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// Element i of a row fragment held as 32-bit words (16-bit types pack two
// elements per word, low half first).
template <typename T>
__device__ __forceinline__ float elem(const uint32_t* words, int i);

template <>
__device__ __forceinline__ float elem<float>(const uint32_t* words, int i) {
    return __uint_as_float(words[i]);
}
template <>
__device__ __forceinline__ float elem<bf16>(const uint32_t* words, int i) {
    const uint32_t w = words[i >> 1];
    return __uint_as_float((i & 1) ? (w & 0xFFFF0000u) : (w << 16));
}
template <>
__device__ __forceinline__ float elem<f16>(const uint32_t* words, int i) {
    const uint32_t w = words[i >> 1];
    const uint16_t h = (i & 1) ? static_cast<uint16_t>(w >> 16) : static_cast<uint16_t>(w & 0xFFFFu);
    return static_cast<float>(__builtin_bit_cast(f16, h));
}

// Two floats packed into one 32-bit word of a 16-bit type (RNE); a
// two-element vector conversion is a single v_cvt_pk_{bf16,f16}_f32.
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi);
template <>
__device__ __forceinline__ uint32_t pack2<bf16>(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo, hi}), bf16x2));
}
template <>
__device__ __forceinline__ uint32_t pack2<f16>(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo, hi}), f16x2));
}

// Bytes 2 sel and 2 sel + 1 of a word of e4m3fn codes as two 16-bit values
// (v_cvt_scalef32_pk_{bf16,f16}_fp8 with scale 1: exact, since every
// e4m3fn value, subnormals included, is a bf16 and an f16 value).
template <typename T, bool SEL>
__device__ __forceinline__ uint32_t widen2_e4m3(uint32_t word) {
    if constexpr (std::is_same_v<T, bf16>)
        return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(word, 1.0f, SEL));
    else
        return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(word, 1.0f, SEL));
}

// 16 e4m3fn values (one 16-byte word) as 16 values of T (two words), exact:
// elements 0-7 in lo, 8-15 in hi.
template <typename T>
__device__ __forceinline__ void widen_e4m3x16(u32x4 in, u32x4& lo, u32x4& hi) {
    lo = u32x4{widen2_e4m3<T, false>(in.x), widen2_e4m3<T, true>(in.x), widen2_e4m3<T, false>(in.y),
               widen2_e4m3<T, true>(in.y)};
    hi = u32x4{widen2_e4m3<T, false>(in.z), widen2_e4m3<T, true>(in.z), widen2_e4m3<T, false>(in.w),
               widen2_e4m3<T, true>(in.w)};
}

// Load 16 bytes into words[0..3] / store words[0..3] as 16 bytes.
template <typename T>
__device__ __forceinline__ void load_words(const T* p, uint32_t* words) {
    const u32x4 v = load16(p);
    words[0] = v.x;
    words[1] = v.y;
    words[2] = v.z;
    words[3] = v.w;
}
template <typename T>
__device__ __forceinline__ void store_words(T* p, const uint32_t* words) {
    store16(p, u32x4{words[0], words[1], words[2], words[3]});
}

// Pack VEC = 16 / sizeof(T) floats into 4 words of T.
template <typename T>
__device__ __forceinline__ void pack_row16(const float* in, uint32_t* words) {
    if constexpr (sizeof(T) == 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) words[i] = __float_as_uint(in[i]);
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) words[i] = pack2<T>(in[2 * i], in[2 * i + 1]);
    }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int status_from_launch() {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : static_cast<int>(e);
}

// A planned row-kernel launch: the kernel (host stub address), its grid and
// block, and how rows map onto waves.  The row entry points launch exactly
// the plan their *_launch_info query describes.
struct RowLaunch {
    const void* fn = nullptr;
    dim3 grid, block;
    int variant = SA_ROW_SCALAR;
    int rows_per_block = 1, waves_per_row = 1, elems_per_load = 1, row_pass_elems = 64;
};

// A dispatch covers grid.x * block.x work-items, a count the dispatch packet
// holds in 32 bits: with one block row per 64 * waves_per_row lanes this caps
// n_rows at 2^26 for one wave per row, 2^24 for 4 and 2^23 for 8.
inline bool grid_fits(dim3 grid, dim3 block) {
    return static_cast<uint64_t>(grid.x) * block.x <= static_cast<uint64_t>(UINT32_MAX);
}

inline int launch_row(const RowLaunch& L, void** args, hipStream_t st) {
    if (!grid_fits(L.grid, L.block)) return SA_ERR_BAD_SHAPE;
    const hipError_t e = hipLaunchKernel(L.fn, L.grid, L.block, args, 0, st);
    return e == hipSuccess ? status_from_launch() : static_cast<int>(e);
}

// *info from a plan plus the compiled kernel's registers, static LDS and
// occupancy on the current device.
inline int describe_row_launch(const RowLaunch& L, sa_launch_info* info) {
    if (!grid_fits(L.grid, L.block)) return SA_ERR_BAD_SHAPE;
    hipFuncAttributes a{};
    hipError_t e = hipFuncGetAttributes(&a, L.fn);
    if (e != hipSuccess) return static_cast<int>(e);
    int nb = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, L.fn, static_cast<int>(L.block.x), 0);
    if (e != hipSuccess) return static_cast<int>(e);
    info->variant = L.variant;
    info->grid_x = static_cast<int>(L.grid.x);
    info->block_threads = static_cast<int>(L.block.x);
    info->rows_per_block = L.rows_per_block;
    info->waves_per_row = L.waves_per_row;
    info->elems_per_load = L.elems_per_load;
    info->row_pass_elems = L.row_pass_elems;
    info->n_vgprs = a.numRegs;
    info->shared_mem_bytes = static_cast<int>(a.sharedSizeBytes);
    info->blocks_per_cu = nb;
    return 0;
}

}  // namespace sa
