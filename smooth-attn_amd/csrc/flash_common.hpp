// Shared pieces of the fused squareplus attention kernels (gfx950 MFMA).
//
// Operand layouts of the MFMAs used here (checked on the device):
//  v_mfma_f32_32x32x16_{bf16,f16}: A (32 x 16) lane l holds row l%32 and k
//    8*(l/32) .. +7; B (16 x 32) lane l holds column l%32 and the same k;
//    C/D (32 x 32 fp32, 16 per lane) lane l holds column l%32 and rows
//    (v/4)*8 + (l/32)*4 + v%4 for v = 0..15.
//  ds_read_b64_tr_b16: inside each group of 16 lanes, lane i receives element
//    j = 0..3 from the address supplied by lane 4j + i/4, plus i%4 elements.
//
// The kernels compute S^T = K Q^T (keys as rows), so each lane ends up with
// one query column and 16 keys of a 32 x 32 tile.  Those scores, once turned
// into weights and rounded, are already laid out as the B operand of
// O^T += V^T P^T, so P never leaves registers.  V^T is read from a row-major
// V tile in LDS with the transposing LDS load.
#pragma once

#include "common.hpp"

namespace sa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

template <typename T>
struct MfmaOps;

template <>
struct MfmaOps<bf16> {
    using vec8 = bf16x8;
    static __device__ __forceinline__ f32x16 mma(vec8 a, vec8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};

template <>
struct MfmaOps<f16> {
    using vec8 = f16x8;
    static __device__ __forceinline__ f32x16 mma(vec8 a, vec8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};

// Reinterpret 4 words as an 8-element MFMA operand.
template <typename V>
__device__ __forceinline__ V as_vec8(u32x4 w) {
    return __builtin_bit_cast(V, w);
}

// Transposing 8-byte LDS read (4 x 16-bit elements); p points into LDS.
__device__ __forceinline__ uint2 lds_read_tr16(const void* p) {
    typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
    typedef __attribute__((address_space(3))) char lds_char;
    const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)((lds_char*)(p)));
    return __builtin_bit_cast(uint2, v);
}

// Two transposing reads assembled into one 8-element MFMA operand (elements
// 0-3 from p0, 4-7 from p1) with a vector shuffle, so the two 64-bit results
// can land directly in the operand's register quad.
template <typename V>
__device__ __forceinline__ V lds_read_tr16_pair(const void* p0, const void* p1) {
    typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
    typedef __attribute__((address_space(3))) char lds_char;
    typedef short s16x8 __attribute__((ext_vector_type(8)));
    const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)((lds_char*)(p0)));
    const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)((lds_char*)(p1)));
    const s16x8 ab = __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(V, ab);
}

// Block -> (step, unit, sub) for grids of n_steps x n_units x n_sub blocks,
// where a unit is a KV head ((b, hk) pair), sub a query head sharing it and
// step the tile position (step 0 runs first: callers map it to their
// heaviest tiles).  Blocks are dealt to the 8 XCDs round-robin by index.
// When n_units is a multiple of 8, XCD x gets units x, x+8, ... (each KV
// head's data is then fetched into one XCD's L2 only), taken a few units at
// a time: a group holds at least xcd_slots blocks (the blocks one XCD runs
// at once), with the steps of the group's heads in order and its heads
// fastest, so the blocks in flight share a handful of K/V (or Q/dO) streams
// and the group's heavy steps still start early.  Otherwise step-major over
// all (unit, sub).
__device__ __forceinline__ void grouped_block(int id, int n_units, int n_sub, int n_steps, int xcd_slots,
                                              int& step, int& unit, int& sub) {
    if ((n_units & 7) == 0) {
        const int x = id & 7;
        const int j = id >> 3;
        const int nh = (n_units >> 3) * n_sub;  // (unit, sub) pairs on this XCD
        const int gu = min(max(1, (xcd_slots + n_sub * n_steps - 1) / (n_sub * n_steps)), n_units >> 3);
        const int gh = gu * n_sub;  // pairs per group
        const int grp = j / (gh * n_steps);
        const int r = j - grp * (gh * n_steps);
        const int ghs = min(gh, nh - grp * gh);  // pairs in this group (the last may be short)
        step = r / ghs;
        const int hl = grp * gh + (r - step * ghs);
        const int ul = hl / n_sub;
        unit = ul * 8 + x;
        sub = hl - ul * n_sub;
    } else {
        const int per = n_units * n_sub;
        step = id / per;
        const int rest = id - step * per;
        unit = rest / n_sub;
        sub = rest - unit * n_sub;
    }
}

// squareplus(a)^2 with a = scale * s - 1/2 already folded in:
//   squareplus(2 s scale - 1) = (2 s scale - 1 + sqrt((2 s scale - 1)^2 + 4)) / 2
//                             = a + sqrt(a^2 + 1),   a = s scale - 1/2.
template <bool EXACT>
__device__ __forceinline__ float sp2_weight(float a) {
    const float u = __builtin_fmaf(a, a, 1.f);
    const float r = EXACT ? __builtin_sqrtf(u) : fast_sqrt(u);
    const float sp = a + r;
    return sp * sp;
}

}  // namespace sa
