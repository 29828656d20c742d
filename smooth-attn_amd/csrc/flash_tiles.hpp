// Helpers shared by the fused-attention kernels: direct-to-LDS tile loads,
// the squareplus weight with its reciprocal root, and branch-free masking.
#pragma once

#include "flash_common.hpp"

namespace sa {

typedef __attribute__((address_space(3))) void tile_lds_void_t;

// Buffer resource over the nbytes bytes from base (raw, no stride): loads at
// or past nbytes return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const void* base, int nbytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, nbytes, 0x00020000);
}

// One 16-byte buffer -> LDS load per lane: lane i writes bytes [16 i, 16 i + 16)
// after lds_base (wave-uniform), read from byte voff of the resource.
__device__ __forceinline__ void tile_dma16(__amdgpu_buffer_rsrc_t rs, int voff, void* lds_base) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (tile_lds_void_t*)(lds_base), 16, voff, 0, 0, 0);
}

// Per-lane byte offset past the buffer resource of every tile the attention
// kernels load (their tiles span at most 64 rows of under 2^25 bytes, so a
// resource holds at most 2^31 - 1024 bytes): the lane's load returns zeros.
// Lanes whose 16-byte chunk lies past the tensors' head dim take it.
constexpr int kPastTile = 0x7FFFFFF0;

// s_waitcnt vmcnt(0): this wave's direct-to-LDS loads have landed.
__device__ __forceinline__ void tile_wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// p, computed from wave-uniform values, as a scalar (buffer resources are built from it).
__device__ __forceinline__ const unsigned char* tile_uniform_ptr(const unsigned char* p) {
    const uint64_t u = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u >> 32));
    return reinterpret_cast<const unsigned char*>((static_cast<uint64_t>(hi) << 32) | lo);
}

// y = squareplus(2 s scale - 1)^2 = (a + r)^2, a = s scale - 1/2,
// r = sqrt(a^2 + 1); rr = 1 / r.
template <bool EXACT>
__device__ __forceinline__ void weight_rr16(float s, float sc, float& y, float& rr) {
    const float a = __builtin_fmaf(s, sc, -0.5f);
    const float u = __builtin_fmaf(a, a, 1.f);
    float r;
    if constexpr (EXACT) {
        r = __builtin_sqrtf(u);
        rr = 1.f / r;
    } else {
        rr = fast_rsqrt(u);
        r = u * rr;
    }
    const float sp = a + r;
    y = sp * sp;
}

// x where c holds, +0 where not, as a bitwise AND: the value is always
// computed, so the compiler cannot turn the choice into a branch around the
// computation (a divergent branch per score, which it does for a select).
__device__ __forceinline__ float keep_if(bool c, float x) {
    return __uint_as_float(__float_as_uint(x) & (0u - static_cast<uint32_t>(c)));
}

}  // namespace sa
