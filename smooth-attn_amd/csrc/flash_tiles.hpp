// Tile helpers shared by the fused-attention kernels that run one wave per
// SIMD with direct-to-LDS tiles (flash_wide.hip, flash_fwd_pipe.hip): tile
// loads, LDS swizzles, MFMA operand reads and the squareplus weights.
#pragma once

#include "flash_common.hpp"

namespace sa {

constexpr int kWW = 4;            // waves per block
constexpr int kWT = 32;           // rows per staged tile
constexpr int kWRows = 32 * kWW;  // rows a block owns

// LDS tiles are unpadded [kWT][D] rows of 16-byte chunks filled by direct
// global -> LDS loads (lane i of a wave writes bytes [16 i, 16 i + 16) after
// the wave's base, so one instruction fills 1 KB).  The LDS serves a 16-byte
// read 16 lanes per cycle and an 8-byte transposing read 32 lanes per cycle,
// conflict-free when the lanes of a cycle cover 256 distinct bytes modulo
// 256.  Rows are 512 bytes (a multiple of 256), so logical chunk c of row r
// is stored at chunk c ^ swz(r):
//  * ROW layout (row reads: 16 rows at one logical chunk): swz = r mod 16
//    gives the 16 rows 16 distinct 16-byte slots;
//  * TR layout (transposing reads: 4 consecutive rows x 64 bytes per 32
//    lanes): swz = 4 (r mod 4) moves the rows' 64-byte groups to 4 distinct
//    64-byte slots.
// A tile read both ways is loaded twice, once per layout.
template <bool TR>
__device__ __forceinline__ int wswz(int r) {
    return TR ? 4 * (r & 3) : (r & 15);
}

typedef __attribute__((address_space(3))) void wide_lds_void_t;

// One 16-byte buffer -> LDS load per lane: lane i writes bytes [16 i, 16 i + 16)
// after lds_base (wave-uniform), read from byte voff of the resource.
__device__ __forceinline__ void wide_dma16(__amdgpu_buffer_rsrc_t rs, int voff, void* lds_base) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (wide_lds_void_t*)(lds_base), 16, voff, 0, 0, 0);
}

// s_waitcnt vmcnt(0): this wave's direct-to-LDS loads have landed.
__device__ __forceinline__ void wide_wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// p, computed from wave-uniform values, as a scalar (buffer resources are built from it).
__device__ __forceinline__ const unsigned char* wide_uniform_ptr(const unsigned char* p) {
    const uint64_t u = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u >> 32));
    return reinterpret_cast<const unsigned char*>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Loads of kWT-row tiles of a [T, D] 16-bit matrix (row stride rstride
// elements) into LDS in layout TR: each wave issues kWT * D * 2 / 1024 / kWW
// instructions of 1 KB.  The per-lane byte offsets depend only on the layout
// and the row stride, so they are computed once; each tile then takes a
// buffer resource at its first row whose size ends at row T - 1 (rows past
// it read as zeros).
template <typename T, int D, bool TR>
struct WideLoader {
    static constexpr int CPR = D / 8;                // 16-byte chunks per row
    static constexpr int NI = kWT * CPR / 64 / kWW;  // instructions per wave
    int voff[NI];
    int lds_off[NI];  // wave-uniform element offset of each instruction's 1 KB
    int64_t row_bytes;
    __device__ __forceinline__ WideLoader(int64_t rstride, int wave, int lane) : row_bytes(rstride * 2) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int base_slot = __builtin_amdgcn_readfirstlane((wave * NI + i) * 64);
            const int slot = base_slot + lane;
            const int r = slot / CPR;
            const int lc = (slot - r * CPR) ^ wswz<TR>(r);
            voff[i] = static_cast<int>(r * row_bytes) + 16 * lc;
            lds_off[i] = base_slot * 8;
        }
    }
    // rows r0 .. r0 + kWT - 1 of the matrix at base into lds
    __device__ __forceinline__ void issue(const T* base, int r0, int T_, T* lds) const {
        const int rows = min(kWT, T_ - r0);
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<T*>(base + static_cast<int64_t>(r0) * (row_bytes / 2)), 0, static_cast<int>(rows * row_bytes),
            0x00020000);
#pragma unroll
        for (int i = 0; i < NI; ++i) wide_dma16(rs, voff[i], lds + lds_off[i]);
    }
};

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

// A lane's D / 16 operand chunks of one row: x[c] = row[16c + 8 hi .. +7].
template <int D, typename T>
__device__ __forceinline__ void load_frags(const T* row, int hi, u32x4 (&x)[D / 16]) {
#pragma unroll
    for (int c = 0; c < D / 16; ++c) x[c] = *reinterpret_cast<const u32x4*>(row + 16 * c + 8 * hi);
}

// C += A B^T over D: A rows from a ROW-layout LDS tile (row l32), B from a
// lane's register chunks.  All reads are issued before the first MFMA, so
// their latency is paid once per call rather than once per MFMA.
template <typename T, int D>
__device__ __forceinline__ f32x16 mma_rows16(const T* lds_rows, int l32, int hi, const u32x4 (&b)[D / 16],
                                             f32x16 c) {
    using V8 = typename MfmaOps<T>::vec8;
    const T* ar = lds_rows + l32 * D;
    const int sw = wswz<false>(l32);
    u32x4 a[D / 16];
#pragma unroll
    for (int i = 0; i < D / 16; ++i) a[i] = *reinterpret_cast<const u32x4*>(ar + 8 * ((2 * i + hi) ^ sw));
    __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the MFMAs
#pragma unroll
    for (int i = 0; i < D / 16; ++i) c = MfmaOps<T>::mma(as_vec8<V8>(a[i]), as_vec8<V8>(b[i]), c);
    return c;
}

// Pack a lane's 16 C-layout values as the two B operands over the tile rows.
template <typename T>
__device__ __forceinline__ void pack_b(const float (&x)[16], u32x4 (&w)[2]) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
        w[j] = u32x4{pack2<T>(x[8 * j + 0], x[8 * j + 1]), pack2<T>(x[8 * j + 2], x[8 * j + 3]),
                     pack2<T>(x[8 * j + 4], x[8 * j + 5]), pack2<T>(x[8 * j + 6], x[8 * j + 7])};
}

// A^T operands of acc[dt] (rows d = 32 dt + ..) += A^T(d, r) X(r, col) over
// a tile's 32 rows r: transposing reads of a TR-layout tile (lane supplies
// row 4 (l / 32) + (l % 16) / 4, column 32 dt + 16 ((l / 16) % 2) + 4 (l % 4);
// the 16 lanes of its group receive column 32 dt + l % 32 of rows +0..3).
// Read before the B operands exist, so the reads overlap the work that
// produces them.
template <typename T, int D>
struct ColOperands {
    using V8 = typename MfmaOps<T>::vec8;
    V8 a[D / 32][2];
    __device__ __forceinline__ void read(const T* lds_tr, int lane) {
        const int r = 4 * (lane >> 5) + ((lane & 15) >> 2);
        const int sw = wswz<true>(r);  // the same for rows r + 8, r + 16, r + 24
        const T* base = lds_tr + r * D + 4 * (lane & 1);
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
            const int chunk = (4 * dt + 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1)) ^ sw;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const T* p0 = base + 16 * j * D + 8 * chunk;
                a[dt][j] = lds_read_tr16_pair<V8>(p0, p0 + 8 * D);
            }
        }
        __builtin_amdgcn_sched_barrier(0);  // issue the reads here, ahead of the caller's VALU work
    }
    // acc[dt] += A^T X, X the packed B operands
    __device__ __forceinline__ void mma(const u32x4 (&x)[2], f32x16 (&acc)[D / 32]) const {
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[dt] = MfmaOps<T>::mma(a[dt][j], as_vec8<V8>(x[j]), acc[dt]);
    }
};

// Write a lane's C-layout rows of acc (d = 32 dt + 8 m + 4 hi .. +3) times f
// into its output row as 8-byte stores.
template <typename T, int D>
__device__ __forceinline__ void store_cols16(T* row, int hi, const f32x16 (&acc)[D / 32], float f) {
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const uint2 w{pack2<T>(acc[dt][4 * m + 0] * f, acc[dt][4 * m + 1] * f),
                          pack2<T>(acc[dt][4 * m + 2] * f, acc[dt][4 * m + 3] * f)};
            *reinterpret_cast<uint2*>(row + dt * 32 + 8 * m + 4 * hi) = w;
        }
    }
}

}  // namespace sa
