// 16-bit (bf16 / fp16) fused causal squareplus attention at head dims 256
// and 512, forward and backward, on v_mfma_f32_16x16x32_{bf16,f16}.  Head
// dims 136..248 and 264..504 (multiples of 8) run on the next of these
// kernels with the columns past them read as zeros and not stored.
//
// Same mathematics and rounding points as the D <= 128 kernels
// (flash_fwd.hip, flash_bwd.hip; reference kernels.py:1536-1631 and
// :1667-1909): fp32 scores and weights, P and dS rounded to the input type
// before their products, fp32 accumulation, row sums of the fp32 weights.
//
// Every kernel here gives a wave 16 rows (queries for the forward and dQ,
// keys for dK and dV) on v_mfma_f32_16x16x32: at D = 256 the accumulators of
// 16 rows (16 tiles of 16 x 16, 64 registers per lane) leave room for two
// waves per SIMD, where 32 rows on the 32x32x16 MFMA would need one wave per
// SIMD.  Blocks of 8 waves own 128 rows and walk 64-row tiles of the other
// side through a 2-stage LDS ring (two 64 KB arrays) filled by direct-to-LDS
// loads, one barrier per tile (D = 512: 4 waves, one per SIMD, own 64 rows
// and walk 32-row tiles); the tile loops are unrolled by two so each
// tile names its stage statically and its LDS reads never wait for the DMA
// filling the other stage.  dK and dV are separate kernels (both
// accumulators plus the K and V operands would not fit two waves per SIMD).
//
// 16x16x32 operands: A lane l holds row l % 16, k = 8 (l / 16) .. +7; B column
// l % 16, the same k; C column l % 16, rows 4 (l / 16) .. +3.  For
// contractions over D one side stays in registers and the other is a 16-byte
// row read of an LDS tile.  For contractions over the tile's rows, the C
// values of 16-row subtiles 2j and 2j + 1 (rows 4 (l / 16) + e and
// 16 + 4 (l / 16) + e) are the B operand of step j as they stand, and the A
// operand comes from two transposing reads of the row-major tile (lane
// supplies row 4 (l / 16) + (l % 16) / 4, and that + 16, columns 16 dt +
// 4 (l % 4): inside its 16-lane group lane i then receives column 16 dt + i of
// those rows).  LDS rows are 512 bytes; logical 16-byte chunk c of row r is
// stored at c ^ swz(r): r & 15 for row reads, 2 (r & 7) for transposing
// reads (8 rows x 32 bytes per cycle), and for tiles read both ways
// fk_swz(r) (below), which serves both.
#include <algorithm>
#include <type_traits>

#include "flash_tiles.hpp"
#include "flash_wide.hpp"
#include "dkdv_split.hpp"

namespace sa {
namespace {

template <typename E>
struct WideParams {
    const E* q;
    const E* k;
    const E* v;
    const E* o;     // backward input
    const E* dout;  // backward input
    const float* rs;  // backward input: forward row sums [B, Hq, T]
    E* out;           // forward output
    float* row_sums;  // forward output (nullable)
    E* dq;
    E* dk;
    E* dv;
    float* delta;  // [B, Hq, T]
    int64_t qs[4], ks[4], vs[4], os[4], dos[4], dqs[4], dks[4], dvs[4];
    int B, Hq, Hkv, T, G, window;
    int dr;  // head dim of the tensors (<= D, a multiple of 8; columns past it read as zero, are not stored)
    float scale;
    int n_split;  // dK/dV: query-range splits of every key block (1: none)
    float* part;  // n_split > 1: fp32 partials [n_split][B * Hkv][T][D] of the dK or dV kernel
};

// 16 bytes of columns d0 .. d0 + 7 of a row; PART (head dim dr below the
// kernel's D): zeros where they lie past dr (the load then reads column 0).
template <bool PART, typename T>
__device__ __forceinline__ u32x4 wide_cols(const T* row, int d0, int dr) {
    if constexpr (!PART) return *reinterpret_cast<const u32x4*>(row + d0);
    const u32x4 v = *reinterpret_cast<const u32x4*>(row + (d0 < dr ? d0 : 0));
    return d0 < dr ? v : u32x4{0u, 0u, 0u, 0u};
}

// Byte offset of a DMA lane's source: row drow, logical chunk c (8 columns);
// PART: chunks past the head dim dr take kPastTile.
template <bool PART>
__device__ __forceinline__ int wide_src_off(int drow, int c, int64_t rs, int dr) {
    if constexpr (!PART) return drow * static_cast<int>(rs) + (c << 4);
    return 8 * c < dr ? drow * static_cast<int>(rs) + (c << 4) : kPastTile;
}


// ---------------------------------------------------------------------------
// Forward: 16 query rows per wave on v_mfma_f32_16x16x32_{bf16,f16}
// ---------------------------------------------------------------------------
// With 32 rows per wave the O accumulators of D = 256 fill a wave's share of
// the register file at one wave per SIMD; 16 rows per wave halve them (O^T
// is 16 tiles of 16 x 16, 64 registers), so a block of 8 waves runs two per
// SIMD.  Per 64-key tile a wave runs S^T = K Q^T (4 key subtiles x 8 k
// steps) and O^T += V^T P^T (16 d tiles x 2 key steps) on the 16x16x32 MFMA:
// A lane l holds row l % 16, k = 8 (l / 16) .. +7; B column l % 16, the
// same k; C column l % 16, rows 4 (l / 16) .. +3.  The S^T accumulators of
// key subtiles 2j and 2j + 1 (keys 4 g + e and 16 + 4 g + e, g = l / 16)
// are the B operand P^T of key step j as they stand; the matching V^T A
// operand comes from two transposing reads of the row-major V tile (lane
// supplies row 4 g + (l % 16) / 4, and that + 16, columns 16 dt + 4 (l % 4):
// inside its 16-lane group lane i then receives d = 16 dt + i of keys 4 g + j
// and 16 + 4 g + j).  K and V tiles go straight from global memory into a
// 2-stage LDS ring (2 x 64 KB); K rows store logical chunk c at c ^ (r & 15)
// (16-byte row reads, 16 rows per cycle), V rows at c ^ 2 (r & 7)
// (transposing reads, 8 rows x 32 bytes per cycle): both conflict-free.
// Block shapes.  D = 256: 8 waves (two per SIMD), 128 rows per block,
// 64-row tiles.  D = 512 (head dims 264..512): the accumulators and
// operands of 16 rows take more than half of a SIMD's registers, so blocks
// of 4 waves run one per SIMD, 64 rows per block, over 32-row tiles.  Both
// stage 2 x 2 tiles of 32 KB (one block per CU).
template <int D>
struct WideCfg {
    static constexpr int NW = D > 256 ? 4 : 8;    // waves per block
    static constexpr int ROWS = 16 * NW;          // query (key) rows per block
    static constexpr int KT = D > 256 ? 32 : 64;  // rows per staged tile
};
constexpr int kWideMaxKT = 64;

// Per-lane source offset of DMA instruction i of a staged tile: the lane's
// chunk lies in tile row drow + i * rpi (drow from the buffer resource of
// instruction i, which starts rpi * i rows in), logical chunk pch ^ swz(row).
// When rpi is a multiple of 16 the swizzles (functions of row bits 0-3) give
// every instruction the same offset.
template <bool PART, int NI, int RPI, typename Swz>
__device__ __forceinline__ void wide_dma_offsets(int (&off)[NI], int drow, int pch, int64_t rs, int dr, Swz swz) {
#pragma unroll
    for (int i = 0; i < NI; ++i)
        off[i] = (RPI % 16 == 0 && i > 0) ? off[0] : wide_src_off<PART>(drow, pch ^ swz(drow + i * RPI), rs, dr);
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
template <typename T>
struct Mfma16;
template <>
struct Mfma16<bf16> {
    static __device__ __forceinline__ f32x4 mma(bf16x8 a, bf16x8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};
template <>
struct Mfma16<f16> {
    static __device__ __forceinline__ f32x4 mma(f16x8 a, f16x8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

// A wave's 16 result rows (C layout of the 16x16 tiles: lane l holds row
// l % 16, columns 16 dt + 4 (l / 16) .. +3), scaled by f, written through
// LDS so that consecutive lanes store whole rows in 16-byte chunks, with
// nontemporal stores (the results are not read again here, and their lines
// then do not evict the tiles other blocks still read from L2).  st: the
// wave's LDS area of 16 rows of 2 D + 16 bytes.  Rows at or past T and
// chunks past dr are not stored.
template <typename T, int D, bool PART>
__device__ __forceinline__ void wide_store_rows(unsigned char* st, const f32x4 (&acc)[D / 16], float f, T* base,
                                                int64_t rs, int row0, int T_, int dr, int lane) {
    constexpr int RB = 2 * D + 16, CPR = 2 * D / 16, RPI = 64 / CPR;
    const int g = lane >> 4, i16 = lane & 15;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt)
        *reinterpret_cast<uint2*>(st + i16 * RB + (16 * dt + 4 * g) * 2) =
            uint2{pack2<T>(acc[dt][0] * f, acc[dt][1] * f), pack2<T>(acc[dt][2] * f, acc[dt][3] * f)};
    // (a wave's LDS accesses complete in order: the reads below see its writes)
#pragma unroll
    for (int r0 = 0; r0 < 16; r0 += RPI) {
        const int r = r0 + lane / CPR, c = lane % CPR;
        const u32x4 v = *reinterpret_cast<const u32x4*>(st + r * RB + c * 16);
        if (row0 + r < T_ && (!PART || c * 8 < dr))
            __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(base + static_cast<int64_t>(row0 + r) * rs + c * 8));
    }
}

// The LDS area of wave w for wide_store_rows once the tile ring is free: the
// first half of the waves in stage array 0, the second in stage array 1.
template <int D>
__device__ __forceinline__ unsigned char* wide_store_area(unsigned char* lds0, unsigned char* lds1, int wave) {
    constexpr int NW = WideCfg<D>::NW;
    static_assert(NW / 2 * 16 * (2 * D + 16) <= 2 * WideCfg<D>::KT * 2 * D, "half the waves' rows per stage array");
    return (wave < NW / 2 ? lds0 : lds1) + (wave % (NW / 2)) * 16 * (2 * D + 16);
}

// FOLD (bf16, moderate positive scales): the S^T chains start at
// c0 = -1/(2 scale), so they hold s' = s - 1/(2 scale) and
// (a + sqrt(a^2 + 1))^2 = scale^2 (s' + sqrt(s'^2 + 1/scale^2))^2: the
// weights carry 1/scale^2 (one FMA per score fewer), cancelled between P V
// and the row sum.
template <typename T, int D, bool EXACT, bool FOLD>
__global__ __launch_bounds__(64 * WideCfg<D>::NW) void flash_fwd_wide_kernel(WideParams<T> p) {
    using V8 = typename MfmaOps<T>::vec8;
    constexpr int kFW = WideCfg<D>::NW, kFRows = WideCfg<D>::ROWS, kFKT = WideCfg<D>::KT;
    constexpr int ROWB = D * 2;          // bytes per K / V row
    constexpr int TB = kFKT * ROWB;      // bytes per tile
    constexpr int CPR = ROWB / 16;       // 16-byte chunks per row
    constexpr int NI = TB / 1024 / kFW;  // DMA instructions per wave per tensor and tile
    constexpr int RPI = 64 * kFW / CPR;  // rows one round of kFW instructions covers
    constexpr int NKS = kFKT / 16;       // 16-key S^T subtiles per tile
    // Two ring stages ([K, V] each) in separate arrays, the tile loop unrolled
    // by two: each tile names its stage statically, so the compiler knows its
    // LDS reads cannot touch the stage the next tile's DMA writes and does
    // not wait for that DMA first.
    __shared__ __attribute__((aligned(1024))) unsigned char lds0[2 * TB];
    __shared__ __attribute__((aligned(1024))) unsigned char lds1[2 * TB];
    auto stage_base = [&](auto st) -> unsigned char* {
        if constexpr (decltype(st)::value == 0) return lds0;
        else return lds1;
    };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4;
    const int i16 = lane & 15;
    const int T_ = p.T;
    const int nqb = (T_ + kFRows - 1) / kFRows;
    int step, unit, sub;
    grouped_block(blockIdx.x, p.B * p.Hkv, p.G, nqb, 32, step, unit, sub);  // heaviest query blocks first
    const int qb = nqb - 1 - step;
    const int b = unit / p.Hkv;
    const int hk = unit - b * p.Hkv;
    const int hq = hk * p.G + sub;

    const unsigned char* kp = tile_uniform_ptr(reinterpret_cast<const unsigned char*>(p.k + b * p.ks[0] + hk * p.ks[1]));
    const unsigned char* vp = tile_uniform_ptr(reinterpret_cast<const unsigned char*>(p.v + b * p.vs[0] + hk * p.vs[1]));
    const int64_t krs = p.ks[2] * 2, vrs = p.vs[2] * 2;

    // 8-wave blocks: waves w and w + 4 share a SIMD, and the second four take
    // the row slots in reverse, so each SIMD pairs an early-row wave with a
    // late-row one
    const int q_start = qb * kFRows;
    const int slot = (kFW == 8 && wave >= 4) ? 11 - wave : wave;
    const int q0w = q_start + 16 * slot;
    const int qi = q0w + i16;
    const int qrow = min(qi, T_ - 1);
    // Q^T as the B operand of S^T: k step ks holds d = 32 ks + 8 g .. +7 of query qi
    u32x4 qf[D / 32];
    {
        const T* qr = p.q + b * p.qs[0] + hq * p.qs[1] + qrow * p.qs[2];
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) qf[ks] = wide_cols<true>(qr, 32 * ks + 8 * g, p.dr);
    }

    const int W = p.window;
    const unsigned weff = W > 0 ? static_cast<unsigned>(W) : 0x7FFFFFFFu;
    const int n_kv = (T_ + kFKT - 1) / kFKT;
    const int kv_end = min((q_start + kFRows + kFKT - 1) / kFKT, n_kv);
    const int kv_begin = W > 0 ? max(0, q_start - W + 1) / kFKT : 0;
    const float sc = p.scale;

    // DMA: slot s = (kFW i + wave) * 64 + lane of a tile holds row s / CPR,
    // physical chunk s % CPR; rows past T read as zeros (they meet only masked
    // weights), and so do columns past the head dim.
    const int drow = (wave * 64 + lane) / CPR;
    const int pch = (wave * 64 + lane) % CPR;
    int koff[NI], voff[NI];
    wide_dma_offsets<true, NI, RPI>(koff, drow, pch, krs, p.dr, [](int r) { return r & 15; });
    wide_dma_offsets<true, NI, RPI>(voff, drow, pch, vrs, p.dr, [](int r) { return 2 * (r & 7); });
    auto issue = [&](int t, auto st) {
        const int k0 = t * kFKT;
        const int nrows = min(T_ - k0, kFKT);
        unsigned char* lk = stage_base(st);
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int skip = i * RPI;
            tile_dma16(__builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(kp + (k0 + skip) * krs), 0,
                                                         max((nrows - skip) * static_cast<int>(krs), 0), 0x00020000),
                       koff[i], lk + (i * kFW + wave) * 1024);
            tile_dma16(__builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(vp + (k0 + skip) * vrs), 0,
                                                         max((nrows - skip) * static_cast<int>(vrs), 0), 0x00020000),
                       voff[i], lk + TB + (i * kFW + wave) * 1024);
        }
    };

    const int vr = 4 * g + (i16 >> 2);
    const int vbase = vr * ROWB + (((lane & 3) >> 1) << 4) + 8 * (lane & 1);
    const int vsw = vr & 7;
    f32x4 oacc[D / 16];
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) oacc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float ssum0 = 0.f, ssum1 = 0.f;
    const float c0 = -0.5f / sc, c2 = 1.f / (sc * sc);

    auto tile = [&](bool masked, int t, auto st) {
        const int k0 = t * kFKT;
        const unsigned char* Kb = stage_base(st);
        const unsigned char* Vb = Kb + TB;
        f32x4 s[NKS];
#pragma unroll
        for (int kst = 0; kst < NKS; ++kst) {
            u32x4 ka[D / 32];
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks)
                ka[ks] = *reinterpret_cast<const u32x4*>(Kb + (16 * kst + i16) * ROWB + (((4 * ks + g) ^ i16) << 4));
            s[kst] = FOLD ? f32x4{c0, c0, c0, c0} : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) s[kst] = Mfma16<T>::mma(as_vec8<V8>(ka[ks]), as_vec8<V8>(qf[ks]), s[kst]);
        }
        // lane: query qi, keys k0 + 16 kst + 4 g + e
        const int dbase = qi - k0 - 4 * g;
        float y[4 * NKS];
#pragma unroll
        for (int kst = 0; kst < NKS; ++kst) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float w;
                if constexpr (FOLD) {
                    const float wf = s[kst][e] + fast_sqrt(__builtin_fmaf(s[kst][e], s[kst][e], c2));
                    w = wf * wf;
                } else {
                    w = sp2_weight<EXACT>(__builtin_fmaf(s[kst][e], sc, -0.5f));
                }
                y[4 * kst + e] = w;
            }
        }
        if (masked) {
#pragma unroll
            for (int i = 0; i < 4 * NKS; ++i)
                y[i] = keep_if(static_cast<unsigned>(dbase - 16 * (i / 4) - i % 4) < weff, y[i]);
        }
#pragma unroll
        for (int i = 0; i < 4 * NKS; ++i) {
            if (i & 1) ssum1 += y[i];
            else ssum0 += y[i];
        }
#pragma unroll
        for (int kk = 0; kk < kFKT / 32; ++kk) {
            const float* yk = y + 8 * kk;
            const u32x4 pw{pack2<T>(yk[0], yk[1]), pack2<T>(yk[2], yk[3]), pack2<T>(yk[4], yk[5]),
                           pack2<T>(yk[6], yk[7])};
            const V8 bop = as_vec8<V8>(pw);
#pragma unroll
            for (int dt = 0; dt < D / 16; ++dt) {
                const unsigned char* p0 = Vb + 32 * kk * ROWB + vbase + ((dt ^ vsw) << 5);
                oacc[dt] = Mfma16<T>::mma(lds_read_tr16_pair<V8>(p0, p0 + 16 * ROWB), bop, oacc[dt]);
            }
        }
    };

    // Iteration t requests tile t + 1 into the stage of tile t - 1 (free since
    // the barrier that ended t - 1), runs tile t, then waits for t + 1 and
    // publishes it.  Waves run only the tiles their rows see (masks only where
    // some pair is outside the causal window or past a window edge) but take
    // every barrier.
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    issue(kv_begin, S0{});
    tile_wait_vmem();
    __syncthreads();
    const int wf = q0w, wl = q0w + 15;  // the wave's query rows
    int t_first = kv_begin;
    if (W > 0 && wf - W + 1 > 0) t_first = max(t_first, (wf - W + 1) / kFKT);
    const int t_last = wf < T_ ? min(wl / kFKT, kv_end - 1) : t_first - 1;
    int ja = t_first;
    if (W > 0 && wl - W >= 0) ja = max(ja, (wl - W) / kFKT + 1);
    const int jb = (wf + 1) / kFKT;
    // Tile t (stage (t - kv_begin) & 1) runs while the DMA fills the other
    // stage with tile t + 1.  Waves run only the tiles their rows see, masked
    // outside [ja, jb), but take every barrier.
    auto run_tile = [&](int t, auto cur) {
        if (t + 1 < kv_end) issue(t + 1, std::integral_constant<int, 1 - decltype(cur)::value>{});
        if (t >= t_first && t <= t_last) tile(t < ja || t >= jb, t, cur);
        if (t + 1 < kv_end) {
            tile_wait_vmem();
            __syncthreads();
        }
    };
    for (int t = kv_begin; t < kv_end; t += 2) {
        run_tile(t, S0{});
        if (t + 1 < kv_end) run_tile(t + 1, S1{});
    }

    // row sums: lanes i16, i16 + 16, + 32, + 48 hold the four key groups of query qi
    float part = ssum0 + ssum1;
    part += __shfl_xor(part, 16);
    part += __shfl_xor(part, 32);
    const float tot = FOLD ? __builtin_fmaf(part, sc * sc, kEps) : part + kEps;
    const float inv = FOLD ? (sc * sc) / tot : 1.f / tot;
    if (qi < T_ && g == 0 && p.row_sums != nullptr) p.row_sums[(static_cast<int64_t>(b) * p.Hq + hq) * T_ + qi] = tot;
    __syncthreads();  // every wave is past its last tile: the ring is free
    wide_store_rows<T, D, true>(wide_store_area<D>(lds0, lds1, wave), oacc, inv, p.out + b * p.os[0] + hq * p.os[1],
                                p.os[2], q0w, T_, p.dr, lane);
}

// ---------------------------------------------------------------------------
// Backward: dQ (and delta), 16 query rows per wave on the 16x16x32 MFMA
// ---------------------------------------------------------------------------
// As the forward: 8 waves x 16 rows, two waves per SIMD, 64-key tiles in a
// 2-stage LDS ring.  Per tile: S^T = K Q^T and dP^T = V dO^T (dP^T chains
// start at -delta of the lane's query), dS on the VALU, then
// dQ^T += K^T dS^T with K^T from transposing reads of the K tile.  The K tile
// is read both ways, so it stores logical chunk c of row r at c ^ fk(r),
// fk(r) = 2 ((r & 7) ^ 4 h) | h with h = (r >> 3) & 1.  Transposing reads:
// bits 1-3 (the 32-byte unit) are injective on 8 consecutive rows and the
// units stay together.  Row reads: injective on 16 consecutive rows, and
// the 16-byte reads are served 8 lanes at a time, so rows r and r + 8 must
// not share an 8-row bank window either: with plain 2 (r & 7) | h they did
// (the head-dim-256 dQ and dK kernels then spent a quarter of their LDS
// cycles in bank conflicts), while flipping bit 2 of the unit for rows 8-15
// puts them in the other half (checked on the device: no conflict for
// either read).  V rows use c ^ (r & 15).
__device__ __forceinline__ int fk_swz(int r) {
    const int h = (r >> 3) & 1;
    return (((r & 7) ^ (h << 2)) << 1) | h;
}

// PART: the tensors' head dim p.dr is below D (columns past it read as zeros
// and are not stored); the kernels with PART false serve dr == D.
template <typename T, int D, bool EXACT, bool PART>
__global__ __launch_bounds__(64 * WideCfg<D>::NW) void flash_bwd_dq_wide_kernel(WideParams<T> p) {
    using V8 = typename MfmaOps<T>::vec8;
    constexpr int kFW = WideCfg<D>::NW, kFRows = WideCfg<D>::ROWS, kFKT = WideCfg<D>::KT;
    constexpr int ROWB = D * 2;
    constexpr int TB = kFKT * ROWB;
    constexpr int CPR = ROWB / 16;
    constexpr int NI = TB / 1024 / kFW;
    constexpr int RPI = 64 * kFW / CPR;
    constexpr int NKS = kFKT / 16;
    // Two ring stages ([K, V] each) in separate arrays, the tile loop unrolled
    // by two: each tile names its stage statically, so the compiler knows its
    // LDS reads cannot touch the stage the next tile's DMA writes and does
    // not wait for that DMA first.
    __shared__ __attribute__((aligned(1024))) unsigned char lds0[2 * TB];
    __shared__ __attribute__((aligned(1024))) unsigned char lds1[2 * TB];
    auto stage_base = [&](auto st) -> unsigned char* {
        if constexpr (decltype(st)::value == 0) return lds0;
        else return lds1;
    };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4;
    const int i16 = lane & 15;
    const int T_ = p.T;
    const int nqb = (T_ + kFRows - 1) / kFRows;
    int step, unit, sub;
    grouped_block(blockIdx.x, p.B * p.Hkv, p.G, nqb, 32, step, unit, sub);
    const int qb = nqb - 1 - step;
    const int b = unit / p.Hkv;
    const int hk = unit - b * p.Hkv;
    const int hq = hk * p.G + sub;
    const unsigned char* kp = tile_uniform_ptr(reinterpret_cast<const unsigned char*>(p.k + b * p.ks[0] + hk * p.ks[1]));
    const unsigned char* vp = tile_uniform_ptr(reinterpret_cast<const unsigned char*>(p.v + b * p.vs[0] + hk * p.vs[1]));
    const int64_t krs = p.ks[2] * 2, vrs = p.vs[2] * 2;

    const int q_start = qb * kFRows;
    const int slot = (kFW == 8 && wave >= 4) ? 11 - wave : wave;
    const int q0w = q_start + 16 * slot;
    const int qi = q0w + i16;
    const int qrow = min(qi, T_ - 1);
    // Q^T and dO^T as B operands: k step ks holds d = 32 ks + 8 g .. +7 of query qi;
    // delta = dO . O of that query (lanes i16 + 16 g share it)
    u32x4 qf[D / 32], df[D / 32];
    float dpart = 0.f;
    {
        const T* qr = p.q + b * p.qs[0] + hq * p.qs[1] + qrow * p.qs[2];
        const T* dr = p.dout + b * p.dos[0] + hq * p.dos[1] + qrow * p.dos[2];
        const T* orw = p.o + b * p.os[0] + hq * p.os[1] + qrow * p.os[2];
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) {
            qf[ks] = wide_cols<PART>(qr, 32 * ks + 8 * g, p.dr);
            df[ks] = wide_cols<PART>(dr, 32 * ks + 8 * g, p.dr);
            const u32x4 ov = wide_cols<PART>(orw, 32 * ks + 8 * g, p.dr);
            const uint32_t ow[4] = {ov[0], ov[1], ov[2], ov[3]};
            const uint32_t dw[4] = {df[ks][0], df[ks][1], df[ks][2], df[ks][3]};
#pragma unroll
            for (int e = 0; e < 8; ++e) dpart = __builtin_fmaf(elem<T>(dw, e), elem<T>(ow, e), dpart);
        }
    }
    dpart += __shfl_xor(dpart, 16);
    const float dl = dpart + __shfl_xor(dpart, 32);
    const int64_t rbase = (static_cast<int64_t>(b) * p.Hq + hq) * T_;
    if (qi < T_ && g == 0) p.delta[rbase + qi] = dl;
    const float inv_r = 1.f / p.rs[rbase + qrow];

    const int W = p.window;
    const unsigned weff = W > 0 ? static_cast<unsigned>(W) : 0x7FFFFFFFu;
    const int n_kv = (T_ + kFKT - 1) / kFKT;
    const int kv_end = min((q_start + kFRows + kFKT - 1) / kFKT, n_kv);
    const int kv_begin = W > 0 ? max(0, q_start - W + 1) / kFKT : 0;
    const float sc = p.scale;

    const int drow = (wave * 64 + lane) / CPR;
    const int pch = (wave * 64 + lane) % CPR;
    int koff[NI], voff[NI];
    wide_dma_offsets<PART, NI, RPI>(koff, drow, pch, krs, p.dr, [](int r) { return fk_swz(r); });
    wide_dma_offsets<PART, NI, RPI>(voff, drow, pch, vrs, p.dr, [](int r) { return r & 15; });
    auto issue = [&](int t, auto st) {
        const int k0 = t * kFKT;
        const int nrows = min(T_ - k0, kFKT);
        unsigned char* lk = stage_base(st);
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int skip = i * RPI;
            tile_dma16(__builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(kp + (k0 + skip) * krs), 0,
                                                         max((nrows - skip) * static_cast<int>(krs), 0), 0x00020000),
                       koff[i], lk + (i * kFW + wave) * 1024);
            tile_dma16(__builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(vp + (k0 + skip) * vrs), 0,
                                                         max((nrows - skip) * static_cast<int>(vrs), 0), 0x00020000),
                       voff[i], lk + TB + (i * kFW + wave) * 1024);
        }
    };

    // K^T operand (16 d x 32 keys) by two transposing reads, as V^T in the forward
    const int vr = 4 * g + (i16 >> 2);
    const int fv = fk_swz(vr);
    const int ktbase = vr * ROWB + (((((lane & 3) >> 1) ^ (fv & 1))) << 4) + 8 * (lane & 1);
    const int ktsw = fv >> 1;
    const int fki = fk_swz(i16);
    f32x4 acc[D / 16];
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    const f32x4 ndl{-dl, -dl, -dl, -dl};

    auto tile = [&](bool masked, int t, auto st) {
        const int k0 = t * kFKT;
        const unsigned char* Kb = stage_base(st);
        const unsigned char* Vb = Kb + TB;
        f32x4 s[NKS], dp[NKS];
#pragma unroll
        for (int kst = 0; kst < NKS; ++kst) {
            u32x4 op[D / 32];
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks)
                op[ks] = *reinterpret_cast<const u32x4*>(Kb + (16 * kst + i16) * ROWB + (((4 * ks + g) ^ fki) << 4));
            s[kst] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) s[kst] = Mfma16<T>::mma(as_vec8<V8>(op[ks]), as_vec8<V8>(qf[ks]), s[kst]);
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks)
                op[ks] = *reinterpret_cast<const u32x4*>(Vb + (16 * kst + i16) * ROWB + (((4 * ks + g) ^ i16) << 4));
            dp[kst] = ndl;
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) dp[kst] = Mfma16<T>::mma(as_vec8<V8>(op[ks]), as_vec8<V8>(df[ks]), dp[kst]);
        }
        const int dbase = qi - k0 - 4 * g;
        float ds[4 * NKS];
#pragma unroll
        for (int kst = 0; kst < NKS; ++kst) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float y, rr;
                weight_rr16<EXACT>(s[kst][e], sc, y, rr);
                ds[4 * kst + e] = dp[kst][e] * y * rr;
            }
        }
        if (masked) {
#pragma unroll
            for (int i = 0; i < 4 * NKS; ++i)
                ds[i] = keep_if(static_cast<unsigned>(dbase - 16 * (i / 4) - i % 4) < weff, ds[i]);
        }
#pragma unroll
        for (int kk = 0; kk < kFKT / 32; ++kk) {
            const float* xk = ds + 8 * kk;
            const u32x4 pw{pack2<T>(xk[0], xk[1]), pack2<T>(xk[2], xk[3]), pack2<T>(xk[4], xk[5]),
                           pack2<T>(xk[6], xk[7])};
            const V8 bop = as_vec8<V8>(pw);
#pragma unroll
            for (int dt = 0; dt < D / 16; ++dt) {
                const unsigned char* p0 = Kb + 32 * kk * ROWB + ktbase + ((dt ^ ktsw) << 5);
                acc[dt] = Mfma16<T>::mma(lds_read_tr16_pair<V8>(p0, p0 + 16 * ROWB), bop, acc[dt]);
            }
        }
    };

    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    issue(kv_begin, S0{});
    tile_wait_vmem();
    __syncthreads();
    const int wf = q0w, wl = q0w + 15;
    int t_first = kv_begin;
    if (W > 0 && wf - W + 1 > 0) t_first = max(t_first, (wf - W + 1) / kFKT);
    const int t_last = wf < T_ ? min(wl / kFKT, kv_end - 1) : t_first - 1;
    int ja = t_first;
    if (W > 0 && wl - W >= 0) ja = max(ja, (wl - W) / kFKT + 1);
    const int jb = (wf + 1) / kFKT;
    // Tile t (stage (t - kv_begin) & 1) runs while the DMA fills the other
    // stage with tile t + 1.  Waves run only the tiles their rows see, masked
    // outside [ja, jb), but take every barrier.
    auto run_tile = [&](int t, auto cur) {
        if (t + 1 < kv_end) issue(t + 1, std::integral_constant<int, 1 - decltype(cur)::value>{});
        if (t >= t_first && t <= t_last) tile(t < ja || t >= jb, t, cur);
        if (t + 1 < kv_end) {
            tile_wait_vmem();
            __syncthreads();
        }
    };
    for (int t = kv_begin; t < kv_end; t += 2) {
        run_tile(t, S0{});
        if (t + 1 < kv_end) run_tile(t + 1, S1{});
    }
    // dS carried without its per-row factor 2 scale / R
    __syncthreads();  // every wave is past its last tile: the ring is free
    wide_store_rows<T, D, PART>(wide_store_area<D>(lds0, lds1, wave), acc, 2.f * sc * inv_r,
                                p.dq + b * p.dqs[0] + hq * p.dqs[1], p.dqs[2], q0w, T_, p.dr, lane);
}

// ---------------------------------------------------------------------------
// Backward: dV (DK = false) or dK (DK = true), 16 key rows per wave on the
// 16x16x32 MFMA: 8 waves x 16 keys (128 keys per block), two waves per SIMD,
// 64-query tiles of every query head of the GQA group in a 2-stage LDS ring.
// S = Q K^T (Q rows from LDS, K in registers) leaves lane l with key
// l % 16 and queries 4 (l / 16) + e of each 16-query subtile: as they stand,
// P (or dS) of subtiles 2j, 2j + 1 are the B operand of dV^T += dO^T P (dK^T
// += Q^T dS) over query step j, with dO^T (Q^T) from transposing reads.  The
// Q tile of dK is read both ways (shared swizzle fk_swz), the other tiles one
// way (row reads: c ^ (r & 15); transposing reads: c ^ 2 (r & 7)).
// ---------------------------------------------------------------------------
template <typename T, int D, bool EXACT, bool DK, bool PART>
__global__ __launch_bounds__(64 * WideCfg<D>::NW) void flash_bwd_kv_wide_kernel(WideParams<T> p) {
    using V8 = typename MfmaOps<T>::vec8;
    constexpr int kFW = WideCfg<D>::NW, kFRows = WideCfg<D>::ROWS, kFKT = WideCfg<D>::KT;
    constexpr int ROWB = D * 2;
    constexpr int TB = kFKT * ROWB;     // bytes per query tile
    constexpr int CPR = ROWB / 16;
    constexpr int NI = TB / 1024 / kFW;
    constexpr int RPI = 64 * kFW / CPR;
    constexpr int NQS = kFKT / 16;      // 16-query subtiles per tile
    // Two ring stages ([Q, dO] each) in separate arrays, the tile loop
    // unrolled by two: each tile names its stage statically, so the compiler
    // knows its LDS reads cannot touch the stage the next tile's DMA writes
    // and does not wait for that DMA first.
    __shared__ __attribute__((aligned(1024))) unsigned char lds0[2 * TB];
    __shared__ __attribute__((aligned(1024))) unsigned char lds1[2 * TB];
    auto stage_base = [&](auto st) -> unsigned char* {
        if constexpr (decltype(st)::value == 0) return lds0;
        else return lds1;
    };
    __shared__ __attribute__((aligned(16))) float ldr[2][2][kFKT];            // [stage][1/R, -delta]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4;
    const int i16 = lane & 15;
    const int T_ = p.T;
    const int per = p.B * p.Hkv;
    // Block -> (ob, split): ob indexes the unsplit grid, split the block's
    // share of ob's (head, query tile) iterations.  When that grid is a
    // multiple of 8 blocks the n_split blocks of one ob run on ob's XCD
    // (blocks are dealt to the XCDs by index mod 8).
    const int n_split = p.n_split;
    int ob = static_cast<int>(blockIdx.x), split = 0;
    if (n_split > 1) {
        if ((((T_ + kFRows - 1) / kFRows * per) & 7) == 0) {
            const int j = ob >> 3;
            split = j % n_split;
            ob = ((j / n_split) << 3) | (ob & 7);
        } else {
            split = ob % n_split;
            ob /= n_split;
        }
    }
    const int kb = ob / per;  // earliest key blocks (most queries) first
    const int rest = ob - kb * per;
    const int b = rest / p.Hkv;
    const int hk = rest - b * p.Hkv;
    const int k_start = kb * kFRows;
    const int wk0 = k_start + 16 * wave;
    const int kj = wk0 + i16;
    const int krow = min(kj, T_ - 1);

    // K (and V) as B operands: k step ks holds d = 32 ks + 8 g .. +7 of key kj
    u32x4 kf[D / 32], vf[DK ? D / 32 : 1];
    {
        const T* kr = p.k + b * p.ks[0] + hk * p.ks[1] + krow * p.ks[2];
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) kf[ks] = wide_cols<PART>(kr, 32 * ks + 8 * g, p.dr);
        if constexpr (DK) {
            const T* vr_ = p.v + b * p.vs[0] + hk * p.vs[1] + krow * p.vs[2];
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) vf[ks] = wide_cols<PART>(vr_, 32 * ks + 8 * g, p.dr);
        }
    }
    f32x4 acc[D / 16];
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int W = p.window;
    const unsigned weff = W > 0 ? static_cast<unsigned>(W) : 0x7FFFFFFFu;
    const int n_qt = (T_ + kFKT - 1) / kFKT;
    const int qt_begin = k_start / kFKT;
    const int qt_end = W > 0 ? min(n_qt, (k_start + kFRows - 1 + W - 1) / kFKT + 1) : n_qt;
    const int nq = qt_end - qt_begin;  // >= 1 (k_start < T)
    const int n_it_all = p.G * nq;
    // this block's iterations [it_lo, it_hi) of the n_it_all (head, query tile) pairs
    const int it_lo = static_cast<int>(static_cast<int64_t>(split) * n_it_all / n_split);
    const int it_hi = static_cast<int>(static_cast<int64_t>(split + 1) * n_it_all / n_split);
    const float sc = p.scale;

    // DMA of the Q and dO rows of a query tile; Q stores chunk c of row r at
    // c ^ qswz(r), dO at c ^ oswz(r)
    auto qswz = [](int r) { return DK ? fk_swz(r) : (r & 15); };
    auto oswz = [](int r) { return DK ? (r & 15) : 2 * (r & 7); };
    const int drow = (wave * 64 + lane) / CPR;
    const int pch = (wave * 64 + lane) % CPR;
    const int64_t qrs = p.qs[2] * 2, ors = p.dos[2] * 2;
    int qoff[NI], ooff[NI];
    wide_dma_offsets<PART, NI, RPI>(qoff, drow, pch, qrs, p.dr, qswz);
    wide_dma_offsets<PART, NI, RPI>(ooff, drow, pch, ors, p.dr, oswz);
    auto tile_of = [&](int it, int& hq, int& q0) {
        const int gg = it / nq;
        q0 = (qt_begin + it - gg * nq) * kFKT;
        hq = hk * p.G + gg;
    };
    auto issue = [&](int it, auto st) {
        int hq, q0;
        tile_of(it, hq, q0);
        const unsigned char* qp = tile_uniform_ptr(reinterpret_cast<const unsigned char*>(p.q + b * p.qs[0] + hq * p.qs[1]));
        const unsigned char* op = tile_uniform_ptr(reinterpret_cast<const unsigned char*>(p.dout + b * p.dos[0] + hq * p.dos[1]));
        const int nrows = min(T_ - q0, kFKT);
        unsigned char* lq = stage_base(st);
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int skip = i * RPI;
            tile_dma16(__builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(qp + (q0 + skip) * qrs), 0,
                                                         max((nrows - skip) * static_cast<int>(qrs), 0), 0x00020000),
                       qoff[i], lq + (i * kFW + wave) * 1024);
            tile_dma16(__builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(op + (q0 + skip) * ors), 0,
                                                         max((nrows - skip) * static_cast<int>(ors), 0), 0x00020000),
                       ooff[i], lq + TB + (i * kFW + wave) * 1024);
        }
    };
    // threads 0..kFKT-1 load the tile's row sums (staged as 1/R), the next
    // kFKT its delta (staged as -delta); the raw value is stored an iteration
    // later
    auto row_value = [&](int it) {
        int hq, q0;
        tile_of(it, hq, q0);
        const int64_t idx = (static_cast<int64_t>(b) * p.Hq + hq) * T_ + min(q0 + (tid & (kFKT - 1)), T_ - 1);
        if constexpr (kFKT == 64) {
            // waves 0 and 1 (wave-uniform: the base pointer stays scalar)
            if (wave == 0) return p.rs[idx];
            if (wave == 1) return p.delta[idx];
        } else {
            if (wave == 0) return lane < kFKT ? p.rs[idx] : p.delta[idx];
        }
        return 0.f;
    };
    auto store_rv = [&](int st, float raw) {
        if (tid < 2 * kFKT) ldr[st][tid / kFKT][tid & (kFKT - 1)] = tid < kFKT ? 1.f / raw : -raw;
    };

    // transposing reads of the tile the accumulators contract over (dK: Q,
    // dV: dO): lane supplies row 4 g + i16 / 4 (+ 16), columns 16 dt + 4 (lane & 3)
    const int vr = 4 * g + (i16 >> 2);
    const int tsw = DK ? fk_swz(vr) : 2 * (vr & 7);
    const int trbase = vr * ROWB + (((((lane & 3) >> 1) ^ (tsw & 1))) << 4) + 8 * (lane & 1);
    const int trsw = tsw >> 1;
    const int qsi = qswz(i16), osi = oswz(i16);

    auto tile = [&](bool masked, int it, auto stage) {
        constexpr int st = decltype(stage)::value;
        int hq, q0;
        tile_of(it, hq, q0);
        (void)hq;
        const unsigned char* Qb = stage_base(stage);
        const unsigned char* Ob = Qb + TB;
        float x[4 * NQS];
#pragma unroll
        for (int qst = 0; qst < NQS; ++qst) {
            u32x4 a[D / 32];
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks)
                a[ks] = *reinterpret_cast<const u32x4*>(Qb + (16 * qst + i16) * ROWB + (((4 * ks + g) ^ qsi) << 4));
            f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) s = Mfma16<T>::mma(as_vec8<V8>(a[ks]), as_vec8<V8>(kf[ks]), s);
            // lane: key kj, queries q0 + 16 qst + 4 g + e
            const float4 ir = *reinterpret_cast<const float4*>(&ldr[st][0][16 * qst + 4 * g]);
            const float irv[4] = {ir.x, ir.y, ir.z, ir.w};
            f32x4 dp;
            if constexpr (DK) {
                const float4 nd = *reinterpret_cast<const float4*>(&ldr[st][1][16 * qst + 4 * g]);
                dp = f32x4{nd.x, nd.y, nd.z, nd.w};
#pragma unroll
                for (int ks = 0; ks < D / 32; ++ks)
                    a[ks] = *reinterpret_cast<const u32x4*>(Ob + (16 * qst + i16) * ROWB + (((4 * ks + g) ^ osi) << 4));
#pragma unroll
                for (int ks = 0; ks < D / 32; ++ks) dp = Mfma16<T>::mma(as_vec8<V8>(a[ks]), as_vec8<V8>(vf[ks]), dp);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float y, rr;
                weight_rr16<EXACT>(s[e], sc, y, rr);
                const float yi = y * irv[e];
                float v;
                if constexpr (DK) v = dp[e] * yi * rr;  // dS (without 2 scale)
                else v = yi;                            // P
                x[4 * qst + e] = v;
            }
        }
        if (masked) {
#pragma unroll
            for (int i = 0; i < 4 * NQS; ++i) {
                const int q = q0 + 16 * (i / 4) + 4 * g + i % 4;
                x[i] = keep_if(static_cast<unsigned>(q - kj) < weff && q < T_, x[i]);
            }
        }
        const unsigned char* Tb = DK ? Qb : Ob;
#pragma unroll
        for (int kk = 0; kk < kFKT / 32; ++kk) {
            const float* xk = x + 8 * kk;
            const u32x4 pw{pack2<T>(xk[0], xk[1]), pack2<T>(xk[2], xk[3]), pack2<T>(xk[4], xk[5]),
                           pack2<T>(xk[6], xk[7])};
            const V8 bop = as_vec8<V8>(pw);
#pragma unroll
            for (int dt = 0; dt < D / 16; ++dt) {
                const unsigned char* p0 = Tb + 32 * kk * ROWB + trbase + ((dt ^ trsw) << 5);
                acc[dt] = Mfma16<T>::mma(lds_read_tr16_pair<V8>(p0, p0 + 16 * ROWB), bop, acc[dt]);
            }
        }
    };

    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    if (it_lo < it_hi) {
        issue(it_lo, S0{});
        store_rv(0, row_value(it_lo));
        tile_wait_vmem();
    }
    __syncthreads();
    // iteration it reads stage (it - it_lo) & 1 while the DMA fills the other with it + 1
    auto step = [&](int it, auto cur) {
        constexpr int nxt = 1 - decltype(cur)::value;
        const bool more = it + 1 < it_hi;
        float rnext = 0.f;
        if (more) {
            issue(it + 1, std::integral_constant<int, nxt>{});  // free since the barrier that ended it - 1
            rnext = row_value(it + 1);
        }
        int hq, q0;
        tile_of(it, hq, q0);
        // wave-uniform: some (query, key) pair of the tile is visible; all are
        const bool active = q0 + kFKT - 1 >= wk0 && q0 < T_ && !(W > 0 && q0 - (wk0 + 15) >= W);
        const bool interior = q0 >= wk0 + 15 && q0 + kFKT <= T_ && !(W > 0 && q0 + kFKT - 1 - wk0 >= W);
        if (active) tile(!interior, it, cur);
        if (more) {
            store_rv(nxt, rnext);
            tile_wait_vmem();
            __syncthreads();
        }
    };
    for (int it = it_lo; it < it_hi; it += 2) {
        step(it, S0{});
        if (it + 1 < it_hi) step(it + 1, S1{});
    }
    if (n_split > 1) {
        // fp32 partial of key kj (zeros for an empty share), unscaled
        if (kj < T_) {
            float* dst = p.part + ((static_cast<int64_t>(split) * per + rest) * T_ + kj) * D + 4 * g;
#pragma unroll
            for (int dt = 0; dt < D / 16; ++dt)
                if (!PART || 16 * dt + 4 * g < p.dr) *reinterpret_cast<f32x4*>(dst + 16 * dt) = acc[dt];
        }
        return;
    }
    __syncthreads();  // every wave is past its last tile: the ring is free
    T* base = DK ? p.dk + b * p.dks[0] + hk * p.dks[1] : p.dv + b * p.dvs[0] + hk * p.dvs[1];
    wide_store_rows<T, D, PART>(wide_store_area<D>(lds0, lds1, wave), acc, DK ? 2.f * sc : 1.f, base,
                                DK ? p.dks[2] : p.dvs[2], wk0, T_, p.dr, lane);
}

// dK (DK) or dV = the sum of the n_split fp32 partials (in split order, so
// the result does not depend on timing), dK times 2 scale; one thread per
// four columns of a key row.
template <typename T, int D, bool DK>
__global__ __launch_bounds__(256) void wide_split_reduce_kernel(WideParams<T> p, int64_t n_quads) {
    const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (gid >= n_quads) return;
    const int64_t row = gid / (D / 4);  // (b * Hkv + hk) * T + key
    const int d0 = static_cast<int>(gid - row * (D / 4)) * 4;
    if (d0 >= p.dr) return;
    const int64_t plane = static_cast<int64_t>(p.B) * p.Hkv * p.T * D;
    const float* src = p.part + row * D + d0;
    float4 a = float4{0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < p.n_split; ++s) {
        const float4 c = *reinterpret_cast<const float4*>(src + s * plane);
        a.x += c.x; a.y += c.y; a.z += c.z; a.w += c.w;
    }
    const float f = DK ? 2.f * p.scale : 1.f;
    const int64_t bh = row / p.T;
    const int key = static_cast<int>(row - bh * p.T);
    const int b = static_cast<int>(bh / p.Hkv);
    const int hk = static_cast<int>(bh - static_cast<int64_t>(b) * p.Hkv);
    T* dst = DK ? p.dk + b * p.dks[0] + hk * p.dks[1] + key * p.dks[2]
                : p.dv + b * p.dvs[0] + hk * p.dvs[1] + key * p.dvs[2];
    *reinterpret_cast<uint2*>(dst + d0) = uint2{pack2<T>(a.x * f, a.y * f), pack2<T>(a.z * f, a.w * f)};
}

// 16-bit tensors: (b, h, t) strides multiples of 8 elements (16-byte rows),
// d stride 1, and a tile's rows within 32-bit byte offsets of its first row.
bool wide_strides_ok(const int64_t* s) {
    return s[3] == 1 && s[0] % 8 == 0 && s[1] % 8 == 0 && s[2] % 8 == 0 && s[2] >= 0 &&
           s[2] * 2 * kWideMaxKT < (int64_t(1) << 31);
}

int check_wide(int B, int Hq, int Hkv, int T, int D, int window_size, int dtype) {
    if (dtype != SA_BF16 && dtype != SA_F16) return SA_ERR_BAD_DTYPE;
    if (B < 0 || Hq <= 0 || Hkv <= 0 || T < 0 || Hq % Hkv != 0 || window_size < 0) return SA_ERR_BAD_SHAPE;
    if (D <= 128 || D > 512 || D % 8 != 0) return SA_ERR_UNSUPPORTED;
    return 0;
}

template <typename T, int D>
int launch_fwd_wide(const WideParams<T>& prm, int exact, hipStream_t st) {
    constexpr int kFW = WideCfg<D>::NW, kFRows = WideCfg<D>::ROWS;
    const int64_t nblk = static_cast<int64_t>((prm.T + kFRows - 1) / kFRows) * prm.B * prm.Hq;
    if (nblk * 64 * kFW >= (int64_t(1) << 32)) return SA_ERR_BAD_SHAPE;
    const dim3 grid(static_cast<unsigned>(nblk));
    if (exact) {
        flash_fwd_wide_kernel<T, D, true, false><<<grid, 64 * kFW, 0, st>>>(prm);
        return status_from_launch();
    }
    // folded weights for bf16 P only (fp16 P would overflow sooner by 1/scale^2)
    if constexpr (std::is_same_v<T, bf16>) {
        if (prm.scale >= 0x1p-20f && prm.scale <= 0x1p20f) {
            flash_fwd_wide_kernel<T, D, false, true><<<grid, 64 * kFW, 0, st>>>(prm);
            return status_from_launch();
        }
    }
    flash_fwd_wide_kernel<T, D, false, false><<<grid, 64 * kFW, 0, st>>>(prm);
    return status_from_launch();
}

template <typename T, int D, bool EXACT, bool PART>
void launch_bwd_wide_kernels(const WideParams<T>& prm, dim3 gq, dim3 gk, hipStream_t st) {
    constexpr int kFW = WideCfg<D>::NW;
    flash_bwd_dq_wide_kernel<T, D, EXACT, PART><<<gq, 64 * kFW, 0, st>>>(prm);
    // dV, then dK; with a split each sums its partials before the next
    // kernel reuses the buffer
    const int64_t n_quads = static_cast<int64_t>(prm.B) * prm.Hkv * prm.T * (D / 4);
    const dim3 gr(static_cast<unsigned>((n_quads + 255) / 256));
    flash_bwd_kv_wide_kernel<T, D, EXACT, false, PART><<<gk, 64 * kFW, 0, st>>>(prm);
    if (prm.n_split > 1) wide_split_reduce_kernel<T, D, false><<<gr, 256, 0, st>>>(prm, n_quads);
    flash_bwd_kv_wide_kernel<T, D, EXACT, true, PART><<<gk, 64 * kFW, 0, st>>>(prm);
    if (prm.n_split > 1) wide_split_reduce_kernel<T, D, true><<<gr, 256, 0, st>>>(prm, n_quads);
}

template <typename T, int D, bool PART>
int launch_bwd_wide_part(const WideParams<T>& prm, int exact, hipStream_t st) {
    constexpr int kFW = WideCfg<D>::NW, kFRows = WideCfg<D>::ROWS;
    const int64_t nq = static_cast<int64_t>((prm.T + kFRows - 1) / kFRows) * prm.B * prm.Hq;
    if (nq * 64 * kFW >= (int64_t(1) << 32)) return SA_ERR_BAD_SHAPE;  // dQ blocks of kFW waves
    const int64_t nk = nq / prm.G * prm.n_split;
    if (nk * 64 * kFW >= (int64_t(1) << 32)) return SA_ERR_BAD_SHAPE;
    const dim3 gq(static_cast<unsigned>(nq)), gk(static_cast<unsigned>(nk));
    if (exact) launch_bwd_wide_kernels<T, D, true, PART>(prm, gq, gk, st);
    else launch_bwd_wide_kernels<T, D, false, PART>(prm, gq, gk, st);
    return status_from_launch();
}

// The masked kernels (PART) only for head dims below the kernel's: the
// masks cost the dK kernel registers (spills in its tile loop at D = 256).
template <typename T>
int launch_bwd_wide(const WideParams<T>& prm, int exact, hipStream_t st) {
    if (prm.dr == 256) return launch_bwd_wide_part<T, 256, false>(prm, exact, st);
    if (prm.dr < 256) return launch_bwd_wide_part<T, 256, true>(prm, exact, st);
    if (prm.dr == 512) return launch_bwd_wide_part<T, 512, false>(prm, exact, st);
    return launch_bwd_wide_part<T, 512, true>(prm, exact, st);
}

template <typename T>
int run_fwd_wide(const void* q, const void* k, const void* v, void* o, float* row_sums, int B, int Hq, int Hkv,
                 int T_, int D, const int64_t* qs, const int64_t* ks, const int64_t* vs, const int64_t* os, float scale,
                 int window_size, int exact_math, hipStream_t st) {
    WideParams<T> prm{};
    prm.q = static_cast<const T*>(q);
    prm.k = static_cast<const T*>(k);
    prm.v = static_cast<const T*>(v);
    prm.out = static_cast<T*>(o);
    prm.row_sums = row_sums;
    for (int i = 0; i < 4; ++i) {
        prm.qs[i] = qs[i];
        prm.ks[i] = ks[i];
        prm.vs[i] = vs[i];
        prm.os[i] = os[i];
    }
    prm.B = B;
    prm.Hq = Hq;
    prm.Hkv = Hkv;
    prm.T = T_;
    prm.G = Hq / Hkv;
    prm.window = window_size;
    prm.dr = D;
    prm.scale = scale;
    if (D <= 256) return launch_fwd_wide<T, 256>(prm, exact_math, st);
    return launch_fwd_wide<T, 512>(prm, exact_math, st);
}

// Kernel head dim for head dim dr in 136..512.
int wide_kernel_d(int dr) { return dr <= 256 ? 256 : 512; }

int64_t wide_part_bytes(int n_split, int B, int Hkv, int T, int dr) {
    return n_split > 1 ? static_cast<int64_t>(n_split) * B * Hkv * T * wide_kernel_d(dr) * 4 : 0;
}

// (head, query tile) iterations of dK/dV key block kb, as the kernels count them.
template <int D>
int wide_kv_iterations(int kb, int T, int G, int W) {
    constexpr int R = WideCfg<D>::ROWS, KT = WideCfg<D>::KT;
    const int n_qt = (T + KT - 1) / KT;
    const int k_start = kb * R;
    const int qt_begin = k_start / KT;
    const int qt_end = W > 0 ? std::min(n_qt, (k_start + R - 1 + W - 1) / KT + 1) : n_qt;
    return G * (qt_end - qt_begin);
}

// Query-range splits of the dK and dV blocks, as for head dims up to 128:
// causally, key block kb sees the query tiles from its own on, so the first
// blocks hold the most work, and a grid that does not fill the chip several
// times over idles while they finish.  The count is the one of 1, 2, 4, 8,
// 16 with the least estimated time: the makespan of an XCD's share (one
// block per CU, 32 at once; a block's set-up and stores at two iterations),
// an iteration of the dV and the dK kernel together at kWideItUs, plus the
// two kernels' partials written and read back at 5 TB/s and two more
// launches.  Both kernels use the count, one after the other, on one buffer
// of at most 512 MiB; grids of 2048 blocks or more are not split.
template <int D>
int wide_split_count_uncached(int B, int Hkv, int T, int G, int W) {
    constexpr double kWideItUs = D > 256 ? 3.0 : 6.0;
    const int nkb = (T + WideCfg<D>::ROWS - 1) / WideCfg<D>::ROWS;
    const int64_t blocks = static_cast<int64_t>(nkb) * B * Hkv;
    int best = 1;
    double best_t = 0.0;
    for (int S = 1; S <= 16; S *= 2) {
        const int64_t bytes = wide_part_bytes(S, B, Hkv, T, D);
        if (blocks * S > 16384 || bytes > (int64_t(512) << 20)) break;
        double t = dkdv_split_makespan(nkb, B * Hkv, S, 32, 2.0,
                                       [&](int kb) { return wide_kv_iterations<D>(kb, T, G, W); }) *
                   kWideItUs;  // us
        if (S > 1) t += 4.0 * static_cast<double>(bytes) / 5e6 + 10.0;
        if (S == 1 || t < best_t) {
            best = S;
            best_t = t;
        }
    }
    return best;
}

int wide_split_count(int B, int Hkv, int T, int G, int W, int dr) {
    const int R = dr <= 256 ? WideCfg<256>::ROWS : WideCfg<512>::ROWS;  // key rows per block
    const int64_t blocks = static_cast<int64_t>((T + R - 1) / R) * B * Hkv;
    if (blocks >= 8 * 32 * 8 || blocks == 0) return 1;
    static SplitCountCache cache;
    const int key[6] = {B, Hkv, T, G, W, wide_kernel_d(dr)};
    return cache.get(key, [&] {
        return dr <= 256 ? wide_split_count_uncached<256>(B, Hkv, T, G, W)
                         : wide_split_count_uncached<512>(B, Hkv, T, G, W);
    });
}

template <typename T>
int run_bwd_wide(const void* q, const void* k, const void* v, const void* o, const void* dout,
                 const float* row_sums, void* dq, void* dk, void* dv, float* delta_ws, int B, int Hq, int Hkv,
                 int T_, int D, const int64_t* const strides[8], float scale, int window_size, int exact_math,
                 int n_split, float* part, hipStream_t st) {
    WideParams<T> prm{};
    prm.q = static_cast<const T*>(q);
    prm.k = static_cast<const T*>(k);
    prm.v = static_cast<const T*>(v);
    prm.o = static_cast<const T*>(o);
    prm.dout = static_cast<const T*>(dout);
    prm.rs = row_sums;
    prm.dq = static_cast<T*>(dq);
    prm.dk = static_cast<T*>(dk);
    prm.dv = static_cast<T*>(dv);
    prm.delta = delta_ws;
    int64_t* dst[8] = {prm.qs, prm.ks, prm.vs, prm.os, prm.dos, prm.dqs, prm.dks, prm.dvs};
    for (int i = 0; i < 8; ++i)
        for (int j = 0; j < 4; ++j) dst[i][j] = strides[i][j];
    prm.B = B;
    prm.Hq = Hq;
    prm.Hkv = Hkv;
    prm.T = T_;
    prm.G = Hq / Hkv;
    prm.window = window_size;
    prm.dr = D;
    prm.scale = scale;
    prm.n_split = n_split;
    prm.part = part;
    return launch_bwd_wide<T>(prm, exact_math, st);
}

}  // namespace

int flash_fwd_wide(const void* q, const void* k, const void* v, void* o, float* row_sums, int B, int Hq, int Hkv,
                   int T, int D, const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                   const int64_t* o_strides, float scale, int window_size, int exact_math, int dtype,
                   hipStream_t st) {
    const int chk = check_wide(B, Hq, Hkv, T, D, window_size, dtype);
    if (chk != 0) return chk;
    if (!q || !k || !v || !o || !q_strides || !k_strides || !v_strides || !o_strides) return SA_ERR_NULL_POINTER;
    if (!wide_strides_ok(q_strides) || !wide_strides_ok(k_strides) || !wide_strides_ok(v_strides) ||
        !wide_strides_ok(o_strides) || !aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
        return SA_ERR_BAD_STRIDE;
    if (B == 0 || T == 0) return 0;
    if (dtype == SA_BF16)
        return run_fwd_wide<bf16>(q, k, v, o, row_sums, B, Hq, Hkv, T, D, q_strides, k_strides, v_strides, o_strides,
                                  scale, window_size, exact_math, st);
    return run_fwd_wide<f16>(q, k, v, o, row_sums, B, Hq, Hkv, T, D, q_strides, k_strides, v_strides, o_strides,
                             scale, window_size, exact_math, st);
}

int64_t flash_bwd_wide_workspace_size(int B, int Hq, int Hkv, int T, int D, int window_size) {
    if (D <= 128 || D > 512 || B == 0 || T == 0) return 0;
    return wide_part_bytes(wide_split_count(B, Hkv, T, Hq / Hkv, window_size, D), B, Hkv, T, D);
}

int flash_bwd_wide(const void* q, const void* k, const void* v, const void* o, const void* dout,
                   const float* row_sums, void* dq, void* dk, void* dv, float* delta_ws, int B, int Hq, int Hkv,
                   int T, int D, const int64_t* const strides[8], float scale, int window_size, int exact_math,
                   int dtype, void* workspace, int64_t workspace_bytes, hipStream_t st) {
    const int chk = check_wide(B, Hq, Hkv, T, D, window_size, dtype);
    if (chk != 0) return chk;
    if (!q || !k || !v || !o || !dout || !row_sums || !dq || !dk || !dv || !delta_ws) return SA_ERR_NULL_POINTER;
    const void* ptrs[8] = {q, k, v, o, dout, dq, dk, dv};
    for (int i = 0; i < 8; ++i) {
        if (!strides[i]) return SA_ERR_NULL_POINTER;
        if (!wide_strides_ok(strides[i]) || !aligned16(ptrs[i])) return SA_ERR_BAD_STRIDE;
    }
    if (B == 0 || T == 0) return 0;
    // the library's split count, or the largest power of two below it whose
    // partials fit the workspace
    int ns = 1;
    if (workspace && workspace_bytes > 0) {
        if (!aligned16(workspace)) return SA_ERR_BAD_STRIDE;
        ns = wide_split_count(B, Hkv, T, Hq / Hkv, window_size, D);
        while (ns > 1 && wide_part_bytes(ns, B, Hkv, T, D) > workspace_bytes) ns /= 2;
    }
    float* part = ns > 1 ? static_cast<float*>(workspace) : nullptr;
    if (dtype == SA_BF16)
        return run_bwd_wide<bf16>(q, k, v, o, dout, row_sums, dq, dk, dv, delta_ws, B, Hq, Hkv, T, D, strides, scale,
                                  window_size, exact_math, ns, part, st);
    return run_bwd_wide<f16>(q, k, v, o, dout, row_sums, dq, dk, dv, delta_ws, B, Hq, Hkv, T, D, strides, scale,
                             window_size, exact_math, ns, part, st);
}

}  // namespace sa
