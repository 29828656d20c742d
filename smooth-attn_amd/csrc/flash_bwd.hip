// Fused causal squareplus attention backward on gfx950 MFMA (bf16 / fp16).
//
// With s = q_i . k_j (raw dot product), a = scale s - 1/2, r = sqrt(a^2 + 1),
// y = (a + r)^2 (= squareplus(2 scale s - 1)^2), R_i = sum_j y_ij + 1e-12 (the
// forward's row sums), P = y / R and O = P V:
//   dP_ij    = dO_i . V_j
//   delta_i  = dO_i . O_i                      (= sum_j P_ij dP_ij)
//   dS_ij    = (dP_ij - delta_i) / R_i * dy/ds = 2 scale (dP_ij - delta_i) y_ij / (r_ij R_i)
//   dQ_i = sum_j dS_ij K_j,  dK_j = sum_i dS_ij Q_i,  dV_j = sum_i P_ij dO_i
// (reference kernels.py:1667-1784 dQ + delta, :1787-1909 dK/dV; the
// reference writes dy/ds as 4 sp sp' scale with sp' = (1 + arg/sqrt(arg^2+4))/2,
// arg = 2a, which equals 2 scale y / r).  P and dS are rounded to the 16-bit
// type before their products, as the reference does.
//
// Two kernels, as in the reference:
//  * flash_bwd_dq_kernel: a block of 4 waves owns 128 query rows of one
//    (batch, query head).  Each wave keeps Q and dO of its 32 rows in
//    registers (B operands), computes delta for them (written to the
//    workspace), and walks the key tiles: S^T = K Q^T and dP^T = V dO^T on
//    MFMA with K, V from LDS, dS^T on the VALU, then dQ^T += K^T dS^T with
//    K^T read from the same LDS tile by the transposing LDS load.
//  * flash_bwd_dkdv_kernel: a block of 4 waves owns 128 key rows of one
//    (batch, KV head); wave w owns keys [32w, 32w+32) and keeps V and most of
//    K of them in registers (at D = 128 the first three and a half 16-byte
//    chunks of K live in LDS, a slot per lane).  It walks every query head of the GQA group and every
//    query tile of 64 rows that sees its keys: S = Q K^T and dP = dO V^T with
//    Q, dO from LDS, P and dS on the VALU (their C layout is the B operand of
//    the next products), then dV^T += dO^T P and dK^T += Q^T dS with dO^T,
//    Q^T from the transposing LDS load.
// Tiles go straight from global memory into LDS (global_load_lds, double
// buffered, one barrier per tile), as in the forward.  The two stages are
// separate LDS arrays and the tile loops are unrolled by two, so a tile's LDS
// reads never wait for the DMA filling the other stage (the compiler waits
// for an in-flight direct-to-LDS load before any read of the same array).
#include "flash_common.hpp"
#include "flash_tiles.hpp"
#include "flash_f32.hpp"
#include "flash_wide.hpp"
#include "dkdv_split.hpp"

#include <algorithm>

namespace sa {
namespace {

constexpr int kBwdThreads = 256;
// Two blocks per CU for both kernels: the register budget is then 256 per
// lane and the compiler keeps every MFMA in the VGPR form (with one block per
// CU it moves the accumulators through AGPRs, which costs more than the few
// dK/dV registers that now spill).
constexpr int kBwdDkdvMinBlocks = 2;
constexpr int kBwdBQ = 128;   // query rows per dQ block (32 per wave)
constexpr int kBwdKT = 64;    // keys per staged tile in the dQ kernel
constexpr int kBwdBK = 128;   // key rows per dK/dV block (32 per wave)
constexpr int kBwdQT = 64;    // query rows per staged tile in the dK/dV kernel
constexpr int kBwdXcdSlots = 64;  // blocks one XCD runs at once (32 CUs x 2)
// D = 128 dK/dV: the first 16-byte chunks of the wave's K and V operands
// kept in LDS (a slot per lane) instead of registers; see
// flash_bwd_dkdv_kernel.  4 KB of LDS per chunk and block: with two blocks
// per CU (80 KB each) three chunks and half of a fourth fit, all from K.
constexpr int kDkdvLdsK = 3, kDkdvLdsV = 0;

struct BwdParams {
    const void* q;
    const void* k;
    const void* v;
    const void* o;
    const void* dout;
    const float* rs;  // [B, Hq, T] row sums of the forward (contiguous)
    void* dq;
    void* dk;
    void* dv;
    float* delta;  // [B, Hq, T] workspace (contiguous)
    int64_t qs[4], ks[4], vs[4], os[4], dos[4], dqs[4], dks[4], dvs[4];
    int B, Hq, Hkv, T, G, window;
    int dr;  // head dim of the tensors (<= D, a multiple of 8; columns past it read as zero, are not stored)
    float scale;
    // dK/dV split over the query tiles: n_split blocks per (key block, KV
    // head), each writing fp32 partials [n_split][2][B * Hkv][T][D] into part
    // (summed by bwd_split_reduce_kernel); 1 = no split, results stored directly
    int n_split;
    float* part;
};

// Plain (cached) 16-byte global load: tiles here are re-read by many blocks.
__device__ __forceinline__ u32x4 ldg16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

// Columns d0 .. d0 + 7 of a row; PART (head dim dr below the kernel's D):
// zeros where they lie past dr (the load then reads column 0).
template <bool PART, typename T>
__device__ __forceinline__ u32x4 ldg16_cols(const T* row, int d0, int dr) {
    if constexpr (!PART) return ldg16(row + d0);
    const u32x4 v = ldg16(row + (d0 < dr ? d0 : 0));
    return d0 < dr ? v : u32x4{0u, 0u, 0u, 0u};
}

// Staged tiles are unpadded [64 rows][D] of the 16-bit type, filled by direct
// global->LDS loads (one 1 KB span of consecutive 16-byte chunks per wave
// instruction).  Each tile is read two ways: as 16-byte A-operand rows (16
// consecutive rows per LDS cycle, same logical chunk) and through the
// transposing read (per 32 lanes: 4 consecutive rows x 64 bytes).  The LDS
// has 64 banks of 4 bytes, so a cycle is conflict-free when its lanes cover
// 256 distinct bytes modulo 256.  Storing logical chunk c of row r at
// c ^ f(r) achieves both: for 256-byte rows (D = 128), f(r) = (r & 3) << 2 |
// (r >> 2) & 3 takes 16 distinct values on 16 consecutive rows, and its
// 64-byte group (f >> 2) 4 distinct values on rows 4k..4k+3; shorter rows
// share a 256-byte window and f uses the row bits above the window.
template <int D>
struct SwzTile {
    static constexpr int ROWB = D * 2;     // bytes per row
    static constexpr int CPR = D / 8;      // 16-byte chunks per row
    static constexpr int BYTES = 64 * ROWB;
    static constexpr int NI = 64 * CPR / kBwdThreads;  // DMA loads per lane per tile
    static __device__ __forceinline__ int f(int r) {
        if constexpr (CPR >= 16) return ((r & 3) << 2) | ((r >> 2) & 3);
        else if constexpr (CPR == 8) return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
        else return (r >> 2) & 3;
    }
    // Byte offset of A-operand chunk c of row r.
    static __device__ __forceinline__ int row_off(int r, int c) { return r * ROWB + ((c ^ f(r)) << 4); }
    // Per-lane byte offset (from row 16c of the tile) of the transposing
    // read of 32-column block dt, half h: row vr + 8h of the 16-row chunk
    // (f depends on bits 0-3 of the row only, so it is the same for every c).
    static __device__ __forceinline__ int tr_off(int lane, int dt, int h) {
        const int vr = (lane >> 5) * 4 + ((lane & 15) >> 2) + 8 * h;
        const int chunk = (dt * 4 + ((lane >> 4) & 1) * 2 + ((lane & 3) >> 1)) ^ f(vr);
        return vr * ROWB + chunk * 16 + (lane & 1) * 8;
    }
};

// A operand = (16 rows x 32 columns of a tile)^T via two transposing reads;
// p points at row 16c of the tile.
template <typename Vec, typename Tl>
__device__ __forceinline__ Vec tr_operand(const unsigned char* p, int lane, int dt) {
    return lds_read_tr16_pair<Vec>(p + Tl::tr_off(lane, dt, 0), p + Tl::tr_off(lane, dt, 1));
}

// Byte offset (from the tile's first row, row stride rsb) of the source of
// this lane's DMA load i of a swizzled [64][D] tile: LDS slot s = (4 i +
// wave) * 64 + lane holds row s / CPR, logical chunk (s % CPR) ^ f(row);
// PART: chunks past the head dim dr take kPastTile (zeros).
template <int D, bool PART>
__device__ __forceinline__ int swz_src_off(int i, int wave, int lane, int rsb, int dr) {
    using Tl = SwzTile<D>;
    const int sl = (i * 4 + wave) * 64 + lane;
    const int row = sl / Tl::CPR;
    const int c = (sl - row * Tl::CPR) ^ Tl::f(row);
    if constexpr (!PART) return row * rsb + (c << 4);
    return 8 * c < dr ? row * rsb + (c << 4) : kPastTile;
}

// Issue the DMA loads of one [64][D] tile whose first row is at `base`
// (wave-uniform; row stride rsb bytes) into the swizzled LDS tile at `dst`;
// rows at or past `nrows` read as zeros.  lane_off: swz_src_off(0, ...).
// Load i covers rows 256/CPR further down than load i - 1 with the same
// swizzle (f depends on row bits that i does not change), so
// swz_src_off(i) = i * (256 / CPR) * rsb + swz_src_off(0): each load gets a
// scalar resource starting i * (256 / CPR) rows in (with the byte count
// shortened to match, so the zero fill past nrows is unchanged) and one
// per-lane offset serves them all.
template <int D>
__device__ __forceinline__ void issue_swz_tile(const unsigned char* base, int rsb, int nrows, unsigned char* dst,
                                               int wave, int lane_off) {
    using Tl = SwzTile<D>;
    constexpr int kRowsPerLoad = 256 / Tl::CPR;
    const int nbytes = nrows * rsb;
#pragma unroll
    for (int i = 0; i < Tl::NI; ++i) {
        const int skip = i * kRowsPerLoad * rsb;
        const __amdgpu_buffer_rsrc_t rs = tile_rsrc(base + skip, max(nbytes - skip, 0));
        tile_dma16(rs, lane_off, dst + (i * 4 + wave) * 64 * 16);
    }
}

template <bool EXACT>
__device__ __forceinline__ void weight_and_rr(float s, float sc, float& y, float& rr) {
    const float a = __builtin_fmaf(s, sc, -0.5f);
    const float u = __builtin_fmaf(a, a, 1.f);
    rr = fast_rsqrt(u);
    const float r = EXACT ? __builtin_sqrtf(u) : u * rr;
    const float sp = a + r;
    y = sp * sp;
}

// ---------------------------------------------------------------------------
// dQ (and delta)
// ---------------------------------------------------------------------------
// PART: the tensors' head dim p.dr is below D (its columns past p.dr read as
// zeros and are not stored); the kernels with PART false serve dr == D.
template <typename T, int D, bool EXACT, bool PART>
__global__ __launch_bounds__(kBwdThreads, 2) void flash_bwd_dq_kernel(BwdParams p) {
    using Ops = MfmaOps<T>;
    using Vec = typename Ops::vec8;
    using Tl = SwzTile<D>;
    // The two ring stages ([K, V] each) are separate arrays and the tile loop
    // is unrolled by two, so each tile names its stage statically: the
    // compiler then knows that the current stage's LDS reads cannot touch the
    // stage the next tile's DMA writes, and does not wait for that DMA first.
    __shared__ __attribute__((aligned(1024))) unsigned char lds0[2 * Tl::BYTES];
    __shared__ __attribute__((aligned(1024))) unsigned char lds1[2 * Tl::BYTES];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hi = lane >> 5;
    const int l32 = lane & 31;

    const int nqb = (p.T + kBwdBQ - 1) / kBwdBQ;
    int step, unit, sub;
    grouped_block(blockIdx.x, p.B * p.Hkv, p.G, nqb, kBwdXcdSlots, step, unit, sub);
    const int qb = nqb - 1 - step;  // heaviest (latest) query blocks first
    const int b = unit / p.Hkv;
    const int hk = unit - b * p.Hkv;
    const int hq = hk * p.G + sub;
    const int bh = b * p.Hq + hq;
    const int T_ = p.T;

    const T* qp = static_cast<const T*>(p.q) + b * p.qs[0] + hq * p.qs[1];
    const unsigned char* kp =
        tile_uniform_ptr(reinterpret_cast<const unsigned char*>(static_cast<const T*>(p.k) + b * p.ks[0] + hk * p.ks[1]));
    const unsigned char* vp =
        tile_uniform_ptr(reinterpret_cast<const unsigned char*>(static_cast<const T*>(p.v) + b * p.vs[0] + hk * p.vs[1]));
    const T* op = static_cast<const T*>(p.o) + b * p.os[0] + hq * p.os[1];
    const T* dop = static_cast<const T*>(p.dout) + b * p.dos[0] + hq * p.dos[1];
    T* dqp = static_cast<T*>(p.dq) + b * p.dqs[0] + hq * p.dqs[1];

    const int q_start = qb * kBwdBQ;
    const int wq0 = q_start + 32 * wave;
    const int qi = wq0 + l32;
    const int qrow = min(qi, T_ - 1);

    // Q and dO rows as B operands (chunk dc: d = 16 dc + 8 hi .. +7); delta
    // from the matching chunks of O (lanes l and l ^ 32 hold the two halves).
    u32x4 qreg[D / 16], doreg[D / 16];
    float dpart = 0.f;
#pragma unroll
    for (int dc = 0; dc < D / 16; ++dc) {
        const int d0 = dc * 16 + hi * 8;
        qreg[dc] = ldg16_cols<PART>(qp + qrow * p.qs[2], d0, p.dr);
        doreg[dc] = ldg16_cols<PART>(dop + qrow * p.dos[2], d0, p.dr);
        const u32x4 ov = ldg16_cols<PART>(op + qrow * p.os[2], d0, p.dr);
        const uint32_t dw[4] = {doreg[dc].x, doreg[dc].y, doreg[dc].z, doreg[dc].w};
        const uint32_t ow[4] = {ov.x, ov.y, ov.z, ov.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) dpart = __builtin_fmaf(elem<T>(dw, e), elem<T>(ow, e), dpart);
    }
    const float dl = dpart + __shfl_xor(dpart, 32);
    const int64_t rbase = static_cast<int64_t>(bh) * T_;
    if (qi < T_ && hi == 0) p.delta[rbase + qi] = dl;
    const float inv_r = 1.f / p.rs[rbase + qrow];
    f32x16 ndl;
#pragma unroll
    for (int v = 0; v < 16; ++v) ndl[v] = -dl;

    f32x16 acc[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) acc[dt] = f32x16{};

    const int W = p.window;
    const unsigned weff = W > 0 ? static_cast<unsigned>(W) : 0x7FFFFFFFu;
    const int n_kv = (T_ + kBwdKT - 1) / kBwdKT;
    const int kv_end = min((q_start + kBwdBQ + kBwdKT - 1) / kBwdKT, n_kv);
    const int kv_begin = W > 0 ? max(0, q_start - W + 1) / kBwdKT : 0;
    const float sc = p.scale;

    const int ksb = static_cast<int>(p.ks[2] * 2), vsb = static_cast<int>(p.vs[2] * 2);  // row strides (bytes)
    const int koff = swz_src_off<D, PART>(0, wave, lane, ksb, p.dr);
    const int voff = swz_src_off<D, PART>(0, wave, lane, vsb, p.dr);
    // Keys past T read as zeros; they only meet masked weights (or rows
    // past T, whose dQ is not written).
    auto stage_base = [&](auto st) -> unsigned char* {
        if constexpr (decltype(st)::value == 0) return lds0;
        else return lds1;
    };
    auto issue_tile = [&](int j, auto st) {
        const int k0 = j * kBwdKT;
        const int nrows = min(T_ - k0, kBwdKT);
        issue_swz_tile<D>(kp + static_cast<int64_t>(k0) * ksb, ksb, nrows, stage_base(st), wave, koff);
        issue_swz_tile<D>(vp + static_cast<int64_t>(k0) * vsb, vsb, nrows, stage_base(st) + Tl::BYTES, wave, voff);
    };

    // Interior tiles [ja, jb): every row of the wave sees every key (jb: the
    // tiles ending at or before the wave's first row; ja: the first tile past
    // the window edge of its last row).
    int ja = kv_begin;
    if (W > 0 && wq0 + 31 - W >= 0) ja = max(ja, (wq0 + 31 - W) / kBwdKT + 1);
    ja = min(ja, kv_end);
    const int jb = max(ja, min((wq0 + 1) / kBwdKT, kv_end));

    // One key tile for the wave's 32 query rows.  Masked tiles (some row of
    // the wave has keys of the tile outside its causal window or past a
    // window edge; a wave-uniform branch) skip the halves no row sees and
    // mask the rest.
    auto tile_step = [&](int j, auto st) {
        const bool masked = j < ja || j >= jb;
        const int k0 = j * kBwdKT;
        const unsigned char* Kb = stage_base(st);
        const unsigned char* Vb = stage_base(st) + Tl::BYTES;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            const int kh0 = k0 + kt * 32;
            // the wave's rows see some key of this half
            const bool act = (kh0 <= wq0 + 31) && !(W > 0 && kh0 + 31 <= wq0 - W);
            if (masked && !act) continue;
            // the dP^T chain starts at -delta (this lane's query), so it ends
            // holding dP - delta
            f32x16 s = f32x16{}, dp = ndl;
            const int r = kt * 32 + l32;
#pragma unroll
            for (int dc = 0; dc < D / 16; ++dc) {
                const int off = Tl::row_off(r, dc * 2 + hi);
                const u32x4 ka = *reinterpret_cast<const u32x4*>(Kb + off);
                const u32x4 va = *reinterpret_cast<const u32x4*>(Vb + off);
                s = Ops::mma(as_vec8<Vec>(ka), as_vec8<Vec>(qreg[dc]), s);
                dp = Ops::mma(as_vec8<Vec>(va), as_vec8<Vec>(doreg[dc]), dp);
            }
            // C layout: column = query l32, rows = keys kh0 + (v/4)*8 + 4 hi + v%4.
            const int dbase = qi - kh0 - hi * 4;
            float ds[16];
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                float y, rr;
                weight_and_rr<EXACT>(s[v], sc, y, rr);
                ds[v] = dp[v] * y * rr;
            }
            if (masked) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int cv = (v >> 2) * 8 + (v & 3);
                    ds[v] = keep_if(static_cast<unsigned>(dbase - cv) < weff, ds[v]);
                }
            }
#pragma unroll
            for (int ch = 0; ch < 2; ++ch) {
                u32x4 pw;
                pw.x = pack2<T>(ds[8 * ch + 0], ds[8 * ch + 1]);
                pw.y = pack2<T>(ds[8 * ch + 2], ds[8 * ch + 3]);
                pw.z = pack2<T>(ds[8 * ch + 4], ds[8 * ch + 5]);
                pw.w = pack2<T>(ds[8 * ch + 6], ds[8 * ch + 7]);
                const Vec bop = as_vec8<Vec>(pw);
                const int c = 2 * kt + ch;  // 16-key chunk of the tile
#pragma unroll
                for (int dt = 0; dt < D / 32; ++dt)
                    acc[dt] = Ops::mma(tr_operand<Vec, Tl>(Kb + 16 * c * Tl::ROWB, lane, dt), bop, acc[dt]);
            }
        }
    };
    // tile j reads stage `cur` while the DMA fills the other with tile j + 1
    auto run_tile = [&](int j, auto cur) {
        if (j + 1 < kv_end) issue_tile(j + 1, std::integral_constant<int, 1 - decltype(cur)::value>{});
        tile_step(j, cur);
        tile_wait_vmem();
        __syncthreads();
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    issue_tile(kv_begin, S0{});
    tile_wait_vmem();
    __syncthreads();
    for (int j = kv_begin; j < kv_end; j += 2) {
        run_tile(j, S0{});
        if (j + 1 < kv_end) run_tile(j + 1, S1{});
    }

    // dS was kept without its per-row factor 2 scale / R_i (applied here).
    // dQ leaves through LDS as whole rows (nontemporal 16-byte chunks).
    {
        constexpr int RB = D * 2 + 16, CPR = D * 2 / 16, RPI = 64 / CPR;
        static_assert(2 * 32 * RB <= 2 * Tl::BYTES, "two waves' rows per stage array");
        // both stages are free after the loop's last barrier
        unsigned char* st = (wave < 2 ? lds0 : lds1) + (wave & 1) * 32 * RB;
        const float f = 2.f * sc * inv_r;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
            for (int vg = 0; vg < 4; ++vg) {
                const int d0 = dt * 32 + vg * 8 + hi * 4;
                uint2 w;
                w.x = pack2<T>(acc[dt][vg * 4 + 0] * f, acc[dt][vg * 4 + 1] * f);
                w.y = pack2<T>(acc[dt][vg * 4 + 2] * f, acc[dt][vg * 4 + 3] * f);
                *reinterpret_cast<uint2*>(st + l32 * RB + d0 * 2) = w;
            }
        }
#pragma unroll
        for (int r0 = 0; r0 < 32; r0 += RPI) {
            const int r = r0 + lane / CPR, c = lane % CPR;
            const int qr = wq0 + r;
            const u32x4 v = *reinterpret_cast<const u32x4*>(st + r * RB + c * 16);
            if (qr < T_ && (!PART || c * 8 < p.dr)) __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(dqp + qr * p.dqs[2] + c * 8));
        }
    }
}

// ---------------------------------------------------------------------------
// dK, dV
// ---------------------------------------------------------------------------
template <typename T, int D, bool EXACT, bool PART>
__global__ __launch_bounds__(kBwdThreads, kBwdDkdvMinBlocks) void flash_bwd_dkdv_kernel(BwdParams p) {
    using Ops = MfmaOps<T>;
    using Vec = typename Ops::vec8;
    using Tl = SwzTile<D>;
    static_assert(kBwdQT == 64, "query tiles are 64 rows");
    // The two ring stages ([Q, dO] each) are separate arrays, and the loop
    // below is unrolled by two so that each iteration names its stages
    // statically: the compiler then knows that the current stage's LDS reads
    // do not touch the stage the next tile's DMA writes, and does not wait
    // for that DMA before them.
    __shared__ __attribute__((aligned(1024))) unsigned char lds0[2 * Tl::BYTES];
    __shared__ __attribute__((aligned(1024))) unsigned char lds1[2 * Tl::BYTES];
    __shared__ __attribute__((aligned(16))) float ldr[2][2][kBwdQT];   // [buf][1/R, -delta]
    // D = 128: the first NXK (NXV) chunks of the wave's K (V) operands, and
    // the low half of K chunk NXK, live in LDS and are read again for every
    // 32-query half.  The 128 accumulators plus all of K and V leave no room
    // under 256 registers, and a compiler spill instead reloads from scratch
    // inside the tile loop, where the wait for it (memory loads complete in
    // order) also waits for the next tile's DMA.  (With fast square roots
    // this leaves no spill; the exact-sqrt build keeps 12 bytes.)
    constexpr int NXK = D == 128 ? kDkdvLdsK : 0, NXV = D == 128 ? kDkdvLdsV : 0;
    __shared__ __attribute__((aligned(16))) u32x4 kvx[NXK + NXV > 0 ? NXK + NXV : 1][4][64];  // [K chunks, V chunks][wave][lane]
    constexpr bool HALFX = D == 128;
    __shared__ __attribute__((aligned(16))) uint2 kvh[HALFX ? 4 : 1][64];  // [wave][lane]: low 8 bytes of K chunk NXK

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hi = lane >> 5;
    const int l32 = lane & 31;

    const int nkb = (p.T + kBwdBK - 1) / kBwdBK;
    // Block -> (ob, split): ob indexes the unsplit grid, split the block's
    // share of ob's query tiles.  When that grid is a multiple of 8 blocks
    // the n_split blocks of one ob run on ob's XCD (blocks are dealt to the
    // XCDs by index mod 8), one after another in its dispatch order.
    const int n_split = p.n_split;
    int ob = static_cast<int>(blockIdx.x), split = 0;
    if (n_split > 1) {
        if (((nkb * p.B * p.Hkv) & 7) == 0) {
            const int j = ob >> 3;
            split = j % n_split;
            ob = ((j / n_split) << 3) | (ob & 7);
        } else {
            split = ob % n_split;
            ob /= n_split;
        }
    }
    int kb, unit, sub;
    // earliest key blocks see the most queries: first
    grouped_block(ob, p.B * p.Hkv, 1, nkb, kBwdXcdSlots, kb, unit, sub);
    const int b = unit / p.Hkv;
    const int hk = unit - b * p.Hkv;
    const int T_ = p.T;

    const T* kp = static_cast<const T*>(p.k) + b * p.ks[0] + hk * p.ks[1];
    const T* vp = static_cast<const T*>(p.v) + b * p.vs[0] + hk * p.vs[1];
    T* dkp = static_cast<T*>(p.dk) + b * p.dks[0] + hk * p.dks[1];
    T* dvp = static_cast<T*>(p.dv) + b * p.dvs[0] + hk * p.dvs[1];

    const int k_start = kb * kBwdBK;
    const int wk0 = k_start + 32 * wave;
    const int kj = wk0 + l32;
    const int krow = min(kj, T_ - 1);

    // K and V rows of the wave as B operands (column = key l32).
    u32x4 kreg[D / 16], vreg[D / 16];
#pragma unroll
    for (int dc = 0; dc < D / 16; ++dc) {
        kreg[dc] = ldg16_cols<PART>(kp + krow * p.ks[2], dc * 16 + hi * 8, p.dr);
        vreg[dc] = ldg16_cols<PART>(vp + krow * p.vs[2], dc * 16 + hi * 8, p.dr);
    }
#pragma unroll
    for (int x = 0; x < NXK; ++x) kvx[x][wave][lane] = kreg[x];
    if constexpr (HALFX) kvh[wave][lane] = uint2{kreg[NXK].x, kreg[NXK].y};
#pragma unroll
    for (int x = 0; x < NXV; ++x) kvx[NXK + x][wave][lane] = vreg[x];

    f32x16 dkacc[D / 32], dvacc[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
        dkacc[dt] = f32x16{};
        dvacc[dt] = f32x16{};
    }

    const int W = p.window;
    const unsigned weff = W > 0 ? static_cast<unsigned>(W) : 0x7FFFFFFFu;
    const int n_qt = (T_ + kBwdQT - 1) / kBwdQT;
    const int qt_begin = k_start / kBwdQT;
    const int qt_end = W > 0 ? min(n_qt, (k_start + kBwdBK - 1 + W - 1) / kBwdQT + 1) : n_qt;
    const int nq = qt_end - qt_begin;  // >= 1 (k_start < T)
    const int n_it_all = p.G * nq;
    // this block's iterations [it_lo, n_it) of the n_it_all (head, query tile) pairs
    const int it_lo = static_cast<int>(static_cast<int64_t>(split) * n_it_all / n_split);
    const int n_it = static_cast<int>(static_cast<int64_t>(split + 1) * n_it_all / n_split);
    const float sc = p.scale;

    const int qsb = static_cast<int>(p.qs[2] * 2), dsb = static_cast<int>(p.dos[2] * 2);  // row strides (bytes)
    const int qoff = swz_src_off<D, PART>(0, wave, lane, qsb, p.dr);
    const int dooff = swz_src_off<D, PART>(0, wave, lane, dsb, p.dr);
    float rst = 0.f;
    // Queries past T read as zeros; their weights are masked.
    auto stage_base = [&](auto st) -> unsigned char* {
        if constexpr (decltype(st)::value == 0) return lds0;
        else return lds1;
    };
    auto issue_tile = [&](int it, auto st) {
        const int g = it / nq;
        const int qt = qt_begin + (it - g * nq);
        const int hq = hk * p.G + g;
        const unsigned char* qp = tile_uniform_ptr(
            reinterpret_cast<const unsigned char*>(static_cast<const T*>(p.q) + b * p.qs[0] + hq * p.qs[1]));
        const unsigned char* dop = tile_uniform_ptr(
            reinterpret_cast<const unsigned char*>(static_cast<const T*>(p.dout) + b * p.dos[0] + hq * p.dos[1]));
        const int q0 = qt * kBwdQT;
        const int nrows = min(T_ - q0, kBwdQT);
        issue_swz_tile<D>(qp + static_cast<int64_t>(q0) * qsb, qsb, nrows, stage_base(st), wave, qoff);
        issue_swz_tile<D>(dop + static_cast<int64_t>(q0) * dsb, dsb, nrows, stage_base(st) + Tl::BYTES, wave, dooff);
        // the raw row sum or delta, turned into 1/R or -delta only when it is
        // stored an iteration later, so this load's latency is not waited for here
        // waves 0 and 1 (wave-uniform: the base pointer stays scalar)
        if (wave < 2) {
            const float* src = wave == 0 ? p.rs : p.delta;
            rst = src[(static_cast<int64_t>(b) * p.Hq + hq) * T_ + min(q0 + lane, T_ - 1)];
        }
    };
    auto store_rs = [&](int buf) {
        if (tid < 2 * kBwdQT) ldr[buf][tid / kBwdQT][tid & (kBwdQT - 1)] = tid < kBwdQT ? 1.f / rst : -rst;
    };

    // One query tile (iteration it: head g = it / nq, tile qt_begin + it % nq)
    // for the wave's 32 keys.  Masks are applied (a wave-uniform branch
    // around them) only when some (query, key) pair of the tile is outside
    // the causal window, past a window edge or past T; halves no query of
    // which sees a key of the wave are skipped.  (One loop with the branch
    // inside keeps the 128 accumulator registers in place; separate loops
    // per tile kind made the compiler spill them.)
    auto tile_step = [&](int it, auto st) {
        constexpr int buf = decltype(st)::value;
        const int g = it / nq;
        const int q0 = (qt_begin + (it - g * nq)) * kBwdQT;
        const bool interior = q0 >= wk0 + 31 && q0 + kBwdQT <= T_ && !(W > 0 && q0 + kBwdQT - 1 - wk0 >= W);
        const unsigned char* Qb = stage_base(st);
        const unsigned char* Ob = stage_base(st) + Tl::BYTES;
#pragma unroll
        for (int qh = 0; qh < 2; ++qh) {
            const int qh0 = q0 + qh * 32;
            // some query of this half sees some key of the wave
            const bool act = (qh0 + 31 >= wk0) && !(W > 0 && qh0 - (wk0 + 31) >= W) && qh0 < T_;
            if (!act) continue;
            // the dP chain starts at -delta of its query rows (C layout, read
            // from the staged -delta), so it ends holding dP - delta
            f32x16 s = f32x16{}, dp;
#pragma unroll
            for (int vg = 0; vg < 4; ++vg) {
                const float4 nd = *reinterpret_cast<const float4*>(&ldr[buf][1][qh * 32 + vg * 8 + hi * 4]);
                dp[vg * 4 + 0] = nd.x;
                dp[vg * 4 + 1] = nd.y;
                dp[vg * 4 + 2] = nd.z;
                dp[vg * 4 + 3] = nd.w;
            }
            const int r = qh * 32 + l32;
            // re-read the LDS-held chunks for this half (not kept in registers across halves)
            if constexpr (NXK + NXV > 0) asm volatile("" ::: "memory");
#pragma unroll
            for (int dc = 0; dc < D / 16; ++dc) {
                const int off = Tl::row_off(r, dc * 2 + hi);
                const u32x4 qa = *reinterpret_cast<const u32x4*>(Qb + off);
                const u32x4 oa = *reinterpret_cast<const u32x4*>(Ob + off);
                u32x4 kb = dc < NXK ? kvx[dc < NXK ? dc : 0][wave][lane] : kreg[dc];
                if (HALFX && dc == NXK) {
                    const uint2 lo = kvh[wave][lane];
                    kb.x = lo.x;
                    kb.y = lo.y;
                }
                const u32x4 vb = dc < NXV ? kvx[dc < NXV ? NXK + dc : 0][wave][lane] : vreg[dc];
                s = Ops::mma(as_vec8<Vec>(qa), as_vec8<Vec>(kb), s);
                dp = Ops::mma(as_vec8<Vec>(oa), as_vec8<Vec>(vb), dp);
            }
            // C layout: column = key kj, rows = queries qh0 + (v/4)*8 + 4 hi + v%4.
            float pv[16], ds[16];
            const int dbase = qh0 + hi * 4 - kj;
            const int qlim = T_ - (qh0 + hi * 4);  // row offsets below this are real queries
#pragma unroll
            for (int vg = 0; vg < 4; ++vg) {
                const int roff = qh * 32 + vg * 8 + hi * 4;
                const float4 ir = *reinterpret_cast<const float4*>(&ldr[buf][0][roff]);
                const float irv[4] = {ir.x, ir.y, ir.z, ir.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int v = vg * 4 + e;
                    float y, rr;
                    weight_and_rr<EXACT>(s[v], sc, y, rr);
                    const float yi = y * irv[e];
                    pv[v] = yi;
                    ds[v] = dp[v] * yi * rr;
                }
            }
            if (!interior) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int cv = (v >> 2) * 8 + (v & 3);
                    const bool ok = (static_cast<unsigned>(dbase + cv) < weff) && (cv < qlim);
                    pv[v] = keep_if(ok, pv[v]);
                    ds[v] = keep_if(ok, ds[v]);
                }
            }
#pragma unroll
            for (int ch = 0; ch < 2; ++ch) {
                u32x4 pw, sw;
                pw.x = pack2<T>(pv[8 * ch + 0], pv[8 * ch + 1]);
                pw.y = pack2<T>(pv[8 * ch + 2], pv[8 * ch + 3]);
                pw.z = pack2<T>(pv[8 * ch + 4], pv[8 * ch + 5]);
                pw.w = pack2<T>(pv[8 * ch + 6], pv[8 * ch + 7]);
                sw.x = pack2<T>(ds[8 * ch + 0], ds[8 * ch + 1]);
                sw.y = pack2<T>(ds[8 * ch + 2], ds[8 * ch + 3]);
                sw.z = pack2<T>(ds[8 * ch + 4], ds[8 * ch + 5]);
                sw.w = pack2<T>(ds[8 * ch + 6], ds[8 * ch + 7]);
                const Vec bp = as_vec8<Vec>(pw);
                const Vec bs = as_vec8<Vec>(sw);
                const int c = 2 * qh + ch;  // 16-query chunk of the tile
#pragma unroll
                for (int dt = 0; dt < D / 32; ++dt) {
                    const int to = 16 * c * Tl::ROWB;
                    dvacc[dt] = Ops::mma(tr_operand<Vec, Tl>(Ob + to, lane, dt), bp, dvacc[dt]);
                    dkacc[dt] = Ops::mma(tr_operand<Vec, Tl>(Qb + to, lane, dt), bs, dkacc[dt]);
                }
            }
        }
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    // (it_lo < n_it for every block unless a split holds no iteration; the
    // branch is block-uniform, so every wave meets the same barriers)
    if (it_lo < n_it) {
        issue_tile(it_lo, S0{});
        store_rs(0);
        tile_wait_vmem();
        __syncthreads();
    }
    // iteration it reads stage `cur` while the DMA fills stage `nxt` with it + 1
    auto iteration = [&](int it, auto cur, auto nxt) {
        const bool has_next = it + 1 < n_it;
        if (has_next) issue_tile(it + 1, nxt);
        tile_step(it, cur);
        if (has_next) store_rs(decltype(nxt)::value);
        tile_wait_vmem();
        __syncthreads();
    };
    for (int it = it_lo; it < n_it; it += 2) {
        iteration(it, S0{}, S1{});
        if (it + 1 < n_it) iteration(it + 1, S1{}, S0{});
    }

    if (n_split > 1) {
        // fp32 partials (zeros for a split without iterations), all D columns
        if (kj < T_) {
            const int64_t bh = static_cast<int64_t>(p.B) * p.Hkv;
            float* pk = p.part + ((static_cast<int64_t>(split) * 2 * bh + unit) * T_ + kj) * D;
            float* pv = pk + bh * T_ * D;
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
                for (int vg = 0; vg < 4; ++vg) {
                    const int d0 = dt * 32 + vg * 8 + hi * 4;
                    *reinterpret_cast<float4*>(pk + d0) = float4{dkacc[dt][vg * 4 + 0], dkacc[dt][vg * 4 + 1],
                                                                 dkacc[dt][vg * 4 + 2], dkacc[dt][vg * 4 + 3]};
                    *reinterpret_cast<float4*>(pv + d0) = float4{dvacc[dt][vg * 4 + 0], dvacc[dt][vg * 4 + 1],
                                                                 dvacc[dt][vg * 4 + 2], dvacc[dt][vg * 4 + 3]};
                }
            }
        }
        return;
    }

    // dS was kept without its factor 2 scale (1/R_i is already in).  dK and
    // dV leave through LDS as whole rows (nontemporal 16-byte chunks).
    {
        constexpr int RB = D * 2 + 16, CPR = D * 2 / 16, RPI = 64 / CPR;
        static_assert(2 * 32 * RB <= 2 * Tl::BYTES, "two waves' rows per stage array");
        unsigned char* st = (wave < 2 ? lds0 : lds1) + (wave & 1) * 32 * RB;
        const float f = 2.f * sc;
#pragma unroll
        for (int which = 0; which < 2; ++which) {
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
                for (int vg = 0; vg < 4; ++vg) {
                    const int d0 = dt * 32 + vg * 8 + hi * 4;
                    uint2 w;
                    if (which == 0) {
                        w.x = pack2<T>(dkacc[dt][vg * 4 + 0] * f, dkacc[dt][vg * 4 + 1] * f);
                        w.y = pack2<T>(dkacc[dt][vg * 4 + 2] * f, dkacc[dt][vg * 4 + 3] * f);
                    } else {
                        w.x = pack2<T>(dvacc[dt][vg * 4 + 0], dvacc[dt][vg * 4 + 1]);
                        w.y = pack2<T>(dvacc[dt][vg * 4 + 2], dvacc[dt][vg * 4 + 3]);
                    }
                    *reinterpret_cast<uint2*>(st + l32 * RB + d0 * 2) = w;
                }
            }
            T* base = which == 0 ? dkp : dvp;
            const int64_t rs = which == 0 ? p.dks[2] : p.dvs[2];
#pragma unroll
            for (int r0 = 0; r0 < 32; r0 += RPI) {
                const int r = r0 + lane / CPR, c = lane % CPR;
                const int kr = wk0 + r;
                const u32x4 v = *reinterpret_cast<const u32x4*>(st + r * RB + c * 16);
                if (kr < T_ && (!PART || c * 8 < p.dr))
                    __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(base + kr * rs + c * 8));
            }
        }
    }
}

// dK, dV = the sum of the n_split fp32 partials (in split order, so the
// result does not depend on timing), dK times 2 scale; one thread per four
// columns of a key row.
template <typename T, int D>
__global__ __launch_bounds__(256) void bwd_split_reduce_kernel(BwdParams p, int64_t n_quads) {
    const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (gid >= n_quads) return;
    const int64_t row = gid / (D / 4);  // (b * Hkv + hk) * T + key
    const int d0 = static_cast<int>(gid - row * (D / 4)) * 4;
    if (d0 >= p.dr) return;
    const int64_t plane = static_cast<int64_t>(p.B) * p.Hkv * p.T * D;
    const float* src = p.part + row * D + d0;
    float4 k4 = float4{0.f, 0.f, 0.f, 0.f}, v4 = float4{0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < p.n_split; ++s) {
        const float4 a = *reinterpret_cast<const float4*>(src + (2 * s) * plane);
        const float4 c = *reinterpret_cast<const float4*>(src + (2 * s + 1) * plane);
        k4.x += a.x; k4.y += a.y; k4.z += a.z; k4.w += a.w;
        v4.x += c.x; v4.y += c.y; v4.z += c.z; v4.w += c.w;
    }
    const float f = 2.f * p.scale;
    const int64_t bh = row / p.T;
    const int key = static_cast<int>(row - bh * p.T);
    const int b = static_cast<int>(bh / p.Hkv);
    const int hk = static_cast<int>(bh - static_cast<int64_t>(b) * p.Hkv);
    T* dk = static_cast<T*>(p.dk) + b * p.dks[0] + hk * p.dks[1] + key * p.dks[2] + d0;
    T* dv = static_cast<T*>(p.dv) + b * p.dvs[0] + hk * p.dvs[1] + key * p.dvs[2] + d0;
    *reinterpret_cast<uint2*>(dk) = uint2{pack2<T>(k4.x * f, k4.y * f), pack2<T>(k4.z * f, k4.w * f)};
    *reinterpret_cast<uint2*>(dv) = uint2{pack2<T>(v4.x, v4.y), pack2<T>(v4.z, v4.w)};
}

template <typename T, int D, bool PART>
int launch_bwd_part(const BwdParams& prm, int exact, hipStream_t st) {
    const unsigned nqb = static_cast<unsigned>((prm.T + kBwdBQ - 1) / kBwdBQ);
    const unsigned nkb = static_cast<unsigned>((prm.T + kBwdBK - 1) / kBwdBK);
    const dim3 gq(nqb * prm.B * prm.Hq), gk(nkb * prm.B * prm.Hkv * prm.n_split), blk(kBwdThreads);
    if (exact) {
        flash_bwd_dq_kernel<T, D, true, PART><<<gq, blk, 0, st>>>(prm);
        flash_bwd_dkdv_kernel<T, D, true, PART><<<gk, blk, 0, st>>>(prm);
    } else {
        flash_bwd_dq_kernel<T, D, false, PART><<<gq, blk, 0, st>>>(prm);
        flash_bwd_dkdv_kernel<T, D, false, PART><<<gk, blk, 0, st>>>(prm);
    }
    if (prm.n_split > 1) {
        const int64_t n_quads = static_cast<int64_t>(prm.B) * prm.Hkv * prm.T * (D / 4);
        bwd_split_reduce_kernel<T, D><<<static_cast<unsigned>((n_quads + 255) / 256), 256, 0, st>>>(prm, n_quads);
    }
    return status_from_launch();
}

// The masked kernels (PART) only where the head dim is below D: the masks
// cost the dK/dV kernel registers, and at D = 128 spills in its tile loop.
template <typename T, int D>
int launch_bwd(const BwdParams& prm, int exact, hipStream_t st) {
    if (prm.dr == D) return launch_bwd_part<T, D, false>(prm, exact, st);
    return launch_bwd_part<T, D, true>(prm, exact, st);
}

// Head dims 8..128 (multiples of 8) run on the kernels for the next of 32,
// 64, 128 with the columns past prm.dr masked.
template <typename T>
int launch_bwd_d(const BwdParams& prm, int exact, hipStream_t st) {
    if (prm.dr <= 32) return launch_bwd<T, 32>(prm, exact, st);
    if (prm.dr <= 64) return launch_bwd<T, 64>(prm, exact, st);
    return launch_bwd<T, 128>(prm, exact, st);
}

// (b, h, t) strides keep every row 16-byte aligned; d stride 1.
bool bwd_strides_ok(const int64_t* s) { return s[3] == 1 && s[0] % 8 == 0 && s[1] % 8 == 0 && s[2] % 8 == 0; }

// Kernel head dim of the 16-bit kernels for head dim dr <= 128.
int bwd_kernel_d(int dr) { return dr <= 32 ? 32 : dr <= 64 ? 64 : 128; }

int64_t bwd_part_bytes(int n_split, int B, int Hkv, int T, int dr) {
    return n_split > 1 ? static_cast<int64_t>(n_split) * 2 * B * Hkv * T * bwd_kernel_d(dr) * 4 : 0;
}

// (head, query tile) iterations of dK/dV key block kb, as the kernel counts them.
int dkdv_iterations(int kb, int T, int G, int W) {
    const int n_qt = (T + kBwdQT - 1) / kBwdQT;
    const int k_start = kb * kBwdBK;
    const int qt_begin = k_start / kBwdQT;
    const int qt_end = W > 0 ? std::min(n_qt, (k_start + kBwdBK - 1 + W - 1) / kBwdQT + 1) : n_qt;
    return G * (qt_end - qt_begin);
}

// Query-tile splits of the dK/dV blocks.  Causally, key block kb sees the
// query tiles from its own on, so the first blocks hold the most work; in a
// grid that does not fill the chip several times over, the GPU idles while
// they finish.  Splitting every block's iterations n_split ways (fp32
// partials, summed by one more kernel) shortens that tail at the cost of the
// partials' traffic.  The count is the one of 1, 2, 4, 8, 16 with the least
// estimated time: blocks dealt to the XCDs round-robin in the kernel's order
// (heaviest key blocks first), each XCD running kBwdXcdSlots at once, a block
// costing its iterations plus two for its set-up and stores, plus a fifth of
// the longest block for the ragged end, an iteration at 5 us (a 64-query
// tile of 128 keys with two blocks per CU), and the partials' writes and
// reads at 5 TB/s; at most 512 MiB of partials.  (Fitted to measured times
// of shapes from 1 x 2 KV heads x 4096 keys to 2 x 8 x 16384, where it picks
// the fastest count of each.)  Grids of 4096 blocks or more are not split.
int dkdv_split_count_uncached(int B, int Hkv, int T, int G, int W, int dr) {
    const int nkb = (T + kBwdBK - 1) / kBwdBK;
    const int64_t blocks = static_cast<int64_t>(nkb) * B * Hkv;
    int best = 1;
    double best_t = 0.0;
    for (int S = 1; S <= 16; S *= 2) {
        // at most 16384 blocks and 512 MiB of partials
        if (blocks * S > 16384 || bwd_part_bytes(S, B, Hkv, T, dr) > (int64_t(512) << 20)) break;
        double t = dkdv_split_makespan(nkb, B * Hkv, S, kBwdXcdSlots, 2.0,
                                       [&](int kb) { return dkdv_iterations(kb, T, G, W); }) *
                   5.0;  // us
        // the partials written, then read by the sum kernel
        if (S > 1) t += 2.0 * static_cast<double>(bwd_part_bytes(S, B, Hkv, T, dr)) / 5e6 + 5.0;
        if (S == 1 || t < best_t) {
            best = S;
            best_t = t;
        }
    }
    return best;
}

int dkdv_split_count(int B, int Hkv, int T, int G, int W, int dr) {
    const int64_t blocks = static_cast<int64_t>((T + kBwdBK - 1) / kBwdBK) * B * Hkv;
    if (blocks >= 8 * kBwdXcdSlots * 8 || blocks == 0) return 1;
    static SplitCountCache cache;
    const int key[6] = {B, Hkv, T, G, W, bwd_kernel_d(dr)};
    return cache.get(key, [&] { return dkdv_split_count_uncached(B, Hkv, T, G, W, dr); });
}

}  // namespace
}  // namespace sa

extern "C" int64_t sa_flash_bwd_workspace_size(int B, int Hq, int Hkv, int T, int D, int window_size, int dtype) {
    using namespace sa;
    if (B < 0 || Hq <= 0 || Hkv <= 0 || T < 0 || D <= 0 || Hq % Hkv != 0 || window_size < 0) return -1;
    if (dtype != SA_BF16 && dtype != SA_F16) return 0;
    if (B == 0 || T == 0 || D > 512) return 0;
    if (D > 128) return flash_bwd_wide_workspace_size(B, Hq, Hkv, T, D, window_size);
    return bwd_part_bytes(dkdv_split_count(B, Hkv, T, Hq / Hkv, window_size, D), B, Hkv, T, D);
}

extern "C" int sa_flash_bwd_ws(const void* q, const void* k, const void* v, const void* o, const void* dout,
                               const float* row_sums, void* dq, void* dk, void* dv, float* delta_ws, int B, int Hq,
                               int Hkv, int T, int D, const int64_t* q_strides, const int64_t* k_strides,
                               const int64_t* v_strides, const int64_t* o_strides, const int64_t* do_strides,
                               const int64_t* dq_strides, const int64_t* dk_strides, const int64_t* dv_strides,
                               float scale, int window_size, int exact_math, int dtype, void* workspace,
                               int64_t workspace_bytes, sa_stream_t stream) {
    using namespace sa;
    if (dtype == SA_F32) {
        const int64_t* const all[8] = {q_strides,  k_strides,  v_strides,  o_strides,
                                       do_strides, dq_strides, dk_strides, dv_strides};
        return flash_bwd_f32(q, k, v, o, dout, row_sums, dq, dk, dv, delta_ws, B, Hq, Hkv, T, D, all, scale,
                             window_size, exact_math, reinterpret_cast<hipStream_t>(stream));
    }
    if (dtype != SA_BF16 && dtype != SA_F16) return SA_ERR_BAD_DTYPE;
    if (D > 128) {
        const int64_t* const all[8] = {q_strides,  k_strides,  v_strides,  o_strides,
                                       do_strides, dq_strides, dk_strides, dv_strides};
        return flash_bwd_wide(q, k, v, o, dout, row_sums, dq, dk, dv, delta_ws, B, Hq, Hkv, T, D, all, scale,
                              window_size, exact_math, dtype, workspace, workspace_bytes,
                              reinterpret_cast<hipStream_t>(stream));
    }
    if (B < 0 || Hq <= 0 || Hkv <= 0 || T < 0 || Hq % Hkv != 0 || window_size < 0) return SA_ERR_BAD_SHAPE;
    if (!q || !k || !v || !o || !dout || !row_sums || !dq || !dk || !dv || !delta_ws) return SA_ERR_NULL_POINTER;
    if (!q_strides || !k_strides || !v_strides || !o_strides || !do_strides || !dq_strides || !dk_strides ||
        !dv_strides)
        return SA_ERR_NULL_POINTER;
    if (D < 8 || D % 8 != 0) return SA_ERR_UNSUPPORTED;
    const int64_t* all[8] = {q_strides, k_strides, v_strides, o_strides, do_strides, dq_strides, dk_strides, dv_strides};
    for (const int64_t* s : all)
        if (!bwd_strides_ok(s)) return SA_ERR_BAD_STRIDE;
    // Q / K / V / dO tiles are addressed with 32-bit offsets within 64 rows.
    for (const int64_t* st : {q_strides, k_strides, v_strides, do_strides})
        if (st[2] * 2 > (int64_t(1) << 24)) return SA_ERR_BAD_STRIDE;
    const void* ptrs[8] = {q, k, v, o, dout, dq, dk, dv};
    for (const void* ptr : ptrs)
        if (!aligned16(ptr)) return SA_ERR_BAD_STRIDE;
    if (B == 0 || T == 0) return 0;
    BwdParams prm{};
    prm.q = q;
    prm.k = k;
    prm.v = v;
    prm.o = o;
    prm.dout = dout;
    prm.rs = row_sums;
    prm.dq = dq;
    prm.dk = dk;
    prm.dv = dv;
    prm.delta = delta_ws;
    for (int i = 0; i < 4; ++i) {
        prm.qs[i] = q_strides[i];
        prm.ks[i] = k_strides[i];
        prm.vs[i] = v_strides[i];
        prm.os[i] = o_strides[i];
        prm.dos[i] = do_strides[i];
        prm.dqs[i] = dq_strides[i];
        prm.dks[i] = dk_strides[i];
        prm.dvs[i] = dv_strides[i];
    }
    prm.B = B;
    prm.Hq = Hq;
    prm.Hkv = Hkv;
    prm.T = T;
    prm.G = Hq / Hkv;
    prm.window = window_size;
    prm.dr = D;
    prm.scale = scale;
    // the library's split count, or the largest power of two below it whose
    // partials fit the workspace
    prm.n_split = 1;
    prm.part = nullptr;
    if (workspace && workspace_bytes > 0) {
        if (!aligned16(workspace)) return SA_ERR_BAD_STRIDE;
        int ns = dkdv_split_count(B, Hkv, T, prm.G, window_size, D);
        while (ns > 1 && bwd_part_bytes(ns, B, Hkv, T, D) > workspace_bytes) ns /= 2;
        prm.n_split = ns;
        prm.part = static_cast<float*>(workspace);
    }
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int ex = exact_math ? 1 : 0;
    if (dtype == SA_BF16) return launch_bwd_d<bf16>(prm, ex, s);
    return launch_bwd_d<f16>(prm, ex, s);
}

extern "C" int sa_flash_bwd(const void* q, const void* k, const void* v, const void* o, const void* dout,
                            const float* row_sums, void* dq, void* dk, void* dv, float* delta_ws, int B, int Hq,
                            int Hkv, int T, int D, const int64_t* q_strides, const int64_t* k_strides,
                            const int64_t* v_strides, const int64_t* o_strides, const int64_t* do_strides,
                            const int64_t* dq_strides, const int64_t* dk_strides, const int64_t* dv_strides,
                            float scale, int window_size, int exact_math, int dtype, sa_stream_t stream) {
    return sa_flash_bwd_ws(q, k, v, o, dout, row_sums, dq, dk, dv, delta_ws, B, Hq, Hkv, T, D, q_strides, k_strides,
                           v_strides, o_strides, do_strides, dq_strides, dk_strides, dv_strides, scale, window_size,
                           exact_math, dtype, nullptr, 0, stream);
}
