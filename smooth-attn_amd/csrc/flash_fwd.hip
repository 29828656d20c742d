// Fused causal squareplus attention forward on gfx950 MFMA: bf16 / fp16, and
// fp8 e4m3fn QK^T with bf16 P V.
//
// O_i = sum_{j <= i, i - j < W} y_ij V_j / (sum_j y_ij + 1e-12),
// y = squareplus(2 s - 1)^2, s = scale q_i . k_j
//   (reference kernels.py:1536-1631 bf16, :2498-2589 fp8)
//
// Squareplus needs no running maximum, so the weights are accumulated
// linearly (sum y in fp32; P V on MFMA with P rounded to the 16-bit type,
// as the reference does at :1617-1621 and :2579) and divided once at the end.
//
// Work decomposition: a block of 8 waves (2 per SIMD) owns 256 query rows of
// one (batch, query head); wave w owns rows [32w, 32w+32).  K and V tiles of
// 64 keys go straight from global memory into a 3-stage LDS ring
// (global_load_lds, no staging registers), one barrier per tile.  Per wave
// and tile: S^T = K Q^T on MFMA, the squareplus weights on the VALU (masks
// only on tiles crossing the diagonal or the window edge), then
// O^T += V^T P^T on MFMA.  The walk is software-pipelined over 32-key
// halves, across the tile boundary too: the barrier that publishes tile t+1
// comes in the middle of tile t, so the first S^T MFMAs of tile t+1 overlap
// the weights and P V of tile t's second half (the third stage keeps tile t
// readable while tile t+2 is in flight).  fp8 V is widened to the 16-bit
// type while it is staged through registers (exact: e4m3fn values are
// representable in bf16) and v_scale is applied once at the end.
// Block order: see block_coords (XCD-aware, heaviest query blocks first).
#include <type_traits>

#include "flash_common.hpp"
#include "flash_tiles.hpp"
#include "flash_f32.hpp"
#include "flash_wide.hpp"

namespace sa {
namespace {

// Block shape: 64-key tiles, one 32-row query tile per wave, 8 waves (the
// code also takes other multiples of 32 keys and two query tiles per wave;
// 32- and 96-key tiles, 4-wave blocks and two query tiles per wave measured
// slower on config 3).
constexpr int kBKV = 64;              // keys per tile (a multiple of 32)
constexpr int kQT = 1;                // 32-row query tiles per wave
constexpr int kWaves = 8 / kQT;       // waves per block (256 query rows)
constexpr int kThreads = 64 * kWaves;
constexpr int kStages = 3;    // LDS ring of K/V tiles

struct FlashParams {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* row_sums;
    const float* q_scale;  // fp8 only (device scalars)
    const float* k_scale;
    const float* v_scale;
    const float* rope_cos;  // RoPE tables [T, D/2] fp32 (RoPE variant only)
    const float* rope_sin;
    int64_t qs[4], ks[4], vs[4], os[4];
    int B, Hq, Hkv, T, G, window, nqb;
    int dr;  // head dim of the tensors (<= D, a multiple of 8; columns past it read as zero, are not stored)
    float scale;
};

// T: 16-bit type of P V (and of q/k/v unless fp8).  QK8: q, k are e4m3fn.
// V8: v is e4m3fn.
//
// LDS tiles are unpadded rows of 16-byte chunks, filled by direct
// global->LDS loads (global_load_lds_dwordx4: lane i of a wave writes bytes
// [16 i, 16 i + 16) after the wave's base, so one instruction fills 1 KB of
// consecutive chunks).  The LDS has 64 banks of 4 bytes (256 bytes per
// cycle): a 16-byte read is served 16 lanes per cycle, an 8-byte
// (transposing) read 32 lanes per cycle, and each group is conflict-free
// when its lanes cover 256 distinct bytes modulo 256.  Storing logical chunk
// c of row r at chunk c ^ swz(r) achieves that:
//  * K (16-byte A-operand rows, 16 consecutive rows per cycle at the same
//    logical chunk): swz_k gives the 16 rows 16 distinct 16-byte slots of
//    the 256-byte bank window;
//  * V (ds_read_b64_tr_b16: per 32 lanes, 4 consecutive rows x 64 bytes):
//    swz_v moves the 4 rows' 64-byte groups to 4 distinct 64-byte slots.
template <typename T, int D, bool QK8, bool V8>
struct Geom {
    static constexpr int QKB = QK8 ? 1 : 2;             // bytes per q/k element
    static constexpr int KROWB = D * QKB;               // K row bytes in LDS
    static constexpr int VROWB = D * 2;                 // V row bytes in LDS (16-bit)
    static constexpr int KT = kBKV * KROWB;             // bytes per K tile
    static constexpr int VT = kBKV * VROWB;             // bytes per V tile
    static constexpr int KCPR = KROWB / 16;             // 16-byte chunks per K row
    static constexpr int VCPRL = VROWB / 16;            // chunks per V row in LDS
    static constexpr int VCPRG = D * (V8 ? 1 : 2) / 16; // chunks per V row in global memory
    static constexpr int KNI = (kBKV * KCPR + kThreads - 1) / kThreads;   // K DMA loads per lane
    static constexpr int VNI = (kBKV * VCPRL + kThreads - 1) / kThreads;  // V DMA loads per lane
    static constexpr int VNL = (kBKV * VCPRG + kThreads - 1) / kThreads;  // staged fp8 V loads
    static constexpr int NQC = QK8 ? (D + 63) / 64 : D / 16;  // MFMAs per 32x32 score tile
    // rows sharing one 256-byte bank window
    static constexpr int KRPW = KCPR >= 16 ? 1 : 16 / KCPR;
    static constexpr int VRPW = VCPRL >= 16 ? 1 : 16 / VCPRL;
    static __device__ __forceinline__ int swz_k(int r) { return (r / KRPW) & (KCPR - 1); }
    static __device__ __forceinline__ int swz_v(int r) { return 4 * ((r / VRPW) & (VCPRL / 4 - 1)); }
};

// e4m3 x e4m3 with block scales 2^(ea-127) and 2^(eb-127) (E8M0; 127 =
// 2^0): D = 2^(ea+eb-254) sum a b + C, the power of two applied exactly.
__device__ __forceinline__ f32x16 mma_fp8(i32x8 a, i32x8 b, f32x16 c, int ea, int eb) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, ea, 0, eb);
}

// Rotate-half RoPE of one pair of 8-element chunks, a = x[d .. d+7] and
// b = x[d + D/2 .. +7] with d < D/2 (reference kernels.py:2150-2158):
//   a' = a cos - b sin,  b' = b cos + a sin   (fp32, rounded to T).
template <typename T>
__device__ __forceinline__ void rope_rotate8(u32x4& a, u32x4& b, const float* cs, const float* sn) {
    const uint32_t aw[4] = {a.x, a.y, a.z, a.w};
    const uint32_t bw[4] = {b.x, b.y, b.z, b.w};
    float ra[8], rb[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float av = elem<T>(aw, e), bv = elem<T>(bw, e);
        ra[e] = av * cs[e] - bv * sn[e];
        rb[e] = bv * cs[e] + av * sn[e];
    }
    a = u32x4{pack2<T>(ra[0], ra[1]), pack2<T>(ra[2], ra[3]), pack2<T>(ra[4], ra[5]), pack2<T>(ra[6], ra[7])};
    b = u32x4{pack2<T>(rb[0], rb[1]), pack2<T>(rb[2], rb[3]), pack2<T>(rb[4], rb[5]), pack2<T>(rb[6], rb[7])};
}

// Rotates every row of K once into a contiguous [B, Hkv, T, D] buffer for the
// RoPE forward (each K tile is re-read by every query block of its head, so
// rotating K once beats rotating it in each block).  One thread per pair of
// 16-byte chunks (d, d + D/2).
template <typename T, int D>
__global__ __launch_bounds__(256) void rope_rotate_rows(const T* __restrict__ k, T* __restrict__ out,
                                                        const float* __restrict__ cs, const float* __restrict__ sn,
                                                        int Hkv, int T_, int64_t s0, int64_t s1, int64_t s2,
                                                        int64_t n_pairs) {
    constexpr int PPR = D / 16;  // chunk pairs per row
    const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (gid >= n_pairs) return;
    const int64_t row = gid / PPR;
    const int c = static_cast<int>(gid - row * PPR);
    const int64_t bh = row / T_;
    const int t = static_cast<int>(row - bh * T_);
    const int b = static_cast<int>(bh / Hkv);
    const int h = static_cast<int>(bh - static_cast<int64_t>(b) * Hkv);
    const T* src = k + b * s0 + h * s1 + t * s2 + c * 8;
    u32x4 a = load16(src);
    u32x4 bb = load16(src + D / 2);
    float cv[8], sv[8];
    const float* cr = cs + static_cast<int64_t>(t) * (D / 2) + c * 8;
    const float* sr = sn + static_cast<int64_t>(t) * (D / 2) + c * 8;
    *reinterpret_cast<float4*>(cv) = *reinterpret_cast<const float4*>(cr);
    *reinterpret_cast<float4*>(cv + 4) = *reinterpret_cast<const float4*>(cr + 4);
    *reinterpret_cast<float4*>(sv) = *reinterpret_cast<const float4*>(sr);
    *reinterpret_cast<float4*>(sv + 4) = *reinterpret_cast<const float4*>(sr + 4);
    rope_rotate8<T>(a, bb, cv, sv);
    T* dst = out + row * D + c * 8;
    *reinterpret_cast<u32x4*>(dst) = a;
    *reinterpret_cast<u32x4*>(dst + D / 2) = bb;
}

// The same rotation for any head dim D that is a multiple of 16 (pairs of
// 16-byte chunks (d, d + D/2)), from strided rows into a contiguous
// [B, H, T, D] buffer: the first pass of RoPE attention at head dims the
// fused Q rotation does not cover.
template <typename T>
__global__ __launch_bounds__(256) void rope_rotate_any(const T* __restrict__ x, T* __restrict__ out,
                                                       const float* __restrict__ cs, const float* __restrict__ sn,
                                                       int H, int T_, int D, int64_t s0, int64_t s1, int64_t s2,
                                                       int64_t n_pairs) {
    const int ppr = D / 16;  // chunk pairs per row
    const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (gid >= n_pairs) return;
    const int64_t row = gid / ppr;
    const int c = static_cast<int>(gid - row * ppr);
    const int64_t bh = row / T_;
    const int t = static_cast<int>(row - bh * T_);
    const int b = static_cast<int>(bh / H);
    const int h = static_cast<int>(bh - static_cast<int64_t>(b) * H);
    const T* src = x + b * s0 + h * s1 + t * s2 + c * 8;
    float cv[8], sv[8];
    const float* cr = cs + static_cast<int64_t>(t) * (D / 2) + c * 8;
    const float* sr = sn + static_cast<int64_t>(t) * (D / 2) + c * 8;
    *reinterpret_cast<float4*>(cv) = *reinterpret_cast<const float4*>(cr);
    *reinterpret_cast<float4*>(cv + 4) = *reinterpret_cast<const float4*>(cr + 4);
    *reinterpret_cast<float4*>(sv) = *reinterpret_cast<const float4*>(sr);
    *reinterpret_cast<float4*>(sv + 4) = *reinterpret_cast<const float4*>(sr + 4);
    T* dst = out + row * D + c * 8;
    if constexpr (std::is_same_v<T, float>) {  // 8 fp32 elements: two 16-byte loads per half
        float a[8], bb[8];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            *reinterpret_cast<float4*>(a + 4 * j) = *reinterpret_cast<const float4*>(src + 4 * j);
            *reinterpret_cast<float4*>(bb + 4 * j) = *reinterpret_cast<const float4*>(src + D / 2 + 4 * j);
        }
        float ra[8], rb[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            ra[e] = a[e] * cv[e] - bb[e] * sv[e];
            rb[e] = bb[e] * cv[e] + a[e] * sv[e];
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            *reinterpret_cast<float4*>(dst + 4 * j) = *reinterpret_cast<const float4*>(ra + 4 * j);
            *reinterpret_cast<float4*>(dst + D / 2 + 4 * j) = *reinterpret_cast<const float4*>(rb + 4 * j);
        }
    } else {
        u32x4 a = load16(src);
        u32x4 bb = load16(src + D / 2);
        rope_rotate8<T>(a, bb, cv, sv);
        *reinterpret_cast<u32x4*>(dst) = a;
        *reinterpret_cast<u32x4*>(dst + D / 2) = bb;
    }
}

// K/V tile loads: every tile is read by all query blocks of its head, so
// these loads are cached (a nontemporal load would stream past L2).
template <typename T>
__device__ __forceinline__ u32x4 tile_load16(const T* p) {
    return *reinterpret_cast<const u32x4*>(p);
}

// Block -> (query block, batch, query head): grouped_block over the KV heads
// (units) and the query heads sharing each (sub), heaviest query block first;
// one block per CU, so an XCD runs 32 at once.
constexpr int kBlocksPerXcd = 32;
__device__ __forceinline__ void block_coords(const FlashParams& p, int& qb, int& b, int& hq) {
    int step, unit, sub;
    grouped_block(blockIdx.x, p.B * p.Hkv, p.G, p.nqb, kBlocksPerXcd, step, unit, sub);
    qb = p.nqb - 1 - step;
    b = unit / p.Hkv;
    hq = (unit - b * p.Hkv) * p.G + sub;
}

constexpr int kBQ2 = 32 * kWaves * kQT;  // query rows per block

// One block per CU: with one query tile per wave, 8 waves (2 per SIMD, 256
// VGPRs per lane); with two, 4 waves (1 per SIMD, 512 registers per lane,
// the O accumulators in AGPRs).
template <typename T, int D, bool QK8, bool V8, bool EXACT, bool ROPE, bool FOLD = false>
__global__ __launch_bounds__(kThreads, 1) void flash_fwd_kernel(FlashParams p) {
    using Gm = Geom<T, D, QK8, V8>;
    using Ops = MfmaOps<T>;
    using Vec = typename Ops::vec8;
    using KFrag = std::conditional_t<QK8, i32x8, Vec>;  // A operand of one S^T MFMA
    static_assert(kBKV % 32 == 0, "the pipeline below walks 32-key parts of a tile");
    constexpr int NH = kBKV / 32;  // 32-key parts per tile
    constexpr int kOStage = kWaves * 32 * (D * 2 + 16);  // the epilogue's O rows (reuses the ring)
    constexpr int kRing = kStages * (Gm::KT + Gm::VT);
    __shared__ __attribute__((aligned(1024))) unsigned char lds[kRing > kOStage ? kRing : kOStage];
    unsigned char* ldsK = lds;                       // [kStages][kBKV][KROWB], swizzled chunks
    unsigned char* ldsVb = lds + kStages * Gm::KT;   // [kStages][kBKV][VROWB], swizzled chunks

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int hi = lane >> 5;  // lane half
    const int l32 = lane & 31;

    int qb, b, hq;
    block_coords(p, qb, b, hq);
    const int bh = b * p.Hq + hq;
    const int hk = hq / p.G;
    const int T_ = p.T;

    const unsigned char* qp = static_cast<const unsigned char*>(p.q) + (b * p.qs[0] + hq * p.qs[1]) * Gm::QKB;
    // head bases as scalars (the tile loads build scalar resources from them)
    const unsigned char* kp =
        tile_uniform_ptr(static_cast<const unsigned char*>(p.k) + (b * p.ks[0] + hk * p.ks[1]) * Gm::QKB);
    const unsigned char* vp =
        tile_uniform_ptr(static_cast<const unsigned char*>(p.v) + (b * p.vs[0] + hk * p.vs[1]) * (V8 ? 1 : 2));
    T* op = static_cast<T*>(p.o) + b * p.os[0] + hq * p.os[1];
    const int64_t qrs = p.qs[2] * Gm::QKB;  // row strides in bytes
    const int64_t krs = p.ks[2] * Gm::QKB;
    const int64_t vrs = p.vs[2] * (V8 ? 1 : 2);

    const int q_start = qb * kBQ2;
    // Query tile qt of wave w: rows q_start + 32 (slot + kWaves qt) .. +31.
    // Waves w and w + 4 share a SIMD; with 8 waves the second four take the
    // row slots in reverse (7, 6, 5, 4), so each SIMD pairs an early-row
    // wave (idle over more of the block's last, diagonal tiles) with a
    // late-row one and the SIMDs carry equal work.
    int wq0[kQT];
    const int slot = (kWaves == 8 && wave >= 4) ? 11 - wave : wave;
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) wq0[qt] = q_start + 32 * (slot + kWaves * qt);
    const int W = p.window;
    const int n_kv = (T_ + kBKV - 1) / kBKV;
    const int kv_end = min((q_start + kBQ2 + kBKV - 1) / kBKV, n_kv);
    const int kv_begin = W > 0 ? max(0, q_start - W + 1) / kBKV : 0;

    // Loads are unconditional with row indices clamped to T-1: rows past T
    // only ever meet masked (zero) weights, and branch-free loads let the
    // compiler count outstanding memory operations exactly, so the tile
    // prefetch below is not drained early.
    // Q^T as the B operand.  16-bit: chunk dc holds d = 16 dc + 8 hi .. +7.
    // fp8: chunk dc holds d = 64 dc + 32 hi .. +31 (zero past D).
    u32x4 qreg[kQT][Gm::NQC][QK8 ? 2 : 1];
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
        const int qrow = min(wq0[qt] + l32, T_ - 1);
#pragma unroll
        for (int dc = 0; dc < Gm::NQC; ++dc) {
            if constexpr (QK8) {
                const int d0 = 64 * dc + 32 * hi;
#pragma unroll
                for (int w = 0; w < 2; ++w) {
                    // columns past D (D = 32) read the row's first 16 bytes and are zeroed
                    const int col = d0 + 16 * w < D ? d0 + 16 * w : 0;
                    const u32x4 raw = load16(qp + qrow * qrs + col);
                    qreg[qt][dc][w] = d0 + 16 * w < D ? raw : u32x4{0u, 0u, 0u, 0u};
                }
            } else {
                // columns past the head dim (dr < D) read column 0 and are zeroed
                const int d0 = dc * 16 + hi * 8;
                const u32x4 raw = load16(qp + qrow * qrs + (d0 < p.dr ? d0 : 0) * 2);
                qreg[qt][dc][0] = d0 < p.dr ? raw : u32x4{0u, 0u, 0u, 0u};
            }
        }
        if constexpr (ROPE && !QK8) {
            // Rotate-half RoPE in registers: chunk dc (d < D/2) pairs with
            // chunk dc + D/32 (d + D/2) of the same lane; both use the table
            // entries [qrow][d], and the result is rounded to T.
#pragma unroll
            for (int dc = 0; dc < D / 32; ++dc) {
                const int d0 = dc * 16 + hi * 8;
                const float* cr = p.rope_cos + static_cast<int64_t>(qrow) * (D / 2) + d0;
                const float* sr = p.rope_sin + static_cast<int64_t>(qrow) * (D / 2) + d0;
                float cs[8], sn[8];
                *reinterpret_cast<float4*>(cs) = *reinterpret_cast<const float4*>(cr);
                *reinterpret_cast<float4*>(cs + 4) = *reinterpret_cast<const float4*>(cr + 4);
                *reinterpret_cast<float4*>(sn) = *reinterpret_cast<const float4*>(sr);
                *reinterpret_cast<float4*>(sn + 4) = *reinterpret_cast<const float4*>(sr + 4);
                rope_rotate8<T>(qreg[qt][dc][0], qreg[qt][dc + D / 32][0], cs, sn);
            }
        }
    }

    float sc = p.scale;
    float vsc = 1.f;
    if constexpr (QK8) sc *= p.q_scale[0] * p.k_scale[0];
    if constexpr (V8) vsc = p.v_scale[0];

    f32x16 oacc[kQT][D / 32];
    // Four partial row sums per query tile (element v adds to ssum[v & 3])
    // keep the accumulation off one serial dependency chain.
    float ssum[kQT][4];
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) oacc[qt][dt] = f32x16{};
#pragma unroll
        for (int i = 0; i < 4; ++i) ssum[qt][i] = 0.f;
    }

    // Tile j into ring stage buf: K (and 16-bit V) by direct global->LDS
    // loads, fp8 V staged through registers (widened to T in finish_tile).
    // Slot s of a tile is written by wave (s / 64) % kWaves, instruction
    // s / kThreads.
    u32x4 vst[V8 ? Gm::VNL : 1];
    // Per-lane byte offset of the DMA loads inside a tile, fixed for the
    // whole walk.  Load i of a tile covers kKRows (kVRows) rows further down
    // than load i - 1 with the same chunk swizzle (where a lane has several
    // loads, the swizzle reads only row bits that i does not change), so
    // one offset serves every load; load i gets its own scalar resource
    // starting i * kKRows rows into the tile, sized to the rows before T, so
    // rows past T read as zeros (they only meet masked weights).  Lanes
    // whose logical chunk lies past the head dim dr take kPastTile (zeros).
    constexpr int kKRows = kThreads / Gm::KCPR, kVRows = kThreads / Gm::VCPRL;
    static_assert(Gm::KNI == 1 || (kThreads % Gm::KCPR == 0 && (kKRows / Gm::KRPW) % Gm::KCPR == 0),
                  "K loads of a lane must share one swizzled offset");
    static_assert(V8 || Gm::VNI == 1 || (kThreads % Gm::VCPRL == 0 && (kVRows / Gm::VRPW) % (Gm::VCPRL / 4) == 0),
                  "V loads of a lane must share one swizzled offset");
    int koff, voff;
    {
        const int sl = wave * 64 + lane;
        const int krow = min(sl / Gm::KCPR, kBKV - 1);
        const int kch = (sl - krow * Gm::KCPR) ^ Gm::swz_k(krow);
        koff = kch * (16 / Gm::QKB) < p.dr ? krow * static_cast<int>(krs) + kch * 16 : kPastTile;
        const int vrow = min(sl / Gm::VCPRL, kBKV - 1);
        const int vch = (sl - vrow * Gm::VCPRL) ^ Gm::swz_v(vrow);
        voff = vch * 8 < p.dr ? vrow * static_cast<int>(vrs) + vch * 16 : kPastTile;
    }
    auto issue_tile = [&](int j, int buf) {
        const int k0 = j * kBKV;
        const int nrows = min(T_ - k0, kBKV);  // rows of this tile before T
        const int kbytes = nrows * static_cast<int>(krs);
#pragma unroll
        for (int i = 0; i < Gm::KNI; ++i) {
            const int sbase = (i * kWaves + wave) * 64;
            if ((kBKV * Gm::KCPR) % kThreads == 0 || sbase < kBKV * Gm::KCPR) {
                const int skip = i * kKRows * static_cast<int>(krs);
                tile_dma16(tile_rsrc(kp + static_cast<int64_t>(k0) * krs + skip, max(kbytes - skip, 0)), koff,
                      ldsK + buf * Gm::KT + sbase * 16);
            }
        }
        if constexpr (!V8) {
            const int vbytes = nrows * static_cast<int>(vrs);
#pragma unroll
            for (int i = 0; i < Gm::VNI; ++i) {
                const int sbase = (i * kWaves + wave) * 64;
                if ((kBKV * Gm::VCPRL) % kThreads == 0 || sbase < kBKV * Gm::VCPRL) {
                    const int skip = i * kVRows * static_cast<int>(vrs);
                    tile_dma16(tile_rsrc(vp + static_cast<int64_t>(k0) * vrs + skip, max(vbytes - skip, 0)), voff,
                          ldsVb + buf * Gm::VT + sbase * 16);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < Gm::VNL; ++i) {
                const int ci = min(tid + kThreads * i, kBKV * Gm::VCPRG - 1);
                const int row = ci / Gm::VCPRG;
                const int c = ci - row * Gm::VCPRG;
                vst[i] = tile_load16(vp + min(k0 + row, T_ - 1) * vrs + c * 16);
            }
        }
    };
    auto finish_tile = [&](int buf) {
        if constexpr (V8) {
#pragma unroll
            for (int i = 0; i < Gm::VNL; ++i) {
                const int ci = tid + kThreads * i;
                const int row = ci / Gm::VCPRG;
                const int c = ci - row * Gm::VCPRG;
                if ((kBKV * Gm::VCPRG) % kThreads == 0 || ci < kBKV * Gm::VCPRG) {
                    // 16 fp8 values = LDS chunks 2c, 2c + 1 (swz_v is even, so they stay adjacent)
                    unsigned char* dst = ldsVb + buf * Gm::VT + row * Gm::VROWB + ((2 * c) ^ Gm::swz_v(row)) * 16;
                    u32x4 lo, hi16;
                    widen_e4m3x16<T>(vst[i], lo, hi16);
                    *reinterpret_cast<u32x4*>(dst) = lo;
                    *reinterpret_cast<u32x4*>(dst + 16) = hi16;
                }
            }
        }
    };

    // Byte offsets (within a 16-key chunk of the V tile) of this lane's
    // transposing reads, one per 32-column block dt: row (lane>>5)*4 +
    // ((lane&15)>>2), columns dt*32 + ((lane>>4)&1)*16 + 4*(lane&3).
    int v_tr_off[D / 32];
    {
        const int vr = (lane >> 5) * 4 + ((lane & 15) >> 2);
        const int vsw = Gm::swz_v(vr);
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
            const int chunk = (dt * 4 + ((lane >> 4) & 1) * 2 + ((lane & 3) >> 1)) ^ vsw;
            v_tr_off[dt] = vr * Gm::VROWB + chunk * 16 + (lane & 1) * 8;
        }
    }
    // K A-operand chunk swizzle of this lane's rows (kt * 32 + l32; the same for every kt).
    const int kswz = Gm::swz_k(l32);
    const unsigned weff = W > 0 ? static_cast<unsigned>(W) : 0x7FFFFFFFu;

    // K fragments (A operands) of the S^T MFMAs of 32-key half kt.
    auto load_k = [&](const unsigned char* Kb, int kt, KFrag (&kf)[Gm::NQC]) {
        const unsigned char* krow = Kb + (kt * 32 + l32) * Gm::KROWB;
#pragma unroll
        for (int dc = 0; dc < Gm::NQC; ++dc) {
            if constexpr (QK8) {
                const int d0 = 64 * dc + 32 * hi;
                u32x4 a0 = u32x4{0u, 0u, 0u, 0u}, a1 = u32x4{0u, 0u, 0u, 0u};
                if (d0 < D) {
                    a0 = *reinterpret_cast<const u32x4*>(krow + ((d0 / 16) ^ kswz) * 16);
                    a1 = *reinterpret_cast<const u32x4*>(krow + ((d0 / 16 + 1) ^ kswz) * 16);
                }
                kf[dc] = i32x8{(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
            } else {
                kf[dc] = as_vec8<Vec>(*reinterpret_cast<const u32x4*>(krow + ((dc * 2 + hi) ^ kswz) * 16));
            }
        }
    };
    // S^T (32 keys x 32 queries) of one half for every query tile; each K
    // fragment feeds one MFMA per query tile.
    struct STiles {
        f32x16 v[kQT];
    };
    // FOLD: every S^T chain starts from c0 = -1/(2 fs) instead of 0, so the
    // accumulator holds s' = s - 1/(2 fs) and a = fs s'.  Then
    // (a + sqrt(a^2 + 1))^2 = fs^2 (s' + sqrt(s'^2 + 1/fs^2))^2: the weights
    // are computed scaled by 1/fs^2 (one FMA per score fewer), which cancels
    // between P V and the row sum (rescaled at the end).  16-bit Q/K: fs = sc
    // (the host folds only moderate positive scales).  fp8 Q/K: the MFMA
    // block scales apply 2^k of sc = fs 2^k exactly (k split over the two
    // E8M0 exponents, each within +-127), leaving fs in [1, 2) for any
    // positive sc.
    float fs = sc;
    int e8a = 127, e8b = 127;
    if constexpr (QK8 && FOLD) {
        if (sc > 0.f) {
            int e;
            fs = 2.f * frexpf(sc, &e);  // sc = fs 2^(e-1)
            const int k = e - 1;
            const int ka = max(-127, min(127, k));
            e8a = 127 + ka;
            e8b = 127 + (k - ka);
        } else {
            // q_scale k_scale scale underflowed to 0: scores 2^-254 s (zero
            // for every e4m3 product), a = -1/2, as sc s - 1/2 gives
            fs = 1.f;
            e8a = 0;
            e8b = 0;
        }
    }
    const float c0 = -0.5f / fs, c2 = 1.f / (fs * fs);
    f32x16 sinit;
#pragma unroll
    for (int v = 0; v < 16; ++v) sinit[v] = FOLD ? c0 : 0.f;
    auto s_tile = [&](const KFrag (&kf)[Gm::NQC]) {
        STiles s;
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) s.v[qt] = FOLD ? sinit : f32x16{};
#pragma unroll
        for (int dc = 0; dc < Gm::NQC; ++dc) {
#pragma unroll
            for (int qt = 0; qt < kQT; ++qt) {
                if constexpr (QK8) {
                    const i32x8 bv{(int)qreg[qt][dc][0].x, (int)qreg[qt][dc][0].y, (int)qreg[qt][dc][0].z,
                                   (int)qreg[qt][dc][0].w, (int)qreg[qt][dc][1].x, (int)qreg[qt][dc][1].y,
                                   (int)qreg[qt][dc][1].z, (int)qreg[qt][dc][1].w};
                    s.v[qt] = mma_fp8(kf[dc], bv, s.v[qt], e8a, e8b);
                } else {
                    s.v[qt] = Ops::mma(kf[dc], as_vec8<Vec>(qreg[qt][dc][0]), s.v[qt]);
                }
            }
        }
        return s;
    };
    // Squareplus weights of one half, added to the row sums and rounded to
    // T as the two B operands (16-key chunks) of O^T += V^T P^T.  MASK: keep
    // key (k0 + kt*32 + cv) iff 0 <= q - key < W_eff (W_eff = W, or INT_MAX
    // for full causal), one unsigned compare per element.
    auto weights = [&](auto mask_tag, const f32x16& s, int qt, int k0, int kt, Vec (&bop)[2]) {
        constexpr bool MASK = decltype(mask_tag)::value;
        const int dbase = wq0[qt] + l32 - k0 - hi * 4 - kt * 32;
        float y[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            float w;
            if constexpr (FOLD) {
                const float wf = s[v] + fast_sqrt(__builtin_fmaf(s[v], s[v], c2));
                w = wf * wf;
            } else {
                w = sp2_weight<EXACT>(__builtin_fmaf(s[v], sc, -0.5f));
            }
            if constexpr (MASK) {
                const int cv = (v >> 2) * 8 + (v & 3);
                w = keep_if(static_cast<unsigned>(dbase - cv) < weff, w);
            }
            y[v] = w;
            ssum[qt][v & 3] += w;
        }
#pragma unroll
        for (int ch = 0; ch < 2; ++ch) {
            u32x4 pw;
            pw.x = pack2<T>(y[8 * ch + 0], y[8 * ch + 1]);
            pw.y = pack2<T>(y[8 * ch + 2], y[8 * ch + 3]);
            pw.z = pack2<T>(y[8 * ch + 4], y[8 * ch + 5]);
            pw.w = pack2<T>(y[8 * ch + 6], y[8 * ch + 7]);
            bop[ch] = as_vec8<Vec>(pw);
        }
    };
    // O^T += V^T P^T for the two 16-key chunks of half kt; each V^T
    // fragment feeds one MFMA per query tile.
    auto pv = [&](const unsigned char* Vb, int kt, const Vec (&bop)[kQT][2]) {
#pragma unroll
        for (int ch = 0; ch < 2; ++ch) {
            const int c = 2 * kt + ch;  // 16-key chunk of the tile
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) {
                const unsigned char* base = Vb + (16 * c) * Gm::VROWB + v_tr_off[dt];
                const Vec aw = lds_read_tr16_pair<Vec>(base, base + 8 * Gm::VROWB);
#pragma unroll
                for (int qt = 0; qt < kQT; ++qt) oacc[qt][dt] = Ops::mma(aw, bop[qt][ch], oacc[qt][dt]);
            }
        }
    };

    auto stage_of = [&](int t) { return (t - kv_begin) % kStages; };
    // S^T of 32-key half h of tile t.
    auto s_half = [&](int t, int h) {
        KFrag kf[Gm::NQC];
        load_k(ldsK + stage_of(t) * Gm::KT, h, kf);
        return s_tile(kf);
    };
    // Barrier B(t+1): tile t+1 has landed (this wave's loads, then every
    // wave's) and is published; then tile t+2 is requested into the stage of
    // tile t-1, which every wave finished reading before B(t+1).  Every wave
    // calls this exactly once per tile of the block, active or not.
    auto boundary = [&](int t) {
        if (t + 1 < kv_end) {
            tile_wait_vmem();
            finish_tile(stage_of(t + 1));
            __syncthreads();
            if (t + 2 < kv_end) issue_tile(t + 2, stage_of(t + 2));
        }
    };
    // Tile t of the wave with s_cur = S^T of its first 32-key part: for each
    // part h, S^T of part h+1 is issued before the weights and P V of part
    // h; before the last part comes B(t+1), then S^T of the first part of
    // tile t+1 (NEXT), so s_cur holds it on exit.
    auto active_tile = [&](auto mask_tag, auto next_tag, int t, STiles& s_cur) {
        constexpr bool NEXT = decltype(next_tag)::value;
        const int k0 = t * kBKV;
        const unsigned char* Vb = ldsVb + stage_of(t) * Gm::VT;
        Vec bop[kQT][2];
#pragma unroll
        for (int h = 0; h + 1 < NH; ++h) {
            const STiles s_nx = s_half(t, h + 1);
#pragma unroll
            for (int qt = 0; qt < kQT; ++qt) weights(mask_tag, s_cur.v[qt], qt, k0, h, bop[qt]);
            pv(Vb, h, bop);
            s_cur = s_nx;
        }
        const STiles s_last = s_cur;
        boundary(t);
        if constexpr (NEXT) s_cur = s_half(t + 1, 0);
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) weights(mask_tag, s_last.v[qt], qt, k0, NH - 1, bop[qt]);
        pv(Vb, NH - 1, bop);
    };

    // Prologue: tile kv_begin staged and published, tile kv_begin + 1 in
    // flight.  kv_begin < kv_end for every block (q_start < T).
    issue_tile(kv_begin, 0);
    tile_wait_vmem();
    finish_tile(0);
    __syncthreads();
    if (kv_begin + 1 < kv_end) issue_tile(kv_begin + 1, 1);

    // The wave's tiles: [t_first, t_last] see some key (before t_first only
    // the window has passed, after t_last only keys past the wave's last
    // row); inside, [ja, jb) need no masks (every row sees every key: jb
    // ends at the wave's first row, ja starts past the window edge of its
    // last row).  Separate loops per kind keep the accumulators in fixed
    // registers.  Waves whose rows all lie past T only keep the barriers.
    // With two query tiles, the span runs from the first tile's first row
    // (wf) to the last tile's last row (wl).
    const int wf = wq0[0], wl = wq0[kQT - 1] + 31;
    int t_first = kv_begin;
    if (W > 0 && wf - W + 1 > 0) t_first = max(t_first, (wf - W + 1) / kBKV);
    const int t_last = wf < T_ ? min(wl / kBKV, kv_end - 1) : t_first - 1;
    int ja = t_first;
    if (W > 0 && wl - W >= 0) ja = max(ja, (wl - W) / kBKV + 1);
    const int jb = (wf + 1) / kBKV;
    int t = kv_begin;
    for (; t < t_first; ++t) boundary(t);
    if (t_first <= t_last) {
        using Y = std::true_type;
        using N = std::false_type;
        STiles s_cur = s_half(t_first, 0);
        for (; t < min(ja, t_last); ++t) active_tile(Y{}, Y{}, t, s_cur);
        for (; t < min(jb, t_last); ++t) active_tile(N{}, Y{}, t, s_cur);
        for (; t < t_last; ++t) active_tile(Y{}, Y{}, t, s_cur);
        // t == t_last: it holds the wave's diagonal (or window edge) unless
        // the interior reaches it.
        if (t >= ja && t < jb)
            active_tile(N{}, N{}, t, s_cur);
        else
            active_tile(Y{}, N{}, t, s_cur);
        ++t;
    }
    for (; t < kv_end; ++t) boundary(t);

    // O goes out through LDS: a lane's accumulators hold 4 columns of one
    // query row, so direct stores write 8 bytes per lane and row, while the
    // staged rows leave in 16-byte chunks, consecutive lanes along a row, so
    // that each store instruction writes whole rows.  Those stores are
    // nontemporal: O is not read again here, and its lines no longer push the
    // K / V tiles the other blocks of the head still read out of L2 (fp8
    // config 4: 167 -> 113 MiB fetched per launch, the algorithmic 112 MiB).
    __syncthreads();  // every wave is past its last tile: the K/V ring is free
    constexpr int OROWB = D * 2 + 16;  // padded LDS row of one query row of O (bytes)
    constexpr int OCPR = D * 2 / 16;   // 16-byte chunks per O row
    constexpr int ORPI = 64 / OCPR;    // rows per store instruction
    unsigned char* ost = lds + wave * (32 * OROWB);
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
        // Row sums: lanes l and l^32 hold the two key halves of one query column.
        const float part = (ssum[qt][0] + ssum[qt][1]) + (ssum[qt][2] + ssum[qt][3]);
        const float both = part + __shfl_xor(part, 32);
        // FOLD: the sums and P V carry the factor 1/fs^2
        const float stot = FOLD ? __builtin_fmaf(both, fs * fs, kEps) : both + kEps;
        const float inv = FOLD ? vsc * (fs * fs) / stot : vsc / stot;
        const int qi = wq0[qt] + l32;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
            for (int vg = 0; vg < 4; ++vg) {
                const int d0 = dt * 32 + vg * 8 + hi * 4;
                uint2 w;
                w.x = pack2<T>(oacc[qt][dt][vg * 4 + 0] * inv, oacc[qt][dt][vg * 4 + 1] * inv);
                w.y = pack2<T>(oacc[qt][dt][vg * 4 + 2] * inv, oacc[qt][dt][vg * 4 + 3] * inv);
                *reinterpret_cast<uint2*>(ost + l32 * OROWB + d0 * 2) = w;
            }
        }
        if (qi < T_ && hi == 0 && p.row_sums != nullptr) p.row_sums[static_cast<int64_t>(bh) * T_ + qi] = stot;
        // (a wave's LDS accesses complete in order: the reads below see its writes)
#pragma unroll
        for (int r0 = 0; r0 < 32; r0 += ORPI) {
            const int r = r0 + lane / OCPR, c = lane % OCPR;
            const int qr = wq0[qt] + r;
            const u32x4 v = *reinterpret_cast<const u32x4*>(ost + r * OROWB + c * 16);
            if (qr < T_ && c * 8 < p.dr) __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(op + qr * p.os[2] + c * 8));
        }
    }
}

// The folded weights (FOLD above) for bf16 P only: fp16 P would overflow
// 65504 sooner by the factor 1/sc^2.  The scale must be positive and
// moderate so that -1/(2 sc), 1/sc^2 and the scaled sums stay well inside
// fp32; the fp8 path's scale is only known on the device and is not folded.
// D = 128 (config 3: 767 -> 752 us) and 16-bit D = 64 ([4,32,4096,64]:
// 377 -> 363 us): the 16 registers holding the chains' start value take
// D = 64 from 154 to 189, which leaves it one 8-wave block per CU as before;
// at D = 32 (108 -> 146) they would halve the resident blocks.
template <typename T, bool QK8, int D>
constexpr bool kCanFold = std::is_same_v<T, bf16> && (D == 128 || (D == 64 && !QK8));

// 16-bit Q/K fold relative to the scale itself; fp8 Q/K fold relative to
// its mantissa (any positive scale: q_scale and k_scale are positive).
template <bool QK8>
bool fold_scale_ok(float scale) {
    if constexpr (QK8) return scale > 0.f && scale <= 3.0e38f;
    return scale >= 0x1p-20f && scale <= 0x1p20f;
}

template <typename T, int D, bool QK8, bool V8>
int launch_flash(const FlashParams& prm, int exact, hipStream_t st) {
    const dim3 grid(static_cast<unsigned>(prm.nqb) * prm.B * prm.Hq);
    const dim3 block(kThreads);
    if (exact) {
        flash_fwd_kernel<T, D, QK8, V8, true, false><<<grid, block, 0, st>>>(prm);
        return status_from_launch();
    }
    if constexpr (kCanFold<T, QK8, D>) {
        if (fold_scale_ok<QK8>(prm.scale)) {
            flash_fwd_kernel<T, D, QK8, V8, false, false, true><<<grid, block, 0, st>>>(prm);
            return status_from_launch();
        }
    }
    flash_fwd_kernel<T, D, QK8, V8, false, false><<<grid, block, 0, st>>>(prm);
    return status_from_launch();
}

// RoPE forward: K rotated into k_rot (contiguous [B, Hkv, T, D]), then the
// forward with Q rotated in registers.
template <typename T, int D>
int launch_rope(FlashParams prm, T* k_rot, hipStream_t st) {
    const int64_t n_pairs = static_cast<int64_t>(prm.B) * prm.Hkv * prm.T * (D / 16);
    const dim3 rgrid(static_cast<unsigned>((n_pairs + 255) / 256));
    rope_rotate_rows<T, D><<<rgrid, 256, 0, st>>>(static_cast<const T*>(prm.k), k_rot, prm.rope_cos, prm.rope_sin,
                                                  prm.Hkv, prm.T, prm.ks[0], prm.ks[1], prm.ks[2], n_pairs);
    int stt = status_from_launch();
    if (stt != 0) return stt;
    prm.k = k_rot;
    prm.ks[0] = static_cast<int64_t>(prm.Hkv) * prm.T * D;
    prm.ks[1] = static_cast<int64_t>(prm.T) * D;
    prm.ks[2] = D;
    prm.ks[3] = 1;
    const dim3 grid(static_cast<unsigned>(prm.nqb) * prm.B * prm.Hq);
    if constexpr (kCanFold<T, false, D>) {
        if (fold_scale_ok<false>(prm.scale)) {
            flash_fwd_kernel<T, D, false, false, false, true, true><<<grid, dim3(kThreads), 0, st>>>(prm);
            return status_from_launch();
        }
    }
    flash_fwd_kernel<T, D, false, false, false, true><<<grid, dim3(kThreads), 0, st>>>(prm);
    return status_from_launch();
}

// Head dims 8..128 (multiples of 8) run on the kernel for the next of 32,
// 64, 128 with the columns past prm.dr masked.
template <typename T, bool QK8, bool V8>
int launch_flash_d(const FlashParams& prm, int exact, hipStream_t st) {
    if (prm.dr <= 32) return launch_flash<T, 32, QK8, V8>(prm, exact, st);
    if (prm.dr <= 64) return launch_flash<T, 64, QK8, V8>(prm, exact, st);
    return launch_flash<T, 128, QK8, V8>(prm, exact, st);
}

// Largest K / V row stride (bytes) the tile loads address with 32-bit offsets.
constexpr int64_t kMaxRowStrideBytes = int64_t(1) << 24;

// (b, h, t) strides must keep every row start 16-byte aligned; d stride 1.
bool strides_ok(const int64_t* s, int elem_bytes) {
    const int64_t a = 16 / elem_bytes;
    return s[3] == 1 && s[0] % a == 0 && s[1] % a == 0 && s[2] % a == 0;
}

int fill_params(FlashParams& prm, const void* q, const void* k, const void* v, void* o, float* row_sums, int B,
                int Hq, int Hkv, int T, int D, const int64_t* q_strides, const int64_t* k_strides,
                const int64_t* v_strides, const int64_t* o_strides, float scale, int window_size, int qk_bytes,
                int v_bytes) {
    if (B < 0 || Hq <= 0 || Hkv <= 0 || T < 0 || Hq % Hkv != 0 || window_size < 0) return SA_ERR_BAD_SHAPE;
    if (!q || !k || !v || !o || !q_strides || !k_strides || !v_strides || !o_strides) return SA_ERR_NULL_POINTER;
    if (D < 8 || D > 128 || D % 8 != 0) return SA_ERR_UNSUPPORTED;
    if (!strides_ok(q_strides, qk_bytes) || !strides_ok(k_strides, qk_bytes) || !strides_ok(v_strides, v_bytes) ||
        !strides_ok(o_strides, 2) || !aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
        return SA_ERR_BAD_STRIDE;
    // K / V tile loads use 32-bit offsets within a tile of kBKV rows.
    if (k_strides[2] * qk_bytes > kMaxRowStrideBytes || v_strides[2] * v_bytes > kMaxRowStrideBytes)
        return SA_ERR_BAD_STRIDE;
    prm.q = q;
    prm.k = k;
    prm.v = v;
    prm.o = o;
    prm.row_sums = row_sums;
    for (int i = 0; i < 4; ++i) {
        prm.qs[i] = q_strides[i];
        prm.ks[i] = k_strides[i];
        prm.vs[i] = v_strides[i];
        prm.os[i] = o_strides[i];
    }
    prm.B = B;
    prm.Hq = Hq;
    prm.Hkv = Hkv;
    prm.T = T;
    prm.G = Hq / Hkv;
    prm.window = window_size;
    prm.nqb = (T + kBQ2 - 1) / kBQ2;
    prm.dr = D;
    prm.scale = scale;
    return 0;
}

}  // namespace
}  // namespace sa

extern "C" int sa_flash_fwd(const void* q, const void* k, const void* v, void* o, float* row_sums, int B, int Hq,
                            int Hkv, int T, int D, const int64_t* q_strides, const int64_t* k_strides,
                            const int64_t* v_strides, const int64_t* o_strides, float scale, int window_size,
                            int exact_math, int dtype, sa_stream_t stream) {
    using namespace sa;
    if (dtype == SA_F32)
        return flash_fwd_f32(q, k, v, o, row_sums, B, Hq, Hkv, T, D, q_strides, k_strides, v_strides, o_strides,
                             scale, window_size, exact_math, reinterpret_cast<hipStream_t>(stream));
    if (dtype != SA_BF16 && dtype != SA_F16) return SA_ERR_BAD_DTYPE;
    if (D > 128)
        return flash_fwd_wide(q, k, v, o, row_sums, B, Hq, Hkv, T, D, q_strides, k_strides, v_strides, o_strides,
                              scale, window_size, exact_math, dtype, reinterpret_cast<hipStream_t>(stream));
    FlashParams prm{};
    const int st = fill_params(prm, q, k, v, o, row_sums, B, Hq, Hkv, T, D, q_strides, k_strides, v_strides,
                               o_strides, scale, window_size, 2, 2);
    if (st != 0) return st;
    if (B == 0 || T == 0) return 0;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int ex = exact_math ? 1 : 0;
    if (dtype == SA_BF16) return launch_flash_d<bf16, false, false>(prm, ex, s);
    return launch_flash_d<f16, false, false>(prm, ex, s);
}

extern "C" int sa_flash_fp8_fwd(const void* q8, const void* k8, const void* v, void* o, float* row_sums,
                                const float* q_scale, const float* k_scale, const float* v_scale, int B, int Hq,
                                int Hkv, int T, int D, const int64_t* q_strides, const int64_t* k_strides,
                                const int64_t* v_strides, const int64_t* o_strides, float attn_scale,
                                int window_size, int v_dtype, sa_stream_t stream) {
    using namespace sa;
    if (v_dtype != SA_FP8_E4M3FN && v_dtype != SA_BF16) return SA_ERR_BAD_DTYPE;
    const bool v8 = v_dtype == SA_FP8_E4M3FN;
    if (!q_scale || !k_scale || (v8 && !v_scale)) return SA_ERR_NULL_POINTER;
    FlashParams prm{};
    const int st = fill_params(prm, q8, k8, v, o, row_sums, B, Hq, Hkv, T, D, q_strides, k_strides, v_strides,
                               o_strides, attn_scale, window_size, 1, v8 ? 1 : 2);
    if (st != 0) return st;
    if (D != 32 && D != 64 && D != 128) return SA_ERR_UNSUPPORTED;  // fp8 kernels: native head dims only
    if (B == 0 || T == 0) return 0;
    prm.q_scale = q_scale;
    prm.k_scale = k_scale;
    prm.v_scale = v_scale;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (v8) return launch_flash_d<bf16, true, true>(prm, 0, s);
    return launch_flash_d<bf16, true, false>(prm, 0, s);
}

extern "C" int sa_rope_rotate(const void* x, void* out, const float* cos_table, const float* sin_table, int B,
                              int H, int T, int D, const int64_t* x_strides, int dtype, sa_stream_t stream) {
    using namespace sa;
    if (dtype != SA_BF16 && dtype != SA_F16 && dtype != SA_F32) return SA_ERR_BAD_DTYPE;
    if (B < 0 || H < 0 || T < 0 || D <= 0 || D % 16 != 0) return SA_ERR_BAD_SHAPE;
    if (!x || !out || !cos_table || !sin_table || !x_strides) return SA_ERR_NULL_POINTER;
    const int64_t* s = x_strides;
    const int64_t q16 = dtype == SA_F32 ? 4 : 8;  // elements per 16 bytes
    if (s[3] != 1 || s[0] % q16 || s[1] % q16 || s[2] % q16 || !aligned16(x) || !aligned16(out) ||
        !aligned16(cos_table) || !aligned16(sin_table))
        return SA_ERR_BAD_STRIDE;
    const int64_t n_pairs = static_cast<int64_t>(B) * H * T * (D / 16);
    if (n_pairs == 0) return 0;
    // one work-item per pair: the dispatch's grid x block count is 32-bit
    if ((n_pairs + 255) / 256 > INT32_MAX) return SA_ERR_BAD_SHAPE;
    const dim3 grid(static_cast<unsigned>((n_pairs + 255) / 256));
    if (!grid_fits(grid, dim3(256))) return SA_ERR_BAD_SHAPE;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (dtype == SA_F32)
        rope_rotate_any<float><<<grid, 256, 0, st>>>(static_cast<const float*>(x), static_cast<float*>(out),
                                                     cos_table, sin_table, H, T, D, s[0], s[1], s[2], n_pairs);
    else if (dtype == SA_BF16)
        rope_rotate_any<bf16><<<grid, 256, 0, st>>>(static_cast<const bf16*>(x), static_cast<bf16*>(out), cos_table,
                                                    sin_table, H, T, D, s[0], s[1], s[2], n_pairs);
    else
        rope_rotate_any<f16><<<grid, 256, 0, st>>>(static_cast<const f16*>(x), static_cast<f16*>(out), cos_table,
                                                   sin_table, H, T, D, s[0], s[1], s[2], n_pairs);
    return status_from_launch();
}

extern "C" int64_t sa_flash_rope_workspace_size(int B, int Hkv, int T, int D) {
    if (B < 0 || Hkv < 0 || T < 0 || D < 0) return -1;
    return static_cast<int64_t>(B) * Hkv * T * D * 2;
}

extern "C" int sa_flash_rope_fwd(const void* q, const void* k, const void* v, const float* cos_table,
                                 const float* sin_table, void* o, float* row_sums, void* k_rot_ws,
                                 int64_t ws_bytes, int B, int Hq, int Hkv, int T, int D,
                                 const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                                 const int64_t* o_strides, float scale, int window_size, int dtype,
                                 sa_stream_t stream) {
    using namespace sa;
    if (dtype != SA_BF16 && dtype != SA_F16) return SA_ERR_BAD_DTYPE;
    if (!cos_table || !sin_table || !k_rot_ws) return SA_ERR_NULL_POINTER;
    FlashParams prm{};
    const int st = fill_params(prm, q, k, v, o, row_sums, B, Hq, Hkv, T, D, q_strides, k_strides, v_strides,
                               o_strides, scale, window_size, 2, 2);
    if (st != 0) return st;
    if (D != 32 && D != 64 && D != 128) return SA_ERR_UNSUPPORTED;  // fused RoPE: native head dims only
    if (B == 0 || T == 0) return 0;
    if (ws_bytes < sa_flash_rope_workspace_size(B, Hkv, T, D)) return SA_ERR_WORKSPACE;
    if (!aligned16(cos_table) || !aligned16(sin_table) || !aligned16(k_rot_ws)) return SA_ERR_BAD_STRIDE;
    prm.rope_cos = cos_table;
    prm.rope_sin = sin_table;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    switch (D) {
        case 32: return dtype == SA_BF16 ? launch_rope<bf16, 32>(prm, static_cast<bf16*>(k_rot_ws), s)
                                         : launch_rope<f16, 32>(prm, static_cast<f16*>(k_rot_ws), s);
        case 64: return dtype == SA_BF16 ? launch_rope<bf16, 64>(prm, static_cast<bf16*>(k_rot_ws), s)
                                         : launch_rope<f16, 64>(prm, static_cast<f16*>(k_rot_ws), s);
        case 128: return dtype == SA_BF16 ? launch_rope<bf16, 128>(prm, static_cast<bf16*>(k_rot_ws), s)
                                          : launch_rope<f16, 128>(prm, static_cast<f16*>(k_rot_ws), s);
        default: return SA_ERR_UNSUPPORTED;
    }
}
