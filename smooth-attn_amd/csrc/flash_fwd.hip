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
// Work decomposition: a block of 4 waves owns 128 query rows of one
// (batch, query head); wave w owns rows [32w, 32w+32).  K and V tiles of 64
// keys go straight from global memory into LDS (global_load_lds, double
// buffered, one barrier per tile; no staging registers): tile j+1 is in
// flight while tile j is computed.  Per wave and tile: S^T = K Q^T on MFMA,
// the squareplus weights on the VALU (masks only on tiles crossing the
// diagonal or the window edge), then O^T += V^T P^T on MFMA.  fp8 V is
// widened to the 16-bit type while it is staged through registers (exact:
// e4m3fn values are representable in bf16) and v_scale is applied once at
// the end.
// Block order: see block_coords (XCD-aware, heaviest query blocks first).
#include <type_traits>

#include "flash_common.hpp"

namespace sa {
namespace {

#ifndef SA_FLASH_BKV
#define SA_FLASH_BKV 64
#endif
#ifndef SA_FLASH_MINB
#define SA_FLASH_MINB 2
#endif
constexpr int kBKV = SA_FLASH_BKV;  // keys per tile (multiple of 32)
#ifndef SA_FLASH_WAVES
#define SA_FLASH_WAVES 4
#endif
constexpr int kWaves = SA_FLASH_WAVES;  // waves per block (each owns 32 query rows per tile)
constexpr int kThreads = 64 * kWaves;

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
    float scale;
};

// T: 16-bit type of P V (and of q/k/v unless fp8).  QK8: q, k are e4m3fn.
// V8: v is e4m3fn.
//
// LDS tiles are unpadded rows of 16-byte chunks, filled by direct
// global->LDS loads (global_load_lds_dwordx4: lane i of a wave writes bytes
// [16 i, 16 i + 16) after the wave's base, so one instruction fills 1 KB of
// consecutive chunks).  Bank conflicts are avoided by storing logical chunk
// c of row r at chunk c ^ swz(r):
//  * K (read as 16-byte A-operand rows, 8 rows per LDS cycle): swz_k spreads
//    8 consecutive rows over the 8 16-byte bank groups of 128 bytes;
//  * V (read by ds_read_b64_tr_b16: per 16 lanes, 4 rows x 32 bytes): swz_v
//    moves the 4 rows' 32-byte pairs to different 32-byte slots.
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
    static __device__ __forceinline__ int swz_k(int r) {
        return KCPR >= 8 ? (r & (KCPR - 1)) : ((r / (8 / KCPR)) & (KCPR - 1));
    }
    static __device__ __forceinline__ int swz_v(int r) { return VCPRL >= 8 ? 2 * (r & 3) : 2 * ((r >> 1) & 1); }
};

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

// One 16-byte global -> LDS load per lane; lds_base must be wave-uniform.
__device__ __forceinline__ void dma16(const void* g, void* lds_base) {
    __builtin_amdgcn_global_load_lds((glb_void_t*)(g), (lds_void_t*)(lds_base), 16, 0, 0);
}

// s_waitcnt vmcnt(0): this wave's direct-to-LDS loads have landed.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

__device__ __forceinline__ f32x16 mma_fp8(i32x8 a, i32x8 b, f32x16 c) {
    // e4m3 x e4m3, unit block scales (E8M0 127 = 2^0)
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

// Widen 16 e4m3fn values (one 16-byte word) to 16 bf16 / f16 values (two words).
template <typename T>
__device__ __forceinline__ void widen_fp8x16(u32x4 in, u32x4& lo, u32x4& hi) {
    uint32_t out[8];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const int word = static_cast<int>(in[w]);
        out[2 * w] = pack2<T>(__builtin_amdgcn_cvt_f32_fp8(word, 0), __builtin_amdgcn_cvt_f32_fp8(word, 1));
        out[2 * w + 1] = pack2<T>(__builtin_amdgcn_cvt_f32_fp8(word, 2), __builtin_amdgcn_cvt_f32_fp8(word, 3));
    }
    lo = u32x4{out[0], out[1], out[2], out[3]};
    hi = u32x4{out[4], out[5], out[6], out[7]};
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

// K/V tile loads: every tile is read by all query blocks of its head, so
// these loads are cached (a nontemporal load would stream past L2).
template <typename T>
__device__ __forceinline__ u32x4 tile_load16(const T* p) {
    return *reinterpret_cast<const u32x4*>(p);
}

// Block -> (query block, batch, query head).  Blocks are dealt to the 8 XCDs
// round-robin by index.  When B*Hkv is a multiple of 8, XCD x gets the KV
// heads u = x, x+8, ... together with all G query heads that read them (so
// each KV head is fetched into one XCD's L2 only), and on every XCD blocks
// run heaviest query block first across its heads (short tail).  Otherwise
// heaviest query block first across all heads.
__device__ __forceinline__ void block_coords(const FlashParams& p, int& qb, int& b, int& hq) {
    const int id = blockIdx.x;
    const int BHk = p.B * p.Hkv;
    if ((BHk & 7) == 0) {
        const int x = id & 7;
        const int j = id >> 3;
        const int nh = (BHk >> 3) * p.G;  // query heads per XCD
        const int step = j / nh;
        const int r = j - step * nh;
        const int kvl = r / p.G;
        const int u = kvl * 8 + x;  // (b, hk)
        b = u / p.Hkv;
        const int hk = u - b * p.Hkv;
        qb = p.nqb - 1 - step;
        hq = hk * p.G + (r - kvl * p.G);
    } else {
        const int BH = p.B * p.Hq;
        qb = p.nqb - 1 - id / BH;
        const int bh = id - (id / BH) * BH;
        b = bh / p.Hq;
        hq = bh - b * p.Hq;
    }
}

#ifndef SA_FLASH_QT
#define SA_FLASH_QT 1
#endif
// Query tiles (32 rows each) per wave.  QT = 1 (the default) keeps a wave
// within 256 VGPRs, so two blocks (8 waves) share each CU and no register
// traffic goes through AGPRs; QT = 2 reuses every K / V^T operand for two
// MFMAs but needs more than 256 registers, and the AGPR copies that the
// compiler then emits cost more than the reuse saves (measured: 987 vs
// 906 us on [4,32,4096,128]).  With QT = 2, wave w owns query tiles w and
// w + 4 of the block, which balances the causal work of the four waves.
constexpr int kQT = SA_FLASH_QT;
constexpr int kBQ2 = 32 * kWaves * kQT;  // query rows per block

template <typename T, int D, bool QK8, bool V8, bool EXACT, bool ROPE>
__global__ __launch_bounds__(kThreads, kQT == 1 ? SA_FLASH_MINB * 4 / kWaves : 1) void flash_fwd_kernel(FlashParams p) {
    using Gm = Geom<T, D, QK8, V8>;
    using Ops = MfmaOps<T>;
    using Vec = typename Ops::vec8;
    __shared__ __attribute__((aligned(1024))) unsigned char lds[2 * (Gm::KT + Gm::VT)];
    unsigned char* ldsK = lds;                 // [2][kBKV][KROWB], swizzled chunks
    unsigned char* ldsVb = lds + 2 * Gm::KT;   // [2][kBKV][VROWB], swizzled chunks

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
    const unsigned char* kp = static_cast<const unsigned char*>(p.k) + (b * p.ks[0] + hk * p.ks[1]) * Gm::QKB;
    const unsigned char* vp =
        static_cast<const unsigned char*>(p.v) + (b * p.vs[0] + hk * p.vs[1]) * (V8 ? 1 : 2);
    T* op = static_cast<T*>(p.o) + b * p.os[0] + hq * p.os[1];
    const int64_t qrs = p.qs[2] * Gm::QKB;  // row strides in bytes
    const int64_t krs = p.ks[2] * Gm::QKB;
    const int64_t vrs = p.vs[2] * (V8 ? 1 : 2);

    const int q_start = qb * kBQ2;
    int wq0[kQT];  // first query row of each of this wave's tiles
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) wq0[qt] = q_start + 32 * (wave + kWaves * qt);
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
                qreg[qt][dc][0] = load16(qp + qrow * qrs + (dc * 16 + hi * 8) * 2);
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
    float ssum[kQT];
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
        ssum[qt] = 0.f;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) oacc[qt][dt] = f32x16{};
    }

    // Tile j into buffer buf: K (and 16-bit V) by direct global->LDS loads,
    // fp8 V staged through registers (widened to T in finish_tile).  Slot s
    // of a tile is written by wave (s / 64) % 4, instruction s / 256.
    u32x4 vst[V8 ? Gm::VNL : 1];
    // Per-lane byte offsets of the DMA loads inside a tile (rows past T are
    // clamped per tile below), so each load is a wave-uniform 64-bit tile
    // base plus a 32-bit lane offset.
    auto issue_tile = [&](int j, int buf) {
        const int k0 = j * kBKV;
        const int rmax = T_ - 1 - k0;  // last valid row of this tile
        const unsigned char* kt_base = kp + static_cast<int64_t>(k0) * krs;
        const unsigned char* vt_base = vp + static_cast<int64_t>(k0) * vrs;
        const int krs32 = static_cast<int>(krs), vrs32 = static_cast<int>(vrs);
#pragma unroll
        for (int i = 0; i < Gm::KNI; ++i) {
            const int sbase = (i * kWaves + wave) * 64;
            if ((kBKV * Gm::KCPR) % kThreads == 0 || sbase < kBKV * Gm::KCPR) {
                const int sl = sbase + lane;
                const int row = sl / Gm::KCPR;
                const int c = (sl - row * Gm::KCPR) ^ Gm::swz_k(row);
                dma16(kt_base + (min(row, rmax) * krs32 + c * 16), ldsK + buf * Gm::KT + sbase * 16);
            }
        }
        if constexpr (!V8) {
#pragma unroll
            for (int i = 0; i < Gm::VNI; ++i) {
                const int sbase = (i * kWaves + wave) * 64;
                if ((kBKV * Gm::VCPRL) % kThreads == 0 || sbase < kBKV * Gm::VCPRL) {
                    const int sl = sbase + lane;
                    const int row = sl / Gm::VCPRL;
                    const int c = (sl - row * Gm::VCPRL) ^ Gm::swz_v(row);
                    dma16(vt_base + (min(row, rmax) * vrs32 + c * 16), ldsVb + buf * Gm::VT + sbase * 16);
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
                    widen_fp8x16<T>(vst[i], lo, hi16);
                    *reinterpret_cast<u32x4*>(dst) = lo;
                    *reinterpret_cast<u32x4*>(dst + 16) = hi16;
                }
            }
        }
    };

    // Per-lane element offset of the transposing V read; see flash_common.hpp.
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

    // One K/V tile for all of this wave's query tiles.  EDGE: some tile of
    // the wave crosses the diagonal or the window edge (per-tile activity
    // and masks are evaluated); otherwise every query tile is fully inside.
    auto tile_step = [&](auto edge_tag, int buf, int k0) {
        constexpr bool EDGE = decltype(edge_tag)::value;
        bool act[kQT], msk[kQT];
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) {
            act[qt] = !EDGE || ((k0 <= wq0[qt] + 31) && !(W > 0 && k0 + kBKV - 1 <= wq0[qt] - W));
            msk[qt] = EDGE && ((k0 + kBKV - 1 > wq0[qt]) || (W > 0 && k0 <= wq0[qt] + 31 - W));
        }
        const unsigned char* Kb = ldsK + buf * Gm::KT;
        const unsigned char* Vb = ldsVb + buf * Gm::VT;
        // One 32-key half at a time: S^T tiles, weights, then the two P V
        // chunks of the half.
#pragma unroll
        for (int kt = 0; kt < kBKV / 32; ++kt) {
            f32x16 s[kQT];
#pragma unroll
            for (int qt = 0; qt < kQT; ++qt) s[qt] = f32x16{};
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
                    const i32x8 av{(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w,
                                   (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
#pragma unroll
                    for (int qt = 0; qt < kQT; ++qt) {
                        if (!act[qt]) continue;
                        const i32x8 bv{(int)qreg[qt][dc][0].x, (int)qreg[qt][dc][0].y, (int)qreg[qt][dc][0].z,
                                       (int)qreg[qt][dc][0].w, (int)qreg[qt][dc][1].x, (int)qreg[qt][dc][1].y,
                                       (int)qreg[qt][dc][1].z, (int)qreg[qt][dc][1].w};
                        s[qt] = mma_fp8(av, bv, s[qt]);
                    }
                } else {
                    const u32x4 a = *reinterpret_cast<const u32x4*>(krow + ((dc * 2 + hi) ^ kswz) * 16);
#pragma unroll
                    for (int qt = 0; qt < kQT; ++qt) {
                        if (!act[qt]) continue;
                        s[qt] = Ops::mma(as_vec8<Vec>(a), as_vec8<Vec>(qreg[qt][dc][0]), s[qt]);
                    }
                }
            }
            Vec bop[kQT][2];
#pragma unroll
            for (int qt = 0; qt < kQT; ++qt) {
                if (!act[qt]) continue;
                // valid(key) <=> 0 <= qi - key < W_eff (W_eff = W, or INT_MAX
                // for full causal): one unsigned compare per element.
                const int dbase = wq0[qt] + l32 - k0 - hi * 4;
                float y[16];
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    float w = sp2_weight<EXACT>(__builtin_fmaf(s[qt][v], sc, -0.5f));
                    if (EDGE && msk[qt]) {
                        const int cv = kt * 32 + (v >> 2) * 8 + (v & 3);
                        w = static_cast<unsigned>(dbase - cv) < weff ? w : 0.f;
                    }
                    y[v] = w;
                    ssum[qt] += w;
                }
#pragma unroll
                for (int ch = 0; ch < 2; ++ch) {
                    u32x4 pw;
                    pw.x = pack2<T>(y[8 * ch + 0], y[8 * ch + 1]);
                    pw.y = pack2<T>(y[8 * ch + 2], y[8 * ch + 3]);
                    pw.z = pack2<T>(y[8 * ch + 4], y[8 * ch + 5]);
                    pw.w = pack2<T>(y[8 * ch + 6], y[8 * ch + 7]);
                    bop[qt][ch] = as_vec8<Vec>(pw);
                }
            }
#pragma unroll
            for (int ch = 0; ch < 2; ++ch) {
                const int c = 2 * kt + ch;  // 16-key chunk of the tile
#pragma unroll
                for (int dt = 0; dt < D / 32; ++dt) {
                    const unsigned char* base = Vb + (16 * c) * Gm::VROWB + v_tr_off[dt];
                    const Vec aw = lds_read_tr16_pair<Vec>(base, base + 8 * Gm::VROWB);
#pragma unroll
                    for (int qt = 0; qt < kQT; ++qt) {
                        if (!act[qt]) continue;
                        oacc[qt][dt] = Ops::mma(aw, bop[qt][ch], oacc[qt][dt]);
                    }
                }
            }
        }
    };

    // kv_begin < kv_end for every block (q_start < T), so the first tile is
    // always staged.
    issue_tile(kv_begin, 0);
    finish_tile(0);
    wait_vmem();
    __syncthreads();

    const int wlast = wq0[kQT - 1];  // the wave's latest query tile
    const int wfirst = wq0[0];
    for (int j = kv_begin; j < kv_end; ++j) {
        const int buf = (j - kv_begin) & 1;
        const bool has_next = j + 1 < kv_end;
        if (has_next) issue_tile(j + 1, buf ^ 1);
        const int k0 = j * kBKV;
        // some query tile of the wave sees this key tile
        const bool any = (k0 <= wlast + 31) && !(W > 0 && k0 + kBKV - 1 <= wfirst - W);
        // every query tile fully sees it (no masks, no inactive tile)
        const bool interior = (k0 + kBKV - 1 <= wfirst) && !(W > 0 && k0 <= wlast + 31 - W);
        if (any) {
            if (interior)
                tile_step(std::false_type{}, buf, k0);
            else
                tile_step(std::true_type{}, buf, k0);
        }
        if (has_next) finish_tile(buf ^ 1);
        wait_vmem();
        __syncthreads();
    }

#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
        // Row sums: lanes l and l^32 hold the two key halves of one query column.
        const float stot = ssum[qt] + __shfl_xor(ssum[qt], 32) + kEps;
        const float inv = vsc / stot;
        const int qi = wq0[qt] + l32;
        if (qi < T_) {
            T* orow = op + qi * p.os[2];
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
                for (int vg = 0; vg < 4; ++vg) {
                    const int d0 = dt * 32 + vg * 8 + hi * 4;
                    uint2 w;
                    w.x = pack2<T>(oacc[qt][dt][vg * 4 + 0] * inv, oacc[qt][dt][vg * 4 + 1] * inv);
                    w.y = pack2<T>(oacc[qt][dt][vg * 4 + 2] * inv, oacc[qt][dt][vg * 4 + 3] * inv);
                    *reinterpret_cast<uint2*>(orow + d0) = w;
                }
            }
            if (hi == 0 && p.row_sums != nullptr) p.row_sums[static_cast<int64_t>(bh) * T_ + qi] = stot;
        }
    }
}

template <typename T, int D, bool QK8, bool V8>
int launch_flash(const FlashParams& prm, int exact, hipStream_t st) {
    const dim3 grid(static_cast<unsigned>(prm.nqb) * prm.B * prm.Hq);
    const dim3 block(kThreads);
    if (exact)
        flash_fwd_kernel<T, D, QK8, V8, true, false><<<grid, block, 0, st>>>(prm);
    else
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
    flash_fwd_kernel<T, D, false, false, false, true><<<grid, dim3(kThreads), 0, st>>>(prm);
    return status_from_launch();
}

template <typename T, bool QK8, bool V8>
int launch_flash_d(const FlashParams& prm, int D, int exact, hipStream_t st) {
    switch (D) {
        case 32: return launch_flash<T, 32, QK8, V8>(prm, exact, st);
        case 64: return launch_flash<T, 64, QK8, V8>(prm, exact, st);
        case 128: return launch_flash<T, 128, QK8, V8>(prm, exact, st);
        default: return SA_ERR_UNSUPPORTED;
    }
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
    if (D != 32 && D != 64 && D != 128) return SA_ERR_UNSUPPORTED;
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
    if (dtype != SA_BF16 && dtype != SA_F16) return SA_ERR_BAD_DTYPE;
    FlashParams prm{};
    const int st = fill_params(prm, q, k, v, o, row_sums, B, Hq, Hkv, T, D, q_strides, k_strides, v_strides,
                               o_strides, scale, window_size, 2, 2);
    if (st != 0) return st;
    if (B == 0 || T == 0) return 0;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int ex = exact_math ? 1 : 0;
    if (dtype == SA_BF16) return launch_flash_d<bf16, false, false>(prm, D, ex, s);
    return launch_flash_d<f16, false, false>(prm, D, ex, s);
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
    if (B == 0 || T == 0) return 0;
    prm.q_scale = q_scale;
    prm.k_scale = k_scale;
    prm.v_scale = v_scale;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (v8) return launch_flash_d<bf16, true, true>(prm, D, 0, s);
    return launch_flash_d<bf16, true, false>(prm, D, 0, s);
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
