// fp32 fused causal squareplus attention, forward and backward, on the fp32
// MFMA of gfx950 (v_mfma_f32_32x32x2_f32: exact fp32 products, fp32 sums).
//
// Same mathematics as the 16-bit kernels (flash_fwd.hip, flash_bwd.hip),
// with P and dS kept in fp32 (the reference keeps P in the input dtype,
// kernels.py:1621, and for fp32 inputs its dots run at Triton's TF32
// default).  Layout of v_mfma_f32_32x32x2_f32 (checked on the device): A
// (32 x 2) lane l holds row l % 32 and k = l / 32; B (2 x 32) lane l holds
// k = l / 32 and column l % 32; C (32 x 32) lane l holds column l % 32 and
// rows 8 (v / 4) + 4 (l / 32) + v % 4, v = 0..15.
//
// Contraction order.  For S^T = K Q^T the k index of MFMA i pairs d = i (k
// = 0) with d = i + D/2 (k = 1), so a lane's D/2 operands of Q (or K) are one
// contiguous half-row.  For products with P or dS as the B operand (O^T +=
// V^T P^T, dQ^T += K^T dS^T, dV^T += dO^T P, dK^T += Q^T dS) MFMA j takes the
// lane's own C element v = j: k = 0 is row 8 (j / 4) + j % 4 and k = 1 that
// row + 4, and the A operand (column d of those rows) is one 4-byte read of
// the row-major tile per MFMA.
//
// Work decomposition: blocks of 4 waves, 32 rows per wave (queries in the
// forward and dQ, keys in dK/dV), tiles of 32 rows staged in LDS, row-major
// [32][D + 4] (V in the forward [32][D + 8]: it is only read by columns);
// the next tile's global loads are in flight while the current one is used.
#include "flash_f32.hpp"
#include "flash_tiles.hpp"

#include <type_traits>

namespace sa {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kFW = 4;             // waves per block
constexpr int kFT = 32;            // rows per staged tile
constexpr int kFRows = 32 * kFW;   // rows a block owns

__device__ __forceinline__ f32x16 mma32(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

struct F32Params {
    const float* q;
    const float* k;
    const float* v;
    const float* o;     // backward input
    const float* dout;  // backward input
    const float* rs;    // backward input: forward row sums [B, Hq, T]
    float* out;         // forward output
    float* row_sums;    // forward output (nullable)
    float* dq;
    float* dk;
    float* dv;
    float* delta;  // [B, Hq, T]
    int64_t qs[4], ks[4], vs[4], os[4], dos[4], dqs[4], dks[4], dvs[4];
    int B, Hq, Hkv, T, G, window;
    int dr;  // head dim of the tensors (<= D, a multiple of 4; columns past it read as zero, are not stored)
    float scale;
};

// One [kFT][D] fp32 tile (rows r0.., clamped to T - 1) held in registers
// between its global loads and its LDS stores.
template <int D>
struct TileRegs {
    static constexpr int PER = kFT * D / 4 / (64 * kFW);  // float4 per thread
    float4 v[PER];
    // PART: the tensors' head dim dr is below D; columns past it load as zeros
    // (the load then reads column 0).
    template <bool PART>
    __device__ __forceinline__ void load(const float* base, int64_t rstride, int r0, int T, int tid, int dr) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int idx = tid + 64 * kFW * i;
            const int r = idx / (D / 4);
            const int c = (idx - r * (D / 4)) * 4;
            const float* rp = base + static_cast<int64_t>(min(r0 + r, T - 1)) * rstride;
            if constexpr (PART) {
                const float4 t = *reinterpret_cast<const float4*>(rp + (c < dr ? c : 0));
                v[i] = c < dr ? t : float4{0.f, 0.f, 0.f, 0.f};
            } else {
                v[i] = *reinterpret_cast<const float4*>(rp + c);
            }
        }
    }
    // row-major [kFT][P]
    template <int P = D + 4>
    __device__ __forceinline__ void store(float* row, int tid) const {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int idx = tid + 64 * kFW * i;
            const int r = idx / (D / 4);
            const int c = (idx - r * (D / 4)) * 4;
            *reinterpret_cast<float4*>(row + r * P + c) = v[i];
        }
    }
};

// y = squareplus(2 s scale - 1)^2 = (a + r)^2 with a = s scale - 1/2,
// r = sqrt(a^2 + 1); rr = 1 / r.
template <bool EXACT>
__device__ __forceinline__ void weight_rr(float s, float sc, float& y, float& rr) {
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

// A lane's half row: x[i] = row[i + hi D/2], i < D/2 (PART: zero past dr).
template <int D, bool PART>
__device__ __forceinline__ void load_half_row(const float* row, int hi, float (&x)[D / 2], int dr) {
#pragma unroll
    for (int i4 = 0; i4 < D / 8; ++i4) {
        const int c = hi * (D / 2) + 4 * i4;
        float4 t;
        if constexpr (PART) {
            t = *reinterpret_cast<const float4*>(row + (c < dr ? c : 0));
            if (c >= dr) t = float4{0.f, 0.f, 0.f, 0.f};
        } else {
            t = *reinterpret_cast<const float4*>(row + c);
        }
        x[4 * i4 + 0] = t.x;
        x[4 * i4 + 1] = t.y;
        x[4 * i4 + 2] = t.z;
        x[4 * i4 + 3] = t.w;
    }
}

// C (32 x 32) += A B^T over D, A rows from a row-major [kFT][D + 4] LDS
// tile (row l32), B rows from a lane's half-row registers.
template <int D>
__device__ __forceinline__ f32x16 mma_rows(const float* lds_rows, int l32, int hi, const float (&b)[D / 2],
                                           f32x16 c) {
    const float* ar = lds_rows + l32 * (D + 4) + hi * (D / 2);
#pragma unroll
    for (int i4 = 0; i4 < D / 8; ++i4) {
        const float4 a = *reinterpret_cast<const float4*>(ar + 4 * i4);
        c = mma32(a.x, b[4 * i4 + 0], c);
        c = mma32(a.y, b[4 * i4 + 1], c);
        c = mma32(a.z, b[4 * i4 + 2], c);
        c = mma32(a.w, b[4 * i4 + 3], c);
    }
    return c;
}

// acc[dt] (rows d = 32 dt + ..) += A^T(d, r) X(r, col) over the tile's 32
// rows r, X the lane's own 16 C-layout values x[v] (row 8 (v / 4) + 4 hi +
// v % 4).  A^T is read from the row-major [kFT][P] tile itself, element (8 m
// + 4 hi + j, 32 dt + l32) for MFMA 4 m + j, one 4-byte read each: the 32
// lanes of a half read consecutive banks, the two halves 4 P floats apart
// (P = D + 8: 32 mod 64, no conflict; P = D + 4, for tiles also read by
// rows: 16 mod 64, two-way on a quarter of the banks).  Reading the tile
// this way replaces a transposed copy, whose scalar stores (16-way bank
// conflicts) stalled every wave between the staging barriers.
template <int D, int P>
__device__ __forceinline__ void mma_cols(const float* lds_rows, int l32, int hi, const float (&x)[16],
                                         f32x16 (&acc)[D / 32]) {
    const float* base = lds_rows + 4 * hi * P + l32;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[dt] = mma32(base[(8 * m + j) * P + 32 * dt], x[4 * m + j], acc[dt]);
        }
    }
}

// Write a lane's C-layout rows of acc (column = its row index of the output,
// d = 32 dt + 8 m + 4 hi .. +3) times f as 16-byte stores (PART: only below dr).
template <int D, bool PART>
__device__ __forceinline__ void store_cols(float* row, int hi, const f32x16 (&acc)[D / 32], float f, int dr) {
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const float4 w{acc[dt][4 * m + 0] * f, acc[dt][4 * m + 1] * f, acc[dt][4 * m + 2] * f,
                           acc[dt][4 * m + 3] * f};
            if (!PART || dt * 32 + 8 * m + 4 * hi < dr) *reinterpret_cast<float4*>(row + dt * 32 + 8 * m + 4 * hi) = w;
        }
    }
}

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
// The 32-row kernels (head dims up to 128) and the 16-row kernels skip the
// tiles that none of a wave's rows sees.  (A 32-row forward at D = 256, one
// wave per SIMD with AGPR accumulators, ran faster without the branch, which
// made the compiler move every accumulator between AGPRs and VGPRs each
// tile: 7.86 vs 7.32 ms on [4,16,4096,256].)
template <int D>
constexpr bool kSkipIdle = D <= 128;

// Every kernel here is held to two waves per SIMD.  Left to itself the
// compiler gives the D = 128 forward 258 registers and one wave (config 3's
// shape in fp32: 7.7 ms vs 5.0 ms), the D = 64 dK/dV kernel 290 registers
// (10.1 vs 8.2 ms for the backward); the D = 128 backward kernels spill at two
// waves and are still faster (21.4 vs 22.0 ms).
// The forward runs the masked loads for every head dim (PART below): at D = 64,
// 128 and 256 that build compiles without the 48-144 B of spills of the
// unmasked one and is as fast or faster (D = 256: 1945 -> 1539 us on
// [4,16,2048,256]; D = 64: 2353 -> 2265 us on [4,32,4096,64]).
template <int D, bool EXACT>
__global__ __launch_bounds__(64 * kFW) __attribute__((amdgpu_waves_per_eu(D > 128 ? 1 : 2, 8))) void flash_fwd_f32_kernel(F32Params p) {
    constexpr bool PART = true;
    __shared__ __attribute__((aligned(16))) float ldsK[kFT * (D + 4)];
    __shared__ __attribute__((aligned(16))) float ldsV[kFT * (D + 8)];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int hi = lane >> 5;
    const int l32 = lane & 31;
    const int T_ = p.T;
    const int nqb = (T_ + kFRows - 1) / kFRows;
    const int per = p.B * p.Hq;
    const int step = blockIdx.x / per;  // heaviest (latest) query blocks first
    const int rest = blockIdx.x - step * per;
    const int qb = nqb - 1 - step;
    const int b = rest / p.Hq;
    const int hq = rest - b * p.Hq;
    const int hk = hq / p.G;
    const float* kp = p.k + b * p.ks[0] + hk * p.ks[1];
    const float* vp = p.v + b * p.vs[0] + hk * p.vs[1];

    const int q0 = qb * kFRows + 32 * wave;
    const int qi = q0 + l32;
    const int qrow = min(qi, T_ - 1);
    float qv[D / 2];
    load_half_row<D, PART>(p.q + b * p.qs[0] + hq * p.qs[1] + qrow * p.qs[2], hi, qv, p.dr);

    f32x16 oacc[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) oacc[dt] = f32x16{};
    float ssum = 0.f;
    const int W = p.window;
    const unsigned weff = W > 0 ? static_cast<unsigned>(W) : 0x7FFFFFFFu;
    const int n_kv = (T_ + kFT - 1) / kFT;
    const int kv_end = min((qb * kFRows + kFRows + kFT - 1) / kFT, n_kv);
    const int kv_begin = W > 0 ? max(0, qb * kFRows - W + 1) / kFT : 0;
    const float sc = p.scale;

    TileRegs<D> kreg, vreg;
    kreg.template load<PART>(kp, p.ks[2], kv_begin * kFT, T_, tid, p.dr);
    vreg.template load<PART>(vp, p.vs[2], kv_begin * kFT, T_, tid, p.dr);
    for (int t = kv_begin; t < kv_end; ++t) {
        __syncthreads();  // every wave is done with tile t - 1
        kreg.store(ldsK, tid);
        vreg.template store<D + 8>(ldsV, tid);
        __syncthreads();
        if (t + 1 < kv_end) {
            kreg.template load<PART>(kp, p.ks[2], (t + 1) * kFT, T_, tid, p.dr);
            vreg.template load<PART>(vp, p.vs[2], (t + 1) * kFT, T_, tid, p.dr);
        }
        const int k0 = t * kFT;
        const bool active = k0 <= q0 + 31 && !(W > 0 && q0 - (k0 + 31) >= W);
        if (kSkipIdle<D> && !active) continue;
        const f32x16 s = mma_rows<D>(ldsK, l32, hi, qv, f32x16{});  // S^T: rows keys, column query
        float pv[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int key = k0 + 8 * (v >> 2) + 4 * hi + (v & 3);
            float y, rr;
            weight_rr<EXACT>(s[v], sc, y, rr);
            y = keep_if(static_cast<unsigned>(qi - key) < weff, y);
            pv[v] = y;
            ssum += y;
        }
        mma_cols<D, D + 8>(ldsV, l32, hi, pv, oacc);  // O^T += V^T P^T
    }

    const float tot = ssum + __shfl_xor(ssum, 32) + kEps;
    if (qi < T_) {
        store_cols<D, PART>(p.out + b * p.os[0] + hq * p.os[1] + qi * p.os[2], hi, oacc, 1.f / tot, p.dr);
        if (hi == 0 && p.row_sums != nullptr) p.row_sums[(static_cast<int64_t>(b) * p.Hq + hq) * T_ + qi] = tot;
    }
}

// ---------------------------------------------------------------------------
// Backward: dQ (and delta)
// ---------------------------------------------------------------------------
template <int D, bool EXACT, bool PART>
__global__ __launch_bounds__(64 * kFW) __attribute__((amdgpu_waves_per_eu(D > 128 ? 1 : 2, 8))) void flash_bwd_dq_f32_kernel(F32Params p) {
    __shared__ __attribute__((aligned(16))) float ldsK[kFT * (D + 4)];
    __shared__ __attribute__((aligned(16))) float ldsV[kFT * (D + 4)];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int hi = lane >> 5;
    const int l32 = lane & 31;
    const int T_ = p.T;
    const int nqb = (T_ + kFRows - 1) / kFRows;
    const int per = p.B * p.Hq;
    const int step = blockIdx.x / per;
    const int rest = blockIdx.x - step * per;
    const int qb = nqb - 1 - step;
    const int b = rest / p.Hq;
    const int hq = rest - b * p.Hq;
    const int hk = hq / p.G;
    const float* kp = p.k + b * p.ks[0] + hk * p.ks[1];
    const float* vp = p.v + b * p.vs[0] + hk * p.vs[1];

    const int q0 = qb * kFRows + 32 * wave;
    const int qi = q0 + l32;
    const int qrow = min(qi, T_ - 1);
    float qv[D / 2], dov[D / 2];
    load_half_row<D, PART>(p.q + b * p.qs[0] + hq * p.qs[1] + qrow * p.qs[2], hi, qv, p.dr);
    load_half_row<D, PART>(p.dout + b * p.dos[0] + hq * p.dos[1] + qrow * p.dos[2], hi, dov, p.dr);
    // delta = rowsum(dO * O) of this lane's query (lanes l and l ^ 32 hold the halves)
    float dpart = 0.f;
    {
        const float* orow = p.o + b * p.os[0] + hq * p.os[1] + qrow * p.os[2] + hi * (D / 2);
#pragma unroll
        for (int i4 = 0; i4 < D / 8; ++i4) {
            // PART: columns past dr read column 0 and are zeroed
            const bool in = !PART || hi * (D / 2) + 4 * i4 < p.dr;
            float4 ov = *reinterpret_cast<const float4*>(orow + (in ? 4 * i4 : -hi * (D / 2)));
            if (!in) ov = float4{0.f, 0.f, 0.f, 0.f};
            dpart = __builtin_fmaf(dov[4 * i4 + 0], ov.x, dpart);
            dpart = __builtin_fmaf(dov[4 * i4 + 1], ov.y, dpart);
            dpart = __builtin_fmaf(dov[4 * i4 + 2], ov.z, dpart);
            dpart = __builtin_fmaf(dov[4 * i4 + 3], ov.w, dpart);
        }
    }
    const float dl = dpart + __shfl_xor(dpart, 32);
    const int64_t rbase = (static_cast<int64_t>(b) * p.Hq + hq) * T_;
    if (qi < T_ && hi == 0) p.delta[rbase + qi] = dl;
    const float inv_r = 1.f / p.rs[rbase + qrow];

    f32x16 acc[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) acc[dt] = f32x16{};
    f32x16 ndl;
#pragma unroll
    for (int v = 0; v < 16; ++v) ndl[v] = -dl;
    const int W = p.window;
    const unsigned weff = W > 0 ? static_cast<unsigned>(W) : 0x7FFFFFFFu;
    const int n_kv = (T_ + kFT - 1) / kFT;
    const int kv_end = min((qb * kFRows + kFRows + kFT - 1) / kFT, n_kv);
    const int kv_begin = W > 0 ? max(0, qb * kFRows - W + 1) / kFT : 0;
    const float sc = p.scale;

    TileRegs<D> kreg, vreg;
    kreg.template load<PART>(kp, p.ks[2], kv_begin * kFT, T_, tid, p.dr);
    vreg.template load<PART>(vp, p.vs[2], kv_begin * kFT, T_, tid, p.dr);
    for (int t = kv_begin; t < kv_end; ++t) {
        __syncthreads();
        kreg.store(ldsK, tid);
        vreg.store(ldsV, tid);
        __syncthreads();
        if (t + 1 < kv_end) {
            kreg.template load<PART>(kp, p.ks[2], (t + 1) * kFT, T_, tid, p.dr);
            vreg.template load<PART>(vp, p.vs[2], (t + 1) * kFT, T_, tid, p.dr);
        }
        const int k0 = t * kFT;
        const bool active = k0 <= q0 + 31 && !(W > 0 && q0 - (k0 + 31) >= W);
        if (kSkipIdle<D> && !active) continue;
        const f32x16 s = mma_rows<D>(ldsK, l32, hi, qv, f32x16{});  // S^T
        const f32x16 dp = mma_rows<D>(ldsV, l32, hi, dov, ndl);     // dP^T - delta
        float ds[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int key = k0 + 8 * (v >> 2) + 4 * hi + (v & 3);
            float y, rr;
            weight_rr<EXACT>(s[v], sc, y, rr);
            ds[v] = keep_if(static_cast<unsigned>(qi - key) < weff, dp[v] * y * rr);
        }
        mma_cols<D, D + 4>(ldsK, l32, hi, ds, acc);  // dQ^T += K^T dS^T
    }
    // dS carried without its per-row factor 2 scale / R
    if (qi < T_) store_cols<D, PART>(p.dq + b * p.dqs[0] + hq * p.dqs[1] + qi * p.dqs[2], hi, acc, 2.f * sc * inv_r, p.dr);
}

// ---------------------------------------------------------------------------
// Backward: dK, dV
// ---------------------------------------------------------------------------
template <int D, bool EXACT, bool PART>
__global__ __launch_bounds__(64 * kFW) __attribute__((amdgpu_waves_per_eu(D > 128 ? 1 : 2, 8))) void flash_bwd_dkdv_f32_kernel(F32Params p) {
    __shared__ __attribute__((aligned(16))) float ldsQ[kFT * (D + 4)];
    __shared__ __attribute__((aligned(16))) float ldsO[kFT * (D + 4)];
    __shared__ __attribute__((aligned(16))) float ldr[2][kFT];  // [1/R, -delta] of the tile's rows
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int hi = lane >> 5;
    const int l32 = lane & 31;
    const int T_ = p.T;
    const int nkb = (T_ + kFRows - 1) / kFRows;
    const int per = p.B * p.Hkv;
    const int kb = blockIdx.x / per;  // earliest key blocks (most queries) first
    const int rest = blockIdx.x - kb * per;
    const int b = rest / p.Hkv;
    const int hk = rest - b * p.Hkv;
    (void)nkb;

    const int k_start = kb * kFRows;
    const int wk0 = k_start + 32 * wave;
    const int kj = wk0 + l32;
    const int krow = min(kj, T_ - 1);
    float kv[D / 2], vv[D / 2];
    load_half_row<D, PART>(p.k + b * p.ks[0] + hk * p.ks[1] + krow * p.ks[2], hi, kv, p.dr);
    load_half_row<D, PART>(p.v + b * p.vs[0] + hk * p.vs[1] + krow * p.vs[2], hi, vv, p.dr);

    f32x16 dkacc[D / 32], dvacc[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
        dkacc[dt] = f32x16{};
        dvacc[dt] = f32x16{};
    }
    const int W = p.window;
    const unsigned weff = W > 0 ? static_cast<unsigned>(W) : 0x7FFFFFFFu;
    const int n_qt = (T_ + kFT - 1) / kFT;
    const int qt_begin = k_start / kFT;
    const int qt_end = W > 0 ? min(n_qt, (k_start + kFRows - 1 + W - 1) / kFT + 1) : n_qt;
    const int nq = qt_end - qt_begin;  // >= 1 (k_start < T)
    const int n_it = p.G * nq;
    const float sc = p.scale;

    TileRegs<D> qreg, oreg;
    float rst = 0.f;
    auto fetch = [&](int it) {
        const int g = it / nq;
        const int q0 = (qt_begin + it - g * nq) * kFT;
        const int hq = hk * p.G + g;
        qreg.template load<PART>(p.q + b * p.qs[0] + hq * p.qs[1], p.qs[2], q0, T_, tid, p.dr);
        oreg.template load<PART>(p.dout + b * p.dos[0] + hq * p.dos[1], p.dos[2], q0, T_, tid, p.dr);
        // raw row sum or delta; 1/R or -delta is formed where it is stored
        if (tid < 2 * kFT) {
            const int64_t idx = (static_cast<int64_t>(b) * p.Hq + hq) * T_ + min(q0 + (tid & (kFT - 1)), T_ - 1);
            rst = (tid < kFT ? p.rs : p.delta)[idx];
        }
    };
    fetch(0);
    for (int it = 0; it < n_it; ++it) {
        __syncthreads();
        qreg.store(ldsQ, tid);
        oreg.store(ldsO, tid);
        if (tid < 2 * kFT) ldr[tid / kFT][tid & (kFT - 1)] = tid < kFT ? 1.f / rst : -rst;
        __syncthreads();
        const int g = it / nq;
        const int q0 = (qt_begin + it - g * nq) * kFT;
        if (it + 1 < n_it) fetch(it + 1);
        // some query of the tile sees some key of the wave
        const bool active = q0 + 31 >= wk0 && !(W > 0 && q0 - (wk0 + 31) >= W) && q0 < T_;
        if (kSkipIdle<D> && !active) continue;
        const f32x16 s = mma_rows<D>(ldsQ, l32, hi, kv, f32x16{});  // S: rows queries, column key
        f32x16 dp;
#pragma unroll
        for (int v = 0; v < 16; ++v) dp[v] = ldr[1][8 * (v >> 2) + 4 * hi + (v & 3)];
        dp = mma_rows<D>(ldsO, l32, hi, vv, dp);  // dP - delta
        float pw[16], ds[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int r = 8 * (v >> 2) + 4 * hi + (v & 3);
            const int q = q0 + r;
            float y, rr;
            weight_rr<EXACT>(s[v], sc, y, rr);
            const float yi = y * ldr[0][r];
            const bool ok = static_cast<unsigned>(q - kj) < weff && q < T_;
            pw[v] = keep_if(ok, yi);
            ds[v] = keep_if(ok, dp[v] * yi * rr);
        }
        mma_cols<D, D + 4>(ldsO, l32, hi, pw, dvacc);  // dV^T += dO^T P
        mma_cols<D, D + 4>(ldsQ, l32, hi, ds, dkacc);  // dK^T += Q^T dS
    }
    if (kj < T_) {
        store_cols<D, PART>(p.dk + b * p.dks[0] + hk * p.dks[1] + kj * p.dks[2], hi, dkacc, 2.f * sc, p.dr);
        store_cols<D, PART>(p.dv + b * p.dvs[0] + hk * p.dvs[1] + kj * p.dvs[2], hi, dvacc, 1.f, p.dr);
    }
}

// fp32 tensors: (b, h, t) strides multiples of 4 elements (16-byte rows), d stride 1.
bool f32_strides_ok(const int64_t* s) { return s[3] == 1 && s[0] % 4 == 0 && s[1] % 4 == 0 && s[2] % 4 == 0; }

int check_common(int B, int Hq, int Hkv, int T, int D, int window_size) {
    if (B < 0 || Hq <= 0 || Hkv <= 0 || T < 0 || Hq % Hkv != 0 || window_size < 0) return SA_ERR_BAD_SHAPE;
    if (D < 4 || D > 512 || D % 4 != 0) return SA_ERR_UNSUPPORTED;
    return 0;
}

// ---------------------------------------------------------------------------
// 16 rows per wave on v_mfma_f32_16x16x4_f32 (the backward from head dim
// 128 up, the forward from 256 up): A (16 x 4): lane l holds row l % 16 and
// k = l / 16; B (4 x 16): k = l / 16, column l % 16; C (16 x 16): column
// l % 16, rows 4 (l / 16) + v.  With 32 rows per wave the D = 128 backward
// held the two operand rows of 32 keys (or queries) as 2 x 64 registers
// plus 2 x 64 accumulators and spilled; 16 rows take half.  The layouts
// mirror the 32-row ones: MFMA i of a D-contraction pairs k-slot g = l / 16
// with d = g D / 4 + i, so a lane's operand is one contiguous quarter row;
// for contractions over a staged tile's 32 rows, MFMA j of 16-row subtile
// st takes the lane's own C element v = j (row 16 st + 4 g + j) as B, and
// its A operand is one 4-byte read of the row-major tile (mma_cols16).
// ---------------------------------------------------------------------------

typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mma16f(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// A lane's quarter row: x[i] = row[g D/4 + i], i < D/4 (PART: zero past dr).
template <int D, bool PART>
__device__ __forceinline__ void load_quarter_row(const float* row, int g, float (&x)[D / 4], int dr) {
#pragma unroll
    for (int i4 = 0; i4 < D / 16; ++i4) {
        const int c = g * (D / 4) + 4 * i4;
        float4 t;
        if constexpr (PART) {
            t = *reinterpret_cast<const float4*>(row + (c < dr ? c : 0));
            if (c >= dr) t = float4{0.f, 0.f, 0.f, 0.f};
        } else {
            t = *reinterpret_cast<const float4*>(row + c);
        }
        x[4 * i4 + 0] = t.x;
        x[4 * i4 + 1] = t.y;
        x[4 * i4 + 2] = t.z;
        x[4 * i4 + 3] = t.w;
    }
}

// C (16 x 16) += A B^T over D: A rows r0 + l16 of a row-major [kFT][D + 4]
// LDS tile, B the lane's quarter-row registers.
template <int D>
__device__ __forceinline__ f32x4 mma_rows16(const float* lds_rows, int r0, int l16, int g, const float (&b)[D / 4],
                                            f32x4 c) {
    const float* ar = lds_rows + (r0 + l16) * (D + 4) + g * (D / 4);
#pragma unroll
    for (int i4 = 0; i4 < D / 16; ++i4) {
        const float4 a = *reinterpret_cast<const float4*>(ar + 4 * i4);
        c = mma16f(a.x, b[4 * i4 + 0], c);
        c = mma16f(a.y, b[4 * i4 + 1], c);
        c = mma16f(a.z, b[4 * i4 + 2], c);
        c = mma16f(a.w, b[4 * i4 + 3], c);
    }
    return c;
}

// acc[dt] (rows d = 16 dt + 4 g + v, column = the lane's row) += A^T(d, r)
// X(r, col) over the tile's 32 rows, X the lane's own C-layout values
// x[st][v] (row 16 st + 4 g + v).  A^T is read from the row-major
// [kFT][D + 4] tile itself: MFMA j of subtile st takes element (16 st + 4 g
// + j, 16 dt + l16), one 4-byte read per MFMA.  Row 4 g lies 4 g (D + 4) =
// 16 g floats (mod 64) from row 0, so a read's 64 lanes hit 64 distinct
// banks, and the tile needs no transposed copy (whose scalar stores, 16-way
// bank conflicts, stalled every wave between the staging barriers).
template <int D>
__device__ __forceinline__ void mma_cols16(const float* lds_rows, int l16, int g, const float (&x)[2][4],
                                           f32x4 (&acc)[D / 16]) {
    const float* base = lds_rows + 4 * g * (D + 4) + l16;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) {
#pragma unroll
        for (int st = 0; st < 2; ++st) {
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[dt] = mma16f(base[(16 * st + j) * (D + 4) + 16 * dt], x[st][j], acc[dt]);
        }
    }
}

// Write a lane's C-layout values of acc (its row of the output, d =
// 16 dt + 4 g .. +3) times f as 16-byte stores (PART: only below dr).
template <int D, bool PART>
__device__ __forceinline__ void store_cols16(float* row, int g, const f32x4 (&acc)[D / 16], float f, int dr) {
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) {
        const float4 w{acc[dt][0] * f, acc[dt][1] * f, acc[dt][2] * f, acc[dt][3] * f};
        if (!PART || dt * 16 + 4 * g < dr) *reinterpret_cast<float4*>(row + dt * 16 + 4 * g) = w;
    }
}

// dQ over one staged 32-key tile (K and V rows in LDS) for the wave's 16
// queries q0 .. q0 + 15 (the lane's query qi); skips tiles none of them sees.
template <int D, bool EXACT>
__device__ __forceinline__ void dq_tile16(const float* ldsK, const float* ldsV, int k0, int q0, int qi, int l16,
                                          int g, const float (&qv)[D / 4], const float (&dov)[D / 4], f32x4 ndl,
                                          float sc, int W, unsigned weff, f32x4 (&acc)[D / 16]) {
    const bool active = k0 <= q0 + 15 && !(W > 0 && q0 - (k0 + 31) >= W);
    if (!active) return;
    float ds[2][4];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
        const f32x4 s = mma_rows16<D>(ldsK, 16 * st, l16, g, qv, f32x4{0.f, 0.f, 0.f, 0.f});  // S^T
        const f32x4 dp = mma_rows16<D>(ldsV, 16 * st, l16, g, dov, ndl);                     // dP^T - delta
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int key = k0 + 16 * st + 4 * g + v;
            float y, rr;
            weight_rr<EXACT>(s[v], sc, y, rr);
            ds[st][v] = keep_if(static_cast<unsigned>(qi - key) < weff, dp[v] * y * rr);
        }
    }
    mma_cols16<D>(ldsK, l16, g, ds, acc);  // dQ^T += K^T dS^T
}


// WHICH: kDkdvBoth (D = 128), or at D = 256, where K, V and both
// accumulators of 16 keys would not leave room for two waves per SIMD, one
// kernel for dV (kDkdvV: K and dV in registers) and one for dK (kDkdvK: K, V
// and dK), each computing S.
constexpr int kDkdvBoth = 0, kDkdvV = 1, kDkdvK = 2;

// dK and/or dV (WHICH) over one staged 32-query tile (Q and dO rows in
// LDS, with its rows' 1/R and -delta in ldr) for the wave's 16 keys wk0 ..
// wk0 + 15 (the lane's key kj); skips tiles none of them sees.
template <int D, bool EXACT, int WHICH, int NV, int NK, int NVA>
__device__ __forceinline__ void kv_tile16(const float* ldsQ, const float* ldsO, const float (&ldr)[2][kFT], int q0,
                                          int wk0, int kj, int T_, int l16, int g, const float (&kv)[D / 4],
                                          const float (&vv)[NV], float sc, int W, unsigned weff,
                                          f32x4 (&dkacc)[NK], f32x4 (&dvacc)[NVA]) {
    constexpr bool DO_V = WHICH != kDkdvK, DO_K = WHICH != kDkdvV;
    // some query of the tile sees some key of the wave
    const bool active = q0 + 31 >= wk0 && !(W > 0 && q0 - (wk0 + 15) >= W) && q0 < T_;
    if (!active) return;
    float pw[2][4], ds[2][4];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
        const f32x4 s = mma_rows16<D>(ldsQ, 16 * st, l16, g, kv, f32x4{0.f, 0.f, 0.f, 0.f});  // S: rows queries
        f32x4 dp;
        if constexpr (DO_K) {
#pragma unroll
            for (int v = 0; v < 4; ++v) dp[v] = ldr[1][16 * st + 4 * g + v];
            dp = mma_rows16<D>(ldsO, 16 * st, l16, g, vv, dp);  // dP - delta
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int r = 16 * st + 4 * g + v;
            const int q = q0 + r;
            float y, rr;
            weight_rr<EXACT>(s[v], sc, y, rr);
            const float yi = y * ldr[0][r];
            const bool ok = static_cast<unsigned>(q - kj) < weff && q < T_;
            pw[st][v] = keep_if(ok, yi);
            if constexpr (DO_K) ds[st][v] = keep_if(ok, dp[v] * yi * rr);
        }
    }
    if constexpr (DO_V) mma_cols16<D>(ldsO, l16, g, pw, dvacc);  // dV^T += dO^T P
    if constexpr (DO_K) mma_cols16<D>(ldsQ, l16, g, ds, dkacc);  // dK^T += Q^T dS
}


// ---------------------------------------------------------------------------
// The 16-row kernels take each 32-row tile straight from global memory
// into LDS (direct-to-LDS buffer loads), so no registers stage it (staged
// through registers, the D = 256 dQ and dK kernels spilled; at D = 512 a
// tile takes 64 KB).  D = 64 to 256: blocks of 8 waves (two per SIMD, four
// at D = 64) and two LDS stages (the next tile loads while the current one
// is used; 2 x 33.8 / 66.5 KB at D = 128 / 256); D = 512: blocks of 4 waves (one per SIMD, 512 registers
// with the AGPRs) and one stage (132 KB: the tile's loads wait).  The
// backward runs them from D = 64 up, the forward from D = 256 up (below
// that the 32-row kernels are as fast or faster).
// ---------------------------------------------------------------------------
template <int D>
struct R16Dma {
    static constexpr int NW = D > 256 ? 4 : 8;      // waves per block
    static constexpr int ROWS = 16 * NW;            // rows a block owns
    static constexpr int STAGES = D > 256 ? 1 : 2;  // LDS stages
    static constexpr int TILE = kFT * (D + 4);      // floats of one staged [kFT][D + 4] tile
    // waves per SIMD allowed: at D = 64 the registers and LDS of four fit
    // (the backward 8.04 -> 7.54-7.73 ms on [4,32,4096,64] against two)
    static constexpr int MAX_WAVES = D <= 64 ? 4 : NW / 4;
};

// Rows r0 .. r0 + kFT - 1 of a [T][D] fp32 tensor (rows rs floats apart,
// base wave-uniform) into an LDS tile of rows D + 4 floats apart.  One
// buffer -> LDS instruction moves up to 1 KB (64 lanes x 16 bytes): a row
// at D <= 256 (below 256 with D / 4 lanes), half of one at 512; wave w
// issues instructions w, w + NW, ...
// Rows at or past T and columns at or past dr (a multiple of 4) read zeros:
// the instruction's buffer resource ends before them.
template <int D, int NW>
__device__ __forceinline__ void dma_tile_f32(const float* base, int64_t rs, int r0, int T, int dr, float* lds,
                                             int wave, int lane) {
    if constexpr (D < 256) {
        // one row per instruction, its first D / 4 lanes active (the LDS rows
        // are D + 4 floats apart, so two rows are not one contiguous 1 KB)
#pragma unroll
        for (int i = 0; i < kFT / NW; ++i) {
            const int r = i * NW + wave;
            const int row = r0 + r;
            const unsigned char* src = tile_uniform_ptr(reinterpret_cast<const unsigned char*>(
                base + static_cast<int64_t>(min(row, T - 1)) * rs));
            if (lane < D / 4) tile_dma16(tile_rsrc(src, row < T ? 4 * min(dr, D) : 0), 16 * lane, lds + r * (D + 4));
        }
        return;
    }
    constexpr int IPR = D / 256 > 0 ? D / 256 : 1;  // instructions per row
    static_assert(kFT * IPR % NW == 0, "whole instructions per wave");
#pragma unroll
    for (int i = 0; i < kFT * IPR / NW; ++i) {
        const int j = i * NW + wave;
        const int r = j / IPR, part = j - r * IPR;
        const int row = r0 + r;
        const int cols = min(max(dr - 256 * part, 0), 256);
        const unsigned char* src = tile_uniform_ptr(reinterpret_cast<const unsigned char*>(
            base + static_cast<int64_t>(min(row, T - 1)) * rs + 256 * part));
        tile_dma16(tile_rsrc(src, row < T ? 4 * cols : 0), 16 * lane, lds + r * (D + 4) + 256 * part);
    }
}

template <int D, bool EXACT, bool PART>
__global__ __launch_bounds__(64 * R16Dma<D>::NW) __attribute__((amdgpu_waves_per_eu(R16Dma<D>::NW / 4, R16Dma<D>::MAX_WAVES)))
void flash_fwd_f32dma_kernel(F32Params p) {
    using C = R16Dma<D>;
    // stage arrays [K][V]; two arrays so that a tile's LDS reads never wait
    // for the direct-to-LDS loads filling the other stage
    __shared__ __attribute__((aligned(16))) float lds0[2 * C::TILE];
    __shared__ __attribute__((aligned(16))) float lds1[C::STAGES > 1 ? 2 * C::TILE : 4];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4;
    const int l16 = lane & 15;
    const int T_ = p.T;
    const int nqb = (T_ + C::ROWS - 1) / C::ROWS;
    const int per = p.B * p.Hq;
    const int step = blockIdx.x / per;  // heaviest (latest) query blocks first
    const int rest = blockIdx.x - step * per;
    const int qb = nqb - 1 - step;
    const int b = rest / p.Hq;
    const int hq = rest - b * p.Hq;
    const int hk = hq / p.G;
    const float* kp = p.k + b * p.ks[0] + hk * p.ks[1];
    const float* vp = p.v + b * p.vs[0] + hk * p.vs[1];

    const int q0 = qb * C::ROWS + 16 * wave;
    const int qi = q0 + l16;
    const int qrow = min(qi, T_ - 1);
    float qv[D / 4];
    load_quarter_row<D, PART>(p.q + b * p.qs[0] + hq * p.qs[1] + qrow * p.qs[2], g, qv, p.dr);
    f32x4 oacc[D / 16];
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) oacc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float ssum = 0.f;
    const int W = p.window;
    const unsigned weff = W > 0 ? static_cast<unsigned>(W) : 0x7FFFFFFFu;
    const int n_kv = (T_ + kFT - 1) / kFT;
    const int kv_end = min((qb * C::ROWS + C::ROWS + kFT - 1) / kFT, n_kv);
    const int kv_begin = W > 0 ? max(0, qb * C::ROWS - W + 1) / kFT : 0;
    const float sc = p.scale;
    auto stage = [&](auto st) -> float* {
        if constexpr (decltype(st)::value == 0) return lds0;
        else return lds1;
    };
    auto issue = [&](int t, auto st) {
        float* l = stage(st);
        dma_tile_f32<D, C::NW>(kp, p.ks[2], t * kFT, T_, p.dr, l, wave, lane);
        dma_tile_f32<D, C::NW>(vp, p.vs[2], t * kFT, T_, p.dr, l + C::TILE, wave, lane);
    };
    auto compute = [&](int t, auto st) {
        const float* l = stage(st);
        const int k0 = t * kFT;
        if (!(k0 <= q0 + 15 && !(W > 0 && q0 - (k0 + 31) >= W))) return;
        float pw[2][4];
#pragma unroll
        for (int st16 = 0; st16 < 2; ++st16) {
            // S^T: lane's column = query qi, rows = keys k0 + 16 st16 + 4 g + v
            const f32x4 s = mma_rows16<D>(l, 16 * st16, l16, g, qv, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int key = k0 + 16 * st16 + 4 * g + v;
                float y, rr;
                weight_rr<EXACT>(s[v], sc, y, rr);
                y = keep_if(static_cast<unsigned>(qi - key) < weff, y);
                pw[st16][v] = y;
                ssum += y;
            }
        }
        mma_cols16<D>(l + C::TILE, l16, g, pw, oacc);  // O^T += V^T P^T
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    if constexpr (C::STAGES == 2) {
        issue(kv_begin, S0{});
        tile_wait_vmem();
        __syncthreads();
        // tile t reads stage (t - kv_begin) & 1 while the other fills with t + 1
        auto run = [&](int t, auto cur) {
            if (t + 1 < kv_end) issue(t + 1, std::integral_constant<int, 1 - decltype(cur)::value>{});
            compute(t, cur);
            if (t + 1 < kv_end) {
                tile_wait_vmem();
                __syncthreads();
            }
        };
        for (int t = kv_begin; t < kv_end; t += 2) {
            run(t, S0{});
            if (t + 1 < kv_end) run(t + 1, S1{});
        }
    } else {
        for (int t = kv_begin; t < kv_end; ++t) {
            if (t > kv_begin) __syncthreads();  // every wave is done with tile t - 1
            issue(t, S0{});
            tile_wait_vmem();
            __syncthreads();
            compute(t, S0{});
        }
    }
    // the query's row sum: its keys lie in lanes l16 + 16 g
    const float sh = ssum + __shfl_xor(ssum, 16);
    const float tot = sh + __shfl_xor(sh, 32) + kEps;
    if (qi < T_) {
        store_cols16<D, PART>(p.out + b * p.os[0] + hq * p.os[1] + qi * p.os[2], g, oacc, 1.f / tot, p.dr);
        if (g == 0 && p.row_sums != nullptr) p.row_sums[(static_cast<int64_t>(b) * p.Hq + hq) * T_ + qi] = tot;
    }
}

template <int D, bool EXACT, bool PART>
__global__ __launch_bounds__(64 * R16Dma<D>::NW) __attribute__((amdgpu_waves_per_eu(R16Dma<D>::NW / 4, R16Dma<D>::MAX_WAVES)))
void flash_bwd_dq_f32dma_kernel(F32Params p) {
    using C = R16Dma<D>;
    // stage arrays [K][V]; two arrays so that a tile's LDS reads never wait
    // for the direct-to-LDS loads filling the other stage
    __shared__ __attribute__((aligned(16))) float lds0[2 * C::TILE];
    __shared__ __attribute__((aligned(16))) float lds1[C::STAGES > 1 ? 2 * C::TILE : 4];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4;
    const int l16 = lane & 15;
    const int T_ = p.T;
    const int nqb = (T_ + C::ROWS - 1) / C::ROWS;
    const int per = p.B * p.Hq;
    const int step = blockIdx.x / per;
    const int rest = blockIdx.x - step * per;
    const int qb = nqb - 1 - step;
    const int b = rest / p.Hq;
    const int hq = rest - b * p.Hq;
    const int hk = hq / p.G;
    const float* kp = p.k + b * p.ks[0] + hk * p.ks[1];
    const float* vp = p.v + b * p.vs[0] + hk * p.vs[1];

    const int q0 = qb * C::ROWS + 16 * wave;
    const int qi = q0 + l16;
    const int qrow = min(qi, T_ - 1);
    float qv[D / 4], dov[D / 4];
    load_quarter_row<D, PART>(p.q + b * p.qs[0] + hq * p.qs[1] + qrow * p.qs[2], g, qv, p.dr);
    load_quarter_row<D, PART>(p.dout + b * p.dos[0] + hq * p.dos[1] + qrow * p.dos[2], g, dov, p.dr);
    float dpart = 0.f;
    {
        const float* orow = p.o + b * p.os[0] + hq * p.os[1] + qrow * p.os[2];
#pragma unroll
        for (int i4 = 0; i4 < D / 16; ++i4) {
            const int c = g * (D / 4) + 4 * i4;
            const bool in = !PART || c < p.dr;
            float4 ov = *reinterpret_cast<const float4*>(orow + (in ? c : 0));
            if (!in) ov = float4{0.f, 0.f, 0.f, 0.f};
            dpart = __builtin_fmaf(dov[4 * i4 + 0], ov.x, dpart);
            dpart = __builtin_fmaf(dov[4 * i4 + 1], ov.y, dpart);
            dpart = __builtin_fmaf(dov[4 * i4 + 2], ov.z, dpart);
            dpart = __builtin_fmaf(dov[4 * i4 + 3], ov.w, dpart);
        }
    }
    const float dh = dpart + __shfl_xor(dpart, 16);
    const float dl = dh + __shfl_xor(dh, 32);
    const int64_t rbase = (static_cast<int64_t>(b) * p.Hq + hq) * T_;
    if (qi < T_ && g == 0) p.delta[rbase + qi] = dl;
    const float inv_r = 1.f / p.rs[rbase + qrow];

    f32x4 acc[D / 16];
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    const f32x4 ndl{-dl, -dl, -dl, -dl};
    const int W = p.window;
    const unsigned weff = W > 0 ? static_cast<unsigned>(W) : 0x7FFFFFFFu;
    const int n_kv = (T_ + kFT - 1) / kFT;
    const int kv_end = min((qb * C::ROWS + C::ROWS + kFT - 1) / kFT, n_kv);
    const int kv_begin = W > 0 ? max(0, qb * C::ROWS - W + 1) / kFT : 0;
    const float sc = p.scale;

    auto stage = [&](auto st) -> float* {
        if constexpr (decltype(st)::value == 0) return lds0;
        else return lds1;
    };
    auto issue = [&](int t, auto st) {
        float* l = stage(st);
        dma_tile_f32<D, C::NW>(kp, p.ks[2], t * kFT, T_, p.dr, l, wave, lane);
        dma_tile_f32<D, C::NW>(vp, p.vs[2], t * kFT, T_, p.dr, l + C::TILE, wave, lane);
    };
    auto compute = [&](int t, auto st) {
        const float* l = stage(st);
        dq_tile16<D, EXACT>(l, l + C::TILE, t * kFT, q0, qi, l16, g, qv, dov, ndl, sc, W, weff, acc);
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    if constexpr (C::STAGES == 2) {
        issue(kv_begin, S0{});
        tile_wait_vmem();
        __syncthreads();
        // tile t reads stage (t - kv_begin) & 1 while the other fills with t + 1
        auto run = [&](int t, auto cur) {
            if (t + 1 < kv_end) issue(t + 1, std::integral_constant<int, 1 - decltype(cur)::value>{});
            compute(t, cur);
            if (t + 1 < kv_end) {
                tile_wait_vmem();
                __syncthreads();
            }
        };
        for (int t = kv_begin; t < kv_end; t += 2) {
            run(t, S0{});
            if (t + 1 < kv_end) run(t + 1, S1{});
        }
    } else {
        for (int t = kv_begin; t < kv_end; ++t) {
            if (t > kv_begin) __syncthreads();
            issue(t, S0{});
            tile_wait_vmem();
            __syncthreads();
            compute(t, S0{});
        }
    }
    if (qi < T_) store_cols16<D, PART>(p.dq + b * p.dqs[0] + hq * p.dqs[1] + qi * p.dqs[2], g, acc, 2.f * sc * inv_r, p.dr);
}

template <int D, bool EXACT, bool PART, int WHICH>
__global__ __launch_bounds__(64 * R16Dma<D>::NW) __attribute__((amdgpu_waves_per_eu(R16Dma<D>::NW / 4, R16Dma<D>::MAX_WAVES)))
void flash_bwd_kv_f32dma_kernel(F32Params p) {
    using C = R16Dma<D>;
    constexpr bool DO_V = WHICH != kDkdvK, DO_K = WHICH != kDkdvV;
    __shared__ __attribute__((aligned(16))) float lds0[2 * C::TILE];  // [Q][dO]
    __shared__ __attribute__((aligned(16))) float lds1[C::STAGES > 1 ? 2 * C::TILE : 4];
    __shared__ __attribute__((aligned(16))) float ldr[C::STAGES][2][kFT];  // [stage][1/R, -delta]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4;
    const int l16 = lane & 15;
    const int T_ = p.T;
    const int per = p.B * p.Hkv;
    const int kb = blockIdx.x / per;  // earliest key blocks (most queries) first
    const int rest = blockIdx.x - kb * per;
    const int b = rest / p.Hkv;
    const int hk = rest - b * p.Hkv;

    const int k_start = kb * C::ROWS;
    const int wk0 = k_start + 16 * wave;
    const int kj = wk0 + l16;
    const int krow = min(kj, T_ - 1);
    float kv[D / 4], vv[DO_K ? D / 4 : 1];
    load_quarter_row<D, PART>(p.k + b * p.ks[0] + hk * p.ks[1] + krow * p.ks[2], g, kv, p.dr);
    if constexpr (DO_K) load_quarter_row<D, PART>(p.v + b * p.vs[0] + hk * p.vs[1] + krow * p.vs[2], g, vv, p.dr);
    f32x4 dkacc[DO_K ? D / 16 : 1], dvacc[DO_V ? D / 16 : 1];
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) {
        if constexpr (DO_K) dkacc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
        if constexpr (DO_V) dvacc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const int W = p.window;
    const unsigned weff = W > 0 ? static_cast<unsigned>(W) : 0x7FFFFFFFu;
    const int n_qt = (T_ + kFT - 1) / kFT;
    const int qt_begin = k_start / kFT;
    const int qt_end = W > 0 ? min(n_qt, (k_start + C::ROWS - 1 + W - 1) / kFT + 1) : n_qt;
    const int nq = qt_end - qt_begin;  // >= 1 (k_start < T)
    const int n_it = p.G * nq;
    const float sc = p.scale;

    auto tile_of = [&](int it, int& hq, int& q0) {
        const int gg = it / nq;
        q0 = (qt_begin + it - gg * nq) * kFT;
        hq = hk * p.G + gg;
    };
    auto stage = [&](auto st) -> float* {
        if constexpr (decltype(st)::value == 0) return lds0;
        else return lds1;
    };
    auto issue = [&](int it, auto st) {
        int hq, q0;
        tile_of(it, hq, q0);
        float* l = stage(st);
        dma_tile_f32<D, C::NW>(p.q + b * p.qs[0] + hq * p.qs[1], p.qs[2], q0, T_, p.dr, l, wave, lane);
        dma_tile_f32<D, C::NW>(p.dout + b * p.dos[0] + hq * p.dos[1], p.dos[2], q0, T_, p.dr, l + C::TILE, wave, lane);
    };
    // threads 0 .. kFT - 1 load the tile's row sums, the next kFT its delta;
    // they are staged as 1/R and -delta
    auto row_value = [&](int it) {
        int hq, q0;
        tile_of(it, hq, q0);
        if (tid >= 2 * kFT) return 0.f;
        const int64_t idx = (static_cast<int64_t>(b) * p.Hq + hq) * T_ + min(q0 + (tid & (kFT - 1)), T_ - 1);
        return (tid < kFT ? p.rs : p.delta)[idx];
    };
    auto store_rv = [&](int st, float raw) {
        if (tid < 2 * kFT) ldr[st][tid / kFT][tid & (kFT - 1)] = tid < kFT ? 1.f / raw : -raw;
    };
    auto compute = [&](int it, auto st) {
        int hq, q0;
        tile_of(it, hq, q0);
        (void)hq;
        const float* l = stage(st);
        kv_tile16<D, EXACT, WHICH>(l, l + C::TILE, ldr[decltype(st)::value], q0, wk0, kj, T_, l16, g, kv, vv, sc, W,
                                   weff, dkacc, dvacc);
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    if constexpr (C::STAGES == 2) {
        issue(0, S0{});
        store_rv(0, row_value(0));
        tile_wait_vmem();
        __syncthreads();
        auto run = [&](int it, auto cur) {
            constexpr int nxt = 1 - decltype(cur)::value;
            const bool more = it + 1 < n_it;
            float rnext = 0.f;
            if (more) {
                issue(it + 1, std::integral_constant<int, nxt>{});
                rnext = row_value(it + 1);
            }
            compute(it, cur);
            if (more) {
                store_rv(nxt, rnext);
                tile_wait_vmem();
                __syncthreads();
            }
        };
        for (int it = 0; it < n_it; it += 2) {
            run(it, S0{});
            if (it + 1 < n_it) run(it + 1, S1{});
        }
    } else {
        for (int it = 0; it < n_it; ++it) {
            if (it > 0) __syncthreads();
            issue(it, S0{});
            store_rv(0, row_value(it));
            tile_wait_vmem();
            __syncthreads();
            compute(it, S0{});
        }
    }
    if (kj < T_) {
        if constexpr (DO_K)
            store_cols16<D, PART>(p.dk + b * p.dks[0] + hk * p.dks[1] + kj * p.dks[2], g, dkacc, 2.f * sc, p.dr);
        if constexpr (DO_V)
            store_cols16<D, PART>(p.dv + b * p.dvs[0] + hk * p.dvs[1] + kj * p.dvs[2], g, dvacc, 1.f, p.dr);
    }
}

template <int D>
int launch_fwd_f32_d(const F32Params& prm, int exact, hipStream_t st) {
    if constexpr (D >= 256) {
        using C = R16Dma<D>;
        const int64_t nblk = static_cast<int64_t>((prm.T + C::ROWS - 1) / C::ROWS) * prm.B * prm.Hq;
        if (nblk * 64 * C::NW >= (int64_t(1) << 32)) return SA_ERR_BAD_SHAPE;
        const dim3 grid(static_cast<unsigned>(nblk));
        const bool part = prm.dr != D;
        if (exact && part) flash_fwd_f32dma_kernel<D, true, true><<<grid, 64 * C::NW, 0, st>>>(prm);
        else if (exact) flash_fwd_f32dma_kernel<D, true, false><<<grid, 64 * C::NW, 0, st>>>(prm);
        else if (part) flash_fwd_f32dma_kernel<D, false, true><<<grid, 64 * C::NW, 0, st>>>(prm);
        else flash_fwd_f32dma_kernel<D, false, false><<<grid, 64 * C::NW, 0, st>>>(prm);
        return status_from_launch();
    } else {
        const int64_t nblk = static_cast<int64_t>((prm.T + kFRows - 1) / kFRows) * prm.B * prm.Hq;
        if (nblk * 64 * kFW >= (int64_t(1) << 32)) return SA_ERR_BAD_SHAPE;
        const dim3 grid(static_cast<unsigned>(nblk));
        if (exact)
            flash_fwd_f32_kernel<D, true><<<grid, 64 * kFW, 0, st>>>(prm);
        else
            flash_fwd_f32_kernel<D, false><<<grid, 64 * kFW, 0, st>>>(prm);
        return status_from_launch();
    }
}

// The 16-row kernels: D = 128, dQ then dK and dV in one kernel, tiles
// staged through registers; D = 256 and 512, dQ, dV, dK, tiles loaded
// straight into LDS.
template <int D, bool EXACT, bool PART>
int launch_bwd_f32r16(const F32Params& prm, hipStream_t st) {
    constexpr int NW = R16Dma<D>::NW, ROWS = 16 * NW;
    const int64_t nq = static_cast<int64_t>((prm.T + ROWS - 1) / ROWS) * prm.B * prm.Hq;
    if (nq * 64 * NW >= (int64_t(1) << 32)) return SA_ERR_BAD_SHAPE;
    const dim3 gq(static_cast<unsigned>(nq)), gk(static_cast<unsigned>(nq / prm.G));
    flash_bwd_dq_f32dma_kernel<D, EXACT, PART><<<gq, 64 * NW, 0, st>>>(prm);
    if constexpr (D <= 128) {
        flash_bwd_kv_f32dma_kernel<D, EXACT, PART, kDkdvBoth><<<gk, 64 * NW, 0, st>>>(prm);
    } else {
        flash_bwd_kv_f32dma_kernel<D, EXACT, PART, kDkdvV><<<gk, 64 * NW, 0, st>>>(prm);
        flash_bwd_kv_f32dma_kernel<D, EXACT, PART, kDkdvK><<<gk, 64 * NW, 0, st>>>(prm);
    }
    return status_from_launch();
}

template <int D>
int launch_bwd_f32_d(const F32Params& prm, int exact, hipStream_t st) {
    if constexpr (D >= 64) {
        // 16 rows per wave; masked builds (PART) only below the kernel's head dim
        const bool part = prm.dr != D;
        if (exact && part) return launch_bwd_f32r16<D, true, true>(prm, st);
        if (exact) return launch_bwd_f32r16<D, true, false>(prm, st);
        if (part) return launch_bwd_f32r16<D, false, true>(prm, st);
        return launch_bwd_f32r16<D, false, false>(prm, st);
    } else {
        // 32 rows per wave (D = 32: the 16-row kernels ran 4.43 vs 4.13 ms on
        // [4,32,4096,32]).  Masked builds (PART) for every head dim: at D = 64
        // they were the faster even when dr == D (8671 -> 8430 us).
        const int64_t nq = static_cast<int64_t>((prm.T + kFRows - 1) / kFRows) * prm.B * prm.Hq;
        if (nq * 64 * kFW >= (int64_t(1) << 32)) return SA_ERR_BAD_SHAPE;
        const dim3 gq(static_cast<unsigned>(nq)), gk(static_cast<unsigned>(nq / prm.G));
        const bool part = true;
        if (exact && part) {
            flash_bwd_dq_f32_kernel<D, true, true><<<gq, 64 * kFW, 0, st>>>(prm);
            flash_bwd_dkdv_f32_kernel<D, true, true><<<gk, 64 * kFW, 0, st>>>(prm);
        } else if (exact) {
            flash_bwd_dq_f32_kernel<D, true, false><<<gq, 64 * kFW, 0, st>>>(prm);
            flash_bwd_dkdv_f32_kernel<D, true, false><<<gk, 64 * kFW, 0, st>>>(prm);
        } else if (part) {
            flash_bwd_dq_f32_kernel<D, false, true><<<gq, 64 * kFW, 0, st>>>(prm);
            flash_bwd_dkdv_f32_kernel<D, false, true><<<gk, 64 * kFW, 0, st>>>(prm);
        } else {
            flash_bwd_dq_f32_kernel<D, false, false><<<gq, 64 * kFW, 0, st>>>(prm);
            flash_bwd_dkdv_f32_kernel<D, false, false><<<gk, 64 * kFW, 0, st>>>(prm);
        }
        return status_from_launch();
    }
}

}  // namespace

int flash_fwd_f32(const void* q, const void* k, const void* v, void* o, float* row_sums, int B, int Hq, int Hkv,
                  int T, int D, const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                  const int64_t* o_strides, float scale, int window_size, int exact_math, hipStream_t st) {
    const int chk = check_common(B, Hq, Hkv, T, D, window_size);
    if (chk != 0) return chk;
    if (!q || !k || !v || !o || !q_strides || !k_strides || !v_strides || !o_strides) return SA_ERR_NULL_POINTER;
    if (!f32_strides_ok(q_strides) || !f32_strides_ok(k_strides) || !f32_strides_ok(v_strides) ||
        !f32_strides_ok(o_strides) || !aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
        return SA_ERR_BAD_STRIDE;
    if (B == 0 || T == 0) return 0;
    F32Params prm{};
    prm.q = static_cast<const float*>(q);
    prm.k = static_cast<const float*>(k);
    prm.v = static_cast<const float*>(v);
    prm.out = static_cast<float*>(o);
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
    prm.dr = D;
    prm.scale = scale;
    // head dims 4..512 (multiples of 4) on the kernel for the next of 32, 64, 128, 256, 512
    if (D <= 32) return launch_fwd_f32_d<32>(prm, exact_math, st);
    if (D <= 64) return launch_fwd_f32_d<64>(prm, exact_math, st);
    if (D <= 128) return launch_fwd_f32_d<128>(prm, exact_math, st);
    if (D <= 256) return launch_fwd_f32_d<256>(prm, exact_math, st);
    return launch_fwd_f32_d<512>(prm, exact_math, st);
}

int flash_bwd_f32(const void* q, const void* k, const void* v, const void* o, const void* dout,
                  const float* row_sums, void* dq, void* dk, void* dv, float* delta_ws, int B, int Hq, int Hkv,
                  int T, int D, const int64_t* const strides[8], float scale, int window_size, int exact_math,
                  hipStream_t st) {
    const int chk = check_common(B, Hq, Hkv, T, D, window_size);
    if (chk != 0) return chk;
    if (!q || !k || !v || !o || !dout || !row_sums || !dq || !dk || !dv || !delta_ws) return SA_ERR_NULL_POINTER;
    const void* ptrs[8] = {q, k, v, o, dout, dq, dk, dv};
    for (int i = 0; i < 8; ++i) {
        if (!strides[i]) return SA_ERR_NULL_POINTER;
        if (!f32_strides_ok(strides[i]) || !aligned16(ptrs[i])) return SA_ERR_BAD_STRIDE;
    }
    if (B == 0 || T == 0) return 0;
    F32Params prm{};
    prm.q = static_cast<const float*>(q);
    prm.k = static_cast<const float*>(k);
    prm.v = static_cast<const float*>(v);
    prm.o = static_cast<const float*>(o);
    prm.dout = static_cast<const float*>(dout);
    prm.rs = row_sums;
    prm.dq = static_cast<float*>(dq);
    prm.dk = static_cast<float*>(dk);
    prm.dv = static_cast<float*>(dv);
    prm.delta = delta_ws;
    int64_t* dst[8] = {prm.qs, prm.ks, prm.vs, prm.os, prm.dos, prm.dqs, prm.dks, prm.dvs};
    for (int i = 0; i < 8; ++i)
        for (int j = 0; j < 4; ++j) dst[i][j] = strides[i][j];
    prm.B = B;
    prm.Hq = Hq;
    prm.Hkv = Hkv;
    prm.T = T;
    prm.G = Hq / Hkv;
    prm.window = window_size;
    prm.dr = D;
    prm.scale = scale;
    if (D <= 32) return launch_bwd_f32_d<32>(prm, exact_math, st);
    if (D <= 64) return launch_bwd_f32_d<64>(prm, exact_math, st);
    if (D <= 128) return launch_bwd_f32_d<128>(prm, exact_math, st);
    if (D <= 256) return launch_bwd_f32_d<256>(prm, exact_math, st);
    return launch_bwd_f32_d<512>(prm, exact_math, st);
}

}  // namespace sa
