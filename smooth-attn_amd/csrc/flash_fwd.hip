// Fused causal squareplus attention forward, bf16 / fp16 on gfx950 MFMA.
//
// O_i = sum_{j <= i, i - j < W} y_ij V_j / (sum_j y_ij + 1e-12),
// y = squareplus(2 s - 1)^2, s = scale q_i . k_j   (reference kernels.py:1536-1631)
//
// Squareplus needs no running maximum, so the weights are accumulated
// linearly (sum y in fp32, P V on MFMA with P rounded to the input type, as
// the reference does at :1617-1621) and divided once at the end.
//
// Work decomposition: a block of 4 waves owns 128 query rows of one
// (batch, query head); wave w owns rows [32w, 32w+32).  K and V tiles of 64
// keys are staged through LDS (double buffered, one barrier per tile):
// global -> registers for tile j+1 while tile j is computed, then registers
// -> LDS.  Per wave and tile: S^T = K Q^T (2 x D/16 MFMA 32x32x16), the
// squareplus weights on the VALU (masks only on tiles crossing the diagonal
// or the window edge), then O^T += V^T P^T (4 x D/32 MFMA).
// Blocks are issued heaviest first (last query blocks first) and, because the
// block index runs over (batch, head) fastest, every query block of one head
// lands on the same XCD when B*Hq is a multiple of 8 (shared K/V in L2).
#include "flash_common.hpp"

namespace sa {
namespace {

constexpr int kBQ = 128;   // query rows per block
constexpr int kBKV = 64;   // keys per tile
constexpr int kWaves = 4;  // 32 query rows per wave

struct FlashParams {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* row_sums;
    int64_t qs[4], ks[4], vs[4], os[4];
    int B, Hq, Hkv, T, G, window, nqb;
    float scale;
};

template <int D>
struct TileGeom {
    static constexpr int RSK = D + 8;    // K row stride in LDS (elements)
    static constexpr int RSV = D + 8;    // V row stride in LDS (elements)
    static constexpr int KT = kBKV * RSK;
    static constexpr int VT = kBKV * RSV;
    static constexpr int CPR = D / 8;                 // 16-byte chunks per row
    static constexpr int NL = kBKV * CPR / (64 * kWaves);  // chunks per thread per tensor
};

template <typename T, int D, bool EXACT>
__global__ __launch_bounds__(256, 2) void flash_fwd_kernel(FlashParams p) {
    using G = TileGeom<D>;
    using Ops = MfmaOps<T>;
    using V8 = typename Ops::vec8;
    __shared__ __attribute__((aligned(16))) T lds[2 * (G::KT + G::VT)];
    T* ldsK = lds;                 // [2][64][RSK]
    T* ldsV = lds + 2 * G::KT;     // [2][64][RSV]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int hi = lane >> 5;      // lane half
    const int l32 = lane & 31;

    const int BH = p.B * p.Hq;
    const int id = blockIdx.x;
    const int qb = p.nqb - 1 - id / BH;
    const int bh = id % BH;
    const int b = bh / p.Hq;
    const int hq = bh - b * p.Hq;
    const int hk = hq / p.G;
    const int T_ = p.T;

    const T* qp = static_cast<const T*>(p.q) + b * p.qs[0] + hq * p.qs[1];
    const T* kp = static_cast<const T*>(p.k) + b * p.ks[0] + hk * p.ks[1];
    const T* vp = static_cast<const T*>(p.v) + b * p.vs[0] + hk * p.vs[1];
    T* op = static_cast<T*>(p.o) + b * p.os[0] + hq * p.os[1];

    const int q_start = qb * kBQ;
    const int wq0 = q_start + wave * 32;
    const int W = p.window;
    const int n_kv = (T_ + kBKV - 1) / kBKV;
    const int kv_end = min((q_start + kBQ + kBKV - 1) / kBKV, n_kv);
    const int kv_begin = W > 0 ? max(0, q_start - W + 1) / kBKV : 0;

    // Q^T as the B operand: lane holds query row wq0 + l32, d = 16 dc + 8 hi .. +7.
    u32x4 qreg[D / 16];
    {
        const int qrow = wq0 + l32;
#pragma unroll
        for (int dc = 0; dc < D / 16; ++dc) {
            qreg[dc] = qrow < T_ ? load16(qp + qrow * p.qs[2] + dc * 16 + hi * 8) : u32x4{0u, 0u, 0u, 0u};
        }
    }

    f32x16 oacc[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) oacc[dt] = f32x16{};
    float ssum = 0.f;

    // Global -> register staging of one K/V tile.
    u32x4 kst[G::NL], vst[G::NL];
    auto load_tile = [&](int j) {
        const int k0 = j * kBKV;
#pragma unroll
        for (int i = 0; i < G::NL; ++i) {
            const int ci = tid + 256 * i;
            const int row = ci / G::CPR;
            const int c8 = ci - row * G::CPR;
            const int key = k0 + row;
            if (key < T_) {
                kst[i] = load16(kp + key * p.ks[2] + c8 * 8);
                vst[i] = load16(vp + key * p.vs[2] + c8 * 8);
            } else {
                kst[i] = u32x4{0u, 0u, 0u, 0u};
                vst[i] = u32x4{0u, 0u, 0u, 0u};
            }
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < G::NL; ++i) {
            const int ci = tid + 256 * i;
            const int row = ci / G::CPR;
            const int c8 = ci - row * G::CPR;
            *reinterpret_cast<u32x4*>(ldsK + buf * G::KT + row * G::RSK + c8 * 8) = kst[i];
            *reinterpret_cast<u32x4*>(ldsV + buf * G::VT + row * G::RSV + c8 * 8) = vst[i];
        }
    };

    // Per-lane element offset of the transposing V read (key part + d part);
    // see flash_common.hpp for the derivation.
    const int v_tr_off = ((lane >> 5) * 4 + ((lane & 15) >> 2)) * G::RSV + ((lane >> 4) & 1) * 16 + 4 * (lane & 3);
    const float scale = p.scale;

    if (kv_begin < kv_end) {
        load_tile(kv_begin);
        store_tile(0);
    }
    __syncthreads();

    for (int j = kv_begin; j < kv_end; ++j) {
        const int buf = (j - kv_begin) & 1;
        const bool has_next = j + 1 < kv_end;
        if (has_next) load_tile(j + 1);
        const int k0 = j * kBKV;
        const bool active = (k0 <= wq0 + 31) && !(W > 0 && k0 + kBKV - 1 <= wq0 - W);
        if (active) {
            const T* Kb = ldsK + buf * G::KT;
            const T* Vb = ldsV + buf * G::VT;
            f32x16 s[2];
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                s[kt] = f32x16{};
#pragma unroll
                for (int dc = 0; dc < D / 16; ++dc) {
                    const u32x4 a = *reinterpret_cast<const u32x4*>(Kb + (kt * 32 + l32) * G::RSK + dc * 16 + hi * 8);
                    s[kt] = Ops::mma(as_vec8<V8>(a), as_vec8<V8>(qreg[dc]), s[kt]);
                }
            }
            const bool edge = (k0 + kBKV - 1 > wq0) || (W > 0 && k0 <= wq0 + 31 - W);
            const int qi = wq0 + l32;
            float y[2][16];
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    float w = sp2_weight<EXACT>(__builtin_fmaf(s[kt][v], scale, -0.5f));
                    if (edge) {
                        const int key = k0 + kt * 32 + (v >> 2) * 8 + hi * 4 + (v & 3);
                        const bool ok = key <= qi && (W <= 0 || qi - key < W);
                        w = ok ? w : 0.f;
                    }
                    y[kt][v] = w;
                    ssum += w;
                }
            }
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                float pv[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) pv[e] = y[c >> 1][(c & 1) * 8 + e];
                u32x4 pw;
                pw.x = pack2<T>(pv[0], pv[1]);
                pw.y = pack2<T>(pv[2], pv[3]);
                pw.z = pack2<T>(pv[4], pv[5]);
                pw.w = pack2<T>(pv[6], pv[7]);
                const V8 bop = as_vec8<V8>(pw);
#pragma unroll
                for (int dt = 0; dt < D / 32; ++dt) {
                    const T* base = Vb + (16 * c) * G::RSV + dt * 32 + v_tr_off;
                    const uint2 lo = lds_read_tr16(base);
                    const uint2 hi8 = lds_read_tr16(base + 8 * G::RSV);
                    const u32x4 aw{lo.x, lo.y, hi8.x, hi8.y};
                    oacc[dt] = Ops::mma(as_vec8<V8>(aw), bop, oacc[dt]);
                }
            }
        }
        if (has_next) store_tile(buf ^ 1);
        __syncthreads();
    }

    // Row sums: lanes l and l^32 hold the two key halves of one query column.
    const float stot = ssum + __shfl_xor(ssum, 32) + kEps;
    const float inv = 1.f / stot;
    const int qi = wq0 + l32;
    if (qi < T_) {
        T* orow = op + qi * p.os[2];
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
            for (int vg = 0; vg < 4; ++vg) {
                const int d0 = dt * 32 + vg * 8 + hi * 4;
                uint2 w;
                w.x = pack2<T>(oacc[dt][vg * 4 + 0] * inv, oacc[dt][vg * 4 + 1] * inv);
                w.y = pack2<T>(oacc[dt][vg * 4 + 2] * inv, oacc[dt][vg * 4 + 3] * inv);
                *reinterpret_cast<uint2*>(orow + d0) = w;
            }
        }
        if (hi == 0 && p.row_sums != nullptr) p.row_sums[static_cast<int64_t>(bh) * T_ + qi] = stot;
    }
}

template <typename T, int D>
int launch_flash(const FlashParams& prm, int exact, hipStream_t st) {
    const dim3 grid(static_cast<unsigned>(prm.nqb) * prm.B * prm.Hq);
    const dim3 block(256);
    if (exact)
        flash_fwd_kernel<T, D, true><<<grid, block, 0, st>>>(prm);
    else
        flash_fwd_kernel<T, D, false><<<grid, block, 0, st>>>(prm);
    return status_from_launch();
}

bool strides_ok(const int64_t* s) {
    return s[3] == 1 && s[0] % 8 == 0 && s[1] % 8 == 0 && s[2] % 8 == 0;
}

}  // namespace
}  // namespace sa

extern "C" int sa_flash_fwd(const void* q, const void* k, const void* v, void* o, float* row_sums, int B, int Hq,
                            int Hkv, int T, int D, const int64_t* q_strides, const int64_t* k_strides,
                            const int64_t* v_strides, const int64_t* o_strides, float scale, int window_size,
                            int exact_math, int dtype, sa_stream_t stream) {
    using namespace sa;
    if (B < 0 || Hq <= 0 || Hkv <= 0 || T < 0 || Hq % Hkv != 0 || window_size < 0) return SA_ERR_BAD_SHAPE;
    if (B == 0 || T == 0) return 0;
    if (!q || !k || !v || !o || !q_strides || !k_strides || !v_strides || !o_strides) return SA_ERR_NULL_POINTER;
    if (D != 32 && D != 64 && D != 128) return SA_ERR_UNSUPPORTED;
    if (!strides_ok(q_strides) || !strides_ok(k_strides) || !strides_ok(v_strides) || !strides_ok(o_strides) ||
        !aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
        return SA_ERR_BAD_STRIDE;
    FlashParams prm{};
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
    prm.nqb = (T + kBQ - 1) / kBQ;
    prm.scale = scale;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int ex = exact_math ? 1 : 0;
    if (dtype == SA_BF16) {
        switch (D) {
            case 32: return launch_flash<bf16, 32>(prm, ex, st);
            case 64: return launch_flash<bf16, 64>(prm, ex, st);
            default: return launch_flash<bf16, 128>(prm, ex, st);
        }
    }
    if (dtype == SA_F16) {
        switch (D) {
            case 32: return launch_flash<f16, 32>(prm, ex, st);
            case 64: return launch_flash<f16, 64>(prm, ex, st);
            default: return launch_flash<f16, 128>(prm, ex, st);
        }
    }
    return SA_ERR_BAD_DTYPE;
}
