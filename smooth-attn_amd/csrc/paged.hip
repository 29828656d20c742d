// Paged single-token squareplus decode through a block table (gfx950).
//
// out[b, h] = sum_{t < ctx_b} y_t V_t / (sum_t y_t + 1e-12),
// y_t = squareplus(2 scale q . K_t - 1)^2,
// K_t = k_cache[block_table[b, t / P], h / G, t % P]
//   (reference kernels.py:2681-2773 and the decode references of
//    tests/test_paged_long_context.py:39-65)
//
// One wavefront per (sequence b, KV head, split of kSplitTok tokens).  The
// wave walks its split in tiles of 32 tokens and reads every K/V row once
// for all G query heads that share the KV head (the reference grid
// (B, Hq) rereads each page G times).  Scores are S^T = K Q^T on MFMA with
// the G query heads as columns; the squareplus weights land in the B-operand
// layout of O^T += V^T P^T, and V^T comes from a wave-private row-major LDS
// tile through the transposing LDS read (see flash_common.hpp).
// Each wave writes its unnormalised partial (O, S); a second kernel sums the
// partials of a sequence in split order (squareplus needs no running
// maximum, so merging is a plain sum) and divides once.
#include "flash_common.hpp"

namespace sa {
namespace {

constexpr int kSplitTok = 512;  // tokens per work unit
constexpr int kTile = 32;       // tokens per MFMA tile

struct PagedParams {
    const void* q;
    const void* k;
    const void* v;
    bf16* out;
    const int32_t* table;
    const int32_t* ctx;
    float* ws_o;  // [B][Hq][n_splits][D]
    float* ws_s;  // [B][Hq][n_splits]
    int64_t qs[4], ks[4], vs[4], os[3];
    int64_t bt_stride;
    int B, Hq, Hkv, G, P, max_pages, n_pages, n_splits;
    float scale;
};

template <typename T, int D>
__global__ __launch_bounds__(64) void paged_partial_kernel(PagedParams p) {
    using Ops = MfmaOps<T>;
    using Vec = typename Ops::vec8;
    constexpr int RSV = D + 8;
    __shared__ __attribute__((aligned(16))) T ldsV[kTile * RSV];

    const int lane = threadIdx.x;
    const int hi = lane >> 5;
    const int l32 = lane & 31;
    const int unit = blockIdx.x;
    const int split = unit % p.n_splits;
    const int bk = unit / p.n_splits;
    const int b = bk / p.Hkv;
    const int hk = bk - b * p.Hkv;
    const int ctx = min(max(p.ctx[b], 0), p.max_pages * p.P);
    const int t_begin = split * kSplitTok;
    if (t_begin >= ctx) return;  // whole wave: nothing in this split
    const int t_end = min(ctx, t_begin + kSplitTok);

    const T* kc = static_cast<const T*>(p.k) + hk * p.ks[1];
    const T* vc = static_cast<const T*>(p.v) + hk * p.vs[1];
    const int32_t* table = p.table + b * p.bt_stride;

    // Q^T as the B operand: column = query head hk*G + l32 (zero past G).
    u32x4 qreg[D / 16];
    {
        const bool live = l32 < p.G;
        const T* qrow = static_cast<const T*>(p.q) + b * p.qs[0] + (hk * p.G + (live ? l32 : 0)) * p.qs[1];
#pragma unroll
        for (int dc = 0; dc < D / 16; ++dc)
            qreg[dc] = live ? load16(qrow + dc * 16 + hi * 8) : u32x4{0u, 0u, 0u, 0u};
    }

    f32x16 oacc[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) oacc[dt] = f32x16{};
    float ssum = 0.f;

    const int v_tr_off = ((lane >> 5) * 4 + ((lane & 15) >> 2)) * RSV + ((lane >> 4) & 1) * 16 + 4 * (lane & 3);
    const int P = p.P;

    for (int t0 = t_begin; t0 < t_end; t0 += kTile) {
        // K operand rows: token t0 + l32.
        u32x4 kreg[D / 16];
        {
            const int t = t0 + l32;
            if (t < t_end) {
                const int phys = min(max(table[t / P], 0), p.n_pages - 1);
                const T* row = kc + static_cast<int64_t>(phys) * p.ks[0] + (t % P) * p.ks[2];
#pragma unroll
                for (int dc = 0; dc < D / 16; ++dc) kreg[dc] = load16(row + dc * 16 + hi * 8);
            } else {
#pragma unroll
                for (int dc = 0; dc < D / 16; ++dc) kreg[dc] = u32x4{0u, 0u, 0u, 0u};
            }
        }
        // V rows: lane covers token t0 + lane/2, half (lane & 1) of the row.
        {
            const int tv = lane >> 1;
            const int part = lane & 1;
            const int t = t0 + tv;
            T* dst = ldsV + tv * RSV + part * (D / 2);
            if (t < t_end) {
                const int phys = min(max(table[t / P], 0), p.n_pages - 1);
                const T* row = vc + static_cast<int64_t>(phys) * p.vs[0] + (t % P) * p.vs[2] + part * (D / 2);
#pragma unroll
                for (int c = 0; c < D / 16; ++c) *reinterpret_cast<u32x4*>(dst + c * 8) = load16(row + c * 8);
            } else {
#pragma unroll
                for (int c = 0; c < D / 16; ++c) *reinterpret_cast<u32x4*>(dst + c * 8) = u32x4{0u, 0u, 0u, 0u};
            }
        }
        __syncthreads();

        f32x16 s = f32x16{};
#pragma unroll
        for (int dc = 0; dc < D / 16; ++dc) s = Ops::mma(as_vec8<Vec>(kreg[dc]), as_vec8<Vec>(qreg[dc]), s);

        float y[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int t = t0 + (v >> 2) * 8 + hi * 4 + (v & 3);
            const float w = sp2_weight<true>(__builtin_fmaf(s[v], p.scale, -0.5f));
            y[v] = t < t_end ? w : 0.f;
            ssum += y[v];
        }
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            u32x4 pw;
            pw.x = pack2<T>(y[8 * c + 0], y[8 * c + 1]);
            pw.y = pack2<T>(y[8 * c + 2], y[8 * c + 3]);
            pw.z = pack2<T>(y[8 * c + 4], y[8 * c + 5]);
            pw.w = pack2<T>(y[8 * c + 6], y[8 * c + 7]);
            const Vec bop = as_vec8<Vec>(pw);
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) {
                const T* base = ldsV + (16 * c) * RSV + dt * 32 + v_tr_off;
                const uint2 lo = lds_read_tr16(base);
                const uint2 hi8 = lds_read_tr16(base + 8 * RSV);
                const u32x4 aw{lo.x, lo.y, hi8.x, hi8.y};
                oacc[dt] = Ops::mma(as_vec8<Vec>(aw), bop, oacc[dt]);
            }
        }
        __syncthreads();
    }

    const float stot = ssum + __shfl_xor(ssum, 32);
    if (l32 < p.G) {
        const int hq = hk * p.G + l32;
        const int64_t slot = (static_cast<int64_t>(b) * p.Hq + hq) * p.n_splits + split;
        float* wo = p.ws_o + slot * D;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
            for (int vg = 0; vg < 4; ++vg) {
                const int d0 = dt * 32 + vg * 8 + hi * 4;
                *reinterpret_cast<float4*>(wo + d0) =
                    float4{oacc[dt][vg * 4 + 0], oacc[dt][vg * 4 + 1], oacc[dt][vg * 4 + 2], oacc[dt][vg * 4 + 3]};
            }
        }
        if (hi == 0) p.ws_s[slot] = stot;
    }
}

// Sum the split partials of one (b, query head) in split order, then divide.
template <int D>
__global__ __launch_bounds__(D) void paged_merge_kernel(PagedParams p) {
    const int bh = blockIdx.x;
    const int b = bh / p.Hq;
    const int hq = bh - b * p.Hq;
    const int d = threadIdx.x;
    const int ctx = min(max(p.ctx[b], 0), p.max_pages * p.P);
    const int n_valid = (ctx + kSplitTok - 1) / kSplitTok;
    const int64_t slot0 = static_cast<int64_t>(bh) * p.n_splits;
    float o = 0.f, s = 0.f;
    for (int i = 0; i < n_valid; ++i) {
        o += p.ws_o[(slot0 + i) * D + d];
        s += p.ws_s[slot0 + i];
    }
    p.out[b * p.os[0] + hq * p.os[1] + d * p.os[2]] = static_cast<bf16>(o / (s + kEps));
}

template <typename T, int D>
int launch_paged(const PagedParams& prm, hipStream_t st) {
    const unsigned units = static_cast<unsigned>(prm.B) * prm.Hkv * prm.n_splits;
    paged_partial_kernel<T, D><<<units, 64, 0, st>>>(prm);
    paged_merge_kernel<D><<<static_cast<unsigned>(prm.B) * prm.Hq, D, 0, st>>>(prm);
    return status_from_launch();
}

int64_t splits_for(int max_pages, int page_size) {
    const int64_t toks = static_cast<int64_t>(max_pages) * page_size;
    return toks <= 0 ? 1 : (toks + kSplitTok - 1) / kSplitTok;
}

}  // namespace
}  // namespace sa

extern "C" int64_t sa_paged_decode_workspace_size(int B, int Hq, int D, int max_pages, int page_size) {
    if (B <= 0 || Hq <= 0 || D <= 0 || max_pages < 0 || page_size <= 0) return 0;
    const int64_t slots = static_cast<int64_t>(B) * Hq * sa::splits_for(max_pages, page_size);
    return slots * (D + 1) * static_cast<int64_t>(sizeof(float));
}

extern "C" int sa_paged_decode(const void* q, const void* k_cache, const void* v_cache, void* out,
                               const int32_t* block_table, const int32_t* context_lens, int B, int Hq, int Hkv,
                               int D, int page_size, int max_pages, int n_pages, const int64_t* q_strides,
                               const int64_t* kv_strides, const int64_t* vv_strides, const int64_t* o_strides,
                               int64_t bt_stride, float scale, int dtype, float* workspace, int64_t workspace_bytes,
                               sa_stream_t stream) {
    using namespace sa;
    if (B < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || max_pages < 0 || n_pages < 0) return SA_ERR_BAD_SHAPE;
    if (Hq / Hkv > 32) return SA_ERR_UNSUPPORTED;  // query heads per KV head fill one 32-wide MFMA column block
    if (page_size != 8 && page_size != 16 && page_size != 32 && page_size != 64) return SA_ERR_UNSUPPORTED;
    if (D != 32 && D != 64 && D != 128) return SA_ERR_UNSUPPORTED;
    if (B == 0) return 0;
    if (n_pages == 0) max_pages = 0;  // no cache: every context is empty
    if (!q || !k_cache || !v_cache || !out || !block_table || !context_lens || !q_strides || !kv_strides ||
        !vv_strides || !o_strides || !workspace)
        return SA_ERR_NULL_POINTER;
    if (workspace_bytes < sa_paged_decode_workspace_size(B, Hq, D, max_pages, page_size)) return SA_ERR_WORKSPACE;
    const auto ok16 = [](const int64_t* s, int n) {
        for (int i = 0; i < n - 1; ++i)
            if (s[i] % 8 != 0) return false;
        return s[n - 1] == 1;
    };
    if (!ok16(q_strides, 4) || !ok16(kv_strides, 4) || !ok16(vv_strides, 4) || o_strides[2] != 1 ||
        !aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache))
        return SA_ERR_BAD_STRIDE;
    if (dtype != SA_BF16 && dtype != SA_F16) return SA_ERR_BAD_DTYPE;
    PagedParams prm{};
    prm.q = q;
    prm.k = k_cache;
    prm.v = v_cache;
    prm.out = static_cast<bf16*>(out);
    prm.table = block_table;
    prm.ctx = context_lens;
    prm.n_splits = static_cast<int>(splits_for(max_pages, page_size));
    prm.ws_o = workspace;
    prm.ws_s = workspace + static_cast<int64_t>(B) * Hq * prm.n_splits * D;
    for (int i = 0; i < 4; ++i) {
        prm.qs[i] = q_strides[i];
        prm.ks[i] = kv_strides[i];
        prm.vs[i] = vv_strides[i];
    }
    for (int i = 0; i < 3; ++i) prm.os[i] = o_strides[i];
    prm.bt_stride = bt_stride;
    prm.B = B;
    prm.Hq = Hq;
    prm.Hkv = Hkv;
    prm.G = Hq / Hkv;
    prm.P = page_size;
    prm.max_pages = max_pages;
    prm.n_pages = n_pages;
    prm.scale = scale;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (dtype == SA_BF16) {
        switch (D) {
            case 32: return launch_paged<bf16, 32>(prm, st);
            case 64: return launch_paged<bf16, 64>(prm, st);
            default: return launch_paged<bf16, 128>(prm, st);
        }
    }
    switch (D) {
        case 32: return launch_paged<f16, 32>(prm, st);
        case 64: return launch_paged<f16, 64>(prm, st);
        default: return launch_paged<f16, 128>(prm, st);
    }
}
