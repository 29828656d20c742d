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
// (B, Hq) rereads each page G times).  Tiles are fetched with coalesced
// 16-byte loads (one 1 KB span per instruction) one tile ahead of the
// compute and staged in wave-private LDS.  Scores are S^T = K Q^T on MFMA
// with the G query heads as columns; the squareplus weights land in the
// B-operand layout of O^T += V^T P^T, and V^T comes from the row-major LDS
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
    int B, Hq, Hkv, G, P, logP, max_pages, n_pages, n_splits;
    float scale;
};

// UNIFORM: every load instruction's tokens lie in one page (64 / (D/8)
// tokens per instruction divide the page size), so the page base is
// wave-uniform and comes from v_readlane of the split's page-id register.
template <typename T, int D, bool UNIFORM>
__global__ __launch_bounds__(64) void paged_partial_kernel(PagedParams p) {
    using Ops = MfmaOps<T>;
    using Vec = typename Ops::vec8;
    // Padded LDS rows.  The LDS has 64 banks of 4 bytes; a 16-byte read is
    // served 16 lanes per cycle, an 8-byte transposing read 32 lanes per
    // cycle.  K (read as 16-byte rows, 16 consecutive rows per cycle at one
    // column): a stride of 2D + 16 bytes puts the 16 rows in 16 distinct
    // 16-byte bank slots.  V (transposing reads: per 32 lanes, 4 consecutive
    // rows x 64 bytes): a stride of 64 bytes modulo 256 puts the 4 rows in 4
    // distinct 64-byte slots.
    constexpr int RS = D + 8;                            // K row stride (elements)
    constexpr int RSV = (2 * D) % 256 == 64 ? D : D + 32;  // V row stride (elements)
    constexpr int CPT = D / 8;             // 16-byte chunks per token row
    constexpr int TPI = 64 / CPT;          // tokens per load instruction
    constexpr int NC = kTile * CPT / 64;   // chunks per lane per tile and tensor
    __shared__ __attribute__((aligned(16))) T ldsK[kTile * RS];
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
    const int logP = p.logP;
    const int pmask = p.P - 1;

    const T* kc = static_cast<const T*>(p.k) + hk * p.ks[1];
    const T* vc = static_cast<const T*>(p.v) + hk * p.vs[1];

    // Page ids of this split, one per lane (a split spans <= 64 pages).
    int page_id;
    {
        const int first = t_begin >> logP;
        const int npg = ((t_end - 1) >> logP) - first + 1;
        page_id = lane < npg ? min(max(p.table[b * p.bt_stride + first + lane], 0), p.n_pages - 1) : 0;
    }
    const int first_page = t_begin >> logP;

    // Q^T as the B operand: column = query head hk*G + l32 (zero past G).
    u32x4 qreg[D / 16];
    {
        const bool live = l32 < p.G;
        const T* qrow = static_cast<const T*>(p.q) + b * p.qs[0] + (hk * p.G + (live ? l32 : 0)) * p.qs[1];
#pragma unroll
        for (int dc = 0; dc < D / 16; ++dc)
            qreg[dc] = live ? load16(qrow + dc * 16 + hi * 8) : u32x4{0u, 0u, 0u, 0u};
    }

    // Coalesced tile loads: instruction i of lane l fetches 16-byte chunk
    // c = 64 i + l of the tile (token c / CPT, columns 8 (c % CPT) .. +7).
    const int lane_tok = lane / CPT;
    const int lane_col = (lane % CPT) * 8;
    u32x4 kbuf[NC], vbuf[NC];
    auto load_tile = [&](int t0) {
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int t = t0 + i * TPI + lane_tok;
            int phys;
            int64_t koff, voff;
            if constexpr (UNIFORM) {
                const int tu = t0 + i * TPI;  // first token of the instruction
                phys = __builtin_amdgcn_readlane(page_id, (tu >> logP) - first_page);
                const int r = tu & pmask;
                koff = phys * p.ks[0] + (r + lane_tok) * p.ks[2];
                voff = phys * p.vs[0] + (r + lane_tok) * p.vs[2];
            } else {
                phys = __shfl(page_id, (t >> logP) - first_page);
                koff = phys * p.ks[0] + (t & pmask) * p.ks[2];
                voff = phys * p.vs[0] + (t & pmask) * p.vs[2];
            }
            if (t < t_end) {
                kbuf[i] = load16(kc + koff + lane_col);
                vbuf[i] = load16(vc + voff + lane_col);
            } else {
                kbuf[i] = u32x4{0u, 0u, 0u, 0u};
                vbuf[i] = u32x4{0u, 0u, 0u, 0u};
            }
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int tok = i * TPI + lane_tok;
            *reinterpret_cast<u32x4*>(ldsK + tok * RS + lane_col) = kbuf[i];
            *reinterpret_cast<u32x4*>(ldsV + tok * RSV + lane_col) = vbuf[i];
        }
    };

    f32x16 oacc[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) oacc[dt] = f32x16{};
    float ssum = 0.f;
    const int v_tr_off = ((lane >> 5) * 4 + ((lane & 15) >> 2)) * RSV + ((lane >> 4) & 1) * 16 + 4 * (lane & 3);

    load_tile(t_begin);
    for (int t0 = t_begin; t0 < t_end; t0 += kTile) {
        // The block is one wavefront: LDS accesses of a wave complete in
        // issue order, so a wave-level scheduling barrier is all the ordering
        // needed (a workgroup barrier would also drain the prefetch below).
        store_tile();
        __builtin_amdgcn_wave_barrier();
        if (t0 + kTile < t_end) load_tile(t0 + kTile);

        f32x16 s = f32x16{};
#pragma unroll
        for (int dc = 0; dc < D / 16; ++dc) {
            const u32x4 a = *reinterpret_cast<const u32x4*>(ldsK + l32 * RS + dc * 16 + hi * 8);
            s = Ops::mma(as_vec8<Vec>(a), as_vec8<Vec>(qreg[dc]), s);
        }
        float y[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int t = t0 + (v >> 2) * 8 + hi * 4 + (v & 3);
            const float w = sp2_weight<false>(__builtin_fmaf(s[v], p.scale, -0.5f));
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
        __builtin_amdgcn_wave_barrier();
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
    if (prm.P * (D / 8) >= 64)
        paged_partial_kernel<T, D, true><<<units, 64, 0, st>>>(prm);
    else
        paged_partial_kernel<T, D, false><<<units, 64, 0, st>>>(prm);
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
    prm.logP = __builtin_ctz(static_cast<unsigned>(page_size));
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
