// Paged single-token squareplus decode through a block table (gfx950).
//
// out[b, h] = sum_{t < ctx_b} y_t V_t / (sum_t y_t + 1e-12),
// y_t = squareplus(2 scale q . K_t - 1)^2,
// K_t = k_cache[block_table[b, t / P], h / G, t % P]
//   (reference kernels.py:2681-2773 and the decode references of
//    tests/test_paged_long_context.py:39-65)
//
// Work split (stream-K style, balanced whatever the context lengths): a
// plan kernel counts each sequence's 32-token tiles, prefix-sums them over
// (sequence, KV head) in that order and fixes the number of active waves
// Ne; a persistent grid of one-wave blocks then gives wave w the tiles
// [floor(w Tt / Ne), floor((w+1) Tt / Ne)) of the Tt in total.  A wave's
// range is cut at (sequence, KV head) boundaries into pieces; each piece is
// walked in tiles of 32 tokens, reading every K/V row once for all G query
// heads that share the KV head (the reference grid (B, Hq) rereads each
// page G times).  Tiles are fetched with coalesced 16-byte loads (one 1 KB
// span per instruction) one tile ahead of the compute and staged in
// wave-private LDS.  Scores are S^T = K Q^T on MFMA with the G query heads
// as columns; the squareplus weights land in the B-operand layout of
// O^T += V^T P^T, and V^T comes from the row-major LDS tile through the
// transposing LDS read (see flash_common.hpp).  Each piece writes its
// unnormalised partial (O, S) into slot k of its (sequence, query head),
// k = its wave minus the wave that owns the segment's first tile; a merge
// kernel sums the slots in order (squareplus needs no running maximum, so
// merging is a plain sum) and divides once.
#include <algorithm>
#include <atomic>
#include <mutex>
#include <type_traits>

#include "flash_common.hpp"

namespace sa {
namespace {

constexpr int kTile = 32;       // tokens per MFMA tile
constexpr int kSplitTok = 512;  // largest minimum of tokens per wave (bounds the pieces per segment)
constexpr int kTargetWaves = 2048;  // about the partial kernel's resident waves (256 CUs x 8)
constexpr int kWinPages = 64;   // page ids held per wave at a time (one per lane)

struct PagedParams {
    const void* q;
    const void* k;
    const void* v;
    bf16* out;
    const int32_t* table;
    const int32_t* ctx;
    int* plan;    // [B + 2]: prefix of Hkv * tiles over sequences (plan[B] = Tt), plan[B + 1] = Ne
    float* ws_o;  // [B][Hq][n_slots][D]
    float* ws_s;  // [B][Hq][n_slots]
    int64_t qs[4], ks[4], vs[4], os[3];
    int64_t bt_stride;
    int B, Hq, Hkv, G, P, logP, max_pages, n_pages, n_slots, n_waves;
    int D;    // head dim (a multiple of 8, at most the kernel's DP)
    int per;  // minimum tiles per active wave
    float scale;
};

// Context length of sequence b as the kernels use it (clamped to the table).
__device__ __forceinline__ int ctx_of(const PagedParams& p, int b) {
    return min(max(p.ctx[b], 0), p.max_pages * p.P);
}

// Plan: plan[b] = sum_{b' < b} Hkv * ceil(ctx_b' / 32) for b <= B (plan[B] =
// Tt, the tiles of all (sequence, KV head) segments), plan[B + 1] = Ne, the
// waves that get work: every wave's range holds at least `per` tiles (so a
// segment of c tokens is cut into at most ceil(c / (32 per)) + 1 pieces),
// and at most n_waves waves run.  One block.
__global__ __launch_bounds__(256) void paged_plan_kernel(PagedParams p) {
    __shared__ int part[256];
    const int tid = threadIdx.x;
    int carry = 0;
    for (int b0 = 0; b0 < p.B; b0 += 256) {
        const int b = b0 + tid;
        const int n = b < p.B ? p.Hkv * ((ctx_of(p, b) + kTile - 1) / kTile) : 0;
        part[tid] = n;
        __syncthreads();
        // inclusive scan of part[] (Hillis-Steele)
        for (int off = 1; off < 256; off <<= 1) {
            const int v = tid >= off ? part[tid - off] : 0;
            __syncthreads();
            part[tid] += v;
            __syncthreads();
        }
        if (b < p.B) p.plan[b] = carry + part[tid] - n;
        carry += part[255];
        __syncthreads();
    }
    if (tid == 0) {
        p.plan[p.B] = carry;
        p.plan[p.B + 1] = carry == 0 ? 0 : max(1, min(p.n_waves, carry / p.per));
    }
}

// Element types of one decode: q (QE) and both caches (CE).  The MFMAs run
// on MT: the 16-bit type itself when q and the caches share it, else bf16,
// with every operand bf16 does not hold exactly split as hi + lo
// (hi = bf16(x), lo = bf16(x - hi), so hi + lo carries 16 significant bits;
// fp16 values split exactly).  With a split operand the fp32 weights are
// split too, and each product becomes the three MFMAs hi*hi + hi*lo + lo*hi:
// about 2^-16 relative error per product, against the reference's fp32
// arithmetic (kernels.py:2716-2717, :2746, :2765).
// e4m3fn cache elements (one byte each).  Every e4m3fn value is a bf16
// value, so fp8 caches widen to bf16 exactly, with no lo part.
struct fp8e4 {
    uint8_t bits;
};

template <typename QE, typename CE>
struct PagedTypes {
    static constexpr bool SAME16 = std::is_same_v<QE, CE> && sizeof(CE) == 2;
    using MT = std::conditional_t<SAME16, CE, bf16>;
    static constexpr bool SPLIT_Q = !std::is_same_v<QE, MT>;
    static constexpr bool SPLIT_C = !std::is_same_v<CE, MT> && !std::is_same_v<CE, fp8e4>;
    static constexpr bool SPLIT_P = !SAME16;
};

// hi = bf16(a), bf16(b) packed; lo = the same of the remainders.
__device__ __forceinline__ void split2_bf16(float a, float b, uint32_t& hi, uint32_t& lo) {
    hi = pack2<bf16>(a, b);
    lo = pack2<bf16>(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xFFFF0000u));
}

// 8 elements of E (one or two 16-byte words, as loaded) as 8 MT values, hi
// and, when SPLIT, lo.
template <typename E, typename MT, bool SPLIT>
__device__ __forceinline__ void to_mt8(const u32x4* w, u32x4& h, u32x4& l) {
    if constexpr (std::is_same_v<E, MT>) {
        h = w[0];
        l = u32x4{0u, 0u, 0u, 0u};
    } else {
        float f[8];
        if constexpr (sizeof(E) == 4) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                f[i] = __uint_as_float(w[0][i]);
                f[4 + i] = __uint_as_float(w[1][i]);
            }
        } else {
            const uint32_t ww[4] = {w[0].x, w[0].y, w[0].z, w[0].w};
#pragma unroll
            for (int i = 0; i < 8; ++i) f[i] = elem<E>(ww, i);
        }
        uint32_t hh[4], ll[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) split2_bf16(f[2 * i], f[2 * i + 1], hh[i], ll[i]);
        h = u32x4{hh[0], hh[1], hh[2], hh[3]};
        l = SPLIT ? u32x4{ll[0], ll[1], ll[2], ll[3]} : u32x4{0u, 0u, 0u, 0u};
    }
}

// The kernels run a padded head dim D (32, 64, 128, 256, 512 or 1024); head dims
// p.D < D (multiples of 8) load only their first p.D columns per row and
// leave zeros in the rest of the LDS rows and Q registers, which add nothing
// to the scores, and write only p.D output columns.
// UNIFORM: every load instruction's tokens lie in one page (the tokens per
// instruction divide the page size), so the page base is wave-uniform and
// comes from v_readlane of the window's page-id register.
// WPB > 1 (cache rows above 512 bytes: 16-bit D = 512 and fp32 D = 256 in
// two parts, fp32 D = 512 in four; head dims above 256 in parts of 256
// columns): a block of WPB waves shares each piece;
// wave v owns columns [v DF / WPB, (v + 1) DF / WPB) of K, V, Q and O, the
// partial S^T tiles meet in LDS (two barriers per tile), and every wave forms
// the same weights.
template <typename QE, typename CE, int DF, bool UNIFORM, int WPB = 1>
__global__ __launch_bounds__(64 * WPB) void paged_partial_kernel(PagedParams p) {
    constexpr int D = DF / WPB;  // columns of this wave
    using Ty = PagedTypes<QE, CE>;
    using T = typename Ty::MT;
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
    constexpr int EPC = 16 / sizeof(CE);   // cache elements per 16-byte chunk
    constexpr int CPT = D / EPC;           // 16-byte chunks per token row
    constexpr int TPI = 64 / CPT;          // tokens per load instruction
    constexpr int NC = kTile * CPT / 64;   // chunks per lane per tile and tensor
    constexpr bool SQ = Ty::SPLIT_Q, SC = Ty::SPLIT_C, SP = Ty::SPLIT_P;
    // MT tiles (one set per wave); the lo parts of split caches in the second pair
    __shared__ __attribute__((aligned(16))) T ldsK_w[WPB][kTile * RS];
    __shared__ __attribute__((aligned(16))) T ldsV_w[WPB][kTile * RSV];
    __shared__ __attribute__((aligned(16))) T ldsKl_w[WPB][SC ? kTile * RS : 8];
    __shared__ __attribute__((aligned(16))) T ldsVl_w[WPB][SC ? kTile * RSV : 8];
    static_assert(WPB == 1 || kTile * RS * sizeof(T) >= 16 * 64 * 4, "a K tile holds a wave's 16 x 64 fp32 scores");

    const int lane = threadIdx.x & 63;
    const int wv = WPB > 1 ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : 0;
    const int col_base = wv * D;  // first column of this wave
    T* const ldsK = ldsK_w[wv];
    T* const ldsV = ldsV_w[wv];
    T* const ldsKl = ldsKl_w[wv];
    T* const ldsVl = ldsVl_w[wv];
    const int hi = lane >> 5;
    const int l32 = lane & 31;
    const int w = blockIdx.x;
    const int Tt = p.plan[p.B];
    const int Ne = p.plan[p.B + 1];
    if (w >= Ne) return;  // no work for this wave (tiny problems)
    const int x_end = static_cast<int>(static_cast<int64_t>(w + 1) * Tt / Ne);
    int x = static_cast<int>(static_cast<int64_t>(w) * Tt / Ne);
    const int logP = p.logP;
    const int pmask = p.P - 1;

    // Sequence b of tile x: the last b with plan[b] <= x (plan[b] ascending).
    int b = 0;
    for (int b0 = 0; b0 < p.B; b0 += 64) {
        const int bi = b0 + lane;
        const bool le = bi < p.B && p.plan[bi] <= x;
        const unsigned long long m = __ballot(le);
        if (m == 0) break;
        b = b0 + 63 - __builtin_clzll(m);
    }

    while (x < x_end) {
        // Segment (b, hk) holding tile x; skip sequences with no tiles.
        while (p.plan[b + 1] <= x) ++b;
        const int seg0 = p.plan[b];
        const int n_b = (p.plan[b + 1] - seg0) / p.Hkv;  // tiles per KV head of b
        const int rel = x - seg0;
        const int hk = rel / n_b;
        const int seg_start = seg0 + hk * n_b;
        const int piece_end = min(x_end, seg_start + n_b);
        const int ctx = ctx_of(p, b);
        const int t_begin = (x - seg_start) * kTile;
        const int t_end = min(ctx, (piece_end - seg_start) * kTile);
        // slot: this wave minus the owner of the segment's first tile
        const int owner0 = static_cast<int>((static_cast<int64_t>(seg_start + 1) * Ne - 1) / Tt);
        const int slot_k = w - owner0;

        const CE* kc = static_cast<const CE*>(p.k) + hk * p.ks[1];
        const CE* vc = static_cast<const CE*>(p.v) + hk * p.vs[1];
        const int32_t* trow = p.table + b * p.bt_stride;

        // Q^T as the B operand: column = query head hk*G + l32 (zero past G);
        // qlo holds the lo parts when q is split.
        u32x4 qreg[D / 16], qlo[SQ ? D / 16 : 1];
        {
            const bool live = l32 < p.G;
            const QE* qrow = static_cast<const QE*>(p.q) + b * p.qs[0] + (hk * p.G + (live ? l32 : 0)) * p.qs[1];
#pragma unroll
            for (int dc = 0; dc < D / 16; ++dc) {
                const int d0 = col_base + dc * 16 + hi * 8;
                u32x4 w[2] = {u32x4{0u, 0u, 0u, 0u}, u32x4{0u, 0u, 0u, 0u}};
                if (live && d0 < p.D) {
                    w[0] = load16(qrow + d0);
                    if constexpr (sizeof(QE) == 4) w[1] = load16(qrow + d0 + 4);
                }
                u32x4 l;
                to_mt8<QE, T, SQ>(w, qreg[dc], l);
                if constexpr (SQ) qlo[dc] = l;
            }
        }

        f32x16 oacc[D / 32];
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) oacc[dt] = f32x16{};
        float ssum = 0.f;
        const int v_tr_off = ((lane >> 5) * 4 + ((lane & 15) >> 2)) * RSV + ((lane >> 4) & 1) * 16 + 4 * (lane & 3);

        // The piece in windows of whole tiles whose pages fit kWinPages.
        for (int ws = t_begin; ws < t_end;) {
            const int first_page = ws >> logP;
            const int we = min(t_end, ws + ((((first_page + kWinPages) << logP) - ws) & ~(kTile - 1)));
            int page_id;
            {
                const int npg = ((we - 1) >> logP) - first_page + 1;
                page_id = lane < npg ? min(max(trow[first_page + lane], 0), p.n_pages - 1) : 0;
            }

            // Coalesced tile loads: instruction i of lane l fetches 16-byte chunk
            // c = 64 i + l of the tile (token c / CPT, columns EPC (c % CPT) ..
            // + EPC - 1).
            const int lane_tok = lane / CPT;
            const int lane_col = (lane % CPT) * EPC;
            const bool col_live = col_base + lane_col < p.D;  // columns past the head dim stay zero
            u32x4 kbuf[NC], vbuf[NC];
            auto load_tile = [&](int t0) {
#pragma unroll
                for (int i = 0; i < NC; ++i) {
                    const int t = t0 + i * TPI + lane_tok;
                    int phys;
                    int64_t koff, voff;
                    if constexpr (UNIFORM) {
                        const int tu = t0 + i * TPI;  // first token of the instruction
                        phys = __builtin_amdgcn_readlane(page_id, min((tu >> logP) - first_page, kWinPages - 1));
                        const int r = tu & pmask;
                        koff = phys * p.ks[0] + (r + lane_tok) * p.ks[2];
                        voff = phys * p.vs[0] + (r + lane_tok) * p.vs[2];
                    } else {
                        phys = __shfl(page_id, min((t >> logP) - first_page, kWinPages - 1));
                        koff = phys * p.ks[0] + (t & pmask) * p.ks[2];
                        voff = phys * p.vs[0] + (t & pmask) * p.vs[2];
                    }
                    if (t < we && col_live) {
                        kbuf[i] = load16(kc + koff + col_base + lane_col);
                        vbuf[i] = load16(vc + voff + col_base + lane_col);
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
                    if constexpr (std::is_same_v<CE, fp8e4>) {
                        // 16 e4m3fn values -> 16 bf16 (32 bytes)
                        u32x4 a, c;
                        widen_e4m3x16<bf16>(kbuf[i], a, c);
                        *reinterpret_cast<u32x4*>(ldsK + tok * RS + lane_col) = a;
                        *reinterpret_cast<u32x4*>(ldsK + tok * RS + lane_col + 8) = c;
                        widen_e4m3x16<bf16>(vbuf[i], a, c);
                        *reinterpret_cast<u32x4*>(ldsV + tok * RSV + lane_col) = a;
                        *reinterpret_cast<u32x4*>(ldsV + tok * RSV + lane_col + 8) = c;
                    } else if constexpr (!SC) {
                        *reinterpret_cast<u32x4*>(ldsK + tok * RS + lane_col) = kbuf[i];
                        *reinterpret_cast<u32x4*>(ldsV + tok * RSV + lane_col) = vbuf[i];
                    } else if constexpr (sizeof(CE) == 4) {
                        // 4 fp32 values -> 4 hi + 4 lo bf16 (8 bytes each)
                        uint32_t kh[2], kl[2], vh[2], vl[2];
#pragma unroll
                        for (int j = 0; j < 2; ++j) {
                            split2_bf16(__uint_as_float(kbuf[i][2 * j]), __uint_as_float(kbuf[i][2 * j + 1]), kh[j],
                                        kl[j]);
                            split2_bf16(__uint_as_float(vbuf[i][2 * j]), __uint_as_float(vbuf[i][2 * j + 1]), vh[j],
                                        vl[j]);
                        }
                        *reinterpret_cast<uint2*>(ldsK + tok * RS + lane_col) = uint2{kh[0], kh[1]};
                        *reinterpret_cast<uint2*>(ldsKl + tok * RS + lane_col) = uint2{kl[0], kl[1]};
                        *reinterpret_cast<uint2*>(ldsV + tok * RSV + lane_col) = uint2{vh[0], vh[1]};
                        *reinterpret_cast<uint2*>(ldsVl + tok * RSV + lane_col) = uint2{vl[0], vl[1]};
                    } else {
                        // 8 fp16 values -> 8 hi + 8 lo bf16 (exact)
                        u32x4 h, l;
                        to_mt8<CE, T, true>(&kbuf[i], h, l);
                        *reinterpret_cast<u32x4*>(ldsK + tok * RS + lane_col) = h;
                        *reinterpret_cast<u32x4*>(ldsKl + tok * RS + lane_col) = l;
                        to_mt8<CE, T, true>(&vbuf[i], h, l);
                        *reinterpret_cast<u32x4*>(ldsV + tok * RSV + lane_col) = h;
                        *reinterpret_cast<u32x4*>(ldsVl + tok * RSV + lane_col) = l;
                    }
                }
            };

            load_tile(ws);
            for (int t0 = ws; t0 < we; t0 += kTile) {
                // The block is one wavefront: LDS accesses of a wave complete
                // in issue order, so a wave-level scheduling barrier is all
                // the ordering needed.
                store_tile();
                __builtin_amdgcn_wave_barrier();
                if (t0 + kTile < we) load_tile(t0 + kTile);

                f32x16 s = f32x16{};
#pragma unroll
                for (int dc = 0; dc < D / 16; ++dc) {
                    const u32x4 a = *reinterpret_cast<const u32x4*>(ldsK + l32 * RS + dc * 16 + hi * 8);
                    s = Ops::mma(as_vec8<Vec>(a), as_vec8<Vec>(qreg[dc]), s);
                    if constexpr (SQ) s = Ops::mma(as_vec8<Vec>(a), as_vec8<Vec>(qlo[dc]), s);
                    if constexpr (SC) {
                        const u32x4 al = *reinterpret_cast<const u32x4*>(ldsKl + l32 * RS + dc * 16 + hi * 8);
                        s = Ops::mma(as_vec8<Vec>(al), as_vec8<Vec>(qreg[dc]), s);
                    }
                }
                if constexpr (WPB > 1) {
                    // Add the other waves' partial scores (their columns of
                    // q . k), exchanged through each wave's K tile, which the
                    // S^T MFMAs above have finished reading (LDS operations of
                    // a wave complete in order; the memory clobber keeps the
                    // compiler from moving these stores above those reads).
                    // The second barrier keeps the next tile's K stores after
                    // the other waves' reads.
                    asm volatile("" ::: "memory");
                    uint32_t* mine = reinterpret_cast<uint32_t*>(ldsK);
#pragma unroll
                    for (int v = 0; v < 16; ++v) mine[v * 64 + lane] = __float_as_uint(s[v]);
                    __syncthreads();
#pragma unroll
                    for (int o = 1; o < WPB; ++o) {
                        const uint32_t* other = reinterpret_cast<const uint32_t*>(ldsK_w[(wv + o) % WPB]);
#pragma unroll
                        for (int v = 0; v < 16; ++v) s[v] += __uint_as_float(other[v * 64 + lane]);
                    }
                    __syncthreads();
                }
                float y[16];
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int t = t0 + (v >> 2) * 8 + hi * 4 + (v & 3);
                    const float wgt = sp2_weight<false>(__builtin_fmaf(s[v], p.scale, -0.5f));
                    y[v] = t < we ? wgt : 0.f;
                    ssum += y[v];
                }
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    uint32_t ph[4], plo[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        if constexpr (SP)
                            split2_bf16(y[8 * c + 2 * j], y[8 * c + 2 * j + 1], ph[j], plo[j]);
                        else
                            ph[j] = pack2<T>(y[8 * c + 2 * j], y[8 * c + 2 * j + 1]);
                    }
                    const u32x4 pw{ph[0], ph[1], ph[2], ph[3]};
                    const u32x4 pl = SP ? u32x4{plo[0], plo[1], plo[2], plo[3]} : u32x4{0u, 0u, 0u, 0u};
                    const Vec bop = as_vec8<Vec>(pw);
#pragma unroll
                    for (int dt = 0; dt < D / 32; ++dt) {
                        const T* base = ldsV + (16 * c) * RSV + dt * 32 + v_tr_off;
                        const uint2 lo = lds_read_tr16(base);
                        const uint2 hi8 = lds_read_tr16(base + 8 * RSV);
                        const u32x4 aw{lo.x, lo.y, hi8.x, hi8.y};
                        oacc[dt] = Ops::mma(as_vec8<Vec>(aw), bop, oacc[dt]);
                        if constexpr (SP) oacc[dt] = Ops::mma(as_vec8<Vec>(aw), as_vec8<Vec>(pl), oacc[dt]);
                        if constexpr (SC) {
                            const T* basel = ldsVl + (16 * c) * RSV + dt * 32 + v_tr_off;
                            const uint2 lol = lds_read_tr16(basel);
                            const uint2 hil = lds_read_tr16(basel + 8 * RSV);
                            const u32x4 awl{lol.x, lol.y, hil.x, hil.y};
                            oacc[dt] = Ops::mma(as_vec8<Vec>(awl), bop, oacc[dt]);
                        }
                    }
                }
                __builtin_amdgcn_wave_barrier();
            }
            ws = we;
        }

        const float stot = ssum + __shfl_xor(ssum, 32);
        if (l32 < p.G) {
            const int hq = hk * p.G + l32;
            const int64_t slot = (static_cast<int64_t>(b) * p.Hq + hq) * p.n_slots + slot_k;
            float* wo = p.ws_o + slot * p.D;
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
                for (int vg = 0; vg < 4; ++vg) {
                    const int d0 = col_base + dt * 32 + vg * 8 + hi * 4;
                    if (d0 < p.D)  // p.D is a multiple of 8: groups of 4 are wholly in or out
                        *reinterpret_cast<float4*>(wo + d0) = float4{oacc[dt][vg * 4 + 0], oacc[dt][vg * 4 + 1],
                                                                     oacc[dt][vg * 4 + 2], oacc[dt][vg * 4 + 3]};
                }
            }
            if (hi == 0 && wv == 0) p.ws_s[slot] = stot;
        }
        x = piece_end;
    }
}

// Sum the piece partials of one (b, query head) in slot order, then divide
// (an empty context gives 0 / eps = 0).
template <int D>
__global__ __launch_bounds__(D) void paged_merge_kernel(PagedParams p) {
    const int bh = blockIdx.x;
    const int b = bh / p.Hq;
    const int hq = bh - b * p.Hq;
    const int hk = hq / p.G;
    const int d = threadIdx.x;
    const int Tt = p.plan[p.B];
    const int Ne = p.plan[p.B + 1];
    const int seg0 = p.plan[b];
    const int n_b = (p.plan[b + 1] - seg0) / p.Hkv;
    float o = 0.f, s = 0.f;
    if (n_b > 0) {
        const int first = seg0 + hk * n_b, last = first + n_b - 1;
        const int w0 = static_cast<int>((static_cast<int64_t>(first + 1) * Ne - 1) / Tt);
        const int w1 = static_cast<int>((static_cast<int64_t>(last + 1) * Ne - 1) / Tt);
        const int64_t slot0 = static_cast<int64_t>(bh) * p.n_slots;
        for (int i = 0; i <= w1 - w0; ++i) {
            o += p.ws_o[(slot0 + i) * p.D + d];
            s += p.ws_s[slot0 + i];
        }
    }
    p.out[b * p.os[0] + hq * p.os[1] + d * p.os[2]] = static_cast<bf16>(o / (s + kEps));
}

// Blocks of paged_partial_kernel<QE, CE, D, U, WPB> resident on the device at
// once (the persistent grid), per device.
template <typename QE, typename CE, int D, bool U, int WPB>
int resident_waves() {
    static int cache[16] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
    const int slot = dev < 16 ? dev : 15;
    if (cache[slot] == 0) {
        int cus = 0, per_cu = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, paged_partial_kernel<QE, CE, D, U, WPB>, 64 * WPB,
                                                         0) !=
                hipSuccess ||
            per_cu <= 0)
            per_cu = 1;
        cache[slot] = cus * per_cu;
    }
    return cache[slot];
}

template <typename QE, typename CE, int D>
int launch_paged(PagedParams prm, hipStream_t st) {
    // waves per block, each owning D / WPB columns: rows above 512 bytes are
    // split into 512-byte parts (their tile registers would not fit one wave)
    // and no wave owns more than 256 columns (Q and O registers)
    constexpr int RB = D * static_cast<int>(sizeof(CE));
    constexpr int WPB_B = RB > 1024 ? 4 : (RB > 512 || D > 256) ? 2 : 1;
    constexpr int WPB = D / WPB_B > 256 ? D / 256 : WPB_B;
    const bool uniform = prm.P * (D / WPB * static_cast<int>(sizeof(CE)) / 16) >= 64;
    const int resident =
        uniform ? resident_waves<QE, CE, D, true, WPB>() : resident_waves<QE, CE, D, false, WPB>();
    // The plan gives work to at most Tt / per waves, and Tt is at most
    // B * Hkv * ceil(max_pages * P / kTile): no more waves are launched.
    const int64_t max_tiles = static_cast<int64_t>(prm.B) * prm.Hkv *
                              ((static_cast<int64_t>(prm.max_pages) * prm.P + kTile - 1) / kTile);
    prm.n_waves = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(resident, max_tiles / prm.per)));
    paged_plan_kernel<<<1, 256, 0, st>>>(prm);
    if (uniform)
        paged_partial_kernel<QE, CE, D, true, WPB><<<prm.n_waves, 64 * WPB, 0, st>>>(prm);
    else
        paged_partial_kernel<QE, CE, D, false, WPB><<<prm.n_waves, 64 * WPB, 0, st>>>(prm);
    paged_merge_kernel<D><<<static_cast<unsigned>(prm.B) * prm.Hq, prm.D, 0, st>>>(prm);
    return status_from_launch();
}

template <typename QE, typename CE>
int launch_paged_d(int dp, const PagedParams& prm, hipStream_t st) {
    switch (dp) {
        case 32: return launch_paged<QE, CE, 32>(prm, st);
        case 64: return launch_paged<QE, CE, 64>(prm, st);
        case 128: return launch_paged<QE, CE, 128>(prm, st);
        case 256: return launch_paged<QE, CE, 256>(prm, st);
        case 512: return launch_paged<QE, CE, 512>(prm, st);
        default:
            // 1024: four waves of 256 columns; caches split into hi and lo
            // tiles would need twice the LDS (refused by validate_paged)
            if constexpr (!PagedTypes<QE, CE>::SPLIT_C) return launch_paged<QE, CE, 1024>(prm, st);
            else return SA_ERR_UNSUPPORTED;
    }
}

// Minimum tiles per active wave: kSplitTok / kTile (few pieces, few
// partials to merge) when the work fills the device, down to 1 for small
// batches, so that their tiles spread over up to kTargetWaves waves instead
// of queueing on a few: clamp(n_segments * max_tiles / kTargetWaves, 1, 16).
int split_for(int64_t segments, int max_pages, int page_size) {
    const int64_t toks = static_cast<int64_t>(max_pages) * page_size;
    const int64_t ub = segments * ((toks + kTile - 1) / kTile);
    return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(kSplitTok / kTile, ub / kTargetWaves)));
}
// The workspace is sized for the split with B * ceil(Hq / 8) segments (KV
// groups of up to 8 query heads); the launch takes the larger of that and
// the split its B * Hkv segments give, so its partial slots always fit.
int split_floor(int B, int Hq, int max_pages, int page_size) {
    return split_for(static_cast<int64_t>(B) * ((Hq + 7) / 8), max_pages, page_size);
}

// Partial slots per (sequence, query head): a segment of c tokens meets at
// most ceil(c / (kTile per)) + 1 waves.
int64_t slots_for(int max_pages, int page_size, int per) {
    const int64_t toks = static_cast<int64_t>(max_pages) * page_size;
    const int64_t span = static_cast<int64_t>(per) * kTile;
    return (toks <= 0 ? 1 : (toks + span - 1) / span) + 1;
}

// Workspace layout: plan (B + 2 int32, padded to 16 bytes), then the O and S
// partials (fp32).
int64_t plan_bytes(int B) { return ((static_cast<int64_t>(B) + 2) * 4 + 15) / 16 * 16; }

int64_t workspace_bytes_for(int B, int Hq, int D, int max_pages, int page_size, int per) {
    const int64_t slots = static_cast<int64_t>(B) * Hq * slots_for(max_pages, page_size, per);
    return plan_bytes(B) + slots * (D + 1) * static_cast<int64_t>(sizeof(float));
}

// The minimum tiles per active wave a launch uses: the workspace is sized
// for split_floor, and the launch takes the larger split its B * Hkv
// segments give (so its slots always fit).
int launch_per(int B, int Hq, int Hkv, int max_pages, int page_size) {
    return std::max(split_floor(B, Hq, max_pages, page_size),
                    split_for(static_cast<int64_t>(B) * Hkv, max_pages, page_size));
}

// q and cache types of a decode's dtype argument (SA_PAGED_DTYPES, or one
// code for both); false for unsupported pairs.  Supported: bf16 / bf16,
// fp16 / fp16, fp32 q over fp32, bf16, fp16 or e4m3fn caches, and bf16 q
// over e4m3fn caches (q is then a plain bf16 operand, no lo part).
bool paged_types(int dtype, int& qt, int& ct) {
    qt = dtype & 0xFF;
    ct = (dtype >> 8) == 0 ? qt : (dtype >> 8) - 1;
    if (dtype < 0 || (dtype >> 16) != 0) return false;
    if (qt == ct) return qt == SA_BF16 || qt == SA_F16 || qt == SA_F32;
    if (qt == SA_BF16) return ct == SA_FP8_E4M3FN;
    return qt == SA_F32 && (ct == SA_BF16 || ct == SA_F16 || ct == SA_FP8_E4M3FN);
}

// Argument checks shared by both decode entry points (0 = launch, 1 =
// nothing to do, < 0 = status).  max_pages becomes 0 when there are no pages.
int validate_paged(const void* q, const void* k_cache, const void* v_cache, const void* out,
                   const int32_t* block_table, const int32_t* context_lens, int B, int Hq, int Hkv, int D,
                   int page_size, int& max_pages, int n_pages, const int64_t* q_strides,
                   const int64_t* kv_strides, const int64_t* vv_strides, const int64_t* o_strides, int dtype) {
    if (B < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || max_pages < 0 || n_pages < 0) return SA_ERR_BAD_SHAPE;
    if (Hq / Hkv > 32) return SA_ERR_UNSUPPORTED;  // query heads per KV head fill one 32-wide MFMA column block
    // any power of two: a tile of 32 tokens spans 32 / P pages (P < 32) or
    // lies in one page; a window of 64 page ids always covers whole tiles
    if (page_size <= 0 || (page_size & (page_size - 1)) != 0 || page_size > (1 << 20)) return SA_ERR_UNSUPPORTED;
    if (D < 8 || D > 1024 || D % 8 != 0) return SA_ERR_UNSUPPORTED;
    if (B == 0) return 1;
    if (n_pages == 0) max_pages = 0;  // no cache: every context is empty
    // The plan keeps token positions, tile counts and their prefix sums over
    // (sequence, KV head) in 32-bit ints.
    const int64_t max_ctx = static_cast<int64_t>(max_pages) * page_size;
    if (max_ctx > INT32_MAX / 2 || static_cast<int64_t>(B) * Hkv * ((max_ctx + kTile - 1) / kTile) > INT32_MAX / 2)
        return SA_ERR_UNSUPPORTED;
    if (!q || !k_cache || !v_cache || !out || !block_table || !context_lens || !q_strides || !kv_strides ||
        !vv_strides || !o_strides)
        return SA_ERR_NULL_POINTER;
    int qt, ct;
    if (!paged_types(dtype, qt, ct)) return SA_ERR_BAD_DTYPE;
    if (ct == SA_FP8_E4M3FN && D % 16 != 0) return SA_ERR_UNSUPPORTED;  // 16-byte rows of 1-byte elements
    // head dims above 512 run on 4 waves of 256 columns; caches read as
    // bf16 hi + lo tiles (fp32, or fp16 under an fp32 q) would need twice
    // the LDS of one block
    if (D > 512 && (ct == SA_F32 || (qt == SA_F32 && ct == SA_F16))) return SA_ERR_UNSUPPORTED;
    // 16-byte rows: element strides that are multiples of 16 / element size
    const auto ok16 = [](const int64_t* s, int n, int t) {
        const int per = t == SA_F32 ? 4 : t == SA_FP8_E4M3FN ? 16 : 8;
        for (int i = 0; i < n - 1; ++i)
            if (s[i] % per != 0) return false;
        return s[n - 1] == 1;
    };
    if (!ok16(q_strides, 4, qt) || !ok16(kv_strides, 4, ct) || !ok16(vv_strides, 4, ct) || o_strides[2] != 1 ||
        !aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache))
        return SA_ERR_BAD_STRIDE;
    return 0;
}

// Plan, partial and merge launches with the workspace at `ws` (laid out for
// `per` minimum tiles per wave).
int run_paged(const void* q, const void* k_cache, const void* v_cache, void* out, const int32_t* block_table,
              const int32_t* context_lens, int B, int Hq, int Hkv, int D, int page_size, int max_pages,
              int n_pages, const int64_t* q_strides, const int64_t* kv_strides, const int64_t* vv_strides,
              const int64_t* o_strides, int64_t bt_stride, float scale, int dtype, float* ws, int per,
              hipStream_t st) {
    PagedParams prm{};
    prm.q = q;
    prm.k = k_cache;
    prm.v = v_cache;
    prm.out = static_cast<bf16*>(out);
    prm.table = block_table;
    prm.ctx = context_lens;
    prm.per = per;
    prm.n_slots = static_cast<int>(slots_for(max_pages, page_size, per));
    prm.plan = reinterpret_cast<int*>(ws);
    prm.ws_o = ws + plan_bytes(B) / 4;
    prm.ws_s = prm.ws_o + static_cast<int64_t>(B) * Hq * prm.n_slots * D;
    prm.D = D;
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
    // padded head dim of the kernels
    const int dp = D <= 32 ? 32 : D <= 64 ? 64 : D <= 128 ? 128 : D <= 256 ? 256 : D <= 512 ? 512 : 1024;
    int qt, ct;
    paged_types(dtype, qt, ct);
    if (qt == SA_BF16 && ct == SA_FP8_E4M3FN) return launch_paged_d<bf16, fp8e4>(dp, prm, st);
    if (qt == SA_BF16) return launch_paged_d<bf16, bf16>(dp, prm, st);
    if (qt == SA_F16) return launch_paged_d<f16, f16>(dp, prm, st);
    if (ct == SA_BF16) return launch_paged_d<float, bf16>(dp, prm, st);
    if (ct == SA_FP8_E4M3FN) return launch_paged_d<float, fp8e4>(dp, prm, st);
    if (ct == SA_F16) return launch_paged_d<float, f16>(dp, prm, st);
    return launch_paged_d<float, float>(dp, prm, st);
}

}  // namespace
}  // namespace sa

extern "C" int64_t sa_paged_decode_workspace_size(int B, int Hq, int D, int max_pages, int page_size) {
    if (B <= 0 || Hq <= 0 || D <= 0 || max_pages < 0 || page_size <= 0) return 0;
    return sa::workspace_bytes_for(B, Hq, D, max_pages, page_size, sa::split_floor(B, Hq, max_pages, page_size));
}

extern "C" int sa_paged_decode(const void* q, const void* k_cache, const void* v_cache, void* out,
                               const int32_t* block_table, const int32_t* context_lens, int B, int Hq, int Hkv,
                               int D, int page_size, int max_pages, int n_pages, const int64_t* q_strides,
                               const int64_t* kv_strides, const int64_t* vv_strides, const int64_t* o_strides,
                               int64_t bt_stride, float scale, int dtype, float* workspace, int64_t workspace_bytes,
                               sa_stream_t stream) {
    using namespace sa;
    const int chk = validate_paged(q, k_cache, v_cache, out, block_table, context_lens, B, Hq, Hkv, D, page_size,
                                   max_pages, n_pages, q_strides, kv_strides, vv_strides, o_strides, dtype);
    if (chk != 0) return chk > 0 ? 0 : chk;
    if (!workspace) return SA_ERR_NULL_POINTER;
    if (workspace_bytes < sa_paged_decode_workspace_size(B, Hq, D, max_pages, page_size)) return SA_ERR_WORKSPACE;
    return run_paged(q, k_cache, v_cache, out, block_table, context_lens, B, Hq, Hkv, D, page_size, max_pages,
                     n_pages, q_strides, kv_strides, vv_strides, o_strides, bt_stride, scale, dtype, workspace,
                     launch_per(B, Hq, Hkv, max_pages, page_size), reinterpret_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------------
// Allocation-free decode.  The plan and partials live in `scratch`, a
// module-scope device array: each device that loads this library holds its
// own copy (SA_PAGED_NOALLOC_SCRATCH_BYTES) until the process ends.  In host
// code the array's name is only a host-side stand-in, so its device address
// is looked up once per device with hipGetSymbolAddress (with that device
// current) and that address is what the kernels receive.
// ---------------------------------------------------------------------------
static __device__ __align__(256) float scratch[SA_PAGED_NOALLOC_SCRATCH_BYTES / sizeof(float)];

namespace sa {
namespace {

constexpr int kMaxDevices = 64;
std::atomic<float*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

// The current device's copy of `scratch` (0 = ok, else a status).
int scratch_of_current_device(float** out) {
    int dev = -1;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return static_cast<int>(e);
    if (dev < 0 || dev >= kMaxDevices) return SA_ERR_UNSUPPORTED;
    float* p = g_scratch[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch[dev].load(std::memory_order_relaxed);
        if (p == nullptr) {
            void* addr = nullptr;
            const hipError_t es = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
            if (es != hipSuccess) return static_cast<int>(es);
            if (addr == nullptr) return SA_ERR_WORKSPACE;
            p = static_cast<float*>(addr);
            g_scratch[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return 0;
}

}  // namespace
}  // namespace sa

extern "C" int sa_paged_decode_noalloc(const void* q, const void* k_cache, const void* v_cache, void* out,
                                       const int32_t* block_table, const int32_t* context_lens, int B, int Hq,
                                       int Hkv, int D, int page_size, int max_pages, int n_pages,
                                       const int64_t* q_strides, const int64_t* kv_strides,
                                       const int64_t* vv_strides, const int64_t* o_strides, int64_t bt_stride,
                                       float scale, int dtype, sa_stream_t stream) {
    using namespace sa;
    const int chk = validate_paged(q, k_cache, v_cache, out, block_table, context_lens, B, Hq, Hkv, D, page_size,
                                   max_pages, n_pages, q_strides, kv_strides, vv_strides, o_strides, dtype);
    if (chk != 0) return chk > 0 ? 0 : chk;
    // The workspace launch's split, or a coarser one (more tiles per wave,
    // fewer partial slots) when its partials would not fit the scratch: the
    // plan honours any per, which only caps how many waves share the work.
    int per = launch_per(B, Hq, Hkv, max_pages, page_size);
    constexpr int64_t cap = SA_PAGED_NOALLOC_SCRATCH_BYTES;
    while (workspace_bytes_for(B, Hq, D, max_pages, page_size, per) > cap &&
           slots_for(max_pages, page_size, per) > 2)
        per *= 2;
    if (workspace_bytes_for(B, Hq, D, max_pages, page_size, per) > cap) return SA_ERR_WORKSPACE;
    float* ws = nullptr;
    const int sst = scratch_of_current_device(&ws);
    if (sst != 0) return sst;
    return run_paged(q, k_cache, v_cache, out, block_table, context_lens, B, Hq, Hkv, D, page_size, max_pages,
                     n_pages, q_strides, kv_strides, vv_strides, o_strides, bt_stride, scale, dtype, ws, per,
                     reinterpret_cast<hipStream_t>(stream));
}
