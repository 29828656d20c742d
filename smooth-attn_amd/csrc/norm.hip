// Row-wise and causal squareplus normalisation, forward and fused backward.
//
// One wavefront per row.  A row is read once with 16-byte nontemporal loads
// (lane l owns columns [(c*64 + l)*VEC, +VEC) for chunk c), held in registers,
// reduced across the wave with DPP, and written once with 16-byte
// nontemporal stores.  Causal rows skip every chunk past the diagonal on the
// read side and stream zeros for it on the write side, so HBM traffic is the
// causal triangle read plus the full row written.
//
// Reference semantics: kernels.py:494-531 (row-wise), :565-676 (causal
// forward, all variants), :679-849 (causal backward, all variants).
//
// Arithmetic.  With a = alpha (x - theta), r = sqrt(a^2 + 4) and t = a + r,
// squareplus(a) = t / 2, so y = squareplus(a)^p = t^p / 2^p.  The kernels
// work with w = t^p and fold 2^p into the epsilon: y / (sum y + 1e-12) =
// w / (sum w + 2^p 1e-12).  For the backward, d squareplus/da =
// squareplus(a) / r, hence dy/dx = alpha p y / r and
//   dx = (alpha p / S') * (w / r) * (dy - T),  S' = sum w + 2^p eps,
//   T = sum(dy w) / S'.

#include "common.hpp"

namespace sa {
namespace {

constexpr int kWavesPerBlock = 4;

// Minimum waves per SIMD requested from the register allocator, from the
// number of 32-bit values a lane keeps live per row (HBM-bound kernels want
// occupancy; each SIMD has 512 VGPRs per lane).
constexpr int waves_for_live(int live) {
    return live <= 48 ? 8 : live <= 72 ? 6 : live <= 96 ? 5 : live <= 112 ? 4 : live <= 160 ? 3 : live <= 224 ? 2 : 1;
}
template <typename T, int NCH>
constexpr int fwd_waves() {
    // raw words + fp32 weights
    return waves_for_live(NCH * 4 + NCH * (16 / static_cast<int>(sizeof(T))));
}
template <typename T, typename TG, int NCH>
constexpr int bwd_waves() {
    constexpr int vec = 16 / static_cast<int>(sizeof(T));
    // dy words + one fp32 array + (on average) half of the x words
    return waves_for_live(NCH * 2 + NCH * vec * static_cast<int>(sizeof(TG)) / 4 + NCH * vec);
}

template <int POWER>
__device__ __forceinline__ float power_of(float t) {
    if constexpr (POWER == 1) return t;
    if constexpr (POWER == 2) return t * t;
    return t * t * t;
}

// Row handled by wave `w`: rows in storage order.  Consecutive waves then
// touch consecutive rows, so the rows in flight at any moment form one dense
// address window, which HBM serves markedly faster (about 15% on the causal
// backward) than the same rows spread over every matrix of a batch.
__device__ __forceinline__ void row_of_wave(int64_t w, int n_cols, bool causal, int64_t& row, int& qpos) {
    row = w;
    qpos = causal ? static_cast<int>(w % n_cols) : n_cols - 1;
}

// ---------------------------------------------------------------------------
// Vectorised kernels (rows 16-byte aligned, n_cols a multiple of VEC).
// ---------------------------------------------------------------------------
template <typename T, int NCH, int POWER>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(fwd_waves<T, NCH>(), 8))) void norm_fwd_vec(const T* __restrict__ x, T* __restrict__ y,
                                                    int64_t n_rows, int n_cols, int64_t xs,
                                                    int64_t ys, int causal, float alpha,
                                                    float neg_alpha_theta, float eps_scaled) {
    constexpr int VEC = 16 / sizeof(T);
    const int lane = threadIdx.x & 63;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
    if (wave >= n_rows) return;
    int64_t row;
    int qpos;
    row_of_wave(wave, n_cols, causal != 0, row, qpos);
    const int limit = qpos + 1;
    const T* xr = x + row * xs;
    T* yr = y + row * ys;

    // Loads and arithmetic run under wave-uniform per-chunk branches (a chunk
    // wholly past the diagonal is skipped by every lane).  Inside the chunk
    // that straddles the diagonal, lanes past it re-read the row's first
    // 16 bytes (in bounds, same cache line for the whole wave) and their
    // values are discarded by the per-element selects below.
    uint32_t raw[NCH][4];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int col0 = (c * 64 + lane) * VEC;
        if (c * 64 * VEC < limit) {
            load_words(xr + (col0 < limit ? col0 : 0), raw[c]);
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) raw[c][k] = 0u;
        }
    }

    float w[NCH][VEC];
    float part = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int col0 = (c * 64 + lane) * VEC;
#pragma unroll
        for (int e = 0; e < VEC; ++e) w[c][e] = 0.f;
        if (c * 64 * VEC < limit) {
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const float a = __builtin_fmaf(alpha, elem<T>(raw[c], e), neg_alpha_theta);
                const float t = a + fast_sqrt(__builtin_fmaf(a, a, 4.f));
                const float wv = (col0 + e <= qpos) ? power_of<POWER>(t) : 0.f;
                w[c][e] = wv;
                part += wv;
            }
        }
    }
    const float inv = 1.f / (wave_sum(part) + eps_scaled);

#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int col0 = (c * 64 + lane) * VEC;
        if (col0 < n_cols) {
            float ov[VEC];
#pragma unroll
            for (int e = 0; e < VEC; ++e) ov[e] = w[c][e] * inv;
            uint32_t packed[4];
            pack_row16<T>(ov, packed);
            store_words(yr + col0, packed);
        }
    }
}

template <typename T, typename TG, int NCH, int POWER>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(bwd_waves<T, TG, NCH>(), 8))) void norm_bwd_vec(const T* __restrict__ x, const TG* __restrict__ dy,
                                                    T* __restrict__ dx, int64_t n_rows, int n_cols,
                                                    int64_t xs, int64_t gs, int64_t dxs, int causal,
                                                    float alpha, float neg_alpha_theta,
                                                    float eps_scaled) {
    constexpr int VEC = 16 / sizeof(T);
    constexpr int GW = (VEC * static_cast<int>(sizeof(TG))) / 16;  // 16-byte words of dy per chunk
    const int lane = threadIdx.x & 63;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
    if (wave >= n_rows) return;
    int64_t row;
    int qpos;
    row_of_wave(wave, n_cols, causal != 0, row, qpos);
    const int limit = qpos + 1;
    const T* xr = x + row * xs;
    const TG* gr = dy + row * gs;
    T* dxr = dx + row * dxs;

    uint32_t rx[NCH][4];
    uint32_t rg[NCH][4 * GW];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int col0 = (c * 64 + lane) * VEC;
        if (c * 64 * VEC < limit) {
            const int off = col0 < limit ? col0 : 0;
            load_words(xr + off, rx[c]);
#pragma unroll
            for (int k = 0; k < GW; ++k) load_words(gr + off + k * (16 / sizeof(TG)), &rg[c][4 * k]);
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) rx[c][k] = 0u;
#pragma unroll
            for (int k = 0; k < 4 * GW; ++k) rg[c][k] = 0u;
        }
    }

    // dy stays packed in rg (unpacked again in the second pass); only the
    // fp32 factor w / r is kept per element.
    float q[NCH][VEC];
    float s_part = 0.f, u_part = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int col0 = (c * 64 + lane) * VEC;
#pragma unroll
        for (int e = 0; e < VEC; ++e) q[c][e] = 0.f;
        if (c * 64 * VEC < limit) {
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const bool live = col0 + e <= qpos;
                const float a = __builtin_fmaf(alpha, elem<T>(rx[c], e), neg_alpha_theta);
                const float s = __builtin_fmaf(a, a, 4.f);
                const float rr = fast_rsqrt(s);
                const float t = __builtin_fmaf(s, rr, a);  // a + sqrt(s)
                const float wv = live ? power_of<POWER>(t) : 0.f;
                q[c][e] = wv * rr;
                s_part += wv;
                u_part = live ? __builtin_fmaf(elem<TG>(rg[c], e), wv, u_part) : u_part;
            }
        }
    }
    const float S = wave_sum(s_part) + eps_scaled;
    const float U = wave_sum(u_part);
    const float Tdot = U / S;
    const float C = alpha * static_cast<float>(POWER) / S;

#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int col0 = (c * 64 + lane) * VEC;
        if (col0 < n_cols) {
            float ov[VEC];
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const float d = (C * q[c][e]) * (elem<TG>(rg[c], e) - Tdot);
                ov[e] = (col0 + e <= qpos) ? d : 0.f;
            }
            uint32_t packed[4];
            pack_row16<T>(ov, packed);
            store_words(dxr + col0, packed);
        }
    }
}

// ---------------------------------------------------------------------------
// Split-row variants: R waves share one row (wave j of the row owns chunks
// j, j + R, j + 2R, ...), combine their partial sums through LDS, and each
// keeps only NCH / R chunks in registers.  Shorter per-wave work keeps the
// rows in flight in a denser address window.
// ---------------------------------------------------------------------------
template <int R>
constexpr int split_block_waves() { return R > kWavesPerBlock ? R : kWavesPerBlock; }

template <typename T, int NCH, int POWER, int R>
__global__ __launch_bounds__(64 * split_block_waves<R>()) void norm_fwd_split(const T* __restrict__ x, T* __restrict__ y, int64_t n_rows,
                                                      int n_cols, int64_t xs, int64_t ys, int causal, float alpha,
                                                      float neg_alpha_theta, float eps_scaled) {
    constexpr int VEC = 16 / sizeof(T);
    constexpr int NW = NCH / R;  // chunks per wave
    constexpr int SW = split_block_waves<R>();
    __shared__ float red[SW];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wr = wave % R;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (SW / R) + wave / R;
    const bool valid = row < n_rows;
    const int qpos = valid ? (causal ? static_cast<int>(row % n_cols) : n_cols - 1) : -1;
    const int limit = qpos + 1;
    const T* xr = x + (valid ? row : 0) * xs;
    T* yr = y + (valid ? row : 0) * ys;

    uint32_t raw[NW][4];
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        const int c = wr + R * i;
        const int col0 = (c * 64 + lane) * VEC;
        if (c * 64 * VEC < limit) {
            load_words(xr + (col0 < limit ? col0 : 0), raw[i]);
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) raw[i][k] = 0u;
        }
    }
    float w[NW][VEC];
    float part = 0.f;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        const int c = wr + R * i;
        const int col0 = (c * 64 + lane) * VEC;
#pragma unroll
        for (int e = 0; e < VEC; ++e) w[i][e] = 0.f;
        if (c * 64 * VEC < limit) {
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const float a = __builtin_fmaf(alpha, elem<T>(raw[i], e), neg_alpha_theta);
                const float t = a + fast_sqrt(__builtin_fmaf(a, a, 4.f));
                const float wv = (col0 + e <= qpos) ? power_of<POWER>(t) : 0.f;
                w[i][e] = wv;
                part += wv;
            }
        }
    }
    const float ws = wave_sum(part);
    if (lane == 0) red[wave] = ws;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int j = 0; j < R; ++j) tot += red[(wave / R) * R + j];
    const float inv = 1.f / (tot + eps_scaled);
    if (!valid) return;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        const int c = wr + R * i;
        const int col0 = (c * 64 + lane) * VEC;
        if (col0 < n_cols) {
            float ov[VEC];
#pragma unroll
            for (int e = 0; e < VEC; ++e) ov[e] = w[i][e] * inv;
            uint32_t packed[4];
            pack_row16<T>(ov, packed);
            store_words(yr + col0, packed);
        }
    }
}

template <typename T, typename TG, int NCH, int POWER, int R>
__global__ __launch_bounds__(64 * split_block_waves<R>()) void norm_bwd_split(const T* __restrict__ x, const TG* __restrict__ dy,
                                                      T* __restrict__ dx, int64_t n_rows, int n_cols, int64_t xs,
                                                      int64_t gs, int64_t dxs, int causal, float alpha,
                                                      float neg_alpha_theta, float eps_scaled) {
    constexpr int VEC = 16 / sizeof(T);
    constexpr int GW = (VEC * static_cast<int>(sizeof(TG))) / 16;
    constexpr int NW = NCH / R;
    constexpr int SW = split_block_waves<R>();
    __shared__ float red[SW][2];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wr = wave % R;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (SW / R) + wave / R;
    const bool valid = row < n_rows;
    const int qpos = valid ? (causal ? static_cast<int>(row % n_cols) : n_cols - 1) : -1;
    const int limit = qpos + 1;
    const T* xr = x + (valid ? row : 0) * xs;
    const TG* gr = dy + (valid ? row : 0) * gs;
    T* dxr = dx + (valid ? row : 0) * dxs;

    uint32_t rx[NW][4];
    uint32_t rg[NW][4 * GW];
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        const int c = wr + R * i;
        const int col0 = (c * 64 + lane) * VEC;
        if (c * 64 * VEC < limit) {
            const int off = col0 < limit ? col0 : 0;
            load_words(xr + off, rx[i]);
#pragma unroll
            for (int k = 0; k < GW; ++k) load_words(gr + off + k * (16 / sizeof(TG)), &rg[i][4 * k]);
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) rx[i][k] = 0u;
#pragma unroll
            for (int k = 0; k < 4 * GW; ++k) rg[i][k] = 0u;
        }
    }
    float q[NW][VEC];
    float s_part = 0.f, u_part = 0.f;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        const int c = wr + R * i;
        const int col0 = (c * 64 + lane) * VEC;
#pragma unroll
        for (int e = 0; e < VEC; ++e) q[i][e] = 0.f;
        if (c * 64 * VEC < limit) {
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const bool live = col0 + e <= qpos;
                const float a = __builtin_fmaf(alpha, elem<T>(rx[i], e), neg_alpha_theta);
                const float s = __builtin_fmaf(a, a, 4.f);
                const float rr = fast_rsqrt(s);
                const float t = __builtin_fmaf(s, rr, a);
                const float wv = live ? power_of<POWER>(t) : 0.f;
                q[i][e] = wv * rr;
                s_part += wv;
                u_part = live ? __builtin_fmaf(elem<TG>(rg[i], e), wv, u_part) : u_part;
            }
        }
    }
    const float sw = wave_sum(s_part), uw = wave_sum(u_part);
    if (lane == 0) {
        red[wave][0] = sw;
        red[wave][1] = uw;
    }
    __syncthreads();
    float S = 0.f, U = 0.f;
#pragma unroll
    for (int j = 0; j < R; ++j) {
        S += red[(wave / R) * R + j][0];
        U += red[(wave / R) * R + j][1];
    }
    S += eps_scaled;
    const float Tdot = U / S;
    const float C = alpha * static_cast<float>(POWER) / S;
    if (!valid) return;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        const int c = wr + R * i;
        const int col0 = (c * 64 + lane) * VEC;
        if (col0 < n_cols) {
            float ov[VEC];
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const float d = (C * q[i][e]) * (elem<TG>(rg[i], e) - Tdot);
                ov[e] = (col0 + e <= qpos) ? d : 0.f;
            }
            uint32_t packed[4];
            pack_row16<T>(ov, packed);
            store_words(dxr + col0, packed);
        }
    }
}

// ---------------------------------------------------------------------------
// Scalar kernels for rows that are not 16-byte aligned: one wave per row,
// element-strided passes over global memory (no register cache).
// ---------------------------------------------------------------------------
template <typename T, int POWER>
__global__ __launch_bounds__(256) void norm_fwd_scalar(const T* __restrict__ x, T* __restrict__ y,
                                                       int64_t n_rows, int n_cols, int64_t xs,
                                                       int64_t ys, int causal, float alpha,
                                                       float neg_alpha_theta, float eps_scaled) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
    if (wave >= n_rows) return;
    int64_t row;
    int qpos;
    row_of_wave(wave, n_cols, causal != 0, row, qpos);
    const T* xr = x + row * xs;
    T* yr = y + row * ys;
    float part = 0.f;
    for (int j = lane; j <= qpos; j += 64) {
        const float a = __builtin_fmaf(alpha, to_f32(xr[j]), neg_alpha_theta);
        part += power_of<POWER>(a + fast_sqrt(__builtin_fmaf(a, a, 4.f)));
    }
    const float inv = 1.f / (wave_sum(part) + eps_scaled);
    for (int j = lane; j < n_cols; j += 64) {
        float o = 0.f;
        if (j <= qpos) {
            const float a = __builtin_fmaf(alpha, to_f32(xr[j]), neg_alpha_theta);
            o = power_of<POWER>(a + fast_sqrt(__builtin_fmaf(a, a, 4.f))) * inv;
        }
        yr[j] = from_f32<T>(o);
    }
}

template <typename T, typename TG, int POWER>
__global__ __launch_bounds__(256) void norm_bwd_scalar(const T* __restrict__ x, const TG* __restrict__ dy,
                                                       T* __restrict__ dx, int64_t n_rows, int n_cols,
                                                       int64_t xs, int64_t gs, int64_t dxs, int causal,
                                                       float alpha, float neg_alpha_theta,
                                                       float eps_scaled) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
    if (wave >= n_rows) return;
    int64_t row;
    int qpos;
    row_of_wave(wave, n_cols, causal != 0, row, qpos);
    const T* xr = x + row * xs;
    const TG* gr = dy + row * gs;
    T* dxr = dx + row * dxs;
    float s_part = 0.f, u_part = 0.f;
    for (int j = lane; j <= qpos; j += 64) {
        const float a = __builtin_fmaf(alpha, to_f32(xr[j]), neg_alpha_theta);
        const float wv = power_of<POWER>(a + fast_sqrt(__builtin_fmaf(a, a, 4.f)));
        s_part += wv;
        u_part = __builtin_fmaf(to_f32(gr[j]), wv, u_part);
    }
    const float S = wave_sum(s_part) + eps_scaled;
    const float Tdot = wave_sum(u_part) / S;
    const float C = alpha * static_cast<float>(POWER) / S;
    for (int j = lane; j < n_cols; j += 64) {
        float o = 0.f;
        if (j <= qpos) {
            const float a = __builtin_fmaf(alpha, to_f32(xr[j]), neg_alpha_theta);
            const float s = __builtin_fmaf(a, a, 4.f);
            const float rr = fast_rsqrt(s);
            const float wv = power_of<POWER>(__builtin_fmaf(s, rr, a));
            o = (C * (wv * rr)) * (to_f32(gr[j]) - Tdot);
        }
        dxr[j] = from_f32<T>(o);
    }
}

// ---------------------------------------------------------------------------
// Host dispatch.
// ---------------------------------------------------------------------------
constexpr int kMaxCols = 8192;
// Waves per row for rows of NCH 1 KB chunks: 4 (one row per block) for 8
// chunks, 8 from 16 chunks up.  Measured: causal bf16 L=4096 fwd 3-4% and
// bwd 1-3% faster, row-wise fp32 L=2048 6% faster; for rows of 2-4 chunks
// (causal bf16 L=1024/2048) splitting was 11-17% slower, so those keep one
// wave per row.  Two chunks per wave does best: 8 waves per row at bf16
// L=4096 (one chunk each) was 17% slower, while at fp32 L=4096 (16 chunks)
// 8 waves beat 4 by 6.7% (fwd 1390 vs 1490 us) and 3.8% (bwd 2129 vs
// 2212 us).
constexpr int split_for(int nch) { return nch >= 16 ? 8 : nch >= 8 ? 4 : 1; }

template <int R>
dim3 split_grid(int64_t n_rows) {
    constexpr int rows = split_block_waves<R>() / R;  // rows per block
    return dim3(static_cast<unsigned>((n_rows + rows - 1) / rows));
}

int chunks_for(int n_cols, int vec) {
    const int need = (n_cols + 64 * vec - 1) / (64 * vec);
    int nch = 1;
    while (nch < need) nch *= 2;
    return nch;
}

float eps_for_power(int power) { return kEps * static_cast<float>(1 << power); }

// The forward launch for these arguments: element kernel for unaligned rows
// (or n_cols not a multiple of the vector width), else one wave per row, or
// split_for(NCH) waves per row for long rows.
template <typename T, int POWER>
int plan_fwd_t(const void* x, const void* y, int64_t n_rows, int n_cols, int64_t xs, int64_t ys, RowLaunch& L) {
    constexpr int VEC = 16 / sizeof(T);
    L.grid = dim3(static_cast<unsigned>((n_rows + kWavesPerBlock - 1) / kWavesPerBlock));
    L.block = dim3(64 * kWavesPerBlock);
    L.rows_per_block = kWavesPerBlock;
    L.waves_per_row = 1;
    const bool vec_ok = (n_cols % VEC == 0) && (xs % VEC == 0) && (ys % VEC == 0) && aligned16(x) && aligned16(y);
    if (!vec_ok) {
        L.fn = reinterpret_cast<const void*>(&norm_fwd_scalar<T, POWER>);
        L.variant = SA_ROW_SCALAR;
        L.elems_per_load = 1;
        L.row_pass_elems = 64;
        return 0;
    }
    const int nch = chunks_for(n_cols, VEC);
    L.elems_per_load = VEC;
    L.row_pass_elems = nch * 64 * VEC;
    switch (nch) {
#define SA_FWD_CASE(N)                                                                        \
    case N:                                                                                   \
        if constexpr (split_for(N) > 1) {                                                     \
            constexpr int R = split_for(N);                                                   \
            L.fn = reinterpret_cast<const void*>(&norm_fwd_split<T, N, POWER, R>);            \
            L.grid = split_grid<R>(n_rows);                                                   \
            L.block = dim3(64 * split_block_waves<R>());                                      \
            L.rows_per_block = split_block_waves<R>() / R;                                    \
            L.waves_per_row = R;                                                              \
            L.variant = SA_ROW_SPLIT;                                                         \
        } else {                                                                              \
            L.fn = reinterpret_cast<const void*>(&norm_fwd_vec<T, N, POWER>);                 \
            L.variant = SA_ROW_VEC;                                                           \
        }                                                                                     \
        return 0;
        SA_FWD_CASE(1)
        SA_FWD_CASE(2)
        SA_FWD_CASE(4)
        SA_FWD_CASE(8)
        SA_FWD_CASE(16)
        SA_FWD_CASE(32)
#undef SA_FWD_CASE
        default:
            return SA_ERR_UNSUPPORTED;
    }
}

template <typename T, int POWER>
int launch_fwd_t(const void* x, void* y, int64_t n_rows, int n_cols, int64_t xs, int64_t ys,
                 int causal, float alpha, float theta, hipStream_t st) {
    RowLaunch L;
    const int pst = plan_fwd_t<T, POWER>(x, y, n_rows, n_cols, xs, ys, L);
    if (pst != 0) return pst;
    // every forward kernel takes (x, y, n_rows, n_cols, xs, ys, causal, alpha, -alpha theta, eps)
    const T* xp = static_cast<const T*>(x);
    T* yp = static_cast<T*>(y);
    float nat = -alpha * theta;
    float eps = eps_for_power(POWER);
    void* args[] = {&xp, &yp, &n_rows, &n_cols, &xs, &ys, &causal, &alpha, &nat, &eps};
    return launch_row(L, args, st);
}

template <typename T>
int launch_fwd_p(const void* x, void* y, int64_t n_rows, int n_cols, int64_t xs, int64_t ys, int causal,
                 float alpha, float theta, int power, hipStream_t st) {
    switch (power) {
        case 1: return launch_fwd_t<T, 1>(x, y, n_rows, n_cols, xs, ys, causal, alpha, theta, st);
        case 2: return launch_fwd_t<T, 2>(x, y, n_rows, n_cols, xs, ys, causal, alpha, theta, st);
        case 3: return launch_fwd_t<T, 3>(x, y, n_rows, n_cols, xs, ys, causal, alpha, theta, st);
        default: return SA_ERR_BAD_FAMILY;
    }
}

template <typename T, typename TG, int POWER>
int launch_bwd_t(const void* x, const void* dy, void* dx, int64_t n_rows, int n_cols, int64_t xs, int64_t gs,
                 int64_t dxs, int causal, float alpha, float theta, hipStream_t st) {
    constexpr int VEC = 16 / sizeof(T);
    constexpr int GVEC = 16 / sizeof(TG);
    const dim3 grid(static_cast<unsigned>((n_rows + kWavesPerBlock - 1) / kWavesPerBlock));
    const dim3 block(64 * kWavesPerBlock);
    const float nat = -alpha * theta;
    const float eps = eps_for_power(POWER);
    const T* xp = static_cast<const T*>(x);
    const TG* gp = static_cast<const TG*>(dy);
    T* dp = static_cast<T*>(dx);
    const bool vec_ok = (n_cols % VEC == 0) && (xs % VEC == 0) && (gs % GVEC == 0) && (dxs % VEC == 0) &&
                        aligned16(x) && aligned16(dy) && aligned16(dx);
    if (!vec_ok) {
        if (!grid_fits(grid, block)) return SA_ERR_BAD_SHAPE;
        norm_bwd_scalar<T, TG, POWER><<<grid, block, 0, st>>>(xp, gp, dp, n_rows, n_cols, xs, gs, dxs, causal,
                                                              alpha, nat, eps);
        return status_from_launch();
    }
    switch (chunks_for(n_cols, VEC)) {
#define SA_BWD_CASE(N)                                                                                   \
    case N:                                                                                              \
        if constexpr (split_for(N) > 1) {                                                                \
            const dim3 sg = split_grid<split_for(N)>(n_rows), sb(64 * split_block_waves<split_for(N)>()); \
            if (!grid_fits(sg, sb)) return SA_ERR_BAD_SHAPE;                                             \
            norm_bwd_split<T, TG, N, POWER, split_for(N)><<<sg, sb, 0, st>>>(                            \
                    xp, gp, dp, n_rows, n_cols, xs, gs, dxs, causal, alpha, nat, eps);                   \
        } else {                                                                                         \
            if (!grid_fits(grid, block)) return SA_ERR_BAD_SHAPE;                                        \
            norm_bwd_vec<T, TG, N, POWER><<<grid, block, 0, st>>>(xp, gp, dp, n_rows, n_cols, xs, gs, dxs, \
                                                                  causal, alpha, nat, eps);              \
        }                                                                                                \
        break;
        SA_BWD_CASE(1)
        SA_BWD_CASE(2)
        SA_BWD_CASE(4)
        SA_BWD_CASE(8)
        SA_BWD_CASE(16)
        SA_BWD_CASE(32)
#undef SA_BWD_CASE
        default:
            return SA_ERR_UNSUPPORTED;
    }
    return status_from_launch();
}

template <typename T, typename TG>
int launch_bwd_p(const void* x, const void* dy, void* dx, int64_t n_rows, int n_cols, int64_t xs, int64_t gs,
                 int64_t dxs, int causal, float alpha, float theta, int power, hipStream_t st) {
    switch (power) {
        case 1: return launch_bwd_t<T, TG, 1>(x, dy, dx, n_rows, n_cols, xs, gs, dxs, causal, alpha, theta, st);
        case 2: return launch_bwd_t<T, TG, 2>(x, dy, dx, n_rows, n_cols, xs, gs, dxs, causal, alpha, theta, st);
        case 3: return launch_bwd_t<T, TG, 3>(x, dy, dx, n_rows, n_cols, xs, gs, dxs, causal, alpha, theta, st);
        default: return SA_ERR_BAD_FAMILY;
    }
}

int check_rows(const void* a, const void* b, int64_t n_rows, int64_t n_cols) {
    if (n_rows < 0 || n_rows > INT32_MAX || n_cols < 0 || n_cols > kMaxCols) return SA_ERR_BAD_SHAPE;
    if (n_rows == 0 || n_cols == 0) return 1;  // nothing to do
    if (a == nullptr || b == nullptr) return SA_ERR_NULL_POINTER;
    return 0;
}

}  // namespace
}  // namespace sa

extern "C" int sa_norm_fwd(const void* x, void* y, int64_t n_rows, int64_t n_cols, int64_t x_row_stride,
                           int64_t y_row_stride, int dtype, int causal, float alpha, float theta, int power,
                           sa_stream_t stream) {
    using namespace sa;
    const int chk = check_rows(x, y, n_rows, n_cols);
    if (chk != 0) return chk > 0 ? 0 : chk;
    if (x_row_stride < n_cols || y_row_stride < n_cols) return SA_ERR_BAD_STRIDE;
    if (power < 1 || power > 3) return SA_ERR_BAD_FAMILY;
    const int nc = static_cast<int>(n_cols);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    switch (dtype) {
        case SA_F32: return launch_fwd_p<float>(x, y, n_rows, nc, x_row_stride, y_row_stride, causal, alpha, theta, power, st);
        case SA_F16: return launch_fwd_p<f16>(x, y, n_rows, nc, x_row_stride, y_row_stride, causal, alpha, theta, power, st);
        case SA_BF16: return launch_fwd_p<bf16>(x, y, n_rows, nc, x_row_stride, y_row_stride, causal, alpha, theta, power, st);
        default: return SA_ERR_BAD_DTYPE;
    }
}

extern "C" int sa_norm_fwd_launch_info(const void* x, const void* y, int64_t n_rows, int64_t n_cols,
                                       int64_t x_row_stride, int64_t y_row_stride, int dtype, int power,
                                       sa_launch_info* info) {
    using namespace sa;
    if (info == nullptr) return SA_ERR_NULL_POINTER;
    if (n_rows < 0 || n_rows > INT32_MAX || n_cols <= 0 || n_cols > kMaxCols) return SA_ERR_BAD_SHAPE;
    if (x_row_stride < n_cols || y_row_stride < n_cols) return SA_ERR_BAD_STRIDE;
    const int nc = static_cast<int>(n_cols);
    RowLaunch L;
    int st = SA_ERR_BAD_FAMILY;
#define SA_PLAN(TT)                                                                                      \
    switch (power) {                                                                                     \
        case 1: st = plan_fwd_t<TT, 1>(x, y, n_rows, nc, x_row_stride, y_row_stride, L); break;           \
        case 2: st = plan_fwd_t<TT, 2>(x, y, n_rows, nc, x_row_stride, y_row_stride, L); break;           \
        case 3: st = plan_fwd_t<TT, 3>(x, y, n_rows, nc, x_row_stride, y_row_stride, L); break;           \
        default: break;                                                                                  \
    }
    switch (dtype) {
        case SA_F32: SA_PLAN(float) break;
        case SA_F16: SA_PLAN(f16) break;
        case SA_BF16: SA_PLAN(bf16) break;
        default: return SA_ERR_BAD_DTYPE;
    }
#undef SA_PLAN
    if (st != 0) return st;
    return describe_row_launch(L, info);
}

extern "C" int sa_norm_bwd(const void* x, const void* dy, void* dx, int64_t n_rows, int64_t n_cols,
                           int64_t x_row_stride, int64_t dy_row_stride, int64_t dx_row_stride, int x_dtype,
                           int dy_dtype, int causal, float alpha, float theta, int power, sa_stream_t stream) {
    using namespace sa;
    const int chk = check_rows(x, dx, n_rows, n_cols);
    if (chk != 0) return chk > 0 ? 0 : chk;
    if (dy == nullptr) return SA_ERR_NULL_POINTER;
    if (x_row_stride < n_cols || dy_row_stride < n_cols || dx_row_stride < n_cols) return SA_ERR_BAD_STRIDE;
    if (power < 1 || power > 3) return SA_ERR_BAD_FAMILY;
    const int nc = static_cast<int>(n_cols);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int64_t xs = x_row_stride, gs = dy_row_stride, ds = dx_row_stride;
    if (x_dtype == SA_F32 && dy_dtype == SA_F32)
        return launch_bwd_p<float, float>(x, dy, dx, n_rows, nc, xs, gs, ds, causal, alpha, theta, power, st);
    if (x_dtype == SA_BF16 && dy_dtype == SA_BF16)
        return launch_bwd_p<bf16, bf16>(x, dy, dx, n_rows, nc, xs, gs, ds, causal, alpha, theta, power, st);
    if (x_dtype == SA_BF16 && dy_dtype == SA_F32)
        return launch_bwd_p<bf16, float>(x, dy, dx, n_rows, nc, xs, gs, ds, causal, alpha, theta, power, st);
    if (x_dtype == SA_F16 && dy_dtype == SA_F16)
        return launch_bwd_p<f16, f16>(x, dy, dx, n_rows, nc, xs, gs, ds, causal, alpha, theta, power, st);
    if (x_dtype == SA_F16 && dy_dtype == SA_F32)
        return launch_bwd_p<f16, float>(x, dy, dx, n_rows, nc, xs, gs, ds, causal, alpha, theta, power, st);
    return SA_ERR_BAD_DTYPE;
}
