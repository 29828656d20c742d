// Row-wise and causal softmax: the comparison baseline of the reference
// (kernels.py:534-562 row-wise, :852-884 causal; APIs :1233-1325).
//
// Same layout as the squareplus normalisation kernels: one wavefront per
// row (eight for rows of 16 KB or more) held in registers (16-byte
// nontemporal loads of the visible part only), a row max, exp(x - max) with
// v_exp_f32 on (x - max) * log2(e), a row sum, one reciprocal, and 16-byte
// stores of the full row (zeros past the diagonal for the causal variant).
// fp32 arithmetic for every dtype.
#include "common.hpp"

namespace sa {
namespace {

constexpr int kSmWavesPerBlock = 4;
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float exp_of_shifted(float v, float m) {
    return __builtin_amdgcn_exp2f((v - m) * kLog2e);
}

template <typename T, int NCH>
__global__ __launch_bounds__(256) void softmax_fwd_vec(const T* __restrict__ x, T* __restrict__ y, int64_t n_rows,
                                                       int n_cols, int64_t xs, int64_t ys, int causal) {
    constexpr int VEC = 16 / sizeof(T);
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kSmWavesPerBlock + (threadIdx.x >> 6);
    if (row >= n_rows) return;
    const int qpos = causal ? static_cast<int>(row % n_cols) : n_cols - 1;
    const int limit = qpos + 1;
    const T* xr = x + row * xs;
    T* yr = y + row * ys;

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
    float m = -__builtin_inff();
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int col0 = (c * 64 + lane) * VEC;
        if (c * 64 * VEC < limit) {
#pragma unroll
            for (int e = 0; e < VEC; ++e)
                if (col0 + e <= qpos) m = __builtin_fmaxf(m, elem<T>(raw[c], e));
        }
    }
    m = wave_max(m);
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
                const float wv = (col0 + e <= qpos) ? exp_of_shifted(elem<T>(raw[c], e), m) : 0.f;
                w[c][e] = wv;
                part += wv;
            }
        }
    }
    const float inv = 1.f / wave_sum(part);
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

// Long rows: R waves per row (one row per block), chunk c of the row on wave
// c % R (interleaved, so the visible part of a causal row spreads over all
// R waves); the row max and the row sum combine the waves' values in LDS.
template <typename T, int NCH, int R>
__global__ __launch_bounds__(64 * R) void softmax_fwd_split(const T* __restrict__ x, T* __restrict__ y,
                                                             int64_t n_rows, int n_cols, int64_t xs, int64_t ys,
                                                             int causal) {
    constexpr int VEC = 16 / sizeof(T);
    constexpr int NW = NCH / R;  // chunks per wave
    static_assert(NW >= 1 && NW * R == NCH, "R divides the chunks of a row");
    __shared__ float red[2][R];
    const int lane = threadIdx.x & 63;
    const int wr = threadIdx.x >> 6;
    const int64_t row = blockIdx.x;
    if (row >= n_rows) return;  // whole block: one row per block
    const int qpos = causal ? static_cast<int>(row % n_cols) : n_cols - 1;
    const int limit = qpos + 1;
    const T* xr = x + row * xs;
    T* yr = y + row * ys;

    uint32_t raw[NW][4];
#pragma unroll
    for (int k = 0; k < NW; ++k) {
        const int c = k * R + wr;
        const int col0 = (c * 64 + lane) * VEC;
        if (c * 64 * VEC < limit) {
            load_words(xr + (col0 < limit ? col0 : 0), raw[k]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) raw[k][e] = 0u;
        }
    }
    float m = -__builtin_inff();
#pragma unroll
    for (int k = 0; k < NW; ++k) {
        const int c = k * R + wr;
        const int col0 = (c * 64 + lane) * VEC;
        if (c * 64 * VEC < limit) {
#pragma unroll
            for (int e = 0; e < VEC; ++e)
                if (col0 + e <= qpos) m = __builtin_fmaxf(m, elem<T>(raw[k], e));
        }
    }
    m = wave_max(m);
    if (lane == 0) red[0][wr] = m;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < R; ++i) m = __builtin_fmaxf(m, red[0][i]);
    float w[NW][VEC];
    float part = 0.f;
#pragma unroll
    for (int k = 0; k < NW; ++k) {
        const int c = k * R + wr;
        const int col0 = (c * 64 + lane) * VEC;
#pragma unroll
        for (int e = 0; e < VEC; ++e) w[k][e] = 0.f;
        if (c * 64 * VEC < limit) {
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const float wv = (col0 + e <= qpos) ? exp_of_shifted(elem<T>(raw[k], e), m) : 0.f;
                w[k][e] = wv;
                part += wv;
            }
        }
    }
    part = wave_sum(part);
    if (lane == 0) red[1][wr] = part;
    __syncthreads();
    float total = 0.f;
#pragma unroll
    for (int i = 0; i < R; ++i) total += red[1][i];
    const float inv = 1.f / total;
#pragma unroll
    for (int k = 0; k < NW; ++k) {
        const int c = k * R + wr;
        const int col0 = (c * 64 + lane) * VEC;
        if (col0 < n_cols) {
            float ov[VEC];
#pragma unroll
            for (int e = 0; e < VEC; ++e) ov[e] = w[k][e] * inv;
            uint32_t packed[4];
            pack_row16<T>(ov, packed);
            store_words(yr + col0, packed);
        }
    }
}

// Waves per row by 1 KB chunks per row: 8 (two chunks each) from 16 chunks
// up.  Measured: row-wise fp32 L=4096 1377-1392 vs 1502-1511 us with one
// wave per row; 4 waves per row at 8 chunks (causal bf16 L=4096) were
// slower (566-579 vs 552-555 us), so rows up to 8 chunks keep one wave.
constexpr int sm_split_for(int nch) { return nch >= 16 ? 8 : 1; }

// Rows that are not 16-byte aligned: three element-strided passes.
template <typename T>
__global__ __launch_bounds__(256) void softmax_fwd_scalar(const T* __restrict__ x, T* __restrict__ y, int64_t n_rows,
                                                          int n_cols, int64_t xs, int64_t ys, int causal) {
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kSmWavesPerBlock + (threadIdx.x >> 6);
    if (row >= n_rows) return;
    const int qpos = causal ? static_cast<int>(row % n_cols) : n_cols - 1;
    const T* xr = x + row * xs;
    T* yr = y + row * ys;
    float m = -__builtin_inff();
    for (int j = lane; j <= qpos; j += 64) m = __builtin_fmaxf(m, to_f32(xr[j]));
    m = wave_max(m);
    float part = 0.f;
    for (int j = lane; j <= qpos; j += 64) part += exp_of_shifted(to_f32(xr[j]), m);
    const float inv = 1.f / wave_sum(part);
    for (int j = lane; j < n_cols; j += 64)
        yr[j] = from_f32<T>(j <= qpos ? exp_of_shifted(to_f32(xr[j]), m) * inv : 0.f);
}

constexpr int kSmMaxCols = 8192;

template <typename T>
int plan_softmax(const void* x, const void* y, int64_t n_rows, int n_cols, int64_t xs, int64_t ys, RowLaunch& L) {
    constexpr int VEC = 16 / sizeof(T);
    L.grid = dim3(static_cast<unsigned>((n_rows + kSmWavesPerBlock - 1) / kSmWavesPerBlock));
    L.block = dim3(64 * kSmWavesPerBlock);
    L.rows_per_block = kSmWavesPerBlock;
    L.waves_per_row = 1;
    const bool vec_ok = (n_cols % VEC == 0) && (xs % VEC == 0) && (ys % VEC == 0) && aligned16(x) && aligned16(y);
    if (!vec_ok) {
        L.fn = reinterpret_cast<const void*>(&softmax_fwd_scalar<T>);
        L.variant = SA_ROW_SCALAR;
        L.elems_per_load = 1;
        L.row_pass_elems = 64;
        return 0;
    }
    int need = (n_cols + 64 * VEC - 1) / (64 * VEC), nch = 1;
    while (nch < need) nch *= 2;
    L.variant = SA_ROW_VEC;
    L.elems_per_load = VEC;
    L.row_pass_elems = nch * 64 * VEC;
    switch (nch) {
#define SA_SM_CASE(N)                                                               \
    case N:                                                                         \
        if constexpr (sm_split_for(N) > 1) {                                        \
            constexpr int R = sm_split_for(N);                                      \
            L.fn = reinterpret_cast<const void*>(&softmax_fwd_split<T, N, R>);      \
            L.grid = dim3(static_cast<unsigned>(n_rows));                           \
            L.block = dim3(64 * R);                                                 \
            L.rows_per_block = 1;                                                   \
            L.waves_per_row = R;                                                    \
            L.variant = SA_ROW_SPLIT;                                               \
        } else {                                                                    \
            L.fn = reinterpret_cast<const void*>(&softmax_fwd_vec<T, N>);           \
        }                                                                           \
        return 0;
        SA_SM_CASE(1)
        SA_SM_CASE(2)
        SA_SM_CASE(4)
        SA_SM_CASE(8)
        SA_SM_CASE(16)
        SA_SM_CASE(32)
#undef SA_SM_CASE
        default:
            return SA_ERR_UNSUPPORTED;
    }
}

template <typename T>
int launch_softmax(const void* x, void* y, int64_t n_rows, int n_cols, int64_t xs, int64_t ys, int causal,
                   hipStream_t st) {
    RowLaunch L;
    const int pst = plan_softmax<T>(x, y, n_rows, n_cols, xs, ys, L);
    if (pst != 0) return pst;
    // both kernels take (x, y, n_rows, n_cols, xs, ys, causal)
    const T* xp = static_cast<const T*>(x);
    T* yp = static_cast<T*>(y);
    void* args[] = {&xp, &yp, &n_rows, &n_cols, &xs, &ys, &causal};
    return launch_row(L, args, st);
}

}  // namespace
}  // namespace sa

extern "C" int sa_softmax_fwd(const void* x, void* y, int64_t n_rows, int64_t n_cols, int64_t x_row_stride,
                              int64_t y_row_stride, int dtype, int causal, sa_stream_t stream) {
    using namespace sa;
    if (n_rows < 0 || n_rows > INT32_MAX || n_cols < 0 || n_cols > kSmMaxCols) return SA_ERR_BAD_SHAPE;
    if (n_rows == 0 || n_cols == 0) return 0;
    if (x == nullptr || y == nullptr) return SA_ERR_NULL_POINTER;
    if (x_row_stride < n_cols || y_row_stride < n_cols) return SA_ERR_BAD_STRIDE;
    const int nc = static_cast<int>(n_cols);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    switch (dtype) {
        case SA_F32: return launch_softmax<float>(x, y, n_rows, nc, x_row_stride, y_row_stride, causal, st);
        case SA_F16: return launch_softmax<f16>(x, y, n_rows, nc, x_row_stride, y_row_stride, causal, st);
        case SA_BF16: return launch_softmax<bf16>(x, y, n_rows, nc, x_row_stride, y_row_stride, causal, st);
        default: return SA_ERR_BAD_DTYPE;
    }
}

extern "C" int sa_softmax_fwd_launch_info(const void* x, const void* y, int64_t n_rows, int64_t n_cols,
                                          int64_t x_row_stride, int64_t y_row_stride, int dtype,
                                          sa_launch_info* info) {
    using namespace sa;
    if (info == nullptr) return SA_ERR_NULL_POINTER;
    if (n_rows < 0 || n_rows > INT32_MAX || n_cols <= 0 || n_cols > kSmMaxCols) return SA_ERR_BAD_SHAPE;
    if (x_row_stride < n_cols || y_row_stride < n_cols) return SA_ERR_BAD_STRIDE;
    const int nc = static_cast<int>(n_cols);
    RowLaunch L;
    int st;
    switch (dtype) {
        case SA_F32: st = plan_softmax<float>(x, y, n_rows, nc, x_row_stride, y_row_stride, L); break;
        case SA_F16: st = plan_softmax<f16>(x, y, n_rows, nc, x_row_stride, y_row_stride, L); break;
        case SA_BF16: st = plan_softmax<bf16>(x, y, n_rows, nc, x_row_stride, y_row_stride, L); break;
        default: return SA_ERR_BAD_DTYPE;
    }
    if (st != 0) return st;
    return describe_row_launch(L, info);
}
