// Transpose of a 2-D matrix of 16-bit elements, dst[c][r] = src[r][c]:
// lays the RoPE projection's weight out for the faster GEMM form (the
// output projection O[B*T, H*D] x W_o[H*D, D_model] runs as
// O x (W_o^T)^T with W_o^T contiguous).
//
// One 64 x 64 tile per block of 256 threads: each thread reads 16 elements
// of the tile as two 16-byte row chunks, the tile goes through LDS (rows
// padded by 4 bytes, so the column-wise reads hit distinct banks), and each
// thread writes 16 elements of the transposed tile as two 16-byte chunks.
// Edge tiles fall back to element accesses.
#include "common.hpp"

namespace sa {
namespace {

constexpr int kTT = 64;                  // tile edge
constexpr int kTPitch = kTT * 2 + 4;     // LDS row pitch in bytes (padded)

__global__ __launch_bounds__(256) void transpose16_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                                          int rows, int cols, int64_t ss, int64_t ds) {
    __shared__ __attribute__((aligned(16))) unsigned char tile[kTT * kTPitch];
    const int r0 = blockIdx.y * kTT, c0 = blockIdx.x * kTT;
    const int tid = threadIdx.x;
    const bool full = r0 + kTT <= rows && c0 + kTT <= cols;
    // load: 64 rows x 8 chunks of 8 elements = 512 chunks, two per thread
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int ch = tid + 256 * k;
        const int r = ch >> 3, cc = (ch & 7) * 8;
        uint16_t v[8];
        if (full) {
            const u32x4 w = *reinterpret_cast<const u32x4*>(src + (r0 + r) * ss + c0 + cc);
            *reinterpret_cast<u32x4*>(v) = w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                v[e] = (r0 + r < rows && c0 + cc + e < cols) ? src[(r0 + r) * ss + c0 + cc + e] : uint16_t(0);
        }
        uint16_t* row = reinterpret_cast<uint16_t*>(tile + r * kTPitch);
#pragma unroll
        for (int e = 0; e < 8; ++e) row[cc + e] = v[e];
    }
    __syncthreads();
    // store: transposed row c (source column) holds source rows r0 .. r0+63
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int ch = tid + 256 * k;
        const int c = ch >> 3, rr = (ch & 7) * 8;
        uint16_t v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = reinterpret_cast<const uint16_t*>(tile + (rr + e) * kTPitch)[c];
        if (full) {
            *reinterpret_cast<u32x4*>(dst + (c0 + c) * ds + r0 + rr) = *reinterpret_cast<const u32x4*>(v);
        } else if (c0 + c < cols) {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (r0 + rr + e < rows) dst[(c0 + c) * ds + r0 + rr + e] = v[e];
        }
    }
}

}  // namespace
}  // namespace sa

extern "C" int sa_transpose16(const void* src, void* dst, int64_t rows, int64_t cols, int64_t src_row_stride,
                              int64_t dst_row_stride, sa_stream_t stream) {
    using namespace sa;
    if (rows < 0 || cols < 0 || rows > (int64_t(1) << 30) || cols > (int64_t(1) << 30)) return SA_ERR_BAD_SHAPE;
    if (rows == 0 || cols == 0) return 0;
    if (!src || !dst) return SA_ERR_NULL_POINTER;
    if (src_row_stride < cols || dst_row_stride < rows || src_row_stride % 8 != 0 || dst_row_stride % 8 != 0 ||
        !aligned16(src) || !aligned16(dst))
        return SA_ERR_BAD_STRIDE;
    const int64_t gx = (cols + kTT - 1) / kTT, gy = (rows + kTT - 1) / kTT;
    if (gy > 65535) return SA_ERR_BAD_SHAPE;
    transpose16_kernel<<<dim3(static_cast<unsigned>(gx), static_cast<unsigned>(gy)), 256, 0,
                         reinterpret_cast<hipStream_t>(stream)>>>(
        static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst), static_cast<int>(rows),
        static_cast<int>(cols), src_row_stride, dst_row_stride);
    return status_from_launch();
}
