// 16-bit fused attention on the kernels built for head dims 256 and 512,
// reached from sa_flash_fwd / sa_flash_bwd for SA_BF16 or SA_F16 head dims
// 136..512 (multiples of 8; columns past D are masked).
#pragma once

#include "common.hpp"

namespace sa {

// Validates and launches the D = 256 / 512 forward (same contract as sa_flash_fwd).
int flash_fwd_wide(const void* q, const void* k, const void* v, void* o, float* row_sums, int B, int Hq, int Hkv,
                   int T, int D, const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                   const int64_t* o_strides, float scale, int window_size, int exact_math, int dtype,
                   hipStream_t st);

// Bytes of fp32 partials the D = 256 / 512 backward splits its dK and dV
// blocks into at this shape (0: no split); D in 136..512.
int64_t flash_bwd_wide_workspace_size(int B, int Hq, int Hkv, int T, int D, int window_size);

// Validates and launches the D = 256 / 512 backward (same contract as
// sa_flash_bwd_ws: without a workspace, or one below the size above, the
// split is coarser or absent).
int flash_bwd_wide(const void* q, const void* k, const void* v, const void* o, const void* dout,
                   const float* row_sums, void* dq, void* dk, void* dv, float* delta_ws, int B, int Hq, int Hkv,
                   int T, int D, const int64_t* const strides[8], float scale, int window_size, int exact_math,
                   int dtype, void* workspace, int64_t workspace_bytes, hipStream_t st);

}  // namespace sa
