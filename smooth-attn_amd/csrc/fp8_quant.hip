// Per-tensor absmax quantisation to float8_e4m3fn, entirely on the device
// (reference kernels.py:2592-2601, which synchronises through .item()):
//   scale = max(amax|x| / 448, 1e-12);  x8 = e4m3fn(clamp(x / scale, +-448))
// Three launches on one stream: zero the amax word, reduce amax with one
// atomicMax per block (non-negative floats order like their bit patterns),
// then quantise.  x / scale is a true division so the codes match torch's
// fp32 division followed by the round-to-nearest-even e4m3fn cast.  Both
// passes read 16 bytes per lane and load when x is 16-byte aligned (the
// remainder, and unaligned inputs, element by element), several loads in
// flight per lane.
#include "common.hpp"

namespace sa {
namespace {

constexpr int kQThreads = 256;
// The amax pass ends in one same-address atomicMax per block; those
// serialise, so the pass runs on at most kAmaxBlocks blocks (one per CU)
// with kAmaxUnroll loads in flight per lane (measured on config 4's Q,
// 67M bf16: 4096 blocks 95 us, 512 blocks 64 us, 256 blocks x 8 loads 62 us
// for amax + quantise together).
constexpr unsigned kAmaxBlocks = 256;
constexpr int kAmaxUnroll = 8;

__global__ void fill_zero_u32(uint32_t* p) { p[0] = 0u; }

template <typename T>
__device__ __forceinline__ float ld(const T* p, int64_t i) { return to_f32(p[i]); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

template <typename T>
__global__ __launch_bounds__(kQThreads) void amax_kernel(const T* __restrict__ x, int64_t n, uint32_t* amax_bits,
                                                         int vec) {
    constexpr int NV = 16 / sizeof(T);  // elements per 16-byte load
    __shared__ float part[kQThreads / 64];
    float m = 0.f;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kQThreads;
    const int64_t tid0 = static_cast<int64_t>(blockIdx.x) * kQThreads + threadIdx.x;
    const int64_t nv = vec ? n / NV : 0;
    int64_t i = tid0;
    // kAmaxUnroll independent 16-byte loads in flight per lane: the grid is
    // small (see launch_quant), so each lane must keep several loads going
    constexpr int U = kAmaxUnroll;
    for (; i + (U - 1) * stride < nv; i += U * stride) {
        uint32_t w[U][4];
#pragma unroll
        for (int u = 0; u < U; ++u) load_words(x + (i + u * stride) * NV, w[u]);
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int e = 0; e < NV; ++e) m = fmaxf(m, fabsf(elem<T>(w[u], e)));
    }
    for (; i < nv; i += stride) {
        uint32_t w[4];
        load_words(x + i * NV, w);
#pragma unroll
        for (int e = 0; e < NV; ++e) m = fmaxf(m, fabsf(elem<T>(w, e)));
    }
    for (int64_t i = nv * NV + tid0; i < n; i += stride) m = fmaxf(m, fabsf(ld(x, i)));
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = part[0];
        for (int w = 1; w < kQThreads / 64; ++w) b = fmaxf(b, part[w]);
        atomicMax(amax_bits, __float_as_uint(b));
    }
}

__device__ __forceinline__ float quant_scale(const uint32_t* amax_bits) {
    const float amax = __uint_as_float(amax_bits[0]);
    return fmaxf(amax / 448.f, 1e-12f);
}

// Round-to-nearest-even conversion of a value already clamped to +-448.
__device__ __forceinline__ uint32_t to_e4m3(float v) {
    return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(v, v, 0, false)) & 0xFFu;
}

// Four clamped values -> one word of e4m3fn codes (element e in byte e).
__device__ __forceinline__ uint32_t pack_e4m3(float v0, float v1, float v2, float v3) {
    const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(v0, v1, 0, false);
    return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(v2, v3, lo, true));
}

template <typename T>
__global__ __launch_bounds__(kQThreads) void quant_kernel(const T* __restrict__ x, uint8_t* __restrict__ x8, int64_t n,
                                                          const uint32_t* amax_bits, float* scale_out, int vec) {
    constexpr int NV = 16 / sizeof(T);  // elements per 16-byte load
    const float scale = quant_scale(amax_bits);
    if (blockIdx.x == 0 && threadIdx.x == 0) scale_out[0] = scale;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kQThreads;
    const int64_t tid0 = static_cast<int64_t>(blockIdx.x) * kQThreads + threadIdx.x;
    if (vec) {
        // NV elements per thread and step: one 16-byte load, NV / 4 word stores
        const int64_t nv = n / NV;
        auto emit = [&](int64_t j, const uint32_t* w) {
            float v[NV];
#pragma unroll
            for (int e = 0; e < NV; ++e) v[e] = fminf(fmaxf(elem<T>(w, e) / scale, -448.f), 448.f);
            if constexpr (NV == 8) {
                *reinterpret_cast<uint2*>(x8 + j * NV) =
                    uint2{pack_e4m3(v[0], v[1], v[2], v[3]), pack_e4m3(v[4], v[5], v[6], v[7])};
            } else {
                *reinterpret_cast<uint32_t*>(x8 + j * NV) = pack_e4m3(v[0], v[1], v[2], v[3]);
            }
        };
        int64_t i = tid0;
        for (; i + stride < nv; i += 2 * stride) {  // two loads in flight per lane
            uint32_t w0[4], w1[4];
            load_words(x + i * NV, w0);
            load_words(x + (i + stride) * NV, w1);
            emit(i, w0);
            emit(i + stride, w1);
        }
        for (; i < nv; i += stride) {
            uint32_t w[4];
            load_words(x + i * NV, w);
            emit(i, w);
        }
        if (blockIdx.x == 0) {
            for (int64_t i = nv * NV + threadIdx.x; i < n; i += kQThreads) {
                const float v = fminf(fmaxf(ld(x, i) / scale, -448.f), 448.f);
                x8[i] = static_cast<uint8_t>(to_e4m3(v));
            }
        }
        return;
    }
    // four elements per thread and step, one 32-bit store
    const int64_t n4 = n / 4;
    for (int64_t i = tid0; i < n4; i += stride) {
        uint32_t word = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float v = fminf(fmaxf(ld(x, 4 * i + e) / scale, -448.f), 448.f);
            word |= to_e4m3(v) << (8 * e);
        }
        reinterpret_cast<uint32_t*>(x8)[i] = word;
    }
    if (blockIdx.x == 0) {
        for (int64_t i = 4 * n4 + threadIdx.x; i < n; i += kQThreads) {
            const float v = fminf(fmaxf(ld(x, i) / scale, -448.f), 448.f);
            x8[i] = static_cast<uint8_t>(to_e4m3(v));
        }
    }
}

template <typename T>
int launch_quant(const void* x, void* x8, int64_t n, float* amax_ws, float* scale_out, hipStream_t st) {
    uint32_t* ab = reinterpret_cast<uint32_t*>(amax_ws);
    fill_zero_u32<<<1, 1, 0, st>>>(ab);
    // 16-byte steps need x 16-byte aligned and x8 aligned to the step's
    // output (8 or 4 bytes; the entry point requires 4)
    constexpr int NV = 16 / sizeof(T);
    const int vec = aligned16(x) && (reinterpret_cast<uintptr_t>(x8) % NV) == 0 ? 1 : 0;
    const int64_t want = (n + kQThreads * 4 * NV - 1) / (kQThreads * 4 * NV);
    const unsigned blocks = static_cast<unsigned>(want < 1 ? 1 : (want > 4096 ? 4096 : want));
    const unsigned ablocks = blocks > kAmaxBlocks ? kAmaxBlocks : blocks;
    amax_kernel<T><<<ablocks, kQThreads, 0, st>>>(static_cast<const T*>(x), n, ab, vec);
    quant_kernel<T><<<blocks, kQThreads, 0, st>>>(static_cast<const T*>(x), static_cast<uint8_t*>(x8), n, ab,
                                                  scale_out, vec);
    return status_from_launch();
}

}  // namespace
}  // namespace sa

extern "C" int sa_fp8_quantize(const void* x, void* x8, int64_t n, int dtype, float* amax_ws, float* scale_out,
                               sa_stream_t stream) {
    using namespace sa;
    if (n < 0) return SA_ERR_BAD_SHAPE;
    if (!amax_ws || !scale_out || (n > 0 && (!x || !x8))) return SA_ERR_NULL_POINTER;
    if ((reinterpret_cast<uintptr_t>(x8) & 3u) != 0) return SA_ERR_BAD_STRIDE;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    switch (dtype) {
        case SA_F32: return launch_quant<float>(x, x8, n, amax_ws, scale_out, st);
        case SA_F16: return launch_quant<f16>(x, x8, n, amax_ws, scale_out, st);
        case SA_BF16: return launch_quant<bf16>(x, x8, n, amax_ws, scale_out, st);
        default: return SA_ERR_BAD_DTYPE;
    }
}
