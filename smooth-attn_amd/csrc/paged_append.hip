// Paged-KV cache writer: appends new tokens' K and V through the block table,
// the step before paged decode.  The reference builds its caches with Python
// loops in its tests (tests/test_paged_attention.py:10-73); this is the
// device-side equivalent for a serving loop.
//
// For sequence b with current length ctx_b and new rows t < n_new:
//   pos = ctx_b + t,  page = block_table[b, pos / P],  slot = pos % P
//   k_cache[page, h, slot, :] = k_new[b, h, t, :]   (same for v)
// One thread per 16-byte chunk of a new row, for K and V (fp32, bf16, fp16 or
// e4m3fn rows: the copy moves bytes and never converts).  Positions whose
// page index is past max_pages, or whose block-table entry is outside
// [0, n_pages), are skipped: nothing is written outside the caches.
#include "common.hpp"

namespace sa {
namespace {

struct AppendParams {
    const void* k_new;
    const void* v_new;
    void* k_cache;
    void* v_cache;
    const int32_t* table;
    const int32_t* ctx;
    int64_t ns[4], kcs[4], vcs[4];  // strides: new (b,h,t,d); caches (page,h,slot,d)
    int64_t bt_stride;
    int B, Hkv, n_new, D, P, max_pages, n_pages;
    int esize;  // bytes per element
};

__global__ __launch_bounds__(256) void paged_append_kernel(AppendParams p, int64_t n_chunks) {
    const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (gid >= n_chunks) return;
    const int cpr = p.D * p.esize / 16;  // 16-byte chunks per row
    const int64_t row = gid / cpr;
    const int c = static_cast<int>(gid - row * cpr);
    const int t = static_cast<int>(row % p.n_new);
    const int64_t bh = row / p.n_new;
    const int h = static_cast<int>(bh % p.Hkv);
    const int b = static_cast<int>(bh / p.Hkv);
    const int ctx = p.ctx[b];
    if (ctx < 0) return;
    const int64_t pos = static_cast<int64_t>(ctx) + t;
    const int64_t page_idx = pos / p.P;
    if (page_idx >= p.max_pages) return;
    const int phys = p.table[b * p.bt_stride + page_idx];
    if (phys < 0 || phys >= p.n_pages) return;
    const int slot = static_cast<int>(pos - page_idx * p.P);
    // byte offsets
    const int64_t src = (b * p.ns[0] + h * p.ns[1] + t * p.ns[2]) * p.esize + c * 16;
    const int64_t dk = (phys * p.kcs[0] + h * p.kcs[1] + slot * p.kcs[2]) * p.esize + c * 16;
    const int64_t dv = (phys * p.vcs[0] + h * p.vcs[1] + slot * p.vcs[2]) * p.esize + c * 16;
    const char* kn = static_cast<const char*>(p.k_new);
    const char* vn = static_cast<const char*>(p.v_new);
    *reinterpret_cast<u32x4*>(static_cast<char*>(p.k_cache) + dk) = *reinterpret_cast<const u32x4*>(kn + src);
    *reinterpret_cast<u32x4*>(static_cast<char*>(p.v_cache) + dv) = *reinterpret_cast<const u32x4*>(vn + src);
}

// 16-byte rows: unit stride along D, the other strides multiples of 16 bytes
bool rows16(const int64_t* s, int esize) {
    const int per = 16 / esize;
    return s[3] == 1 && s[0] % per == 0 && s[1] % per == 0 && s[2] % per == 0;
}

}  // namespace
}  // namespace sa

extern "C" int sa_paged_kv_append(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                                  const int32_t* block_table, const int32_t* context_lens, int B, int Hkv,
                                  int n_new, int D, int page_size, int max_pages, int n_pages,
                                  const int64_t* new_strides, const int64_t* kc_strides,
                                  const int64_t* vc_strides, int64_t bt_stride, int dtype, sa_stream_t stream) {
    using namespace sa;
    if (dtype != SA_BF16 && dtype != SA_F16 && dtype != SA_F32 && dtype != SA_FP8_E4M3FN) return SA_ERR_BAD_DTYPE;
    const int esize = dtype == SA_F32 ? 4 : dtype == SA_FP8_E4M3FN ? 1 : 2;
    if (B < 0 || Hkv <= 0 || n_new < 0 || max_pages < 0 || n_pages < 0 || page_size <= 0) return SA_ERR_BAD_SHAPE;
    if (D <= 0 || (D * esize) % 16 != 0) return SA_ERR_UNSUPPORTED;
    if (B == 0 || n_new == 0 || max_pages == 0 || n_pages == 0) return 0;
    if (!k_new || !v_new || !k_cache || !v_cache || !block_table || !context_lens || !new_strides || !kc_strides ||
        !vc_strides)
        return SA_ERR_NULL_POINTER;
    if (!rows16(new_strides, esize) || !rows16(kc_strides, esize) || !rows16(vc_strides, esize) ||
        bt_stride < max_pages ||
        !aligned16(k_new) || !aligned16(v_new) || !aligned16(k_cache) || !aligned16(v_cache))
        return SA_ERR_BAD_STRIDE;
    AppendParams prm{};
    prm.k_new = k_new;
    prm.v_new = v_new;
    prm.k_cache = k_cache;
    prm.v_cache = v_cache;
    prm.table = block_table;
    prm.ctx = context_lens;
    for (int i = 0; i < 4; ++i) {
        prm.ns[i] = new_strides[i];
        prm.kcs[i] = kc_strides[i];
        prm.vcs[i] = vc_strides[i];
    }
    prm.bt_stride = bt_stride;
    prm.B = B;
    prm.Hkv = Hkv;
    prm.n_new = n_new;
    prm.D = D;
    prm.P = page_size;
    prm.max_pages = max_pages;
    prm.n_pages = n_pages;
    prm.esize = esize;
    const int64_t n_chunks = static_cast<int64_t>(B) * Hkv * n_new * (D * esize / 16);
    const dim3 grid(static_cast<unsigned>((n_chunks + 255) / 256));
    paged_append_kernel<<<grid, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(prm, n_chunks);
    return status_from_launch();
}
