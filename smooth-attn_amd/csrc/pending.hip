// Entry points whose kernels are not built yet: they reject every call.
#include "common.hpp"

extern "C" int sa_flash_bwd(const void*, const void*, const void*, const void*, const void*, const float*, void*,
                            void*, void*, float*, int, int, int, int, int, const int64_t*, const int64_t*,
                            const int64_t*, const int64_t*, const int64_t*, const int64_t*, const int64_t*,
                            const int64_t*, float, int, int, int, sa_stream_t) {
    return SA_ERR_UNSUPPORTED;
}
extern "C" int64_t sa_paged_decode_workspace_size(int, int, int, int, int) { return 0; }
extern "C" int sa_paged_decode(const void*, const void*, const void*, void*, const int32_t*, const int32_t*, int, int,
                               int, int, int, int, const int64_t*, const int64_t*, const int64_t*, const int64_t*,
                               int64_t, float, int, float*, int64_t, sa_stream_t) { return SA_ERR_UNSUPPORTED; }
