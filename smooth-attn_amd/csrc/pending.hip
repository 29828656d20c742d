// Entry points whose kernels are not built yet: they reject every call.
#include "common.hpp"

extern "C" int sa_flash_bwd(const void*, const void*, const void*, const void*, const void*, const float*, void*,
                            void*, void*, float*, int, int, int, int, int, const int64_t*, const int64_t*,
                            const int64_t*, const int64_t*, const int64_t*, const int64_t*, const int64_t*,
                            const int64_t*, float, int, int, int, sa_stream_t) {
    return SA_ERR_UNSUPPORTED;
}
