// Status strings for the C ABI.
#include "common.hpp"

extern "C" const char* sa_status_string(int status) {
    switch (status) {
        case 0: return "success";
        case SA_ERR_NULL_POINTER: return "null pointer argument";
        case SA_ERR_BAD_SHAPE: return "unsupported or inconsistent shape";
        case SA_ERR_BAD_DTYPE: return "unsupported dtype";
        case SA_ERR_BAD_FAMILY: return "power must be 1, 2 or 3";
        case SA_ERR_BAD_STRIDE: return "unsupported stride or alignment";
        case SA_ERR_UNSUPPORTED: return "unsupported configuration";
        case SA_ERR_WORKSPACE:
            return "workspace too small (sa_paged_decode_noalloc: the call needs more than its fixed "
                   "SA_PAGED_NOALLOC_SCRATCH_BYTES of scratch)";
        default:
            if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
            return "unknown error";
    }
}
