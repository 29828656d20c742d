"""ctypes binding of ``libsmooth_attn_amd.so`` (the C ABI in include/smooth_attn_amd.h).

The library is loaded lazily on first use and must exist: there is no
fallback path.  A missing or stale build raises ``RuntimeError`` naming the
build command.
"""
from __future__ import annotations

import ctypes
import os
import threading
from ctypes import POINTER, c_float, c_int, c_int32, c_int64, c_void_p
from pathlib import Path

# SMOOTH_ATTN_LIB selects an alternate build of the same library (tuning runs).
LIB_PATH = Path(os.environ.get("SMOOTH_ATTN_LIB") or Path(__file__).resolve().parent / "libsmooth_attn_amd.so")

# Element-type codes (SA_F32 ... in the header).
SA_F32, SA_F16, SA_BF16, SA_FP8_E4M3FN = 0, 1, 2, 3


def paged_dtypes(q_type: int, cache_type: int) -> int:
    """SA_PAGED_DTYPES(q_type, cache_type): the paged decode's dtype argument
    for q and caches of different element types."""
    return q_type | ((cache_type + 1) << 8)


# SA_PAGED_NOALLOC_SCRATCH_BYTES: the fixed scratch of sa_paged_decode_noalloc.
PAGED_NOALLOC_SCRATCH_BYTES = 64 << 20

_I64P = POINTER(c_int64)


class LaunchInfo(ctypes.Structure):
    """``sa_launch_info`` of include/smooth_attn_amd.h."""

    _fields_ = [(name, c_int) for name in (
        "variant", "grid_x", "block_threads", "rows_per_block", "waves_per_row", "elems_per_load",
        "row_pass_elems", "n_vgprs", "shared_mem_bytes", "blocks_per_cu")]


ROW_VARIANTS = {0: "scalar", 1: "vec", 2: "split"}

# name -> (restype, argtypes); mirrors include/smooth_attn_amd.h.
SIGNATURES = {
    "sa_status_string": (ctypes.c_char_p, [c_int]),
    "sa_norm_fwd": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int, c_int,
                            c_float, c_float, c_int, c_void_p]),
    "sa_norm_bwd": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64,
                            c_int, c_int, c_int, c_float, c_float, c_int, c_void_p]),
    "sa_softmax_fwd": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int, c_int, c_void_p]),
    "sa_transpose16": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p]),
    "sa_norm_fwd_launch_info": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int, c_int,
                                        POINTER(LaunchInfo)]),
    "sa_softmax_fwd_launch_info": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int,
                                           POINTER(LaunchInfo)]),
    "sa_flash_fwd": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                             c_int, _I64P, _I64P, _I64P, _I64P, c_float, c_int, c_int, c_int, c_void_p]),
    "sa_flash_bwd": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                             c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, _I64P, _I64P, _I64P,
                             _I64P, _I64P, _I64P, _I64P, _I64P, c_float, c_int, c_int, c_int, c_void_p]),
    "sa_flash_bwd_workspace_size": (c_int64, [c_int, c_int, c_int, c_int, c_int, c_int, c_int]),
    "sa_flash_bwd_ws": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, _I64P, _I64P, _I64P,
                                _I64P, _I64P, _I64P, _I64P, _I64P, c_float, c_int, c_int, c_int, c_void_p, c_int64,
                                c_void_p]),
    "sa_fp8_quantize": (c_int, [c_void_p, c_void_p, c_int64, c_int, c_void_p, c_void_p, c_void_p]),
    "sa_flash_fp8_fwd": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                 c_void_p, c_int, c_int, c_int, c_int, c_int, _I64P, _I64P, _I64P, _I64P,
                                 c_float, c_int, c_int, c_void_p]),
    "sa_flash_rope_workspace_size": (c_int64, [c_int, c_int, c_int, c_int]),
    "sa_rope_rotate": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, _I64P, c_int,
                               c_void_p]),
    "sa_flash_rope_fwd": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                  c_void_p, c_int64, c_int, c_int, c_int, c_int, c_int, _I64P, _I64P, _I64P,
                                  _I64P, c_float, c_int, c_int, c_void_p]),
    "sa_paged_decode_workspace_size": (c_int64, [c_int, c_int, c_int, c_int, c_int]),
    "sa_paged_decode": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                c_int, c_int, c_int, c_int, c_int, _I64P, _I64P, _I64P, _I64P, c_int64, c_float,
                                c_int, c_void_p, c_int64, c_void_p]),
    "sa_paged_decode_noalloc": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                        c_int, c_int, c_int, c_int, c_int, _I64P, _I64P, _I64P, _I64P, c_int64,
                                        c_float, c_int, c_void_p]),
    "sa_paged_kv_append": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                   c_int, c_int, c_int, c_int, c_int, _I64P, _I64P, _I64P, c_int64, c_int,
                                   c_void_p]),
}

_lock = threading.Lock()
_lib = None


def load():
    """Load (once) and return the configured ctypes library handle."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"smooth_attn HIP library not found at {LIB_PATH}; build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` from the repository root"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def check(status: int, what: str) -> None:
    """Raise RuntimeError for a nonzero status returned by the C ABI."""
    if status != 0:
        msg = load().sa_status_string(int(status)).decode()
        raise RuntimeError(f"{what} failed (status {status}): {msg}")


def strides(t) -> ctypes.Array:
    """Element strides of a torch tensor as an int64[ndim] array."""
    return (c_int64 * t.dim())(*t.stride())


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()
