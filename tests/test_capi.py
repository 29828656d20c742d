"""The C-ABI library loads and exports every entry point the header declares —
CPU only (no kernel launch; sa_status_string is host code)."""
import ctypes
import re
from pathlib import Path

import pytest

from smooth_attn import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "smooth_attn_amd.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(sa_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_entry_points():
    names = declared_functions()
    for n in ["sa_norm_fwd", "sa_norm_bwd", "sa_flash_fwd", "sa_flash_bwd", "sa_fp8_quantize", "sa_flash_fp8_fwd",
              "sa_paged_decode", "sa_paged_decode_workspace_size", "sa_status_string"]:
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"missing exports: {missing}"
    # the ctypes signature table covers exactly the declared functions
    assert sorted(_lib.SIGNATURES) == declared_functions()


def test_status_strings():
    lib = _lib.load()
    assert lib.sa_status_string(0) == b"success"
    assert b"dtype" in lib.sa_status_string(-3)
    with pytest.raises(RuntimeError, match="dtype"):
        _lib.check(-3, "probe")


def test_launch_info_struct_matches_header():
    # field names and order of sa_launch_info, all int
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    body = re.search(r"typedef struct sa_launch_info \{(.*?)\} sa_launch_info;", text, flags=re.S).group(1)
    fields = re.findall(r"int\s+(\w+)\s*;", body)
    assert fields == [name for name, _ in _lib.LaunchInfo._fields_]
    assert len(re.findall(r";", body)) == len(fields)
    assert _lib.LaunchInfo().__sizeof__() >= 4 * len(fields)


def test_launch_info_argument_errors():
    # rejected before any HIP call, so these run without a GPU
    lib = _lib.load()
    info = _lib.LaunchInfo()
    assert lib.sa_norm_fwd_launch_info(None, None, 4, 64, 64, 64, _lib.SA_BF16, 2, None) == -1
    assert lib.sa_norm_fwd_launch_info(None, None, 4, 0, 64, 64, _lib.SA_BF16, 2, ctypes.byref(info)) == -2
    assert lib.sa_norm_fwd_launch_info(None, None, 4, 9000, 9000, 9000, _lib.SA_BF16, 2, ctypes.byref(info)) == -2
    assert lib.sa_norm_fwd_launch_info(None, None, 4, 64, 32, 64, _lib.SA_BF16, 2, ctypes.byref(info)) == -5
    assert lib.sa_norm_fwd_launch_info(None, None, 4, 64, 64, 64, 7, 2, ctypes.byref(info)) == -3
    assert lib.sa_norm_fwd_launch_info(None, None, 4, 64, 64, 64, _lib.SA_BF16, 4, ctypes.byref(info)) == -4
    assert lib.sa_softmax_fwd_launch_info(None, None, 4, 64, 64, 64, _lib.SA_F32, None) == -1
    assert lib.sa_softmax_fwd_launch_info(None, None, 4, 64, 64, 64, 7, ctypes.byref(info)) == -3
    # 2^31 rows: the one-block-per-row grids would wrap, so the row count is refused
    big = 1 << 31
    assert lib.sa_norm_fwd_launch_info(None, None, big, 64, 64, 64, _lib.SA_BF16, 2, ctypes.byref(info)) == -2
    assert lib.sa_softmax_fwd_launch_info(None, None, big, 64, 64, 64, _lib.SA_F32, ctypes.byref(info)) == -2
    assert lib.sa_norm_fwd(None, None, big, 64, 64, 64, _lib.SA_BF16, 1, 2.0, 0.5, 2, None) == -2
    assert lib.sa_norm_bwd(None, None, None, big, 64, 64, 64, 64, _lib.SA_BF16, _lib.SA_BF16, 1, 2.0, 0.5, 2,
                           None) == -2
    assert lib.sa_softmax_fwd(None, None, big, 64, 64, 64, _lib.SA_F32, 0, None) == -2


def test_row_launches_refuse_grids_past_32_bit_work_items():
    # a dispatch holds grid * block work-items in 32 bits: 2^26 rows of one
    # wave each, 2^24 rows of 4 waves (bf16 rows of 8 KB), 2^23 of 8 waves
    # (fp32 rows of 16 KB).  Refused by the plan before any HIP call (the
    # pointers are 16-byte aligned dummies that nothing dereferences).
    lib = _lib.load()
    info = _lib.LaunchInfo()
    d = ctypes.c_void_p(16)
    for n_cols, dtype, limit in ((1024, _lib.SA_BF16, 1 << 26), (4096, _lib.SA_BF16, 1 << 24),
                                 (4096, _lib.SA_F32, 1 << 23)):
        assert lib.sa_norm_fwd_launch_info(d, d, limit, n_cols, n_cols, n_cols, dtype, 2, ctypes.byref(info)) == -2
        assert lib.sa_norm_fwd(d, d, limit, n_cols, n_cols, n_cols, dtype, 1, 2.0, 0.5, 2, None) == -2
        assert lib.sa_norm_bwd(d, d, d, limit, n_cols, n_cols, n_cols, n_cols, dtype, dtype, 1, 2.0, 0.5, 2,
                               None) == -2
    assert lib.sa_softmax_fwd_launch_info(d, d, 1 << 23, 4096, 4096, 4096, _lib.SA_F32, ctypes.byref(info)) == -2
    assert lib.sa_softmax_fwd(d, d, 1 << 23, 4096, 4096, 4096, _lib.SA_F32, 0, None) == -2
    assert lib.sa_softmax_fwd(d, d, 1 << 26, 256, 256, 256, _lib.SA_F32, 0, None) == -2


def test_paged_decode_rejects_plans_past_int32():
    # B * Hkv * ceil(max context / 32) tiles must fit the plan's 32-bit
    # prefix sums; rejected before any HIP call, so this runs without a GPU
    lib = _lib.load()
    strides = (ctypes.c_int64 * 4)(128 * 32, 128, 128, 1)
    kv = (ctypes.c_int64 * 4)(8 * 16 * 128, 16 * 128, 128, 1)
    o = (ctypes.c_int64 * 3)(32 * 128, 128, 1)
    dummy = ctypes.c_void_p(16)
    st = lib.sa_paged_decode(dummy, dummy, dummy, dummy, dummy, dummy, 4096, 32, 8, 128, 16, 1 << 20, 1 << 20,
                             strides, kv, kv, o, 1 << 20, 0.1, _lib.SA_BF16, dummy, 1 << 62, None)
    assert st == -6  # SA_ERR_UNSUPPORTED


def test_transpose16_argument_errors():
    lib = _lib.load()
    d = ctypes.c_void_p(16)
    assert lib.sa_transpose16(None, d, 8, 8, 8, 8, None) == -1
    assert lib.sa_transpose16(d, d, -1, 8, 8, 8, None) == -2
    assert lib.sa_transpose16(d, d, 8, 16, 8, 8, None) == -5   # source stride below cols
    assert lib.sa_transpose16(d, d, 8, 8, 12, 8, None) == -5   # stride not a multiple of 8
    assert lib.sa_transpose16(ctypes.c_void_p(18), d, 8, 8, 8, 8, None) == -5  # unaligned
    assert lib.sa_transpose16(d, d, 0, 8, 8, 8, None) == 0


def test_paged_workspace_sizes():
    # plan (B + 2 int32, padded to 16 bytes) + fp32 partials [B, Hq, n_slots, D + 1];
    # n_slots = ceil(max_pages * P / (32 m)) + 1 with the tile floor
    # m = clamp(B * ceil(Hq / 8) * ceil(max_pages * P / 32) / 2048, 1, 16)
    lib = _lib.load()

    def expect(B, Hq, D, max_pages, P):
        tiles = -(-max_pages * P // 32)
        m = max(1, min(16, B * -(-Hq // 8) * tiles // 2048))
        slots = -(-max_pages * P // (32 * m)) + 1
        return ((B + 2) * 4 + 15) // 16 * 16 + B * Hq * slots * (D + 1) * 4, m, slots

    cases = {  # shape -> (m, n_slots)
        (64, 32, 128, 1024, 16): (16, 33),  # config 5: the full split, as for large batches
        (4, 8, 128, 16, 16): (1, 9),        # 4 short sequences: one tile per wave
        (16, 32, 128, 128, 16): (2, 33),    # 16 x 2K tokens, Hq 32
        (0, 8, 128, 16, 16): None,          # empty batch: nothing to size
    }
    for (B, Hq, D, mp, P), ms in cases.items():
        got = lib.sa_paged_decode_workspace_size(B, Hq, D, mp, P)
        if ms is None:
            assert got == 0
            continue
        want, m, slots = expect(B, Hq, D, mp, P)
        assert (m, slots) == ms and got == want


def test_paged_decode_noalloc_refuses_what_its_scratch_cannot_hold():
    # two partials per (sequence, query head) are the least any split needs:
    # 4096 x 32 x 2 x 129 fp32 = 135 MB > SA_PAGED_NOALLOC_SCRATCH_BYTES, so
    # the call returns SA_ERR_WORKSPACE before any HIP call (dummy pointers)
    lib = _lib.load()
    q = (ctypes.c_int64 * 4)(32 * 128, 128, 128, 1)
    kv = (ctypes.c_int64 * 4)(8 * 16 * 128, 16 * 128, 128, 1)
    o = (ctypes.c_int64 * 3)(32 * 128, 128, 1)
    d = ctypes.c_void_p(256)
    args = (d, d, d, d, d, d, 4096, 32, 8, 128, 16, 4, 1 << 14, q, kv, kv, o, 4, 0.1, _lib.SA_BF16, None)
    assert lib.sa_paged_decode_noalloc(*args) == -7
    assert _lib.PAGED_NOALLOC_SCRATCH_BYTES == 64 << 20
    header = HEADER.read_text()
    assert "#define SA_PAGED_NOALLOC_SCRATCH_BYTES (64LL << 20)" in header
    # argument errors as the workspace entry point
    bad = list(args)
    bad[10] = 12  # page size not a power of two
    assert lib.sa_paged_decode_noalloc(*bad) == -6
    bad = list(args)
    bad[0] = None
    assert lib.sa_paged_decode_noalloc(*bad) == -1


def test_flash_fp32_argument_errors():
    # fp32 q/k/v (SA_F32 = 0): (b, h, t) strides multiples of 4 elements
    # (16 bytes), D a multiple of 4 up to 512; every check runs before any launch
    lib = _lib.load()
    d = ctypes.c_void_p(16)
    good = (ctypes.c_int64 * 4)(2 * 64 * 64, 64 * 64, 64, 1)
    odd = (ctypes.c_int64 * 4)(2 * 64 * 66, 64 * 66, 66, 1)  # rows 264 bytes apart
    fwd = lambda s, D=64, dt=_lib.SA_F32, B=1, ptr=d: lib.sa_flash_fwd(
        ptr, d, d, d, None, B, 2, 2, 64, D, s, good, good, good, 0.1, 0, 0, dt, None)
    assert fwd(odd) == -5
    assert fwd(good, ptr=ctypes.c_void_p(20)) == -5  # base not 16-byte aligned
    assert fwd(good, D=50) == -6
    assert fwd(good, D=516) == -6
    assert fwd(good, D=264, B=0) == 0 and fwd(good, D=512, B=0) == 0
    assert fwd(good, dt=7) == -3
    assert fwd(good, B=0) == 0
    bwd = lambda s, D=64: lib.sa_flash_bwd(d, d, d, d, d, d, d, d, d, d, 0, 2, 2, 64, D, good, good, good, good,
                                           s, good, good, good, 0.1, 0, 0, _lib.SA_F32, None)
    assert bwd(odd) == -5
    assert bwd(good, D=18) == -6
    assert bwd(good, D=36) == 0  # B = 0: accepted, nothing launched
    assert bwd(good) == 0


def test_flash_bwd_workspace_size():
    # fp32 partials of dK / dV for split key blocks: only for 16-bit head dims
    # and grids that leave the GPU idle behind the first key blocks; the size
    # is n_split * 2 (dK, dV) * B * Hkv * T * kernel head dim * 4 for head
    # dims up to 128, and n_split * B * Hkv * T * kernel head dim * 4 (one
    # buffer the dV and the dK kernel take in turn) for the kernels of head
    # dim 256 and 512
    lib = _lib.load()
    ws = lambda B, Hq, Hkv, T, D, W=0, dt=_lib.SA_BF16: lib.sa_flash_bwd_workspace_size(B, Hq, Hkv, T, D, W, dt)
    for B, Hq, Hkv, T, D, Dk, planes in ((1, 32, 8, 8192, 128, 128, 2), (1, 8, 1, 65536, 128, 128, 2),
                                         (1, 4, 2, 333, 40, 64, 2), (1, 16, 2, 16384, 256, 256, 1),
                                         (1, 4, 2, 333, 200, 256, 1), (1, 8, 1, 16384, 512, 512, 1),
                                         (1, 2, 1, 260, 400, 512, 1)):
        n = ws(B, Hq, Hkv, T, D)
        unit = planes * B * Hkv * T * Dk * 4
        assert n > 0 and n % unit == 0 and n // unit in (2, 4, 8, 16), (B, Hq, Hkv, T, D, n)
        assert ws(B, Hq, Hkv, T, D, dt=_lib.SA_F16) == n
    assert ws(1, 32, 8, 8192, 128, dt=_lib.SA_F32) == 0  # fp32 kernels do not split
    assert ws(16, 32, 8, 4096, 128) == 0  # 4096 key blocks fill the GPU
    assert ws(4, 16, 16, 4096, 256) == 0  # 2048 blocks of the head-dim-256 kernels too
    assert ws(0, 32, 8, 8192, 128) == 0 and ws(1, 32, 8, 0, 128) == 0
    assert ws(1, 30, 8, 8192, 128) == -1 and ws(-1, 32, 8, 64, 128) == -1
    # a workspace that is not 16-byte aligned is refused before any launch
    d = ctypes.c_void_p(256)
    s = (ctypes.c_int64 * 4)(8 * 64 * 128, 64 * 128, 128, 1)
    st = lib.sa_flash_bwd_ws(d, d, d, d, d, d, d, d, d, d, 1, 8, 8, 64, 128, s, s, s, s, s, s, s, s, 0.1, 0, 0,
                             _lib.SA_BF16, ctypes.c_void_p(264), 1 << 20, None)
    assert st == -5


def test_paged_decode_head_dims():
    # D must be a multiple of 8 in 8..1024 (8..512 over caches read as bf16
    # hi + lo tiles: fp32, or fp16 under an fp32 q); checked before any HIP call
    lib = _lib.load()
    dummy = ctypes.c_void_p(16)
    for D, dt, want in ((4, _lib.SA_BF16, -6), (12, _lib.SA_BF16, -6), (516, _lib.SA_BF16, -6),
                        (1028, _lib.SA_BF16, -6), (1032, _lib.SA_BF16, -6), (2048, _lib.SA_BF16, -6),
                        (520, _lib.SA_F32, -6), (1024, _lib.paged_dtypes(_lib.SA_F32, _lib.SA_F16), -6)):
        s4 = (ctypes.c_int64 * 4)(8 * D, D, D, 1)
        o = (ctypes.c_int64 * 3)(8 * D, D, 1)
        st = lib.sa_paged_decode(dummy, dummy, dummy, dummy, dummy, dummy, 2, 8, 2, D, 16, 4, 8,
                                 s4, s4, s4, o, 4, 0.1, dt, dummy, 1 << 30, None)
        assert st == want, D
    for D in (8, 24, 200, 256, 264, 512, 520, 576, 1024):  # accepted: B = 0 returns before any launch
        s4 = (ctypes.c_int64 * 4)(8 * D, D, D, 1)
        o = (ctypes.c_int64 * 3)(8 * D, D, 1)
        assert lib.sa_paged_decode(dummy, dummy, dummy, dummy, dummy, dummy, 0, 8, 2, D, 16, 4, 8,
                                   s4, s4, s4, o, 4, 0.1, _lib.SA_BF16, dummy, 1 << 30, None) == 0
        assert lib.sa_paged_decode_workspace_size(2, 8, D, 4, 16) > 0


def test_rope_rotate_argument_errors():
    # checked before any HIP call: dtype, D a multiple of 16, null pointers,
    # 16-byte strides and alignment; B = 0 launches nothing
    lib = _lib.load()
    d = ctypes.c_void_p(16)
    s = (ctypes.c_int64 * 4)(4 * 64 * 64, 64 * 64, 64, 1)
    assert lib.sa_rope_rotate(d, d, d, d, 1, 4, 64, 64, s, 7, None) == -3
    assert lib.sa_rope_rotate(d, d, d, d, 1, 4, 64, 40, s, _lib.SA_BF16, None) == -2
    assert lib.sa_rope_rotate(None, d, d, d, 1, 4, 64, 64, s, _lib.SA_BF16, None) == -1
    odd = (ctypes.c_int64 * 4)(4 * 64 * 68, 64 * 68, 68, 1)  # rows 136 bytes apart (bf16)
    assert lib.sa_rope_rotate(d, d, d, d, 1, 4, 64, 64, odd, _lib.SA_BF16, None) == -5
    assert lib.sa_rope_rotate(ctypes.c_void_p(24), d, d, d, 1, 4, 64, 64, s, _lib.SA_BF16, None) == -5
    assert lib.sa_rope_rotate(d, d, d, d, 0, 4, 64, 64, s, _lib.SA_BF16, None) == 0


def test_flash_16bit_head_dims():
    # bf16 / fp16: any multiple of 8 in 8..512 (kernels for 32, 64, 128, 256, 512
    # read only the first D columns); the fp8 and fused-RoPE kernels take 32,
    # 64, 128 only.  Every check runs before any launch (B = 0 launches nothing).
    lib = _lib.load()
    d = ctypes.c_void_p(256)
    s = (ctypes.c_int64 * 4)(2 * 64 * 256, 64 * 256, 256, 1)
    fwd = lambda D, B=0: lib.sa_flash_fwd(d, d, d, d, None, B, 2, 2, 64, D, s, s, s, s, 0.1, 0, 0, _lib.SA_BF16,
                                          None)
    bwd = lambda D, B=0: lib.sa_flash_bwd(d, d, d, d, d, d, d, d, d, d, B, 2, 2, 64, D, s, s, s, s, s, s, s, s, 0.1,
                                          0, 0, _lib.SA_F16, None)
    for D in (0, 4, 12, 132, 250, 516, 520, 1024):
        assert fwd(D) == -6, D
        assert bwd(D) == -6, D
    for D in (8, 24, 40, 96, 128, 136, 200, 248, 256, 264, 400, 504, 512):
        assert fwd(D) == 0, D
        assert bwd(D) == 0, D
    fp8 = lambda D: lib.sa_flash_fp8_fwd(d, d, d, d, None, d, d, d, 0, 2, 2, 64, D, s, s, s, s, 0.1, 0,
                                         _lib.SA_FP8_E4M3FN, None)
    rope = lambda D: lib.sa_flash_rope_fwd(d, d, d, d, d, d, None, d, 1 << 20, 0, 2, 2, 64, D, s, s, s, s, 0.1, 0,
                                           _lib.SA_BF16, None)
    for D in (48, 96, 256):
        assert fp8(D) == -6, D
        assert rope(D) == -6, D
    assert fp8(64) == 0 and rope(64) == 0


def test_paged_decode_dtype_pairs():
    # SA_PAGED_DTYPES(q, cache): fp32 q over fp32 / bf16 / fp16 / e4m3fn
    # caches, bf16 q over e4m3fn caches, or one 16-bit type for both; other
    # pairs are refused before any HIP call, and e4m3fn caches need D a
    # multiple of 16
    lib = _lib.load()
    dummy = ctypes.c_void_p(16)
    D = 64
    s4 = (ctypes.c_int64 * 4)(8 * D, D, D, 1)
    o = (ctypes.c_int64 * 3)(8 * D, D, 1)
    pd = _lib.paged_dtypes
    assert pd(_lib.SA_F32, _lib.SA_BF16) == 0 | (3 << 8)
    for code in (pd(_lib.SA_BF16, _lib.SA_F32), pd(_lib.SA_BF16, _lib.SA_F16), pd(_lib.SA_F16, _lib.SA_BF16),
                 pd(_lib.SA_F16, _lib.SA_F32), _lib.SA_FP8_E4M3FN, pd(_lib.SA_F16, _lib.SA_FP8_E4M3FN), 7,
                 1 << 16, -1):
        st = lib.sa_paged_decode(dummy, dummy, dummy, dummy, dummy, dummy, 2, 8, 2, D, 16, 4, 8,
                                 s4, s4, s4, o, 4, 0.1, code, dummy, 1 << 30, None)
        assert st == -3, code  # SA_ERR_BAD_DTYPE
        st = lib.sa_paged_decode_noalloc(dummy, dummy, dummy, dummy, dummy, dummy, 2, 8, 2, D, 16, 4, 8,
                                         s4, s4, s4, o, 4, 0.1, code, None)
        assert st == -3, code
    s40 = (ctypes.c_int64 * 4)(8 * 40, 40, 40, 1)
    o40 = (ctypes.c_int64 * 3)(8 * 40, 40, 1)
    for q_type in (_lib.SA_F32, _lib.SA_BF16):
        st = lib.sa_paged_decode(dummy, dummy, dummy, dummy, dummy, dummy, 2, 8, 2, 40, 16, 4, 8, s40, s40, s40,
                                 o40, 4, 0.1, pd(q_type, _lib.SA_FP8_E4M3FN), dummy, 1 << 30, None)
        assert st == -6, q_type  # SA_ERR_UNSUPPORTED (an accepted pair, refused for D % 16)
    # fp32 rows need element strides that are multiples of 4, 16-bit rows of 8
    s_odd = (ctypes.c_int64 * 4)(8 * 68, 68, 68, 1)
    st = lib.sa_paged_decode(dummy, dummy, dummy, dummy, dummy, dummy, 2, 8, 2, D, 16, 4, 8,
                             s4, s_odd, s_odd, o, 4, 0.1, _lib.SA_BF16, dummy, 1 << 30, None)
    assert st == -5  # SA_ERR_BAD_STRIDE
