/*
 * smooth_attn_amd.h — C ABI of the MI355X (gfx950) smooth-attn hot path.
 *
 * Plain pointers, sizes and element strides; no torch types.  Every entry
 * point is asynchronous on the given HIP stream, allocates nothing (device
 * memory beyond the arguments is a caller workspace, or for
 * sa_paged_decode_noalloc a fixed module-scope array), and returns a status:
 *      0            success
 *     < 0           invalid argument (see sa_status_string)
 *     > 0           a hipError_t from the launch
 * Device pointers must stay valid until the stream reaches the launched work.
 *
 * Squareplus family: y = squareplus(alpha * (x - theta))^power,
 *   squareplus(a) = (a + sqrt(a^2 + 4)) / 2,  power in {1, 2, 3}.
 * Fused attention and decode use the default family (alpha=2, theta=0.5, p=2),
 * as the reference's fused kernels do.
 *
 * Citations are path:line into the reference (NoSelection/smooth-attn).
 */
#ifndef SMOOTH_ATTN_AMD_H
#define SMOOTH_ATTN_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* sa_stream_t; /* == hipStream_t */

/* Element types (also used for the fp8 storage type). */
enum {
    SA_F32 = 0,
    SA_F16 = 1,
    SA_BF16 = 2,
    SA_FP8_E4M3FN = 3
};

/* Status codes < 0. */
enum {
    SA_ERR_NULL_POINTER = -1,
    SA_ERR_BAD_SHAPE = -2,
    SA_ERR_BAD_DTYPE = -3,
    SA_ERR_BAD_FAMILY = -4,
    SA_ERR_BAD_STRIDE = -5,
    SA_ERR_UNSUPPORTED = -6,
    SA_ERR_WORKSPACE = -7
};

/* Human-readable text for a status code (static storage). */
const char* sa_status_string(int status);

/*
 * Row-wise or causal squareplus normalisation forward over the rows of a 2-D
 * view x[n_rows, n_cols] (element row strides; columns contiguous).
 *   causal == 0: y_ij = w_ij / (sum_j w_ij + 1e-12)
 *   causal != 0: row r attends to columns j <= (r mod n_cols); the rest of the
 *                row is written as exact zeros.
 * dtype: SA_F32 / SA_F16 / SA_BF16 for both x and y; fp32 arithmetic.
 * n_cols <= 8192.  n_rows * 64 * waves_per_row < 2^32 (one launch's work-item
 * count), i.e. n_rows < 2^26 for rows of up to four 1 KB chunks (one wave
 * per row), 2^24 for eight (4 waves) and 2^23 beyond (8 waves); more rows
 * return SA_ERR_BAD_SHAPE.  sa_norm_fwd_launch_info reports waves_per_row.
 * Replaces the launches of _softplus_norm_fwd (kernels.py:494-531, launched
 * by _launch_row_kernel_out :887-939), _softplus_norm_causal_fwd (:565-604),
 * _winner_squareplus_p2_causal_fwd (:607-637) and the tiered path
 * (:640-676, :1042-1094), reached from softplus_norm_triton_out (:1006-1031)
 * and softplus_norm_causal_triton_out (:1274-1297).
 */
int sa_norm_fwd(const void* x, void* y, int64_t n_rows, int64_t n_cols,
                int64_t x_row_stride, int64_t y_row_stride, int dtype,
                int causal, float alpha, float theta, int power,
                sa_stream_t stream);

/*
 * Fused backward of sa_norm_fwd:
 *   dx_j = dw_j/dx_j / S * (dy_j - sum_k dy_k P_k),  S = sum w + 1e-12, P = w/S
 * recomputing w from x.  Causal rows write exact zeros above the diagonal.
 * x_dtype is the dtype of x and dx; dy_dtype may be SA_F32 or x_dtype.
 * Replaces _softplus_norm_causal_backward (kernels.py:1197-1230) with its
 * kernels _softplus_norm_causal_bwd (:679-743),
 * _winner_squareplus_p2_causal_bwd (:746-794) and the tiered backward
 * (:797-849, :1097-1121); the row-wise case replaces autograd of
 * softplus_norm_eager (:1332-1346), for which the reference has no kernel.
 */
int sa_norm_bwd(const void* x, const void* dy, void* dx, int64_t n_rows,
                int64_t n_cols, int64_t x_row_stride, int64_t dy_row_stride,
                int64_t dx_row_stride, int x_dtype, int dy_dtype, int causal,
                float alpha, float theta, int power, sa_stream_t stream);

/*
 * Softmax over each row of a [n_rows, n_cols] matrix (the comparison
 * baseline).  causal != 0: row r sees columns 0 .. r mod n_cols (others are
 * written as 0).  fp32 arithmetic, exp(x - rowmax) / sum.  dtype as
 * sa_norm_fwd; n_cols <= 8192; n_rows * 64 * waves_per_row < 2^32
 * (sa_softmax_fwd_launch_info reports waves_per_row: 8 for rows of 16 or
 * more 1 KB chunks, else 1), else SA_ERR_BAD_SHAPE.
 * Replaces softmax_triton[_out] / softmax_causal_triton[_out]
 * (kernels.py:1233-1325) and the kernels _softmax_fwd (:534-562) and
 * _softmax_causal_fwd (:852-884).
 */
int sa_softmax_fwd(const void* x, void* y, int64_t n_rows, int64_t n_cols,
                   int64_t x_row_stride, int64_t y_row_stride, int dtype,
                   int causal, sa_stream_t stream);

/*
 * dst[c][r] = src[r][c] for a rows x cols matrix of 16-bit elements (bf16
 * or fp16; element row strides, multiples of 8, both pointers 16-byte
 * aligned).  Lays out the RoPE projection's W_o as [D_model, Hq*D] so the
 * projection runs as the faster GEMM form O (W_o^T)^T.  No counterpart in
 * the reference, whose projection kernel reads W_o per head
 * (kernels.py:2373-2426).
 */
int sa_transpose16(const void* src, void* dst, int64_t rows, int64_t cols,
                   int64_t src_row_stride, int64_t dst_row_stride,
                   sa_stream_t stream);

/* Row kernel variants (sa_launch_info.variant). */
enum {
    SA_ROW_SCALAR = 0, /* element loads (unaligned rows or n_cols % vec != 0) */
    SA_ROW_VEC = 1,    /* one wave per row, 16-byte loads */
    SA_ROW_SPLIT = 2   /* several waves per row, 16-byte loads */
};

/* The launch a row entry point makes for given arguments, and the compiled
 * kernel's resources (queried from the HIP runtime on the current device). */
typedef struct sa_launch_info {
    int variant;          /* SA_ROW_* */
    int grid_x;           /* blocks launched */
    int block_threads;    /* threads per block (64 per wave) */
    int rows_per_block;
    int waves_per_row;
    int elems_per_load;   /* elements per lane load: 16 bytes / element, or 1 */
    int row_pass_elems;   /* columns one pass over a row covers (power of 2) */
    int n_vgprs;          /* registers per lane of the compiled kernel */
    int shared_mem_bytes; /* static LDS per block */
    int blocks_per_cu;    /* resident blocks per CU (occupancy) */
} sa_launch_info;

/*
 * Describe, without launching, the kernel sa_norm_fwd (resp. sa_softmax_fwd)
 * runs for these arguments (x, y are only inspected for 16-byte alignment).
 * Returns a status as the launchers do.  Backs the launch metadata
 * (block_size, num_warps, num_programs, n_regs, shared_mem, occupancy) of
 * return_meta=True (kernels.py:287-317, :1154-1172), which the reference
 * reads from the compiled Triton kernel.
 */
int sa_norm_fwd_launch_info(const void* x, const void* y, int64_t n_rows,
                            int64_t n_cols, int64_t x_row_stride,
                            int64_t y_row_stride, int dtype, int power,
                            sa_launch_info* info);
int sa_softmax_fwd_launch_info(const void* x, const void* y, int64_t n_rows,
                               int64_t n_cols, int64_t x_row_stride,
                               int64_t y_row_stride, int dtype,
                               sa_launch_info* info);

/*
 * Fused causal squareplus attention forward (bf16, fp16 or fp32 q/k/v/o,
 * dtype SA_BF16 / SA_F16 / SA_F32; fp32 runs on the fp32 MFMA with P kept in
 * fp32):
 *   O_i = sum_{j<=i, i-j<W} y_ij V_j / (sum_j y_ij + 1e-12),
 *   y = squareplus(2 s - 1)^2,  s = scale * q_i . k_j
 * q,o: [B, Hq, T, D]; k,v: [B, Hkv, T, D]; Hq % Hkv == 0 (query head h reads
 * KV head h / (Hq/Hkv)).  *_strides are element strides for (b, h, t, d):
 * the d stride must be 1, the others multiples of 16 bytes (8 elements of a
 * 16-bit type, 4 of fp32), base pointers 16-byte aligned, and for bf16/fp16
 * K and V row strides at most 16 MiB.  row_sums (nullable): fp32 [B, Hq, T] contiguous,
 * receives sum_j y_ij + 1e-12.  window_size 0 = full causal.  D: bf16 /
 * fp16 any multiple of 8 in 8..512 (kernels built for 32, 64, 128, 256 and
 * 512 read only the first D columns and store only those), fp32 any
 * multiple of 4 in 4..512 (the same way).  exact_math != 0 selects a correctly rounded
 * sqrt.
 * Replaces _sp2norm_flash_fwd (kernels.py:1912-1931) and its kernel
 * _sp2norm_flash_fwd_with_rowsum_kernel (:1536-1631).
 */
int sa_flash_fwd(const void* q, const void* k, const void* v, void* o,
                 float* row_sums, int B, int Hq, int Hkv, int T, int D,
                 const int64_t* q_strides, const int64_t* k_strides,
                 const int64_t* v_strides, const int64_t* o_strides,
                 float scale, int window_size, int exact_math, int dtype,
                 sa_stream_t stream);

/*
 * Fused attention backward: dq, dk, dv of sa_flash_fwd given o, do and the
 * forward's row_sums.  Same layouts and constraints as sa_flash_fwd; dq has
 * q's strides argument dq_strides, dk/dv have KV shape.  delta_ws: fp32
 * workspace of B*Hq*T floats (receives rowsum(do * o)).
 * Replaces _sp2norm_flash_bwd (kernels.py:1934-1989) with its kernels
 * _sp2norm_flash_bwd_dq_kernel (:1667-1784) and
 * _sp2norm_flash_bwd_dkv_kernel (:1787-1909).
 */
int sa_flash_bwd(const void* q, const void* k, const void* v, const void* o,
                 const void* dout, const float* row_sums, void* dq, void* dk,
                 void* dv, float* delta_ws, int B, int Hq, int Hkv, int T,
                 int D, const int64_t* q_strides, const int64_t* k_strides,
                 const int64_t* v_strides, const int64_t* o_strides,
                 const int64_t* do_strides, const int64_t* dq_strides,
                 const int64_t* dk_strides, const int64_t* dv_strides,
                 float scale, int window_size, int exact_math, int dtype,
                 sa_stream_t stream);

/*
 * Bytes of workspace sa_flash_bwd_ws uses for these sizes: fp32 partial
 * dK / dV of the key blocks split over their query tiles, which the library
 * does for causal rows long against the grid (few batch x KV heads), where
 * the first key blocks, which see every query, would otherwise run alone at
 * the end; at most 512 MiB (head dims above 128: one buffer the dV and the
 * dK kernel take in turn).  0 when it does not split (fp32, grids that fill
 * the GPU); -1 for invalid sizes.
 */
int64_t sa_flash_bwd_workspace_size(int B, int Hq, int Hkv, int T, int D,
                                    int window_size, int dtype);

/*
 * sa_flash_bwd with the workspace above (16-byte aligned).  A smaller
 * workspace runs fewer splits (none when NULL or 0 bytes); results are the
 * same up to fp32 summation order in dK and dV.  The split path adds a
 * kernel summing the partials in a fixed order (head dims above 128: one
 * after the dV and one after the dK kernel), so results do not depend on
 * timing.  Replaces the same reference functions as sa_flash_bwd.
 */
int sa_flash_bwd_ws(const void* q, const void* k, const void* v, const void* o,
                    const void* dout, const float* row_sums, void* dq, void* dk,
                    void* dv, float* delta_ws, int B, int Hq, int Hkv, int T,
                    int D, const int64_t* q_strides, const int64_t* k_strides,
                    const int64_t* v_strides, const int64_t* o_strides,
                    const int64_t* do_strides, const int64_t* dq_strides,
                    const int64_t* dk_strides, const int64_t* dv_strides,
                    float scale, int window_size, int exact_math, int dtype,
                    void* workspace, int64_t workspace_bytes,
                    sa_stream_t stream);

/*
 * Per-tensor absmax quantisation to float8_e4m3fn, entirely on the device:
 *   scale = max(amax|x| / 448, 1e-12);  x8 = e4m3fn(clamp(x / scale, +-448))
 * x: n contiguous elements of dtype (SA_F32/SA_F16/SA_BF16); x8: n bytes.
 * amax_ws: one fp32 of workspace; scale_out: one fp32 (device) receiving
 * the scale.  No host synchronisation.
 * Replaces _quantize_to_fp8 (kernels.py:2592-2601), which syncs via .item().
 */
int sa_fp8_quantize(const void* x, void* x8, int64_t n, int dtype,
                    float* amax_ws, float* scale_out, sa_stream_t stream);

/*
 * fp8 fused causal attention forward.  q8, k8: float8_e4m3fn; v: e4m3fn
 * (v_dtype SA_FP8_E4M3FN, as the reference entry point quantises V) or bf16
 * (v_dtype SA_BF16).  Scales are device pointers to one fp32 each (v_scale
 * ignored, may be NULL, for bf16 v).  Scores = (q8 . k8) * q_s * k_s *
 * attn_scale on fp8 MFMA; y rounded to bf16 and multiplied with v (as bf16)
 * on bf16 MFMA, times v_s.  o: bf16 [B, Hq, T, D]; row_sums nullable.
 * Layout rules as sa_flash_fwd; D in {32, 64, 128} (the Python wrapper runs
 * head dims 129..512 on sa_flash_fwd with the fp8 codes widened to bf16).
 * Replaces _sp2norm_fp8_flash_fwd (kernels.py:2604-2627) and its kernel
 * _sp2norm_fp8_flash_fwd_kernel (:2498-2589).
 */
int sa_flash_fp8_fwd(const void* q8, const void* k8, const void* v, void* o,
                     float* row_sums, const float* q_scale,
                     const float* k_scale, const float* v_scale, int B,
                     int Hq, int Hkv, int T, int D, const int64_t* q_strides,
                     const int64_t* k_strides, const int64_t* v_strides,
                     const int64_t* o_strides, float attn_scale,
                     int window_size, int v_dtype, sa_stream_t stream);

/*
 * Rotate-half RoPE of a [B, H, T, D] tensor x (dtype SA_BF16, SA_F16 or
 * SA_F32; element strides x_strides, d stride 1, the others multiples of 16
 * bytes) into the contiguous
 * [B, H, T, D] buffer out: for each pair (d, d + D/2) of row t,
 * a' = a cos - b sin, b' = b cos + a sin in fp32 with cos/sin = fp32
 * contiguous [T, D/2] tables, rounded to the input type.  D a multiple of
 * 16; B * H * T * D / 16 (one work-item per pair) below 2^32, else
 * SA_ERR_BAD_SHAPE.  RoPE attention at head dims other than 32, 64 and 128 is this
 * rotation of Q and K followed by sa_flash_fwd.
 * Replaces the rotation step of _sp2norm_rope_flash_fwd_kernel
 * (kernels.py:2104-2224), which the reference runs only inside the fused
 * kernel.
 */
int sa_rope_rotate(const void* x, void* out, const float* cos_table,
                   const float* sin_table, int B, int H, int T, int D,
                   const int64_t* x_strides, int dtype, sa_stream_t stream);

/*
 * Bytes of workspace sa_flash_rope_fwd needs (the rotated K, contiguous
 * [B, Hkv, T, D] of the 16-bit type).  -1 for negative sizes.
 */
int64_t sa_flash_rope_workspace_size(int B, int Hkv, int T, int D);

/*
 * Fused attention forward with rotate-half RoPE on Q and K (V unrotated).
 *   cos_table, sin_table: fp32 contiguous [T, D/2], 16-byte aligned
 *     (precompute_rope_cos_sin); position t of every (b, h) row uses row t.
 *   k_rot_ws: workspace of sa_flash_rope_workspace_size() bytes; receives the
 *     rotated K (rotated once per row there; Q is rotated in registers).
 * Rotation in fp32, a' = a cos - b sin, b' = b cos + a sin for the pair
 * (d, d + D/2), rounded to the 16-bit type; everything else as sa_flash_fwd
 * (exact_math off).  dtype: SA_BF16 or SA_F16 (the reference rounds rotated
 * values to bf16 whatever the input type).
 * Replaces sp2norm_rope_flash_attention (kernels.py:2373-2426) and its kernel
 * _sp2norm_rope_flash_fwd_kernel (:2104-2224).  The RoPE + W_o variant
 * (kernels.py:2429-2487) is this entry point writing O in [B, T, Hq, D]
 * order (o_strides) followed by one library GEMM O[B*T, Hq*D] x
 * W_o[Hq*D, D_model] with fp32 accumulation, in place of the reference's
 * per-head bf16 atomic adds.
 */
int sa_flash_rope_fwd(const void* q, const void* k, const void* v,
                      const float* cos_table, const float* sin_table, void* o,
                      float* row_sums, void* k_rot_ws, int64_t ws_bytes, int B,
                      int Hq, int Hkv, int T, int D, const int64_t* q_strides,
                      const int64_t* k_strides, const int64_t* v_strides,
                      const int64_t* o_strides, float scale, int window_size,
                      int dtype, sa_stream_t stream);

/*
 * Bytes of workspace sa_paged_decode needs for these sizes: a plan of B + 2
 * int32 (padded to 16 bytes), then fp32 partials [B, Hq, n_slots, D] and
 * [B, Hq, n_slots] with n_slots = ceil(max_pages * page_size / (32 m)) + 1,
 * m = clamp(B * ceil(Hq / 8) * ceil(max_pages * page_size / 32) / 2048, 1,
 * 16), a floor on the 32-token tiles each wave takes (smaller batches spread
 * over more waves).
 */
int64_t sa_paged_decode_workspace_size(int B, int Hq, int D, int max_pages,
                                       int page_size);

/* dtype argument of the paged decode entry points: q's element type in the
 * low byte, the caches' type plus one in the next (0 there: the caches share
 * q's type, so a plain SA_BF16 / SA_F16 / SA_F32 means both). */
#define SA_PAGED_DTYPES(q_type, cache_type) ((q_type) | (((cache_type) + 1) << 8))

/*
 * Paged single-token decode through a block table.
 *   q: [B, Hq, 1, D] (strides q_strides, d stride 1)
 *   k_cache, v_cache: [n_pages, Hkv, page_size, D] (strides kv_strides /
 *     vv_strides, d stride 1)
 *   block_table: int32 [B, max_pages] (row stride bt_stride, unit col stride),
 *     entries in [0, n_pages) for the pages a sequence uses
 *   context_lens: int32 [B], each in [0, max_pages * page_size]
 * Out-of-range page ids and context lengths are clamped on the device (the
 * result is then meaningless but no memory outside the cache is read).
 *   out: bf16 [B, Hq, D] (strides o_strides)
 * out[b,h] = sum_{t<ctx_b} y_t V_t / (sum_t y_t + 1e-12) with
 * K_t = k_cache[block_table[b, t/P], h/(Hq/Hkv), t%P].  dtype:
 * SA_PAGED_DTYPES(q type, cache type), or one code for both; supported
 * pairs: bf16 / bf16, fp16 / fp16, fp32 / fp32, fp32 q over bf16, fp16 or
 * e4m3fn caches, bf16 q over e4m3fn caches (the reference upcasts q, K and V to fp32,
 * kernels.py:2716-2717, :2746, :2765; mixed pairs and fp32 run their
 * products as bf16 hi + lo splits, about 16 significant bits; e4m3fn values
 * widen to bf16 exactly, unscaled, and need D a multiple of 16).  Row strides (element units)
 * must be 16-byte multiples.  D a multiple of 8 in 8..1024 (kernels for 32,
 * 64, 128, 256, 512 and 1024, the last two with two and four waves per
 * block splitting the columns; smaller D read only their own columns), at
 * most 512 over fp32 caches and over fp16 caches with an fp32 q; page_size
 * a power of two (at most 2^20).
 * workspace: at least sa_paged_decode_workspace_size() bytes, 16-byte
 * aligned, no initialisation needed (a plan kernel writes it).
 * Replaces sp2norm_paged_attention (kernels.py:2776-2829) and its kernel
 * _sp2norm_paged_attention_kernel (:2681-2773).
 */
int sa_paged_decode(const void* q, const void* k_cache, const void* v_cache,
                    void* out, const int32_t* block_table,
                    const int32_t* context_lens, int B, int Hq, int Hkv,
                    int D, int page_size, int max_pages, int n_pages,
                    const int64_t* q_strides, const int64_t* kv_strides,
                    const int64_t* vv_strides, const int64_t* o_strides,
                    int64_t bt_stride, float scale, int dtype,
                    float* workspace, int64_t workspace_bytes,
                    sa_stream_t stream);

/* Device memory sa_paged_decode_noalloc keeps per device for its plan and
 * partials (64 MiB). */
#define SA_PAGED_NOALLOC_SCRATCH_BYTES (64LL << 20)

/*
 * sa_paged_decode without a workspace argument: allocates nothing and takes
 * no caller memory beyond its inputs and output, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference.  The plan and
 * the partials live in a module-scope device array of
 * SA_PAGED_NOALLOC_SCRATCH_BYTES that every device using the library holds
 * until the process ends; its address is looked up on the first call on a
 * device.  When sa_paged_decode's partials would not fit, the split is
 * coarsened (more 32-token tiles per wave, fewer partials); when even two
 * partials per (sequence, query head) do not fit (B * Hq * 2 * (D + 1) * 4
 * bytes plus the plan over 64 MiB) it returns SA_ERR_WORKSPACE.  Nothing in
 * the array needs to start at zero (the plan kernel writes what the other
 * kernels read).  Calls that overlap on one device (other streams, other
 * host threads) share the array and race: serialise them.  The first call
 * on a device (and the first per element type and head-dim class) looks up
 * the array's address and the kernels' occupancy on the host: make it
 * before capturing the call into a HIP graph.  Arguments and result as
 * sa_paged_decode.
 */
int sa_paged_decode_noalloc(const void* q, const void* k_cache,
                            const void* v_cache, void* out,
                            const int32_t* block_table,
                            const int32_t* context_lens, int B, int Hq,
                            int Hkv, int D, int page_size, int max_pages,
                            int n_pages, const int64_t* q_strides,
                            const int64_t* kv_strides,
                            const int64_t* vv_strides,
                            const int64_t* o_strides, int64_t bt_stride,
                            float scale, int dtype, sa_stream_t stream);

/*
 * Paged-KV cache writer (the step before sa_paged_decode): for sequence b
 * with current length context_lens[b] and new rows t < n_new,
 *   pos = context_lens[b] + t,  page = block_table[b, pos / page_size]
 *   k_cache[page, h, pos % page_size, :] = k_new[b, h, t, :]   (and v)
 * k_new, v_new: [B, Hkv, n_new, D] (new_strides, d stride 1); caches as in
 * sa_paged_decode.  Rows whose page index reaches max_pages or whose table
 * entry is outside [0, n_pages) are skipped.  context_lens is not updated
 * (the caller adds n_new).  dtype SA_F32, SA_BF16, SA_F16 or
 * SA_FP8_E4M3FN (the caches' type; the rows are copied as bytes); rows of
 * 16-byte multiples (D a multiple of 4 for fp32, of 8 for 16-bit types, of
 * 16 for e4m3fn).
 * No reference kernel: the reference fills caches with Python loops in its
 * tests (tests/test_paged_attention.py:10-73).
 */
int sa_paged_kv_append(const void* k_new, const void* v_new, void* k_cache,
                       void* v_cache, const int32_t* block_table,
                       const int32_t* context_lens, int B, int Hkv, int n_new,
                       int D, int page_size, int max_pages, int n_pages,
                       const int64_t* new_strides, const int64_t* kc_strides,
                       const int64_t* vc_strides, int64_t bt_stride, int dtype,
                       sa_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SMOOTH_ATTN_AMD_H */
