/* g950rt.h -- C ABI of the gfx950 hot-path module loader and launcher.
 *
 * One shared library (libg950rt.so) loads ONE code object (g950.hsaco, every
 * hot-path kernel built for gfx950) and launches an operator on caller-owned
 * device buffers.  It replaces, for the hot-path operators, the reference's
 * native runtime boundary:
 *
 *   reference                                   here
 *   a100c/runtime/a100rt.h:79-89  a100rt_view    g950_view   (same fields, 56 B)
 *   a100c/runtime/a100rt.h:94-98  a100rt_scalar  g950_scalar (same fields, 16 B)
 *   a100c/runtime/a100rt.h:58-72  dtype codes    G950_DTYPE_* (same values)
 *   a100c/runtime/a100rt.h:50-55  exit codes     G950_* return codes (same values)
 *   a100c/runtime/a100rt.h:176    operator_entry(launch)  -> g950_launch(...)
 *   a100c/runtime/main.c:50-177   operator_exec process    -> g950_open/launch/sync/close
 *
 * Views and scalars are passed in SORTED ARGUMENT-NAME order, exactly as the
 * reference host packer lays them out (a100_support/native_io.py:74,81); the
 * binary carries no names.  `data` of a view is a DEVICE pointer; shape and
 * strides (bytes) are host arrays.  Output views carry flag bit 0.
 *
 * Calls are asynchronous on `stream` (a hipStream_t; NULL = the null stream);
 * g950_sync() waits, so "launch then sync" meets the reference contract that a
 * launch has finished before it returns (ops/harness/compiler_api/
 * COMPILE_CONTRACT.md:73-74).  No C++ exception crosses this boundary.  Every
 * refusal happens on the host before any kernel is launched.
 */
#ifndef G950RT_H
#define G950RT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define G950_ABI_VERSION 1

/* return codes (values of A100RT_EXIT_*, a100c/runtime/a100rt.h:50-55) */
#define G950_OK 0
#define G950_USAGE 2      /* operator contract / shape / scalar refused */
#define G950_REJECTED 3   /* a view violates its storage or layout rules */
#define G950_RESOURCE 4   /* HIP error: module load, launch, allocation */
#define G950_REPEAT_MISMATCH 5 /* g950_exec: repeats produced different outputs */
#define G950_SYNC 6       /* stream synchronisation failed */

/* dtype codes (a100c/runtime/a100rt.h:58-72) */
enum g950_dtype {
  G950_DTYPE_BOOL = 1, G950_DTYPE_INT8 = 2, G950_DTYPE_UINT8 = 3,
  G950_DTYPE_INT16 = 4, G950_DTYPE_UINT16 = 5, G950_DTYPE_INT32 = 6,
  G950_DTYPE_UINT32 = 7, G950_DTYPE_INT64 = 8, G950_DTYPE_UINT64 = 9,
  G950_DTYPE_FLOAT16 = 10, G950_DTYPE_BFLOAT16 = 11, G950_DTYPE_FLOAT32 = 12,
  G950_DTYPE_FLOAT64 = 13
};

#define G950_VIEW_OUTPUT 1u

/* A strided view over one device allocation (layout of a100rt_view). */
typedef struct g950_view {
  void *data;              /* element base (device address) */
  const int64_t *shape;    /* ndim extents (host) */
  const int64_t *strides;  /* ndim BYTE strides (host) */
  uint64_t storage_size;   /* bytes of the allocation `storage` points at */
  uint32_t dtype;          /* enum g950_dtype */
  uint32_t ndim;
  uint32_t flags;          /* bit 0: output */
  uint32_t reserved_;
  void *storage;           /* allocation base (device address) */
} g950_view;

/* A typed scalar (layout of a100rt_scalar): raw little-endian value bits. */
typedef struct g950_scalar {
  uint32_t dtype;
  uint32_t size;
  uint64_t bits;
} g950_scalar;

/* Operator contracts.  Each names the reference kernel whose call signature
 * it takes; views / scalars are that kernel's arguments in sorted-name order.
 *
 * G950_OP_SOFTMAX      softmax_kernel (ops/suite/perf/softmax.py:21-32)
 *   views   x_ptr[R,C], y_ptr[R,C]                  f32 | bf16 | f16 (same)
 *   scalars n_cols
 * G950_OP_RMS_LAYERNORM  rms_layernorm_forward_kernel
 *                      (ops/suite/perf/fast_rms_layernorm.py:20-42)
 *   views   W[C], X[R,C], Y[R,C], r[R]
 *   scalars W_row_stride, X_row_stride, Y_row_stride, eps, n_cols, r_row_stride
 * G950_OP_LAYERNORM    layernorm_kernel (ops/suite/dev/fused_layernorm_triton.py:27-42)
 *   views   B[C], Mean[R], Rstd[R], W[C], X[R,C], Y[R,C]
 *   scalars N, eps, stride
 * G950_OP_MATMUL       matmul_kernel (ops/suite/perf/matmul.py:21-37)
 *   views   a_ptr[M,K], b_ptr[K,N] (any strides; K-contiguous b = column-major
 *           takes the MFMA path), y_ptr[M,N]
 *   scalars K, M, N
 * G950_OP_MATMUL_I8    8-bit integer tl.dot, int32 accumulate modulo 2^32, in the
 *                      four signedness pairs of the reference's i8 family
 *                      (a100c/plan/tiles.py:118-131: s x s, u x u, u x s, s x u)
 *   views   a_ptr i8|u8[M,K], b_ptr i8|u8[K,N], c_ptr i32[M,N]
 *   scalars K, M, N
 * G950_OP_MATMUL_I8_DEQUANT  8-bit integer GEMM + dequant epilogue
 *                      (per-column rule of ops/suite/perf/dequantize_matmul.py:29-38
 *                      plus a per-row A scale): y = bf16(acc * sa[m] * sb[n])
 *   views   a_ptr i8|u8[M,K], b_ptr i8|u8[K,N], sa_ptr f32[M], sb_ptr f32[N], y_ptr[M,N]
 *   scalars K, M, N
 * G950_OP_ATTENTION    attn_fwd_causal_kernel (ops/suite/perf/attn_fwd_causal.py:20-55)
 *                      with GQA (K/V may have fewer heads, ops/suite/dev/gqa.py:29)
 *   views   k_ptr[Z,Hkv,S,D], out_ptr[Z,H,S,D], q_ptr[Z,H,S,D], v_ptr[Z,Hkv,S,D]
 *   scalars CAUSAL, H, N_CTX, Z, scale, stride_* (16 element strides)
 * G950_OP_ATTENTION_LSE  same plus the per-row logsumexp output
 *                      (ops/suite/dev/flash_varlen_fwd_kernel.py:309,318-320)
 *   views   k_ptr, lse_ptr f32[Z,H,S], out_ptr, q_ptr, v_ptr
 *   scalars as G950_OP_ATTENTION
 * G950_OP_COPY         y = x, contiguous, 16-byte multiple (no reference
 *                      counterpart: the streaming-copy kernel that calibrates
 *                      the HBM traffic counters; same load/store path as the
 *                      row kernels)
 *   views   x, y
 * G950_OP_LOGSUMEXP    logsumexp_kernel (ops/suite/perf/logsumexp.py:16-38):
 *                      y[r] = max + log(sum(exp(x - max))) with the max taken
 *                      over non-NaN entries; NaN if the row holds a NaN, the
 *                      max itself if it is infinite
 *   views   x_ptr[R,C] f32 | bf16 | f16, y_ptr[R] (f32 in the reference)
 *   scalars n_cols
 * G950_OP_DEQUANTIZE   dequantize_kernel (ops/suite/perf/dequantize_matmul.py:28-43):
 *                      fpb[k,n] = float(b[k,n]) * b_scale[n], rounded once to
 *                      fpb's dtype (exact product: bit-equal to float64 then round)
 *   views   b_ptr i8[K,N], b_scale_ptr[N], fpb_ptr[K,N]; b_scale_ptr and fpb_ptr
 *           share one dtype (f32 | bf16 | f16)
 *   scalars K, N, stride_bk, stride_bn, stride_fpbk, stride_fpbn (element
 *           strides; must agree with the views wherever the extent exceeds 1)
 * G950_OP_FLASH_VARLEN flash_varlen_fwd_kernel (ops/suite/dev/flash_varlen_fwd_kernel.py:22-320):
 *                      variable-length batches (cu_seqlens_q/k, seqused_k),
 *                      GQA, causal and local windows (bottom-right aligned),
 *                      paged K/V; O = 0 and LSE = +inf for a row without keys
 *   views   alibi_slopes_ptr, cu_seqlens_k_ptr i32, cu_seqlens_q_ptr i32, k_ptr,
 *           o_ptr, p_ptr, page_table_ptr i32, philox_args, q_ptr, seqused_k_ptr i32,
 *           softmax_lse_ptr f32 (all 1-D flat buffers; q/k/v/o share one dtype)
 *   scalars the kernel's 46 non-pointer arguments with semantics, sorted
 *           (alibi_slopes_batch_stride, b, bk, block_size, d, h, h_hk_ratio, hk,
 *           is_alibi, is_causal, ... window_size_left, window_size_right);
 *           is_softcap, is_dropout, return_softmax, seqlenq_ngroups_swapped and
 *           is_alibi must be 0 (refused otherwise)
 * G950_OP_DEQUANT_MATMUL  dequantize_matmul fused into the GEMM: the
 *                      reference's dequantize_kernel (ops/suite/perf/
 *                      dequantize_matmul.py:28-43) feeding matmul_kernel
 *                      (ops/suite/perf/matmul.py:21-37) as one kernel:
 *                      y = a . (b * b_scale[n]), fp32 accumulation of a . b
 *                      (int8 exact in 16-bit floats), scale on the accumulator
 *   views   a_ptr[M,K] f32 | bf16 | f16, b_ptr i8[K,N] (K-contiguous for the MFMA
 *           path), b_scale_ptr[N] (a's dtype), y_ptr[M,N] float
 *   scalars K, M, N
 * G950_OP_SOFTMAX_INNER  softmax_kernel_inner (ops/suite/dev/softmax_kernel_inner.py:12-72):
 *                      row softmax of M rows of N contiguous elements at
 *                      input_ptr + m*N, written to output_ptr + m*N
 *   views   input_ptr, output_ptr: flat (any rank, C-contiguous, >= M*N
 *           elements), one float dtype
 *   scalars M, N; or M, N, ONE_TILE_PER_CTA, TILE_N (the constexprs): with
 *           ONE_TILE_PER_CTA != 0 and TILE_N < N only the first TILE_N
 *           elements of each row are normalised and written (:13-24); any
 *           other pair covers the whole row
 * G950_OP_LAYERNORM_ROW  _layer_norm_forward_row (ops/suite/dev/layer_norm_forward_row.py:11-36):
 *                      mean = sum(x)/n, rstd = 1/sqrt(sum(x^2)/n - mean^2 + eps),
 *                      x_hat = (x - mean)*rstd rounded to X's dtype, Y = x_hat*W + B
 *   views   B_ptr, Mean_ptr, RSTD_ptr, W_ptr, X_ptr, Y_ptr: flat (any rank,
 *           C-contiguous), addressed through the row strides; X/Y/W/B one float
 *           dtype, Mean/RSTD one float dtype
 *   scalars Mean_row_stride, RSTD_row_stride, X_row_stride, Y_row_stride, eps,
 *           n_cols, n_rows (eps, n_cols, n_rows are the kernel's constexprs;
 *           BLOCK_SIZE only shapes its tile)
 * G950_OP_GQA          gqa_kernel (ops/suite/dev/gqa.py:20-59): non-causal GQA
 *                      attention, query head h reads KV head h // GROUP
 *   views   K[Z,H_KV,N_CTX,D], Out[Z,H_Q,N_CTX,D], Q[Z,H_Q,N_CTX,D],
 *           V[Z,H_KV,N_CTX,D]; one float dtype; batch stride = heads x head
 *           stride (the kernel's batch offset, gqa.py:30-33)
 *   scalars GROUP, HEAD_DIM, H_KV, H_Q, N_CTX, scale, stride_kh, stride_kk,
 *           stride_kn, stride_oh, stride_om, stride_on, stride_qh, stride_qk,
 *           stride_qm, stride_vh, stride_vk, stride_vn (BLOCK_N only shapes the tile)
 */
enum g950_op {
  G950_OP_SOFTMAX = 1,
  G950_OP_RMS_LAYERNORM = 2,
  G950_OP_LAYERNORM = 3,
  G950_OP_MATMUL = 4,
  G950_OP_MATMUL_I8 = 5,
  G950_OP_MATMUL_I8_DEQUANT = 6,
  G950_OP_ATTENTION = 7,
  G950_OP_ATTENTION_LSE = 8,
  G950_OP_COPY = 9,
  G950_OP_LOGSUMEXP = 10,
  G950_OP_DEQUANTIZE = 11,
  G950_OP_FLASH_VARLEN = 12,
  G950_OP_DEQUANT_MATMUL = 13,
  G950_OP_SOFTMAX_INNER = 14,
  G950_OP_LAYERNORM_ROW = 15,
  G950_OP_GQA = 16
};

typedef struct g950_module g950_module;

/* Load the code object at `code_object_path` on the current HIP device.
 * Replaces the reference's per-operator executable load (a100c/runtime/main.c:50-110). */
int g950_open(const char *code_object_path, g950_module **out);

/* Validate the views/scalars against the operator contract, choose the kernel
 * variant from dtypes, shapes and strides, and launch it on `stream`.
 * Replaces operator_entry (a100c/runtime/a100rt.h:176) run by the worker pool
 * (a100c/runtime/pool.c:155-161). */
int g950_launch(g950_module *module, uint32_t op, const g950_view *views, uint32_t nviews,
                const g950_scalar *scalars, uint32_t nscalars, void *stream);

/* Bytes of the static device scratch array behind g950_launch_noalloc (one
 * per GPU, held from the module's load until the process ends); all of it
 * serves as workspace. */
#define G950_NOALLOC_SCRATCH_BYTES (32u << 20)

/* g950_launch that allocates nothing.  No counterpart in the reference: it is
 * for callers that cannot call hipMalloc (code under HIP graph capture, tight
 * serving loops, harnesses that forbid allocation).  Same contracts, checks
 * and results as g950_launch; workspace comes from the library's static
 * scratch array instead of hipMalloc, and no hipMalloc, hipFree or memset is
 * issued (no route needs memory cleared before it runs).  A call whose
 * workspace exceeds the scratch is refused with G950_USAGE, except the routes
 * that copy B first, which have a workspace-free alternative taken when the
 * copy does not fit: the widened W8A16 route (G950_OP_DEQUANT_MATMUL with
 * K-contiguous int8 b) takes the fused W8A16 kernel, and the row-major-B
 * routes that need a copy (G950_OP_MATMUL with row-major b the _rb kernels
 * do not take: fp32, M or N under 256, K not a multiple of 64;
 * G950_OP_DEQUANT_MATMUL with row-major int8 b) run g950_gemm_general, the
 * scalar-FMA kernel: same results within the GEMM tolerance, much slower;
 * g950_last_kernel names it.  All calls on one GPU share its array and it
 * keeps the last call's contents: calls that overlap on one GPU (different
 * streams or threads) race and must be ordered by the caller. */
int g950_launch_noalloc(g950_module *module, uint32_t op, const g950_view *views, uint32_t nviews,
                        const g950_scalar *scalars, uint32_t nscalars, void *stream);

/* Bytes of device workspace the module holds for launches on `stream` (0 if
 * it holds none): what g950_launch allocated there for split rows, copies of
 * B and int8 sums, grown on demand and freed by g950_close.  The runtime-side
 * counterpart of the reference's workspace queries
 * (operator_workspace_private/_shared, a100c/runtime/a100rt.h:180-181); it
 * lets a caller see that g950_launch_noalloc left it untouched. */
size_t g950_workspace_bytes(g950_module *module, void *stream);

/* Run every contract check and the kernel choice of g950_launch without
 * touching a device (no module, no HIP call).  On success
 * g950_last_kernel() names the kernel g950_launch would run.  The views'
 * pointers are only compared, never dereferenced. */
int g950_validate(uint32_t op, const g950_view *views, uint32_t nviews,
                  const g950_scalar *scalars, uint32_t nscalars);

/* Name of the kernel symbol the last successful g950_launch on this thread
 * ran (for profiling and tests); empty string if none. */
const char *g950_last_kernel(void);

/* Wait for all work on `stream`. */
int g950_sync(void *stream);

/* Static description of a return code. */
const char *g950_strerror(int code);

/* Detailed message of the last failure on this thread (like
 * a100rt_reject_reason, a100c/runtime/bundle.c:59-88, but with context). */
const char *g950_last_error(void);

/* Unload the code object. */
void g950_close(g950_module *module);

/* ---------------------------------------------------------------------------
 * a100-native-io/v1 bundles: the reference's host<->native argument image
 * (writer a100_support/native_io.py:49-150, reader a100c/runtime/bundle.c).
 * These calls replace the reference's bundle reader and the repeat loop of its
 * single-operator executable (a100c/runtime/main.c:50-177); the
 * `g950_exec` program (compiler_amd/csrc/g950_exec.cpp) is the command-line
 * counterpart of `operator_exec --bundle`.
 * ------------------------------------------------------------------------- */
typedef struct g950_bundle g950_bundle;

/* Map the file shared and write outputs back on close (the reference's
 * behaviour); without it the mapping is private and the file never changes. */
#define G950_BUNDLE_WRITE_BACK 1u

/* Rejection reasons: the reference reader's codes and names, same values
 * (a100c/runtime/bundle.c:31-88). */
enum g950_bundle_reason {
  G950_R_OPEN = 1, G950_R_SIZE, G950_R_MAGIC, G950_R_VERSION, G950_R_RESERVED, G950_R_MAP,
  G950_R_STORAGE_BOUNDS, G950_R_COUNT_BOUNDS, G950_R_ALLOC, G950_R_VIEW_TRUNCATED,
  G950_R_VIEW_STORAGE, G950_R_VIEW_DTYPE, G950_R_VIEW_OFFSET, G950_R_VIEW_DIM, G950_R_VIEW_REACH,
  G950_R_VIEW_FLAGS, G950_R_SCALAR_TRUNCATED, G950_R_SCALAR_WIDTH, G950_R_RELOC_TRUNCATED,
  G950_R_RELOC_VIEW, G950_R_RELOC_TABLE_WIDTH, G950_R_RELOC_TABLE_OUTPUT, G950_R_RELOC_ENTRY,
  G950_R_RELOC_OFFSET, G950_R_STORAGE_OVERLAPS_METADATA
};

/* Open, map and validate a bundle image (replaces a100rt_bundle_open,
 * a100c/runtime/bundle.c:111-339).  Every record is checked, in the
 * reference's order, before anything is returned: a violation returns
 * G950_REJECTED with *reason set and leaves the file untouched.  Host only. */
int g950_bundle_open(const char *path, uint32_t flags, g950_bundle **out, int *reason);

/* The same validation on an in-memory image (no file, nothing written). */
int g950_bundle_check(const void *image, uint64_t size, int *reason);

/* Name of a rejection reason (replaces a100rt_reject_reason,
 * a100c/runtime/bundle.c:59-88). */
const char *g950_bundle_reason(int reason);

/* Record counts: what = 0 storages, 1 views, 2 scalars, 3 relocations. */
uint32_t g950_bundle_count(const g950_bundle *bundle, int what);

/* View i over the mapped (host) image, and scalar i, in the image's order. */
int g950_bundle_view(const g950_bundle *bundle, uint32_t i, g950_view *out);
int g950_bundle_scalar(const g950_bundle *bundle, uint32_t i, g950_scalar *out);

/* Run operator `op` on the bundle `repeats` times on the current device
 * (replaces main.c:96-150 and the pool call): every storage is staged into its
 * own device allocation (pointer tables patched with device addresses), each
 * repeat restores all storages from the image first, outputs are compared
 * with the first repeat's byte for byte (*repeats_equal), and the first
 * repeat's outputs are written into the mapped image.  `lead` scalars are
 * prepended to the bundle's own (for constexprs with semantics that the image
 * does not carry, e.g. attention's CAUSAL).  Returns the launcher's code. */
int g950_bundle_exec(g950_module *module, g950_bundle *bundle, uint32_t op, const g950_scalar *lead,
                     uint32_t nlead, uint32_t repeats, void *stream, int *repeats_equal);

/* Unmap (syncing a write-back mapping to its file: G950_SYNC on failure). */
int g950_bundle_close(g950_bundle *bundle);

#ifdef __cplusplus
}
#endif

#endif /* G950RT_H */
