/*
 * C ABI of the gfx950 tile-local Strassen GEMM library (libstrassen_mi355x.so).
 *
 * Plain pointers and sizes only; the caller owns every buffer. Calls are
 * asynchronous on the given HIP stream (hipStream_t passed as void*, NULL =
 * the default stream), do not synchronise the host and keep no state beyond
 * an immutable kernel table and a thread-local error message.
 *
 * Reference interface replaced (paths relative to the reference checkout):
 *   smx_gemm  <- strassen_pallas.strassen_matmul(a, b, *, bm, bn, bk,
 *                interleave_products, epilogue, residual, bias, rope_cos,
 *                rope_sin, rope_scale, rope_head_dim, rope_eps, ...)
 *                (strassen_pallas.py:882-1221) with algo = SMX_ALGO_STRASSEN;
 *             <- benchmark_cubic_control.cubic_matmul(a, b, variant="blocked",
 *                bm, bn, bk) (experiments/qwen3/benchmark_cubic_control.py:116-177)
 *                with algo = SMX_ALGO_CUBIC (the matched 8-product control).
 *   smx_last_error / status codes <- the ValueError/RuntimeError raised by
 *                strassen_matmul's argument checks (strassen_pallas.py:927-1047).
 *   smx_tile_requirements <- check_tiling (strassen_pallas.py:127-140): the
 *                gfx950 kernel's divisibility rule for (bm, bn, bk).
 *   smx_strassen_weight_layout <- the offline weight relayouts
 *                (swiglu_weight_layout / rope_weight_layout,
 *                strassen_pallas.py:1315-1411): one more offline transform of a
 *                static weight, which stores the seven classical B operand sums
 *                of every (bk, bn) tile (strassen_pallas.py:324-379) so that
 *                smx_gemm only forms the A sums at run time.
 *   smx_version: no reference counterpart (ABI version query for bindings).
 */
#ifndef STRASSEN_MI355X_H
#define STRASSEN_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SMX_VERSION 2

/* Status codes. */
#define SMX_OK 0
#define SMX_ERR_INVALID 1     /* bad argument: maps to ValueError */
#define SMX_ERR_UNSUPPORTED 2 /* valid for the reference, not for this kernel: ValueError */
#define SMX_ERR_LAUNCH 3      /* HIP launch failure: RuntimeError */

/* Algorithms. */
#define SMX_ALGO_STRASSEN 7 /* one-level classical Strassen, 7 products */
#define SMX_ALGO_CUBIC 8    /* matched blocked cubic, 8 products */

/* Epilogues (strassen_pallas.py:739-879). */
#define SMX_EPI_NONE 0
#define SMX_EPI_SWIGLU 1       /* out[M, N/2] = silu(gate) * up; :762-777 */
#define SMX_EPI_RESIDUAL_ADD 2 /* out = acc + residual;          :778-792 */
#define SMX_EPI_BIAS_ADD 3     /* out = acc + bias[col];         :867-874 */
#define SMX_EPI_QK_NORM_ROPE 4 /* per-head RMSNorm + RoPE;       :793-835 */

/* Layout of B. */
#define SMX_B_KCONTIG 1   /* B^T stored row-major [N, K] (ldb >= K) */
#define SMX_B_PRESUMMED 2 /* Strassen weight [N/2 * 7, K/2] from smx_strassen_weight_layout (ldb >= K/2) */

/* desc.flags bits. */
#define SMX_FLAG_COMPACT_TILE 1 /* cubic: use the compact-tile (plain-weight Strassen) kernel */

/* aux_f32 bits: element type of the small auxiliary vectors. */
#define SMX_AUX_BIAS_F32 1  /* bias is float32 (else bf16) */
#define SMX_AUX_SCALE_F32 2 /* rope_scale is float32 (else bf16) */

typedef struct smx_gemm_desc {
  int64_t m, n, k;       /* C[m, n] = A[m, k] @ B[k, n] */
  int64_t lda, ldb, ldc; /* row strides in elements (A rows, B^T rows, C rows) */
  int64_t ldr;           /* residual row stride (residual_add) */
  int32_t bm, bn, bk;    /* Strassen quadrant tile: the reference's (bm, bn, bk) */
  int32_t algo;          /* SMX_ALGO_* */
  int32_t epilogue;      /* SMX_EPI_* */
  int32_t b_layout;      /* SMX_B_KCONTIG or SMX_B_PRESUMMED */
  int32_t rope_head_dim; /* qk_norm_rope head width (128) */
  float rope_eps;        /* qk_norm_rope epsilon */
  int32_t aux_f32;       /* SMX_AUX_* bits */
  int32_t flags;         /* SMX_FLAG_* bits */
} smx_gemm_desc;

/*
 * C = epilogue(A @ B). A: bf16 [m, k] row-major. B: bf16, layout b_layout
 * (SMX_B_PRESUMMED only with SMX_ALGO_STRASSEN, built for the same bn, bk).
 * C: bf16 [m, n] (or [m, n/2] for SwiGLU). residual: bf16 [m, n] (ldr).
 * bias: [n] bf16 or f32. rope_cos / rope_sin: bf16 [m, bn/2] tables indexed
 * by output row (rope_layout_tables). rope_scale: [bn] bf16 or f32
 * (rope_scale_layout). Unused pointers may be NULL.
 * Returns SMX_OK or an SMX_ERR_* code; smx_last_error() describes it.
 */
int smx_gemm(const smx_gemm_desc* desc, const void* a, const void* b, void* c, const void* residual,
             const void* bias, const void* rope_cos, const void* rope_sin, const void* rope_scale,
             void* stream);

/* Product-space workgroup tile (tm, tn) and K stage (tk) of the kernel that
 * serves (algo, epilogue, b_layout, flags): bm must be a multiple of 2*tm,
 * bn of 2*tn, bk of 2*tk. */
int smx_tile_requirements(int32_t algo, int32_t epilogue, int32_t b_layout, int32_t flags, int32_t* tm, int32_t* tn,
                          int32_t* tk);

/*
 * Pre-summed Strassen weight for the (bn, bk) tile: from B^T bf16 [n, k]
 * (row stride ldb) writes out bf16 [n/2 * 7, k/2] (row stride ldo): row
 * (p*7 + o) holds operand T_(o+1) of product-space column p, in order
 * B0+B3, B0, B1-B3, B2-B0, B3, B0+B1, B2+B3, each sum rounded once to bf16.
 * Needs n % bn == 0, k % bk == 0, bk % 16 == 0. Asynchronous on stream.
 */
int smx_strassen_weight_layout(int64_t n, int64_t k, const void* bt, int64_t ldb, int32_t bn, int32_t bk, void* out,
                               int64_t ldo, void* stream);

/* Message of the last failing call on this thread ("" if none). */
const char* smx_last_error(void);

/* SMX_VERSION of the built library. */
int smx_version(void);

#ifdef __cplusplus
}
#endif

#endif /* STRASSEN_MI355X_H */
