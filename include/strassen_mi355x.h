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
 *   smx_norm_residual_add <- the norm_residual_add epilogue (strassen_pallas.py:836-866),
 *                run as a second pass over an FP32 smx_gemm result.
 *   smx_qk_norm_rope <- the qk_norm_rope epilogue (strassen_pallas.py:793-835)
 *                for head widths other than 128, likewise a second pass.
 *   smx_last_error / status codes <- the ValueError/RuntimeError raised by
 *                strassen_matmul's argument checks (strassen_pallas.py:927-1047).
 *   smx_tile_requirements <- check_tiling (strassen_pallas.py:127-140): the
 *                gfx950 kernel's divisibility rule for (bm, bn, bk).
 *   smx_pack_operand / smx_packed_bytes <- the offline weight relayouts
 *                (swiglu_weight_layout / rope_weight_layout,
 *                strassen_pallas.py:1315-1411) and the in-kernel quadrant
 *                sums (strassen_pallas.py:324-379): a weight is packed once
 *                (its seven classical B operand sums per (bk, bn) tile, or its
 *                four quadrants for the cubic) and an activation once per call
 *                (its A sums / quadrants), into the fragment order the packed
 *                kernel streams into LDS.
 *   smx_version: no reference counterpart (ABI version query for bindings).
 */
#ifndef STRASSEN_MI355X_H
#define STRASSEN_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SMX_VERSION 12

/* Status codes. */
#define SMX_OK 0
#define SMX_ERR_INVALID 1     /* bad argument: maps to ValueError */
#define SMX_ERR_UNSUPPORTED 2 /* valid for the reference, not for this kernel: ValueError */
#define SMX_ERR_LAUNCH 3      /* HIP launch failure: RuntimeError */

/* Algorithms. */
#define SMX_ALGO_STRASSEN 7 /* one-level classical Strassen, 7 products */
#define SMX_ALGO_CUBIC 8    /* matched blocked cubic, 8 products */

/* Strassen formula variants (strassen_pallas.py formula_variant). */
#define SMX_FORMULA_CLASSICAL 0 /* P1..P7, :324-379 */
#define SMX_FORMULA_DUAL 1      /* Q1..Q7, :461-517 */
#define SMX_FORMULA_POWERS 2    /* R1..R7 into a decoded output basis, :381-459 / :744-760; no fused epilogue */

/* Epilogues (strassen_pallas.py:739-879). */
#define SMX_EPI_NONE 0
#define SMX_EPI_SWIGLU 1       /* out[M, N/2] = silu(gate) * up; :762-777 */
#define SMX_EPI_RESIDUAL_ADD 2 /* out = acc + residual;          :778-792 */
#define SMX_EPI_BIAS_ADD 3     /* out = acc + bias[col];         :867-874 */
#define SMX_EPI_QK_NORM_ROPE 4 /* per-head RMSNorm + RoPE;       :793-835 */
#define SMX_EPI_GEGLU 5        /* out[M, N/2] = gelu_tanh(gate) * up; :143-153 */

/* Layout of A. */
#define SMX_A_ROWMAJOR 0 /* A row-major [M, K] (lda >= K) */
#define SMX_A_PACKED 1   /* smx_pack_operand(algo, SMX_SIDE_LHS, ...) output */

/* Layout of B. */
#define SMX_B_KCONTIG 1 /* B^T stored row-major [N, K] (ldb >= K) */
#define SMX_B_PACKED 2  /* smx_pack_operand(algo, SMX_SIDE_RHS, ...) output */

/* Operand side for smx_pack_operand. */
#define SMX_SIDE_LHS 0 /* A [M, K] */
#define SMX_SIDE_RHS 1 /* B^T [N, K] */
#define SMX_SIDE_LHS_T 2 /* A stored transposed as [K, M] (strassen_matmul_lhs_transposed, :1224-1312) */

/* desc.flags bits. */
#define SMX_FLAG_OUT_F32 1 /* C is float32 (the unrounded FP32 result, output_dtype=float32, :1048-1057) */
/* Strassen on packed operands: run the product-major kernel, which takes the
 * seven products of a 128 x 256 product-space tile one after another over
 * the whole K range into three FP32 register sets (the default kernel keeps
 * seven sets of a 128 x 128 tile), parking two partial sets per workgroup in
 * the workspace (smx_gemm_workspace_bytes). It streams 384 operand bytes per
 * MFMA instead of 512. Calls it cannot take run the default kernel: another
 * formula, the qk_norm_rope epilogue, an FP32 partial, bm/2 not a multiple of
 * 128, bn/2 not a multiple of 256, or K not a multiple of 128. No counterpart
 * in the reference (a kernel choice of gfx950). */
#define SMX_FLAG_PRODUCT_MAJOR 2
/* Strassen on packed operands: the product-major kernel for the leading
 * tile columns whose tiles fill whole rounds of the device's CUs, the
 * default kernel (with its K split of a partly filled last round) for the
 * columns after them. The product-major kernel streams fewer operand bytes
 * per MFMA but has no K split, so a partly filled last round of its tiles
 * (twice the default kernel's size) runs as long as a full one: this flag
 * keeps it to whole rounds. The head's columns end on a bn tile boundary.
 * A call whose product-major tiles fill no whole round, with K below 4096
 * (where the product-major kernel's per-tile costs outweigh its lead), or
 * that the product-major kernel cannot take (as for SMX_FLAG_PRODUCT_MAJOR),
 * runs on the default kernel alone. The workspace (smx_gemm_workspace_bytes) then
 * serves both parts, one after the other. Not together with
 * SMX_FLAG_PRODUCT_MAJOR. No counterpart in the reference (a kernel choice
 * of gfx950). */
#define SMX_FLAG_PRODUCT_MAJOR_ROUNDS 4

/* aux_f32 bits: element type of the small auxiliary vectors. */
#define SMX_AUX_BIAS_F32 1  /* bias is float32 (else bf16) */
#define SMX_AUX_SCALE_F32 2 /* rope_scale is float32 (else bf16) */
#define SMX_AUX_RESIDUAL_F32 4 /* residual is float32 (else bf16) */

/* Source element type for smx_pack_operand. */
#define SMX_DTYPE_BF16 0
#define SMX_DTYPE_F32 1 /* FP32 inputs: operand sums formed in float, each operand rounded once to bf16 */

/* smx_norm_residual_add dtype bits (else bf16). */
#define SMX_NRA_SCALE_F32 1
#define SMX_NRA_RESIDUAL_F32 2
#define SMX_NRA_OUT_F32 4

/* smx_qk_norm_rope dtype bits (else bf16). */
#define SMX_QK_SCALE_F32 1
#define SMX_QK_OUT_F32 4

typedef struct smx_gemm_desc {
  int64_t m, n, k;       /* C[m, n] = A[m, k] @ B[k, n] */
  int64_t lda, ldb, ldc; /* row strides in elements (A rows, B^T rows, C rows) */
  int64_t ldr;           /* residual row stride (residual_add) */
  int32_t bm, bn, bk;    /* Strassen quadrant tile: the reference's (bm, bn, bk) */
  int32_t algo;          /* SMX_ALGO_* */
  int32_t epilogue;      /* SMX_EPI_* */
  int32_t a_layout;      /* SMX_A_ROWMAJOR or SMX_A_PACKED */
  int32_t b_layout;      /* SMX_B_KCONTIG or SMX_B_PACKED */
  int32_t rope_head_dim; /* qk_norm_rope head width (128) */
  float rope_eps;        /* qk_norm_rope epsilon */
  int32_t aux_f32;       /* SMX_AUX_* bits */
  int32_t flags;         /* SMX_FLAG_* bits */
  int32_t formula;       /* SMX_FORMULA_* (Strassen; packed operands built with the same formula) */
  int32_t block_permutation; /* 0..7: bit 0 swaps row halves, bit 1 K halves, bit 2 column halves (:205-226) */
  /* Cubic only, packed operands: NULL, or an FP32 [m, n] partial product
   * (row stride ldp >= n, 16-byte aligned rows) added to the quadrants
   * before the epilogue. An exact-panel schedule
   * (classical_panels / panel_schedule, :575-586, :713-735) is the Strassen
   * GEMM over the ordinary K panels with an FP32 result, then the cubic GEMM
   * over the exact panels with that result as its partial. */
  const float* partial;
  int64_t ldp;
  /* Optional device workspace (NULL, or workspace_bytes >= the
   * smx_gemm_workspace_bytes of this descriptor, 16-byte aligned). With it,
   * the tiles of a packed launch's last, partly filled round (every tile of
   * a launch under one round) run as K shares, up to 16, so that the round
   * finishes soonest; the shares go into this FP32 buffer and a pass sums
   * them and applies the epilogue. Without it every tile runs over full K.
   * The result is the same up to FP32 summation order. */
  void* workspace;
  int64_t workspace_bytes;
} smx_gemm_desc;

/*
 * C = epilogue(A @ B). Operands: either A bf16 [m, k] row-major (lda) with
 * B^T bf16 [n, k] row-major (ldb), served by the compact kernel that forms
 * the operand sums in registers; or both packed by smx_pack_operand for the
 * same algo and (bm, bk) / (bn, bk), served by the packed kernel (lda / ldb
 * ignored). C: bf16 [m, n] (or [m, n/2] for SwiGLU / GeGLU), float32 with
 * SMX_FLAG_OUT_F32. residual: [m, n] (ldr), bf16 or float32
 * (SMX_AUX_RESIDUAL_F32). bias: [n] bf16 or f32. rope_cos / rope_sin: bf16 [m, bn/2] tables
 * indexed by output row (rope_layout_tables). rope_scale: [bn] bf16 or f32
 * (rope_scale_layout). Unused pointers may be NULL. The epilogue moves C,
 * residual and partial rows, and reads the RoPE tables and scale, in 16-byte chunks:
 * those pointers must be 16-byte aligned and their row strides keep every
 * row 16-byte aligned (ldc, ldr a multiple of 8 elements for bf16, 4 for
 * float32; ldp a multiple of 4). The packed kernel orders its tiles over the
 * XCDs by the packed operand sizes (what of them the 256 MB MALL keeps across
 * rounds); SMX_RASTER=spread|chunks|blocks in the environment, read once per
 * process, forces an order. Every order gives the same result.
 * Returns SMX_OK or an SMX_ERR_* code; smx_last_error() describes it.
 */
int smx_gemm(const smx_gemm_desc* desc, const void* a, const void* b, void* c, const void* residual,
             const void* bias, const void* rope_cos, const void* rope_sin, const void* rope_scale,
             void* stream);

/*
 * Allocation-free variant of smx_gemm, with no counterpart in the reference:
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). It takes
 * a row-major bf16 A (desc->a_layout = SMX_A_ROWMAJOR, row stride lda) and a
 * packed B (desc->b_layout = SMX_B_PACKED, from smx_pack_operand for the
 * same algo, formula, block permutation and tile), packs A into a device
 * scratch array that the library holds for the life of the process (256 MiB
 * on every GPU it runs on), then runs the packed kernel: the result equals
 * smx_pack_operand of A into a caller buffer followed by smx_gemm. The packed
 * A needs smx_packed_bytes(algo, M, K) bytes (about M/2 * K/2 * nops * 2, nops
 * 7 for Strassen, 4 for the cubic), so M * K must stay at or below about
 * 76,695,844 (Strassen) or 134,217,728 (cubic); larger calls fail with SMX_ERR_UNSUPPORTED before any launch. No
 * FP32 partial (desc->partial must be null). A workspace in the descriptor
 * (smx_gemm_workspace_bytes sizes this descriptor as the packed call it
 * becomes) is checked, with every other argument, before anything is
 * launched. Calls allocate nothing. Every
 * call on one GPU shares that GPU's scratch: calls that overlap on one GPU
 * (different streams, or another thread) race, so a caller serialises them.
 */
int smx_gemm_noalloc(const smx_gemm_desc* desc, const void* a, const void* b, void* c, const void* residual,
                     const void* bias, const void* rope_cos, const void* rope_sin, const void* rope_scale,
                     void* stream);

/* Bytes of device workspace with which smx_gemm runs this descriptor's
 * call: for a call on the product-major kernel (SMX_FLAG_PRODUCT_MAJOR),
 * 256 KB per 128 x 256 product tile, (M/2 / 128) (N/2 / 256) tiles, which
 * the call then requires. With SMX_FLAG_PRODUCT_MAJOR_ROUNDS, the larger of
 * that for the product-major head and the K split's bytes below for the
 * rest (required when a head runs). Otherwise the bytes (s * r * 256 KB: one dense
 * 256 x 256 FP32 block per K share and split tile) with which
 * smx_gemm splits tiles of this descriptor's launch over K, on the current
 * device. T tiles on the device's C CUs make T / C whole rounds and a last
 * round of r = T mod C tiles; those r tiles split into the s shares,
 * 2 <= s <= min(16, K / 512, 2^30 / (r * 256 KB)), that minimise
 * ceil(s r / C) (1/s + f) + s r g (f = 400 / K, g = (5/3) / K: a workgroup's
 * fixed time and the summing pass's traffic, in units of a full-K tile's
 * time), when that is under 0.95 (1 + f). 0 when no split applies: an
 * unpacked call, an FP32 partial, K below 2048, r = 0, or no s that shortens
 * the round. Takes a descriptor smx_gemm accepts; no operand pointer is read.
 * SMX_TAIL_SPLIT=0 in the environment turns the split off. No counterpart in
 * the reference (a launch shape of gfx950). A row-major A with a packed B
 * (smx_gemm_noalloc's descriptor) is sized as the packed call it becomes. */
int smx_gemm_workspace_bytes(const smx_gemm_desc* desc, int64_t* bytes);

/* Tile granules of the kernels that serve (algo, epilogue, b_layout): bm
 * must be a multiple of 2*tm, bn of 2*tn, bk of 2*tk. Packed operands: 8, 128,
 * 32 (every bm the reference's check_tiling allows, strassen_pallas.py:127-140;
 * a bm/2 that is not a multiple of the kernels' 128-row product tile runs
 * their thin-tiling instantiations); unpacked: 128, 64, 32. */
int smx_tile_requirements(int32_t algo, int32_t epilogue, int32_t b_layout, int32_t flags, int32_t* tm, int32_t* tn,
                          int32_t* tk);

/* Bytes of the packed form of a [rows, k] operand for algo: R * k/2 * nops *
 * 2, with R = rows/2 rounded up to a multiple of 128 (product rows of a thin
 * tiling's last tile are zero padding) and nops = 7 for Strassen, 4 for the
 * cubic. */
int smx_packed_bytes(int32_t algo, int64_t rows, int64_t k, int64_t* bytes);

/*
 * Packs one operand for the packed kernel. side SMX_SIDE_LHS: src is A
 * [rows = m, k] and tile_rows = bm; SMX_SIDE_LHS_T: src is the same A stored
 * transposed, [k, rows = m] with row stride ld >= m; SMX_SIDE_RHS: src is
 * B^T [rows = n, k] and tile_rows = bn. src_dtype: SMX_DTYPE_BF16, or
 * SMX_DTYPE_F32 for FP32 inputs (operand sums formed in float, every operand
 * rounded once to bf16: the one-pass bf16 product of the reference's FP32
 * path at DEFAULT precision). passes: bf16 passes per product, 1, or for a
 * float32 source 3 (dot_precision HIGH) or 6 (HIGHEST): each operand v is
 * split into bf16 parts p0 = bf16(v), p1 = bf16(v - p0), p2 = bf16(v - p0 - p1).
 * The packed K runs pass-major: with slots = k / (passes * bk) panels per
 * pass, packed panel j holds pass j / slots of panel slot j % slots; the A
 * side carries parts (1, 0, 0) or (2, 1, 0, 1, 0, 0) over the passes and the
 * B side (0, 1, 0) or (0, 1, 2, 0, 1, 0) (smallest products first), so that
 * one GEMM over the packed K = passes x the source K sums every pass product
 * in FP32.
 * Strassen (algo 7) stores the seven operand sums of
 * P1..P7 (A0+A3, A2+A3, A0, A3, A0+A1, A2-A0, A1-A3; B0+B3, B0, B1-B3,
 * B2-B0, B3, B0+B1, B2+B3), each rounded once to bf16, or those of the dual /
 * powers formula, after the block permutation's quadrant swaps (A uses bits 0
 * and 1, B bits 1 and 2); the cubic (algo 8, formula 0, permutation 0) stores
 * the four quadrants. panels: NULL, or device int32 [slots] naming the
 * source K panel (of bk columns) that each slot reads (in every pass), from a
 * source src_k wide (entries are clamped to 0 .. src_k/bk - 1); this packs
 * the ordinary or the exact panels of an exact-panel schedule (without a map,
 * src_k = k / passes). out
 * (smx_packed_bytes bytes, 16-byte aligned)
 * is laid out [R/128][k/32][nops][4][64][8] bf16 (R as in smx_packed_bytes):
 * fragment (tile of 128 product rows, stage of 16 product k, operand, 32-row
 * block), lane l holding row l%32, depth 8*(l/32)..+8. Product row P is row
 * P % (tile_rows/2) of row tile P / (tile_rows/2); rows past rows/2 are
 * zeros. Needs rows % tile_rows == 0, k % (passes * bk) == 0, tile_rows % 16
 * == 0 (A sides) or % 256 == 0 (RHS), bk % 64 == 0, ld >= src_k, rows 16-byte
 * aligned (ld % 8 for bf16, % 4 for float32; LHS_T: ld >= m). Asynchronous
 * on stream.
 */
int smx_pack_operand(int32_t algo, int32_t formula, int32_t block_permutation, int32_t side, int64_t rows, int64_t k,
                     const void* src, int32_t src_dtype, int32_t passes, int64_t ld, int32_t tile_rows,
                     int32_t bk, const int32_t* panels, int64_t src_k, void* out, void* stream);

/*
 * Second pass of the norm_residual_add epilogue (strassen_pallas.py:836-866),
 * whose norm spans a whole output row: from the FP32 product x [m, n] (an
 * smx_gemm with SMX_FLAG_OUT_F32 and no epilogue) writes
 * out = x * rsqrt(mean_row(x^2) + eps) * scale[col] + residual, with
 * residual and out [m, n] and scale [n]; each bf16 or float32 by the dtypes
 * bits (SMX_NRA_*).
 * Asynchronous on stream.
 */
int smx_norm_residual_add(int64_t m, int64_t n, const float* x, int64_t ldx, const void* residual, int64_t ldr,
                          const void* scale, int32_t dtypes, float eps, void* out, int64_t ldo, void* stream);

/*
 * Second pass of the qk_norm_rope epilogue (strassen_pallas.py:793-835) for
 * head widths the fused epilogue does not take (it fuses head_dim 128): from
 * the FP32 product x [m, n] (an smx_gemm with SMX_FLAG_OUT_F32 and no
 * epilogue, on the rope-laid-out weight) writes out [m, n]. In each column
 * tile of bn, head h of the bn / head_dim heads pairs columns c in
 * [h head_dim/2, (h+1) head_dim/2) of the first half (a) and the second half
 * (b): recip = 1/sqrt((sum a^2 + sum b^2)/head_dim + eps), na = a recip
 * scale[c], nb = b recip scale[bn/2 + c], out_a = na cos - nb sin, out_b =
 * nb cos + na sin, with rope_cos / rope_sin bf16 [m, bn/2] at (row, c) and
 * rope_scale [bn] (the layouts of rope_layout_tables / rope_scale_layout).
 * dtypes: SMX_QK_* bits. Needs bn % (2 head_dim) == 0, n % bn == 0 and
 * (bn + bn/head_dim) * 4 <= 65536. Asynchronous on stream.
 */
int smx_qk_norm_rope(int64_t m, int64_t n, const float* x, int64_t ldx, const void* rope_cos, const void* rope_sin,
                     const void* rope_scale, int32_t dtypes, int32_t bn, int32_t head_dim, float eps, void* out,
                     int64_t ldo, void* stream);

/* Message of the last failing call on this thread ("" if none). */
const char* smx_last_error(void);

/* SMX_VERSION of the built library. */
int smx_version(void);

#ifdef __cplusplus
}
#endif

#endif /* STRASSEN_MI355X_H */
