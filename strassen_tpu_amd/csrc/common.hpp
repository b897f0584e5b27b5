// Shared device helpers for the gfx950 Strassen / cubic GEMM kernels:
// bf16 packing, kernel parameters, workgroup-to-tile mapping and the fused
// epilogues (strassen_pallas.py:739-879).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/strassen_mi355x.h"

namespace smx {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;  // 4 waves of 64

// ---------------------------------------------------------------------------
// bf16 helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ float lo_f32(uint32_t x) { return __uint_as_float(x << 16); }
__device__ __forceinline__ float hi_f32(uint32_t x) { return __uint_as_float(x & 0xffff0000u); }

// Round two floats to bf16 (ties to even) and pack: v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  bf16x2 v;
  v[0] = (__bf16)lo;
  v[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t x) { return __uint_as_float(((uint32_t)x) << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
  __bf16 v = (__bf16)x;
  return __builtin_bit_cast(uint16_t, v);
}

// Eight bf16 values unpacked to float.
struct F8 {
  float v[8];
};

__device__ __forceinline__ F8 unpack8(u32x4 x) {
  F8 f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f.v[2 * i] = lo_f32(x[i]);
    f.v[2 * i + 1] = hi_f32(x[i]);
  }
  return f;
}

// bf16(x + y) or bf16(x - y) per element. Two bf16 values sum exactly or
// within half a float ulp in float, and float keeps >= 2*8+2 bits, so
// rounding the float sum to bf16 gives the correctly rounded bf16 sum.
template <bool kSub>
__device__ __forceinline__ u32x4 sum8(const F8& x, const F8& y) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float s0 = kSub ? x.v[2 * i] - y.v[2 * i] : x.v[2 * i] + y.v[2 * i];
    float s1 = kSub ? x.v[2 * i + 1] - y.v[2 * i + 1] : x.v[2 * i + 1] + y.v[2 * i + 1];
    r[i] = pack_bf16(s0, s1);
  }
  return r;
}

// The seven classical A operands of P1..P7 (strassen_pallas.py:324-379) from
// the four raw A quadrants: A0+A3, A2+A3, A0, A3, A0+A1, A2-A0, A1-A3.
__device__ __forceinline__ void strassen_a_ops(const u32x4 (&q)[4], u32x4 (&ops)[7]) {
  const F8 a0 = unpack8(q[0]), a1 = unpack8(q[1]), a2 = unpack8(q[2]), a3 = unpack8(q[3]);
  ops[0] = sum8<false>(a0, a3);
  ops[1] = sum8<false>(a2, a3);
  ops[2] = q[0];
  ops[3] = q[3];
  ops[4] = sum8<false>(a0, a1);
  ops[5] = sum8<true>(a2, a0);
  ops[6] = sum8<true>(a1, a3);
}

// The seven classical B operands of P1..P7 from the four raw B quadrants:
// B0+B3, B0, B1-B3, B2-B0, B3, B0+B1, B2+B3.
__device__ __forceinline__ void strassen_b_ops(const u32x4 (&q)[4], u32x4 (&ops)[7]) {
  const F8 b0 = unpack8(q[0]), b1 = unpack8(q[1]), b2 = unpack8(q[2]), b3 = unpack8(q[3]);
  ops[0] = sum8<false>(b0, b3);
  ops[1] = q[0];
  ops[2] = sum8<true>(b1, b3);
  ops[3] = sum8<true>(b2, b0);
  ops[4] = q[3];
  ops[5] = sum8<false>(b0, b1);
  ops[6] = sum8<false>(b2, b3);
}

// bf16 round trip of a float (round to nearest even).
__device__ __forceinline__ float round_bf16(float x) { return bf16_to_f32(f32_to_bf16(x)); }

// Elementwise x + y or x - y in float, unrounded.
template <bool kSub>
__device__ __forceinline__ F8 add8(const F8& x, const F8& y) {
  F8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r.v[i] = kSub ? x.v[i] - y.v[i] : x.v[i] + y.v[i];
  return r;
}

// Elementwise map of four unpacked quadrants to one float operand.
template <class F>
__device__ __forceinline__ F8 map8(const F8& x0, const F8& x1, const F8& x2, const F8& x3, F f) {
  F8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r.v[i] = f(x0.v[i], x1.v[i], x2.v[i], x3.v[i]);
  return r;
}

// Formula variants of strassen_pallas.py (formula_variant): 0 classical
// (:324-379), 1 dual (:461-517), 2 powers (:381-459).
constexpr int kFormulaClassical = 0, kFormulaDual = 1, kFormulaPowers = 2;

// Eight floats rounded to bf16 and packed (round to nearest even).
__device__ __forceinline__ u32x4 pack8(const F8& x) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = pack_bf16(x.v[2 * i], x.v[2 * i + 1]);
  return r;
}

// Part `part` of the bf16 expansion of a float v = p0 + p1 + p2 + r:
// p0 = bf16(v), p1 = bf16(v - p0), p2 = bf16(v - p0 - p1). Each remainder
// is exact in float (v and its bf16 rounding share the exponent range), so
// the parts are those of the exact value.
__device__ __forceinline__ float bf16_part(float v, int part) {
  const float p0 = round_bf16(v);
  if (part == 0) return p0;
  const float r1 = v - p0;
  const float p1 = round_bf16(r1);
  return part == 1 ? p1 : round_bf16(r1 - p1);
}

__device__ __forceinline__ u32x4 pack8_part(const F8& x, int part) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = pack_bf16(bf16_part(x.v[2 * i], part), bf16_part(x.v[2 * i + 1], part));
  return r;
}

// Multi-pass bf16 products of FP32 operands (dot_precision HIGH: 3 passes,
// HIGHEST: 6). Pass i multiplies part pass_part(A, i) of the A operand by
// part pass_part(B, i) of the B operand, smallest products first so that
// the FP32 accumulator takes the leading p0*p0 pass last: p1*p0, p0*p1,
// p0*p0 (3 passes); p2*p0, p1*p1, p0*p2, p1*p0, p0*p1, p0*p0 (6 passes).
// The tables hold the part of pass i in bits 4i..4i+3.
constexpr uint32_t kPassPartsA3 = 0x001, kPassPartsB3 = 0x010;
constexpr uint32_t kPassPartsA6 = 0x001012, kPassPartsB6 = 0x010210;

__device__ __forceinline__ int pass_part(bool side_b, int passes, int pass) {
  const uint32_t table = passes == 3 ? (side_b ? kPassPartsB3 : kPassPartsA3)
                         : passes == 6 ? (side_b ? kPassPartsB6 : kPassPartsA6) : 0u;
  return (int)((table >> (4 * pass)) & 15u);
}

// Operands of products 1..7 of a formula from the four (permuted) quadrants
// in float, A side (kSide 0) or B side (kSide 1), before their final bf16
// rounding (pack8, or pack8_part for a multi-pass product).
// kBf16Compute: the reference's compute dtype is bf16 (bf16 inputs), so each
// jnp bf16 operation rounds: two-term sums round once (as they also do in
// float), and the powers formula's balanced four-term expressions round
// both halves and their sum. With FP32 inputs the compute dtype is float and
// only the finished operand is rounded, by the one-pass bf16 MXU product at
// DEFAULT precision (or split into bf16 parts by a multi-pass product). Raw
// quadrants (A0, B3, ...) are rounded the same way, which leaves bf16 inputs
// unchanged; scaling by 1/2 and 1/4 is exact.
template <int kSide, bool kBf16Compute>
__device__ __forceinline__ void formula_vals(int formula, const F8 (&x)[4], F8 (&ops)[7]) {
  const F8 &x0 = x[0], &x1 = x[1], &x2 = x[2], &x3 = x[3];
  auto rnd = [](float v) { return kBf16Compute ? round_bf16(v) : v; };
  if (formula == kFormulaClassical) {
    if constexpr (kSide == 0) {  // A0+A3, A2+A3, A0, A3, A0+A1, A2-A0, A1-A3 (:324-379)
      ops[0] = add8<false>(x0, x3);
      ops[1] = add8<false>(x2, x3);
      ops[2] = x0;
      ops[3] = x3;
      ops[4] = add8<false>(x0, x1);
      ops[5] = add8<true>(x2, x0);
      ops[6] = add8<true>(x1, x3);
    } else {  // B0+B3, B0, B1-B3, B2-B0, B3, B0+B1, B2+B3
      ops[0] = add8<false>(x0, x3);
      ops[1] = x0;
      ops[2] = add8<true>(x1, x3);
      ops[3] = add8<true>(x2, x0);
      ops[4] = x3;
      ops[5] = add8<false>(x0, x1);
      ops[6] = add8<false>(x2, x3);
    }
    return;
  }
  if (formula == kFormulaDual) {
    if constexpr (kSide == 0) {  // A0+A3, A0, A2-A3, A1-A0, A3, A0+A2, A1+A3 (:461-517)
      ops[0] = add8<false>(x0, x3);
      ops[1] = x0;
      ops[2] = add8<true>(x2, x3);
      ops[3] = add8<true>(x1, x0);
      ops[4] = x3;
      ops[5] = add8<false>(x0, x2);
      ops[6] = add8<false>(x1, x3);
    } else {  // B0+B3, B1+B3, B0, B3, B0+B2, B1-B0, B2-B3
      ops[0] = add8<false>(x0, x3);
      ops[1] = add8<false>(x1, x3);
      ops[2] = x0;
      ops[3] = x3;
      ops[4] = add8<false>(x0, x2);
      ops[5] = add8<true>(x1, x0);
      ops[6] = add8<true>(x2, x3);
    }
    return;
  }
  // Powers (Dumas--Pernet--Sedoglavic, :381-459).
  if constexpr (kSide == 0) {
    ops[0] = map8(x0, x1, x2, x3, [](float a0, float a1, float a2, float a3) { return a2 - a1; });
    ops[1] = map8(x0, x1, x2, x3, [&](float a0, float a1, float a2, float a3) {
      return rnd(a0 - a2 * 0.5f) + rnd(a1 * 0.5f - a3 * 0.25f);
    });
    ops[2] = map8(x0, x1, x2, x3, [](float a0, float a1, float a2, float a3) { return a2 - a3 * 0.5f; });
    ops[3] = map8(x0, x1, x2, x3, [](float a0, float a1, float a2, float a3) { return a1 - a3 * 0.5f; });
    ops[4] = map8(x0, x1, x2, x3, [](float a0, float a1, float a2, float a3) { return a2 + a3 * 0.5f; });
    ops[5] = map8(x0, x1, x2, x3, [&](float a0, float a1, float a2, float a3) {
      return rnd(a0 - a1 * 0.5f) + rnd(a2 * 0.5f - a3 * 0.25f);
    });
    ops[6] = map8(x0, x1, x2, x3, [](float a0, float a1, float a2, float a3) { return a1 + a3 * 0.5f; });
  } else {
    ops[0] = map8(x0, x1, x2, x3, [](float b0, float b1, float b2, float b3) { return b0 - b3; });
    ops[1] = map8(x0, x1, x2, x3, [](float b0, float b1, float b2, float b3) { return b0 + b1 * 0.5f; });
    ops[2] = map8(x0, x1, x2, x3, [](float b0, float b1, float b2, float b3) { return b1 * 0.5f - b3; });
    ops[3] = map8(x0, x1, x2, x3, [&](float b0, float b1, float b2, float b3) {
      return rnd(b0 * 0.5f - b2) + rnd(b1 * 0.25f - b3 * 0.5f);
    });
    ops[4] = map8(x0, x1, x2, x3, [](float b0, float b1, float b2, float b3) { return b1 * 0.5f + b3; });
    ops[5] = map8(x0, x1, x2, x3, [](float b0, float b1, float b2, float b3) { return b0 - b1 * 0.5f; });
    ops[6] = map8(x0, x1, x2, x3, [&](float b0, float b1, float b2, float b3) {
      return rnd(b0 * 0.5f + b2) - rnd(b1 * 0.25f + b3 * 0.5f);
    });
  }
}

// Block permutation (strassen_pallas.py:205-226): quadrant (row, col) takes
// the original quadrant (row ^ swap_rows, col ^ swap_cols).
template <class T>
__device__ __forceinline__ void permute_quadrants(T (&q)[4], int swap_rows, int swap_cols) {
  if (swap_rows) {
    const T t0 = q[0], t1 = q[1];
    q[0] = q[2];
    q[1] = q[3];
    q[2] = t0;
    q[3] = t1;
  }
  if (swap_cols) {
    const T t0 = q[0], t2 = q[2];
    q[0] = q[1];
    q[2] = q[3];
    q[1] = t0;
    q[3] = t2;
  }
}

// ---------------------------------------------------------------------------
// Parameters and tile mapping
// ---------------------------------------------------------------------------

struct Params {
  const uint16_t* a;
  const uint16_t* b;  // B^T [N, K] (plain) or the pre-summed operands [N/2*7, K/2]
  void* c;           // bf16, or float32 when out_f32
  const void* residual;      // bf16, or float32 when residual_f32
  const void* bias;
  const uint16_t* rope_cos;  // bf16 [M, bn/2]
  const uint16_t* rope_sin;
  const void* rope_scale;
  int64_t m, n, k;
  int64_t lda, ldb, ldc, ldr;
  int32_t bm, bn, bk;
  int32_t bias_f32, scale_f32, residual_f32;
  int32_t head_dim;
  float eps;
  int32_t tiles_m, tiles_n;  // product-space workgroup grid
  int32_t group_m;           // tile rows per rasterization group
  int32_t raster;            // tile order (kRaster*, tile_of)
  int32_t out_f32;           // store float32 instead of bf16
  int32_t formula;           // kFormula* (Strassen family)
  int32_t perm;              // block permutation bits: 1 rows, 2 K, 4 columns
  const float* partial;      // cubic: FP32 [M, N] added before the epilogue, or null
  int64_t ldp;
  // Launch shape (packed kernels): grid workgroups (0: tiles_m * tiles_n).
  // A K-split launch (ksplit s > 1, grid s u) gives workgroup h u + w the
  // tile tile_base + w and share h of its S K stages, stages
  // floor(h S / s) .. floor((h + 1) S / s) - 1 (S >= s), and stores that
  // share as a dense FP32 block (dense_share_output): share h of split tile
  // w at h * split_stride + w * kSplitTileFloats floats, split_stride =
  // u * kSplitTileFloats.
  int32_t grid;
  int32_t ksplit;
  int32_t tile_base;
  int64_t split_stride;
  // Product-major Strassen kernel (kernel_pm.hpp): FP32 space for one parked
  // quadrant set per workgroup (pm::kParkBytes each).
  void* park;
};

// A workgroup's logical tile and its share of the K stages (see Params).
struct WorkShare {
  int tile;     // logical tile index, for tile_of
  int stage0;   // first K stage
  int nstages;  // K stages of this share
  int share;    // 0 .. ksplit-1
};

__device__ __forceinline__ WorkShare work_share(const Params& p, int nstages_all) {
  WorkShare w;
  if (p.ksplit > 1) {
    // Share h runs on workgroups h u .. h u + u - 1: with tile_base and u
    // multiples of 8, workgroup h u + w lands on the XCD that tile_of
    // gathers tile tile_base + w on.
    const uint32_t tiles = gridDim.x / (uint32_t)p.ksplit;
    const uint32_t share = blockIdx.x / tiles;
    w.share = (int)share;
    w.tile = p.tile_base + (int)(blockIdx.x - share * tiles);
    w.stage0 = (int)(share * (uint32_t)nstages_all / (uint32_t)p.ksplit);
    w.nstages = (int)((share + 1) * (uint32_t)nstages_all / (uint32_t)p.ksplit) - w.stage0;
    // The divisions run on VALU; the results are uniform, and in SGPRs they
    // leave the VGPRs to the accumulators.
    w.share = __builtin_amdgcn_readfirstlane(w.share);
    w.tile = __builtin_amdgcn_readfirstlane(w.tile);
    w.stage0 = __builtin_amdgcn_readfirstlane(w.stage0);
    w.nstages = __builtin_amdgcn_readfirstlane(w.nstages);
  } else {
    w.share = 0;
    w.tile = (int)blockIdx.x;
    w.nstages = nstages_all;
    w.stage0 = 0;
  }
  return w;
}

// Workgroup id -> product-space tile. Workgroups are dispatched round-robin
// over the 8 XCDs (bid % 8), and an XCD's 32 CUs run its workgroups in the
// order bid / 8, 32 at a time. Tiles walk column groups of group_m rows, so
// that 32 concurrent tiles on an XCD are group_m rows x 32 / group_m
// columns (8 A and 4 B panels for group_m = 8: the fewest for 32 tiles)
// and share them in its L2. Where the 8 XCDs' concurrent tiles sit decides
// how often an L2 miss is served by the MALL (memory-side cache, 256 MB)
// rather than HBM, which the Strassen kernel's operand stream feels:
//   kRasterSpread: XCD x takes the x-th eighth of the order. All tile rows
//     run at once and each B panel is shared by several XCDs: the order for
//     a packed A that stays in the MALL;
//   kRasterChunks: XCD x takes chunks x, x + 8, ... of 32 tiles of the
//     order, so a round is 8 consecutive chunks: few tile rows, each shared
//     by several XCDs, and all B columns of a narrow launch, which then stay
//     in the MALL;
//   kRasterBlocks: chunks as above over super-blocks of 2 group_m rows x
//     4 chunk widths, so a round is a 2 x 4 grid of XCD blocks that shares
//     each A panel 4 ways and each B panel 2 ways, for launches where
//     neither operand stays in the MALL.
constexpr int kRasterSpread = 0, kRasterChunks = 1, kRasterBlocks = 2;
constexpr int kXcds = 8, kXcdTiles = 32;

__host__ __device__ inline int xcd_order(int bid, int total, int raster) {
  if (total % kXcds) return bid;
  const int per_xcd = total / kXcds, x = bid % kXcds, slot = bid / kXcds;
  if (raster == kRasterSpread) return x * per_xcd + slot;
  const int full = per_xcd / kXcdTiles * kXcdTiles;
  return slot < full ? ((slot / kXcdTiles) * kXcds + x) * kXcdTiles + slot % kXcdTiles
                     : full * kXcds + x * (per_xcd - full) + (slot - full);
}

__host__ __device__ inline void tile_of(int bid, int tiles_m, int tiles_n, int group_m, int raster, int& tm,
                                        int& tn) {
  const int logical = xcd_order(bid, tiles_m * tiles_n, raster);
  if (raster == kRasterBlocks) {
    const int chunk_cols = kXcdTiles / group_m > 0 ? kXcdTiles / group_m : 1;
    const int sg_rows = 2 * group_m, strip = 4 * chunk_cols;
    const int sg = logical / (sg_rows * tiles_n);
    const int h = min(sg_rows, tiles_m - sg * sg_rows);
    const int in_sg = logical - sg * sg_rows * tiles_n;
    const int t = in_sg / (h * strip);
    const int w = min(strip, tiles_n - t * strip);
    const int in_strip = in_sg - t * h * strip;
    const int h1 = min(group_m, h);
    const bool second = in_strip >= h1 * w;
    const int k = second ? in_strip - h1 * w : in_strip, rows = second ? h - h1 : h1;
    tm = sg * sg_rows + (second ? h1 : 0) + k % rows;
    tn = t * strip + k / rows;
    return;
  }
  const int group_size = group_m * tiles_n;
  const int group = logical / group_size;
  const int first_m = group * group_m;
  const int rows_in_group = min(tiles_m - first_m, group_m);
  const int in_group = logical - group * group_size;
  tm = first_m + in_group % rows_in_group;
  tn = in_group / rows_in_group;
}

// Physical origin of a product-space workgroup tile (prow0, pcol0).
struct TileOrigin {
  int64_t ti, tr;  // row tile index and row inside the half (thin tilings: 0 and the product row)
  int64_t tj, tc;  // column tile index and column inside the half
};

// The origin is uniform over the workgroup. Product-space coordinates fit in
// 32 bits (the host refuses M/2 or N/2 >= 2^31), so the divisions run on
// 32-bit values, and readfirstlane moves the results to SGPRs: VGPR copies
// would stay live across the main loop next to the accumulators and spill.
// kThin: bm/2 is not a multiple of the product tile's rows, so the tile's
// rows belong to several row tiles; the origin keeps the product row and the
// epilogue maps every row on its own (ThinRows).
template <bool kThin = false>
__device__ __forceinline__ TileOrigin tile_origin(const Params& p, int64_t prow0, int64_t pcol0) {
  const uint32_t hm = (uint32_t)(p.bm / 2), hn = (uint32_t)(p.bn / 2);
  const uint32_t r = (uint32_t)prow0, c = (uint32_t)pcol0;
  auto uniform = [](uint32_t v) { return (int64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)v); };
  TileOrigin o;
  if constexpr (kThin) {
    o.ti = 0;
    o.tr = uniform(r);
  } else {
    o.ti = uniform(r / hm);
    o.tr = uniform(r % hm);
  }
  o.tj = uniform(c / hn);
  o.tc = uniform(c % hn);
  return o;
}

// FP32 elements of one K share of one split tile: its 256 x 256 outputs.
constexpr int64_t kSplitTileFloats = 256 * 256;

// A K share's output (the no-epilogue FP32 store of a K-split launch) goes to
// the workspace as a dense 256 x 256 block per split tile: the tile's four
// 128 x 128 quadrant blocks at row and column offsets 0 and 128, row stride
// 256, in the order the block permutation stores them. The store code is the
// ordinary epilogue's, on the geometry of a 256 x 256 tiling whose only tile
// sits at the origin (a thin tiling then maps every product row straight to
// a row of its half). Its M keeps the tile's real product rows (prow0 is
// the tile's first): a thin tiling's padding rows, past M/2, are not stored.
// split_fixup reads the blocks back.
__device__ __forceinline__ void dense_share_output(Params& p, TileOrigin& o, const WorkShare& ws, int64_t prow0) {
  const int64_t rows = p.m / 2 - prow0;
  p.c = reinterpret_cast<float*>(p.c) + ws.share * p.split_stride + (int64_t)(ws.tile - p.tile_base) * kSplitTileFloats;
  p.bm = p.bn = 256;
  p.m = 2 * (rows < 128 ? rows : 128);
  p.n = 256;
  p.ldc = 256;
  o = TileOrigin{0, 0, 0, 0};
}

// Output rows of a thin tiling. Product row P (of M/2) is row P % hm of row
// tile P / hm, whose two row halves are output rows (P / hm) * bm + P % hm
// and that plus hm (strassen_pallas.py:188-204 splits every bm-row tile into
// those halves). The packed A holds its rows in product order, zero-padded
// to whole 128-row product tiles, so the main loop is that of any tiling;
// only the epilogue's row addresses change, and padding rows (P >= M/2) are
// neither read nor written.
struct ThinRows {
  uint32_t hm, bm, prows;
  __device__ __forceinline__ int64_t row(uint32_t prow, int half) const {
    const uint32_t t = prow / hm;
    return (int64_t)t * bm + (int64_t)half * hm + (prow - t * hm);
  }
  __device__ __forceinline__ bool valid(uint32_t prow) const { return prow < prows; }
};

// ---------------------------------------------------------------------------
// Epilogue
// ---------------------------------------------------------------------------

// Lane index within the wave (v_mbcnt over a full mask), as a volatile asm
// that the compiler can neither hoist nor merge with an earlier lane index.
__device__ __forceinline__ int opaque_lane_id() {
  int lane;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane));
  return lane;
}

// SiLU as jax.nn.silu computes it, x * sigmoid(x), with sigmoid(x) =
// 1 / (1 + 2^(-x log2 e)) on the hardware exp2 and reciprocal (each within
// about one float ulp, far below the result's bf16 rounding).
__device__ __forceinline__ float silu_f32(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}

// GELU, tanh approximation (jax.nn.gelu(approximate=True), the GeGLU gate of
// strassen_pallas.py:143-153): 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))).
__device__ __forceinline__ float gelu_tanh_f32(float x) {
  const float k = 0.7978845608028654f;  // sqrt(2/pi)
  return 0.5f * x * (1.0f + tanhf(k * (x + 0.044715f * x * x * x)));
}

template <int kEpi>
__device__ __forceinline__ float gate_f32(float x) {
  if constexpr (kEpi == SMX_EPI_GEGLU)
    return gelu_tanh_f32(x);
  else
    return silu_f32(x);
}

__device__ __forceinline__ float load_vec(const void* v, int is_f32, int64_t i) {
  return is_f32 ? reinterpret_cast<const float*>(v)[i] : bf16_to_f32(reinterpret_cast<const uint16_t*>(v)[i]);
}

// Eight values of an [.., ld] array at element i (i % 8 == 0 for bf16,
// i % 4 == 0 for float32 rows: 16-byte loads).
__device__ __forceinline__ F8 load8(const void* base, int is_f32, int64_t i) {
  if (is_f32) {
    const f32x4 lo = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(base) + i);
    const f32x4 hi = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(base) + i + 4);
    return F8{{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]}};
  }
  return unpack8(*reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(base) + i));
}

__device__ __forceinline__ void store8(void* base, int out_f32, int64_t i, const F8& x) {
  if (out_f32) {
    float* const o = reinterpret_cast<float*>(base) + i;
    *reinterpret_cast<f32x4*>(o) = f32x4{x.v[0], x.v[1], x.v[2], x.v[3]};
    *reinterpret_cast<f32x4*>(o + 4) = f32x4{x.v[4], x.v[5], x.v[6], x.v[7]};
  } else {
    *reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(base) + i) = pack8(x);
  }
}

// Sum over the 32 lanes of a half-wave (lanes sharing lane>>5), the same
// total in every lane. DPP adds within rows of 16 lanes (quad_perm
// [1,0,3,2] and [2,3,0,1]: pairs and quads; row_half_mirror: lane i with
// 7-i, halves of 8; row_mirror: lane i with 15-i, rows of 16), after which
// each row's lanes hold their row's total; then v_permlane16_swap (gfx950)
// on two copies of the value swaps the odd rows of the first with the even
// rows of the second, so that in both lanes i and i ^ 16 the first result
// holds the lower row's total and the second the upper row's. Each DPP step
// adds two partial sums that its partner lane adds in the other order (float
// addition is commutative) and the last adds lower + upper in every lane, so
// all 32 lanes end with bit-identical totals. Every step is a plain VALU op:
// nothing waits on the LDS, and the sums of independent rows interleave.
__device__ __forceinline__ float half_wave_sum(float x) {
  auto as_int = [](float v) __attribute__((always_inline)) { return __builtin_bit_cast(int, v); };
  auto as_float = [](int v) __attribute__((always_inline)) { return __builtin_bit_cast(float, v); };
  x += as_float(__builtin_amdgcn_update_dpp(0, as_int(x), 0xB1, 0xF, 0xF, false));   // quad_perm [1,0,3,2]
  x += as_float(__builtin_amdgcn_update_dpp(0, as_int(x), 0x4E, 0xF, 0xF, false));   // quad_perm [2,3,0,1]
  x += as_float(__builtin_amdgcn_update_dpp(0, as_int(x), 0x141, 0xF, 0xF, false));  // row_half_mirror
  x += as_float(__builtin_amdgcn_update_dpp(0, as_int(x), 0x140, 0xF, 0xF, false));  // row_mirror
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto rows = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __builtin_bit_cast(float, (unsigned)rows[0]) + __builtin_bit_cast(float, (unsigned)rows[1]);
}

// One wave's epilogue staging tile in LDS: kRows x kCols floats, row stride
// kStride bytes. An accumulator register holds rows r (lanes 0-31) and r+4
// (lanes 32-63) of 32 consecutive columns; the 32-byte row pad puts the two
// half-waves of a store 32 banks apart. Elements are addressed as a per-lane
// base plus a compile-time offset, and global memory is read and written in
// coalesced 16-byte chunks by whole rows.
template <int kRows_, int kCols_>
struct StageTile {
  static constexpr int kRows = kRows_, kCols = kCols_;
  static constexpr int kStride = kCols * 4 + 32;
  static constexpr int kBytes = kRows * kStride;
  // Register r of 32x32 block (i, j), lane part excluded.
  static constexpr int at(int i, int j, int r) { return (i * 32 + 8 * (r >> 2) + (r & 3)) * kStride + j * 128; }
  static __device__ __forceinline__ int lane_part(int lane) { return (lane >> 5) * 4 * kStride + (lane & 31) * 4; }
  static_assert(kRows * kCols % 512 == 0, "whole 16-byte chunks per lane");
};

// Staging tiles per wave of an epilogue (q/k writes its a and b blocks at
// once), and the LDS bytes four waves of kRows x kCols tiles need.
template <int kEpi>
constexpr int kEpiTiles = kEpi == SMX_EPI_QK_NORM_ROPE ? 2 : 1;
template <int kEpi, int kRows, int kCols>
constexpr int kEpiLds = 4 * kEpiTiles<kEpi> * StageTile<kRows, kCols>::kBytes;

// Rows of a global [*, ld] matrix (bf16, or float when f32; 16-byte aligned
// rows) -> the staging tile as float.
template <class T>
__device__ __forceinline__ void tile_load(uint8_t* tile, const char* src, int64_t ld, int f32, int lane) {
  if (f32) {
    constexpr int kChunks = T::kCols / 4;
#pragma unroll
    for (int t = 0; t < T::kRows * kChunks / 64; ++t) {
      const int idx = lane + 64 * t, row = idx / kChunks, ch = idx % kChunks;
      const f32x4 v = *reinterpret_cast<const f32x4*>(src + (row * ld + ch * 4) * 4);
      *reinterpret_cast<f32x4*>(tile + row * T::kStride + ch * 16) = v;
    }
  } else {
    constexpr int kChunks = T::kCols / 8;
#pragma unroll
    for (int t = 0; t < T::kRows * kChunks / 64; ++t) {
      const int idx = lane + 64 * t, row = idx / kChunks, ch = idx % kChunks;
      const F8 f = unpack8(*reinterpret_cast<const u32x4*>(src + (row * ld + ch * 8) * 2));
      const f32x4 v0 = {f.v[0], f.v[1], f.v[2], f.v[3]}, v1 = {f.v[4], f.v[5], f.v[6], f.v[7]};
      *reinterpret_cast<f32x4*>(tile + row * T::kStride + ch * 32) = v0;
      *reinterpret_cast<f32x4*>(tile + row * T::kStride + ch * 32 + 16) = v1;
    }
  }
}

// The staging tile -> rows of a global [*, ld] matrix, rounded once to bf16
// (or stored as float when f32).
template <class T>
__device__ __forceinline__ void tile_store(const uint8_t* tile, char* dst, int64_t ld, int f32, int lane) {
  constexpr int kChunks = T::kCols / 8;  // 8 elements per lane and step
#pragma unroll
  for (int t = 0; t < T::kRows * kChunks / 64; ++t) {
    const int idx = lane + 64 * t, row = idx / kChunks, ch = idx % kChunks;
    const f32x4 v0 = *reinterpret_cast<const f32x4*>(tile + row * T::kStride + ch * 32);
    const f32x4 v1 = *reinterpret_cast<const f32x4*>(tile + row * T::kStride + ch * 32 + 16);
    if (f32) {
      char* const out = dst + (row * ld + ch * 8) * 4;
      *reinterpret_cast<f32x4*>(out) = v0;
      *reinterpret_cast<f32x4*>(out + 16) = v1;
    } else {
      F8 f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f.v[e] = v0[e];
        f.v[4 + e] = v1[e];
      }
      *reinterpret_cast<u32x4*>(dst + (row * ld + ch * 8) * 2) = pack8(f);
    }
  }
}

// tile_load / tile_store over rows at arbitrary addresses: row_at(row) gives
// the row's first element (already offset to the tile's first column), or
// null for a row that is skipped (its staging row is left as it is).
template <class T, class RowAt>
__device__ __forceinline__ void tile_load_rows(uint8_t* tile, RowAt row_at, int f32, int lane) {
  if (f32) {
    constexpr int kChunks = T::kCols / 4;
#pragma unroll
    for (int t = 0; t < T::kRows * kChunks / 64; ++t) {
      const int idx = lane + 64 * t, row = idx / kChunks, ch = idx % kChunks;
      const char* const src = row_at(row);
      if (src) *reinterpret_cast<f32x4*>(tile + row * T::kStride + ch * 16) =
          *reinterpret_cast<const f32x4*>(src + ch * 16);
    }
  } else {
    constexpr int kChunks = T::kCols / 8;
#pragma unroll
    for (int t = 0; t < T::kRows * kChunks / 64; ++t) {
      const int idx = lane + 64 * t, row = idx / kChunks, ch = idx % kChunks;
      const char* const src = row_at(row);
      if (!src) continue;
      const F8 f = unpack8(*reinterpret_cast<const u32x4*>(src + ch * 16));
      const f32x4 v0 = {f.v[0], f.v[1], f.v[2], f.v[3]}, v1 = {f.v[4], f.v[5], f.v[6], f.v[7]};
      *reinterpret_cast<f32x4*>(tile + row * T::kStride + ch * 32) = v0;
      *reinterpret_cast<f32x4*>(tile + row * T::kStride + ch * 32 + 16) = v1;
    }
  }
}

template <class T, class RowAt>
__device__ __forceinline__ void tile_store_rows(const uint8_t* tile, RowAt row_at, int f32, int lane) {
  constexpr int kChunks = T::kCols / 8;
#pragma unroll
  for (int t = 0; t < T::kRows * kChunks / 64; ++t) {
    const int idx = lane + 64 * t, row = idx / kChunks, ch = idx % kChunks;
    char* const dst = row_at(row);
    if (!dst) continue;
    const f32x4 v0 = *reinterpret_cast<const f32x4*>(tile + row * T::kStride + ch * 32);
    const f32x4 v1 = *reinterpret_cast<const f32x4*>(tile + row * T::kStride + ch * 32 + 16);
    if (f32) {
      *reinterpret_cast<f32x4*>(dst + ch * 32) = v0;
      *reinterpret_cast<f32x4*>(dst + ch * 32 + 16) = v1;
    } else {
      F8 f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f.v[e] = v0[e];
        f.v[4 + e] = v1[e];
      }
      *reinterpret_cast<u32x4*>(dst + ch * 16) = pack8(f);
    }
  }
}

// Quadrant sources of the epilogue: the cubic's quadrants (plus an FP32
// partial product), or Strassen's seven product sets under the classical,
// dual or powers formula. The block permutation is applied by addressing:
// it only moves where a quadrant is stored (and which quadrant gates, for
// SwiGLU / GeGLU, or is the a half, for q/k).
constexpr int kQuadCubic = 0, kQuadCubicPartial = 1, kQuadClassical = 2, kQuadDual = 3, kQuadPowers = 4;

template <int kQ>
using QuadC = std::integral_constant<int, kQ>;

// Logical output quadrant kQ of accumulator element (i, j, r). The
// accumulators are only read, so no quadrant set is materialised next to
// the 448 product registers.
template <int kQuad, int kQ, int kMB, int kNB, int kNacc>
__device__ __forceinline__ float quadrant_value(const f32x16 (&acc)[kNacc][kMB][kNB], int i, int j, int r) {
  if constexpr (kQuad == kQuadCubic || kQuad == kQuadCubicPartial) {
    return acc[kQ][i][j][r];
  } else {
    const float p1 = acc[0][i][j][r], p2 = acc[1][i][j][r], p3 = acc[2][i][j][r], p4 = acc[3][i][j][r];
    const float p5 = acc[4][i][j][r], p6 = acc[5][i][j][r], p7 = acc[6][i][j][r];
    if constexpr (kQuad == kQuadClassical) {
      // C0 = P1+P4-P5+P7, C1 = P3+P5, C2 = P2+P4, C3 = P1-P2+P3+P6
      if constexpr (kQ == 0) return ((p4 - p5) + p7) + p1;
      if constexpr (kQ == 1) return p5 + p3;
      if constexpr (kQ == 2) return p4 + p2;
      if constexpr (kQ == 3) return ((p6 - p2) + p3) + p1;
    } else if constexpr (kQuad == kQuadDual) {
      // C0 = Q1+Q4-Q5+Q7, C1 = Q2+Q4, C2 = Q3+Q5, C3 = Q1-Q2+Q3+Q6
      if constexpr (kQ == 0) return ((p4 - p5) + p7) + p1;
      if constexpr (kQ == 1) return p4 + p2;
      if constexpr (kQ == 2) return p5 + p3;
      if constexpr (kQ == 3) return ((p6 + p3) - p2) + p1;
    } else {
      // powers: basis z0 = R3+R5, z1 = R6+R7, z2 = R2-R4, z3 = R1-R3+R4+R7,
      // decoded as in strassen_pallas.py:744-760
      const float z0 = p3 + p5;
      if constexpr (kQ == 3) return z0;
      const float z1 = p6 + p7, z2 = p2 - p4, z3 = ((p4 - p3) + p7) + p1;
      if constexpr (kQ == 0) return (z1 + z2) * 0.5f + z0 * 0.25f;
      if constexpr (kQ == 1) return ((z2 - z1) + z3) + z0 * 0.5f;
      if constexpr (kQ == 2) return z3 + z0 * 0.5f;
    }
  }
}

// Combines the accumulator sets into the four quadrants, applies the
// epilogue and stores bf16 (or float32). acc has kNacc sets (7 Strassen
// products P1..P7, or the 4 quadrants for the cubic) of kMB x kNB 32x32
// blocks; the wave's block (i, j) sits at product-space rows row0 + 32 i and
// columns col0 + 32 j, relative to the tile origin o. Accumulator lane
// layout (v_mfma_f32_32x32x16_bf16): column lane%32, row
// 8*(r/4) + 4*(lane/32) + r%4 for register r.
//
// Logical quadrant (row, col) is stored at physical (row ^ swap_m, col ^
// swap_n) for the block permutation (strassen_pallas.py:205-226), so the
// permutation changes addresses only; SwiGLU / GeGLU and q/k, whose roles
// follow physical columns, swap their two operands with one select.
//
// One output block at a time passes through the wave's staging tile `tile`
// (StageTile<32 kMB, 32 kNB>::kBytes of LDS, private to the wave): a
// residual block is loaded into it, each element's result replaces the
// element in place, and the block is stored. Registers meet LDS at
// compile-time offsets; global memory sees whole 16-byte row chunks.
//
// kThin: the rows of a thin tiling go through ThinRows one by one (o.tr is
// then the tile's first product row).
template <int kMB, int kNB, int kEpi, int kNacc, int kQuad, bool kThin = false>
__device__ __forceinline__ void epilogue_body(const Params& p, const TileOrigin& o, int row0, int col0,
                                              f32x16 (&acc)[kNacc][kMB][kNB], uint8_t* tile) {
  using T = StageTile<32 * kMB, 32 * kNB>;
  // The lane index is produced here by its own volatile asm, after the main
  // loop's drain: every per-lane epilogue address depends on it, so none can
  // be computed ahead of the loop and held (or spilled) across it, and the
  // compiler cannot reuse a lane index it computed before the loop.
  const int lane = opaque_lane_id();
  const int hm = p.bm / 2, hn = p.bn / 2;
  const int lcol = lane & 31;
  const int swap_m = p.perm & 1, swap_n = (p.perm >> 2) & 1;
  // Top-left output element of this wave (quadrant 0) and its column inside
  // the tile half.
  const int64_t row_base = o.ti * p.bm + o.tr + row0;
  const int64_t cc_base = o.tc + col0;
  const int64_t col_base = o.tj * p.bn + cc_base;
  // thin tilings: row_base is the wave's first product row
  const ThinRows thin{(uint32_t)hm, (uint32_t)p.bm, (uint32_t)(p.m / 2)};
  uint8_t* const te = tile + T::lane_part(lane);
  // LDS operations of one wave complete in order; this keeps the compiler
  // from moving one lane's tile access across another lane's.
  auto fence = []() __attribute__((always_inline)) { asm volatile("" ::: "memory"); };
  auto put = [&](int i, int j, int r, float v) __attribute__((always_inline)) {
    *reinterpret_cast<float*>(te + T::at(i, j, r)) = v;
  };
  auto get = [&](int i, int j, int r) __attribute__((always_inline)) {
    return *reinterpret_cast<const float*>(te + T::at(i, j, r));
  };
  auto value = [&](auto q, int i, int j, int r) __attribute__((always_inline)) {
    return quadrant_value<kQuad, decltype(q)::value>(acc, i, j, r);
  };
  // Physical quadrant (row half pr, column half pc) of an [M, N] operand
  // (row stride ld, element size es, float when f32) -> the staging tile.
  auto load_quadrant = [&](const void* base, int64_t ld, int es, int f32, int pr, int pc)
                           __attribute__((always_inline)) {
    const char* const cols = reinterpret_cast<const char*>(base) + (col_base + pc * hn) * es;
    if constexpr (kThin) {
      tile_load_rows<T>(tile, [&](int row) __attribute__((always_inline)) -> const char* {
        const uint32_t prow = (uint32_t)(row_base + row);
        return thin.valid(prow) ? cols + thin.row(prow, pr) * ld * es : nullptr;
      }, f32, lane);
    } else {
      tile_load<T>(tile, cols + (row_base + pr * hm) * ld * es, ld, f32, lane);
    }
  };
  // The staging tile `t` -> the output block in row half `half` at column col.
  auto emit_from = [&](uint8_t* t, int half, int64_t col) __attribute__((always_inline)) {
    fence();
    const int es = p.out_f32 ? 4 : 2;
    if constexpr (kThin) {
      char* const cols = reinterpret_cast<char*>(p.c) + col * es;
      tile_store_rows<T>(t, [&](int row) __attribute__((always_inline)) -> char* {
        const uint32_t prow = (uint32_t)(row_base + row);
        return thin.valid(prow) ? cols + thin.row(prow, half) * p.ldc * es : nullptr;
      }, p.out_f32, lane);
    } else {
      tile_store<T>(t, reinterpret_cast<char*>(p.c) + ((row_base + half * hm) * p.ldc + col) * es, p.ldc,
                    p.out_f32, lane);
    }
    fence();
  };

  // Cubic only: an FP32 partial product of the same output (the Strassen
  // panels of an exact-panel schedule) joins the quadrants first.
  if constexpr (kQuad == kQuadCubicPartial) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      load_quadrant(p.partial, p.ldp, 4, 1, q >> 1, q & 1);
      fence();
#pragma unroll
      for (int i = 0; i < kMB; ++i)
#pragma unroll
        for (int j = 0; j < kNB; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[q][i][j][r] += get(i, j, r);
      fence();
    }
  }

  if constexpr (kEpi == SMX_EPI_SWIGLU || kEpi == SMX_EPI_GEGLU) {
    // Physical quadrants 0/2 are gate, 1/3 up; output [M, N/2]. Logical row
    // half lr lands on physical row half lr ^ swap_m; its gate is logical
    // column swap_n.
    const int64_t ocol = o.tj * hn + cc_base;
    auto gated = [&](auto q_left, auto q_right, int lr) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < kMB; ++i)
#pragma unroll
        for (int j = 0; j < kNB; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float left = value(q_left, i, j, r), right = value(q_right, i, j, r);
            const float gate = swap_n ? right : left, up = swap_n ? left : right;
            put(i, j, r, gate_f32<kEpi>(gate) * up);
          }
      emit_from(tile, lr ^ swap_m, ocol);
    };
    gated(QuadC<0>{}, QuadC<1>{}, 0);
    gated(QuadC<2>{}, QuadC<3>{}, 1);
  } else if constexpr (kEpi == SMX_EPI_QK_NORM_ROPE) {
    // Per-head RMSNorm then RoPE (strassen_pallas.py:793-835). A head owns
    // head_dim/2 = 64 consecutive columns of a tile half: the wave's column
    // blocks j = 2h, 2h+1 (the caller guarantees kNB % 2 == 0 and 64-aligned
    // wave columns). Physical quadrants 0/2 hold the a half, 1/3 the b half.
    static_assert(kNB % 2 == 0, "qk epilogue needs 64-column waves");
    // The norm spans both quadrants of a tile half and both halves are
    // needed to the end: the logical quadrants are formed once, in place in
    // sets 0-3 (straight-line code), which frees the other three sets.
    if constexpr (kNacc == 7) {
#pragma unroll
      for (int i = 0; i < kMB; ++i)
#pragma unroll
        for (int j = 0; j < kNB; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float q0 = value(QuadC<0>{}, i, j, r), q1 = value(QuadC<1>{}, i, j, r);
            const float q2 = value(QuadC<2>{}, i, j, r), q3 = value(QuadC<3>{}, i, j, r);
            acc[0][i][j][r] = q0;
            acc[1][i][j][r] = q1;
            acc[2][i][j][r] = q2;
            acc[3][i][j][r] = q3;
          }
    }
    const float inv_width = 1.0f / (float)p.head_dim;
    // Two staging tiles per wave: the a and b halves of each row, first as
    // a * recip and b * recip (FP32, exact), then rotated and stored by the
    // pass below.
    uint8_t* const tile_b = tile + T::kBytes;
    uint8_t* const te_b = tile_b + T::lane_part(lane);
    // Rotation and store by 16-byte row chunks (the staging tile's store
    // pattern). A lane always takes the same chunk column, eight columns c0..
    // of the tile half: it reads their scale (gamma) once per row half, and
    // the scale and the RoPE tables ([M, hn] bf16, by output row and column
    // inside the half) eight values per 16-byte-aligned load. out_a = a' cos - b' sin and out_b =
    // b' cos + a' sin with a' = (a * recip) * gamma_a, b' = (b * recip) *
    // gamma_b, as the reference orders them (strassen_pallas.py:821-827).
    constexpr int kChunks = T::kCols / 8;
    static_assert(64 % kChunks == 0, "a lane keeps one chunk column");
    const int ch = lane % kChunks;
    const int64_t c0 = cc_base + ch * 8;
    auto rotate_store = [&](int half) __attribute__((always_inline)) {
      fence();
      const F8 ga = load8(p.rope_scale, p.scale_f32, c0), gb = load8(p.rope_scale, p.scale_f32, hn + c0);
      const int es = p.out_f32 ? 4 : 2;
      char* const out_cols = reinterpret_cast<char*>(p.c) + (col_base + ch * 8) * es;
#pragma unroll
      for (int t = 0; t < T::kRows * kChunks / 64; ++t) {
        const int row = (lane + 64 * t) / kChunks;
        int64_t orow;
        bool store = true;
        if constexpr (kThin) {
          const uint32_t prow = (uint32_t)(row_base + row);
          store = thin.valid(prow);
          orow = thin.row(store ? prow : thin.prows - 1, half);  // padding rows read a real table row
        } else {
          orow = row_base + half * hm + row;
        }
        const F8 cs = unpack8(*reinterpret_cast<const u32x4*>(p.rope_cos + orow * hn + c0));
        const F8 sn = unpack8(*reinterpret_cast<const u32x4*>(p.rope_sin + orow * hn + c0));
        const uint8_t* const sa = tile + row * T::kStride + ch * 32;
        const uint8_t* const sb = tile_b + row * T::kStride + ch * 32;
        const f32x4 a_lo = *reinterpret_cast<const f32x4*>(sa), a_hi = *reinterpret_cast<const f32x4*>(sa + 16);
        const f32x4 b_lo = *reinterpret_cast<const f32x4*>(sb), b_hi = *reinterpret_cast<const f32x4*>(sb + 16);
        F8 oa, ob;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float na = (e < 4 ? a_lo[e & 3] : a_hi[e & 3]) * ga.v[e];
          const float nb = (e < 4 ? b_lo[e & 3] : b_hi[e & 3]) * gb.v[e];
          oa.v[e] = na * cs.v[e] - nb * sn.v[e];
          ob.v[e] = nb * cs.v[e] + na * sn.v[e];
        }
        if (!store) continue;
        char* const out_a = out_cols + orow * p.ldc * es;
        char* const out_b = out_a + (int64_t)hn * es;
        if (p.out_f32) {
          *reinterpret_cast<f32x4*>(out_a) = f32x4{oa.v[0], oa.v[1], oa.v[2], oa.v[3]};
          *reinterpret_cast<f32x4*>(out_a + 16) = f32x4{oa.v[4], oa.v[5], oa.v[6], oa.v[7]};
          *reinterpret_cast<f32x4*>(out_b) = f32x4{ob.v[0], ob.v[1], ob.v[2], ob.v[3]};
          *reinterpret_cast<f32x4*>(out_b + 16) = f32x4{ob.v[4], ob.v[5], ob.v[6], ob.v[7]};
        } else {
          *reinterpret_cast<u32x4*>(out_a) = pack8(oa);
          *reinterpret_cast<u32x4*>(out_b) = pack8(ob);
        }
      }
      fence();
    };
    // Logical row half lr (sets 2 lr, 2 lr + 1) lands on physical row half
    // lr ^ swap_m; its a half is logical column swap_n.
    auto rows = [&](auto q_left, auto q_right, int lr) __attribute__((always_inline)) {
      constexpr int kL = decltype(q_left)::value, kR = decltype(q_right)::value;
      const int half = lr ^ swap_m;
      auto qa = [&](int i, int j, int r) __attribute__((always_inline)) {
        return swap_n ? acc[kR][i][j][r] : acc[kL][i][j][r];
      };
      auto qb = [&](int i, int j, int r) __attribute__((always_inline)) {
        return swap_n ? acc[kL][i][j][r] : acc[kR][i][j][r];
      };
#pragma unroll
      for (int i = 0; i < kMB; ++i) {
#pragma unroll
        for (int h = 0; h < kNB / 2; ++h) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float a0 = qa(i, 2 * h, r), a1 = qa(i, 2 * h + 1, r);
            const float b0 = qb(i, 2 * h, r), b1 = qb(i, 2 * h + 1, r);
            const float ssa = half_wave_sum(a0 * a0 + a1 * a1);
            const float ssb = half_wave_sum(b0 * b0 + b1 * b1);
            // the reference's jax.lax.rsqrt (strassen_pallas.py:818) as the
            // hardware reciprocal square root, within 1 ulp of 1 / sqrt
            const float recip = __builtin_amdgcn_rsqf((ssa + ssb) * inv_width + p.eps);
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
              const int j = 2 * h + jj;
              put(i, j, r, qa(i, j, r) * recip);
              *reinterpret_cast<float*>(te_b + T::at(i, j, r)) = qb(i, j, r) * recip;
            }
          }
        }
      }
      rotate_store(half);
    };
    rows(QuadC<0>{}, QuadC<1>{}, 0);
    rows(QuadC<2>{}, QuadC<3>{}, 1);
  } else {
    // Logical quadrant q -> physical (row half (q >> 1) ^ swap_m, column
    // half (q & 1) ^ swap_n); the residual and bias are those of the
    // physical position.
    auto block = [&](auto q) __attribute__((always_inline)) {
      constexpr int kQ = decltype(q)::value;
      const int pr = (kQ >> 1) ^ swap_m, pc = (kQ & 1) ^ swap_n;
      if constexpr (kEpi == SMX_EPI_RESIDUAL_ADD) {
        load_quadrant(p.residual, p.ldr, p.residual_f32 ? 4 : 2, p.residual_f32, pr, pc);
        fence();
      }
#pragma unroll
      for (int j = 0; j < kNB; ++j) {
        float b = 0.f;
        if constexpr (kEpi == SMX_EPI_BIAS_ADD) b = load_vec(p.bias, p.bias_f32, col_base + pc * hn + j * 32 + lcol);
#pragma unroll
        for (int i = 0; i < kMB; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            float v = value(q, i, j, r);
            if constexpr (kEpi == SMX_EPI_RESIDUAL_ADD) v += get(i, j, r);
            if constexpr (kEpi == SMX_EPI_BIAS_ADD) v += b;
            put(i, j, r, v);
          }
      }
      emit_from(tile, pr, col_base + pc * hn);
    };
    block(QuadC<0>{});
    block(QuadC<1>{});
    block(QuadC<2>{});
    block(QuadC<3>{});
  }
}

// The epilogue for the quadrant source kQuad. Each source has a kernel of
// its own: a runtime choice between bodies would leave the 448 live
// accumulators to be split across two arms, which spills. The workgroup
// barrier first makes the LDS free for the staging tiles: every wave has
// finished its main-loop reads and the last DMA has landed.
template <int kQuad, int kMB, int kNB, int kEpi, int kNacc, bool kThin = false>
__device__ __forceinline__ void epilogue(const Params& p, const TileOrigin& o, int row0, int col0,
                                         f32x16 (&acc)[kNacc][kMB][kNB], uint8_t* tile) {
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  epilogue_body<kMB, kNB, kEpi, kNacc, kQuad, kThin>(p, o, row0, col0, acc, tile);
}

template <int kNacc, int kMB, int kNB>
__device__ __forceinline__ void zero_acc(f32x16 (&acc)[kNacc][kMB][kNB]) {
#pragma unroll
  for (int s = 0; s < kNacc; ++s)
#pragma unroll
    for (int i = 0; i < kMB; ++i)
#pragma unroll
      for (int j = 0; j < kNB; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[s][i][j][r] = 0.0f;
}

}  // namespace smx
