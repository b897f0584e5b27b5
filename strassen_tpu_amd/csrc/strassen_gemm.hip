// Tile-local one-level Strassen GEMM (7 products) and the matched blocked
// cubic GEMM (8 products) for gfx950, with fused epilogues, behind a C ABI.
//
// Semantics follow the reference's strassen_pallas.py:
//   * the caller's (bm, bn, bk) tile defines the 2x2 quadrant split of every
//     A tile (bm x bk) and B tile (bk x bn) (strassen_pallas.py:188-204);
//   * operand sums are the classical ones, each rounded once to bf16
//     (P1..P7, strassen_pallas.py:324-379);
//   * products accumulate in FP32; the epilogue runs on the FP32 quadrant
//     values and the result is rounded once to bf16 (:739-879).
//
// Work decomposition ("product space"). Let hm=bm/2, hn=bn/2, hk=bk/2. Every
// quadrant-level product is an (M/2 x K/2) by (K/2 x N/2) GEMM once the row
// halves of all tiles are stacked: product-space row R = (tile i, row r<hm),
// column C = (tile j, col c<hn), depth k' = (panel s, kk<hk). A workgroup owns
// a TM x TN block of product space, i.e. the same (r, c) positions in all four
// output quadrants. Consequently:
//   * each thread holds all four quadrant values of an output position, so
//     SwiGLU (gate|up), RoPE (a|b) and residual/bias epilogues are
//     register-local;
//   * a TK-deep K slab of the four A quadrants (and four B quadrants) is a set
//     of contiguous row segments in HBM.
// Per K slab the workgroup loads the raw quadrant segments into registers,
// forms the operand sums there (bf16, round-to-nearest-even), writes the
// seven A operands and seven B operands to LDS, and runs the seven products
// on v_mfma_f32_32x32x16_bf16 into seven persistent FP32 accumulators. The
// quadrants are combined once, after the last slab:
//   C0 = P1 + P4 - P5 + P7, C1 = P3 + P5, C2 = P2 + P4, C3 = P1 - P2 + P3 + P6.
// The cubic control uses the same staging and tiling with the raw quadrants
// and eight products into four accumulators
// (experiments/qwen3/benchmark_cubic_control.py:76-113).
//
// Operand layouts in HBM: A is [M, K] row-major (lda >= K). B is supplied
// K-contiguous, i.e. as B^T stored [N, K] row-major (ldb >= K); this is the
// natural storage of a [out, in] projection weight. C is [M, N] (or [M, N/2]
// for SwiGLU) row-major bf16.

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <type_traits>

#include "../../include/strassen_mi355x.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWaveSize = 64;
constexpr int kThreads = 256;  // 4 waves

// ---------------------------------------------------------------------------
// bf16 arithmetic on packed pairs
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

// Eight bf16 lanes unpacked to float.
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

// bf16(x + sy*y) per lane, where sy = +1 or -1. The float sum of two bf16
// values rounded to bf16 is the correctly rounded bf16 sum.
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

// ---------------------------------------------------------------------------
// Kernel configuration
// ---------------------------------------------------------------------------

template <int kAlgo, int kWavesM, int kWavesN, int kMB, int kNB, int kTK>
struct Cfg {
  static constexpr int algo = kAlgo;          // 7 = Strassen, 8 = cubic
  static constexpr int nops = kAlgo == 7 ? 7 : 4;  // operands per side in LDS
  static constexpr int nacc = kAlgo == 7 ? 7 : 4;  // accumulator sets
  static constexpr int wm = kWavesM, wn = kWavesN;
  static constexpr int mb = kMB, nb = kNB;    // 32x32 blocks per wave
  static constexpr int TM = 32 * kMB * kWavesM;
  static constexpr int TN = 32 * kNB * kWavesN;
  static constexpr int TK = kTK;              // product-space K per slab
  static constexpr int kRowBytes = TK * 2 + 16;  // padded LDS row
  static constexpr int kChunksPerRow = TK / 8;   // 16-byte chunks per row
  static constexpr int kAVec = TM * kChunksPerRow / kThreads;  // per quadrant
  static constexpr int kBVec = TN * kChunksPerRow / kThreads;
  static constexpr int kLdsA = nops * TM * kRowBytes;
  static constexpr int kLdsB = nops * TN * kRowBytes;
  static constexpr int kLds = kLdsA + kLdsB;
  static_assert(kWavesM * kWavesN * kWaveSize == kThreads, "4 waves");
  static_assert(TM * kChunksPerRow % kThreads == 0, "A staging divides");
  static_assert(TN * kChunksPerRow % kThreads == 0, "B staging divides");
  static_assert(TK % 16 == 0, "TK is a multiple of the MFMA depth");
};

struct Params {
  const uint16_t* a;
  const uint16_t* b;  // B^T, [N, K]
  uint16_t* c;
  const uint16_t* residual;
  const void* bias;
  const uint16_t* rope_cos;
  const uint16_t* rope_sin;
  const void* rope_scale;
  int64_t m, n, k;
  int64_t lda, ldb, ldc, ldr;
  int32_t bm, bn, bk;
  int32_t bias_f32, scale_f32;
  int32_t head_dim;
  float eps;
  int32_t tiles_m, tiles_n;  // product-space workgroup grid
};

// Maps a workgroup id to a product-space tile. Workgroups are dispatched
// round-robin over the 8 XCDs; consecutive logical tiles are gathered on one
// XCD so that neighbouring tiles share its L2, and inside an XCD tiles walk
// column-groups of kGroupM rows.
__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  int logical = bid;
  if (total % 8 == 0) {
    const int per_xcd = total / 8;
    logical = (bid % 8) * per_xcd + bid / 8;
  }
  constexpr int kGroupM = 8;
  const int group_size = kGroupM * tiles_n;
  const int group = logical / group_size;
  const int first_m = group * kGroupM;
  const int rows_in_group = min(tiles_m - first_m, kGroupM);
  const int in_group = logical - group * group_size;
  tm = first_m + in_group % rows_in_group;
  tn = in_group / rows_in_group;
}

template <class C>
__device__ __forceinline__ void load_slab(const Params& p, int64_t a_row0[2], int64_t b_row0[2],
                                          int slab, u32x4 (&ra)[4][C::kAVec],
                                          u32x4 (&rb)[4][C::kBVec]) {
  // K offset of the slab inside its panel, for both K halves.
  const int hk = p.bk / 2;
  const int64_t kprod = (int64_t)slab * C::TK;
  const int64_t panel = kprod / hk;
  const int64_t kk = kprod - panel * hk;
  const int64_t kcol0 = panel * p.bk + kk;  // K half 0; half 1 adds hk
  const int t = threadIdx.x;
#pragma unroll
  for (int v = 0; v < C::kAVec; ++v) {
    const int idx = t + v * kThreads;
    const int row = idx / C::kChunksPerRow;
    const int ch = idx % C::kChunksPerRow;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int rh = q >> 1, kh = q & 1;
      const uint16_t* src = p.a + (a_row0[rh] + row) * p.lda + kcol0 + kh * hk + ch * 8;
      ra[q][v] = *reinterpret_cast<const u32x4*>(src);
    }
  }
#pragma unroll
  for (int v = 0; v < C::kBVec; ++v) {
    const int idx = t + v * kThreads;
    const int row = idx / C::kChunksPerRow;
    const int ch = idx % C::kChunksPerRow;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      // b quadrant q = (K half q>>1, N half q&1); B^T rows are n.
      const int kh = q >> 1, nh = q & 1;
      const uint16_t* src = p.b + (b_row0[nh] + row) * p.ldb + kcol0 + kh * hk + ch * 8;
      rb[q][v] = *reinterpret_cast<const u32x4*>(src);
    }
  }
}

template <class C>
__device__ __forceinline__ void store_operands(uint8_t* lds, const u32x4 (&ra)[4][C::kAVec],
                                               const u32x4 (&rb)[4][C::kBVec]) {
  const int t = threadIdx.x;
  uint8_t* lds_a = lds;
  uint8_t* lds_b = lds + C::kLdsA;
#pragma unroll
  for (int v = 0; v < C::kAVec; ++v) {
    const int idx = t + v * kThreads;
    const int row = idx / C::kChunksPerRow;
    const int ch = idx % C::kChunksPerRow;
    const int off = row * C::kRowBytes + ch * 16;
    if constexpr (C::algo == 7) {
      const F8 a0 = unpack8(ra[0][v]), a1 = unpack8(ra[1][v]);
      const F8 a2 = unpack8(ra[2][v]), a3 = unpack8(ra[3][v]);
      // A operands of P1..P7: A0+A3, A2+A3, A0, A3, A0+A1, A2-A0, A1-A3.
      u32x4 ops[7];
      ops[0] = sum8<false>(a0, a3);
      ops[1] = sum8<false>(a2, a3);
      ops[2] = ra[0][v];
      ops[3] = ra[3][v];
      ops[4] = sum8<false>(a0, a1);
      ops[5] = sum8<true>(a2, a0);
      ops[6] = sum8<true>(a1, a3);
#pragma unroll
      for (int o = 0; o < 7; ++o)
        *reinterpret_cast<u32x4*>(lds_a + o * C::TM * C::kRowBytes + off) = ops[o];
    } else {
#pragma unroll
      for (int o = 0; o < 4; ++o)
        *reinterpret_cast<u32x4*>(lds_a + o * C::TM * C::kRowBytes + off) = ra[o][v];
    }
  }
#pragma unroll
  for (int v = 0; v < C::kBVec; ++v) {
    const int idx = t + v * kThreads;
    const int row = idx / C::kChunksPerRow;
    const int ch = idx % C::kChunksPerRow;
    const int off = row * C::kRowBytes + ch * 16;
    if constexpr (C::algo == 7) {
      const F8 b0 = unpack8(rb[0][v]), b1 = unpack8(rb[1][v]);
      const F8 b2 = unpack8(rb[2][v]), b3 = unpack8(rb[3][v]);
      // B operands of P1..P7: B0+B3, B0, B1-B3, B2-B0, B3, B0+B1, B2+B3.
      u32x4 ops[7];
      ops[0] = sum8<false>(b0, b3);
      ops[1] = rb[0][v];
      ops[2] = sum8<true>(b1, b3);
      ops[3] = sum8<true>(b2, b0);
      ops[4] = rb[3][v];
      ops[5] = sum8<false>(b0, b1);
      ops[6] = sum8<false>(b2, b3);
#pragma unroll
      for (int o = 0; o < 7; ++o)
        *reinterpret_cast<u32x4*>(lds_b + o * C::TN * C::kRowBytes + off) = ops[o];
    } else {
#pragma unroll
      for (int o = 0; o < 4; ++o)
        *reinterpret_cast<u32x4*>(lds_b + o * C::TN * C::kRowBytes + off) = rb[o][v];
    }
  }
}

// MFMA over one LDS slab. acc[set][i][j] for the wave's mb x nb blocks.
template <class C>
__device__ __forceinline__ void mma_slab(const uint8_t* lds, f32x16 (&acc)[C::nacc][C::mb][C::nb],
                                         int wave_m, int wave_n) {
  const int lane = threadIdx.x & 63;
  const uint8_t* lds_a = lds;
  const uint8_t* lds_b = lds + C::kLdsA;
  const int lrow = lane & 31;
  const int lk = (lane >> 5) * 16;
#pragma unroll
  for (int ks = 0; ks < C::TK / 16; ++ks) {
    const int koff = ks * 32 + lk;
    if constexpr (C::algo == 7) {
#pragma unroll
      for (int pidx = 0; pidx < 7; ++pidx) {
        // Interleaved issue order P4 P6 P5 P2 P7 P3 P1 (strassen_pallas.py:556-565).
        constexpr int order[7] = {3, 5, 4, 1, 6, 2, 0};
        const int o = order[pidx];
        bf16x8 fa[C::mb], fb[C::nb];
#pragma unroll
        for (int i = 0; i < C::mb; ++i) {
          const int row = (wave_m * C::mb + i) * 32 + lrow;
          fa[i] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(
                                                  lds_a + (o * C::TM + row) * C::kRowBytes + koff));
        }
#pragma unroll
        for (int j = 0; j < C::nb; ++j) {
          const int row = (wave_n * C::nb + j) * 32 + lrow;
          fb[j] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(
                                                  lds_b + (o * C::TN + row) * C::kRowBytes + koff));
        }
#pragma unroll
        for (int i = 0; i < C::mb; ++i)
#pragma unroll
          for (int j = 0; j < C::nb; ++j)
            acc[o][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[o][i][j], 0, 0, 0);
      }
    } else {
      // Cubic: (a0,b0)->0 (a0,b1)->1 (a2,b0)->2 (a2,b1)->3 (a1,b2)->0 (a1,b3)->1
      // (a3,b2)->2 (a3,b3)->3, in that order.
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int ao0 = half ? 1 : 0, ao1 = half ? 3 : 2;
        const int bo0 = half ? 2 : 0, bo1 = half ? 3 : 1;
        bf16x8 fa0[C::mb], fa1[C::mb], fb0[C::nb], fb1[C::nb];
#pragma unroll
        for (int i = 0; i < C::mb; ++i) {
          const int row = (wave_m * C::mb + i) * 32 + lrow;
          fa0[i] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(
                                                   lds_a + (ao0 * C::TM + row) * C::kRowBytes + koff));
          fa1[i] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(
                                                   lds_a + (ao1 * C::TM + row) * C::kRowBytes + koff));
        }
#pragma unroll
        for (int j = 0; j < C::nb; ++j) {
          const int row = (wave_n * C::nb + j) * 32 + lrow;
          fb0[j] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(
                                                   lds_b + (bo0 * C::TN + row) * C::kRowBytes + koff));
          fb1[j] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(
                                                   lds_b + (bo1 * C::TN + row) * C::kRowBytes + koff));
        }
#pragma unroll
        for (int i = 0; i < C::mb; ++i)
#pragma unroll
          for (int j = 0; j < C::nb; ++j) {
            acc[0][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa0[i], fb0[j], acc[0][i][j], 0, 0, 0);
            acc[1][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa0[i], fb1[j], acc[1][i][j], 0, 0, 0);
            acc[2][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa1[i], fb0[j], acc[2][i][j], 0, 0, 0);
            acc[3][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa1[i], fb1[j], acc[3][i][j], 0, 0, 0);
          }
      }
    }
  }
}

__device__ __forceinline__ float silu_f32(float x) { return x / (1.0f + expf(-x)); }

__device__ __forceinline__ float load_vec(const void* v, int is_f32, int64_t i) {
  return is_f32 ? reinterpret_cast<const float*>(v)[i] : bf16_to_f32(reinterpret_cast<const uint16_t*>(v)[i]);
}

// Sum over the 32 lanes of a half-wave (lanes sharing lane>>5).
__device__ __forceinline__ float half_wave_sum(float x) {
#pragma unroll
  for (int s = 16; s >= 1; s >>= 1) x += __shfl_xor(x, s, 64);
  return x;
}

template <class C, int kEpi>
__global__ __launch_bounds__(kThreads, 1) void gemm_kernel(Params p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int wave_m = wave / C::wn;
  const int wave_n = wave % C::wn;

  int tile_m, tile_n;
  tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tile_m, tile_n);
  const int hm = p.bm / 2, hn = p.bn / 2, hk = p.bk / 2;
  // Product-space origin of this workgroup.
  const int64_t prow0 = (int64_t)tile_m * C::TM;
  const int64_t pcol0 = (int64_t)tile_n * C::TN;
  // Physical rows of the two row halves (A) and columns of the two column
  // halves (B^T rows, C columns) for this workgroup.
  const int64_t ti = prow0 / hm, tr = prow0 % hm;
  const int64_t tj = pcol0 / hn, tc = pcol0 % hn;
  int64_t a_row0[2] = {ti * p.bm + tr, ti * p.bm + hm + tr};
  int64_t b_row0[2] = {tj * p.bn + tc, tj * p.bn + hn + tc};

  f32x16 acc[C::nacc][C::mb][C::nb];
#pragma unroll
  for (int s = 0; s < C::nacc; ++s)
#pragma unroll
    for (int i = 0; i < C::mb; ++i)
#pragma unroll
      for (int j = 0; j < C::nb; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[s][i][j][r] = 0.0f;

  const int nslabs = (int)((p.k / 2) / C::TK);
  u32x4 ra[4][C::kAVec], rb[4][C::kBVec];
  load_slab<C>(p, a_row0, b_row0, 0, ra, rb);
  for (int slab = 0; slab < nslabs; ++slab) {
    store_operands<C>(lds, ra, rb);
    __syncthreads();
    if (slab + 1 < nslabs) load_slab<C>(p, a_row0, b_row0, slab + 1, ra, rb);
    mma_slab<C>(lds, acc, wave_m, wave_n);
    __syncthreads();
  }

  // ---- epilogue ----------------------------------------------------------
  // Lane layout of a 32x32 accumulator block: column lane%32, row
  // 8*(r/4) + 4*(lane/32) + r%4 for register r.
  const int lcol = lane & 31;
  const int lrow4 = (lane >> 5) * 4;
#pragma unroll
  for (int i = 0; i < C::mb; ++i) {
#pragma unroll
    for (int j = 0; j < C::nb; ++j) {
      const int64_t cc = tc + (wave_n * C::nb + j) * 32 + lcol;  // col inside the half
      const int64_t col_l = tj * p.bn + cc;                       // left-half column
      const int64_t col_r = col_l + hn;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t rr = tr + (wave_m * C::mb + i) * 32 + 8 * (r >> 2) + lrow4 + (r & 3);
        const int64_t row_t = ti * p.bm + rr;
        const int64_t row_b = row_t + hm;
        float q0, q1, q2, q3;
        if constexpr (C::algo == 7) {
          const float p1 = acc[0][i][j][r], p2 = acc[1][i][j][r], p3 = acc[2][i][j][r];
          const float p4 = acc[3][i][j][r], p5 = acc[4][i][j][r], p6 = acc[5][i][j][r];
          const float p7 = acc[6][i][j][r];
          q0 = ((p4 - p5) + p7) + p1;
          q1 = p5 + p3;
          q2 = p4 + p2;
          q3 = ((p6 - p2) + p3) + p1;
        } else {
          q0 = acc[0][i][j][r];
          q1 = acc[1][i][j][r];
          q2 = acc[2][i][j][r];
          q3 = acc[3][i][j][r];
        }
        if constexpr (kEpi == SMX_EPI_SWIGLU) {
          // Quadrants 0/2 are gate, 1/3 up; output [M, N/2] at column (tj*hn + cc).
          const int64_t ocol = tj * hn + cc;
          p.c[row_t * p.ldc + ocol] = f32_to_bf16(silu_f32(q0) * q1);
          p.c[row_b * p.ldc + ocol] = f32_to_bf16(silu_f32(q2) * q3);
        } else if constexpr (kEpi == SMX_EPI_RESIDUAL_ADD) {
          q0 += bf16_to_f32(p.residual[row_t * p.ldr + col_l]);
          q1 += bf16_to_f32(p.residual[row_t * p.ldr + col_r]);
          q2 += bf16_to_f32(p.residual[row_b * p.ldr + col_l]);
          q3 += bf16_to_f32(p.residual[row_b * p.ldr + col_r]);
          p.c[row_t * p.ldc + col_l] = f32_to_bf16(q0);
          p.c[row_t * p.ldc + col_r] = f32_to_bf16(q1);
          p.c[row_b * p.ldc + col_l] = f32_to_bf16(q2);
          p.c[row_b * p.ldc + col_r] = f32_to_bf16(q3);
        } else if constexpr (kEpi == SMX_EPI_BIAS_ADD) {
          const float bl = load_vec(p.bias, p.bias_f32, col_l);
          const float br = load_vec(p.bias, p.bias_f32, col_r);
          p.c[row_t * p.ldc + col_l] = f32_to_bf16(q0 + bl);
          p.c[row_t * p.ldc + col_r] = f32_to_bf16(q1 + br);
          p.c[row_b * p.ldc + col_l] = f32_to_bf16(q2 + bl);
          p.c[row_b * p.ldc + col_r] = f32_to_bf16(q3 + br);
        } else if constexpr (kEpi == SMX_EPI_QK_NORM_ROPE) {
          // Stored as-is here; the normalisation needs whole head segments and
          // is done in the dedicated pass below.
          acc[0][i][j][r] = q0;
          acc[1][i][j][r] = q1;
          acc[2][i][j][r] = q2;
          acc[3][i][j][r] = q3;
        } else {
          p.c[row_t * p.ldc + col_l] = f32_to_bf16(q0);
          p.c[row_t * p.ldc + col_r] = f32_to_bf16(q1);
          p.c[row_b * p.ldc + col_l] = f32_to_bf16(q2);
          p.c[row_b * p.ldc + col_r] = f32_to_bf16(q3);
        }
      }
    }
  }

  if constexpr (kEpi == SMX_EPI_QK_NORM_ROPE) {
    // Per-head RMSNorm then RoPE (strassen_pallas.py:793-835). A head owns
    // head_dim/2 = 64 consecutive columns of a tile half, which are the wave's
    // column blocks j = 2h, 2h+1 (the host guarantees nb % 2 == 0 and
    // 64-aligned wave columns). Quadrants 0/2 hold the a half, 1/3 the b half.
    const float inv_width = 1.0f / (float)p.head_dim;
    static_assert(kEpi != SMX_EPI_QK_NORM_ROPE || C::nb % 2 == 0, "qk epilogue needs 64-wide waves");
#pragma unroll
    for (int i = 0; i < C::mb; ++i) {
#pragma unroll
      for (int h = 0; h < C::nb / 2; ++h) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t rr = tr + (wave_m * C::mb + i) * 32 + 8 * (r >> 2) + lrow4 + (r & 3);
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            const int sa = 2 * half, sb = 2 * half + 1;  // a / b quadrant sets
            const float a0 = acc[sa][i][2 * h][r], a1 = acc[sa][i][2 * h + 1][r];
            const float b0 = acc[sb][i][2 * h][r], b1 = acc[sb][i][2 * h + 1][r];
            const float ssa = half_wave_sum(a0 * a0 + a1 * a1);
            const float ssb = half_wave_sum(b0 * b0 + b1 * b1);
            const float recip = 1.0f / sqrtf((ssa + ssb) * inv_width + p.eps);
            const int64_t row = ti * p.bm + rr + half * hm;
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
              const int j = 2 * h + jj;
              const int64_t cc = tc + (wave_n * C::nb + j) * 32 + lcol;
              const float ga = load_vec(p.rope_scale, p.scale_f32, cc);
              const float gb = load_vec(p.rope_scale, p.scale_f32, hn + cc);
              const float cs = bf16_to_f32(p.rope_cos[row * hn + cc]);
              const float sn = bf16_to_f32(p.rope_sin[row * hn + cc]);
              const float na = acc[sa][i][j][r] * recip * ga;
              const float nbv = acc[sb][i][j][r] * recip * gb;
              const int64_t col_l = tj * p.bn + cc;
              p.c[row * p.ldc + col_l] = f32_to_bf16(na * cs - nbv * sn);
              p.c[row * p.ldc + col_l + hn] = f32_to_bf16(nbv * cs + na * sn);
            }
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Dispatch
// ---------------------------------------------------------------------------

thread_local char g_error[512] = "";

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

template <class C, int kEpi>
int launch(const Params& p0, hipStream_t stream) {
  Params p = p0;
  p.tiles_m = (int)((p.m / 2) / C::TM);
  p.tiles_n = (int)((p.n / 2) / C::TN);
  auto kern = gemm_kernel<C, kEpi>;
  static bool attr_set = false;  // per instantiation
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, C::kLds);
    if (e != hipSuccess) return fail(SMX_ERR_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(e));
    attr_set = true;
  }
  const int grid = p.tiles_m * p.tiles_n;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kThreads), C::kLds, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SMX_ERR_LAUNCH, "kernel launch: %s", hipGetErrorString(e));
  return SMX_OK;
}

// Tile configurations. The general one uses 64x32 wave tiles; the q/k
// epilogue needs 64-column waves, so it uses 32x64 wave tiles.
using Strassen = Cfg<7, 2, 2, 2, 1, 32>;       // TM=128, TN=64
using StrassenQK = Cfg<7, 4, 1, 1, 2, 32>;     // TM=128, TN=64
using Cubic = Cfg<8, 2, 2, 2, 1, 32>;          // TM=128, TN=64
using CubicQK = Cfg<8, 4, 1, 1, 2, 32>;        // TM=128, TN=64

template <int kAlgo>
int dispatch(const Params& p, int epilogue, hipStream_t s) {
  using G = typename std::conditional<kAlgo == 7, Strassen, Cubic>::type;
  using Q = typename std::conditional<kAlgo == 7, StrassenQK, CubicQK>::type;
  switch (epilogue) {
    case SMX_EPI_NONE: return launch<G, SMX_EPI_NONE>(p, s);
    case SMX_EPI_SWIGLU: return launch<G, SMX_EPI_SWIGLU>(p, s);
    case SMX_EPI_RESIDUAL_ADD: return launch<G, SMX_EPI_RESIDUAL_ADD>(p, s);
    case SMX_EPI_BIAS_ADD: return launch<G, SMX_EPI_BIAS_ADD>(p, s);
    case SMX_EPI_QK_NORM_ROPE: return launch<Q, SMX_EPI_QK_NORM_ROPE>(p, s);
  }
  return fail(SMX_ERR_INVALID, "unknown epilogue %d", epilogue);
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

}  // namespace

extern "C" {

int smx_version(void) { return SMX_VERSION; }

const char* smx_last_error(void) { return g_error; }

int smx_tile_requirements(int32_t algo, int32_t epilogue, int32_t* tm, int32_t* tn, int32_t* tk) {
  if (algo != SMX_ALGO_STRASSEN && algo != SMX_ALGO_CUBIC) return fail(SMX_ERR_INVALID, "algo must be 7 or 8");
  // All current configurations share TM=128, TN=64, TK=32.
  (void)epilogue;
  if (tm) *tm = Strassen::TM;
  if (tn) *tn = Strassen::TN;
  if (tk) *tk = Strassen::TK;
  return SMX_OK;
}

int smx_gemm(const smx_gemm_desc* d, const void* a, const void* b, void* c, const void* residual,
             const void* bias, const void* rope_cos, const void* rope_sin, const void* rope_scale,
             void* stream) {
  g_error[0] = 0;
  if (!d) return fail(SMX_ERR_INVALID, "null descriptor");
  if (d->algo != SMX_ALGO_STRASSEN && d->algo != SMX_ALGO_CUBIC)
    return fail(SMX_ERR_INVALID, "algo must be %d (Strassen) or %d (cubic), got %d", SMX_ALGO_STRASSEN,
                SMX_ALGO_CUBIC, d->algo);
  if (d->m <= 0 || d->n <= 0 || d->k <= 0) return fail(SMX_ERR_INVALID, "empty problem m=%lld n=%lld k=%lld",
                                                      (long long)d->m, (long long)d->n, (long long)d->k);
  if (d->bm <= 0 || d->bn <= 0 || d->bk <= 0 || d->m % d->bm || d->n % d->bn || d->k % d->bk)
    return fail(SMX_ERR_INVALID, "M, N, K must be divisible by bm, bn, bk");
  const int hm = d->bm / 2, hn = d->bn / 2, hk = d->bk / 2;
  if (d->bm % 2 || d->bn % 2 || d->bk % 2 || hm % Strassen::TM || hn % Strassen::TN || hk % Strassen::TK)
    return fail(SMX_ERR_UNSUPPORTED,
                "tile (bm=%d, bn=%d, bk=%d) unsupported on gfx950: need bm %% %d == 0, bn %% %d == 0, bk %% %d == 0",
                d->bm, d->bn, d->bk, 2 * Strassen::TM, 2 * Strassen::TN, 2 * Strassen::TK);
  if (d->b_layout != SMX_B_KCONTIG)
    return fail(SMX_ERR_UNSUPPORTED, "only K-contiguous B (B^T stored [N,K]) is supported");
  if (!a || !b || !c) return fail(SMX_ERR_INVALID, "null operand pointer");
  if (!aligned16(a) || !aligned16(b)) return fail(SMX_ERR_INVALID, "A and B must be 16-byte aligned");
  if (d->lda < d->k || d->ldb < d->k || d->lda % 8 || d->ldb % 8)
    return fail(SMX_ERR_INVALID, "lda/ldb must be >= K and multiples of 8 elements");
  const int64_t out_cols = d->epilogue == SMX_EPI_SWIGLU ? d->n / 2 : d->n;
  if (d->ldc < out_cols) return fail(SMX_ERR_INVALID, "ldc must be >= output width");
  Params p{};
  p.a = (const uint16_t*)a;
  p.b = (const uint16_t*)b;
  p.c = (uint16_t*)c;
  p.m = d->m;
  p.n = d->n;
  p.k = d->k;
  p.lda = d->lda;
  p.ldb = d->ldb;
  p.ldc = d->ldc;
  p.ldr = d->ldr;
  p.bm = d->bm;
  p.bn = d->bn;
  p.bk = d->bk;
  p.head_dim = d->rope_head_dim;
  p.eps = d->rope_eps;
  p.bias_f32 = d->aux_f32 & SMX_AUX_BIAS_F32 ? 1 : 0;
  p.scale_f32 = d->aux_f32 & SMX_AUX_SCALE_F32 ? 1 : 0;
  switch (d->epilogue) {
    case SMX_EPI_NONE:
    case SMX_EPI_SWIGLU:
      break;
    case SMX_EPI_RESIDUAL_ADD:
      if (!residual) return fail(SMX_ERR_INVALID, "residual_add epilogue requires residual");
      if (d->ldr < d->n) return fail(SMX_ERR_INVALID, "ldr must be >= N");
      p.residual = (const uint16_t*)residual;
      break;
    case SMX_EPI_BIAS_ADD:
      if (!bias) return fail(SMX_ERR_INVALID, "bias_add epilogue requires bias");
      p.bias = bias;
      break;
    case SMX_EPI_QK_NORM_ROPE:
      if (!rope_cos || !rope_sin || !rope_scale)
        return fail(SMX_ERR_INVALID, "qk_norm_rope requires rope_cos, rope_sin and rope_scale");
      if (d->rope_head_dim != 128)
        return fail(SMX_ERR_UNSUPPORTED, "qk_norm_rope on gfx950 supports head_dim 128, got %d", d->rope_head_dim);
      if (d->bn % (2 * d->rope_head_dim))
        return fail(SMX_ERR_INVALID, "qk_norm_rope needs bn a multiple of 2*head_dim");
      p.rope_cos = (const uint16_t*)rope_cos;
      p.rope_sin = (const uint16_t*)rope_sin;
      p.rope_scale = rope_scale;
      break;
    default:
      return fail(SMX_ERR_INVALID, "unknown epilogue %d", d->epilogue);
  }
  hipStream_t s = (hipStream_t)stream;
  return d->algo == SMX_ALGO_STRASSEN ? dispatch<7>(p, d->epilogue, s) : dispatch<8>(p, d->epilogue, s);
}

}  // extern "C"
