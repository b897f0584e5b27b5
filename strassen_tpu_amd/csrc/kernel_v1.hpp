// Compact-tile gfx950 kernel: both operand sums formed in registers.
//
// Serves strassen_matmul with a plain weight (B^T [N, K]), the drop-in call
// that has no pre-summed weight: per K slab the workgroup loads the raw A and
// B quadrant segments into registers, forms the seven A operands and the
// seven B operands there, writes them to LDS and runs the seven products into
// seven persistent FP32 accumulators. The same staging with the raw quadrants
// and eight products gives the compact-tile cubic control.
#pragma once

#include "common.hpp"

namespace smx {
namespace v1 {

template <int kAlgo, int kWavesM, int kWavesN, int kMB, int kNB, int kTK>
struct Cfg {
  static constexpr int algo = kAlgo;
  static constexpr int nops = kAlgo == 7 ? 7 : 4;  // operands per side in LDS
  static constexpr int nacc = kAlgo == 7 ? 7 : 4;  // accumulator sets
  static constexpr int wm = kWavesM, wn = kWavesN;
  static constexpr int mb = kMB, nb = kNB;  // 32x32 blocks per wave
  static constexpr int TM = 32 * kMB * kWavesM;
  static constexpr int TN = 32 * kNB * kWavesN;
  static constexpr int TK = kTK;                 // product-space K per slab
  static constexpr int kRowBytes = TK * 2 + 16;  // padded LDS row
  static constexpr int kChunksPerRow = TK / 8;   // 16-byte chunks per row
  static constexpr int kAVec = TM * kChunksPerRow / kThreads;
  static constexpr int kBVec = TN * kChunksPerRow / kThreads;
  static constexpr int kLdsA = nops * TM * kRowBytes;
  static constexpr int kLdsB = nops * TN * kRowBytes;
  static constexpr int kLds = kLdsA + kLdsB;
  static_assert(kWavesM * kWavesN * 64 == kThreads, "4 waves");
  static_assert(TM * kChunksPerRow % kThreads == 0, "A staging divides");
  static_assert(TN * kChunksPerRow % kThreads == 0, "B staging divides");
  static_assert(TK % 16 == 0, "TK is a multiple of the MFMA depth");
};

template <class C>
__device__ __forceinline__ void load_slab(const Params& p, const int64_t (&a_row0)[2], const int64_t (&b_row0)[2],
                                          int slab, u32x4 (&ra)[4][C::kAVec], u32x4 (&rb)[4][C::kBVec]) {
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
      ra[q][v] = *reinterpret_cast<const u32x4*>(p.a + (a_row0[rh] + row) * p.lda + kcol0 + kh * hk + ch * 8);
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
      rb[q][v] = *reinterpret_cast<const u32x4*>(p.b + (b_row0[nh] + row) * p.ldb + kcol0 + kh * hk + ch * 8);
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
    const int off = (idx / C::kChunksPerRow) * C::kRowBytes + (idx % C::kChunksPerRow) * 16;
    const u32x4 q[4] = {ra[0][v], ra[1][v], ra[2][v], ra[3][v]};
    if constexpr (C::algo == 7) {
      u32x4 ops[7];
      strassen_a_ops(q, ops);
#pragma unroll
      for (int o = 0; o < 7; ++o) *reinterpret_cast<u32x4*>(lds_a + o * C::TM * C::kRowBytes + off) = ops[o];
    } else {
#pragma unroll
      for (int o = 0; o < 4; ++o) *reinterpret_cast<u32x4*>(lds_a + o * C::TM * C::kRowBytes + off) = q[o];
    }
  }
#pragma unroll
  for (int v = 0; v < C::kBVec; ++v) {
    const int idx = t + v * kThreads;
    const int off = (idx / C::kChunksPerRow) * C::kRowBytes + (idx % C::kChunksPerRow) * 16;
    const u32x4 q[4] = {rb[0][v], rb[1][v], rb[2][v], rb[3][v]};
    if constexpr (C::algo == 7) {
      u32x4 ops[7];
      strassen_b_ops(q, ops);
#pragma unroll
      for (int o = 0; o < 7; ++o) *reinterpret_cast<u32x4*>(lds_b + o * C::TN * C::kRowBytes + off) = ops[o];
    } else {
#pragma unroll
      for (int o = 0; o < 4; ++o) *reinterpret_cast<u32x4*>(lds_b + o * C::TN * C::kRowBytes + off) = q[o];
    }
  }
}

template <class C>
__device__ __forceinline__ bf16x8 frag(const uint8_t* base, int o, int rows, int row, int koff) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(base + (o * rows + row) * C::kRowBytes + koff));
}

// MFMA over one LDS slab; acc[set][i][j] over the wave's mb x nb blocks.
template <class C>
__device__ __forceinline__ void mma_slab(const uint8_t* lds, f32x16 (&acc)[C::nacc][C::mb][C::nb], int wave_m,
                                         int wave_n) {
  const int lane = threadIdx.x & 63;
  const uint8_t* lds_a = lds;
  const uint8_t* lds_b = lds + C::kLdsA;
  const int lrow = lane & 31;
  const int lk = (lane >> 5) * 16;
#pragma unroll
  for (int ks = 0; ks < C::TK / 16; ++ks) {
    const int koff = ks * 32 + lk;
    if constexpr (C::algo == 7) {
      // Issue order P4 P6 P5 P2 P7 P3 P1 (strassen_pallas.py:556-565).
      constexpr int order[7] = {3, 5, 4, 1, 6, 2, 0};
#pragma unroll
      for (int x = 0; x < 7; ++x) {
        const int o = order[x];
        bf16x8 fa[C::mb], fb[C::nb];
#pragma unroll
        for (int i = 0; i < C::mb; ++i) fa[i] = frag<C>(lds_a, o, C::TM, (wave_m * C::mb + i) * 32 + lrow, koff);
#pragma unroll
        for (int j = 0; j < C::nb; ++j) fb[j] = frag<C>(lds_b, o, C::TN, (wave_n * C::nb + j) * 32 + lrow, koff);
#pragma unroll
        for (int i = 0; i < C::mb; ++i)
#pragma unroll
          for (int j = 0; j < C::nb; ++j)
            acc[o][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[o][i][j], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int ao0 = half ? 1 : 0, ao1 = half ? 3 : 2;
        const int bo0 = half ? 2 : 0, bo1 = half ? 3 : 1;
        bf16x8 fa0[C::mb], fa1[C::mb], fb0[C::nb], fb1[C::nb];
#pragma unroll
        for (int i = 0; i < C::mb; ++i) {
          const int row = (wave_m * C::mb + i) * 32 + lrow;
          fa0[i] = frag<C>(lds_a, ao0, C::TM, row, koff);
          fa1[i] = frag<C>(lds_a, ao1, C::TM, row, koff);
        }
#pragma unroll
        for (int j = 0; j < C::nb; ++j) {
          const int row = (wave_n * C::nb + j) * 32 + lrow;
          fb0[j] = frag<C>(lds_b, bo0, C::TN, row, koff);
          fb1[j] = frag<C>(lds_b, bo1, C::TN, row, koff);
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

template <class C, int kEpi>
__global__ __launch_bounds__(kThreads, 1) void gemm_v1(Params p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int wave = threadIdx.x >> 6;
  const int wave_m = wave / C::wn;
  const int wave_n = wave % C::wn;

  int tile_m, tile_n;
  tile_of(blockIdx.x, p.tiles_m, p.tiles_n, p.group_m, p.raster, tile_m, tile_n);
  const TileOrigin o = tile_origin(p, (int64_t)tile_m * C::TM, (int64_t)tile_n * C::TN);
  const int hm = p.bm / 2, hn = p.bn / 2;
  const int64_t a_row0[2] = {o.ti * p.bm + o.tr, o.ti * p.bm + hm + o.tr};
  const int64_t b_row0[2] = {o.tj * p.bn + o.tc, o.tj * p.bn + hn + o.tc};

  f32x16 acc[C::nacc][C::mb][C::nb];
  zero_acc(acc);

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
  using T = StageTile<32 * C::mb, 32 * C::nb>;
  static_assert(kEpiLds<kEpi, 32 * C::mb, 32 * C::nb> <= 160 * 1024, "epilogue staging fits the LDS");
  // The compact path runs the classical formula unpermuted (the host sends
  // formula variants, permutations and partial products to the packed path).
  constexpr int kQuad = C::algo == 7 ? kQuadClassical : kQuadCubic;
  epilogue<kQuad, C::mb, C::nb, kEpi>(p, o, wave_m * C::mb * 32, wave_n * C::nb * 32, acc,
                                      lds + wave * kEpiTiles<kEpi> * T::kBytes);
}

// The general configuration uses 64x32 wave tiles; the q/k epilogue needs
// 64-column waves, so it uses 32x64 wave tiles. Both have TM=128, TN=64.
template <int kAlgo>
using General = Cfg<kAlgo, 2, 2, 2, 1, 32>;
template <int kAlgo>
using ForQK = Cfg<kAlgo, 4, 1, 1, 2, 32>;

}  // namespace v1
}  // namespace smx
