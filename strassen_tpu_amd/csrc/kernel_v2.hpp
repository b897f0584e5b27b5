// Pipelined gfx950 kernel: 128x128 product-space workgroup tile, four waves
// of 64x64, K advanced 16 product-space columns per stage through a
// double-buffered, fragment-ordered LDS layout.
//
// LDS fragment: the 16-byte chunks of one 32x16 bf16 MFMA operand in lane
// order (lane l: row/column l%32, k 8*(l/32)..+8), 1 KB, read with one
// conflict-free ds_read_b128 per lane.
//
// Per stage (16 product-space k):
//   A: every thread loads one 16-byte chunk of each of the four raw A
//      quadrants (global -> VGPR). Strassen forms the seven A operands there
//      (bf16 sums, strassen_pallas.py:324-379); the cubic keeps the raw four.
//      They are written to LDS in fragment order.
//   B: loaded straight into LDS (global_load_lds_dwordx4, no VGPRs). Strassen
//      reads the seven B operands from the pre-summed weight [N/2*7, K/2]
//      (strassen_weight_layout); the cubic reads the four raw quadrants from
//      B^T [N, K].
//   MFMA: each wave runs 7 (Strassen) or 8 (cubic) products over its 2x2
//      blocks of 32x32, into 7 or 4 persistent FP32 accumulator sets.
// One barrier per stage: buffer s%2 is read while s+1 is being filled.
#pragma once

#include "common.hpp"

namespace smx {
namespace v2 {

constexpr int TM = 128, TN = 128, TK = 16;
constexpr int kFrag = 1024;
constexpr int kBlocks = 4;  // 32-row (or 32-column) blocks per tile side

template <int kAlgo>
struct Lay {
  static constexpr int nops = kAlgo == 7 ? 7 : 4;
  static constexpr int kA = nops * kBlocks * kFrag;
  static constexpr int kB = nops * kBlocks * kFrag;
  static constexpr int kStage = kA + kB;
  static constexpr int kLds = 2 * kStage;
  static constexpr int kBFragsPerWave = nops;  // nops*4 fragments over 4 waves
};

__device__ __forceinline__ void lds_barrier() {
  // Make this wave's LDS writes and LDS-DMA loads complete, then barrier.
  // The "memory" clobber keeps the compiler from moving LDS accesses across.
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// v_mfma_f32_32x32x16_bf16 with the accumulator pinned to AGPRs / VGPRs.
// An accumulator is reused only 16+ MFMAs later and read by VALU only after
// mfma_drain(), so no MFMA result hazard is left to the compiler.
__device__ __forceinline__ void mfma_agpr(f32x16& c, const bf16x8& a, const bf16x8& b) {
  asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma_vgpr(f32x16& c, const bf16x8& a, const bf16x8& b) {
  asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
}
// Wait states between the last MFMA writes and VALU / v_accvgpr_read reads
// of the accumulators (more than the longest MFMA result latency). Each
// accumulator then passes through an empty volatile asm that "defines" it,
// so no read of it can be scheduled above the s_nops.
template <int kSets>
__device__ __forceinline__ void mfma_drain(f32x16 (&acc)[kSets][2][2]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
  for (int s = 0; s < kSets; ++s)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (s < 4)
          asm volatile("" : "+a"(acc[s][i][j]));
        else
          asm volatile("" : "+v"(acc[s][i][j]));
      }
}

__device__ __forceinline__ bf16x8 ld_frag(const uint8_t* p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(p));
}

template <int kAlgo, int kEpi>
__global__ __launch_bounds__(kThreads, 1) void gemm_v2(Params p) {
  using L = Lay<kAlgo>;
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;

  int tile_m, tile_n;
  tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tile_m, tile_n);
  const TileOrigin o = tile_origin(p, (int64_t)tile_m * TM, (int64_t)tile_n * TN);
  const int hm = p.bm / 2, hn = p.bn / 2, hk = p.bk / 2;

  // ---- A staging: thread -> (row ar of the tile, k half ah) ----
  const int ar = tid >> 1, ah = tid & 1;
  const uint16_t* a_top = p.a + (o.ti * p.bm + o.tr + ar) * p.lda + ah * 8;
  const uint16_t* a_bot = a_top + (int64_t)hm * p.lda;
  const int a_chunk = (ar >> 5) * kFrag + ((ah << 5) | (ar & 31)) * 16;

  // ---- B staging: this wave's fragments f = wave + 4 x, x < nops ----
  // Strassen: f = op*4 + cb, source row (pcol*7 + op) of the pre-summed weight.
  // Cubic:    f = quadrant*4 + cb, source row of B^T.
  // Addresses are a wave-uniform base plus a 32-bit per-lane byte offset.
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const uint16_t* b_wave;  // row of lane 0 for this workgroup
  uint32_t b_lane_off;     // bytes from b_wave to this lane's 16-byte chunk
  if constexpr (kAlgo == 7) {
    b_wave = p.b + ((o.tj * hn + o.tc) * 7) * p.ldb;
    b_lane_off = (uint32_t)(((lane & 31) * 7) * p.ldb + (lane >> 5) * 8) * 2u;
  } else {
    b_wave = p.b + (o.tj * p.bn + o.tc) * p.ldb;
    b_lane_off = (uint32_t)((lane & 31) * p.ldb + (lane >> 5) * 8) * 2u;
  }

  f32x16 acc[L::nops][2][2];
  zero_acc(acc);

  const int nstages = (int)((p.k / 2) / TK);
  // Physical column of the loaded stage in K half 0 (half 1 adds hk) and its
  // product-space k (column of the pre-summed weight). Advancing stops at the
  // last stage, so the pipeline's two trailing prefetches re-load it instead
  // of branching (one uniform loop body, no peeled tail).
  int64_t kcol = 0, kprod = 0;
  int kk = 0, loaded = 0;
  auto advance = [&]() {
    const bool more = loaded + 1 < nstages;
    const int kk_next = kk + TK;
    const bool wrap = kk_next == hk;
    kprod = more ? kprod + TK : kprod;
    kcol = more ? kcol + TK + (wrap ? hk : 0) : kcol;
    kk = more ? (wrap ? 0 : kk_next) : kk;
    loaded = more ? loaded + 1 : loaded;
  };

  u32x4 ra[4];
  auto load_a = [&]() {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint16_t* src = ((q >> 1) ? a_bot : a_top) + kcol + (q & 1) * hk;
      ra[q] = *reinterpret_cast<const u32x4*>(src);
    }
  };
  auto store_a = [&](uint8_t* sa) {
    if constexpr (kAlgo == 7) {
      // A operands of P1..P7: A0+A3, A2+A3, A0, A3, A0+A1, A2-A0, A1-A3, one
      // packed pair of elements at a time to keep few values live.
      u32x4 s1, s2, s5, s6, s7;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a0l = lo_f32(ra[0][i]), a0h = hi_f32(ra[0][i]);
        const float a1l = lo_f32(ra[1][i]), a1h = hi_f32(ra[1][i]);
        const float a2l = lo_f32(ra[2][i]), a2h = hi_f32(ra[2][i]);
        const float a3l = lo_f32(ra[3][i]), a3h = hi_f32(ra[3][i]);
        s1[i] = pack_bf16(a0l + a3l, a0h + a3h);
        s2[i] = pack_bf16(a2l + a3l, a2h + a3h);
        s5[i] = pack_bf16(a0l + a1l, a0h + a1h);
        s6[i] = pack_bf16(a2l - a0l, a2h - a0h);
        s7[i] = pack_bf16(a1l - a3l, a1h - a3h);
        __builtin_amdgcn_sched_barrier(0);
      }
      uint8_t* dst = sa + a_chunk;
      *reinterpret_cast<u32x4*>(dst + 0 * kBlocks * kFrag) = s1;
      *reinterpret_cast<u32x4*>(dst + 1 * kBlocks * kFrag) = s2;
      *reinterpret_cast<u32x4*>(dst + 2 * kBlocks * kFrag) = ra[0];
      *reinterpret_cast<u32x4*>(dst + 3 * kBlocks * kFrag) = ra[3];
      *reinterpret_cast<u32x4*>(dst + 4 * kBlocks * kFrag) = s5;
      *reinterpret_cast<u32x4*>(dst + 5 * kBlocks * kFrag) = s6;
      *reinterpret_cast<u32x4*>(dst + 6 * kBlocks * kFrag) = s7;
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) *reinterpret_cast<u32x4*>(sa + q * kBlocks * kFrag + a_chunk) = ra[q];
    }
  };
  auto dma_b = [&](uint8_t* sb) {
#pragma unroll
    for (int x = 0; x < L::kBFragsPerWave; ++x) {
      const int f = wave_u + 4 * x;
      const int op = f >> 2, cb = f & 3;
      const uint16_t* base;
      if constexpr (kAlgo == 7) {
        base = b_wave + (int64_t)(cb * 32 * 7 + op) * p.ldb + kprod;
      } else {
        const int kh = op >> 1, nh = op & 1;
        base = b_wave + (int64_t)(nh * hn + cb * 32) * p.ldb + kcol + kh * hk;
      }
      const void* src = reinterpret_cast<const uint8_t*>(base) + b_lane_off;
      __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(sb + f * kFrag), 16, 0, 0);
    }
  };
  // Fragments of one product (Strassen) or one quadrant pair (cubic):
  // A blocks 2wm, 2wm+1 and B blocks 2wn, 2wn+1.
  struct Frags {
    bf16x8 a0, a1, b0, b1;
  };
  const int lo = lane * 16;
  auto load_frags = [&](const uint8_t* sa, const uint8_t* sb, int opa, int opb) {
    Frags f;
    f.a0 = ld_frag(sa + opa * kBlocks * kFrag + (2 * wm) * kFrag + lo);
    f.a1 = ld_frag(sa + opa * kBlocks * kFrag + (2 * wm + 1) * kFrag + lo);
    f.b0 = ld_frag(sb + opb * kBlocks * kFrag + (2 * wn) * kFrag + lo);
    f.b1 = ld_frag(sb + opb * kBlocks * kFrag + (2 * wn + 1) * kFrag + lo);
    return f;
  };
  auto mfma4 = [&](const Frags& f, int set) {
    if constexpr (kAlgo == 8) {
      // The cubic's 256 accumulator registers fit the AGPR file: compiler
      // builtins (with the compiler's own hazard handling).
      acc[set][0][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a0, f.b0, acc[set][0][0], 0, 0, 0);
      acc[set][0][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a0, f.b1, acc[set][0][1], 0, 0, 0);
      acc[set][1][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a1, f.b0, acc[set][1][0], 0, 0, 0);
      acc[set][1][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a1, f.b1, acc[set][1][1], 0, 0, 0);
      return;
    }
    // Strassen: accumulator sets 0-3 live in AGPRs and 4-6 in VGPRs (pinned
    // through the operand constraint), so 448 accumulator registers never
    // move between the two files.
    if (set < 4) {
      mfma_agpr(acc[set][0][0], f.a0, f.b0);
      mfma_agpr(acc[set][0][1], f.a0, f.b1);
      mfma_agpr(acc[set][1][0], f.a1, f.b0);
      mfma_agpr(acc[set][1][1], f.a1, f.b1);
    } else {
      mfma_vgpr(acc[set][0][0], f.a0, f.b0);
      mfma_vgpr(acc[set][0][1], f.a0, f.b1);
      mfma_vgpr(acc[set][1][0], f.a1, f.b0);
      mfma_vgpr(acc[set][1][1], f.a1, f.b1);
    }
  };
  // Products (Strassen, issue order P4 P6 P5 P2 P7 P3 P1,
  // strassen_pallas.py:556-565) or quadrant pairs (cubic, a0b0 a0b1 a2b0
  // a2b1 a1b2 a1b3 a3b2 a3b3, benchmark_cubic_control.py:96-106), each as
  // (A operand, B operand, accumulator set). The next step's fragments load
  // while the current step's MFMAs run.
  constexpr int kSteps = kAlgo == 7 ? 7 : 8;
  constexpr int kStepA[8] = {kAlgo == 7 ? 3 : 0, kAlgo == 7 ? 5 : 0, kAlgo == 7 ? 4 : 2, kAlgo == 7 ? 1 : 2,
                             kAlgo == 7 ? 6 : 1, kAlgo == 7 ? 2 : 1, kAlgo == 7 ? 0 : 3, 3};
  constexpr int kStepB[8] = {kAlgo == 7 ? 3 : 0, kAlgo == 7 ? 5 : 1, kAlgo == 7 ? 4 : 0, kAlgo == 7 ? 1 : 1,
                             kAlgo == 7 ? 6 : 2, kAlgo == 7 ? 2 : 3, kAlgo == 7 ? 0 : 2, 3};
  constexpr int kStepAcc[8] = {kAlgo == 7 ? 3 : 0, kAlgo == 7 ? 5 : 1, kAlgo == 7 ? 4 : 2, kAlgo == 7 ? 1 : 3,
                               kAlgo == 7 ? 6 : 0, kAlgo == 7 ? 2 : 1, kAlgo == 7 ? 0 : 2, 3};
  auto mma = [&](const uint8_t* sa, const uint8_t* sb) {
    Frags cur = load_frags(sa, sb, kStepA[0], kStepB[0]);
#pragma unroll
    for (int x = 0; x < kSteps; ++x) {
      Frags next;
      if (x + 1 < kSteps) next = load_frags(sa, sb, kStepA[x + 1], kStepB[x + 1]);
      mfma4(cur, kStepAcc[x]);
      __builtin_amdgcn_sched_barrier(0);
      if (x + 1 < kSteps) cur = next;
    }
  };

  auto stage_buf = [&](int s) { return lds + (s & 1) * L::kStage; };

  // Prologue: stage 0 into buffer 0, stage 1 (or stage 0 again when there is
  // one stage) loads in flight.
  dma_b(stage_buf(0) + L::kA);
  load_a();
  advance();
  store_a(stage_buf(0));
  dma_b(stage_buf(1) + L::kA);
  load_a();
  advance();
  lds_barrier();

  // Compute stage s from buffer s%2 while stage s+1 (loaded during stage
  // s-1) is written into the other buffer, then start loading stage s+2 into
  // the buffer just consumed. Past the end the writes and loads are redundant
  // but in bounds (the last stage again) and never read.
  // The host guarantees nstages >= 1; a do-while leaves no zero-trip path
  // whose register assignment would have to be reconciled with copies.
  int s = 0;
  do {
    uint8_t* cur = stage_buf(s);
    mma(cur, cur + L::kA);
    store_a(stage_buf(s + 1));
    lds_barrier();
    dma_b(cur + L::kA);
    load_a();
    advance();
  } while (++s < nstages);

  // Both algorithms: the drain also pins every accumulator in its register
  // file up to this point, so the allocator cannot copy them out early.
  mfma_drain(acc);
  epilogue<kAlgo, 2, 2, kEpi>(p, o, wm * 64, wn * 64, acc);
}

}  // namespace v2
}  // namespace smx
