// Product-major Strassen kernel (gfx950): the seven products of a
// 128 x 256 product-space tile run one after another, each over the whole K
// range, into three FP32 accumulator sets instead of seven.
//
// Why: gemm_split keeps the seven products of a 128 x 128 product tile in
// registers for the whole K loop (448 registers per lane), so each 1 KB
// operand fragment it streams from L2 into LDS feeds four MFMAs: 512 bytes
// per MFMA, twice the matched cubic's, which keeps the texture address unit
// (TA, 16 cycles per 64-lane 16-byte DMA) as busy as the MFMAs. Three sets
// of a 128 x 256 tile are 384 registers per lane, and each A fragment feeds
// 4 MFMAs, each B fragment 2: 384 bytes per MFMA.
//
// The products contribute to the four output quadrants as
//   C0 = P1 + P4 - P5 + P7,  C1 = P3 + P5,  C2 = P2 + P4,  C3 = P1 - P2 + P3 + P6
// (strassen_pallas.py:324-379). No VALU instruction touches an accumulator
// between two products: every combination comes from the MFMA itself, whose
// first instruction of a product may read its C operand from another set of
// the same register file (D = A B + C), and from two FP32 partial sets
// parked in global memory. Sets: V (VGPRs), A1 and A2 (AGPRs); parks q1, q3.
//   P5 -> V          park q1 = V = P5
//   P3 -> V (chain)  V = P3 + P5 = C1
//   P4 -> A1         A1 = P4
//   P1 -> A2 from A1 A2 = P1 + P4;   park q3 = A2 + V = P1 + P3 + P4 + P5
//   P7 -> A2 (chain) A2 = P1 + P4 + P7; row half 0: C0 = A2 - q1, C1 = V
//   P6 -> A2         A2 = P6
//   P2 -> A1 (chain) A1 = P2 + P4 = C2; row half 1: C2 = A1,
//                    C3 = q3 + A2 - q1 - A1 = P1 + P3 + P6 - P2
// V is dead after row half 0, so the second half's epilogue has the VGPRs
// for its parked blocks.
// Each row half's two quadrants (gate | up for SwiGLU / GeGLU) are complete
// together. The parks cost 256 KB written and 384 KB read per tile, against
// about 14 MB of operand fragments at the gate|up shape; each row half's
// epilogue reads its parked blocks two blocks ahead (kParkAhead).
//
// The packed operands are those of gemm_split (packed::Lay<7>): the tile
// reads packed A tile tile_m and packed B tiles 2 tile_n and 2 tile_n + 1,
// one operand (the current product's) per stage.
//
// Pipeline: a stage is 64 product-space k (four packed 16-k stages,
// "quarters") of one product, 16 KB of A and 32 KB of B; a ring of three
// stages is refilled two stages ahead, and the DMA stream runs on across
// product boundaries. One barrier per stage, before its last quarter's
// MFMAs: it sees the next stage landed and every wave done reading the
// stage, whose slot the refill then starts on. Per wave and stage: 24
// fragment reads, 32 MFMAs and 12 DMAs, three per quarter, each issued
// between two MFMAs (after the second, fifth and eighth of the quarter):
// DMAs issued back to back hold back the next MFMA's issue (4% on the
// gate|up launch).
//
// Waves: wave (wm, wn) owns product rows 64 wm .. + 63 and columns
// 128 wn .. + 127 of the tile, 2 x 4 blocks of 32 x 32 per set; per 16 k it
// reads 2 A and 4 B fragments for 8 MFMAs.
#pragma once

#include "kernel_packed.hpp"

namespace smx {
namespace pm {

using packed::kBlocks;
using packed::kFrag;

constexpr int TM = 128;  // product rows of a tile (one packed A tile)
constexpr int TN = 256;  // product columns (two packed B tiles)
constexpr int kOps = 7;
// One packed 16-k stage of one operand of one packed tile: 4 KB; of all
// seven operands: 28 KB.
constexpr int kOpStage = kBlocks * kFrag;
constexpr int kPackedStage = kOps * kOpStage;
// Pipeline stage: four packed 16-k stages ("quarters") of one product; a
// quarter holds A blocks 0-3, then B tile 0 blocks 0-3, then B tile 1
// blocks 0-3.
constexpr int kQuarters = 4;
constexpr int kQuarterBytes = 3 * kOpStage;            // 12 KB
constexpr int kStageBytes = kQuarters * kQuarterBytes;  // 48 KB
constexpr int kSlots = 3;
constexpr int kDist = kSlots - 1;  // refill distance in stages
constexpr int kDmaPerWave = kStageBytes / kFrag / 4;  // 12
// VMEM operations a wave may leave in flight at the barrier of stage g,
// which needs stage g + 1: the refill of stage g + 2.
constexpr int kPending = (kDist - 1) * kDmaPerWave;
constexpr int kRingBytes = kSlots * kStageBytes;
// Epilogue staging tile of a wave: 32 x 32 floats, rows unpadded (the ring
// leaves 16 KB of the LDS). Same interface as StageTile.
struct Tile {
  static constexpr int kRows = 32, kCols = 32;
  static constexpr int kStride = kCols * 4;
  static constexpr int kBytes = kRows * kStride;
  static constexpr int at(int i, int j, int r) { return (i * 32 + 8 * (r >> 2) + (r & 3)) * kStride + j * 128; }
  static __device__ __forceinline__ int lane_part(int lane) { return (lane >> 5) * 4 * kStride + (lane & 31) * 4; }
};
constexpr int kLds = kRingBytes + 4 * Tile::kBytes;
static_assert(kLds <= 160 * 1024, "LDS budget");
static_assert(kPending < 64, "vmcnt range");
// One parked set of one workgroup (FP32, 128 x 256), in the registers' lane
// order: [wave][block][4 register groups][64 lanes][4 floats]; a workgroup
// parks two.
constexpr int64_t kParkSet = (int64_t)TM * TN * 4;
constexpr int64_t kParkBytes = 2 * kParkSet;

// Product (0-based: P1 = 0) of phase ph, four bits per phase:
// P5 P3 P4 P1 P7 P6 P2.
constexpr uint32_t kOrder = 4u | 2u << 4 | 3u << 8 | 0u << 12 | 6u << 16 | 5u << 20 | 1u << 24;
__host__ __device__ constexpr int product_of(int ph) { return (int)((kOrder >> (4 * ph)) & 15u); }

typedef f32x16 Set[2][4];

struct Frags {
  bf16x8 a[2];
  bf16x8 b[4];
};

// File of a set's accumulators: V in VGPRs, A1 and A2 in AGPRs.
constexpr int kV = 0, kA1 = 1, kA2 = 2;
__host__ __device__ constexpr bool in_agprs(int set) { return set != kV; }

// The MFMAs of one 16-k half on a set's 2 x 4 blocks. kStart 0: chain
// (D = A B + D); 1: the product's first half from zero (D = A B); 2: its
// first half from set `from` of the same file (D = A B + from).
template <int kSet, int kStart>
__device__ __forceinline__ void mfma8(Set& acc, const Set& from, const Frags& f) {
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (kStart == 0) {
        if constexpr (in_agprs(kSet))
          packed::mfma_agpr(acc[i][j], f.a[i], f.b[j]);
        else
          packed::mfma_vgpr(acc[i][j], f.a[i], f.b[j]);
      } else if constexpr (kStart == 1) {
        if constexpr (in_agprs(kSet))
          asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&a"(acc[i][j]) : "v"(f.a[i]), "v"(f.b[j]));
        else
          asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(acc[i][j]) : "v"(f.a[i]), "v"(f.b[j]));
      } else {
        static_assert(in_agprs(kSet), "only the AGPR sets start from another set");
        asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %3"
            : "=&a"(acc[i][j])
            : "v"(f.a[i]), "v"(f.b[j]), "a"(from[i][j]));
      }
    }
}

// mfma8 with hook(k) after MFMA k (k = 0..7), each hook between scheduling
// barriers.
template <int kSet, int kStart, class Hook>
__device__ __forceinline__ void mfma8_dma(Set& acc, const Set& from, const Frags& f, Hook hook) {
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (kStart == 0) {
        if constexpr (in_agprs(kSet))
          packed::mfma_agpr(acc[i][j], f.a[i], f.b[j]);
        else
          packed::mfma_vgpr(acc[i][j], f.a[i], f.b[j]);
      } else if constexpr (kStart == 1) {
        if constexpr (in_agprs(kSet))
          asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&a"(acc[i][j]) : "v"(f.a[i]), "v"(f.b[j]));
        else
          asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(acc[i][j]) : "v"(f.a[i]), "v"(f.b[j]));
      } else {
        static_assert(in_agprs(kSet), "only the AGPR sets start from another set");
        asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %3"
            : "=&a"(acc[i][j])
            : "v"(f.a[i]), "v"(f.b[j]), "a"(from[i][j]));
      }
      __builtin_amdgcn_sched_barrier(0);
      hook(4 * i + j);
      __builtin_amdgcn_sched_barrier(0);
    }
}

// Wait states past the MFMA result latency, then every accumulator of the
// set is bound (volatile asm, in program order after the s_nops), so no
// read of it moves above them.
template <int kSet>
__device__ __forceinline__ void drain(Set& acc) {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (in_agprs(kSet))
        asm volatile("" : "+a"(acc[i][j]));
      else
        asm volatile("" : "+v"(acc[i][j]));
    }
  __builtin_amdgcn_sched_barrier(0);
}

// Parked sets go through a buffer resource over the workgroup's park
// region: a uniform base, the lane's 32-bit byte offset (derived where it is
// used, so no per-lane 64-bit address is held across the main loops) and a
// compile-time offset. Lane l of register group g of block (i, j) of set x
// of wave w sits at x kParkSet + w kParkSet / 4 + (4 (4 i + j) + g) KB + 16 l.
__device__ __forceinline__ uint32_t park_offset(int set, int wave, int i, int j, int g) {
  return (uint32_t)(set * kParkSet + wave * (kParkSet / 4) + ((4 * i + j) * 4 + g) * 1024);
}

// Stores x (plus y, when kAdd) as parked set kSetIdx.
template <int kSetIdx, bool kAdd>
__device__ __forceinline__ void park_store(__amdgpu_buffer_rsrc_t park, int wave, const Set& x, const Set& y) {
  const uint32_t lane16 = opaque_lane_id() * 16;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = kAdd ? x[i][j][4 * g + e] + y[i][j][4 * g + e] : x[i][j][4 * g + e];
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), park, lane16,
                                               park_offset(kSetIdx, wave, i, j, g), 0);
      }
}

// Block (i, j) of parked set kSetIdx.
template <int kSetIdx>
__device__ __forceinline__ f32x16 park_block(__amdgpu_buffer_rsrc_t park, int wave, uint32_t lane16, int i, int j) {
  f32x16 v;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const f32x4 x = __builtin_bit_cast(
        f32x4, __builtin_amdgcn_raw_buffer_load_b128(park, lane16, park_offset(kSetIdx, wave, i, j, g), 0));
#pragma unroll
    for (int e = 0; e < 4; ++e) v[4 * g + e] = x[e];
  }
  return v;
}

// Parked blocks are loaded this many blocks ahead of their use: the parks
// were written long before and come back from beyond the L2. Two ahead
// measured 0.7% faster than one on the gate|up site; three gained nothing
// more, and more spill.
constexpr int kParkAhead = 2;

// Epilogue of logical row half lr. quads(i, j, pk, left, right) yields
// the FP32 values of quadrants (lr, 0) and (lr, 1) of the wave's block
// (i, j), given block (i, j) of parked sets 0 .. kParks-1 (pk[0], pk[1]),
// loaded kParkAhead blocks ahead. One 32 x 32 block at a
// time passes through the wave's staging tile (strassen_pallas.py:739-792,
// :867-874): SwiGLU / GeGLU store gate(left) * right into [M, N/2];
// residual_add and bias_add (and no epilogue) store each quadrant. Logical
// quadrant (row, col) is stored at physical (row ^ swap_m, col ^ swap_n)
// for the block permutation (strassen_pallas.py:205-226).
template <int kEpi, int kParks, class Quads>
__device__ __forceinline__ void emit_half(const Params& p, const TileOrigin& o, int wave, int lr,
                                          __amdgpu_buffer_rsrc_t park, Quads quads, uint8_t* tile) {
  const int wm = wave >> 1, wn = wave & 1;
  using T = Tile;
  const int lane = opaque_lane_id();
  const int lcol = lane & 31;
  const int64_t hm = p.bm / 2, hn = p.bn / 2;
  const int swap_m = p.perm & 1, swap_n = (p.perm >> 2) & 1;
  const int64_t half = lr ^ swap_m;
  const int es = p.out_f32 ? 4 : 2;
  uint8_t* const te = tile + T::lane_part(lane);
  auto fence = []() __attribute__((always_inline)) { asm volatile("" ::: "memory"); };
  auto put = [&](int r, float v) __attribute__((always_inline)) {
    *reinterpret_cast<float*>(te + T::at(0, 0, r)) = v;
  };
  auto get = [&](int r) __attribute__((always_inline)) {
    return *reinterpret_cast<const float*>(te + T::at(0, 0, r));
  };
  const uint32_t lane16 = lane * 16;
  f32x16 pk[kParkAhead + 1][kParks];
  auto fetch = [&](f32x16 (&to)[kParks], int b) __attribute__((always_inline)) {
    to[0] = park_block<0>(park, wave, lane16, b >> 2, b & 3);
    if constexpr (kParks > 1) to[kParks - 1] = park_block<kParks - 1>(park, wave, lane16, b >> 2, b & 3);
  };
#pragma unroll
  for (int f = 0; f < kParkAhead; ++f) fetch(pk[f], f);
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    const int i = b >> 2, j = b & 3;
    if (b + kParkAhead < 8) fetch(pk[(b + kParkAhead) % (kParkAhead + 1)], b + kParkAhead);
    const int64_t row = o.ti * p.bm + o.tr + wm * 64 + i * 32 + half * hm;
    const int64_t cc = o.tc + wn * 128 + j * 32;  // column inside a column half
    f32x16 left, right;
    quads(i, j, pk[b % (kParkAhead + 1)], left, right);
    if constexpr (kEpi == SMX_EPI_SWIGLU || kEpi == SMX_EPI_GEGLU) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float gate = swap_n ? right[r] : left[r], up = swap_n ? left[r] : right[r];
        put(r, gate_f32<kEpi>(gate) * up);
      }
      fence();
      tile_store<T>(tile, reinterpret_cast<char*>(p.c) + (row * p.ldc + o.tj * hn + cc) * es, p.ldc, p.out_f32,
                    lane);
      fence();
    } else {
#pragma unroll
      for (int lc = 0; lc < 2; ++lc) {
        const int64_t col = o.tj * p.bn + cc + (lc ^ swap_n) * hn;
        if constexpr (kEpi == SMX_EPI_RESIDUAL_ADD) {
          const int res = p.residual_f32 ? 4 : 2;
          tile_load<T>(tile, reinterpret_cast<const char*>(p.residual) + (row * p.ldr + col) * res, p.ldr,
                       p.residual_f32, lane);
          fence();
        }
        float bv = 0.f;
        if constexpr (kEpi == SMX_EPI_BIAS_ADD) bv = load_vec(p.bias, p.bias_f32, col + lcol);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float v = lc ? right[r] : left[r];
          if constexpr (kEpi == SMX_EPI_RESIDUAL_ADD) v += get(r);
          if constexpr (kEpi == SMX_EPI_BIAS_ADD) v += bv;
          put(r, v);
        }
        fence();
        tile_store<T>(tile, reinterpret_cast<char*>(p.c) + (row * p.ldc + col) * es, p.ldc, p.out_f32, lane);
        fence();
      }
    }
  }
}

template <int kEpi>
__global__ __launch_bounds__(kThreads, 1) void gemm_pm(Params p) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  int tile_m, tile_n;
  tile_of((int)blockIdx.x, p.tiles_m, p.tiles_n, p.group_m, p.raster, tile_m, tile_n);
  tile_m = __builtin_amdgcn_readfirstlane(tile_m);
  tile_n = __builtin_amdgcn_readfirstlane(tile_n);
  const TileOrigin o = tile_origin<false>(p, (int64_t)tile_m * TM, (int64_t)tile_n * TN);

  // Packed 16-k stages over K, and pipeline stages per product (the host
  // takes K % 128 == 0).
  const int nst16 = (int)(p.k / 32);
  const int nstages = nst16 / kQuarters;
  // One packed tile's panel (all stages, all operands); B's second tile
  // follows its first.
  const uint32_t panel = (uint32_t)nst16 * kPackedStage;
  const __amdgpu_buffer_rsrc_t a_src = packed::panel_rsrc(
      reinterpret_cast<const uint8_t*>(p.a) + (int64_t)tile_m * panel + wave * kFrag, panel - wave * kFrag);
  const __amdgpu_buffer_rsrc_t b_src = packed::panel_rsrc(
      reinterpret_cast<const uint8_t*>(p.b) + (int64_t)(2 * tile_n) * panel + wave * kFrag, 2 * panel - wave * kFrag);
  // The workgroup's parked sets q1 and q3.
  const __amdgpu_buffer_rsrc_t park = packed::panel_rsrc(
      reinterpret_cast<const uint8_t*>(p.park) + (int64_t)blockIdx.x * kParkBytes, (uint32_t)kParkBytes);
  uint8_t* const tile = lds + kRingBytes + wave * Tile::kBytes;

  // DMA x of quarter q of stage (ph, s) into ring slot `slot`: wave w moves
  // block w of A (x = 0) and of each B tile (x = 1, 2). Stages past the
  // last one re-load it (in bounds, never read).
  auto dma_one = [&](int ph, int s, int q, int slot, uint32_t lane_off, int x) __attribute__((always_inline)) {
    if (ph >= kOps) {
      ph = kOps - 1;
      s = nstages - 1;
    }
    const uint32_t off = (uint32_t)((kQuarters * s + q) * kOps + product_of(ph)) * kOpStage;
    uint8_t* const to = lds + slot * kStageBytes + q * kQuarterBytes + wave * kFrag;
    if (x == 0) packed::dma_frag(a_src, lane_off, off, to);
    if (x == 1) packed::dma_frag(b_src, lane_off, off, to + kOpStage);
    if (x == 2) packed::dma_frag(b_src, lane_off, off + panel, to + 2 * kOpStage);
  };
  auto dma_quarter = [&](int ph, int s, int q, int slot, uint32_t lane_off) __attribute__((always_inline)) {
#pragma unroll
    for (int x = 0; x < 3; ++x) dma_one(ph, s, q, slot, lane_off, x);
  };
  // Hook for mfma8_dma: the three DMAs of quarter q after MFMAs 1, 4 and 7.
  auto dma_hook = [&](int ph, int s, int q, int slot, uint32_t lane_off) __attribute__((always_inline)) {
    return [=, &dma_one](int k) __attribute__((always_inline)) {
      if (k == 1) dma_one(ph, s, q, slot, lane_off, 0);
      if (k == 4) dma_one(ph, s, q, slot, lane_off, 1);
      if (k == 7) dma_one(ph, s, q, slot, lane_off, 2);
    };
  };
  auto load = [&](int slot, int q) __attribute__((always_inline)) {
    const int lo = opaque_lane_id() * 16;
    const uint8_t* const base = lds + slot * kStageBytes + q * kQuarterBytes + lo;
    Frags f;
#pragma unroll
    for (int i = 0; i < 2; ++i) f.a[i] = packed::ld_frag(base + (2 * wm + i) * kFrag);
#pragma unroll
    for (int j = 0; j < 4; ++j) f.b[j] = packed::ld_frag(base + (4 + 4 * wn + j) * kFrag);
    return f;
  };

  // Prologue: stages 0 .. kDist-1 of the stream, and quarter 0 of stage
  // kDist (the stage loop refills quarters 1-3 of the slot it reads, and
  // quarter 0 of the next refill after its barrier).
  int dph = kDist / nstages, ds = kDist % nstages;
  {
    const uint32_t lane_off = opaque_lane_id() * 16;
#pragma unroll
    for (int st = 0; st < kDist; ++st)
#pragma unroll
      for (int q = 0; q < kQuarters; ++q) dma_quarter(st / nstages, st % nstages, q, st, lane_off);
    dma_quarter(dph, ds, 0, kDist, lane_off);
  }
  packed::stage_barrier<kPending + 3>();

  Set V, A1, A2;
  int slot = 0;
  Frags cur = load(0, 0);

  // One pipeline stage: each quarter's fragments read under the previous
  // quarter's MFMAs; quarters 1-3 of the refill of the slot read at the
  // previous stage under the first three quarters' MFMAs; the barrier; then
  // the next stage's first quarter read, and quarter 0 of the refill of the
  // slot this stage read, under the last quarter's MFMAs. Every wave has
  // read all of that slot by the barrier (its quarter 0 before the previous
  // one), and at the barrier a wave leaves only the current refill's 12
  // DMAs in flight, so the previous refill (the next stage) has landed.
  // kStart applies to the first quarter (the product's first stage).
  auto stage = [&](auto setc, auto startc, Set& acc, const Set& from) __attribute__((always_inline)) {
    constexpr int kSet = decltype(setc)::value, kStart = decltype(startc)::value;
    const int next = slot == kSlots - 1 ? 0 : slot + 1;
    const int fill = slot == 0 ? kSlots - 1 : slot - 1;
    const uint32_t lane_off = opaque_lane_id() * 16;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < kQuarters - 1; ++q) {
      const Frags nxt = load(slot, q + 1);
      __builtin_amdgcn_sched_barrier(0);
      if (q == 0)
        mfma8_dma<kSet, kStart>(acc, from, cur, dma_hook(dph, ds, q + 1, fill, lane_off));
      else
        mfma8_dma<kSet, 0>(acc, from, cur, dma_hook(dph, ds, q + 1, fill, lane_off));
      __builtin_amdgcn_sched_barrier(0);
      cur = nxt;
    }
    if (++ds == nstages) {
      ds = 0;
      ++dph;
    }
    packed::stage_barrier<kPending>();
    const Frags h0 = load(next, 0);  // past the last stage: a re-loaded copy, unused
    __builtin_amdgcn_sched_barrier(0);
    mfma8_dma<kSet, 0>(acc, from, cur, dma_hook(dph, ds, 0, slot, lane_off));
    __builtin_amdgcn_sched_barrier(0);
    cur = h0;
    slot = next;
  };
  // One product over all stages into set kSet, its first stage started as
  // kStart says.
  auto run = [&](auto setc, auto startc, Set& acc, const Set& from) __attribute__((always_inline)) {
    stage(setc, startc, acc, from);
    for (int s = 1; s < nstages; ++s) stage(setc, QuadC<0>{}, acc, from);
  };
  using SV = QuadC<kV>;
  using SA1 = QuadC<kA1>;
  using SA2 = QuadC<kA2>;
  using Zero = QuadC<1>;
  using From = QuadC<2>;
  using Chain = QuadC<0>;

  // P5 -> V, parked as q1.
  run(SV{}, Zero{}, V, V);
  drain<kV>(V);
  park_store<0, false>(park, wave, V, V);
  // The parked stores leave the VMEM count before the next barrier counts
  // refills again.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  // P3 chained into V: V = C1.
  run(SV{}, Chain{}, V, V);
  drain<kV>(V);
  // P4 -> A1.
  run(SA1{}, Zero{}, A1, A1);
  // P1 -> A2 from A1: A2 = P1 + P4; q3 = A2 + V parked.
  run(SA2{}, From{}, A2, A1);
  drain<kA2>(A2);
  park_store<1, true>(park, wave, A2, V);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  // P7 chained into A2: row half 0, C0 = A2 - q1, C1 = V.
  run(SA2{}, Chain{}, A2, A2);
  drain<kA2>(A2);
  emit_half<kEpi, 1>(p, o, wave, 0, park, [&](int i, int j, const f32x16 (&pk)[1], f32x16& left, f32x16& right)
                                              __attribute__((always_inline)) {
    left = A2[i][j] - pk[0];
    right = V[i][j];
  }, tile);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  // P6 -> A2.
  run(SA2{}, Zero{}, A2, A2);
  // P2 chained into A1: row half 1, C2 = A1, C3 = q3 + A2 - q1 - A1.
  run(SA1{}, Chain{}, A1, A1);
  drain<kA1>(A1);
  drain<kA2>(A2);
  emit_half<kEpi, 2>(p, o, wave, 1, park, [&](int i, int j, const f32x16 (&pk)[2], f32x16& left, f32x16& right)
                                              __attribute__((always_inline)) {
    left = A1[i][j];
    right = ((pk[1] + A2[i][j]) - pk[0]) - A1[i][j];
  }, tile);
  // Every wave's DMA (the unread re-loads past the last stage) has landed
  // before the workgroup ends.
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
}

}  // namespace pm
}  // namespace smx
