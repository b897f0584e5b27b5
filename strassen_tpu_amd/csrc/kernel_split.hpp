// Product-split Strassen kernel: the packed kernel's operands, DMA ring and
// stage pipeline, with the seven products divided among the waves instead
// of the output.
//
// The 128x128 product-space workgroup tile holds 7 products x 4 block rows
// = 28 strips of 32x128 (one product, one 32-row block row, all four
// 32-column blocks). Wave w owns strips 7w .. 7w+6 in (product, row) order,
// so it accumulates 28 32x32 blocks (448 registers, as in gemm_packed) but
// reads each A fragment once and each product's four B fragments once per
// stage: 7 + 4 x (products touched) fragments for 28 MFMAs, against 28 for
// 28 when every wave owns a 64x64 region of all seven products. Per stage
// the workgroup reads 68 KB of LDS instead of 112 KB (0.61 KB per MFMA
// instead of 1.0), while the DMA writes are unchanged.
//
// Stage ring (all 160 KB of LDS): B holds three stages of its seven
// operands (prefetched two stages ahead); A holds three stages of operands
// 0-4 and two of operands 5-6 (refilled right after the barrier that frees
// their slot, one stage and a strip ahead). A full three-
// stage ring of both (168 KB) does not fit; of the splits that do, this one
// measured fastest (the weight operand B, streamed from HBM, needs the
// distance most).
//
// After the last stage the waves exchange accumulator blocks through LDS so
// that wave (wm, wn) holds all seven products of its 64x64 region, the
// layout gemm_packed ends with; the shared epilogue then combines and
// stores them.
#pragma once

#include "kernel_packed.hpp"

namespace smx {
namespace split {

using packed::kBlocks;
using packed::kFrag;
using packed::TK;

// Strip plan of wave kWave. Forced inline: a call would return its value in
// a VGPR, which the compiler must treat as divergent, and the strip schedule
// would turn into exec-masked branches inside the main loop.
template <int kWave>
struct Plan {
  static constexpr int kFirst = 7 * kWave;
  __device__ __forceinline__ static constexpr int product(int j) { return (kFirst + j) / 4; }
  __device__ __forceinline__ static constexpr int row(int j) { return (kFirst + j) % 4; }
  // Whether strip j starts a product (its B fragments must be read).
  __device__ __forceinline__ static constexpr bool opens(int j) { return j == 0 || product(j) != product(j - 1); }
  // The strip of product q and block row r, or -1 if another wave owns it.
  __device__ __forceinline__ static constexpr int strip_of(int q, int r) {
    for (int j = 0; j < 7; ++j)
      if (product(j) == q && row(j) == r) return j;
    return -1;
  }
};

// Accumulators of strips 0-3 live in AGPRs, strips 4-6 in VGPRs.
__device__ __forceinline__ void drain(f32x16 (&acc)[7][4]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
  for (int j = 0; j < 7; ++j)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (j < 4)
        asm volatile("" : "+a"(acc[j][c]));
      else
        asm volatile("" : "+v"(acc[j][c]));
    }
}

struct StripFrags {
  bf16x8 a;
  bf16x8 b[4];
};

// LDS layout of the stage ring. A operand x < kLongOps of stage s sits in
// slot s % 3 of the long region, operand x >= kLongOps in slot s % 2 of the
// short region; B stage s in slot s % 3. Each wave moves fragment (op x,
// row block = wave) of every operand, i.e. 7 DMAs per operand and stage.
struct Ring {
  using L = packed::Lay<7>;
  static constexpr int kLongOps = 5;
  static constexpr int kShortOps = 7 - kLongOps;
  static constexpr int kALong = kLongOps * kBlocks * kFrag;    // one A stage, operands 0-4
  static constexpr int kAShort = kShortOps * kBlocks * kFrag;  // one A stage, operands 5-6
  static constexpr int kAShortBase = 3 * kALong;
  static constexpr int kBBase = kAShortBase + 2 * kAShort;
  static constexpr int kBytes = kBBase + 3 * L::kStage;
  // Each wave issues, in this order: right after the barrier that ends
  // stage s-1, A operands 5-6 of stage s+1 (into the short slot stage s-1
  // used); during stage s, A operands 0-4 and B of stage s+2. At the barrier
  // that ends stage s only the last two groups may still be in flight
  // (vmcnt completes in order).
  static constexpr int kLoopDma = kLongOps + 7;
  static constexpr int kPending = kLongOps + 7;
  static_assert(kBytes <= 160 * 1024, "stage ring exceeds the LDS");
  static_assert(kPending < 64, "vmcnt range");
};

// One wave's main loop, accumulator exchange and epilogue.
template <int kWave, int kEpi, int kQuad, bool kThin>
__device__ __forceinline__ void run_wave(const Params& p, const TileOrigin& o, int nstages,
                                         __amdgpu_buffer_rsrc_t a_src, __amdgpu_buffer_rsrc_t b_src, uint8_t* lds) {
  using L = packed::Lay<7>;
  using P = Plan<kWave>;
  uint8_t* const a_long = lds;
  uint8_t* const a_short = lds + Ring::kAShortBase;
  uint8_t* const b_region = lds + Ring::kBBase;
  // The lane's byte offset is derived here, inside the wave's own code path:
  // a value computed before the switch over waves would stay live through
  // every other wave's path (the branches are laid out one after another)
  // and spill there.
  const uint32_t lane_off = opaque_lane_id() * 16;
  const int lo = (int)lane_off;
  // Operand and slot choices depend only on the strip (a compile-time
  // constant after unrolling), so each read is one LDS load from a slot base.
  auto load_a = [&](const uint8_t* sl, const uint8_t* ss, int j) {
    constexpr int kL = Ring::kLongOps;
    return P::product(j) < kL ? packed::ld_frag(sl + (P::product(j) * kBlocks + P::row(j)) * kFrag + lo)
                              : packed::ld_frag(ss + ((P::product(j) - kL) * kBlocks + P::row(j)) * kFrag + lo);
  };
  auto load_b = [&](const uint8_t* sb, int j, bf16x8 (&b)[4]) {
#pragma unroll
    for (int c = 0; c < 4; ++c) b[c] = packed::ld_frag(sb + (P::product(j) * kBlocks + c) * kFrag + lo);
  };

  f32x16 acc[7][4];
#pragma unroll
  for (int j = 0; j < 7; ++j)
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][c][r] = 0.0f;
  auto mfma_strip = [&](int j, const bf16x8& a, const bf16x8 (&b)[4]) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (j < 4)
        packed::mfma_agpr(acc[j][c], a, b[c]);
      else
        packed::mfma_vgpr(acc[j][c], a, b[c]);
    }
  };
  // The same with hook(c) after MFMA c between scheduling barriers: the
  // stage's DMAs go out one at a time in the MFMAs' shadow.
  auto mfma_strip_dma = [&](int j, const bf16x8& a, const bf16x8 (&b)[4], auto hook) __attribute__((always_inline)) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (j < 4)
        packed::mfma_agpr(acc[j][c], a, b[c]);
      else
        packed::mfma_vgpr(acc[j][c], a, b[c]);
      __builtin_amdgcn_sched_barrier(0);
      hook(c);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Stage s: the 12 long-distance prefetch DMAs spread over strips 0-5 (two
  // per strip, after its second and fourth MFMA), with the next strip's
  // fragments read under the current strip's MFMAs; barrier; the
  // short-distance A prefetch of stage s+2; the next stage's strip-0
  // fragments read under strip 6's MFMAs. The barrier sees every read of
  // stage s complete and every wave's DMA of stage s+1 landed. Issuing the
  // short-distance prefetch right after the barrier, instead of with the
  // others, gave 0.7%. A DMA issued between two MFMAs, rather than two in a
  // row after a strip, keeps the wave from stalling the MFMA pipe on the
  // second DMA's issue (1.5% on the gate|up launch).
  int s = 0, l_slot = 0, s_slot = 0;
  bf16x8 a_cur = load_a(a_long, a_short, 0);
  bf16x8 b_cur[4];
  load_b(b_region, 0, b_cur);
  do {
    // Long slots: the one read at stage s-1 is refilled with stage s+2.
    const int l_fill = l_slot == 0 ? 2 : l_slot - 1, l_next = l_slot == 2 ? 0 : l_slot + 1;
    const int s_next = s_slot ^ 1;
    // The lane offset is re-derived opaquely each stage: otherwise the
    // compiler hoists (operand base + lane offset) out of the loop as 64-bit
    // per-lane addresses held across it, where the VGPRs next to the
    // accumulators cannot afford them; this way the loads take a uniform
    // base plus a 32-bit lane offset.
    uint32_t dma_lane = lane_off;
    asm volatile("" : "+v"(dma_lane));
    const uint32_t far = (uint32_t)min(s + 2, nstages - 1) * L::kStage;
    uint8_t* const al_to = a_long + l_fill * Ring::kALong + kWave * kFrag;
    uint8_t* const b_to = b_region + l_fill * L::kStage + kWave * kFrag;
    // q < 5: A operand q; q >= 5: B operand q - 5
    auto dma_op = [&](int q) {
      constexpr int kL = Ring::kLongOps;
      if (q < kL)
        packed::dma_frag(a_src, dma_lane, far + q * 4 * kFrag, al_to + q * 4 * kFrag);
      else
        packed::dma_frag(b_src, dma_lane, far + (q - kL) * 4 * kFrag, b_to + (q - kL) * 4 * kFrag);
    };
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t* const sal = a_long + l_slot * Ring::kALong;
    const uint8_t* const sas = a_short + s_slot * Ring::kAShort;
    const uint8_t* const sb = b_region + l_slot * L::kStage;
#pragma unroll
    for (int j = 0; j < 6; ++j) {
      const bf16x8 a_next = load_a(sal, sas, j + 1);
      static_assert(Ring::kLoopDma == 2 * 6, "two DMAs per strip");
      auto hook = [&](int c) __attribute__((always_inline)) {
        if (c == 1) dma_op(2 * j);
        if (c == 3) dma_op(2 * j + 1);
      };
      if (P::opens(j + 1)) {
        bf16x8 b_next_frags[4];
        load_b(sb, j + 1, b_next_frags);
        mfma_strip_dma(j, a_cur, b_cur, hook);
#pragma unroll
        for (int c = 0; c < 4; ++c) b_cur[c] = b_next_frags[c];
      } else {
        mfma_strip_dma(j, a_cur, b_cur, hook);
      }
      __builtin_amdgcn_sched_barrier(0);
      a_cur = a_next;
    }
    packed::stage_barrier<Ring::kPending>();
    {
      // A operands 5-6 of stage s+2 into the short slot stage s used.
      const uint32_t near = (uint32_t)min(s + 2, nstages - 1) * L::kStage;
      uint8_t* const as_to = a_short + s_slot * Ring::kAShort + kWave * kFrag;
#pragma unroll
      for (int q = 0; q < Ring::kShortOps; ++q)
        packed::dma_frag(a_src, dma_lane, near + (Ring::kLongOps + q) * 4 * kFrag, as_to + q * 4 * kFrag);
    }
    // Stage s+1's strip 0 (past the last stage: a re-loaded copy, unused).
    const bf16x8 a_first = load_a(a_long + l_next * Ring::kALong, a_short + s_next * Ring::kAShort, 0);
    bf16x8 b_first[4];
    load_b(b_region + l_next * L::kStage, 0, b_first);
    mfma_strip(6, a_cur, b_cur);
    __builtin_amdgcn_sched_barrier(0);
    a_cur = a_first;
#pragma unroll
    for (int c = 0; c < 4; ++c) b_cur[c] = b_first[c];
    l_slot = l_next;
    s_slot = s_next;
  } while (++s < nstages);
  drain(acc);

  // Every wave's DMAs (including the unread prefetches past the last stage)
  // have landed and every wave is past its last LDS read of the ring before
  // the exchange reuses it.
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");

  // Exchange, four rounds: in round t = 2i + jj every wave receives the
  // blocks (i, jj) of its 64x64 region for all seven products, i.e. strip
  // rows r with r % 2 == i and columns c with c % 2 == jj. Slot (dest wave,
  // product) is one 32x32 FP32 block stored as [4 register groups][64
  // lanes][4 floats]: source and destination share the MFMA accumulator
  // lane layout, so a block moves register for register.
  //
  // Each round's block goes through the epilogue as soon as it arrives (the
  // q/k epilogue, whose heads span 64 columns, takes the blocks (i, 0) and
  // (i, 1) together), so the products of a finished block are dead before
  // the next round: holding all seven products of the whole 64x64 region
  // through the epilogue needed more than the register file and spilled.
  //
  // Epilogues other than q/k stage their output in a tile of their own past
  // the receive slots, so a wave sends the next round's blocks as soon as
  // every wave has read the current round's, and that send overlaps the
  // current block's epilogue. The q/k epilogue's two staging tiles per wave
  // do not fit beside the slots: it stages in the wave's own receive slots,
  // which are free from the moment their blocks are read until the barrier
  // that ends the round (no wave writes them before it).
  constexpr int kBlockBytes = 64 * 16 * 4;
  constexpr int kSlotBytes = 4 * 7 * kBlockBytes;
  constexpr bool kPairs = kEpi == SMX_EPI_QK_NORM_ROPE;
  constexpr int kStageBytes = kEpiTiles<kEpi> * StageTile<32, kPairs ? 64 : 32>::kBytes;
  static_assert(!kPairs || kStageBytes <= 7 * kBlockBytes, "q/k staging fits the wave's receive slots");
  static_assert(kPairs || kSlotBytes + 4 * kStageBytes <= Ring::kBytes, "staging fits past the receive slots");
  const int wm = kWave >> 1, wn = kWave & 1;
  uint8_t* const mine = lds + kWave * 7 * kBlockBytes;
  // The rounds are spelled out with compile-time indices: a loop the
  // compiler declines to unroll (its body holds the inlined epilogue) would
  // index the block arrays at run time and move them to scratch.
  //
  // Round t's blocks of this wave's strips into their destination slots;
  // outside q/k, a block this wave receives itself stays in its registers
  // (receive). The q/k kernels, whose epilogue holds two blocks' quadrant
  // sets, spill when those registers stay live, so they move every block.
  constexpr bool kKeepOwn = !kPairs;
  auto send = [&](auto tc) __attribute__((always_inline)) {
    constexpr int t = decltype(tc)::value, i = t >> 1, jj = t & 1;
    // the lane's byte offset, re-derived opaquely each round so that no copy
    // of it stays live through the epilogues
    const uint32_t lane16 = opaque_lane_id() * 16;
#pragma unroll
    for (int j = 0; j < 7; ++j) {
      const int r = P::row(j);
      if (r % 2 != i) continue;
#pragma unroll
      for (int c = jj; c < 4; c += 2) {
        const int dest = 2 * (r / 2) + c / 2;
        if (kKeepOwn && dest == kWave) continue;
        uint8_t* const slot = lds + (dest * 7 + P::product(j)) * kBlockBytes + lane16;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          f32x4 v = {acc[j][c][4 * g], acc[j][c][4 * g + 1], acc[j][c][4 * g + 2], acc[j][c][4 * g + 3]};
          *reinterpret_cast<f32x4*>(slot + g * 1024) = v;
        }
      }
    }
  };
  // The seven products of round t's block: from this wave's own strips where
  // it owns them, else from its slots.
  auto receive = [&](auto tc, f32x16 (&blk)[7][1][1]) __attribute__((always_inline)) {
    constexpr int t = decltype(tc)::value, i = t >> 1, jj = t & 1;
    const uint32_t lane16 = opaque_lane_id() * 16;
#pragma unroll
    for (int q = 0; q < 7; ++q) {
      if constexpr (kKeepOwn) {
        const int own = P::strip_of(q, 2 * (kWave >> 1) + i);
        if (own >= 0) {
#pragma unroll
          for (int e = 0; e < 16; ++e) blk[q][0][0][e] = acc[own][2 * (kWave & 1) + jj][e];
          continue;
        }
      }
      const uint8_t* const slot = mine + q * kBlockBytes + lane16;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(slot + g * 1024);
#pragma unroll
        for (int e = 0; e < 4; ++e) blk[q][0][0][4 * g + e] = v[e];
      }
    }
  };
  if constexpr (kPairs) {
    // q/k: the four quadrant sets of block (i, 0), formed on arrival, wait
    // for block (i, 1).
    f32x16 quads[4][1][2];
    auto round = [&](auto tc) __attribute__((always_inline)) {
      constexpr int t = decltype(tc)::value, i = t >> 1, jj = t & 1;
      send(tc);
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      f32x16 blk[7][1][1];
      receive(tc, blk);
      // the block's reads complete before its slots turn into staging tiles
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        quads[0][0][jj][r] = quadrant_value<kQuad, 0>(blk, 0, 0, r);
        quads[1][0][jj][r] = quadrant_value<kQuad, 1>(blk, 0, 0, r);
        quads[2][0][jj][r] = quadrant_value<kQuad, 2>(blk, 0, 0, r);
        quads[3][0][jj][r] = quadrant_value<kQuad, 3>(blk, 0, 0, r);
      }
      // the quadrant sets go through the epilogue as the cubic's would
      if constexpr (jj == 1)
        epilogue_body<1, 2, kEpi, 4, kQuadCubic, kThin>(p, o, wm * 64 + i * 32, wn * 64, quads, mine);
      // every staging access has completed before the next round's blocks
      // land in these slots
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    round(QuadC<0>{});
    round(QuadC<1>{});
    round(QuadC<2>{});
    round(QuadC<3>{});
  } else {
    uint8_t* const stage = lds + kSlotBytes + kWave * kStageBytes;
    // Round t: receive; once every wave has read its slots, send round
    // t + 1 and run round t's epilogue; the barrier after both makes round
    // t + 1's blocks visible.
    auto step = [&](auto tc) __attribute__((always_inline)) {
      constexpr int t = decltype(tc)::value, i = t >> 1, jj = t & 1;
      f32x16 blk[7][1][1];
      receive(tc, blk);
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      if constexpr (t < 3) send(QuadC<t + 1>{});
      epilogue_body<1, 1, kEpi, 7, kQuad, kThin>(p, o, wm * 64 + i * 32, wn * 64 + jj * 32, blk, stage);
      if constexpr (t < 3) asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    send(QuadC<0>{});
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    step(QuadC<0>{});
    step(QuadC<1>{});
    step(QuadC<2>{});
    step(QuadC<3>{});
  }
}

// kThin: a tiling whose bm/2 is not a multiple of 128 (ThinRows).
template <int kEpi, int kQuad, bool kThin = false>
__global__ __launch_bounds__(kThreads, 1) void gemm_split(Params p) {
  using L = packed::Lay<7>;
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int nstages_all = (int)(p.k / (2 * TK));
  const WorkShare ws = work_share(p, nstages_all);
  int tile_m, tile_n;
  tile_of(ws.tile, p.tiles_m, p.tiles_n, p.group_m, p.raster, tile_m, tile_n);
  // The tile indices are uniform, but the integer divisions that produce
  // them run on VALU; readfirstlane moves them (and every operand address
  // derived from them) to SGPRs, which keeps VGPRs for the accumulators.
  tile_m = __builtin_amdgcn_readfirstlane(tile_m);
  tile_n = __builtin_amdgcn_readfirstlane(tile_n);
  TileOrigin o = tile_origin<kThin>(p, (int64_t)tile_m * packed::TM, (int64_t)tile_n * packed::TN);
  // K-split shares run without an epilogue and store dense FP32 blocks.
  if constexpr (kEpi == SMX_EPI_NONE)
    if (p.ksplit > 1) dense_share_output(p, o, ws, (int64_t)tile_m * packed::TM);
  const int nstages = ws.nstages;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t panel_bytes = (uint32_t)nstages * L::kStage - wave * kFrag;
  const __amdgpu_buffer_rsrc_t a_src = packed::panel_rsrc(
      reinterpret_cast<const uint8_t*>(p.a) + ((int64_t)tile_m * nstages_all + ws.stage0) * L::kStage + wave * kFrag,
      panel_bytes);
  const __amdgpu_buffer_rsrc_t b_src = packed::panel_rsrc(
      reinterpret_cast<const uint8_t*>(p.b) + ((int64_t)tile_n * nstages_all + ws.stage0) * L::kStage + wave * kFrag,
      panel_bytes);

  // Prologue: stage 0 of everything, then stage 1 of A's long operands, of
  // B and of A's short operands (the loop's order); stage 0 has landed once
  // only stage 1 remains in flight.
  const uint32_t lane_off = lane * 16;
  auto dma = [&](__amdgpu_buffer_rsrc_t src, int stage, int x0, int x1, uint8_t* slot) {
    const uint32_t from = (uint32_t)min(stage, nstages - 1) * L::kStage;
#pragma unroll
    for (int x = x0; x < x1; ++x)
      packed::dma_frag(src, lane_off, from + x * 4 * kFrag, slot + (wave + 4 * (x - x0)) * kFrag);
  };
  uint8_t* const b_region = lds + Ring::kBBase;
  dma(a_src, 0, Ring::kLongOps, 7, lds + Ring::kAShortBase);
  dma(a_src, 0, 0, Ring::kLongOps, lds);
  dma(b_src, 0, 0, 7, b_region);
  dma(a_src, 1, 0, Ring::kLongOps, lds + Ring::kALong);
  dma(b_src, 1, 0, 7, b_region + L::kStage);
  dma(a_src, 1, Ring::kLongOps, 7, lds + Ring::kAShortBase + Ring::kAShort);
  packed::stage_barrier<Ring::kPending + Ring::kShortOps>();

  // One code path per wave (its strip plan is a compile-time constant); no
  // accumulator is live across the branches.
  switch (wave) {
    case 0:
      run_wave<0, kEpi, kQuad, kThin>(p, o, nstages, a_src, b_src, lds);
      break;
    case 1:
      run_wave<1, kEpi, kQuad, kThin>(p, o, nstages, a_src, b_src, lds);
      break;
    case 2:
      run_wave<2, kEpi, kQuad, kThin>(p, o, nstages, a_src, b_src, lds);
      break;
    default:
      run_wave<3, kEpi, kQuad, kThin>(p, o, nstages, a_src, b_src, lds);
      break;
  }
}

}  // namespace split
}  // namespace smx
