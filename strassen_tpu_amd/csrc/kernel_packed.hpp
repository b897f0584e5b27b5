// Packed-operand gfx950 kernel: 128x128 product-space workgroup tile, four
// waves of 64x64, 16 product-space k per stage, both operands streamed from
// HBM straight into LDS (buffer_load_dwordx4 ... lds, no VGPR staging, no
// VALU in the main loop).
//
// Packed operand layout (written by pack_operand below, once per weight and
// once per call for the activation). An operand of R product rows (M/2 for
// A, N/2 for B) and K/2 product-space depth is stored as
//   [R/128 tiles][K/32 stages][nops][4 blocks of 32 rows][64 lanes][8 bf16]
// where lane l of a 1 KB fragment holds row l%32, depth 8*(l/32)..+8 of the
// 32x16 MFMA operand, i.e. exactly the order a lane's ds_read_b128 wants.
// nops is 7 for Strassen (the operand sums of P1..P7, each rounded once to
// bf16, strassen_pallas.py:324-379) and 4 for the cubic (raw quadrants). One
// stage of one operand for one workgroup is therefore nops*4 KB contiguous,
// and every DMA instruction moves one contiguous 1 KB fragment.
//
// Pipeline: a ring of kASlots A stages and three B stages in LDS. At stage s
// a wave issues the DMA of A stage s+kASlots-1 and B stage s+2, runs its
// MFMAs on stage s and meets the other waves at one barrier that waits for
// everything but the newest prefetches.
#pragma once

#include "common.hpp"

namespace smx {
namespace packed {

constexpr int TM = 128, TN = 128, TK = 16;
// K granule of the packed kernel: bk % (2 * kKGranule) == 0 keeps the stage
// count (K/32) even.
constexpr int kKGranule = 2 * TK;
constexpr int kFrag = 1024;  // one 32x16 bf16 operand fragment in lane order
constexpr int kBlocks = 4;   // 32-row blocks per 128-row tile
constexpr int kPackStages = 4;  // stages one pack wave handles (128 B per source row)

__host__ __device__ constexpr int nops_of(int algo) { return algo == 7 ? 7 : 4; }

// Product rows of a packed [rows, k] operand: rows/2 rounded up to whole
// 128-row tiles (a thin tiling's last tile is zero-padded).
__host__ __device__ constexpr int64_t padded_product_rows(int64_t rows) { return (rows / 2 + TM - 1) / TM * TM; }

// Byte offset of fragment (tile, stage, op, block) in a packed operand.
__host__ __device__ inline int64_t frag_offset(int64_t tile, int64_t stage, int64_t nstages, int op, int nops,
                                               int block) {
  return (((tile * nstages + stage) * nops + op) * kBlocks + block) * (int64_t)kFrag;
}

// kCubicSlots: LDS ring depth of the cubic (both operands); the ring is
// refilled kCubicSlots-1 stages ahead.
template <int kAlgo, int kCubicSlots = 3>
struct Lay {
  static constexpr int nops = nops_of(kAlgo);
  static constexpr int kStage = nops * kBlocks * kFrag;  // one operand, one stage
  // Strassen's 28 KB stages allow two A slots next to three B slots.
  static constexpr int kASlots = kAlgo == 7 ? 2 : kCubicSlots;
  static constexpr int kBSlots = kAlgo == 7 ? 3 : kCubicSlots;
  static constexpr int kLds = (kASlots + kBSlots) * kStage;
  static constexpr int kDmaPerWave = nops;  // nops*4 fragments over 4 waves
  // VMEM operations a wave may leave in flight at the stage barrier: the
  // prefetches that target stages after s+1 (Strassen: B stage s+2; cubic:
  // A and B stages s+2 .. s+kCubicSlots-1).
  static constexpr int kPending = kAlgo == 7 ? kDmaPerWave : (kCubicSlots - 2) * 2 * kDmaPerWave;
  static_assert(kLds <= 160 * 1024, "LDS budget");
  static_assert(kPending < 64, "vmcnt range");
};

// s_waitcnt immediate (gfx9 encoding) for vmcnt(vm) lgkmcnt(lgkm), no
// export-count wait.
constexpr int waitcnt_imm(int vm, int lgkm) { return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | (lgkm << 8); }

// Barrier after this wave's LDS reads and all but its newest kPending VMEM
// operations have completed. The wait is issued through the builtin so the
// compiler's own wait tracking knows the LDS reads are complete (and adds no
// later wait for them); the asm repeats it next to the barrier, and its
// "memory" clobber keeps the compiler from moving LDS accesses across.
template <int kPending>
__device__ __forceinline__ void stage_barrier() {
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(kPending, 0));
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"i"(kPending) : "memory");
}

// v_mfma_f32_32x32x16_bf16 with the accumulator pinned to AGPRs / VGPRs.
// An accumulator is reused only 4+ MFMAs later and read by VALU only after
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

// Operand DMA goes through buffer loads into LDS (buffer_load_dwordx4 ...
// lds). Measured on gfx950, the FLAT form of the same DMA
// (global_load_lds_dwordx4) holds back the MFMAs of every wave on the CU
// while its data arrives: an MFMA stream and a DMA stream on one CU took
// about the sum of their separate times, at full chip load and on 32 CUs
// alike; with buffer loads they overlap (1.89 against 1.57 PFLOP/s for 32 KB
// and 128 MFMAs per CU and stage).
//
// A wave's operand panel as a buffer resource: base = the wave's first
// fragment in the workgroup's packed panel, num_records = the bytes from
// there to the panel's end. Word 3 selects raw 32-bit-format access (gfx9
// DATA_FORMAT 32). A load past num_records returns zeros instead of
// touching memory.
constexpr int kBufferWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t panel_rsrc(const uint8_t* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), 0, (int)bytes, kBufferWord3);
}

// One fragment-sized DMA: every lane moves 16 bytes at panel offset
// soffset (uniform) + voffset (the lane's 16 * lane) into LDS at `to` + 16 *
// lane.
__device__ __forceinline__ void dma_frag(__amdgpu_buffer_rsrc_t rsrc, uint32_t voffset, uint32_t soffset,
                                         uint8_t* to) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)to, 16, voffset, soffset,
                                           0, 0);
}

__device__ __forceinline__ bf16x8 ld_frag(const uint8_t* p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(p));
}

// kThin: a tiling whose bm/2 is not a multiple of 128 (ThinRows).
template <int kAlgo, int kEpi, int kQuad, int kCubicSlots = 3, bool kThin = false>
__global__ __launch_bounds__(kThreads, 1) void gemm_packed(Params p) {
  static_assert(kAlgo == 8, "the packed kernel serves the cubic; Strassen runs on gemm_split");
  using L = Lay<kAlgo, kCubicSlots>;
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
  static_assert(kEpiLds<kEpi, 64, 64> <= 160 * 1024, "epilogue staging fits the LDS");
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;

  const int nstages_all = (int)(p.k / (2 * TK));
  const WorkShare ws = work_share(p, nstages_all);
  int tile_m, tile_n;
  tile_of(ws.tile, p.tiles_m, p.tiles_n, p.group_m, p.raster, tile_m, tile_n);
  TileOrigin o = tile_origin<kThin>(p, (int64_t)tile_m * TM, (int64_t)tile_n * TN);
  // K-split shares run without an epilogue and store dense FP32 blocks.
  if constexpr (kEpi == SMX_EPI_NONE)
    if (p.ksplit > 1) dense_share_output(p, o, ws, (int64_t)tile_m * TM);
  const int nstages = ws.nstages;

  // DMA sources: this workgroup's packed stages are contiguous runs of
  // L::kStage bytes; wave w moves fragments f = w + 4x of each.
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t panel_bytes = (uint32_t)nstages * L::kStage - wave_u * kFrag;
  const __amdgpu_buffer_rsrc_t a_src = panel_rsrc(
      reinterpret_cast<const uint8_t*>(p.a) + ((int64_t)tile_m * nstages_all + ws.stage0) * L::kStage + wave_u * kFrag,
      panel_bytes);
  const __amdgpu_buffer_rsrc_t b_src = panel_rsrc(
      reinterpret_cast<const uint8_t*>(p.b) + ((int64_t)tile_n * nstages_all + ws.stage0) * L::kStage + wave_u * kFrag,
      panel_bytes);
  const uint32_t lane_off = lane * 16;
  uint8_t* const a_region = lds;
  uint8_t* const b_region = lds + L::kASlots * L::kStage;

  // Prefetches past the last stage re-load it (in bounds, never read)
  // instead of branching.
  auto dma = [&](__amdgpu_buffer_rsrc_t src, int stage, uint8_t* slot) {
    const uint32_t from = (uint32_t)min(stage, nstages - 1) * L::kStage;
#pragma unroll
    for (int x = 0; x < L::kDmaPerWave; ++x) dma_frag(src, lane_off, from + x * 4 * kFrag, slot + (wave_u + 4 * x) * kFrag);
  };

  f32x16 acc[L::nops][2][2];
  zero_acc(acc);

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
    // Accumulator sets 0-3 live in AGPRs and (Strassen) 4-6 in VGPRs, pinned
    // through the operand constraint, so the accumulators never move between
    // the two files and the VGPRs stay free for fragments.
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
  // Cubic products a0b0 a0b1 a2b0 a2b1 a1b2 a1b3 a3b2 a3b3
  // (benchmark_cubic_control.py:96-106) run one K half at a time, A
  // quadrants (top, bottom) x B quadrants (left, right), every fragment
  // feeding two MFMAs (the cubic loop below).

  // Prologue: stages 0..kASlots-2 of A and 0..kBSlots-2 of B.
  dma(a_src, 0, a_region);
  dma(b_src, 0, b_region);
#pragma unroll
  for (int st = 1; st + 1 < L::kBSlots; ++st) {
    if (st + 1 < L::kASlots) dma(a_src, st, a_region + st * L::kStage);
    dma(b_src, st, b_region + st * L::kStage);
  }
  stage_barrier<L::kPending>();

  if constexpr (kAlgo == 8) {
    // Cubic: a whole stage of fragments (16) fits in VGPRs next to the AGPR
    // accumulators, so the barrier moves to mid-stage and the reads of stage
    // s+1 run under the second half of stage s's MFMAs:
    //   DMA stage s+kSlots-1 | MFMAs K half 0 of s | barrier | read s+1 | MFMAs K half 1 of s
    // The barrier guarantees that every wave's DMA of stage s+1 has landed
    // (vmcnt leaves only later stages in flight) and that every wave
    // finished reading stage s (its reads completed before its first MFMA
    // of s), so stage s's slot may be refilled after it.
    struct Stage {
      Frags h0t, h0b, h1t, h1b;  // K half x (A top + B left, A bottom + B right)
    };
    auto load_stage = [&](int slot) {
      const uint8_t* sa = a_region + slot * L::kStage;
      const uint8_t* sb = b_region + slot * L::kStage;
      return Stage{load_frags(sa, sb, 0, 0), load_frags(sa, sb, 2, 1), load_frags(sa, sb, 1, 2),
                   load_frags(sa, sb, 3, 3)};
    };
    auto half = [&](const Frags& t, const Frags& b) {
      mfma4(Frags{t.a0, t.a1, t.b0, t.b1}, 0);
      mfma4(Frags{t.a0, t.a1, b.b0, b.b1}, 1);
      mfma4(Frags{b.a0, b.a1, t.b0, t.b1}, 2);
      mfma4(Frags{b.a0, b.a1, b.b0, b.b1}, 3);
    };
    int s = 0, slot = 0;
    constexpr int kSlots = kCubicSlots;
    auto body = [&](const Stage& cur) {
      // Slot of stage s+1, and of stage s+kSlots-1 (the one read at s-1).
      const int slot1 = slot == kSlots - 1 ? 0 : slot + 1, refill = slot == 0 ? kSlots - 1 : slot - 1;
      // The stage's DMA fragments (A then B) go out one at a time between the
      // first half's MFMAs, after the second and fourth of each group of
      // four, rather than in bursts: a DMA issued right after another holds
      // back the next MFMA's issue (measured 5% on the gate|up launch). All
      // are issued before the mid-stage barrier, so its vmcnt accounting is
      // unchanged.
      const uint32_t from = (uint32_t)min(s + kSlots - 1, nstages - 1) * L::kStage;
      uint8_t* const a_to = a_region + refill * L::kStage + wave_u * kFrag;
      uint8_t* const b_to = b_region + refill * L::kStage + wave_u * kFrag;
      auto dma_one = [&](int q) __attribute__((always_inline)) {
        const bool is_a = q < L::kDmaPerWave;
        const int x = is_a ? q : q - L::kDmaPerWave;
        dma_frag(is_a ? a_src : b_src, lane_off, from + x * 4 * kFrag, (is_a ? a_to : b_to) + 4 * x * kFrag);
      };
      // Group g's four MFMAs on quadrant set g, with DMAs 2g and 2g + 1.
      auto mfma4_dma = [&](const Frags& f, int g) __attribute__((always_inline)) {
        auto step = [&](f32x16& c, const bf16x8& a, const bf16x8& b, int k) __attribute__((always_inline)) {
          mfma_agpr(c, a, b);
          __builtin_amdgcn_sched_barrier(0);
          if (k == 1) dma_one(2 * g);
          if (k == 3) dma_one(2 * g + 1);
          __builtin_amdgcn_sched_barrier(0);
        };
        step(acc[g][0][0], f.a0, f.b0, 0);
        step(acc[g][0][1], f.a0, f.b1, 1);
        step(acc[g][1][0], f.a1, f.b0, 2);
        step(acc[g][1][1], f.a1, f.b1, 3);
      };
      static_assert(2 * L::kDmaPerWave == 8, "two DMAs per MFMA group");
      __builtin_amdgcn_sched_barrier(0);
      {
        const Frags& t = cur.h0t;
        const Frags& b = cur.h0b;
        mfma4_dma(Frags{t.a0, t.a1, t.b0, t.b1}, 0);
        mfma4_dma(Frags{t.a0, t.a1, b.b0, b.b1}, 1);
        mfma4_dma(Frags{b.a0, b.a1, t.b0, t.b1}, 2);
        mfma4_dma(Frags{b.a0, b.a1, b.b0, b.b1}, 3);
      }
      __builtin_amdgcn_sched_barrier(0);
      stage_barrier<L::kPending>();
      const Stage next = load_stage(slot1);  // past the last stage: re-reads it, unused
      __builtin_amdgcn_sched_barrier(0);
      half(cur.h1t, cur.h1b);
      __builtin_amdgcn_sched_barrier(0);
      slot = slot1;
      return next;
    };
    // Unrolled by two so the fragment sets swap roles without copies. The
    // host guarantees an even stage count (bk % 64 == 0), so the loop is
    // bottom-tested with no tail: a branch between the two bodies would let
    // the compiler sink the second body's reads past it (out of the MFMA
    // shadow), and any path that skips the loop gets its own copy of the
    // accumulator initialisation.
    Stage f0 = load_stage(0);
    do {
      const Stage f1 = body(f0);
      ++s;
      f0 = body(f1);
      ++s;
    } while (s < nstages);
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    mfma_drain(acc);
    epilogue<kQuad, 2, 2, kEpi, L::nops, kThin>(p, o, wm * 64, wn * 64, acc,
                                                lds + wave * kEpiTiles<kEpi> * StageTile<64, 64>::kBytes);
    return;
  }

}

// Packs one operand. kSide 0: A [m, k] row-major (kSide 2: the same A stored
// transposed as [k, m]), product row R = (tile i,
// row r < bm/2) -> physical rows i*bm + r (top) and + bm/2 (bottom).
// kSide 1: B^T [n, k] row-major, product column C = (tile j, c < bn/2) ->
// rows j*bn + c (left) and + bn/2 (right) of B^T. Product depth k' = (panel
// s, kk < bk/2) -> columns s*bk + kk and + bk/2. Quadrants: A0 = (top, k
// left), A1 = (top, k right), A2 = (bottom, k left), A3 = (bottom, k right);
// B0 = (k top, left), B1 = (k top, right), B2 = (k bottom, left),
// B3 = (k bottom, right) (strassen_pallas.py:188-204). With a panel map,
// packed K panel s reads source panel panels[s] (the Strassen or the exact
// panels of an exact-panel schedule); without one, panel s. One wave packs one
// 32-row product block over kPackStages stages: each lane loads 16 bytes of
// each quadrant per stage and stores nops 16-byte chunks, so the stores of
// a wave are whole 1 KB fragments.
// One lane's share of one packed stage: from the four quadrant values x
// (A: [row half][K half]; B: [K half][column half]) of its 8 consecutive k,
// the nops operands of the formula, each stored as 16 bytes at dst + op x 4 KB
// (lane-contiguous, so every store instruction writes 1 KB).
template <int kAlgo, int kSide, bool kF32>
__device__ __forceinline__ void store_fragments(F8 (&x)[4], int formula, int perm, int part, uint8_t* dst) {
  auto store = [&](int op, const F8& v) {
    *reinterpret_cast<u32x4*>(dst + op * kBlocks * kFrag) = kF32 ? pack8_part(v, part) : pack8(v);
  };
  if constexpr (kAlgo == 7) {
    F8 ops[7];
    if constexpr (kSide != 1) {
      permute_quadrants(x, perm & 1, (perm >> 1) & 1);  // A: (rows, K halves)
      formula_vals<0, !kF32>(formula, x, ops);
    } else {
      permute_quadrants(x, (perm >> 1) & 1, (perm >> 2) & 1);  // B: (K halves, columns)
      formula_vals<1, !kF32>(formula, x, ops);
    }
#pragma unroll
    for (int op = 0; op < 7; ++op) store(op, ops[op]);
  } else {
#pragma unroll
    for (int op = 0; op < 4; ++op) store(op, x[op]);
  }
}

template <int kAlgo, int kSide, bool kF32>
__global__ __launch_bounds__(256) void pack_operand(const void* __restrict__ src_v, int64_t ld, int64_t rows,
                                                    int64_t k, int32_t tile_rows, int32_t bk, int32_t formula,
                                                    int32_t perm, const int32_t* __restrict__ panels,
                                                    int32_t src_panels, int32_t passes,
                                                    uint8_t* __restrict__ out) {
  // Source elements: bf16, or float (FP32 inputs: the operand sums are
  // formed in float and each operand is rounded once to bf16, or, for a
  // product of `passes` bf16 passes, split into bf16 parts: the packed K runs
  // pass-major, packed panel j holding pass j / slots of slot j % slots,
  // slots = k / (passes * bk)).
  using Elem = typename std::conditional<kF32, float, uint16_t>::type;
  const Elem* const src = reinterpret_cast<const Elem*>(src_v);
  constexpr int nops = nops_of(kAlgo);
  const int lane = threadIdx.x & 63;
  const int64_t gwave = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
  const int64_t nstages = k / (2 * TK);
  const int64_t sgroups = (nstages + kPackStages - 1) / kPackStages;
  const int64_t rblock = gwave / sgroups;  // 32-row product block
  if (rblock >= padded_product_rows(rows) / 32) return;
  const int64_t sg = gwave - rblock * sgroups;
  const int hr = tile_rows / 2, hk = bk / 2;
  const int64_t r = rblock * 32 + (lane & 31);
  // Product rows past rows/2 pad the last 128-row tile: they pack as zeros
  // (their source rows are clamped to row 0 and the values replaced).
  const bool pad = r >= rows / 2;
  const int64_t row_first = pad ? 0 : (r / hr) * tile_rows + r % hr, row_second = row_first + hr;
  const Elem* const first = src + row_first * ld;
  const Elem* const second = first + (int64_t)hr * ld;
  // Eight consecutive elements (columns col0 .. col0+7) of a row-major row.
  auto load_row = [&](const Elem* row, int64_t col0) {
    F8 f;
    if constexpr (kF32) {
      const f32x4 v0 = *reinterpret_cast<const f32x4*>(row + col0);
      const f32x4 v1 = *reinterpret_cast<const f32x4*>(row + col0 + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f.v[e] = v0[e];
        f.v[4 + e] = v1[e];
      }
    } else {
      f = unpack8(*reinterpret_cast<const u32x4*>(row + col0));
    }
    return f;
  };
  // kSide 2: A stored transposed, [k, rows] with row stride ld; element
  // (row, col) of A is src[col * ld + row]. Eight consecutive k of one row
  // are gathered from eight source rows (lanes cover consecutive rows, so
  // each load instruction reads 64 contiguous bytes of one source row, 128
  // for float).
  auto gather = [&](int64_t row, int64_t col0) {
    F8 f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if constexpr (kF32)
        f.v[e] = src[(col0 + e) * ld + row];
      else
        f.v[e] = bf16_to_f32(src[(col0 + e) * ld + row]);
    }
    return f;
  };
  const int half = lane >> 5;
  uint8_t* const dst_tile = out + frag_offset(rblock / 4, 0, nstages, 0, nops, (int)(rblock % 4)) + lane * 16;
#pragma unroll
  for (int j = 0; j < kPackStages; ++j) {
    const int64_t st = sg * kPackStages + j;
    if (st >= nstages) break;
    const int64_t kp = st * TK + half * 8;
    const int64_t panel = kp / hk;
    const int64_t slots = k / ((int64_t)passes * bk);
    const int64_t pass = kF32 ? panel / slots : 0;
    const int64_t slot = panel - pass * slots;
    const int part = kF32 ? pass_part(kSide == 1, passes, (int)pass) : 0;
    // Map entries are clamped to the source, so a bad map cannot read out of bounds.
    const int64_t src_panel = panels ? min(max(panels[slot], 0), src_panels - 1) : slot;
    const int64_t lo = src_panel * bk + kp % hk, hi = lo + hk;
    F8 x[4];
    if (pad) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 8; ++e) x[q].v[e] = 0.0f;
    } else if constexpr (kSide == 2) {
      x[0] = gather(row_first, lo);
      x[1] = gather(row_first, hi);
      x[2] = gather(row_second, lo);
      x[3] = gather(row_second, hi);
    } else if constexpr (kSide == 0) {
      x[0] = load_row(first, lo);
      x[1] = load_row(first, hi);
      x[2] = load_row(second, lo);
      x[3] = load_row(second, hi);
    } else {
      x[0] = load_row(first, lo);
      x[1] = load_row(second, lo);
      x[2] = load_row(first, hi);
      x[3] = load_row(second, hi);
    }
    store_fragments<kAlgo, kSide, kF32>(x, formula, perm, part, dst_tile + st * (int64_t)(nops * kBlocks * kFrag));
  }
}

// pack_operand for bf16 row-major sources (A [rows, k], or a weight stored
// [n, k]) at one pass, with coalesced reads. pack_operand's lanes read 32
// source rows per instruction, 32 bytes of each; here a workgroup first
// copies, for 32 product rows and kRowStages stages, the four source
// segments of each product row (first / second source row x lower / upper
// K half, 16 k per stage) into LDS, 16 threads per contiguous 256-byte run.
// Each wave then forms whole stages from LDS exactly as pack_operand does.
// The row stride carries a 16-byte pad, so the 8 lanes of one LDS read
// phase (consecutive rows) fall in distinct banks.
constexpr int kRowStages = 8;
constexpr int kRowRun = kRowStages * TK * 2;   // bytes of one segment: 16 k per stage
constexpr int kRowStride = 4 * kRowRun + 16;  // LDS bytes per product row

template <int kAlgo, int kSide>
__global__ __launch_bounds__(256) void pack_rows(const uint16_t* __restrict__ src, int64_t ld, int64_t rows,
                                                 int64_t k, int32_t tile_rows, int32_t bk, int32_t formula,
                                                 int32_t perm, const int32_t* __restrict__ panels,
                                                 int32_t src_panels, uint8_t* __restrict__ out) {
  static_assert(kSide == 0 || kSide == 1, "row-major sources only");
  static_assert(kRowStages % 4 == 0, "whole stages per wave");
  __shared__ __attribute__((aligned(16))) uint8_t tile[32 * kRowStride];
  constexpr int nops = nops_of(kAlgo);
  const int64_t nstages = k / (2 * TK);
  const int64_t sgroups = (nstages + kRowStages - 1) / kRowStages;
  const int64_t rblock = blockIdx.x / sgroups;  // 32-row product block
  if (rblock >= padded_product_rows(rows) / 32) return;  // uniform per workgroup
  const int64_t st0 = (blockIdx.x - rblock * sgroups) * kRowStages;
  const int hr = tile_rows / 2, hk = bk / 2;
  // Copy: 32 rows x 4 segments x kRowStages stages x two 16-byte pieces.
  constexpr int kPieces = 32 * 4 * kRowStages * 2;
  static_assert(kPieces % 256 == 0, "whole copy rounds");
#pragma unroll
  for (int i = 0; i < kPieces / 256; ++i) {
    const int piece = i * 256 + (int)threadIdx.x;
    const int sub = piece & 1, j = (piece >> 1) % kRowStages, rs = (piece >> 1) / kRowStages;
    const int row = rs >> 2, seg = rs & 3;  // seg bit 1: second source row; bit 0: upper K half
    const int64_t st = st0 + j;
    if (st < nstages) {
      const int64_t r = rblock * 32 + row;
      uint8_t* const to = tile + row * kRowStride + seg * kRowRun + j * 32 + sub * 16;
      if (r >= rows / 2) {  // padding of the last 128-row product tile: zeros
        *reinterpret_cast<u32x4*>(to) = u32x4{0u, 0u, 0u, 0u};
        continue;
      }
      const int64_t srow = (r / hr) * tile_rows + r % hr + ((seg & 2) ? hr : 0);
      // A stage's 16 k never cross a panel half (hk is a multiple of 32).
      const int64_t kp = st * TK;
      const int64_t panel = kp / hk;
      // Map entries are clamped to the source, so a bad map cannot read out of bounds.
      const int64_t src_panel = panels ? min(max(panels[panel], 0), src_panels - 1) : panel;
      const int64_t col = src_panel * bk + kp % hk + ((seg & 1) ? hk : 0) + sub * 8;
      *reinterpret_cast<u32x4*>(to) = *reinterpret_cast<const u32x4*>(src + srow * ld + col);
    }
  }
  __syncthreads();
  const int wave = (int)threadIdx.x >> 6, lane = (int)threadIdx.x & 63;
  const uint8_t* const from = tile + (lane & 31) * kRowStride + (lane >> 5) * 16;
  uint8_t* const dst_tile = out + frag_offset(rblock / 4, 0, nstages, 0, nops, (int)(rblock % 4)) + lane * 16;
#pragma unroll
  for (int jj = 0; jj < kRowStages / 4; ++jj) {
    const int j = jj * 4 + wave;
    const int64_t st = st0 + j;
    if (st >= nstages) break;
    auto seg = [&](int sg) { return unpack8(*reinterpret_cast<const u32x4*>(from + sg * kRowRun + j * 32)); };
    F8 x[4];
    if constexpr (kSide == 0) {
      x[0] = seg(0);  // first row, lower K half
      x[1] = seg(1);  // first row, upper K half
      x[2] = seg(2);  // second row, lower K half
      x[3] = seg(3);  // second row, upper K half
    } else {
      x[0] = seg(0);
      x[1] = seg(2);
      x[2] = seg(1);
      x[3] = seg(3);
    }
    store_fragments<kAlgo, kSide, false>(x, formula, perm, 0, dst_tile + st * (int64_t)(nops * kBlocks * kFrag));
  }
}

}  // namespace packed
}  // namespace smx
