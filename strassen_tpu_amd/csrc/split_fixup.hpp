// Second pass of a K-split launch (smx_gemm with a workspace): some tiles
// of a packed launch ran as p.ksplit shares of their K stages, each share
// writing its FP32 result into the workspace as one dense 256 x 256 block per
// split tile (dense_share_output). This pass sums the shares in share order
// and applies the epilogue the fused kernels apply
// (strassen_pallas.py:739-879), on the physical output positions.
#pragma once

#include "common.hpp"
#include "kernel_packed.hpp"

namespace smx {

// Workgroups per split tile: each takes 32 of the tile's 256 output rows, so
// a pass over r tiles runs 8 r workgroups and keeps enough loads in flight
// to stream at HBM speed.
constexpr int kFixupSlices = 8;

// Workgroup w serves split tile u = w / kFixupSlices (tile tile_base + u of
// the launch's grid): its 128 x 128 product-space block is 128 product rows
// in each output row half by 128 columns of each column half. Thread t takes
// columns 8 (t % 16) .. + 7 of both column halves (the a | b or gate | up
// pair of the epilogues) on rows 32 (w % kFixupSlices) + t / 16 + 16 i,
// i < 2, of the 256. Product row P is output row (P / hm) bm + half hm +
// P % hm (one row tile per product tile unless the tiling is thin); rows
// past M/2 (a thin tiling's padding) are neither read nor written. `ws`
// holds the p.ksplit shares, split_stride floats apart; in a share, split
// tile u's block starts at u * kSplitTileFloats and holds the tile's row
// lr (row half lr / 128) and column half c at lr * 256 + 128 c. p is the
// fused call's Params.
template <int kEpi>
__global__ __launch_bounds__(256) void split_fixup(Params p, const float* __restrict__ ws) {
  const int u = (int)blockIdx.x / kFixupSlices, slice = (int)blockIdx.x % kFixupSlices;
  int tile_m, tile_n;
  tile_of(p.tile_base + u, p.tiles_m, p.tiles_n, p.group_m, p.raster, tile_m, tile_n);
  const TileOrigin o = tile_origin<false>(p, (int64_t)tile_m * packed::TM, (int64_t)tile_n * packed::TN);
  const ThinRows rows{(uint32_t)(p.bm / 2), (uint32_t)p.bm, (uint32_t)(p.m / 2)};
  const uint32_t prow0 = (uint32_t)tile_m * packed::TM;
  const int64_t hn = p.bn / 2;
  const int t = (int)threadIdx.x;
  const int64_t cin = o.tc + (t & 15) * 8;  // column inside a column half
  const int64_t col_a = o.tj * p.bn + cin, col_b = col_a + hn;
  F8 bias_a{}, bias_b{}, ga{}, gb{};
  if constexpr (kEpi == SMX_EPI_BIAS_ADD) {
    // the bias has no alignment requirement: element loads
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      bias_a.v[e] = load_vec(p.bias, p.bias_f32, col_a + e);
      bias_b.v[e] = load_vec(p.bias, p.bias_f32, col_b + e);
    }
  }
  if constexpr (kEpi == SMX_EPI_QK_NORM_ROPE) {
    ga = load8(p.rope_scale, p.scale_f32, cin);
    gb = load8(p.rope_scale, p.scale_f32, hn + cin);
  }
  const float inv_width = 1.0f / (float)p.head_dim;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int lr = 32 * slice + (t >> 4) + 16 * i;  // row half lr / 128, row lr % 128 of the tile
    const uint32_t prow = prow0 + (uint32_t)(lr & 127);
    if (!rows.valid(prow)) continue;  // uniform over the 16 lanes of a row
    const int64_t row = rows.row(prow, lr >> 7);
    const int64_t at = (int64_t)u * kSplitTileFloats + lr * 256 + (t & 15) * 8;
    F8 a = load8(ws, 1, at), b = load8(ws, 1, at + 128);
    for (int h = 1; h < p.ksplit; ++h) {
      const float* const wh = ws + h * p.split_stride;
      const F8 ah = load8(wh, 1, at), bh = load8(wh, 1, at + 128);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        a.v[e] += ah.v[e];
        b.v[e] += bh.v[e];
      }
    }
    if constexpr (kEpi == SMX_EPI_SWIGLU || kEpi == SMX_EPI_GEGLU) {
      // gate | up: the tile's first and second column halves
      F8 g;
#pragma unroll
      for (int e = 0; e < 8; ++e) g.v[e] = gate_f32<kEpi>(a.v[e]) * b.v[e];
      store8(p.c, p.out_f32, row * p.ldc + o.tj * hn + cin, g);
      continue;
    }
    if constexpr (kEpi == SMX_EPI_RESIDUAL_ADD) {
      const F8 ra = load8(p.residual, p.residual_f32, row * p.ldr + col_a);
      const F8 rb = load8(p.residual, p.residual_f32, row * p.ldr + col_b);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        a.v[e] += ra.v[e];
        b.v[e] += rb.v[e];
      }
    }
    if constexpr (kEpi == SMX_EPI_BIAS_ADD) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        a.v[e] += bias_a.v[e];
        b.v[e] += bias_b.v[e];
      }
    }
    if constexpr (kEpi == SMX_EPI_QK_NORM_ROPE) {
      // A head is 64 columns of each half: eight lanes (t % 8 equal
      // neighbours) of a row. recip = rsqrt((sum a^2 + sum b^2) /
      // head_dim + eps) (v_rsq_f32, as in the fused epilogue); a' = (a recip) gamma_a, b' = (b recip) gamma_b;
      // out_a = a' cos - b' sin, out_b = b' cos + a' sin (cos, sin at the
      // output row and the column inside the half).
      float ssa = 0.f, ssb = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        ssa += a.v[e] * a.v[e];
        ssb += b.v[e] * b.v[e];
      }
#pragma unroll
      for (int x = 1; x < 8; x <<= 1) {
        ssa += __shfl_xor(ssa, x);
        ssb += __shfl_xor(ssb, x);
      }
      const float recip = __builtin_amdgcn_rsqf((ssa + ssb) * inv_width + p.eps);
      const F8 cs = unpack8(*reinterpret_cast<const u32x4*>(p.rope_cos + row * hn + cin));
      const F8 sn = unpack8(*reinterpret_cast<const u32x4*>(p.rope_sin + row * hn + cin));
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float na = (a.v[e] * recip) * ga.v[e], nb = (b.v[e] * recip) * gb.v[e];
        a.v[e] = na * cs.v[e] - nb * sn.v[e];
        b.v[e] = nb * cs.v[e] + na * sn.v[e];
      }
    }
    store8(p.c, p.out_f32, row * p.ldc + col_a, a);
    store8(p.c, p.out_f32, row * p.ldc + col_b, b);
  }
}

}  // namespace smx
