// Tile-local one-level Strassen GEMM (7 products) and the matched blocked
// cubic GEMM (8 products) for gfx950, with fused epilogues, behind the C ABI
// of include/strassen_mi355x.h.
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
// a block of product space, i.e. the same (r, c) positions in all four output
// quadrants, so every thread holds all four quadrant values of its outputs
// and SwiGLU (gate|up), RoPE (a|b), residual and bias epilogues are
// register-local. The seven products accumulate into seven persistent FP32
// accumulator sets, combined once after the last K panel:
//   C0 = P1 + P4 - P5 + P7, C1 = P3 + P5, C2 = P2 + P4, C3 = P1 - P2 + P3 + P6.
//
// Kernels:
//   split (kernel_split.hpp): the Strassen kernel for packed operands. The
//      packed kernel's operands, LDS ring and DMA, with each wave owning
//      seven (product, 32-row strip) pairs of the 128x128 product-space tile
//      instead of a 64x64 region of all seven products; the accumulators are
//      regrouped by region through LDS before the shared epilogue.
//   packed (kernel_packed.hpp): the cubic's kernel: 128x128 product-space
//      tiles, 64x64 waves, both operands pre-packed (smx_pack_operand: the
//      Strassen operand sums or the cubic quadrants, in MFMA fragment order)
//      and streamed into an LDS ring by DMA.
//   v1 (kernel_v1.hpp): 128x64 tiles, row-major A and B^T, both operand sums
//      formed in registers; serves unpacked calls whose tile the packed
//      kernels cannot take, or all of them under SMX_PLAIN_WEIGHTS=compact.
// The split and packed kernels are instantiated in translation units of
// their own (gemm_strassen*.hip, gemm_cubic*.hip) and reached through the
// launchers of launch.hpp; a thin tiling (bm/2 not a multiple of the 128-row
// product tile, bm % 16 == 0 as the reference allows) runs their kThin
// instantiations, whose epilogues map rows one by one (ThinRows).

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <numeric>

#include "common.hpp"
#include "kernel_packed.hpp"
#include "kernel_pm.hpp"
#include "kernel_v1.hpp"
#include "launch.hpp"
#include "split_fixup.hpp"

namespace smx {
namespace {
thread_local char g_error[512] = "";
}  // namespace

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

namespace {

template <class K>
int set_lds(K kern, int bytes) {
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e != hipSuccess) return fail(SMX_ERR_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(e));
  return SMX_OK;
}

// Tile rows per rasterization group; SMX_GROUP_M overrides the default for
// tuning sweeps.
int group_m_setting() {
  static const int value = [] {
    const char* env = getenv("SMX_GROUP_M");
    const int v = env ? atoi(env) : 0;
    return v > 0 && v <= 64 ? v : 8;
  }();
  return value;
}

// Tile order of a packed launch (tile_of): SMX_RASTER=spread, chunks or
// blocks forces one; unset (-1), packed_grid chooses.
int raster_setting() {
  static const int value = [] {
    const char* env = getenv("SMX_RASTER");
    if (!env) return -1;
    if (!strcmp(env, "spread")) return (int)kRasterSpread;
    if (!strcmp(env, "chunks")) return (int)kRasterChunks;
    if (!strcmp(env, "blocks")) return (int)kRasterBlocks;
    return -1;
  }();
  return value;
}

template <class C, int kEpi>
int launch_v1(Params p, hipStream_t stream) {
  p.tiles_m = (int)((p.m / 2) / C::TM);
  p.tiles_n = (int)((p.n / 2) / C::TN);
  p.group_m = group_m_setting();
  auto kern = v1::gemm_v1<C, kEpi>;
  // operand slabs, then the epilogue's staging tiles, share the LDS
  constexpr int lds = C::kLds > kEpiLds<kEpi, 32 * C::mb, 32 * C::nb> ? C::kLds : kEpiLds<kEpi, 32 * C::mb, 32 * C::nb>;
  if (int rc = set_lds(kern, lds)) return rc;
  hipLaunchKernelGGL(kern, dim3(p.tiles_m * p.tiles_n), dim3(kThreads), lds, stream, p);
  return check_launch();
}

template <int kAlgo>
int dispatch_v1(const Params& p, int epilogue, hipStream_t s) {
  switch (epilogue) {
    case SMX_EPI_NONE: return launch_v1<v1::General<kAlgo>, SMX_EPI_NONE>(p, s);
    case SMX_EPI_SWIGLU: return launch_v1<v1::General<kAlgo>, SMX_EPI_SWIGLU>(p, s);
    case SMX_EPI_GEGLU: return launch_v1<v1::General<kAlgo>, SMX_EPI_GEGLU>(p, s);
    case SMX_EPI_RESIDUAL_ADD: return launch_v1<v1::General<kAlgo>, SMX_EPI_RESIDUAL_ADD>(p, s);
    case SMX_EPI_BIAS_ADD: return launch_v1<v1::General<kAlgo>, SMX_EPI_BIAS_ADD>(p, s);
    case SMX_EPI_QK_NORM_ROPE: return launch_v1<v1::ForQK<kAlgo>, SMX_EPI_QK_NORM_ROPE>(p, s);
  }
  return fail(SMX_ERR_INVALID, "unknown epilogue %d", epilogue);
}

// Tile granules of a path: bm % (2 tm), bn % (2 tn), bk % (2 tk). Packed
// operands take any bm the reference allows (bm % 16; thin tilings map rows
// in the epilogue); the v1 kernels need whole 128-row product tiles.
constexpr int32_t kThinRowGranule = 8;

void tile_of_path(bool packed_path, int32_t* tm, int32_t* tn, int32_t* tk) {
  if (packed_path) {
    *tm = kThinRowGranule;
    *tn = packed::TN;
    *tk = packed::kKGranule;
  } else {  // both v1 configurations are 128 x 64 x 32
    *tm = v1::General<7>::TM;
    *tn = v1::General<7>::TN;
    *tk = v1::General<7>::TK;
  }
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

// Formula / block-permutation arguments shared by smx_gemm and smx_pack_operand.
int check_variant(int32_t algo, int32_t formula, int32_t perm) {
  if (formula < SMX_FORMULA_CLASSICAL || formula > SMX_FORMULA_POWERS)
    return fail(SMX_ERR_INVALID, "formula must be classical (0), dual (1) or powers (2), got %d", formula);
  if (perm < 0 || perm > 7) return fail(SMX_ERR_INVALID, "block_permutation must be 0..7, got %d", perm);
  if (algo == SMX_ALGO_CUBIC && (formula || perm))
    return fail(SMX_ERR_INVALID, "the cubic control has no formula variant or block permutation");
  return SMX_OK;
}

template <int kAlgo, int kSide>
int launch_pack(const void* src, bool src_f32, int64_t ld, int64_t rows, int64_t k, int32_t tile_rows, int32_t bk,
                int32_t formula, int32_t perm, const int32_t* panels, int32_t src_panels, int32_t passes,
                uint8_t* out, hipStream_t stream) {
  const int64_t nstages = k / (2 * packed::TK);
  if constexpr (kSide != 2) {
    if (!src_f32) {  // bf16 row-major source: the LDS-staged kernel
      const int64_t blocks =
          (packed::padded_product_rows(rows) / 32) * ((nstages + packed::kRowStages - 1) / packed::kRowStages);
      if (blocks >= ((int64_t)1 << 31)) return fail(SMX_ERR_UNSUPPORTED, "operand too large to pack");
      hipLaunchKernelGGL((packed::pack_rows<kAlgo, kSide>), dim3((unsigned)blocks), dim3(256), 0, stream,
                         (const uint16_t*)src, ld, rows, k, tile_rows, bk, formula, perm, panels, src_panels, out);
      return check_launch();
    }
  }
  const int64_t waves =
      (packed::padded_product_rows(rows) / 32) * ((nstages + packed::kPackStages - 1) / packed::kPackStages);
  const int64_t blocks = (waves + 3) / 4;
  if (blocks >= ((int64_t)1 << 31)) return fail(SMX_ERR_UNSUPPORTED, "operand too large to pack");
  if (src_f32)
    hipLaunchKernelGGL((packed::pack_operand<kAlgo, kSide, true>), dim3((unsigned)blocks), dim3(256), 0, stream, src,
                       ld, rows, k, tile_rows, bk, formula, perm, panels, src_panels, passes, out);
  else
    hipLaunchKernelGGL((packed::pack_operand<kAlgo, kSide, false>), dim3((unsigned)blocks), dim3(256), 0, stream, src,
                       ld, rows, k, tile_rows, bk, formula, perm, panels, src_panels, 1, out);
  return check_launch();
}

// norm_residual_add's second pass (strassen_pallas.py:836-866): one
// workgroup per output row of the FP32 product x [m, n]:
// out = bf16(x * rsqrt(mean(x^2) + eps) * scale + residual). The row's sum of
// squares is accumulated in FP32 per thread, then across the workgroup.
__global__ __launch_bounds__(256) void norm_residual_rows(const float* __restrict__ x, int64_t ldx,
                                                          const void* __restrict__ residual, int64_t ldr,
                                                          const void* __restrict__ scale, int32_t dtypes,
                                                          float eps, int64_t n, void* __restrict__ out,
                                                          int64_t ldo) {
  __shared__ float partial[4];
  const int64_t row = blockIdx.x;
  const float* xr = x + row * ldx;
  float ss = 0.f;
  for (int64_t c = threadIdx.x; c < n; c += blockDim.x) ss += xr[c] * xr[c];
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) ss += __shfl_xor(ss, s, 64);
  if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float total = (partial[0] + partial[1]) + (partial[2] + partial[3]);
  const float recip = 1.0f / sqrtf(total / (float)n + eps);
  const int scale_f32 = dtypes & SMX_NRA_SCALE_F32, residual_f32 = dtypes & SMX_NRA_RESIDUAL_F32;
  for (int64_t c = threadIdx.x; c < n; c += blockDim.x) {
    const float v = xr[c] * recip * load_vec(scale, scale_f32, c) + load_vec(residual, residual_f32, row * ldr + c);
    if (dtypes & SMX_NRA_OUT_F32)
      reinterpret_cast<float*>(out)[row * ldo + c] = v;
    else
      reinterpret_cast<uint16_t*>(out)[row * ldo + c] = f32_to_bf16(v);
  }
}

// Checks a GEMM descriptor and its operands and fills the kernel parameters;
// launches nothing. Shared by smx_gemm and smx_gemm_noalloc.
int gemm_params(const smx_gemm_desc* d, const void* a, const void* b, void* c, const void* residual,
                const void* bias, const void* rope_cos, const void* rope_sin, const void* rope_scale, Params& p) {
  if (!d) return fail(SMX_ERR_INVALID, "null descriptor");
  if (d->algo != SMX_ALGO_STRASSEN && d->algo != SMX_ALGO_CUBIC)
    return fail(SMX_ERR_INVALID, "algo must be %d (Strassen) or %d (cubic), got %d", SMX_ALGO_STRASSEN,
                SMX_ALGO_CUBIC, d->algo);
  if (d->a_layout != SMX_A_ROWMAJOR && d->a_layout != SMX_A_PACKED)
    return fail(SMX_ERR_INVALID, "a_layout must be SMX_A_ROWMAJOR or SMX_A_PACKED, got %d", d->a_layout);
  if (d->b_layout != SMX_B_KCONTIG && d->b_layout != SMX_B_PACKED)
    return fail(SMX_ERR_INVALID, "b_layout must be SMX_B_KCONTIG or SMX_B_PACKED, got %d", d->b_layout);
  const bool packed_path = d->b_layout == SMX_B_PACKED;
  if (packed_path != (d->a_layout == SMX_A_PACKED))
    return fail(SMX_ERR_UNSUPPORTED, "A and B must both be packed (smx_pack_operand) or both unpacked");
  if (d->flags & ~(SMX_FLAG_OUT_F32 | SMX_FLAG_PRODUCT_MAJOR | SMX_FLAG_PRODUCT_MAJOR_ROUNDS))
    return fail(SMX_ERR_INVALID, "unknown flags 0x%x", d->flags);
  if ((d->flags & SMX_FLAG_PRODUCT_MAJOR) && (d->flags & SMX_FLAG_PRODUCT_MAJOR_ROUNDS))
    return fail(SMX_ERR_INVALID, "SMX_FLAG_PRODUCT_MAJOR and SMX_FLAG_PRODUCT_MAJOR_ROUNDS exclude each other");
  if (int rc = check_variant(d->algo, d->formula, d->block_permutation)) return rc;
  if ((d->formula || d->block_permutation) && !packed_path)
    return fail(SMX_ERR_UNSUPPORTED, "formula variants and block permutations run on packed operands");
  if (d->formula == SMX_FORMULA_POWERS && d->epilogue != SMX_EPI_NONE)
    return fail(SMX_ERR_INVALID, "fused epilogues require a quadrant-basis formula");
  if (d->partial && d->algo != SMX_ALGO_CUBIC)
    return fail(SMX_ERR_INVALID, "an FP32 partial is added by the cubic algorithm only");
  if (d->partial && d->a_layout != SMX_A_PACKED)
    return fail(SMX_ERR_UNSUPPORTED, "an FP32 partial needs packed operands (smx_pack_operand)");
  if (d->partial && (d->ldp < d->n || d->ldp % 4 || !aligned16(d->partial)))
    return fail(SMX_ERR_INVALID, "partial needs ldp >= N, ldp %% 4 == 0 and 16-byte alignment");
  if (d->m <= 0 || d->n <= 0 || d->k <= 0)
    return fail(SMX_ERR_INVALID, "empty problem m=%lld n=%lld k=%lld", (long long)d->m, (long long)d->n,
                (long long)d->k);
  if (d->bm <= 0 || d->bn <= 0 || d->bk <= 0 || d->m % d->bm || d->n % d->bn || d->k % d->bk)
    return fail(SMX_ERR_INVALID, "M, N, K must be divisible by bm, bn, bk");
  // Product-space coordinates (rows of M/2, columns of N/2) are 32-bit in the kernels.
  if (d->m / 2 >= ((int64_t)1 << 31) || d->n / 2 >= ((int64_t)1 << 31))
    return fail(SMX_ERR_UNSUPPORTED, "M/2 and N/2 must stay below 2^31 (m=%lld, n=%lld)", (long long)d->m,
                (long long)d->n);
  int32_t tm, tn, tk;
  tile_of_path(packed_path, &tm, &tn, &tk);
  const int hm = d->bm / 2, hn = d->bn / 2, hk = d->bk / 2;
  if (d->bm % 2 || d->bn % 2 || d->bk % 2 || hm % tm || hn % tn || hk % tk)
    return fail(SMX_ERR_UNSUPPORTED,
                "tile (bm=%d, bn=%d, bk=%d) unsupported on gfx950: need bm %% %d == 0, bn %% %d == 0, bk %% %d == 0",
                d->bm, d->bn, d->bk, 2 * tm, 2 * tn, 2 * tk);
  if (!a || !b || !c) return fail(SMX_ERR_INVALID, "null operand pointer");
  if (!aligned16(a) || !aligned16(b)) return fail(SMX_ERR_INVALID, "A and B must be 16-byte aligned");
  if (!packed_path && (d->lda < d->k || d->ldb < d->k || d->lda % 8 || d->ldb % 8))
    return fail(SMX_ERR_INVALID, "lda and ldb must be >= K and multiples of 8 elements");
  const int64_t out_cols = (d->epilogue == SMX_EPI_SWIGLU || d->epilogue == SMX_EPI_GEGLU) ? d->n / 2 : d->n;
  if (d->ldc < out_cols) return fail(SMX_ERR_INVALID, "ldc must be >= output width");
  // The epilogue moves output (and residual / partial) rows in 16-byte chunks.
  const bool out_f32 = (d->flags & SMX_FLAG_OUT_F32) != 0;
  if (!aligned16(c) || d->ldc % (out_f32 ? 4 : 8))
    return fail(SMX_ERR_INVALID, "C rows must be 16-byte aligned (C 16-byte aligned, ldc %% %d == 0)", out_f32 ? 4 : 8);
  if (d->workspace_bytes < 0 || !aligned16(d->workspace))
    return fail(SMX_ERR_INVALID, "the workspace must be 16-byte aligned with workspace_bytes >= 0");
  // The q/k epilogue addresses its RoPE tables ([M, bn/2] per tile half)
  // with 32-bit element offsets.
  if ((int64_t)hm * d->bn >= ((int64_t)1 << 31))
    return fail(SMX_ERR_UNSUPPORTED, "bm/2 * bn must stay below 2^31 (bm=%d, bn=%d)", d->bm, d->bn);
  // A thin tiling's q/k epilogue addresses the whole [M, bn/2] tables so.
  if (packed_path && hm % packed::TM && d->epilogue == SMX_EPI_QK_NORM_ROPE && d->m * (d->bn / 2) >= ((int64_t)1 << 31))
    return fail(SMX_ERR_UNSUPPORTED, "thin tilings (bm/2 %% 128 != 0) with qk_norm_rope need M * bn/2 below 2^31");
  p = Params{};
  p.a = (const uint16_t*)a;
  p.b = (const uint16_t*)b;
  p.c = c;
  p.out_f32 = (d->flags & SMX_FLAG_OUT_F32) ? 1 : 0;
  p.formula = d->formula;
  p.perm = d->block_permutation;
  p.partial = d->partial;
  p.ldp = d->partial ? d->ldp : 0;
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
  p.residual_f32 = d->aux_f32 & SMX_AUX_RESIDUAL_F32 ? 1 : 0;
  switch (d->epilogue) {
    case SMX_EPI_NONE:
    case SMX_EPI_SWIGLU:
    case SMX_EPI_GEGLU:
      break;
    case SMX_EPI_RESIDUAL_ADD:
      if (!residual) return fail(SMX_ERR_INVALID, "residual_add epilogue requires residual");
      if (d->ldr < d->n) return fail(SMX_ERR_INVALID, "ldr must be >= N");
      if (!aligned16(residual) || d->ldr % (p.residual_f32 ? 4 : 8))
        return fail(SMX_ERR_INVALID, "residual rows must be 16-byte aligned (residual 16-byte aligned, ldr %% %d == 0)",
                    p.residual_f32 ? 4 : 8);
      p.residual = residual;
      break;
    case SMX_EPI_BIAS_ADD:
      if (!bias) return fail(SMX_ERR_INVALID, "bias_add epilogue requires bias");
      p.bias = bias;
      break;
    case SMX_EPI_QK_NORM_ROPE:
      if (!rope_cos || !rope_sin || !rope_scale)
        return fail(SMX_ERR_INVALID, "qk_norm_rope requires rope_cos, rope_sin and rope_scale");
      // the epilogue reads the tables and the scale 16 bytes at a time
      if (!aligned16(rope_cos) || !aligned16(rope_sin) || !aligned16(rope_scale))
        return fail(SMX_ERR_INVALID, "rope_cos, rope_sin and rope_scale must be 16-byte aligned");
      if (d->rope_head_dim != 128)
        return fail(SMX_ERR_UNSUPPORTED,
                    "the fused qk_norm_rope takes head_dim 128, got %d: run smx_gemm with SMX_FLAG_OUT_F32 and no "
                    "epilogue, then smx_qk_norm_rope",
                    d->rope_head_dim);
      if (d->bn % (2 * d->rope_head_dim))
        return fail(SMX_ERR_INVALID, "qk_norm_rope needs bn a multiple of 2*head_dim");
      p.rope_cos = (const uint16_t*)rope_cos;
      p.rope_sin = (const uint16_t*)rope_sin;
      p.rope_scale = rope_scale;
      break;
    default:
      return fail(SMX_ERR_INVALID, "unknown epilogue %d", d->epilogue);
  }
  return SMX_OK;
}

constexpr int kMaxDevices = 64;

// Compute units of the current device, looked up once per device.
int device_cus(int* cus) {
  static std::atomic<int> known[kMaxDevices] = {};
  int device = -1;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return fail(SMX_ERR_LAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
  if (device < 0 || device >= kMaxDevices) return fail(SMX_ERR_UNSUPPORTED, "device %d out of range", device);
  int v = known[device].load(std::memory_order_relaxed);
  if (v <= 0) {
    e = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device);
    if (e != hipSuccess || v <= 0) return fail(SMX_ERR_LAUNCH, "compute unit count: %s", hipGetErrorString(e));
    known[device].store(v, std::memory_order_relaxed);
  }
  *cus = v;
  return SMX_OK;
}

// SMX_TAIL_SPLIT=0 keeps every tile of a launch over full K (for timing
// the launch shapes against each other).
bool split_setting() {
  static const bool value = [] {
    const char* env = getenv("SMX_TAIL_SPLIT");
    return !(env && env[0] == '0');
  }();
  return value;
}

// Bytes of packed operand the MALL (the 256 MB memory-side cache shared by
// the XCDs) keeps across a launch's rounds next to the streaming operand.
constexpr int64_t kMallResident = (int64_t)192 << 20;

// Tile order (tile_of) of a packed launch, from its packed operand sizes.
// Measured on MI355X (whole rounds, Strassen): a packed A that the MALL
// holds runs fastest spread over all tile rows (8192 x 5120 x 20480: 1.47 ms
// spread, 1.55 chunks); a larger A with a B that fits runs fastest in chunks
// (16384 x 5120 x 10240: 1.63 ms spread, 1.51 chunks); when neither fits
// but a round's 32 panels do, in blocks (8192 x 8192 x 20480: 2.47 ms
// spread, 2.35 blocks); with panels beyond that no order gains (8192 x 25600
// x 5120: 2.09-2.11 ms).
int raster_for(const Params& p, int algo, int tile_cols) {
  const int64_t nops = packed::nops_of(algo), depth = p.k / 2;
  const int64_t panel = (int64_t)packed::TM * depth * nops * 2;
  const int64_t b_panel = panel * (tile_cols / packed::TN);
  const int64_t a_bytes = (int64_t)p.tiles_m * panel, b_bytes = (int64_t)p.tiles_n * b_panel;
  if (a_bytes <= kMallResident) return kRasterSpread;
  if (b_bytes <= kMallResident) return kRasterChunks;
  // a blocks round reads 16 A and 16 B panels
  if (16 * (panel + b_panel) <= ((int64_t)256 << 20)) return kRasterBlocks;
  return kRasterSpread;
}

// Packed launch grid (p.tiles_m, p.tiles_n, p.group_m, p.raster) of a
// checked call.
void packed_grid(Params& p, int algo) {
  p.tiles_m = (int)(packed::padded_product_rows(p.m) / packed::TM);
  p.tiles_n = (int)((p.n / 2) / packed::TN);
  p.group_m = group_m_setting();
  const int forced = raster_setting();
  p.raster = forced >= 0 ? forced : raster_for(p, algo, packed::TN);
}

// Depth below which a split's rounds are short enough that its two extra
// launches take much of the saving (a 128 x 128 Strassen product tile over
// K = 2048 is 235 MFLOP: 24 us at one CU's peak).
constexpr int64_t kSplitMinK = 2048;
// A K share keeps at least this many 32-deep K stages; a launch splits its
// tiles at most this many ways, and into no more shares than keep the
// workspace (shares x split tiles x 256 KB) within kSplitMaxBytes.
constexpr int kSplitMinStages = 16;
constexpr int kMaxKSplit = 16;
constexpr int64_t kSplitMaxBytes = (int64_t)1 << 30;

// Which tiles of a packed launch run as K shares. A launch runs one tile per
// CU and round: T tiles on C CUs make T / C whole rounds and a last round of
// r = T mod C (r = T for a launch under one round). Those r tiles can run as
// s shares of their K stages, s r workgroups in ceil(s r / C) rounds. In
// units of one full-K tile's time (about 0.03 K us on MI355X), the split
// round costs
//   ceil(s r / C) (1/s + f) + s r g,   f = 400 / K,  g = (5/3) / K:
// f is a workgroup's fixed prologue and epilogue (about 12 us), g the
// summing pass's read of one share of one tile (256 KB at about 5 TB/s).
// The cheapest s of 2 .. s_max splits when it costs under 0.95 of the
// unsplit round (1 + f). On 256 CUs a launch of 20 tiles over K = 25600
// splits 12 ways, 128 tiles two ways, a last round of 32 tiles at K = 8192
// five ways (the workspace bound), one of 224 tiles not at all. FP32
// partials, K below kSplitMinK and a whole last round keep every tile whole.
struct SplitPlan {
  int whole;   // tiles 0 .. whole - 1 run over full K, with the epilogue
  int split;   // tiles whole .. whole + split - 1 run as ksplit shares
  int ksplit;
};

double split_cost(int s, int r, int cus, int64_t k) {
  const double f = 400.0 / (double)k, g = (5.0 / 3.0) / (double)k;
  const int rounds = (s * r + cus - 1) / cus;
  return (double)rounds * (1.0 / (double)s + f) + (double)(s * r) * g;
}

int split_plan(const Params& p, SplitPlan* plan) {
  *plan = SplitPlan{p.tiles_m * p.tiles_n, 0, 1};
  if (p.partial || !split_setting() || p.k < kSplitMinK) return SMX_OK;
  int cus = 0;
  if (int rc = device_cus(&cus)) return rc;
  const int tiles = p.tiles_m * p.tiles_n;
  const int r = tiles % cus;
  if (r == 0) return SMX_OK;
  const int stages = (int)(p.k / (2 * packed::TK));
  const int64_t share_bytes = (int64_t)r * kSplitTileFloats * (int64_t)sizeof(float);
  const int s_max = (int)std::min<int64_t>(std::min(kMaxKSplit, stages / kSplitMinStages), kSplitMaxBytes / share_bytes);
  int best_s = 1;
  double best = 0.95 * split_cost(1, r, cus, p.k);
  for (int s = 2; s <= s_max; ++s) {
    const double c = split_cost(s, r, cus, p.k);
    if (c < best) {
      best = c;
      best_s = s;
    }
  }
  if (best_s > 1) *plan = SplitPlan{tiles - r, r, best_s};
  return SMX_OK;
}

int64_t split_bytes(const Params&, const SplitPlan& plan) {
  return (int64_t)plan.ksplit * plan.split * kSplitTileFloats * (int64_t)sizeof(float);
}

template <int kEpi>
int launch_fixup(const Params& p, const float* ws, int tiles, hipStream_t s) {
  hipLaunchKernelGGL(split_fixup<kEpi>, dim3((unsigned)(tiles * kFixupSlices)), dim3(256), 0, s, p, ws);
  return check_launch();
}

int launch_split_fixup(const Params& p, int epilogue, const float* ws, int tiles, hipStream_t s) {
  switch (epilogue) {
    case SMX_EPI_NONE: return launch_fixup<SMX_EPI_NONE>(p, ws, tiles, s);
    case SMX_EPI_SWIGLU: return launch_fixup<SMX_EPI_SWIGLU>(p, ws, tiles, s);
    case SMX_EPI_GEGLU: return launch_fixup<SMX_EPI_GEGLU>(p, ws, tiles, s);
    case SMX_EPI_RESIDUAL_ADD: return launch_fixup<SMX_EPI_RESIDUAL_ADD>(p, ws, tiles, s);
    case SMX_EPI_BIAS_ADD: return launch_fixup<SMX_EPI_BIAS_ADD>(p, ws, tiles, s);
    case SMX_EPI_QK_NORM_ROPE: return launch_fixup<SMX_EPI_QK_NORM_ROPE>(p, ws, tiles, s);
  }
  return fail(SMX_ERR_INVALID, "unknown epilogue %d", epilogue);
}

int launch_packed(const Params& p, int algo, int epilogue, hipStream_t s) {
  const bool thin = (p.bm / 2) % packed::TM != 0;
  if (algo == SMX_ALGO_STRASSEN)
    return thin ? launch_strassen<true>(p, epilogue, s) : launch_strassen<false>(p, epilogue, s);
  return thin ? launch_cubic<true>(p, epilogue, s) : launch_cubic<false>(p, epilogue, s);
}

// Whether a checked packed Strassen call asks for (SMX_FLAG_PRODUCT_MAJOR or
// SMX_FLAG_PRODUCT_MAJOR_ROUNDS) and can take the product-major kernel
// (kernel_pm.hpp): the classical formula, no FP32 partial, whole 128 x 256
// product tiles inside every (bm, bn) tile, K a multiple of 128, and an
// epilogue it fuses.
bool pm_eligible(const Params& p, const smx_gemm_desc& d) {
  if (!(d.flags & (SMX_FLAG_PRODUCT_MAJOR | SMX_FLAG_PRODUCT_MAJOR_ROUNDS))) return false;
  if (d.algo != SMX_ALGO_STRASSEN || d.b_layout != SMX_B_PACKED || p.partial) return false;
  if (p.formula != SMX_FORMULA_CLASSICAL || (p.bm / 2) % pm::TM || (p.bn / 2) % pm::TN) return false;
  if ((p.k / 32) % pm::kQuarters) return false;  // whole pipeline stages of 64 product-space k
  return d.epilogue == SMX_EPI_NONE || d.epilogue == SMX_EPI_SWIGLU || d.epilogue == SMX_EPI_GEGLU ||
         d.epilogue == SMX_EPI_RESIDUAL_ADD || d.epilogue == SMX_EPI_BIAS_ADD;
}

// Grid of a product-major launch: 128 x 256 product tiles, the tile order
// chosen from its packed operands as for the other packed kernels.
void pm_grid(Params& p) {
  p.tiles_m = (int)((p.m / 2) / pm::TM);
  p.tiles_n = (int)((p.n / 2) / pm::TN);
  p.group_m = group_m_setting();
  const int forced = raster_setting();
  p.raster = forced >= 0 ? forced : raster_for(p, SMX_ALGO_STRASSEN, pm::TN);
}

// Workspace of a product-major launch: two parked FP32 sets per workgroup.
int64_t pm_park_bytes(const Params& p) { return (int64_t)p.tiles_m * p.tiles_n * pm::kParkBytes; }

// Depth below which a SMX_FLAG_PRODUCT_MAJOR_ROUNDS call runs on the split
// kernel alone. The product-major kernel's per-tile costs (two mid-kernel
// epilogues, two parked sets) are fixed while its lead per unit of K is
// small: on whole rounds (8192 x K x 16384, one MI355X) it takes 15% longer
// than the split kernel at K = 1024, 3% at 2048, the same at 3072, 1% less
// at 4096, 1-2% at 5120 and 10% at 25600.
constexpr int64_t kPmRoundsMinK = 4096;

// Product-major tile columns that a SMX_FLAG_PRODUCT_MAJOR_ROUNDS call runs on
// the product-major kernel (q on its grid, pm_grid): the most whose tiles
// fill whole rounds of `cus` CUs (tiles_m columns a multiple of cus) and
// end on a bn tile boundary (a multiple of bn/2 / 256 columns); none below
// kPmRoundsMinK.
int pm_round_columns(const Params& q, int cus) {
  if (q.k < kPmRoundsMinK) return 0;
  const int per_bn = (int)((q.bn / 2) / pm::TN);
  const int per_round = cus / std::gcd(q.tiles_m, cus);
  const int step = std::lcm(per_bn, per_round);
  return q.tiles_n / step * step;
}

// The product-space columns pcol0 .. pcol0 + pcols - 1 of a checked packed
// Strassen call as a call of its own (pcol0 and pcols multiples of bn/2):
// B's packed tiles from pcol0 / 128 on, and C, residual and bias from
// physical column 2 pcol0 on (C from pcol0 for SwiGLU / GeGLU, whose output
// has N/2 columns). A tile's physical columns relative to its part are
// those it has in the whole call, so the parts store what the whole does.
Params column_part(const Params& p, int epilogue, int64_t pcol0, int64_t pcols) {
  Params q = p;
  q.n = 2 * pcols;
  // One packed B tile (128 product columns) is K/32 stages of the seven
  // operands' fragments (packed::Lay<7>::kStage bytes each).
  const int64_t tile_bytes = (p.k / (2 * packed::TK)) * packed::Lay<7>::kStage;
  q.b = reinterpret_cast<const uint16_t*>(reinterpret_cast<const uint8_t*>(p.b) + pcol0 / packed::TN * tile_bytes);
  const int64_t col = 2 * pcol0;
  const bool gated = epilogue == SMX_EPI_SWIGLU || epilogue == SMX_EPI_GEGLU;
  q.c = reinterpret_cast<uint8_t*>(p.c) + (gated ? pcol0 : col) * (p.out_f32 ? 4 : 2);
  if (p.residual) q.residual = reinterpret_cast<const uint8_t*>(p.residual) + col * (p.residual_f32 ? 4 : 2);
  if (p.bias) q.bias = reinterpret_cast<const uint8_t*>(p.bias) + col * (p.bias_f32 ? 4 : 2);
  return q;
}

// How a checked packed call runs: a head of product-major tile columns on the
// product-major kernel (every column with SMX_FLAG_PRODUCT_MAJOR, whole
// rounds with SMX_FLAG_PRODUCT_MAJOR_ROUNDS), then the rest on the split
// (or cubic) kernel, with that part's K split when a workspace is given.
struct Parts {
  int pm_cols = 0;    // product-major tile columns (0: no head)
  bool rest = true;   // whether a split-kernel part follows
  Params head{};      // on pm_grid
  Params rest_p{};    // on packed_grid
};

int plan_parts(const Params& p, const smx_gemm_desc& d, Parts* out) {
  Parts t;
  t.rest_p = p;
  if (pm_eligible(p, d)) {
    Params q = p;
    pm_grid(q);
    int cols = q.tiles_n;
    if (d.flags & SMX_FLAG_PRODUCT_MAJOR_ROUNDS) {
      int cus = 0;
      if (int rc = device_cus(&cus)) return rc;
      cols = pm_round_columns(q, cus);
    }
    if (cols == q.tiles_n) {
      t.pm_cols = cols;
      t.head = q;
      t.rest = false;
    } else if (cols > 0) {
      const int64_t pcols = (int64_t)cols * pm::TN;
      t.pm_cols = cols;
      t.head = column_part(p, d.epilogue, 0, pcols);
      pm_grid(t.head);
      t.rest_p = column_part(p, d.epilogue, pcols, p.n / 2 - pcols);
    }
  }
  if (t.rest) packed_grid(t.rest_p, d.algo);
  *out = t;
  return SMX_OK;
}

// Workspace bytes of a planned call: the head's parked sets and the rest's
// K shares (split_plan), which run one after the other on one stream and
// share the buffer.
int parts_workspace(const Parts& t, int64_t* bytes) {
  int64_t need = t.pm_cols ? pm_park_bytes(t.head) : 0;
  if (t.rest) {
    SplitPlan plan{};
    if (int rc = split_plan(t.rest_p, &plan)) return rc;
    if (plan.split) need = std::max(need, split_bytes(t.rest_p, plan));
  }
  *bytes = need;
  return SMX_OK;
}

// The workspace checks of a checked call, run before anything is launched
// (launch_gemm, and smx_gemm_noalloc before its packing pass): a
// product-major head needs its parked sets (and then the whole call's
// workspace); otherwise a given workspace must hold the K split's shares.
int check_workspace(const Params& p, const smx_gemm_desc& d) {
  if (d.b_layout != SMX_B_PACKED) return SMX_OK;
  Parts t;
  if (int rc = plan_parts(p, d, &t)) return rc;
  if (!t.pm_cols && !d.workspace) return SMX_OK;
  int64_t need = 0;
  if (int rc = parts_workspace(t, &need)) return rc;
  if (t.pm_cols && (!d.workspace || d.workspace_bytes < need))
    return fail(SMX_ERR_INVALID,
                "the product-major kernel needs workspace_bytes >= %lld (smx_gemm_workspace_bytes), got %lld",
                (long long)need, (long long)(d.workspace ? d.workspace_bytes : 0));
  if (d.workspace_bytes < need)
    return fail(SMX_ERR_INVALID, "workspace_bytes %lld is below the %lld this call needs (smx_gemm_workspace_bytes)",
                (long long)d.workspace_bytes, (long long)need);
  return SMX_OK;
}

int launch_rest(Params p, const smx_gemm_desc& d, hipStream_t s);

// A packed call: a product-major head (plan_parts) parks two partial sets
// per workgroup in the workspace; the rest runs as launch_rest says.
int launch_gemm(Params p, const smx_gemm_desc& d, hipStream_t s) {
  if (d.b_layout != SMX_B_PACKED)
    return d.algo == SMX_ALGO_STRASSEN ? dispatch_v1<7>(p, d.epilogue, s) : dispatch_v1<8>(p, d.epilogue, s);
  if (int rc = check_workspace(p, d)) return rc;
  Parts t;
  if (int rc = plan_parts(p, d, &t)) return rc;
  if (t.pm_cols) {
    Params q = t.head;
    q.park = d.workspace;
    if (int rc = launch_strassen_pm(q, d.epilogue, s)) return rc;
  }
  return t.rest ? launch_rest(t.rest_p, d, s) : SMX_OK;
}

// The split (or cubic) kernel's part of a packed call (on packed_grid), with
// tiles split over K when a workspace is given (smx_gemm_desc.workspace,
// split_plan): the whole tiles with the fused epilogue, then the split
// tiles' K shares into the workspace (FP32, no epilogue), then split_fixup,
// all on the caller's stream in that order.
int launch_rest(Params p, const smx_gemm_desc& d, hipStream_t s) {
  SplitPlan plan{p.tiles_m * p.tiles_n, 0, 1};
  if (d.workspace)
    if (int rc = split_plan(p, &plan)) return rc;
  if (!plan.split) return launch_packed(p, d.algo, d.epilogue, s);
  if (plan.whole > 0) {
    Params q = p;
    q.grid = plan.whole;
    if (int rc = launch_packed(q, d.algo, d.epilogue, s)) return rc;
  }
  Params h = p;
  h.c = d.workspace;
  h.out_f32 = 1;
  h.residual = h.bias = nullptr;
  h.rope_cos = h.rope_sin = nullptr;
  h.rope_scale = nullptr;
  h.grid = plan.ksplit * plan.split;
  h.ksplit = plan.ksplit;
  h.tile_base = plan.whole;
  h.split_stride = (int64_t)plan.split * kSplitTileFloats;
  if (int rc = launch_packed(h, d.algo, SMX_EPI_NONE, s)) return rc;
  Params f = p;
  f.ksplit = plan.ksplit;
  f.tile_base = plan.whole;
  f.split_stride = (int64_t)plan.split * kSplitTileFloats;
  return launch_split_fixup(f, d.epilogue, (const float*)d.workspace, plan.split, s);
}

// Device scratch of smx_gemm_noalloc: the packed activation of one call,
// at most kNoAllocScratchBytes. Each GPU the library runs on holds its own
// copy from module load until the process ends. Host code never passes the
// array's name to a kernel or a copy (on the host it is only a stand-in
// symbol): scratch_address() looks up the device address once per device,
// with that device current, and every use goes through that pointer.
constexpr size_t kNoAllocScratchBytes = (size_t)256 << 20;
__device__ __attribute__((aligned(256))) uint8_t scratch[kNoAllocScratchBytes];
// A non-null, 16-byte-aligned placeholder for the packed A while a
// descriptor is checked (never dereferenced or launched with).
const void* const kNoAllocScratchProbe = reinterpret_cast<const void*>((uintptr_t)256);

std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_address(void** out) {
  int device = -1;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return fail(SMX_ERR_LAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
  if (device < 0 || device >= kMaxDevices) return fail(SMX_ERR_UNSUPPORTED, "device %d out of range", device);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[device]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(SMX_ERR_LAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", device, hipGetErrorString(e));
    g_scratch_ptr[device] = ptr;
  }
  *out = g_scratch_ptr[device];
  return SMX_OK;
}

// qk_norm_rope's second pass (strassen_pallas.py:793-835) for head widths
// the fused epilogue does not take: one workgroup per (output row, column
// tile of bn). A tile half holds bn / head_dim heads of head_dim/2 columns;
// head h pairs its columns c of the first half (a) with the same columns of
// the second half (b). recip = 1 / sqrt((sum a^2 + sum b^2) / head_dim + eps)
// over the head; na = a recip scale[c], nb = b recip scale[bn/2 + c];
// out_a = na cos - nb sin, out_b = nb cos + na sin, with cos, sin [m, bn/2] at
// (row, c). Squares go to LDS ([a^2 | b^2], bn floats), one thread per head
// sums its segment (first half, then second, in column order), and the
// reciprocals ([bn / head_dim]) follow them in LDS.
__global__ __launch_bounds__(256) void qk_norm_rope_rows(const float* __restrict__ x, int64_t ldx,
                                                         const uint16_t* __restrict__ cos_t,
                                                         const uint16_t* __restrict__ sin_t,
                                                         const void* __restrict__ scale, int32_t dtypes, int32_t bn,
                                                         int32_t head_dim, float eps, void* __restrict__ out,
                                                         int64_t ldo) {
  extern __shared__ float sq[];
  const int64_t row = blockIdx.x;
  const int hn = bn / 2, seg = head_dim / 2, heads = hn / seg;
  const float* const xa = x + row * ldx + (int64_t)blockIdx.y * bn;
  const float* const xb = xa + hn;
  for (int c = threadIdx.x; c < hn; c += blockDim.x) {
    sq[c] = xa[c] * xa[c];
    sq[hn + c] = xb[c] * xb[c];
  }
  __syncthreads();
  float* const recip = sq + bn;
  const float inv_width = 1.0f / (float)head_dim;
  for (int h = threadIdx.x; h < heads; h += blockDim.x) {
    float ssa = 0.f, ssb = 0.f;
    for (int c = 0; c < seg; ++c) {
      ssa += sq[h * seg + c];
      ssb += sq[hn + h * seg + c];
    }
    recip[h] = 1.0f / sqrtf((ssa + ssb) * inv_width + eps);
  }
  __syncthreads();
  const int scale_f32 = dtypes & SMX_QK_SCALE_F32;
  const int64_t out0 = row * ldo + (int64_t)blockIdx.y * bn;
  for (int c = threadIdx.x; c < hn; c += blockDim.x) {
    const float r = recip[c / seg];
    const float na = xa[c] * r * load_vec(scale, scale_f32, c);
    const float nb = xb[c] * r * load_vec(scale, scale_f32, hn + c);
    const float cs = bf16_to_f32(cos_t[row * hn + c]), sn = bf16_to_f32(sin_t[row * hn + c]);
    const float oa = na * cs - nb * sn, ob = nb * cs + na * sn;
    if (dtypes & SMX_QK_OUT_F32) {
      reinterpret_cast<float*>(out)[out0 + c] = oa;
      reinterpret_cast<float*>(out)[out0 + hn + c] = ob;
    } else {
      reinterpret_cast<uint16_t*>(out)[out0 + c] = f32_to_bf16(oa);
      reinterpret_cast<uint16_t*>(out)[out0 + hn + c] = f32_to_bf16(ob);
    }
  }
}

}  // namespace
}  // namespace smx

using namespace smx;

extern "C" {

int smx_version(void) { return SMX_VERSION; }

const char* smx_last_error(void) { return g_error; }

int smx_tile_requirements(int32_t algo, int32_t epilogue, int32_t b_layout, int32_t flags, int32_t* tm, int32_t* tn,
                          int32_t* tk) {
  g_error[0] = 0;
  (void)epilogue;
  if (algo != SMX_ALGO_STRASSEN && algo != SMX_ALGO_CUBIC) return fail(SMX_ERR_INVALID, "algo must be 7 or 8");
  if (b_layout != SMX_B_KCONTIG && b_layout != SMX_B_PACKED) return fail(SMX_ERR_INVALID, "unknown b_layout");
  if (flags) return fail(SMX_ERR_INVALID, "flags must be 0");
  int32_t a, b, c;
  tile_of_path(b_layout == SMX_B_PACKED, &a, &b, &c);
  if (tm) *tm = a;
  if (tn) *tn = b;
  if (tk) *tk = c;
  return SMX_OK;
}

int smx_packed_bytes(int32_t algo, int64_t rows, int64_t k, int64_t* bytes) {
  g_error[0] = 0;
  if (algo != SMX_ALGO_STRASSEN && algo != SMX_ALGO_CUBIC) return fail(SMX_ERR_INVALID, "algo must be 7 or 8");
  if (rows <= 0 || k <= 0 || rows % 2 || k % 2) return fail(SMX_ERR_INVALID, "rows and k must be positive and even");
  if (!bytes) return fail(SMX_ERR_INVALID, "null output");
  *bytes = packed::padded_product_rows(rows) * (k / 2) * packed::nops_of(algo) * 2;
  return SMX_OK;
}

int smx_pack_operand(int32_t algo, int32_t formula, int32_t block_permutation, int32_t side, int64_t rows, int64_t k,
                     const void* src, int32_t src_dtype, int32_t passes, int64_t ld, int32_t tile_rows,
                     int32_t bk, const int32_t* panels, int64_t src_k, void* out, void* stream) {
  g_error[0] = 0;
  if (algo != SMX_ALGO_STRASSEN && algo != SMX_ALGO_CUBIC) return fail(SMX_ERR_INVALID, "algo must be 7 or 8");
  if (int rc = check_variant(algo, formula, block_permutation)) return rc;
  if (side != SMX_SIDE_LHS && side != SMX_SIDE_RHS && side != SMX_SIDE_LHS_T)
    return fail(SMX_ERR_INVALID, "side must be LHS (0), RHS (1) or LHS_T (2)");
  if (rows <= 0 || k <= 0 || tile_rows <= 0 || bk <= 0 || rows % tile_rows || k % bk)
    return fail(SMX_ERR_INVALID, "packing needs rows %% tile_rows == 0 and K %% bk == 0");
  // A's tile rows may be thin (ThinRows); B's must fill whole product tiles.
  const int32_t row_granule = side == SMX_SIDE_RHS ? 2 * packed::TN : 2 * kThinRowGranule;
  if (tile_rows % row_granule || bk % (2 * packed::kKGranule))
    return fail(SMX_ERR_UNSUPPORTED, "packed tiles need %s %% %d == 0 and bk %% %d == 0 (got %d, %d)",
                side == SMX_SIDE_RHS ? "bn" : "bm", row_granule, 2 * packed::kKGranule, tile_rows, bk);
  if (!src || !out) return fail(SMX_ERR_INVALID, "null pointer");
  if (!aligned16(src) || !aligned16(out)) return fail(SMX_ERR_INVALID, "pointers must be 16-byte aligned");
  if (src_dtype != SMX_DTYPE_BF16 && src_dtype != SMX_DTYPE_F32)
    return fail(SMX_ERR_INVALID, "src_dtype must be SMX_DTYPE_BF16 (0) or SMX_DTYPE_F32 (1), got %d", src_dtype);
  const bool src_f32 = src_dtype == SMX_DTYPE_F32;
  if (passes != 1 && passes != 3 && passes != 6)
    return fail(SMX_ERR_INVALID, "passes must be 1, 3 or 6, got %d", passes);
  if (passes > 1 && !src_f32) return fail(SMX_ERR_INVALID, "multi-pass products need a float32 source");
  if (k % ((int64_t)passes * bk))
    return fail(SMX_ERR_INVALID, "the packed K (%lld) must hold whole passes of bk panels", (long long)k);
  if (!panels) src_k = k / passes;
  if (src_k <= 0 || src_k % bk || src_k / bk >= ((int64_t)1 << 31))
    return fail(SMX_ERR_INVALID, "the source K (%lld) must be a positive multiple of bk", (long long)src_k);
  // Row-major sources are read 16 bytes at a time: rows must stay 16-byte aligned.
  if (side == SMX_SIDE_LHS_T ? ld < rows : (ld < src_k || ld % (src_f32 ? 4 : 8)))
    return fail(SMX_ERR_INVALID, side == SMX_SIDE_LHS_T ? "ld must be >= rows for a transposed A"
                                                        : "ld must be >= K and a multiple of 16 bytes");
  const void* s16 = src;
  uint8_t* o8 = (uint8_t*)out;
  hipStream_t st = (hipStream_t)stream;
  const int32_t sp = (int32_t)(src_k / bk);
  if (algo == SMX_ALGO_STRASSEN) {
    if (side == SMX_SIDE_LHS) return launch_pack<7, 0>(s16, src_f32, ld, rows, k, tile_rows, bk, formula, block_permutation, panels, sp, passes, o8, st);
    if (side == SMX_SIDE_RHS) return launch_pack<7, 1>(s16, src_f32, ld, rows, k, tile_rows, bk, formula, block_permutation, panels, sp, passes, o8, st);
    return launch_pack<7, 2>(s16, src_f32, ld, rows, k, tile_rows, bk, formula, block_permutation, panels, sp, passes, o8, st);
  }
  if (side == SMX_SIDE_LHS) return launch_pack<8, 0>(s16, src_f32, ld, rows, k, tile_rows, bk, formula, block_permutation, panels, sp, passes, o8, st);
  if (side == SMX_SIDE_RHS) return launch_pack<8, 1>(s16, src_f32, ld, rows, k, tile_rows, bk, formula, block_permutation, panels, sp, passes, o8, st);
  return launch_pack<8, 2>(s16, src_f32, ld, rows, k, tile_rows, bk, formula, block_permutation, panels, sp, passes, o8, st);
}

int smx_gemm(const smx_gemm_desc* d, const void* a, const void* b, void* c, const void* residual, const void* bias,
             const void* rope_cos, const void* rope_sin, const void* rope_scale, void* stream) {
  g_error[0] = 0;
  Params p{};
  if (int rc = gemm_params(d, a, b, c, residual, bias, rope_cos, rope_sin, rope_scale, p)) return rc;
  return launch_gemm(p, *d, (hipStream_t)stream);
}

int smx_gemm_workspace_bytes(const smx_gemm_desc* d, int64_t* bytes) {
  g_error[0] = 0;
  if (!bytes) return fail(SMX_ERR_INVALID, "null output");
  *bytes = 0;
  if (!d) return fail(SMX_ERR_INVALID, "null descriptor");
  // The descriptor is checked as smx_gemm checks it, with placeholders for
  // the operand pointers (never dereferenced). A row-major A with a packed B
  // (smx_gemm_noalloc's descriptor) is sized as the packed call it becomes.
  smx_gemm_desc desc = *d;
  if (desc.a_layout == SMX_A_ROWMAJOR && desc.b_layout == SMX_B_PACKED) desc.a_layout = SMX_A_PACKED;
  d = &desc;
  const void* x = kNoAllocScratchProbe;
  Params p{};
  if (int rc = gemm_params(d, x, x, const_cast<void*>(x), x, x, x, x, x, p)) return rc;
  if (d->b_layout != SMX_B_PACKED) return SMX_OK;
  Parts t;
  if (int rc = plan_parts(p, *d, &t)) return rc;
  return parts_workspace(t, bytes);
}

int smx_gemm_noalloc(const smx_gemm_desc* d, const void* a, const void* b, void* c, const void* residual,
                     const void* bias, const void* rope_cos, const void* rope_sin, const void* rope_scale,
                     void* stream) {
  g_error[0] = 0;
  if (!d) return fail(SMX_ERR_INVALID, "null descriptor");
  if (d->a_layout != SMX_A_ROWMAJOR || d->b_layout != SMX_B_PACKED)
    return fail(SMX_ERR_INVALID,
                "smx_gemm_noalloc takes a row-major bf16 A (SMX_A_ROWMAJOR) and a packed B (SMX_B_PACKED)");
  if (d->partial) return fail(SMX_ERR_UNSUPPORTED, "smx_gemm_noalloc takes no FP32 partial");
  if (!a) return fail(SMX_ERR_INVALID, "null operand pointer");
  // Every check of the GEMM runs on the descriptor the packed call will see,
  // before anything is launched; the scratch stands in for the packed A.
  smx_gemm_desc packed = *d;
  packed.a_layout = SMX_A_PACKED;
  Params p{};
  if (int rc = gemm_params(&packed, kNoAllocScratchProbe, b, c, residual, bias, rope_cos, rope_sin, rope_scale, p))
    return rc;
  if (d->lda < d->k || d->lda % 8) return fail(SMX_ERR_INVALID, "lda must be >= K and a multiple of 8 elements");
  if (!aligned16(a)) return fail(SMX_ERR_INVALID, "A must be 16-byte aligned");
  const int64_t bytes = packed::padded_product_rows(d->m) * (d->k / 2) * packed::nops_of(d->algo) * 2;
  if (bytes > (int64_t)kNoAllocScratchBytes)
    return fail(SMX_ERR_UNSUPPORTED,
                "smx_gemm_noalloc packs A into a %lld-byte device scratch; this call needs %lld bytes "
                "(M*K <= %lld for algo %d)",
                (long long)kNoAllocScratchBytes, (long long)bytes,
                (long long)(kNoAllocScratchBytes / (packed::nops_of(d->algo) / 2.0)), d->algo);
  if (int rc = check_workspace(p, packed)) return rc;
  void* scratch_ptr = nullptr;
  if (int rc = scratch_address(&scratch_ptr)) return rc;
  if (int rc = smx_pack_operand(d->algo, d->formula, d->block_permutation, SMX_SIDE_LHS, d->m, d->k, a,
                                SMX_DTYPE_BF16, 1, d->lda, d->bm, d->bk, nullptr, 0, scratch_ptr, stream))
    return rc;
  p.a = (const uint16_t*)scratch_ptr;
  return launch_gemm(p, packed, (hipStream_t)stream);
}

int smx_norm_residual_add(int64_t m, int64_t n, const float* x, int64_t ldx, const void* residual, int64_t ldr,
                          const void* scale, int32_t dtypes, float eps, void* out, int64_t ldo, void* stream) {
  g_error[0] = 0;
  if (m <= 0 || n <= 0) return fail(SMX_ERR_INVALID, "empty problem m=%lld n=%lld", (long long)m, (long long)n);
  if (!x || !residual || !scale || !out) return fail(SMX_ERR_INVALID, "null pointer");
  if (ldx < n || ldr < n || ldo < n) return fail(SMX_ERR_INVALID, "row strides must be >= n");
  if (m >= ((int64_t)1 << 31)) return fail(SMX_ERR_UNSUPPORTED, "too many rows");
  if (dtypes & ~(SMX_NRA_SCALE_F32 | SMX_NRA_RESIDUAL_F32 | SMX_NRA_OUT_F32))
    return fail(SMX_ERR_INVALID, "unknown dtype bits 0x%x", dtypes);
  hipLaunchKernelGGL(norm_residual_rows, dim3((unsigned)m), dim3(256), 0, (hipStream_t)stream, x, ldx,
                     residual, ldr, scale, dtypes, eps, n, out, ldo);
  return check_launch();
}

int smx_qk_norm_rope(int64_t m, int64_t n, const float* x, int64_t ldx, const void* rope_cos, const void* rope_sin,
                     const void* rope_scale, int32_t dtypes, int32_t bn, int32_t head_dim, float eps, void* out,
                     int64_t ldo, void* stream) {
  g_error[0] = 0;
  if (m <= 0 || n <= 0) return fail(SMX_ERR_INVALID, "empty problem m=%lld n=%lld", (long long)m, (long long)n);
  if (!x || !rope_cos || !rope_sin || !rope_scale || !out) return fail(SMX_ERR_INVALID, "null pointer");
  if (head_dim <= 0 || head_dim % 2 || bn <= 0 || bn % (2 * head_dim))
    return fail(SMX_ERR_INVALID, "qk_norm_rope needs an even head_dim and bn a multiple of 2*head_dim (bn=%d, "
                "head_dim=%d)", bn, head_dim);
  if (n % bn) return fail(SMX_ERR_INVALID, "N=%lld is not divisible by bn=%d", (long long)n, bn);
  if (ldx < n || ldo < n) return fail(SMX_ERR_INVALID, "row strides must be >= n");
  if (dtypes & ~(SMX_QK_SCALE_F32 | SMX_QK_OUT_F32)) return fail(SMX_ERR_INVALID, "unknown dtype bits 0x%x", dtypes);
  // LDS: the tile's bn squares and its bn / head_dim reciprocals.
  const int64_t lds = ((int64_t)bn + bn / head_dim) * 4;
  if (lds > 64 * 1024)
    return fail(SMX_ERR_UNSUPPORTED, "bn=%d: the row pass holds bn + bn/head_dim floats in at most 64 KiB of LDS", bn);
  if (m >= ((int64_t)1 << 31) || n / bn >= 65536) return fail(SMX_ERR_UNSUPPORTED, "too many rows or tiles");
  hipLaunchKernelGGL(qk_norm_rope_rows, dim3((unsigned)m, (unsigned)(n / bn)), dim3(256), (unsigned)lds,
                     (hipStream_t)stream, x, ldx, (const uint16_t*)rope_cos, (const uint16_t*)rope_sin, rope_scale,
                     dtypes, bn, head_dim, eps, out, ldo);
  return check_launch();
}

}  // extern "C"
