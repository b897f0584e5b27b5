// Definitions of launch_strassen / launch_cubic (launch.hpp), included by the
// translation units that instantiate them.
#pragma once

#include "kernel_split.hpp"
#include "launch.hpp"

namespace smx {

// The epilogue's quadrant source (the Strassen formula, or the cubic with or
// without a partial product) is a kernel template argument, so every
// epilogue is straight-line code; the block permutation is applied by
// addressing at run time. The stage ring, then the epilogue's staging tiles,
// share the LDS.
template <bool kThin, int kEpi>
int launch_strassen_epilogue(const Params& p, hipStream_t stream) {
  constexpr int epi_lds = kEpiLds<kEpi, 64, 64>;
  constexpr int lds = split::Ring::kBytes > epi_lds ? split::Ring::kBytes : epi_lds;
  void (*kern)(Params);
  if (p.formula == SMX_FORMULA_DUAL) {
    kern = split::gemm_split<kEpi, kQuadDual, kThin>;
  } else if (p.formula == SMX_FORMULA_POWERS) {
    if constexpr (kEpi == SMX_EPI_NONE)
      kern = split::gemm_split<SMX_EPI_NONE, kQuadPowers, kThin>;
    else
      return fail(SMX_ERR_INVALID, "fused epilogues require a quadrant-basis formula");
  } else {
    kern = split::gemm_split<kEpi, kQuadClassical, kThin>;
  }
  return launch_kernel(kern, p, p.grid > 0 ? p.grid : p.tiles_m * p.tiles_n, lds, stream);
}

template <bool kThin, int kEpi>
int launch_cubic_epilogue(const Params& p, hipStream_t stream) {
  constexpr int epi_lds = kEpiLds<kEpi, 64, 64>;
  constexpr int lds = packed::Lay<8>::kLds > epi_lds ? packed::Lay<8>::kLds : epi_lds;
  void (*kern)(Params) = p.partial ? packed::gemm_packed<8, kEpi, kQuadCubicPartial, 3, kThin>
                                   : packed::gemm_packed<8, kEpi, kQuadCubic, 3, kThin>;
  return launch_kernel(kern, p, p.grid > 0 ? p.grid : p.tiles_m * p.tiles_n, lds, stream);
}

template <bool kThin>
int launch_strassen(const Params& p, int epilogue, hipStream_t s) {
  switch (epilogue) {
    case SMX_EPI_NONE: return launch_strassen_epilogue<kThin, SMX_EPI_NONE>(p, s);
    case SMX_EPI_SWIGLU: return launch_strassen_epilogue<kThin, SMX_EPI_SWIGLU>(p, s);
    case SMX_EPI_GEGLU: return launch_strassen_epilogue<kThin, SMX_EPI_GEGLU>(p, s);
    case SMX_EPI_RESIDUAL_ADD: return launch_strassen_epilogue<kThin, SMX_EPI_RESIDUAL_ADD>(p, s);
    case SMX_EPI_BIAS_ADD: return launch_strassen_epilogue<kThin, SMX_EPI_BIAS_ADD>(p, s);
    case SMX_EPI_QK_NORM_ROPE: return launch_strassen_epilogue<kThin, SMX_EPI_QK_NORM_ROPE>(p, s);
  }
  return fail(SMX_ERR_INVALID, "unknown epilogue %d", epilogue);
}

template <bool kThin>
int launch_cubic(const Params& p, int epilogue, hipStream_t s) {
  switch (epilogue) {
    case SMX_EPI_NONE: return launch_cubic_epilogue<kThin, SMX_EPI_NONE>(p, s);
    case SMX_EPI_SWIGLU: return launch_cubic_epilogue<kThin, SMX_EPI_SWIGLU>(p, s);
    case SMX_EPI_GEGLU: return launch_cubic_epilogue<kThin, SMX_EPI_GEGLU>(p, s);
    case SMX_EPI_RESIDUAL_ADD: return launch_cubic_epilogue<kThin, SMX_EPI_RESIDUAL_ADD>(p, s);
    case SMX_EPI_BIAS_ADD: return launch_cubic_epilogue<kThin, SMX_EPI_BIAS_ADD>(p, s);
    case SMX_EPI_QK_NORM_ROPE: return launch_cubic_epilogue<kThin, SMX_EPI_QK_NORM_ROPE>(p, s);
  }
  return fail(SMX_ERR_INVALID, "unknown epilogue %d", epilogue);
}

}  // namespace smx
