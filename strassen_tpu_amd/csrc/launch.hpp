// Launchers of the packed-operand GEMM kernels, shared by the C ABI's
// translation unit (strassen_gemm.hip) and the translation units that
// instantiate the kernels (gemm_strassen*.hip, gemm_cubic*.hip). Each kernel
// is instantiated, registered and launched in exactly one translation unit;
// the units compile in parallel.
#pragma once

#include "common.hpp"

namespace smx {

// Records the message of a failing call (smx_last_error) and returns code.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

inline int check_launch() {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SMX_ERR_LAUNCH, "kernel launch: %s", hipGetErrorString(e));
  return SMX_OK;
}

// Dynamic LDS of `kern` raised to `bytes`, then one launch of `blocks`
// workgroups of kThreads on `stream`.
template <class K>
int launch_kernel(K kern, const Params& p, int blocks, int lds, hipStream_t stream) {
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e != hipSuccess) return fail(SMX_ERR_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(e));
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(kThreads), lds, stream, p);
  return check_launch();
}

// The Strassen (product-split) and cubic GEMMs on packed operands, for the
// epilogue `epilogue`; p.tiles_m, p.tiles_n and p.group_m are set. kThin:
// bm/2 is not a multiple of the 128-row product tile (ThinRows).
template <bool kThin>
int launch_strassen(const Params& p, int epilogue, hipStream_t stream);
template <bool kThin>
int launch_cubic(const Params& p, int epilogue, hipStream_t stream);

// The product-major Strassen kernel (kernel_pm.hpp) on packed operands:
// 128 x 256 product-space tiles, p.tiles_n counted in those, p.park set.
int launch_strassen_pm(const Params& p, int epilogue, hipStream_t stream);

extern template int launch_strassen<false>(const Params&, int, hipStream_t);
extern template int launch_strassen<true>(const Params&, int, hipStream_t);
extern template int launch_cubic<false>(const Params&, int, hipStream_t);
extern template int launch_cubic<true>(const Params&, int, hipStream_t);

}  // namespace smx
