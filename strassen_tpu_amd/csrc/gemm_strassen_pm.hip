// The product-major Strassen kernels (kernel_pm.hpp): instantiated,
// registered and launched here (launch.hpp).
#include "kernel_pm.hpp"
#include "launch.hpp"

namespace smx {

template <int kEpi>
int launch_pm_epilogue(const Params& p, hipStream_t stream) {
  return launch_kernel(pm::gemm_pm<kEpi>, p, p.tiles_m * p.tiles_n, pm::kLds, stream);
}

int launch_strassen_pm(const Params& p, int epilogue, hipStream_t s) {
  switch (epilogue) {
    case SMX_EPI_NONE: return launch_pm_epilogue<SMX_EPI_NONE>(p, s);
    case SMX_EPI_SWIGLU: return launch_pm_epilogue<SMX_EPI_SWIGLU>(p, s);
    case SMX_EPI_GEGLU: return launch_pm_epilogue<SMX_EPI_GEGLU>(p, s);
    case SMX_EPI_RESIDUAL_ADD: return launch_pm_epilogue<SMX_EPI_RESIDUAL_ADD>(p, s);
    case SMX_EPI_BIAS_ADD: return launch_pm_epilogue<SMX_EPI_BIAS_ADD>(p, s);
  }
  return fail(SMX_ERR_INVALID, "the product-major kernel takes no epilogue %d", epilogue);
}

}  // namespace smx
