// The matched cubic kernels, tilings whose bm/2 is a multiple of 128:
// instantiated, registered and launched here (launch.hpp).
#include "gemm_launch.hpp"

template int smx::launch_cubic<false>(const smx::Params&, int, hipStream_t);
