// The Strassen (product-split) kernels, tilings whose bm/2 is a multiple of
// 128: instantiated, registered and launched here (launch.hpp).
#include "gemm_launch.hpp"

template int smx::launch_strassen<false>(const smx::Params&, int, hipStream_t);
