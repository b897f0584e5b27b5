// The Strassen (product-split) kernels, thin tilings (bm/2 not a multiple of
// 128): instantiated, registered and launched here (launch.hpp).
#include "gemm_launch.hpp"

template int smx::launch_strassen<true>(const smx::Params&, int, hipStream_t);
