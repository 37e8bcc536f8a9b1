// int8 GEMM kernels instantiated for: EPI_DEQUANT / F16T.
#include "gemm_i8_kernels.hpp"

namespace xmh3 {
XMH3_INSTANTIATE_GEMM(EPI_DEQUANT, F16T)
}  // namespace xmh3
