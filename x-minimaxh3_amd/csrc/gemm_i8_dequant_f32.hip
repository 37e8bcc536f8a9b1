// int8 GEMM kernels instantiated for: EPI_DEQUANT / F32T, EPI_INT32 / F32T.
#include "gemm_i8_kernels.hpp"

namespace xmh3 {
XMH3_INSTANTIATE_GEMM(EPI_DEQUANT, F32T)
XMH3_INSTANTIATE_GEMM(EPI_INT32, F32T)
}  // namespace xmh3
