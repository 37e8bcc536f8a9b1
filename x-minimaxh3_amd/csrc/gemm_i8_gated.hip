// int8 GEMM kernels instantiated for: EPI_GATED / BF16T, EPI_GATED / F16T.
#include "gemm_i8_kernels.hpp"

namespace xmh3 {
XMH3_INSTANTIATE_GEMM(EPI_GATED, BF16T)
XMH3_INSTANTIATE_GEMM(EPI_GATED, F16T)
}  // namespace xmh3
