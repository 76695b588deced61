// Instantiations: i8 GEMM, residual epilogue, bf16 output.
#include "gemm_kernels.hpp"

namespace d3 {
template hipError_t launch_epi<kInt8, kEpiResidual, kBF16>(GemmParams, int, hipStream_t);
}  // namespace d3
