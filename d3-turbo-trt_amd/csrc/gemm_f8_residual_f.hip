// Instantiations: f8 GEMM, residual epilogue, fp16 and fp32 outputs.
#include "gemm_kernels.hpp"

namespace d3 {
template hipError_t launch_epi<kFp8, kEpiResidual, kF16>(GemmParams, int, hipStream_t);
template hipError_t launch_epi<kFp8, kEpiResidual, kF32>(GemmParams, int, hipStream_t);
}  // namespace d3
