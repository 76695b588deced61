// Instantiations: f8 GEMM, SwiGLU epilogue, fp16 and fp32 outputs.
#include "gemm_kernels.hpp"

namespace d3 {
template hipError_t launch_epi<kFp8, kEpiSwiGLU, kF16>(GemmParams, int, hipStream_t);
template hipError_t launch_epi<kFp8, kEpiSwiGLU, kF32>(GemmParams, int, hipStream_t);
}  // namespace d3
