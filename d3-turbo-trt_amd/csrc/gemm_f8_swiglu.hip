// Instantiations: f8 GEMM, SwiGLU epilogue, bf16 output.
#include "gemm_kernels.hpp"

namespace d3 {
template hipError_t launch_epi<kFp8, kEpiSwiGLU, kBF16>(GemmParams, int, hipStream_t);
}  // namespace d3
