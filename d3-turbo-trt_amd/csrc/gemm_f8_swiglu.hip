// Instantiations: f8 GEMM, swiglu epilogue.
#include "gemm_kernels.hpp"

namespace d3 {
template hipError_t launch_epi<kFp8, kEpiSwiGLU, kBF16>(GemmParams, int, hipStream_t);
template hipError_t launch_epi<kFp8, kEpiSwiGLU, kF16>(GemmParams, int, hipStream_t);
template hipError_t launch_epi<kFp8, kEpiSwiGLU, kF32>(GemmParams, int, hipStream_t);
}  // namespace d3
