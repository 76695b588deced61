// Instantiations: i8 GEMM, 16-bit dequant epilogues.
#include "gemm_kernels.hpp"

namespace d3 {
template hipError_t launch_epi<kInt8, kEpiDequant, kBF16>(GemmParams, int, hipStream_t);
template hipError_t launch_epi<kInt8, kEpiDequant, kF16>(GemmParams, int, hipStream_t);
}  // namespace d3
