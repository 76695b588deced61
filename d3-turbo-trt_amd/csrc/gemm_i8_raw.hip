// Instantiations: i8 GEMM, raw accumulators and fp32 dequant.
#include "gemm_kernels.hpp"

namespace d3 {
template hipError_t launch_epi<kInt8, kEpiRaw, kF32>(GemmParams, int, hipStream_t);
template hipError_t launch_epi<kInt8, kEpiDequant, kF32>(GemmParams, int, hipStream_t);
}  // namespace d3
