// W8A8 GEMM dispatch: mode / epilogue / output dtype -> the kernel family
// instantiated in gemm_<mode>_<epilogue>.hip (the kernels themselves are in
// gemm_kernels.hpp; one translation unit per family keeps the build parallel).
#include "common.hpp"
#include "kernels.hpp"

namespace d3 {

template <int MODE, int EPI, int OUT>
hipError_t launch_epi(GemmParams p, int tile, hipStream_t st);

#define D3_EXTERN_EPI(MODE)                                   \
  extern template hipError_t launch_epi<MODE, kEpiRaw, kF32>(GemmParams, int, hipStream_t);       \
  extern template hipError_t launch_epi<MODE, kEpiDequant, kBF16>(GemmParams, int, hipStream_t);  \
  extern template hipError_t launch_epi<MODE, kEpiDequant, kF16>(GemmParams, int, hipStream_t);   \
  extern template hipError_t launch_epi<MODE, kEpiDequant, kF32>(GemmParams, int, hipStream_t);   \
  extern template hipError_t launch_epi<MODE, kEpiSwiGLU, kBF16>(GemmParams, int, hipStream_t);   \
  extern template hipError_t launch_epi<MODE, kEpiSwiGLU, kF16>(GemmParams, int, hipStream_t);    \
  extern template hipError_t launch_epi<MODE, kEpiSwiGLU, kF32>(GemmParams, int, hipStream_t);    \
  extern template hipError_t launch_epi<MODE, kEpiResidual, kBF16>(GemmParams, int, hipStream_t); \
  extern template hipError_t launch_epi<MODE, kEpiResidual, kF16>(GemmParams, int, hipStream_t);  \
  extern template hipError_t launch_epi<MODE, kEpiResidual, kF32>(GemmParams, int, hipStream_t);
D3_EXTERN_EPI(kInt8)
D3_EXTERN_EPI(kFp8)
#undef D3_EXTERN_EPI

template <int MODE>
static hipError_t launch_mode(GemmParams p, int epi, int out_dt, int tile, hipStream_t st) {
  switch (epi) {
    case kEpiRaw: return launch_epi<MODE, kEpiRaw, kF32>(p, tile, st);
    case kEpiDequant:
      if (out_dt == kBF16) return launch_epi<MODE, kEpiDequant, kBF16>(p, tile, st);
      if (out_dt == kF16) return launch_epi<MODE, kEpiDequant, kF16>(p, tile, st);
      return launch_epi<MODE, kEpiDequant, kF32>(p, tile, st);
    case kEpiSwiGLU:
      if (out_dt == kBF16) return launch_epi<MODE, kEpiSwiGLU, kBF16>(p, tile, st);
      if (out_dt == kF16) return launch_epi<MODE, kEpiSwiGLU, kF16>(p, tile, st);
      return launch_epi<MODE, kEpiSwiGLU, kF32>(p, tile, st);
    case kEpiResidual:
      if (out_dt == kBF16) return launch_epi<MODE, kEpiResidual, kBF16>(p, tile, st);
      if (out_dt == kF16) return launch_epi<MODE, kEpiResidual, kF16>(p, tile, st);
      return launch_epi<MODE, kEpiResidual, kF32>(p, tile, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_gemm(int mode, GemmParams p, int epi, int out_dt, int tile, hipStream_t st) {
  if (p.M == 0 || p.N == 0) return hipSuccess;
  return mode == kInt8 ? launch_mode<kInt8>(p, epi, out_dt, tile, st) : launch_mode<kFp8>(p, epi, out_dt, tile, st);
}

}  // namespace d3
