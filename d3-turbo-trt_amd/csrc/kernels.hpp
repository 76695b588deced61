// Host-side launch interface shared by the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace d3 {

struct GemmParams {
  const uint8_t* a;
  int64_t lda;
  const float* a_scale;
  const uint8_t* w;
  int64_t ldw;
  const float* w_scale;
  int64_t M, N, K;
  void* out;
  int64_t ldo;
  const void* res;
  int64_t ldr;
  float* row_amax;
  const int32_t* row_map;
  int vec;  // output, residual and channel scales allow 4-element vector access
  int tiles_m, tiles_n;
};

hipError_t launch_quant_rows(int mode, int dt, const void* x, int64_t ldx, int64_t M, int64_t K, void* q,
                             int64_t ldq, float* scale, bool vec, hipStream_t st);
hipError_t launch_quant_rows_amax(int mode, int dt, const void* h, int64_t ldh, const float* amax, int64_t M,
                                  int64_t K, void* q, int64_t ldq, float* scale, hipStream_t st);
hipError_t launch_rmsnorm_quant(int mode, int dt, int dtw, const void* x, int64_t ldx, const void* w, int64_t M,
                                int64_t K, float eps, int zc, void* q, int64_t ldq, float* scale, void* normed,
                                int64_t ldn, float* clear_amax, hipStream_t st);
// Packed-row offsets of a ragged batch, passed by value in the kernel arguments:
// segment b owns packed rows [off[b], off[b + 1]).
constexpr int kMaxSegments = 256;
struct SegOffsets {
  int32_t off[kMaxSegments + 1];
};

hipError_t launch_quant_ragged(int mode, int dt, int out_es, const void* x, int64_t ldx, const SegOffsets& segs,
                               int64_t nseg, int64_t width, int64_t K, void* q, int64_t ldq, float* scale,
                               int32_t* row_map, void* out, int64_t ldo, int64_t N, hipStream_t st);
hipError_t launch_gemm(int mode, GemmParams p, int epi, int out_dt, int tile, hipStream_t st);

constexpr int64_t kMaxVecK = 32 * 512;  // longest row the one-pass quant kernels hold in registers

}  // namespace d3
