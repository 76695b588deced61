// Shared definitions for the gfx950 W8A8 Linear kernels.
//
// Numerics that every kernel here keeps (they are what makes the INT8 path
// bit-exact against the reference's quantization, d3trt/model/quant.py:77-100):
//   * fp32 division and sqrt are correctly rounded (hipcc's default
//     -fhip-fp32-correctly-rounded-divide-sqrt; no fast-math anywhere);
//   * floating-point contraction is off (-ffp-contract=off), so a*b+c is two
//     roundings, as in the eager torch chain;
//   * rounding to integer is round-half-to-even (rintf), as torch.round;
//   * bf16/fp16 conversions are round-to-nearest-even.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace d3 {

enum Mode : int { kInt8 = 0, kFp8 = 1 };
enum DType : int { kBF16 = 0, kF16 = 1, kF32 = 2 };
enum Epilogue : int { kEpiDequant = 0, kEpiRaw = 1, kEpiSwiGLU = 2, kEpiResidual = 3 };

constexpr float kInt8Max = 127.0f;
constexpr float kFp8Max = 448.0f;
constexpr float kAmaxFloor = 1e-12f;  // quant.py:34, as the fp32 value torch compares against

typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

// ---- scalar conversions -----------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
  return __uint_as_float(b << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);  // v_cvt_pk_bf16_f32, RNE
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  // Materialize the fp32 value first: without the barrier the compiler folds
  // fptrunc(fmul(a, b)) into v_fma_mixlo_f16, which rounds the exact product
  // to fp16 once instead of fp32-then-fp16 as the eager chain does.
  asm volatile("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ float bf16_round(float f) {  // fp32 -> bf16 -> fp32
  return bf16_bits_to_f32(f32_to_bf16_bits(f));
}

template <int DT>
__device__ __forceinline__ float load_elem(const void* p, int64_t i) {
  if constexpr (DT == kBF16) return bf16_bits_to_f32(((const uint16_t*)p)[i]);
  else if constexpr (DT == kF16) return f16_bits_to_f32(((const uint16_t*)p)[i]);
  else return ((const float*)p)[i];
}
template <int DT>
__device__ __forceinline__ void store_elem(void* p, int64_t i, float v) {
  if constexpr (DT == kBF16) ((uint16_t*)p)[i] = f32_to_bf16_bits(v);
  else if constexpr (DT == kF16) ((uint16_t*)p)[i] = f32_to_f16_bits(v);
  else ((float*)p)[i] = v;
}
// value as stored in DT and read back (the rounding a torch tensor of that dtype applies)
template <int DT>
__device__ __forceinline__ float round_to(float v) {
  if constexpr (DT == kBF16) return bf16_round(v);
  else if constexpr (DT == kF16) return f16_bits_to_f32(f32_to_f16_bits(v));
  else return v;
}

// ---- quantization of one value ------------------------------------------------
// int8: clamp(rint(x / scale), -127, 127)   (quant.py:86, 100)
__device__ __forceinline__ int quant_i8(float x, float scale) {
  float q = rintf(x / scale);
  q = fminf(fmaxf(q, -kInt8Max), kInt8Max);
  return (int)q;
}
// fp8: e4m3fn_rne(clamp(x / scale, -448, 448))   (quant.py:83, 98); the
// hardware converter rounds to nearest even and is OCP E4M3 on gfx950.
__device__ __forceinline__ uint32_t quant_f8_pair(float x0, float x1, float scale) {
  float a = fminf(fmaxf(x0 / scale, -kFp8Max), kFp8Max);
  float b = fminf(fmaxf(x1 / scale, -kFp8Max), kFp8Max);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xffffu;
}

// ---- wave reductions (64 lanes) --------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum_tree(float v) {
  // pairwise tree: lane i adds lane i^o for o = 1, 2, ..., 32 (fixed order)
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v = v + __shfl_xor(v, o, 64);
  return v;
}

}  // namespace d3
