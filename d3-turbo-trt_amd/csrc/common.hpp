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
// both values as stored in DT and read back; one packed conversion for the pair
template <int DT>
__device__ __forceinline__ void round_pair_to(float& a, float& b) {
  if constexpr (DT == kBF16) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    typedef float f2 __attribute__((ext_vector_type(2)));
    const uint32_t w = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a, b}, bf2));  // v_cvt_pk_bf16_f32, RNE
    a = __uint_as_float(w << 16);
    b = __uint_as_float(w & 0xffff0000u);
  } else if constexpr (DT == kF16) {
    a = f16_bits_to_f32(f32_to_f16_bits(a));
    b = f16_bits_to_f32(f32_to_f16_bits(b));
  }
}
template <int DT>
__device__ __forceinline__ float round_to(float v) {
  if constexpr (DT == kBF16) return bf16_round(v);
  else if constexpr (DT == kF16) return f16_bits_to_f32(f32_to_f16_bits(v));
  else return v;
}

// ---- quantization of one value ------------------------------------------------
// The reference divides every element by its row's fp32 scale (x / scale,
// quant.py:86, 100). With r = RN(1 / scale) formed once per row (a correctly
// rounded fp32 division), Markstein's correction step
//   q = RN(x * r);  e = RN(x - q * scale) (FMA, exact);  q' = RN(e * r + q) (FMA)
// gives q' == RN(x / scale) bit for bit whenever |x| >= 2^-100 and the quotient
// is a normal float: r is the correctly rounded reciprocal and q lies within
// one ulp of x / scale. Below that the residual can underflow, but then both
// q' and x / scale are below 2^-40 in magnitude and round to the same signed
// zero in int8 and FP8 once the sign of x is put back on q'. Three VALU ops
// per element replace a correctly rounded fp32 division (~10 ops); the
// exhaustive CPU check of this identity is tests/c/fma_division.c.
//
// Non-finite scales (a row holding an inf or a NaN) keep torch's quotients:
// scale NaN gives r = NaN and a NaN quotient; scale inf gives r = 0, and the
// correction runs with c = 0 (e = x, q' = q = x * 0), so a finite x yields a
// zero of x's sign and an infinite x a NaN, as x / inf does. With c = scale,
// q * inf would turn every finite element's residual into a NaN.
struct RowScale {
  float s;  // the scale (stored per token)
  float r;  // RN(1 / s)
  float c;  // s, or 0 when s is infinite (the correction step's multiplier)
};
__device__ __forceinline__ RowScale make_row_scale(float s) {
  return RowScale{s, 1.0f / s, __builtin_isinf(s) ? 0.0f : s};
}
__device__ __forceinline__ float div_row(float x, const RowScale& r) {
  const float q = x * r.r;
  const float e = __builtin_fmaf(-q, r.c, x);
  return __builtin_fmaf(e, r.r, q);
}

// Running max of magnitudes that keeps a NaN, as torch's x.abs().amax() does:
// the bit patterns of values >= 0 order like the values as unsigned integers,
// and |NaN| (sign cleared) lies above +inf. m is a previous result (>= 0 or NaN).
__device__ __forceinline__ float amax_acc(float m, float v) {
  return __uint_as_float(max(__float_as_uint(m), __float_as_uint(fabsf(v))));
}
// max of two such results
__device__ __forceinline__ float amax_join(float a, float b) {
  return __uint_as_float(max(__float_as_uint(a), __float_as_uint(b)));
}

// int8: clamp(rint(x / scale), -127, 127) (quant.py:86, 100). Adding 1.5 * 2^23
// rounds to nearest even and leaves the integer, two's complement, in the low
// byte of the float's bits (the sign of a zero quotient does not matter).
// CLAMP: when the scale comes from the amax of the very values quantized
// (scale = RN(amax / 127), |x| <= amax), |x / scale| <= 127 (1 + 2^-23), which
// rounds to at most 127, so the reference's clamp never acts and is skipped;
// a row amax supplied from outside keeps it. Clamping before rounding gives
// the same integers as after (127.5 rounds to 128, then clamps to 127).
template <bool CLAMP>
__device__ __forceinline__ uint32_t quant_i8_word(float x, const RowScale& r) {  // int8 in the low byte
  float v = div_row(x, r);
  if constexpr (CLAMP) v = fminf(fmaxf(v, -kInt8Max), kInt8Max);
  v = v + 12582912.0f;
  return __float_as_uint(v);
}
template <bool CLAMP>
__device__ __forceinline__ uint32_t quant_i8_bits(float x, const RowScale& r) {
  return quant_i8_word<CLAMP>(x, r) & 0xffu;
}
// fp8: e4m3fn_rne(clamp(x / scale, -448, 448))   (quant.py:83, 98); the
// hardware converter rounds to nearest even and is OCP E4M3 on gfx950. The
// quotient carries the sign of x also when it is zero (-0 encodes as 0x80).
// CLAMP as for int8: with the scale from the row's own amax, |x / scale| <=
// 448 (1 + 2^-23), which rounds to 448 (the next E4M3 step would be 480, so
// everything below 464 rounds down), and a NaN quotient reaches the converter
// as a NaN (fminf / fmaxf would turn it into +-448).
// div_row_signed is div_row's correction with the residual negated: e' = RN(q·c − x) = −e and
// q' = RN(q − e'·r), the same value as div_row's for every x ≠ 0. For x = ±0, q = ±0, e' = +0 and
// q' = (−0) + q keeps the sign of x, where div_row's last step turns −0 into +0 (−0 + +0).
__device__ __forceinline__ float div_row_signed(float x, const RowScale& r) {
  const float q = x * r.r;
  const float e = __builtin_fmaf(q, r.c, -x);
  return __builtin_fmaf(-e, r.r, q);
}
template <bool CLAMP>
__device__ __forceinline__ float f8_quotient(float x, const RowScale& r) {
  const float v = div_row_signed(x, r);
  return CLAMP ? fminf(fmaxf(v, -kFp8Max), kFp8Max) : v;
}
template <bool CLAMP = false>
__device__ __forceinline__ uint32_t quant_f8_pair(float x0, float x1, const RowScale& r) {
  const float a = f8_quotient<CLAMP>(x0, r), b = f8_quotient<CLAMP>(x1, r);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xffffu;
}
// four values -> four E4M3 bytes of one word (the second conversion writes the high half)
template <bool CLAMP = false>
__device__ __forceinline__ uint32_t quant_f8_quad(const float* x, const RowScale& r) {
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = f8_quotient<CLAMP>(x[i], r);
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(v[0], v[1], 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v[2], v[3], lo, true);
}
// four int8 results (the low bytes of quant_i8_bits words) -> one word, by byte permutes
__device__ __forceinline__ uint32_t pack_low_bytes(uint32_t b0, uint32_t b1, uint32_t b2, uint32_t b3) {
  const uint32_t a = __builtin_amdgcn_perm(b1, b0, 0x0c0c0400u);  // [b0.0, b1.0, 0, 0]
  const uint32_t c = __builtin_amdgcn_perm(b3, b2, 0x0c0c0400u);  // [b2.0, b3.0, 0, 0]
  return __builtin_amdgcn_perm(c, a, 0x05040100u);                // [b0.0, b1.0, b2.0, b3.0]
}

// ---- wave reductions (64 lanes) --------------------------------------------------
// DPP steps within rows of 16 lanes (row_shr 1, 2, 4, 8), then across rows
// (row_bcast 15, 31): lane 63 ends up with the reduction of all 64 lanes,
// which readlane broadcasts through an SGPR. Lanes a step has no source for
// read 0, so the operation needs op(a, 0) == a: a sum, or a max of values
// >= 0. Every step is a VALU op; no LDS round trip.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}
template <typename OP>
__device__ __forceinline__ float wave_reduce(float v, OP op) {
  v = op(v, dpp_f32<0x111, 0xf>(v));  // row_shr:1
  v = op(v, dpp_f32<0x112, 0xf>(v));  // row_shr:2
  v = op(v, dpp_f32<0x114, 0xf>(v));  // row_shr:4
  v = op(v, dpp_f32<0x118, 0xf>(v));  // row_shr:8
  v = op(v, dpp_f32<0x142, 0xa>(v));  // row_bcast:15 into rows 1 and 3
  v = op(v, dpp_f32<0x143, 0xc>(v));  // row_bcast:31 into rows 2 and 3
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// max over the wave of magnitudes (values >= 0, or NaN, which wins: amax_join)
__device__ __forceinline__ float wave_max(float v) {
  return wave_reduce(v, [](float a, float b) { return amax_join(a, b); });
}
// sum over the wave, in the fixed order of the DPP steps above
__device__ __forceinline__ float wave_sum(float v) {
  return wave_reduce(v, [](float a, float b) { return a + b; });
}

}  // namespace d3
