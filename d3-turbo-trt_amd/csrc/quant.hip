// Per-token quantization kernels for gfx950: plain, fused with RMSNorm,
// from a precomputed row amax (after SwiGLU), and the ragged gather form.
//
// One 64-lane wave owns one row. A lane holds NCH chunks of 8 consecutive
// elements (chunk c covers columns [512c, 512c+512); lane l holds columns
// 512c + 8l .. +8), loaded with 128-bit loads, so the row is read from HBM
// exactly once and the amax is a register + cross-lane reduction.
//
// Reference arithmetic: d3trt/model/quant.py:92-100 (quantize_rows) and
// :77-89 (quantize_weight, the same per-row arithmetic over [N, K]);
// RMSNorm is transformers' Qwen3_5RMSNorm (modeling_qwen3_5.py:720-734).
#include "common.hpp"
#include "kernels.hpp"

namespace d3 {

constexpr int kQuantWaves = 4;  // rows per 256-thread block

// acc + lo^2 + hi^2 of the two 16-bit values packed in w (v_dot2_f32_bf16 / _f16)
template <int DT>
__device__ __forceinline__ float dot2_sq(uint32_t w, float acc) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  if constexpr (DT == kBF16) {
    const bf2 v = __builtin_bit_cast(bf2, w);
    return __builtin_amdgcn_fdot2_f32_bf16(v, v, acc, false);
  } else {
    const h2 v = __builtin_bit_cast(h2, w);
    return __builtin_amdgcn_fdot2(v, v, acc, false);
  }
}

// One row of a [*, K] tensor held by one wave: lane l owns the 8-element
// chunks at columns 512 c + 8 l (c < NCH), kept as raw 16-byte words (32 for
// fp32) so that a row of 16-bit values costs 4 VGPRs per chunk.
//
// load() issues every chunk's load before any is consumed: a chunk past the
// end of the row reads the row's last 8 elements instead (K % 8 == 0 and
// K >= 8, so the address is always inside the row) and is masked by valid().
// Putting the loads under `if (col < K)` instead makes the compiler wait for
// each load before issuing the next, serializing NCH HBM round trips.
template <int DT, int NCH>
struct RowChunks {
  static constexpr int kWords = DT == kF32 ? 2 : 1;
  static constexpr int kES = DT == kF32 ? 4 : 2;
  uint4 raw[NCH][kWords];

  __device__ __forceinline__ static int64_t col(int c, int lane) { return (int64_t)c * 512 + lane * 8; }
  __device__ __forceinline__ static bool valid(int c, int lane, int64_t K) { return col(c, lane) < K; }

  __device__ __forceinline__ void load(const char* row, int64_t K, int lane) {
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int64_t cc = min(col(c, lane), K - 8);
      const uint4* src = (const uint4*)(row + cc * kES);
#pragma unroll
      for (int w = 0; w < kWords; ++w) raw[c][w] = src[w];
    }
  }
  __device__ __forceinline__ void get(int c, float* v) const {
    if constexpr (DT == kF32) {
      const uint4 a = raw[c][0], b = raw[c][1];
      v[0] = __uint_as_float(a.x); v[1] = __uint_as_float(a.y); v[2] = __uint_as_float(a.z); v[3] = __uint_as_float(a.w);
      v[4] = __uint_as_float(b.x); v[5] = __uint_as_float(b.y); v[6] = __uint_as_float(b.z); v[7] = __uint_as_float(b.w);
    } else {
      const uint4 u = raw[c][0];
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (DT == kBF16) {
          v[2 * i] = bf16_bits_to_f32(w[i] & 0xffffu);
          v[2 * i + 1] = bf16_bits_to_f32(w[i] >> 16);
        } else {
          v[2 * i] = f16_bits_to_f32(w[i] & 0xffffu);
          v[2 * i + 1] = f16_bits_to_f32(w[i] >> 16);
        }
      }
    }
  }

  // 8 floats -> chunk c in DT (values already representable in DT, as after round_to<DT>)
  __device__ __forceinline__ void put(int c, const float* v) {
    if constexpr (DT == kF32) {
      raw[c][0] = make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3]));
      raw[c][1] = make_uint4(__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]), __float_as_uint(v[7]));
    } else {
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t lo = DT == kBF16 ? f32_to_bf16_bits(v[2 * i]) : f32_to_f16_bits(v[2 * i]);
        const uint32_t hi = DT == kBF16 ? f32_to_bf16_bits(v[2 * i + 1]) : f32_to_f16_bits(v[2 * i + 1]);
        w[i] = lo | (hi << 16);
      }
      raw[c][0] = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
  // chunk c -> dst (16-byte aligned; 32 bytes for fp32)
  __device__ __forceinline__ void store_raw(int c, char* dst) const {
#pragma unroll
    for (int w = 0; w < kWords; ++w) ((uint4*)dst)[w] = raw[c][w];
  }

  // Re-materialize the raw words: keeps the compiler from carrying the unpacked floats of the
  // amax pass into the quantize pass (that would hold 8 VGPRs per chunk instead of 4 and halve
  // the waves a SIMD can hold).
  __device__ __forceinline__ void fence() {
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int w = 0; w < kWords; ++w) {
        uint32_t a = raw[c][w].x, b = raw[c][w].y, d = raw[c][w].z, e = raw[c][w].w;
        asm volatile("" : "+v"(a), "+v"(b), "+v"(d), "+v"(e));
        raw[c][w] = make_uint4(a, b, d, e);
      }
  }

  // max |x| over the valid chunks
  __device__ __forceinline__ float amax(int64_t K, int lane) const {
    float m = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (valid(c, lane, K)) {
        float v[8];
        get(c, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i]));
      }
    }
    return m;
  }
};

template <int DT>
__device__ __forceinline__ void store8(void* p, const float* v) {
  if constexpr (DT == kF32) {
    float4* q = (float4*)p;
    q[0] = make_float4(v[0], v[1], v[2], v[3]);
    q[1] = make_float4(v[4], v[5], v[6], v[7]);
  } else {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t lo, hi;
      if constexpr (DT == kBF16) { lo = f32_to_bf16_bits(v[2 * i]); hi = f32_to_bf16_bits(v[2 * i + 1]); }
      else { lo = f32_to_f16_bits(v[2 * i]); hi = f32_to_f16_bits(v[2 * i + 1]); }
      w[i] = lo | (hi << 16);
    }
    *(uint4*)p = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// Quantize 8 values with a row scale and store 8 bytes at q (CLAMP: see quant_i8_bits).
template <int MODE, bool CLAMP = false>
__device__ __forceinline__ void quant_store8(void* q, const float* v, const RowScale& r) {
  uint32_t lo, hi;
  if constexpr (MODE == kInt8) {
    uint32_t b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) b[i] = quant_i8_word<CLAMP>(v[i], r);
    lo = pack_low_bytes(b[0], b[1], b[2], b[3]);
    hi = pack_low_bytes(b[4], b[5], b[6], b[7]);
  } else {
    lo = quant_f8_quad(v, r);
    hi = quant_f8_quad(v + 4, r);
  }
  *(uint2*)q = make_uint2(lo, hi);
}

// scale = max(amax, 1e-12) / (127 | 448)   (quant.py:95-99: clamp_min, then an fp32 division)
template <int MODE>
__device__ __forceinline__ RowScale scale_from_amax(float amax) {
  amax = fmaxf(amax, kAmaxFloor);
  return make_row_scale(amax / (MODE == kInt8 ? kInt8Max : kFp8Max));
}

// ---------------------------------------------------------------------------
// quantize_rows: x [M, K] (ld ldx) -> q [M, K] (ld ldq) + scale [M]
// Vector path: K % 8 == 0, rows 16B aligned; NCH = ceil(K / 512).
// With row_map != nullptr (ragged gather), logical row r reads source row
// src_row(r) computed from the segment lengths; see quant_rows_ragged.
// ---------------------------------------------------------------------------
template <int MODE, int DT, int NCH>
__global__ __launch_bounds__(256) void quant_rows_vec(const void* __restrict__ x, int64_t ldx,
                                                     int64_t M, int64_t K, void* __restrict__ q,
                                                     int64_t ldq, float* __restrict__ scale) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kQuantWaves + (threadIdx.x >> 6);
  if (row >= M) return;
  using RC = RowChunks<DT, NCH>;
  RC x_;
  x_.load((const char*)x + row * ldx * RC::kES, K, lane);
  const RowScale s = scale_from_amax<MODE>(wave_max(x_.amax(K, lane)));
  if constexpr (NCH > 12) x_.fence();  // wide rows: keep them packed between the passes (occupancy)
  char* qr = (char*)q + row * ldq;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (RC::valid(c, lane, K)) {
      float v[8];
      x_.get(c, v);
      quant_store8<MODE>(qr + RC::col(c, lane), v, s);
    }
  }
  if (lane == 0) scale[row] = s.s;
}

// Generic path for any K / alignment: two passes over the row (amax, then quantize).
template <int MODE, int DT>
__global__ __launch_bounds__(256) void quant_rows_generic(const void* __restrict__ x, int64_t ldx,
                                                         int64_t M, int64_t K, void* __restrict__ q,
                                                         int64_t ldq, float* __restrict__ scale) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kQuantWaves + (threadIdx.x >> 6);
  if (row >= M) return;
  const int64_t base = row * ldx;
  float amax = 0.0f;
  for (int64_t k = lane; k < K; k += 64) amax = fmaxf(amax, fabsf(load_elem<DT>(x, base + k)));
  amax = wave_max(amax);
  const RowScale s = scale_from_amax<MODE>(amax);
  uint8_t* qr = (uint8_t*)q + row * ldq;
  for (int64_t k = lane; k < K; k += 64) {
    const float xv = load_elem<DT>(x, base + k);
    if constexpr (MODE == kInt8) qr[k] = (uint8_t)quant_i8_bits<false>(xv, s);
    else qr[k] = (uint8_t)(quant_f8_pair(xv, 0.0f, s) & 0xff);
  }
  if (lane == 0) scale[row] = s.s;
}

// ---------------------------------------------------------------------------
// Requantization with a known row amax (SwiGLU output h [M, K]).
// ---------------------------------------------------------------------------
template <int MODE, int DT, int NCH>
__global__ __launch_bounds__(256) void quant_rows_amax_vec(const void* __restrict__ h, int64_t ldh,
                                                          const float* __restrict__ amax_in, int64_t M,
                                                          int64_t K, void* __restrict__ q, int64_t ldq,
                                                          float* __restrict__ scale) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kQuantWaves + (threadIdx.x >> 6);
  if (row >= M) return;
  using RC = RowChunks<DT, NCH>;
  RC h_;
  h_.load((const char*)h + row * ldh * RC::kES, K, lane);
  const RowScale s = scale_from_amax<MODE>(amax_in[row]);
  char* qr = (char*)q + row * ldq;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (RC::valid(c, lane, K)) {
      float v[8];
      h_.get(c, v);
      quant_store8<MODE, true>(qr + RC::col(c, lane), v, s);  // amax from outside: keep the clamp
    }
  }
  if (lane == 0) scale[row] = s.s;
}

// ---------------------------------------------------------------------------
// Fused zero-centred RMSNorm + per-token quantization.
//   y = DT( (x * rstd) * g ),  g = 1 + w (zero_centered) or w,
//   rstd = 1 / sqrt(sum(x*x) / K + eps)  (sqrt and division each correctly rounded), then q(y).
// Optional: normed output y, and clear_amax[row] = 0 (the SwiGLU amax
// buffer of the same rows, so the next GEMM can atomically max into it).
// ---------------------------------------------------------------------------
template <int MODE, int DT, int DTW, int NCH, bool ZC>
__global__ __launch_bounds__(256) void rmsnorm_quant_vec(
    const void* __restrict__ x, int64_t ldx, const void* __restrict__ w, int64_t M, int64_t K,
    float eps, void* __restrict__ q, int64_t ldq, float* __restrict__ scale,
    void* __restrict__ normed, int64_t ldn, float* __restrict__ clear_amax) {
  extern __shared__ __attribute__((aligned(16))) float gain_lds[];  // K floats: g = 1 + w (ZC) or w
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kQuantWaves + (threadIdx.x >> 6);
  const bool live = row < M;
  using RC = RowChunks<DT, NCH>;
  RC x_;
  if (live) x_.load((const char*)x + row * ldx * RC::kES, K, lane);
  // The gain is the same for every row: the block forms it once in fp32 (the
  // values the reference's (1 + w.float()) holds) and every wave reads it from
  // LDS, instead of each wave loading and widening the weight row.
  {
    // 8-element pieces of w, all loads issued before any is used (K % 8 == 0, w 16-byte aligned)
    using RW = RowChunks<DTW, 1>;
    constexpr int PIECES = (NCH * 64 + 255) / 256;  // per thread: NCH * 64 pieces over 256 threads
    RW wp[PIECES];
#pragma unroll
    for (int i = 0; i < PIECES; ++i) {
      const int64_t k = (int64_t)(threadIdx.x + 256 * i) * 8;
      if (k < K) {
        const uint4* src = (const uint4*)((const char*)w + k * RW::kES);
#pragma unroll
        for (int u = 0; u < RW::kWords; ++u) wp[i].raw[0][u] = src[u];
      }
    }
#pragma unroll
    for (int i = 0; i < PIECES; ++i) {
      const int64_t k = (int64_t)(threadIdx.x + 256 * i) * 8;
      if (k < K) {
        float g[8];
        wp[i].get(0, g);
#pragma unroll
        for (int u = 0; u < 8; ++u) g[u] = ZC ? 1.0f + g[u] : g[u];
        *(float4*)(gain_lds + k) = make_float4(g[0], g[1], g[2], g[3]);
        *(float4*)(gain_lds + k + 4) = make_float4(g[4], g[5], g[6], g[7]);
      }
    }
  }
  __syncthreads();
  if (!live) return;
  // sum of squares: for 16-bit inputs one v_dot2 per packed pair (the squares of bf16 / fp16 values
  // are exact in fp32, as torch's x.float().pow(2) is)
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (RC::valid(c, lane, K)) {
      if constexpr (DT == kF32) {
        float v[8];
        x_.get(c, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float sq = v[i] * v[i];
          ss = ss + sq;
        }
      } else {
        const uint32_t w4[4] = {x_.raw[c][0].x, x_.raw[c][0].y, x_.raw[c][0].z, x_.raw[c][0].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) ss = dot2_sq<DT>(w4[i], ss);
      }
    }
  }
  ss = wave_sum(ss);
  const float var = ss / (float)K;
  const float t = var + eps;
  const float rstd = 1.0f / sqrtf(t);  // torch.rsqrt on the CPU: 1 / sqrt(t), each step correctly rounded
  float y[NCH][8];
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (RC::valid(c, lane, K)) {
      float v[8];
      x_.get(c, v);
      const float4 g0 = *(const float4*)(gain_lds + RC::col(c, lane));
      const float4 g1 = *(const float4*)(gain_lds + RC::col(c, lane) + 4);
      const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        float p0 = v[i] * rstd, p1 = v[i + 1] * rstd;
        p0 = p0 * g[i];
        p1 = p1 * g[i + 1];
        round_pair_to<DT>(p0, p1);
        y[c][i] = p0;
        y[c][i + 1] = p1;
        amax = fmaxf(fmaxf(amax, fabsf(p0)), fabsf(p1));
      }
    }
  }
  const RowScale s = scale_from_amax<MODE>(wave_max(amax));
  char* qr = (char*)q + row * ldq;
  char* nr = normed ? (char*)normed + row * ldn * RC::kES : nullptr;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (RC::valid(c, lane, K)) {
      const int64_t col = RC::col(c, lane);
      quant_store8<MODE>(qr + col, y[c], s);
      if (nr) store8<DT>(nr + col * RC::kES, y[c]);
    }
  }
  if (lane == 0) {
    scale[row] = s.s;
    if (clear_amax) clear_amax[row] = 0.0f;
  }
}

// ---------------------------------------------------------------------------
// Ragged gather: x is the right-padded [nseg, width, K] question batch;
// segment b holds off[b+1] - off[b] valid rows. Valid row (b, t) is quantized
// into packed row off[b] + t and row_map[packed] = b * width + t. Padded rows
// (t >= length) instead get their output row zeroed (out [nseg*width, N] of
// out_dtype, ld ldo), so the GEMM, which only visits packed rows, leaves a
// fully defined output. The offsets travel by value in the kernel arguments:
// no host-to-device copy precedes the launch, and a captured graph keeps them.
// ---------------------------------------------------------------------------
template <int MODE, int DT, int NCH, int OUTES>
__global__ __launch_bounds__(256) void quant_rows_ragged_vec(
    const void* __restrict__ x, int64_t ldx, const SegOffsets segs, int64_t nseg,
    int64_t width, int64_t K, void* __restrict__ q, int64_t ldq, float* __restrict__ scale,
    int32_t* __restrict__ row_map, void* __restrict__ out, int64_t ldo, int64_t N) {
  const int lane = threadIdx.x & 63;
  const int64_t prow = (int64_t)blockIdx.x * kQuantWaves + (threadIdx.x >> 6);
  if (prow >= nseg * width) return;
  const int64_t b = prow / width, t = prow - b * width;
  const int64_t part = segs.off[b];
  const int64_t len = segs.off[b + 1] - part;
  if (t >= len) {
    if (out) {
      // the host guarantees 16-byte aligned output rows and N * OUTES % 16 == 0
      char* orow = (char*)out + prow * ldo * OUTES;
      for (int64_t byte = (int64_t)lane * 16; byte < N * OUTES; byte += 64 * 16)
        *(uint4*)(orow + byte) = make_uint4(0, 0, 0, 0);
    }
    return;
  }
  const int64_t dst = part + t;
  using RC = RowChunks<DT, NCH>;
  RC x_;
  x_.load((const char*)x + prow * ldx * RC::kES, K, lane);
  const RowScale s = scale_from_amax<MODE>(wave_max(x_.amax(K, lane)));
  if constexpr (NCH > 12) x_.fence();  // wide rows: keep them packed between the passes (occupancy)
  char* qr = (char*)q + dst * ldq;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (RC::valid(c, lane, K)) {
      float v[8];
      x_.get(c, v);
      quant_store8<MODE>(qr + RC::col(c, lane), v, s);
    }
  }
  if (lane == 0) {
    scale[dst] = s.s;
    row_map[dst] = (int32_t)prow;
  }
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
#define D3_NCH_DISPATCH(K, FN)                                   \
  do {                                                           \
    const int64_t nch_ = ((K) + 511) / 512;                      \
    if (nch_ <= 1) { FN(1); }                                    \
    else if (nch_ <= 2) { FN(2); }                               \
    else if (nch_ <= 4) { FN(4); }                               \
    else if (nch_ <= 8) { FN(8); }                               \
    else if (nch_ <= 12) { FN(12); }                             \
    else if (nch_ <= 16) { FN(16); }                             \
    else if (nch_ <= 24) { FN(24); }                             \
    else { FN(32); }                                             \
  } while (0)


static inline dim3 quant_grid(int64_t rows) { return dim3((unsigned)((rows + kQuantWaves - 1) / kQuantWaves)); }

template <int MODE, int DT>
hipError_t launch_quant_rows_t(const void* x, int64_t ldx, int64_t M, int64_t K, void* q, int64_t ldq,
                               float* scale, bool vec, hipStream_t st) {
  if (M == 0) return hipSuccess;
  if (vec && K <= kMaxVecK) {
#define L(N) hipLaunchKernelGGL((quant_rows_vec<MODE, DT, N>), quant_grid(M), dim3(256), 0, st, x, ldx, M, K, q, ldq, scale)
    D3_NCH_DISPATCH(K, L);
#undef L
  } else {
    hipLaunchKernelGGL((quant_rows_generic<MODE, DT>), quant_grid(M), dim3(256), 0, st, x, ldx, M, K, q, ldq, scale);
  }
  return hipGetLastError();
}

hipError_t launch_quant_rows(int mode, int dt, const void* x, int64_t ldx, int64_t M, int64_t K, void* q,
                             int64_t ldq, float* scale, bool vec, hipStream_t st) {
#define C(MO, D) if (mode == MO && dt == D) return launch_quant_rows_t<MO, D>(x, ldx, M, K, q, ldq, scale, vec, st)
  C(kInt8, kBF16); C(kInt8, kF16); C(kInt8, kF32);
  C(kFp8, kBF16); C(kFp8, kF16); C(kFp8, kF32);
#undef C
  return hipErrorInvalidValue;
}

template <int MODE, int DT>
hipError_t launch_quant_rows_amax_t(const void* h, int64_t ldh, const float* amax, int64_t M, int64_t K, void* q,
                                    int64_t ldq, float* scale, hipStream_t st) {
  if (M == 0) return hipSuccess;
#define L(N) hipLaunchKernelGGL((quant_rows_amax_vec<MODE, DT, N>), quant_grid(M), dim3(256), 0, st, h, ldh, amax, M, K, q, ldq, scale)
  D3_NCH_DISPATCH(K, L);
#undef L
  return hipGetLastError();
}

hipError_t launch_quant_rows_amax(int mode, int dt, const void* h, int64_t ldh, const float* amax, int64_t M,
                                  int64_t K, void* q, int64_t ldq, float* scale, hipStream_t st) {
  if (K > kMaxVecK) return hipErrorInvalidValue;
#define C(MO, D) if (mode == MO && dt == D) return launch_quant_rows_amax_t<MO, D>(h, ldh, amax, M, K, q, ldq, scale, st)
  C(kInt8, kBF16); C(kInt8, kF16); C(kInt8, kF32);
  C(kFp8, kBF16); C(kFp8, kF16); C(kFp8, kF32);
#undef C
  return hipErrorInvalidValue;
}

template <int MODE, int DT, int DTW>
hipError_t launch_rmsnorm_quant_t(const void* x, int64_t ldx, const void* w, int64_t M, int64_t K, float eps,
                                  int zc, void* q, int64_t ldq, float* scale, void* normed, int64_t ldn,
                                  float* clear_amax, hipStream_t st) {
  if (M == 0) return hipSuccess;
  const size_t lds = (size_t)K * sizeof(float);  // the staged gain (K <= kMaxVecK: at most 64 KiB)
#define L(N)                                                                                                        \
  if (zc) hipLaunchKernelGGL((rmsnorm_quant_vec<MODE, DT, DTW, N, true>), quant_grid(M), dim3(256), lds, st, x, ldx, w, M, K, eps, q, ldq, scale, normed, ldn, clear_amax); \
  else hipLaunchKernelGGL((rmsnorm_quant_vec<MODE, DT, DTW, N, false>), quant_grid(M), dim3(256), lds, st, x, ldx, w, M, K, eps, q, ldq, scale, normed, ldn, clear_amax)
  D3_NCH_DISPATCH(K, L);
#undef L
  return hipGetLastError();
}

hipError_t launch_rmsnorm_quant(int mode, int dt, int dtw, const void* x, int64_t ldx, const void* w, int64_t M,
                                int64_t K, float eps, int zc, void* q, int64_t ldq, float* scale, void* normed,
                                int64_t ldn, float* clear_amax, hipStream_t st) {
  if (K > kMaxVecK) return hipErrorInvalidValue;
#define C(MO, D, W) if (mode == MO && dt == D && dtw == W) return launch_rmsnorm_quant_t<MO, D, W>(x, ldx, w, M, K, eps, zc, q, ldq, scale, normed, ldn, clear_amax, st)
  C(kInt8, kBF16, kBF16); C(kInt8, kBF16, kF32); C(kInt8, kF16, kF16); C(kInt8, kF16, kF32); C(kInt8, kF32, kF32);
  C(kFp8, kBF16, kBF16); C(kFp8, kBF16, kF32); C(kFp8, kF16, kF16); C(kFp8, kF16, kF32); C(kFp8, kF32, kF32);
#undef C
  return hipErrorInvalidValue;
}

template <int MODE, int DT, int OUTES>
hipError_t launch_quant_ragged_t(const void* x, int64_t ldx, const SegOffsets& segs, int64_t nseg, int64_t width,
                                 int64_t K, void* q, int64_t ldq, float* scale, int32_t* row_map, void* out,
                                 int64_t ldo, int64_t N, hipStream_t st) {
  const int64_t rows = nseg * width;
  if (rows == 0) return hipSuccess;
#define L(NC) hipLaunchKernelGGL((quant_rows_ragged_vec<MODE, DT, NC, OUTES>), quant_grid(rows), dim3(256), 0, st, x, ldx, segs, nseg, width, K, q, ldq, scale, row_map, out, ldo, N)
  D3_NCH_DISPATCH(K, L);
#undef L
  return hipGetLastError();
}

hipError_t launch_quant_ragged(int mode, int dt, int out_es, const void* x, int64_t ldx, const SegOffsets& segs,
                               int64_t nseg, int64_t width, int64_t K, void* q, int64_t ldq, float* scale,
                               int32_t* row_map, void* out, int64_t ldo, int64_t N, hipStream_t st) {
  if (K > kMaxVecK) return hipErrorInvalidValue;
#define C(MO, D, E) if (mode == MO && dt == D && out_es == E) return launch_quant_ragged_t<MO, D, E>(x, ldx, segs, nseg, width, K, q, ldq, scale, row_map, out, ldo, N, st)
  C(kInt8, kBF16, 2); C(kInt8, kBF16, 4); C(kInt8, kF16, 2); C(kInt8, kF16, 4); C(kInt8, kF32, 2); C(kInt8, kF32, 4);
  C(kFp8, kBF16, 2); C(kFp8, kBF16, 4); C(kFp8, kF16, 2); C(kFp8, kF16, 4); C(kFp8, kF32, 2); C(kFp8, kF32, 4);
#undef C
  return hipErrorInvalidValue;
}

}  // namespace d3
