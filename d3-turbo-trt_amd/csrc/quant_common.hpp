// Device helpers shared by the per-token quantization kernels (quant.hip,
// norm_quant.hip): the register-resident row, the 8-value quantize-and-store,
// the row scale, the row pipeline and the host-side grid choice.
//
// Reference arithmetic: d3trt/model/quant.py:92-100 (quantize_rows) and
// :77-89 (quantize_weight, the same per-row arithmetic over [N, K]).
#pragma once

#include "common.hpp"
#include "kernels.hpp"

namespace d3 {

constexpr int kQuantWaves = 4;  // waves per 256-thread block

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

// Running max of magnitudes over packed bf16 pairs. With the sign bits cleared, the two 16-bit halves
// order like the values (NaN above inf) as unsigned integers, so one AND and one packed 16-bit max per
// pair give what amax_acc gives after unpacking both to fp32 (three ops and the two unpacks): the bf16
// magnitude shifted into the high half is the fp32 bit pattern of the same value.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
struct Bf16PairAmax {
  u16x2 m = {0, 0};
  __device__ __forceinline__ void add(uint32_t w) {
    m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, w & 0x7fff7fffu));
  }
  __device__ __forceinline__ float value() const {
    return __uint_as_float((uint32_t)(m.x > m.y ? m.x : m.y) << 16);
  }
};

// One row of a [*, K] tensor held by one wave: lane l owns the 8-element
// chunks at columns 512 c + 8 l (c < NCH), kept as raw 32-bit words (4 per
// chunk for 16-bit types, 8 for fp32), so a row of 16-bit values costs 4 VGPRs
// per chunk.
//
// FULL (K == 512 NCH): every chunk of every lane lies inside the row, so no
// chunk is checked. Otherwise a chunk past the end of the row reads the row's
// last 8 elements (K % 8 == 0 and K >= 8, so the address stays inside the row)
// and is masked by valid(): every load is issued unconditionally, before any is
// consumed. Loads under `if (col < K)` make the compiler wait for each load
// before issuing the next, serializing NCH HBM round trips.
template <int DT, int NCH, bool FULL>
struct RowChunks {
  static constexpr int kWords = DT == kF32 ? 8 : 4;
  static constexpr int kES = DT == kF32 ? 4 : 2;
  uint32_t w[NCH][kWords];

  __device__ __forceinline__ static int64_t col(int c, int lane) { return (int64_t)c * 512 + lane * 8; }
  __device__ __forceinline__ static bool valid(int c, int lane, int64_t K) { return FULL || col(c, lane) < K; }

  __device__ __forceinline__ void load(const char* row, int64_t K, int lane) {
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int64_t cc = FULL ? col(c, lane) : min(col(c, lane), K - 8);
      const uint4* src = (const uint4*)(row + cc * kES);
#pragma unroll
      for (int u = 0; u < kWords / 4; ++u) {
        const uint4 t = src[u];
        w[c][4 * u] = t.x;
        w[c][4 * u + 1] = t.y;
        w[c][4 * u + 2] = t.z;
        w[c][4 * u + 3] = t.w;
      }
    }
  }
  __device__ __forceinline__ void get(int c, float* v) const {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (DT == kF32) {
        v[2 * i] = __uint_as_float(w[c][2 * i]);
        v[2 * i + 1] = __uint_as_float(w[c][2 * i + 1]);
      } else if constexpr (DT == kBF16) {
        v[2 * i] = bf16_bits_to_f32(w[c][i] & 0xffffu);
        v[2 * i + 1] = __uint_as_float(w[c][i] & 0xffff0000u);
      } else {
        v[2 * i] = f16_bits_to_f32(w[c][i] & 0xffffu);
        v[2 * i + 1] = f16_bits_to_f32(w[c][i] >> 16);
      }
    }
  }
  // Round (a, b) to DT, keep the pair as elements 2i, 2i+1 of chunk c, and
  // return the rounded values in a and b (one v_cvt_pk_bf16_f32 for bf16).
  __device__ __forceinline__ void put_pair(int c, int i, float& a, float& b) {
    if constexpr (DT == kF32) {
      w[c][2 * i] = __float_as_uint(a);
      w[c][2 * i + 1] = __float_as_uint(b);
    } else if constexpr (DT == kBF16) {
      typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
      typedef float f2 __attribute__((ext_vector_type(2)));
      const uint32_t p = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a, b}, bf2));  // RNE
      w[c][i] = p;
      a = __uint_as_float(p << 16);
      b = __uint_as_float(p & 0xffff0000u);
    } else {
      const uint32_t lo = f32_to_f16_bits(a), hi = f32_to_f16_bits(b);
      w[c][i] = lo | (hi << 16);
      a = f16_bits_to_f32(lo);
      b = f16_bits_to_f32(hi);
    }
  }
  // bf16 only: round (a, b) to bf16, keep the pair as elements 2i, 2i+1 of chunk c and return the packed
  // word (a in the low half), without unpacking the rounded values
  __device__ __forceinline__ uint32_t put_pair_bits(int c, int i, float a, float b) {
    static_assert(DT == kBF16, "packed bf16 pairs");
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    typedef float f2 __attribute__((ext_vector_type(2)));
    const uint32_t p = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a, b}, bf2));  // RNE
    w[c][i] = p;
    return p;
  }
  // chunk c -> dst (16-byte aligned; 32 bytes for fp32)
  __device__ __forceinline__ void store_raw(int c, char* dst) const {
#pragma unroll
    for (int u = 0; u < kWords / 4; ++u)
      ((uint4*)dst)[u] = make_uint4(w[c][4 * u], w[c][4 * u + 1], w[c][4 * u + 2], w[c][4 * u + 3]);
  }

  // Re-materialize the raw words: keeps the compiler from carrying the
  // unpacked floats of one pass into the next (that would hold 8 VGPRs per
  // chunk instead of 4 and halve the waves a SIMD can hold).
  __device__ __forceinline__ void fence() {
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int u = 0; u < kWords; ++u) asm volatile("" : "+v"(w[c][u]));
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
        for (int i = 0; i < 8; i += 2) m = amax_acc(amax_acc(m, v[i]), v[i + 1]);
      }
    }
    return m;
  }
};

// Visit rows row0, row0 + stride, ... < M of a [M, K] tensor (row pitch
// ld_bytes) with one wave, calling f(row_chunks, row). The loads of the next
// row are issued before f runs on the current one, so that row's HBM traffic
// overlaps the current row's arithmetic; the finished buffer then takes the
// next row's words (register moves, after the wait those words need anyway).
// The prefetch issued with the last row re-reads that same row (an L2 hit)
// rather than sitting under a branch: a load under a branch makes the
// compiler wait for every outstanding load (vmcnt(0)) where the paths join.
// `pre` runs once, after the first row's loads are issued (set-up work that
// then overlaps their latency).
template <typename RC, typename P, typename F>
__device__ __forceinline__ void pipeline_rows(const char* base, int64_t ld_bytes, int64_t row0, int64_t stride,
                                              int64_t M, int64_t K, int lane, P&& pre, F&& f) {
  RC cur, nxt;
  int64_t r = row0;
  cur.load(base + r * ld_bytes, K, lane);
  pre();
  for (;;) {
    const int64_t n = r + stride;
    nxt.load(base + (n < M ? n : r) * ld_bytes, K, lane);
    f(cur, r);
    if (n >= M) return;
    cur = nxt;
    r = n;
  }
}

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
    lo = quant_f8_quad<CLAMP>(v, r);
    hi = quant_f8_quad<CLAMP>(v + 4, r);
  }
  *(uint2*)q = make_uint2(lo, hi);
}

// scale = max(amax, 1e-12) / (127 | 448)   (quant.py:95-99: clamp_min, then an fp32 division);
// a NaN amax stays NaN, as torch's clamp_min keeps it (fmaxf would return the floor)
template <int MODE>
__device__ __forceinline__ RowScale scale_from_amax(float amax) {
  amax = amax < kAmaxFloor ? kAmaxFloor : amax;
  return make_row_scale(amax / (MODE == kInt8 ? kInt8Max : kFp8Max));
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

// Row-bucket dispatch of the one-pass kernels: NCH = chunks of 512 elements
// per row, rounded up to a compiled bucket; FULL when K fills the bucket.
#define D3_NCH_DISPATCH(K, FN)                                   \
  do {                                                           \
    const int64_t nch_ = ((K) + 511) / 512;                      \
    int b_;                                                      \
    if (nch_ <= 1) b_ = 1;                                       \
    else if (nch_ <= 2) b_ = 2;                                  \
    else if (nch_ <= 4) b_ = 4;                                  \
    else if (nch_ <= 8) b_ = 8;                                  \
    else if (nch_ <= 12) b_ = 12;                                \
    else if (nch_ <= 16) b_ = 16;                                \
    else if (nch_ <= 24) b_ = 24;                                \
    else b_ = 32;                                                \
    const bool full_ = (K) == 512 * (int64_t)b_;                 \
    switch (b_) {                                                \
      case 1: if (full_) FN(1, true); else FN(1, false); break;  \
      case 2: if (full_) FN(2, true); else FN(2, false); break;  \
      case 4: if (full_) FN(4, true); else FN(4, false); break;  \
      case 8: if (full_) FN(8, true); else FN(8, false); break;  \
      case 12: if (full_) FN(12, true); else FN(12, false); break; \
      case 16: if (full_) FN(16, true); else FN(16, false); break; \
      case 24: if (full_) FN(24, true); else FN(24, false); break; \
      default: if (full_) FN(32, true); else FN(32, false); break; \
    }                                                            \
  } while (0)

// One block per 4 rows (kernels that give each wave exactly one row).
inline dim3 quant_grid(int64_t rows) { return dim3((unsigned)((rows + kQuantWaves - 1) / kQuantWaves)); }

// Grid of a row-pipelined kernel: enough blocks for every row, capped at the
// blocks the device holds at once (the kernel's occupancy times the CU count,
// at most kRowBlocksPerCU per CU), so each wave walks several rows and
// overlaps one row's loads with the previous row's arithmetic.
constexpr int kRowBlocksPerCU = 1;  // 4 waves per CU, 1 per SIMD (measured best: the pipeline hides the rest)
// The fused RMSNorm + quantize does more arithmetic per element (~13 VALU ops against ~5), so one
// wave per SIMD leaves its loads and its arithmetic in series: every wave takes one row and the
// occupancy sets the blocks per CU (4096 x 4096 INT8: 13.2 -> 12.0 us; 8192 x 4096: 22.2 -> 21.0).
constexpr int kNormRowBlocksPerCU = 1024;
// `dflt`, or D3W8A8_ROW_BLOCKS_PER_CU from the environment (a tuning
// override for every row-pipelined kernel, read once; a large value gives
// every wave a single row).
int row_blocks_per_cu(int dflt);
int device_cu_count();
// Blocks of `kernel` (256 threads, lds_bytes of dynamic LDS) one CU holds at
// once, cached per kernel.
int kernel_blocks_per_cu(const void* kernel, size_t lds_bytes);
template <typename K>
inline dim3 row_grid(K kernel, int64_t rows, size_t lds_bytes, int per_cu_default = kRowBlocksPerCU) {
  const int occ = kernel_blocks_per_cu((const void*)kernel, lds_bytes);
  const int64_t need = (rows + kQuantWaves - 1) / kQuantWaves;
  const int per_cu = row_blocks_per_cu(per_cu_default);
  const int64_t cap = (int64_t)device_cu_count() * (occ < per_cu ? occ : per_cu);
  return dim3((unsigned)(need < cap ? need : cap));
}

}  // namespace d3
