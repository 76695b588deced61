// W8A8 GEMM for gfx950: out[m, n] = epilogue( sum_k a[m, k] * w[n, k] ).
//
// Both operands are K-contiguous 8-bit matrices (a: per-token quantized
// activations [M, K]; w: per-output-channel quantized weights [N, K]), the
// "TN" product the reference asks of torch._int_mm / torch._scaled_mm
// (d3trt/model/quant.py:171-177, 196).
//
// Structure (one workgroup = one BM x BN output tile):
//   * K advances in steps of 128 bytes; A and B tiles of the step are staged
//     in LDS, double-buffered: the global loads of step t+1 are in flight
//     (128-bit, 8 lanes per 128-byte row segment) while the MFMAs of step t
//     run, so there is one barrier per step.
//   * LDS rows are 128 bytes; the 16-byte chunk c of row r is stored at chunk
//     c ^ ((r >> 1) & 7), so the 16 lanes a ds_read_b128 serves per cycle (16
//     consecutive rows, one chunk each) hit 16 distinct 16-byte bank groups.
//   * WM x WN waves; each owns a (BM/WM) x (BN/WN) sub-tile made of 32x32
//     MFMA blocks: v_mfma_i32_32x32x32_i8 (INT8) or
//     v_mfma_f32_32x32x64_f8f6f4 with format E4M3 (FP8).
//     Operand lane l carries row (l & 31) and the K chunk selected by l >> 5;
//     both operands use the same K assignment, so the dot product is complete.
//     The weights are the MFMA's first operand and the activations its
//     second, so each 32x32 result block is transposed: register r of lane l
//     holds output row l%32, column 8*(r/4) + 4*(l/32) + (r%4).
//   * Workgroups are remapped so that each XCD (the hardware deals
//     workgroups round-robin over 8 XCDs) receives a contiguous run of tiles,
//     ordered in groups of GROUP_M tile-rows, so concurrently running tiles on
//     one XCD share A and B panels in that XCD's L2.
//
// Epilogues (all fp32 with contraction off, then rounded like the eager chain):
//   dequant : out = OUT( (float(acc) * s_tok[m]) * s_ch[n] )      (quant.py:162, 197)
//   raw     : out = acc (int32 for INT8, fp32 for FP8)             (parity hook)
//   swiglu  : weights interleaved in blocks of 32 rows [g0..g31, u0..u31, g32..];
//             g = OUT(deq(gate)), u = OUT(deq(up)),
//             h = OUT( OUT(g / (1 + exp(-g))) * u )                 (trtllm_stack.py:131-134)
//             (exp and the reciprocal on the hardware exp2 / v_rcp_f32: ~1e-6
//             relative, absorbed by the bf16 rounding of silu but next to a
//             rounding boundary)
//             and row_amax[m] = max(row_amax[m], |h|) by atomic max.
//   residual: out = OUT( float(res[m, n]) + OUT(deq(acc)) )         (core.py:215)
#pragma once

#include "common.hpp"
#include "kernels.hpp"

#include <type_traits>

namespace d3 {


constexpr int kBK = 128;  // bytes of K per pipeline step
// M tiles per group of the tile order (XCD-contiguous ranges, then groups of kGroupM M tiles
// walked N-major). Measured (FP8, M = 4096): 2 runs 1-1.5% faster than 4 (gate_up 352 vs 355 us) but
// re-reads each weight panel twice as often (L2-to-fabric traffic of gate_up 1.23 GB vs 0.93 GB);
// 8 and 16 are slower (16: gate_up 382 us).
constexpr int kGroupM = 4;

template <int MODE>
struct Mfma;
template <>
struct Mfma<kInt8> {
  typedef v4i frag;    // 16 bytes of K per lane, 32 K per instruction
  typedef v16i acc;
  static constexpr int kSub = kBK / 32;
  __device__ static __forceinline__ acc run(frag a, frag b, acc c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma<kFp8> {
  typedef v8i frag;    // 32 bytes of K per lane, 64 K per instruction
  typedef v16f acc;
  static constexpr int kSub = kBK / 64;
  __device__ static __forceinline__ acc run(frag a, frag b, acc c) {
    // Format 0 = FP8 E4M3 for both operands. With scale operands 0 the compiler emits the plain
    // v_mfma_f32_32x32x64_f8f6f4: one 8-byte instruction per MFMA. The unit-scale form (E8M0 127 =
    // 1.0) keeps the 16-byte scaled encoding, whose prefix loads the two scales for every MFMA, and
    // measured 1.5-2% slower on the state-pass GEMMs. The FP8 GEMM tests pin the plain product.
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
  }
};

// 128-byte rows: a ds_read_b128 serves 16 lanes per cycle from 64 banks (256 B), i.e. two rows of 8
// chunks; XOR-ing the chunk with (row >> 1) & 7 puts the 16 rows of one cycle on 16 distinct chunks.
__device__ __forceinline__ int lds_off(int row, int chunk) { return row * kBK + ((chunk ^ ((row >> 1) & 7)) << 4); }

// Map a linear workgroup id to (tile_m, tile_n): XCD-contiguous, then grouped.
__device__ __forceinline__ void tile_of(int bid, int nb, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int full = nb >> 3, rem = nb & 7;
  const int xcd = bid & 7, local = bid >> 3;
  const int logical = xcd * full + (xcd < rem ? xcd : rem) + local;
  const int per_group = kGroupM * tiles_n;
  const int group = logical / per_group;
  const int first_m = group * kGroupM;
  const int gsz = min(tiles_m - first_m, kGroupM);
  const int in_group = logical - group * per_group;
  tm = first_m + in_group % gsz;
  tn = in_group / gsz;
}

// Epilogue shared by the GEMM kernels. The MFMAs take the weights as their
// first operand and the activations as their second, so acc[i][j] is the
// transposed 32x32 output block: lane l holds output row
//   wrow0 + 32 i + (l & 31)
// and, in register 4 g + c (g, c in 0..3), output column
//   wcol0 + 32 j + 8 g + 4 (l >> 5) + c.
// Every lane therefore owns runs of 4 consecutive columns of one row: one
// token scale per block row and float4 channel scales.

// Edge tiles (partly outside the output, or outputs without 16-byte row
// alignment): every element is checked and stored on its own, with its
// scales loaded where they are used. Correct for any shape; the full-tile
// path below carries the throughput.
template <int MODE, int TM, int TN, int EPI, int OUT, bool MAP, typename ACC>
__device__ __forceinline__ void epilogue_edge(const GemmParams& p, ACC (&acc)[TM][TN], int64_t wrow0, int64_t wcol0,
                                              int lane) {
  const int64_t M = p.M, N = p.N;
  const int lrow = lane & 31, lhalf = lane >> 5;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int64_t row = wrow0 + i * 32 + lrow;
    const bool rok = row < M;
    const float st = (EPI != kEpiRaw && rok) ? p.a_scale[row] : 0.0f;
    const int64_t orow = MAP ? (rok ? (int64_t)p.row_map[row] : 0) : row;
    if constexpr (EPI == kEpiSwiGLU) {
      float rmax = 0.0f;
#pragma unroll
      for (int jp = 0; jp < TN / 2; ++jp)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t cg = wcol0 + jp * 64 + (r >> 2) * 8 + lhalf * 4 + (r & 3);  // gate column; up is cg + 32
          if (rok && cg + 32 < N) {
            float gv = (float)acc[i][2 * jp][r];
            gv = gv * st;
            gv = round_to<OUT>(gv * p.w_scale[cg]);
            float uv = (float)acc[i][2 * jp + 1][r];
            uv = uv * st;
            uv = round_to<OUT>(uv * p.w_scale[cg + 32]);
            const float sl = round_to<OUT>(gv * __builtin_amdgcn_rcpf(1.0f + __expf(-gv)));
            const float h = round_to<OUT>(sl * uv);
            store_elem<OUT>(p.out, orow * p.ldo + (cg >> 6) * 32 + (cg & 31), h);
            rmax = amax_acc(rmax, h);
          }
        }
      if (p.row_amax) {
        rmax = amax_join(rmax, __shfl_xor(rmax, 32, 64));
        if (lhalf == 0 && rok) atomicMax((unsigned int*)(p.row_amax + row), __float_as_uint(rmax));
      }
    } else {
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t col = wcol0 + j * 32 + (r >> 2) * 8 + lhalf * 4 + (r & 3);
          if (rok && col < N) {
            const int64_t o = orow * p.ldo + col;
            if constexpr (EPI == kEpiRaw) {
              if constexpr (MODE == kInt8) ((int32_t*)p.out)[o] = acc[i][j][r];
              else ((float*)p.out)[o] = acc[i][j][r];
            } else {
              float x = (float)acc[i][j][r];
              x = x * st;
              x = x * p.w_scale[col];
              if constexpr (EPI == kEpiResidual) {
                x = round_to<OUT>(x);
                x = load_elem<OUT>(p.res, orow * p.ldr + col) + x;
              }
              store_elem<OUT>(p.out, o, x);
            }
          }
        }
    }
  }
}

// Full-tile epilogue through LDS. For each 32-row block row of the wave tile,
// every lane writes its runs of 4 finished output values (rounded to OUT) into
// this wave's LDS region, row-major; the wave then reads the rows back as
// 16-byte chunks, 16 consecutive lanes per 256-byte row segment, and stores
// them with 16-byte global stores, so every store instruction writes whole
// cache lines. The residual (core.py:215: bf16 add of the rounded projection)
// is applied in the read-back, where its loads are coalesced the same way.
//
// PACK: rows unpadded (RS = RB), the 16-byte chunk c of row r stored at chunk
// c ^ (r & (CPR - 1)) (CPR a power of two, at most 16 used): 32 rows in 32 RB
// bytes, for kernels whose LDS has no room for the padding; the lanes of one
// write (32 rows, one chunk each) then meet each bank at most twice.
template <int TN, int EPI, int OUT, bool PACK = false>
struct EpiLds {
  static constexpr int ES = EPI == kEpiRaw ? 4 : (OUT == kF32 ? 4 : 2);  // output element bytes
  static constexpr int OC = EPI == kEpiSwiGLU ? TN * 16 : TN * 32;        // output columns per wave tile
  static constexpr int RB = OC * ES;                                      // bytes per output row
  static constexpr int RS = PACK ? RB : RB + 16;                          // LDS row stride
  static constexpr int CPR = RB / 16;                                     // 16-byte chunks per row
  static constexpr int NRB = 32 * CPR / 64;                               // read-back chunks per lane
  static constexpr int BYTES = 32 * RS;                                   // LDS bytes per wave
  static constexpr int SWZ = PACK ? (CPR < 16 ? CPR - 1 : 15) : 0;
  static_assert((32 * CPR) % 64 == 0, "read-back split");
  static_assert(!PACK || (CPR & (CPR - 1)) == 0, "the packed layout needs a power-of-two chunk count");
  // byte offset of byte `b` of row `row` in the staging area
  __device__ static __forceinline__ int at(int row, int b) { return row * RS + ((((b >> 4) ^ (row & SWZ))) << 4) + (b & 15); }
};

template <int OUT, int ES>
__device__ __forceinline__ void lds_put4(uint8_t* dst, const float* v) {
  if constexpr (ES == 4) {
    *(float4*)dst = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    uint32_t b[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) b[c] = OUT == kBF16 ? f32_to_bf16_bits(v[c]) : f32_to_f16_bits(v[c]);
    *(uint2*)dst = make_uint2(b[0] | (b[1] << 16), b[2] | (b[3] << 16));
  }
}

template <int MODE, int TM, int TN, int EPI, int OUT, bool MAP, bool PACK, typename ACC, typename H>
__device__ __forceinline__ void epilogue_lds(const GemmParams& p, ACC (&acc)[TM][TN], int64_t wrow0, int64_t wcol0,
                                             int lane, uint8_t* stage, H&& after_scales) {
  using E = EpiLds<TN, EPI, OUT, PACK>;
  const int lrow = lane & 31, lhalf = lane >> 5;
  float st[TM];
  int64_t orow[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int64_t row = wrow0 + i * 32 + lrow;
    st[i] = EPI != kEpiRaw ? p.a_scale[row] : 0.0f;
    if constexpr (MAP) orow[i] = (int64_t)p.row_map[row];
    else orow[i] = row;
  }
  // channel scales: float4 per (block, group); SwiGLU needs the gate and up columns
  constexpr int NSB = EPI == kEpiRaw ? 1 : TN;
  float sc[NSB][4][4];
  if constexpr (EPI != kEpiRaw) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 s4 = *(const float4*)(p.w_scale + wcol0 + j * 32 + g * 8 + lhalf * 4);
        sc[j][g][0] = s4.x; sc[j][g][1] = s4.y; sc[j][g][2] = s4.z; sc[j][g][3] = s4.w;
      }
  }
  const int64_t ocol0 = EPI == kEpiSwiGLU ? wcol0 / 2 : wcol0;  // first output column of the wave tile
  after_scales();

#pragma unroll
  for (int i = 0; i < TM; ++i) {
    // 1. finish this lane's values of block row i and stage them
    if constexpr (EPI == kEpiSwiGLU) {
      float rmax = 0.0f;
#pragma unroll
      for (int jp = 0; jp < TN / 2; ++jp)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float h[4];
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            float gv = (float)acc[i][2 * jp][4 * g + c];
            gv = gv * st[i];
            gv = round_to<OUT>(gv * sc[2 * jp][g][c]);
            float uv = (float)acc[i][2 * jp + 1][4 * g + c];
            uv = uv * st[i];
            uv = round_to<OUT>(uv * sc[2 * jp + 1][g][c]);
            const float sl = round_to<OUT>(gv * __builtin_amdgcn_rcpf(1.0f + __expf(-gv)));
            h[c] = round_to<OUT>(sl * uv);
            rmax = amax_acc(rmax, h[c]);
          }
          lds_put4<OUT, E::ES>(stage + E::at(lrow, (jp * 32 + g * 8 + lhalf * 4) * E::ES), h);
          if (g == 3) __builtin_amdgcn_sched_barrier(0);
        }
      if (p.row_amax) {
        rmax = amax_join(rmax, __shfl_xor(rmax, 32, 64));  // lanes l and l + 32 share the row
        if (lhalf == 0) atomicMax((unsigned int*)(p.row_amax + wrow0 + i * 32 + lrow), __float_as_uint(rmax));
      }
    } else {
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          uint8_t* dst = stage + E::at(lrow, (j * 32 + g * 8 + lhalf * 4) * E::ES);
          if constexpr (EPI == kEpiRaw) {
            if constexpr (MODE == kInt8)
              *(int4*)dst = make_int4(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
            else
              *(float4*)dst = make_float4(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
          } else {
            float v[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              float x = (float)acc[i][j][4 * g + c];
              x = x * st[i];
              v[c] = x * sc[j][g][c];
            }
            lds_put4<OUT, E::ES>(dst, v);  // rounds to OUT (the residual adds to the rounded value)
          }
          if (g == 3) __builtin_amdgcn_sched_barrier(0);
        }
    }
    // 2. read the staged rows back as 16-byte chunks and store them
    uint4 chunk[E::NRB];
    int64_t obase[E::NRB];
#pragma unroll
    for (int t = 0; t < E::NRB; ++t) {
      const int q = t * 64 + lane, r = q / E::CPR, ch = q % E::CPR;
      chunk[t] = *(const uint4*)(stage + E::at(r, ch * 16));
      const int64_t orr = MAP ? __shfl(orow[i], r, 64) : wrow0 + i * 32 + r;
      obase[t] = orr;
    }
    if constexpr (EPI == kEpiResidual) {
      uint4 rs[E::NRB];
#pragma unroll
      for (int t = 0; t < E::NRB; ++t) {
        const int ch = (t * 64 + lane) % E::CPR;
        rs[t] = *(const uint4*)((const uint8_t*)p.res + (obase[t] * p.ldr + ocol0) * E::ES + ch * 16);
      }
#pragma unroll
      for (int t = 0; t < E::NRB; ++t) {
        const uint32_t* a = (const uint32_t*)&chunk[t];
        const uint32_t* b = (const uint32_t*)&rs[t];
        uint32_t o[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          if constexpr (E::ES == 4) {
            o[w] = __float_as_uint(__uint_as_float(b[w]) + __uint_as_float(a[w]));
          } else {
            float lo, hi;
            if constexpr (OUT == kBF16) {
              lo = bf16_bits_to_f32(b[w] & 0xffffu) + bf16_bits_to_f32(a[w] & 0xffffu);
              hi = bf16_bits_to_f32(b[w] >> 16) + bf16_bits_to_f32(a[w] >> 16);
              o[w] = (uint32_t)f32_to_bf16_bits(lo) | ((uint32_t)f32_to_bf16_bits(hi) << 16);
            } else {
              lo = f16_bits_to_f32(b[w] & 0xffffu) + f16_bits_to_f32(a[w] & 0xffffu);
              hi = f16_bits_to_f32(b[w] >> 16) + f16_bits_to_f32(a[w] >> 16);
              o[w] = (uint32_t)f32_to_f16_bits(lo) | ((uint32_t)f32_to_f16_bits(hi) << 16);
            }
          }
        }
        chunk[t] = make_uint4(o[0], o[1], o[2], o[3]);
      }
    }
#pragma unroll
    for (int t = 0; t < E::NRB; ++t) {
      const int ch = (t * 64 + lane) % E::CPR;
      *(uint4*)((uint8_t*)p.out + (obase[t] * p.ldo + ocol0) * E::ES + ch * 16) = chunk[t];
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Full tiles (inside the output, vector-aligned) take the LDS path; edge tiles
// check and store every element. `stage` is this wave's LDS region
// (EpiLds<.., PACK>::BYTES), free of any in-flight use when the epilogue
// starts. after_scales() runs once the full path's row / channel scales are
// in registers (the edge path runs it first): the persistent kernel issues
// the next tile's DMA there, so the epilogue's own loads need not wait for it.
template <int MODE, int TM, int TN, int EPI, int OUT, bool PACK = false, typename ACC, typename H>
__device__ __forceinline__ void epilogue(const GemmParams& p, ACC (&acc)[TM][TN], int64_t wrow0, int64_t wcol0,
                                         int lane, uint8_t* stage, H&& after_scales) {
  const bool full = p.vec && wrow0 + TM * 32 <= p.M && wcol0 + TN * 32 <= p.N;
  if (full) {
    if (EPI != kEpiSwiGLU && p.row_map)
      epilogue_lds<MODE, TM, TN, EPI, OUT, true, PACK>(p, acc, wrow0, wcol0, lane, stage, after_scales);
    else epilogue_lds<MODE, TM, TN, EPI, OUT, false, PACK>(p, acc, wrow0, wcol0, lane, stage, after_scales);
  } else {
    after_scales();
    if (EPI != kEpiSwiGLU && p.row_map) epilogue_edge<MODE, TM, TN, EPI, OUT, true>(p, acc, wrow0, wcol0, lane);
    else epilogue_edge<MODE, TM, TN, EPI, OUT, false>(p, acc, wrow0, wcol0, lane);
  }
}
template <int MODE, int TM, int TN, int EPI, int OUT, typename ACC>
__device__ __forceinline__ void epilogue(const GemmParams& p, ACC (&acc)[TM][TN], int64_t wrow0, int64_t wcol0,
                                         int lane, uint8_t* stage) {
  epilogue<MODE, TM, TN, EPI, OUT, false>(p, acc, wrow0, wcol0, lane, stage, [] {});
}

// Register-staged tiles: row-major operands only (plan_gemm never gives them a K-blocked one).
template <int MODE, int BM, int BN, int WM, int WN, int EPI, int OUT>
__global__ __launch_bounds__(WM* WN * 64, 1) void gemm_w8a8(GemmParams p) {
  using MF = Mfma<MODE>;
  typedef typename MF::frag frag_t;
  typedef typename MF::acc acc_t;
  constexpr int NT = WM * WN * 64;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  constexpr int A_LD = BM * 8 / NT, B_LD = BN * 8 / NT;
  constexpr int STAGE = (BM + BN) * kBK;
  static_assert(TM >= 1 && TN >= 1 && A_LD >= 1 && B_LD >= 1, "tile config");
  static_assert(EPI != kEpiSwiGLU || (TN % 2 == 0), "swiglu needs gate/up block pairs");
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  int tm, tn;
  tile_of(blockIdx.x, gridDim.x, p.tiles_m, p.tiles_n, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int64_t M = p.M, N = p.N, K = p.K;

  v4i ra[A_LD], rb[B_LD];
  auto gload = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const int id = i * NT + tid, row = id >> 3, ch = id & 7;
      const int64_t gm = m0 + row, kk = k0 + ch * 16;
      ra[i] = (gm < M && kk < K) ? *(const v4i*)(p.a + gm * p.lda + kk) : v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < B_LD; ++i) {
      const int id = i * NT + tid, row = id >> 3, ch = id & 7;
      const int64_t gn = n0 + row, kk = k0 + ch * 16;
      rb[i] = (gn < N && kk < K) ? *(const v4i*)(p.w + gn * p.ldw + kk) : v4i{0, 0, 0, 0};
    }
  };
  auto swrite = [&](int buf) {
    uint8_t* sa = lds + buf * STAGE;
    uint8_t* sb = sa + BM * kBK;
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const int id = i * NT + tid, row = id >> 3, ch = id & 7;
      *(v4i*)(sa + lds_off(row, ch)) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_LD; ++i) {
      const int id = i * NT + tid, row = id >> 3, ch = id & 7;
      *(v4i*)(sb + lds_off(row, ch)) = rb[i];
    }
  };

  acc_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  const int nk = (int)((K + kBK - 1) / kBK);
  gload(0);
  swrite(0);
  __syncthreads();
  const int lrow = lane & 31, lhalf = lane >> 5;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload((int64_t)(kt + 1) * kBK);
    const uint8_t* sa = lds + buf * STAGE;
    const uint8_t* sb = sa + BM * kBK;
#pragma unroll
    for (int s = 0; s < MF::kSub; ++s) {
      frag_t af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = wm * WTM + i * 32 + lrow;
        if constexpr (MODE == kInt8) {
          af[i] = *(const v4i*)(sa + lds_off(row, 2 * s + lhalf));
        } else {
          const v4i lo = *(const v4i*)(sa + lds_off(row, 4 * s + 2 * lhalf));
          const v4i hi = *(const v4i*)(sa + lds_off(row, 4 * s + 2 * lhalf + 1));
          af[i] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int row = wn * WTN + j * 32 + lrow;
        if constexpr (MODE == kInt8) {
          bf[j] = *(const v4i*)(sb + lds_off(row, 2 * s + lhalf));
        } else {
          const v4i lo = *(const v4i*)(sb + lds_off(row, 4 * s + 2 * lhalf));
          const v4i hi = *(const v4i*)(sb + lds_off(row, 4 * s + 2 * lhalf + 1));
          bf[j] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = MF::run(bf[j], af[i], acc[i][j]);
    }
    if (kt + 1 < nk) swrite(buf ^ 1);
    __syncthreads();
  }

  static_assert(NT / 64 * EpiLds<TN, EPI, OUT>::BYTES <= (int)sizeof(lds), "epilogue staging");
  epilogue<MODE, TM, TN, EPI, OUT>(p, acc, m0 + wm * WTM, n0 + wn * WTN, lane,
                                   lds + (tid >> 6) * EpiLds<TN, EPI, OUT>::BYTES);
}


// ---------------------------------------------------------------------------
// Pipelined kernel (K % BK == 0): BK-byte K steps (64, or 128 for the
// weight-streaming tile), 4 LDS stages filled by direct global->LDS DMA
// (global_load_lds_dwordx4), one barrier per step.
//
//   * DMA: each instruction of a wave writes 1 KiB of LDS (64 lanes x 16 B):
//     1024/BK rows of BK bytes. Lane j carries row r0 + j/(BK/16) and physical
//     chunk j%(BK/16), i.e. logical K chunk (j%(BK/16)) ^ swz(row): the XOR
//     swizzle that makes the MFMA operand reads (one 16-byte chunk of 32
//     consecutive rows) conflict-free (a ds_read_b128 serves 16 lanes per
//     cycle from 64 banks). 128-byte steps fetch whole 128-byte lines of each
//     row, which HBM streams at ~6 TB/s where 64-byte pieces of many rows
//     reach ~4 TB/s (measured on MI355X): the skinny-M tile uses them.
//     Sources are a uniform base (SGPRs, advanced by BK bytes per step) plus
//     a 32-bit per-lane offset; the LDS address is this wave's slot in stage
//     0 plus a compile-time stage/row offset. Rows past M (or N) are clamped
//     to the last row: they only feed output rows (columns) never stored.
//   * Operands: A fragments are single-buffered (the fragment for the next
//     step is read right after its last MFMA of this step); B fragments are
//     double-buffered by step parity.
//   * Step kt (stage U = kt % 4 holds its operands): PRE MFMAs; wait for this
//     wave's LDS reads and for its DMA of step kt+1; barrier (so every wave's
//     DMA of step kt+1 has landed and every wave is done reading stage U);
//     then the remaining MFMAs, each followed by its share of the next step's
//     fragment reads (stage U+1) and of the DMA of step kt+4 (into stage U).
//     sched_barrier after every slot keeps that interleave: the matrix pipe
//     always has queued work while LDS and DMA requests issue.
//   * Steps with a full pipeline ahead run unchecked; the last steps of the
//     K loop (CHECKED) guard the reads and DMAs that would pass the end.
// ---------------------------------------------------------------------------
constexpr int kStages = 4;

// LDS swizzle of BK-byte rows. 64-byte rows: the 16 lanes of one ds_read_b128 cycle read rows
// r..r+15 (four rows per 256-byte bank line); XOR-ing the chunk with (row >> 2) & 3 spreads them over
// the 16 bank groups. 128-byte rows: two rows per bank line; XOR with (row >> 1) & 7.
template <int BK>
__host__ __device__ __forceinline__ int lds_swz(int row) {
  static_assert(BK == 64 || BK == 128, "step bytes");
  return BK == 64 ? (row >> 2) & 3 : (row >> 1) & 7;
}
template <int BK>
__device__ __forceinline__ int lds_offk(int row, int chunk) { return row * BK + ((chunk ^ lds_swz<BK>(row)) << 4); }

// s_barrier without the fence __syncthreads() adds (whose vmcnt(0) would drain
// the DMA pipeline); the empty asm keeps the compiler from moving LDS accesses
// across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Calls f(std::integral_constant<int, I>) for I in [B, E), in order.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  // s_waitcnt encoding (gfx9): vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

#define D3_LDS_PTR(p) ((__attribute__((address_space(3))) const void*)(p))

// One wave-wide 16-byte-per-lane DMA: lane l's 16 bytes at gbase + voff land
// at LDS lds_base + OFF + 16 l. Issued as inline asm so the compiler does not
// model the LDS write (it would otherwise insert vmcnt(0) before LDS reads it
// cannot prove disjoint, draining the pipeline); every wait on this DMA is
// explicit (wait_vmcnt + barrier). M0 holds the LDS address: it is an input
// operand bound to m0 ("{m0}"), so the compiler writes m0 itself and knows
// its value at every point. The compiler does not insert wait states for an
// inline asm's operands, so the asm carries its own: s_nop 4 gives the 5 wait
// states a VMEM instruction needs after a VALU write of an SGPR it reads (the
// base comes from v_readfirstlane, often only an instruction or two earlier;
// with fewer, the DMA can read the register's previous value), which also
// covers the single wait state after an M0 write.
// A wave-uniform pointer, pinned to SGPRs (the DMA asm takes it as an SGPR pair).
__device__ __forceinline__ const uint8_t* uniform_ptr(const uint8_t* q) {
  const uint64_t v = (uint64_t)(uintptr_t)q;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const uint8_t*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

template <int OFF>
__device__ __forceinline__ void dma16(const uint8_t* gbase, uint32_t voff, uint32_t lds_base) {
  asm volatile(
      "s_nop 4\n\t"
      "global_load_lds_dwordx4 %0, %1"
      :
      : "v"(voff), "s"(gbase), "{m0}"(lds_base + (uint32_t)OFF)
      : "memory");
}

// Split-K, first half: every workgroup of a tile stores its raw accumulators
// in its own slot of the workspace. Slot layout: 16-byte word (i, j, g) of
// wave w is 1 KiB of consecutive bytes over the wave's lanes (registers
// 4g..4g+3 of acc[i][j]), so every store writes whole cache lines.
template <int NW, int TM, int TN>
__host__ __device__ constexpr int splitk_wave_words() { return TM * TN * 4 * 64; }

// Tiles that carry the split-K path.
template <int BM, int BN>
constexpr bool kSplitTile = BM == 128 && BN == 128;

template <int MODE, int NW, int TM, int TN, typename ACC>
__device__ __forceinline__ void splitk_store(const GemmParams& p, ACC (&acc)[TM][TN], int tile, int split, int wave,
                                             int lane) {
  using E = typename std::conditional<MODE == kInt8, int, float>::type;
  constexpr int WAVE_U4 = splitk_wave_words<NW, TM, TN>(), TILE_U4 = NW * WAVE_U4;
  uint4* mine = (uint4*)p.partial + ((int64_t)tile * p.ksplit + split) * TILE_U4 + wave * WAVE_U4 + lane;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        mine[((i * TN + j) * 4 + g) * 64] =
            make_uint4(__builtin_bit_cast(uint32_t, (E)acc[i][j][4 * g]), __builtin_bit_cast(uint32_t, (E)acc[i][j][4 * g + 1]),
                       __builtin_bit_cast(uint32_t, (E)acc[i][j][4 * g + 2]), __builtin_bit_cast(uint32_t, (E)acc[i][j][4 * g + 3]));
}

// Split-K, second half (its own launch, so the slots are visible device-wide).
// One workgroup per 32-row block of a GEMM wave's sub-tile (tiles x NW x TM
// workgroups, so every CU reads) runs the same epilogue the unsplit kernel
// runs, on the sum of the ksplit slots. Its kSumWaves waves load the slots
// at once: wave r sums splits r, r + kSumWaves, ... in increasing order, and
// wave 0 adds the other waves' sums, taken through LDS, in wave order. The
// floating-point order is fixed (results do not depend on scheduling), and all
// the slots' loads are in flight together: one wave taking the splits two at a
// time waited for ksplit / 2 round trips.
constexpr int kSumWaves = 4;
template <int MODE, int BM, int BN, int WM, int WN, int EPI, int OUT>
__global__ __launch_bounds__(64 * kSumWaves) void gemm_splitk_reduce(GemmParams p) {
  using MF = Mfma<MODE>;
  typedef typename MF::acc acc_t;
  using E = typename std::conditional<MODE == kInt8, int, float>::type;
  constexpr int NW = WM * WN, WTM = BM / WM, WTN = BN / WN, TM = WTM / 32, TN = WTN / 32;
  constexpr int WAVE_U4 = splitk_wave_words<NW, TM, TN>(), TILE_U4 = NW * WAVE_U4;
  __shared__ __attribute__((aligned(16))) uint8_t lds[EpiLds<TN, EPI, OUT>::BYTES];
  __shared__ uint4 sums[kSumWaves - 1][TN * 4][64];  // waves 1.. : lane-contiguous, 1 KiB per store
  const int lane = threadIdx.x & 63, r = threadIdx.x >> 6;
  int b = (int)blockIdx.x;
  const int i = b % TM;
  b /= TM;
  const int wave = b % NW;
  const int tile = b / NW;
  const int tm = tile / p.tiles_n, tn = tile - (tile / p.tiles_n) * p.tiles_n;
  const int wm = wave / WN, wn = wave % WN;
  const int S = p.ksplit;
  const uint4* src = (const uint4*)p.partial + (int64_t)tile * S * TILE_U4 + wave * WAVE_U4 + i * TN * 4 * 64 + lane;
  acc_t acc[1][TN];
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[0][j][e] = 0;
  auto add4 = [&](int j, int g, const uint4 v) {
    acc[0][j][4 * g] = (E)acc[0][j][4 * g] + __builtin_bit_cast(E, v.x);
    acc[0][j][4 * g + 1] = (E)acc[0][j][4 * g + 1] + __builtin_bit_cast(E, v.y);
    acc[0][j][4 * g + 2] = (E)acc[0][j][4 * g + 2] + __builtin_bit_cast(E, v.z);
    acc[0][j][4 * g + 3] = (E)acc[0][j][4 * g + 3] + __builtin_bit_cast(E, v.w);
  };
#pragma unroll 2
  for (int s = r; s < S; s += kSumWaves) {
    uint4 u[TN * 4];
#pragma unroll
    for (int w = 0; w < TN * 4; ++w) u[w] = src[(int64_t)s * TILE_U4 + w * 64];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) add4(j, g, u[j * 4 + g]);
  }
  if (r > 0 && r < S) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        sums[r - 1][j * 4 + g][lane] =
            make_uint4(__builtin_bit_cast(uint32_t, (E)acc[0][j][4 * g]), __builtin_bit_cast(uint32_t, (E)acc[0][j][4 * g + 1]),
                       __builtin_bit_cast(uint32_t, (E)acc[0][j][4 * g + 2]), __builtin_bit_cast(uint32_t, (E)acc[0][j][4 * g + 3]));
  }
  __syncthreads();
  if (r != 0) return;  // no barrier follows: the epilogue is wave-local
  const int nsum = S < kSumWaves ? S : kSumWaves;
  for (int q = 1; q < nsum; ++q)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) add4(j, g, sums[q - 1][j * 4 + g][lane]);
  epilogue<MODE, 1, TN, EPI, OUT>(p, acc, (int64_t)tm * BM + wm * WTM + i * 32, (int64_t)tn * BN + wn * WTN, lane, lds);
}

// Persistent form of the pipelined kernel: one workgroup per CU walks the
// tiles blockIdx.x, + gridDim.x, ... and issues the next tile's DMA prologue
// inside the current tile's epilogue, whose rows are then staged in an LDS
// region of their own beside the stages (padded rows when they fit, else the
// packed layout). Only where that region fits into the 160 KiB of LDS, for
// 16-bit outputs of the dequantizing epilogues, and never with split-K.
constexpr int kLdsBytes = 160 * 1024;
template <int MODE, int BM, int BN, int WM, int WN, int EPI, int OUT, int BK>
struct PersistLayout {
  static constexpr int NW = WM * WN, TN = BN / WN / 32;
  static constexpr int STAGES = kStages * (BM + BN) * BK;
  using Pad = EpiLds<TN, EPI, OUT, false>;
  static constexpr bool kPadFits = STAGES + NW * Pad::BYTES <= kLdsBytes;
  static constexpr bool kPackable = (Pad::CPR & (Pad::CPR - 1)) == 0;
  static constexpr bool PACK = !kPadFits && kPackable;
  using E = EpiLds<TN, EPI, OUT, PACK>;
  static constexpr bool value =
      !kSplitTile<BM, BN> && EPI != kEpiRaw && OUT != kF32 && STAGES + NW * E::BYTES <= kLdsBytes;
};

// WALK: the persistent form (one workgroup per CU walking tiles; only where PersistLayout allows it).
// Otherwise one workgroup per tile, whose epilogue stages its rows in the freed stage memory.
template <int MODE, int BM, int BN, int WM, int WN, int EPI, int OUT, int BK, bool WALK>
__global__ __launch_bounds__(WM* WN * 64, 1) void gemm_w8a8_dma(GemmParams p) {
  using MF = Mfma<MODE>;
  typedef typename MF::frag frag_t;
  typedef typename MF::acc acc_t;
  constexpr int NW = WM * WN;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  constexpr int A_BYTES = BM * BK, B_BYTES = BN * BK, STAGE = A_BYTES + B_BYTES;
  constexpr int A_DMA = A_BYTES / (1024 * NW), B_DMA = B_BYTES / (1024 * NW);
  constexpr int DPS = A_DMA + B_DMA;            // DMA instructions per wave per step
  constexpr int CPR = BK / 16, RPD = 64 / CPR;  // 16-byte chunks per row, rows per DMA instruction
  constexpr int SUB = MODE == kInt8 ? BK / 32 : BK / 64;  // MFMAs along K per step
  constexpr int FW = MODE == kInt8 ? 1 : 2;     // 16-byte LDS words per MFMA operand
  constexpr int NMF = SUB * TM * TN;            // MFMAs per step
  // MFMAs issued before the barrier (cover the waves' skew at it); 4 for the three-column-block tiles
  // (256x192: QKV 107.7 -> 101.1 us at M = 4096, same box) and the FP8 128-byte-step tile (M = 128
  // question GEMMs: 1-3%), 2 elsewhere (256x256 unchanged by 4)
  constexpr int PRE = (TN == 3 || (BK == 128 && MODE == kFp8)) ? 4 : (NMF >= 4 ? 2 : 1);
  constexpr int SLOTS = NMF - PRE;
  constexpr int NBW = SUB * TN * FW;            // B words read per step
  static_assert(A_BYTES % (1024 * NW) == 0 && B_BYTES % (1024 * NW) == 0, "DMA split");
  static_assert(EPI != kEpiSwiGLU || (TN % 2 == 0), "swiglu needs gate/up block pairs");
  static_assert(SLOTS >= 1, "tile too small for the interleave");
  using PL = PersistLayout<MODE, BM, BN, WM, WN, EPI, OUT, BK>;
  static_assert(!WALK || PL::value, "the persistent form needs room for its epilogue staging");
  constexpr bool PERSIST = WALK;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kStages * STAGE + (PERSIST ? NW * PL::E::BYTES : 0)];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;
  // ksplit consecutive workgroups share a tile, split s taking K steps [s nk/S, (s+1) nk/S).
  // Only the 128x128 tiles carry the split path (the 256-row tiles hold too many accumulators to
  // add it without spilling).
  const int S = kSplitTile<BM, BN> ? p.ksplit : 1;
  const int split = kSplitTile<BM, BN> ? (int)blockIdx.x % S : 0;
  const int ntiles = p.tiles_m * p.tiles_n;
  int tile = kSplitTile<BM, BN> ? (int)blockIdx.x / S : (int)blockIdx.x;
  int tm, tn;
  int64_t m0, n0;
  const int nk_all = (int)(p.K / BK);
  const int kbeg = kSplitTile<BM, BN> ? (int)((int64_t)split * nk_all / S) : 0;
  // >= 1: the host keeps S <= nk_all
  const int nk = kSplitTile<BM, BN> ? (int)((int64_t)(split + 1) * nk_all / S) - kbeg : nk_all;
  const int lrow = lane & 31, lhalf = lane >> 5;

  // DMA sources: uniform tile bases + per-lane 32-bit offsets (the host keeps every operand
  // offset below 2^32 for this kernel). Each operand is row-major or K-blocked (QDst, kernels.hpp):
  // byte (m, k) at m * rs + (k / 64) * bs + k % 64.
  const uint8_t* a_base;
  const uint8_t* b_base;
  uint32_t a_off[A_DMA], b_off[B_DMA];
  const int64_t a_rs = p.a_kblk ? 64 : p.lda, a_bs = p.a_kblk ? 64 * p.lda : 64;
  const int64_t b_rs = p.w_kblk ? 64 : p.ldw, b_bs = p.w_kblk ? 64 * p.ldw : 64;
  const int64_t a_step = (BK / 64) * a_bs, b_step = (BK / 64) * b_bs;  // bytes per K step
  auto setup = [&](int t) {
    if constexpr (kSplitTile<BM, BN>) tile_of(t, (int)gridDim.x / S, p.tiles_m, p.tiles_n, tm, tn);
    else tile_of(t, ntiles, p.tiles_m, p.tiles_n, tm, tn);
    m0 = (int64_t)tm * BM;
    n0 = (int64_t)tn * BN;
    a_base = uniform_ptr(p.a + m0 * a_rs + (int64_t)kbeg * a_step);
    b_base = uniform_ptr(p.w + n0 * b_rs + (int64_t)kbeg * b_step);
#pragma unroll
    for (int i = 0; i < A_DMA; ++i) {
      const int row = (i * NW + wave) * RPD + lane / CPR;
      const int ch = (lane % CPR) ^ lds_swz<BK>(row);  // logical 16-byte chunk of the step's K bytes
      a_off[i] = (uint32_t)((min(m0 + row, p.M - 1) - m0) * a_rs + (ch >> 2) * a_bs + (ch & 3) * 16);
    }
#pragma unroll
    for (int i = 0; i < B_DMA; ++i) {
      const int row = (i * NW + wave) * RPD + lane / CPR;
      const int ch = (lane % CPR) ^ lds_swz<BK>(row);
      b_off[i] = (uint32_t)((min(n0 + row, p.N - 1) - n0) * b_rs + (ch >> 2) * b_bs + (ch & 3) * 16);
    }
  };
  setup(tile);
  const uint32_t lds_wave =
      __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)D3_LDS_PTR(lds) + (uint32_t)wave * 1024u);

  // DMA d of step kt into stage U
  auto dma_one = [&](auto u_c, auto d_c, int kt) {
    constexpr int U = decltype(u_c)::value % kStages, d = decltype(d_c)::value;
    if constexpr (d < A_DMA) dma16<U * STAGE + d * NW * 1024>(a_base + (int64_t)kt * a_step, a_off[d], lds_wave);
    else dma16<U * STAGE + A_BYTES + (d - A_DMA) * NW * 1024>(b_base + (int64_t)kt * b_step, b_off[d - A_DMA], lds_wave);
  };
  auto dma_stage = [&](auto u_c, int kt) { static_for<0, DPS>([&](auto d_c) { dma_one(u_c, d_c, kt); }); };

  acc_t acc[TM][TN];
  frag_t fa[SUB][TM];     // A operands of the current step (single buffer)
  frag_t fb[2][SUB][TN];  // B operands, by step parity

  // A word (s, i, h) / B word w of stage U (h: 16-byte half of an FP8 operand)
  auto read_a = [&](auto u_c, auto s_c, auto i_c, auto h_c) {
    constexpr int U = decltype(u_c)::value % kStages, s = decltype(s_c)::value;
    constexpr int i = decltype(i_c)::value, h = decltype(h_c)::value;
    const int chunk = MODE == kInt8 ? 2 * s + lhalf : 4 * s + 2 * lhalf + h;
    const v4i v = *(const v4i*)(lds + U * STAGE + lds_offk<BK>(wm * WTM + i * 32 + lrow, chunk));
    if constexpr (MODE == kInt8) fa[s][i] = v;
    else if constexpr (h == 0) fa[s][i].lo = v;
    else fa[s][i].hi = v;
  };
  auto read_b = [&](auto u_c, auto p_c, auto w_c) {
    constexpr int U = decltype(u_c)::value % kStages, P = decltype(p_c)::value, w = decltype(w_c)::value;
    constexpr int s = w / (TN * FW), j = (w / FW) % TN, h = w % FW;
    const int chunk = MODE == kInt8 ? 2 * s + lhalf : 4 * s + 2 * lhalf + h;
    const v4i v = *(const v4i*)(lds + U * STAGE + A_BYTES + lds_offk<BK>(wn * WTN + j * 32 + lrow, chunk));
    if constexpr (MODE == kInt8) fb[P][s][j] = v;
    else if constexpr (h == 0) fb[P][s][j].lo = v;
    else fb[P][s][j].hi = v;
  };
  // all operands of one step (prologue)
  auto read_all = [&](auto u_c, auto p_c) {
    static_for<0, SUB>([&](auto s_c) {
      static_for<0, TM>([&](auto i_c) {
        static_for<0, FW>([&](auto h_c) { read_a(u_c, s_c, i_c, h_c); });
      });
    });
    static_for<0, NBW>([&](auto w_c) { read_b(u_c, p_c, w_c); });
  };
  auto mfma_q = [&](auto p_c, auto q_c) {
    constexpr int P = decltype(p_c)::value, q = decltype(q_c)::value;
    constexpr int s = q / (TM * TN), i = (q / TN) % TM, j = q % TN;
    acc[i][j] = MF::run(fb[P][s][j], fa[s][i], acc[i][j]);
  };

  // Step kt with operands in stage U = kt % 4 and B parity P = kt & 1.
  auto step = [&](auto u_c, auto chk_c, int kt) {
    constexpr int U = decltype(u_c)::value;
    constexpr int P = U & 1;
    constexpr bool CHECKED = decltype(chk_c)::value;
    static_for<0, PRE>([&](auto q_c) { mfma_q(std::integral_constant<int, P>{}, q_c); });
    __builtin_amdgcn_sched_barrier(0);
    const bool rd = !CHECKED || kt + 1 < nk;
    const bool fetch = !CHECKED || kt + kStages < nk;
    wait_lgkm0();
    if constexpr (!CHECKED) {
      wait_vmcnt<2 * DPS>();
    } else {
      const int after = min(kStages - 2, nk - 2 - kt);  // DMA steps issued after step kt+1
      if (after >= 2) wait_vmcnt<2 * DPS>();
      else if (after == 1) wait_vmcnt<DPS>();
      else wait_vmcnt<0>();
    }
    lds_barrier();
    static_for<PRE, NMF>([&](auto q_c) {
      constexpr int q = decltype(q_c)::value, k = q - PRE;
      mfma_q(std::integral_constant<int, P>{}, q_c);
      // B words of the next step in this slot's share
      static_for<k * NBW / SLOTS, (k + 1) * NBW / SLOTS>([&](auto w_c) {
        if (rd) read_b(std::integral_constant<int, U + 1>{}, std::integral_constant<int, P ^ 1>{}, w_c);
      });
      // A operand (s, i) of the next step once its last MFMA of this step has issued
      static_for<0, SUB * TM>([&](auto a_c) {
        constexpr int s = decltype(a_c)::value / TM, i = decltype(a_c)::value % TM;
        constexpr int last = s * TM * TN + i * TN + TN - 1;
        if constexpr ((last < PRE ? PRE : last) == q) {
          static_for<0, FW>([&](auto h_c) {
            if (rd) read_a(std::integral_constant<int, U + 1>{}, std::integral_constant<int, s>{},
                           std::integral_constant<int, i>{}, h_c);
          });
        }
      });
      // DMA of step kt+4 into stage U, in this slot's share
      static_for<k * DPS / SLOTS, (k + 1) * DPS / SLOTS>([&](auto d_c) {
        if (fetch) dma_one(u_c, d_c, kt + kStages);
      });
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // Prologue: DMA of steps 0..3 fills every stage; then the operands of step 0.
  auto prologue_dma = [&] {
    dma_stage(std::integral_constant<int, 0>{}, 0);
    if (nk > 1) dma_stage(std::integral_constant<int, 1>{}, 1);
    if (nk > 2) dma_stage(std::integral_constant<int, 2>{}, 2);
    if (nk > 3) dma_stage(std::integral_constant<int, 3>{}, 3);
  };
  prologue_dma();
  bool first = true;
  for (;;) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
    if (first) {
      const int after = min(kStages - 1, nk - 1);  // DMA steps issued after step 0
      if (after >= 3) wait_vmcnt<3 * DPS>();
      else if (after == 2) wait_vmcnt<2 * DPS>();
      else if (after == 1) wait_vmcnt<DPS>();
      else wait_vmcnt<0>();
    } else {
      wait_vmcnt<0>();  // this tile's prologue DMA (issued in the last epilogue) and that epilogue's stores
    }
    first = false;
    lds_barrier();
    read_all(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});

    using Steady = std::integral_constant<bool, false>;
    using Checked = std::integral_constant<bool, true>;
    int kt0 = 0;
    for (; kt0 + 2 * kStages <= nk; kt0 += 4) {
      step(std::integral_constant<int, 0>{}, Steady{}, kt0);
      step(std::integral_constant<int, 1>{}, Steady{}, kt0 + 1);
      step(std::integral_constant<int, 2>{}, Steady{}, kt0 + 2);
      step(std::integral_constant<int, 3>{}, Steady{}, kt0 + 3);
    }
    for (; kt0 < nk; kt0 += 4) {
      step(std::integral_constant<int, 0>{}, Checked{}, kt0);
      if (kt0 + 1 < nk) step(std::integral_constant<int, 1>{}, Checked{}, kt0 + 1);
      if (kt0 + 2 < nk) step(std::integral_constant<int, 2>{}, Checked{}, kt0 + 2);
      if (kt0 + 3 < nk) step(std::integral_constant<int, 3>{}, Checked{}, kt0 + 3);
    }

    if constexpr (kSplitTile<BM, BN>) {
      if (S > 1) {
        splitk_store<MODE, NW, TM, TN>(p, acc, tm * p.tiles_n + tn, split, wave, lane);
        return;
      }
    }
    // every wave has finished reading the stages (before they take the epilogue's rows, or the next
    // tile's DMA)
    wait_lgkm0();
    lds_barrier();
    if constexpr (PERSIST) {
      const int next = tile + (int)gridDim.x;
      const bool more = next < ntiles;  // uniform over the workgroup
      const int64_t wrow0 = m0 + wm * WTM, wcol0 = n0 + wn * WTN;
      static_assert(kStages * STAGE + NW * PL::E::BYTES <= (int)sizeof(lds), "epilogue staging");
      epilogue<MODE, TM, TN, EPI, OUT, PL::PACK>(p, acc, wrow0, wcol0, lane, lds + kStages * STAGE + wave * PL::E::BYTES,
                                                 [&] {
                                                   if (more) {
                                                     // the epilogue's scales have landed, so its later
                                                     // waits do not cover this DMA
                                                     asm volatile("" ::: "memory");
                                                     wait_vmcnt<0>();
                                                     setup(next);
                                                     prologue_dma();
                                                   }
                                                 });
      if (!more) return;
      tile = next;
    } else {
      static_assert(NW * EpiLds<TN, EPI, OUT>::BYTES <= (int)sizeof(lds), "epilogue staging");
      epilogue<MODE, TM, TN, EPI, OUT>(p, acc, m0 + wm * WTM, n0 + wn * WTN, lane,
                                       lds + wave * EpiLds<TN, EPI, OUT>::BYTES);
      return;
    }
  }
}

// ---------------------------------------------------------------------------
// host side: tile-config selection and dispatch
// ---------------------------------------------------------------------------

template <int MODE, int BM, int BN, int WM, int WN, int EPI, int OUT>
static hipError_t launch_cfg(GemmParams p, hipStream_t st) {
  p.tiles_m = (int)((p.M + BM - 1) / BM);
  p.tiles_n = (int)((p.N + BN - 1) / BN);
  const int64_t nb = (int64_t)p.tiles_m * p.tiles_n;
  hipLaunchKernelGGL((gemm_w8a8<MODE, BM, BN, WM, WN, EPI, OUT>), dim3((unsigned)nb), dim3(WM * WN * 64), 0, st, p);
  return hipGetLastError();
}

template <int MODE, int BM, int BN, int WM, int WN, int EPI, int OUT, int BK = 64>
static hipError_t launch_dma(GemmParams p, hipStream_t st) {
  p.tiles_m = (int)((p.M + BM - 1) / BM);
  p.tiles_n = (int)((p.N + BN - 1) / BN);
  const int64_t tiles = (int64_t)p.tiles_m * p.tiles_n;
  // the walk is built for the 256-row tiles it was measured on; the 192-row tiles always run one
  // workgroup per tile (fewer kernels to compile)
  if constexpr (PersistLayout<MODE, BM, BN, WM, WN, EPI, OUT, BK>::value && BM == 256) {
    // one workgroup per CU; a multiple of the 8 XCDs keeps each workgroup's tiles on its own XCD
    const int64_t cus = device_cu_count() & ~7;
    if (gemm_persistent() && cus >= 8 && tiles > cus) {
      hipLaunchKernelGGL((gemm_w8a8_dma<MODE, BM, BN, WM, WN, EPI, OUT, BK, true>), dim3((unsigned)cus),
                         dim3(WM * WN * 64), 0, st, p);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((gemm_w8a8_dma<MODE, BM, BN, WM, WN, EPI, OUT, BK, false>), dim3((unsigned)(tiles * p.ksplit)),
                     dim3(WM * WN * 64), 0, st, p);
  if (kSplitTile<BM, BN> && p.ksplit > 1) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    constexpr int WAVE_BLOCKS = WM * WN * (BM / WM / 32);  // reduce workgroups per tile
    hipLaunchKernelGGL((gemm_splitk_reduce<MODE, BM, BN, WM, WN, EPI, OUT>), dim3((unsigned)(tiles * WAVE_BLOCKS)),
                       dim3(64 * kSumWaves), 0, st, p);
  }
  return hipGetLastError();
}

template <int MODE, int EPI, int OUT>
static hipError_t launch_ws(GemmParams p, hipStream_t st);  // gemm_ws.hpp

template <int MODE, int EPI, int OUT>
hipError_t launch_epi(GemmParams p, int tile, hipStream_t st) {
  if (p.ksplit < 1 || (p.ksplit > 1 && tile < kDma256w8)) return hipErrorInvalidValue;
  switch (tile) {
    case kTile256: return launch_cfg<MODE, 256, 256, 2, 2, EPI, OUT>(p, st);
    case kTile128: return launch_cfg<MODE, 128, 128, 2, 2, EPI, OUT>(p, st);
    case kTile64x128: return launch_cfg<MODE, 64, 128, 2, 2, EPI, OUT>(p, st);
    case kDma256w8: return launch_dma<MODE, 256, 256, 2, 4, EPI, OUT>(p, st);
    case kDma256w4: return launch_dma<MODE, 256, 256, 2, 2, EPI, OUT>(p, st);
    case kDma128w4: return launch_dma<MODE, 128, 128, 2, 2, EPI, OUT>(p, st);
    case kDma256x128w4: return launch_dma<MODE, 256, 128, 2, 2, EPI, OUT>(p, st);
    case kDma128w4k128: return launch_dma<MODE, 128, 128, 2, 2, EPI, OUT, 128>(p, st);
    case kDma256x192w4:
      if constexpr (EPI == kEpiSwiGLU) return hipErrorInvalidValue;  // 3 column blocks per wave: no gate/up pairs
      else return launch_dma<MODE, 256, 192, 2, 2, EPI, OUT>(p, st);
    case kWs: return launch_ws<MODE, EPI, OUT>(p, st);
    case kDma192x192w4:
      if constexpr (EPI == kEpiSwiGLU) return hipErrorInvalidValue;  // 3 column blocks per wave: no gate/up pairs
      else return launch_dma<MODE, 192, 192, 2, 2, EPI, OUT>(p, st);
    case kDma192x128w4: return launch_dma<MODE, 192, 128, 2, 2, EPI, OUT>(p, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace d3

#include "gemm_ws.hpp"
