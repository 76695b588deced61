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
//     v_mfma_scale_f32_32x32x64_f8f6f4 with format E4M3 and unit scales (FP8).
//     Operand lane l carries row (l & 31) and the K chunk selected by l >> 5;
//     A and B use the same K assignment, so the dot product is complete.
//   * Result lane layout (32x32 blocks): register r of lane l is
//     row 8*(r/4) + 4*(l/32) + (r%4), column l%32.
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
//             and row_amax[m] = max(row_amax[m], |h|) by atomic max.
//   residual: out = OUT( float(res[m, n]) + OUT(deq(acc)) )         (core.py:215)
#include "common.hpp"
#include "kernels.hpp"

#include <type_traits>

namespace d3 {


constexpr int kBK = 128;  // bytes of K per pipeline step
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
    // format 0 = FP8 E4M3 for both operands; E8M0 scale 127 = 1.0
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
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

// Epilogue shared by the GEMM kernels. acc[i][j] is the 32x32 MFMA block at
// rows wrow0 + 32 i, columns wcol0 + 32 j of the output; register r of lane l
// holds row 8*(r/4) + 4*(l/32) + (r%4), column l%32 of its block.
//
// vmcnt counts loads and stores in issue order, so a load issued after stores
// waits for them too: every token scale, row-map entry and channel scale the
// tile needs is loaded before the first store (residuals per 32-row block).
// FULL (the whole wave tile lies inside the output) drops every per-element
// predicate, so the stores are straight-line code with no waits between them.
template <int MODE, int TM, int TN, int EPI, int OUT, bool FULL, bool MAP, typename ACC>
__device__ __forceinline__ void epilogue_impl(const GemmParams& p, ACC (&acc)[TM][TN], int64_t wrow0, int64_t wcol0,
                                              int lane) {
  const int64_t M = p.M, N = p.N;
  const int lrow = lane & 31, lhalf = lane >> 5;
  const float* __restrict__ a_scale = p.a_scale;
  const float* __restrict__ w_scale = p.w_scale;
  const int32_t* __restrict__ row_map = p.row_map;
  auto row_of = [&](int i, int r) -> int64_t { return wrow0 + i * 32 + (r >> 2) * 8 + lhalf * 4 + (r & 3); };

  if constexpr (EPI == kEpiSwiGLU) {
    float sg[TN / 2], su[TN / 2];
    int64_t hcol[TN / 2];
    bool cok[TN / 2];
#pragma unroll
    for (int jp = 0; jp < TN / 2; ++jp) {
      const int64_t cg = wcol0 + (2 * jp) * 32 + lrow;  // interleaved gate column; its up column is cg + 32
      cok[jp] = FULL || cg + 32 < N;
      hcol[jp] = (cg >> 6) * 32 + (cg & 31);
      sg[jp] = cok[jp] ? w_scale[cg] : 0.0f;
      su[jp] = cok[jp] ? w_scale[cg + 32] : 0.0f;
    }
    // all token scales up front when the accumulators leave room (AGPR-resident tiles), else per block
    constexpr bool kHoist = TM * TN * 16 > 128;
    float st[kHoist ? TM : 1][16];
    auto load_st = [&](int i, float* dst) {
#pragma unroll
      for (int r = 0; r < 16; ++r) dst[r] = (FULL || row_of(i, r) < M) ? a_scale[row_of(i, r)] : 0.0f;
    };
    if constexpr (kHoist) {
#pragma unroll
      for (int i = 0; i < TM; ++i) load_st(i, st[i]);
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      if constexpr (!kHoist) load_st(i, st[0]);
      float* sti = st[kHoist ? i : 0];
      float rmax[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        rmax[r] = 0.0f;
        const int64_t row = row_of(i, r);
#pragma unroll
        for (int jp = 0; jp < TN / 2; ++jp) {
          if (FULL || (row < M && cok[jp])) {
            float g = (float)acc[i][2 * jp][r];
            g = g * sti[r];
            g = round_to<OUT>(g * sg[jp]);
            float u = (float)acc[i][2 * jp + 1][r];
            u = u * sti[r];
            u = round_to<OUT>(u * su[jp]);
            const float e = expf(-g);
            const float den = 1.0f + e;
            const float sl = round_to<OUT>(g / den);
            const float h = round_to<OUT>(sl * u);
            store_elem<OUT>(p.out, row * p.ldo + hcol[jp], h);
            rmax[r] = fmaxf(rmax[r], fabsf(h));
          }
        }
      }
      if (p.row_amax) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float v = rmax[r];
#pragma unroll
          for (int o = 1; o < 32; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
          const int64_t row = row_of(i, r);
          if (lrow == 0 && (FULL || row < M)) atomicMax((unsigned int*)(p.row_amax + row), __float_as_uint(v));
        }
      }
    }
  } else {
    float sc[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t col = wcol0 + j * 32 + lrow;
      sc[j] = (EPI != kEpiRaw && (FULL || col < N)) ? w_scale[col] : 0.0f;
    }
    // all token scales / output rows up front when the accumulators leave room, else per block
    constexpr bool kHoist = TM * TN * 16 > 128;
    float st_[kHoist ? TM : 1][16];
    int32_t orow_[kHoist ? TM : 1][16];
    auto load_rows = [&](int i, float* st, int32_t* orow) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = row_of(i, r);
        const bool ok = FULL || row < M;
        if constexpr (MAP) orow[r] = ok ? row_map[row] : -1;
        else orow[r] = ok ? (int32_t)row : -1;
        st[r] = (EPI != kEpiRaw && ok) ? a_scale[row] : 0.0f;
      }
    };
    if constexpr (kHoist) {
#pragma unroll
      for (int i = 0; i < TM; ++i) load_rows(i, st_[i], orow_[i]);
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      if constexpr (!kHoist) load_rows(i, st_[0], orow_[0]);
      const float* st = st_[kHoist ? i : 0];
      const int32_t* orow = orow_[kHoist ? i : 0];
      float res[EPI == kEpiResidual ? 16 : 1][EPI == kEpiResidual ? TN : 1];
      if constexpr (EPI == kEpiResidual) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            const int64_t col = wcol0 + j * 32 + lrow;
            res[r][j] = (FULL || (orow[r] >= 0 && col < N)) ? load_elem<OUT>(p.res, (int64_t)orow[r] * p.ldr + col)
                                                              : 0.0f;
          }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        if (!FULL && orow[r] < 0) continue;
        const int64_t obase = (int64_t)orow[r] * p.ldo;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int64_t col = wcol0 + j * 32 + lrow;
          if (!FULL && col >= N) continue;
          if constexpr (EPI == kEpiRaw) {
            if constexpr (MODE == kInt8) ((int32_t*)p.out)[obase + col] = acc[i][j][r];
            else ((float*)p.out)[obase + col] = acc[i][j][r];
          } else {
            float v = (float)acc[i][j][r];
            v = v * st[r];
            v = v * sc[j];
            if constexpr (EPI == kEpiResidual) {
              v = round_to<OUT>(v);
              v = res[r][j] + v;
            }
            store_elem<OUT>(p.out, obase + col, v);
          }
        }
      }
    }
  }
}

template <int MODE, int TM, int TN, int EPI, int OUT, typename ACC>
__device__ __forceinline__ void epilogue(const GemmParams& p, ACC (&acc)[TM][TN], int64_t wrow0, int64_t wcol0,
                                         int lane) {
  const bool full = wrow0 + TM * 32 <= p.M && wcol0 + TN * 32 <= p.N;
  if constexpr (EPI == kEpiSwiGLU) {
    if (full) epilogue_impl<MODE, TM, TN, EPI, OUT, true, false>(p, acc, wrow0, wcol0, lane);
    else epilogue_impl<MODE, TM, TN, EPI, OUT, false, false>(p, acc, wrow0, wcol0, lane);
  } else if (p.row_map) {
    if (full) epilogue_impl<MODE, TM, TN, EPI, OUT, true, true>(p, acc, wrow0, wcol0, lane);
    else epilogue_impl<MODE, TM, TN, EPI, OUT, false, true>(p, acc, wrow0, wcol0, lane);
  } else {
    if (full) epilogue_impl<MODE, TM, TN, EPI, OUT, true, false>(p, acc, wrow0, wcol0, lane);
    else epilogue_impl<MODE, TM, TN, EPI, OUT, false, false>(p, acc, wrow0, wcol0, lane);
  }
}

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
        for (int j = 0; j < TN; ++j) acc[i][j] = MF::run(af[i], bf[j], acc[i][j]);
    }
    if (kt + 1 < nk) swrite(buf ^ 1);
    __syncthreads();
  }

  epilogue<MODE, TM, TN, EPI, OUT>(p, acc, m0 + wm * WTM, n0 + wn * WTN, lane);
}


// ---------------------------------------------------------------------------
// Pipelined kernel (K % 64 == 0): 64-byte K steps, STAGES LDS buffers filled
// by direct global->LDS DMA (global_load_lds_dwordx4), one barrier per step.
//
//   * Each DMA instruction of a wave writes 1 KiB of LDS (64 lanes x 16 B):
//     16 rows of 64 bytes. Lane j carries row r0 + j/4 and physical chunk
//     j%4, i.e. logical K chunk (j%4) ^ ((row >> 2) & 3): the XOR swizzle that
//     makes the MFMA operand reads (one 16-byte chunk of 32 consecutive rows)
//     conflict-free (a ds_read_b128 serves 16 lanes per cycle from 64 banks).
//   * Rows past M (or N) are clamped to the last row: they only feed output
//     rows (columns) that are never stored.
//   * Fragments are double-buffered in registers: step t reads the MFMA
//     operands of step t+1 from LDS while its own MFMAs (operands read during
//     step t-1) run, so LDS latency hides behind the matrix pipe.
//   * Step t waits for the DMA of step t+1 (vmcnt counts only this wave's
//     DMA, so the wait is followed by a barrier); after that barrier every
//     wave has finished reading stage t (its reads completed before step t-1
//     ended), so the DMA of step t+STAGES goes into stage t: three steps of lead.
//   * The stage buffers are separate __shared__ arrays and the K loop is
//     unrolled by STAGES, so the compiler sees which buffer each access uses
//     and adds no waits of its own beyond the explicit ones; sched_barrier
//     keeps the read / MFMA / wait phases in program order.
// ---------------------------------------------------------------------------
constexpr int kBK2 = 64;

// 64-byte rows: the 16 lanes of one ds_read_b128 cycle read rows r..r+15 (four rows per 256-byte bank
// line); XOR-ing the chunk with (row >> 2) & 3 spreads them over the 16 bank groups.
__device__ __forceinline__ int lds_off64(int row, int chunk) { return row * kBK2 + ((chunk ^ ((row >> 2) & 3)) << 4); }

// s_barrier without the fence __syncthreads() adds (whose vmcnt(0) would drain
// the DMA pipeline); the empty asm keeps the compiler from moving LDS accesses
// across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  // s_waitcnt encoding (gfx9): vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

#define D3_LDS_PTR(p) ((__attribute__((address_space(3))) const void*)(p))

// One wave-wide 16-byte-per-lane DMA: lane l's 16 bytes at gsrc land at LDS
// lds_dst + 16 l. Issued as inline asm so the compiler does not model the LDS
// write: it would otherwise insert vmcnt(0) before LDS reads it cannot prove
// disjoint (draining the whole pipeline); every wait on this DMA is explicit
// (wait_vmcnt + s_barrier) in the kernel. M0 holds the LDS base; the s_nop
// covers the M0-write -> LDS-DMA hazard.
__device__ __forceinline__ void dma16(const void* gsrc, const uint8_t* lds_dst) {
  const uint32_t m0 = (uint32_t)(uintptr_t)D3_LDS_PTR(lds_dst);
  asm volatile(
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, off"
      :
      : "v"(gsrc), "s"(__builtin_amdgcn_readfirstlane(m0))
      : "memory", "m0");
}

template <int MODE, int BM, int BN, int WM, int WN, int STAGES, int EPI, int OUT>
__global__ __launch_bounds__(WM* WN * 64, 1) void gemm_w8a8_dma(GemmParams p) {
  using MF = Mfma<MODE>;
  typedef typename MF::frag frag_t;
  typedef typename MF::acc acc_t;
  constexpr int NW = WM * WN;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  constexpr int A_BYTES = BM * kBK2, B_BYTES = BN * kBK2;
  constexpr int A_DMA = A_BYTES / (1024 * NW), B_DMA = B_BYTES / (1024 * NW);
  constexpr int DPS = A_DMA + B_DMA;  // DMA instructions per wave per stage
  constexpr int SUB = (MODE == kInt8) ? 2 : 1;  // MFMAs along K per 64-byte step
  static_assert(A_BYTES % (1024 * NW) == 0 && B_BYTES % (1024 * NW) == 0, "DMA split");
  static_assert(STAGES == 4, "the step unroll below assumes 4 stages");
  static_assert(EPI != kEpiSwiGLU || (TN % 2 == 0), "swiglu needs gate/up block pairs");
  __shared__ __attribute__((aligned(1024))) uint8_t st0[A_BYTES + B_BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t st1[A_BYTES + B_BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t st2[A_BYTES + B_BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t st3[STAGES > 3 ? A_BYTES + B_BYTES : 16];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;
  int tm, tn;
  tile_of(blockIdx.x, gridDim.x, p.tiles_m, p.tiles_n, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int nk = (int)(p.K / kBK2);

  // per-lane DMA source rows (clamped) and K-chunk byte offsets
  const uint8_t* a_src[A_DMA];
  const uint8_t* b_src[B_DMA];
#pragma unroll
  for (int i = 0; i < A_DMA; ++i) {
    const int row = (i * NW + wave) * 16 + (lane >> 2);
    const int ch = (lane & 3) ^ ((row >> 2) & 3);
    const int64_t gm = min(m0 + row, p.M - 1);
    a_src[i] = p.a + gm * p.lda + ch * 16;
  }
#pragma unroll
  for (int i = 0; i < B_DMA; ++i) {
    const int row = (i * NW + wave) * 16 + (lane >> 2);
    const int ch = (lane & 3) ^ ((row >> 2) & 3);
    const int64_t gn = min(n0 + row, p.N - 1);
    b_src[i] = p.w + gn * p.ldw + ch * 16;
  }

  auto dma = [&](uint8_t* stage, int kt) {
    const int64_t kb = (int64_t)kt * kBK2;
#pragma unroll
    for (int i = 0; i < A_DMA; ++i) dma16(a_src[i] + kb, stage + (i * NW + wave) * 1024);
#pragma unroll
    for (int i = 0; i < B_DMA; ++i) dma16(b_src[i] + kb, stage + A_BYTES + (i * NW + wave) * 1024);
  };

  acc_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  const int lrow = lane & 31, lhalf = lane >> 5;
  // fragments of one 64-byte K step: SUB MFMA K-slices x (TM A blocks, TN B blocks)
  struct Frags {
    frag_t a[SUB][TM];
    frag_t b[SUB][TN];
  };
  auto read_frags = [&](const uint8_t* stage, Frags& f) {
    const uint8_t* sa = stage;
    const uint8_t* sb = stage + A_BYTES;
#pragma unroll
    for (int s = 0; s < SUB; ++s) {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = wm * WTM + i * 32 + lrow;
        if constexpr (MODE == kInt8) {
          f.a[s][i] = *(const v4i*)(sa + lds_off64(row, 2 * s + lhalf));
        } else {
          const v4i lo = *(const v4i*)(sa + lds_off64(row, 2 * lhalf));
          const v4i hi = *(const v4i*)(sa + lds_off64(row, 2 * lhalf + 1));
          f.a[s][i] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int row = wn * WTN + j * 32 + lrow;
        if constexpr (MODE == kInt8) {
          f.b[s][j] = *(const v4i*)(sb + lds_off64(row, 2 * s + lhalf));
        } else {
          const v4i lo = *(const v4i*)(sb + lds_off64(row, 2 * lhalf));
          const v4i hi = *(const v4i*)(sb + lds_off64(row, 2 * lhalf + 1));
          f.b[s][j] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
      }
    }
  };
  auto mfmas = [&](const Frags& f) {
#pragma unroll
    for (int s = 0; s < SUB; ++s)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = MF::run(f.a[s][i], f.b[s][j], acc[i][j]);
  };
  auto stage_ptr = [&](auto u_c) -> uint8_t* {
    constexpr int U = decltype(u_c)::value % STAGES;
    return U == 0 ? st0 : U == 1 ? st1 : U == 2 ? st2 : st3;
  };

  // Prologue: DMA of steps 0 .. STAGES-1 fills every stage; then the fragments of step 0.
  dma(st0, 0);
  if (nk > 1) dma(st1, 1);
  if (nk > 2) dma(st2, 2);
  if (STAGES > 3 && nk > 3) dma(st3, 3);
  {
    const int after = min(STAGES - 1, nk - 1);  // steps issued after step 0
    if (after >= 3) wait_vmcnt<3 * DPS>();
    else if (after == 2) wait_vmcnt<2 * DPS>();
    else if (after == 1) wait_vmcnt<DPS>();
    else wait_vmcnt<0>();
  }
  lds_barrier();
  Frags f0, f1;
  read_frags(st0, f0);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)

  // Step kt (fragments in registers): wait for stage kt+1, barrier (all waves finished step kt-1,
  // whose fragment reads of stage kt completed before it), DMA step kt+STAGES into the stage of
  // step kt, read the fragments of step kt+1 while the MFMAs of step kt run.
  auto step = [&](auto u_c, int kt, Frags& cur, Frags& nxt) {
    constexpr int U = decltype(u_c)::value;
    if (kt + 1 < nk) {
      const int after = min(STAGES - 2, nk - 2 - kt);  // steps issued after step kt+1
      if (after >= 2) wait_vmcnt<2 * DPS>();
      else if (after == 1) wait_vmcnt<DPS>();
      else wait_vmcnt<0>();
      lds_barrier();
      if (kt + STAGES < nk) dma(stage_ptr(std::integral_constant<int, U>{}), kt + STAGES);
      __builtin_amdgcn_sched_barrier(0);
      read_frags(stage_ptr(std::integral_constant<int, U + 1>{}), nxt);
      __builtin_amdgcn_sched_barrier(0);
    }
    mfmas(cur);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): fragments of step kt+1 are in registers
  };

  for (int kt0 = 0; kt0 < nk; kt0 += 4) {
    step(std::integral_constant<int, 0>{}, kt0, f0, f1);
    if (kt0 + 1 < nk) step(std::integral_constant<int, 1>{}, kt0 + 1, f1, f0);
    if (kt0 + 2 < nk) step(std::integral_constant<int, 2>{}, kt0 + 2, f0, f1);
    if (kt0 + 3 < nk) step(std::integral_constant<int, 3>{}, kt0 + 3, f1, f0);
  }

  epilogue<MODE, TM, TN, EPI, OUT>(p, acc, m0 + wm * WTM, n0 + wn * WTN, lane);
}

// ---------------------------------------------------------------------------
// host side: tile-config selection and dispatch
// ---------------------------------------------------------------------------
enum TileCfg : int {
  kTileAuto = -1,
  kTile256 = 0,      // register-staged 256x256, 4 waves
  kTile128 = 1,      // register-staged 128x128, 4 waves
  kTile64x128 = 2,   // register-staged 64x128, 4 waves
  kDma256w8 = 3,     // DMA pipeline 256x256, 8 waves (128x64 each), 4 stages
  kDma256w4 = 4,     // DMA pipeline 256x256, 4 waves (128x128 each), 4 stages
  kDma128w4 = 5,     // DMA pipeline 128x128, 4 waves (64x64 each), 4 stages
  kDma256x128w4 = 6, // DMA pipeline 256x128, 4 waves (128x64 each), 4 stages
  kTileCount = 7
};

template <int MODE, int BM, int BN, int WM, int WN, int EPI, int OUT>
static hipError_t launch_cfg(GemmParams p, hipStream_t st) {
  p.tiles_m = (int)((p.M + BM - 1) / BM);
  p.tiles_n = (int)((p.N + BN - 1) / BN);
  const int64_t nb = (int64_t)p.tiles_m * p.tiles_n;
  hipLaunchKernelGGL((gemm_w8a8<MODE, BM, BN, WM, WN, EPI, OUT>), dim3((unsigned)nb), dim3(WM * WN * 64), 0, st, p);
  return hipGetLastError();
}

template <int MODE, int BM, int BN, int WM, int WN, int EPI, int OUT>
static hipError_t launch_dma(GemmParams p, hipStream_t st) {
  p.tiles_m = (int)((p.M + BM - 1) / BM);
  p.tiles_n = (int)((p.N + BN - 1) / BN);
  const int64_t nb = (int64_t)p.tiles_m * p.tiles_n;
  hipLaunchKernelGGL((gemm_w8a8_dma<MODE, BM, BN, WM, WN, 4, EPI, OUT>), dim3((unsigned)nb), dim3(WM * WN * 64), 0,
                     st, p);
  return hipGetLastError();
}

static int choose_tile(int64_t M, int64_t N, int64_t K) {
  const int64_t t256 = ((M + 255) / 256) * ((N + 255) / 256);
  const int64_t t128 = ((M + 127) / 128) * ((N + 127) / 128);
  if (K % kBK2 == 0) {
    if (t256 >= 256) return kDma256w8;
    if (t128 >= 192) return kDma128w4;
    return kTile64x128;
  }
  if (t256 >= 256) return kTile256;
  if (t128 >= 192) return kTile128;
  return kTile64x128;
}

template <int MODE, int EPI, int OUT>
static hipError_t launch_epi(GemmParams p, int tile, hipStream_t st) {
  if (tile == kTileAuto) tile = choose_tile(p.M, p.N, p.K);
  if (tile >= kDma256w8 && p.K % kBK2 != 0) return hipErrorInvalidValue;
  switch (tile) {
    case kTile256: return launch_cfg<MODE, 256, 256, 2, 2, EPI, OUT>(p, st);
    case kTile128: return launch_cfg<MODE, 128, 128, 2, 2, EPI, OUT>(p, st);
    case kTile64x128: return launch_cfg<MODE, 64, 128, 2, 2, EPI, OUT>(p, st);
    case kDma256w8: return launch_dma<MODE, 256, 256, 2, 4, EPI, OUT>(p, st);
    case kDma256w4: return launch_dma<MODE, 256, 256, 2, 2, EPI, OUT>(p, st);
    case kDma128w4: return launch_dma<MODE, 128, 128, 2, 2, EPI, OUT>(p, st);
    case kDma256x128w4: return launch_dma<MODE, 256, 128, 2, 2, EPI, OUT>(p, st);
  }
  return hipErrorInvalidValue;
}

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
