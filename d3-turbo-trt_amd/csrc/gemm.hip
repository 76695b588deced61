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
//     c ^ (r & 7), so the 32 lanes of an MFMA operand read (rows r..r+31, one
//     chunk each) spread over all banks.
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

__device__ __forceinline__ int lds_off(int row, int chunk) { return row * kBK + ((chunk ^ (row & 7)) << 4); }

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

  // ------------------------------------------------------------------ epilogue
  const int64_t wrow0 = m0 + wm * WTM, wcol0 = n0 + wn * WTN;
  if constexpr (EPI == kEpiSwiGLU) {
    const int64_t NH = N >> 1;  // h columns
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      float rmax[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) rmax[r] = 0.0f;
#pragma unroll
      for (int jp = 0; jp < TN / 2; ++jp) {
        const int64_t cg = wcol0 + (2 * jp) * 32 + lrow;  // interleaved gate column
        const int64_t cu = cg + 32;                       // its up column
        const int64_t hc = (cg >> 6) * 32 + (cg & 31);    // h column
        const bool cok = cu < N;
        const float sg = cok ? p.w_scale[cg] : 0.0f, su = cok ? p.w_scale[cu] : 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = wrow0 + i * 32 + (r >> 2) * 8 + lhalf * 4 + (r & 3);
          if (row < M && cok) {
            const float st = p.a_scale[row];
            float g = (float)acc[i][2 * jp][r];
            g = g * st;
            g = round_to<OUT>(g * sg);
            float u = (float)acc[i][2 * jp + 1][r];
            u = u * st;
            u = round_to<OUT>(u * su);
            const float e = expf(-g);
            const float den = 1.0f + e;
            const float sl = round_to<OUT>(g / den);
            const float h = round_to<OUT>(sl * u);
            store_elem<OUT>(p.out, row * p.ldo + hc, h);
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
          const int64_t row = wrow0 + i * 32 + (r >> 2) * 8 + lhalf * 4 + (r & 3);
          if (lrow == 0 && row < M) atomicMax((unsigned int*)(p.row_amax + row), __float_as_uint(v));
        }
      }
    }
    (void)NH;
  } else {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = wrow0 + i * 32 + (r >> 2) * 8 + lhalf * 4 + (r & 3);
        if (row >= M) continue;
        const int64_t orow = p.row_map ? (int64_t)p.row_map[row] : row;
        const float st = (EPI == kEpiRaw) ? 0.0f : p.a_scale[row];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int64_t col = wcol0 + j * 32 + lrow;
          if (col >= N) continue;
          if constexpr (EPI == kEpiRaw) {
            if constexpr (MODE == kInt8) ((int32_t*)p.out)[orow * p.ldo + col] = acc[i][j][r];
            else ((float*)p.out)[orow * p.ldo + col] = acc[i][j][r];
          } else {
            float v = (float)acc[i][j][r];
            v = v * st;
            v = v * p.w_scale[col];
            if constexpr (EPI == kEpiResidual) {
              v = round_to<OUT>(v);
              v = load_elem<OUT>(p.res, orow * p.ldr + col) + v;
            }
            store_elem<OUT>(p.out, orow * p.ldo + col, v);
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// host side: tile-config selection and dispatch
// ---------------------------------------------------------------------------
enum TileCfg : int { kTileAuto = -1, kTile256 = 0, kTile128 = 1, kTile64x128 = 2 };

template <int MODE, int BM, int BN, int WM, int WN, int EPI, int OUT>
static hipError_t launch_cfg(GemmParams p, hipStream_t st) {
  p.tiles_m = (int)((p.M + BM - 1) / BM);
  p.tiles_n = (int)((p.N + BN - 1) / BN);
  const int64_t nb = (int64_t)p.tiles_m * p.tiles_n;
  hipLaunchKernelGGL((gemm_w8a8<MODE, BM, BN, WM, WN, EPI, OUT>), dim3((unsigned)nb), dim3(WM * WN * 64), 0, st, p);
  return hipGetLastError();
}

static int choose_tile(int64_t M, int64_t N) {
  const int64_t t256 = ((M + 255) / 256) * ((N + 255) / 256);
  const int64_t t128 = ((M + 127) / 128) * ((N + 127) / 128);
  if (t256 >= 256) return kTile256;
  if (t128 >= 192) return kTile128;
  return kTile64x128;
}

template <int MODE, int EPI, int OUT>
static hipError_t launch_epi(GemmParams p, int tile, hipStream_t st) {
  if (tile == kTileAuto) tile = choose_tile(p.M, p.N);
  switch (tile) {
    case kTile256: return launch_cfg<MODE, 256, 256, 2, 2, EPI, OUT>(p, st);
    case kTile128: return launch_cfg<MODE, 128, 128, 2, 2, EPI, OUT>(p, st);
    default: return launch_cfg<MODE, 64, 128, 2, 2, EPI, OUT>(p, st);
  }
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
