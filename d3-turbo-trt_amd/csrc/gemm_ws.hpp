// Weight-streaming W8A8 GEMM for skinny M (question batches, M <= 128 tokens;
// correct for any M): one launch, no split-K workspace.
//
// A question batch runs every projection at small M, where the GEMM is a
// stream of the weight matrix (N x K bytes) past a few activation rows that
// stay in L2. What bounds it is how many weight bytes each CU keeps in flight
// and how early a short-lived workgroup asks for them, not the MFMAs.
//
//   * A workgroup owns a slab of 32 * NB output columns (NB = 2 for the SwiGLU
//     gate/up pairs) and MB blocks of 32 rows, over the whole of K. Its four
//     waves split K: wave w takes the 128-byte K blocks w, w + 4, w + 8, ...
//   * Weights: each wave DMAs its own K blocks of the slab into a private LDS
//     ring (global_load_lds_dwordx4, 8 rows of 128 bytes per instruction:
//     whole 128-byte lines of each weight row), RW blocks deep. No wave reads
//     another wave's ring, so the K loop has no barrier.
//   * Activations: each wave loads its K blocks of the MB x 32 rows straight
//     into VGPRs (DA blocks deep); nothing is shared, so nothing goes through
//     LDS.
//   * K order inside a 128-byte block: lane (row r, half h) holds the 64
//     contiguous bytes [64 h, 64 h + 64) of row r; MFMA a of the block takes
//     its piece a (32 bytes for FP8 32x32x64, 16 for INT8 32x32x32). Both
//     operands use the same assignment, so every product of the block is
//     taken exactly once; the weight rows in LDS are read with the same
//     64-byte split (XOR-swizzled 16-byte chunks, conflict-free).
//   * Every wave ends with a partial sum of its K blocks. The partials meet in
//     LDS and are added in wave order 0, 1, 2, 3 (INT8 exact; FP8 in a fixed
//     fp32 order that depends on K only, so any M gives the same bits), then
//     wave i runs the shared epilogue on M block i.
//   * All memory operations of the K loop are inline asm with explicit
//     vmcnt waits (in issue order: weights of block t + RW - 1, then
//     activations of block t + DA - 1, then the wait for block t), so the
//     compiler's own waits never cover a load that is not needed yet.
#pragma once

#include "gemm_kernels.hpp"

namespace d3 {

constexpr int kWsKB = 128;               // bytes of K per block
constexpr int kWsWaveLds = 35 * 1024;    // LDS per wave for its weight ring (and later its partials)

template <int MODE, int MB, int NB, int EPI, int OUT>
struct WsCfg {
  static constexpr int SUB = MODE == kInt8 ? 4 : 2;          // MFMAs along K per block
  static constexpr int WBLK = NB * 32 * kWsKB;                // weight bytes per block (one wave)
  static constexpr int WDMA = WBLK / 1024;                    // DMA instructions per block
  static constexpr int ADMA = MB * 4;                         // 16-byte activation loads per lane per block
  static constexpr int DA = MB <= 2 ? 4 : 3;                  // activation blocks in VGPRs
  static constexpr int RING = kWsWaveLds / WBLK;              // weight blocks the LDS ring holds
  // at most 63 memory operations may be outstanding (vmcnt is 6 bits)
  static constexpr int RW_VM = (63 - (DA - 1) * ADMA) / WDMA + 1;
  static constexpr int RW = RING < RW_VM ? RING : RW_VM;      // weight blocks in the ring
  static constexpr int STEADY_WAIT = (DA - 1) * (WDMA + ADMA);
  using E = EpiLds<NB, EPI, OUT>;
  static constexpr int LDS = 4 * kWsWaveLds + 4 * E::BYTES;
  static_assert(RW >= DA && DA >= 2, "ring depth");
  static_assert(STEADY_WAIT <= 63, "vmcnt range");
  static_assert(MB * NB * 4096 <= kWsWaveLds, "partials fit the wave's region");
  static_assert(LDS <= 160 * 1024, "LDS");
};

// 16-byte global load into VGPRs, invisible to the compiler's wait insertion (explicit vmcnt waits).
__device__ __forceinline__ uint4 ws_load16(const uint8_t* p) {
  uint4 v;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(p) : "memory");
  return v;
}

// s_waitcnt vmcnt(n) for a wave-uniform runtime n in [0, MAXN]
template <int MAXN>
__device__ __forceinline__ void ws_wait_vm(int n) {
  static_for<0, MAXN + 1>([&](auto c) {
    if (n == decltype(c)::value) wait_vmcnt<decltype(c)::value>();
  });
}

template <int MODE, int MB, int NB, int EPI, int OUT>
__global__ __launch_bounds__(256, 1) void gemm_w8a8_ws(GemmParams p) {
  using C = WsCfg<MODE, MB, NB, EPI, OUT>;
  using MF = Mfma<MODE>;
  typedef typename MF::frag frag_t;
  typedef typename MF::acc acc_t;
  constexpr int SUB = C::SUB, DA = C::DA, RW = C::RW, WDMA = C::WDMA, ADMA = C::ADMA;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[C::LDS];

  const int lane = threadIdx.x & 63, lrow = lane & 31, lhalf = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // workgroup -> (column slab, row part); the row parts of one slab run on the same XCD (ids 8 apart),
  // so the second read of the slab's weights hits that XCD's L2
  const int bid = blockIdx.x, xcd = bid & 7, local = bid >> 3;
  const int part = local % p.tiles_m;
  const int slab = (local / p.tiles_m) * 8 + xcd;
  if (slab >= p.tiles_n) return;
  const int64_t n0 = (int64_t)slab * (32 * NB);
  const int64_t m0 = (int64_t)part * (32 * MB);
  const int nkb = (int)(p.K / kWsKB);
  const int cnt = nkb > wave ? (nkb - wave + 3) / 4 : 0;  // this wave's K blocks: wave, wave + 4, ...

  // weight DMA: instruction d of a block covers slab rows 8 d .. 8 d + 7; lane j -> row 8 d + j / 8,
  // physical chunk j % 8 = logical chunk (j % 8) ^ swz(row); rows past N repeat row N - 1 (never stored)
  uint32_t w_off[WDMA];
#pragma unroll
  for (int d = 0; d < WDMA; ++d) {
    const int row = 8 * d + (lane >> 3);
    const int ch = (lane & 7) ^ lds_swz<kWsKB>(row);
    w_off[d] = (uint32_t)((min(n0 + row, p.N - 1) - n0) * p.ldw + ch * 16);
  }
  const uint8_t* w_slab = p.w + n0 * p.ldw;
  const uint32_t ring0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)D3_LDS_PTR(lds) +
                                                        (uint32_t)wave * (uint32_t)kWsWaveLds);
  // activations: lane (r, h) of M block i reads row m0 + 32 i + r (clamped), bytes [64 h, 64 h + 64)
  const uint8_t* a_row[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) a_row[i] = p.a + min(m0 + 32 * i + lrow, p.M - 1) * p.lda + 64 * lhalf;

  auto issue_w = [&](int t) {  // weights of this wave's block t into ring slot t % RW
    const int kb = wave + 4 * t;
    const uint8_t* g = uniform_ptr(w_slab + (int64_t)kb * kWsKB);
    const uint32_t slot = ring0 + (uint32_t)(t % RW) * C::WBLK;
    static_for<0, WDMA>([&](auto d_c) {
      constexpr int d = decltype(d_c)::value;
      dma16<d * 1024>(g, w_off[d], slot);
    });
  };
  uint4 ra[DA][MB][4];
  auto issue_a = [&](auto s_c, int t) {  // activations of block t into register slot s
    constexpr int s = decltype(s_c)::value;
    const int64_t kb = wave + 4 * t;
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int c = 0; c < 4; ++c) ra[s][i][c] = ws_load16(a_row[i] + kb * kWsKB + 16 * c);
  };

  acc_t acc[MB][NB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  // prologue: the issue pattern of iterations -(RW - 1) .. -1 (weights of blocks 0 .. RW - 2, with the
  // activations of blocks 0 .. DA - 2 after the weights of the iterations they belong to)
  static_for<0, RW - 1>([&](auto v_c) {
    constexpr int v = decltype(v_c)::value;  // iteration v - (RW - 1)
    if (v < cnt) issue_w(v);
    constexpr int ab = v - (RW - 1) + DA - 1;  // activation block of that iteration
    if constexpr (ab >= 0) {
      if (ab < cnt) issue_a(std::integral_constant<int, ab % DA>{}, ab);
    }
  });

  // one block: iteration t with activations in register slot s = t % DA
  auto block = [&](auto s_c, int t) {
    constexpr int s = decltype(s_c)::value;
    if (t + RW - 1 < cnt) issue_w(t + RW - 1);
    if (t + DA - 1 < cnt) issue_a(std::integral_constant<int, (s + DA - 1) % DA>{}, t + DA - 1);
    // wait for block t: every operation issued after its activation loads may stay outstanding
    if (t + RW - 1 < cnt) {
      wait_vmcnt<C::STEADY_WAIT>();
    } else {
      int n = 0;
#pragma unroll
      for (int u = 1; u < DA; ++u) {  // iterations t - DA + 1 + u, the ones after block t's loads were issued
        const int it = t - DA + 1 + u;
        n += (it + RW - 1 < cnt ? WDMA : 0) + (it + DA - 1 < cnt ? ADMA : 0);
      }
      ws_wait_vm<C::STEADY_WAIT>(n);
    }
    asm volatile("" ::: "memory");  // the ring was written by DMA the compiler does not see
    __builtin_amdgcn_sched_barrier(0);
    // weight fragments of block t from the ring: lane (r, h) of N block j, MFMA a reads its row's logical
    // chunks (SUB == 2: 4 h + 2 a, 4 h + 2 a + 1; SUB == 4: 4 h + a)
    const uint8_t* slot = lds + (size_t)wave * kWsWaveLds + (size_t)(t % RW) * C::WBLK;
    frag_t wf[NB][SUB];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int row = 32 * j + lrow;
#pragma unroll
      for (int a = 0; a < SUB; ++a) {
        if constexpr (MODE == kInt8) {
          wf[j][a] = *(const v4i*)(slot + lds_offk<kWsKB>(row, 4 * lhalf + a));
        } else {
          const v4i lo = *(const v4i*)(slot + lds_offk<kWsKB>(row, 4 * lhalf + 2 * a));
          const v4i hi = *(const v4i*)(slot + lds_offk<kWsKB>(row, 4 * lhalf + 2 * a + 1));
          wf[j][a] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // every weight read of the block ahead of its MFMAs: one LDS latency
#pragma unroll
    for (int a = 0; a < SUB; ++a)
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        frag_t af;
        if constexpr (MODE == kInt8) {
          const uint4 v = ra[s][i][a];
          af = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
        } else {
          const uint4 lo = ra[s][i][2 * a], hi = ra[s][i][2 * a + 1];
          af = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        }
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = MF::run(wf[j][a], af, acc[i][j]);
      }
    // this slot's LDS reads are done before a later DMA refills it
    wait_lgkm0();
    __builtin_amdgcn_sched_barrier(0);
  };
  for (int t0 = 0; t0 < cnt; t0 += DA) {
    static_for<0, DA>([&](auto s_c) {
      if (t0 + decltype(s_c)::value < cnt) block(s_c, t0 + decltype(s_c)::value);
    });
  }

  // partials -> this wave's region: 16-byte word (i, j, g) of lane l at ((i NB + j) 4 + g) 64 + l
  uint4* mine = (uint4*)(lds + (size_t)wave * kWsWaveLds);
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        using EL = typename std::conditional<MODE == kInt8, int, float>::type;
        mine[((i * NB + j) * 4 + g) * 64 + lane] =
            make_uint4(__builtin_bit_cast(uint32_t, (EL)acc[i][j][4 * g]), __builtin_bit_cast(uint32_t, (EL)acc[i][j][4 * g + 1]),
                       __builtin_bit_cast(uint32_t, (EL)acc[i][j][4 * g + 2]), __builtin_bit_cast(uint32_t, (EL)acc[i][j][4 * g + 3]));
      }
  __syncthreads();
  if (wave >= MB) return;
  // wave i: M block i, the four partials added in wave order
  acc_t sum[1][NB];
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) sum[0][j][r] = 0;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const uint4* part_u = (const uint4*)(lds + (size_t)u * kWsWaveLds);
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        using EL = typename std::conditional<MODE == kInt8, int, float>::type;
        const uint4 v = part_u[((wave * NB + j) * 4 + g) * 64 + lane];
        sum[0][j][4 * g] = (EL)sum[0][j][4 * g] + __builtin_bit_cast(EL, v.x);
        sum[0][j][4 * g + 1] = (EL)sum[0][j][4 * g + 1] + __builtin_bit_cast(EL, v.y);
        sum[0][j][4 * g + 2] = (EL)sum[0][j][4 * g + 2] + __builtin_bit_cast(EL, v.z);
        sum[0][j][4 * g + 3] = (EL)sum[0][j][4 * g + 3] + __builtin_bit_cast(EL, v.w);
      }
  }
  epilogue<MODE, 1, NB, EPI, OUT>(p, sum, m0 + 32 * wave, n0, lane, lds + 4 * kWsWaveLds + wave * C::E::BYTES);
}

// Host side: MB row blocks per workgroup, p.tiles_m row parts, p.tiles_n column slabs.
template <int MODE, int EPI, int OUT, int MB>
static hipError_t launch_ws_mb(GemmParams p, hipStream_t st) {
  constexpr int NB = EPI == kEpiSwiGLU ? 2 : 1;
  const int64_t slabs8 = ((int64_t)p.tiles_n + 7) / 8 * 8;
  hipLaunchKernelGGL((gemm_w8a8_ws<MODE, MB, NB, EPI, OUT>), dim3((unsigned)(slabs8 * p.tiles_m)), dim3(256), 0, st, p);
  return hipGetLastError();
}

// Row blocks per part (1-4) and row parts for M rows and `slabs` column slabs: the split with the
// fewest bytes per CU (each workgroup reads its rows' activations and its slab's weights over all of
// K; workgroups beyond one per CU run in further rounds).
inline void ws_partition(int64_t M, int64_t slabs, int nb, int64_t cus, int& mb, int& parts) {
  const int64_t mblocks = (M + 31) / 32;
  int64_t best = -1;
  mb = 4;
  parts = (int)((mblocks + 3) / 4);
  for (int p = (int)((mblocks + 3) / 4); p <= mblocks && p <= 4 * ((mblocks + 3) / 4); p *= 2) {
    const int64_t b = (mblocks + p - 1) / p;
    const int64_t rounds = (slabs * p + cus - 1) / cus;
    const int64_t cost = rounds * (b + nb);
    if (best < 0 || cost < best) {
      best = cost;
      mb = (int)b;
      parts = p;
    }
  }
}

template <int MODE, int EPI, int OUT>
static hipError_t launch_ws(GemmParams p, hipStream_t st) {
  if (p.ksplit != 1) return hipErrorInvalidValue;
  constexpr int NB = EPI == kEpiSwiGLU ? 2 : 1;
  int mb, parts;
  ws_partition(p.M, (p.N + 32 * NB - 1) / (32 * NB), NB, device_cu_count(), mb, parts);
  p.tiles_m = parts;
  p.tiles_n = (int)((p.N + 32 * NB - 1) / (32 * NB));
  switch (mb) {
    case 1: return launch_ws_mb<MODE, EPI, OUT, 1>(p, st);
    case 2: return launch_ws_mb<MODE, EPI, OUT, 2>(p, st);
    case 3: return launch_ws_mb<MODE, EPI, OUT, 3>(p, st);
    default: return launch_ws_mb<MODE, EPI, OUT, 4>(p, st);
  }
}

}  // namespace d3
