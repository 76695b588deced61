// Weight-streaming W8A8 GEMM for skinny M (question batches, M <= 128 tokens
// per workgroup; any M by row parts): one launch, no split-K workspace, a
// dedicated weight-streaming wave.
//
// At M <= 128 the GEMM is a stream of the weight matrix (N x K bytes, HBM)
// past a few activation rows (L2-resident). Two facts shape the kernel:
//
//   * vmcnt counts a wave's memory operations in issue order, so a wave that
//     loads both operands can only keep its weights as far ahead as its
//     activations. Weights come from HBM (microseconds away under load) and
//     activations from L2, so they need different lead. Here they are issued
//     by different waves: one producer wave DMAs the weight slab into a deep
//     LDS ring (DW blocks) and does nothing else; the consumer waves DMA
//     their own activation rows into shallow private rings (DA blocks) and
//     run the MFMAs. Each wave waits only on its own counter.
//   * Whole 128-byte lines per request: every DMA instruction moves 8 rows x
//     128 bytes (one K block of 8 rows) of either operand, so the vector
//     memory path handles 8 lines per KiB.
//
// Layout. A workgroup owns a slab of 32 * NB output columns (NB = 2 for the
// SwiGLU gate/up pairs) and MB blocks of 32 rows. Consumer c (of CW) owns
// row blocks c * RB .. c * RB + RB - 1 (RB = MB / CW) and every column of the
// slab: it reads every weight block (shared through the ring) and only its
// own activation rows. K blocks are 128 bytes; inside a block the MFMA
// operand chunks are assigned as in the pipelined tiles (FP8 sub-step s, lane
// half h: 16-byte chunks 4 s + 2 h and 4 s + 2 h + 1; INT8: 2 s + h), and
// blocks are summed in K order, so results equal the unsplit 128x128 tile with
// 128-byte K steps bit for bit.
//
// Synchronization, per K block t: the producer waits for its DMA of weight
// block t and joins barrier t; a consumer waits for its activation block t and
// joins barrier t, then reads both operands. After barrier t every consumer
// has finished block t - 1 (its LDS reads completed before it arrived), so the
// producer refills that slot with block t + DW - 1. Activation slots are
// private: a consumer refills the slot of block t - 1 at the start of
// iteration t. Every wave passes the same nkb barriers; the producer then
// leaves and each consumer runs the shared epilogue on its rows, staging
// through its own activation ring.
//
// Cost (MI355X, M = 128, weights from HBM). Every workgroup reads all M x K
// activation bytes from L2, and that stream runs at ~47 GB/s per CU, so the
// kernel wins where M x K is small against the split-K alternative's partial
// sums and second launch: QKV 128 x 6144 x 4096 13.5 us and o_proj
// 128 x 4096 x 4096 13.0 us, against 17.6 and 16.5 us for the 128x128 tile
// split over K; down (K = 12288) 34.5 against 21.8 us. Deeper weight or
// activation rings and more producer waves measured no faster.
#pragma once

#include "gemm_kernels.hpp"

namespace d3 {

constexpr int kWsKB = 128;  // bytes of K per block

// s_waitcnt vmcnt(n) for a wave-uniform runtime n in [0, MAXN]
template <int MAXN>
__device__ __forceinline__ void ws_wait_vm(int n) {
  static_for<0, MAXN + 1>([&](auto c) {
    if (n == decltype(c)::value) wait_vmcnt<decltype(c)::value>();
  });
}


template <int MODE, int MB, int NB, int CW, int DW, int DA, int EPI, int OUT>
struct WsCfg {
  static_assert(MB % CW == 0, "row blocks split evenly over the consumers");
  static constexpr int RB = MB / CW;                    // row blocks per consumer
  static constexpr int SUB = MODE == kInt8 ? 4 : 2;     // MFMAs along K per block
  static constexpr int WBLK = NB * 32 * kWsKB;           // weight bytes per block
  static constexpr int WDMA = WBLK / 1024;               // producer DMA instructions per block
  static constexpr int ABLK = RB * 32 * kWsKB;           // activation bytes per block per consumer
  static constexpr int ADMA = ABLK / 1024;               // consumer DMA instructions per block
  static constexpr int W_STEADY = (DW - 2) * WDMA;       // producer: blocks t+1 .. t+DW-2 may be in flight
  static constexpr int A_STEADY = (DA - 1) * ADMA;       // consumer: blocks t+1 .. t+DA-1 may be in flight
  static constexpr int W_BYTES = DW * WBLK;
  static constexpr int A_BYTES = CW * DA * ABLK;
  static constexpr int LDS = W_BYTES + A_BYTES;
  using E = EpiLds<NB, EPI, OUT>;
  static_assert(DW >= 2 && DA >= 2, "ring depth");
  static_assert(W_STEADY <= 63 && A_STEADY <= 63, "vmcnt range");
  static_assert(E::BYTES <= DA * ABLK, "epilogue staging fits the consumer's ring");
  static_assert(LDS <= 160 * 1024, "LDS");
};

template <int MODE, int MB, int NB, int CW, int DW, int DA, int EPI, int OUT>
__global__ __launch_bounds__((CW + 1) * 64, 1) void gemm_w8a8_ws(GemmParams p) {
  using C = WsCfg<MODE, MB, NB, CW, DW, DA, EPI, OUT>;
  using MF = Mfma<MODE>;
  typedef typename MF::frag frag_t;
  typedef typename MF::acc acc_t;
  constexpr int RB = C::RB, SUB = C::SUB, WDMA = C::WDMA, ADMA = C::ADMA;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[C::LDS];

  const int lane = threadIdx.x & 63, lrow = lane & 31, lhalf = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // workgroup -> (column slab, row part): consecutive slabs on one XCD
  const int bid = blockIdx.x, xcd = bid & 7, local = bid >> 3;
  const int part = local % p.tiles_m;
  const int slab = (local / p.tiles_m) * 8 + xcd;
  if (slab >= p.tiles_n) return;  // the whole workgroup leaves: no barrier is pending
  const int64_t n0 = (int64_t)slab * (32 * NB);
  const int64_t m0 = (int64_t)part * (32 * MB);
  const int nkb = (int)(p.K / kWsKB);
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)D3_LDS_PTR(lds));

  if (wave == CW) {
    // ---------------- producer: the weight slab, DW blocks deep ----------------
    // instruction d covers slab rows 8 d .. 8 d + 7: lane j -> row 8 d + j / 8, LDS chunk j % 8 holds
    // logical chunk (j % 8) ^ swz(row); rows past N repeat row N - 1 (their outputs are never stored)
    // W row-major or K-blocked (QDst, kernels.hpp), as A below
    const int64_t w_rs = p.w_kblk ? 64 : p.ldw, w_bs = p.w_kblk ? 64 * p.ldw : 64;
    uint32_t w_off[WDMA];
#pragma unroll
    for (int d = 0; d < WDMA; ++d) {
      const int row = 8 * d + (lane >> 3);
      const int ch = (lane & 7) ^ lds_swz<kWsKB>(row);
      w_off[d] = (uint32_t)((min(n0 + row, p.N - 1) - n0) * w_rs + (ch >> 2) * w_bs + (ch & 3) * 16);
    }
    const uint8_t* w_slab = p.w + n0 * w_rs;
    auto issue_w = [&](int t) {
      const uint8_t* g = uniform_ptr(w_slab + (int64_t)t * 2 * w_bs);
      const uint32_t slot = lds0 + (uint32_t)(t % DW) * C::WBLK;
      static_for<0, WDMA>([&](auto d_c) {
        constexpr int d = decltype(d_c)::value;
        dma16<d * 1024>(g, w_off[d], slot);
      });
    };
    for (int t = 0; t < DW - 1 && t < nkb; ++t) issue_w(t);
    for (int t = 0; t < nkb; ++t) {
      // blocks issued so far: 0 .. min(nkb, t + DW - 1) - 1; all after block t may stay in flight
      if (t + DW - 1 <= nkb) {
        wait_vmcnt<C::W_STEADY>();
      } else {
        ws_wait_vm<C::W_STEADY>((nkb - t - 1) * WDMA);
      }
      lds_barrier();  // barrier t: block t is in LDS; every consumer is done with block t - 1
      if (t + DW - 1 < nkb) issue_w(t + DW - 1);  // into the slot of block t - 1
    }
    return;
  }

  // ---------------- consumer c: row blocks c RB .. c RB + RB - 1 ----------------
  const int c = wave;
  const int64_t r0 = m0 + 32 * RB * c;  // first row of this consumer
  // A row-major or K-blocked (QDst, kernels.hpp): byte (m, k) at m * a_rs + (k / 64) * a_bs + k % 64;
  // a 128-byte block spans two 64-byte K blocks
  const int64_t a_rs = p.a_kblk ? 64 : p.lda, a_bs = p.a_kblk ? 64 * p.lda : 64;
  uint32_t a_off[ADMA];
#pragma unroll
  for (int d = 0; d < ADMA; ++d) {
    const int row = 8 * d + (lane >> 3);
    const int ch = (lane & 7) ^ lds_swz<kWsKB>(row);
    a_off[d] = (uint32_t)((min(r0 + row, p.M - 1) - r0) * a_rs + (ch >> 2) * a_bs + (ch & 3) * 16);
  }
  // rows past M read row M - 1; if this consumer's first row is past M it still runs the loop (the
  // barriers are shared) on clamped rows and stores nothing
  const uint8_t* a_rows = p.a + min(r0, p.M - 1) * a_rs;
  if (r0 >= p.M) {
#pragma unroll
    for (int d = 0; d < ADMA; ++d) {
      const int ch = (lane & 7) ^ lds_swz<kWsKB>(8 * d + (lane >> 3));
      a_off[d] = (uint32_t)((ch >> 2) * a_bs + (ch & 3) * 16);
    }
  }
  const uint32_t aring = lds0 + (uint32_t)C::W_BYTES + (uint32_t)c * (uint32_t)(DA * C::ABLK);
  auto issue_a = [&](int t) {
    const uint8_t* g = uniform_ptr(a_rows + (int64_t)t * 2 * a_bs);
    const uint32_t slot = aring + (uint32_t)(t % DA) * C::ABLK;
    static_for<0, ADMA>([&](auto d_c) {
      constexpr int d = decltype(d_c)::value;
      dma16<d * 1024>(g, a_off[d], slot);
    });
  };

  acc_t acc[RB][NB];
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  for (int t = 0; t < DA - 1 && t < nkb; ++t) issue_a(t);
  const uint8_t* a_lds = lds + C::W_BYTES + (size_t)c * (DA * C::ABLK);
  for (int t = 0; t < nkb; ++t) {
    if (t + DA - 1 < nkb) issue_a(t + DA - 1);  // into the slot of block t - 1 (read last iteration)
    // blocks issued so far: 0 .. min(nkb, t + DA) - 1; all after block t may stay in flight
    if (t + DA <= nkb) {
      wait_vmcnt<C::A_STEADY>();
    } else {
      ws_wait_vm<C::A_STEADY>((nkb - t - 1) * ADMA);
    }
    lds_barrier();  // barrier t: the producer's weight block t is in LDS as well
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t* ws = lds + (size_t)(t % DW) * C::WBLK;
    const uint8_t* as = a_lds + (size_t)(t % DA) * C::ABLK;
    frag_t wf[SUB][NB], af[SUB][RB];
#pragma unroll
    for (int s = 0; s < SUB; ++s) {
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int row = 32 * j + lrow;
        if constexpr (MODE == kInt8) {
          wf[s][j] = *(const v4i*)(ws + lds_offk<kWsKB>(row, 2 * s + lhalf));
        } else {
          const v4i lo = *(const v4i*)(ws + lds_offk<kWsKB>(row, 4 * s + 2 * lhalf));
          const v4i hi = *(const v4i*)(ws + lds_offk<kWsKB>(row, 4 * s + 2 * lhalf + 1));
          wf[s][j] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
      }
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const int row = 32 * i + lrow;
        if constexpr (MODE == kInt8) {
          af[s][i] = *(const v4i*)(as + lds_offk<kWsKB>(row, 2 * s + lhalf));
        } else {
          const v4i lo = *(const v4i*)(as + lds_offk<kWsKB>(row, 4 * s + 2 * lhalf));
          const v4i hi = *(const v4i*)(as + lds_offk<kWsKB>(row, 4 * s + 2 * lhalf + 1));
          af[s][i] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
      }
    }
#pragma unroll
    for (int s = 0; s < SUB; ++s)
#pragma unroll
      for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = MF::run(wf[s][j], af[s][i], acc[i][j]);
    wait_lgkm0();  // this block's LDS reads are done before its slots are refilled
    __builtin_amdgcn_sched_barrier(0);
  }
  if (r0 >= p.M) return;
  // the last activation slots were read (wait_lgkm0 above) and no DMA targets them any more
  epilogue<MODE, RB, NB, EPI, OUT>(p, acc, r0, n0, lane, (uint8_t*)a_lds);
}

// Host side: MB row blocks per workgroup (p.tiles_m row parts), p.tiles_n column slabs of 32 NB columns.
// One consumer per row block; activations 3 blocks deep (4 with at most two consumers: o_proj in two
// row parts 11.0 -> 10.6 us); the weight ring 8 blocks deep (5 for NB = 4, whose 16 DMAs per block
// would otherwise pass vmcnt's 63 and LDS).
template <int MODE, int EPI, int OUT, int MB, int NB>
static hipError_t launch_ws_mb(GemmParams p, hipStream_t st) {
  constexpr int CW = MB, DW = NB == 4 ? 5 : 8, DA = MB <= 2 ? 4 : 3;
  const int64_t slabs8 = ((int64_t)p.tiles_n + 7) / 8 * 8;
  hipLaunchKernelGGL((gemm_w8a8_ws<MODE, MB, NB, CW, DW, DA, EPI, OUT>), dim3((unsigned)(slabs8 * p.tiles_m)),
                     dim3((CW + 1) * 64), 0, st, p);
  return hipGetLastError();
}

// Row blocks per workgroup: every workgroup reads all K of its rows' activations, and that stream
// bounds it, so the rows are split into more parts while the slabs x parts still fit one round of
// CUs (M = 128: o_proj's 128 slabs in two parts of 64 rows, 13.0 -> 10.6 us; QKV's 192 slabs stay
// whole: two parts would need a second round, 13.7 -> 15.9 us). A row's result does not depend on
// the split.
inline int ws_row_blocks(int64_t M, int64_t slabs, int64_t cus) {
  const int64_t mblocks = (M + 31) / 32;
  int mb = (int)std::min<int64_t>(mblocks, 4);
  while (mb > 1 && slabs * ((mblocks + mb / 2 - 1) / (mb / 2)) <= cus) mb /= 2;
  return mb;
}

template <int MODE, int EPI, int OUT, int NB>
static hipError_t launch_ws_nb(GemmParams p, hipStream_t st) {
  const int64_t mblocks = (p.M + 31) / 32;
  p.tiles_n = (int)((p.N + 32 * NB - 1) / (32 * NB));
  const int mb = ws_row_blocks(p.M, p.tiles_n, device_cu_count());
  p.tiles_m = (int)((mblocks + mb - 1) / mb);
  switch (mb) {
    case 1: return launch_ws_mb<MODE, EPI, OUT, 1, NB>(p, st);
    case 2: return launch_ws_mb<MODE, EPI, OUT, 2, NB>(p, st);
    case 3: return launch_ws_mb<MODE, EPI, OUT, 3, NB>(p, st);
    default: return launch_ws_mb<MODE, EPI, OUT, 4, NB>(p, st);
  }
}

template <int MODE, int EPI, int OUT>
static hipError_t launch_ws(GemmParams p, hipStream_t st) {
  if (p.ksplit != 1) return hipErrorInvalidValue;
  if constexpr (EPI == kEpiSwiGLU) {
    if (ws_slab_blocks(p.N, EPI, device_cu_count()) == 4) return launch_ws_nb<MODE, EPI, OUT, 4>(p, st);
    return launch_ws_nb<MODE, EPI, OUT, 2>(p, st);
  } else {
    return launch_ws_nb<MODE, EPI, OUT, 1>(p, st);
  }
}

}  // namespace d3
