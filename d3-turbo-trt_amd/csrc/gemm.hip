// W8A8 GEMM dispatch: mode / epilogue / output dtype -> the kernel family
// instantiated in gemm_<mode>_<epilogue>.hip (the kernels themselves are in
// gemm_kernels.hpp; one translation unit per family keeps the build parallel).
#include "common.hpp"
#include "kernels.hpp"

#include <stdlib.h>
#include <string.h>

#include <algorithm>

namespace d3 {

// The persistent walk (one workgroup per CU walking tiles) runs only when D3W8A8_GEMM_PERSIST=1 is set
// (read at every launch). Measured on MI355X (state-pass shapes, K-blocked activations), one workgroup
// per tile is faster: FP8 gate_up 4096 x 24576 x 4096 352 -> 319-332 us, qkv 91.2 -> 86.0 us, INT8
// gate_up 394 -> 350 us. That form stages its epilogue rows in the stage memory the K loop has freed
// (padded rows) and carries no state from tile to tile, so it needs no scratch; the walk packs its
// staging into the 32 KiB beside the four stages and spills 71 VGPRs.
bool gemm_persistent() {
  const char* e = getenv("D3W8A8_GEMM_PERSIST");
  return e && strcmp(e, "1") == 0;
}

template <int MODE, int EPI, int OUT>
hipError_t launch_epi(GemmParams p, int tile, hipStream_t st);

#define D3_EXTERN_EPI(MODE)                                   \
  extern template hipError_t launch_epi<MODE, kEpiRaw, kF32>(GemmParams, int, hipStream_t);       \
  extern template hipError_t launch_epi<MODE, kEpiDequant, kBF16>(GemmParams, int, hipStream_t);  \
  extern template hipError_t launch_epi<MODE, kEpiDequant, kF16>(GemmParams, int, hipStream_t);   \
  extern template hipError_t launch_epi<MODE, kEpiDequant, kF32>(GemmParams, int, hipStream_t);   \
  extern template hipError_t launch_epi<MODE, kEpiSwiGLU, kBF16>(GemmParams, int, hipStream_t);   \
  extern template hipError_t launch_epi<MODE, kEpiSwiGLU, kF16>(GemmParams, int, hipStream_t);    \
  extern template hipError_t launch_epi<MODE, kEpiSwiGLU, kF32>(GemmParams, int, hipStream_t);    \
  extern template hipError_t launch_epi<MODE, kEpiResidual, kBF16>(GemmParams, int, hipStream_t); \
  extern template hipError_t launch_epi<MODE, kEpiResidual, kF16>(GemmParams, int, hipStream_t);  \
  extern template hipError_t launch_epi<MODE, kEpiResidual, kF32>(GemmParams, int, hipStream_t);
D3_EXTERN_EPI(kInt8)
D3_EXTERN_EPI(kFp8)
#undef D3_EXTERN_EPI

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

namespace {

struct TileShape {
  int bm, bn;
  bool dma;
  int bk;      // bytes of K per pipeline step (K must be a multiple)
};

TileShape shape_of(int tile) {
  switch (tile) {
    case kTile256: return {256, 256, false, 16};
    case kTile128: return {128, 128, false, 16};
    case kTile64x128: return {64, 128, false, 16};
    case kDma256w8: return {256, 256, true, 64};
    case kDma256w4: return {256, 256, true, 64};
    case kDma128w4: return {128, 128, true, 64};
    case kDma256x128w4: return {256, 128, true, 64};
    case kDma128w4k128: return {128, 128, true, 128};
    case kDma256x192w4: return {256, 192, true, 64};
    case kWs: return {128, 32, true, 128};
    case kDma192x192w4: return {192, 192, true, 64};
    case kDma192x128w4: return {192, 128, true, 64};
  }
  return {0, 0, false, 0};
}

constexpr int kMinSplitBytes = 1024;   // bytes of K per split at least

// The DMA kernels address operands as a tile base plus a 32-bit per-lane offset. A K-blocked operand
// keeps its offsets within a tile's rows and two K blocks (ld < kMaxKblkRows, checked by the caller).
bool dma_offsets_fit(int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldw, bool a_kblk, bool w_kblk) {
  const int64_t lim = (int64_t)1 << 32;
  return (a_kblk || (M - 1) * lda + K < lim) && (w_kblk || (N - 1) * ldw + K < lim);
}

// Rounds of tiles the chip runs one after the other (one workgroup per CU).
int64_t rounds(int64_t tiles, int64_t cus) { return (tiles + cus - 1) / cus; }

// Tile choice (measured on MI355X): with K % 64 == 0, the 4-wave 256x256 DMA
// tile once there are enough such tiles to cover the chip, 256x128 for
// mid-size problems, 128x128 otherwise. Where 256x256 tiles leave the last
// round partly idle (fused QKV at M = 4096, N = 6144: 384 tiles, 1.5 rounds)
// and 256x192 tiles fill whole rounds (512 tiles, 2 rounds), the narrower
// tile wins: it is taken when its rounds x tile area is at least 10% below
// that of 256x256, or of 256x128 where that tile would be chosen (N % 192 == 0,
// epilogues without gate/up pairs). Measured: 1440 x 6144 x 4096 INT8 70.0 ->
// 60.6 us; 1280 rows keep 256x128 (44.2 us, 256x192 52.5 us), as the rule says. M <= 128 (a
// 256-row tile would compute half its rows for nothing) streams the weights. When K % 128 == 0,
// the weight-streaming kernel (gemm_ws.hpp, tile kWs) runs where K <= 4096 (each of its workgroups
// reads M x K <= 512 KiB of activations) and its column slabs fit one round of CUs: no split-K
// partials and no second launch (M = 128: QKV 13.5 vs 17.6 us, o_proj 13.0 vs 16.5 us, gate_up +
// SwiGLU in 128-column slabs 28.9 vs 30.8 us). The rule
// does not look at M, so every M <= 128 takes the same tile and split (a packed question batch
// equals its blocks run one by one, FP8 included). Otherwise the
// 128x128 tile with 128-byte K steps, split over K by the planner (down, K = 12288: 21.8 vs 34.5 us).
// Tile counts are weighed against the device's compute units (`cus`; the thresholds were measured on
// 256).
// INT8 takes the 8-wave 256x256 tile (two waves per SIMD, 128x64 accumulators in VGPRs) where the
// 4-wave one would run: same-box, K-blocked operands, INT8 gate_up 4096 x 24576 x 4096 350.3 -> 340.5 us
// (SwiGLU 361.2 -> 356.3), 8192 x 6144 x 4096 175.0 -> 170.8 us, single-round shapes even. FP8 keeps
// the 4-wave tile (even on gate_up, down 141.4 against 146.3 us).
// A 192-row tile in place of the chosen 256-row one where its rounds x tile area is at least 10%
// below the chosen tile's (ragged batches whose 256-row tiles leave part of a round idle: 1440 rows are
// 6 tile rows of 256, 192 tiles at N = 4096 or 6144, but 8 tile rows of 192, one whole round).
// The larger of two equal-cost tiles stays.
int prefer_192_rows(int tile, int64_t cost, int64_t M, int64_t N, int epi, int64_t cus) {
  const int64_t tm = (M + 191) / 192;
  const int64_t bar = cost * 9;
  int best = tile;
  int64_t best_cost = cost;
  if (epi != kEpiSwiGLU && N % 192 == 0) {
    const int64_t c = rounds(tm * (N / 192), cus) * 192 * 192;
    if (c * 10 <= bar && c < best_cost) best = kDma192x192w4, best_cost = c;
  }
  const int64_t c = rounds(tm * ((N + 127) / 128), cus) * 192 * 128;
  if (c * 10 <= bar && c < best_cost) best = kDma192x128w4;
  return best;
}

int choose_tile(int64_t M, int64_t N, int64_t K, bool fit, int epi, int64_t cus, int mode) {
  const int64_t t256 = ((M + 255) / 256) * ((N + 255) / 256);
  const int64_t t256x128 = ((M + 255) / 256) * ((N + 127) / 128);
  const int64_t t128 = ((M + 127) / 128) * ((N + 127) / 128);
  if (K % 64 == 0 && fit) {
    if (M <= 128) {
      if (K % 128 != 0) return kDma128w4;
      const int64_t cols = 32 * ws_slab_blocks(N, epi, cus);
      return K <= 4096 && (N + cols - 1) / cols <= cus ? kWs : kDma128w4k128;
    }
    if (4 * t256 >= 3 * cus) {  // 192 tiles on 256 CUs
      if (epi != kEpiSwiGLU && N % 192 == 0) {
        const int64_t t192 = ((M + 255) / 256) * (N / 192);
        if (rounds(t192, cus) * 192 * 10 <= rounds(t256, cus) * 256 * 9)
          return prefer_192_rows(kDma256x192w4, rounds(t192, cus) * 256 * 192, M, N, epi, cus);
      }
      return prefer_192_rows(mode == kInt8 ? kDma256w8 : kDma256w4, rounds(t256, cus) * 256 * 256, M, N, epi, cus);
    }
    if (8 * t256x128 >= 5 * cus) {  // 160 tiles on 256 CUs
      // the same round count rule against 256x128 (ragged question batches: 1440 rows x N = 6144 is
      // 288 tiles of 256x128, one round and 32 tiles, but 192 tiles of 256x192, one round)
      if (epi != kEpiSwiGLU && N % 192 == 0) {
        const int64_t t192 = ((M + 255) / 256) * (N / 192);
        if (rounds(t192, cus) * 192 * 10 <= rounds(t256x128, cus) * 128 * 9)
          return prefer_192_rows(kDma256x192w4, rounds(t192, cus) * 256 * 192, M, N, epi, cus);
      }
      return prefer_192_rows(kDma256x128w4, rounds(t256x128, cus) * 256 * 128, M, N, epi, cus);
    }
    return kDma128w4;
  }
  if (t256 >= cus) return kTile256;
  if (4 * t128 >= 3 * cus) return kTile128;
  return kTile64x128;
}

// Split-K when the tiles leave most CUs idle: about one workgroup per CU,
// each split at least kMinSplitBytes of K. Measured on MI355X at M = 128
// (weights streamed from HBM): more splits cost more in partial sums and the
// reduce launch than the extra workgroups gain.
int choose_ksplit(int64_t tiles, int nk, int bk, int64_t cus) {
  const int64_t target = cus;
  if (2 * tiles > target) return 1;
  int64_t s = (target + tiles - 1) / tiles;
  s = std::min<int64_t>(s, nk / (kMinSplitBytes / bk));
  s = std::min<int64_t>(s, kMaxKSplit);
  return (int)std::max<int64_t>(s, 1);
}

}  // namespace

GemmPlan plan_gemm(int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldw, int tile, int ksplit,
                   int64_t ws_bytes, int epi, bool a_kblk, bool w_kblk, int mode) {
  GemmPlan pl{};
  pl.ksplit = 1;
  const bool fit = dma_offsets_fit(M, N, K, lda, ldw, a_kblk, w_kblk);
  const int64_t cus = device_cu_count();
  pl.tile = tile < 0 ? choose_tile(M, N, K, fit, epi, cus, mode) : tile;
  if (pl.tile >= kTileCount) return pl.error = "unknown tile", pl;
  if ((pl.tile == kDma256x192w4 || pl.tile == kDma192x192w4) && epi == kEpiSwiGLU)
    return pl.error = "the 192-column tiles have 3 column blocks per wave; SwiGLU needs gate/up pairs", pl;
  const TileShape sh = shape_of(pl.tile);
  if ((a_kblk || w_kblk) && !sh.dma) return pl.error = "a K-blocked operand needs a pipelined (DMA) tile", pl;
  if (sh.dma && K % sh.bk != 0)
    return pl.error = sh.bk == 128 ? "the 128-byte-step tile needs K % 128 == 0" : "the pipelined tiles need K % 64 == 0",
           pl;
  if (sh.dma && !fit) return pl.error = "the pipelined tiles address each operand with 32-bit offsets", pl;
  pl.tiles_m = (int)((M + sh.bm - 1) / sh.bm);
  pl.tiles_n = (int)((N + sh.bn - 1) / sh.bn);
  const int64_t tiles = (int64_t)pl.tiles_m * pl.tiles_n;
  const int nk = (int)(K / (sh.dma ? sh.bk : 64));
  const int64_t slot = (int64_t)sh.bm * sh.bn * 4;
  if (ksplit >= 1) {
    if (ksplit > 1) {
      if (!sh.dma || sh.bm != 128 || sh.bn != 128) return pl.error = "split-K needs a pipelined 128x128 tile", pl;
      if (ksplit > kMaxKSplit || ksplit > nk) return pl.error = "ksplit exceeds K / 64 or the split limit", pl;
      if (tiles * ksplit * slot > ws_bytes) return pl.error = "split-K workspace too small", pl;
    }
    pl.ksplit = ksplit;
  } else if (sh.dma && sh.bm == 128 && sh.bn == 128 && tiles > 0 && ws_bytes > 0) {
    const int64_t room = ws_bytes / (tiles * slot);
    const int s = (int)std::min<int64_t>(choose_ksplit(tiles, nk, sh.bk, cus), room);
    pl.ksplit = s >= 2 ? s : 1;
  }
  pl.ws_bytes = pl.ksplit > 1 ? tiles * pl.ksplit * slot : 0;
  return pl;
}

hipError_t launch_gemm(int mode, GemmParams p, int epi, int out_dt, const GemmPlan& plan, hipStream_t st) {
  if (p.M == 0 || p.N == 0) return hipSuccess;
  if (plan.error) return hipErrorInvalidValue;
  p.ksplit = plan.ksplit;
  return mode == kInt8 ? launch_mode<kInt8>(p, epi, out_dt, plan.tile, st)
                       : launch_mode<kFp8>(p, epi, out_dt, plan.tile, st);
}

}  // namespace d3
