// Host-side launch interface shared by the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace d3 {

// Layouts of quantized activations. Row-major: byte (m, k) at m * ld + k. K-blocked: each 64-byte
// slice of K holds all rows back to back, byte (m, k) at ((k / 64) * ld + m) * 64 + k % 64 (ld >= M:
// the row capacity). A pipelined GEMM tile loads 64 bytes of K from each of its rows per step; row-major
// rows make each load half a 128-byte line of many rows, K-blocked rows make it whole lines of
// consecutive rows (MI355X, FP8 state pass at M = 4096, K-blocked activations: qkv 105.8 -> 90.7 us,
// gate_up 387 -> 355 us, down 169 -> 153 us). Both are addressed as row * rs + (k / 64) * bs + k % 64.
struct QDst {
  char* q;
  int64_t rs;  // bytes between rows
  int64_t bs;  // bytes between 64-byte K blocks
  static QDst of(void* q, int64_t ld, bool kblk) {
    return kblk ? QDst{(char*)q, 64, 64 * ld} : QDst{(char*)q, ld, 64};
  }
  __host__ __device__ QDst rows_from(int64_t r0) const { return QDst{q + r0 * rs, rs, bs}; }
  // K-blocked with room for more than one row (a one-row K-blocked q is also row-major)
  __host__ __device__ bool kblocked() const { return rs == 64 && bs > 64; }
  __device__ __forceinline__ char* row(int64_t r) const { return q + r * rs; }
  // column col (a multiple of 8 for the vector stores: an 8-byte store stays in one K block)
  __device__ __forceinline__ static char* at(char* qrow, int64_t col, int64_t bs) {
    return qrow + (col >> 6) * bs + (col & 63);
  }
};

struct GemmParams {
  const uint8_t* a;
  int64_t lda;  // row-major: elements between rows; K-blocked (a_kblk): the row capacity (>= M)
  int a_kblk;   // A is K-blocked (pipelined tiles only)
  const float* a_scale;
  const uint8_t* w;
  int64_t ldw;  // as lda, for w (w_kblk)
  int w_kblk;   // W is K-blocked (pipelined tiles only)
  const float* w_scale;
  int64_t M, N, K;
  void* out;
  int64_t ldo;
  const void* res;
  int64_t ldr;
  float* row_amax;
  const int32_t* row_map;
  int vec;  // output, residual and channel scales allow 4-element vector access
  int tiles_m, tiles_n;
  // Split-K (pipelined tiles only): ksplit workgroups share one output tile,
  // each over a contiguous range of K steps, and store their raw accumulators
  // in `partial` (ksplit tile-sized slots per tile); a second launch sums the
  // slots in a fixed order and runs the epilogue.
  int ksplit;
  uint32_t* partial;  // tiles * ksplit * BM * BN 32-bit words
};

hipError_t launch_quant_rows(int mode, int dt, const void* x, int64_t ldx, int64_t M, int64_t K, QDst q,
                             float* scale, bool vec, hipStream_t st);
hipError_t launch_quant_rows_amax(int mode, int dt, const void* h, int64_t ldh, const float* amax, int64_t M,
                                  int64_t K, QDst q, float* scale, hipStream_t st);
hipError_t launch_rmsnorm_quant(int mode, int dt, int dtw, const void* x, int64_t ldx, const void* w, int64_t M,
                                int64_t K, float eps, int zc, QDst q, float* scale, void* normed,
                                int64_t ldn, float* clear_amax, hipStream_t st);
// o_proj input of a gated attention layer: quantize_rows(x * sigmoid(gate)); head_dim > 0 reads the
// gate in place from the per-head [query | gate] rows of the q_proj output. 16-bit inputs only.
hipError_t launch_gate_quant(int mode, int dt, const void* x, int64_t ldx, const void* gate, int64_t ldg,
                             int64_t head_dim, int64_t M, int64_t K, QDst q, float* scale, void* y_out,
                             int64_t ldy, hipStream_t st);
// GDN output: gated RMSNorm over heads of head_dim (64, 128, 256 or 512), then quantize_rows over the
// whole row. 16-bit inputs; w is head_dim entries of the input dtype or fp32.
hipError_t launch_gdn_norm_quant(int mode, int dt, int dtw, const void* x, int64_t ldx, const void* z, int64_t ldz,
                                 const void* w, int head_dim, float eps, int64_t M, int64_t K, QDst q,
                                 float* scale, void* y_out, int64_t ldy, hipStream_t st);
// Packed-row offsets of a ragged batch, passed by value in the kernel arguments:
// segment b owns packed rows [off[b], off[b + 1]).
constexpr int kMaxSegments = 256;
struct SegOffsets {
  int32_t off[kMaxSegments + 1];
};

hipError_t launch_quant_ragged(int mode, int dt, int out_es, const void* x, int64_t ldx, const SegOffsets& segs,
                               int64_t nseg, int64_t width, int64_t K, QDst q, float* scale,
                               int32_t* row_map, void* out, int64_t ldo, int64_t N, hipStream_t st);
enum TileCfg : int {
  kTileAuto = -1,
  kTile256 = 0,      // register-staged 256x256, 4 waves
  kTile128 = 1,      // register-staged 128x128, 4 waves
  kTile64x128 = 2,   // register-staged 64x128, 4 waves
  kDma256w8 = 3,     // DMA pipeline 256x256, 8 waves (128x64 each), 4 stages
  kDma256w4 = 4,     // DMA pipeline 256x256, 4 waves (128x128 each), 4 stages
  kDma128w4 = 5,     // DMA pipeline 128x128, 4 waves (64x64 each), 4 stages
  kDma256x128w4 = 6, // DMA pipeline 256x128, 4 waves (128x64 each), 4 stages
  kDma128w4k128 = 7, // DMA pipeline 128x128, 4 waves, 128-byte K steps (weight streaming, K % 128 == 0)
  kDma256x192w4 = 8, // DMA pipeline 256x192, 4 waves (128x96 each), 4 stages; not for SwiGLU
  kWs = 9,           // weight streaming for skinny M: 32- or 64-column slabs, waves split K (K % 128 == 0)
  kDma192x192w4 = 10, // DMA pipeline 192x192, 4 waves (96x96 each), 4 stages; not for SwiGLU
  kDma192x128w4 = 11, // DMA pipeline 192x128, 4 waves (96x64 each), 4 stages
  kTileCount = 12
};

constexpr int kMaxKSplit = 32;

// Tile and split-K choice for one GEMM. `tile` / `ksplit` < 0 ask for the
// automatic choice; a workspace of `ws_bytes` (0: none) bounds ksplit.
struct GemmPlan {
  int tile, ksplit;
  int tiles_m, tiles_n;
  int64_t ws_bytes;  // workspace the plan uses (0 when ksplit == 1)
  const char* error; // non-null: the request is not valid
};
// `epi` (an Epilogue) rules out tiles the epilogue cannot use; a K-blocked operand (`a_kblk`,
// `w_kblk`) rules out the register-staged tiles.
// `mode` (kInt8 / kFp8) picks between tiles that compute the same result.
GemmPlan plan_gemm(int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldw, int tile, int ksplit,
                   int64_t ws_bytes, int epi, bool a_kblk = false, bool w_kblk = false, int mode = kFp8);

// Largest row capacity of a K-blocked operand: the pipelined tiles keep per-lane offsets (two K blocks
// apart at most) below 2^32.
constexpr int64_t kMaxKblkRows = (int64_t)1 << 25;
// Launches the plan; p.partial must point to a workspace of plan.ws_bytes.
hipError_t launch_gemm(int mode, GemmParams p, int epi, int out_dt, const GemmPlan& plan, hipStream_t st);

constexpr int64_t kMaxVecK = 32 * 512;  // longest row the one-pass quant kernels hold in registers

// Compute units of the current device (queried once per device).
int device_cu_count();
// Whether the pipelined GEMMs that can run persistently (one workgroup per CU
// walking several tiles) do so: only with D3W8A8_GEMM_PERSIST=1 in the
// environment (read at every launch; one workgroup per tile is faster).
bool gemm_persistent();

// Column slab of the weight-streaming tile: 32 columns, 64 (one gate/up pair) with SwiGLU, and two
// pairs where 64-column slabs would not fit one round of CUs (gate_up, N = 24576 at M = 128: 28.9
// against 35.5 us for 384 slabs of 64, and 30.8 us for the 128x128 tile).
inline int ws_slab_blocks(int64_t N, int epi, int64_t cus) {
  if (epi != kEpiSwiGLU) return 1;
  return (N + 63) / 64 <= cus ? 2 : 4;
}

}  // namespace d3
