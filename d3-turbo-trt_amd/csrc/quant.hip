// Per-token quantization kernels for gfx950: plain, from a precomputed row
// amax (after SwiGLU), and the ragged gather form. The fused RMSNorm form is
// in norm_quant.hip.
//
// Every row is read from HBM exactly once, with 128-bit loads, and held in
// registers while its amax is formed. The plain and requantizing kernels give
// each row a 256-thread block (thread t: the 8-element chunks t, t + 256, ...);
// the gated and ragged kernels give each row one 64-lane wave (lane l: the
// chunks at columns 512 c + 8 l).
//
// Reference arithmetic: d3trt/model/quant.py:92-100 (quantize_rows) and
// :77-89 (quantize_weight, the same per-row arithmetic over [N, K]).
#include "quant_common.hpp"

#include <stdlib.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <utility>
#include <vector>

namespace d3 {

int kernel_blocks_per_cu(const void* kernel, size_t lds_bytes) {
  static std::mutex mu;
  static std::vector<std::pair<const void*, int>> cache;  // one entry per kernel (the LDS size is fixed per kernel)
  std::lock_guard<std::mutex> lock(mu);
  for (const auto& e : cache)
    if (e.first == kernel) return e.second;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, 256, lds_bytes) != hipSuccess || n < 1) n = 1;
  cache.emplace_back(kernel, n);
  return n;
}

int row_blocks_per_cu(int dflt) {
  static const int v = [] {
    const char* e = getenv("D3W8A8_ROW_BLOCKS_PER_CU");
    const int n = e ? atoi(e) : 0;
    return n >= 1 && n <= 1024 ? n : 0;
  }();
  return v ? v : dflt;
}

int device_cu_count() {
  static std::atomic<int> cus[64];  // 0 until queried; concurrent first calls store the same value
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) n = 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// ---------------------------------------------------------------------------
// quantize_rows: x [M, K] (ld ldx) -> q [M, K] + scale [M]; q is row-major
// or K-blocked (QDst, kernels.hpp).
// Vector path: K % 8 == 0, rows 16B aligned.
// ---------------------------------------------------------------------------
// One 256-thread block per row: thread t takes the 8-element chunks t, t + 256,
// ... (NCT of them, K <= 2048 NCT; a chunk past the row's end re-reads the last
// chunk and is not used). Every load issues first; the amax is reduced over
// the wave (fixed DPP order) and then over the four waves through LDS. Many
// small blocks per CU keep other rows' loads in flight while a row is
// quantized: FP8, 4096 x 4096 bf16 11.1 -> 10.5 us and 4096 x 12288
// 30.5 -> 25.3 us (74% of 8 TB/s) against one wave per row walking rows with
// one row prefetched.
template <int MODE, int DT, int NCT>
__global__ __launch_bounds__(256) void quant_rows_stream(const void* __restrict__ x, int64_t ldx, int64_t K,
                                                        const QDst qd, float* __restrict__ scale) {
  using RC = RowChunks<DT, 1, true>;
  __shared__ float red[kQuantWaves];
  const int64_t row = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t nch = K / 8;
  const char* xr = (const char*)x + row * ldx * RC::kES;
  RC v[NCT];
#pragma unroll
  for (int i = 0; i < NCT; ++i) {
    const int64_t c = min((int64_t)t + 256 * i, nch - 1);
    v[i].load(xr + c * 8 * RC::kES, 8, 0);
  }
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < NCT; ++i)
    if (t + 256 * i < nch) m = amax_join(m, v[i].amax(8, 0));
  m = wave_max(m);
  if (lane == 0) red[wave] = m;
  __syncthreads();
  m = amax_join(amax_join(red[0], red[1]), amax_join(red[2], red[3]));
  const RowScale s = scale_from_amax<MODE>(m);
  char* qr = qd.row(row);
#pragma unroll
  for (int i = 0; i < NCT; ++i) {
    const int64_t c = (int64_t)t + 256 * i;
    if (c < nch) {
      float f[8];
      v[i].get(0, f);
      quant_store8<MODE>(QDst::at(qr, c * 8, qd.bs), f, s);
    }
  }
  if (t == 0) scale[row] = s.s;
}

// ---------------------------------------------------------------------------
// K-blocked q (QDst, kernels.hpp): two rows per block. In that layout the 64-byte K block of rows 2p
// and 2p + 1 is one 128-byte line; with one row per block every line would be written in two halves
// by two blocks (FP8, 4096 x 4096 bf16: 10.5 -> 12.2 us; requantize 4096 x 12288: 25.5 -> 33.6 us).
// Here lane l of wave w takes row 2p + l / 32 and the 8-element chunks (l % 32) + 32 w + 128 i, so
// each store instruction writes K blocks of both rows: whole lines. The row amax is reduced over the
// lanes of the row's half wave (DPP) and then over the four waves through LDS; AMAX_IN takes it from
// the SwiGLU epilogue instead (requantization). A missing second row (odd M) re-reads the last row
// and stores nothing.
// ---------------------------------------------------------------------------
// max over each half wave (lanes 0-31, 32-63) of values >= 0, returned to the lanes of that half
__device__ __forceinline__ float half_wave_max(float v, int lane) {
  const auto join = [](float a, float b) { return amax_join(a, b); };
  v = join(v, dpp_f32<0x111, 0xf>(v));  // row_shr:1
  v = join(v, dpp_f32<0x112, 0xf>(v));  // row_shr:2
  v = join(v, dpp_f32<0x114, 0xf>(v));  // row_shr:4
  v = join(v, dpp_f32<0x118, 0xf>(v));  // row_shr:8
  v = join(v, dpp_f32<0x142, 0xa>(v));  // row_bcast:15 into rows 1 and 3: lane 31 holds lanes 0-31, lane 63 32-63
  const float lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
  const float hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
  return lane < 32 ? lo : hi;
}

template <int MODE, int DT, int NCT, bool AMAX_IN>
__global__ __launch_bounds__(256) void quant_rows_pair(const void* __restrict__ x, int64_t ldx,
                                                      const float* __restrict__ amax_in, int64_t M, int64_t K,
                                                      const QDst qd, float* __restrict__ scale) {
  using RC = RowChunks<DT, 1, true>;
  __shared__ float red[2][kQuantWaves];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, half = lane >> 5, j = lane & 31;
  const int64_t row = 2 * (int64_t)blockIdx.x + half;
  const int64_t rrow = min(row, M - 1);
  const int64_t nch = K / 8;
  const char* xr = (const char*)x + rrow * ldx * RC::kES;
  RC v[NCT];
#pragma unroll
  for (int i = 0; i < NCT; ++i) {
    const int64_t c = min((int64_t)j + 32 * wave + 128 * i, nch - 1);
    v[i].load(xr + c * 8 * RC::kES, 8, 0);
  }
  float m;
  if constexpr (AMAX_IN) {
    m = amax_in[rrow];
  } else {
    m = 0.0f;
#pragma unroll
    for (int i = 0; i < NCT; ++i)
      if (j + 32 * wave + 128 * i < nch) m = amax_join(m, v[i].amax(8, 0));
    m = half_wave_max(m, lane);
    if (j == 0) red[half][wave] = m;
    __syncthreads();
    m = amax_join(amax_join(red[half][0], red[half][1]), amax_join(red[half][2], red[half][3]));
  }
  const RowScale s = scale_from_amax<MODE>(m);
  if (row >= M) return;
  char* qr = qd.row(row);
#pragma unroll
  for (int i = 0; i < NCT; ++i) {
    const int64_t c = (int64_t)j + 32 * wave + 128 * i;
    if (c < nch) {
      float f[8];
      v[i].get(0, f);
      quant_store8<MODE, AMAX_IN>(QDst::at(qr, c * 8, qd.bs), f, s);  // amax from outside: keep the clamp
    }
  }
  if (wave == 0 && j == 0) scale[row] = s.s;
}

// Generic path for any K / alignment: two passes over the row (amax, then quantize).
template <int MODE, int DT>
__global__ __launch_bounds__(256) void quant_rows_generic(const void* __restrict__ x, int64_t ldx,
                                                         int64_t M, int64_t K, const QDst qd,
                                                         float* __restrict__ scale) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kQuantWaves + (threadIdx.x >> 6);
  if (row >= M) return;
  const int64_t base = row * ldx;
  float amax = 0.0f;
  for (int64_t k = lane; k < K; k += 64) amax = amax_acc(amax, load_elem<DT>(x, base + k));
  amax = wave_max(amax);
  const RowScale s = scale_from_amax<MODE>(amax);
  char* qr = qd.row(row);
  for (int64_t k = lane; k < K; k += 64) {
    const float xv = load_elem<DT>(x, base + k);
    uint8_t* qk = (uint8_t*)QDst::at(qr, k, qd.bs);
    if constexpr (MODE == kInt8) *qk = (uint8_t)quant_i8_bits<false>(xv, s);
    else *qk = (uint8_t)(quant_f8_pair(xv, 0.0f, s) & 0xff);
  }
  if (lane == 0) scale[row] = s.s;
}

// ---------------------------------------------------------------------------
// Requantization with a known row amax (SwiGLU output h [M, K]).
// The scale comes from outside, so nothing waits for a whole row: the kernel
// is a plain stream. One 256-thread block per row; thread t takes the
// 8-element chunks t, t + 256, ... (NCT of them, K <= 2048 NCT), issues all
// its loads (a chunk past the row's end re-reads the row's last chunk and is
// not stored), forms the row scale while they fly, then quantizes and stores
// 8 bytes per chunk. Many small blocks per CU keep the HBM queue full
// (4096 x 12288 bf16: 31.0 us in the row-pipelined form, one wave per row).
// ---------------------------------------------------------------------------
template <int MODE, int DT, int NCT>
__global__ __launch_bounds__(256) void quant_rows_amax_stream(const void* __restrict__ h, int64_t ldh,
                                                             const float* __restrict__ amax_in, int64_t K,
                                                             const QDst qd, float* __restrict__ scale) {
  using RC = RowChunks<DT, 1, true>;
  const int64_t row = blockIdx.x;
  const int t = threadIdx.x;
  const int64_t nch = K / 8;
  const char* hr = (const char*)h + row * ldh * RC::kES;
  RC v[NCT];
#pragma unroll
  for (int i = 0; i < NCT; ++i) {
    const int64_t c = min((int64_t)t + 256 * i, nch - 1);
    v[i].load(hr + c * 8 * RC::kES, 8, 0);
  }
  const RowScale s = scale_from_amax<MODE>(amax_in[row]);
  char* qr = qd.row(row);
#pragma unroll
  for (int i = 0; i < NCT; ++i) {
    const int64_t c = (int64_t)t + 256 * i;
    if (c < nch) {
      float f[8];
      v[i].get(0, f);
      quant_store8<MODE, true>(QDst::at(qr, c * 8, qd.bs), f, s);  // amax from outside: keep the clamp
    }
  }
  if (t == 0) scale[row] = s.s;
}

// ---------------------------------------------------------------------------
// Gated o_proj input: y = DT( x * DT(sigmoid(gate)) ), then quantize_rows(y)
// (d3trt/model/core.py:297: o_proj(out * torch.sigmoid(gate)); torch rounds
// the sigmoid to the tensor dtype, then the product). The gate is either a
// [M, K] tensor (head_dim == 0) or read in place from the q_proj output, whose
// rows hold per head [query (head_dim) | gate (head_dim)] (core.py:231, the
// chunk of the q_proj output viewed as [.., heads, 2 head_dim]): gate column k
// sits at (k / head_dim) * 2 head_dim + head_dim + k % head_dim
// (head_dim % 8 == 0, so an 8-element chunk never straddles two heads).
// One wave per row; optional y output (the bf16 product). The sigmoid uses the
// hardware exp2 and reciprocal: the kernel is VALU-bound, and their ~1e-6
// relative error only moves the bf16 rounding of the sigmoid next to a
// rounding boundary.
// ---------------------------------------------------------------------------
template <int MODE, int DT, int NCH, bool FULL>
__global__ __launch_bounds__(256) void gate_quant_vec(const void* __restrict__ x, int64_t ldx,
                                                     const void* __restrict__ gate, int64_t ldg, int64_t head_dim,
                                                     int64_t M, int64_t K, const QDst qd,
                                                     float* __restrict__ scale, void* __restrict__ y_out,
                                                     int64_t ldy) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kQuantWaves + (threadIdx.x >> 6);
  if (row >= M) return;
  using RC = RowChunks<DT, NCH, FULL>;
  RC x_, g_;
  x_.load((const char*)x + row * ldx * RC::kES, K, lane);
  {
    const char* grow = (const char*)gate + row * ldg * RC::kES;
    // (k / hd) * 2 hd + hd + k % hd = k + hd * (k / hd + 1), with k / hd = umulhi(k, m),
    // m = floor((2^32 - 1) / hd) + 1: exact for k < 2^16 and 8 <= hd < 2^16 (K <= kMaxVecK), since
    // k * m / 2^32 exceeds k / hd by less than k / 2^32 <= 2^-16 < 1 / hd
    const uint32_t hd = (uint32_t)head_dim;
    const uint32_t m = hd ? 0xffffffffu / hd + 1u : 0u;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const uint32_t k = (uint32_t)(FULL ? RC::col(c, lane) : min(RC::col(c, lane), K - 8));
      const uint32_t gk = hd ? k + hd * (__umulhi(k, m) + 1u) : k;
      const uint4 t = *(const uint4*)(grow + (int64_t)gk * RC::kES);
      g_.w[c][0] = t.x;
      g_.w[c][1] = t.y;
      g_.w[c][2] = t.z;
      g_.w[c][3] = t.w;
    }
  }
  RC y;
  float amax = 0.0f;
  Bf16PairAmax am16;  // bf16: the amax of the rounded products, taken on the packed pairs
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (RC::valid(c, lane, K)) {
      float v[8], gv[8];
      x_.get(c, v);
      g_.get(c, gv);
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        // hardware exp2 and reciprocal (~1e-6 relative): the bf16 rounding that follows absorbs that
        // except within ~1e-6 of a rounding boundary (a 1-ulp difference on < 1e-3 of elements)
        float s0 = __builtin_amdgcn_rcpf(1.0f + __expf(-gv[i]));
        float s1 = __builtin_amdgcn_rcpf(1.0f + __expf(-gv[i + 1]));
        round_pair_to<DT>(s0, s1);  // torch.sigmoid's output in the tensor dtype
        float p0 = v[i] * s0, p1 = v[i + 1] * s1;
        if constexpr (DT == kBF16) {
          am16.add(y.put_pair_bits(c, i / 2, p0, p1));
        } else {
          y.put_pair(c, i / 2, p0, p1);
          amax = amax_acc(amax_acc(amax, p0), p1);
        }
      }
    }
  }
  if constexpr (DT == kBF16) amax = am16.value();
  const RowScale s = scale_from_amax<MODE>(wave_max(amax));
  char* qr = qd.row(row);
  char* yr = y_out ? (char*)y_out + row * ldy * RC::kES : nullptr;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (RC::valid(c, lane, K)) {
      float v[8];
      y.get(c, v);
      quant_store8<MODE>(QDst::at(qr, RC::col(c, lane), qd.bs), v, s);
      if (yr) y.store_raw(c, yr + RC::col(c, lane) * RC::kES);
    }
  }
  if (lane == 0) scale[row] = s.s;
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
template <int MODE, int DT, int NCH, bool FULL, int OUTES>
__global__ __launch_bounds__(256) void quant_rows_ragged_vec(
    const void* __restrict__ x, int64_t ldx, const SegOffsets segs, int64_t nseg,
    int64_t width, int64_t K, const QDst qd, float* __restrict__ scale,
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
  using RC = RowChunks<DT, NCH, FULL>;
  RC x_;
  x_.load((const char*)x + prow * ldx * RC::kES, K, lane);
  const RowScale s = scale_from_amax<MODE>(wave_max(x_.amax(K, lane)));
  if constexpr (NCH > 12) x_.fence();  // wide rows: keep them packed between the passes (occupancy)
  char* qr = qd.row(dst);
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (RC::valid(c, lane, K)) {
      float v[8];
      x_.get(c, v);
      quant_store8<MODE>(QDst::at(qr, RC::col(c, lane), qd.bs), v, s);
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

constexpr int64_t kMaxRowBlocks = (int64_t)1 << 30;  // rows per launch of the block-per-row kernels

// The two-row kernel for a K-blocked q (rows of 64-byte pieces 64 bytes apart), in launches of at most
// kMaxRowBlocks blocks. AMAX_IN: the row amax comes from `amax` (requantization).
template <int MODE, int DT, bool AMAX_IN>
hipError_t launch_quant_pair(const void* x, int64_t ldx, const float* amax, int64_t M, int64_t K, QDst q,
                             float* scale, hipStream_t st) {
  const int64_t nct = (K / 8 + 127) / 128;  // chunks per thread, K <= kMaxVecK: at most 16
  for (int64_t r0 = 0; r0 < M; r0 += 2 * kMaxRowBlocks) {
    const int64_t rows = std::min<int64_t>(M - r0, 2 * kMaxRowBlocks);
    const char* xr = (const char*)x + r0 * ldx * (DT == kF32 ? 4 : 2);
    const QDst qr = q.rows_from(r0);
    const float* ar = AMAX_IN ? amax + r0 : nullptr;
#define L(N) hipLaunchKernelGGL((quant_rows_pair<MODE, DT, N, AMAX_IN>), dim3((unsigned)((rows + 1) / 2)), dim3(256), 0, st, xr, ldx, ar, rows, K, qr, scale + r0)
    if (nct <= 1) L(1);
    else if (nct <= 2) L(2);
    else if (nct <= 4) L(4);
    else if (nct <= 6) L(6);
    else if (nct <= 8) L(8);
    else if (nct <= 12) L(12);
    else L(16);
#undef L
  }
  return hipGetLastError();
}

template <int MODE, int DT>
hipError_t launch_quant_rows_t(const void* x, int64_t ldx, int64_t M, int64_t K, QDst q, float* scale, bool vec,
                               hipStream_t st) {
  if (M == 0) return hipSuccess;
  if (vec && K <= kMaxVecK && q.kblocked()) return launch_quant_pair<MODE, DT, false>(x, ldx, nullptr, M, K, q, scale, st);
  if (vec && K <= kMaxVecK) {
    const int64_t nct = (K / 8 + 255) / 256;
    // one block per row, in launches of at most kMaxRowBlocks rows (the grid's x limit)
    for (int64_t r0 = 0; r0 < M; r0 += kMaxRowBlocks) {
      const unsigned rows = (unsigned)std::min<int64_t>(M - r0, kMaxRowBlocks);
      const char* xr = (const char*)x + r0 * ldx * (DT == kF32 ? 4 : 2);
      const QDst qr = q.rows_from(r0);
#define L(N) hipLaunchKernelGGL((quant_rows_stream<MODE, DT, N>), dim3(rows), dim3(256), 0, st, xr, ldx, K, qr, scale + r0)
      if (nct <= 1) L(1);
      else if (nct <= 2) L(2);
      else if (nct <= 4) L(4);
      else if (nct <= 6) L(6);
      else L(8);
#undef L
    }
  } else {
    hipLaunchKernelGGL((quant_rows_generic<MODE, DT>), quant_grid(M), dim3(256), 0, st, x, ldx, M, K, q, scale);
  }
  return hipGetLastError();
}

hipError_t launch_quant_rows(int mode, int dt, const void* x, int64_t ldx, int64_t M, int64_t K, QDst q,
                             float* scale, bool vec, hipStream_t st) {
#define C(MO, D) if (mode == MO && dt == D) return launch_quant_rows_t<MO, D>(x, ldx, M, K, q, scale, vec, st)
  C(kInt8, kBF16); C(kInt8, kF16); C(kInt8, kF32);
  C(kFp8, kBF16); C(kFp8, kF16); C(kFp8, kF32);
#undef C
  return hipErrorInvalidValue;
}

template <int MODE, int DT>
hipError_t launch_quant_rows_amax_t(const void* h, int64_t ldh, const float* amax, int64_t M, int64_t K, QDst q,
                                    float* scale, hipStream_t st) {
  if (M == 0) return hipSuccess;
  if (q.kblocked()) return launch_quant_pair<MODE, DT, true>(h, ldh, amax, M, K, q, scale, st);
  const int64_t nct = (K / 8 + 255) / 256;  // chunks per thread, K <= kMaxVecK: at most 8
  for (int64_t r0 = 0; r0 < M; r0 += kMaxRowBlocks) {
    const unsigned rows = (unsigned)std::min<int64_t>(M - r0, kMaxRowBlocks);
    const char* hr = (const char*)h + r0 * ldh * (DT == kF32 ? 4 : 2);
    const QDst qr = q.rows_from(r0);
#define L(N) hipLaunchKernelGGL((quant_rows_amax_stream<MODE, DT, N>), dim3(rows), dim3(256), 0, st, hr, ldh, amax + r0, K, qr, scale + r0)
    if (nct <= 1) L(1);
    else if (nct <= 2) L(2);
    else if (nct <= 4) L(4);
    else if (nct <= 6) L(6);
    else L(8);
#undef L
  }
  return hipGetLastError();
}

hipError_t launch_quant_rows_amax(int mode, int dt, const void* h, int64_t ldh, const float* amax, int64_t M,
                                  int64_t K, QDst q, float* scale, hipStream_t st) {
  if (K > kMaxVecK) return hipErrorInvalidValue;
#define C(MO, D) if (mode == MO && dt == D) return launch_quant_rows_amax_t<MO, D>(h, ldh, amax, M, K, q, scale, st)
  C(kInt8, kBF16); C(kInt8, kF16); C(kInt8, kF32);
  C(kFp8, kBF16); C(kFp8, kF16); C(kFp8, kF32);
#undef C
  return hipErrorInvalidValue;
}

template <int MODE, int DT>
hipError_t launch_gate_quant_t(const void* x, int64_t ldx, const void* gate, int64_t ldg, int64_t head_dim, int64_t M,
                               int64_t K, QDst q, float* scale, void* y_out, int64_t ldy, hipStream_t st) {
  if (M == 0) return hipSuccess;
#define L(N, F) hipLaunchKernelGGL((gate_quant_vec<MODE, DT, N, F>), quant_grid(M), dim3(256), 0, st, x, ldx, gate, ldg, head_dim, M, K, q, scale, y_out, ldy)
  D3_NCH_DISPATCH(K, L);
#undef L
  return hipGetLastError();
}

hipError_t launch_gate_quant(int mode, int dt, const void* x, int64_t ldx, const void* gate, int64_t ldg,
                             int64_t head_dim, int64_t M, int64_t K, QDst q, float* scale, void* y_out,
                             int64_t ldy, hipStream_t st) {
  if (K > kMaxVecK) return hipErrorInvalidValue;
#define C(MO, D) if (mode == MO && dt == D) return launch_gate_quant_t<MO, D>(x, ldx, gate, ldg, head_dim, M, K, q, scale, y_out, ldy, st)
  C(kInt8, kBF16); C(kInt8, kF16); C(kFp8, kBF16); C(kFp8, kF16);
#undef C
  return hipErrorInvalidValue;
}

template <int MODE, int DT, int OUTES>
hipError_t launch_quant_ragged_t(const void* x, int64_t ldx, const SegOffsets& segs, int64_t nseg, int64_t width,
                                 int64_t K, QDst q, float* scale, int32_t* row_map, void* out,
                                 int64_t ldo, int64_t N, hipStream_t st) {
  const int64_t rows = nseg * width;
  if (rows == 0) return hipSuccess;
#define L(NC, F) hipLaunchKernelGGL((quant_rows_ragged_vec<MODE, DT, NC, F, OUTES>), quant_grid(rows), dim3(256), 0, st, x, ldx, segs, nseg, width, K, q, scale, row_map, out, ldo, N)
  D3_NCH_DISPATCH(K, L);
#undef L
  return hipGetLastError();
}

hipError_t launch_quant_ragged(int mode, int dt, int out_es, const void* x, int64_t ldx, const SegOffsets& segs,
                               int64_t nseg, int64_t width, int64_t K, QDst q, float* scale,
                               int32_t* row_map, void* out, int64_t ldo, int64_t N, hipStream_t st) {
  if (K > kMaxVecK) return hipErrorInvalidValue;
#define C(MO, D, E) if (mode == MO && dt == D && out_es == E) return launch_quant_ragged_t<MO, D, E>(x, ldx, segs, nseg, width, K, q, scale, row_map, out, ldo, N, st)
  C(kInt8, kBF16, 2); C(kInt8, kBF16, 4); C(kInt8, kF16, 2); C(kInt8, kF16, 4); C(kInt8, kF32, 2); C(kInt8, kF32, 4);
  C(kFp8, kBF16, 2); C(kFp8, kBF16, 4); C(kFp8, kF16, 2); C(kFp8, kF16, 4); C(kFp8, kF32, 2); C(kFp8, kF32, 4);
#undef C
  return hipErrorInvalidValue;
}

}  // namespace d3
