// Fused zero-centred RMSNorm + per-token quantization for gfx950.
//
//   y = DT( (x * rstd) * g ),  g = 1 + w (zero_centered) or w,
//   rstd = 1 / sqrt(sum(x*x) / K + eps)  (sqrt and division each correctly rounded), then q(y).
//
// RMSNorm is transformers' Qwen3_5RMSNorm (modeling_qwen3_5.py:720-734), the
// norm TRT-LLM's RMSNorm(use_gemma=True) applies before each linear group
// (d3trt/model/trtllm_stack.py:217-228, core.py:207, 215); the quantization
// is d3trt/model/quant.py:92-100.
//
// Optional outputs: the normed rows y, and clear_amax[row] = 0 (the SwiGLU
// row-amax buffer of the same rows, so the next GEMM can atomically max into
// it without a memset).
#include "quant_common.hpp"

namespace d3 {

template <int MODE, int DT, int DTW, int NCH, bool FULL>
__global__ __launch_bounds__(256) void rmsnorm_quant_vec(
    const void* __restrict__ x, int64_t ldx, const void* __restrict__ w, int64_t M, int64_t K,
    float eps, int zc, const QDst qd, float* __restrict__ scale,
    void* __restrict__ normed, int64_t ldn, float* __restrict__ clear_amax) {
  extern __shared__ __attribute__((aligned(16))) float gain_lds[];  // K floats: g = 1 + w (zc) or w
  const int lane = threadIdx.x & 63;
  const int64_t row0 = (int64_t)blockIdx.x * kQuantWaves + (threadIdx.x >> 6);
  using RC = RowChunks<DT, NCH, FULL>;
  // Waves past the last row still take part in the gain set-up and its barrier.
  const bool live = row0 < M;
  auto stage_gain = [&] {
    // The gain is the same for every row: the block forms it once in fp32 (the
    // values the reference's (1 + w.float()) holds) and every wave reads it from
    // LDS, instead of each wave loading and widening the weight row.
    {
      using RW = RowChunks<DTW, 1, true>;
      constexpr int PIECES = (NCH * 64 + 255) / 256;  // 8-element pieces per thread: NCH * 64 over 256 threads
      RW wp[PIECES];
#pragma unroll
      for (int i = 0; i < PIECES; ++i) {
        const int64_t k = (int64_t)(threadIdx.x + 256 * i) * 8;
        if (k < K) {
          const uint4* src = (const uint4*)((const char*)w + k * RW::kES);
#pragma unroll
          for (int u = 0; u < RW::kWords / 4; ++u) {
            const uint4 t = src[u];
            wp[i].w[0][4 * u] = t.x;
            wp[i].w[0][4 * u + 1] = t.y;
            wp[i].w[0][4 * u + 2] = t.z;
            wp[i].w[0][4 * u + 3] = t.w;
          }
        }
      }
#pragma unroll
      for (int i = 0; i < PIECES; ++i) {
        const int64_t k = (int64_t)(threadIdx.x + 256 * i) * 8;
        if (k < K) {
          float g[8];
          wp[i].get(0, g);
#pragma unroll
          for (int u = 0; u < 8; ++u) g[u] = zc ? 1.0f + g[u] : g[u];
          *(float4*)(gain_lds + k) = make_float4(g[0], g[1], g[2], g[3]);
          *(float4*)(gain_lds + k + 4) = make_float4(g[4], g[5], g[6], g[7]);
        }
      }
    }
    __syncthreads();
  };
  if (!live) {
    stage_gain();
    return;
  }
  pipeline_rows<RC>(
      (const char*)x, ldx * RC::kES, row0, (int64_t)gridDim.x * kQuantWaves, M, K, lane, stage_gain, [&](RC& x_, int64_t row) {
        // sum of squares: for 16-bit inputs one v_dot2 per packed pair (the squares of bf16 / fp16
        // values are exact in fp32, as torch's x.float().pow(2) is)
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
#pragma unroll
              for (int i = 0; i < 4; ++i) ss = dot2_sq<DT>(x_.w[c][i], ss);
            }
          }
        }
        ss = wave_sum(ss);
        const float var = ss / (float)K;
        const float t = var + eps;
        const float rstd = 1.0f / sqrtf(t);  // torch.rsqrt on the CPU: 1 / sqrt(t), each step correctly rounded
        // y, rounded to DT, kept packed (the normed output is stored from these words as they are)
        RC y;
        float amax = 0.0f;
        [[maybe_unused]] Bf16PairAmax am16;
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
        if constexpr (NCH > 12) y.fence();  // wide rows: keep y packed between the passes (registers)
        char* qr = qd.row(row);
        char* nr = normed ? (char*)normed + row * ldn * RC::kES : nullptr;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
          if (RC::valid(c, lane, K)) {
            const int64_t col = RC::col(c, lane);
            float v[8];
            y.get(c, v);
            quant_store8<MODE>(QDst::at(qr, col, qd.bs), v, s);
            if (nr) y.store_raw(c, nr + col * RC::kES);
          }
        }
        if (lane == 0) {
          scale[row] = s.s;
          if (clear_amax) clear_amax[row] = 0.0f;
        }
      });
}

// The same RMSNorm + quantize for few rows: one 256-thread block per row, thread
// t taking the 8-element chunks t, t + 256, ... (NCT of them, K <= 2048 NCT; a
// chunk past the row's end re-reads the row's last chunk and is not used). All
// loads (the row and its gain) issue first; the sum of squares and the amax are
// reduced over the wave (fixed DPP order) and then over the four waves through
// LDS (in wave order). Each row's work is spread over 4x the lanes, so a batch
// of a few hundred rows occupies more CUs with a shorter chain per row; at
// M = 4096 the row-pipelined kernel above is faster (12.0 against 14.1 us).
template <int MODE, int DT, int DTW, int NCT>
__global__ __launch_bounds__(256) void rmsnorm_quant_rowblock(
    const void* __restrict__ x, int64_t ldx, const void* __restrict__ w, int64_t K, float eps, int zc,
    const QDst qd, float* __restrict__ scale, void* __restrict__ normed, int64_t ldn,
    float* __restrict__ clear_amax) {
  using RC = RowChunks<DT, 1, true>;
  using RW = RowChunks<DTW, 1, true>;
  __shared__ float red[2][kQuantWaves];
  const int64_t row = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t nch = K / 8;
  const char* xr = (const char*)x + row * ldx * RC::kES;
  RC xv[NCT];
  RW wv[NCT];
#pragma unroll
  for (int i = 0; i < NCT; ++i) {
    const int64_t c = min((int64_t)t + 256 * i, nch - 1);
    xv[i].load(xr + c * 8 * RC::kES, 8, 0);
  }
#pragma unroll
  for (int i = 0; i < NCT; ++i) {
    const int64_t c = min((int64_t)t + 256 * i, nch - 1);
    wv[i].load((const char*)w + c * 8 * RW::kES, 8, 0);
  }
  // sum of squares (for 16-bit inputs one v_dot2 per packed pair: the squares are exact in fp32)
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NCT; ++i) {
    if (t + 256 * i < nch) {
      if constexpr (DT == kF32) {
        float v[8];
        xv[i].get(0, v);
#pragma unroll
        for (int k = 0; k < 8; ++k) ss = ss + v[k] * v[k];
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) ss = dot2_sq<DT>(xv[i].w[0][k], ss);
      }
    }
  }
  ss = wave_sum(ss);
  if (lane == 0) red[0][wave] = ss;
  __syncthreads();
  ss = ((red[0][0] + red[0][1]) + red[0][2]) + red[0][3];
  const float var = ss / (float)K;
  const float tv = var + eps;
  const float rstd = 1.0f / sqrtf(tv);  // torch.rsqrt on the CPU: 1 / sqrt(t), each step correctly rounded
  // y, rounded to DT and kept packed
  RC y[NCT];
  float amax = 0.0f;
  [[maybe_unused]] Bf16PairAmax am16;
#pragma unroll
  for (int i = 0; i < NCT; ++i) {
    if (t + 256 * i < nch) {
      float v[8], g[8];
      xv[i].get(0, v);
      wv[i].get(0, g);
#pragma unroll
      for (int k = 0; k < 8; k += 2) {
        const float g0 = zc ? 1.0f + g[k] : g[k], g1 = zc ? 1.0f + g[k + 1] : g[k + 1];
        float p0 = v[k] * rstd, p1 = v[k + 1] * rstd;
        p0 = p0 * g0;
        p1 = p1 * g1;
        if constexpr (DT == kBF16) {
          am16.add(y[i].put_pair_bits(0, k / 2, p0, p1));
        } else {
          y[i].put_pair(0, k / 2, p0, p1);
          amax = amax_acc(amax_acc(amax, p0), p1);
        }
      }
    }
  }
  if constexpr (DT == kBF16) amax = am16.value();
  amax = wave_max(amax);
  if (lane == 0) red[1][wave] = amax;
  __syncthreads();
  amax = amax_join(amax_join(red[1][0], red[1][1]), amax_join(red[1][2], red[1][3]));
  const RowScale s = scale_from_amax<MODE>(amax);
  char* qr = qd.row(row);
  char* nr = normed ? (char*)normed + row * ldn * RC::kES : nullptr;
#pragma unroll
  for (int i = 0; i < NCT; ++i) {
    const int64_t c = (int64_t)t + 256 * i;
    if (c < nch) {
      float v[8];
      y[i].get(0, v);
      quant_store8<MODE>(QDst::at(qr, c * 8, qd.bs), v, s);
      if (nr) y[i].store_raw(0, nr + c * 8 * RC::kES);
    }
  }
  if (t == 0) {
    scale[row] = s.s;
    if (clear_amax) clear_amax[row] = 0.0f;
  }
}

// ---------------------------------------------------------------------------
// GDN output: gated RMSNorm over heads of head_dim, then the per-token quantize
// of out_proj's input (d3trt/model/core.py:390-391: delta.norm(core, z) on rows
// of head_v_dim, reshaped back to [tokens, heads * head_v_dim]; the norm is
// transformers' Qwen3_5RMSNormGated, modeling_qwen3_5.py:168-184, built in the
// model dtype, trtllm_stack.py:198):
//   h = x * rstd_head  (fp32; rstd = 1 / sqrt(mean over the head of x^2 + eps))
//   h = w * DT(h)      (rounded to DT when w is DT; fp32 when w is fp32)
//   y = DT( h * silu(z) ),  silu(z) = z / (1 + exp(-z)) in fp32 (hardware exp2 and
//                            reciprocal: the kernel is VALU-bound)
// then q(y) per token over the whole row. w has head_dim entries, shared by the
// heads. head_dim divides 512 (64, 128, 256, 512): the 8-element pieces of one
// head sit in head_dim / 8 consecutive lanes of one chunk, whose sum of squares
// is a butterfly over those lanes (group_sum). One wave per row.
// ---------------------------------------------------------------------------
// Sum over aligned groups of `group` lanes (8, 16, 32 or 64); every lane of a group ends with the same
// value. Within 16-lane rows the partners come from DPP lane permutes (VALU ops): lane ^ 1, lane ^ 2,
// then the mirror lane of the 8-lane half (the other quad) and of the 16-lane row (the other half).
// Each level adds two values that every lane of the new group holds the same way round (addition
// commutes), so the group stays uniform.
__device__ __forceinline__ float group_sum(float v, int group) {
  v = v + dpp_f32<0xB1, 0xf>(v);   // quad_perm [1, 0, 3, 2]
  v = v + dpp_f32<0x4E, 0xf>(v);   // quad_perm [2, 3, 0, 1]
  v = v + dpp_f32<0x141, 0xf>(v);  // row_half_mirror
  if (group >= 16) v = v + dpp_f32<0x140, 0xf>(v);  // row_mirror
  if (group >= 32) v = v + __shfl_xor(v, 16, 64);
  if (group >= 64) v = v + __shfl_xor(v, 32, 64);
  return v;
}

template <int MODE, int DT, int DTW, int NCH, bool FULL>
__global__ __launch_bounds__(256) void gdn_norm_quant_vec(
    const void* __restrict__ x, int64_t ldx, const void* __restrict__ z, int64_t ldz, const void* __restrict__ w,
    int head_dim, float eps, int64_t M, int64_t K, const QDst qd, float* __restrict__ scale,
    void* __restrict__ y_out, int64_t ldy) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kQuantWaves + (threadIdx.x >> 6);
  if (row >= M) return;
  using RC = RowChunks<DT, NCH, FULL>;
  RC x_, z_;
  x_.load((const char*)x + row * ldx * RC::kES, K, lane);
  z_.load((const char*)z + row * ldz * RC::kES, K, lane);
  // this lane's 8 weights: columns 512 c + 8 lane of every chunk fall on head offset (8 lane) % head_dim
  float wv[8];
  {
    using RW = RowChunks<DTW, 1, true>;
    RW wp;
    const uint4* src = (const uint4*)((const char*)w + (int64_t)((8 * lane) % head_dim) * RW::kES);
#pragma unroll
    for (int u = 0; u < RW::kWords / 4; ++u) {
      const uint4 t = src[u];
      wp.w[0][4 * u] = t.x;
      wp.w[0][4 * u + 1] = t.y;
      wp.w[0][4 * u + 2] = t.z;
      wp.w[0][4 * u + 3] = t.w;
    }
    wp.get(0, wv);
  }
  const int group = head_dim >> 3;  // lanes per head
  // Each head's rstd is computed once, not by every lane that holds a piece of it: the heads' sums of
  // squares go to this wave's LDS slots, slot (g, c) = g * NCH + c for the head that lanes
  // [g * group, (g + 1) * group) hold in chunk c; lanes take the slots in turn and put the rstd back.
  __shared__ __attribute__((aligned(16))) float rstd_lds[kQuantWaves][NCH * 8];
  float* const slots = rstd_lds[threadIdx.x >> 6];
  const int g = lane / group;
  {
    float ss[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      // every lane of the wave takes part in the butterfly; lanes past the row contribute nothing used
      float a = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) a = dot2_sq<DT>(x_.w[c][i], a);
      ss[c] = group_sum(a, group);
    }
    if (lane % group == 0) {
#pragma unroll
      for (int c = 0; c < NCH; ++c) slots[g * NCH + c] = ss[c];
    }
  }
  // the LDS operations of one wave complete in order; the fences keep the compiler from moving the
  // reads of other lanes' slots ahead of the writes
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  {
    // head_dim is a power of two, so ss * (1 / head_dim) is ss / head_dim bit for bit
    const float inv_hd = 1.0f / (float)head_dim;
    const int nslots = NCH * (512 / head_dim);
    for (int j = lane; j < nslots; j += 64) {
      const float t = slots[j] * inv_hd + eps;
      slots[j] = 1.0f / sqrtf(t);  // torch.rsqrt on the CPU: 1 / sqrt(t), each step correctly rounded
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  RC y;
  float amax = 0.0f;
  Bf16PairAmax am16;  // bf16: the amax of the rounded outputs, taken on the packed pairs
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (RC::valid(c, lane, K)) {
      const float rstd = slots[g * NCH + c];
      float v[8], zv[8];
      x_.get(c, v);
      z_.get(c, zv);
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        float h0 = v[i] * rstd, h1 = v[i + 1] * rstd;
        round_pair_to<DT>(h0, h1);  // h.to(input_dtype)
        h0 = wv[i] * h0;
        h1 = wv[i + 1] * h1;
        if constexpr (DTW == DT) round_pair_to<DT>(h0, h1);  // w (DT) * h (DT) is a DT tensor
        // silu with the hardware exp2 and reciprocal (~1e-6 relative; only moves the final bf16
        // rounding next to a rounding boundary)
        const float e0 = __expf(-zv[i]), e1 = __expf(-zv[i + 1]);
        const float d0 = 1.0f + e0, d1 = 1.0f + e1;
        const float s0 = zv[i] * __builtin_amdgcn_rcpf(d0), s1 = zv[i + 1] * __builtin_amdgcn_rcpf(d1);
        float p0 = h0 * s0, p1 = h1 * s1;
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
  if constexpr (NCH > 12) y.fence();
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

template <int MODE, int DT, int DTW>
hipError_t launch_gdn_norm_quant_t(const void* x, int64_t ldx, const void* z, int64_t ldz, const void* w,
                                   int head_dim, float eps, int64_t M, int64_t K, QDst q, float* scale,
                                   void* y_out, int64_t ldy, hipStream_t st) {
  if (M == 0) return hipSuccess;
#define L(N, F) hipLaunchKernelGGL((gdn_norm_quant_vec<MODE, DT, DTW, N, F>), quant_grid(M), dim3(256), 0, st, x, ldx, z, ldz, w, head_dim, eps, M, K, q, scale, y_out, ldy)
  D3_NCH_DISPATCH(K, L);
#undef L
  return hipGetLastError();
}

hipError_t launch_gdn_norm_quant(int mode, int dt, int dtw, const void* x, int64_t ldx, const void* z, int64_t ldz,
                                 const void* w, int head_dim, float eps, int64_t M, int64_t K, QDst q,
                                 float* scale, void* y_out, int64_t ldy, hipStream_t st) {
  if (K > kMaxVecK) return hipErrorInvalidValue;
#define C(MO, D, W) if (mode == MO && dt == D && dtw == W) return launch_gdn_norm_quant_t<MO, D, W>(x, ldx, z, ldz, w, head_dim, eps, M, K, q, scale, y_out, ldy, st)
  C(kInt8, kBF16, kBF16); C(kInt8, kBF16, kF32); C(kInt8, kF16, kF16); C(kInt8, kF16, kF32);
  C(kFp8, kBF16, kBF16); C(kFp8, kBF16, kF32); C(kFp8, kF16, kF16); C(kFp8, kF16, kF32);
#undef C
  return hipErrorInvalidValue;
}

// Row count up to which the block-per-row form runs (question batches).
#ifndef D3_NORM_ROWBLOCK_MAX
#define D3_NORM_ROWBLOCK_MAX 1024
#endif
constexpr int64_t kNormRowBlockMaxRows = D3_NORM_ROWBLOCK_MAX;

template <int MODE, int DT, int DTW>
hipError_t launch_rmsnorm_quant_t(const void* x, int64_t ldx, const void* w, int64_t M, int64_t K, float eps,
                                  int zc, QDst q, float* scale, void* normed, int64_t ldn,
                                  float* clear_amax, hipStream_t st) {
  if (M == 0) return hipSuccess;
  if (M <= kNormRowBlockMaxRows) {
    const int64_t nct = (K / 8 + 255) / 256;  // chunks per thread, K <= kMaxVecK: at most 8
#define R(N)                                                                                                 \
  hipLaunchKernelGGL((rmsnorm_quant_rowblock<MODE, DT, DTW, N>), dim3((unsigned)M), dim3(256), 0, st, x, ldx, w, K, \
                     eps, zc, q, scale, normed, ldn, clear_amax)
    if (nct <= 1) R(1);
    else if (nct <= 2) R(2);
    else if (nct <= 4) R(4);
    else if (nct <= 6) R(6);
    else R(8);
#undef R
    return hipGetLastError();
  }
  const size_t lds = (size_t)K * sizeof(float);  // the staged gain (K <= kMaxVecK: at most 64 KiB)
#define L(N, F)                                                                                               \
  hipLaunchKernelGGL((rmsnorm_quant_vec<MODE, DT, DTW, N, F>),                                                 \
                     row_grid(rmsnorm_quant_vec<MODE, DT, DTW, N, F>, M, lds, kNormRowBlocksPerCU),             \
                     dim3(256), lds, st, x, ldx, w, M, K, eps, zc, q, scale, normed, ldn, clear_amax)
  D3_NCH_DISPATCH(K, L);
#undef L
  return hipGetLastError();
}

hipError_t launch_rmsnorm_quant(int mode, int dt, int dtw, const void* x, int64_t ldx, const void* w, int64_t M,
                                int64_t K, float eps, int zc, QDst q, float* scale, void* normed,
                                int64_t ldn, float* clear_amax, hipStream_t st) {
  if (K > kMaxVecK) return hipErrorInvalidValue;
#define C(MO, D, W) if (mode == MO && dt == D && dtw == W) return launch_rmsnorm_quant_t<MO, D, W>(x, ldx, w, M, K, eps, zc, q, scale, normed, ldn, clear_amax, st)
  C(kInt8, kBF16, kBF16); C(kInt8, kBF16, kF32); C(kInt8, kF16, kF16); C(kInt8, kF16, kF32); C(kInt8, kF32, kF32);
  C(kFp8, kBF16, kBF16); C(kFp8, kBF16, kF32); C(kFp8, kF16, kF16); C(kFp8, kF16, kF32); C(kFp8, kF32, kF32);
#undef C
  return hipErrorInvalidValue;
}

}  // namespace d3
