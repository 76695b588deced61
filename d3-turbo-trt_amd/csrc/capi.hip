// C ABI of the gfx950 W8A8 Linear library (declared in include/d3w8a8.h).
//
// Every entry point validates its arguments on the host, so a kernel is only
// ever launched on shapes, strides and alignments it was written for; a bad
// argument returns D3W8A8_EINVAL with a message instead of reaching the GPU.
#include <stdio.h>
#include <stdarg.h>

#include <atomic>
#include <mutex>

#include "common.hpp"
#include "kernels.hpp"
#include "../../include/d3w8a8.h"

static_assert(d3::kMaxSegments == D3W8A8_MAX_SEGMENTS, "segment limit of the C ABI and the kernels");
static_assert(d3::kTileCount == D3W8A8_TILE_LAST + 1, "tile codes of the C ABI and the planner");

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return D3W8A8_OK;
  if (e == hipErrorInvalidValue) return fail(D3W8A8_EINVAL, "%s: unsupported argument combination", what);
  return fail(D3W8A8_EHIP, "%s: %s", what, hipGetErrorString(e));
}

// mode: D3W8A8_INT8 / D3W8A8_FP8, optionally with the layout flags D3W8A8_KBLOCK (q / a) and
// D3W8A8_W_KBLOCK (w of the GEMMs)
int base_mode(int m) { return m & ~(D3W8A8_KBLOCK | D3W8A8_W_KBLOCK); }
bool kblk(int m) { return (m & D3W8A8_KBLOCK) != 0; }
bool w_kblk(int m) { return (m & D3W8A8_W_KBLOCK) != 0; }
bool mode_ok(int m) { return base_mode(m) == D3W8A8_INT8 || base_mode(m) == D3W8A8_FP8; }
bool quant_mode_ok(int m) { return mode_ok(m) && !w_kblk(m); }

// Layout of a quantize entry point's q: row-major [rows, K] (ldq >= K; a multiple of 8 where the
// kernel stores 8 bytes at a time) or, with D3W8A8_KBLOCK, K-blocked (K % 64 == 0, ldq >= rows).
const char* q_layout_error(int mode, int64_t rows, int64_t K, int64_t ldq, bool need8) {
  if (kblk(mode)) {
    if (K % 64 != 0) return "a K-blocked q needs K % 64 == 0";
    if (ldq < rows) return "a K-blocked q needs ldq >= its rows (ldq is the row capacity)";
    return nullptr;
  }
  if (ldq < K) return "ldq must be at least K";
  if (need8 && ldq % 8 != 0) return "ldq must be a multiple of 8";
  return nullptr;
}
d3::QDst q_dst(int mode, void* q, int64_t ldq) { return d3::QDst::of(q, ldq, kblk(mode)); }
bool dtype_ok(int d) { return d == D3W8A8_BF16 || d == D3W8A8_F16 || d == D3W8A8_F32; }
int esize(int d) { return d == D3W8A8_F32 ? 4 : 2; }
bool aligned(const void* p, int a) { return ((uintptr_t)p % (uintptr_t)a) == 0; }

// Split-K scratch of d3w8a8_gemm_noalloc: device memory of the library's own code object, one copy
// per GPU, held until the process ends. In host code `scratch` names a host-side stand-in, not the
// device array: kernels and copies get the address hipGetSymbolAddress returns for the current
// device (scratch_device_ptr), never the name.
constexpr int64_t kScratchBytes = D3W8A8_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// The scratch array's address on the current device, looked up once per device (with that device
// current, as every later call on it is).
int scratch_device_ptr(void** out) {
  int dev = 0;
  const hipError_t ge = hipGetDevice(&dev);
  if (ge != hipSuccess) return fail(D3W8A8_EHIP, "gemm_noalloc: hipGetDevice: %s", hipGetErrorString(ge));
  if (dev < 0 || dev >= kMaxDevices) return fail(D3W8A8_EINVAL, "gemm_noalloc: device %d beyond %d", dev, kMaxDevices);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p)
        return fail(D3W8A8_EHIP, "gemm_noalloc: hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return D3W8A8_OK;
}

}  // namespace

extern "C" {

const char* d3w8a8_version(void) { return "d3w8a8 0.1.0 gfx950"; }

const char* d3w8a8_last_error(void) { return g_err; }

int d3w8a8_quantize_rows(int mode, int in_dtype, const void* x, int64_t ldx, int64_t M, int64_t K, void* q,
                         int64_t ldq, float* scale, void* stream) {
  if (!quant_mode_ok(mode)) return fail(D3W8A8_EINVAL, "quantize_rows: unknown mode %d", mode);
  if (!dtype_ok(in_dtype)) return fail(D3W8A8_EINVAL, "quantize_rows: unknown dtype %d", in_dtype);
  if (M < 0 || K < 1 || ldx < K) return fail(D3W8A8_EINVAL, "quantize_rows: bad shape M=%lld K=%lld ldx=%lld ldq=%lld", (long long)M, (long long)K, (long long)ldx, (long long)ldq);
  if (const char* e = q_layout_error(mode, M, K, ldq, false)) return fail(D3W8A8_EINVAL, "quantize_rows: %s", e);
  if (M == 0) return D3W8A8_OK;
  if (!x || !q || !scale) return fail(D3W8A8_EINVAL, "quantize_rows: null pointer");
  const int es = esize(in_dtype);
  const int va = es == 4 ? 32 : 16;  // bytes per 8 elements
  const bool vec = K % 8 == 0 && (ldx * es) % va == 0 && aligned(x, va) && (kblk(mode) || ldq % 8 == 0) && aligned(q, 8);
  return hip_status(d3::launch_quant_rows(base_mode(mode), in_dtype, x, ldx, M, K, q_dst(mode, q, ldq), scale, vec,
                                          (hipStream_t)stream),
                    "quantize_rows");
}

int d3w8a8_rmsnorm_quantize(int mode, int in_dtype, const void* x, int64_t ldx, int w_dtype, const void* w,
                            int64_t M, int64_t K, float eps, int zero_centered, void* q, int64_t ldq, float* scale,
                            void* normed, int64_t ldn, float* clear_amax, void* stream) {
  if (!quant_mode_ok(mode)) return fail(D3W8A8_EINVAL, "rmsnorm_quantize: unknown mode %d", mode);
  if (!dtype_ok(in_dtype) || !dtype_ok(w_dtype)) return fail(D3W8A8_EINVAL, "rmsnorm_quantize: unknown dtype");
  if (w_dtype != D3W8A8_F32 && w_dtype != in_dtype)
    return fail(D3W8A8_EINVAL, "rmsnorm_quantize: weight dtype must be fp32 or the input dtype");
  if (M < 0 || K < 8 || K % 8 != 0 || K > d3::kMaxVecK || ldx < K || (normed && ldn < K))
    return fail(D3W8A8_EINVAL, "rmsnorm_quantize: bad shape M=%lld K=%lld (K must be a multiple of 8, <= %lld)",
                (long long)M, (long long)K, (long long)d3::kMaxVecK);
  if (const char* e = q_layout_error(mode, M, K, ldq, true)) return fail(D3W8A8_EINVAL, "rmsnorm_quantize: %s", e);
  if (M == 0) return D3W8A8_OK;
  if (!x || !w || !q || !scale) return fail(D3W8A8_EINVAL, "rmsnorm_quantize: null pointer");
  const int es = esize(in_dtype), va = es == 4 ? 32 : 16, vw = w_dtype == D3W8A8_F32 ? 32 : 16;
  if ((ldx * es) % va || !aligned(x, va) || !aligned(w, vw) || !aligned(q, 8) ||
      (normed && ((ldn * es) % va || !aligned(normed, va))))
    return fail(D3W8A8_EINVAL, "rmsnorm_quantize: rows must be 16-byte aligned (32 for fp32)");
  return hip_status(d3::launch_rmsnorm_quant(base_mode(mode), in_dtype, w_dtype, x, ldx, w, M, K, eps,
                                             zero_centered ? 1 : 0, q_dst(mode, q, ldq), scale, normed, ldn,
                                             clear_amax, (hipStream_t)stream),
                    "rmsnorm_quantize");
}

int d3w8a8_quantize_rows_amax(int mode, int in_dtype, const void* h, int64_t ldh, const float* amax, int64_t M,
                              int64_t K, void* q, int64_t ldq, float* scale, void* stream) {
  if (!quant_mode_ok(mode)) return fail(D3W8A8_EINVAL, "quantize_rows_amax: unknown mode %d", mode);
  if (!dtype_ok(in_dtype)) return fail(D3W8A8_EINVAL, "quantize_rows_amax: unknown dtype %d", in_dtype);
  if (M < 0 || K < 8 || K % 8 != 0 || K > d3::kMaxVecK || ldh < K)
    return fail(D3W8A8_EINVAL, "quantize_rows_amax: bad shape M=%lld K=%lld", (long long)M, (long long)K);
  if (const char* e = q_layout_error(mode, M, K, ldq, true)) return fail(D3W8A8_EINVAL, "quantize_rows_amax: %s", e);
  if (M == 0) return D3W8A8_OK;
  if (!h || !amax || !q || !scale) return fail(D3W8A8_EINVAL, "quantize_rows_amax: null pointer");
  const int es = esize(in_dtype), va = es == 4 ? 32 : 16;
  if ((ldh * es) % va || !aligned(h, va) || !aligned(q, 8))
    return fail(D3W8A8_EINVAL, "quantize_rows_amax: rows must be 16-byte aligned");
  return hip_status(d3::launch_quant_rows_amax(base_mode(mode), in_dtype, h, ldh, amax, M, K, q_dst(mode, q, ldq),
                                               scale, (hipStream_t)stream),
                    "quantize_rows_amax");
}

int d3w8a8_gate_quantize(int mode, int in_dtype, const void* x, int64_t ldx, const void* gate, int64_t ldg,
                         int64_t gate_head_dim, int64_t M, int64_t K, void* q, int64_t ldq, float* scale,
                         void* y_out, int64_t ldy, void* stream) {
  if (!quant_mode_ok(mode)) return fail(D3W8A8_EINVAL, "gate_quantize: unknown mode %d", mode);
  if (in_dtype != D3W8A8_BF16 && in_dtype != D3W8A8_F16)
    return fail(D3W8A8_EINVAL, "gate_quantize: inputs must be bf16 or fp16");
  if (M < 0 || K < 8 || K % 8 != 0 || K > d3::kMaxVecK || ldx < K || (y_out && ldy < K))
    return fail(D3W8A8_EINVAL, "gate_quantize: bad shape M=%lld K=%lld (K must be a multiple of 8, <= %lld)",
                (long long)M, (long long)K, (long long)d3::kMaxVecK);
  if (const char* e = q_layout_error(mode, M, K, ldq, true)) return fail(D3W8A8_EINVAL, "gate_quantize: %s", e);
  if (gate_head_dim < 0 || (gate_head_dim > 0 && (gate_head_dim % 8 != 0 || K % gate_head_dim != 0)))
    return fail(D3W8A8_EINVAL, "gate_quantize: gate_head_dim must be 0 or a multiple of 8 dividing K");
  if (ldg < (gate_head_dim > 0 ? 2 * K : K))
    return fail(D3W8A8_EINVAL, "gate_quantize: ldg must cover the gate row (2 K for the q_proj layout)");
  if (M == 0) return D3W8A8_OK;
  if (!x || !gate || !q || !scale) return fail(D3W8A8_EINVAL, "gate_quantize: null pointer");
  if ((ldx * 2) % 16 || (ldg * 2) % 16 || !aligned(x, 16) || !aligned(gate, 16) || !aligned(q, 8) ||
      (y_out && ((ldy * 2) % 16 || !aligned(y_out, 16))))
    return fail(D3W8A8_EINVAL, "gate_quantize: rows must be 16-byte aligned");
  return hip_status(d3::launch_gate_quant(base_mode(mode), in_dtype, x, ldx, gate, ldg, gate_head_dim, M, K,
                                          q_dst(mode, q, ldq), scale, y_out, ldy, (hipStream_t)stream),
                    "gate_quantize");
}

int d3w8a8_gdn_norm_quantize(int mode, int in_dtype, const void* x, int64_t ldx, const void* z, int64_t ldz,
                             int w_dtype, const void* w, int64_t head_dim, float eps, int64_t M, int64_t K, void* q,
                             int64_t ldq, float* scale, void* y_out, int64_t ldy, void* stream) {
  if (!quant_mode_ok(mode)) return fail(D3W8A8_EINVAL, "gdn_norm_quantize: unknown mode %d", mode);
  if (in_dtype != D3W8A8_BF16 && in_dtype != D3W8A8_F16)
    return fail(D3W8A8_EINVAL, "gdn_norm_quantize: inputs must be bf16 or fp16");
  if (w_dtype != in_dtype && w_dtype != D3W8A8_F32)
    return fail(D3W8A8_EINVAL, "gdn_norm_quantize: weight dtype must be fp32 or the input dtype");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256 && head_dim != 512)
    return fail(D3W8A8_EINVAL, "gdn_norm_quantize: head_dim must be 64, 128, 256 or 512");
  if (M < 0 || K < head_dim || K % head_dim != 0 || K > d3::kMaxVecK || ldx < K || ldz < K || (y_out && ldy < K))
    return fail(D3W8A8_EINVAL, "gdn_norm_quantize: bad shape M=%lld K=%lld (whole heads, K <= %lld)", (long long)M,
                (long long)K, (long long)d3::kMaxVecK);
  if (const char* e = q_layout_error(mode, M, K, ldq, true)) return fail(D3W8A8_EINVAL, "gdn_norm_quantize: %s", e);
  if (M == 0) return D3W8A8_OK;
  if (!x || !z || !w || !q || !scale) return fail(D3W8A8_EINVAL, "gdn_norm_quantize: null pointer");
  if ((ldx * 2) % 16 || (ldz * 2) % 16 || !aligned(x, 16) || !aligned(z, 16) || !aligned(w, 16) ||
      !aligned(q, 8) || (y_out && ((ldy * 2) % 16 || !aligned(y_out, 16))))
    return fail(D3W8A8_EINVAL, "gdn_norm_quantize: rows must be 16-byte aligned");
  return hip_status(d3::launch_gdn_norm_quant(base_mode(mode), in_dtype, w_dtype, x, ldx, z, ldz, w, (int)head_dim, eps,
                                              M, K, q_dst(mode, q, ldq), scale, y_out, ldy, (hipStream_t)stream),
                    "gdn_norm_quantize");
}

int d3w8a8_quantize_rows_ragged(int mode, int in_dtype, const void* x, int64_t ldx, const int32_t* lengths,
                                int64_t nseg, int64_t width, int64_t K, void* q, int64_t ldq, float* scale,
                                int32_t* row_map, void* out, int out_dtype, int64_t ldo, int64_t N, void* stream) {
  if (!quant_mode_ok(mode)) return fail(D3W8A8_EINVAL, "quantize_rows_ragged: unknown mode %d", mode);
  if (!dtype_ok(in_dtype) || (out && !dtype_ok(out_dtype)))
    return fail(D3W8A8_EINVAL, "quantize_rows_ragged: unknown dtype");
  if (nseg < 0 || nseg > D3W8A8_MAX_SEGMENTS || width < 0 || K < 8 || K % 8 != 0 || K > d3::kMaxVecK || ldx < K)
    return fail(D3W8A8_EINVAL, "quantize_rows_ragged: bad shape nseg=%lld (at most %d) width=%lld K=%lld",
                (long long)nseg, D3W8A8_MAX_SEGMENTS, (long long)width, (long long)K);
  if (nseg * width > INT32_MAX) return fail(D3W8A8_EINVAL, "quantize_rows_ragged: too many rows");
  if (nseg == 0 || width == 0) return D3W8A8_OK;
  if (!x || !lengths || !q || !scale || !row_map) return fail(D3W8A8_EINVAL, "quantize_rows_ragged: null pointer");
  d3::SegOffsets segs;
  segs.off[0] = 0;
  for (int64_t b = 0; b < nseg; ++b) {
    if (lengths[b] < 0 || lengths[b] > width)
      return fail(D3W8A8_EINVAL, "quantize_rows_ragged: length %d of segment %lld outside [0, %lld]", lengths[b],
                  (long long)b, (long long)width);
    segs.off[b + 1] = segs.off[b] + lengths[b];
  }
  if (const char* e = q_layout_error(mode, segs.off[nseg], K, ldq, true))
    return fail(D3W8A8_EINVAL, "quantize_rows_ragged: %s (rows: the sum of the lengths)", e);
  const int es = esize(in_dtype), va = es == 4 ? 32 : 16;
  if ((ldx * es) % va || !aligned(x, va) || !aligned(q, 8))
    return fail(D3W8A8_EINVAL, "quantize_rows_ragged: rows must be 16-byte aligned");
  int oes = 2;
  if (out) {
    oes = esize(out_dtype);
    if (N < 1 || ldo < N || (N * oes) % 16 || (ldo * oes) % 16 || !aligned(out, 16))
      return fail(D3W8A8_EINVAL, "quantize_rows_ragged: output rows must be 16-byte multiples and aligned");
  }
  return hip_status(d3::launch_quant_ragged(base_mode(mode), in_dtype, oes, x, ldx, segs, nseg, width, K,
                                            q_dst(mode, q, ldq), scale, row_map, out, ldo, N, (hipStream_t)stream),
                    "quantize_rows_ragged");
}

static int gemm_impl(int mode, const void* a, int64_t lda, const float* a_scale, const void* w, int64_t ldw,
                     const float* w_scale, int64_t M, int64_t N, int64_t K, int epilogue, int out_dtype, void* out,
                     int64_t ldo, const void* res, int64_t ldr, float* row_amax, const int32_t* row_map, int tile,
                     int ksplit, void* workspace, int64_t workspace_bytes, void* stream) {
  if (!mode_ok(mode)) return fail(D3W8A8_EINVAL, "gemm: unknown mode %d", mode);
  if (epilogue < D3W8A8_EPI_DEQUANT || epilogue > D3W8A8_EPI_RESIDUAL)
    return fail(D3W8A8_EINVAL, "gemm: unknown epilogue %d", epilogue);
  if (epilogue != D3W8A8_EPI_RAW && !dtype_ok(out_dtype)) return fail(D3W8A8_EINVAL, "gemm: unknown out dtype");
  if (tile < D3W8A8_TILE_AUTO || tile > D3W8A8_TILE_LAST) return fail(D3W8A8_EINVAL, "gemm: unknown tile %d", tile);
  if (ksplit < D3W8A8_KSPLIT_AUTO || ksplit == 0) return fail(D3W8A8_EINVAL, "gemm: bad ksplit %d", ksplit);
  if (workspace_bytes < 0 || (workspace_bytes > 0 && (!workspace || !aligned(workspace, 256))))
    return fail(D3W8A8_EINVAL, "gemm: the workspace must be 256-byte aligned device memory");
  if (M < 0 || N < 0 || K < 0 || K % 16 != 0)
    return fail(D3W8A8_EINVAL, "gemm: bad shape M=%lld N=%lld K=%lld (K must be a multiple of 16)", (long long)M,
                (long long)N, (long long)K);
  if (M > INT32_MAX / 2 || N > INT32_MAX / 2) return fail(D3W8A8_EINVAL, "gemm: M or N too large");
  const int64_t ncols = epilogue == D3W8A8_EPI_SWIGLU ? N / 2 : N;
  const bool a_kblk = kblk(mode);
  if (a_kblk) {
    if (K % 64 != 0 || lda < M || lda >= d3::kMaxKblkRows)
      return fail(D3W8A8_EINVAL, "gemm: a K-blocked A needs K %% 64 == 0 and M <= lda < %lld (lda: its row capacity)",
                  (long long)d3::kMaxKblkRows);
  } else if (lda < K || lda % 16) {
    return fail(D3W8A8_EINVAL, "gemm: leading dimensions must cover the rows and be multiples of 16");
  }
  const bool wk = w_kblk(mode);
  if (wk) {
    if (K % 64 != 0 || ldw < N || ldw >= d3::kMaxKblkRows)
      return fail(D3W8A8_EINVAL, "gemm: a K-blocked w needs K %% 64 == 0 and N <= ldw < %lld (ldw: its row capacity)",
                  (long long)d3::kMaxKblkRows);
  } else if (ldw < K || ldw % 16) {
    return fail(D3W8A8_EINVAL, "gemm: leading dimensions must cover the rows and be multiples of 16");
  }
  if (ldo < ncols) return fail(D3W8A8_EINVAL, "gemm: ldo must cover the output row");
  const d3::GemmPlan plan =
      d3::plan_gemm(M, N, K, lda, ldw, tile, ksplit, workspace_bytes, epilogue, a_kblk, wk, base_mode(mode));
  if (plan.error) return fail(D3W8A8_EINVAL, "gemm: %s", plan.error);
  if (M == 0 || N == 0) return D3W8A8_OK;
  if (!a || !w || !out || (epilogue != D3W8A8_EPI_RAW && (!a_scale || !w_scale)))
    return fail(D3W8A8_EINVAL, "gemm: null pointer");
  if (!aligned(a, 16) || !aligned(w, 16)) return fail(D3W8A8_EINVAL, "gemm: operands must be 16-byte aligned");
  if (epilogue == D3W8A8_EPI_SWIGLU) {
    if (N % 64 != 0) return fail(D3W8A8_EINVAL, "gemm: swiglu needs N %% 64 == 0 (interleaved gate/up)");
    if (row_map) return fail(D3W8A8_EINVAL, "gemm: swiglu output stays in GEMM row order (no row_map)");
  }
  if (epilogue == D3W8A8_EPI_RESIDUAL && (!res || ldr < N)) return fail(D3W8A8_EINVAL, "gemm: residual missing");
  d3::GemmParams p{};
  p.a = (const uint8_t*)a; p.lda = lda; p.a_kblk = a_kblk ? 1 : 0; p.a_scale = a_scale;
  p.w = (const uint8_t*)w; p.ldw = ldw; p.w_kblk = wk ? 1 : 0; p.w_scale = w_scale;
  p.M = M; p.N = N; p.K = K;
  p.out = out; p.ldo = ldo; p.res = res; p.ldr = ldr;
  p.row_amax = row_amax; p.row_map = row_map;
  p.partial = (uint32_t*)workspace;
  const int oes = epilogue == D3W8A8_EPI_RAW ? 4 : esize(out_dtype);
  // full tiles store 16-byte row chunks: rows of out (and res) must be 16-byte aligned
  p.vec = (ldo * oes) % 16 == 0 && aligned(out, 16) && (epilogue == D3W8A8_EPI_RAW || aligned(w_scale, 16)) &&
          (epilogue != D3W8A8_EPI_RESIDUAL || ((ldr * oes) % 16 == 0 && aligned(res, 16)));
  return hip_status(d3::launch_gemm(base_mode(mode), p, epilogue, out_dtype, plan, (hipStream_t)stream), "gemm");
}

int d3w8a8_gemm(int mode, const void* a, int64_t lda, const float* a_scale, const void* w, int64_t ldw,
                const float* w_scale, int64_t M, int64_t N, int64_t K, int epilogue, int out_dtype, void* out,
                int64_t ldo, const void* res, int64_t ldr, float* row_amax, const int32_t* row_map, int tile,
                void* stream) {
  return gemm_impl(mode, a, lda, a_scale, w, ldw, w_scale, M, N, K, epilogue, out_dtype, out, ldo, res, ldr,
                   row_amax, row_map, tile, 1, nullptr, 0, stream);
}

int d3w8a8_gemm_ws(int mode, const void* a, int64_t lda, const float* a_scale, const void* w, int64_t ldw,
                   const float* w_scale, int64_t M, int64_t N, int64_t K, int epilogue, int out_dtype, void* out,
                   int64_t ldo, const void* res, int64_t ldr, float* row_amax, const int32_t* row_map, int tile,
                   int ksplit, void* workspace, int64_t workspace_bytes, void* stream) {
  return gemm_impl(mode, a, lda, a_scale, w, ldw, w_scale, M, N, K, epilogue, out_dtype, out, ldo, res, ldr,
                   row_amax, row_map, tile, ksplit, workspace, workspace_bytes, stream);
}

int d3w8a8_gemm_noalloc(int mode, const void* a, int64_t lda, const float* a_scale, const void* w, int64_t ldw,
                        const float* w_scale, int64_t M, int64_t N, int64_t K, int epilogue, int out_dtype, void* out,
                        int64_t ldo, const void* res, int64_t ldr, float* row_amax, const int32_t* row_map, int tile,
                        int ksplit, void* stream) {
  if (ksplit > 1 && M > 0 && N > 0 && K > 0 && K % 16 == 0 && (kblk(mode) ? lda >= M : lda >= K) &&
      (w_kblk(mode) ? ldw >= N : ldw >= K) && M <= INT32_MAX / 2 && N <= INT32_MAX / 2 &&
      tile >= D3W8A8_TILE_AUTO && tile <= D3W8A8_TILE_LAST) {
    // an explicit split larger than the scratch: name both sizes rather than the generic plan error
    const d3::GemmPlan want =
        d3::plan_gemm(M, N, K, lda, ldw, tile, ksplit, INT64_MAX, epilogue, kblk(mode), w_kblk(mode), base_mode(mode));
    if (!want.error && want.ws_bytes > kScratchBytes)
      return fail(D3W8A8_EINVAL, "gemm_noalloc: ksplit %d needs %lld bytes of split-K scratch; the library holds %lld",
                  ksplit, (long long)want.ws_bytes, (long long)kScratchBytes);
  }
  void* ws = nullptr;
  if (const int rc = scratch_device_ptr(&ws)) return rc;
  return gemm_impl(mode, a, lda, a_scale, w, ldw, w_scale, M, N, K, epilogue, out_dtype, out, ldo, res, ldr,
                   row_amax, row_map, tile, ksplit, ws, kScratchBytes, stream);
}

int64_t d3w8a8_gemm_workspace(int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldw, int tile, int ksplit,
                              int64_t max_bytes) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 16 || lda < K || ldw < K || M > INT32_MAX / 2 || N > INT32_MAX / 2 ||
      tile < D3W8A8_TILE_AUTO || tile > D3W8A8_TILE_LAST || ksplit < D3W8A8_KSPLIT_AUTO || ksplit == 0) {
    fail(D3W8A8_EINVAL, "gemm_workspace: bad arguments");
    return -1;
  }
  // the epilogue only rules tiles out; none of those it could rule out splits K, so the bytes do not depend on it
  const d3::GemmPlan plan =
      d3::plan_gemm(M, N, K, lda, ldw, tile, ksplit, max_bytes < 0 ? 0 : max_bytes, D3W8A8_EPI_DEQUANT);
  if (plan.error) {
    fail(D3W8A8_EINVAL, "gemm_workspace: %s", plan.error);
    return -1;
  }
  return plan.ws_bytes;
}

}  // extern "C"
