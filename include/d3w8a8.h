/* d3w8a8 -- gfx950 (MI355X) W8A8 quantized Linear kernels behind a plain C ABI.
 *
 * The reference's boundary for this path is a Python module API, not an FFI:
 * d3trt/model/quant.py (quantize_rows :92-100, quantize_weight :77-89,
 * QuantLinear._int8 :190-197, QuantLinear._fp8 :164-188) and the MLP chain
 * around it (trtllm_stack.py:131-134, core.py:214-215). Each entry point below
 * replaces one of those torch call sequences; the Python mirror of the module
 * (d3trt_amd.quant) binds them with ctypes.
 *
 * Conventions
 *   - All pointers are device pointers owned by the caller; the library never
 *     allocates. Matrices are row-major with explicit leading dimensions in
 *     elements. Work is enqueued on `stream` (a hipStream_t; NULL = default
 *     stream) and nothing synchronizes.
 *   - Return 0 on success; D3W8A8_EINVAL for a bad mode/dtype/shape/stride/
 *     alignment (the Python layer raises ValueError), D3W8A8_EHIP for a HIP
 *     launch failure (RuntimeError). d3w8a8_last_error() returns the message of
 *     the calling thread's last failure.
 *   - Stateless and reentrant: concurrent calls on different streams are safe.
 */
#ifndef D3W8A8_H
#define D3W8A8_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define D3W8A8_OK 0
#define D3W8A8_EINVAL 1
#define D3W8A8_EHIP 2

/* modes (quant.py:28 "fp8" / "int8") */
#define D3W8A8_INT8 0
#define D3W8A8_FP8 1

/* Layout flag, OR-ed into `mode`: K-blocked quantized activations. Given to a
 * quantize entry point it sets the layout of q; given to a GEMM entry point,
 * the layout of a. Byte (m, k) sits at ((k / 64) * ld + m) * 64 + k % 64: each
 * 64-byte slice of K holds all rows back to back, ld (ldq / lda) is the row
 * capacity (>= M) and K % 64 == 0. No counterpart in the reference, whose
 * activations are row-major tensors: it exists for the pipelined GEMM tiles,
 * which read 64 bytes of K per row per step, half a 128-byte line of each
 * row when rows are row-major and whole lines when K-blocked. GEMM results
 * are identical for both layouts. The register-staged tiles (0-2) take
 * row-major a only; a K-blocked a needs lda < 2^25. */
#define D3W8A8_KBLOCK 0x100
/* The same layout for the weights of a GEMM entry point (w, ldw = its row
 * capacity >= N; K % 64 == 0; ldw < 2^25): OR-ed into `mode` of d3w8a8_gemm,
 * _gemm_ws and _gemm_noalloc. d3w8a8_quantize_rows with D3W8A8_KBLOCK writes
 * quantized weights [N, K] in it. */
#define D3W8A8_W_KBLOCK 0x200

/* element types of floating-point tensors */
#define D3W8A8_BF16 0
#define D3W8A8_F16 1
#define D3W8A8_F32 2

/* GEMM epilogues */
#define D3W8A8_EPI_DEQUANT 0  /* out = OUT((float(acc) * a_scale[m]) * w_scale[n])      quant.py:162,197 */
#define D3W8A8_EPI_RAW 1      /* out = acc: int32 (INT8) or fp32 (FP8)                 parity hook      */
#define D3W8A8_EPI_SWIGLU 2   /* h = OUT(OUT(silu(g)) * u), g/u dequantized; row amax  trtllm_stack.py:131-134 */
#define D3W8A8_EPI_RESIDUAL 3 /* out = OUT(res + OUT(dequant))                         core.py:215      */

/* GEMM tile configurations (D3W8A8_TILE_AUTO picks one from M, N and K).
 * REG tiles stage K through registers and accept any K % 16 == 0; DMA tiles
 * use the direct global->LDS pipeline and need K % 64 == 0 and each operand
 * within 4 GiB of its first row ((rows - 1) * ld + K < 2^32). */
#define D3W8A8_TILE_AUTO (-1)
#define D3W8A8_TILE_256 0           /* REG 256x256, 4 waves */
#define D3W8A8_TILE_128 1           /* REG 128x128, 4 waves */
#define D3W8A8_TILE_64x128 2        /* REG 64x128, 4 waves */
#define D3W8A8_TILE_DMA_256_W8 3    /* DMA 256x256, 8 waves */
#define D3W8A8_TILE_DMA_256_W4 4    /* DMA 256x256, 4 waves */
#define D3W8A8_TILE_DMA_128_W4 5    /* DMA 128x128, 4 waves */
#define D3W8A8_TILE_DMA_256x128_W4 6 /* DMA 256x128, 4 waves */
#define D3W8A8_TILE_DMA_128_W4_K128 7 /* DMA 128x128, 4 waves, 128-byte K steps (K % 128 == 0): weight streaming */
#define D3W8A8_TILE_DMA_256x192_W4 8 /* DMA 256x192, 4 waves: whole tile rounds where 256x256 leaves one ragged
                                      * (fused QKV, N = 6144); not with D3W8A8_EPI_SWIGLU */
#define D3W8A8_TILE_WS 9             /* weight streaming for skinny M (question batches): 32-column slabs
                                      * (64 with SwiGLU), one wave streams the weights, one per 32 rows
                                      * computes; no split-K workspace; K % 128 == 0; results equal
                                      * tile 7 unsplit bit for bit (so FP8 rows do not depend on M) */
#define D3W8A8_TILE_DMA_192x192_W4 10 /* DMA 192x192, 4 waves: whole rounds for ragged batches whose
                                       * 256-row tiles leave part of one idle (1440 rows, N = 6144);
                                       * not with D3W8A8_EPI_SWIGLU */
#define D3W8A8_TILE_DMA_192x128_W4 11 /* DMA 192x128, 4 waves (1440 rows, N = 4096) */
#define D3W8A8_TILE_LAST D3W8A8_TILE_DMA_192x128_W4

const char* d3w8a8_version(void);
const char* d3w8a8_last_error(void);

/* Per-token dynamic quantization.
 * Replaces quant.py:92-100 quantize_rows(x, mode) and, applied to a weight
 * [N, K], quant.py:77-89 quantize_weight (same per-row arithmetic).
 *   x [M, K] (in_dtype, ld ldx) -> q [M, K] int8 / e4m3fn (ld ldq), scale [M] fp32
 *   scale = max(max|x_m|, 1e-12) / (127 | 448); q = clamp(rne(x / scale))
 * Every quantize entry point writes q row-major (ldq >= K) or, with
 * D3W8A8_KBLOCK in mode, K-blocked (ldq >= rows of q). */
int d3w8a8_quantize_rows(int mode, int in_dtype, const void* x, int64_t ldx, int64_t M, int64_t K,
                         void* q, int64_t ldq, float* scale, void* stream);

/* Fused zero-centred RMSNorm + per-token quantization.
 * Replaces the input/post-attention RMSNorm (trtllm_stack.py:217-228,
 * Qwen3_5RMSNorm semantics) followed by quant.py:92-100 on its output.
 *   y = in_dtype((x * rsqrt(mean(x^2) + eps)) * (zero_centered ? 1 + w : w)); q, scale = quant(y)
 * normed (optional, ld ldn) receives y; clear_amax (optional) gets clear_amax[m] = 0
 * for every row, preparing the SwiGLU epilogue's row-amax buffer. */
int d3w8a8_rmsnorm_quantize(int mode, int in_dtype, const void* x, int64_t ldx, int w_dtype, const void* w,
                            int64_t M, int64_t K, float eps, int zero_centered, void* q, int64_t ldq,
                            float* scale, void* normed, int64_t ldn, float* clear_amax, void* stream);

/* Quantization with the row amax already known (SwiGLU output h, amax from
 * the SwiGLU epilogue): the quant.py:95-100 arithmetic after the amax. */
int d3w8a8_quantize_rows_amax(int mode, int in_dtype, const void* h, int64_t ldh, const float* amax,
                              int64_t M, int64_t K, void* q, int64_t ldq, float* scale, void* stream);

/* o_proj input of a gated attention layer, quantized per token: y = OUT(x * OUT(sigmoid(gate))), then
 * quantize_rows(y). Replaces `attn.o_proj(out * torch.sigmoid(gate))`'s elementwise product and
 * quantize (d3trt/model/core.py:297 with quant.py:92-100). x [M, K] (ld ldx), bf16 or fp16.
 * gate_head_dim == 0: gate is [M, K] (ld ldg >= K). gate_head_dim > 0 (a multiple of 8 dividing K):
 * gate is read in place from the q_proj output [M, 2K] (ld ldg >= 2K), whose rows hold per head
 * [query (head_dim) | gate (head_dim)] (core.py:231). y_out (optional, ld ldy): the product. */
int d3w8a8_gate_quantize(int mode, int in_dtype, const void* x, int64_t ldx, const void* gate, int64_t ldg,
                         int64_t gate_head_dim, int64_t M, int64_t K, void* q, int64_t ldq, float* scale,
                         void* y_out, int64_t ldy, void* stream);

/* GDN output projection's input, quantized per token: Qwen3_5RMSNormGated over heads of head_dim
 * (`delta.norm(core, z)`, d3trt/model/core.py:390-391; transformers modeling_qwen3_5.py:168-184, built
 * in the model dtype, trtllm_stack.py:198), then quantize_rows over the whole row (quant.py:92-100):
 *   h = x * rsqrt(mean_head(x^2) + eps) (fp32); h = w * IN(h) (rounded to IN when w is IN);
 *   y = IN(h * silu(z)); q(y).
 * x, z [M, K] (K = heads * head_dim), bf16 or fp16; w [head_dim] of the input dtype or fp32, shared by
 * the heads; head_dim 64, 128, 256 or 512. y_out (optional, ld ldy): the normed, gated rows. */
int d3w8a8_gdn_norm_quantize(int mode, int in_dtype, const void* x, int64_t ldx, const void* z, int64_t ldz,
                             int w_dtype, const void* w, int64_t head_dim, float eps, int64_t M, int64_t K, void* q,
                             int64_t ldq, float* scale, void* y_out, int64_t ldy, void* stream);

/* Ragged gather-quantize for a right-padded question batch x [nseg, width, K]
 * (backends/trtllm.py:149-179 builds such batches; core.py:158-181 runs them):
 * valid row (b, t < lengths[b]) is quantized into packed row off(b) + t with
 * row_map[off(b) + t] = b * width + t, off(b) = lengths[0] + ... + lengths[b-1];
 * padded rows of `out` (optional, [nseg * width, N] of out_dtype, ld ldo) are
 * zeroed. `lengths` is a HOST array of nseg <= D3W8A8_MAX_SEGMENTS entries,
 * read during the call and passed to the kernel by value: no host-to-device
 * copy precedes the launch. */
#define D3W8A8_MAX_SEGMENTS 256
int d3w8a8_quantize_rows_ragged(int mode, int in_dtype, const void* x, int64_t ldx, const int32_t* lengths,
                                int64_t nseg, int64_t width, int64_t K, void* q, int64_t ldq, float* scale,
                                int32_t* row_map, void* out, int out_dtype, int64_t ldo, int64_t N,
                                void* stream);

/* W8A8 GEMM with a fused epilogue. Replaces quant.py:196-197 (torch._int_mm +
 * dequant) and quant.py:171-177 (torch._scaled_mm rowwise).
 *   a [M, K] quantized activations (ld lda), a_scale [M]; w [N, K] quantized
 *   weights (ld ldw), w_scale [N]; out per `epilogue` (ld ldo; N/2 columns for
 *   SWIGLU); res (RESIDUAL only, ld ldr, out_dtype); row_amax [M] (SWIGLU,
 *   atomically max-ed, must start at 0 or a lower bound); row_map [M]
 *   (optional; output row of GEMM row m, from d3w8a8_quantize_rows_ragged).
 * Requirements: K % 16 == 0; lda, ldw % 16 == 0; a, w 16-byte aligned;
 * SWIGLU needs N % 64 == 0 with weights interleaved in blocks of 32 rows. */
int d3w8a8_gemm(int mode, const void* a, int64_t lda, const float* a_scale, const void* w, int64_t ldw,
                const float* w_scale, int64_t M, int64_t N, int64_t K, int epilogue, int out_dtype, void* out,
                int64_t ldo, const void* res, int64_t ldr, float* row_amax, const int32_t* row_map, int tile,
                void* stream);

/* d3w8a8_gemm with a caller-owned workspace that lets skinny problems split K.
 * Same operation, arguments and results as d3w8a8_gemm (the reference's
 * question passes, backends/trtllm.py:149-179, run every projection at a small
 * M; with too few output tiles to occupy the GPU, `ksplit` workgroups share
 * each tile over disjoint K ranges). The partial sums are added in a fixed
 * order (a second launch reads them), so results do not depend on
 * scheduling: INT8 equals d3w8a8_gemm bit for bit; FP8 differs from it only
 * by fp32 summation order.
 *   ksplit: D3W8A8_KSPLIT_AUTO (chosen from the shape and the workspace size),
 *           or 1..32 (>1 needs a 128x128 DMA tile, 5 or 7, and at least
 *           one K step per split).
 *   workspace: device memory, 256-byte aligned, `workspace_bytes` long, of
 *           any contents (it holds partial sums between the two launches).
 *           Calls that share a workspace must be ordered (same stream);
 *           NULL / 0 means no split. */
#define D3W8A8_KSPLIT_AUTO (-1)
int d3w8a8_gemm_ws(int mode, const void* a, int64_t lda, const float* a_scale, const void* w, int64_t ldw,
                   const float* w_scale, int64_t M, int64_t N, int64_t K, int epilogue, int out_dtype, void* out,
                   int64_t ldo, const void* res, int64_t ldr, float* row_amax, const int32_t* row_map, int tile,
                   int ksplit, void* workspace, int64_t workspace_bytes, void* stream);

/* d3w8a8_gemm_ws without a workspace argument: the split-K partial sums go to
 * the library's own scratch, a static device array of
 * D3W8A8_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends).
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc); the call itself allocates nothing. Same operation,
 * arguments and results as d3w8a8_gemm_ws given a workspace of that size
 * (ksplit AUTO picks a split that fits it; an explicit ksplit that needs more
 * returns D3W8A8_EINVAL). Every call on one GPU uses that GPU's one scratch
 * array, so calls on one GPU must be ordered (one stream): calls that overlap
 * race on it. The stream's device must be current. Nothing needs clearing
 * between calls: each split overwrites its whole slot before the reduce
 * reads it. */
#define D3W8A8_NOALLOC_SCRATCH_BYTES (16 << 20)
int d3w8a8_gemm_noalloc(int mode, const void* a, int64_t lda, const float* a_scale, const void* w, int64_t ldw,
                        const float* w_scale, int64_t M, int64_t N, int64_t K, int epilogue, int out_dtype, void* out,
                        int64_t ldo, const void* res, int64_t ldr, float* row_amax, const int32_t* row_map, int tile,
                        int ksplit, void* stream);

/* Workspace bytes d3w8a8_gemm_ws uses for this problem, tile and ksplit when
 * given at most `max_bytes` (0 when it would not split); -1 on bad arguments.
 * For a K-blocked a or w, pass lda = K or ldw = K. */
int64_t d3w8a8_gemm_workspace(int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldw, int tile, int ksplit,
                              int64_t max_bytes);

#ifdef __cplusplus
}
#endif

#endif /* D3W8A8_H */
