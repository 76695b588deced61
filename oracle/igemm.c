/* int64 brute-force GEMM over int8 operands (TEST ORACLE).
 *
 * C[m][n] = sum_k A[m][k] * W[n][k]  -- the product QuantLinear._int8 asks of
 * torch._int_mm(q, weight.t()) (reference d3trt/model/quant.py:196), with both
 * operands K-contiguous. Partial sums are kept in int32 over chunks of 4096
 * (|partial| <= 127*127*4096 < 2**31) and added into int64, so the result is
 * exact for any K.
 */
#include <stdint.h>

int oracle_igemm_i8(const int8_t* A, const int8_t* W, int64_t* C,
                    int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldw) {
  if (M < 0 || N < 0 || K < 0 || lda < K || ldw < K) return 1;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t m = 0; m < M; ++m) {
    const int8_t* a = A + m * lda;
    for (int64_t n = 0; n < N; ++n) {
      const int8_t* w = W + n * ldw;
      int64_t total = 0;
      for (int64_t k0 = 0; k0 < K; k0 += 4096) {
        int64_t k1 = k0 + 4096 < K ? k0 + 4096 : K;
        int32_t part = 0;
        for (int64_t k = k0; k < k1; ++k) part += (int32_t)a[k] * (int32_t)w[k];
        total += part;
      }
      C[m * N + n] = total;
    }
  }
  return 0;
}
