/* CPU oracle in plain C -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 *
 * A second, independent restatement of two reference oracles, used by tests/ (through ctypes) to cross-check the
 * numpy oracle at sizes where numpy's integer matmul is too slow, and by nothing in the product:
 *
 *   fgo_w4_dequant_f32   forge/kernels/layouts/w4.py:294-305   W[n,k] = (q - z) * s, one fp32 rounding
 *   fgo_w4a16_gemm_f32   forge/kernels/ref/gemm_w4a16.py:9-27   y = x @ W^T (+ bias), fp32 sequential accumulation
 *   fgo_int8_gemm_i32    forge/kernels/ref/gemm_int8.py:62-65    exact int32 accumulator (int64 running sum)
 *
 * Packed layout: forge/kernels/layouts/w4.py:15-17 (portable_row): qweight int32 [N, ldq], nibble j of word w holds
 * q[n, 8w + j]; scales [G, lds] (here pre-widened to float); zeros int32 [G, ldz], nibble j of word v holds the
 * zero of channel 8v + j (NULL = symmetric, zero-point 8).
 */
#include <stdint.h>
#include <stddef.h>

static inline int nib(uint32_t w, int j) { return (int)((w >> (4 * j)) & 0xFu); }

static inline float w_at(const int32_t* qw, int64_t ldq, const float* sc, int64_t lds, const int32_t* zr, int64_t ldz,
                         const int32_t* g_idx, int gs, int64_t n, int64_t k) {
  int64_t g = g_idx ? (int64_t)g_idx[k] : k / gs;
  int q = nib((uint32_t)qw[n * ldq + k / 8], (int)(k % 8));
  int z = zr ? nib((uint32_t)zr[g * ldz + n / 8], (int)(n % 8)) : 8;
  float d = (float)q - (float)z; /* exact */
  return d * sc[g * lds + n];    /* one rounding, as torch's fp32 multiply */
}

void fgo_w4_dequant_f32(const int32_t* qw, int64_t ldq, const float* sc, int64_t lds, const int32_t* zr, int64_t ldz,
                        const int32_t* g_idx, int gs, int64_t N, int64_t K, float* out) {
  for (int64_t n = 0; n < N; ++n)
    for (int64_t k = 0; k < K; ++k) out[n * K + k] = w_at(qw, ldq, sc, lds, zr, ldz, g_idx, gs, n, k);
}

void fgo_w4a16_gemm_f32(const float* x, int64_t M, int64_t K, const int32_t* qw, int64_t ldq, const float* sc,
                        int64_t lds, const int32_t* zr, int64_t ldz, const int32_t* g_idx, int gs, int64_t N,
                        const float* bias, float* y) {
  for (int64_t n = 0; n < N; ++n) {
    for (int64_t m = 0; m < M; ++m) {
      float acc = 0.0f;
      for (int64_t k = 0; k < K; ++k) {
        float prod = x[m * K + k] * w_at(qw, ldq, sc, lds, zr, ldz, g_idx, gs, n, k);
        acc = acc + prod;
      }
      if (bias) acc = acc + bias[n];
      y[m * N + n] = acc;
    }
  }
}

void fgo_int8_gemm_i32(const int8_t* a, int64_t M, int64_t K, const int8_t* b, int64_t N, int32_t* c) {
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      int64_t acc = 0;
      const int8_t* ar = a + m * K;
      const int8_t* br = b + n * K;
      for (int64_t k = 0; k < K; ++k) acc += (int64_t)ar[k] * (int64_t)br[k];
      c[m * N + n] = (int32_t)acc;
    }
}
