// INT8 W8A8 decode GEMV (1..2 rows of A): C[m, n] = sum_k A[m, k] B[n, k] in exact int32, then EpiInt8's fp32
// epilogue.  The W8A16 decode GEMV's structure: a wavefront owns R = 8 channels (rows of B) and one K slice of at most
// S 16-byte chunks per lane (chunk c = slice start + lane + 64 i); lane l reads 16 bytes of each of its 8 rows of B and
// of each row of A per chunk and multiplies them with v_dot4_i32_i8 (four int8 products per instruction into an int32
// accumulator, exact); the int32 partials are summed over the 64 lanes and then over the KS slices of the workgroup,
// in a fixed order (integer sums are exact in any order anyway).  A workgroup is the KS wavefronts of one channel
// block.  All loads are raw buffer loads issued unconditionally; a chunk past the slice reads past A's span (0, no
// traffic) and adds 0.
#include "fg_mm.h"

namespace fg {

struct I8GemvArgs {
  int KC, cps;
  uint32_t abytes, bbytes;
};

template <int MT, int S>
__global__ void __launch_bounds__(1024) int8_gemv_kernel(const int8_t* __restrict__ a, int64_t lda,
                                                         const int8_t* __restrict__ b, int64_t ldb, int M, int N,
                                                         I8GemvArgs g, EpiInt8 epi) {
  constexpr int R = 8;
  static_assert(R * MT == 8 || R * MT == 16, "rows x batch must be 8 or 16");
  __shared__ int red[16][R * MT];
  const int lane = threadIdx.x & (kWave - 1);
  const int wb = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int ks = __builtin_amdgcn_readfirstlane(threadIdx.y);
  const int BW = (int)(blockDim.x / kWave), KS = (int)blockDim.y;
  const int n0 = (blockIdx.x * BW + wb) * R;
  const int nr = min(n0, N - R);
  const int c0 = ks * g.cps, c1 = min(c0 + g.cps, g.KC);
  const __amdgpu_buffer_rsrc_t ra = buf_rsrc(a, g.abytes), rb = buf_rsrc(b, g.bbytes);

  uint32_t ao[S], bo[S];
#pragma unroll
  for (int i = 0; i < S; ++i) {
    const int c = c0 + lane + kWave * i;
    const bool ok = c < c1;
    ao[i] = ok ? (uint32_t)c * 16u : g.abytes;
    bo[i] = ok ? (uint32_t)c * 16u : g.bbytes;
  }
  uint4 av[MT][S];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int i = 0; i < S; ++i) av[m][i] = buf_ld16(ra, ao[i], (uint32_t)min(m, M - 1) * (uint32_t)lda);
  uint4 bv[R][S];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int i = 0; i < S; ++i) bv[r][i] = buf_ld16_nt(rb, bo[i], ((uint32_t)nr + (uint32_t)r) * (uint32_t)ldb);

  int acc[R * MT];
#pragma unroll
  for (int v = 0; v < R * MT; ++v) acc[v] = 0;
#pragma unroll
  for (int i = 0; i < S; ++i)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t bw[4] = {bv[r][i].x, bv[r][i].y, bv[r][i].z, bv[r][i].w};
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const uint32_t aw[4] = {av[m][i].x, av[m][i].y, av[m][i].z, av[m][i].w};
#pragma unroll
        for (int q = 0; q < 4; ++q)
          acc[r * MT + m] = __builtin_amdgcn_sdot4((int)aw[q], (int)bw[q], acc[r * MT + m], false);
      }
    }
  const int tot = wave_transpose_sum_i32<R * MT>(acc, lane);
  constexpr int span = kWave / (R * MT);
  auto store = [&](int idx, int v) {
    const int r = idx / MT, m = idx - (idx / MT) * MT;
    if (m < M && n0 + r < N) epi.store(m, n0 + r, v);
  };
  if (KS == 1) {
    if ((lane % span) == 0) store(lane / span, tot);
  } else {
    if ((lane % span) == 0) red[ks * BW + wb][lane / span] = tot;
    __syncthreads();
    if (ks == 0 && lane < R * MT) {
      int v = 0;
      for (int k2 = 0; k2 < KS; ++k2) v += red[k2 * BW + wb][lane];
      store(lane, v);
    }
  }
}

// S chunks per lane: 1 while K <= 4096, 2 to K = 8192, else 4; KS = ceil(chunks / (64 S)) slices (at most 16); one
// channel block per workgroup.
static bool int8_gemv_plan(int M, int N, int K, int* mt, int* S, int* KS) {
  const int KC = K / 16;
  *mt = M <= 1 ? 1 : 2;
  *S = KC <= 4 * kWave ? 1 : (KC <= 8 * kWave ? 2 : 4);
  *KS = (KC + kWave * *S - 1) / (kWave * *S);
  return M >= 1 && M <= 2 && *KS <= 16 && N % 8 == 0;
}

bool int8_gemv_ok(const void* a, int64_t lda, const void* b, int64_t ldb, int64_t M, int64_t N, int64_t K) {
  const int64_t k4g = 1LL << 32;
  int mt, S, KS;
  return K % 16 == 0 && lda % 16 == 0 && ldb % 16 == 0 && reinterpret_cast<uintptr_t>(a) % 16 == 0 &&
         reinterpret_cast<uintptr_t>(b) % 16 == 0 && N * ldb < k4g && M * lda < k4g && K < k4g / 64 &&
         int8_gemv_plan((int)M, (int)N, (int)K, &mt, &S, &KS);
}

hipError_t launch_int8_gemv(const int8_t* a, int64_t lda, const float* sa, int64_t sa_len, const int8_t* b,
                            int64_t ldb, const float* sb, int64_t sb_len, const void* bias, int bdt, void* y,
                            int64_t ldy, int ydt, int M, int N, int K, hipStream_t s) {
  int mt, S, KS;
  if (!int8_gemv_plan(M, N, K, &mt, &S, &KS)) return hipErrorInvalidValue;
  I8GemvArgs g;
  g.KC = K / 16;
  g.cps = (g.KC + KS - 1) / KS;
  g.abytes = (uint32_t)((int64_t)M * lda);
  g.bbytes = (uint32_t)((int64_t)N * ldb);
  const EpiInt8 epi{sa, sa_len, sb, sb_len, bias, bdt, y, ldy, ydt};
  const dim3 grid(N / 8), block(kWave, KS);
#define FG_I8G(MT_, S_)                                                                              \
  do {                                                                                               \
    note_kernel("int8_gemv_kernel<%d,%d>", MT_, S_);                                                 \
    hipLaunchKernelGGL((int8_gemv_kernel<MT_, S_>), grid, block, 0, s, a, lda, b, ldb, M, N, g, epi); \
  } while (0)
  if (mt == 1) {
    if (S == 1) FG_I8G(1, 1); else if (S == 2) FG_I8G(1, 2); else FG_I8G(1, 4);
  } else {
    if (S == 1) FG_I8G(2, 1); else if (S == 2) FG_I8G(2, 2); else FG_I8G(2, 4);
  }
#undef FG_I8G
  return hipGetLastError();
}

}  // namespace fg
