// W8A8 GEMMs on gfx950 matrix cores: INT8 (v_mfma_i32_16x16x64_i8, exact int32) and FP8 OCP e4m3fn
// (v_mfma_f32_16x16x128_f8f6f4, fp32 accumulation).
//
// C[M,N] = A[M,K] @ B[N,K]^T with both operands K-contiguous (Forge stores activations [M,K] and weights [N,K]), so
// every lane's MFMA fragment is one contiguous 16/32-byte run along K in LDS.
//
// Workgroup: 256 threads = 2x2 wavefronts; wave tile (16*TM) x (16*TN) made of 16x16 MFMA tiles; workgroup tile
// BM x BN = 32*TM x 32*TN; K is walked in 128-byte slices staged through a double-buffered LDS ring (global ->
// registers -> LDS, one barrier per slice).  LDS rows are padded by 16 bytes so the 16 lanes that read one fragment
// column hit 16 distinct bank quads.  Tiles are ordered so that each XCD (workgroups are dealt round-robin over the
// 8 XCDs) works on a compact block of output tiles that shares A and B slices in its own L2.
//
// Used for outputs that do not fill the 256 x 256 kernel of fg_mm_big.hip (small M or N, K not a multiple of 128,
// unaligned operands) and for the K-blocked FP8 scale mode.
#include "fg_mm.h"

namespace fg {

template <class Mma, int TM, int TN, bool ALIGNED, class Epi>
__global__ void __launch_bounds__(256) mm_kernel(const uint8_t* __restrict__ A, int64_t lda,
                                                 const uint8_t* __restrict__ B, int64_t ldb, int M, int N, int K,
                                                 Epi epi) {
  constexpr int BM = 32 * TM, BN = 32 * TN, BK = 128, LDSP = BK + 16;
  constexpr int A_ROUNDS = BM * BK / (256 * 16), B_ROUNDS = BN * BK / (256 * 16);
  constexpr int STAGE = (BM + BN) * LDSP;
  extern __shared__ __align__(16) uint8_t smem[];

  const int ntm = (M + BM - 1) / BM, ntn = (N + BN - 1) / BN;
  int tm_, tn_;
  tile_of(blockIdx.x, ntm, ntn, tm_, tn_);
  const int m0 = tm_ * BM, n0 = tn_ * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lrow = tid >> 3, lcol = (tid & 7) * 16;  // global->LDS copy: 32 rows x 8 chunks per round

  auto fetch = [&](const uint8_t* base, int64_t ld, int rows_total, int row0, int k0, uint4* regs, int rounds) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (r >= rounds) break;
      const int row = row0 + lrow + 32 * r;
      const int k = k0 + lcol;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (row < rows_total) {
        const uint8_t* p = base + (int64_t)row * ld + k;
        if (ALIGNED) {
          if (k < K) v = *reinterpret_cast<const uint4*>(p);
        } else {
          uint8_t b[16];
#pragma unroll
          for (int j = 0; j < 16; ++j) b[j] = (k + j < K) ? p[j] : 0;
          __builtin_memcpy(&v, b, 16);
        }
      }
      regs[r] = v;
    }
  };
  auto stash = [&](uint8_t* tile, const uint4* regs, int rounds) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (r >= rounds) break;
      *reinterpret_cast<uint4*>(tile + (lrow + 32 * r) * LDSP + lcol) = regs[r];
    }
  };

  typename Mma::acc_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[i][j][e] = 0;

  uint4 ra[4], rb[4];
  const int nk = (K + BK - 1) / BK;
  fetch(A, lda, M, m0, 0, ra, A_ROUNDS);
  fetch(B, ldb, N, n0, 0, rb, B_ROUNDS);
  stash(smem, ra, A_ROUNDS);
  stash(smem + BM * LDSP, rb, B_ROUNDS);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    uint8_t* cur = smem + (kt & 1) * STAGE;
    uint8_t* nxt = smem + ((kt + 1) & 1) * STAGE;
    const bool more = kt + 1 < nk;
    if (more) {
      fetch(A, lda, M, m0, (kt + 1) * BK, ra, A_ROUNDS);
      fetch(B, ldb, N, n0, (kt + 1) * BK, rb, B_ROUNDS);
    }
    const uint8_t* sA = cur + (wm * 16 * TM + (lane & 15)) * LDSP + (lane >> 4) * Mma::LB;
    const uint8_t* sB = cur + BM * LDSP + (wn * 16 * TN + (lane & 15)) * LDSP + (lane >> 4) * Mma::LB;
    if constexpr (Epi::kBlocked) {
      typename Mma::acc_t part[TM][TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) part[i][j][e] = 0;
#pragma unroll
      for (int s = 0; s < BK / Mma::KB; ++s) {
        typename Mma::frag_t fa[TM], fb[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) fa[i] = Mma::load(sA + i * 16 * LDSP + s * Mma::KB);
#pragma unroll
        for (int j = 0; j < TN; ++j) fb[j] = Mma::load(sB + j * 16 * LDSP + s * Mma::KB);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) part[i][j] = Mma::mma(fa[i], fb[j], part[i][j]);
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int m = m0 + wm * 16 * TM + i * 16 + 4 * (lane >> 4) + e;
            const int n = n0 + wn * 16 * TN + j * 16 + (lane & 15);
            acc[i][j][e] = __builtin_fmaf(part[i][j][e], epi.kscale(m, n, kt), acc[i][j][e]);
          }
    } else {
#pragma unroll
      for (int s = 0; s < BK / Mma::KB; ++s) {
        typename Mma::frag_t fa[TM], fb[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) fa[i] = Mma::load(sA + i * 16 * LDSP + s * Mma::KB);
#pragma unroll
        for (int j = 0; j < TN; ++j) fb[j] = Mma::load(sB + j * 16 * LDSP + s * Mma::KB);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = Mma::mma(fa[i], fb[j], acc[i][j]);
      }
    }
    if (more) {
      stash(nxt, ra, A_ROUNDS);
      stash(nxt + BM * LDSP, rb, B_ROUNDS);
    }
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + wm * 16 * TM + i * 16 + 4 * (lane >> 4) + e;
        const int n = n0 + wn * 16 * TN + j * 16 + (lane & 15);
        if (m < M && n < N) epi.store(m, n, acc[i][j][e]);
      }
}

template <class Mma, int TM, int TN, class Epi>
static hipError_t launch_mm(const uint8_t* A, int64_t lda, const uint8_t* B, int64_t ldb, int M, int N, int K,
                            const Epi& epi, hipStream_t s) {
  constexpr int BM = 32 * TM, BN = 32 * TN, LDSP = 128 + 16;
  const size_t shm = 2 * (size_t)(BM + BN) * LDSP;
  const bool aligned = (lda % 16 == 0) && (ldb % 16 == 0) && (K % 16 == 0) &&
                       ((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B)) % 16 == 0);
  const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  auto k = aligned ? mm_kernel<Mma, TM, TN, true, Epi> : mm_kernel<Mma, TM, TN, false, Epi>;
  if (shm > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
    if (e != hipSuccess) return e;
  }
  note_kernel("mm_kernel %dx%d", BM, BN);
  hipLaunchKernelGGL(k, dim3(tiles), dim3(256), shm, s, A, lda, B, ldb, M, N, K, epi);
  return hipGetLastError();
}

hipError_t launch_int8_gemm(const int8_t* a, int64_t lda, const float* sa, int64_t sa_len, const int8_t* b,
                            int64_t ldb, const float* sb, int64_t sb_len, const void* bias, int bdt, void* y,
                            int64_t ldy, int ydt, int M, int N, int K, int tile, hipStream_t s) {
  EpiInt8 epi{sa, sa_len, sb, sb_len, bias, bdt, y, ldy, ydt};
  const uint8_t* A = reinterpret_cast<const uint8_t*>(a);
  const uint8_t* B = reinterpret_cast<const uint8_t*>(b);
  if (tile == 64) return launch_mm<MmaI8, 2, 2>(A, lda, B, ldb, M, N, K, epi, s);
  return launch_mm<MmaI8, 4, 4>(A, lda, B, ldb, M, N, K, epi, s);
}

hipError_t launch_fp8_gemm(const uint8_t* a, int64_t lda, const float* sa, int64_t sa_sm, const uint8_t* b,
                           int64_t ldb, const float* sb, int64_t sb_sn, const void* bias, int bdt, void* y,
                           int64_t ldy, int ydt, int M, int N, int K, int tile, hipStream_t s) {
  EpiFp8 epi{sa, sa_sm, sb, sb_sn, bias, bdt, y, ldy, ydt};
  if (tile == 64) return launch_mm<MmaF8, 2, 2>(a, lda, b, ldb, M, N, K, epi, s);
  return launch_mm<MmaF8, 4, 4>(a, lda, b, ldb, M, N, K, epi, s);
}

hipError_t launch_fp8_gemm_blocked(const uint8_t* a, int64_t lda, const float* sa, int64_t sa_sm, int64_t sa_sk,
                                   const uint8_t* b, int64_t ldb, const float* sb, int64_t sb_sn, int64_t sb_sk,
                                   int sb_div, const void* bias, int bdt, void* y, int64_t ldy, int ydt, int M, int N,
                                   int K, hipStream_t s) {
  EpiFp8Blocked epi{sa, sa_sm, sa_sk, sb, sb_sn, sb_sk, sb_div, bias, bdt, y, ldy, ydt, M, N};
  if (M <= 64 || N <= 64) return launch_mm<MmaF8, 2, 2>(a, lda, b, ldb, M, N, K, epi, s);
  return launch_mm<MmaF8, 4, 4>(a, lda, b, ldb, M, N, K, epi, s);
}

}  // namespace fg
