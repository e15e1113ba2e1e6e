// W8A8 skinny GEMMs on matrix cores for M <= 64 (decode batches, HBM-bound): C[M,N] = A[M,K] @ B[N,K]^T with the
// INT8 / FP8 scale epilogues of EpiInt8 / EpiFp8.
//
// The structure of the W4 skinny kernel without the dequantisation: a wavefront owns T tiles of 16 output channels
// and one K slice, walked in 256-byte steps; the KS wavefronts of a workgroup take the KS slices of the same channels
// and sum their partials in slice order through LDS (int32 partials for INT8, so the sum stays exact; fp32 for FP8).
// Operands go from global memory straight into registers through raw buffer loads (32-bit lane offsets, no 64-bit
// address math), two steps ahead of the MFMAs.
//
// Operand layout per 256-byte step.  Lane l (row / channel l % 16, lane group j = l / 16) loads the 64 contiguous
// bytes 64 j .. 64 j + 63 of the step from its weight row (one 16-byte load per 16 bytes) and the same bytes of its x
// row.  MFMA k-step s takes the lane's bytes 16 s .. (INT8: v_mfma_i32_16x16x64_i8, 16 bytes per lane, 4 k-steps) or
// 32 s .. (FP8: v_mfma_f32_16x16x128_f8f6f4, 32 bytes per lane, 2 k-steps): one instruction covers one piece of each
// lane group's 64 bytes, A and B the same pieces, and the products are summed over every K element once.
//
// Requirements (w8_skinny_ok): K % 256 == 0, 16-byte aligned A and B with lda, ldb multiples of 16, operands under
// 4 GiB.
#include "fg_mm.h"

namespace fg {

__device__ __forceinline__ __amdgpu_buffer_rsrc_t w8sk_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ uint4 w8sk_ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// Threads per workgroup at most: 512 when the tiles times the m-tiles reach 2 (more than 128 registers), else 1024.
constexpr int w8_skinny_max_threads(int mb, int t) { return mb * t >= 2 ? 512 : 1024; }

template <bool F8>
struct W8Op {
  typedef typename std::conditional<F8, f32x4, i32x4>::type acc_t;
  static constexpr int KSTEPS = F8 ? 2 : 4;  // MFMA k-steps per 256-byte step
  // k-step s of one lane's 64 bytes (4 x 16)
  static __device__ __forceinline__ acc_t mma(const uint4 (&a)[4], const uint4 (&b)[4], int s, acc_t c) {
    if constexpr (F8) {
      const uint4 a0 = a[2 * s], a1 = a[2 * s + 1], b0 = b[2 * s], b1 = b[2 * s + 1];
      const i32x8 fa = {(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
      const i32x8 fb = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
      return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(fa, fb, c, 0, 0, 0, 0, 0, 0);
    } else {
      const i32x4 fa = {(int)a[s].x, (int)a[s].y, (int)a[s].z, (int)a[s].w};
      const i32x4 fb = {(int)b[s].x, (int)b[s].y, (int)b[s].z, (int)b[s].w};
      return __builtin_amdgcn_mfma_i32_16x16x64_i8(fa, fb, c, 0, 0, 0);
    }
  }
};

template <int MB, int T, bool F8, class Epi>
__global__ void __launch_bounds__(w8_skinny_max_threads(MB, T)) w8_skinny_kernel(
    const uint8_t* __restrict__ A, int64_t lda, const uint8_t* __restrict__ B, int64_t ldb, int M, int N, int K,
    int KS, Epi epi) {
  typedef W8Op<F8> Op;
  typedef typename Op::acc_t acc_t;
  typedef typename std::conditional<F8, float, int>::type elem_t;
  constexpr int NV = T * MB * 4;
  extern __shared__ __align__(16) uint8_t w8red_raw[];
  elem_t* red = reinterpret_cast<elem_t*>(w8red_raw);  // [waves][NV][64]
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int BW = (int)(blockDim.x / kWave) / KS;
  const int ks = wave % KS, nb = blockIdx.x * BW + wave / KS;
  const int n0 = nb * 16 * T;
  const int nsteps = K / 256;
  const int st0 = (int)((int64_t)ks * nsteps / KS), st1 = (int)((int64_t)(ks + 1) * nsteps / KS);
  const int r16 = lane & 15, j = lane >> 4;

  const uint32_t aspan = (uint32_t)M * (uint32_t)lda, bspan = (uint32_t)N * (uint32_t)ldb;
  const __amdgpu_buffer_rsrc_t ra = w8sk_rsrc(A, aspan);
  const __amdgpu_buffer_rsrc_t rb = w8sk_rsrc(B, bspan);
  uint32_t boff[T], aoff[MB];
#pragma unroll
  for (int t = 0; t < T; ++t) boff[t] = (uint32_t)min(n0 + 16 * t + r16, N - 1) * (uint32_t)ldb + 64u * j;
#pragma unroll
  for (int i = 0; i < MB; ++i)  // rows past M start at the end of A: their loads read 0 and fetch nothing
    aoff[i] = 16 * i + r16 < M ? (uint32_t)(16 * i + r16) * (uint32_t)lda + 64u * j : (uint32_t)M * (uint32_t)lda;

  struct Buf {
    uint4 a[MB][4], b[T][4];
  };
  Buf bufa, bufb;
  auto fetch = [&](int st, Buf& f) __attribute__((always_inline)) {
    const bool live = st < st1;
    const uint32_t so = (uint32_t)st * 256u;
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) f.a[i][q] = w8sk_ld16(ra, live ? aoff[i] + so + 16u * q : aspan);
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int q = 0; q < 4; ++q) f.b[t][q] = w8sk_ld16(rb, live ? boff[t] + so + 16u * q : bspan);
  };
  acc_t acc[T][MB];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[t][i] = acc_t{0, 0, 0, 0};
  auto compute = [&](const Buf& f) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < Op::KSTEPS; ++s)
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int i = 0; i < MB; ++i) acc[t][i] = Op::mma(f.a[i], f.b[t], s, acc[t][i]);
  };
  // Steps past the slice are fetched through offsets past the operands' spans: the same load instructions (so each
  // wait before a compute counts exactly the older loads) that read zeros and move no memory.
  if (st0 < st1) {
    fetch(st0, bufa);
    fetch(st0 + 1, bufb);
    for (int st = st0; st < st1; st += 2) {
      compute(bufa);
      fetch(st + 2, bufa);
      if (st + 1 < st1) compute(bufb);
      fetch(st + 3, bufb);
    }
  }

  // sum the KS slices of this channel block in slice order; wavefront ks stores value indices ks, ks + KS, ...
  elem_t* mine = red + (size_t)wave * NV * kWave;
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) mine[((t * MB + i) * 4 + e) * kWave + lane] = acc[t][i][e];
  __syncthreads();
  const elem_t* base = red + (size_t)(wave - ks) * NV * kWave;
  for (int v = ks; v < NV; v += KS) {
    elem_t sum = 0;
    for (int k2 = 0; k2 < KS; ++k2) sum += base[((size_t)k2 * NV + v) * kWave + lane];
    const int t = v / (MB * 4), i = (v / 4) % MB, e = v % 4;
    const int m = 16 * i + 4 * j + e, n = n0 + 16 * t + r16;
    if (m < M && n < N) epi.store(m, n, sum);
  }
}

bool w8_skinny_ok(const void* a, int64_t lda, const void* b, int64_t ldb, int64_t M, int64_t N, int64_t K) {
  const int64_t k4g = 1LL << 32;
  return M > 0 && M <= 64 && (K % 256) == 0 && (lda % 16) == 0 && (ldb % 16) == 0 &&
         (reinterpret_cast<uintptr_t>(a) % 16) == 0 && (reinterpret_cast<uintptr_t>(b) % 16) == 0 &&
         M * lda < k4g && N * ldb < k4g;
}

// Launch shape: T tiles of 16 channels per wavefront, the largest of 4 / 2 / 1 (2 for M <= 32, 1 for M <= 64: the x
// registers) leaving at least 3/4 of a channel block per CU; KS K slices so that about 4 wavefronts per CU exist (at
// most the workgroup limit and the 256-byte steps); two channel blocks per workgroup from 1.5 blocks per CU.
void w8_skinny_plan(int M, int N, int K, int* mb, int* T, int* KS, int* BW) {
  const int cus = device_cus();
  const int b = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  int t = b == 1 ? 4 : (b == 2 ? 2 : 1);
  while (t > 1 && 4 * ((N + 16 * t - 1) / (16 * t)) < 3 * cus) t /= 2;
  const int nblk = (N + 16 * t - 1) / (16 * t);
  const int maxw = w8_skinny_max_threads(b, t) / kWave;
  int ks = (4 * cus + nblk - 1) / nblk;
  ks = max(1, min(ks, min(maxw, K / 256)));
  *mb = b; *T = t; *KS = ks; *BW = skinny_balance(nblk, ks, maxw, cus);
}

template <int MB, int T, bool F8, class Epi>
static hipError_t launch_w8sk_t(const uint8_t* a, int64_t lda, const uint8_t* b, int64_t ldb, int M, int N, int K,
                                int KS, int BW, const Epi& epi, hipStream_t s) {
  const int nblk = (N + 16 * T - 1) / (16 * T);
  const size_t shm = (size_t)BW * KS * (T * MB * 4) * kWave * 4;
  auto kern = w8_skinny_kernel<MB, T, F8, Epi>;
  if (shm > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
    if (e != hipSuccess) return e;
  }
  note_kernel("w8_skinny_kernel KS=%d", KS);
  hipLaunchKernelGGL(kern, dim3((nblk + BW - 1) / BW), dim3(kWave * BW * KS), shm, s, a, lda, b, ldb, M, N, K, KS,
                     epi);
  return hipGetLastError();
}

template <bool F8, class Epi>
static hipError_t launch_w8sk(const uint8_t* a, int64_t lda, const uint8_t* b, int64_t ldb, int M, int N, int K,
                              const Epi& epi, hipStream_t s) {
  int mb, T, KS, BW;
  w8_skinny_plan(M, N, K, &mb, &T, &KS, &BW);
#define FG_W8SK(MB_, T_) return launch_w8sk_t<MB_, T_, F8, Epi>(a, lda, b, ldb, M, N, K, KS, BW, epi, s)
  if (mb == 1) {
    if (T == 4) FG_W8SK(1, 4);
    if (T == 2) FG_W8SK(1, 2);
    FG_W8SK(1, 1);
  }
  if (mb == 2) {
    if (T == 2) FG_W8SK(2, 2);
    FG_W8SK(2, 1);
  }
  FG_W8SK(4, 1);
#undef FG_W8SK
}

hipError_t launch_int8_gemm_skinny(const int8_t* a, int64_t lda, const float* sa, int64_t sa_len, const int8_t* b,
                                   int64_t ldb, const float* sb, int64_t sb_len, const void* bias, int bdt, void* y,
                                   int64_t ldy, int ydt, int M, int N, int K, hipStream_t s) {
  const EpiInt8 epi{sa, sa_len, sb, sb_len, bias, bdt, y, ldy, ydt};
  return launch_w8sk<false>(reinterpret_cast<const uint8_t*>(a), lda, reinterpret_cast<const uint8_t*>(b), ldb, M,
                            N, K, epi, s);
}

hipError_t launch_fp8_gemm_skinny(const uint8_t* a, int64_t lda, const float* sa, int64_t sa_sm, const uint8_t* b,
                                  int64_t ldb, const float* sb, int64_t sb_sn, const void* bias, int bdt, void* y,
                                  int64_t ldy, int ydt, int M, int N, int K, hipStream_t s) {
  const EpiFp8 epi{sa, sa_sm, sb, sb_sn, bias, bdt, y, ldy, ydt};
  return launch_w8sk<true>(a, lda, b, ldb, M, N, K, epi, s);
}

}  // namespace fg
