// Large-output W8A8 GEMMs (INT8 and FP8 e4m3fn), C[M,N] = A[M,K] @ B[N,K]^T with both operands K-contiguous.
//
// Workgroup tile 256 x BN (BN = 256, or 320 for INT8 with 16-bit outputs where that fills the last round of
// workgroups better), 512 threads = 2 x 4 wavefronts of 128 x BN/4 (8 x BN/64 MFMA tiles of 16 x 16, 128 or 160
// accumulator registers per lane).  K is walked in 128-byte slices.  Each slice of A and B (32 KiB + BN/8 KiB) is
// written straight from global memory into one half of a double-buffered LDS ring (128 or 144 KiB) by
// global_load_lds_dwordx4 (no staging registers, no VALU), one wavefront instruction = 1 KiB = 8 rows x 128 bytes.
// Within a 128-byte LDS row the 16-byte unit c of global row r is stored at position c ^ key(r): the load lanes pick
// their global column so that this holds.  The key makes the fragment reads (16 rows of one 16-row slab per
// instruction) free of LDS bank conflicts, as measured with the SQ_LDS_BANK_CONFLICT counter on gfx950: r & 7 for the
// INT8 reads (unit 4 s + lane / 16 per lane), and (r & 7) ^ ((r >> 3) & 1) for the FP8 reads (units 2 (lane / 16)
// and + 1), which conflict 4 cycles per instruction under r & 7.
//
// Epilogue for 16-bit outputs: the fp32 result of each 16-row slab of a wavefront tile is scaled, rounded and written
// to a per-wavefront LDS buffer, then stored as 16-byte row segments (row scales read once per row, column scales and
// bias once per column).  32-bit outputs are stored element by element.
//
// mm_ring_kernel (below) is the same design for small M: 64- or 128-row tiles, an S-stage ring with S - 1 slices in
// flight.
//
// Requirements (checked by mm_big_ok, for both kernels): K % 128 == 0, 16-byte aligned A and B with lda, ldb multiples
// of 16.  Rows of A or B past M or N are read from row M-1 or N-1 (valid memory) and their results are not stored.
#include "fg_mm.h"

namespace fg {

template <class E, class = void>
struct IsVec16 : std::false_type {};
template <class E>
struct IsVec16<E, std::void_t<decltype(E::kVec16)>> : std::integral_constant<bool, E::kVec16> {};

// Fragment of row `rp` (one row of a 16-row slab, 128 bytes in LDS, units swizzled by key(r16), r16 = row % 16) for
// k-step s.
struct MmaI8Big : MmaI8 {  // 16 bytes per lane: unit 4s + lane/16
  static __device__ __forceinline__ int key(int r) { return r & 7; }
  static __device__ __forceinline__ frag_t load_sw(const uint8_t* rp, int r16, int lane, int s) {
    const int c = (4 * s + (lane >> 4)) ^ key(r16);
    return *reinterpret_cast<const i32x4*>(rp + c * 16);
  }
};
struct MmaF8Big : MmaF8 {  // 32 bytes per lane: units 2 * (lane/16) and +1 (one k-step per 128-byte slice)
  static __device__ __forceinline__ int key(int r) { return (r & 7) ^ ((r >> 3) & 1); }
  static __device__ __forceinline__ frag_t load_sw(const uint8_t* rp, int r16, int lane, int) {
    const int k = key(r16);
    const int c0 = (2 * (lane >> 4)) ^ k, c1 = (2 * (lane >> 4) + 1) ^ k;
    const i32x4 lo = *reinterpret_cast<const i32x4*>(rp + c0 * 16);
    const i32x4 hi = *reinterpret_cast<const i32x4*>(rp + c1 * 16);
    frag_t f;
    f[0] = lo[0]; f[1] = lo[1]; f[2] = lo[2]; f[3] = lo[3];
    f[4] = hi[0]; f[5] = hi[1]; f[6] = hi[2]; f[7] = hi[3];
    return f;
  }
};

// 16-bit-output epilogues: value = (acc * row_scale) * col_scale (+ bias), one rounding per operation, in the order of
// EpiInt8 / EpiFp8 (and of the oracles), then one rounding to bf16 / fp16.
struct EpiInt8V {
  static constexpr bool kVec16 = true;
  const float* sa; int64_t sa_len;
  const float* sb; int64_t sb_len;
  const void* bias; int bdt;
  uint16_t* y; int64_t ldy; bool bf16; bool vec_ok;
  __device__ __forceinline__ float row_scale(int m) const { return sa[sa_len == 1 ? 0 : m]; }
  __device__ __forceinline__ float col_scale(int n) const { return sb[sb_len == 1 ? 0 : n]; }
  __device__ __forceinline__ float col_bias(int n) const { return bias ? load_f(bias, bdt, n) : 0.f; }
  __device__ __forceinline__ float value(int acc, float rs, float cs, float cb) const {
    float v = (float)acc * rs;
    v = v * cs;
    return bias ? v + cb : v;
  }
  __device__ __forceinline__ uint16_t cvt(float v) const { return bf16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v); }
  __device__ __forceinline__ uint16_t* row_ptr(int m) const { return y + (int64_t)m * ldy; }
};

struct EpiFp8V {
  static constexpr bool kVec16 = true;
  const float* sa; int64_t sa_sm;
  const float* sb; int64_t sb_sn;
  const void* bias; int bdt;
  uint16_t* y; int64_t ldy; bool bf16; bool vec_ok;
  __device__ __forceinline__ float row_scale(int m) const { return sa[(int64_t)m * sa_sm]; }
  __device__ __forceinline__ float col_scale(int n) const { return sb[(int64_t)n * sb_sn]; }
  __device__ __forceinline__ float col_bias(int n) const { return bias ? load_f(bias, bdt, n) : 0.f; }
  __device__ __forceinline__ float value(float acc, float rs, float cs, float cb) const {
    float v = acc * rs;
    v = v * cs;
    return bias ? v + cb : v;
  }
  __device__ __forceinline__ uint16_t cvt(float v) const { return bf16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v); }
  __device__ __forceinline__ uint16_t* row_ptr(int m) const { return y + (int64_t)m * ldy; }
};

// Epilogue of one wavefront's TM x TN tiles of 16 x 16 (rows mw.., columns nw..).  16-bit outputs: the fp32 result of
// each 16-row slab is scaled, rounded and written to the wavefront's LDS buffer `slab` (16 rows x 16 TN + 8 halves),
// then stored as 16-byte row segments (row scales read once per row, column scales and bias once per column).
// 32-bit outputs are stored element by element.
template <class Epi, int TM, int TN, class Acc>
__device__ __forceinline__ void big_epilogue(const Acc (&acc)[TM][TN], uint16_t* slab, const Epi& epi, int mw, int nw,
                                             int lane, int M, int N) {
  if constexpr (IsVec16<Epi>::value) {
    constexpr int SW = 16 * TN;  // slab width in columns
    constexpr int SP = SW + 8;   // LDS row pitch in halves (16-byte aligned rows, staggered banks)
    float cs[TN], cb[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = min(nw + j * 16 + (lane & 15), N - 1);
      cs[j] = epi.col_scale(n);
      cb[j] = epi.col_bias(n);
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      float rs[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) rs[e] = epi.row_scale(min(mw + i * 16 + 4 * (lane >> 4) + e, M - 1));
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          slab[(4 * (lane >> 4) + e) * SP + j * 16 + (lane & 15)] = epi.cvt(epi.value(acc[i][j][e], rs[e], cs[j], cb[j]));
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's slab writes are done before it reads them
      constexpr int NU = 16 * SW / 8;  // 16-byte units of the slab: 2 TN per row (32 .. 160)
#pragma unroll
      for (int u0 = 0; u0 < NU; u0 += 64) {
        const int u = u0 + lane, r = u / (SW / 8), c8 = u % (SW / 8);
        if (NU % 64 != 0 && u >= NU) break;  // a pass with fewer than 64 units left (NU = 32 or 160)
        const int m = mw + i * 16 + r, n = nw + c8 * 8;
        const uint4 v = *reinterpret_cast<const uint4*>(slab + r * SP + c8 * 8);
        if (m < M) {
          if (n + 8 <= N && epi.vec_ok) {
            *reinterpret_cast<uint4*>(epi.row_ptr(m) + n) = v;
          } else {
            const uint16_t h[8] = {(uint16_t)v.x, (uint16_t)(v.x >> 16), (uint16_t)v.y, (uint16_t)(v.y >> 16),
                                   (uint16_t)v.z, (uint16_t)(v.z >> 16), (uint16_t)v.w, (uint16_t)(v.w >> 16)};
            for (int t = 0; t < 8 && n + t < N; ++t) epi.row_ptr(m)[n + t] = h[t];
          }
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads done before the next slab overwrites the buffer
    }
  } else {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = mw + i * 16 + 4 * (lane >> 4) + e;
          const int n = nw + j * 16 + (lane & 15);
          if (m < M && n < N) epi.store(m, n, acc[i][j][e]);
        }
  }
}

constexpr int kBigBM = 256, kBigBN = 256, kBigWM = 2, kBigWN = 4, kBigBK = 128;
constexpr size_t big_lds_bytes(int bn) { return 2 * (size_t)(kBigBM + bn) * kBigBK; }

template <class Mma, class Epi, int BN>
__global__ void __launch_bounds__(kBigWM * kBigWN * 64) mm_big_kernel(const uint8_t* __restrict__ A, int64_t lda,
                                                                      const uint8_t* __restrict__ B, int64_t ldb,
                                                                      int M, int N, int K, Epi epi) {
  constexpr int BM = kBigBM, WM = kBigWM, WN = kBigWN, BK = kBigBK;
  constexpr int NT = WM * WN * 64;
  constexpr int TM = BM / WM / 16, TN = BN / WN / 16;
  constexpr int A_INSTR = BM * BK / 16 / NT, B_INSTR = BN * BK / 16 / NT;  // 1 KiB load instructions per wave
  static_assert(A_INSTR * NT * 16 == BM * BK && B_INSTR * NT * 16 == BN * BK, "tile / thread count mismatch");
  constexpr int STAGE = (BM + BN) * BK;
  extern __shared__ __align__(16) uint8_t smem[];

  const int ntm = (M + BM - 1) / BM, ntn = (N + BN - 1) / BN;
  int tm_, tn_;
  tile_of(blockIdx.x, ntm, ntn, tm_, tn_);
  const int m0 = tm_ * BM, n0 = tn_ * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  // Load instruction i of wave w fills LDS units (w * INSTR + i) * 64 + lane, i.e. row r = (w * INSTR + i) * 8 +
  // lane / 8, position lane % 8, which holds global unit (lane % 8) ^ key(r) (the swizzle is its own inverse).
  const int lrow = lane >> 3;
  const int arow0 = wave * A_INSTR * 8 + lrow, brow0 = wave * B_INSTR * 8 + lrow;
  auto issue = [&](int kt, uint8_t* st) __attribute__((always_inline)) {
    const int64_t ko = (int64_t)kt * BK;
#pragma unroll
    for (int i = 0; i < A_INSTR; ++i) {
      const int col = ((lane & 7) ^ Mma::key(arow0 + 8 * i)) * 16;
      __builtin_amdgcn_global_load_lds(A + (int64_t)min(m0 + arow0 + 8 * i, M - 1) * lda + ko + col,
                                       st + (wave * A_INSTR + i) * 1024, 16, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < B_INSTR; ++i) {
      const int col = ((lane & 7) ^ Mma::key(brow0 + 8 * i)) * 16;
      __builtin_amdgcn_global_load_lds(B + (int64_t)min(n0 + brow0 + 8 * i, N - 1) * ldb + ko + col,
                                       st + BM * BK + (wave * B_INSTR + i) * 1024, 16, 0, 0);
    }
  };

  typename Mma::acc_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[i][j][e] = 0;

  const int r16 = lane & 15;
  const int nk = K / BK;
  issue(0, smem);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const uint8_t* cur = smem + (kt & 1) * STAGE;
    if (kt + 1 < nk) issue(kt + 1, smem + ((kt + 1) & 1) * STAGE);  // the other buffer: free since the last barrier
    const uint8_t* sA = cur + (wm * TM * 16) * BK;
    const uint8_t* sB = cur + BM * BK + (wn * TN * 16) * BK;
#pragma unroll
    for (int s = 0; s < BK / Mma::KB; ++s) {
      typename Mma::frag_t fa[TM];
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[i] = Mma::load_sw(sA + (i * 16 + r16) * BK, r16, lane, s);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const typename Mma::frag_t fb = Mma::load_sw(sB + (j * 16 + r16) * BK, r16, lane, s);
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[i][j] = Mma::mma(fa[i], fb, acc[i][j]);
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // next slice landed in LDS
    __syncthreads();                                  // ... for every wave; and this slice is no longer read
  }

  constexpr int SW = 16 * TN;
  big_epilogue<Epi, TM, TN>(acc, reinterpret_cast<uint16_t*>(smem) + wave * 16 * (SW + 8), epi, m0 + wm * 16 * TM,
                            n0 + wn * SW, lane, M, N);  // the ring is free after the last barrier
}

// Small-M W8A8 GEMMs (M up to a few hundred rows, where 256-row tiles would leave most CUs idle): BM x BN tiles,
// WM x WN wavefronts, K in 128-byte slices written straight into an S-stage LDS ring by global_load_lds_dwordx4,
// S - 1 slices in flight.  A workgroup here does little MFMA work per slice (BM x BN x 128), so a two-stage ring
// leaves every slice waiting for its loads' full HBM latency; the deep ring keeps the loads of the next S - 1 slices
// in flight while one is multiplied.  Every slice issues the same loads (slices past the last re-read it, into a stage
// no one reads again), so `vmcnt((S - 2) * loads per slice)` is exactly "slice kt + 1 has landed".  Same swizzle,
// fragment reads and epilogue as mm_big_kernel.
template <class Mma, class Epi, int BM, int BN, int WM, int WN, int S>
__global__ void __launch_bounds__(WM * WN * 64) mm_ring_kernel(const uint8_t* __restrict__ A, int64_t lda,
                                                               const uint8_t* __restrict__ B, int64_t ldb, int M,
                                                               int N, int K, Epi epi) {
  constexpr int BK = kBigBK, NT = WM * WN * 64;
  constexpr int TM = BM / WM / 16, TN = BN / WN / 16;
  constexpr int A_INSTR = BM * BK / 16 / NT, B_INSTR = BN * BK / 16 / NT, NI = A_INSTR + B_INSTR;
  static_assert(TM * WM * 16 == BM && TN * WN * 16 == BN, "wavefront tiles must cover the workgroup tile");
  static_assert(A_INSTR >= 1 && B_INSTR >= 1 && A_INSTR * NT * 16 == BM * BK && B_INSTR * NT * 16 == BN * BK,
                "tile / thread count mismatch");
  static_assert(S >= 2 && (S - 2) * NI <= 63, "the wait count must fit vmcnt");
  constexpr int STAGE = (BM + BN) * BK;
  extern __shared__ __align__(16) uint8_t smem[];

  const int ntm = (M + BM - 1) / BM, ntn = (N + BN - 1) / BN;
  int tm_, tn_;
  tile_of(blockIdx.x, ntm, ntn, tm_, tn_);
  const int m0 = tm_ * BM, n0 = tn_ * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  const int lrow = lane >> 3;
  const int arow0 = wave * A_INSTR * 8 + lrow, brow0 = wave * B_INSTR * 8 + lrow;
  auto issue = [&](int kt, uint8_t* st) __attribute__((always_inline)) {
    const int64_t ko = (int64_t)kt * BK;
#pragma unroll
    for (int i = 0; i < A_INSTR; ++i) {
      const int col = ((lane & 7) ^ Mma::key(arow0 + 8 * i)) * 16;
      __builtin_amdgcn_global_load_lds(A + (int64_t)min(m0 + arow0 + 8 * i, M - 1) * lda + ko + col,
                                       st + (wave * A_INSTR + i) * 1024, 16, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < B_INSTR; ++i) {
      const int col = ((lane & 7) ^ Mma::key(brow0 + 8 * i)) * 16;
      __builtin_amdgcn_global_load_lds(B + (int64_t)min(n0 + brow0 + 8 * i, N - 1) * ldb + ko + col,
                                       st + BM * BK + (wave * B_INSTR + i) * 1024, 16, 0, 0);
    }
  };

  typename Mma::acc_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[i][j][e] = 0;

  const int r16 = lane & 15;
  const int nk = K / BK;
#pragma unroll
  for (int p = 0; p < S - 1; ++p) issue(min(p, nk - 1), smem + p * STAGE);
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((S - 2) * NI) : "memory");  // slice 0 has landed
  // The stage being read and the stage being loaded reach the body as __restrict__ pointers, so the compiler does not
  // wait for the loads in flight before the fragment reads.
  auto body = [&](int kt, const uint8_t* __restrict__ cur, uint8_t* __restrict__ nxt) __attribute__((always_inline)) {
    issue(min(kt + S - 1, nk - 1), nxt);  // the stage of slice kt - 1: every wave has read it (last barrier)
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t* sA = cur + (wm * TM * 16) * BK;
    const uint8_t* sB = cur + BM * BK + (wn * TN * 16) * BK;
#pragma unroll
    for (int s = 0; s < BK / Mma::KB; ++s) {
      typename Mma::frag_t fa[TM];
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[i] = Mma::load_sw(sA + (i * 16 + r16) * BK, r16, lane, s);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const typename Mma::frag_t fb = Mma::load_sw(sB + (j * 16 + r16) * BK, r16, lane, s);
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[i][j] = Mma::mma(fa[i], fb, acc[i][j]);
      }
    }
    // slice kt + 1 has landed (the S - 2 slices after it may be in flight) and this wave's fragment reads are done;
    // then the barrier, after which stage kt may be overwritten.  Not __syncthreads(): its release fence would wait
    // for every load in flight.
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((S - 2) * NI) : "memory");
  };
  int st = 0;  // stage of slice kt
  for (int kt = 0; kt < nk; ++kt) {
    const int sl = st == 0 ? S - 1 : st - 1;  // stage of slice kt - 1 = stage of slice kt + S - 1
    body(kt, smem + st * STAGE, smem + sl * STAGE);
    st = st + 1 == S ? 0 : st + 1;
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the re-read loads of the last slices
  __syncthreads();                                  // the epilogue reuses the ring
  constexpr int SW = 16 * TN;
  big_epilogue<Epi, TM, TN>(acc, reinterpret_cast<uint16_t*>(smem) + wave * 16 * (SW + 8), epi, m0 + wm * 16 * TM,
                            n0 + wn * SW, lane, M, N);
}

bool mm_big_ok(const void* a, int64_t lda, const void* b, int64_t ldb, int64_t K) {
  return K % kBigBK == 0 && lda % 16 == 0 && ldb % 16 == 0 &&
         ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) % 16) == 0;
}

// Workgroups of the 256 x 256 kernel for an M x N output.
int64_t mm_big_tiles(int64_t M, int64_t N) { return ((M + kBigBM - 1) / kBigBM) * ((N + kBigBN - 1) / kBigBN); }

// Tile width for an M x N output: 320 when its rounds of workgroups over the CUs, weighted by the tile width, cost
// less than those of 256 (K=8192, N=10240, M=4096: 640 tiles of 256 take 3 rounds, the last half empty; 512 tiles of
// 320 take 2).
int mm_big_bn(int64_t M, int64_t N) {
  const int64_t cus = device_cus(), tm = (M + kBigBM - 1) / kBigBM;
  const int64_t r256 = (tm * ((N + 255) / 256) + cus - 1) / cus, r320 = (tm * ((N + 319) / 320) + cus - 1) / cus;
  return r320 * 320 < r256 * 256 ? 320 : 256;
}

template <class Mma, int BN, class Epi>
static hipError_t launch_big_t(const uint8_t* A, int64_t lda, const uint8_t* B, int64_t ldb, int M, int N, int K,
                               const Epi& epi, hipStream_t s) {
  auto k = mm_big_kernel<Mma, Epi, BN>;
  constexpr size_t lds = big_lds_bytes(BN);
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)lds);
  if (e != hipSuccess) return e;
  const unsigned tiles = (unsigned)(((M + kBigBM - 1) / kBigBM) * ((N + BN - 1) / BN));
  note_kernel("mm_big_kernel 256x%d", BN);
  hipLaunchKernelGGL(k, dim3(tiles), dim3(kBigWM * kBigWN * 64), lds, s, A, lda, B, ldb, M, N, K, epi);
  return hipGetLastError();
}

// The 320-wide tile only for INT8 with 16-bit outputs: it takes 234 registers per lane there, and spills for FP8
// fragments (8 registers each) or the element-wise 32-bit epilogue.
template <class Mma, class Epi>
static hipError_t launch_big(const uint8_t* A, int64_t lda, const uint8_t* B, int64_t ldb, int M, int N, int K,
                             const Epi& epi, hipStream_t s) {
  if constexpr (std::is_same<Mma, MmaI8Big>::value && IsVec16<Epi>::value) {
    if (mm_big_bn(M, N) == 320) return launch_big_t<Mma, 320>(A, lda, B, ldb, M, N, K, epi, s);
  }
  return launch_big_t<Mma, 256>(A, lda, B, ldb, M, N, K, epi, s);
}

static bool vec16_ok(const void* y, int64_t ldy) { return ldy % 8 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0; }

hipError_t launch_int8_gemm_big(const int8_t* a, int64_t lda, const float* sa, int64_t sa_len, const int8_t* b,
                                int64_t ldb, const float* sb, int64_t sb_len, const void* bias, int bdt, void* y,
                                int64_t ldy, int ydt, int M, int N, int K, hipStream_t s) {
  const uint8_t* A = reinterpret_cast<const uint8_t*>(a);
  const uint8_t* B = reinterpret_cast<const uint8_t*>(b);
  if (ydt == FG_BF16 || ydt == FG_F16) {
    EpiInt8V epi{sa, sa_len, sb, sb_len, bias, bdt, static_cast<uint16_t*>(y), ldy, ydt == FG_BF16, vec16_ok(y, ldy)};
    return launch_big<MmaI8Big>(A, lda, B, ldb, M, N, K, epi, s);
  }
  EpiInt8 epi{sa, sa_len, sb, sb_len, bias, bdt, y, ldy, ydt};
  return launch_big<MmaI8Big>(A, lda, B, ldb, M, N, K, epi, s);
}

hipError_t launch_fp8_gemm_big(const uint8_t* a, int64_t lda, const float* sa, int64_t sa_sm, const uint8_t* b,
                               int64_t ldb, const float* sb, int64_t sb_sn, const void* bias, int bdt, void* y,
                               int64_t ldy, int ydt, int M, int N, int K, hipStream_t s) {
  if (ydt == FG_BF16 || ydt == FG_F16) {
    EpiFp8V epi{sa, sa_sm, sb, sb_sn, bias, bdt, static_cast<uint16_t*>(y), ldy, ydt == FG_BF16, vec16_ok(y, ldy)};
    return launch_big<MmaF8Big>(a, lda, b, ldb, M, N, K, epi, s);
  }
  EpiFp8 epi{sa, sa_sm, sb, sb_sn, bias, bdt, y, ldy, ydt};
  return launch_big<MmaF8Big>(a, lda, b, ldb, M, N, K, epi, s);
}

// Tile width of the ring kernel for BM-row tiles: 128 for BM = 128; for BM = 64 the widest of 128, 64 and 32 whose
// tiles number at least 5/8 of the CUs, else 32.  Measured (K = 8192, random operands): fp8 N = 8192 at M = 16 / 64
// best with 32 (256 tiles: 16.7 / 19.3 us, 64-wide 18.6 / 23.5), M = 128 with 64, M = 256 with 128; int8 N = 10240 at
// M <= 64 with 64 (160 tiles: 20-26 us; 32-wide 35-37 us), N = 57344 with 128 or 64 (within 2%).
int mm_ring_bn(int64_t M, int64_t N, int bm) {
  if (bm == 128) return 128;
  const int64_t thr = device_cus() * 5 / 8, tm = (M + 63) / 64;
  for (int bn : {128, 64})
    if (tm * ((N + bn - 1) / bn) >= thr) return bn;
  return 32;
}

template <class Mma, int BM, int BN, int WM, int WN, int S, class Epi>
static hipError_t launch_ring_t(const uint8_t* A, int64_t lda, const uint8_t* B, int64_t ldb, int M, int N, int K,
                                const Epi& epi, hipStream_t s) {
  auto k = mm_ring_kernel<Mma, Epi, BM, BN, WM, WN, S>;
  constexpr size_t lds = (size_t)S * (BM + BN) * kBigBK;
  static_assert(lds <= 160 * 1024, "ring exceeds the LDS");
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)lds);
  if (e != hipSuccess) return e;
  const unsigned tiles = (unsigned)(((M + BM - 1) / BM) * ((N + BN - 1) / BN));
  note_kernel("mm_ring_kernel %dx%d S=%d", BM, BN, S);
  hipLaunchKernelGGL(k, dim3(tiles), dim3(WM * WN * 64), lds, s, A, lda, B, ldb, M, N, K, epi);
  return hipGetLastError();
}

// Instances (BM x BN, wavefronts, stages), each the fastest of those measured for its width: 64 x 32 with 2 x 2
// wavefronts and 8 stages, 64 x 64 with 2 x 4 and 6, 64 x 128 with 2 x 4 and 4, 128 x 128 with 2 x 4 and 3.
template <class Mma, class Epi>
static hipError_t launch_ring(const uint8_t* A, int64_t lda, const uint8_t* B, int64_t ldb, int M, int N, int K,
                              const Epi& epi, int bm, int bn, hipStream_t s) {
  if (bm == 128) return launch_ring_t<Mma, 128, 128, 2, 4, 3>(A, lda, B, ldb, M, N, K, epi, s);
  if (bn == 128) return launch_ring_t<Mma, 64, 128, 2, 4, 4>(A, lda, B, ldb, M, N, K, epi, s);
  if (bn == 64) return launch_ring_t<Mma, 64, 64, 2, 4, 6>(A, lda, B, ldb, M, N, K, epi, s);
  return launch_ring_t<Mma, 64, 32, 2, 2, 8>(A, lda, B, ldb, M, N, K, epi, s);
}

hipError_t launch_int8_gemm_ring(const int8_t* a, int64_t lda, const float* sa, int64_t sa_len, const int8_t* b,
                                 int64_t ldb, const float* sb, int64_t sb_len, const void* bias, int bdt, void* y,
                                 int64_t ldy, int ydt, int M, int N, int K, int bm, int bn, hipStream_t s) {
  const uint8_t* A = reinterpret_cast<const uint8_t*>(a);
  const uint8_t* B = reinterpret_cast<const uint8_t*>(b);
  if (ydt == FG_BF16 || ydt == FG_F16) {
    EpiInt8V epi{sa, sa_len, sb, sb_len, bias, bdt, static_cast<uint16_t*>(y), ldy, ydt == FG_BF16, vec16_ok(y, ldy)};
    return launch_ring<MmaI8Big>(A, lda, B, ldb, M, N, K, epi, bm, bn, s);
  }
  EpiInt8 epi{sa, sa_len, sb, sb_len, bias, bdt, y, ldy, ydt};
  return launch_ring<MmaI8Big>(A, lda, B, ldb, M, N, K, epi, bm, bn, s);
}

hipError_t launch_fp8_gemm_ring(const uint8_t* a, int64_t lda, const float* sa, int64_t sa_sm, const uint8_t* b,
                                int64_t ldb, const float* sb, int64_t sb_sn, const void* bias, int bdt, void* y,
                                int64_t ldy, int ydt, int M, int N, int K, int bm, int bn, hipStream_t s) {
  if (ydt == FG_BF16 || ydt == FG_F16) {
    EpiFp8V epi{sa, sa_sm, sb, sb_sn, bias, bdt, static_cast<uint16_t*>(y), ldy, ydt == FG_BF16, vec16_ok(y, ldy)};
    return launch_ring<MmaF8Big>(a, lda, b, ldb, M, N, K, epi, bm, bn, s);
  }
  EpiFp8 epi{sa, sa_sm, sb, sb_sn, bias, bdt, y, ldy, ydt};
  return launch_ring<MmaF8Big>(a, lda, b, ldb, M, N, K, epi, bm, bn, s);
}

}  // namespace fg
