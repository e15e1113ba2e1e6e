// W4A16 skinny GEMM on matrix cores for 4 < M <= 64 (decode batches): y[M,N] = x[M,K] @ dequant(W)[N,K]^T (+bias).
//
// The split GEMV's structure with v_mfma_f32_16x16x32_{bf16,f16} in place of v_dot2: a wavefront owns T tiles of 16
// output channels and one K slice, walked in 128-column steps; the KS wavefronts of a workgroup take the KS slices of
// the same channels and sum their partials in slice order through LDS at the end (one launch, no workspace,
// deterministic).  No LDS on the hot path: every operand goes from global memory into registers.
//
// Operand layout per 128-column step.  Lane l (channel or row l % 16, lane group j = l / 16) holds 16 bytes = 4 packed
// words of its weight row, columns 32 j .. 32 j + 31 of the step (one coalesced 16-byte load per tile), and 64 bytes of
// its x row over the same columns.  MFMA k-step s (s = 0..3) takes word s: lane group j supplies columns 32 j + 8 s ..
// + 7, so one MFMA covers four 8-column pieces of the step (the sum over k does not care which).  A word's nibbles
// become four exact bf16 / fp16 pairs B + (q0,q2) (q1,q3) (q4,q6) (q5,q7) (two masks and four byte-permutes against
// the magic exponent byte: bf16 0x43 -> 128 + q, fp16 0x64 -> 1024 + q), and x is put in the same order with four
// byte-permutes per 8 columns.  The offset leaves per group: sum x (q - z) = sum x (B + q) - (B + z) sum x; the row sums of
// x come from one more MFMA per m-tile and k-step against all-ones, which lands them in the accumulator layout.  Each
// step is one group or part of one (group size a multiple of 128, or one group per row), so after a step's MFMAs
//   acc += s[n, g] * (acc_step - (B + z[n, g]) * xsum)     (fp32, per accumulator element)
// and acc_step restarts at zero.
//
// Requirements (w4_skinny_ok): K % 128 == 0, group size % 128 == 0 or one group, 16-bit scales, 16-byte aligned x with
// ldx % 8 == 0, 16-byte aligned qweight with ldq % 4 == 0, no act-order perm.
#include "fg_device.h"

namespace fg {

typedef __bf16 bf16x8_sk_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_sk_t __attribute__((ext_vector_type(8)));
typedef float f32x4_sk_t __attribute__((ext_vector_type(4)));

template <bool XBF16>
__device__ __forceinline__ f32x4_sk_t sk_mfma(uint4 a, uint4 b, f32x4_sk_t c) {
  if constexpr (XBF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_sk_t, a),
                                                   __builtin_bit_cast(bf16x8_sk_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_sk_t, a),
                                                  __builtin_bit_cast(f16x8_sk_t, b), c, 0, 0, 0);
  }
}

// 8 x values (x0..x7 as 4 packed pairs) in the order (x0,x2) (x1,x3) (x4,x6) (x5,x7)
__device__ __forceinline__ uint4 sk_xorder(uint4 v) {
  return make_uint4(__builtin_amdgcn_perm(v.y, v.x, 0x05040100u), __builtin_amdgcn_perm(v.y, v.x, 0x07060302u),
                    __builtin_amdgcn_perm(v.w, v.z, 0x05040100u), __builtin_amdgcn_perm(v.w, v.z, 0x07060302u));
}

// a packed word's nibbles as the exact 16-bit pairs B + (q0,q2) (q1,q3) (q4,q6) (q5,q7): two masks split even and
// odd nibbles into bytes, four byte-permutes put the magic exponent byte above each
template <bool XBF16>
__device__ __forceinline__ uint4 sk_wunpack(uint32_t w) {
  constexpr uint32_t kMagicBytes = XBF16 ? 0x43434343u : 0x64646464u;
  const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
  return make_uint4(__builtin_amdgcn_perm(kMagicBytes, lo, 0x04010400u), __builtin_amdgcn_perm(kMagicBytes, hi, 0x04010400u),
                    __builtin_amdgcn_perm(kMagicBytes, lo, 0x04030402u), __builtin_amdgcn_perm(kMagicBytes, hi, 0x04030402u));
}

// Raw buffer resource over `bytes` bytes from p (gfx9 dword3: 32-bit data format); loads through it take a 32-bit
// per-lane offset, need no 64-bit address math, and read 0 past the end.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t sk_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// Threads per workgroup at most: 512 when the tile count times the m-tiles reaches 2 (those need more than 128
// registers per lane), else 1024.
constexpr int w4_skinny_max_threads(int mb, int t) { return mb * t >= 2 ? 512 : 1024; }

template <int MB, int T, bool XBF16, bool SBF16>
__global__ void __launch_bounds__(w4_skinny_max_threads(MB, T)) w4_skinny_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const int32_t* __restrict__ qw, int64_t ldq,
    const uint16_t* __restrict__ scales, int64_t lds, const int32_t* __restrict__ zeros, int64_t ldz, int hasz,
    const void* __restrict__ bias, int bdt, uint16_t* __restrict__ y, int64_t ldy, int M, int N, int K, int gsteps,
    int KS) {
  constexpr float kB = XBF16 ? 128.f : 1024.f;
  constexpr uint32_t kOnes = XBF16 ? 0x3F803F80u : 0x3C003C00u;
  constexpr int NV = T * MB * 4;  // accumulator values per lane
  extern __shared__ __align__(16) float red[];  // [waves][NV][64]
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int BW = (int)(blockDim.x / kWave) / KS;
  const int ks = wave % KS, nb = blockIdx.x * BW + wave / KS;
  const int n0 = nb * 16 * T;
  const int nsteps = K / 128;
  const int st0 = (int)((int64_t)ks * nsteps / KS), st1 = (int)((int64_t)(ks + 1) * nsteps / KS);
  const int r16 = lane & 15, j = lane >> 4;

  // per tile: this lane's weight row and the column of its accumulator values (the same channel n0 + 16 t + r16).
  // Offsets are 32-bit from the uniform base pointers (the host checks that every operand spans < 4 GiB).
  const int G = gsteps > 0 ? (K / 128 + gsteps - 1) / gsteps : 1;
  const uint32_t qspan = (uint32_t)N * (uint32_t)ldq * 4u, xspan = (uint32_t)M * (uint32_t)ldx * 2u;
  const uint32_t sspan = (uint32_t)G * (uint32_t)lds * 2u, zspan = hasz ? (uint32_t)G * (uint32_t)ldz * 4u : 4u;
  const __amdgpu_buffer_rsrc_t rq = sk_rsrc(qw, qspan);
  const __amdgpu_buffer_rsrc_t rx = sk_rsrc(x, xspan);
  const __amdgpu_buffer_rsrc_t rs = sk_rsrc(scales, sspan);
  const __amdgpu_buffer_rsrc_t rz = sk_rsrc(zeros, zspan);
  uint32_t woff[T], soff[T], zoff[T];
  int ncol[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    ncol[t] = min(n0 + 16 * t + r16, N - 1);
    woff[t] = (uint32_t)ncol[t] * (uint32_t)ldq * 4u + 16u * j;
    soff[t] = (uint32_t)ncol[t];
    zoff[t] = (uint32_t)(ncol[t] >> 3);
  }
  uint32_t xoff[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i)  // rows past M start at the end of x: their loads read 0 and fetch nothing
    xoff[i] = 16 * i + r16 < M ? (uint32_t)(16 * i + r16) * (uint32_t)ldx * 2u + 64u * j
                                : (uint32_t)M * (uint32_t)ldx * 2u;
  const FastDiv gdiv((uint32_t)max(gsteps, 1));
  const uint32_t lds32 = (uint32_t)lds, ldz32 = (uint32_t)ldz;

  // two-step register ring: the loads of steps st + 1 and st + 2 are in flight while step st is computed
  struct Buf {
    uint4 w[T], x[MB][4];
    uint32_t s[T], z[T];
  };
  Buf bufa, bufb;
  auto ld16 = [](__amdgpu_buffer_rsrc_t r, uint32_t off) __attribute__((always_inline)) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
  };
  auto fetch = [&](int st, Buf& b) __attribute__((always_inline)) {
    const bool live = st < st1;
    const uint32_t g = gsteps > 0 ? gdiv.div((uint32_t)st) : 0u;
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) b.x[i][q] = ld16(rx, live ? xoff[i] + (uint32_t)st * 256u + 16u * q : xspan);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      b.s[t] = __builtin_amdgcn_raw_buffer_load_b16(rs, live ? (int)((g * lds32 + soff[t]) * 2u) : (int)sspan, 0, 0);
      b.z[t] = __builtin_amdgcn_raw_buffer_load_b32(rz, live ? (int)((g * ldz32 + zoff[t]) * 4u) : (int)zspan, 0, 0);
    }
#pragma unroll
    for (int t = 0; t < T; ++t) b.w[t] = ld16(rq, live ? woff[t] + (uint32_t)st * 64u : qspan);
  };

  f32x4_sk_t acc[T][MB];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[t][i] = f32x4_sk_t{0.f, 0.f, 0.f, 0.f};

  const uint4 ones = make_uint4(kOnes, kOnes, kOnes, kOnes);
  auto compute = [&](const Buf& b) __attribute__((always_inline)) {
    uint4 xa[MB][4];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) xa[i][q] = sk_xorder(b.x[i][q]);
    f32x4_sk_t xs[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      xs[i] = f32x4_sk_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) xs[i] = sk_mfma<XBF16>(xa[i][s], ones, xs[i]);
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const float sc = SBF16 ? bf16_bits_to_f32(b.s[t]) : f16_bits_to_f32((uint16_t)b.s[t]);
      const float zb = kB + (hasz ? (float)nibble(b.z[t], ncol[t] & 7) : 8.f);
      const uint32_t wd[4] = {b.w[t].x, b.w[t].y, b.w[t].z, b.w[t].w};
      f32x4_sk_t as[MB];
#pragma unroll
      for (int i = 0; i < MB; ++i) as[i] = f32x4_sk_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint4 bw = sk_wunpack<XBF16>(wd[s]);
#pragma unroll
        for (int i = 0; i < MB; ++i) as[i] = sk_mfma<XBF16>(xa[i][s], bw, as[i]);
      }
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          acc[t][i][e] = __builtin_fmaf(sc, __builtin_fmaf(-zb, xs[i][e], as[i][e]), acc[t][i][e]);
    }
  };

  // Steps past the slice are fetched through offsets past the operands' spans: the same load instructions (so the
  // waits before each compute count exactly the older loads) that read zeros and move no memory.
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

  // sum the KS slices of this channel block in slice order; wavefront ks then stores value indices ks, ks + KS, ...
  float* mine = red + (size_t)wave * NV * kWave;
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) mine[((t * MB + i) * 4 + e) * kWave + lane] = acc[t][i][e];
  __syncthreads();
  const float* base = red + (size_t)(wave - ks) * NV * kWave;
  for (int v = ks; v < NV; v += KS) {
    float sum = 0.f;
    for (int k2 = 0; k2 < KS; ++k2) sum += base[((size_t)k2 * NV + v) * kWave + lane];
    const int t = v / (MB * 4), i = (v / 4) % MB, e = v % 4;
    const int m = 16 * i + 4 * j + e, n = n0 + 16 * t + r16;
    if (m < M && n < N) {
      if (bias) sum += load_f(bias, bdt, n);
      y[(int64_t)m * ldy + n] = XBF16 ? f32_to_bf16_bits(sum) : f32_to_f16_bits(sum);
    }
  }
}

bool w4_skinny_ok(const void* x, int64_t ldx, const int32_t* qw, int64_t ldq, const int32_t* perm, int sdt,
                  int64_t lds, int64_t ldz, int M, int64_t N, int64_t K, int gs, int64_t G) {
  const int64_t k4g = 1LL << 32;  // byte offsets are 32-bit
  return M > 0 && M <= 64 && perm == nullptr && sdt != FG_F32 && (K % 128) == 0 && ((gs % 128) == 0 || G == 1) &&
         (ldx % 8) == 0 && (reinterpret_cast<uintptr_t>(x) % 16) == 0 && (ldq % 4) == 0 &&
         (reinterpret_cast<uintptr_t>(qw) % 16) == 0 && N * ldq * 4 < k4g && (int64_t)M * ldx * 2 < k4g &&
         G * lds * 2 < k4g && G * ldz * 4 < k4g &&  // scale / zero buffer spans in bytes
         group_div_exact(K, gs, G, 128);
}

// Launch shape, from a sweep over the Llama-3-8B shapes at M = 8..64: T tiles of 16 channels per wavefront, the largest
// of 4 / 2 / 1 (capped at 2 for M <= 32 and 1 for M <= 64 by the x registers) that leaves at least 3/4 of a channel
// block per CU; KS = 4 K slices for one m-tile with T <= 2, else 2 (more slices cost more than the parallelism they
// add); two channel blocks per workgroup from 1.5 blocks per CU.
void w4_skinny_plan(int M, int N, int K, int* mb, int* T, int* KS, int* BW) {
  const int cus = device_cus();
  const int b = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  int t = b == 1 ? 4 : (b == 2 ? 2 : 1);
  while (t > 1 && 4 * ((N + 16 * t - 1) / (16 * t)) < 3 * cus) t /= 2;
  const int nblk = (N + 16 * t - 1) / (16 * t);
  const int maxw = w4_skinny_max_threads(b, t) / kWave;
  int ks = (b == 1 && t <= 2) ? 4 : 2;
  // few rows over a long K: 8 slices (down at M = 1 / 4: 12.2 / 14.1 us against 14.1 / 14.8; 4 from M = 8 on)
  if (b == 1 && t <= 2 && M <= 4 && K >= 8192) ks = 8;
  ks = max(1, min(ks, K / 128));
  *mb = b; *T = t; *KS = ks; *BW = skinny_balance(nblk, ks, maxw, cus);
}

template <int MB, int T, bool XBF16, bool SBF16>
static hipError_t launch_skinny_t(const void* x, int64_t ldx, const int32_t* qw, int64_t ldq, const void* scales,
                                  int64_t lds, const int32_t* zeros, int64_t ldz, const void* bias, int bdt, void* y,
                                  int64_t ldy, int M, int N, int K, int gsteps, int KS, int BW, hipStream_t s) {
  const int nblk = (N + 16 * T - 1) / (16 * T);
  const int hasz = zeros != nullptr;
  const int32_t* zp = hasz ? zeros : qw;  // symmetric: a valid dummy word, ignored
  const size_t shm = (size_t)BW * KS * (T * MB * 4) * kWave * sizeof(float);
  auto kern = w4_skinny_kernel<MB, T, XBF16, SBF16>;
  if (shm > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
    if (e != hipSuccess) return e;
  }
  note_kernel("w4_skinny_kernel KS=%d", KS);
  hipLaunchKernelGGL(kern, dim3((nblk + BW - 1) / BW), dim3(kWave * BW * KS), shm, s,
                     static_cast<const uint16_t*>(x), ldx, qw, ldq, static_cast<const uint16_t*>(scales), lds, zp,
                     hasz ? ldz : 0, hasz, bias, bdt, static_cast<uint16_t*>(y), ldy, M, N, K, gsteps, KS);
  return hipGetLastError();
}

template <bool XBF16, bool SBF16>
static hipError_t launch_skinny_x(int mb, int T, const void* x, int64_t ldx, const int32_t* qw, int64_t ldq,
                                  const void* scales, int64_t lds, const int32_t* zeros, int64_t ldz,
                                  const void* bias, int bdt, void* y, int64_t ldy, int M, int N, int K, int gsteps,
                                  int KS, int BW, hipStream_t s) {
#define FG_SK(MB_, T_)                                                                                            \
  return launch_skinny_t<MB_, T_, XBF16, SBF16>(x, ldx, qw, ldq, scales, lds, zeros, ldz, bias, bdt, y, ldy, M, N, K, \
                                                gsteps, KS, BW, s)
  if (mb == 1) {
    if (T == 4) FG_SK(1, 4);
    if (T == 2) FG_SK(1, 2);
    FG_SK(1, 1);
  }
  if (mb == 2) {
    if (T == 2) FG_SK(2, 2);
    FG_SK(2, 1);
  }
  FG_SK(4, 1);
#undef FG_SK
}

hipError_t launch_w4_skinny(const void* x, int64_t ldx, bool xbf16, const int32_t* qw, int64_t ldq,
                            const void* scales, int sdt, int64_t lds, const int32_t* zeros, int64_t ldz,
                            const void* bias, int bdt, void* y, int64_t ldy, int M, int N, int K, int gs,
                            bool single_group, hipStream_t s) {
  int mb, T, KS, BW;
  w4_skinny_plan(M, N, K, &mb, &T, &KS, &BW);
  const int gsteps = single_group ? 0 : gs / 128;
  const bool sbf = sdt == FG_BF16;
  if (xbf16) {
    if (sbf) return launch_skinny_x<true, true>(mb, T, x, ldx, qw, ldq, scales, lds, zeros, ldz, bias, bdt, y, ldy, M, N, K, gsteps, KS, BW, s);
    return launch_skinny_x<true, false>(mb, T, x, ldx, qw, ldq, scales, lds, zeros, ldz, bias, bdt, y, ldy, M, N, K, gsteps, KS, BW, s);
  }
  if (sbf) return launch_skinny_x<false, true>(mb, T, x, ldx, qw, ldq, scales, lds, zeros, ldz, bias, bdt, y, ldy, M, N, K, gsteps, KS, BW, s);
  return launch_skinny_x<false, false>(mb, T, x, ldx, qw, ldq, scales, lds, zeros, ldz, bias, bdt, y, ldy, M, N, K, gsteps, KS, BW, s);
}

}  // namespace fg
