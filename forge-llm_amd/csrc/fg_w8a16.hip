// W8A16 (int8 weight-only): y[M,N] = x[M,K] @ dequant(W)[N,K]^T (+bias), W[n,k] = q[n,k] * s[g(k), n], q signed int8
// (symmetric, no zero-point), x bf16 / fp16.  The portable_row W8 layout: qweight int8 [N, K] row-major, scales [G, N].
//
// The policy (fg_w8a16_gemm) runs 17..64 rows, and 3..16 rows over N >= 16384 or K >= 8192, on the W4 LDS-ring kernel's
// int8 form (w8a16_ring_kernel, fg_w4_ring.hip); the skinny kernel below serves the other 3..64-row calls, and the
// prefill kernels (fg_w4_big.hip, fg_w4_pp.hip) the larger ones.
//
// Skinny kernel (M <= 64): the W4 skinny kernel's split-K structure (a wavefront owns T tiles of 16 channels and one K
// slice in 128-column steps; KS slices per workgroup summed in slice order through LDS; operands straight from global
// memory into registers by raw buffer loads, two steps ahead).  Lane l (row l % 16, lane group j = l / 16) loads the
// 32 weight bytes 32 j .. 32 j + 31 of its row per step and the 64 bytes of x over the same columns; MFMA k-step s
// takes weight bytes 8 s .. 8 s + 7 and x columns 32 j + 8 s .. + 7 in natural order.  The signed byte q becomes
// u = q ^ 0x80 = q + 128 (0..255):
//   fp16 x: one exact fp16 per byte, 0x6400 | u = 1024 + u (byte-permutes against the magic exponent byte), one MFMA
//           per k-step:  sum x q = A - 1152 sum x;
//   bf16 x: u itself (0..255) is exact in bf16: v_cvt_f32_ubyte{b} and a packed fp32 -> bf16 conversion, one MFMA
//           per k-step:  sum x q = A - 128 sum x.
// The row sums of x come from one MFMA per k-step against all-ones (in the accumulator layout); each step lies in one
// group (group size a multiple of 128, or one group), so after a step  acc += s[n, g] * (that expression).
//
// Decode GEMV (M <= 4): the W4 split GEMV's structure (16 weight bytes per lane and row, K slices summed in order
// through LDS) with the bytes turned into floats and multiplied in fp32, where 15 of the skinny kernel's 16 MFMA rows
// would be empty.
//
// Generic kernel: any shape, stride, alignment, group size and scale dtype; one wavefront per output channel and up
// to 4 rows of x, lanes stride over K, fp32 products q * s * x in the oracle's order of dequantise-then-multiply.
#include "fg_device.h"

namespace fg {

typedef __bf16 bf16x8_w8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_w8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_w8_t __attribute__((ext_vector_type(4)));

template <bool XBF16>
__device__ __forceinline__ f32x4_w8_t w8_mfma(uint4 a, uint4 b, f32x4_w8_t c) {
  if constexpr (XBF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_w8_t, a),
                                                   __builtin_bit_cast(bf16x8_w8_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_w8_t, a),
                                                  __builtin_bit_cast(f16x8_w8_t, b), c, 0, 0, 0);
  }
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t w8a_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ uint4 w8a_ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

constexpr int w8a16_max_threads(int mb, int t) { return mb * t >= 2 ? 512 : 1024; }

template <int MB, int T, bool XBF16, bool SBF16>
__global__ void __launch_bounds__(w8a16_max_threads(MB, T)) w8a16_skinny_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const int8_t* __restrict__ qw, int64_t ldq,
    const uint16_t* __restrict__ scales, int64_t lds, const void* __restrict__ bias, int bdt,
    uint16_t* __restrict__ y, int64_t ldy, int M, int N, int K, int gsteps, int KS) {
  constexpr uint32_t kOnes = XBF16 ? 0x3F803F80u : 0x3C003C00u;
  constexpr float kCorr = XBF16 ? 128.f : 1152.f;  // u = q + 128 (bf16) / 1024 + u = q + 1152 (fp16)
  constexpr int NV = T * MB * 4;
  extern __shared__ __align__(16) float red[];  // [waves][NV][64]
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int BW = (int)(blockDim.x / kWave) / KS;
  const int ks = wave % KS, nb = blockIdx.x * BW + wave / KS;
  const int n0 = nb * 16 * T;
  const int nsteps = K / 128;
  const int st0 = (int)((int64_t)ks * nsteps / KS), st1 = (int)((int64_t)(ks + 1) * nsteps / KS);
  const int r16 = lane & 15, j = lane >> 4;
  const int G = gsteps > 0 ? (nsteps + gsteps - 1) / gsteps : 1;

  const uint32_t qspan = (uint32_t)N * (uint32_t)ldq, xspan = (uint32_t)M * (uint32_t)ldx * 2u;
  const uint32_t sspan = (uint32_t)G * (uint32_t)lds * 2u;
  const __amdgpu_buffer_rsrc_t rq = w8a_rsrc(qw, qspan);
  const __amdgpu_buffer_rsrc_t rx = w8a_rsrc(x, xspan);
  const __amdgpu_buffer_rsrc_t rs = w8a_rsrc(scales, sspan);
  uint32_t woff[T], soff[T];
  int ncol[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    ncol[t] = min(n0 + 16 * t + r16, N - 1);
    woff[t] = (uint32_t)ncol[t] * (uint32_t)ldq + 32u * j;
    soff[t] = (uint32_t)ncol[t];
  }
  uint32_t xoff[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i)  // rows past M start at the end of x: their loads read 0 and fetch nothing
    xoff[i] = 16 * i + r16 < M ? (uint32_t)(16 * i + r16) * (uint32_t)ldx * 2u + 64u * j
                                : (uint32_t)M * (uint32_t)ldx * 2u;
  const FastDiv gdiv((uint32_t)max(gsteps, 1));
  const uint32_t lds32 = (uint32_t)lds;

  struct Buf {
    uint4 w[T][2], x[MB][4];
    uint32_t s[T];
  };
  Buf bufa, bufb;
  auto fetch = [&](int st, Buf& b) __attribute__((always_inline)) {
    const bool live = st < st1;
    const uint32_t g = gsteps > 0 ? gdiv.div((uint32_t)st) : 0u;
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) b.x[i][q] = w8a_ld16(rx, live ? xoff[i] + (uint32_t)st * 256u + 16u * q : xspan);
#pragma unroll
    for (int t = 0; t < T; ++t)
      b.s[t] = __builtin_amdgcn_raw_buffer_load_b16(rs, live ? (int)((g * lds32 + soff[t]) * 2u) : (int)sspan, 0, 0);
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int h = 0; h < 2; ++h) b.w[t][h] = w8a_ld16(rq, live ? woff[t] + (uint32_t)st * 128u + 16u * h : qspan);
  };

  f32x4_w8_t acc[T][MB];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[t][i] = f32x4_w8_t{0.f, 0.f, 0.f, 0.f};
  const uint4 ones = make_uint4(kOnes, kOnes, kOnes, kOnes);

  auto compute = [&](const Buf& b) __attribute__((always_inline)) {
    f32x4_w8_t xs[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      xs[i] = f32x4_w8_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) xs[i] = w8_mfma<XBF16>(b.x[i][s], ones, xs[i]);
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const float sc = SBF16 ? bf16_bits_to_f32(b.s[t]) : f16_bits_to_f32((uint16_t)b.s[t]);
      const uint32_t wd[8] = {b.w[t][0].x, b.w[t][0].y, b.w[t][0].z, b.w[t][0].w,
                              b.w[t][1].x, b.w[t][1].y, b.w[t][1].z, b.w[t][1].w};
      f32x4_w8_t a1[MB];
#pragma unroll
      for (int i = 0; i < MB; ++i) a1[i] = f32x4_w8_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint32_t u0 = wd[2 * s] ^ 0x80808080u, u1 = wd[2 * s + 1] ^ 0x80808080u;  // q + 128 per byte
        if constexpr (XBF16) {
          // u (0..255) is exact in bf16: v_cvt_f32_ubyte{b} then a packed conversion, one MFMA per k-step
          const uint4 bu = make_uint4(w8a_bf16_pair(u0, 0), w8a_bf16_pair(u0, 1), w8a_bf16_pair(u1, 0),
                                      w8a_bf16_pair(u1, 1));
#pragma unroll
          for (int i = 0; i < MB; ++i) a1[i] = w8_mfma<XBF16>(b.x[i][s], bu, a1[i]);
        } else {
          const uint4 bu = make_uint4(w8a_pair_lo(0x64646464u, u0), w8a_pair_hi(0x64646464u, u0),
                                      w8a_pair_lo(0x64646464u, u1), w8a_pair_hi(0x64646464u, u1));
#pragma unroll
          for (int i = 0; i < MB; ++i) a1[i] = w8_mfma<XBF16>(b.x[i][s], bu, a1[i]);
        }
      }
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[t][i][e] = __builtin_fmaf(sc, __builtin_fmaf(-kCorr, xs[i][e], a1[i][e]), acc[t][i][e]);
        }
    }
  };

  // Steps past the slice are fetched through offsets past the operands' spans: same loads, no memory moved.
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

// ------------------------------------------------------------------------------------------ decode GEMV (M <= 4)
// The W4 split GEMV's structure for int8 weights: a wavefront owns R consecutive output channels and one K slice of at
// most S 16-column chunks per lane (chunk c = slice start + lane + 64 i: 16 weight bytes of each row, 32 bytes of each
// row of x); the KS slices of a channel block are the KS wavefronts of one workgroup, summed in slice order through LDS
// at the end (no workspace, deterministic).  Per chunk a lane turns its 16 x values into fp32 once, with their sum, and
// reuses them for all R channels: byte b of u = q ^ 0x80 = q + 128 becomes a float by v_cvt_f32_ubyte{b} and meets x
// in an fma, so d = sum x u - 128 sum x = sum x q with every product exact in fp32; then acc += s[g(c), n] * d.  All
// loads are raw buffer loads issued unconditionally in the order of first use (x, scales, weights); a chunk past the
// slice reads past the operands' spans (0, no traffic) and adds exactly 0.
struct W8GemvArgs {
  int KC;         // 16-column chunks of K
  int cps;        // chunks per K slice
  int gs16;       // group size / 16, 0 for one group per row
  uint32_t gmul;  // group of chunk c = umulhi(c, gmul) when gs16 > 1 (floor((2^32 - 1) / gs16) + 1)
  uint32_t qbytes, xbytes, sbytes;
};

constexpr int w8a16_gemv_max_threads(int mt) { return mt == 4 ? 512 : 1024; }

template <int MT, int S, int R, bool XBF16, bool SBF16>
__global__ void __launch_bounds__(w8a16_gemv_max_threads(MT)) w8a16_gemv_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const int8_t* __restrict__ qw, int64_t ldq,
    const uint16_t* __restrict__ scales, int64_t lds, const void* __restrict__ bias, int bdt,
    uint16_t* __restrict__ y, int64_t ldy, int M, int N, W8GemvArgs a) {
  static_assert(R * MT == 4 || R * MT == 8 || R * MT == 16, "rows x batch must be 4, 8 or 16");
  static_assert(R == 4 || R == 8, "4 or 8 channels per wavefront");
  __shared__ float red[16][R * MT];
  const int lane = threadIdx.x & (kWave - 1);
  const int wb = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // channel block within the workgroup
  const int ks = __builtin_amdgcn_readfirstlane(threadIdx.y);         // K slice
  const int BW = (int)(blockDim.x / kWave), KS = (int)blockDim.y;
  const int n0 = (blockIdx.x * BW + wb) * R;
  const int nr = min(n0, N - R);  // first channel read (blocks past the end re-read the last block)
  const int c0 = ks * a.cps, c1 = min(c0 + a.cps, a.KC);
  const __amdgpu_buffer_rsrc_t rq = buf_rsrc(qw, a.qbytes), rx = buf_rsrc(x, a.xbytes), rs = buf_rsrc(scales, a.sbytes);

  uint32_t xo[S], wo[S], so[S];
#pragma unroll
  for (int i = 0; i < S; ++i) {
    const int c = c0 + lane + kWave * i;
    const bool ok = c < c1;
    const uint32_t g = a.gs16 > 1 ? __umulhi((uint32_t)c, a.gmul) : (a.gs16 == 1 ? (uint32_t)c : 0u);
    xo[i] = ok ? (uint32_t)c * 32u : a.xbytes;
    wo[i] = ok ? (uint32_t)c * 16u : a.qbytes;
    so[i] = ok ? g * (uint32_t)lds * 2u : a.sbytes;
  }
  uint4 xv[MT][S][2];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int i = 0; i < S; ++i)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        xv[m][i][h] = buf_ld16(rx, xo[i] + 16u * h, (uint32_t)min(m, M - 1) * (uint32_t)ldx * 2u);
  uint32_t sraw[S][R / 2];
#pragma unroll
  for (int i = 0; i < S; ++i) {
    if constexpr (R == 8) {
      const uint4 t = buf_ld16(rs, so[i], (uint32_t)nr * 2u);
      sraw[i][0] = t.x; sraw[i][1] = t.y; sraw[i][2] = t.z; sraw[i][3] = t.w;
    } else {
      const uint2 t = buf_ld8(rs, so[i], (uint32_t)nr * 2u);
      sraw[i][0] = t.x; sraw[i][1] = t.y;
    }
  }
  uint4 wv[R][S];
  const uint32_t ldqb = (uint32_t)ldq;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int i = 0; i < S; ++i) wv[r][i] = buf_ld16_nt(rq, wo[i], ((uint32_t)nr + (uint32_t)r) * ldqb);

  float acc[R * MT];
#pragma unroll
  for (int v = 0; v < R * MT; ++v) acc[v] = 0.f;
#pragma unroll
  for (int i = 0; i < S; ++i) {
    float xf[MT][16], xs[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const uint32_t wd[8] = {xv[m][i][0].x, xv[m][i][0].y, xv[m][i][0].z, xv[m][i][0].w,
                              xv[m][i][1].x, xv[m][i][1].y, xv[m][i][1].z, xv[m][i][1].w};
      float sum = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        xf[m][2 * e] = XBF16 ? __uint_as_float(wd[e] << 16) : f16_bits_to_f32((uint16_t)wd[e]);
        xf[m][2 * e + 1] = XBF16 ? __uint_as_float(wd[e] & 0xffff0000u) : f16_bits_to_f32((uint16_t)(wd[e] >> 16));
        sum += xf[m][2 * e];
        sum += xf[m][2 * e + 1];
      }
      xs[m] = sum;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t sb = (r & 1) ? sraw[i][r >> 1] >> 16 : sraw[i][r >> 1] & 0xffffu;
      const float sc = SBF16 ? bf16_bits_to_f32(sb) : f16_bits_to_f32((uint16_t)sb);
      float d[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m) d[m] = -128.f * xs[m];
      const uint32_t wq[4] = {wv[r][i].x, wv[r][i].y, wv[r][i].z, wv[r][i].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t u = wq[q] ^ 0x80808080u;  // q + 128 per byte
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const float fu = (float)((u >> (8 * b)) & 0xffu);
#pragma unroll
          for (int m = 0; m < MT; ++m) d[m] = __builtin_fmaf(xf[m][4 * q + b], fu, d[m]);
        }
      }
#pragma unroll
      for (int m = 0; m < MT; ++m) acc[r * MT + m] = __builtin_fmaf(sc, d[m], acc[r * MT + m]);
    }
  }
  const float tot = wave_transpose_sum<R * MT>(acc, lane);
  constexpr int span = kWave / (R * MT);
  auto store = [&](int idx, float v) {
    const int r = idx / MT, m = idx - (idx / MT) * MT;
    if (m < M && n0 + r < N) {
      if (bias) v += load_f(bias, bdt, n0 + r);
      y[(int64_t)m * ldy + n0 + r] = XBF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
    }
  };
  if (KS == 1) {
    if ((lane % span) == 0) store(lane / span, tot);
  } else {
    if ((lane % span) == 0) red[ks * BW + wb][lane / span] = tot;
    __syncthreads();
    if (ks == 0 && lane < R * MT) {  // the K slices of this block, summed in slice order
      float v = 0.f;
      for (int k2 = 0; k2 < KS; ++k2) v += red[k2 * BW + wb][lane];
      store(lane, v);
    }
  }
}

// Generic: one wavefront per (channel n, up to 4 rows of x); fixed-order lane and cross-lane sums.
__global__ void __launch_bounds__(256) w8a16_generic_kernel(const void* __restrict__ x, int64_t ldx, int xdt,
                                                            const int8_t* __restrict__ qw, int64_t ldq,
                                                            const void* __restrict__ scales, int sdt, int64_t lds,
                                                            const void* __restrict__ bias, int bdt, void* __restrict__ y,
                                                            int64_t ldy, int M, int N, int K, int gs) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t item = (int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  const int mblocks = (M + 3) / 4;
  if (item >= (int64_t)N * mblocks) return;  // whole wavefronts leave together
  const int n = (int)(item / mblocks), m0 = (int)(item % mblocks) * 4;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int k = lane; k < K; k += kWave) {
    const float w = (float)qw[(int64_t)n * ldq + k] * load_f(scales, sdt, (int64_t)(k / gs) * lds + n);
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (m0 + r < M) acc[r] = __builtin_fmaf(load_f(x, xdt, (int64_t)(m0 + r) * ldx + k), w, acc[r]);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float v = wave_sum(acc[r]);
    if (lane == 0 && m0 + r < M) store_f(y, xdt, (int64_t)(m0 + r) * ldy + n, bias ? v + load_f(bias, bdt, n) : v);
  }
}

bool w8a16_skinny_ok(const void* x, int64_t ldx, const int8_t* qw, int64_t ldq, int sdt, int64_t lds, int64_t M,
                     int64_t N, int64_t K, int gs, int64_t G) {
  const int64_t k4g = 1LL << 32;
  return M > 0 && M <= 64 && sdt != FG_F32 && (K % 128) == 0 && ((gs % 128) == 0 || G == 1) && (ldx % 8) == 0 &&
         (reinterpret_cast<uintptr_t>(x) % 16) == 0 && (ldq % 16) == 0 &&
         (reinterpret_cast<uintptr_t>(qw) % 16) == 0 && N * ldq < k4g && M * ldx * 2 < k4g && G * lds * 2 < k4g &&
         group_div_exact(K, gs, G, 128);
}

// Same shape rules as the W4 skinny kernel (the weight bytes per step double, the register budget is the same):
// T tiles (4 / 2 / 1, capped by the rows of x) leaving at least 3/4 of a channel block per CU, 2-4 K slices, channel
// blocks per workgroup chosen so that workgroups spread evenly over the CUs.
static void w8a16_plan(int M, int N, int K, int* mb, int* T, int* KS, int* BW) {
  const int cus = device_cus();
  const int b = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  int t = b == 1 ? 4 : (b == 2 ? 2 : 1);
  while (t > 1 && 4 * ((N + 16 * t - 1) / (16 * t)) < 3 * cus) t /= 2;
  const int nblk = (N + 16 * t - 1) / (16 * t);
  const int maxw = w8a16_max_threads(b, t) / kWave;
  int ks = (b == 1 && t <= 2) ? 4 : 2;
  // few rows over a long K: 8 slices (down at M = 1: 15.8 against 16.9 us; 4 stay ahead from M = 8)
  if (b == 1 && t <= 2 && M <= 4 && K >= 8192) ks = 8;
  ks = max(1, min(ks, K / 128));
  *mb = b; *T = t; *KS = ks; *BW = skinny_balance(nblk, ks, maxw, cus);
}

template <int MB, int T, bool XBF16, bool SBF16>
static hipError_t launch_w8a16_skinny_t(const void* x, int64_t ldx, const int8_t* qw, int64_t ldq,
                                        const void* scales, int64_t lds, const void* bias, int bdt, void* y,
                                        int64_t ldy, int M, int N, int K, int gsteps, int KS, int BW, hipStream_t s) {
  const int nblk = (N + 16 * T - 1) / (16 * T);
  const size_t shm = (size_t)BW * KS * (T * MB * 4) * kWave * sizeof(float);
  auto kern = w8a16_skinny_kernel<MB, T, XBF16, SBF16>;
  if (shm > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
    if (e != hipSuccess) return e;
  }
  note_kernel("w8a16_skinny_kernel KS=%d", KS);
  hipLaunchKernelGGL(kern, dim3((nblk + BW - 1) / BW), dim3(kWave * BW * KS), shm, s,
                     static_cast<const uint16_t*>(x), ldx, qw, ldq, static_cast<const uint16_t*>(scales), lds, bias,
                     bdt, static_cast<uint16_t*>(y), ldy, M, N, K, gsteps, KS);
  return hipGetLastError();
}

template <bool XBF16, bool SBF16>
static hipError_t launch_w8a16_skinny_x(int mb, int T, const void* x, int64_t ldx, const int8_t* qw, int64_t ldq,
                                        const void* scales, int64_t lds, const void* bias, int bdt, void* y,
                                        int64_t ldy, int M, int N, int K, int gsteps, int KS, int BW, hipStream_t s) {
#define FG_W8A(MB_, T_)                                                                                      \
  return launch_w8a16_skinny_t<MB_, T_, XBF16, SBF16>(x, ldx, qw, ldq, scales, lds, bias, bdt, y, ldy, M, N, K, \
                                                      gsteps, KS, BW, s)
  if (mb == 1) {
    if (T == 4) FG_W8A(1, 4);
    if (T == 2) FG_W8A(1, 2);
    FG_W8A(1, 1);
  }
  if (mb == 2) {
    if (T == 2) FG_W8A(2, 2);
    FG_W8A(2, 1);
  }
  FG_W8A(4, 1);
#undef FG_W8A
}

hipError_t launch_w8a16_skinny(const void* x, int64_t ldx, bool xbf16, const int8_t* qw, int64_t ldq,
                               const void* scales, int sdt, int64_t lds, const void* bias, int bdt, void* y,
                               int64_t ldy, int M, int N, int K, int gs, bool single_group, hipStream_t s) {
  int mb, T, KS, BW;
  w8a16_plan(M, N, K, &mb, &T, &KS, &BW);
  const int gsteps = single_group ? 0 : gs / 128;
  const bool sbf = sdt == FG_BF16;
  if (xbf16) {
    if (sbf) return launch_w8a16_skinny_x<true, true>(mb, T, x, ldx, qw, ldq, scales, lds, bias, bdt, y, ldy, M, N, K, gsteps, KS, BW, s);
    return launch_w8a16_skinny_x<true, false>(mb, T, x, ldx, qw, ldq, scales, lds, bias, bdt, y, ldy, M, N, K, gsteps, KS, BW, s);
  }
  if (sbf) return launch_w8a16_skinny_x<false, true>(mb, T, x, ldx, qw, ldq, scales, lds, bias, bdt, y, ldy, M, N, K, gsteps, KS, BW, s);
  return launch_w8a16_skinny_x<false, false>(mb, T, x, ldx, qw, ldq, scales, lds, bias, bdt, y, ldy, M, N, K, gsteps, KS, BW, s);
}

// Decode GEMV launch shape: R = 8 channels per wavefront (4 for four rows of x); S = 1 chunk per lane while K <= 4096
// (KS = 4 slices of 1024 columns), else 4 (2 with four rows of x); one channel block per workgroup, i.e. a workgroup is
// the KS wavefronts of one block.  Graph replays over a 1.2 GB ring, M = 1, us (this shape / 16-wavefront workgroups):
// gate+up 19.2 / 23.9 (6.1 TB/s), down (S = 4, 4 slices) 11.6 / 11.9, o_proj 4.9 / 5.6, qkv 6.1 / 6.5: small
// workgroups retire and refill independently.
struct W8GemvPlan {
  int mt, S, R, KS, BW;
};
static bool w8a16_gemv_plan(int M, int N, int K, W8GemvPlan* p) {
  const int mt = M <= 1 ? 1 : (M <= 2 ? 2 : 4);
  const int KC = K / 16, R = mt == 4 ? 4 : 8;
  // one chunk per lane while the K slices fit one workgroup (1-2 rows: K <= 16384), else 4 (2 for four rows).  Graph
  // replays, us, one chunk / four: K = 8192, N = 10240 / 8192 / 57344 15.6 / 12.9 / 74.8 against 18.9 / 16.2 / 83.9;
  // K = 14336, N = 4096 12.0 / 12.5 (M = 1 / 2) against 12.4 / 14.3; K = 28672 (28 slices) stays on four
  const int S = KC <= 4 * kWave || (mt <= 2 && KC <= 16 * kWave) ? 1 : (mt == 4 ? 2 : 4);
  const int ks = (KC + kWave * S - 1) / (kWave * S);
  const int maxw = w8a16_gemv_max_threads(mt) / kWave;
  if (ks > maxw || N % R != 0) return false;
  *p = W8GemvPlan{mt, S, R, ks, 1};
  return true;
}

bool w8a16_gemv_ok(const void* x, int64_t ldx, const int8_t* qw, int64_t ldq, const void* scales, int sdt,
                   int64_t lds, int64_t M, int64_t N, int64_t K, int gs, int64_t G) {
  const int64_t k4g = 1LL << 32;
  W8GemvPlan p;
  return M > 0 && M <= 4 && sdt != FG_F32 && (K % 16) == 0 && ((gs % 16) == 0 || G == 1) && (ldx % 8) == 0 &&
         (reinterpret_cast<uintptr_t>(x) % 16) == 0 && (ldq % 16) == 0 &&
         (reinterpret_cast<uintptr_t>(qw) % 16) == 0 && (lds % 8) == 0 &&
         (reinterpret_cast<uintptr_t>(scales) % 16) == 0 && N * ldq < k4g && M * ldx * 2 < k4g &&
         G * lds * 2 < k4g && K < k4g / 32 && group_div_exact(K, gs, G, 16) && w8a16_gemv_plan((int)M, (int)N, (int)K, &p);
}

template <int MT, int S, int R, bool XBF16, bool SBF16>
static hipError_t launch_w8a16_gemv_t(const W8GemvPlan& p, const void* x, int64_t ldx, const int8_t* qw, int64_t ldq,
                                      const void* scales, int64_t lds, const void* bias, int bdt, void* y,
                                      int64_t ldy, int M, int N, int K, int gs16, int64_t G, hipStream_t s) {
  W8GemvArgs a;
  a.KC = K / 16;
  a.cps = (a.KC + p.KS - 1) / p.KS;
  a.gs16 = gs16;
  a.gmul = gs16 > 1 ? 0xffffffffu / (uint32_t)gs16 + 1u : 0u;
  a.qbytes = (uint32_t)((int64_t)N * ldq);
  a.xbytes = (uint32_t)((int64_t)M * ldx * 2);
  a.sbytes = (uint32_t)(G * lds * 2);
  const int nblk = N / R;
  note_kernel("w8a16_gemv_kernel<%d,%d,%d>", MT, S, R);
  hipLaunchKernelGGL((w8a16_gemv_kernel<MT, S, R, XBF16, SBF16>), dim3((nblk + p.BW - 1) / p.BW),
                     dim3(kWave * p.BW, p.KS), 0, s, static_cast<const uint16_t*>(x), ldx, qw, ldq,
                     static_cast<const uint16_t*>(scales), lds, bias, bdt, static_cast<uint16_t*>(y), ldy, M, N, a);
  return hipGetLastError();
}

template <bool XBF16, bool SBF16>
static hipError_t launch_w8a16_gemv_x(const W8GemvPlan& p, const void* x, int64_t ldx, const int8_t* qw, int64_t ldq,
                                      const void* scales, int64_t lds, const void* bias, int bdt, void* y,
                                      int64_t ldy, int M, int N, int K, int gs16, int64_t G, hipStream_t s) {
#define FG_W8G(MT_, S_, R_)                                                                                       \
  return launch_w8a16_gemv_t<MT_, S_, R_, XBF16, SBF16>(p, x, ldx, qw, ldq, scales, lds, bias, bdt, y, ldy, M, N, \
                                                        K, gs16, G, s)
  if (p.mt == 1) {
    if (p.S == 4) FG_W8G(1, 4, 8);
    FG_W8G(1, 1, 8);
  }
  if (p.mt == 2) {
    if (p.S == 4) FG_W8G(2, 4, 8);
    FG_W8G(2, 1, 8);
  }
  if (p.S == 2) FG_W8G(4, 2, 4);
  FG_W8G(4, 1, 4);
#undef FG_W8G
}

hipError_t launch_w8a16_gemv(const void* x, int64_t ldx, bool xbf16, const int8_t* qw, int64_t ldq,
                             const void* scales, int sdt, int64_t lds, const void* bias, int bdt, void* y,
                             int64_t ldy, int M, int N, int K, int gs, bool single_group, int64_t G, hipStream_t s) {
  W8GemvPlan p;
  if (!w8a16_gemv_plan(M, N, K, &p)) return hipErrorInvalidValue;
  const int gs16 = single_group ? 0 : gs / 16;
  const bool sbf = sdt == FG_BF16;
  if (xbf16) {
    if (sbf) return launch_w8a16_gemv_x<true, true>(p, x, ldx, qw, ldq, scales, lds, bias, bdt, y, ldy, M, N, K, gs16, G, s);
    return launch_w8a16_gemv_x<true, false>(p, x, ldx, qw, ldq, scales, lds, bias, bdt, y, ldy, M, N, K, gs16, G, s);
  }
  if (sbf) return launch_w8a16_gemv_x<false, true>(p, x, ldx, qw, ldq, scales, lds, bias, bdt, y, ldy, M, N, K, gs16, G, s);
  return launch_w8a16_gemv_x<false, false>(p, x, ldx, qw, ldq, scales, lds, bias, bdt, y, ldy, M, N, K, gs16, G, s);
}

hipError_t launch_w8a16_generic(const void* x, int64_t ldx, int xdt, const int8_t* qw, int64_t ldq,
                                const void* scales, int sdt, int64_t lds, const void* bias, int bdt, void* y,
                                int64_t ldy, int M, int N, int K, int gs, hipStream_t s) {
  const int64_t waves = (int64_t)N * ((M + 3) / 4);
  note_kernel("w8a16_generic_kernel");
  hipLaunchKernelGGL(w8a16_generic_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, x, ldx, xdt, qw, ldq,
                     scales, sdt, lds, bias, bdt, y, ldy, M, N, K, gs);
  return hipGetLastError();
}

}  // namespace fg
