// W4A16 kernels for gfx950: decode GEMV (M <= 4), generic per-element kernel, dense dequantisation.
//
// Packed layout (Forge portable_row, forge/kernels/layouts/w4.py:15-17): qweight int32 [N, ldq], nibble j of word w
// holds q[n, 8w+j]; scales [G, lds]; zeros int32 [G, ldz] with 8 channels per word (NULL = symmetric, zero-point 8).
//
// Decode GEMV design (HBM-bound: >96% of the bytes are qweight):
//  * one wavefront owns R consecutive output channels and walks the whole K range; lane l reads the 16-byte chunk
//    c = l + 64*i of each row, so every global load instruction of a wave covers 1 KiB of contiguous qweight;
//  * x is staged once per workgroup into LDS, already arranged as bf16/fp16 pairs (x[8w+j], x[8w+j+4]) that line up
//    with the nibble pairs (q_j, q_{j+4}) = bits {4j..4j+3, 16+4j..16+4j+3} of a word, plus the fp32 sum of each
//    32-column chunk;
//  * nibbles become 16-bit floats with one AND-OR against a magic exponent: bf16 0x4300|q == 128+q exactly (fp16:
//    0x6400|q == 1024+q), and v_dot2_f32_{bf16,f16} multiplies them with the x pairs into an fp32 accumulator;
//  * the offset is removed once per chunk: sum_k x_k (q_k - z) = sum_k x_k (B+q_k) - (B+z) * sum_k x_k (B = 128 or
//    1024), and the group scale multiplies the chunk's partial sum (a chunk never straddles a group);
//  * the 64 lane partials of each channel are summed with cross-lane shuffles; no split-K, no workspace, one launch.
#include "fg_device.h"

namespace fg {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

template <bool XBF16>
__device__ __forceinline__ float dot2_acc(uint32_t xpair, uint32_t wpair, float acc) {
  if constexpr (XBF16) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, xpair), __builtin_bit_cast(bf16x2_t, wpair),
                                           acc, false);
  } else {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, xpair), __builtin_bit_cast(f16x2_t, wpair), acc, false);
  }
}

template <bool XBF16>
__device__ __forceinline__ float x_to_f32(uint32_t bits16) {
  return XBF16 ? bf16_bits_to_f32(bits16) : f16_bits_to_f32((uint16_t)bits16);
}

// Stage x[0:MT, 0:K] (gathered through perm when given) into LDS as pair units and per-chunk sums.
//   xq: uint4 units indexed ((m*4 + i) * KC + c) = pairs of word 4c+i of row m;  xs: float [MT*KC]
template <int MT, bool XBF16>
__device__ __forceinline__ void stage_x(const uint16_t* __restrict__ x, int64_t ldx, const int32_t* __restrict__ perm,
                                        int M, int K, int KW, int KC, uint4* xq, float* xs) {
  const int nunits = MT * 4 * KC;
  for (int u = threadIdx.x; u < nunits; u += blockDim.x) {
    const int m = u / (4 * KC);
    const int rem = u - m * 4 * KC;
    const int i = rem / KC;
    const int c = rem - i * KC;
    const int w = 4 * c + i;
    uint32_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = 0;
    if (m < M && w < KW) {
      const uint16_t* xr = x + (int64_t)m * ldx;
      const int k0 = 8 * w;
      if (perm == nullptr && k0 + 8 <= K && ((reinterpret_cast<uintptr_t>(xr + k0) & 15) == 0)) {
        uint4 t = *reinterpret_cast<const uint4*>(xr + k0);
        v[0] = t.x & 0xffffu; v[1] = t.x >> 16; v[2] = t.y & 0xffffu; v[3] = t.y >> 16;
        v[4] = t.z & 0xffffu; v[5] = t.z >> 16; v[6] = t.w & 0xffffu; v[7] = t.w >> 16;
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int k = k0 + j;
          if (k < K) v[j] = xr[perm ? perm[k] : k];
        }
      }
    }
    uint4 p;
    p.x = v[0] | (v[4] << 16);
    p.y = v[1] | (v[5] << 16);
    p.z = v[2] | (v[6] << 16);
    p.w = v[3] | (v[7] << 16);
    xq[u] = p;
  }
  __syncthreads();
  for (int t = threadIdx.x; t < MT * KC; t += blockDim.x) {
    const int m = t / KC;
    const int c = t - m * KC;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 p = xq[(m * 4 + i) * KC + c];
      const uint32_t a[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) s += x_to_f32<XBF16>(a[j] & 0xffffu) + x_to_f32<XBF16>(a[j] >> 16);
    }
    xs[t] = s;
  }
  __syncthreads();
}

// y[M,N] = x[M,K] @ dequant(W)^T (+bias), M <= MT, group size a multiple of 32 (or one group per row).
// Requires ldq % 4 == 0 and a 16-byte aligned qweight base (16-byte chunk loads).
template <int MT, int R, bool XBF16>
__global__ void __launch_bounds__(256) w4_gemv_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const int32_t* __restrict__ qw, int64_t ldq,
    const void* __restrict__ scales, int sdt, int64_t lds, const int32_t* __restrict__ zeros, int64_t ldz,
    const int32_t* __restrict__ perm, const void* __restrict__ bias, int bdt, uint16_t* __restrict__ y, int64_t ldy,
    int M, int N, int K, int gs) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int KW = (K + 7) / 8;
  const int KC = (KW + 3) / 4;
  uint4* xq = reinterpret_cast<uint4*>(smem);
  float* xs = reinterpret_cast<float*>(smem + (size_t)MT * 4 * KC * 16);
  stage_x<MT, XBF16>(x, ldx, perm, M, K, KW, KC, xq, xs);

  constexpr uint32_t kMagic = XBF16 ? 0x43004300u : 0x64006400u;
  constexpr float kBias = XBF16 ? 128.f : 1024.f;
  const int lane = threadIdx.x & (kWave - 1);
  const int waves = blockDim.x / kWave;
  const int NB = (N + R - 1) / R;
  const int64_t ldq4 = ldq / 4;
  const uint4* __restrict__ qw4 = reinterpret_cast<const uint4*>(qw);

  for (int rb = blockIdx.x * waves + (int)(threadIdx.x / kWave); rb < NB; rb += gridDim.x * waves) {
    const int n0 = rb * R;
    int nr[R];
#pragma unroll
    for (int r = 0; r < R; ++r) nr[r] = min(n0 + r, N - 1);
    float acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < MT; ++m) acc[r][m] = 0.f;

    for (int c = lane; c < KC; c += kWave) {
      uint4 wv[R];
#pragma unroll
      for (int r = 0; r < R; ++r) wv[r] = load16_stream(qw4 + nr[r] * ldq4 + c);
      const int g = (32 * c) / gs;
      float s[R], zb[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        s[r] = load_f(scales, sdt, (int64_t)g * lds + nr[r]);
        const uint32_t z = zeros ? nibble((uint32_t)zeros[(int64_t)g * ldz + nr[r] / 8], nr[r] & 7) : 8u;
        zb[r] = kBias + (float)z;
      }
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        uint4 xu[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) xu[i] = xq[(m * 4 + i) * KC + c];
        const float xsum = xs[m * KC + c];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          float d = -zb[r] * xsum;
          const uint32_t w4[4] = {wv[r].x, wv[r].y, wv[r].z, wv[r].w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t xw[4] = {xu[i].x, xu[i].y, xu[i].z, xu[i].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const uint32_t pair = ((w4[i] >> (4 * j)) & 0x000F000Fu) | kMagic;
              d = dot2_acc<XBF16>(xw[j], pair, d);
            }
          }
          acc[r][m] = __builtin_fmaf(s[r], d, acc[r][m]);
        }
      }
    }
    float out = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float v = wave_sum(acc[r][m]);
        if (lane == r * MT + m) out = v;
      }
    if (lane < R * MT) {
      const int r = lane / MT, m = lane - (lane / MT) * MT;
      const int n = n0 + r;
      if (n < N && m < M) {
        if (bias) out += load_f(bias, bdt, n);
        y[(int64_t)m * ldy + n] = XBF16 ? f32_to_bf16_bits(out) : f32_to_f16_bits(out);
      }
    }
  }
}

// Generic kernel: any group size (multiple of 8), per-column g_idx, any ldq / alignment, any M.
// One wavefront per (output channel n, block of 4 rows of x); each weight element is dequantised exactly as the
// oracle does ((q - z) * s in fp32) and accumulated in fp32.
__global__ void __launch_bounds__(256) w4_generic_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int xdt, const int32_t* __restrict__ qw, int64_t ldq,
    const void* __restrict__ scales, int sdt, int64_t lds, const int32_t* __restrict__ zeros, int64_t ldz,
    const int32_t* __restrict__ perm, const int32_t* __restrict__ g_idx, const void* __restrict__ bias, int bdt,
    uint16_t* __restrict__ y, int64_t ldy, int M, int N, int K, int gs) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wid = (int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  const int64_t nwork = (int64_t)N * ((M + 3) / 4);
  if (wid >= nwork) return;
  const int n = (int)(wid % N);
  const int m0 = (int)(wid / N) * 4;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int k = lane; k < K; k += kWave) {
    const int g = g_idx ? g_idx[k] : k / gs;
    const uint32_t q = nibble((uint32_t)qw[(int64_t)n * ldq + k / 8], k & 7);
    const uint32_t z = zeros ? nibble((uint32_t)zeros[(int64_t)g * ldz + n / 8], n & 7) : 8u;
    const float w = ((float)q - (float)z) * load_f(scales, sdt, (int64_t)g * lds + n);
    const int xk = perm ? perm[k] : k;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (m0 + i < M) acc[i] = __builtin_fmaf(load_f(x, xdt, (int64_t)(m0 + i) * ldx + xk), w, acc[i]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float v = wave_sum(acc[i]);
    if (lane == i && m0 + i < M) {
      store_f(y, xdt, (int64_t)(m0 + i) * ldy + n, bias ? v + load_f(bias, bdt, n) : v);
    }
  }
}

// out[n, k] = (q - z) * s in fp32, rounded once to out dtype.  One thread per packed word (8 columns).
__global__ void __launch_bounds__(256) w4_dequant_kernel(
    const int32_t* __restrict__ qw, int64_t ldq, const void* __restrict__ scales, int sdt, int64_t lds,
    const int32_t* __restrict__ zeros, int64_t ldz, const int32_t* __restrict__ g_idx, void* __restrict__ out,
    int odt, int64_t ldo, int N, int K, int gs) {
  const int KW = (K + 7) / 8;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)N * KW) return;
  const int n = (int)(t / KW);
  const int w = (int)(t - (int64_t)n * KW);
  const uint32_t word = (uint32_t)qw[(int64_t)n * ldq + w];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int k = 8 * w + j;
    if (k >= K) break;
    const int g = g_idx ? g_idx[k] : k / gs;
    const uint32_t z = zeros ? nibble((uint32_t)zeros[(int64_t)g * ldz + n / 8], n & 7) : 8u;
    const float v = ((float)nibble(word, j) - (float)z) * load_f(scales, sdt, (int64_t)g * lds + n);
    store_f(out, odt, (int64_t)n * ldo + k, v);
  }
}

// ------------------------------------------------------------------------------------------------ launchers
size_t w4_gemv_lds_bytes(int mt, int K) {
  const int KW = (K + 7) / 8, KC = (KW + 3) / 4;
  return (size_t)mt * 4 * KC * 16 + (size_t)mt * KC * 4;
}

template <int MT, int R, bool XBF16>
static hipError_t launch_gemv_t(const void* x, int64_t ldx, const int32_t* qw, int64_t ldq, const void* scales,
                                int sdt, int64_t lds, const int32_t* zeros, int64_t ldz, const int32_t* perm,
                                const void* bias, int bdt, void* y, int64_t ldy, int M, int N, int K, int gs,
                                int max_blocks, hipStream_t stream) {
  auto kern = w4_gemv_kernel<MT, R, XBF16>;
  const size_t shm = w4_gemv_lds_bytes(MT, K);
  if (shm > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
    if (e != hipSuccess) return e;
  }
  const int threads = 256;
  const int waves = threads / kWave;
  const int NB = (N + R - 1) / R;
  int blocks = (NB + waves - 1) / waves;
  if (max_blocks > 0 && blocks > max_blocks) blocks = max_blocks;
  hipLaunchKernelGGL(kern, dim3(blocks), dim3(threads), shm, stream, static_cast<const uint16_t*>(x), ldx, qw, ldq,
                     scales, sdt, lds, zeros, ldz, perm, bias, bdt, static_cast<uint16_t*>(y), ldy, M, N, K, gs);
  return hipGetLastError();
}

template <int MT, bool XBF16>
static hipError_t launch_gemv_r(int R, const void* x, int64_t ldx, const int32_t* qw, int64_t ldq,
                                const void* scales, int sdt, int64_t lds, const int32_t* zeros, int64_t ldz,
                                const int32_t* perm, const void* bias, int bdt, void* y, int64_t ldy, int M, int N,
                                int K, int gs, int max_blocks, hipStream_t s) {
  switch (R) {
    case 1: return launch_gemv_t<MT, 1, XBF16>(x, ldx, qw, ldq, scales, sdt, lds, zeros, ldz, perm, bias, bdt, y, ldy, M, N, K, gs, max_blocks, s);
    case 2: return launch_gemv_t<MT, 2, XBF16>(x, ldx, qw, ldq, scales, sdt, lds, zeros, ldz, perm, bias, bdt, y, ldy, M, N, K, gs, max_blocks, s);
    default: return launch_gemv_t<MT, 4, XBF16>(x, ldx, qw, ldq, scales, sdt, lds, zeros, ldz, perm, bias, bdt, y, ldy, M, N, K, gs, max_blocks, s);
  }
}

hipError_t launch_w4_gemv(int mt, int R, bool xbf16, const void* x, int64_t ldx, const int32_t* qw, int64_t ldq,
                          const void* scales, int sdt, int64_t lds, const int32_t* zeros, int64_t ldz,
                          const int32_t* perm, const void* bias, int bdt, void* y, int64_t ldy, int M, int N, int K,
                          int gs, int max_blocks, hipStream_t s) {
#define FG_GEMV(MT_, XB_) \
  return launch_gemv_r<MT_, XB_>(R, x, ldx, qw, ldq, scales, sdt, lds, zeros, ldz, perm, bias, bdt, y, ldy, M, N, K, gs, max_blocks, s)
  if (xbf16) {
    if (mt == 1) FG_GEMV(1, true);
    if (mt == 2) FG_GEMV(2, true);
    FG_GEMV(4, true);
  } else {
    if (mt == 1) FG_GEMV(1, false);
    if (mt == 2) FG_GEMV(2, false);
    FG_GEMV(4, false);
  }
#undef FG_GEMV
}

hipError_t launch_w4_generic(const void* x, int64_t ldx, int xdt, const int32_t* qw, int64_t ldq, const void* scales,
                             int sdt, int64_t lds, const int32_t* zeros, int64_t ldz, const int32_t* perm,
                             const int32_t* g_idx, const void* bias, int bdt, void* y, int64_t ldy, int M, int N,
                             int K, int gs, hipStream_t s) {
  const int64_t nwork = (int64_t)N * ((M + 3) / 4);
  const int64_t blocks = (nwork + 3) / 4;
  hipLaunchKernelGGL(w4_generic_kernel, dim3((unsigned)blocks), dim3(256), 0, s, static_cast<const uint16_t*>(x), ldx,
                     xdt, qw, ldq, scales, sdt, lds, zeros, ldz, perm, g_idx, bias, bdt, static_cast<uint16_t*>(y),
                     ldy, M, N, K, gs);
  return hipGetLastError();
}

hipError_t launch_w4_dequant(const int32_t* qw, int64_t ldq, const void* scales, int sdt, int64_t lds,
                             const int32_t* zeros, int64_t ldz, const int32_t* g_idx, void* out, int odt, int64_t ldo,
                             int N, int K, int gs, hipStream_t s) {
  const int64_t total = (int64_t)N * ((K + 7) / 8);
  const int64_t blocks = (total + 255) / 256;
  hipLaunchKernelGGL(w4_dequant_kernel, dim3((unsigned)blocks), dim3(256), 0, s, qw, ldq, scales, sdt, lds, zeros, ldz,
                     g_idx, out, odt, ldo, N, K, gs);
  return hipGetLastError();
}

}  // namespace fg
