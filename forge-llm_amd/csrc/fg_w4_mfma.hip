// W4A16 on matrix cores (M > 4: skinny decode batches and prefill): dequantise weight tiles into LDS, then
// v_mfma_f32_16x16x32_{bf16,f16} with fp32 accumulation.
//
// Per 64-column K slice a workgroup copies its x tile [BM x 64] (16-byte loads) and its packed weight tile
// [BN x 8 words] into registers, then writes x as-is and the weights dequantised -- (q - z) * s in fp32, exactly the
// oracle's value, rounded once to the MFMA input type -- into a double-buffered LDS ring; no dequantised copy of W
// ever reaches HBM (the reference's large-M path writes one and re-reads it,
// forge/kernels/triton/gemm_w4_dequant.py:194-256).  Any group size that is a multiple of 8 works because every packed
// word (8 columns) lies in one group.
//
// Split-K (gridDim.y > 1) writes fp32 partials to the caller's workspace [S, M, N]; w4_splitk_reduce_kernel sums them
// in a fixed order (bit-reproducible run to run) and adds the bias -- the role of the reference's
// _splitk_reduce_kernel (forge/kernels/triton/gemm_wq.py:114-135).
#include "fg_device.h"

namespace fg {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <bool XBF16>
__device__ __forceinline__ f32x4_t mfma16x16x32(uint4 a, uint4 b, f32x4_t c) {
  if constexpr (XBF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                   0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
  }
}

// two fp32 -> packed 16-bit pair (bf16: v_cvt_pk_bf16_f32, round to nearest even; fp16: v_cvt_pkrtz is NOT used --
// each half is converted with round to nearest even)
template <bool XBF16>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (XBF16) {
    typedef float f2_t __attribute__((ext_vector_type(2)));
    typedef __bf16 b2_t __attribute__((ext_vector_type(2)));
    const b2_t p = __builtin_convertvector(f2_t{lo, hi}, b2_t);
    return __builtin_bit_cast(uint32_t, p);
  } else {
    return (uint32_t)f32_to_f16_bits(lo) | ((uint32_t)f32_to_f16_bits(hi) << 16);
  }
}

template <int WM, int WN, int TM, int TN, bool XBF16>
__global__ void __launch_bounds__(256) w4_mfma_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const int32_t* __restrict__ perm, const int32_t* __restrict__ qw,
    int64_t ldq, const void* __restrict__ scales, int sdt, int64_t lds, const int32_t* __restrict__ zeros, int64_t ldz,
    const void* __restrict__ bias, int bdt, uint16_t* __restrict__ y, int64_t ldy, float* __restrict__ ws, int M,
    int N, int K, int gs, int kchunk) {
  static_assert(WM * WN == 4, "four wavefronts");
  constexpr int BM = WM * TM * 16, BN = WN * TN * 16, BK = 64, PITCH = BK * 2 + 16;
  constexpr int STAGE = (BM + BN) * PITCH;
  constexpr int XCH = BM * 8, WCH = BN * 2;  // 16-byte chunks per slice: x rows hold 8, weight rows hold 2
  constexpr int XPT = (XCH + 255) / 256, WPT = (WCH + 255) / 256;
  extern __shared__ __align__(16) uint8_t smem[];

  const int ntm = (M + BM - 1) / BM, ntn = (N + BN - 1) / BN;
  int tmi, tni;
  tile_of(blockIdx.x, ntm, ntn, tmi, tni);
  const int m0 = tmi * BM, n0 = tni * BN;
  const int kbeg = blockIdx.y * kchunk;
  const int kend = min(K, kbeg + kchunk);
  const int nk = (kend - kbeg + BK - 1) / BK;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int64_t ldq4 = ldq / 4;
  const uint4* __restrict__ qw4 = reinterpret_cast<const uint4*>(qw);

  uint4 rx[XPT], rw[WPT];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int t = 0; t < XPT; ++t) {
      const int ch = tid + 256 * t;
      uint4 v = make_uint4(0, 0, 0, 0);
      const int row = ch >> 3, m = m0 + row, k = k0 + (ch & 7) * 8;
      if (ch < XCH && m < M && k < kend) {
        if (perm == nullptr) {
          v = *reinterpret_cast<const uint4*>(x + (int64_t)m * ldx + k);
        } else {
          uint32_t h[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) h[j] = x[(int64_t)m * ldx + perm[k + j]];
          v = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
        }
      }
      rx[t] = v;
    }
#pragma unroll
    for (int t = 0; t < WPT; ++t) {
      const int ch = tid + 256 * t;
      uint4 v = make_uint4(0, 0, 0, 0);
      const int row = ch >> 1, n = n0 + row, k = k0 + (ch & 1) * 32;
      if (ch < WCH && n < N && k < kend) v = load16_stream(qw4 + n * ldq4 + k / 32);
      rw[t] = v;
    }
  };
  auto stash = [&](uint8_t* st, int k0) {
#pragma unroll
    for (int t = 0; t < XPT; ++t) {
      const int ch = tid + 256 * t;
      if (ch < XCH) *reinterpret_cast<uint4*>(st + (ch >> 3) * PITCH + (ch & 7) * 16) = rx[t];
    }
#pragma unroll
    for (int t = 0; t < WPT; ++t) {
      const int ch = tid + 256 * t;
      if (ch >= WCH) continue;
      const int row = ch >> 1, n = n0 + row, kc = k0 + (ch & 1) * 32;
      const uint32_t words[4] = {rw[t].x, rw[t].y, rw[t].z, rw[t].w};
      uint32_t out[16];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kw = kc + 8 * i;
        float s = 0.f, z = 0.f;
        if (n < N && kw < kend) {
          const int g = kw / gs;
          s = load_f(scales, sdt, (int64_t)g * lds + n);
          z = zeros ? (float)nibble((uint32_t)zeros[(int64_t)g * ldz + n / 8], n & 7) : 8.f;
        }
        float d[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) d[j] = ((float)nibble(words[i], j) - z) * s;  // oracle's fp32 value
#pragma unroll
        for (int j = 0; j < 4; ++j) out[4 * i + j] = pack2<XBF16>(d[2 * j], d[2 * j + 1]);
      }
      uint4* dst = reinterpret_cast<uint4*>(st + BM * PITCH + row * PITCH + (ch & 1) * 64);
#pragma unroll
      for (int q = 0; q < 4; ++q) dst[q] = make_uint4(out[4 * q], out[4 * q + 1], out[4 * q + 2], out[4 * q + 3]);
    }
  };

  f32x4_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  if (nk > 0) {
    fetch(kbeg);
    stash(smem, kbeg);
  }
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    uint8_t* cur = smem + (kt & 1) * STAGE;
    uint8_t* nxt = smem + ((kt + 1) & 1) * STAGE;
    const bool more = kt + 1 < nk;
    if (more) fetch(kbeg + (kt + 1) * BK);
    const uint8_t* sA = cur + (wm * TM * 16 + (lane & 15)) * PITCH + (lane >> 4) * 16;
    const uint8_t* sB = cur + BM * PITCH + (wn * TN * 16 + (lane & 15)) * PITCH + (lane >> 4) * 16;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      uint4 fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[i] = *reinterpret_cast<const uint4*>(sA + i * 16 * PITCH + s * 64);
#pragma unroll
      for (int j = 0; j < TN; ++j) fb[j] = *reinterpret_cast<const uint4*>(sB + j * 16 * PITCH + s * 64);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma16x16x32<XBF16>(fa[i], fb[j], acc[i][j]);
    }
    if (more) stash(nxt, kbeg + (kt + 1) * BK);
    __syncthreads();
  }

  const bool split = gridDim.y > 1;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + wm * TM * 16 + i * 16 + 4 * (lane >> 4) + e;
        const int n = n0 + wn * TN * 16 + j * 16 + (lane & 15);
        if (m >= M || n >= N) continue;
        float v = acc[i][j][e];
        if (split) {
          ws[((int64_t)blockIdx.y * M + m) * N + n] = v;
        } else {
          if (bias) v += load_f(bias, bdt, n);
          y[(int64_t)m * ldy + n] = XBF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
        }
      }
}

template <bool XBF16>
__global__ void __launch_bounds__(256) w4_splitk_reduce_kernel(const float* __restrict__ ws, int S, int M, int N,
                                                               const void* __restrict__ bias, int bdt,
                                                               uint16_t* __restrict__ y, int64_t ldy) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t MN = (int64_t)M * N;
  if (t >= MN) return;
  // fixed order; the partials are loaded four splits at a time before any is added (adding each as it arrives waits
  // out one L2 round trip per split)
  float v = 0.f;
  for (int s = 0; s < S; s += 4) {
    float p[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) p[u] = ws[(int64_t)min(s + u, S - 1) * MN + t];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (s + u < S) v += p[u];
  }
  const int m = (int)(t / N), n = (int)(t - (int64_t)m * N);
  if (bias) v += load_f(bias, bdt, n);
  y[(int64_t)m * ldy + n] = XBF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
}

// The same sum, four outputs of one row per thread (N % 4 == 0, 16-byte aligned partials): 16-byte loads of eight
// splits in flight, one 8-byte store when y allows it.  Bit-identical to the one-output form.
template <bool XBF16>
__global__ void __launch_bounds__(256) w4_splitk_reduce4_kernel(const float* __restrict__ ws, int S, int M, int N,
                                                                const void* __restrict__ bias, int bdt,
                                                                uint16_t* __restrict__ y, int64_t ldy, int vec_store) {
  typedef float f32x4_t __attribute__((ext_vector_type(4)));
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // group of 4 outputs
  const int64_t MN = (int64_t)M * N;
  if (t * 4 >= MN) return;
  const f32x4_t* p = reinterpret_cast<const f32x4_t*>(ws) + t;
  f32x4_t v = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < S; s += 8) {
    f32x4_t q[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) q[u] = p[(int64_t)min(s + u, S - 1) * (MN / 4)];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (s + u < S) v += q[u];
  }
  const int m = (int)(t * 4 / N), n = (int)(t * 4 - (int64_t)m * N);
  uint16_t h[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float o = v[e];
    if (bias) o += load_f(bias, bdt, n + e);
    h[e] = XBF16 ? f32_to_bf16_bits(o) : f32_to_f16_bits(o);
  }
  uint16_t* yr = y + (int64_t)m * ldy + n;
  if (vec_store) {
    *reinterpret_cast<uint2*>(yr) = make_uint2(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16));
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) yr[e] = h[e];
  }
}

template <bool XBF16>
hipError_t launch_w4_splitk_reduce(const float* ws, int S, int M, int N, const void* bias, int bdt, void* y,
                                   int64_t ldy, hipStream_t s) {
  const int64_t MN = (int64_t)M * N;
  if (N % 4 == 0 && reinterpret_cast<uintptr_t>(ws) % 16 == 0) {
    const int vec = reinterpret_cast<uintptr_t>(y) % 8 == 0 && ldy % 4 == 0;
    hipLaunchKernelGGL(w4_splitk_reduce4_kernel<XBF16>, dim3((unsigned)((MN / 4 + 255) / 256)), dim3(256), 0, s, ws,
                       S, M, N, bias, bdt, static_cast<uint16_t*>(y), ldy, vec);
  } else {
    hipLaunchKernelGGL(w4_splitk_reduce_kernel<XBF16>, dim3((unsigned)((MN + 255) / 256)), dim3(256), 0, s, ws, S, M,
                       N, bias, bdt, static_cast<uint16_t*>(y), ldy);
  }
  return hipGetLastError();
}
template hipError_t launch_w4_splitk_reduce<true>(const float*, int, int, int, const void*, int, void*, int64_t,
                                                  hipStream_t);
template hipError_t launch_w4_splitk_reduce<false>(const float*, int, int, int, const void*, int, void*, int64_t,
                                                   hipStream_t);

// Tile shape per M bucket (wave grid WM x WN, wave tile (16 TM) x (16 TN)).
struct W4Tile {
  int bm, bn;
};

W4Tile w4_mfma_tile(int M, int tile_m) {
  const int t = tile_m > 0 ? tile_m : (M <= 16 ? 16 : (M <= 32 ? 32 : (M <= 64 ? 64 : 128)));
  if (t <= 16) return {16, 64};
  if (t <= 32) return {32, 64};
  if (t <= 64) return {64, 64};
  return {128, 128};
}

// K splits for the MFMA path: enough workgroups to cover the 256 CUs twice, at least 256 K columns per split.
// kchunk (columns per split) is a multiple of the 64-column slice; `used` is the number of non-empty splits.
void w4_mfma_split_plan(int M, int N, int K, int tile_m, int split_k, int* kchunk, int* used) {
  const W4Tile t = w4_mfma_tile(M, tile_m);
  int s = split_k;
  if (s <= 0) {
    const int tiles = ((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn);
    s = (512 + tiles - 1) / tiles;
    const int max_s = K / 256 > 0 ? K / 256 : 1;
    if (s > max_s) s = max_s;
    if (s > 16) s = 16;
    if (s < 1) s = 1;
  }
  int kc = (K + s - 1) / s;
  kc = (kc + 63) / 64 * 64;
  *kchunk = kc;
  *used = (K + kc - 1) / kc;
}

template <int WM, int WN, int TM, int TN, bool XBF16>
static hipError_t launch_w4_mfma_t(const void* x, int64_t ldx, const int32_t* qw, int64_t ldq, const void* scales,
                                   int sdt, int64_t lds, const int32_t* zeros, int64_t ldz, const int32_t* perm,
                                   const void* bias, int bdt, void* y, int64_t ldy, float* ws, int M, int N, int K,
                                   int gs, int splits, hipStream_t s) {
  constexpr int BM = WM * TM * 16, BN = WN * TN * 16, PITCH = 64 * 2 + 16;
  const size_t shm = 2 * (size_t)(BM + BN) * PITCH;
  auto kern = w4_mfma_kernel<WM, WN, TM, TN, XBF16>;
  if (shm > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
    if (e != hipSuccess) return e;
  }
  const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  int kchunk = 0, used = 0;
  w4_mfma_split_plan(M, N, K, BM, splits, &kchunk, &used);
  note_kernel("w4_mfma_kernel splits=%d%s", used, used > 1 ? " + w4_splitk_reduce_kernel" : "");
  hipLaunchKernelGGL(kern, dim3(tiles, used), dim3(256), shm, s, static_cast<const uint16_t*>(x), ldx, perm, qw, ldq,
                     scales, sdt, lds, zeros, ldz, bias, bdt, static_cast<uint16_t*>(y), ldy, ws, M, N, K, gs, kchunk);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || used == 1) return e;
  return launch_w4_splitk_reduce<XBF16>(ws, used, M, N, bias, bdt, y, ldy, s);
}

template <bool XBF16>
static hipError_t launch_w4_mfma_x(const void* x, int64_t ldx, const int32_t* qw, int64_t ldq, const void* scales,
                                   int sdt, int64_t lds, const int32_t* zeros, int64_t ldz, const int32_t* perm,
                                   const void* bias, int bdt, void* y, int64_t ldy, float* ws, int M, int N, int K,
                                   int gs, int tile_m, int splits, hipStream_t s) {
  const W4Tile t = w4_mfma_tile(M, tile_m);
  if (t.bm == 16) return launch_w4_mfma_t<1, 4, 1, 1, XBF16>(x, ldx, qw, ldq, scales, sdt, lds, zeros, ldz, perm, bias, bdt, y, ldy, ws, M, N, K, gs, splits, s);
  if (t.bm == 32) return launch_w4_mfma_t<2, 2, 1, 2, XBF16>(x, ldx, qw, ldq, scales, sdt, lds, zeros, ldz, perm, bias, bdt, y, ldy, ws, M, N, K, gs, splits, s);
  if (t.bm == 64) return launch_w4_mfma_t<2, 2, 2, 2, XBF16>(x, ldx, qw, ldq, scales, sdt, lds, zeros, ldz, perm, bias, bdt, y, ldy, ws, M, N, K, gs, splits, s);
  return launch_w4_mfma_t<2, 2, 4, 4, XBF16>(x, ldx, qw, ldq, scales, sdt, lds, zeros, ldz, perm, bias, bdt, y, ldy, ws, M, N, K, gs, splits, s);
}

hipError_t launch_w4_mfma(const void* x, int64_t ldx, bool xbf16, const int32_t* qw, int64_t ldq, const void* scales,
                          int sdt, int64_t lds, const int32_t* zeros, int64_t ldz, const int32_t* perm,
                          const void* bias, int bdt, void* y, int64_t ldy, float* ws, int M, int N, int K, int gs,
                          int tile_m, int splits, hipStream_t s) {
  if (xbf16)
    return launch_w4_mfma_x<true>(x, ldx, qw, ldq, scales, sdt, lds, zeros, ldz, perm, bias, bdt, y, ldy, ws, M, N, K, gs, tile_m, splits, s);
  return launch_w4_mfma_x<false>(x, ldx, qw, ldq, scales, sdt, lds, zeros, ldz, perm, bias, bdt, y, ldy, ws, M, N, K, gs, tile_m, splits, s);
}

}  // namespace fg
