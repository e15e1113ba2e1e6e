// Per-token activation quantisers (memory-bound pre-passes of the W8A8 GEMMs): one 256-thread workgroup per row.
//
// INT8 (forge/kernels/ref/gemm_int8.py:17-35): s = amax / 127 with IEEE division (1 where amax > 0 is false),
//   q = clamp(round_half_even(x / s), -127, 127), x / s again IEEE-divided, so codes equal the CPU oracle's bit for
//   bit, ties included.  NaN inputs give code 0, like the oracle's float->int8 cast.
// FP8 (forge/kernels/ref/gemm_fp8.py:43-85,130-150): optional fused RMSNorm y = x * (1 / sqrt(mean(x^2) + eps)) * w in
//   fp32, s = amax(y) / 448 (IEEE; 1 where amax > 0 is false, so NaN rows get scale 1 as in the oracle), or a static
//   device scale; q = e4m3fn(clamp(y / s, -448, 448)) with gfx950's round-to-nearest-even OCP fp8 conversion.
#include "fg_device.h"

namespace fg {

__device__ __forceinline__ float block_reduce(float v, bool is_max, float* red) {
  v = is_max ? wave_max(v) : wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
  return r;
}

__global__ void __launch_bounds__(256) quant_int8_rowwise_kernel(const void* __restrict__ x, int64_t ldx, int xdt,
                                                                 int8_t* __restrict__ q, int64_t ldq,
                                                                 float* __restrict__ s, int K) {
  __shared__ float red[8];
  __shared__ int nan_flag;
  const int64_t row = blockIdx.x;
  if (threadIdx.x == 0) nan_flag = 0;
  __syncthreads();
  float amax = 0.f;
  bool has_nan = false;
  for (int k = threadIdx.x; k < K; k += blockDim.x) {
    const float v = load_f(x, xdt, row * ldx + k);
    has_nan |= __builtin_isnan(v);
    amax = fmaxf(amax, fabsf(v));
  }
  if (has_nan) nan_flag = 1;
  amax = block_reduce(amax, true, red);
  // torch.amax propagates NaN and `NaN > 0` is false: such rows take scale 1
  const float scale = (!nan_flag && amax > 0.f) ? __fdiv_rn(amax, 127.f) : 1.f;
  if (threadIdx.x == 0) s[row] = scale;
  for (int k = threadIdx.x; k < K; k += blockDim.x) {
    const float v = __fdiv_rn(load_f(x, xdt, row * ldx + k), scale);
    const float r = __builtin_isnan(v) ? 0.f : rintf(fminf(fmaxf(v, -127.f), 127.f));
    q[row * ldq + k] = (int8_t)(int)r;
  }
}

__device__ __forceinline__ uint8_t f32_to_e4m3(float v) {
  // v_cvt_pk_fp8_f32: OCP e4m3 (gfx950), round to nearest even; inputs are pre-clamped to +-448.  A NaN becomes the
  // e4m3fn NaN code with its sign (0x7F / 0xFF), as torch's cast writes it.
  const int packed = __builtin_amdgcn_cvt_pk_fp8_f32(v, 0.f, 0, false);
  const uint8_t nan_code = (__float_as_uint(v) >> 24 & 0x80) | 0x7F;
  return __builtin_isnan(v) ? nan_code : (uint8_t)(packed & 0xff);
}

__global__ void __launch_bounds__(256) quant_fp8_rowwise_kernel(const void* __restrict__ x, int64_t ldx, int xdt,
                                                                uint8_t* __restrict__ q, int64_t ldq,
                                                                float* __restrict__ s, int K,
                                                                const float* __restrict__ static_scale,
                                                                const void* __restrict__ rms_w, int wdt, float eps,
                                                                int fuse) {
  __shared__ float red[8];
  __shared__ int nan_flag;
  const int64_t row = blockIdx.x;
  if (threadIdx.x == 0) nan_flag = 0;
  __syncthreads();
  float rs = 1.f;
  if (fuse) {
    float ss = 0.f;
    for (int k = threadIdx.x; k < K; k += blockDim.x) {
      const float v = load_f(x, xdt, row * ldx + k);
      ss = __builtin_fmaf(v, v, ss);
    }
    ss = block_reduce(ss, false, red);
    rs = __fdiv_rn(1.f, __fsqrt_rn(__fdiv_rn(ss, (float)K) + eps));
  }
  auto yval = [&](int k) {
    float v = load_f(x, xdt, row * ldx + k);
    if (fuse) {
      v = v * rs;
      if (rms_w) v = v * load_f(rms_w, wdt, k);
    }
    return v;
  };
  float scale;
  if (static_scale) {
    scale = static_scale[row];
  } else {
    float amax = 0.f;
    bool has_nan = false;
    for (int k = threadIdx.x; k < K; k += blockDim.x) {
      const float v = yval(k);
      has_nan |= __builtin_isnan(v);
      amax = fmaxf(amax, fabsf(v));
    }
    if (has_nan) nan_flag = 1;
    amax = block_reduce(amax, true, red);
    scale = (!nan_flag && amax > 0.f) ? __fdiv_rn(amax, 448.f) : 1.f;
    if (threadIdx.x == 0) s[row] = scale;
  }
  for (int k = threadIdx.x; k < K; k += blockDim.x) {
    const float v = __fdiv_rn(yval(k), scale);
    const float c = __builtin_isnan(v) ? v : fminf(fmaxf(v, -448.f), 448.f);
    q[row * ldq + k] = f32_to_e4m3(c);
  }
}

// One workgroup per [block_m x block_k] tile: amax over the tile, one scale, then the codes.
__global__ void __launch_bounds__(256) quant_fp8_block_kernel(const void* __restrict__ x, int64_t ldx, int xdt,
                                                              uint8_t* __restrict__ q, int64_t ldq,
                                                              float* __restrict__ s, int64_t lds, int M, int K,
                                                              int bm, int bk, const float* __restrict__ static_scale) {
  __shared__ float red[8];
  __shared__ int nan_flag;
  const int r0 = blockIdx.y * bm, c0 = blockIdx.x * bk;
  const int rows = min(bm, M - r0), cols = min(bk, K - c0);
  const int64_t n = (int64_t)rows * cols;
  if (threadIdx.x == 0) nan_flag = 0;
  __syncthreads();
  float scale;
  if (static_scale) {
    scale = static_scale[0];
  } else {
    float amax = 0.f;
    bool has_nan = false;
    for (int64_t t = threadIdx.x; t < n; t += blockDim.x) {
      const int r = (int)(t / cols), c = (int)(t - (int64_t)r * cols);
      const float v = load_f(x, xdt, (int64_t)(r0 + r) * ldx + c0 + c);
      has_nan |= __builtin_isnan(v);
      amax = fmaxf(amax, fabsf(v));
    }
    if (has_nan) nan_flag = 1;
    amax = block_reduce(amax, true, red);
    scale = (!nan_flag && amax > 0.f) ? __fdiv_rn(amax, 448.f) : 1.f;
    if (threadIdx.x == 0) s[(int64_t)blockIdx.y * lds + blockIdx.x] = scale;
  }
  for (int64_t t = threadIdx.x; t < n; t += blockDim.x) {
    const int r = (int)(t / cols), c = (int)(t - (int64_t)r * cols);
    const float v = __fdiv_rn(load_f(x, xdt, (int64_t)(r0 + r) * ldx + c0 + c), scale);
    const float cl = __builtin_isnan(v) ? v : fminf(fmaxf(v, -448.f), 448.f);
    q[(int64_t)(r0 + r) * ldq + c0 + c] = f32_to_e4m3(cl);
  }
}

// Few large tiles (a per-tensor scale: one tile of M x K) would leave all but a few CUs idle in the kernel above.  Then
// each tile is cut into `parts` contiguous element ranges, one workgroup each, over up to four launches: zero the
// amax words, fold each part's amax into its tile's word (atomic max on the bit pattern: amax >= 0, and a NaN's
// pattern exceeds every number's, so NaN wins like torch.amax), turn the words into scales, then encode.  The scale
// buffer holds the amax bits in between, so no workspace is needed.
__global__ void __launch_bounds__(256) quant_fp8_tile_zero_kernel(float* __restrict__ s, int64_t lds, int mb, int kb) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t < mb * kb) s[(int64_t)(t / kb) * lds + t % kb] = 0.f;
}

__device__ __forceinline__ void tile_part(int M, int K, int bm, int bk, int parts, int64_t* r0, int64_t* c0,
                                          int64_t* cols, int64_t* e0, int64_t* e1) {
  *r0 = (int64_t)blockIdx.y * bm;
  *c0 = (int64_t)blockIdx.x * bk;
  const int64_t rows = min((int64_t)bm, M - *r0);
  *cols = min((int64_t)bk, K - *c0);
  const int64_t n = rows * *cols, chunk = (n + parts - 1) / parts;
  *e0 = min(n, (int64_t)blockIdx.z * chunk);
  *e1 = min(n, *e0 + chunk);
}

__global__ void __launch_bounds__(256) quant_fp8_tile_amax_kernel(const void* __restrict__ x, int64_t ldx, int xdt,
                                                                  float* __restrict__ s, int64_t lds, int M, int K,
                                                                  int bm, int bk, int parts) {
  __shared__ float red[8];
  __shared__ int nan_flag;
  int64_t r0, c0, cols, e0, e1;
  tile_part(M, K, bm, bk, parts, &r0, &c0, &cols, &e0, &e1);
  if (threadIdx.x == 0) nan_flag = 0;
  __syncthreads();
  float amax = 0.f;
  bool has_nan = false;
  for (int64_t t = e0 + threadIdx.x; t < e1; t += blockDim.x) {
    const int64_t r = t / cols, c = t - r * cols;
    const float v = load_f(x, xdt, (r0 + r) * ldx + c0 + c);
    has_nan |= __builtin_isnan(v);
    amax = fmaxf(amax, fabsf(v));
  }
  if (has_nan) nan_flag = 1;
  amax = block_reduce(amax, true, red);  // its barriers also publish nan_flag
  if (threadIdx.x == 0) {
    unsigned* word = reinterpret_cast<unsigned*>(s + (int64_t)blockIdx.y * lds + blockIdx.x);
    atomicMax(word, nan_flag ? 0x7FC00000u : __float_as_uint(amax));
  }
}

__global__ void __launch_bounds__(256) quant_fp8_tile_scale_kernel(float* __restrict__ s, int64_t lds, int mb,
                                                                   int kb) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= mb * kb) return;
  float* p = s + (int64_t)(t / kb) * lds + t % kb;
  const float amax = *p;  // the bit pattern the atomics left is the amax itself (or a NaN)
  *p = (!__builtin_isnan(amax) && amax > 0.f) ? __fdiv_rn(amax, 448.f) : 1.f;
}

__global__ void __launch_bounds__(256) quant_fp8_tile_encode_kernel(const void* __restrict__ x, int64_t ldx, int xdt,
                                                                    uint8_t* __restrict__ q, int64_t ldq,
                                                                    const float* __restrict__ s, int64_t lds,
                                                                    int64_t ldx_s, int M, int K, int bm, int bk,
                                                                    int parts) {
  int64_t r0, c0, cols, e0, e1;
  tile_part(M, K, bm, bk, parts, &r0, &c0, &cols, &e0, &e1);
  const float scale = s[(int64_t)blockIdx.y * lds + blockIdx.x * ldx_s];  // strides 0, 0: one static scale
  for (int64_t t = e0 + threadIdx.x; t < e1; t += blockDim.x) {
    const int64_t r = t / cols, c = t - r * cols;
    const float v = __fdiv_rn(load_f(x, xdt, (r0 + r) * ldx + c0 + c), scale);
    const float cl = __builtin_isnan(v) ? v : fminf(fmaxf(v, -448.f), 448.f);
    q[(r0 + r) * ldq + c0 + c] = f32_to_e4m3(cl);
  }
}

hipError_t launch_quant_fp8_block(const void* x, int64_t ldx, int xdt, uint8_t* q, int64_t ldq, float* s,
                                  int64_t lds, int M, int K, int bm, int bk, const float* static_scale,
                                  hipStream_t st) {
  const int kb = (K + bk - 1) / bk, mb = (M + bm - 1) / bm;
  const int64_t tiles = (int64_t)kb * mb, per_tile = (int64_t)min(bm, M) * min(bk, K);
  const int64_t cus = device_cus();
  // one workgroup per tile while the tiles cover the CUs or are small; else parts of 64 Ki elements, up to 4 rounds
  int64_t parts = 1;
  if (tiles < cus && per_tile > 65536) parts = min((per_tile + 65535) / 65536, (4 * cus + tiles - 1) / tiles);
  if (parts == 1) {
    hipLaunchKernelGGL(quant_fp8_block_kernel, dim3(kb, mb), dim3(256), 0, st, x, ldx, xdt, q, ldq, s, lds, M, K, bm,
                       bk, static_scale);
    return hipGetLastError();
  }
  const dim3 grid(kb, mb, (unsigned)parts);
  const float* scale = static_scale;
  int64_t slds = 0, sldx = 0;
  if (!static_scale) {
    const unsigned small = (unsigned)((tiles + 255) / 256);
    hipLaunchKernelGGL(quant_fp8_tile_zero_kernel, dim3(small), dim3(256), 0, st, s, lds, mb, kb);
    hipLaunchKernelGGL(quant_fp8_tile_amax_kernel, grid, dim3(256), 0, st, x, ldx, xdt, s, lds, M, K, bm, bk,
                       (int)parts);
    hipLaunchKernelGGL(quant_fp8_tile_scale_kernel, dim3(small), dim3(256), 0, st, s, lds, mb, kb);
    scale = s;
    slds = lds;
    sldx = 1;
  }
  hipLaunchKernelGGL(quant_fp8_tile_encode_kernel, grid, dim3(256), 0, st, x, ldx, xdt, q, ldq, scale, slds, sldx, M,
                     K, bm, bk, (int)parts);
  return hipGetLastError();
}

hipError_t launch_quant_int8(const void* x, int64_t ldx, int xdt, int8_t* q, int64_t ldq, float* s, int M, int K,
                             hipStream_t st) {
  hipLaunchKernelGGL(quant_int8_rowwise_kernel, dim3(M), dim3(256), 0, st, x, ldx, xdt, q, ldq, s, K);
  return hipGetLastError();
}

hipError_t launch_quant_fp8(const void* x, int64_t ldx, int xdt, uint8_t* q, int64_t ldq, float* s, int M, int K,
                            const float* static_scale, const void* rms_w, int wdt, float eps, int fuse,
                            hipStream_t st) {
  hipLaunchKernelGGL(quant_fp8_rowwise_kernel, dim3(M), dim3(256), 0, st, x, ldx, xdt, q, ldq, s, K, static_scale,
                     rms_w, wdt, eps, fuse);
  return hipGetLastError();
}

}  // namespace fg
