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
  // v_cvt_pk_fp8_f32: OCP e4m3 (gfx950), round to nearest even; inputs are pre-clamped to +-448
  const int packed = __builtin_amdgcn_cvt_pk_fp8_f32(v, 0.f, 0, false);
  return (uint8_t)(packed & 0xff);
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

hipError_t launch_quant_fp8_block(const void* x, int64_t ldx, int xdt, uint8_t* q, int64_t ldq, float* s,
                                  int64_t lds, int M, int K, int bm, int bk, const float* static_scale,
                                  hipStream_t st) {
  const dim3 grid((K + bk - 1) / bk, (M + bm - 1) / bm);
  hipLaunchKernelGGL(quant_fp8_block_kernel, grid, dim3(256), 0, st, x, ldx, xdt, q, ldq, s, lds, M, K, bm, bk,
                     static_scale);
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
