// Shared pieces of the W8A8 GEMM kernels (fg_mm.hip: 128-row tiles and the K-blocked FP8 mode; fg_mm_big.hip:
// 256 x 256 tiles fed by direct global->LDS loads): MFMA wrappers and epilogues.
//
// MFMA register layouts (16x16 tiles): operand lane l holds row/column (l % 16) and the K sub-slice (l / 16); the
// result lane l holds column (l % 16), rows 4*(l/16) + i, i = 0..3.  A and B use the same K sub-slice mapping, so the
// product sums every K element exactly once whatever order the hardware uses inside the instruction.
#pragma once

#include "fg_device.h"

namespace fg {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct MmaI8 {  // v_mfma_i32_16x16x64_i8
  static constexpr int KB = 64;  // K bytes per instruction
  static constexpr int LB = 16;  // operand bytes per lane
  typedef i32x4 frag_t;
  typedef i32x4 acc_t;
  static __device__ __forceinline__ acc_t mma(frag_t a, frag_t b, acc_t c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ frag_t load(const uint8_t* p) {
    return *reinterpret_cast<const i32x4*>(p);
  }
};

struct MmaF8 {  // v_mfma_f32_16x16x128_f8f6f4, both operands OCP e4m3 (format code 0), no block scales
  static constexpr int KB = 128;
  static constexpr int LB = 32;
  typedef i32x8 frag_t;
  typedef f32x4 acc_t;
  static __device__ __forceinline__ acc_t mma(frag_t a, frag_t b, acc_t c) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
  }
  static __device__ __forceinline__ frag_t load(const uint8_t* p) {
    const i32x4 lo = *reinterpret_cast<const i32x4*>(p);
    const i32x4 hi = *reinterpret_cast<const i32x4*>(p + 16);
    frag_t f;
    f[0] = lo[0]; f[1] = lo[1]; f[2] = lo[2]; f[3] = lo[3];
    f[4] = hi[0]; f[5] = hi[1]; f[6] = hi[2]; f[7] = hi[3];
    return f;
  }
};

// ------------------------------------------------------------------------------------------------ epilogues
struct EpiInt8 {
  static constexpr bool kBlocked = false;
  const float* sa; int64_t sa_len;
  const float* sb; int64_t sb_len;
  const void* bias; int bdt;
  void* y; int64_t ldy; int ydt;
  __device__ __forceinline__ void store(int m, int n, int acc) const {
    if (ydt == FG_I32) {
      static_cast<int32_t*>(y)[(int64_t)m * ldy + n] = acc;
      return;
    }
    // (float(acc) * sa[m]) * sb[n] (+ bias[n]): one fp32 rounding per operation, no contraction
    float v = (float)acc * sa[sa_len == 1 ? 0 : m];
    v = v * sb[sb_len == 1 ? 0 : n];
    if (bias) v = v + load_f(bias, bdt, n);
    store_f(y, ydt, (int64_t)m * ldy + n, v);
  }
};

struct EpiFp8 {
  static constexpr bool kBlocked = false;
  const float* sa; int64_t sa_sm;
  const float* sb; int64_t sb_sn;
  const void* bias; int bdt;
  void* y; int64_t ldy; int ydt;
  __device__ __forceinline__ void store(int m, int n, float acc) const {
    float v = acc * sa[(int64_t)m * sa_sm];
    v = v * sb[(int64_t)n * sb_sn];
    if (bias) v = v + load_f(bias, bdt, n);
    store_f(y, ydt, (int64_t)m * ldy + n, v);
  }
};


// FP8 with K-blocked scales (activations 1 x block, weights per row or block x block): every 128-byte K slice is one
// scale block, so each slice's MFMA partial is scaled by sa[m, kb] * sb[n / sb_div, kb] before it joins the fp32 sum.
struct EpiFp8Blocked {
  static constexpr bool kBlocked = true;
  const float* sa; int64_t sa_sm, sa_sk;
  const float* sb; int64_t sb_sn, sb_sk; int sb_div;
  const void* bias; int bdt;
  void* y; int64_t ldy; int ydt;
  int M, N;
  __device__ __forceinline__ float kscale(int m, int n, int kb) const {
    m = min(m, M - 1);
    n = min(n, N - 1);
    return sa[(int64_t)m * sa_sm + (int64_t)kb * sa_sk] * sb[(int64_t)(n / sb_div) * sb_sn + (int64_t)kb * sb_sk];
  }
  __device__ __forceinline__ void store(int m, int n, float acc) const {
    float v = acc;
    if (bias) v = v + load_f(bias, bdt, n);
    store_f(y, ydt, (int64_t)m * ldy + n, v);
  }
};

}  // namespace fg
