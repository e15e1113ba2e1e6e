// Device-side helpers shared by the gfx950 kernels: number-format conversions, typed loads, wave reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/forge_mi355x.h"

namespace fg {

constexpr int kWave = 64;

// ----------------------------------------------------------------------------------------------- conversions
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);                                            // round half to even
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
  _Float16 h;
  __builtin_memcpy(&h, &b, 2);
  return (float)h;
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;  // v_cvt_f16_f32, round to nearest even
  uint16_t b;
  __builtin_memcpy(&b, &h, 2);
  return b;
}

// Load element i of a buffer of element type `dt` (FG_F32/F16/BF16) as float.
__device__ __forceinline__ float load_f(const void* p, int dt, int64_t i) {
  if (dt == FG_F32) return static_cast<const float*>(p)[i];
  uint16_t b = static_cast<const uint16_t*>(p)[i];
  return dt == FG_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}

// Store float v as element i of a buffer of element type `dt` (FG_F32/F16/BF16).
__device__ __forceinline__ void store_f(void* p, int dt, int64_t i, float v) {
  if (dt == FG_F32) {
    static_cast<float*>(p)[i] = v;
  } else {
    static_cast<uint16_t*>(p)[i] = dt == FG_BF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
  }
}

// ----------------------------------------------------------------------------------------------- reductions
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// Map a linear workgroup id to an output tile: first deal consecutive logical tiles to one XCD, then walk tiles in
// groups of `gm` tile-rows so neighbouring workgroups share B (weight) slices and A (activation) slices.
__device__ __forceinline__ void tile_of(int bid, int ntm, int ntn, int& tm, int& tn) {
  const int total = ntm * ntn;
  const int per = total / 8;
  int t = bid;
  if (bid < per * 8) t = (bid % 8) * per + bid / 8;
  const int gm = 8;
  const int group = t / (gm * ntn);
  const int first = group * gm;
  const int gsz = min(ntm - first, gm);
  const int r = t - group * gm * ntn;
  tm = first + r % gsz;
  tn = r / gsz;
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte streaming load (non-temporal: weights are read once per call and should not evict reusable lines)
__device__ __forceinline__ uint4 load16_stream(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// nibble j (bits 4j..4j+3) of a packed word
__device__ __forceinline__ uint32_t nibble(uint32_t w, int j) { return (w >> (4 * j)) & 0xFu; }

}  // namespace fg
