// Helpers shared by the gfx950 kernels (number-format conversions, typed and buffer loads, wave reductions, tile
// order) and by their host launchers (CU count, workgroup balance).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <type_traits>

#include "../../include/forge_mi355x.h"

namespace fg {

constexpr int kWave = 64;

// Records (printf-style) the kernel and launch form of the calling thread's current launch; fg_last_kernel() returns
// it.  Host code only.
void note_kernel(const char* fmt, ...);

// ----------------------------------------------------------------------------------------------- conversions
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);                                            // round half to even
  return (uint16_t)(u >> 16);
}

// Hardware conversion (v_cvt_pk_bf16_f32): round to nearest even, NaN stays NaN.
__device__ __forceinline__ uint16_t f32_to_bf16_bits_hw(float f) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
  const bf16x2v_t h = __builtin_convertvector((f32x2_t){f, f}, bf16x2v_t);
  return (uint16_t)__builtin_bit_cast(uint32_t, h);
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

// Quotient n / d for n * d < 2^32 with one multiply-high (d == 1 passes n through): m = floor((2^32 - 1) / d) + 1 is
// floor(2^32 / d) + 1 (or 2^32 / d for powers of two), and n * m / 2^32 = n / d + n * e / 2^32 with 0 <= e <= 1 never
// carries past the next integer while n * d < 2^32.
struct FastDiv {
  uint32_t d, m;
  __device__ __forceinline__ explicit FastDiv(uint32_t d_) : d(d_), m(d_ > 1 ? 0xffffffffu / d_ + 1u : 0u) {}
  __device__ __forceinline__ uint32_t div(uint32_t n) const { return d > 1 ? __umulhi(n, m) : n; }
};

// Whether a kernel's group index, the chunk index (chunks of `unit` columns below K) divided by the chunks per group
// with one multiply-high (FastDiv, or the same m inline), is exact for every chunk: one group, a power-of-two group
// (m = 2^32 / d exactly), or (K / unit) * (gs / unit) < 2^32.
inline bool group_div_exact(int64_t K, int64_t gs, int64_t G, int64_t unit) {
  const int64_t d = gs / unit, c = (K + unit - 1) / unit;
  return G == 1 || d <= 1 || (d & (d - 1)) == 0 || c * d < (1LL << 32);
}

// Value of lane l ^ o (o = 1, 2) or of a partner in the other o-half of its 8/16-lane group (o = 4: mirror within 8
// lanes, o = 8: rotate by 8 within 16 lanes) through DPP, without LDS traffic.
template <int O>
__device__ __forceinline__ float dpp_partner(float v) {
  constexpr int ctrl = O == 1 ? 0xB1 : (O == 2 ? 0x4E : (O == 4 ? 0x141 : 0x128));
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl, 0xF, 0xF, false));
}

// In-place v_permlane32_swap_b32 / v_permlane16_swap_b32: a's lanes 32-63 trade places with b's lanes 0-31 (32), or
// a's odd 16-lane rows with b's even rows (16).  Written as asm because this compiler folds the builtin's second
// result into its first when both feed one add.  s_nop 1 gives the two wait states a VALU write needs before a
// permlane swap reads it (and the same after, for the consumer).
__device__ __forceinline__ void permlane32_swap(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void permlane16_swap(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}

// Sum each of V (4, 8 or 16) values over the 64 lanes; every lane of the group of 64/V lanes that starts at
// (l / (64/V)) * (64/V) ends with the same total of value l / (64/V).  Halving steps exchange half of the live values
// with the partner half of the wave: across 32 lanes with v_permlane32_swap, across 16 with v_permlane16_swap, then
// within 16-lane rows through DPP, so V values cost V-1 exchanges plus the log2 of the final group size.
template <int V>
__device__ __forceinline__ float wave_transpose_sum(float (&v)[V], int lane) {
  static_assert(V == 4 || V == 8 || V == 16, "V");
  float cur[V];
#pragma unroll
  for (int i = 0; i < V; ++i) cur[i] = v[i];
#pragma unroll
  for (int i = 0; i < V / 2; ++i) {  // lanes 0-31 keep values [0, V/2), lanes 32-63 keep [V/2, V)
    float a = cur[i], b = cur[i + V / 2];
    permlane32_swap(a, b);  // a = [cur_i lanes 0-31, cur_j lanes 0-31], b = [cur_i lanes 32-63, cur_j lanes 32-63]
    cur[i] = a + b;
  }
#pragma unroll
  for (int i = 0; i < V / 4; ++i) {  // even 16-lane rows keep the lower quarter, odd rows the upper one
    float a = cur[i], b = cur[i + V / 4];
    permlane16_swap(a, b);
    cur[i] = a + b;
  }
  auto step = [&](auto o_tag, int n) {
    constexpr int O = decltype(o_tag)::value;
    const bool up = (lane & O) != 0;
    if (n > 1) {
#pragma unroll
      for (int i = 0; i < V / 8; ++i) {
        if (i < n / 2) {
          const float send = up ? cur[i] : cur[i + n / 2];
          const float keep = up ? cur[i + n / 2] : cur[i];
          cur[i] = keep + dpp_partner<O>(send);
        }
      }
    } else {
      cur[0] += dpp_partner<O>(cur[0]);
    }
  };
  step(std::integral_constant<int, 8>{}, V / 4);
  step(std::integral_constant<int, 4>{}, V / 8 > 0 ? V / 8 : 1);
  step(std::integral_constant<int, 2>{}, V / 16 > 0 ? V / 16 : 1);
  step(std::integral_constant<int, 1>{}, 1);
  return cur[0];
}

// wave_transpose_sum for int32 partials (exact integer adds; the lane moves are the same bit moves).
template <int V>
__device__ __forceinline__ int wave_transpose_sum_i32(int (&v)[V], int lane) {
  static_assert(V == 4 || V == 8 || V == 16, "V");
  int cur[V];
#pragma unroll
  for (int i = 0; i < V; ++i) cur[i] = v[i];
#pragma unroll
  for (int i = 0; i < V / 2; ++i) {
    float a = __builtin_bit_cast(float, cur[i]), b = __builtin_bit_cast(float, cur[i + V / 2]);
    permlane32_swap(a, b);
    cur[i] = __builtin_bit_cast(int, a) + __builtin_bit_cast(int, b);
  }
#pragma unroll
  for (int i = 0; i < V / 4; ++i) {
    float a = __builtin_bit_cast(float, cur[i]), b = __builtin_bit_cast(float, cur[i + V / 4]);
    permlane16_swap(a, b);
    cur[i] = __builtin_bit_cast(int, a) + __builtin_bit_cast(int, b);
  }
  auto partner = [&](auto o_tag, int v) {
    constexpr int O = decltype(o_tag)::value;
    return __builtin_bit_cast(int, dpp_partner<O>(__builtin_bit_cast(float, v)));
  };
  auto step = [&](auto o_tag, int n) {
    constexpr int O = decltype(o_tag)::value;
    const bool up = (lane & O) != 0;
    if (n > 1) {
#pragma unroll
      for (int i = 0; i < V / 8; ++i) {
        if (i < n / 2) {
          const int send = up ? cur[i] : cur[i + n / 2];
          const int keep = up ? cur[i + n / 2] : cur[i];
          cur[i] = keep + partner(o_tag, send);
        }
      }
    } else {
      cur[0] += partner(o_tag, cur[0]);
    }
  };
  step(std::integral_constant<int, 8>{}, V / 4);
  step(std::integral_constant<int, 4>{}, V / 8 > 0 ? V / 8 : 1);
  step(std::integral_constant<int, 2>{}, V / 16 > 0 ? V / 16 : 1);
  step(std::integral_constant<int, 1>{}, 1);
  return cur[0];
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

// Raw buffer resource over `bytes` bytes from p (gfx9 dword3: 32-bit data format).  Loads through it take a per-lane
// 32-bit voffset plus a wavefront-uniform soffset (a scalar register), need no 64-bit address math, and read 0 past the
// end.  The caller guarantees bytes < 2^32.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
// 16 bytes at voff + soff; the _nt form sets the non-temporal cache policy (data read once per call).
__device__ __forceinline__ uint4 buf_ld16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint4 buf_ld16_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 2);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint2 buf_ld8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, 0);
  return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ uint32_t buf_ld4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0);
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte streaming load (non-temporal: weights are read once per call and should not evict reusable lines)
__device__ __forceinline__ uint4 load16_stream(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// int8 weights as exact 16-bit values (u = q ^ 0x80 = q + 128, 0..255, used by the W8A16 kernels).
// four bytes b0..b3 (each < 256) as two 16-bit pairs (M + b0, M + b1), (M + b2, M + b3) above the magic byte M
__device__ __forceinline__ uint32_t w8a_pair_lo(uint32_t magic, uint32_t bytes) {
  return __builtin_amdgcn_perm(magic, bytes, 0x04010400u);
}
__device__ __forceinline__ uint32_t w8a_pair_hi(uint32_t magic, uint32_t bytes) {
  return __builtin_amdgcn_perm(magic, bytes, 0x04030402u);
}

// bytes 2h, 2h + 1 of w (each < 256, exact in bf16) as one packed bf16 pair
__device__ __forceinline__ uint32_t w8a_bf16_pair(uint32_t w, int h) {
  typedef float f32x2_w8_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_w8_t __attribute__((ext_vector_type(2)));
  const f32x2_w8_t f = {(float)((w >> (16 * h)) & 0xffu), (float)((w >> (16 * h + 8)) & 0xffu)};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_w8_t));
}

// nibble j (bits 4j..4j+3) of a packed word
__device__ __forceinline__ uint32_t nibble(uint32_t w, int j) { return (w >> (4 * j)) & 0xFu; }

__device__ __forceinline__ float raw_bits_to_f32(uint32_t raw, int dt) {
  return dt == FG_F32 ? __builtin_bit_cast(float, raw)
                      : (dt == FG_BF16 ? bf16_bits_to_f32(raw) : f16_bits_to_f32((uint16_t)raw));
}

// Element i of a 16- or 32-bit float array as raw bits (converted after the wait by raw_bits_to_f32).
__device__ __forceinline__ uint32_t load_raw(const void* p, int dt, int64_t i) {
  return dt == FG_F32 ? static_cast<const uint32_t*>(p)[i] : (uint32_t) static_cast<const uint16_t*>(p)[i];
}

// ----------------------------------------------------------------------------------------------- host helpers
// Compute units of the current device, queried once per device.
inline int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  (void)hipGetDevice(&dev);
  if (dev < 0 || dev >= 64) dev = 0;
  int cus = cache[dev].load(std::memory_order_relaxed);
  if (cus == 0) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cache[dev].store(cus, std::memory_order_relaxed);
  }
  return cus;
}

// Channel blocks per workgroup (1, 2 or 4, with that many times ks wavefronts within maxw): the count whose workgroups
// spread most evenly over the CUs, by busy fraction (workgroups / cus) / ceil(workgroups / cus) -- all are resident at
// once, so 1.25 workgroups per CU take as long as 2 (measured 2x slower) -- the widest on ties: gate+up (448 blocks of
// 64 channels) runs 5-7% (W4) and 13% (W8A16) faster as 224 workgroups of two blocks than as 448 of one.
inline int skinny_balance(int nblk, int ks, int maxw, int cus) {
  int best = 1;
  double best_eff = -1.0;
  for (int bw = 1; bw <= 4 && bw * ks <= maxw; bw *= 2) {
    const int wgs = (nblk + bw - 1) / bw;
    const double per_cu = (double)wgs / cus;
    const double eff = per_cu / ((wgs + cus - 1) / cus);
    if (eff > best_eff - 1e-9) {
      best = bw;
      best_eff = eff > best_eff ? eff : best_eff;
    }
  }
  return best;
}

}  // namespace fg
