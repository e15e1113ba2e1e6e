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

// ------------------------------------------------------------------------------------------------ GEMV (tiled)
constexpr int kTileMaxWaves = 12;  // wavefronts per workgroup of the tiled GEMV (three per SIMD)

constexpr int kStageU = 8;         // items per thread and pass of the tile staging

// Wavefront cap of a tiled-GEMV variant, from its register need (fetch buffers grow with the chunks per lane S, x
// pairs and accumulators with the rows of x MT): three waves per SIMD leave 168 VGPRs, two leave 256, one 512.
__host__ __device__ constexpr int w4_tile_max_waves(int mt, int s) {
  return mt == 1 ? (s <= 2 ? kTileMaxWaves : 8) : (mt == 2 ? (s <= 6 ? 8 : 4) : (s <= 3 ? 8 : 4));
}

// Sum of a value over the four lanes of an aligned quad (row-local DPP, no LDS traffic).  Every lane of the quad gets
// the same total, (v0 + v1) + (v2 + v3) in one order.
__device__ __forceinline__ float quad_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
  return v;
}

// Stage everything a tile of TN channels [tile0, tile0+TN) reads besides qweight into LDS:
//   xq[(m*4 + i) * KC + c] = word 4c+i of x row m as 16-bit pairs (x0,x2) (x1,x3) (x4,x6) (x5,x7), the order in
//                            which the byte-permute unpack produces nibble pairs;  xs[m*KC + c] = fp32 sum of chunk c;
//   ssc[g*TN + r] = fp32 scale of channel tile0+r in group g;  szb[g*TN + r] = fp32 (B + zero-point);
//   sbias[r] = fp32 bias (0 without bias).
// Each pass first issues every global load it needs (up to kStageU x words and kStageU scales per thread, one zero
// word and one bias value), then converts and stores, so a pass costs one memory round trip; decode shapes need a
// single pass.  Item indices are split with multiply-high division.
template <int MT, bool XBF16>
__device__ __forceinline__ void stage_tile(const uint16_t* __restrict__ x, int64_t ldx,
                                           const int32_t* __restrict__ perm, const void* __restrict__ scales, int sdt,
                                           int64_t lds, const int32_t* __restrict__ zeros, int64_t ldz,
                                           const void* __restrict__ bias, int bdt, int M, int N, int K, int KW, int KC,
                                           int G, int TN, int tile0, int nthr, uint4* xq, float* xs, float* ssc,
                                           float* szb, float* sbias) {
  constexpr float kBias = XBF16 ? 128.f : 1024.f;
  const int tid = threadIdx.x;
  const int nw = 4 * KC;       // x words per row, padded to whole chunks
  const int nx = MT * nw;      // item u = m * nw + w
  const int ns = G * TN;
  const int zpr = TN / 8;      // zero words per group row of the tile (tile0 and TN are multiples of 8)
  const int nz = G * zpr;
  const FastDiv div_w(nw), div_tn(TN), div_z(zpr);
  const int per = kStageU * nthr;
  const int passes = max(max((nx + per - 1) / per, (ns + per - 1) / per),
                         max((nz + nthr - 1) / nthr, (TN + nthr - 1) / nthr));
  const bool vec = perm == nullptr && (K & 7) == 0 && (ldx & 7) == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
  for (int p = 0; p < passes; ++p) {
    uint4 xr[kStageU];
    uint32_t sr[kStageU];
#pragma unroll
    for (int j = 0; j < kStageU; ++j) {
      const int u = (p * kStageU + j) * nthr + tid;
      const int m = (int)div_w.div((uint32_t)u), w = u - m * nw;
      xr[j] = make_uint4(0u, 0u, 0u, 0u);
      if (u < nx && m < M && w < KW) {
        const uint16_t* xrow = x + (int64_t)m * ldx;
        if (vec) {
          xr[j] = reinterpret_cast<const uint4*>(xrow)[w];
        } else {
          uint32_t h[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int k = 8 * w + e;
            h[e] = k < K ? xrow[perm ? perm[k] : k] : 0u;
          }
          xr[j] = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
        }
      }
    }
    // one dtype branch around the whole batch keeps the scale loads back to back
    if (sdt == FG_F32) {
#pragma unroll
      for (int j = 0; j < kStageU; ++j) {
        const int t = (p * kStageU + j) * nthr + tid;
        const int g = (int)div_tn.div((uint32_t)t), r = t - g * TN;
        if (t < ns) sr[j] = static_cast<const uint32_t*>(scales)[(int64_t)g * lds + min(tile0 + r, N - 1)];
      }
    } else {
#pragma unroll
      for (int j = 0; j < kStageU; ++j) {
        const int t = (p * kStageU + j) * nthr + tid;
        const int g = (int)div_tn.div((uint32_t)t), r = t - g * TN;
        if (t < ns) sr[j] = static_cast<const uint16_t*>(scales)[(int64_t)g * lds + min(tile0 + r, N - 1)];
      }
    }
    const int tz = p * nthr + tid;
    const int gz = (int)div_z.div((uint32_t)tz), vz = tz - gz * zpr;
    uint32_t zr = 0x88888888u;
    if (zeros && tz < nz) zr = (uint32_t)zeros[(int64_t)gz * ldz + min(tile0 / 8 + vz, (N - 1) / 8)];
    uint32_t br = 0u;
    if (bias && tz < TN) br = load_raw(bias, bdt, min(tile0 + tz, N - 1));

    // ---- convert and store
#pragma unroll
    for (int j = 0; j < kStageU; ++j) {
      const int u = (p * kStageU + j) * nthr + tid;
      if (u < nx) {  // whole quads: nx and the quad's first item are multiples of 4
        const int m = (int)div_w.div((uint32_t)u), w = u - m * nw;
        const uint32_t e4[4] = {xr[j].x, xr[j].y, xr[j].z, xr[j].w};
        uint32_t h[8];
        float sum = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          h[2 * e] = e4[e] & 0xffffu;
          h[2 * e + 1] = e4[e] >> 16;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) sum += x_to_f32<XBF16>(h[e]);
        sum = quad_sum(sum);  // the four words of a chunk sit in four consecutive lanes
        const int c = w >> 2, i = w & 3;
        xq[(m * 4 + i) * KC + c] = make_uint4(h[0] | (h[2] << 16), h[1] | (h[3] << 16), h[4] | (h[6] << 16),
                                              h[5] | (h[7] << 16));
        if (i == 0) xs[m * KC + c] = sum;
      }
    }
#pragma unroll
    for (int j = 0; j < kStageU; ++j) {
      const int t = (p * kStageU + j) * nthr + tid;
      if (t < ns) ssc[t] = raw_bits_to_f32(sr[j], sdt);
    }
    if (tz < nz) {
#pragma unroll
      for (int e = 0; e < 8; ++e) szb[gz * TN + 8 * vz + e] = kBias + (float)nibble(zr, e);
    }
    if (tz < TN) sbias[tz] = raw_bits_to_f32(br, bias ? bdt : FG_F32);
  }
}

// LDS bytes of the tiled GEMV: x pair units + chunk sums, then per-tile fp32 scales and fp32 (B + zero) [G][TN],
// then the tile's fp32 bias [TN].
__host__ __device__ inline size_t w4_gemv_tile_scale_offset(int mt, int KC) {
  return ((size_t)mt * KC * (4 * 16 + 4) + 15) / 16 * 16;  // 16-byte aligned for float4 reads
}

size_t w4_gemv_tile_lds_bytes(int mt, int K, int G, int TN) {
  const int KW = (K + 7) / 8, KC = (KW + 3) / 4;
  return w4_gemv_tile_scale_offset(mt, KC) + (size_t)G * TN * 8 + (size_t)TN * 4;
}

struct W4TilePlan {
  int s;       // 16-byte chunks per lane and channel
  int tn;      // channels per workgroup tile
  int waves;   // wavefronts per workgroup
  size_t lds;  // dynamic LDS bytes
};

// y[M,N] = x[M,K] @ dequant(W)^T (+bias) for M <= MT, K <= 2048*S, group size a multiple of 32 (or one group).
// Workgroup = one tile of TN consecutive output channels (TN a multiple of 8, sized by the host so that the tiles
// spread evenly over the CUs, one workgroup each); its `waves` wavefronts take the tile's 4-channel row blocks
// round-robin.  The tile's x, scales, zero-points and bias are staged into LDS in one memory round trip (the [G, N]
// scale layout otherwise costs one cache line per group per block), converted once to fp32 scale and fp32 (B + zero).
// A block's S chunk loads per channel are issued together; the first block's loads go out before the staging, and
// for S <= 2 the next block is fetched while the current one is computed.  Nibble pairs (q0,q2) (q1,q3) (q4,q6) (q5,q7) of a word come from two masks and
// four byte-permutes against the magic exponent byte (bf16 0x43: 128+q, fp16 0x64: 1024+q).
// Requires ldq % 4 == 0 and a 16-byte aligned qweight.
template <int MT, int S, bool XBF16>
__global__ void __launch_bounds__(w4_tile_max_waves(MT, S) * kWave) w4_gemv_tile_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const int32_t* __restrict__ qw, int64_t ldq,
    const void* __restrict__ scales, int sdt, int64_t lds, const int32_t* __restrict__ zeros, int64_t ldz,
    const int32_t* __restrict__ perm, const void* __restrict__ bias, int bdt, uint16_t* __restrict__ y, int64_t ldy,
    int M, int N, int K, int gs, int G, int TN, int waves) {
  constexpr int R = 4;
  constexpr bool PF = S <= 2;
  constexpr uint32_t kMagicBytes = XBF16 ? 0x43434343u : 0x64646464u;
  extern __shared__ __align__(16) uint8_t smem[];
  const int KW = (K + 7) / 8;
  const int KC = (KW + 3) / 4;
  uint4* xq = reinterpret_cast<uint4*>(smem);
  float* xs = reinterpret_cast<float*>(smem + (size_t)MT * 4 * KC * 16);
  float* ssc = reinterpret_cast<float*>(smem + w4_gemv_tile_scale_offset(MT, KC));
  float* szb = ssc + (size_t)G * TN;
  float* sbias = szb + (size_t)G * TN;

  const int lane = threadIdx.x & (kWave - 1);
  // Wave-uniform (scalar) block index: the block loop then branches on scalars and row addresses are scalar math.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int tile0 = blockIdx.x * TN;
  const int rows = min(TN, N - tile0);
  const int nblk = (rows + R - 1) / R;
  const int64_t ldq4 = ldq / 4;
  const uint4* __restrict__ qw4 = reinterpret_cast<const uint4*>(qw);
  const bool full = (KC % kWave) == 0 && KC == S * kWave;  // every chunk slot of every lane is real

  // Branch-free fetch of one 4-channel block: rows past N re-read row N-1 and chunk slots past KC re-read chunk KC-1
  // (their products are skipped), so every lane issues the same straight-line run of 16-byte loads.
  int cl[S];
#pragma unroll
  for (int i = 0; i < S; ++i) cl[i] = min(lane + kWave * i, KC - 1);
  auto fetch = [&](int blk, uint4 (&w)[R][S]) {
    const int n0 = tile0 + blk * R;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint4* rp = qw4 + (int64_t)min(n0 + r, N - 1) * ldq4;
#pragma unroll
      for (int i = 0; i < S; ++i) w[r][i] = load16_stream(rp + cl[i]);
    }
  };

  uint4 wa[R][S], wb[R][S];
  int blk = wave;
  fetch(min(blk, nblk - 1), wa);  // weight bytes are in flight while x, scales and zeros are staged

  stage_tile<MT, XBF16>(x, ldx, perm, scales, sdt, lds, zeros, ldz, bias, bdt, M, N, K, KW, KC, G, TN, tile0,
                        waves * kWave, xq, xs, ssc, szb, sbias);
  __syncthreads();

  auto compute = [&](int blk, const uint4 (&w)[R][S]) {
    const int r0 = blk * R;
    float acc[R * MT];
#pragma unroll
    for (int i = 0; i < R * MT; ++i) acc[i] = 0.f;
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const int c = lane + kWave * i;
      if (!full && c >= KC) continue;
      const int g = (32 * c) / gs;
      const float4 sc4 = *reinterpret_cast<const float4*>(ssc + g * TN + r0);
      const float4 zb4 = *reinterpret_cast<const float4*>(szb + g * TN + r0);
      const float sc[R] = {sc4.x, sc4.y, sc4.z, sc4.w};
      const float zb[R] = {zb4.x, zb4.y, zb4.z, zb4.w};
      uint4 xu[MT][4];
      float xsum[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m) {
#pragma unroll
        for (int q = 0; q < 4; ++q) xu[m][q] = xq[(m * 4 + q) * KC + c];
        xsum[m] = xs[m * KC + c];
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float d[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) d[m] = -zb[r] * xsum[m];
        const uint32_t wq[4] = {w[r][i].x, w[r][i].y, w[r][i].z, w[r][i].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          // nibble pairs (q0,q2) (q1,q3) (q4,q6) (q5,q7) as exact 16-bit floats B + q
          const uint32_t lo = wq[q] & 0x0F0F0F0Fu, hi = (wq[q] >> 4) & 0x0F0F0F0Fu;
          const uint32_t p0 = __builtin_amdgcn_perm(kMagicBytes, lo, 0x04010400u);
          const uint32_t p1 = __builtin_amdgcn_perm(kMagicBytes, hi, 0x04010400u);
          const uint32_t p2 = __builtin_amdgcn_perm(kMagicBytes, lo, 0x04030402u);
          const uint32_t p3 = __builtin_amdgcn_perm(kMagicBytes, hi, 0x04030402u);
#pragma unroll
          for (int m = 0; m < MT; ++m) {
            d[m] = dot2_acc<XBF16>(xu[m][q].x, p0, d[m]);
            d[m] = dot2_acc<XBF16>(xu[m][q].y, p1, d[m]);
            d[m] = dot2_acc<XBF16>(xu[m][q].z, p2, d[m]);
            d[m] = dot2_acc<XBF16>(xu[m][q].w, p3, d[m]);
          }
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r * MT + m] = __builtin_fmaf(sc[r], d[m], acc[r * MT + m]);
      }
    }
    const float tot = wave_transpose_sum<R * MT>(acc, lane);
    constexpr int span = kWave / (R * MT);
    if ((lane % span) == 0) {
      const int idx = lane / span;
      const int r = idx / MT, m = idx - (idx / MT) * MT;
      const int n = tile0 + r0 + r;
      if (r0 + r < rows && m < M) {
        const float v = tot + sbias[r0 + r];
        y[(int64_t)m * ldy + n] = XBF16 ? f32_to_bf16_bits_hw(v) : f32_to_f16_bits(v);
      }
    }
  };

  const int cnt = blk < nblk ? (nblk - 1 - blk) / waves + 1 : 0;  // blocks of this wave: blk, blk + waves, ...
  if constexpr (PF) {
    // Counted loop over pairs while at least three blocks remain, then a peeled tail of one or two blocks: every
    // path into the loop header has only buffer A in flight, so compute on one buffer waits only for its own loads
    // while the other buffer's loads stay in flight, and no block is fetched without being used.
    int left = cnt;
    for (; left > 2; left -= 2) {
      fetch(blk + waves, wb);
      compute(blk, wa);
      fetch(blk + 2 * waves, wa);
      compute(blk + waves, wb);
      blk += 2 * waves;
    }
    if (left == 2) {
      fetch(blk + waves, wb);
      compute(blk, wa);
      compute(blk + waves, wb);
    } else if (left == 1) {
      compute(blk, wa);
    }
  } else {
    for (int i = 0; i < cnt; ++i, blk += waves) {
      if (i) fetch(blk, wa);
      compute(blk, wa);
    }
  }
}


// ------------------------------------------------------------------------------------------------ GEMV (split-K)
// w4_gemv_split_kernel MODE: the scale type of the FAST forms, plus kSplitSz8 for scales / zero words blocked by 8
// channels ([N / 8][G][8] 16-bit scales, [N / 8][G] zero words) instead of the portable [G, lds] / [G, ldz]
enum { kSplitGeneral = 0, kSplitF16Scales = 1, kSplitBf16Scales = 2, kSplitSz8 = 4 };
// Decode GEMV for M <= MT <= 4 with no LDS on the hot path.  A wavefront owns R consecutive output channels and one K
// slice of at most S 32-column chunks per lane (chunk c = slice start + lane + 64 i); the K slices of a channel block
// are the KS wavefronts of one workgroup, summed in a fixed order through LDS at the end.  The lane's x chunks are read
// once (they are cache resident: every wavefront reads the same x), put into the nibble-pair order of the weight
// unpack, and kept in registers with their sums; the R scales of a chunk's group and the zero-point word come straight
// from global memory next to the weights.  Every wavefront is independent until the final sum, so many of them per CU
// keep HBM busy while others compute.
// The FAST modes (N % R == 0, K % 32 == 0, fp16 or bf16 scales with lds % 8 == 0, 16-byte aligned x and scales,
// ldx % 8 == 0, no perm, every operand spanning < 4 GiB; the scale type is a template parameter) issue every load of
// the wavefront unconditionally, back to back, in the order of first use: a load under a branch, or a branch on the
// scale type between loads and their use, makes the compiler wait for all earlier loads.  They are buffer loads: the
// per-lane offset (the chunk) is one 32-bit value and the row parts, the same for the whole wavefront, go in scalar
// registers, so a row costs no 64-bit address arithmetic.  Symmetric weights then read a dummy word (`zeros` points at
// any valid memory, ldz = 0) and replace it by 0x88888888.  The general form takes ragged N, K tails, fp32 scales,
// unaligned or permuted x with per-element loads.
//   gs32: group size / 32 (groups are whole chunks), 0 for one group per row.
// Threads per workgroup at most (BW * KS wavefronts): 512 for four rows of x, which need more than 128 registers.
constexpr int w4_split_max_threads(int mt) { return mt == 4 ? 512 : 1024; }

// Launch constants of the split GEMV, computed on the host so that the kernel prologue (run by every wavefront at the
// same moment, on the CU's shared scalar unit) has no integer division before the loads go out.
struct SplitArgs {
  int KC;         // 32-column chunks of K
  int cps;        // chunks per K slice (the last slice may be shorter)
  int gs32;       // group size / 32, 0 for one group per row
  uint32_t gmul;  // group of chunk c = umulhi(c, gmul) when gs32 > 1 (floor((2^32 - 1) / gs32) + 1)
  uint32_t qbytes, xbytes, sbytes, zbytes;  // FAST: byte spans of qweight, x, scales, zeros (each < 2^32)
  uint32_t sz8_block;  // kSplitSz8: bytes of one 8-channel block of scales (G * 16)
};

// Workgroup: blockDim.x = 64 * BW (one wavefront per channel block), blockDim.y = KS (one row of wavefronts per K
// slice).
template <int MT, int S, int R, bool XBF16, int MODE>
__global__ void __launch_bounds__(w4_split_max_threads(MT)) w4_gemv_split_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const int32_t* __restrict__ perm, const int32_t* __restrict__ qw,
    int64_t ldq, const void* __restrict__ scales, int sdt, int64_t lds, const int32_t* __restrict__ zeros, int64_t ldz,
    int hasz, const void* __restrict__ bias, int bdt, uint16_t* __restrict__ y, int64_t ldy, int M, int N, int K,
    SplitArgs a) {
  static_assert(R * MT == 4 || R * MT == 8 || R * MT == 16, "rows x batch must be 4, 8 or 16");
  constexpr bool FAST = MODE != kSplitGeneral, SZ8 = (MODE & kSplitSz8) != 0;
  constexpr int SM = MODE & 3;  // scale type
  constexpr uint32_t kMagicBytes = XBF16 ? 0x43434343u : 0x64646464u;
  constexpr uint32_t kOnes = XBF16 ? 0x3f803f80u : 0x3c003c00u;  // (1, 1) as bf16 / fp16 pairs
  constexpr float kB = XBF16 ? 128.f : 1024.f;
  __shared__ float red[16][R * MT];
  const int lane = threadIdx.x & (kWave - 1);
  const int wb = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // channel block within the workgroup
  const int ks = __builtin_amdgcn_readfirstlane(threadIdx.y);         // K slice
  const int BW = (int)(blockDim.x / kWave), KS = (int)blockDim.y;
  const int KC = a.KC;
  const int blk = blockIdx.x * BW + wb;
  const int n0 = blk * R;
  const int nr = min(n0, N - R);  // FAST: first row read (blocks past the end re-read the last block)
  const int c0 = ks * a.cps, c1 = min(c0 + a.cps, KC);
  const int64_t ldq4 = ldq / 4;
  const uint4* __restrict__ qw4 = reinterpret_cast<const uint4*>(qw);
  const __amdgpu_buffer_rsrc_t rq = buf_rsrc(qw, a.qbytes);
  const __amdgpu_buffer_rsrc_t rx = buf_rsrc(x, a.xbytes);
  const __amdgpu_buffer_rsrc_t rs = buf_rsrc(scales, a.sbytes);
  const __amdgpu_buffer_rsrc_t rz = buf_rsrc(zeros, a.zbytes);

  int cl[S], gl[S];
  bool ok[S];
#pragma unroll
  for (int i = 0; i < S; ++i) {
    const int c = c0 + lane + kWave * i;
    ok[i] = c < c1;
    cl[i] = min(c, KC - 1);
    gl[i] = a.gs32 > 1 ? (int)__umulhi((uint32_t)cl[i], a.gmul) : (a.gs32 == 1 ? cl[i] : 0);
  }
  // Loads in the order of first use for one row of x: x (its chunk sums start every row), scales and zero words, then
  // the weights row by row (general form: rows past N re-read row N-1).  With 2-4 rows of x the weights go first:
  // holding the raw x of every row through the weight loads would spill.
  uint4 xv[MT][S][4];
  auto load_x = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int i = 0; i < S; ++i) {
        const uint16_t* xr = x + (int64_t)min(m, M - 1) * ldx;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int wi = 4 * cl[i] + q;
          if constexpr (FAST) {
            xv[m][i][q] = buf_ld16(rx, (uint32_t)cl[i] * 64u + 16u * q, (uint32_t)min(m, M - 1) * (uint32_t)ldx * 2u);
          } else {
            uint32_t h[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const int k = 8 * wi + e;
              h[e] = k < K ? xr[perm ? perm[k] : k] : 0u;
            }
            xv[m][i][q] = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
          }
        }
      }
  };
  uint32_t sraw[S][FAST ? (R + 1) / 2 : R];  // FAST: two 16-bit scales per word
  uint32_t zw[S][(R + 7) / 8];
  auto load_sz = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const int64_t srow = (int64_t)gl[i] * lds;
      if constexpr (SZ8) {  // group gl's 16 bytes (per lane) in the blocks of the wavefront's channels (uniform)
        const uint32_t sv = (uint32_t)gl[i] * 16u, b8 = (uint32_t)nr / 8u;
        if constexpr (R == 4) {
          const uint2 t = buf_ld8(rs, sv, b8 * a.sz8_block + (uint32_t)(nr & 7) * 2u);
          sraw[i][0] = t.x;
          sraw[i][1] = t.y;
        } else {
#pragma unroll
          for (int h = 0; h < R / 8; ++h) {
            const uint4 t = buf_ld16(rs, sv, (b8 + (uint32_t)h) * a.sz8_block);
            sraw[i][4 * h] = t.x;
            sraw[i][4 * h + 1] = t.y;
            sraw[i][4 * h + 2] = t.z;
            sraw[i][4 * h + 3] = t.w;
          }
        }
#pragma unroll
        for (int h = 0; h < (R + 7) / 8; ++h)
          zw[i][h] = buf_ld4(rz, (uint32_t)gl[i] * 4u, (b8 + (uint32_t)h) * (a.sz8_block / 4u));
      } else if constexpr (FAST) {  // group row gl * lds (per lane, < 2^24 each) + the block's first channel (uniform)
        const uint32_t sv = __umul24((uint32_t)gl[i], (uint32_t)lds) * 2u;
        if constexpr (R == 4) {
          const uint2 t = buf_ld8(rs, sv, (uint32_t)nr * 2u);
          sraw[i][0] = t.x;
          sraw[i][1] = t.y;
        } else {
#pragma unroll
          for (int h = 0; h < R / 8; ++h) {
            const uint4 t = buf_ld16(rs, sv, (uint32_t)(nr + 8 * h) * 2u);
            sraw[i][4 * h] = t.x;
            sraw[i][4 * h + 1] = t.y;
            sraw[i][4 * h + 2] = t.z;
            sraw[i][4 * h + 3] = t.w;
          }
        }
        const uint32_t zv = __umul24((uint32_t)gl[i], (uint32_t)ldz) * 4u;
#pragma unroll
        for (int h = 0; h < (R + 7) / 8; ++h) zw[i][h] = buf_ld4(rz, zv, (uint32_t)(nr / 8 + h) * 4u);
      } else {
#pragma unroll
        for (int r = 0; r < R; ++r) sraw[i][r] = load_raw(scales, sdt, srow + min(n0 + r, N - 1));
#pragma unroll
        for (int h = 0; h < (R + 7) / 8; ++h)
          zw[i][h] = (uint32_t)zeros[(int64_t)gl[i] * ldz + min(n0 / 8 + h, (N - 1) / 8)];
      }
    }
  };
  uint4 w[R][S];
  const uint32_t ldqb = (uint32_t)ldq * 4u;  // FAST: bytes per weight row
  auto load_w = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int i = 0; i < S; ++i) {
        if constexpr (FAST) {
          w[r][i] = buf_ld16_nt(rq, (uint32_t)cl[i] * 16u, (uint32_t)nr * ldqb + (uint32_t)r * ldqb);
        } else {
          w[r][i] = load16_stream(qw4 + (int64_t)min(n0 + r, N - 1) * ldq4 + cl[i]);
        }
      }
  };
  if constexpr (MT == 1) {
    load_x();
    load_sz();
    load_w();
  } else {
    load_w();
    load_sz();
    load_x();
  }

  // x chunks in nibble-pair order, and their sums
  uint4 xu[MT][S][4];
  float xs[MT][S];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int i = 0; i < S; ++i) {
      float sum = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint4 v = xv[m][i][q];
        // (x0,x1)(x2,x3)(x4,x5)(x6,x7) -> (x0,x2)(x1,x3)(x4,x6)(x5,x7), the order of the nibble pairs below
        xu[m][i][q] = make_uint4(__builtin_amdgcn_perm(v.y, v.x, 0x05040100u), __builtin_amdgcn_perm(v.y, v.x, 0x07060302u),
                                 __builtin_amdgcn_perm(v.w, v.z, 0x05040100u), __builtin_amdgcn_perm(v.w, v.z, 0x07060302u));
        sum = dot2_acc<XBF16>(xu[m][i][q].x, kOnes, sum);
        sum = dot2_acc<XBF16>(xu[m][i][q].y, kOnes, sum);
        sum = dot2_acc<XBF16>(xu[m][i][q].z, kOnes, sum);
        sum = dot2_acc<XBF16>(xu[m][i][q].w, kOnes, sum);
      }
      xs[m][i] = sum;
    }

  const int zsh = R == 4 ? ((FAST ? nr : n0) & 7) : 0;  // nibble of the block's first row in its zero word
  float acc[R * MT];
#pragma unroll
  for (int i = 0; i < R * MT; ++i) acc[i] = 0.f;
#pragma unroll
  for (int i = 0; i < S; ++i) {
    if (!ok[i]) continue;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float sc;
      if constexpr (SM == kSplitF16Scales) {
        sc = f16_bits_to_f32((uint16_t)((r & 1) ? sraw[i][r >> 1] >> 16 : sraw[i][r >> 1]));
      } else if constexpr (SM == kSplitBf16Scales) {
        sc = __uint_as_float((r & 1) ? sraw[i][r >> 1] & 0xffff0000u : sraw[i][r >> 1] << 16);
      } else {
        sc = raw_bits_to_f32(sraw[i][r], sdt);
      }
      const uint32_t zword = hasz ? zw[i][r / 8] : 0x88888888u;
      const float zb = kB + (float)nibble(zword, (r + zsh) & 7);
      float d[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m) d[m] = -zb * xs[m][i];
      const uint32_t wq[4] = {w[r][i].x, w[r][i].y, w[r][i].z, w[r][i].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t lo = wq[q] & 0x0F0F0F0Fu, hi = (wq[q] >> 4) & 0x0F0F0F0Fu;
        const uint32_t p0 = __builtin_amdgcn_perm(kMagicBytes, lo, 0x04010400u);
        const uint32_t p1 = __builtin_amdgcn_perm(kMagicBytes, hi, 0x04010400u);
        const uint32_t p2 = __builtin_amdgcn_perm(kMagicBytes, lo, 0x04030402u);
        const uint32_t p3 = __builtin_amdgcn_perm(kMagicBytes, hi, 0x04030402u);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          d[m] = dot2_acc<XBF16>(xu[m][i][q].x, p0, d[m]);
          d[m] = dot2_acc<XBF16>(xu[m][i][q].y, p1, d[m]);
          d[m] = dot2_acc<XBF16>(xu[m][i][q].z, p2, d[m]);
          d[m] = dot2_acc<XBF16>(xu[m][i][q].w, p3, d[m]);
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
      y[(int64_t)m * ldy + n0 + r] = XBF16 ? f32_to_bf16_bits_hw(v) : f32_to_f16_bits(v);
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

// Launch shape of the split-K GEMV: S chunks per lane (1 while K <= 32768, else 2 for one row of x), KS =
// ceil(chunks / (64 S)) K slices (at most 16), R rows per wavefront (16 for one row of x over 8 or more slices, 8 for
// wide outputs or long K, else 4; R * MT <= 16), BW channel blocks per workgroup (8 .. 16 wavefronts, 8 with four rows of x).  Returns false when the shape is outside its reach (four rows of x: K > 16384).
// sz8: the scales and zero words come as 8-channel blocks (fg_w4a16_gemv_sz8).
bool w4_gemv_split_plan(int mt, int N, int K, int* S, int* R, int* KS, int* BW, bool sz8) {
  const int KW = (K + 7) / 8, KC = (KW + 3) / 4;
  const int s = KC <= 16 * kWave ? 1 : (KC <= 32 * kWave && mt == 1 ? 2 : 0);
  if (s == 0) return false;
  const int ks = (KC + kWave * s - 1) / (kWave * s);
  const int per_cu = N / device_cus();
  // 8 rows for wide outputs or long K, else 4 (graph replays over a 1.2 GB ring, M = 1: gate+up 12.2 us with 8 rows in
  // 448 workgroups of 16 wavefronts against 13.2 with 16 rows in one workgroup per CU; qkv 4.75 against 5.03 with 8
  // rows): fewer rows per wavefront shorten the arithmetic left once a wavefront's last bytes arrive
  int r = (per_cu >= 64 || ks >= 4) ? 8 : 4;
  // one row of x split 8 or more ways over K: 16 rows per wavefront, half the wavefronts (K = 28672, N = 8192: 26.3 us
  // against 32.3 with 8 rows; K = 14336, 7 slices: level)
  if (mt == 1 && ks >= 8) r = 16;
  if (mt == 2) r = min(r, 8);
  if (mt == 4) r = 4;
  if (s == 2) r = 4;  // 8 rows x 2 chunks would spill
  const int max_waves = w4_split_max_threads(mt) / kWave;
  if (ks > max_waves) return false;
  // One workgroup per CU when the channel blocks divide evenly (measured best on all four Llama-3-8B shapes; uneven
  // counts such as 1.2-1.4 workgroups per CU cost up to 40%), else the widest workgroup for wide outputs (gate+up, 3584
  // blocks of 8 rows: 448 workgroups of 16 wavefronts 12.2 us against 12.6 for 896 of 8 and 14.4 for 1195 of 12) and
  // 8-16 wavefronts otherwise.
  const int nblk = (N + r - 1) / r, cus = device_cus();
  // two rows of x over wide outputs: two channel blocks per workgroup (4-8 wavefronts; M = 2, us, gate+up 15.8 against
  // 18.6 with the widest workgroups, K = 8192, N = 57344 56.0 against 62.5); one row over wide outputs with the scales
  // in 8-channel blocks likewise (graph replays, medians of five: gate+up 12.4 against 12.8-13.1 us, K = 8192,
  // N = 57344 42.6 against 46.4), where the portable scales keep the widest workgroups (gate+up 13.1 against 13.7)
  int bw = nblk >= 8 * cus ? (mt == 2 || (sz8 && mt == 1) ? 2 : max_waves / ks) : max(2, 8 / ks);
  if (nblk % cus == 0 && (nblk / cus) * ks <= max_waves) bw = nblk / cus;
  while (bw * ks > max_waves && bw > 1) --bw;
  *S = s; *R = r; *KS = ks; *BW = bw;
  return true;
}

template <int MT, int S, int R, bool XBF16>
static hipError_t launch_split_t(bool fast, bool sz8, const void* x, int64_t ldx, const int32_t* perm,
                                 const int32_t* qw, int64_t ldq, const void* scales, int sdt, int64_t lds,
                                 const int32_t* zeros, int64_t ldz, const void* bias, int bdt, void* y, int64_t ldy,
                                 int M, int N, int K, int gs32, int KS, int BW, hipStream_t s) {
  const int nblk = (N + R - 1) / R;
  const int hasz = zeros != nullptr;
  // symmetric weights: the zero word is read from qweight (always valid memory) and ignored
  const int32_t* zp = hasz ? zeros : qw;
  const int64_t ldzp = hasz ? ldz : 0;
  SplitArgs a;
  a.KC = ((K + 7) / 8 + 3) / 4;
  a.cps = (a.KC + KS - 1) / KS;
  a.gs32 = gs32;
  a.gmul = gs32 > 1 ? 0xffffffffu / (uint32_t)gs32 + 1u : 0u;
  const int64_t G = gs32 > 0 ? (a.KC + gs32 - 1) / gs32 : 1;
  // byte spans for the FAST buffer loads (split_fast checked each is < 2^32; unused by the general form)
  a.qbytes = fast ? (uint32_t)((int64_t)N * ldq * 4) : 0u;
  a.xbytes = fast ? (uint32_t)((int64_t)M * ldx * 2) : 0u;
  // sz8: [N / 8][G][8] scales and [N / 8][G] zero words (split_sz8_ok checked N % 8 == 0 and the spans)
  a.sbytes = fast ? (uint32_t)(G * (sz8 ? N : lds) * 2) : 0u;
  a.zbytes = fast ? (hasz ? (uint32_t)(G * (sz8 ? N / 8 : ldz) * 4) : a.qbytes) : 0u;
  a.sz8_block = (uint32_t)(G * 16);
  const dim3 grid((nblk + BW - 1) / BW), block(kWave * BW, KS);
  const bool bf = sdt == FG_BF16;
  auto kern = !fast ? w4_gemv_split_kernel<MT, S, R, XBF16, kSplitGeneral>
              : sz8 ? (bf ? w4_gemv_split_kernel<MT, S, R, XBF16, kSplitBf16Scales | kSplitSz8>
                          : w4_gemv_split_kernel<MT, S, R, XBF16, kSplitF16Scales | kSplitSz8>)
                    : (bf ? w4_gemv_split_kernel<MT, S, R, XBF16, kSplitBf16Scales>
                          : w4_gemv_split_kernel<MT, S, R, XBF16, kSplitF16Scales>);
  note_kernel("w4_gemv_split_kernel<%d,%d,%d,%s>%s KS=%d", MT, S, R, XBF16 ? "bf16" : "f16",
              !fast ? " general" : (sz8 ? " sz8" : ""), KS);
  hipLaunchKernelGGL(kern, grid, block, 0, s, static_cast<const uint16_t*>(x), ldx, perm, qw, ldq, scales, sdt, lds, zp,
                     ldzp, hasz, bias, bdt, static_cast<uint16_t*>(y), ldy, M, N, K, a);
  return hipGetLastError();
}

template <bool XBF16>
static hipError_t launch_split_x(int mt, int S, int R, bool fast, bool sz8, const void* x, int64_t ldx,
                                 const int32_t* perm, const int32_t* qw, int64_t ldq, const void* scales, int sdt,
                                 int64_t lds, const int32_t* zeros, int64_t ldz, const void* bias, int bdt, void* y,
                                 int64_t ldy, int M, int N, int K, int gs32, int KS, int BW, hipStream_t s) {
#define FG_SPLIT(MT_, S_, R_)                                                                                        \
  return launch_split_t<MT_, S_, R_, XBF16>(fast, sz8, x, ldx, perm, qw, ldq, scales, sdt, lds, zeros, ldz, bias, bdt, \
                                            y, ldy, M, N, K, gs32, KS, BW, s)
  if (mt == 1) {
    if (S == 2) FG_SPLIT(1, 2, 4);
    if (R == 4) FG_SPLIT(1, 1, 4);
    if (R == 8) FG_SPLIT(1, 1, 8);
    FG_SPLIT(1, 1, 16);
  }
  if (mt == 2) { if (R == 4) FG_SPLIT(2, 1, 4); FG_SPLIT(2, 1, 8); }
  FG_SPLIT(4, 1, 4);
#undef FG_SPLIT
}

// True when the split GEMV can take its branch-free form for these operands.
static bool split_fast(int R, const void* x, int64_t ldx, const int32_t* perm, const void* scales, int sdt,
                       int64_t lds, int64_t ldq, int64_t ldz, int M, int N, int K, int gs32) {
  const int64_t KC = (K + 31) / 32, G = gs32 > 0 ? (KC + gs32 - 1) / gs32 : 1;
  const int64_t lim = int64_t(1) << 32, lim24 = int64_t(1) << 24;  // buffer spans; 24-bit per-lane group offsets
  return perm == nullptr && (K % 32) == 0 && (N % R) == 0 && (ldx % 8) == 0 &&
         (reinterpret_cast<uintptr_t>(x) % 16) == 0 && sdt != FG_F32 && (lds % 8) == 0 &&
         (reinterpret_cast<uintptr_t>(scales) % 16) == 0 && (int64_t)N * ldq * 4 < lim &&
         (int64_t)M * ldx * 2 < lim && G * lds * 2 < lim && G * ldz * 4 < lim && lds < lim24 && ldz < lim24 &&
         G < lim24;
}

hipError_t launch_w4_gemv_split(int mt, bool xbf16, const void* x, int64_t ldx, const int32_t* qw, int64_t ldq,
                                const void* scales, int sdt, int64_t lds, const int32_t* zeros, int64_t ldz,
                                const int32_t* perm, const void* bias, int bdt, void* y, int64_t ldy, int M, int N,
                                int K, int gs, bool single_group, hipStream_t s) {
  int S, R, KS, BW;
  if (!w4_gemv_split_plan(mt, N, K, &S, &R, &KS, &BW, false)) return hipErrorInvalidValue;
  const int gs32 = single_group ? 0 : gs / 32;
  const bool fast = split_fast(R, x, ldx, perm, scales, sdt, lds, ldq, zeros ? ldz : 0, M, N, K, gs32);
  if (xbf16)
    return launch_split_x<true>(mt, S, R, fast, false, x, ldx, perm, qw, ldq, scales, sdt, lds, zeros, ldz, bias, bdt,
                                y, ldy, M, N, K, gs32, KS, BW, s);
  return launch_split_x<false>(mt, S, R, fast, false, x, ldx, perm, qw, ldq, scales, sdt, lds, zeros, ldz, bias, bdt,
                               y, ldy, M, N, K, gs32, KS, BW, s);
}

// The split GEMV's branch-free form reading scales / zero words blocked by 8 channels ([N / 8][G][8] 16-bit scales,
// [N / 8][G] zero words): each wavefront's scales and zero words of a K slice are one contiguous run instead of one
// strided word per group.
bool w4_gemv_sz8_ok(const void* x, int64_t ldx, const int32_t* qw, int64_t ldq, const void* scales8, int sdt, int M,
                    int N, int K, int gs) {
  int S, R, KS, BW;
  const int mt = M <= 1 ? 1 : (M <= 2 ? 2 : 4);
  if (M < 1 || M > 4 || !w4_gemv_split_plan(mt, N, K, &S, &R, &KS, &BW, false)) return false;
  const int gs32 = gs > 0 ? gs / 32 : 0;
  if ((gs > 0 && gs % 32 != 0) || N % 8 != 0 || (reinterpret_cast<uintptr_t>(qw) % 16) != 0 || (ldq % 4) != 0)
    return false;
  // the portable form's checks with the blocked arrays' strides (N per group row of scales, N / 8 of zero words)
  return split_fast(R, x, ldx, nullptr, scales8, sdt, N, ldq, N / 8, M, N, K, gs32);
}

hipError_t launch_w4_gemv_sz8(int mt, bool xbf16, const void* x, int64_t ldx, const int32_t* qw, int64_t ldq,
                              const void* scales8, int sdt, const int32_t* zeros8, const void* bias, int bdt, void* y,
                              int64_t ldy, int M, int N, int K, int gs, bool single_group, hipStream_t s) {
  int S, R, KS, BW;
  if (!w4_gemv_split_plan(mt, N, K, &S, &R, &KS, &BW, true)) return hipErrorInvalidValue;
  const int gs32 = single_group ? 0 : gs / 32;
  if (xbf16)
    return launch_split_x<true>(mt, S, R, true, true, x, ldx, nullptr, qw, ldq, scales8, sdt, N, zeros8, N / 8, bias,
                                bdt, y, ldy, M, N, K, gs32, KS, BW, s);
  return launch_split_x<false>(mt, S, R, true, true, x, ldx, nullptr, qw, ldq, scales8, sdt, N, zeros8, N / 8, bias,
                               bdt, y, ldy, M, N, K, gs32, KS, BW, s);
}

bool w4_gemv_split_ok(int mt, int N, int K) {
  int S, R, KS, BW;
  return w4_gemv_split_plan(mt, N, K, &S, &R, &KS, &BW, false);
}

// Whether the policy takes the split GEMV: its branch-free form applies to these operands, and the shape is not one
// where the tiled kernel measured faster (3-4 rows of x over wide outputs: at K=4096, N=28672 the tiled kernel takes
// 22 us against 28 us; at N=4096..6144 the split kernel is as fast or faster).
bool w4_gemv_split_preferred(int mt, const void* x, int64_t ldx, const int32_t* perm, const void* scales, int sdt,
                             int64_t lds, int64_t ldq, const int32_t* zeros, int64_t ldz, int M, int N, int K, int gs,
                             bool single_group) {
  int S, R, KS, BW;
  if (mt == 4 && N / device_cus() >= 64) return false;
  return w4_gemv_split_plan(mt, N, K, &S, &R, &KS, &BW, false) &&
         split_fast(R, x, ldx, perm, scales, sdt, lds, ldq, zeros ? ldz : 0, M, N, K, single_group ? 0 : gs / 32);
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

// Dense dequantisation to a 16-bit output: one wavefront per 2048 columns of one channel row, lane l converting
// columns c0 + 512 i + 8 l .. + 7 (i = 0..3) from one dword of qweight each, so every dword load reads 256 and every
// 16-byte store writes 1024 contiguous bytes per wavefront (a thread per 32 columns wrote 16 of every 64 bytes per
// store instruction and ran at 2.5-3.1 TB/s).  (q - z) * s = fma(q, s, -z * s) is exact in fp32 (both products and
// their sum are exact for |q - z| <= 15 and a 16-bit scale) and rounded once to nearest even by the packed hardware
// conversion -- the generic kernel's value, bit for bit.  Group of column c: c / gs by a multiply-high with the host's
// constant (gdiv = 0: one group).  Needs K % 32 == 0, groups of whole 32-column chunks (or one group), 16-bit scales,
// no g_idx, 4-byte aligned qweight, 16-byte aligned out with ldo % 8 == 0.
template <bool OBF16>
__global__ void __launch_bounds__(256) w4_dequant16_kernel(const int32_t* __restrict__ qw, int64_t ldq,
                                                           const uint16_t* __restrict__ scales, int sbf16, int64_t lds,
                                                           const int32_t* __restrict__ zeros, int64_t ldz,
                                                           uint16_t* __restrict__ out, int64_t ldo, int N, int K,
                                                           int wpr, uint32_t gdiv, uint32_t gmul) {
  typedef float f32x2_dq_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_dq_t __attribute__((ext_vector_type(2)));
  typedef _Float16 f16x2_dq_t __attribute__((ext_vector_type(2)));
  const int64_t wv = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  if (wv >= (int64_t)N * wpr) return;  // whole wavefronts
  const int lane = threadIdx.x & (kWave - 1);
  const int n = (int)(wv / wpr), c0 = (int)(wv - (int64_t)n * wpr) * 2048 + 8 * lane;
  const int32_t* qr = qw + (int64_t)n * ldq;
  uint16_t* orow = out + (int64_t)n * ldo;
  uint32_t w[4];
  float sc[4], cz[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = c0 + 512 * i;
    if (c < K) {
      w[i] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(qr) + c / 8);
      const uint32_t g = gdiv > 1 ? __umulhi((uint32_t)c, gmul) : (gdiv == 1 ? (uint32_t)c : 0u);
      const uint16_t sb = scales[(int64_t)g * lds + n];
      sc[i] = sbf16 ? bf16_bits_to_f32(sb) : f16_bits_to_f32(sb);
      const float z = zeros ? (float)nibble((uint32_t)zeros[(int64_t)g * ldz + n / 8], n & 7) : 8.f;
      cz[i] = -z * sc[i];
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = c0 + 512 * i;
    if (c < K) {
      const uint32_t lo = w[i] & 0x0F0F0F0Fu, hi = (w[i] >> 4) & 0x0F0F0F0Fu;  // nibbles 2j / 2j + 1 in byte j
      uint32_t h[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x2_dq_t v = {__builtin_fmaf((float)((lo >> (8 * j)) & 0xFFu), sc[i], cz[i]),
                              __builtin_fmaf((float)((hi >> (8 * j)) & 0xFFu), sc[i], cz[i])};
        if constexpr (OBF16) {
          h[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_dq_t));
        } else {
          h[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_dq_t));
        }
      }
      *reinterpret_cast<uint4*>(orow + c) = make_uint4(h[0], h[1], h[2], h[3]);
    }
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
  note_kernel("w4_gemv_kernel<%d,%d,%s>", MT, R, XBF16 ? "bf16" : "f16");
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

template <int MT, int S, bool XBF16>
static hipError_t launch_gemv_tile_t(const void* x, int64_t ldx, const int32_t* qw, int64_t ldq, const void* scales,
                                     int sdt, int64_t lds, const int32_t* zeros, int64_t ldz, const int32_t* perm,
                                     const void* bias, int bdt, void* y, int64_t ldy, int M, int N, int K, int gs,
                                     int G, const W4TilePlan& tp, hipStream_t s) {
  auto kern = w4_gemv_tile_kernel<MT, S, XBF16>;
  if (tp.lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)tp.lds);
    if (e != hipSuccess) return e;
  }
  const int blocks = (N + tp.tn - 1) / tp.tn;
  note_kernel("w4_gemv_tile_kernel<%d,%d,%s> TN=%d", MT, S, XBF16 ? "bf16" : "f16", tp.tn);
  hipLaunchKernelGGL(kern, dim3(blocks), dim3(tp.waves * kWave), tp.lds, s, static_cast<const uint16_t*>(x), ldx, qw,
                     ldq, scales, sdt, lds, zeros, ldz, perm, bias, bdt, static_cast<uint16_t*>(y), ldy, M, N, K, gs, G,
                     tp.tn, tp.waves);
  return hipGetLastError();
}

template <int MT, bool XBF16>
static hipError_t launch_gemv_tile_s(const void* x, int64_t ldx, const int32_t* qw, int64_t ldq, const void* scales,
                                     int sdt, int64_t lds, const int32_t* zeros, int64_t ldz, const int32_t* perm,
                                     const void* bias, int bdt, void* y, int64_t ldy, int M, int N, int K, int gs,
                                     int G, const W4TilePlan& tp, hipStream_t s) {
#define FG_GT(S_) \
  return launch_gemv_tile_t<MT, S_, XBF16>(x, ldx, qw, ldq, scales, sdt, lds, zeros, ldz, perm, bias, bdt, y, ldy, M, N, K, gs, G, tp, s)
  switch (tp.s) {
    case 1: FG_GT(1);
    case 2: FG_GT(2);
    case 3: FG_GT(3);
    case 4: FG_GT(4);
    case 5: FG_GT(5);
    case 6: FG_GT(6);
    case 7: FG_GT(7);
    default: FG_GT(8);
  }
#undef FG_GT
}

// Launch shape of the tiled GEMV.  Tiles: TN = 8 * ceil(N / (8 * CUs)) channels (or the caller's tile_n, rounded up
// to a multiple of 8), halved while the tile's LDS exceeds 160 KiB.  Wavefronts: the tile's ceil(TN/4) row blocks are
// shared evenly when a divisor in [4, cap] exists (the largest one), else min(blocks, cap), cap = w4_tile_max_waves.  Returns false when K is
// beyond the kernel's reach (more than 8 chunks per lane) or nothing fits in LDS.
bool w4_gemv_tile_plan(int mt, int N, int K, int G, int tile_n, W4TilePlan* tp) {
  const int KC = ((K + 7) / 8 + 3) / 4;
  const int S = (KC + 63) / 64;
  if (S > 8 || N <= 0) return false;
  int tn = tile_n > 0 ? (tile_n + 7) / 8 * 8 : 8 * ((N + 8 * device_cus() - 1) / (8 * device_cus()));
  tn = max(tn, 8);
  while (w4_gemv_tile_lds_bytes(mt, K, G, tn) > 160 * 1024 && tn > 8) tn = max(8, (tn / 2 + 7) / 8 * 8);
  const size_t shm = w4_gemv_tile_lds_bytes(mt, K, G, tn);
  if (shm > 160 * 1024) return false;
  const int nb = (tn + 3) / 4;
  const int cap = w4_tile_max_waves(mt, S);
  int waves = min(nb, cap);
  if (nb > cap) {
    for (int w = cap; w >= 4; --w)
      if (nb % w == 0) { waves = w; break; }
  }
  *tp = W4TilePlan{S, tn, waves, shm};
  return true;
}

bool w4_gemv_tile_ok(int mt, int N, int K, int G, int tile_n) {
  W4TilePlan tp;
  return w4_gemv_tile_plan(mt, N, K, G, tile_n, &tp);
}

hipError_t launch_w4_gemv_tile(int mt, bool xbf16, const void* x, int64_t ldx, const int32_t* qw, int64_t ldq,
                               const void* scales, int sdt, int64_t lds, const int32_t* zeros, int64_t ldz,
                               const int32_t* perm, const void* bias, int bdt, void* y, int64_t ldy, int M, int N,
                               int K, int gs, int G, int tile_n, hipStream_t s) {
  W4TilePlan tp;
  if (!w4_gemv_tile_plan(mt, N, K, G, tile_n, &tp)) return hipErrorInvalidValue;
#define FG_GTM(MT_, XB_) \
  return launch_gemv_tile_s<MT_, XB_>(x, ldx, qw, ldq, scales, sdt, lds, zeros, ldz, perm, bias, bdt, y, ldy, M, N, K, gs, G, tp, s)
  if (xbf16) {
    if (mt == 1) FG_GTM(1, true);
    if (mt == 2) FG_GTM(2, true);
    FG_GTM(4, true);
  } else {
    if (mt == 1) FG_GTM(1, false);
    if (mt == 2) FG_GTM(2, false);
    FG_GTM(4, false);
  }
#undef FG_GTM
}

hipError_t launch_w4_generic(const void* x, int64_t ldx, int xdt, const int32_t* qw, int64_t ldq, const void* scales,
                             int sdt, int64_t lds, const int32_t* zeros, int64_t ldz, const int32_t* perm,
                             const int32_t* g_idx, const void* bias, int bdt, void* y, int64_t ldy, int M, int N,
                             int K, int gs, hipStream_t s) {
  const int64_t nwork = (int64_t)N * ((M + 3) / 4);
  const int64_t blocks = (nwork + 3) / 4;
  note_kernel("w4_generic_kernel");
  hipLaunchKernelGGL(w4_generic_kernel, dim3((unsigned)blocks), dim3(256), 0, s, static_cast<const uint16_t*>(x), ldx,
                     xdt, qw, ldq, scales, sdt, lds, zeros, ldz, perm, g_idx, bias, bdt, static_cast<uint16_t*>(y),
                     ldy, M, N, K, gs);
  return hipGetLastError();
}

hipError_t launch_w4_dequant(const int32_t* qw, int64_t ldq, const void* scales, int sdt, int64_t lds,
                             const int32_t* zeros, int64_t ldz, const int32_t* g_idx, void* out, int odt, int64_t ldo,
                             int N, int K, int gs, hipStream_t s) {
  const bool one_group = gs >= K;
  if (!g_idx && (odt == FG_BF16 || odt == FG_F16) && (sdt == FG_BF16 || sdt == FG_F16) && K % 32 == 0 &&
      group_div_exact(K, gs, one_group ? 1 : 2, 1) && (gs % 32 == 0 || one_group) &&
      reinterpret_cast<uintptr_t>(qw) % 4 == 0 && ldo % 8 == 0 &&
      reinterpret_cast<uintptr_t>(out) % 16 == 0) {
    const int wpr = (K + 2047) / 2048;  // wavefronts per channel row
    const int64_t blocks = ((int64_t)N * wpr + 3) / 4;
    const uint32_t gdiv = one_group ? 0u : (uint32_t)gs;
    const uint32_t gmul = gdiv > 1 ? (uint32_t)(0xffffffffu / gdiv + 1u) : 0u;  // c / gs = umulhi(c, gmul)
    auto kern = odt == FG_BF16 ? w4_dequant16_kernel<true> : w4_dequant16_kernel<false>;
    note_kernel("w4_dequant16_kernel");
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), 0, s, qw, ldq, static_cast<const uint16_t*>(scales),
                       (int)(sdt == FG_BF16), lds, zeros, ldz, static_cast<uint16_t*>(out), ldo, N, K, wpr, gdiv, gmul);
    return hipGetLastError();
  }
  const int64_t total = (int64_t)N * ((K + 7) / 8);
  const int64_t blocks = (total + 255) / 256;
  note_kernel("w4_dequant_kernel");
  hipLaunchKernelGGL(w4_dequant_kernel, dim3((unsigned)blocks), dim3(256), 0, s, qw, ldq, scales, sdt, lds, zeros, ldz,
                     g_idx, out, odt, ldo, N, K, gs);
  return hipGetLastError();
}

}  // namespace fg
