// W4A16 prefill for large M x N with producer and consumer wavefronts: y[M,N] = x[M,K] @ dequant(W)[N,K]^T (+bias).
//
// A workgroup owns a 256 x 128 output tile and walks K in 64-column slices through a three-stage LDS ring.  Its eight
// wavefronts split the work by role, one of each role per SIMD (wavefronts 0-3 on SIMDs 0-3, 4-7 likewise):
//   * consumers (wavefronts 0-3, a 2 x 2 grid of 128 x 64 tiles): read A and B fragments from LDS and run
//     v_mfma_f32_16x16x32_{bf16,f16}; they issue no global memory instruction;
//   * producers (wavefronts 4-7): every global access of the slice is a direct-to-LDS load (global_load_lds, no
//     registers): the 256 x 64 tile of x (eight 1 KiB loads per producer), the 128 x 64 tile of packed int4 weights
//     (one 1 KiB load per producer: its own 32 rows), and the scales and zero-point words of those 32 rows (one 4-byte
//     per lane load); then each producer lane reads back its 16 bytes of packed weights (32 columns of one row),
//     dequantises them -- (q - z) * s in fp32, exactly the oracle's value (q * s + (-z * s) is exact and the fma
//     rounds nothing), rounded once to bf16 / fp16 -- and stores them into the stage's weight rows.
// So the dequantisation VALU of one wavefront runs while the other wavefront of its SIMD keeps the matrix core busy,
// instead of both wavefronts alternating the two under one barrier (the all-rounder w4_big_kernel, fg_w4_big.hip).
//
// Ring schedule, slice t in stage t % 3 (iteration t ends with the workgroup barrier that publishes stage t + 1):
//   producers, iteration t: x of slice t + 2 -> stage (t + 2) % 3 (consumed in t - 1); packed weights, scales and
//     zero words of slice t + 3 -> the staging areas of stage t % 3 (read by the producers in t - 1); wait until
//     slice t + 1's staging loads have landed, dequantise slice t + 1 into stage (t + 1) % 3's weight rows (consumed
//     in t - 2); wait until slice t + 1's x rows have landed; barrier.
//   consumers, iteration t: 64 MFMAs per k-step pair over stage t % 3; barrier.
// Every producer issues the same loads in the same order each iteration (slices past the end re-read the last one,
// into areas no one reads again), so `s_waitcnt vmcnt(N)` with a constant N is exactly "these loads have landed"
// (loads complete in issue order); the direct-to-LDS loads are invisible to the compiler's wait analysis, so those
// waits are explicit.  Packed weights and scales get two slices (~2 us at full rate) to arrive, x two as well.
//
// LDS per stage: x 256 rows x 128 B (16-byte unit c of row r at c ^ (r & 7): conflict-free fragment reads), weight
// rows 128 x 128 B (same swizzle), packed-weight staging 4 KiB (producer p's lane l at p * 1024 + 16 l), scale and
// zero staging 1 KiB (producer p: 32 fp16 scales at p * 256, its 4 zero words at p * 256 + 64).  Three stages:
// 162816 bytes.
//
// Split-K (gridDim.y > 1): each split covers `kchunk` columns and writes fp32 partials [S, M, N] to the caller's
// workspace; w4_splitk_reduce_kernel (fg_w4_mfma.hip) sums them in a fixed order and adds the bias.
//
// Requirements (w4_pc_ok): K % 64 == 0, group a multiple of 64 (or one group), N % 8 == 0, 16-bit scales with an even
// row stride, 16-byte aligned x (ldx % 8 == 0) and qweight (ldq % 4 == 0), 4-byte aligned scales, no act-order perm.
// Rows past M and channels past N read row M - 1 / channel N - 1 and are not stored.
#include <algorithm>

#include "fg_device.h"

namespace fg {

typedef __bf16 bf16x8_pc_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_pc_t __attribute__((ext_vector_type(8)));
typedef float f32x4_pc_t __attribute__((ext_vector_type(4)));
typedef float f32x2_pc_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_pc_t __attribute__((ext_vector_type(2)));

constexpr int kPcBM = 256, kPcBN = 128, kPcBK = 64, kPcRow = 128, kPcThreads = 512;
constexpr int kPcXBytes = kPcBM * kPcRow;                      // x rows
constexpr int kPcWBytes = kPcBN * kPcRow;                      // dequantised weight rows
constexpr int kPcQBytes = kPcBN * kPcBK / 2;                   // packed weights of the slice
constexpr int kPcSBytes = 4 * 256;                             // scales and zero words
constexpr int kPcStage = kPcXBytes + kPcWBytes + kPcQBytes + kPcSBytes;
constexpr int kPcLds = 3 * kPcStage;
static_assert(kPcLds <= 160 * 1024, "the ring exceeds the LDS");
// direct-to-LDS loads one producer issues per slice: x rows, packed weights, scales + zero words
constexpr int kPcXI = kPcXBytes / 1024 / 4, kPcQI = 1, kPcSI = 1;
static_assert(kPcXI == 8, "eight x loads per producer and slice");

struct PcArgs {
  const uint16_t* x;
  int64_t ldx;
  const int32_t* qw;
  int64_t ldq;  // int32 words per row
  const uint16_t* scales;
  int64_t lds;
  const int32_t* zeros;  // qweight when symmetric (a valid address, never used)
  int64_t ldz;
  const void* bias;
  float* ws;
  uint16_t* y;
  int64_t ldy;
  int M, N, K;
  int kchunk;        // columns per K split (a multiple of 64)
  uint32_t gdiv;     // 64-column slices per group (0: one group)
  uint32_t gmul;     // slice / gdiv = umulhi(slice, gmul) (gdiv > 1)
  int hasz, sbf16, bdt;
};

template <bool XBF16>
__device__ __forceinline__ f32x4_pc_t pc_mfma(uint4 a, uint4 b, f32x4_pc_t c) {
  if constexpr (XBF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_pc_t, a),
                                                   __builtin_bit_cast(bf16x8_pc_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_pc_t, a),
                                                  __builtin_bit_cast(f16x8_pc_t, b), c, 0, 0, 0);
  }
}

// two fp32 values as one packed 16-bit pair, each rounded to nearest even
template <bool XBF16>
__device__ __forceinline__ uint32_t pc_pack(float lo, float hi) {
  if constexpr (XBF16) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_pc_t{lo, hi}, bf16x2_pc_t));
  } else {
    return (uint32_t)f32_to_f16_bits(lo) | ((uint32_t)f32_to_f16_bits(hi) << 16);
  }
}

// 16-byte fragment of one swizzled 128-byte LDS row for k-step s: unit 4 s + lane / 16
__device__ __forceinline__ uint4 pc_frag(const uint8_t* rp, int r16, int lane, int s) {
  const int c = (4 * s + (lane >> 4)) ^ (r16 & 7);
  return *reinterpret_cast<const uint4*>(rp + c * 16);
}

template <bool XBF16>
__global__ void __launch_bounds__(kPcThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) w4_pc_kernel(const PcArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int ntm = (a.M + kPcBM - 1) / kPcBM, ntn = (a.N + kPcBN - 1) / kPcBN;
  int tm, tn;
  tile_of(blockIdx.x, ntm, ntn, tm, tn);
  const int m0 = tm * kPcBM, n0 = tn * kPcBN;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int kbeg = blockIdx.y * a.kchunk;
  const int nk = (min(a.K, kbeg + a.kchunk) - kbeg) / kPcBK;

  if (wave < 4) {
    // ------------------------------------------------------------------------------------------- consumers
    const int wm = wave >> 1, wn = wave & 1, r16 = lane & 15;
    f32x4_pc_t acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_pc_t{0.f, 0.f, 0.f, 0.f};
    asm volatile("s_barrier" ::: "memory");  // slice 0 is in stage 0
    // Fragments of k-step 0 of a slice (f0) and of k-step 1 (f1), in registers.  The loop is software-pipelined
    // around the barrier: k-step 0 of slice t + 1 is read right after the barrier that ends slice t, while the last
    // eight MFMAs of slice t (whose fragments are already in registers) run, so a consumer -- the only MFMA issuer of
    // its SIMD -- does not sit out the LDS latency at the top of every slice.
    uint4 fa0[8], fb0[4], fa1[8], fb1[4];
    auto read_ks = [&](const uint8_t* st, int s, uint4 (&fa)[8], uint4 (&fb)[4]) __attribute__((always_inline)) {
      const uint8_t* sA = st + (wm * 128 + r16) * kPcRow;
      const uint8_t* sB = st + kPcXBytes + (wn * 64 + r16) * kPcRow;
#pragma unroll
      for (int j = 0; j < 4; ++j) fb[j] = pc_frag(sB + j * 16 * kPcRow, r16, lane, s);
#pragma unroll
      for (int i = 0; i < 8; ++i) fa[i] = pc_frag(sA + i * 16 * kPcRow, r16, lane, s);
    };
    auto mfma_rows = [&](int i0, int i1, const uint4 (&fa)[8], const uint4 (&fb)[4]) __attribute__((always_inline)) {
#pragma unroll
      for (int i = i0; i < i1; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = pc_mfma<XBF16>(fa[i], fb[j], acc[i][j]);
    };
    const uint8_t* st = smem;
    read_ks(st, 0, fa0, fb0);
    for (int t = 0; t < nk; ++t) {
      read_ks(st, 1, fa1, fb1);
      mfma_rows(0, 8, fa0, fb0);
      mfma_rows(0, 6, fa1, fb1);
      // this stage's fragments are in registers before the barrier lets the producers refill it
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      st = st == smem + 2 * kPcStage ? smem : st + kPcStage;
      read_ks(st, 0, fa0, fb0);  // slice t + 1 (past the last slice: a stage no one writes any more, unused)
      __builtin_amdgcn_sched_barrier(0);
      mfma_rows(6, 8, fa1, fb1);
      __builtin_amdgcn_sched_barrier(0);
    }
    asm volatile("s_barrier" ::: "memory");  // the producers' last loads have drained: the ring is free

    const int mw = m0 + wm * 128, nw = n0 + wn * 64;
    if (gridDim.y > 1) {  // fp32 partials of this split
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int m = mw + i * 16 + 4 * (lane >> 4) + e, n = nw + j * 16 + (lane & 15);
            if (m < a.M && n < a.N) a.ws[((int64_t)blockIdx.y * a.M + m) * a.N + n] = acc[i][j][e];
          }
      return;
    }
    // 16-bit output through a per-wavefront LDS slab of 16 rows x 64 columns, stored as 16-byte row segments
    constexpr int SP = 64 + 8;
    uint16_t* slab = reinterpret_cast<uint16_t*>(smem) + wave * 16 * SP;
    float cb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) cb[j] = a.bias ? load_f(a.bias, a.bdt, min(nw + j * 16 + (lane & 15), a.N - 1)) : 0.f;
    const bool vec_ok = (a.ldy % 8) == 0 && (reinterpret_cast<uintptr_t>(a.y) % 16) == 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float v = a.bias ? acc[i][j][e] + cb[j] : acc[i][j][e];
          slab[(4 * (lane >> 4) + e) * SP + j * 16 + (lane & 15)] = XBF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
        }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's slab writes are done before it reads them
#pragma unroll
      for (int u0 = 0; u0 < 16 * 64 / 8; u0 += 64) {
        const int u = u0 + lane, r = u / 8, c8 = u % 8;
        const int m = mw + i * 16 + r, n = nw + c8 * 8;
        const uint4 v = *reinterpret_cast<const uint4*>(slab + r * SP + c8 * 8);
        if (m < a.M) {
          uint16_t* yr = a.y + (int64_t)m * a.ldy;
          if (n + 8 <= a.N && vec_ok) {
            *reinterpret_cast<uint4*>(yr + n) = v;
          } else {
            const uint16_t h[8] = {(uint16_t)v.x, (uint16_t)(v.x >> 16), (uint16_t)v.y, (uint16_t)(v.y >> 16),
                                   (uint16_t)v.z, (uint16_t)(v.z >> 16), (uint16_t)v.w, (uint16_t)(v.w >> 16)};
            for (int q = 0; q < 8 && n + q < a.N; ++q) yr[n + q] = h[q];
          }
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads done before the next slab overwrites the buffer
    }
    return;
  }

  // --------------------------------------------------------------------------------------------- producers
  const int p = wave - 4;
  // x: load i of producer p fills tile rows (8 p + i) * 8 .. + 8; lane l writes position l % 8 of row
  // (8 p + i) * 8 + l / 8, i.e. global unit (l % 8) ^ (l / 8) (the row's swizzle key is l / 8)
  const int lrow = lane >> 3, lcol = ((lane & 7) ^ (lane >> 3)) * 8;
  const uint16_t* xr[kPcXI];
#pragma unroll
  for (int i = 0; i < kPcXI; ++i) xr[i] = a.x + (int64_t)min(m0 + (8 * p + i) * 8 + lrow, a.M - 1) * a.ldx + lcol;
  // packed weights: lane l owns tile row 32 p + l / 2, columns 32 (l % 2) .. + 32 of each slice (16 bytes)
  const int wr = 32 * p + (lane >> 1), wh = lane & 1;
  const int32_t* wq = a.qw + (int64_t)min(n0 + wr, a.N - 1) * a.ldq + 4 * wh;
  // scales and zero words of the producer's 32 channels: lanes 0-15 read scale pairs, lanes 16-19 zero words, the
  // rest repeat lane 0's pair (every lane of a direct-to-LDS load writes its 4 bytes)
  const uint8_t* szb;
  int64_t szstride;  // bytes per group
  {
    const int c0 = n0 + 32 * p;
    if (lane >= 16 && lane < 20 && a.hasz) {
      const int w = min(c0 / 8 + (lane - 16), (a.N - 1) / 8);
      szb = reinterpret_cast<const uint8_t*>(a.zeros + w);
      szstride = a.ldz * 4;
    } else {
      const int c = min(c0 + 2 * (lane < 16 ? lane : 0), a.N - 2);
      szb = reinterpret_cast<const uint8_t*>(a.scales + c);
      szstride = a.lds * 2;
    }
  }
  const int slice0 = kbeg / kPcBK;
  auto group_of = [&](int t) -> uint32_t {  // group of local slice t (clamped to the last slice)
    const uint32_t sl = (uint32_t)(slice0 + min(t, nk - 1));
    return a.gdiv == 0 ? 0u : (a.gdiv == 1 ? sl : __umulhi(sl, a.gmul));
  };
  // x rows of slice t into a stage's x area
  auto issue_x = [&](int t, uint8_t* dst) __attribute__((always_inline)) {
    const int k0 = kbeg + min(t, nk - 1) * kPcBK;
    dst += p * kPcXI * 1024;
#pragma unroll
    for (int i = 0; i < kPcXI; ++i) __builtin_amdgcn_global_load_lds(xr[i] + k0, dst + i * 1024, 16, 0, 0);
  };
  // packed weights, scales and zero words of slice t into a stage's staging areas (base: the stage's packed-weight
  // area, the scale area follows it)
  auto issue_q = [&](int t, uint8_t* dst) __attribute__((always_inline)) {
    const int k0 = kbeg + min(t, nk - 1) * kPcBK;
    __builtin_amdgcn_global_load_lds(wq + k0 / 8, dst + p * 1024, 16, 0, 0);
    __builtin_amdgcn_global_load_lds(szb + (int64_t)group_of(t) * szstride, dst + kPcQBytes + p * 256, 4, 0, 0);
  };
  uint32_t nmask = 0x0F0F0F0Fu;
  asm("" : "+v"(nmask));  // hidden from known-bits analysis: bytes of masked words convert with v_cvt_f32_ubyte{k}
  const uint32_t zsel = a.hasz ? 0xffffffffu : 0u;
  // one slice's weights from a stage's staging areas (q) into its weight rows (w)
  auto dequant = [&](const uint8_t* __restrict__ q, uint8_t* __restrict__ w) __attribute__((always_inline)) {
    const uint4 qv = *reinterpret_cast<const uint4*>(q + p * 1024 + lane * 16);
    const uint8_t* sz = q + kPcQBytes + p * 256;
    const uint32_t sraw = *reinterpret_cast<const uint16_t*>(sz + (lane >> 1) * 2);
    const uint32_t zw = (*reinterpret_cast<const uint32_t*>(sz + 64 + ((lane >> 1) >> 3) * 4) & zsel) |
                        (0x88888888u & ~zsel);  // symmetric: zero-point 8
    const float sc = a.sbf16 ? bf16_bits_to_f32(sraw) : f16_bits_to_f32((uint16_t)sraw);
    const float c = -(float)nibble(zw, (lane >> 1) & 7) * sc;
    const uint32_t wd[4] = {qv.x, qv.y, qv.z, qv.w};
    uint8_t* rp = w + wr * kPcRow;
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // word i = columns 8 i .. 8 i + 7 of the lane's 32 = unit 4 wh + i of the row
      const uint32_t lo = wd[i] & nmask, hi = (wd[i] >> 4) & nmask;  // nibbles 0,2,4,6 / 1,3,5,7
      float d[8];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        d[2 * b] = __builtin_fmaf((float)((lo >> (8 * b)) & 0xFFu), sc, c);
        d[2 * b + 1] = __builtin_fmaf((float)((hi >> (8 * b)) & 0xFFu), sc, c);
      }
      const uint4 v = make_uint4(pc_pack<XBF16>(d[0], d[1]), pc_pack<XBF16>(d[2], d[3]), pc_pack<XBF16>(d[4], d[5]),
                                 pc_pack<XBF16>(d[6], d[7]));
      *reinterpret_cast<uint4*>(rp + (((4 * wh + i) ^ (wr & 7)) * 16)) = v;
    }
  };
  constexpr int kQ = kPcXBytes + kPcWBytes;  // offset of a stage's staging areas
  // Iteration t.  The four regions reach the body as __restrict__ pointers: without them the compiler cannot tell
  // the direct-to-LDS loads from the staging reads and weight-row stores, and waits for every outstanding load.
  auto body = [&](int t, const uint8_t* __restrict__ q_rd, uint8_t* __restrict__ w_wr, uint8_t* __restrict__ x_dst,
                  uint8_t* __restrict__ q_dst) __attribute__((always_inline)) {
    issue_x(t + 2, x_dst);
    issue_q(t + 3, q_dst);
    // slice t + 1's staging landed (issued two iterations ago; everything after it may still be in flight)
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * kPcXI + 2 * (kPcQI + kPcSI)) : "memory");
    dequant(q_rd, w_wr);
    // slice t + 1's x rows landed and this wave's weight stores are done; then the barrier publishes stage t + 1
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(kPcXI + 2 * (kPcQI + kPcSI)) : "memory");
  };

  uint8_t* const s0 = smem;
  uint8_t* const s1 = smem + kPcStage;
  uint8_t* const s2 = smem + 2 * kPcStage;
  // prologue, in the steady state's issue order: [q0] [x0 q1] [x1 q2]
  issue_q(0, s0 + kQ);
  issue_x(0, s0);
  issue_q(1, s1 + kQ);
  issue_x(1, s1);
  issue_q(2, s2 + kQ);
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * kPcXI + 2 * (kPcQI + kPcSI)) : "memory");  // slice 0's staging
  dequant(s0 + kQ, s0 + kPcXBytes);
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(kPcXI + 2 * (kPcQI + kPcSI)) : "memory");
  // stage of slice t: t % 3; rotate (a, b, c) = stages of (t, t + 1, t + 2)
  uint8_t *sa = s0, *sb = s1, *sc = s2;
  for (int t = 0; t < nk; ++t) {
    body(t, sb + kQ, sb + kPcXBytes, sc, sa + kQ);
    uint8_t* tmp = sa;
    sa = sb;
    sb = sc;
    sc = tmp;
  }
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");  // drain before the consumers reuse the ring
}

bool w4_pc_ok(const void* x, int64_t ldx, const int32_t* qw, int64_t ldq, const int32_t* perm, const void* scales,
              int sdt, int64_t lds, int64_t N, int64_t K, int gs, int64_t G) {
  return perm == nullptr && (K % kPcBK) == 0 && ((gs % kPcBK) == 0 || G == 1) && (N % 8) == 0 && N >= 8 &&
         sdt != FG_F32 && (lds % 2) == 0 && (reinterpret_cast<uintptr_t>(scales) % 4) == 0 && (ldx % 8) == 0 &&
         (reinterpret_cast<uintptr_t>(x) % 16) == 0 && (ldq % 4) == 0 && (reinterpret_cast<uintptr_t>(qw) % 16) == 0 &&
         group_div_exact(K, gs, G, kPcBK);
}

// K splits: one when the tiles cover the CUs, else as many as keep the workgroups within one round over the CUs, each
// at least 512 columns.
void w4_pc_plan(int M, int N, int K, int split_k, int* splits, int* kchunk) {
  const int cus = device_cus();
  const int64_t tiles = (int64_t)((M + kPcBM - 1) / kPcBM) * ((N + kPcBN - 1) / kPcBN);
  int s = split_k;
  if (s <= 0) {
    s = tiles >= cus ? 1 : (int)(cus / tiles);
    const int max_s = K / 512 > 0 ? K / 512 : 1;
    s = std::min(std::min(s, max_s), 16);
  }
  int kc = (K + s - 1) / s;
  kc = (kc + kPcBK - 1) / kPcBK * kPcBK;
  *kchunk = kc;
  *splits = (K + kc - 1) / kc;
}

size_t w4_pc_workspace_bytes(int M, int N, int K, int split_k) {
  int s, kc;
  w4_pc_plan(M, N, K, split_k, &s, &kc);
  return s > 1 ? (size_t)s * (size_t)M * (size_t)N * sizeof(float) : 0;
}

template <bool XBF16>
hipError_t launch_w4_splitk_reduce(const float* ws, int S, int M, int N, const void* bias, int bdt, void* y,
                                   int64_t ldy, hipStream_t s);

hipError_t launch_w4_pc(const void* x, int64_t ldx, bool xbf16, const int32_t* qw, int64_t ldq, const void* scales,
                        int sdt, int64_t lds, const int32_t* zeros, int64_t ldz, const void* bias, int bdt, void* y,
                        int64_t ldy, float* ws, int M, int N, int K, int gs, bool single_group, int split_k,
                        hipStream_t s) {
  int splits, kchunk;
  w4_pc_plan(M, N, K, split_k, &splits, &kchunk);
  PcArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.qw = qw;
  a.ldq = ldq;
  a.scales = static_cast<const uint16_t*>(scales);
  a.lds = lds;
  a.hasz = zeros != nullptr;
  a.zeros = zeros ? zeros : qw;
  a.ldz = zeros ? ldz : 0;
  a.bias = bias;
  a.bdt = bdt;
  a.ws = ws;
  a.y = static_cast<uint16_t*>(y);
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  a.kchunk = kchunk;
  a.gdiv = single_group ? 0u : (uint32_t)(gs / kPcBK);
  a.gmul = a.gdiv > 1 ? 0xffffffffu / a.gdiv + 1u : 0u;
  a.sbf16 = sdt == FG_BF16;
  if (splits > 1 && ws == nullptr) return hipErrorInvalidValue;
  auto kern = xbf16 ? w4_pc_kernel<true> : w4_pc_kernel<false>;
  hipError_t e =
      hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, kPcLds);
  if (e != hipSuccess) return e;
  const int tiles = ((M + kPcBM - 1) / kPcBM) * ((N + kPcBN - 1) / kPcBN);
  note_kernel("w4_pc_kernel<%s> 256x128 splits=%d%s", xbf16 ? "bf16" : "f16", splits,
              splits > 1 ? " + w4_splitk_reduce_kernel" : "");
  hipLaunchKernelGGL(kern, dim3(tiles, splits), dim3(kPcThreads), kPcLds, s, a);
  e = hipGetLastError();
  if (e != hipSuccess || splits == 1) return e;
  return xbf16 ? launch_w4_splitk_reduce<true>(ws, splits, M, N, bias, bdt, y, ldy, s)
               : launch_w4_splitk_reduce<false>(ws, splits, M, N, bias, bdt, y, ldy, s);
}

}  // namespace fg
