// W4A16 prefill on matrix cores for large M x N: y[M,N] = x[M,K] @ dequant(W)[N,K]^T (+bias).
//
// Workgroup tile BM x 256 (BM = 256, 128 or 64), 512 threads = 2 x 4 wavefronts of (BM/2) x 64 (BM = 64: 1 x 8
// wavefronts of 64 x 32), 16 x 16 output tiles of
// v_mfma_f32_16x16x32_{bf16,f16}.  K is walked in 64-column slices (128 bytes of x per row) through a double-buffered
// LDS ring:
//   * x: written straight from global memory into LDS by global_load_lds_dwordx4 (no registers, no VALU), one
//     wavefront instruction = 8 rows x 128 bytes;
//   * W: each thread loads 16 bytes of packed weights (32 columns of one row) one slice ahead into registers, with the
//     row's scale and zero-point for that group, and after the current slice's MFMAs writes the 32 dequantised
//     values -- (q - z) * s in fp32, exactly the oracle's value (q * s + (-z * s) is exact in fp32 and the fma rounds
//     nothing), rounded once to bf16 / fp16 with round-to-nearest-even -- into the other half of the ring.  No
//     dequantised copy of W reaches HBM (the reference's large-M path writes one and re-reads it,
//     forge/kernels/triton/gemm_w4_dequant.py:194-256).
// Within a 128-byte LDS row the 16-byte unit c (8 columns) of row r is stored at c ^ (r & 7), so the 16-row fragment
// reads of one MFMA fall on 8 distinct bank groups.
//
// Split-K (gridDim.y > 1): each split covers `kchunk` columns and writes fp32 partials to the caller's workspace
// [S, M, N]; w4_splitk_reduce_kernel (fg_w4_mfma.hip) sums them in a fixed order and adds the bias.
//
// Requirements (w4_big_ok): K % 64 == 0, group size a multiple of 32 (or one group), x 16-byte aligned with
// ldx % 8 == 0, qweight 16-byte aligned with ldq % 4 == 0, no act-order perm.  Rows past M or N read row M-1 / N-1.
#include <algorithm>

#include "fg_device.h"

namespace fg {

typedef __bf16 bf16x8_big_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_big_t __attribute__((ext_vector_type(8)));
typedef float f32x4_big_t __attribute__((ext_vector_type(4)));
typedef float f32x2_big_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_big_t __attribute__((ext_vector_type(2)));

constexpr int kW4BigBN = 256, kW4BigBK = 64, kW4BigThreads = 512;

template <bool XBF16>
__device__ __forceinline__ f32x4_big_t w4big_mfma(uint4 a, uint4 b, f32x4_big_t c) {
  if constexpr (XBF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_big_t, a),
                                                   __builtin_bit_cast(bf16x8_big_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_big_t, a),
                                                  __builtin_bit_cast(f16x8_big_t, b), c, 0, 0, 0);
  }
}

// Two fp32 values as one packed 16-bit pair, each rounded to nearest even.
template <bool XBF16>
__device__ __forceinline__ uint32_t w4big_pack(float lo, float hi) {
  if constexpr (XBF16) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_big_t{lo, hi}, bf16x2_big_t));
  } else {
    return (uint32_t)f32_to_f16_bits(lo) | ((uint32_t)f32_to_f16_bits(hi) << 16);
  }
}

// Byte b of w as a float (v_cvt_f32_ubyte{b}).
__device__ __forceinline__ float ubyte_f32(uint32_t w, int b) { return (float)((w >> (8 * b)) & 0xFFu); }

// Fragment of one 128-byte LDS row for k-step s (32 columns): 16 bytes, unit 4 s + lane / 16, swizzled.
__device__ __forceinline__ uint4 w4big_frag(const uint8_t* rp, int r16, int lane, int s) {
  const int c = (4 * s + (lane >> 4)) ^ (r16 & 7);
  return *reinterpret_cast<const uint4*>(rp + c * 16);
}

// WB = 4: packed int4 qweight (int32 words, ldq in words) with zero-points; WB = 8: int8 qweight (ldq in bytes),
// symmetric (W8A16).
// PF (16-bit scales, K chunks of whole 128-column pairs of slices; PF = 0 otherwise): the loop is unrolled by two with
// no branch in it, and the next slice's loads are issued before this slice's MFMAs, which no longer wait for them.
// PF = 2 (64- and 128-row tiles): the weights, scale and zero word of slice kt + 2 are fetched while slice kt's MFMAs
// run and slice kt + 1's are dequantised into LDS -- two register sets -- so a slice's HBM latency is covered by two
// slices of work instead of one (small M has little work per slice); every fetch is exactly three loads, issued after
// the slice's x loads (pinned by sched_barrier), and the end-of-slice wait for the x loads leaves those three in
// flight.  PF = 1 (256-row tiles, no registers for a second set): slice kt + 1's weights load during slice kt's
// MFMAs.  Loads past the last slice re-read it (clamped) into registers or into an LDS half no one reads again.
template <int BM, bool XBF16, int WB, int PF>
__global__ void __launch_bounds__(kW4BigThreads) w4_big_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const void* __restrict__ qw, int64_t ldq,
    const void* __restrict__ scales, int sdt, int64_t lds, const int32_t* __restrict__ zeros, int64_t ldz, int hasz,
    const void* __restrict__ bias, int bdt, uint16_t* __restrict__ y, int64_t ldy, float* __restrict__ ws, int M,
    int N, int K, int gs32, int kchunk) {
  constexpr int BN = kW4BigBN, BK = kW4BigBK, NT = kW4BigThreads, WM = BM >= 128 ? 2 : 1, WN = 8 / WM;
  constexpr int ROW = BK * 2;                  // bytes per LDS row
  constexpr int TM = BM / WM / 16, TN = BN / WN / 16;
  constexpr int X_INSTR = BM * ROW / 16 / NT;  // 1 KiB x load instructions per wavefront and slice
  static_assert(X_INSTR * NT * 16 == BM * ROW, "x tile / thread count mismatch");
  static_assert(BN * 2 == NT, "one thread per half weight row");
  constexpr int STAGE = (BM + BN) * ROW;
  extern __shared__ __align__(16) uint8_t smem[];

  const int ntm = (M + BM - 1) / BM, ntn = (N + BN - 1) / BN;
  int tm_, tn_;
  tile_of(blockIdx.x, ntm, ntn, tm_, tn_);
  const int m0 = tm_ * BM, n0 = tn_ * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int kbeg = blockIdx.y * kchunk, kend = min(K, kbeg + kchunk);
  const int nk = (kend - kbeg) / BK;

  // x: load instruction i of wave w fills LDS units (w * X_INSTR + i) * 64 + lane = row (w * X_INSTR + i) * 8 +
  // lane / 8, position lane % 8, which holds global unit (lane % 8) ^ (row % 8) = (lane % 8) ^ (lane / 8).
  const int lrow = lane >> 3, lcol = ((lane & 7) ^ (lane >> 3)) * 8;  // column offset in elements
  const int xrow0 = wave * X_INSTR * 8 + lrow;
  auto issue_x = [&](int k0, uint8_t* st) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < X_INSTR; ++i)
      __builtin_amdgcn_global_load_lds(x + (int64_t)min(m0 + xrow0 + 8 * i, M - 1) * ldx + k0 + lcol,
                                       st + (wave * X_INSTR + i) * 1024, 16, 0, 0);
  };
  // W: thread t owns row t / 2 of the tile, columns 32 (t % 2) .. + 32 of each slice (4 packed words)
  const int wrow = tid >> 1, whalf = tid & 1;
  const int wn_ = min(n0 + wrow, N - 1);
  // this thread's 32 columns of each slice: 16 bytes of packed int4 or 32 bytes of int8
  const uint4* __restrict__ wsrc =
      WB == 4 ? reinterpret_cast<const uint4*>(static_cast<const int32_t*>(qw) + (int64_t)wn_ * ldq) + whalf
              : reinterpret_cast<const uint4*>(static_cast<const int8_t*>(qw) + (int64_t)wn_ * ldq) + 2 * whalf;
  // Branch-free group index, scale and zero-point (a uniform condition inside the loop would become a scalar branch,
  // which splits the loop body and makes the compiler wait for every load at the join): group of chunk c =
  // umulhi(c, gmul) | (c & gsel) (gs32 > 1: floor(c / gs32); gs32 == 1: c; one group: 0).
  const uint32_t gmul = gs32 > 1 ? 0xffffffffu / (uint32_t)gs32 + 1u : 0u, gsel = gs32 == 1 ? 0xffffffffu : 0u;
  const uint32_t zmask = hasz ? 0xffffffffu : 0u, sbf16 = sdt == FG_BF16 ? 0xffffffffu : 0u;
  struct WRegs {  // one slice of this thread's weights, its group's scale and zero-point word
    uint4 w, w2;
    uint32_t s, z;
  };
  // Vector-memory instructions one fetch_w issues (4-bit: weights, scale, zero word; 8-bit: two weight halves,
  // scale).  The PF = 2 loop waits with vmcnt(kFetchVmem) for the x rows it issued just before them;
  // tests/test_isa_waits.py checks in the built code object that this many loads follow the last x load.
  constexpr int kFetchVmem = 3;
  auto fetch_w = [&](int k0, WRegs& r) __attribute__((always_inline)) {
    const uint32_t c = (uint32_t)((k0 >> 5) + whalf);  // 32-column chunk index
    const int g = (int)(__umulhi(c, gmul) | (c & gsel));
    if constexpr (WB == 4) {
      r.w = load16_stream(wsrc + (k0 >> 5));
    } else {
      r.w = load16_stream(wsrc + (k0 >> 4));
      r.w2 = load16_stream(wsrc + (k0 >> 4) + 1);
    }
    if constexpr (PF > 0) {  // fp16 / bf16 scales only (the launcher takes PF > 0 for no other)
      r.s = static_cast<const uint16_t*>(scales)[(int64_t)g * lds + wn_];
    } else {  // any scale type
      r.s = load_raw(scales, sdt, (int64_t)g * lds + wn_);
    }
    if constexpr (WB == 4) r.z = (uint32_t)zeros[(int64_t)g * ldz + (wn_ >> 3)];
  };
  // wbase: the weight rows of an LDS half (its x rows come first)
  auto stash_w = [&](uint8_t* wbase, const WRegs& r) __attribute__((always_inline)) {
    const uint4 wreg = r.w, wreg2 = r.w2;
    const uint32_t sreg = r.s, zreg = (r.z & zmask) | (0x88888888u & ~zmask);  // symmetric: zero-point 8
    const uint32_t f16 = __float_as_uint(f16_bits_to_f32((uint16_t)sreg));
    const float s = PF > 0 ? __uint_as_float(((sreg << 16) & sbf16) | (f16 & ~sbf16)) : raw_bits_to_f32(sreg, sdt);
    uint8_t* rp = wbase + wrow * ROW;
    if constexpr (WB == 8) {  // 32 signed bytes: q * s exactly as the oracle's fp32 product, rounded once
      const uint32_t wd[8] = {wreg.x, wreg.y, wreg.z, wreg.w, wreg2.x, wreg2.y, wreg2.z, wreg2.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float d[8];
#pragma unroll
        for (int b = 0; b < 8; ++b) d[b] = (float)(int8_t)(wd[2 * i + b / 4] >> (8 * (b % 4))) * s;
        const uint4 v = make_uint4(w4big_pack<XBF16>(d[0], d[1]), w4big_pack<XBF16>(d[2], d[3]),
                                   w4big_pack<XBF16>(d[4], d[5]), w4big_pack<XBF16>(d[6], d[7]));
        *reinterpret_cast<uint4*>(rp + (((4 * whalf + i) ^ (wrow & 7)) * 16)) = v;
      }
      return;
    }
    const float z = (float)nibble(zreg, wn_ & 7);
    const float c = -z * s;
    const uint32_t wd[4] = {wreg.x, wreg.y, wreg.z, wreg.w};
    // The nibble mask is hidden from known-bits analysis: with it visible, byte k of a masked word (at most 15) is
    // extracted with v_bfe_u32 and then converted, instead of converted directly by v_cvt_f32_ubyte{k}.
    uint32_t nmask = 0x0F0F0F0Fu;
    asm("" : "+v"(nmask));
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // word i = columns 8 i .. 8 i + 7 of this thread's 32 = LDS unit 4 whalf + i
      const uint32_t lo = wd[i] & nmask, hi = (wd[i] >> 4) & nmask;  // nibbles 0,2,4,6 / 1,3,5,7
      float d[8];
      d[0] = __builtin_fmaf(ubyte_f32(lo, 0), s, c);
      d[1] = __builtin_fmaf(ubyte_f32(hi, 0), s, c);
      d[2] = __builtin_fmaf(ubyte_f32(lo, 1), s, c);
      d[3] = __builtin_fmaf(ubyte_f32(hi, 1), s, c);
      d[4] = __builtin_fmaf(ubyte_f32(lo, 2), s, c);
      d[5] = __builtin_fmaf(ubyte_f32(hi, 2), s, c);
      d[6] = __builtin_fmaf(ubyte_f32(lo, 3), s, c);
      d[7] = __builtin_fmaf(ubyte_f32(hi, 3), s, c);
      const uint4 v = make_uint4(w4big_pack<XBF16>(d[0], d[1]), w4big_pack<XBF16>(d[2], d[3]),
                                 w4big_pack<XBF16>(d[4], d[5]), w4big_pack<XBF16>(d[6], d[7]));
      const int unit = (4 * whalf + i) ^ (wrow & 7);
      *reinterpret_cast<uint4*>(rp + unit * 16) = v;
    }
  };

  f32x4_big_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4_big_t{0.f, 0.f, 0.f, 0.f};

  const int r16 = lane & 15;
  auto mfma_slice = [&](const uint8_t* cur) __attribute__((always_inline)) {
    const uint8_t* sA = cur + (wm * TM * 16) * ROW;
    const uint8_t* sB = cur + BM * ROW + (wn * TN * 16) * ROW;
#pragma unroll
    for (int s = 0; s < BK / 32; ++s) {
      uint4 fa[TM];
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[i] = w4big_frag(sA + (i * 16 + r16) * ROW, r16, lane, s);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const uint4 fb = w4big_frag(sB + (j * 16 + r16) * ROW, r16, lane, s);
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[i][j] = w4big_mfma<XBF16>(fa[i], fb, acc[i][j]);
      }
    }
  };
  uint8_t* const h0 = smem;
  uint8_t* const h1 = smem + STAGE;
  if constexpr (PF == 2) {
    // Slice kt is in LDS half cur; rnext holds slice kt + 1; rfree is free.  The three regions are passed as
    // __restrict__ pointers: the compiler otherwise cannot tell the x rows being loaded into the other half (LDS DMA)
    // from the fragment reads of this half, or from the weight rows stored into the other half, and waits for every
    // outstanding load -- the prefetch included -- before each of them.
    //
    // With a direct-to-LDS load in flight the compiler waits for every outstanding load (vmcnt(0)) before the first
    // use of any register load, so every other slice's dequantisation waits for the loads issued at its top; the
    // other slice's data is already covered by that wait.
    auto body = [&](int kt, WRegs& rfree, const WRegs& rnext, const uint8_t* __restrict__ cur,
                    uint8_t* __restrict__ nxt_x, uint8_t* __restrict__ nxt_w) __attribute__((always_inline)) {
      issue_x(kbeg + min(kt + 1, nk - 1) * BK, nxt_x);  // that half is free since the last barrier
      __builtin_amdgcn_sched_barrier(0);
      fetch_w(kbeg + min(kt + 2, nk - 1) * BK, rfree);
      __builtin_amdgcn_sched_barrier(0);
      mfma_slice(cur);
      __builtin_amdgcn_sched_barrier(0);  // keep the dequantisation (and its wait for rnext) after the MFMAs
      stash_w(nxt_w, rnext);
      // Slice kt + 1's x rows have landed (slice kt + 2's three loads may still be in flight) and this wave's LDS
      // stores are done; then the workgroup barrier.  Not __syncthreads(): its release fence waits for every load,
      // the prefetch included.  The memory clobber keeps the compiler from moving LDS accesses across it.
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(kFetchVmem) : "memory");
    };
    WRegs ra, rb;
    if (nk > 0) {
      issue_x(kbeg, smem);
      fetch_w(kbeg, ra);
      stash_w(smem + BM * ROW, ra);
      fetch_w(kbeg + min(1, nk - 1) * BK, rb);
    }
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(kFetchVmem) : "memory");
    for (int kt = 0; kt < nk; kt += 2) {  // nk is even (the host splits K in 128-column multiples)
      body(kt, ra, rb, h0, h1, h1 + BM * ROW);
      body(kt + 1, rb, ra, h1, h0, h0 + BM * ROW);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();  // the epilogue reuses the ring
  } else if constexpr (PF == 1) {
    // as PF = 2 with one register set: the loads of slice kt + 1 go out before slice kt's MFMAs, the weights are
    // dequantised after them, and the slice ends once everything has landed
    auto body = [&](int kt, WRegs& rw, const uint8_t* __restrict__ cur, uint8_t* __restrict__ nxt_x,
                    uint8_t* __restrict__ nxt_w) __attribute__((always_inline)) {
      const int kn = kbeg + min(kt + 1, nk - 1) * BK;
      issue_x(kn, nxt_x);  // that half is free since the last barrier
      fetch_w(kn, rw);
      __builtin_amdgcn_sched_barrier(0);
      mfma_slice(cur);
      __builtin_amdgcn_sched_barrier(0);  // keep the dequantisation (and its wait for rw) after the MFMAs
      stash_w(nxt_w, rw);
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    WRegs rw;
    if (nk > 0) {
      issue_x(kbeg, smem);
      fetch_w(kbeg, rw);
      stash_w(smem + BM * ROW, rw);
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    for (int kt = 0; kt < nk; kt += 2) {  // nk is even (the host splits K in 128-column multiples)
      body(kt, rw, h0, h1, h1 + BM * ROW);
      body(kt + 1, rw, h1, h0, h0 + BM * ROW);
    }
    __syncthreads();  // the epilogue reuses the ring
  } else {
    WRegs rw;
    if (nk > 0) {
      issue_x(kbeg, smem);
      fetch_w(kbeg, rw);
      stash_w(smem + BM * ROW, rw);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      uint8_t* nxt = smem + ((kt + 1) & 1) * STAGE;
      const bool more = kt + 1 < nk;
      if (more) {  // the other half of the ring is free since the last barrier
        issue_x(kbeg + (kt + 1) * BK, nxt);
        fetch_w(kbeg + (kt + 1) * BK, rw);
      }
      mfma_slice(smem + (kt & 1) * STAGE);
      __builtin_amdgcn_sched_barrier(0);  // keep the dequantisation (and its wait for the loads) after the MFMAs
      if (more) stash_w(nxt + BM * ROW, rw);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // next x slice landed in LDS
      __syncthreads();                                  // ... for every wave; and this slice is no longer read
    }
  }

  const int mw = m0 + wm * 16 * TM, nw = n0 + wn * 16 * TN;
  if (gridDim.y > 1) {  // fp32 partials of this split
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = mw + i * 16 + 4 * (lane >> 4) + e, n = nw + j * 16 + (lane & 15);
          if (m < M && n < N) ws[((int64_t)blockIdx.y * M + m) * N + n] = acc[i][j][e];
        }
    return;
  }
  // 16-bit output through a per-wavefront LDS slab (16 rows x 16 TN columns), stored as 16-byte row segments
  constexpr int SW = 16 * TN, SP = SW + 8;
  uint16_t* slab = reinterpret_cast<uint16_t*>(smem) + wave * 16 * SP;  // the ring is free after the last barrier
  float cb[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) cb[j] = bias ? load_f(bias, bdt, min(nw + j * 16 + (lane & 15), N - 1)) : 0.f;
  const bool vec_ok = (ldy % 8) == 0 && (reinterpret_cast<uintptr_t>(y) % 16) == 0;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float v = bias ? acc[i][j][e] + cb[j] : acc[i][j][e];
        slab[(4 * (lane >> 4) + e) * SP + j * 16 + (lane & 15)] = XBF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
      }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's slab writes are done before it reads them
#pragma unroll
    for (int u0 = 0; u0 < 16 * SW / 8; u0 += 64) {
      const int u = u0 + lane, r = u / (SW / 8), c8 = u % (SW / 8);
      const int m = mw + i * 16 + r, n = nw + c8 * 8;
      const uint4 v = *reinterpret_cast<const uint4*>(slab + r * SP + c8 * 8);
      if (m < M) {
        uint16_t* yr = y + (int64_t)m * ldy;
        if (n + 8 <= N && vec_ok) {
          *reinterpret_cast<uint4*>(yr + n) = v;
        } else {
          const uint16_t h[8] = {(uint16_t)v.x, (uint16_t)(v.x >> 16), (uint16_t)v.y, (uint16_t)(v.y >> 16),
                                 (uint16_t)v.z, (uint16_t)(v.z >> 16), (uint16_t)v.w, (uint16_t)(v.w >> 16)};
          for (int t = 0; t < 8 && n + t < N; ++t) yr[n + t] = h[t];
        }
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads done before the next slab overwrites the buffer
  }
}

bool w4_big_ok(const void* x, int64_t ldx, const int32_t* qw, int64_t ldq, const int32_t* perm, int64_t K, int gs,
               int64_t G) {
  return perm == nullptr && (K % kW4BigBK) == 0 && ((gs % 32) == 0 || G == 1) && (ldx % 8) == 0 &&
         (reinterpret_cast<uintptr_t>(x) % 16) == 0 && (ldq % 4) == 0 && (reinterpret_cast<uintptr_t>(qw) % 16) == 0 &&
         group_div_exact(K, gs, G, 32);
}

// Row tile and K splits: 256 x 256 tiles when they alone cover the CUs, 64 x 256 for M <= 64, else 128 x 256, split
// over K (in 64-column slices, at least 512 columns each) into as many parts as keep the workgroups within one round
// over the CUs.  8-bit weights over K >= 8192 take 256-row tiles from 129 rows when those fill the round at least as
// well (each tile reads half as many weight bytes per row of x).
void w4_big_plan(int M, int N, int K, int split_k, int* bm, int* splits, int* kchunk, bool w8) {
  const int cus = device_cus();
  const int64_t t256 = (int64_t)((M + 255) / 256) * ((N + kW4BigBN - 1) / kW4BigBN);
  const int64_t t128 = (int64_t)((M + 127) / 128) * ((N + kW4BigBN - 1) / kW4BigBN);
  const int64_t t64 = (int64_t)((M + 63) / 64) * ((N + kW4BigBN - 1) / kW4BigBN);
  // 256-row tiles from three quarters of a round of them (graph replays, random weights: qkv M = 2048, 192 tiles,
  // 132 us against 178 with 128-row tiles; gate+up M = 512, 224 tiles, 141 against 194; o_proj / down M = 2048 at 128
  // tiles stay on 128 rows: 98 / 319 us against 125 / 385)
  *bm = 4 * t256 >= 3 * cus ? 256 : (M <= 64 ? 64 : 128);
  // as many splits as fit in one round of workgroups (gate+up at M = 64 / 128, 112 tiles: 2 splits take 57.5 / 71.3
  // us, 3 -- a round and a third -- 60.1 / 85.0)
  auto auto_splits = [&](int64_t tiles) {
    int s = tiles >= cus ? 1 : (int)(cus / tiles);
    const int max_s = K / 512 > 0 ? K / 512 : 1;
    return s > max_s ? max_s : (s > 16 ? 16 : s);
  };
  // W8A16 down (K = 14336, N = 4096), us, 256- / 128-row tiles: M = 192 59.5 / 65.3, 384 93 / 96, 512 95 / 112, 640
  // 130 / 137; K = 8192, N = 28672, M = 192 180 / 203 (4-bit weights and K = 4096 shapes: level or behind)
  if (w8 && *bm == 128 && M > 128 && K >= 8192 && split_k <= 0 &&
      std::min<int64_t>(t256 * auto_splits(t256), cus) >= std::min<int64_t>(t128 * auto_splits(t128), cus))
    *bm = 256;
  const int64_t tiles = *bm == 256 ? t256 : (*bm == 128 ? t128 : t64);
  int s = split_k;
  if (s <= 0) s = auto_splits(tiles);
  int kc = (K + s - 1) / s;
  const int unit = K % (2 * kW4BigBK) == 0 ? 2 * kW4BigBK : kW4BigBK;  // whole slice pairs where K allows them
  kc = (kc + unit - 1) / unit * unit;
  *kchunk = kc;
  *splits = (K + kc - 1) / kc;
}

size_t w4_big_workspace_bytes(int M, int N, int K, int split_k, bool w8) {
  int bm, s, kc;
  w4_big_plan(M, N, K, split_k, &bm, &s, &kc, w8);
  return s > 1 ? (size_t)s * (size_t)M * (size_t)N * sizeof(float) : 0;
}

template <bool XBF16>
hipError_t launch_w4_splitk_reduce(const float* ws, int S, int M, int N, const void* bias, int bdt, void* y,
                                   int64_t ldy, hipStream_t s);

template <int BM, bool XBF16, int WB>
static hipError_t launch_w4_big_t(const void* x, int64_t ldx, const void* qw, int64_t ldq, const void* scales,
                                  int sdt, int64_t lds, const int32_t* zeros, int64_t ldz, const void* bias, int bdt,
                                  void* y, int64_t ldy, float* ws, int M, int N, int K, int gs32, int splits,
                                  int kchunk, hipStream_t s) {
  constexpr size_t shm = 2 * (size_t)(BM + kW4BigBN) * kW4BigBK * 2;
  // the unrolled forms: 16-bit scales, and every K chunk an even number of slices (w4_big_plan rounds chunks to 128
  // columns when K allows); two register sets for 64- and 128-row tiles, one for 256 (no registers left)
  const bool pf = sdt != FG_F32 && K % (2 * kW4BigBK) == 0;
  constexpr int kPf = BM <= 128 ? 2 : 1;
  auto kern = pf ? w4_big_kernel<BM, XBF16, WB, kPf> : w4_big_kernel<BM, XBF16, WB, 0>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)shm);
  if (e != hipSuccess) return e;
  const int hasz = zeros != nullptr;
  const int32_t* zp = hasz ? zeros : static_cast<const int32_t*>(qw);  // symmetric: a valid dummy word, ignored
  const int64_t ldzp = hasz ? ldz : 0;
  const int tiles = ((M + BM - 1) / BM) * ((N + kW4BigBN - 1) / kW4BigBN);
  note_kernel("w4_big_kernel<%d,%s,w%d> splits=%d%s", BM, XBF16 ? "bf16" : "f16", WB, splits,
              splits > 1 ? " + w4_splitk_reduce_kernel" : "");
  hipLaunchKernelGGL(kern, dim3(tiles, splits), dim3(kW4BigThreads), shm, s, static_cast<const uint16_t*>(x), ldx, qw,
                     ldq, scales, sdt, lds, zp, ldzp, hasz, bias, bdt, static_cast<uint16_t*>(y), ldy, ws, M, N, K,
                     gs32, kchunk);
  e = hipGetLastError();
  if (e != hipSuccess || splits == 1) return e;
  return launch_w4_splitk_reduce<XBF16>(ws, splits, M, N, bias, bdt, y, ldy, s);
}

hipError_t launch_w4_big(const void* x, int64_t ldx, bool xbf16, const int32_t* qw, int64_t ldq, const void* scales,
                         int sdt, int64_t lds, const int32_t* zeros, int64_t ldz, const void* bias, int bdt, void* y,
                         int64_t ldy, float* ws, int M, int N, int K, int gs, bool single_group, int split_k,
                         hipStream_t s) {
  int bm, splits, kchunk;
  w4_big_plan(M, N, K, split_k, &bm, &splits, &kchunk, false);
  const int gs32 = single_group ? 0 : gs / 32;
#define FG_W4BIG(BM_, XB_)                                                                                             \
  return launch_w4_big_t<BM_, XB_, 4>(x, ldx, qw, ldq, scales, sdt, lds, zeros, ldz, bias, bdt, y, ldy, ws, M, N, K, \
                                      gs32, splits, kchunk, s)
  if (xbf16) {
    if (bm == 256) FG_W4BIG(256, true);
    if (bm == 64) FG_W4BIG(64, true);
    FG_W4BIG(128, true);
  }
  if (bm == 256) FG_W4BIG(256, false);
  if (bm == 64) FG_W4BIG(64, false);
  FG_W4BIG(128, false);
#undef FG_W4BIG
}

// W8A16 through the same kernel (int8 qweight, ldq in bytes, no zero-points).
bool w8_big_ok(const void* x, int64_t ldx, const int8_t* qw, int64_t ldq, int64_t K, int gs, int64_t G) {
  return (K % kW4BigBK) == 0 && ((gs % 32) == 0 || G == 1) && (ldx % 8) == 0 &&
         (reinterpret_cast<uintptr_t>(x) % 16) == 0 && (ldq % 16) == 0 && (reinterpret_cast<uintptr_t>(qw) % 16) == 0 &&
         group_div_exact(K, gs, G, 32);
}

hipError_t launch_w8_big(const void* x, int64_t ldx, bool xbf16, const int8_t* qw, int64_t ldq, const void* scales,
                         int sdt, int64_t lds, const void* bias, int bdt, void* y, int64_t ldy, float* ws, int M,
                         int N, int K, int gs, bool single_group, int split_k, hipStream_t s) {
  int bm, splits, kchunk;
  w4_big_plan(M, N, K, split_k, &bm, &splits, &kchunk, true);
  const int gs32 = single_group ? 0 : gs / 32;
#define FG_W8BIG(BM_, XB_)                                                                                         \
  return launch_w4_big_t<BM_, XB_, 8>(x, ldx, qw, ldq, scales, sdt, lds, nullptr, 0, bias, bdt, y, ldy, ws, M, N, \
                                      K, gs32, splits, kchunk, s)
  if (xbf16) {
    if (bm == 256) FG_W8BIG(256, true);
    if (bm == 64) FG_W8BIG(64, true);
    FG_W8BIG(128, true);
  }
  if (bm == 256) FG_W8BIG(256, false);
  if (bm == 64) FG_W8BIG(64, false);
  FG_W8BIG(128, false);
#undef FG_W8BIG
}

}  // namespace fg
