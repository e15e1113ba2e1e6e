// W4A16 for 1..64 rows of x on the CDNA4 MFMA-fragment weight layout (w4.cdna4_mfma_k128n16), with every operand of a
// 128-column K step brought into an S-stage LDS ring by direct-to-LDS buffer loads:
//   y[M,N] = x[M,K] @ dequant(W)[N,K]^T (+bias),  v_mfma_f32_16x16x32_{bf16,f16}.
//
// A workgroup of BW wavefronts owns BW * T 16-channel tiles and one K split.  Per step it loads, straight into LDS
// (no registers, no VALU):
//   x      the MB * 16 rows x 128 columns of the step, 256 bytes per row, 16-byte unit u of row r stored at
//          u ^ (r % 16) (the 16 rows of one A-fragment read fall on 16 distinct bank groups); shared by all BW * T
//          tiles, so x crosses the L2 once per workgroup and step instead of once per wavefront;
//   W      each tile's 1 KiB for the step, lane l's 16 bytes at l * 16 (the B operand of the four k-steps, in the
//          order the layout stores them);
//   s, z   the scales and zero words of the wavefront's channels for the step's group.
// Each wavefront issues the same NI = 4 MB / BW + T + 2 loads per step, and no other vector-memory load in the loop,
// so `s_waitcnt vmcnt((S - 2) * NI)` before the step's barrier is exactly "this step has landed" (the loads of the next
// S - 2 steps stay in flight).  Steps past the split go through a zero-length buffer resource: the same instructions
// (so the count holds), reading 0 and moving no memory.  Rows of x past M and tiles past N read out of range (0).
//
// Arithmetic, as w4_frag_kernel: B = magic | nibble pair ((word >> 4 p) & 0x000F000F | 0x4300 4300 for bf16, 0x6400
// 6400 for fp16: the exact values 128 + q / 1024 + q), one v_and_or_b32 per pair (plus a shift for p > 0); per step
// acc += s * (acc_step - (B + z) * xsum), the x row sums from MFMAs against all-ones.  The row sums of a step are the
// same for every wavefront: on eight wavefronts, wavefront b < MB computes those of row block b into an LDS pair
// buffered by step parity, and every wavefront subtracts s * (B + z) * xsum one step later, after the next step's
// barrier has made them visible (the last step's after one more barrier at the end).
//
// K splits (KS > 1): each split writes its fp32 partial to the caller's workspace [KS, M, N] and w4_ring_reduce_kernel
// sums them in split order (bit-reproducible), adds the bias and rounds, four outputs per thread.  (Letting the last
// split of a group reduce instead measured slower both ways it was built: with a device-scope release per workgroup,
// an L2 writeback, 60-100x; with partials stored and re-read at device scope and an arrival counter, 1.2-6 us per
// call, the last workgroup's store, atomic and load round trips running in series.)
//
// Requirements (w4_ring_ok): M <= 64, N % 16 == 0, K % 128 == 0, group size % 128 == 0 or one group, 16-bit scales
// with lds even and 4-byte aligned scales / zeros, 16-byte aligned x with ldx % 8 == 0, 16-byte aligned qweight with
// ldq % 4 == 0, every operand spanning < 2 GiB.
#include "fg_device.h"

namespace fg {

typedef __bf16 bf16x8_rg_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_rg_t __attribute__((ext_vector_type(8)));
typedef float f32x4_rg_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;

template <bool XBF16>
__device__ __forceinline__ f32x4_rg_t rg_mfma(uint4 a, uint4 b, f32x4_rg_t c) {
  if constexpr (XBF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_rg_t, a),
                                                   __builtin_bit_cast(bf16x8_rg_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_rg_t, a),
                                                  __builtin_bit_cast(f16x8_rg_t, b), c, 0, 0, 0);
  }
}

// (a & mask) | magic: one v_and_or_b32 once the caller has hidden the constants from the compiler (mask in a scalar
// register, magic in a vector register; with literals it emits a v_and + v_or pair).  Plain C rather than inline asm:
// the result feeds MFMA B operands, and the hazard recognizer inserts the wait states a VALU write needs before an
// MFMA reads it only for instructions it can see (an asm v_and_or_b32 one instruction ahead of its MFMA produced
// wrong products).
__device__ __forceinline__ uint32_t rg_and_or(uint32_t a, uint32_t mask, uint32_t magic) { return (a & mask) | magic; }

// one k-step's word -> the lane's eight B values as four exact 16-bit pairs
__device__ __forceinline__ uint4 rg_unpack(uint32_t w, uint32_t mask, uint32_t magic) {
  return make_uint4(rg_and_or(w, mask, magic), rg_and_or(w >> 4, mask, magic), rg_and_or(w >> 8, mask, magic),
                    rg_and_or(w >> 12, mask, magic));
}

// portable_row word (nibble t = column t) -> the same four pairs in column order: byte p of w and of w >> 4 moved to
// bytes 0 and 2 by one v_perm_b32 (bytes 1 and 3 zero), then masked and tagged (nibble 2p | magic, 2p + 1 | magic)
__device__ __forceinline__ uint4 rg_unpack_portable(uint32_t w, uint32_t mask, uint32_t magic) {
  const uint32_t h = w >> 4;
  return make_uint4(rg_and_or(__builtin_amdgcn_perm(h, w, 0x0C040C00u), mask, magic),
                    rg_and_or(__builtin_amdgcn_perm(h, w, 0x0C050C01u), mask, magic),
                    rg_and_or(__builtin_amdgcn_perm(h, w, 0x0C060C02u), mask, magic),
                    rg_and_or(__builtin_amdgcn_perm(h, w, 0x0C070C03u), mask, magic));
}

template <int MB, int T, int BW, bool W8 = false>
struct RingShape {
  static_assert((4 * MB) % BW == 0, "the x rows of a step split evenly over the wavefronts");
  static constexpr int X = MB * 16 * 256;     // x rows of one step
  static constexpr int TB = W8 ? 2048 : 1024;  // one 16-channel tile's weights per step
  static constexpr int W = BW * T * TB;       // weight tiles of one step
  static constexpr int SB = W8 ? 256 : 512;   // per wavefront: 256 bytes of scales (+ 256 of zero words for W4)
  static constexpr int SZ = BW * SB;
  static constexpr int STAGE = X + W + SZ;
  static constexpr bool SHARE = MB >= 2 && BW == 8;  // x row sums computed once per workgroup (w4_ring_kernel)
  static constexpr int XS = SHARE ? 2 * MB * 16 * 4 : 0;  // the row sums of two steps (fp32), after the S stages
  static constexpr int XI = 4 * MB / BW;      // x loads (1 KiB = 4 rows each) per wavefront and step
  static constexpr int NI = XI + (W8 ? 2 * T + 1 : T + 2);  // loads per wavefront and step
};

// Swizzle of a W8 tile's 128-byte rows in LDS: 16-byte unit u of row r at position u ^ key (the units 2 j, 2 j + 1
// that lane group j reads of 16 rows fall on distinct bank groups; the same key as the FP8 MFMA operand's rows).
__device__ __forceinline__ int w8_ring_key(int r) { return (r & 7) ^ ((r >> 3) & 1); }

struct RingArgs {
  const uint16_t* x;
  int64_t ldx;
  const int32_t* qw;
  int64_t ldq;  // W4: int32 words per row (portable) or per 16-channel tile row (CDNA4); W8: bytes per row
  const uint16_t* scales;
  int64_t lds;
  const int32_t* zeros;
  int64_t ldz;
  const void* bias;
  float* part;  // KS > 1: fp32 partials [KS, M, N]
  uint16_t* y;
  int64_t ldy;
  int M, N, K, gsteps, KS, ngrp, hasz, bdt;
  uint32_t qbytes, xbytes, sbytes, zbytes;
};

// FMT 1: W4 weights in portable_row ([N, ldq] int32 words, row n = channel n): a tile's step is 16 rows x 64 bytes,
// loaded into LDS row by row with the 16-byte quarter q of row r at position q ^ ((r / 4) % 4) (the 16 rows of one
// B read fall on distinct bank groups), and lane group j takes quarter j: MFMA k-step s of lane group j is word 4 j + s
// (columns 32 j + 8 s ..), so x's unit 4 j + s goes with it (the sum over K does not care which 32 columns go to
// which k-step).  FMT 0: the CDNA4 layout: lane l's 16 bytes at l * 16, k-step s = word s (columns 32 s + 8 j ..).
// FMT 2: W8A16 weights (int8 [N, ldq] bytes, symmetric, scales [G, N]): a tile's step is 16 rows x 128 bytes (two
// loads), unit u of row r at position u ^ w8_ring_key(r); lane group j reads units 2 j, 2 j + 1 of its row, the
// 32 bytes of columns 32 j .. 32 j + 31, k-step s takes bytes 8 s .. 8 s + 7 (x's unit 4 j + s, as for FMT 1).  A
// byte q becomes u = q ^ 0x80 = q + 128, exact as a bf16 (0..255) or, for fp16 x, as 1024 + u above the magic
// exponent byte, so  sum x q = sum x B - (128 or 1152) sum x  in place of W4's  - (B + z) sum x.
template <int MB, int T, int BW, int S, bool XBF16, bool SBF16, int FMT>
__device__ __forceinline__ void ring_body(const RingArgs& a) {
  constexpr bool PORT = FMT != 0, W8 = FMT == 2;
  using Sh = RingShape<MB, T, BW, W8>;
  static_assert(S >= 2 && (S - 2) * Sh::NI <= 63, "the wait count must fit vmcnt");
  // Row sums shared through LDS on eight wavefronts of 17..64 rows (wavefront b < MB computes row block b's).
  // Elsewhere every wavefront computes its MB blocks' sums itself: with fewer row blocks than wavefronts wavefront 0
  // computes as many either way, and on four wavefronts the fewer MFMAs did not make up for the extra LDS reads of x
  // (M = 64: qkv 17.2 -> 16.5 us, down 25.2 -> 23.7 with sharing; o_proj 14.4 -> 14.8, gate+up level on four
  // wavefronts).
  constexpr bool SHARE = Sh::SHARE;
  constexpr float kB = XBF16 ? 128.f : 1024.f;
  const float zsel = a.hasz ? 1.f : 0.f;  // zero-points present
  constexpr float kCorr8 = XBF16 ? 128.f : 1152.f;  // W8: B = q + 128 (bf16) / 1024 + q + 128 (fp16)
  constexpr uint32_t kOnes = XBF16 ? 0x3F803F80u : 0x3C003C00u;
  extern __shared__ __align__(16) uint8_t smem[];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave);
  const int grp = blockIdx.x % a.ngrp, ks = blockIdx.x / a.ngrp;
  const int nsteps = a.K / 128;
  const int st0 = (int)((int64_t)ks * nsteps / a.KS), ns = (int)((int64_t)(ks + 1) * nsteps / a.KS) - st0;
  const int NT = a.N / 16;
  const int tile0 = (grp * BW + wave) * T;  // first tile of this wavefront
  const int r16 = lane & 15, j = lane >> 4;

  const __amdgpu_buffer_rsrc_t rx = buf_rsrc(a.x, a.xbytes), rq = buf_rsrc(a.qw, a.qbytes);
  const __amdgpu_buffer_rsrc_t rs = buf_rsrc(a.scales, a.sbytes), rz = buf_rsrc(a.zeros, a.zbytes);
  const __amdgpu_buffer_rsrc_t rx0 = buf_rsrc(a.x, 0u), rq0 = buf_rsrc(a.qw, 0u);
  const __amdgpu_buffer_rsrc_t rs0 = buf_rsrc(a.scales, 0u), rz0 = buf_rsrc(a.zeros, 0u);

  // per-lane load offsets (step 0); rows past M and tiles past N point past their operand
  uint32_t xv[Sh::XI];
#pragma unroll
  for (int q = 0; q < Sh::XI; ++q) {
    const int row = (wave * Sh::XI + q) * 4 + (lane >> 4);
    const int u = (lane & 15) ^ (row & 15);
    xv[q] = row < a.M ? (uint32_t)row * (uint32_t)a.ldx * 2u + 16u * (uint32_t)u : a.xbytes;
  }
  constexpr int WH = W8 ? 2 : 1;  // weight loads per tile and step
  uint32_t wv[T][WH];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    if constexpr (W8) {  // load h: LDS position lane = row 8 h + lane / 8, slot lane % 8, holding unit slot ^ key(row)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int row = 8 * h + (lane >> 3), unit = (lane & 7) ^ w8_ring_key(row);
        wv[t][h] = tile0 + t < NT
                       ? ((uint32_t)(tile0 + t) * 16u + (uint32_t)row) * (uint32_t)a.ldq + 16u * (uint32_t)unit
                       : a.qbytes;
      }
    } else if constexpr (PORT) {  // LDS position lane = row lane / 4, slot lane % 4: quarter slot ^ (row / 4 % 4)
      const int row = lane >> 2, quarter = (lane & 3) ^ ((lane >> 4) & 3);
      wv[t][0] = tile0 + t < NT
                     ? ((uint32_t)(tile0 + t) * 16u + (uint32_t)row) * (uint32_t)a.ldq * 4u + 16u * (uint32_t)quarter
                     : a.qbytes;
    } else {
      wv[t][0] = tile0 + t < NT ? (uint32_t)(tile0 + t) * (uint32_t)a.ldq * 4u + 16u * (uint32_t)lane : a.qbytes;
    }
  }
  // scales: lane i < 8 T loads the channel pair 2i, 2i + 1 of the wavefront's tiles; zero words: lane i < 2 T loads
  // word i (eight channels each)
  const bool sl = lane < 8 * T && tile0 + lane / 8 < NT, zl = lane < 2 * T && tile0 + lane / 2 < NT;
  const uint32_t sv = (uint32_t)tile0 * 32u + 4u * (uint32_t)lane, zv = (uint32_t)tile0 * 8u + 4u * (uint32_t)lane;
  const FastDiv gdiv((uint32_t)max(a.gsteps, 1));
  const uint32_t lds2 = (uint32_t)a.lds * 2u, ldz4 = (uint32_t)a.ldz * 4u;

  // stage i of the split into the ring slot at stg (i >= ns: zero-length resources, nothing moves)
  auto issue = [&](int i, uint8_t* stg) __attribute__((always_inline)) {
    const bool live = i < ns;
    const int st = st0 + (live ? i : 0);
    const uint32_t g = a.gsteps > 0 ? gdiv.div((uint32_t)st) : 0u;
    const __amdgpu_buffer_rsrc_t x_ = live ? rx : rx0, q_ = live ? rq : rq0;
    const __amdgpu_buffer_rsrc_t s_ = live ? rs : rs0, z_ = live ? rz : rz0;
#pragma unroll
    for (int q = 0; q < Sh::XI; ++q)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(x_, (lds_void_t*)(stg + (wave * Sh::XI + q) * 1024), 16, (int)xv[q],
                                               st * 256, 0, 0);
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int h = 0; h < WH; ++h)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(q_, (lds_void_t*)(stg + Sh::X + (wave * T + t) * Sh::TB + h * 1024),
                                                 16, (int)wv[t][h], st * (W8 ? 128 : (PORT ? 64 : 1024)), 0, 2);
    // the group row goes into the per-lane offset (past-the-end lanes must stay past the end)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(s_, (lds_void_t*)(stg + Sh::X + Sh::W + wave * Sh::SB), 4,
                                             sl ? (int)(g * lds2 + sv) : (int)a.sbytes, 0, 0, 0);
    if constexpr (!W8)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(z_, (lds_void_t*)(stg + Sh::X + Sh::W + wave * Sh::SB + 256), 4,
                                               zl ? (int)(g * ldz4 + zv) : (int)a.zbytes, 0, 0, 0);
  };

  f32x4_rg_t acc[T][MB];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[t][i] = f32x4_rg_t{0.f, 0.f, 0.f, 0.f};
  uint32_t mask = 0x000F000Fu, magic = XBF16 ? 0x43004300u : 0x64006400u;
  asm("" : "+s"(mask));  // opaque to constant folding: v_and_or_b32 with a scalar mask and a vector magic
  asm("" : "+v"(magic));
  const uint4 ones = make_uint4(kOnes, kOnes, kOnes, kOnes);

  // row sums by step parity: step i's are written into xsb[i % 2] and read at step i + 1
  float* const xsb = reinterpret_cast<float*>(smem + S * Sh::STAGE);
  if constexpr (SHARE)  // read at step 0 (times zero)
    for (int q = (int)threadIdx.x; q < 2 * MB * 16; q += BW * kWave) xsb[q] = 0.f;
  float szb[T];  // s * (B + z) of the previous step, per tile
#pragma unroll
  for (int t = 0; t < T; ++t) szb[t] = 0.f;

  auto compute = [&](const uint8_t* __restrict__ stg, float* __restrict__ xsw, const float* __restrict__ xsr)
                     __attribute__((always_inline)) {
    if (SHARE && wave < MB) {  // first, this step's row sums of row block `wave`, for every wavefront
      const uint8_t* xr = stg + (16 * wave + r16) * 256;
      f32x4_rg_t xs = f32x4_rg_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s)
        xs = rg_mfma<XBF16>(*reinterpret_cast<const uint4*>(xr + (((PORT ? 4 * j + s : 4 * s + j) ^ r16) * 16)), ones,
                            xs);
      if (r16 == 0) *reinterpret_cast<f32x4_rg_t*>(xsw + 16 * wave + 4 * j) = xs;
    }
    const uint8_t* sw = stg + Sh::X;
    const uint8_t* ssz = stg + Sh::X + Sh::W + wave * Sh::SB;
    uint4 raw[T][WH];
    float sc[T], zb[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      if constexpr (W8) {
        const uint8_t* tr = sw + (wave * T + t) * Sh::TB + r16 * 128;
#pragma unroll
        for (int h = 0; h < 2; ++h)
          raw[t][h] = *reinterpret_cast<const uint4*>(tr + (((2 * j + h) ^ w8_ring_key(r16)) * 16));
      } else {
        const int wpos = PORT ? r16 * 64 + ((j ^ ((r16 >> 2) & 3)) * 16) : lane * 16;
        raw[t][0] = *reinterpret_cast<const uint4*>(sw + (wave * T + t) * 1024 + wpos);
      }
      const uint16_t sb = reinterpret_cast<const uint16_t*>(ssz)[t * 16 + r16];
      sc[t] = SBF16 ? bf16_bits_to_f32(sb) : f16_bits_to_f32(sb);
      if constexpr (W8) {
        zb[t] = kCorr8;
      } else {
        // B + z without a branch (symmetric: zsel = 0 and the zero words read as 0): behind a branch the compiler
        // waits for this one LDS read before issuing the step's fragment reads
        const uint32_t zw = reinterpret_cast<const uint32_t*>(ssz + 256)[t * 2 + (r16 >> 3)];
        zb[t] = __builtin_fmaf(zsel, (float)nibble(zw, r16 & 7) - 8.f, kB + 8.f);
      }
    }
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      uint4 af[4];
#pragma unroll
      for (int s = 0; s < 4; ++s)
        af[s] = *reinterpret_cast<const uint4*>(stg + (16 * i + r16) * 256 +
                                                (((PORT ? 4 * j + s : 4 * s + j) ^ r16) * 16));
      f32x4_rg_t xp;  // SHARE: the previous step's row sums; else this step's
      if constexpr (SHARE) {
        xp = *reinterpret_cast<const f32x4_rg_t*>(xsr + 16 * i + 4 * j);
      } else {
        xp = f32x4_rg_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) xp = rg_mfma<XBF16>(af[s], ones, xp);
      }
#pragma unroll
      for (int t = 0; t < T; ++t) {
        f32x4_rg_t as = f32x4_rg_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          uint4 bop;
          if constexpr (W8) {  // bytes 8 s .. 8 s + 7 of the lane's 32
            const uint4 rw = raw[t][s >> 1];
            const uint32_t u0 = ((s & 1) ? rw.z : rw.x) ^ 0x80808080u, u1 = ((s & 1) ? rw.w : rw.y) ^ 0x80808080u;
            bop = XBF16 ? make_uint4(w8a_bf16_pair(u0, 0), w8a_bf16_pair(u0, 1), w8a_bf16_pair(u1, 0),
                                     w8a_bf16_pair(u1, 1))
                        : make_uint4(w8a_pair_lo(0x64646464u, u0), w8a_pair_hi(0x64646464u, u0),
                                     w8a_pair_lo(0x64646464u, u1), w8a_pair_hi(0x64646464u, u1));
          } else {
            const uint4 rw = raw[t][0];
            const uint32_t wq = s == 0 ? rw.x : (s == 1 ? rw.y : (s == 2 ? rw.z : rw.w));
            bop = PORT ? rg_unpack_portable(wq, mask, magic) : rg_unpack(wq, mask, magic);
          }
          as = rg_mfma<XBF16>(af[s], bop, as);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e)
          acc[t][i][e] = SHARE ? __builtin_fmaf(sc[t], as[e], __builtin_fmaf(-szb[t], xp[e], acc[t][i][e]))
                               : __builtin_fmaf(sc[t], __builtin_fmaf(-zb[t], xp[e], as[e]), acc[t][i][e]);
      }
    }
    if constexpr (SHARE) {
#pragma unroll
      for (int t = 0; t < T; ++t) szb[t] = sc[t] * zb[t];
    }
  };

#pragma unroll
  for (int p = 0; p < S - 1; ++p) issue(p, smem + p * Sh::STAGE);
  // The slot being read and the slot being loaded reach the body as __restrict__ pointers, so the compiler does not
  // wait for the loads in flight before the LDS reads.
  auto body = [&](int i, const uint8_t* __restrict__ cur, uint8_t* __restrict__ nxt) __attribute__((always_inline)) {
    issue(i + S - 1, nxt);  // the slot of step i - 1: every wavefront has read it (last barrier)
    __builtin_amdgcn_sched_barrier(0);
    compute(cur, xsb + (i & 1) * MB * 16, xsb + ((i + 1) & 1) * MB * 16);
  };
  // Before each step: this step's loads have landed for every wavefront, every wavefront is done with step i - 1's
  // slot and with the row sums of step i - 2, and step i - 1's row sums are in LDS.  With four wavefronts and 17..64
  // rows the loop is unrolled by S so that every ring slot is a constant offset (no per-step address arithmetic: M = 64
  // o_proj 14.45 -> 13.5 us on the CDNA4 layout, and as much on two-tile wavefronts); on eight wavefronts and on 1..16
  // rows the unrolled form measured slower (portable qkv M = 64 17.5 -> 18.7, down M = 16 14.9 -> 15.5) and the loop
  // stays rolled.
  if constexpr (BW == 4 && MB >= 2) {
    int i = 0;
    for (; i + S <= ns; i += S) {
#pragma unroll
      for (int u = 0; u < S; ++u) {
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((S - 2) * Sh::NI) : "memory");
        body(i + u, smem + u * Sh::STAGE, smem + ((u + S - 1) % S) * Sh::STAGE);
      }
    }
#pragma unroll
    for (int u = 0; u < S - 1; ++u) {  // the last ns % S steps (i is a multiple of S)
      if (i + u < ns) {
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((S - 2) * Sh::NI) : "memory");
        body(i + u, smem + u * Sh::STAGE, smem + ((u + S - 1) % S) * Sh::STAGE);
      }
    }
  } else {
    for (int i = 0; i < ns; ++i) {
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((S - 2) * Sh::NI) : "memory");
      body(i, smem + (i % S) * Sh::STAGE, smem + ((i + S - 1) % S) * Sh::STAGE);
    }
  }
  // the last step's row sums
  if constexpr (SHARE) {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    const float* xsr = xsb + ((ns + 1) & 1) * MB * 16;
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      const f32x4_rg_t xp = *reinterpret_cast<const f32x4_rg_t*>(xsr + 16 * i + 4 * j);
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[t][i][e] = __builtin_fmaf(-szb[t], xp[e], acc[t][i][e]);
    }
  }

  // KS == 1: y (+ bias); KS > 1: this split's fp32 partial
  float* part = a.part + (int64_t)ks * a.M * a.N;
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = 16 * i + 4 * j + e, n = (tile0 + t) * 16 + r16;
        if (m < a.M && tile0 + t < NT) {
          float v = acc[t][i][e];
          if (a.KS > 1) {
            part[(int64_t)m * a.N + n] = v;
          } else {
            if (a.bias) v += load_f(a.bias, a.bdt, n);
            a.y[(int64_t)m * a.ldy + n] = XBF16 ? f32_to_bf16_bits_hw(v) : f32_to_f16_bits(v);
          }
        }
      }
}

template <int MB, int T, int BW, int S, bool XBF16, bool SBF16, bool PORT>
__global__ void __launch_bounds__(BW * kWave) w4_ring_kernel(RingArgs a) {
  ring_body<MB, T, BW, S, XBF16, SBF16, PORT ? 1 : 0>(a);
}

// W8A16 (int8 weight-only, portable [N, K] bytes) for 1..64 rows of x: the same LDS ring (FMT 2 above).
template <int MB, int T, int BW, int S, bool XBF16, bool SBF16>
__global__ void __launch_bounds__(BW * kWave) w8a16_ring_kernel(RingArgs a) {
  ring_body<MB, T, BW, S, XBF16, SBF16, 2>(a);
}

// y[m, n .. n + 3] = sum over the KS partials in split order (+ bias), one thread per 4 outputs (N % 16 == 0).  The
// partials are loaded eight splits at a time before any is added (a loop that adds each split as it arrives waits out
// one round trip per split: 4.2 us for 4 splits of a 64 x 4096 output), then summed in split order.  Four outputs per
// thread rather than eight: twice the workgroups for the short outputs of 16 rows, and with the plans' K splits (at
// most 8) every load of a thread in one round trip.
template <bool XBF16>
__global__ void __launch_bounds__(256) w4_ring_reduce_kernel(const float* __restrict__ part, int KS, int M, int N,
                                                             const void* __restrict__ bias, int bdt,
                                                             uint16_t* __restrict__ y, int64_t ldy, int vec_store) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // group of 4 outputs
  const int n4 = N / 4;
  if (idx >= (int64_t)M * n4) return;
  const int m = (int)(idx / n4), n = (int)(idx - (int64_t)m * n4) * 4;
  const int64_t MN4 = (int64_t)M * N / 4;
  f32x4_rg_t acc = f32x4_rg_t{0.f, 0.f, 0.f, 0.f};
  const f32x4_rg_t* p = reinterpret_cast<const f32x4_rg_t*>(part + (int64_t)m * N + n);
  for (int k = 0; k < KS; k += 8) {
    f32x4_rg_t v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = p[(int64_t)min(k + u, KS - 1) * MN4];  // past the last split: re-read it
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (k + u < KS) acc += v[u];  // ... and add nothing
  }
  uint16_t h[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float v = acc[e];
    if (bias) v += load_f(bias, bdt, n + e);
    h[e] = XBF16 ? f32_to_bf16_bits_hw(v) : f32_to_f16_bits(v);
  }
  uint16_t* yr = y + (int64_t)m * ldy + n;
  if (vec_store) {
    *reinterpret_cast<uint2*>(yr) = make_uint2(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16));
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) yr[e] = h[e];
  }
}

// portable: qweight [N, ldq] int32 (ldq >= K / 8); otherwise the CDNA4 tile rows [N / 16, ldq] (ldq >= 2 K)
bool w4_ring_ok(bool portable, const void* x, int64_t ldx, const int32_t* qw, int64_t ldq, const void* scales, int sdt,
                int64_t lds, const int32_t* zeros, int64_t ldz, int M, int64_t N, int64_t K, int gs, int64_t G) {
  const int64_t k2g = 1LL << 31;  // offsets past a span plus a step offset stay below 2^32
  const int64_t qspan = portable ? N * ldq * 4 : (N / 16) * ldq * 4;
  return M > 0 && M <= 64 && sdt != FG_F32 && N % 16 == 0 && (K % 128) == 0 && ((gs % 128) == 0 || G == 1) &&
         (ldx % 8) == 0 && (reinterpret_cast<uintptr_t>(x) % 16) == 0 && (ldq % 4) == 0 &&
         ldq >= (portable ? K / 8 : 2 * K) && (reinterpret_cast<uintptr_t>(qw) % 16) == 0 && (lds % 2) == 0 &&
         (reinterpret_cast<uintptr_t>(scales) % 4) == 0 && (reinterpret_cast<uintptr_t>(zeros) % 4) == 0 &&
         qspan < k2g && (int64_t)M * ldx * 2 < k2g && G * lds * 2 < k2g && G * ldz * 4 < k2g &&
         group_div_exact(K, gs, G, 128);
}

// Launch shape, from a sweep of (BW, T, KS) against the register-ring kernel (w4_frag_kernel) on the Llama-3-8B
// shapes at M = 1 / 16 / 32 / 64 (graph replays over a 1.2 GB weight ring): BW = 4 or 8 wavefronts, one tile each
// (T = 2 tiles per wavefront on four wavefronts was the gate+up choice before eight wavefronts shared the x row sums;
// now slower: M = 33 / 64 on the CDNA4 layout 34.7 / 35.9 us against 31.1 / 33.8, W8A16 M = 64 45.8 against 42.2,
// so the T = 2 instances are not built); KS = 1 when the
// channel groups fill three quarters of the CUs, else the smallest power of two that gives one wavefront per SIMD,
// doubled while a split is longer than 16 steps over K >= 8192 (down: 8 splits of 14 steps, 26.0 us at M = 64 against
// 30.7 with 4).
// Measured (us, this kernel + reduce / w4_frag_kernel): M = 64 qkv 18.4 / 21.2, o_proj 14.7 / 18.8, gate+up 37.9 /
// 44.0, down 26.0 / 54.7; M = 32 down 18.7 / 29.9; M = 16 down 15.9 / 17.0.  Below that the register ring is as fast
// or faster on the CDNA4 layout (w4_ring_preferred).
struct RingPlan {
  int mb, T, BW, KS, ngrp;
};

static RingPlan w4_ring_plan(int M, int N, int K) {
  RingPlan p;
  p.mb = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  const int NT = N / 16, nsteps = K / 128, cus = device_cus();
  p.T = 1;
  // eight wavefronts (x shared by 128 channels, row sums once per workgroup) for 17..64 rows on qkv-sized, wide or
  // long-K weights: M = 64 qkv 17.1 us against 18.5, down 25.7 against 28.2; M = 17..32 (portable) qkv 11.9-13.0
  // against 12.3-13.3, gate+up 26.0-26.8 against 27.2-28.3, down 17.2-18.8 against 18.4-20.0, W8A16 down M = 24 19.4
  // against 23.8; o_proj stays on four (M = 64 15.7 against 14.6, M = 17..32 10.4-11.4 against 10.0-10.6)
  p.BW = p.mb >= 2 && (NT >= 384 || nsteps >= 64) ? 8 : 4;
  p.ngrp = (NT + p.BW * p.T - 1) / (p.BW * p.T);
  int ks = 1;
  if (4 * p.ngrp < 3 * cus)
    while (p.ngrp * ks * p.BW < 4 * cus && 2 * ks <= nsteps) ks *= 2;
  if (nsteps >= 64)
    while (nsteps / ks > 16 && p.ngrp * ks < 4 * cus && 2 * ks <= nsteps) ks *= 2;
  p.KS = ks;
  return p;
}

// CDNA4 layout: 29..64 rows, and 9..28 over K >= 8192; below that the register ring is as fast or faster (us, LDS
// ring / register ring: M = 32 qkv 12.6 / 12.8, o_proj 10.3 / 11.3, gate+up 24.4 / 26.8; M = 24 qkv 12.2 / 11.6,
// o_proj and gate+up level; M = 17 qkv 11.7 / 10.3, o_proj 9.7 / 8.9).
// portable_row: also 17..32 rows, and 4..16 rows over wide outputs, where the ring replaces the skinny kernel (us,
// ring / skinny: M = 32 qkv 13.4 / 14.5, o_proj 11.1 / 12.2, gate+up 31.4 / 44.4; M = 24 gate+up 30.1 / 38.8; M = 16
// gate+up 23.6 / 25.9, qkv 11.0 / 10.0; gate+up M = 12 21.0-23.0 / 24.0, M = 8 22.2 / 23.3, M = 4 22.0 / 23.8,
// M = 3 level).
bool w4_ring_preferred(bool portable, int M, int N, int K) {
  if (M > 28 || (M > 8 && K >= 8192)) return true;
  return portable && (M > 16 || (M > 3 && N >= 16384));
}

size_t w4_ring_workspace_bytes(bool portable, int M, int N, int K) {
  if (M <= 0 || M > 64 || N % 16 != 0 || K % 128 != 0 || !w4_ring_preferred(portable, M, N, K)) return 0;
  const RingPlan p = w4_ring_plan(M, N, K);
  return p.KS == 1 ? 0 : (size_t)p.KS * M * N * sizeof(float);
}

static hipError_t launch_ring_reduce(bool xbf16, const float* part, int KS, int M, int N, const void* bias, int bdt,
                                     void* y, int64_t ldy, hipStream_t s) {
  const int64_t groups = (int64_t)M * (N / 4);
  const int vec = (reinterpret_cast<uintptr_t>(y) % 8) == 0 && (ldy % 4) == 0;
  const dim3 grid((unsigned)((groups + 255) / 256));
  if (xbf16) {
    hipLaunchKernelGGL(w4_ring_reduce_kernel<true>, grid, dim3(256), 0, s, part, KS, M, N, bias, bdt,
                       static_cast<uint16_t*>(y), ldy, vec);
  } else {
    hipLaunchKernelGGL(w4_ring_reduce_kernel<false>, grid, dim3(256), 0, s, part, KS, M, N, bias, bdt,
                       static_cast<uint16_t*>(y), ldy, vec);
  }
  return hipGetLastError();
}

template <int MB, int T, int BW, int S, bool XBF16, bool SBF16, bool PORT>
static hipError_t launch_ring_t(const RingArgs& a, hipStream_t s) {
  using Sh = RingShape<MB, T, BW>;
  const size_t shm = (size_t)S * Sh::STAGE + Sh::XS;
  auto kern = w4_ring_kernel<MB, T, BW, S, XBF16, SBF16, PORT>;
  note_kernel("w4_ring_kernel<%d,%d,%d,%d,%s,%s> KS=%d%s", MB, T, BW, S, XBF16 ? "bf16" : "f16",
              PORT ? "portable_row" : "cdna4", a.KS, a.KS > 1 ? " + w4_ring_reduce_kernel" : "");
  if (shm > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kern, dim3(a.ngrp * a.KS), dim3(BW * kWave), shm, s, a);
  return hipGetLastError();
}

template <bool XBF16, bool SBF16, bool PORT>
static hipError_t launch_ring_x(const RingPlan& p, const RingArgs& a, hipStream_t s) {
  if (p.mb == 1) return launch_ring_t<1, 1, 4, 4, XBF16, SBF16, PORT>(a, s);
  if (p.mb == 2) return p.BW == 8 ? launch_ring_t<2, 1, 8, 3, XBF16, SBF16, PORT>(a, s)
                                   : launch_ring_t<2, 1, 4, 3, XBF16, SBF16, PORT>(a, s);
  return p.BW == 8 ? launch_ring_t<4, 1, 8, 3, XBF16, SBF16, PORT>(a, s)
                   : launch_ring_t<4, 1, 4, 3, XBF16, SBF16, PORT>(a, s);
}

template <bool PORT>
static hipError_t launch_ring_p(bool xbf16, bool sbf, const RingPlan& p, const RingArgs& a, hipStream_t s) {
  if (xbf16) return sbf ? launch_ring_x<true, true, PORT>(p, a, s) : launch_ring_x<true, false, PORT>(p, a, s);
  return sbf ? launch_ring_x<false, true, PORT>(p, a, s) : launch_ring_x<false, false, PORT>(p, a, s);
}

hipError_t launch_w4_ring(bool portable, const void* x, int64_t ldx, bool xbf16, const int32_t* qw, int64_t ldq,
                          const void* scales,
                          int sdt, int64_t lds, const int32_t* zeros, int64_t ldz, const void* bias, int bdt, void* y,
                          int64_t ldy, int M, int N, int K, int gs, bool single_group, int G, void* ws, size_t ws_bytes,
                          hipStream_t s) {
  const RingPlan p = w4_ring_plan(M, N, K);
  RingArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.qw = qw;
  a.ldq = ldq;
  a.scales = static_cast<const uint16_t*>(scales);
  a.lds = lds;
  a.hasz = zeros != nullptr;
  a.zeros = zeros ? zeros : qw;  // symmetric: never read (zero-length resource below)
  a.ldz = zeros ? ldz : 0;
  a.bias = bias;
  a.bdt = bdt;
  a.y = static_cast<uint16_t*>(y);
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  a.gsteps = single_group ? 0 : gs / 128;
  a.KS = p.KS;
  a.ngrp = p.ngrp;
  a.qbytes = (uint32_t)((int64_t)(portable ? N : N / 16) * ldq * 4);
  a.xbytes = (uint32_t)((int64_t)M * ldx * 2);
  a.sbytes = (uint32_t)((int64_t)G * lds * 2);
  a.zbytes = zeros ? (uint32_t)((int64_t)G * ldz * 4) : 0u;
  a.part = static_cast<float*>(ws);
  if (p.KS > 1 && (ws == nullptr || ws_bytes < (size_t)p.KS * M * N * sizeof(float) ||
                   reinterpret_cast<uintptr_t>(ws) % 16 != 0))
    return hipErrorInvalidValue;
  const bool sbf = sdt == FG_BF16;
  const hipError_t e = portable ? launch_ring_p<true>(xbf16, sbf, p, a, s) : launch_ring_p<false>(xbf16, sbf, p, a, s);
  if (e != hipSuccess || p.KS == 1) return e;
  return launch_ring_reduce(xbf16, a.part, p.KS, M, N, bias, bdt, y, ldy, s);
}

// ------------------------------------------------------------------------------------------------ W8A16 ring
// int8 [N, ldq] weights (ldq bytes per row, a multiple of 16), scales [G, lds] 16-bit, no zero-points.
bool w8a16_ring_ok(const void* x, int64_t ldx, const int8_t* qw, int64_t ldq, const void* scales, int sdt,
                   int64_t lds, int64_t M, int64_t N, int64_t K, int gs, int64_t G) {
  const int64_t k2g = 1LL << 31;  // offsets past a span plus a step offset stay below 2^32
  return M > 0 && M <= 64 && sdt != FG_F32 && N % 16 == 0 && (K % 128) == 0 && ((gs % 128) == 0 || G == 1) &&
         (ldx % 8) == 0 && (reinterpret_cast<uintptr_t>(x) % 16) == 0 && (ldq % 16) == 0 && ldq >= K &&
         (reinterpret_cast<uintptr_t>(qw) % 16) == 0 && (lds % 2) == 0 &&
         (reinterpret_cast<uintptr_t>(scales) % 4) == 0 && N * ldq < k2g && M * ldx * 2 < k2g && G * lds * 2 < k2g &&
         group_div_exact(K, gs, G, 128);
}

size_t w8a16_ring_workspace_bytes(int M, int N, int K) {
  if (M <= 0 || M > 64 || N % 16 != 0 || K % 128 != 0) return 0;
  const RingPlan p = w4_ring_plan(M, N, K);
  return p.KS == 1 ? 0 : (size_t)p.KS * M * N * sizeof(float);
}

template <int MB, int T, int BW, int S, bool XBF16, bool SBF16>
static hipError_t launch_w8ring_t(const RingArgs& a, hipStream_t s) {
  using Sh = RingShape<MB, T, BW, true>;
  const size_t shm = (size_t)S * Sh::STAGE + Sh::XS;
  auto kern = w8a16_ring_kernel<MB, T, BW, S, XBF16, SBF16>;
  note_kernel("w8a16_ring_kernel<%d,%d,%d,%d,%s> KS=%d%s", MB, T, BW, S, XBF16 ? "bf16" : "f16", a.KS,
              a.KS > 1 ? " + w4_ring_reduce_kernel" : "");
  if (shm > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kern, dim3(a.ngrp * a.KS), dim3(BW * kWave), shm, s, a);
  return hipGetLastError();
}

template <bool XBF16, bool SBF16>
static hipError_t launch_w8ring_x(const RingPlan& p, const RingArgs& a, hipStream_t s) {
  if (p.mb == 1) return launch_w8ring_t<1, 1, 4, 4, XBF16, SBF16>(a, s);
  if (p.mb == 2) return p.BW == 8 ? launch_w8ring_t<2, 1, 8, 3, XBF16, SBF16>(a, s)
                                   : launch_w8ring_t<2, 1, 4, 3, XBF16, SBF16>(a, s);
  return p.BW == 8 ? launch_w8ring_t<4, 1, 8, 3, XBF16, SBF16>(a, s) : launch_w8ring_t<4, 1, 4, 3, XBF16, SBF16>(a, s);
}

hipError_t launch_w8a16_ring(const void* x, int64_t ldx, bool xbf16, const int8_t* qw, int64_t ldq,
                             const void* scales, int sdt, int64_t lds, const void* bias, int bdt, void* y, int64_t ldy,
                             int M, int N, int K, int gs, bool single_group, int G, void* ws, size_t ws_bytes,
                             hipStream_t s) {
  const RingPlan p = w4_ring_plan(M, N, K);
  RingArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.qw = reinterpret_cast<const int32_t*>(qw);
  a.ldq = ldq;
  a.scales = static_cast<const uint16_t*>(scales);
  a.lds = lds;
  a.hasz = 0;
  a.zeros = a.qw;  // never read (no zero-point loads in the W8 form)
  a.ldz = 0;
  a.bias = bias;
  a.bdt = bdt;
  a.y = static_cast<uint16_t*>(y);
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  a.gsteps = single_group ? 0 : gs / 128;
  a.KS = p.KS;
  a.ngrp = p.ngrp;
  a.qbytes = (uint32_t)((int64_t)N * ldq);
  a.xbytes = (uint32_t)((int64_t)M * ldx * 2);
  a.sbytes = (uint32_t)((int64_t)G * lds * 2);
  a.zbytes = 0;
  a.part = static_cast<float*>(ws);
  if (p.KS > 1 && (ws == nullptr || ws_bytes < (size_t)p.KS * M * N * sizeof(float) ||
                   reinterpret_cast<uintptr_t>(ws) % 16 != 0))
    return hipErrorInvalidValue;
  const bool sbf = sdt == FG_BF16;
  hipError_t e;
  if (xbf16) {
    e = sbf ? launch_w8ring_x<true, true>(p, a, s) : launch_w8ring_x<true, false>(p, a, s);
  } else {
    e = sbf ? launch_w8ring_x<false, true>(p, a, s) : launch_w8ring_x<false, false>(p, a, s);
  }
  if (e != hipSuccess || p.KS == 1) return e;
  return launch_ring_reduce(xbf16, a.part, p.KS, M, N, bias, bdt, y, ldy, s);
}

}  // namespace fg
