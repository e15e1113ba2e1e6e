// W4A16 / W8A16 prefill for large M x N: y[M,N] = x[M,K] @ dequant(W)[N,K]^T (+bias), two teams of wavefronts
// alternating between matrix and vector work (ping-pong).
//
// A workgroup of eight wavefronts owns a 256 x 256 output tile.  Wavefront w owns all 256 rows and channels 32 w .. + 32:
// 16 x 2 tiles of v_mfma_f32_16x16x32_{bf16,f16}, 128 fp32 accumulators per lane, kept in AGPRs.  Wavefronts 0..3 form
// team A, 4..7 team B; each SIMD holds one wavefront of each team.  K is walked in 64-column slices through a
// three-stage LDS ring; time is cut into half-periods separated by workgroup barriers, and in every half-period one team
// runs an M phase while the other runs a V phase:
//   * M phase (slice s): the slice's 64 MFMAs, A fragments read from the LDS x tile (32 per wavefront, four in
//     flight), B operands from registers -- no VALU, no global memory; at its end the wavefront reads the staging words
//     its next V phase converts (their LDS latency passes in the barrier);
//   * V phase (slice s): dequantise slice s's B operands (the wavefront's 32 channels x 64 columns) into registers from
//     those words -- lane (r, j) of channel tile b takes the 8 nibbles of packed word 2 j + k (k-step k, columns
//     16 j + 8 k .. + 7; the A fragments are read to match) and computes (q - z) * s in fp32, exactly the oracle's
//     value (q * s + (-z * s) is exact and the fma rounds nothing; W8A16: q * s), rounded once to bf16 / fp16 -- and
//     issue direct-to-LDS loads: its quarter of one team's half of the x tile of slice s + 2 (x rows 64 q .. + 32 for
//     team B's wavefront q, the next 32 for team A's) and the staging (packed weights, scales, zero words) of its
//     channels for a later slice.
// Team A runs M(s) in half-period 2 s and V(s + 1) in 2 s + 1; team B runs V(s) in 2 s and M(s) in 2 s + 1.  So the
// matrix core of every SIMD runs the M phases of the two teams back to back, while the vector work and load issue of
// one team hide under the other team's MFMAs (a wavefront's own VALU and MFMA instructions do not overlap; those of
// two wavefronts on one SIMD do).  A dequantised B operand serves 256 rows, which keeps the V phase near the M phase.
//
// Ring: x of slice s in stage s % 3, loaded in V(s - 2) (team B in half-period 2 s - 4, team A in 2 s - 3) into a
// stage both teams last read in half-period 2 s - 3 or earlier; both teams wait for their halves before the barrier
// that ends half-period 2 s - 1, which makes the tile visible to both.  A wavefront's staging of slice s (stage s % 3)
// is loaded and read by that wavefront alone, two V phases apart.  Every wavefront issues the same loads in the same
// order each V phase (slices past the end re-read the last one into areas no one reads again), so
// `s_waitcnt vmcnt(N)` with a constant N means exactly "these loads have landed" (loads complete in issue order; the
// loads are invisible to the compiler's wait analysis, so every wait is explicit; the ISA test checks the counts).
//
// LDS per stage: x 256 rows x 128 B (16-byte unit c of row r at c ^ key(r), key(r) = (r & 7) ^ ((r >> 3) & 1): for
// fragment reads of units 2 (lane / 16) + k this is free of bank conflicts on gfx950 (SQ_LDS_BANK_CONFLICT), where
// r & 7 alone costs 4 cycles per read, as in fg_mm_big.hip's FP8 reads) and eight
// staging areas (packed weights of 32 channels: 32 B (W8A16: 64 B) per channel, scales 256 B, zero words 256 B).  Three
// stages: 135168 bytes (W8A16 153600).
//
// Split-K (gridDim.y > 1): each split covers `kchunk` columns and writes fp32 partials [S, M, N] to the caller's
// workspace; w4_splitk_reduce_kernel (fg_w4_mfma.hip) sums them in a fixed order and adds the bias.
//
// Requirements (w4_pp_ok / w8_pp_ok): K % 64 == 0, group a multiple of 64 (or one group), N % 8 == 0, 16-bit scales with
// an even row stride, 16-byte aligned x (ldx % 8 == 0) and qweight (W4: ldq % 4 == 0, W8: ldq % 16 == 0), 4-byte
// aligned scales, no act-order perm, every operand under 2 GiB (32-bit buffer offsets).  Rows past M and channels past
// N read row M - 1 / channel N - 1 and are not stored.
#include <algorithm>

#include "fg_device.h"

namespace fg {

typedef __bf16 bf16x2_pp_t __attribute__((ext_vector_type(2)));
typedef float f32x4_pp_t __attribute__((ext_vector_type(4)));
typedef float f32x2_pp_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) uint8_t lds_u8_pp_t;

constexpr int kPpBM = 256, kPpBN = 256, kPpBK = 64, kPpRow = 128, kPpThreads = 512;
constexpr int kPpX = kPpBM * kPpRow;  // x rows of a stage
// a wavefront's staging area: packed weights of 32 channels (W4 32 B, W8 64 B per channel and slice), 32 scales (a
// 256-byte area), 4 zero words (a 256-byte area)
template <int WB>
struct PpStg {
  static constexpr int Q = 32 * (WB == 4 ? 32 : 64), S = Q, Z = Q + 256, BYTES = Q + (WB == 4 ? 512 : 256);
  static constexpr int QI = Q / 1024;                   // 1 KiB packed-weight loads per slice
  static constexpr int LOADS = QI + (WB == 4 ? 2 : 1);  // + scales (+ zero words)
  static constexpr int STAGE = kPpX + 8 * BYTES;
};
static_assert(3 * PpStg<4>::STAGE <= 160 * 1024 && 3 * PpStg<8>::STAGE <= 160 * 1024, "ring exceeds the LDS");
constexpr int kPpXI = 4;  // x loads per wavefront and slice (1 KiB each)
constexpr int kPpAhead = 4;  // A fragments in flight in an M phase (more slows the other team's LDS reads)

struct PpArgs {
  const uint16_t* x;
  int64_t ldx;
  const void* qw;
  int64_t ldq;  // W4: int32 words per row; W8: bytes per row
  const uint16_t* scales;
  int64_t lds;
  const int32_t* zeros;  // a valid buffer when symmetric, never used
  int64_t ldz;
  const void* bias;
  float* ws;
  uint16_t* y;
  int64_t ldy;
  int M, N, K;
  int kchunk;     // columns per K split (a multiple of 64)
  uint32_t gmul;  // group of a slice = umulhi(slice, gmul) | (slice & gsel): gmul = 2^32 / (slices per group)
  uint32_t gsel;  // rounded up for groups of several slices (else 0), gsel = all ones for one slice per group
  int hasz, sbf16, bdt;
  uint32_t xbytes, qbytes, sbytes, zbytes;  // buffer spans (each < 2^31)
};

// One MFMA as inline asm, the accumulator in AGPRs and updated in place (given 128 accumulators per lane as values the
// compiler copies them between AGPRs and VGPRs).  The compiler's hazard recognizer does not see inside the asm, so the
// code keeps every hazard out of reach by construction: the statements are volatile (they stay between the barriers of
// their M phase, in order), the B operands are pinned in VGPRs by pp_pin before the barrier that ends their V phase (no
// VALU write reaches into the M phase), the A operands come from LDS (the compiler waits for asm operands too), an
// accumulator's next MFMA comes 32 MFMAs later, and the epilogue reads the AGPRs after explicit wait states.
template <bool XBF16>
__device__ __forceinline__ void pp_mfma(f32x4_pp_t& c, uint4 a, uint4 b) {
  if constexpr (XBF16) {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0"
        : "+a"(c)
        : "v"(__builtin_bit_cast(u32x4_t, a)), "v"(__builtin_bit_cast(u32x4_t, b)));
  } else {
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0"
        : "+a"(c)
        : "v"(__builtin_bit_cast(u32x4_t, a)), "v"(__builtin_bit_cast(u32x4_t, b)));
  }
}

// Values computed before this point stay computed before it (a volatile asm that reads and rewrites them).
__device__ __forceinline__ void pp_pin(uint4& v) {
  u32x4_t t = __builtin_bit_cast(u32x4_t, v);
  asm volatile("" : "+v"(t));
  v = __builtin_bit_cast(uint4, t);
}
__device__ __forceinline__ void pp_pin_acc(f32x4_pp_t& c) { asm volatile("" : "+a"(c)); }

// Buffer resource of `bytes` bytes at p (stride 0, raw buffer, out-of-range loads return zero).
__device__ __forceinline__ u32x4_t pp_rsrc(const void* p, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  return u32x4_t{(uint32_t)a, (uint32_t)(a >> 32) & 0xffffu, bytes, 0x00020000u};
}

// One direct-to-LDS buffer load: lane l's B bytes at voff + soff land at LDS address lds + B l.  Written as asm so the
// compiler's wait analysis does not see an LDS write: it would otherwise wait for every such load in flight before any
// LDS read (vmcnt(0)), which defeats the ring; the kernel's explicit vmcnt waits order them instead.  M0 carries the
// LDS address (one wait state before the load reads it); nothing else in the kernel uses M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
template <int B>
__device__ __forceinline__ void pp_dma(const u32x4_t& rsrc, uint32_t lds, uint32_t voff, uint32_t soff) {
  if constexpr (B == 16) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(lds), "v"(voff),
                 "s"(rsrc), "s"(soff)
                 : "memory", "m0");
  } else {
    static_assert(B == 4, "16- or 4-byte lanes");
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, %3 offen lds" ::"s"(lds), "v"(voff),
                 "s"(rsrc), "s"(soff)
                 : "memory", "m0");
  }
}
#pragma clang diagnostic pop

template <bool XBF16>
__device__ __forceinline__ uint32_t pp_pack(float lo, float hi) {
  if constexpr (XBF16) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_pp_t{lo, hi}, bf16x2_pp_t));
  } else {
    return (uint32_t)f32_to_f16_bits(lo) | ((uint32_t)f32_to_f16_bits(hi) << 16);
  }
}

// 8 columns of one packed int4 word (nibble t = column t) as an MFMA B operand: (q - z) * s rounded to 16 bits
template <bool XBF16>
__device__ __forceinline__ uint4 pp_dequant4(uint32_t w, uint32_t nmask, float s, float c) {
  const uint32_t lo = w & nmask, hi = (w >> 4) & nmask;  // nibbles 0,2,4,6 / 1,3,5,7 in bytes 0..3
  float d[8];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    d[2 * b] = __builtin_fmaf((float)((lo >> (8 * b)) & 0xFFu), s, c);
    d[2 * b + 1] = __builtin_fmaf((float)((hi >> (8 * b)) & 0xFFu), s, c);
  }
  return make_uint4(pp_pack<XBF16>(d[0], d[1]), pp_pack<XBF16>(d[2], d[3]), pp_pack<XBF16>(d[4], d[5]),
                    pp_pack<XBF16>(d[6], d[7]));
}

// 8 columns of int8 weights (two words, byte t = column t) as an MFMA B operand: q * s rounded to 16 bits
template <bool XBF16>
__device__ __forceinline__ uint4 pp_dequant8(uint32_t w0, uint32_t w1, float s) {
  float d[8];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    d[b] = (float)(int8_t)(w0 >> (8 * b)) * s;
    d[4 + b] = (float)(int8_t)(w1 >> (8 * b)) * s;
  }
  return make_uint4(pp_pack<XBF16>(d[0], d[1]), pp_pack<XBF16>(d[2], d[3]), pp_pack<XBF16>(d[4], d[5]),
                    pp_pack<XBF16>(d[6], d[7]));
}

template <bool XBF16, int WB>
__global__ void __launch_bounds__(kPpThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) w4_pp_kernel(const PpArgs a) {
  using St = PpStg<WB>;
  extern __shared__ __align__(16) uint8_t smem[];
  const int ntm = (a.M + kPpBM - 1) / kPpBM, ntn = (a.N + kPpBN - 1) / kPpBN;
  int tm, tn;
  tile_of(blockIdx.x, ntm, ntn, tm, tn);
  const int m0 = tm * kPpBM, n0 = tn * kPpBN;
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // w: wave-uniform
  const int team = w >> 2, wq = w & 3;  // team 0 = A, 1 = B
  const int r16 = lane & 15, j4 = lane >> 4;
  const int kbeg = blockIdx.y * a.kchunk;
  const int nk = (min(a.K, kbeg + a.kchunk) - kbeg) / kPpBK;
  const int c0 = n0 + 32 * w;  // first channel of the wavefront

  // ---- direct-to-LDS sources: raw buffer loads with 32-bit per-lane offsets (the slice's column offset and group row
  // go in the scalar offset)
  const u32x4_t rx = pp_rsrc(a.x, a.xbytes), rq = pp_rsrc(a.qw, a.qbytes);
  const u32x4_t rs = pp_rsrc(a.scales, a.sbytes), rz = pp_rsrc(a.zeros, a.zbytes);
  // x: load i of wavefront w fills tile rows 8 xg + 8 i .. + 8 with xg = 8 wq + 4 (1 - team) (team B the first half of
  // rows 64 wq .. + 64, team A the second); lane l writes position l % 8 of row r = 8 (xg + i) + l / 8, i.e. global
  // unit (l % 8) ^ key(r) with key(r) = (l / 8) ^ ((xg + i) & 1)
  const int xg = 8 * wq + 4 * (1 - team);
  uint32_t xv[kPpXI];
  {
    const int lrow = lane >> 3;
#pragma unroll
    for (int i = 0; i < kPpXI; ++i) {
      const int lunit = (lane & 7) ^ (lane >> 3) ^ ((xg + i) & 1);
      xv[i] = (uint32_t)min(m0 + (xg + i) * 8 + lrow, a.M - 1) * (uint32_t)a.ldx * 2u + 16u * (uint32_t)lunit;
    }
  }
  // packed weights: load h fills 1 KiB of the wavefront's staging: W4 channels l / 2 (16-byte half l % 2 of a 32-byte
  // slice row), W8 channels 16 h + l / 4 (quarter l % 4 of a 64-byte row)
  constexpr int CPL = WB == 4 ? 2 : 4;  // lanes per channel row
  uint32_t qv[St::QI];
#pragma unroll
  for (int h = 0; h < St::QI; ++h) {
    const int ch = min(c0 + (32 / St::QI) * h + lane / CPL, a.N - 1);
    qv[h] = WB == 4 ? (uint32_t)ch * (uint32_t)a.ldq * 4u + 16u * (uint32_t)(lane % CPL)
                    : (uint32_t)ch * (uint32_t)a.ldq + 16u * (uint32_t)(lane % CPL);
  }
  // scales: lane l < 16 the pair 2 l, 2 l + 1 (the rest repeat lane 0's); zero words: lane l < 4 word l
  const uint32_t sv = (uint32_t)min(c0 + 2 * (lane < 16 ? lane : 0), a.N - 2) * 2u;
  const uint32_t zv = (uint32_t)min(c0 / 8 + (lane < 4 ? lane : 0), (a.N - 1) / 8) * 4u;
  const int slice0 = kbeg / kPpBK;
  // LDS addresses (wave-uniform) of a stage and of this wavefront's staging area in it
  const uint32_t lds0 = (uint32_t)(size_t)(lds_u8_pp_t*)smem;
  auto stage_addr = [&](int s) { return lds0 + (uint32_t)((s % 3) * St::STAGE); };
  auto stage = [&](int s) { return smem + (s % 3) * St::STAGE; };
  auto stg = [&](int s) { return stage(s) + kPpX + w * St::BYTES; };
  // the staging loads of slice s for this wavefront's channels
  auto issue_stg = [&](int s) __attribute__((always_inline)) {
    const int sc = min(s, nk - 1);
    const int k0 = kbeg + sc * kPpBK;
    const uint32_t sl = (uint32_t)(slice0 + sc);
    const uint32_t g = __umulhi(sl, a.gmul) | (sl & a.gsel);
    const uint32_t d = stage_addr(s) + (uint32_t)(kPpX + w * St::BYTES);
#pragma unroll
    for (int h = 0; h < St::QI; ++h) pp_dma<16>(rq, d + h * 1024, qv[h], WB == 4 ? k0 / 2 : k0);
    pp_dma<4>(rs, d + St::S, sv, g * (uint32_t)a.lds * 2u);
    if constexpr (WB == 4) pp_dma<4>(rz, d + St::Z, zv, g * (uint32_t)a.ldz * 4u);
  };
  // this wavefront's x rows of slice s
  auto issue_x = [&](int s) __attribute__((always_inline)) {
    const int k0 = kbeg + min(s, nk - 1) * kPpBK;
    const uint32_t d = stage_addr(s) + (uint32_t)(xg * 1024);
#pragma unroll
    for (int i = 0; i < kPpXI; ++i) pp_dma<16>(rx, d + i * 1024, xv[i], k0 * 2);
  };

  uint32_t nmask = 0x0F0F0F0Fu;
  asm("" : "+v"(nmask));  // hidden from known-bits analysis: bytes of masked words convert with v_cvt_f32_ubyte{k}
  const uint32_t zsel = a.hasz ? 0xffffffffu : 0u;
  uint4 fb[2][2];  // B operands: k-step, channel tile
  // The staging words of slice s that this lane converts: scale, zero word and packed weights of its two channels.
  // They are read at the end of the M phase before the V phase that converts them, so the LDS latency passes in the
  // barrier between.
  struct Words {
    uint32_t sraw[2], zw[2];
    uint4 q[2];
  };
  auto read_words = [&](int s) __attribute__((always_inline)) {
    const uint8_t* d = stg(s);
    Words wd;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int c = 16 * b + r16;
      wd.sraw[b] = *reinterpret_cast<const uint16_t*>(d + St::S + 2 * c);
      if constexpr (WB == 4) {
        const uint2 q2 = *reinterpret_cast<const uint2*>(d + c * 32 + 8 * j4);
        wd.q[b] = make_uint4(q2.x, q2.y, 0u, 0u);
        wd.zw[b] = *reinterpret_cast<const uint32_t*>(d + St::Z + (c >> 3) * 4);
      } else {  // 16 bytes: columns 16 j + 0 .. 7 (k-step 0) and 16 j + 8 .. 15 (k-step 1)
        wd.q[b] = *reinterpret_cast<const uint4*>(d + c * 64 + 16 * j4);
        wd.zw[b] = 0u;
      }
    }
    return wd;
  };
  // V phase: this wavefront's B operands from the staging words, and `loads` (the phase's direct-to-LDS issue)
  auto convert = [&](const Words& wd, auto&& loads) __attribute__((always_inline)) {
    loads();
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int c = 16 * b + r16;
      const float sc = a.sbf16 ? bf16_bits_to_f32(wd.sraw[b]) : f16_bits_to_f32((uint16_t)wd.sraw[b]);
      if constexpr (WB == 4) {
        const uint32_t z = (wd.zw[b] & zsel) | (0x88888888u & ~zsel);  // symmetric: zero-point 8
        const float cz = -(float)nibble(z, c & 7) * sc;
        fb[0][b] = pp_dequant4<XBF16>(wd.q[b].x, nmask, sc, cz);
        fb[1][b] = pp_dequant4<XBF16>(wd.q[b].y, nmask, sc, cz);
      } else {
        fb[0][b] = pp_dequant8<XBF16>(wd.q[b].x, wd.q[b].y, sc);
        fb[1][b] = pp_dequant8<XBF16>(wd.q[b].z, wd.q[b].w, sc);
      }
      pp_pin(fb[0][b]);  // the VALU work stays in this V phase
      pp_pin(fb[1][b]);
    }
  };

  f32x4_pp_t acc[16][2];
#pragma unroll
  for (int i = 0; i < 16; ++i)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[i][b] = f32x4_pp_t{0.f, 0.f, 0.f, 0.f};
  // M phase of slice s: 32 A fragments (rows 16 i + r16, columns 16 j4 + 8 k .. + 7 = unit 2 j4 + k), each for two
  // MFMAs, read kPpAhead ahead
  auto mphase = [&](int s) __attribute__((always_inline)) {
    const uint8_t* arow = stage(s) + r16 * kPpRow;
    const int rkey = (r16 & 7) ^ (r16 >> 3);  // key of rows 16 i + r16
    auto read_a = [&](int g) __attribute__((always_inline)) {
      const int k = g >> 4, i = g & 15;
      return *reinterpret_cast<const uint4*>(arow + i * 16 * kPpRow + (((2 * j4 + k) ^ rkey) * 16));
    };
    uint4 f[kPpAhead];
#pragma unroll
    for (int g = 0; g < kPpAhead; ++g) f[g] = read_a(g);
#pragma unroll
    for (int g = 0; g < 32; ++g) {
      const uint4 cur = f[g % kPpAhead];
      if (g + kPpAhead < 32) f[g % kPpAhead] = read_a(g + kPpAhead);
      const int k = g >> 4, i = g & 15;
#pragma unroll
      for (int b = 0; b < 2; ++b) pp_mfma<XBF16>(acc[i][b], cur, fb[k][b]);
    }
  };
  // Every V phase of a wavefront issues its x rows of one slice, then its staging of a later one: team A x(s + 2) and
  // stg(s + 3) in V(s + 1), team B x(s + 2) and stg(s + 2) in V(s).  Waits: a staging group before its words are read
  // (an x group and a staging group were issued after it; for team B this also covers the x group of the next slice),
  // and for team A the x group of slice s + 1 before the barrier that ends half-period 2 s + 1 (a staging group, an x
  // group and a staging group after it).  The barriers need no LDS wait: every LDS read before one is either consumed
  // (A fragments, staging words of the phase) or reads an area no one writes for several half-periods (the words read
  // ahead).
  constexpr int kStgWait = kPpXI + St::LOADS;
  constexpr int kXWait = kPpXI + 2 * St::LOADS;

  if (team == 0) {
    // prologue: the issue order of the V phases before V(0), then V(0)
    issue_stg(0);
    issue_x(0);
    issue_stg(1);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kStgWait) : "memory");
    convert(read_words(0), [&] {
      issue_x(1);
      issue_stg(2);
    });
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(kXWait) : "memory");  // x of slice 0 landed
    for (int s = 0; s < nk; ++s) {
      mphase(s);
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kStgWait) : "memory");  // staging of slice s + 1 landed
      const Words wd = read_words(s + 1);
      asm volatile("s_barrier" ::: "memory");  // end of half-period 2 s
      convert(wd, [&] {  // V(s + 1)
        issue_x(s + 2);
        issue_stg(s + 3);
      });
      // the x rows of slice s + 1 landed (both teams read them from the next half-period on)
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(kXWait) : "memory");  // end of 2 s + 1
    }
  } else {
    issue_x(0);
    issue_stg(0);
    issue_x(1);
    issue_stg(1);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kStgWait) : "memory");  // x and staging of slice 0 landed
    Words wd = read_words(0);
    asm volatile("s_barrier" ::: "memory");
    for (int s = 0; s < nk; ++s) {
      convert(wd, [&] {  // V(s)
        issue_x(s + 2);
        issue_stg(s + 2);
      });
      asm volatile("s_barrier" ::: "memory");  // end of half-period 2 s
      mphase(s);
      // x and staging of slice s + 1 landed (team A reads the x rows next half-period)
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kStgWait) : "memory");
      wd = read_words(s + 1);
      asm volatile("s_barrier" ::: "memory");  // end of 2 s + 1
    }
  }
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");  // drain: the epilogue reuses the ring
  // the last MFMAs' results are in the AGPRs before the epilogue reads them (more wait states than an MFMA of 8
  // passes needs ahead of a dependent read; the compiler does not see inside the asm)
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
  for (int i = 0; i < 16; ++i)
#pragma unroll
    for (int b = 0; b < 2; ++b) pp_pin_acc(acc[i][b]);  // AGPR reads come after the wait states

  if (gridDim.y > 1) {  // fp32 partials of this split
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = m0 + i * 16 + 4 * j4 + e, n = c0 + b * 16 + r16;
          if (m < a.M && n < a.N) a.ws[((int64_t)blockIdx.y * a.M + m) * a.N + n] = acc[i][b][e];
        }
    return;
  }
  // 16-bit output through a per-wavefront LDS slab of 16 rows x 32 channels, stored as 16-byte row segments
  constexpr int SP = 32 + 8;
  uint16_t* slab = reinterpret_cast<uint16_t*>(smem) + w * 16 * SP;
  float cb[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) cb[b] = a.bias ? load_f(a.bias, a.bdt, min(c0 + b * 16 + r16, a.N - 1)) : 0.f;
  const bool vec_ok = (a.ldy % 8) == 0 && (reinterpret_cast<uintptr_t>(a.y) % 16) == 0;
  const int r = lane >> 2, c8 = lane & 3;  // the row segment this lane stores
#pragma unroll
  for (int i = 0; i < 16; ++i) {
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float v = a.bias ? acc[i][b][e] + cb[b] : acc[i][b][e];
        slab[(4 * j4 + e) * SP + b * 16 + r16] = XBF16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
      }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's slab writes are done before it reads them
    const int m = m0 + i * 16 + r, n = c0 + c8 * 8;
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
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads done before the next slab overwrites the buffer
  }
}

template <int WB>
static bool pp_ok(const void* x, int64_t ldx, const void* qw, int64_t ldq, const void* scales, int sdt, int64_t lds,
                  const int32_t* zeros, int64_t ldz, int64_t M, int64_t N, int64_t K, int gs, int64_t G) {
  const int64_t lim = int64_t(1) << 31;  // buffer spans (offsets are 32-bit)
  const int64_t qbytes = WB == 4 ? N * ldq * 4 : N * ldq;
  return (K % kPpBK) == 0 && ((gs % kPpBK) == 0 || G == 1) && (N % 8) == 0 && N >= 8 && sdt != FG_F32 &&
         (lds % 2) == 0 && (reinterpret_cast<uintptr_t>(scales) % 4) == 0 && (ldx % 8) == 0 &&
         (reinterpret_cast<uintptr_t>(x) % 16) == 0 && (WB == 4 ? (ldq % 4) == 0 : (ldq % 16) == 0) &&
         (reinterpret_cast<uintptr_t>(qw) % 16) == 0 && M * ldx * 2 < lim && qbytes < lim && G * lds * 2 < lim &&
         (!zeros || G * ldz * 4 < lim) && group_div_exact(K, gs, G, kPpBK);
}

bool w4_pp_ok(const void* x, int64_t ldx, const int32_t* qw, int64_t ldq, const int32_t* perm, const void* scales,
              int sdt, int64_t lds, const int32_t* zeros, int64_t ldz, int64_t M, int64_t N, int64_t K, int gs,
              int64_t G) {
  return perm == nullptr && pp_ok<4>(x, ldx, qw, ldq, scales, sdt, lds, zeros, ldz, M, N, K, gs, G);
}

bool w8_pp_ok(const void* x, int64_t ldx, const int8_t* qw, int64_t ldq, const void* scales, int sdt, int64_t lds,
              int64_t M, int64_t N, int64_t K, int gs, int64_t G) {
  return pp_ok<8>(x, ldx, qw, ldq, scales, sdt, lds, nullptr, 0, M, N, K, gs, G);
}

// K splits: one when the tiles cover the CUs, else as many as keep the workgroups within one round over the CUs, each
// at least 512 columns.
void w4_pp_plan(int M, int N, int K, int split_k, int* splits, int* kchunk) {
  const int cus = device_cus();
  const int64_t tiles = (int64_t)((M + kPpBM - 1) / kPpBM) * ((N + kPpBN - 1) / kPpBN);
  int s = split_k;
  if (s <= 0) {
    s = tiles >= cus ? 1 : (int)(cus / tiles);
    const int max_s = K / 512 > 0 ? K / 512 : 1;
    s = std::min(std::min(s, max_s), 16);
  }
  int kc = (K + s - 1) / s;
  kc = (kc + kPpBK - 1) / kPpBK * kPpBK;
  *kchunk = kc;
  *splits = (K + kc - 1) / kc;
}

size_t w4_pp_workspace_bytes(int M, int N, int K, int split_k) {
  int s, kc;
  w4_pp_plan(M, N, K, split_k, &s, &kc);
  return s > 1 ? (size_t)s * (size_t)M * (size_t)N * sizeof(float) : 0;
}

template <bool XBF16>
hipError_t launch_w4_splitk_reduce(const float* ws, int S, int M, int N, const void* bias, int bdt, void* y,
                                   int64_t ldy, hipStream_t s);

template <int WB>
static hipError_t launch_pp(const void* x, int64_t ldx, bool xbf16, const void* qw, int64_t ldq, const void* scales,
                            int sdt, int64_t lds, const int32_t* zeros, int64_t ldz, const void* bias, int bdt,
                            void* y, int64_t ldy, float* ws, int M, int N, int K, int gs, bool single_group,
                            int split_k, hipStream_t s) {
  int splits, kchunk;
  w4_pp_plan(M, N, K, split_k, &splits, &kchunk);
  if (splits > 1 && ws == nullptr) return hipErrorInvalidValue;
  PpArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.qw = qw;
  a.ldq = ldq;
  a.scales = static_cast<const uint16_t*>(scales);
  a.lds = lds;
  a.hasz = zeros != nullptr;
  a.zeros = zeros ? zeros : static_cast<const int32_t*>(scales);  // symmetric: a valid buffer, never read
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
  const uint32_t gdiv = single_group ? 0u : (uint32_t)(gs / kPpBK);  // slices per group
  a.gmul = gdiv > 1 ? 0xffffffffu / gdiv + 1u : 0u;
  a.gsel = gdiv == 1 ? 0xffffffffu : 0u;
  a.sbf16 = sdt == FG_BF16;
  const int64_t G = single_group ? 1 : (K + gs - 1) / gs;
  a.xbytes = (uint32_t)((int64_t)M * ldx * 2);
  a.qbytes = (uint32_t)(WB == 4 ? (int64_t)N * ldq * 4 : (int64_t)N * ldq);
  a.sbytes = (uint32_t)(G * lds * 2);
  a.zbytes = zeros ? (uint32_t)(G * ldz * 4) : a.sbytes;
  auto kern = xbf16 ? w4_pp_kernel<true, WB> : w4_pp_kernel<false, WB>;
  constexpr int lds_bytes = 3 * PpStg<WB>::STAGE;
  hipError_t e =
      hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes);
  if (e != hipSuccess) return e;
  const int tiles = ((M + kPpBM - 1) / kPpBM) * ((N + kPpBN - 1) / kPpBN);
  note_kernel("w4_pp_kernel<%s,w%d> 256x256 splits=%d%s", xbf16 ? "bf16" : "f16", WB, splits,
              splits > 1 ? " + w4_splitk_reduce_kernel" : "");
  hipLaunchKernelGGL(kern, dim3(tiles, splits), dim3(kPpThreads), lds_bytes, s, a);
  e = hipGetLastError();
  if (e != hipSuccess || splits == 1) return e;
  return xbf16 ? launch_w4_splitk_reduce<true>(ws, splits, M, N, bias, bdt, y, ldy, s)
               : launch_w4_splitk_reduce<false>(ws, splits, M, N, bias, bdt, y, ldy, s);
}

hipError_t launch_w4_pp(const void* x, int64_t ldx, bool xbf16, const int32_t* qw, int64_t ldq, const void* scales,
                        int sdt, int64_t lds, const int32_t* zeros, int64_t ldz, const void* bias, int bdt, void* y,
                        int64_t ldy, float* ws, int M, int N, int K, int gs, bool single_group, int split_k,
                        hipStream_t s) {
  return launch_pp<4>(x, ldx, xbf16, qw, ldq, scales, sdt, lds, zeros, ldz, bias, bdt, y, ldy, ws, M, N, K, gs,
                      single_group, split_k, s);
}

hipError_t launch_w8_pp(const void* x, int64_t ldx, bool xbf16, const int8_t* qw, int64_t ldq, const void* scales,
                        int sdt, int64_t lds, const void* bias, int bdt, void* y, int64_t ldy, float* ws, int M, int N,
                        int K, int gs, bool single_group, int split_k, hipStream_t s) {
  return launch_pp<8>(x, ldx, xbf16, qw, ldq, scales, sdt, lds, nullptr, 0, bias, bdt, y, ldy, ws, M, N, K, gs,
                      single_group, split_k, s);
}

}  // namespace fg
