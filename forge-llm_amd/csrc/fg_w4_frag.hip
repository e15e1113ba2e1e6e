// W4A16 for up to 64 rows of x (decode batches) on the CDNA4 MFMA-fragment weight layout (w4.cdna4_mfma_k128n16):
// y[M,N] = x[M,K] @ dequant(W)[N,K]^T (+bias) with v_mfma_f32_16x16x32_{bf16,f16}.
//
// The layout stores each 16-channel x 128-column tile as 1 KiB in the order the MFMA B operand wants it: lane
// l = 16 j + r of a wavefront loads 16 bytes (words 4 l .. 4 l + 3 of the tile); word s holds channel r, columns
// 32 s + 8 j + t (t = 0..7) with t in nibble slot t / 2 (even) or 4 + t / 2 (odd).  So one 16-byte load per lane and
// tile brings the B values of all four k-steps of a 128-column step, and (word >> 4 p) & 0x000F000F | magic is, in one
// v_and_or_b32 (plus a shift for p > 0), the exact 16-bit pair B + (q_2p, q_2p+1): bf16 0x43 -> 128 + q, fp16 0x64 ->
// 1024 + q.  x is read in MFMA A order as it lies in memory (lane l: row r, columns 32 s + 8 j .. + 7: one 16-byte
// load per m-tile and k-step), so neither operand is shuffled.
//
// Zero-points and scales (group size a multiple of 128, or one group per row; scales and zero words stored as in
// portable_row): sum_k x (q - z) = sum_k x (B + q) - (B + z) sum_k x, the row sums of x from one MFMA per m-tile and
// k-step against all-ones, and per 128-column step
//   acc += s[n, g] * (acc_step - (B + z[n, g]) * xsum)     (fp32, per accumulator element).
// A wavefront owns T tiles (16 T channels) and one K slice; the B operands of a step are unpacked once and used by all
// MB m-tiles, the A operands of an m-tile by all T tiles.  The KS wavefronts of a workgroup take the KS slices of the
// same channels and sum their partials in slice order through LDS (one launch, no workspace, deterministic).
//
// Requirements (w4_frag_ok): M <= 64, K % 128 == 0, group size % 128 == 0 or one group, 16-bit scales, 16-byte
// aligned x with ldx % 8 == 0, 16-byte aligned qweight with ldq % 4 == 0, operands spanning < 4 GiB.
#include "fg_device.h"

namespace fg {

typedef __bf16 bf16x8_fr_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_fr_t __attribute__((ext_vector_type(8)));
typedef float f32x4_fr_t __attribute__((ext_vector_type(4)));

template <bool XBF16>
__device__ __forceinline__ f32x4_fr_t fr_mfma(uint4 a, uint4 b, f32x4_fr_t c) {
  if constexpr (XBF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_fr_t, a),
                                                   __builtin_bit_cast(bf16x8_fr_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_fr_t, a),
                                                  __builtin_bit_cast(f16x8_fr_t, b), c, 0, 0, 0);
  }
}

// (a & mask) | magic: one v_and_or_b32 once the caller has hidden the constants from the compiler (mask in a scalar
// register, magic in a vector register; with literals it emits a v_and + v_or pair).  Plain C rather than inline asm:
// the result feeds MFMA B operands, and the hazard recognizer inserts the wait states a VALU write needs before an
// MFMA reads it only for instructions it can see (an asm v_and_or_b32 one instruction ahead of its MFMA produced
// wrong products).
__device__ __forceinline__ uint32_t fr_and_or(uint32_t a, uint32_t mask, uint32_t magic) { return (a & mask) | magic; }

// one k-step's word -> the lane's eight B values (columns 8 j .. 8 j + 7 of the k-step) as four exact 16-bit pairs
__device__ __forceinline__ uint4 fr_unpack(uint32_t w, uint32_t mask, uint32_t magic) {
  return make_uint4(fr_and_or(w, mask, magic), fr_and_or(w >> 4, mask, magic), fr_and_or(w >> 8, mask, magic),
                    fr_and_or(w >> 12, mask, magic));
}

constexpr int w4_frag_max_threads(int mb, int t) { return mb * t >= 4 ? 256 : 512; }

// Byte spans of the operands (each < 2^32, checked on the host) for the buffer resources: loads past a span read 0.
struct FragSpans {
  uint32_t q, x, s, z;
};

template <int MB, int T, int D, bool XBF16, bool SBF16>
__global__ void __launch_bounds__(w4_frag_max_threads(MB, T)) w4_frag_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const int32_t* __restrict__ qw, int64_t ldq,
    const uint16_t* __restrict__ scales, int64_t lds, const int32_t* __restrict__ zeros, int64_t ldz, int hasz,
    const void* __restrict__ bias, int bdt, uint16_t* __restrict__ y, int64_t ldy, int M, int N, int K, int gsteps,
    int KS, FragSpans sp) {
  constexpr float kB = XBF16 ? 128.f : 1024.f;
  constexpr uint32_t kOnes = XBF16 ? 0x3F803F80u : 0x3C003C00u;
  constexpr int NV = T * MB * 4;  // accumulator values per lane
  extern __shared__ __align__(16) float red[];  // [waves][NV][64]
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave);  // K slice and block: uniform
  const int ks = wave % KS, nb = blockIdx.x * ((int)(blockDim.x / kWave) / KS) + wave / KS;
  const int n0 = nb * 16 * T;
  const int nsteps = K / 128;
  const int st0 = (int)((int64_t)ks * nsteps / KS), st1 = (int)((int64_t)(ks + 1) * nsteps / KS);
  const int r16 = lane & 15, j = lane >> 4;
  const int NT = (N + 15) / 16;

  const __amdgpu_buffer_rsrc_t rq = buf_rsrc(qw, sp.q);
  const __amdgpu_buffer_rsrc_t rx = buf_rsrc(x, sp.x);
  const __amdgpu_buffer_rsrc_t rs = buf_rsrc(scales, sp.s);
  const __amdgpu_buffer_rsrc_t rz = buf_rsrc(zeros, sp.z);
  const __amdgpu_buffer_rsrc_t rq0 = buf_rsrc(qw, 0u), rx0 = buf_rsrc(x, 0u);  // zero length: every load reads 0
  const __amdgpu_buffer_rsrc_t rs0 = buf_rsrc(scales, 0u), rz0 = buf_rsrc(zeros, 0u);
  // per tile: the lane's 16 bytes of tile-row nt at step 0, and its channel (tiles past the last re-read the last)
  uint32_t woff[T], soff[T], zoff[T];
  int ncol[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int nt = min(nb * T + t, NT - 1);
    woff[t] = (uint32_t)nt * (uint32_t)ldq * 4u + 16u * (uint32_t)lane;
    ncol[t] = min(16 * nt + r16, N - 1);
    soff[t] = (uint32_t)ncol[t] * 2u;
    zoff[t] = (uint32_t)(ncol[t] >> 3) * 4u;
  }
  uint32_t xoff[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i)  // rows past M start at the end of x: their loads read 0 and fetch nothing
    xoff[i] = 16 * i + r16 < M ? (uint32_t)(16 * i + r16) * (uint32_t)ldx * 2u + 16u * (uint32_t)j : sp.x;
  const FastDiv gdiv((uint32_t)max(gsteps, 1));
  const uint32_t lds2 = (uint32_t)lds * 2u, ldz4 = (uint32_t)ldz * 4u;

  // D-step register ring: the loads of the next D steps are in flight while a step is computed
  struct Buf {
    uint4 w[T], x[MB][4];
    uint32_t s[T], z[T];
  };
  Buf buf[D];
  // A step past the slice is fetched through zero-length buffer resources: the same load instructions (so the waits
  // before each compute count exactly the older loads) that read zeros and move no memory.  The step and group parts
  // of each offset are wavefront-uniform (scalar soffset), the lane parts fixed (voffset), so a fetch costs no VALU.
  auto fetch = [&](int st, Buf& b) __attribute__((always_inline)) {
    const bool live = st < st1;
    const uint32_t g = gsteps > 0 ? gdiv.div((uint32_t)st) : 0u;
    const __amdgpu_buffer_rsrc_t x_ = live ? rx : rx0, q_ = live ? rq : rq0;
    const __amdgpu_buffer_rsrc_t s_ = live ? rs : rs0, z_ = live ? rz : rz0;
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int s = 0; s < 4; ++s) b.x[i][s] = buf_ld16(x_, xoff[i] + 64u * (uint32_t)s, (uint32_t)st * 256u);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      b.s[t] = __builtin_amdgcn_raw_buffer_load_b16(s_, (int)soff[t], (int)(g * lds2), 0);
      b.z[t] = __builtin_amdgcn_raw_buffer_load_b32(z_, (int)zoff[t], (int)(g * ldz4), 0);
    }
#pragma unroll
    for (int t = 0; t < T; ++t) b.w[t] = buf_ld16_nt(q_, woff[t], (uint32_t)st * 1024u);
  };

  f32x4_fr_t acc[T][MB];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[t][i] = f32x4_fr_t{0.f, 0.f, 0.f, 0.f};

  const uint4 ones = make_uint4(kOnes, kOnes, kOnes, kOnes);
  uint32_t mask = 0x000F000Fu, magic = XBF16 ? 0x43004300u : 0x64006400u;
  asm("" : "+s"(mask));  // opaque to constant folding: v_and_or_b32 with a scalar mask and a vector magic
  asm("" : "+v"(magic));
  auto compute = [&](const Buf& b) __attribute__((always_inline)) {
    uint4 bw[T][4];
    float sc[T], zb[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      bw[t][0] = fr_unpack(b.w[t].x, mask, magic);
      bw[t][1] = fr_unpack(b.w[t].y, mask, magic);
      bw[t][2] = fr_unpack(b.w[t].z, mask, magic);
      bw[t][3] = fr_unpack(b.w[t].w, mask, magic);
      sc[t] = SBF16 ? bf16_bits_to_f32(b.s[t]) : f16_bits_to_f32((uint16_t)b.s[t]);
      zb[t] = kB + (hasz ? (float)nibble(b.z[t], ncol[t] & 7) : 8.f);
    }
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      f32x4_fr_t xs = f32x4_fr_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) xs = fr_mfma<XBF16>(b.x[i][s], ones, xs);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        f32x4_fr_t as = f32x4_fr_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) as = fr_mfma<XBF16>(b.x[i][s], bw[t][s], as);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          acc[t][i][e] = __builtin_fmaf(sc[t], __builtin_fmaf(-zb[t], xs[e], as[e]), acc[t][i][e]);
      }
    }
  };

  if (st0 < st1) {
#pragma unroll
    for (int d = 0; d < D; ++d) fetch(st0 + d, buf[d]);
    for (int st = st0; st < st1; st += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        if (st + d < st1) compute(buf[d]);
        fetch(st + d + D, buf[d]);
      }
    }
  }

  // sum the KS slices of this channel block in slice order; wavefront ks then stores value indices ks, ks + KS, ...
  float* mine = red + (size_t)wave * NV * kWave;
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) mine[((t * MB + i) * 4 + e) * kWave + lane] = acc[t][i][e];
  __syncthreads();
  const float* base = red + (size_t)(wave - ks) * NV * kWave;
  for (int v = ks; v < NV; v += KS) {
    float sum = 0.f;
    for (int k2 = 0; k2 < KS; ++k2) sum += base[((size_t)k2 * NV + v) * kWave + lane];
    const int t = v / (MB * 4), i = (v / 4) % MB, e = v % 4;
    const int m = 16 * i + 4 * j + e, n = n0 + 16 * t + r16;
    if (m < M && n < N) {
      if (bias) sum += load_f(bias, bdt, n);
      y[(int64_t)m * ldy + n] = XBF16 ? f32_to_bf16_bits(sum) : f32_to_f16_bits(sum);
    }
  }
}

bool w4_frag_ok(const void* x, int64_t ldx, const int32_t* qw, int64_t ldq, int sdt, int64_t lds, int64_t ldz, int M,
                int64_t N, int64_t K, int gs, int64_t G) {
  const int64_t k4g = 1LL << 32;  // byte offsets are 32-bit
  const int64_t nt = (N + 15) / 16;
  return M > 0 && M <= 64 && sdt != FG_F32 && (K % 128) == 0 && ((gs % 128) == 0 || G == 1) && (ldx % 8) == 0 &&
         (reinterpret_cast<uintptr_t>(x) % 16) == 0 && (ldq % 4) == 0 && ldq >= 2 * K &&
         (reinterpret_cast<uintptr_t>(qw) % 16) == 0 && nt * ldq * 4 < k4g && (int64_t)M * ldx * 2 < k4g &&
         G * lds * 2 < k4g && G * ldz * 4 < k4g && group_div_exact(K, gs, G, 128);
}

// Launch shape, from a sweep of (T, KS) on the Llama-3-8B shapes at M = 1 / 16 / 64 (graph replays over a 1.2 GB
// weight ring): MB = ceil(M / 16) m-tiles (1, 2 or 4); T = 1 tile per wavefront up to 4096 channels (o_proj, down:
// 256 channel blocks, one per CU), 2 up to 8192 (qkv), else 4 (gate+up); KS = 4 K slices (2 with 4 tiles), fewer
// when a slice would be shorter than two steps.  Measured (us): o_proj M=16 7.0 (T1 KS4) against 7.5-16.7 for the
// others, qkv M=16 8.5 (T2 KS4), gate+up M=16 21.3 (T4 KS2) against 22.0 (T2 KS1) and 25.1 (T4 KS4), down M=16 17.1
// (T1 KS4); gate+up M = 1..4 16.4-17.0 with 4 tiles against 19.4-20.1 with 2.
void w4_frag_plan(int M, int N, int K, int* mb, int* T, int* KS) {
  const int b = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  const int nsteps = K / 128;
  const int t = N <= 4096 ? 1 : (N <= 8192 ? 2 : 4);
  int ks = t == 4 ? 2 : 4;
  while (ks > 1 && 2 * ks > nsteps) ks /= 2;
  ks = min(ks, w4_frag_max_threads(b, t) / kWave);
  *mb = b;
  *T = t;
  *KS = ks;
}

template <int MB, int T, bool XBF16, bool SBF16>
static hipError_t launch_frag_t(const void* x, int64_t ldx, const int32_t* qw, int64_t ldq, const void* scales,
                                int64_t lds, const int32_t* zeros, int64_t ldz, const void* bias, int bdt, void* y,
                                int64_t ldy, int M, int N, int K, int gsteps, int G, int KS, hipStream_t s) {
  const int nblk = (N + 16 * T - 1) / (16 * T);
  const int hasz = zeros != nullptr;
  const int32_t* zp = hasz ? zeros : qw;  // symmetric: a valid dummy word, ignored
  const size_t shm = (size_t)KS * (T * MB * 4) * kWave * sizeof(float);
  constexpr int D = MB == 1 ? 4 : (MB == 2 ? 3 : 2);
  auto kern = w4_frag_kernel<MB, T, D, XBF16, SBF16>;
  if (shm > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
    if (e != hipSuccess) return e;
  }
  const int64_t nt = (N + 15) / 16;
  const FragSpans sp{(uint32_t)(nt * ldq * 4), (uint32_t)((int64_t)M * ldx * 2), (uint32_t)((int64_t)G * lds * 2),
                     hasz ? (uint32_t)((int64_t)G * ldz * 4) : 4u};
  note_kernel("w4_frag_kernel KS=%d", KS);
  hipLaunchKernelGGL(kern, dim3(nblk), dim3(kWave * KS), shm, s, static_cast<const uint16_t*>(x), ldx, qw, ldq,
                     static_cast<const uint16_t*>(scales), lds, zp, hasz ? ldz : 0, hasz, bias, bdt,
                     static_cast<uint16_t*>(y), ldy, M, N, K, gsteps, KS, sp);
  return hipGetLastError();
}

template <bool XBF16, bool SBF16>
static hipError_t launch_frag_x(int mb, int T, const void* x, int64_t ldx, const int32_t* qw, int64_t ldq,
                                const void* scales, int64_t lds, const int32_t* zeros, int64_t ldz, const void* bias,
                                int bdt, void* y, int64_t ldy, int M, int N, int K, int gsteps, int G, int KS,
                                hipStream_t s) {
#define FG_FR(MB_, T_)                                                                                        \
  return launch_frag_t<MB_, T_, XBF16, SBF16>(x, ldx, qw, ldq, scales, lds, zeros, ldz, bias, bdt, y, ldy, M, N, \
                                              K, gsteps, G, KS, s)
  if (mb == 1) {
    if (T == 4) FG_FR(1, 4);
    if (T == 2) FG_FR(1, 2);
    FG_FR(1, 1);
  }
  if (mb == 2) {
    if (T == 4) FG_FR(2, 4);
    if (T == 2) FG_FR(2, 2);
    FG_FR(2, 1);
  }
  if (T == 4) FG_FR(4, 4);
  if (T == 2) FG_FR(4, 2);
  FG_FR(4, 1);
#undef FG_FR
}

hipError_t launch_w4_frag(const void* x, int64_t ldx, bool xbf16, const int32_t* qw, int64_t ldq, const void* scales,
                          int sdt, int64_t lds, const int32_t* zeros, int64_t ldz, const void* bias, int bdt, void* y,
                          int64_t ldy, int M, int N, int K, int gs, bool single_group, int G, hipStream_t s) {
  int mb, T, KS;
  w4_frag_plan(M, N, K, &mb, &T, &KS);
  const int gsteps = single_group ? 0 : gs / 128;
  const bool sbf = sdt == FG_BF16;
  if (xbf16) {
    if (sbf) return launch_frag_x<true, true>(mb, T, x, ldx, qw, ldq, scales, lds, zeros, ldz, bias, bdt, y, ldy, M, N, K, gsteps, G, KS, s);
    return launch_frag_x<true, false>(mb, T, x, ldx, qw, ldq, scales, lds, zeros, ldz, bias, bdt, y, ldy, M, N, K, gsteps, G, KS, s);
  }
  if (sbf) return launch_frag_x<false, true>(mb, T, x, ldx, qw, ldq, scales, lds, zeros, ldz, bias, bdt, y, ldy, M, N, K, gsteps, G, KS, s);
  return launch_frag_x<false, false>(mb, T, x, ldx, qw, ldq, scales, lds, zeros, ldz, bias, bdt, y, ldy, M, N, K, gsteps, G, KS, s);
}

}  // namespace fg
