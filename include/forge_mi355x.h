/* forge_mi355x -- C ABI of the MI355X-native (gfx950) quantized-linear hot path.
 *
 * One shared library, libforge_mi355x.so, built with hipcc --offload-arch=gfx950.  Every entry point takes plain
 * device pointers, element strides and sizes, enqueues its kernels on `stream` and returns immediately (no host
 * synchronisation, no device allocation: callers own every buffer, so launches can be captured in a HIP graph).
 *
 * Return value: FG_OK (0) or an error code; fg_last_error() gives a message for the calling thread.
 *
 * Each entry point names the reference interface it replaces (paths are in the Forge-LLM source tree).
 */
#ifndef FORGE_MI355X_H
#define FORGE_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* fg_stream_t; /* a hipStream_t; NULL = the default stream */

/* element type codes */
enum {
  FG_F32 = 0,
  FG_F16 = 1,
  FG_BF16 = 2,
  FG_E4M3 = 3, /* OCP float8 e4m3fn */
  FG_I8 = 4,
  FG_I32 = 5
};

/* status codes */
enum { FG_OK = 0, FG_EINVAL = 1, FG_EUNSUPPORTED = 2, FG_EHIP = 3 };

/* W4A16 implementation selector (fg_w4_config.impl) */
enum { FG_W4_AUTO = 0, FG_W4_GEMV = 1, FG_W4_MFMA = 2, FG_W4_GENERIC = 3, FG_W4_PREFILL = 4, FG_W4_DEQUANT_GEMM = 5 };
/* FG_W4_PREFILL: the prefill kernels, x straight to LDS, weights dequantised tile by tile and fed to bf16 / fp16 MFMA
   (large M x N; needs K % 64 == 0, group % 32 == 0 or one group, aligned x / qweight, no act-order perm): from 256
   rows the ping-pong kernel (256 x 256 tiles, two teams of wavefronts alternating MFMA and dequantisation; group %
   64 == 0, N % 8 == 0, 16-bit scales) once the problem has >= 160 such tiles, else the producer / consumer kernel
   (256 x 128 tiles), else the all-rounder (128 / 256 x 256 tiles, split-K).  fg_w4_config.tile_n = 256 / 128 / 64
   forces one of them where its conditions hold.
   FG_W4_DEQUANT_GEMM: the reference's dequant_matmul route (forge/kernels/triton/gemm_w4_dequant.py:194-256,
   dequantise then a library GEMM); here a name for FG_W4_PREFILL, whose kernels fuse the two steps. */

/* GEMV kernel selector (fg_w4_config.gemv_kernel) */
enum { FG_GEMV_AUTO = 0, FG_GEMV_SPLIT = 1, FG_GEMV_TILE = 2, FG_GEMV_WAVE = 3 };

/* Launch knobs; pass NULL for the built-in per-shape policy.  Zero fields mean "policy default". */
typedef struct fg_w4_config {
  int32_t impl;         /* FG_W4_* */
  int32_t rows_per_wave; /* GEMV: output channels per wavefront (1, 2 or 4) */
  int32_t max_blocks;   /* GEMV: cap on workgroups (grid-stride beyond it) */
  int32_t tile_m;       /* MFMA: rows of x per workgroup tile (16, 32, 64 or 128); setting it (or split_k) selects
                           the LDS-tiled MFMA kernel over the register-resident split-K kernel used for M <= 64 */
  int32_t split_k;      /* MFMA / PREFILL: K splits (fp32 partials in the workspace, reduced in fixed order) */
  int32_t tile_n;       /* GEMV tile kernel: output channels per workgroup tile (rounded up to a multiple of 8);
                           PREFILL: 256 / 128 / 64 = ping-pong / producer-consumer / all-round kernel */
  int32_t gemv_kernel;  /* GEMV: FG_GEMV_SPLIT = split-K register kernel (M <= 4, K <= 65536), FG_GEMV_TILE = LDS-tiled
                           kernel, FG_GEMV_WAVE = one-wavefront-per-row-block kernel; AUTO = split when it fits,
                           else tile, else wave.  Setting rows_per_wave implies WAVE, tile_n implies TILE. */
  int32_t reserved[1];
} fg_w4_config;

typedef struct fg_mm_config {
  int32_t tile_m; /* 0 = policy; 64 / 128 = 64- / 128-row tiles: with K % 128 == 0 and 16-byte aligned A, B whose
                     lda, ldb are multiples of 16, the ring kernel (direct-to-LDS loads, several K slices in flight;
                     width from tile_n or the policy), otherwise square register-staged tiles; 256 = the 256-row
                     direct-to-LDS kernel (256 x 256 tiles, 256 x 320 for INT8 with 16-bit outputs where that fills
                     the CUs' last round better) (needs the same K and alignment, else FG_EUNSUPPORTED); 16 = the
                     skinny split-K kernel (M <= 64, K % 256 == 0, same alignment; modes 0 / 1); 1 = the INT8
                     decode GEMV (fg_int8_gemm only: M <= 2, K % 16 == 0, N % 8 == 0, same alignment), which the policy
                     takes for 1..2 rows */
  int32_t tile_n; /* ring kernel tile width: 32, 64 or 128 with tile_m = 64, 128 with tile_m = 128 (needs the ring
                     kernel's conditions, else FG_EUNSUPPORTED); 0 = policy; ignored for tile_m 16 / 256 */
  int32_t reserved[6];
} fg_mm_config;

/* ---------------------------------------------------------------------------------------------------------------
 * W4A16:  y[M,N] = x[M,K] @ dequant(W)[N,K]^T (+ bias),  W[n,k] = (q[n,k] - zero[n,g(k)]) * scale[n,g(k)].
 * Replaces the Triton launchers behind w4a16_linear: forge/kernels/ops_gemm.py:287-317 ->
 * forge/kernels/triton/gemm_w4a16.py:69-153 (w4a16_gemm_triton), gemm_w4_fast.py:274-343 (w4_fast_gemm, gemv/dot),
 * gemm_w4_dequant.py:194-236 (w4_dequant_matmul), gemm_wq.py:138-204 (legacy wq_gemm).
 *   x        x_dtype (FG_BF16 | FG_F16) [M, ldx], unit stride along K
 *   qweight  int32 [N, ldq] portable_row words (forge/kernels/layouts/w4.py:15-17), ldq >= ceil(K/8)
 *   scales   scale_dtype (FG_F16 | FG_BF16 | FG_F32) [n_groups, lds], lds >= N
 *   zeros    int32 [n_groups, ldz] packed 8 channels per word, or NULL (symmetric, zero-point 8)
 *   perm     int32 [K] or NULL: column order of a group-sorted act-order weight; x is read as x[:, perm[k]]
 *   g_idx    int32 [K] or NULL: per-column group id (irregular act-order; selects the generic kernel)
 *   bias     bias_dtype [N] or NULL
 *   y        x_dtype [M, ldy]
 *   group_size  > 0 (multiple of 8) or <= 0 for one group per row
 *   workspace   device scratch of at least fg_w4a16_workspace_bytes(...) bytes (may be NULL when that is 0); the
 *               caller allocates it (e.g. from the torch caching allocator on the same stream), as the reference's
 *               split-K workspace (forge/kernels/triton/gemm_w4_fast.py:316-318)
 * ------------------------------------------------------------------------------------------------------------- */
int fg_w4a16_gemm(const void* x, int64_t ldx, int x_dtype, const int32_t* qweight, int64_t ldq, const void* scales,
                  int scale_dtype, int64_t lds, const int32_t* zeros, int64_t ldz, const int32_t* perm,
                  const int32_t* g_idx, const void* bias, int bias_dtype, void* y, int64_t ldy, int64_t M, int64_t N,
                  int64_t K, int32_t group_size, int32_t n_groups, const fg_w4_config* cfg, void* workspace,
                  size_t workspace_bytes, fg_stream_t stream);

/* W4A16 without a caller workspace.  No counterpart in the reference: an entry point for callers that cannot allocate
 * device memory (code under HIP graph capture in harnesses that forbid hipMalloc, tight serving loops).  Arguments and
 * results are those of fg_w4a16_gemm minus the workspace: split-K partials go to a static device buffer of
 * FG_W4A16_SCRATCH_BYTES that the library holds on every GPU it runs on until the process ends.  A launch whose plan
 * needs more scratch than that returns FG_EINVAL (call fg_w4a16_gemm with a workspace instead).  Nothing is allocated
 * and nothing in the buffer needs clearing (each launch writes all the partials it reduces).  Calls that overlap on
 * one GPU (concurrent streams or host threads) share the buffer and race.  The calling thread's current device must be
 * the device of `stream` and of the tensors. */
#define FG_W4A16_SCRATCH_BYTES ((size_t)64 << 20)
int fg_w4a16_gemm_noalloc(const void* x, int64_t ldx, int x_dtype, const int32_t* qweight, int64_t ldq,
                          const void* scales, int scale_dtype, int64_t lds, const int32_t* zeros, int64_t ldz,
                          const int32_t* perm, const int32_t* g_idx, const void* bias, int bias_dtype, void* y,
                          int64_t ldy, int64_t M, int64_t N, int64_t K, int32_t group_size, int32_t n_groups,
                          const fg_w4_config* cfg, fg_stream_t stream);

/* Workspace bytes fg_w4a16_gemm needs for this problem and config (0 for single-pass launches).  The alignment and
 * g_idx flags must match the later call: x_aligned = x and ldx allow 16-byte row loads, q_aligned = qweight and ldq
 * allow 16-byte chunk loads, has_g_idx = a per-column g_idx will be passed. */
size_t fg_w4a16_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t group_size, int32_t x_aligned,
                                int32_t q_aligned, int32_t has_g_idx, const fg_w4_config* cfg);

/* W4A16 on the CDNA4 MFMA-fragment layout w4.cdna4_mfma_k128n16 (forge_amd.layouts.CDNA4_W4), for 1 <= M <= 64.
 * The reference reserves a "native" executor for fragment-ordered W4 layouts that kernels read without shuffles
 * (forge/kernels/layouts/layout.py:14-17,158-190, w4.py:18-24) but ships no kernel for it; this is that kernel for
 * gfx950, over this build's fragment order (v_mfma_f32_16x16x32 B operands; load-time repack in
 * forge_amd.layouts.repack / ops_gemm.prepare_w4).  Same arguments and results as fg_w4a16_gemm except:
 *   qweight  int32 [ceil(N/16), ldq]: 16-channel tile rows, 256 words per 128-column tile, ldq >= 2 * K (K % 128 == 0)
 *   no perm / g_idx (act-order weights are column-sorted first)
 *   workspace  16-byte aligned, at least fg_w4a16_cdna4_workspace_bytes(M, N, K, group_size) bytes (NULL when that
 *              is 0): fp32 K-split partials of the LDS-ring kernel (29..64 rows, or 9..64 over K >= 8192), summed by a
 *              second launch in split order; smaller M runs one launch that sums its K slices in LDS
 * Needs group_size % 128 == 0 (or one group), fp16 / bf16 scales, 16-byte aligned x (ldx % 8 == 0) and qweight. */
int fg_w4a16_gemm_cdna4(const void* x, int64_t ldx, int x_dtype, const int32_t* qweight, int64_t ldq,
                        const void* scales, int scale_dtype, int64_t lds, const int32_t* zeros, int64_t ldz,
                        const void* bias, int bias_dtype, void* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                        int32_t group_size, int32_t n_groups, void* workspace, size_t workspace_bytes,
                        fg_stream_t stream);

/* Workspace bytes fg_w4a16_gemm_cdna4 may need for this problem (an upper bound: 0 when its launch plan has no K
 * split). */
size_t fg_w4a16_cdna4_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t group_size);

/* W4A16 decode GEMV (1 <= M <= 4) on portable_row weights whose scales and zero-points are re-blocked by 8 channels.
 * No counterpart in the reference: the reference's GEMV reads the portable [G, N] scales (forge/kernels/layouts/w4.py
 * :15-17), and this entry point serves the copy that forge_amd's packed-linear module keeps beside them
 * (forge_amd.layouts.sz8_blocks, KernelW4A16Linear.prepare): with it each wavefront reads the scales and zero words of
 * its channels and K slice as one contiguous run instead of one strided word per group.  Same arguments and results
 * as fg_w4a16_gemm (split-K decode GEMV, bit-identical output) except:
 *   scales8  fp16|bf16 [N / 8][G][8]: scale (g, n) at ((n / 8) * G + g) * 8 + n % 8
 *   zeros8   int32 [N / 8][G]: the zero word of group g and channels 8 b .. 8 b + 7 at b * G + g (nibble n % 8 =
 *            channel n's zero-point); NULL = symmetric (zero-point 8)
 *   n_groups must equal ceil(K / group_size); no perm / g_idx, no workspace
 * Needs N % 8 == 0, K % 32 == 0, group_size % 32 == 0 (or one group), 16-byte aligned x (ldx % 8 == 0), qweight
 * (ldq % 4 == 0) and scales8; FG_EUNSUPPORTED otherwise. */
int fg_w4a16_gemv_sz8(const void* x, int64_t ldx, int x_dtype, const int32_t* qweight, int64_t ldq,
                      const void* scales8, int scale_dtype, const int32_t* zeros8, const void* bias, int bias_dtype,
                      void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, int32_t group_size, int32_t n_groups,
                      fg_stream_t stream);

/* Dense dequantisation out[n,k] = (q - z) * s computed in fp32 and rounded once to out_dtype (FG_F32|FG_F16|FG_BF16).
 * Replaces forge/kernels/triton/gemm_w4_dequant.py:143-191 (w4_dequant) and PackedW4.dequantize
 * (forge/kernels/layouts/w4.py:137-140 -> dequantize_parts :294-305). */
int fg_w4_dequant(const int32_t* qweight, int64_t ldq, const void* scales, int scale_dtype, int64_t lds,
                  const int32_t* zeros, int64_t ldz, const int32_t* g_idx, void* out, int out_dtype, int64_t ldo,
                  int64_t N, int64_t K, int32_t group_size, int32_t n_groups, fg_stream_t stream);

/* ---------------------------------------------------------------------------------------------------------------
 * W8A16:  y[M,N] = x[M,K] @ dequant(W)[N,K]^T (+ bias),  W[n,k] = q[n,k] * scale[g(k), n],  q signed int8 (symmetric).
 * Replaces the Triton launcher behind w8a16_linear: forge/kernels/ops_gemm.py:320-346 ->
 * forge/kernels/triton/gemm_w8a16.py:14-31 (wq_gemm with bits=8, forge/kernels/triton/gemm_wq.py:138-205).
 *   x        bf16|fp16 [M, K] (row stride ldx)
 *   qweight  int8 [N, K] (row stride ldq, bytes; portable_row PackedW8, forge/kernels/layouts/w8.py:18-104)
 *   scales   fp16|bf16|fp32 [G, N] (row stride lds);  group_size <= 0: one group per row (per-channel)
 *   cfg      NULL (policy: decode GEMV for 1..2 rows and 3..4 over N <= 8192 and K < 8192; LDS-ring kernel for
 *            17..64 rows and for 3..16 over N >= 16384 or K >= 8192; skinny kernel for the other rows up to 64;
 *            then the prefill kernels: from 256 rows the ping-pong kernel once the problem has >= 160 tiles of
 *            256 x 256, below that the ping-pong kernel with K split 2 or 4 ways when tiles x splits reaches 160,
 *            else the all-rounder) or impl FG_W4_GEMV (split-K decode GEMV, M <= 4), FG_W4_MFMA (skinny
 *            kernel, M <= 64), FG_W4_PREFILL / FG_W4_DEQUANT_GEMM (the prefill kernels; tile_n = 256 / 64 forces
 *            the ping-pong / all-round kernel), FG_W4_GENERIC (any shape); split_k for the prefill kernels
 *   workspace  fg_w8a16_workspace_bytes bytes (split-K partials of the prefill kernels or, under the policy, of the
 *              LDS-ring kernel; 0 when none applies)
 * ------------------------------------------------------------------------------------------------------------- */
size_t fg_w8a16_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t group_size, const fg_w4_config* cfg);
int fg_w8a16_gemm(const void* x, int64_t ldx, int x_dtype, const int8_t* qweight, int64_t ldq, const void* scales,
                  int scale_dtype, int64_t lds, const void* bias, int bias_dtype, void* y, int64_t ldy, int64_t M,
                  int64_t N, int64_t K, int32_t group_size, int32_t n_groups, const fg_w4_config* cfg,
                  void* workspace, size_t workspace_bytes, fg_stream_t stream);

/* ---------------------------------------------------------------------------------------------------------------
 * INT8 W8A8:  acc[M,N] = a[M,K] @ b[N,K]^T in exact int32;  y = (float(acc) * sa[m]) * sb[n] (+ bias[n]).
 * Replaces forge/kernels/triton/gemm_int8.py:95-137 (int8_gemm_triton), called from int8_linear
 * (forge/kernels/ops_gemm.py:483-515).
 *   sa  float [sa_len], sa_len in {1, M};  sb float [sb_len], sb_len in {1, N}
 *   y_dtype  FG_F32 | FG_F16 | FG_BF16, or FG_I32 to store the raw int32 accumulator (scales ignored; a bias is rejected)
 * ------------------------------------------------------------------------------------------------------------- */
int fg_int8_gemm(const int8_t* a, int64_t lda, const float* sa, int64_t sa_len, const int8_t* b, int64_t ldb,
                 const float* sb, int64_t sb_len, const void* bias, int bias_dtype, void* y, int64_t ldy, int y_dtype,
                 int64_t M, int64_t N, int64_t K, const fg_mm_config* cfg, fg_stream_t stream);

/* ---------------------------------------------------------------------------------------------------------------
 * FP8 W8A8 (OCP e4m3fn operands, fp32 accumulation):  y = sum_k (a*sa)(b*sb) (+ bias).
 * Replaces forge/kernels/triton/gemm_fp8.py:194-248 (fp8_gemm_triton) with the scale normalisation of
 * prepare_fp8_scales (gemm_fp8.py:151-191), called from fp8_linear (forge/kernels/ops_gemm.py:396-461).
 *   scale_mode 0: per-tensor sa[0], sb[0];  1: sa[m * sa_sm], sb[n * sb_sn] (stride 0 broadcasts);
 *              2: K-blocked: sa[m * sa_sm + kb * sa_sk], sb[(n / sb_div) * sb_sn + kb * sb_sk], kb = k / block
 *   y_dtype FG_F32 | FG_F16 | FG_BF16
 * ------------------------------------------------------------------------------------------------------------- */
int fg_fp8_gemm(const uint8_t* a, int64_t lda, const float* sa, int64_t sa_sm, int64_t sa_sk, const uint8_t* b,
                int64_t ldb, const float* sb, int64_t sb_sn, int64_t sb_sk, int32_t sb_div, int32_t scale_mode,
                int32_t block, const void* bias, int bias_dtype, void* y, int64_t ldy, int y_dtype, int64_t M,
                int64_t N, int64_t K, const fg_mm_config* cfg, fg_stream_t stream);

/* ---------------------------------------------------------------------------------------------------------------
 * Per-token activation quantisers (one scale per row of x).
 * INT8: s = amax /_IEEE 127 (1 if amax is not > 0), q = clamp(round_half_even(x /_IEEE s), -127, 127).
 *   Replaces forge/kernels/triton/gemm_int8.py:140-151 (int8_quant_triton) behind quantize_act_int8
 *   (forge/kernels/ops_gemm.py:467-480); oracle forge/kernels/ref/gemm_int8.py:17-35.
 * FP8:  optional fused RMSNorm y = x * rsqrt(mean(x^2) + eps) * w (fp32), then s = amax / 448 (1 if amax is not > 0),
 *       q = e4m3fn(clamp(y / s, -448, 448)), round-half-even.  static_scale (device float[M], one per row)
 *       replaces s when given (s may then be NULL).
 *   Replaces forge/kernels/triton/gemm_fp8.py:251-304 (act_quant_fp8_triton, per_token / per_tensor-static) behind
 *   quantize_act_fp8 (forge/kernels/ops_gemm.py:359-388); oracles forge/kernels/ref/gemm_fp8.py:43-85,130-150.
 * ------------------------------------------------------------------------------------------------------------- */
int fg_quant_int8_rowwise(const void* x, int64_t ldx, int x_dtype, int8_t* q, int64_t ldq, float* s, int64_t M,
                          int64_t K, fg_stream_t stream);

int fg_quant_fp8_rowwise(const void* x, int64_t ldx, int x_dtype, uint8_t* q, int64_t ldq, float* s, int64_t M,
                         int64_t K, const float* static_scale, const void* rms_weight, int rms_weight_dtype,
                         float rms_eps, int32_t fuse_rmsnorm, fg_stream_t stream);

/* FP8 quantisation with one scale per [block_m x block_k] tile of x: s[i, j] (row stride lds) covers rows
 * i*block_m.. and columns j*block_k..; s = amax / 448 (1 if amax is not > 0) or *static_scale for every tile.
 * block_m = 1, block_k = 128 is the reference's 1x128 activation blocks (gemm_fp8.py act_quant_blockwise),
 * block_m = block_k = 128 its 128x128 weight blocks and block_m = M, block_k = K one per-tensor scale
 * (oracle forge/kernels/ref/gemm_fp8.py:43-85, granularities block / block2d / per_tensor). */
int fg_quant_fp8_block(const void* x, int64_t ldx, int x_dtype, uint8_t* q, int64_t ldq, float* s, int64_t lds,
                       int64_t M, int64_t K, int32_t block_m, int32_t block_k, const float* static_scale,
                       fg_stream_t stream);

/* ---------------------------------------------------------------------------------------------------------------
 * Library information.  fg_device_ok replaces the capability gate triton_usable (forge/kernels/ops_gemm.py:159-175):
 * returns 1 when `device` is a gfx950 GPU this build can run on, else 0 (message in fg_last_error).
 * ------------------------------------------------------------------------------------------------------------- */
const char* fg_version(void);
const char* fg_last_error(void);
int fg_device_ok(int device);

/* Name of the kernel, with its launch form, that the calling thread's last successful launch through this library
 * ran, e.g. "w4_gemv_split_kernel<1,1,8>" or "w4_ring_kernel KS=4 + w4_ring_reduce_kernel"; "" before the first.
 * The reference records the path each op took (last_path, forge/kernels/ops_gemm.py:81-99, and the bench's per-case
 * `path`, forge/kernels/bench.py:188,648); this names the kernel below that path.  Valid until the same thread's next
 * call into the library. */
const char* fg_last_kernel(void);

#ifdef __cplusplus
}
#endif

#endif /* FORGE_MI355X_H */
