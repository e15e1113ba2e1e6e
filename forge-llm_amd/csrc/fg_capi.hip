// extern "C" entry points of libforge_mi355x.so: argument validation, per-shape kernel policy, launch.
// Declarations and the reference interface each one replaces: include/forge_mi355x.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/forge_mi355x.h"
#include "fg_device.h"

namespace fg {
hipError_t launch_w4_gemv(int mt, int R, bool xbf16, const void* x, int64_t ldx, const int32_t* qw, int64_t ldq,
                          const void* scales, int sdt, int64_t lds, const int32_t* zeros, int64_t ldz,
                          const int32_t* perm, const void* bias, int bdt, void* y, int64_t ldy, int M, int N, int K,
                          int gs, int max_blocks, hipStream_t s);
hipError_t launch_w4_generic(const void* x, int64_t ldx, int xdt, const int32_t* qw, int64_t ldq, const void* scales,
                             int sdt, int64_t lds, const int32_t* zeros, int64_t ldz, const int32_t* perm,
                             const int32_t* g_idx, const void* bias, int bdt, void* y, int64_t ldy, int M, int N,
                             int K, int gs, hipStream_t s);
hipError_t launch_w4_dequant(const int32_t* qw, int64_t ldq, const void* scales, int sdt, int64_t lds,
                             const int32_t* zeros, int64_t ldz, const int32_t* g_idx, void* out, int odt, int64_t ldo,
                             int N, int K, int gs, hipStream_t s);
hipError_t launch_w4_mfma(const void* x, int64_t ldx, bool xbf16, const int32_t* qw, int64_t ldq, const void* scales,
                          int sdt, int64_t lds, const int32_t* zeros, int64_t ldz, const int32_t* perm,
                          const void* bias, int bdt, void* y, int64_t ldy, float* ws, int M, int N, int K, int gs,
                          int tile_m, int splits, hipStream_t s);
void w4_mfma_split_plan(int M, int N, int K, int tile_m, int split_k, int* kchunk, int* used);
bool w4_big_ok(const void* x, int64_t ldx, const int32_t* qw, int64_t ldq, const int32_t* perm, int64_t K, int gs,
               int64_t G);
size_t w4_big_workspace_bytes(int M, int N, int K, int split_k, bool w8);
bool w4_pc_ok(const void* x, int64_t ldx, const int32_t* qw, int64_t ldq, const int32_t* perm, const void* scales,
              int sdt, int64_t lds, int64_t N, int64_t K, int gs, int64_t G);
size_t w4_pc_workspace_bytes(int M, int N, int K, int split_k);
bool w4_pp_ok(const void* x, int64_t ldx, const int32_t* qw, int64_t ldq, const int32_t* perm, const void* scales,
              int sdt, int64_t lds, const int32_t* zeros, int64_t ldz, int64_t M, int64_t N, int64_t K, int gs,
              int64_t G);
bool w8_pp_ok(const void* x, int64_t ldx, const int8_t* qw, int64_t ldq, const void* scales, int sdt, int64_t lds,
              int64_t M, int64_t N, int64_t K, int gs, int64_t G);
size_t w4_pp_workspace_bytes(int M, int N, int K, int split_k);
hipError_t launch_w4_pp(const void* x, int64_t ldx, bool xbf16, const int32_t* qw, int64_t ldq, const void* scales,
                        int sdt, int64_t lds, const int32_t* zeros, int64_t ldz, const void* bias, int bdt, void* y,
                        int64_t ldy, float* ws, int M, int N, int K, int gs, bool single_group, int split_k,
                        hipStream_t s);
hipError_t launch_w8_pp(const void* x, int64_t ldx, bool xbf16, const int8_t* qw, int64_t ldq, const void* scales,
                        int sdt, int64_t lds, const void* bias, int bdt, void* y, int64_t ldy, float* ws, int M, int N,
                        int K, int gs, bool single_group, int split_k, hipStream_t s);
hipError_t launch_w4_pc(const void* x, int64_t ldx, bool xbf16, const int32_t* qw, int64_t ldq, const void* scales,
                        int sdt, int64_t lds, const int32_t* zeros, int64_t ldz, const void* bias, int bdt, void* y,
                        int64_t ldy, float* ws, int M, int N, int K, int gs, bool single_group, int split_k,
                        hipStream_t s);
bool w8a16_skinny_ok(const void* x, int64_t ldx, const int8_t* qw, int64_t ldq, int sdt, int64_t lds, int64_t M,
                     int64_t N, int64_t K, int gs, int64_t G);
hipError_t launch_w8a16_skinny(const void* x, int64_t ldx, bool xbf16, const int8_t* qw, int64_t ldq,
                               const void* scales, int sdt, int64_t lds, const void* bias, int bdt, void* y,
                               int64_t ldy, int M, int N, int K, int gs, bool single_group, hipStream_t s);
hipError_t launch_w8a16_generic(const void* x, int64_t ldx, int xdt, const int8_t* qw, int64_t ldq,
                                const void* scales, int sdt, int64_t lds, const void* bias, int bdt, void* y,
                                int64_t ldy, int M, int N, int K, int gs, hipStream_t s);
bool w8a16_ring_ok(const void* x, int64_t ldx, const int8_t* qw, int64_t ldq, const void* scales, int sdt,
                   int64_t lds, int64_t M, int64_t N, int64_t K, int gs, int64_t G);
size_t w8a16_ring_workspace_bytes(int M, int N, int K);
hipError_t launch_w8a16_ring(const void* x, int64_t ldx, bool xbf16, const int8_t* qw, int64_t ldq,
                             const void* scales, int sdt, int64_t lds, const void* bias, int bdt, void* y, int64_t ldy,
                             int M, int N, int K, int gs, bool single_group, int G, void* ws, size_t ws_bytes,
                             hipStream_t s);
bool w8a16_gemv_ok(const void* x, int64_t ldx, const int8_t* qw, int64_t ldq, const void* scales, int sdt,
                   int64_t lds, int64_t M, int64_t N, int64_t K, int gs, int64_t G);
hipError_t launch_w8a16_gemv(const void* x, int64_t ldx, bool xbf16, const int8_t* qw, int64_t ldq,
                             const void* scales, int sdt, int64_t lds, const void* bias, int bdt, void* y,
                             int64_t ldy, int M, int N, int K, int gs, bool single_group, int64_t G, hipStream_t s);
bool w8_big_ok(const void* x, int64_t ldx, const int8_t* qw, int64_t ldq, int64_t K, int gs, int64_t G);
hipError_t launch_w8_big(const void* x, int64_t ldx, bool xbf16, const int8_t* qw, int64_t ldq, const void* scales,
                         int sdt, int64_t lds, const void* bias, int bdt, void* y, int64_t ldy, float* ws, int M,
                         int N, int K, int gs, bool single_group, int split_k, hipStream_t s);
bool w4_skinny_ok(const void* x, int64_t ldx, const int32_t* qw, int64_t ldq, const int32_t* perm, int sdt,
                  int64_t lds, int64_t ldz, int M, int64_t N, int64_t K, int gs, int64_t G);
hipError_t launch_w4_skinny(const void* x, int64_t ldx, bool xbf16, const int32_t* qw, int64_t ldq,
                            const void* scales, int sdt, int64_t lds, const int32_t* zeros, int64_t ldz,
                            const void* bias, int bdt, void* y, int64_t ldy, int M, int N, int K, int gs,
                            bool single_group, hipStream_t s);
hipError_t launch_w4_big(const void* x, int64_t ldx, bool xbf16, const int32_t* qw, int64_t ldq, const void* scales,
                         int sdt, int64_t lds, const int32_t* zeros, int64_t ldz, const void* bias, int bdt, void* y,
                         int64_t ldy, float* ws, int M, int N, int K, int gs, bool single_group, int split_k,
                         hipStream_t s);
size_t w4_gemv_lds_bytes(int mt, int K);
bool w4_frag_ok(const void* x, int64_t ldx, const int32_t* qw, int64_t ldq, int sdt, int64_t lds, int64_t ldz, int M,
                int64_t N, int64_t K, int gs, int64_t G);
hipError_t launch_w4_frag(const void* x, int64_t ldx, bool xbf16, const int32_t* qw, int64_t ldq, const void* scales,
                          int sdt, int64_t lds, const int32_t* zeros, int64_t ldz, const void* bias, int bdt, void* y,
                          int64_t ldy, int M, int N, int K, int gs, bool single_group, int G, hipStream_t s);
bool w4_ring_ok(bool portable, const void* x, int64_t ldx, const int32_t* qw, int64_t ldq, const void* scales, int sdt,
                int64_t lds, const int32_t* zeros, int64_t ldz, int M, int64_t N, int64_t K, int gs, int64_t G);
bool w4_ring_preferred(bool portable, int M, int N, int K);
bool int8_gemv_ok(const void* a, int64_t lda, const void* b, int64_t ldb, int64_t M, int64_t N, int64_t K);
hipError_t launch_int8_gemv(const int8_t* a, int64_t lda, const float* sa, int64_t sa_len, const int8_t* b,
                            int64_t ldb, const float* sb, int64_t sb_len, const void* bias, int bdt, void* y,
                            int64_t ldy, int ydt, int M, int N, int K, hipStream_t s);
size_t w4_ring_workspace_bytes(bool portable, int M, int N, int K);
hipError_t launch_w4_ring(bool portable, const void* x, int64_t ldx, bool xbf16, const int32_t* qw, int64_t ldq,
                          const void* scales, int sdt, int64_t lds, const int32_t* zeros, int64_t ldz, const void* bias,
                          int bdt, void* y, int64_t ldy, int M, int N, int K, int gs, bool single_group, int G, void* ws,
                          size_t ws_bytes, hipStream_t s);
hipError_t launch_w4_gemv_tile(int mt, bool xbf16, const void* x, int64_t ldx, const int32_t* qw, int64_t ldq,
                               const void* scales, int sdt, int64_t lds, const int32_t* zeros, int64_t ldz,
                               const int32_t* perm, const void* bias, int bdt, void* y, int64_t ldy, int M, int N,
                               int K, int gs, int G, int tile_n, hipStream_t s);
bool w4_gemv_tile_ok(int mt, int N, int K, int G, int tile_n);
hipError_t launch_w4_gemv_split(int mt, bool xbf16, const void* x, int64_t ldx, const int32_t* qw, int64_t ldq,
                                const void* scales, int sdt, int64_t lds, const int32_t* zeros, int64_t ldz,
                                const int32_t* perm, const void* bias, int bdt, void* y, int64_t ldy, int M, int N,
                                int K, int gs, bool single_group, hipStream_t s);
bool w4_gemv_split_ok(int mt, int N, int K);
bool w4_gemv_sz8_ok(const void* x, int64_t ldx, const int32_t* qw, int64_t ldq, const void* scales8, int sdt, int M,
                    int N, int K, int gs);
hipError_t launch_w4_gemv_sz8(int mt, bool xbf16, const void* x, int64_t ldx, const int32_t* qw, int64_t ldq,
                              const void* scales8, int sdt, const int32_t* zeros8, const void* bias, int bdt, void* y,
                              int64_t ldy, int M, int N, int K, int gs, bool single_group, hipStream_t s);
bool w4_gemv_split_preferred(int mt, const void* x, int64_t ldx, const int32_t* perm, const void* scales, int sdt,
                             int64_t lds, int64_t ldq, const int32_t* zeros, int64_t ldz, int M, int N, int K, int gs,
                             bool single_group);
size_t w4_gemv_tile_lds_bytes(int mt, int K, int G, int TN);
hipError_t launch_int8_gemm(const int8_t* a, int64_t lda, const float* sa, int64_t sa_len, const int8_t* b,
                            int64_t ldb, const float* sb, int64_t sb_len, const void* bias, int bdt, void* y,
                            int64_t ldy, int ydt, int M, int N, int K, int tile, hipStream_t s);
hipError_t launch_fp8_gemm(const uint8_t* a, int64_t lda, const float* sa, int64_t sa_sm, const uint8_t* b,
                           int64_t ldb, const float* sb, int64_t sb_sn, const void* bias, int bdt, void* y,
                           int64_t ldy, int ydt, int M, int N, int K, int tile, hipStream_t s);
bool mm_big_ok(const void* a, int64_t lda, const void* b, int64_t ldb, int64_t K);
bool w8_skinny_ok(const void* a, int64_t lda, const void* b, int64_t ldb, int64_t M, int64_t N, int64_t K);
hipError_t launch_int8_gemm_skinny(const int8_t* a, int64_t lda, const float* sa, int64_t sa_len, const int8_t* b,
                                   int64_t ldb, const float* sb, int64_t sb_len, const void* bias, int bdt, void* y,
                                   int64_t ldy, int ydt, int M, int N, int K, hipStream_t s);
hipError_t launch_fp8_gemm_skinny(const uint8_t* a, int64_t lda, const float* sa, int64_t sa_sm, const uint8_t* b,
                                  int64_t ldb, const float* sb, int64_t sb_sn, const void* bias, int bdt, void* y,
                                  int64_t ldy, int ydt, int M, int N, int K, hipStream_t s);
int64_t mm_big_tiles(int64_t M, int64_t N);
hipError_t launch_int8_gemm_big(const int8_t* a, int64_t lda, const float* sa, int64_t sa_len, const int8_t* b,
                                int64_t ldb, const float* sb, int64_t sb_len, const void* bias, int bdt, void* y,
                                int64_t ldy, int ydt, int M, int N, int K, hipStream_t s);
hipError_t launch_fp8_gemm_big(const uint8_t* a, int64_t lda, const float* sa, int64_t sa_sm, const uint8_t* b,
                               int64_t ldb, const float* sb, int64_t sb_sn, const void* bias, int bdt, void* y,
                               int64_t ldy, int ydt, int M, int N, int K, hipStream_t s);
int mm_ring_bn(int64_t M, int64_t N, int bm);
hipError_t launch_int8_gemm_ring(const int8_t* a, int64_t lda, const float* sa, int64_t sa_len, const int8_t* b,
                                 int64_t ldb, const float* sb, int64_t sb_len, const void* bias, int bdt, void* y,
                                 int64_t ldy, int ydt, int M, int N, int K, int bm, int bn, hipStream_t s);
hipError_t launch_fp8_gemm_ring(const uint8_t* a, int64_t lda, const float* sa, int64_t sa_sm, const uint8_t* b,
                                int64_t ldb, const float* sb, int64_t sb_sn, const void* bias, int bdt, void* y,
                                int64_t ldy, int ydt, int M, int N, int K, int bm, int bn, hipStream_t s);
hipError_t launch_fp8_gemm_blocked(const uint8_t* a, int64_t lda, const float* sa, int64_t sa_sm, int64_t sa_sk,
                                   const uint8_t* b, int64_t ldb, const float* sb, int64_t sb_sn, int64_t sb_sk,
                                   int sb_div, const void* bias, int bdt, void* y, int64_t ldy, int ydt, int M, int N,
                                   int K, hipStream_t s);
hipError_t launch_quant_int8(const void* x, int64_t ldx, int xdt, int8_t* q, int64_t ldq, float* s, int M, int K,
                             hipStream_t st);
hipError_t launch_quant_fp8(const void* x, int64_t ldx, int xdt, uint8_t* q, int64_t ldq, float* s, int M, int K,
                            const float* static_scale, const void* rms_w, int wdt, float eps, int fuse,
                            hipStream_t st);
hipError_t launch_quant_fp8_block(const void* x, int64_t ldx, int xdt, uint8_t* q, int64_t ldq, float* s,
                                  int64_t lds, int M, int K, int bm, int bk, const float* static_scale,
                                  hipStream_t st);
}  // namespace fg

namespace fg {

namespace {
thread_local char g_kernel[160];
}

void note_kernel(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_kernel, sizeof(g_kernel), fmt, ap);
  va_end(ap);
}

}  // namespace fg

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return FG_OK;
  return fail(FG_EHIP, "%s: %s", what, hipGetErrorString(e));
}

bool is_float_dt(int dt) { return dt == FG_F32 || dt == FG_F16 || dt == FG_BF16; }

constexpr int64_t kMaxDim = (int64_t)1 << 31;

// W8A8 tile policy.  tile_m = 256 (config or automatic) selects the 256-row direct-to-LDS kernel; tile_m = 64 / 128
// select 64- / 128-row tiles: the ring kernel (direct-to-LDS loads, several slices in flight) wherever the 256-row
// kernel's conditions hold (K % 128 == 0, 16-byte aligned operands with 16-byte multiple leading dimensions), with
// tile_n (32, 64, 128; 128 only for 128-row tiles) or mm_ring_bn choosing the width, else the register-staged tiled
// kernel with square tiles.  Tile 16 selects the skinny kernel (M <= 64, K % 256 == 0, same alignment;
// register-resident split-K).  Returns the tile (16, 64, 128, 256) and sets *ring when the ring kernel runs; -1 for a
// configuration the operands do not allow, -2 for a tile_m outside 0 / 16 / 64 / 128 / 256.
int mm_tile(int64_t M, int64_t N, int64_t K, bool int8, const void* a, int64_t lda, const void* b, int64_t ldb,
            const fg_mm_config* cfg, bool* ring) {
  const bool big_ok = fg::mm_big_ok(a, lda, b, ldb, K);
  const bool skinny_ok = fg::w8_skinny_ok(a, lda, b, ldb, M, N, K);
  *ring = false;
  if (cfg && cfg->tile_m) {
    const int t = cfg->tile_m, tn = cfg->tile_n;
    if (t != 16 && t != 64 && t != 128 && t != 256) return -2;
    if ((t == 256 && !big_ok) || (t == 16 && !skinny_ok)) return -1;
    if (t == 64 || t == 128) {
      if (tn && (!big_ok || (t == 64 && tn != 32 && tn != 64 && tn != 128) || (t == 128 && tn != 128))) return -1;
      *ring = big_ok;
    }
    return t;
  }
  if (big_ok) {
    // Measured on the configs' shapes (us, bf16 output, random operands):
    //  * the skinny kernel for M <= 16 at K >= 16384 (int8 K=28672, N=8192: 45 / 56 at M = 1 / 16 against 58 / 60 for
    //    the ring kernel), and for M <= 32 where the ring's 64 x 32 tiles would not cover the CUs (int8 K=14336,
    //    N=4096: 15.3 / 22.6 / 26.0 at M = 4 / 24 / 32 against 29.6-30.1; fp8 K=N=4096: 6.8 / 9.0 against 9.6 / 9.8 at
    //    M = 4 / 24, level at 32, behind from 48); with the CUs covered the ring kernel is ahead from M = 1 (int8 K=8192,
    //    N=10240: 20 against 27; fp8 N=8192 at M=16: 17 against 19; int8 N=57344: 96 against 112; K=4096, N=14336 or
    //    28672: 15.8 / 27.8 against 19.1 / 32.7 at M = 4), and at M = 32..64 everywhere (int8 K=28672, M=64: 63
    //    against 139);
    //  * the 256-row kernel once its tiles number 5/8 of the CUs, whatever M (int8 M=1024, K=8192, N=10240: 160 tiles,
    //    113 against 130 for 128-row ring tiles; K=8192, M=160..224, N=57344: 224 tiles, 146-150 against 180-186
    //    int8 and 150-156 against 168-180 fp8; M=300..448, N=28672: 118-128 against 131-177; M=640, N=14336: 168
    //    tiles, 102 against 120); at 112-128 tiles the ring is ahead (fp8 M=1024, K=N=8192, 89 against 117; int8
    //    K=28672, N=8192, 297 against 353; K=8192, N=28672, M=160..224, 110-124 against 88-96);
    //  * below that the ring kernel: 128-row tiles once they number 5/8 of the CUs (fp8 M=512: 256 tiles, 47 against
    //    62 for 64 x 128) unless 64 x 128 tiles fit one per CU (int8 K=8192, N=10240, M=160..192: 240 tiles, 34-35
    //    against 41; M=224: 320 tiles, 57 against 43), else 64-row tiles (fp8 M=256: 33 against 65 for the
    //    register-staged 64 x 64 tiles).
    const int64_t tiles = fg::mm_big_tiles(M, N), cus = fg::device_cus();
    if (skinny_ok && ((M <= 16 && K >= 16384) || (M <= 32 && (N + 31) / 32 < cus))) return 16;
    if (8 * tiles >= 5 * cus) return 256;
    *ring = true;
    const int64_t t128 = ((M + 127) / 128) * ((N + 127) / 128), t64 = ((M + 63) / 64) * ((N + 127) / 128);
    return (M > 64 && 8 * t128 >= 5 * cus && t64 > cus) ? 128 : 64;
  }
  // Unaligned operands or K % 128 != 0: the skinny kernel where it applies and was measured faster, else the
  // register-staged tiles (64-row while 128-row tiles would leave fewer than two per CU).
  if (skinny_ok && N < 32768 && (M <= 16 || N < 16384) && !(int8 && M > 32 && K < 16384)) return 16;
  const int64_t tiles128 = ((M + 127) / 128) * ((N + 127) / 128);
  return (M <= 64 || N <= 64 || tiles128 < 512) ? 64 : 128;
}

}  // namespace

extern "C" {

const char* fg_version(void) { return "forge_mi355x 0.1.0 (gfx950)"; }

const char* fg_last_error(void) { return g_err.c_str(); }

const char* fg_last_kernel(void) { return fg::g_kernel; }

int fg_device_ok(int device) {
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) {
    fail(FG_EHIP, "hipGetDeviceProperties(%d): %s", device, hipGetErrorString(e));
    return 0;
  }
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    fail(FG_EUNSUPPORTED, "device %d is %s; this library is built for gfx950 only", device, prop.gcnArchName);
    return 0;
  }
  return 1;
}

}  // extern "C"

namespace {

// Rows of x from which the policy takes the prefill kernel (64/128/256-row tiles, split-K) over the skinny MFMA
// kernel: measured on the Llama-3-8B shapes, the skinny kernel wins up to 32 rows (and to 64 rows for N, K <= 4096),
// the prefill kernel from 48 rows (gate+up at M = 64: 1.10 against 0.60 TB/s).
constexpr int64_t kPrefillMinM = 33;
// Whether the automatic policy sends a 4..64-row call to the LDS-ring kernel (portable_row weights): 17..64 rows,
// 4..16 over N >= 16384 and 9..16 over K >= 8192 (fg::w4_ring_preferred; measured on the Llama-3-8B shapes, us, ring
// / previous choice: M = 64 qkv 17.8 / 22.4, o_proj 15.1 / 20.4, gate+up 37.8 / 51.3, down 25.4 / 32.6; M = 32
// gate+up 31.4 / 44.4; M = 16 down 14.4 / 20.3; M = 4 gate+up 22.0 / 23.8), when its shape conditions can hold
// (N % 16 == 0, K % 128 == 0, group % 128 == 0 or one group); the operands decide the rest at launch.
bool ring_policy(const fg_w4_config* cfg, int64_t M, int64_t N, int64_t K) {
  return (!cfg || (cfg->impl == FG_W4_AUTO && !cfg->tile_m && !cfg->split_k)) && M <= 64 && N % 16 == 0 &&
         K % 128 == 0 && fg::w4_ring_preferred(true, (int)M, (int)N, (int)K);
}

// Prefill kernel among those whose conditions hold (pp: ping-pong 256 x 256, pc: producer / consumer 256 x 128, big:
// the all-rounder), 2 / 4 / 5 as in the launch switch; 1 (skinny) when `skinny_first`.  tile_n = 256 / 128 / 64
// forces ping-pong / producer-consumer / all-rounder.  Otherwise from 256 rows: the ping-pong kernel once its tiles
// come near one per CU (>= 160 of 256 x 256), else the producer / consumer kernel (graph replays over four distinct
// weights, us, ping-pong / producer-consumer / all-rounder: M = 512 qkv 53.0 / 50.4 / 60.5, o_proj 48.1 / 36.9 / 40.9,
// gate+up 114.6 / 138.6 / 135.1, down 87.4 / 75.0 / 96.9; M = 2048 qkv 108.9 / 135.2 / 131.0, o_proj 98.3 / 78.4 /
// 93.4, gate+up 449.5 / 501.7 / 502.3, down 234.8 / 232.5 / 297.4; M = 8192 qkv 367 / 434 / 413, o_proj 246 / 294 /
// 273, gate+up 1624 / 1916 / 1799, down 779 / 894 / 878); below 256 rows the all-rounder.
constexpr int64_t kPpMinTiles = 160;
int64_t pp_tiles(int64_t M, int64_t N) { return ((M + 255) / 256) * ((N + 255) / 256); }
int prefill_kernel(int tile_n, int64_t M, int64_t N, bool pp, bool pc, bool big, bool skinny_first) {
  if (tile_n == 256 && pp) return 5;
  if (tile_n == 128 && pc) return 4;
  if (tile_n == 64 && big) return 2;
  if (skinny_first) return 1;
  if (M >= 256 && pp && pp_tiles(M, N) >= kPpMinTiles) return 5;
  if (M >= 256 && pc) return 4;
  return big ? 2 : 0;
}

// W8A16 has no producer / consumer kernel.  Below kPpMinTiles tiles from 256 rows, the ping-pong kernel with its K
// split two or four ways (the fewest that bring tiles x splits to kPpMinTiles) still beats the all-rounder; where four
// ways stay short of it, the all-rounder wins (graph replays over four distinct weights, us, all-rounder / ping-pong
// split 2 / split 4: qkv M = 512 65.7 / 66.3 / 51.2, M = 1024 86.9 / 77.8 / 90.9; o_proj M = 512 44.8 / 62.8 / 46.0,
// M = 1024 67.1 / 70.4 / 61.3, M = 2048 96.4 / 93.8 / 114.2; down M = 512 95.4 / 163.8 / 98.9, M = 1024 159.0 /
// 174.9 / 133.7, M = 2048 262.8 / 228.5 / 243.6).  Returns that split, 1 from kPpMinTiles tiles, 0 for the
// all-rounder.
int w8_pp_split(int64_t M, int64_t N) {
  if (M < 256) return 0;
  const int64_t t = pp_tiles(M, N);
  return t >= kPpMinTiles ? 1 : (2 * t >= kPpMinTiles ? 2 : (4 * t >= kPpMinTiles ? 4 : 0));
}

// Split-K workspace of the prefill kernel prefill_kernel picks for this shape and tile_n (for W8A16 also the split
// ping-pong launch w8_pp_split picks), and of those it falls back to when the operands rule a kernel out at launch
// (the ping-pong kernel falls back to the producer / consumer kernel, W4 only, and both to the all-rounder).
size_t prefill_workspace_bytes(int tile_n, int64_t M, int64_t N, int64_t K, int split_k, bool w4) {
  const bool pp = tile_n == 256 || (tile_n == 0 && M >= 256 && pp_tiles(M, N) >= kPpMinTiles);
  const bool pc = w4 && (tile_n == 128 || tile_n == 256 || (tile_n == 0 && M >= 256));
  size_t b = fg::w4_big_workspace_bytes((int)M, (int)N, (int)K, split_k, !w4);
  if (pp) b = std::max(b, fg::w4_pp_workspace_bytes((int)M, (int)N, (int)K, split_k));
  if (!w4 && tile_n == 0 && w8_pp_split(M, N) > 1)
    b = std::max(b, fg::w4_pp_workspace_bytes((int)M, (int)N, (int)K, split_k > 0 ? split_k : w8_pp_split(M, N)));
  if (pc) b = std::max(b, fg::w4_pc_workspace_bytes((int)M, (int)N, (int)K, split_k));
  return b;
}

// Kernel choice and launch shape for one W4A16 call; fg_w4a16_workspace_bytes and fg_w4a16_gemm share it so the
// workspace a caller sizes is the workspace the launch uses.
struct W4Plan {
  int impl;
  int gemv, mt, rows, max_blocks;  // GEMV: FG_GEMV_* kernel, rows of x per pass, wave-kernel knobs
  int tile_m, splits;              // MFMA
  size_t ws_bytes;
};

int plan_w4(int64_t M, int64_t N, int64_t K, int32_t group_size, bool x_aligned, bool q_aligned, bool has_g_idx,
            const fg_w4_config* cfg, W4Plan* p) {
  const int gs = group_size > 0 ? group_size : (int)K;
  const int impl = cfg ? cfg->impl : FG_W4_AUTO;
  const int G = (int)((K + gs - 1) / gs);
  const int mt = M <= 1 ? 1 : (M <= 2 ? 2 : 4);
  const bool gemv_shape = !has_g_idx && q_aligned && (gs % 32 == 0 || G == 1) && M <= 4;
  const bool split_fits = fg::w4_gemv_split_ok(mt, (int)N, (int)K);
  const bool tile_fits = fg::w4_gemv_tile_ok(mt, (int)N, (int)K, G, cfg ? cfg->tile_n : 0);
  const bool wave_fits = fg::w4_gemv_lds_bytes(4, (int)K) <= 150 * 1024;
  int gemv = cfg ? cfg->gemv_kernel : FG_GEMV_AUTO;
  if (gemv == FG_GEMV_AUTO && cfg && cfg->rows_per_wave) gemv = FG_GEMV_WAVE;
  if (gemv == FG_GEMV_AUTO && cfg && cfg->tile_n) gemv = FG_GEMV_TILE;
  if (gemv < FG_GEMV_AUTO || gemv > FG_GEMV_WAVE) return fail(FG_EINVAL, "fg_w4a16_gemm: unknown gemv_kernel %d", gemv);
  // AUTO is resolved at launch, where the operand addresses decide between the split and the tiled kernel
  const bool gemv_ok = gemv_shape && (gemv == FG_GEMV_SPLIT   ? split_fits
                                      : gemv == FG_GEMV_TILE  ? tile_fits
                                      : gemv == FG_GEMV_WAVE  ? wave_fits
                                                              : (split_fits || tile_fits || wave_fits));
  const bool mfma_ok = !has_g_idx && q_aligned && x_aligned && (K % 8 == 0);
  // the prefill kernel's shape conditions (an act-order perm, known only at launch, sends the call to MFMA instead)
  const bool prefill_ok = mfma_ok && (K % 64 == 0) && (gs % 32 == 0 || G == 1);
  // FG_W4_DEQUANT_GEMM (the reference's dequant_matmul) names the prefill kernels: they dequantise tiles into LDS and
  // feed them to bf16 / fp16 MFMA, the two steps of that route fused
  int use = impl == FG_W4_DEQUANT_GEMM ? FG_W4_PREFILL : impl;
  if (use == FG_W4_AUTO)
    use = gemv_ok ? FG_W4_GEMV : (prefill_ok && M >= kPrefillMinM ? FG_W4_PREFILL : (mfma_ok ? FG_W4_MFMA : FG_W4_GENERIC));
  if (use == FG_W4_PREFILL && !prefill_ok)
    return fail(FG_EUNSUPPORTED, "fg_w4a16_gemm: prefill kernel needs K%%64==0, group%%32==0 (or one group), no g_idx, "
                                 "ldq%%4==0, ldx%%8==0 and 16-byte aligned x/qweight");
  if (use == FG_W4_GEMV && !gemv_ok)
    return fail(FG_EUNSUPPORTED, "fg_w4a16_gemm: GEMV kernel %d needs M<=4, no g_idx, group%%32==0, ldq%%4==0, "
                                 "aligned qweight and a K / N it covers", gemv);
  if (use == FG_W4_MFMA && !mfma_ok)
    return fail(FG_EUNSUPPORTED, "fg_w4a16_gemm: MFMA path needs no g_idx, K%%8==0, ldq%%4==0, ldx%%8==0 and "
                                 "16-byte aligned x/qweight");
  if (use != FG_W4_GEMV && use != FG_W4_MFMA && use != FG_W4_GENERIC && use != FG_W4_PREFILL)
    return fail(FG_EINVAL, "fg_w4a16_gemm: unknown impl %d", impl);
  *p = W4Plan{use, gemv, mt, 4, 0, 0, 1, 0};
  if (use == FG_W4_GEMV) {
    p->rows = cfg && cfg->rows_per_wave ? cfg->rows_per_wave : 4;
    if (p->rows != 1 && p->rows != 2 && p->rows != 4) return fail(FG_EINVAL, "fg_w4a16_gemm: rows_per_wave must be 1, 2 or 4");
    p->max_blocks = cfg ? cfg->max_blocks : 0;
  } else if (use == FG_W4_MFMA || use == FG_W4_PREFILL) {
    p->tile_m = cfg ? cfg->tile_m : 0;
    int kchunk = 0, used = 1;
    fg::w4_mfma_split_plan((int)M, (int)N, (int)K, p->tile_m, cfg ? cfg->split_k : 0, &kchunk, &used);
    p->splits = cfg && cfg->split_k ? cfg->split_k : 0;
    const size_t wm = used > 1 ? (size_t)used * (size_t)M * (size_t)N * sizeof(float) : 0;
    if (wm > p->ws_bytes) p->ws_bytes = wm;
    // the launch picks among the skinny, prefill and tiled MFMA kernels once the operand addresses are known (an
    // act-order perm or misaligned operands rule some out): size the workspace for either split-K kernel
    if (prefill_ok) {
      const size_t wb = prefill_workspace_bytes(cfg ? cfg->tile_n : 0, M, N, K, p->splits, true);
      if (wb > p->ws_bytes) p->ws_bytes = wb;
    }
    // ... and for the LDS-ring kernel when the policy sends the call there
    if (ring_policy(cfg, M, N, K)) {
      const size_t wr = fg::w4_ring_workspace_bytes(true, (int)M, (int)N, (int)K);
      if (wr > p->ws_bytes) p->ws_bytes = wr;
    }
  }
  return FG_OK;
}

}  // namespace

extern "C" {

size_t fg_w4a16_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t group_size, int32_t x_aligned,
                                int32_t q_aligned, int32_t has_g_idx, const fg_w4_config* cfg) {
  if (M <= 0 || N <= 0 || K <= 0 || M >= kMaxDim || N >= kMaxDim || K >= kMaxDim) return 0;
  W4Plan p;
  if (plan_w4(M, N, K, group_size, x_aligned != 0, q_aligned != 0, has_g_idx != 0, cfg, &p) != FG_OK) return 0;
  return p.ws_bytes;
}

}  // extern "C"

namespace {

// fg_w4a16_gemm and fg_w4a16_gemm_noalloc: validation, plan and launch.  `static_ws` marks the library's own scratch
// buffer as the workspace (a plan that needs more than it holds is rejected rather than served by an allocation).
int w4a16_run(const void* x, int64_t ldx, int x_dtype, const int32_t* qweight, int64_t ldq, const void* scales,
              int scale_dtype, int64_t lds, const int32_t* zeros, int64_t ldz, const int32_t* perm,
              const int32_t* g_idx, const void* bias, int bias_dtype, void* y, int64_t ldy, int64_t M, int64_t N,
              int64_t K, int32_t group_size, int32_t n_groups, const fg_w4_config* cfg, void* workspace,
              size_t workspace_bytes, fg_stream_t stream, bool static_ws) {
  if (M < 0 || N <= 0 || K <= 0 || M >= kMaxDim || N >= kMaxDim || K >= kMaxDim)
    return fail(FG_EINVAL, "fg_w4a16_gemm: bad sizes M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
  if (M == 0) return FG_OK;
  if (x_dtype != FG_BF16 && x_dtype != FG_F16) return fail(FG_EUNSUPPORTED, "fg_w4a16_gemm: x must be bf16 or fp16");
  if (!is_float_dt(scale_dtype)) return fail(FG_EINVAL, "fg_w4a16_gemm: bad scale dtype %d", scale_dtype);
  if (bias && !is_float_dt(bias_dtype)) return fail(FG_EINVAL, "fg_w4a16_gemm: bad bias dtype %d", bias_dtype);
  if (!x || !qweight || !scales || !y) return fail(FG_EINVAL, "fg_w4a16_gemm: null tensor");
  const int64_t KW = (K + 7) / 8;
  const int gs = group_size > 0 ? group_size : (int)K;
  const int64_t G = (K + gs - 1) / gs;
  if (group_size > 0 && group_size % 8 != 0)
    return fail(FG_EINVAL, "fg_w4a16_gemm: group_size must be a multiple of 8 or <= 0, got %d", group_size);
  if (ldq < KW || lds < N || ldx < K || ldy < N || (zeros && ldz < (N + 7) / 8))
    return fail(FG_EINVAL, "fg_w4a16_gemm: leading dimensions too small");
  if (n_groups <= 0 || (!g_idx && n_groups < G))
    return fail(FG_EINVAL, "fg_w4a16_gemm: n_groups=%d does not cover K=%lld with group %d", n_groups, (long long)K, gs);

  const bool x_aligned = (ldx % 8 == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0);
  const bool q_aligned = (ldq % 4 == 0) && (reinterpret_cast<uintptr_t>(qweight) % 16 == 0);
  W4Plan p;
  const int rc = plan_w4(M, N, K, group_size, x_aligned, q_aligned, g_idx != nullptr, cfg, &p);
  if (rc != FG_OK) return rc;
  if (static_ws && p.ws_bytes > workspace_bytes)
    return fail(FG_EINVAL, "fg_w4a16_gemm_noalloc: this launch needs %zu bytes of split-K scratch, the library's static "
                           "buffer holds %zu (FG_W4A16_SCRATCH_BYTES); call fg_w4a16_gemm with a workspace instead",
                p.ws_bytes, workspace_bytes);
  if (p.ws_bytes > 0 && (workspace == nullptr || workspace_bytes < p.ws_bytes))
    return fail(FG_EINVAL, "fg_w4a16_gemm: workspace of %zu bytes needed, %zu given", p.ws_bytes,
                workspace ? workspace_bytes : (size_t)0);

  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool xbf16 = x_dtype == FG_BF16;
  hipError_t e;
  // 3-4 rows over weights larger than 4096 x 4096: the skinny MFMA kernel where it applies (it needs no workspace).
  // Measured at M = 4 (us): qkv 8.2 against 8.7 for the GEMV, gate+up 20.5 against 22.8, down 14.8 against 16.2;
  // o_proj (4096 x 4096) 6.8 against 6.1 stays on the GEMV, as do 1-2 rows.
  if (p.impl == FG_W4_GEMV && p.gemv == FG_GEMV_AUTO && (!cfg || cfg->impl == FG_W4_AUTO) && M > 2 &&
      N * K > 4096LL * 4096 &&
      fg::w4_skinny_ok(x, ldx, qweight, ldq, perm, scale_dtype, lds, zeros ? ldz : 0, (int)M, N, K, gs, G))
    p.impl = FG_W4_MFMA;
  if (p.impl == FG_W4_GEMV && p.gemv == FG_GEMV_AUTO) {
    // the split kernel in its branch-free form, else the tiled kernel, else whichever covers the shape
    if (fg::w4_gemv_split_preferred(p.mt, x, ldx, perm, scales, scale_dtype, lds, ldq, zeros, ldz, (int)M, (int)N,
                                    (int)K, gs, G == 1))
      p.gemv = FG_GEMV_SPLIT;
    else if (fg::w4_gemv_tile_ok(p.mt, (int)N, (int)K, (int)G, 0))
      p.gemv = FG_GEMV_TILE;
    else
      p.gemv = fg::w4_gemv_split_ok(p.mt, (int)N, (int)K) ? FG_GEMV_SPLIT : FG_GEMV_WAVE;
  }
  if (p.impl == FG_W4_GEMV && p.gemv == FG_GEMV_SPLIT) {
    e = fg::launch_w4_gemv_split(p.mt, xbf16, x, ldx, qweight, ldq, scales, scale_dtype, lds, zeros, ldz, perm, bias,
                                 bias_dtype, y, ldy, (int)M, (int)N, (int)K, gs, G == 1, s);
  } else if (p.impl == FG_W4_GEMV && p.gemv == FG_GEMV_TILE) {
    e = fg::launch_w4_gemv_tile(p.mt, xbf16, x, ldx, qweight, ldq, scales, scale_dtype, lds, zeros, ldz, perm, bias,
                                bias_dtype, y, ldy, (int)M, (int)N, (int)K, gs, (int)G, cfg ? cfg->tile_n : 0, s);
  } else if (p.impl == FG_W4_GEMV) {
    e = fg::launch_w4_gemv(p.mt, p.rows, xbf16, x, ldx, qweight, ldq, scales, scale_dtype, lds, zeros, ldz, perm, bias,
                           bias_dtype, y, ldy, (int)M, (int)N, (int)K, gs, p.max_blocks, s);
  } else if (p.impl == FG_W4_MFMA || p.impl == FG_W4_PREFILL) {
    const bool auto_impl = !cfg || cfg->impl == FG_W4_AUTO;
    const bool skinny = !(cfg && (cfg->tile_m || cfg->split_k)) &&
                        fg::w4_skinny_ok(x, ldx, qweight, ldq, perm, scale_dtype, lds, zeros ? ldz : 0, (int)M, N, K,
                                         gs, G);
    const bool big = fg::w4_big_ok(x, ldx, qweight, ldq, perm, K, gs, G) && !(cfg && cfg->tile_m);
    const bool pc = fg::w4_pc_ok(x, ldx, qweight, ldq, perm, scales, scale_dtype, lds, N, K, gs, G) &&
                    !(cfg && cfg->tile_m);
    const bool pp = fg::w4_pp_ok(x, ldx, qweight, ldq, perm, scales, scale_dtype, lds, zeros, zeros ? ldz : 0, M, N,
                                 K, gs, G) &&
                    !(cfg && cfg->tile_m);
    // 0: LDS-tiled MFMA, 1: skinny, 2: all-round prefill, 3: LDS ring, 4: producer / consumer prefill, 5: ping-pong
    // prefill
    int kern = 0;
    if (p.impl == FG_W4_PREFILL)
      kern = prefill_kernel(cfg ? cfg->tile_n : 0, M, N, pp, pc, big,
                            auto_impl && skinny && M <= 64 && N <= 4096 && K <= 4096);
    else
      kern = skinny ? 1 : ((auto_impl && big) ? 2 : 0);
    if (ring_policy(cfg, M, N, K) && perm == nullptr &&
        fg::w4_ring_ok(true, x, ldx, qweight, ldq, scales, scale_dtype, lds, zeros, zeros ? ldz : 0, (int)M, N, K, gs,
                       G) &&
        (fg::w4_ring_workspace_bytes(true, (int)M, (int)N, (int)K) == 0 ||
         (workspace && reinterpret_cast<uintptr_t>(workspace) % 16 == 0)))
      kern = 3;
    if (kern == 3)
      e = fg::launch_w4_ring(true, x, ldx, xbf16, qweight, ldq, scales, scale_dtype, lds, zeros, ldz, bias,
                             bias_dtype, y, ldy, (int)M, (int)N, (int)K, gs, G == 1, (int)G, workspace,
                             workspace_bytes, s);
    else if (kern == 1)
      e = fg::launch_w4_skinny(x, ldx, xbf16, qweight, ldq, scales, scale_dtype, lds, zeros, ldz, bias, bias_dtype, y,
                               ldy, (int)M, (int)N, (int)K, gs, G == 1, s);
    else if (kern == 5)
      e = fg::launch_w4_pp(x, ldx, xbf16, qweight, ldq, scales, scale_dtype, lds, zeros, ldz, bias, bias_dtype, y, ldy,
                           static_cast<float*>(workspace), (int)M, (int)N, (int)K, gs, G == 1, p.splits, s);
    else if (kern == 4)
      e = fg::launch_w4_pc(x, ldx, xbf16, qweight, ldq, scales, scale_dtype, lds, zeros, ldz, bias, bias_dtype, y, ldy,
                           static_cast<float*>(workspace), (int)M, (int)N, (int)K, gs, G == 1, p.splits, s);
    else if (kern == 2)
      e = fg::launch_w4_big(x, ldx, xbf16, qweight, ldq, scales, scale_dtype, lds, zeros, ldz, bias, bias_dtype, y,
                            ldy, static_cast<float*>(workspace), (int)M, (int)N, (int)K, gs, G == 1, p.splits, s);
    else
      e = fg::launch_w4_mfma(x, ldx, xbf16, qweight, ldq, scales, scale_dtype, lds, zeros, ldz, perm, bias,
                             bias_dtype, y, ldy, static_cast<float*>(workspace), (int)M, (int)N, (int)K, gs, p.tile_m,
                             p.splits, s);
  } else {
    e = fg::launch_w4_generic(x, ldx, x_dtype, qweight, ldq, scales, scale_dtype, lds, zeros, ldz, perm, g_idx, bias,
                              bias_dtype, y, ldy, (int)M, (int)N, (int)K, gs, s);
  }
  return hip_status(e, static_ws ? "fg_w4a16_gemm_noalloc launch" : "fg_w4a16_gemm launch");
}

// Split-K scratch of fg_w4a16_gemm_noalloc: one copy per GPU, placed by the code object loader (no hipMalloc).  The
// kernels write every element of the partials they later reduce, so nothing in it needs clearing between calls.
static __device__ __align__(256) unsigned char scratch[FG_W4A16_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
std::atomic<void*> g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the current device, looked up once per device with that device current.  The
// array's name is a host-side stand-in; only this address may reach a kernel or a copy.
int scratch_of_current_device(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, "fg_w4a16_gemm_noalloc: hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(FG_EUNSUPPORTED, "fg_w4a16_gemm_noalloc: device %d out of range", dev);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || p == nullptr)
        return hip_status(e != hipSuccess ? e : hipErrorInvalidSymbol,
                          "fg_w4a16_gemm_noalloc: hipGetSymbolAddress(scratch)");
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return FG_OK;
}

}  // namespace

extern "C" {

int fg_w4a16_gemm(const void* x, int64_t ldx, int x_dtype, const int32_t* qweight, int64_t ldq, const void* scales,
                  int scale_dtype, int64_t lds, const int32_t* zeros, int64_t ldz, const int32_t* perm,
                  const int32_t* g_idx, const void* bias, int bias_dtype, void* y, int64_t ldy, int64_t M, int64_t N,
                  int64_t K, int32_t group_size, int32_t n_groups, const fg_w4_config* cfg, void* workspace,
                  size_t workspace_bytes, fg_stream_t stream) {
  return w4a16_run(x, ldx, x_dtype, qweight, ldq, scales, scale_dtype, lds, zeros, ldz, perm, g_idx, bias, bias_dtype,
                   y, ldy, M, N, K, group_size, n_groups, cfg, workspace, workspace_bytes, stream, false);
}

int fg_w4a16_gemm_noalloc(const void* x, int64_t ldx, int x_dtype, const int32_t* qweight, int64_t ldq,
                          const void* scales, int scale_dtype, int64_t lds, const int32_t* zeros, int64_t ldz,
                          const int32_t* perm, const int32_t* g_idx, const void* bias, int bias_dtype, void* y,
                          int64_t ldy, int64_t M, int64_t N, int64_t K, int32_t group_size, int32_t n_groups,
                          const fg_w4_config* cfg, fg_stream_t stream) {
  void* ws = nullptr;
  const int rc = scratch_of_current_device(&ws);
  if (rc != FG_OK) return rc;
  return w4a16_run(x, ldx, x_dtype, qweight, ldq, scales, scale_dtype, lds, zeros, ldz, perm, g_idx, bias, bias_dtype,
                   y, ldy, M, N, K, group_size, n_groups, cfg, ws, FG_W4A16_SCRATCH_BYTES, stream, true);
}

size_t fg_w4a16_cdna4_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t group_size) {
  (void)group_size;
  if (M <= 0 || M > 64 || N <= 0 || K <= 0 || N >= kMaxDim || K >= kMaxDim) return 0;
  return fg::w4_ring_workspace_bytes(false, (int)M, (int)N, (int)K);
}

int fg_w4a16_gemm_cdna4(const void* x, int64_t ldx, int x_dtype, const int32_t* qweight, int64_t ldq,
                        const void* scales, int scale_dtype, int64_t lds, const int32_t* zeros, int64_t ldz,
                        const void* bias, int bias_dtype, void* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                        int32_t group_size, int32_t n_groups, void* workspace, size_t workspace_bytes,
                        fg_stream_t stream) {
  if (M < 0 || N <= 0 || K <= 0 || M >= kMaxDim || N >= kMaxDim || K >= kMaxDim)
    return fail(FG_EINVAL, "fg_w4a16_gemm_cdna4: bad sizes M=%lld N=%lld K=%lld", (long long)M, (long long)N,
                (long long)K);
  if (M == 0) return FG_OK;
  if (x_dtype != FG_BF16 && x_dtype != FG_F16)
    return fail(FG_EUNSUPPORTED, "fg_w4a16_gemm_cdna4: x must be bf16 or fp16");
  if (!is_float_dt(scale_dtype)) return fail(FG_EINVAL, "fg_w4a16_gemm_cdna4: bad scale dtype %d", scale_dtype);
  if (bias && !is_float_dt(bias_dtype)) return fail(FG_EINVAL, "fg_w4a16_gemm_cdna4: bad bias dtype %d", bias_dtype);
  if (!x || !qweight || !scales || !y) return fail(FG_EINVAL, "fg_w4a16_gemm_cdna4: null tensor");
  const int gs = group_size > 0 ? group_size : (int)K;
  const int64_t G = (K + gs - 1) / gs;
  if (group_size > 0 && group_size % 8 != 0)
    return fail(FG_EINVAL, "fg_w4a16_gemm_cdna4: group_size must be a multiple of 8 or <= 0, got %d", group_size);
  const int64_t kpad = (K + 127) / 128 * 128;
  if (ldq < 2 * kpad || lds < N || ldx < K || ldy < N || (zeros && ldz < (N + 7) / 8))
    return fail(FG_EINVAL, "fg_w4a16_gemm_cdna4: leading dimensions too small (ldq counts int32 words per 16-channel "
                           "tile row: at least 2 * K rounded up to 128)");
  if (n_groups < G)
    return fail(FG_EINVAL, "fg_w4a16_gemm_cdna4: n_groups=%d does not cover K=%lld with group %d", n_groups,
                (long long)K, gs);
  if (!fg::w4_frag_ok(x, ldx, qweight, ldq, scale_dtype, lds, zeros ? ldz : 0, (int)M, N, K, gs, G))
    return fail(FG_EUNSUPPORTED, "fg_w4a16_gemm_cdna4: needs M <= 64, K %% 128 == 0, group %% 128 == 0 (or one group), "
                                 "16-bit scales, 16-byte aligned x and qweight, ldx %% 8 == 0, ldq %% 4 == 0");
  if (fg::w4_ring_preferred(false, (int)M, (int)N, (int)K) &&
      fg::w4_ring_ok(false, x, ldx, qweight, ldq, scales, scale_dtype, lds, zeros, zeros ? ldz : 0, (int)M, N, K, gs,
                     G)) {
    const size_t need = fg::w4_ring_workspace_bytes(false, (int)M, (int)N, (int)K);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need || reinterpret_cast<uintptr_t>(workspace) % 16))
      return fail(FG_EINVAL, "fg_w4a16_gemm_cdna4: needs a 16-byte aligned workspace of %zu bytes, got %zu", need,
                  workspace ? workspace_bytes : (size_t)0);
    return hip_status(fg::launch_w4_ring(false, x, ldx, x_dtype == FG_BF16, qweight, ldq, scales, scale_dtype, lds, zeros,
                                         ldz, bias, bias_dtype, y, ldy, (int)M, (int)N, (int)K, gs, G == 1, (int)G,
                                         workspace, workspace_bytes, static_cast<hipStream_t>(stream)),
                      "fg_w4a16_gemm_cdna4 launch");
  }
  return hip_status(fg::launch_w4_frag(x, ldx, x_dtype == FG_BF16, qweight, ldq, scales, scale_dtype, lds, zeros, ldz,
                                       bias, bias_dtype, y, ldy, (int)M, (int)N, (int)K, gs, G == 1, (int)G,
                                       static_cast<hipStream_t>(stream)),
                    "fg_w4a16_gemm_cdna4 launch");
}

int fg_w4a16_gemv_sz8(const void* x, int64_t ldx, int x_dtype, const int32_t* qweight, int64_t ldq,
                      const void* scales8, int scale_dtype, const int32_t* zeros8, const void* bias, int bias_dtype,
                      void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, int32_t group_size, int32_t n_groups,
                      fg_stream_t stream) {
  if (M < 0 || N <= 0 || K <= 0 || M >= kMaxDim || N >= kMaxDim || K >= kMaxDim)
    return fail(FG_EINVAL, "fg_w4a16_gemv_sz8: bad sizes M=%lld N=%lld K=%lld", (long long)M, (long long)N,
                (long long)K);
  if (M == 0) return FG_OK;
  if (x_dtype != FG_BF16 && x_dtype != FG_F16) return fail(FG_EUNSUPPORTED, "fg_w4a16_gemv_sz8: x must be bf16 or fp16");
  if (scale_dtype != FG_F16 && scale_dtype != FG_BF16)
    return fail(FG_EUNSUPPORTED, "fg_w4a16_gemv_sz8: scales must be fp16 or bf16");
  if (bias && !is_float_dt(bias_dtype)) return fail(FG_EINVAL, "fg_w4a16_gemv_sz8: bad bias dtype %d", bias_dtype);
  if (!x || !qweight || !scales8 || !y) return fail(FG_EINVAL, "fg_w4a16_gemv_sz8: null tensor");
  const int gs = group_size > 0 ? group_size : (int)K;
  const int64_t G = (K + gs - 1) / gs;
  if (ldq < (K + 7) / 8 || ldx < K || ldy < N) return fail(FG_EINVAL, "fg_w4a16_gemv_sz8: leading dimensions too small");
  // the blocked arrays hold exactly the groups K needs: [N / 8][G][8] scales, [N / 8][G] zero words
  if (n_groups != G)
    return fail(FG_EINVAL, "fg_w4a16_gemv_sz8: n_groups=%d, but K=%lld with group %d has %lld", n_groups,
                (long long)K, gs, (long long)G);
  if (!fg::w4_gemv_sz8_ok(x, ldx, qweight, ldq, scales8, scale_dtype, (int)M, (int)N, (int)K, group_size))
    return fail(FG_EUNSUPPORTED, "fg_w4a16_gemv_sz8: needs M <= 4, N %% 8 == 0, K %% 32 == 0, group %% 32 == 0 (or one "
                                 "group), 16-byte aligned x / qweight / scales, ldx %% 8 == 0, ldq %% 4 == 0 and a "
                                 "split-GEMV plan for the shape");
  const int mt = M <= 1 ? 1 : (M <= 2 ? 2 : 4);
  return hip_status(fg::launch_w4_gemv_sz8(mt, x_dtype == FG_BF16, x, ldx, qweight, ldq, scales8, scale_dtype, zeros8,
                                           bias, bias_dtype, y, ldy, (int)M, (int)N, (int)K, gs, G == 1,
                                           static_cast<hipStream_t>(stream)),
                    "fg_w4a16_gemv_sz8 launch");
}

int fg_w4_dequant(const int32_t* qweight, int64_t ldq, const void* scales, int scale_dtype, int64_t lds,
                  const int32_t* zeros, int64_t ldz, const int32_t* g_idx, void* out, int out_dtype, int64_t ldo,
                  int64_t N, int64_t K, int32_t group_size, int32_t n_groups, fg_stream_t stream) {
  if (N <= 0 || K <= 0 || N >= kMaxDim || K >= kMaxDim) return fail(FG_EINVAL, "fg_w4_dequant: bad sizes");
  if (!qweight || !scales || !out) return fail(FG_EINVAL, "fg_w4_dequant: null tensor");
  if (!is_float_dt(scale_dtype) || !is_float_dt(out_dtype)) return fail(FG_EINVAL, "fg_w4_dequant: bad dtype");
  const int gs = group_size > 0 ? group_size : (int)K;
  if (group_size > 0 && group_size % 8 != 0) return fail(FG_EINVAL, "fg_w4_dequant: group_size must be a multiple of 8");
  if (ldq < (K + 7) / 8 || lds < N || ldo < K || (zeros && ldz < (N + 7) / 8))
    return fail(FG_EINVAL, "fg_w4_dequant: leading dimensions too small");
  if (n_groups <= 0 || (!g_idx && n_groups < (K + gs - 1) / gs))
    return fail(FG_EINVAL, "fg_w4_dequant: n_groups does not cover K");
  return hip_status(fg::launch_w4_dequant(qweight, ldq, scales, scale_dtype, lds, zeros, ldz, g_idx, out, out_dtype,
                                          ldo, (int)N, (int)K, gs, static_cast<hipStream_t>(stream)),
                    "fg_w4_dequant launch");
}

// Whether the automatic W8A16 policy takes the LDS-ring kernel (when its conditions hold): 17..64 rows, and 3..16 rows
// over wide or long weights.  Graph replays over a 1.2 GB weight ring, us, ring / skinny: M = 64 qkv 18.4 / 37.9,
// o_proj 14.4 / 21.1, gate+up 44.4 / 143.5, down 27.2 / 61.2; M = 32 13.9 / 16.1, 10.9 / 13.0, 31.5 / 51.9,
// 21.5 / 36.0; M = 16 11.9 / 11.7, 9.5 / 9.1, 26.9 / 30.7, 17.9 / 23.7; M = 3 11.3 / 9.8, 9.3 / 7.5, 28.0 / 29.1,
// 17.1 / 18.3.
static bool w8a16_ring_rows(int64_t M, int64_t N, int64_t K) {
  return M > 16 ? M <= 64 : (M > 2 && (N >= 16384 || K >= 8192));
}

size_t fg_w8a16_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t group_size, const fg_w4_config* cfg) {
  if (M <= 0 || N <= 0 || K <= 0 || M >= kMaxDim || N >= kMaxDim || K >= kMaxDim) return 0;
  const int gs = group_size > 0 ? group_size : (int)K;
  const int64_t G = (K + gs - 1) / gs;
  const int impl = cfg ? cfg->impl : FG_W4_AUTO;
  // the prefill kernels' split-K partials, whenever one may run (their alignment conditions are checked at launch)
  const bool prefill_shape = (K % 64 == 0) && (gs % 32 == 0 || G == 1);
  if (!prefill_shape || impl == FG_W4_GENERIC || impl == FG_W4_MFMA || impl == FG_W4_GEMV) return 0;
  const size_t ring = impl == FG_W4_AUTO && w8a16_ring_rows(M, N, K) ? fg::w8a16_ring_workspace_bytes((int)M, (int)N, (int)K)
                                                               : 0;
  return std::max(ring, prefill_workspace_bytes(cfg ? cfg->tile_n : 0, M, N, K, cfg ? cfg->split_k : 0, false));
}

int fg_w8a16_gemm(const void* x, int64_t ldx, int x_dtype, const int8_t* qweight, int64_t ldq, const void* scales,
                  int scale_dtype, int64_t lds, const void* bias, int bias_dtype, void* y, int64_t ldy, int64_t M,
                  int64_t N, int64_t K, int32_t group_size, int32_t n_groups, const fg_w4_config* cfg,
                  void* workspace, size_t workspace_bytes, fg_stream_t stream) {
  if (M < 0 || N <= 0 || K <= 0 || M >= kMaxDim || N >= kMaxDim || K >= kMaxDim)
    return fail(FG_EINVAL, "fg_w8a16_gemm: bad sizes M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
  if (M == 0) return FG_OK;
  if (x_dtype != FG_BF16 && x_dtype != FG_F16) return fail(FG_EUNSUPPORTED, "fg_w8a16_gemm: x must be bf16 or fp16");
  if (!is_float_dt(scale_dtype)) return fail(FG_EINVAL, "fg_w8a16_gemm: bad scale dtype %d", scale_dtype);
  if (bias && !is_float_dt(bias_dtype)) return fail(FG_EINVAL, "fg_w8a16_gemm: bad bias dtype %d", bias_dtype);
  if (!x || !qweight || !scales || !y) return fail(FG_EINVAL, "fg_w8a16_gemm: null tensor");
  const int gs = group_size > 0 ? group_size : (int)K;
  const int64_t G = (K + gs - 1) / gs;
  if (ldq < K || lds < N || ldx < K || ldy < N) return fail(FG_EINVAL, "fg_w8a16_gemm: leading dimensions too small");
  if (n_groups < G)
    return fail(FG_EINVAL, "fg_w8a16_gemm: n_groups=%d does not cover K=%lld with group %d", n_groups, (long long)K, gs);
  // FG_W4_DEQUANT_GEMM names the prefill kernels, as for W4A16
  const int impl = cfg && cfg->impl == FG_W4_DEQUANT_GEMM ? FG_W4_PREFILL : (cfg ? cfg->impl : FG_W4_AUTO);
  if (impl != FG_W4_AUTO && impl != FG_W4_GEMV && impl != FG_W4_MFMA && impl != FG_W4_PREFILL && impl != FG_W4_GENERIC)
    return fail(FG_EINVAL, "fg_w8a16_gemm: unknown impl %d", cfg->impl);
  const bool xbf16 = x_dtype == FG_BF16;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool gemv = fg::w8a16_gemv_ok(x, ldx, qweight, ldq, scales, scale_dtype, lds, M, N, K, gs, G);
  const bool skinny = fg::w8a16_skinny_ok(x, ldx, qweight, ldq, scale_dtype, lds, M, N, K, gs, G);
  const bool big = fg::w8_big_ok(x, ldx, qweight, ldq, K, gs, G);
  const bool ring = fg::w8a16_ring_ok(x, ldx, qweight, ldq, scales, scale_dtype, lds, M, N, K, gs, G);
  int kern = impl == FG_W4_GENERIC ? 0
             : impl == FG_W4_MFMA  ? 1
             : impl == FG_W4_PREFILL ? 2
             : impl == FG_W4_GEMV  ? 3
                                   : -1;
  // 1..2 rows, and 3..4 over N <= 8192 and K < 8192: the decode GEMV (graph replays, M = 1, us, GEMV / skinny: qkv
  // 6.2 / 9.6, o_proj 5.1 / 8.0, gate+up 20.7 / 28.7, down 12.6 / 17.3; M = 3 / 4 o_proj 6.8 / 7.0 against 7.3 / 7.5,
  // qkv level, gate+up 33.2 against 27.1 on the ring); then the LDS ring (w8a16_ring_rows), else the skinny kernel up
  // to 64 rows
  const bool gemv_rows = M <= 2 || (M <= 4 && N <= 8192 && K < 8192);
  if (kern < 0)
    kern = (gemv && gemv_rows) ? 3 : ((ring && w8a16_ring_rows(M, N, K)) ? 4 : ((skinny && M <= 64) ? 1 : (big ? 2 : 0)));
  if (kern == 3 && !gemv)
    return fail(FG_EUNSUPPORTED, "fg_w8a16_gemm: decode GEMV needs M<=4, K%%16==0, group%%16==0 (or one group), "
                                 "16-bit scales with lds%%8==0, ldq%%16==0, ldx%%8==0, 16-byte aligned x/qweight/"
                                 "scales and N a multiple of its channels per wavefront");
  if (kern == 1 && !skinny)
    return fail(FG_EUNSUPPORTED, "fg_w8a16_gemm: skinny kernel needs M<=64, K%%128==0, group%%128==0 (or one group), "
                                 "16-bit scales, ldq%%16==0, ldx%%8==0 and 16-byte aligned x/qweight");
  if (kern == 2 && !big)
    return fail(FG_EUNSUPPORTED, "fg_w8a16_gemm: prefill kernel needs K%%64==0, group%%32==0 (or one group), "
                                 "ldq%%16==0, ldx%%8==0 and 16-byte aligned x/qweight");
  hipError_t e;
  if (kern == 4) {
    const size_t need = fg::w8a16_ring_workspace_bytes((int)M, (int)N, (int)K);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need))
      return fail(FG_EINVAL, "fg_w8a16_gemm: workspace of %zu bytes needed, %zu given", need,
                  workspace ? workspace_bytes : (size_t)0);
    e = fg::launch_w8a16_ring(x, ldx, xbf16, qweight, ldq, scales, scale_dtype, lds, bias, bias_dtype, y, ldy, (int)M,
                              (int)N, (int)K, gs, G == 1, (int)G, workspace, workspace_bytes, s);
  } else if (kern == 3) {
    e = fg::launch_w8a16_gemv(x, ldx, xbf16, qweight, ldq, scales, scale_dtype, lds, bias, bias_dtype, y, ldy, (int)M,
                              (int)N, (int)K, gs, G == 1, G, s);
  } else if (kern == 1) {
    e = fg::launch_w8a16_skinny(x, ldx, xbf16, qweight, ldq, scales, scale_dtype, lds, bias, bias_dtype, y, ldy,
                                (int)M, (int)N, (int)K, gs, G == 1, s);
  } else if (kern == 2) {
    // the ping-pong kernel or the all-rounder, by the W4A16 rule; where W4A16 would take the producer / consumer
    // kernel (none for int8 weights), the ping-pong kernel with its K split as w8_pp_split says
    const bool pp = fg::w8_pp_ok(x, ldx, qweight, ldq, scales, scale_dtype, lds, M, N, K, gs, G) &&
                    !(cfg && cfg->tile_m);
    const int tn = cfg ? cfg->tile_n : 0;
    int pk = prefill_kernel(tn, M, N, pp, false, big, false);
    int split = cfg ? cfg->split_k : 0;
    if (pk != 5 && pp && tn == 0 && w8_pp_split(M, N) > 1) {
      pk = 5;
      if (split <= 0) split = w8_pp_split(M, N);
    }
    const size_t need = pk == 5 ? fg::w4_pp_workspace_bytes((int)M, (int)N, (int)K, split)
                                : fg::w4_big_workspace_bytes((int)M, (int)N, (int)K, split, true);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need))
      return fail(FG_EINVAL, "fg_w8a16_gemm: workspace of %zu bytes needed, %zu given", need,
                  workspace ? workspace_bytes : (size_t)0);
    if (pk == 5)
      e = fg::launch_w8_pp(x, ldx, xbf16, qweight, ldq, scales, scale_dtype, lds, bias, bias_dtype, y, ldy,
                           static_cast<float*>(workspace), (int)M, (int)N, (int)K, gs, G == 1, split, s);
    else
      e = fg::launch_w8_big(x, ldx, xbf16, qweight, ldq, scales, scale_dtype, lds, bias, bias_dtype, y, ldy,
                            static_cast<float*>(workspace), (int)M, (int)N, (int)K, gs, G == 1, split, s);
  } else {
    e = fg::launch_w8a16_generic(x, ldx, x_dtype, qweight, ldq, scales, scale_dtype, lds, bias, bias_dtype, y, ldy,
                                 (int)M, (int)N, (int)K, gs, s);
  }
  return hip_status(e, "fg_w8a16_gemm launch");
}

int fg_int8_gemm(const int8_t* a, int64_t lda, const float* sa, int64_t sa_len, const int8_t* b, int64_t ldb,
                 const float* sb, int64_t sb_len, const void* bias, int bias_dtype, void* y, int64_t ldy, int y_dtype,
                 int64_t M, int64_t N, int64_t K, const fg_mm_config* cfg, fg_stream_t stream) {
  if (M < 0 || N <= 0 || K <= 0 || M >= kMaxDim || N >= kMaxDim || K >= kMaxDim)
    return fail(FG_EINVAL, "fg_int8_gemm: bad sizes");
  if (M == 0) return FG_OK;
  if (!a || !b || !y) return fail(FG_EINVAL, "fg_int8_gemm: null tensor");
  if (y_dtype != FG_I32) {
    if (!is_float_dt(y_dtype)) return fail(FG_EINVAL, "fg_int8_gemm: bad output dtype %d", y_dtype);
    if (!sa || !sb || (sa_len != 1 && sa_len != M) || (sb_len != 1 && sb_len != N))
      return fail(FG_EINVAL, "fg_int8_gemm: scale sizes %lld/%lld do not match M=%lld/N=%lld", (long long)sa_len,
                  (long long)sb_len, (long long)M, (long long)N);
    if (bias && !is_float_dt(bias_dtype)) return fail(FG_EINVAL, "fg_int8_gemm: bad bias dtype");
  }
  if (lda < K || ldb < K || ldy < N) return fail(FG_EINVAL, "fg_int8_gemm: leading dimensions too small");
  if (y_dtype == FG_I32 && bias)
    return fail(FG_EINVAL, "fg_int8_gemm: a bias cannot be added to the raw int32 accumulator (y_dtype FG_I32)");
  // 1..2 rows of A: the decode GEMV (tile_m = 1 forces it)
  const bool gemv = fg::int8_gemv_ok(a, lda, b, ldb, M, N, K);
  if (cfg && cfg->tile_m == 1 && !gemv)
    return fail(FG_EUNSUPPORTED, "fg_int8_gemm: tile_m=1 (decode GEMV) needs M <= 2, K %% 16 == 0, N %% 8 == 0 and "
                                 "16-byte aligned operands with leading dimensions that are multiples of 16");
  if (gemv && ((cfg && cfg->tile_m == 1) || (!(cfg && cfg->tile_m) && M <= 2)))
    return hip_status(fg::launch_int8_gemv(a, lda, sa, sa_len, b, ldb, sb, sb_len, bias, bias_dtype, y, ldy, y_dtype,
                                           (int)M, (int)N, (int)K, static_cast<hipStream_t>(stream)),
                      "fg_int8_gemm launch");
  bool ring;
  const int tile = mm_tile(M, N, K, true, a, lda, b, ldb, cfg, &ring);
  if (tile == -2) return fail(FG_EINVAL, "fg_int8_gemm: tile_m must be 0, 16, 64, 128 or 256, got %d", cfg->tile_m);
  if (tile < 0)
    return fail(FG_EUNSUPPORTED, "fg_int8_gemm: tile_m=256 needs K %% 128 == 0, tile_m=16 M <= 64 and K %% 256 == 0, "
                                 "both 16-byte aligned operands; tile_n (32, 64, 128 for tile_m=64, 128 for "
                                 "tile_m=128) the same");
  if (ring) {
    const int bn = cfg && cfg->tile_n ? cfg->tile_n : fg::mm_ring_bn(M, N, tile);
    return hip_status(fg::launch_int8_gemm_ring(a, lda, sa, sa_len, b, ldb, sb, sb_len, bias, bias_dtype, y, ldy,
                                                y_dtype, (int)M, (int)N, (int)K, tile, bn,
                                                static_cast<hipStream_t>(stream)),
                      "fg_int8_gemm launch");
  }
  if (tile == 16)
    return hip_status(fg::launch_int8_gemm_skinny(a, lda, sa, sa_len, b, ldb, sb, sb_len, bias, bias_dtype, y, ldy,
                                                  y_dtype, (int)M, (int)N, (int)K, static_cast<hipStream_t>(stream)),
                      "fg_int8_gemm launch");
  if (tile == 256)
    return hip_status(fg::launch_int8_gemm_big(a, lda, sa, sa_len, b, ldb, sb, sb_len, bias, bias_dtype, y, ldy,
                                               y_dtype, (int)M, (int)N, (int)K, static_cast<hipStream_t>(stream)),
                      "fg_int8_gemm launch");
  return hip_status(fg::launch_int8_gemm(a, lda, sa, sa_len, b, ldb, sb, sb_len, bias, bias_dtype, y, ldy, y_dtype,
                                         (int)M, (int)N, (int)K, tile, static_cast<hipStream_t>(stream)),
                    "fg_int8_gemm launch");
}

int fg_fp8_gemm(const uint8_t* a, int64_t lda, const float* sa, int64_t sa_sm, int64_t sa_sk, const uint8_t* b,
                int64_t ldb, const float* sb, int64_t sb_sn, int64_t sb_sk, int32_t sb_div, int32_t scale_mode,
                int32_t block, const void* bias, int bias_dtype, void* y, int64_t ldy, int y_dtype, int64_t M,
                int64_t N, int64_t K, const fg_mm_config* cfg, fg_stream_t stream) {
  if (M < 0 || N <= 0 || K <= 0 || M >= kMaxDim || N >= kMaxDim || K >= kMaxDim)
    return fail(FG_EINVAL, "fg_fp8_gemm: bad sizes");
  if (M == 0) return FG_OK;
  if (!a || !b || !y || !sa || !sb) return fail(FG_EINVAL, "fg_fp8_gemm: null tensor");
  if (!is_float_dt(y_dtype)) return fail(FG_EINVAL, "fg_fp8_gemm: bad output dtype %d", y_dtype);
  if (bias && !is_float_dt(bias_dtype)) return fail(FG_EINVAL, "fg_fp8_gemm: bad bias dtype");
  if (lda < K || ldb < K || ldy < N) return fail(FG_EINVAL, "fg_fp8_gemm: leading dimensions too small");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (scale_mode == 0 || scale_mode == 1) {
    if (scale_mode == 0) sa_sm = sb_sn = 0;
    bool ring;
    const int tile = mm_tile(M, N, K, false, a, lda, b, ldb, cfg, &ring);
    if (tile == -2) return fail(FG_EINVAL, "fg_fp8_gemm: tile_m must be 0, 16, 64, 128 or 256, got %d", cfg->tile_m);
    if (tile < 0)
      return fail(FG_EUNSUPPORTED, "fg_fp8_gemm: tile_m=256 needs K %% 128 == 0, tile_m=16 M <= 64 and K %% 256 == 0, "
                                   "both 16-byte aligned operands; tile_n (32, 64, 128 for tile_m=64, 128 for "
                                   "tile_m=128) the same");
    if (ring) {
      const int bn = cfg && cfg->tile_n ? cfg->tile_n : fg::mm_ring_bn(M, N, tile);
      return hip_status(fg::launch_fp8_gemm_ring(a, lda, sa, sa_sm, b, ldb, sb, sb_sn, bias, bias_dtype, y, ldy,
                                                 y_dtype, (int)M, (int)N, (int)K, tile, bn, s),
                        "fg_fp8_gemm launch");
    }
    if (tile == 16)
      return hip_status(fg::launch_fp8_gemm_skinny(a, lda, sa, sa_sm, b, ldb, sb, sb_sn, bias, bias_dtype, y, ldy,
                                                   y_dtype, (int)M, (int)N, (int)K, s),
                        "fg_fp8_gemm launch");
    if (tile == 256)
      return hip_status(fg::launch_fp8_gemm_big(a, lda, sa, sa_sm, b, ldb, sb, sb_sn, bias, bias_dtype, y, ldy, y_dtype,
                                                (int)M, (int)N, (int)K, s),
                        "fg_fp8_gemm launch");
    return hip_status(fg::launch_fp8_gemm(a, lda, sa, sa_sm, b, ldb, sb, sb_sn, bias, bias_dtype, y, ldy, y_dtype,
                                          (int)M, (int)N, (int)K, tile, s),
                      "fg_fp8_gemm launch");
  }
  if (scale_mode == 2) {
    if (block != 128) return fail(FG_EUNSUPPORTED, "fg_fp8_gemm: block scales need block=128, got %d", block);
    if (sb_div != 1 && sb_div != 128) return fail(FG_EINVAL, "fg_fp8_gemm: sb_div must be 1 or the block");
    return hip_status(fg::launch_fp8_gemm_blocked(a, lda, sa, sa_sm, sa_sk, b, ldb, sb, sb_sn, sb_sk, sb_div, bias,
                                                  bias_dtype, y, ldy, y_dtype, (int)M, (int)N, (int)K, s),
                      "fg_fp8_gemm launch");
  }
  return fail(FG_EINVAL, "fg_fp8_gemm: unknown scale_mode %d", scale_mode);
}

int fg_quant_int8_rowwise(const void* x, int64_t ldx, int x_dtype, int8_t* q, int64_t ldq, float* s, int64_t M,
                          int64_t K, fg_stream_t stream) {
  if (M < 0 || K <= 0 || M >= kMaxDim || K >= kMaxDim) return fail(FG_EINVAL, "fg_quant_int8_rowwise: bad sizes");
  if (M == 0) return FG_OK;
  if (!x || !q || !s) return fail(FG_EINVAL, "fg_quant_int8_rowwise: null tensor");
  if (!is_float_dt(x_dtype)) return fail(FG_EINVAL, "fg_quant_int8_rowwise: bad x dtype");
  if (ldx < K || ldq < K) return fail(FG_EINVAL, "fg_quant_int8_rowwise: leading dimensions too small");
  return hip_status(fg::launch_quant_int8(x, ldx, x_dtype, q, ldq, s, (int)M, (int)K, static_cast<hipStream_t>(stream)),
                    "fg_quant_int8_rowwise launch");
}

int fg_quant_fp8_rowwise(const void* x, int64_t ldx, int x_dtype, uint8_t* q, int64_t ldq, float* s, int64_t M,
                         int64_t K, const float* static_scale, const void* rms_weight, int rms_weight_dtype,
                         float rms_eps, int32_t fuse_rmsnorm, fg_stream_t stream) {
  if (M < 0 || K <= 0 || M >= kMaxDim || K >= kMaxDim) return fail(FG_EINVAL, "fg_quant_fp8_rowwise: bad sizes");
  if (M == 0) return FG_OK;
  if (!x || !q || (!s && !static_scale)) return fail(FG_EINVAL, "fg_quant_fp8_rowwise: null tensor");
  if (!is_float_dt(x_dtype)) return fail(FG_EINVAL, "fg_quant_fp8_rowwise: bad x dtype");
  if (rms_weight && !is_float_dt(rms_weight_dtype)) return fail(FG_EINVAL, "fg_quant_fp8_rowwise: bad weight dtype");
  if (ldx < K || ldq < K) return fail(FG_EINVAL, "fg_quant_fp8_rowwise: leading dimensions too small");
  return hip_status(fg::launch_quant_fp8(x, ldx, x_dtype, q, ldq, s, (int)M, (int)K, static_scale, rms_weight,
                                         rms_weight_dtype, rms_eps, fuse_rmsnorm, static_cast<hipStream_t>(stream)),
                    "fg_quant_fp8_rowwise launch");
}

int fg_quant_fp8_block(const void* x, int64_t ldx, int x_dtype, uint8_t* q, int64_t ldq, float* s, int64_t lds,
                       int64_t M, int64_t K, int32_t block_m, int32_t block_k, const float* static_scale,
                       fg_stream_t stream) {
  if (M < 0 || K <= 0 || M >= kMaxDim || K >= kMaxDim || block_m <= 0 || block_k <= 0)
    return fail(FG_EINVAL, "fg_quant_fp8_block: bad sizes");
  if (M == 0) return FG_OK;
  if (!x || !q || (!s && !static_scale)) return fail(FG_EINVAL, "fg_quant_fp8_block: null tensor");
  if (!is_float_dt(x_dtype)) return fail(FG_EINVAL, "fg_quant_fp8_block: bad x dtype");
  const int64_t kb = (K + block_k - 1) / block_k, mb = (M + block_m - 1) / block_m;
  if (ldx < K || ldq < K || (s && lds < kb)) return fail(FG_EINVAL, "fg_quant_fp8_block: leading dimensions too small");
  if (kb >= 65536 * 32768LL || mb >= 65536) return fail(FG_EINVAL, "fg_quant_fp8_block: too many blocks");
  return hip_status(fg::launch_quant_fp8_block(x, ldx, x_dtype, q, ldq, s, lds, (int)M, (int)K, block_m, block_k,
                                               static_scale, static_cast<hipStream_t>(stream)),
                    "fg_quant_fp8_block launch");
}

}  // extern "C"
