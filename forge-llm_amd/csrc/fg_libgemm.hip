// W4A16 (and W8A16) for many rows of x along the reference's own large-M route (forge/kernels/triton/gemm_w4_dequant.py:194-256,
// chosen by forge/kernels/w4_tuning.py:22-28 from 64 rows): the weights are dequantised once into the caller's
// workspace by the dense dequantisation kernel -- (q - z) * s in fp32, rounded once to x's dtype, the value the fused
// prefill kernel stores into LDS -- and then multiplied by hipBLASLt's bf16 / fp16 GEMM (fp32 accumulation, the bias
// added in fp32 by its epilogue before the single rounding of the output).  A plain library GEMM is what the matrix
// cores run best from M ~ 1024: the dequantisation costs 2.5 N K bytes of traffic once per call (3 N K for int8
// weights, q * s rounded once, the value the W8A16 prefill kernel stores into LDS), the GEMM then has no unpack in its
// loop.  Weights larger than kChunkBytes once dequantised go through in channel chunks.
//
// Row-major y[M, N] = x[M, K] W[N, K]^T is, column-major, Y^T (N x M, ld ldy) = op(W^T) op(x^T): A = the dequantised
// W (K x N, ld K) transposed, B = x^T (K x M, ld ldx), D = Y^T.
//
// One hipBLASLt handle per device and one matmul description + heuristic choice per problem signature are created on
// first use and kept for the life of the process (a mutex guards the tables); the matmul itself only enqueues work on
// the caller's stream.
#include <hipblaslt/hipblaslt.h>

#include <cstring>
#include <map>
#include <mutex>
#include <tuple>

#include "fg_device.h"

namespace fg {

hipError_t launch_w4_dequant(const int32_t* qw, int64_t ldq, const void* scales, int sdt, int64_t lds,
                             const int32_t* zeros, int64_t ldz, const int32_t* g_idx, void* out, int odt, int64_t ldo,
                             int N, int K, int gs, hipStream_t s);
hipError_t launch_w8_dequant16(const int8_t* qw, int64_t ldq, const void* scales, int sdt, int64_t lds, void* out,
                               int odt, int64_t ldo, int N, int K, int gs, hipStream_t s);

namespace {

constexpr size_t kChunkBytes = 512ull << 20;  // dequantised weights per chunk
constexpr size_t kLtWorkspace = 32ull << 20;  // hipBLASLt's own workspace, at the end of ours
constexpr int kLibMaxDevices = 64;

int chunk_rows(int N, int K) {
  const int64_t per = (int64_t)K * 2;
  if ((int64_t)N * per <= (int64_t)kChunkBytes) return N;
  return (int)(((int64_t)kChunkBytes / per) / 256 * 256);
}

struct PlanKey {
  int dev, M, N, K, xdt, bdt;
  int64_t ldx, ldy;
  bool operator<(const PlanKey& o) const {
    return std::tie(dev, M, N, K, xdt, bdt, ldx, ldy) < std::tie(o.dev, o.M, o.N, o.K, o.xdt, o.bdt, o.ldx, o.ldy);
  }
};

struct Plan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
  hipblasLtMatmulAlgo_t algo;
  size_t ws = 0;
};

std::mutex g_mu;
hipblasLtHandle_t g_handle[kLibMaxDevices] = {};
std::map<PlanKey, Plan> g_plans;

hipDataType lt_type(int dt) { return dt == FG_BF16 ? HIP_R_16BF : (dt == FG_F16 ? HIP_R_16F : HIP_R_32F); }

// The plan for one problem signature (created under the lock on first use); nullptr when hipBLASLt offers none.
const Plan* get_plan(const PlanKey& k, hipblasLtHandle_t h) {
  auto it = g_plans.find(k);
  if (it != g_plans.end()) return it->second.desc ? &it->second : nullptr;
  Plan p;
  bool ok = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS;
  const int32_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  ok = ok && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) == HIPBLAS_STATUS_SUCCESS;
  if (ok && k.bdt >= 0) {
    const uint32_t epi = HIPBLASLT_EPILOGUE_BIAS;
    const int32_t bt = lt_type(k.bdt);
    ok = hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi)) == HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof(bt)) == HIPBLAS_STATUS_SUCCESS;
  }
  const hipDataType t = lt_type(k.xdt);
  ok = ok && hipblasLtMatrixLayoutCreate(&p.a, t, k.K, k.N, k.K) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&p.b, t, k.K, k.M, k.ldx) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&p.d, t, k.N, k.M, k.ldy) == HIPBLAS_STATUS_SUCCESS;
  hipblasLtMatmulPreference_t pref = nullptr;
  ok = ok && hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS;
  const uint64_t maxws = kLtWorkspace;
  ok = ok && hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &maxws,
                                                   sizeof(maxws)) == HIPBLAS_STATUS_SUCCESS;
  hipblasLtMatmulHeuristicResult_t res[1];
  int found = 0;
  ok = ok && hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.a, p.b, p.d, p.d, pref, 1, res, &found) ==
                 HIPBLAS_STATUS_SUCCESS && found > 0 && res[0].state == HIPBLAS_STATUS_SUCCESS &&
       res[0].workspaceSize <= kLtWorkspace;
  if (pref) hipblasLtMatmulPreferenceDestroy(pref);
  if (ok) {
    p.algo = res[0].algo;
    p.ws = res[0].workspaceSize;
  } else {
    if (p.a) hipblasLtMatrixLayoutDestroy(p.a);
    if (p.b) hipblasLtMatrixLayoutDestroy(p.b);
    if (p.d) hipblasLtMatrixLayoutDestroy(p.d);
    if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
    p = Plan{};
  }
  auto ins = g_plans.emplace(k, p).first;
  return ins->second.desc ? &ins->second : nullptr;
}

}  // namespace

// Workspace of the dequantise + library GEMM route: one chunk of dequantised weights (16-bit, 256-byte aligned) and
// hipBLASLt's workspace after it.
size_t libgemm_workspace_bytes(int N, int K) {
  const size_t deq = ((size_t)chunk_rows(N, K) * (size_t)K * 2 + 255) / 256 * 256;
  return deq + kLtWorkspace;
}

// Whether the route applies to these operands: 16-bit x, a bias (if any) in fp32 or x's dtype, and x, y and K with
// 16-byte aligned rows.  Under graph capture only a problem whose handle and plan already exist takes it (creating
// them may allocate or synchronise, which a capture forbids); the caller's fused kernel serves the rest.
bool libgemm_ok(int xdt, const void* x, const void* bias, int bdt, const void* y, int64_t M, int64_t N, int64_t K,
                int64_t ldx, int64_t ldy, hipStream_t s) {
  if (!((xdt == FG_BF16 || xdt == FG_F16) && (!bias || bdt == FG_F32 || bdt == xdt) && K % 8 == 0 && ldx % 8 == 0 &&
        ldy % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0))
    return false;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cs) != hipSuccess) return false;
  if (cs == hipStreamCaptureStatusNone) return true;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kLibMaxDevices) return false;
  const int rows = chunk_rows((int)N, (int)K);
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_handle[dev]) return false;
  for (int n0 = 0; n0 < N; n0 += rows) {
    const int nc = N - n0 < rows ? (int)(N - n0) : rows;
    auto it = g_plans.find(PlanKey{dev, (int)M, nc, (int)K, xdt, bias ? bdt : -1, ldx, ldy});
    if (it == g_plans.end() || !it->second.desc) return false;
  }
  return true;
}

namespace {

// Dequantise channel chunk after channel chunk into the workspace (deq(n0, nc, out, stream) writes a 16-bit [nc, K]
// matrix) and multiply each by x with hipBLASLt.
template <class Deq>
hipError_t libgemm_run(const void* x, int64_t ldx, int xdt, const void* bias, int bdt, void* y, int64_t ldy, int M, int N,
                       int K, void* ws, size_t ws_bytes, hipStream_t s, Deq deq) {
  if (ws_bytes < libgemm_workspace_bytes(N, K) || reinterpret_cast<uintptr_t>(ws) % 256) return hipErrorInvalidValue;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kLibMaxDevices) return hipErrorInvalidDevice;
  const int rows = chunk_rows(N, K);
  uint8_t* dq = static_cast<uint8_t*>(ws);
  uint8_t* ltws = dq + (libgemm_workspace_bytes(N, K) - kLtWorkspace);
  for (int n0 = 0; n0 < N; n0 += rows) {
    const int nc = N - n0 < rows ? N - n0 : rows;
    e = deq(n0, nc, dq, s);
    if (e != hipSuccess) return e;
    const Plan* p;
    hipblasLtHandle_t h;
    {
      std::lock_guard<std::mutex> lk(g_mu);
      if (!g_handle[dev] && hipblasLtCreate(&g_handle[dev]) != HIPBLAS_STATUS_SUCCESS) {
        g_handle[dev] = nullptr;
        return hipErrorNotSupported;
      }
      h = g_handle[dev];
      p = get_plan(PlanKey{dev, M, nc, K, xdt, bias ? bdt : -1, ldx, ldy}, h);
    }
    if (!p) return hipErrorNotSupported;
    // the plan is shared by every call of this signature: its bias pointer is set and consumed under the lock
    std::lock_guard<std::mutex> lk(g_mu);
    if (bias) {
      const void* bp = static_cast<const uint8_t*>(bias) + (size_t)n0 * (bdt == FG_F32 ? 4 : 2);
      if (hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bp, sizeof(bp)) !=
          HIPBLAS_STATUS_SUCCESS)
        return hipErrorNotSupported;
    }
    const float alpha = 1.f, beta = 0.f;
    void* yc = static_cast<uint8_t*>(y) + (size_t)n0 * 2;
    if (hipblasLtMatmul(h, p->desc, &alpha, dq, p->a, x, p->b, &beta, yc, p->d, yc, p->d, &p->algo, ltws, p->ws, s) !=
        HIPBLAS_STATUS_SUCCESS)
      return hipErrorLaunchFailure;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_w4_libgemm(const void* x, int64_t ldx, int xdt, const int32_t* qw, int64_t ldq, const void* scales,
                             int sdt, int64_t lds, const int32_t* zeros, int64_t ldz, const int32_t* g_idx,
                             const void* bias, int bdt, void* y, int64_t ldy, int M, int N, int K, int gs,
                             void* ws, size_t ws_bytes, hipStream_t s) {
  const size_t esz = sdt == FG_F32 ? 4 : 2;
  const hipError_t e = libgemm_run(x, ldx, xdt, bias, bdt, y, ldy, M, N, K, ws, ws_bytes, s,
                     [&](int n0, int nc, void* out, hipStream_t st) {
                       return launch_w4_dequant(qw + (int64_t)n0 * ldq, ldq,
                                                static_cast<const uint8_t*>(scales) + (size_t)n0 * esz, sdt, lds,
                                                zeros ? zeros + n0 / 8 : nullptr, ldz, g_idx, out, xdt, K, nc, K, gs,
                                                st);
                     });
  note_kernel("w4_dequant16_kernel + hipBLASLt GEMM");
  return e;
}

// W8A16: symmetric int8 weights [N, ldq] with scales [G, lds] (w8_dequant16_ok must hold).
hipError_t launch_w8a16_libgemm(const void* x, int64_t ldx, int xdt, const int8_t* qw, int64_t ldq, const void* scales,
                                int sdt, int64_t lds, const void* bias, int bdt, void* y, int64_t ldy, int M, int N,
                                int K, int gs, void* ws, size_t ws_bytes, hipStream_t s) {
  const size_t esz = sdt == FG_F32 ? 4 : 2;
  const hipError_t e = libgemm_run(x, ldx, xdt, bias, bdt, y, ldy, M, N, K, ws, ws_bytes, s,
                     [&](int n0, int nc, void* out, hipStream_t st) {
                       return launch_w8_dequant16(qw + (int64_t)n0 * ldq, ldq,
                                                  static_cast<const uint8_t*>(scales) + (size_t)n0 * esz, sdt, lds, out,
                                                  xdt, K, nc, K, gs, st);
                     });
  note_kernel("w8_dequant16_kernel + hipBLASLt GEMM");
  return e;
}

}  // namespace fg
