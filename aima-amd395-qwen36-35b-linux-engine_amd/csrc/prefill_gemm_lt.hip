// Prefill projection GEMM through hipBLASLt: y[m, n] = x[m, k] W[n, k]^T,
// bf16 in and out, fp32 accumulation -- the same product as
// qwen36_prefill_gemm_bf16 (prefill_gemm.hip), run as the library GEMM the
// reference's native prefill plans for these projections
// (native/src/native_full_prefill.hip.cpp:552-560, hipBLASLt plans).  The host
// picks this path per shape where hipBLASLt's kernel is the faster one (the
// K = 4096 output projections at long prompts), the native MFMA kernel
// elsewhere.
//
// Column-major view: row-major y [m][n] (row stride ldy) is the column-major
// n x m matrix D = op(A) op(B) with A = W as a column-major k x n matrix (ld
// k) transposed and B = x as a column-major k x m matrix (ld ldx).
// A handle per device and the heuristic's algorithm per shape are cached
// behind a mutex; the caller passes the workspace (at least
// qwen36_prefill_gemm_lt_workspace_bytes()), so the call allocates nothing
// once a shape has been seen.
#include "common.h"

#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

namespace q36 {
namespace {

constexpr size_t kLtWorkspace = 32u << 20;   // heuristic limit for the algorithm's workspace
constexpr int kLtMaxDevices = 64;

struct LtPlan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  size_t ws = 0;
};

std::mutex g_lt_mutex;
hipblasLtHandle_t g_lt_handle[kLtMaxDevices] = {};
std::map<std::tuple<int, unsigned, unsigned, unsigned, unsigned, unsigned>, LtPlan> g_lt_plans;

// The cached plan for (device, shape, strides), creating it on first use;
// nullptr if hipBLASLt has no algorithm for it.
const LtPlan* lt_plan(int dev, unsigned m, unsigned n, unsigned k, unsigned ldx, unsigned ldy) {
  std::lock_guard<std::mutex> lock(g_lt_mutex);
  const auto key = std::make_tuple(dev, m, n, k, ldx, ldy);
  auto it = g_lt_plans.find(key);
  if (it != g_lt_plans.end()) return &it->second;
  if (g_lt_handle[dev] == nullptr && hipblasLtCreate(&g_lt_handle[dev]) != HIPBLAS_STATUS_SUCCESS) {
    g_lt_handle[dev] = nullptr;
    return nullptr;
  }
  LtPlan p;
  bool ok = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) ==
            HIPBLAS_STATUS_SUCCESS;
  const hipblasOperation_t op_t = HIPBLAS_OP_T, op_n = HIPBLAS_OP_N;
  ok = ok && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &op_t,
                                             sizeof(op_t)) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &op_n,
                                             sizeof(op_n)) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&p.la, HIP_R_16BF, k, n, k) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&p.lb, HIP_R_16BF, k, m, ldx) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&p.lc, HIP_R_16BF, n, m, ldy) == HIPBLAS_STATUS_SUCCESS;
  hipblasLtMatmulPreference_t pref = nullptr;
  ok = ok && hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS;
  const uint64_t max_ws = kLtWorkspace;
  ok = ok && hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                                   &max_ws, sizeof(max_ws)) ==
                 HIPBLAS_STATUS_SUCCESS;
  // the heuristic's first algorithm whose workspace fits the advertised size
  hipblasLtMatmulHeuristicResult_t res[8];
  int found = 0, pick = -1;
  ok = ok && hipblasLtMatmulAlgoGetHeuristic(g_lt_handle[dev], p.desc, p.la, p.lb, p.lc, p.lc,
                                             pref, 8, res, &found) == HIPBLAS_STATUS_SUCCESS;
  for (int i = 0; ok && i < found && pick < 0; ++i)
    if (res[i].state == HIPBLAS_STATUS_SUCCESS && res[i].workspaceSize <= kLtWorkspace) pick = i;
  ok = ok && pick >= 0;
  if (pref != nullptr) hipblasLtMatmulPreferenceDestroy(pref);
  if (!ok) {
    if (p.la) hipblasLtMatrixLayoutDestroy(p.la);
    if (p.lb) hipblasLtMatrixLayoutDestroy(p.lb);
    if (p.lc) hipblasLtMatrixLayoutDestroy(p.lc);
    if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
    return nullptr;
  }
  p.algo = res[pick].algo;
  p.ws = res[pick].workspaceSize;
  return &(g_lt_plans[key] = p);
}

}  // namespace
}  // namespace q36

using namespace q36;

Q36_EXPORT size_t qwen36_prefill_gemm_lt_workspace_bytes(void) { return kLtWorkspace; }

Q36_EXPORT int qwen36_prefill_gemm_bf16_lt(const void* x, unsigned ldx, const void* w, void* y,
                                           unsigned ldy, unsigned m, unsigned n, unsigned k,
                                           void* ws, size_t ws_bytes, void* stream) {
  if (x == nullptr || w == nullptr || y == nullptr || m == 0 || n == 0 || k == 0 ||
      m > kMaxTokens || n > 65536u || k > 16384u || ldx < k || ldy < n ||
      (ws == nullptr && ws_bytes != 0))
    return Q36_EINVAL;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kLtMaxDevices) return Q36_EINVAL;
  // Output widths past a multiple of 4096 run as two products (the first
  // n1 = 4096-multiple columns, then the rest) from 513 rows on: the
  // heuristic's algorithm for the fused widths is far from its best there
  // (MI355X, T = 8192: N = 12352 443 us vs 12288 + 64 in 285 + 10 us; N =
  // 9216 274 us vs 8192 + 1024 in 196 + 33 us), while for short prompts the
  // second launch costs more than it saves (T = 256: N = 9216 22.4 vs 28.5
  // us, N = 12352 22.6 vs 30.8; T = 512: 26.0 vs 30.6, 33.0 vs 35.9).
  const unsigned n1 =
      (m > 512u && n > 4096u && n % 4096u != 0u) ? n / 4096u * 4096u : n;
  const LtPlan* p = lt_plan(dev, m, n1, k, ldx, ldy);
  const LtPlan* p2 = n1 < n ? lt_plan(dev, m, n - n1, k, ldx, ldy) : nullptr;
  if (p == nullptr || (n1 < n && p2 == nullptr))
    return static_cast<int>(hipErrorNotSupported);   // no hipBLASLt algorithm
  if (p->ws > ws_bytes || (p2 != nullptr && p2->ws > ws_bytes)) return Q36_EINVAL;
  const float alpha = 1.0f, beta = 0.0f;
  const hipStream_t hs = static_cast<hipStream_t>(stream);
  hipblasStatus_t st = hipblasLtMatmul(g_lt_handle[dev], p->desc, &alpha, w, p->la, x, p->lb,
                                       &beta, y, p->lc, y, p->lc, &p->algo, ws, ws_bytes, hs);
  if (st == HIPBLAS_STATUS_SUCCESS && p2 != nullptr) {
    const void* w2 = static_cast<const bf16*>(w) + (size_t)n1 * k;
    void* y2 = static_cast<bf16*>(y) + n1;
    st = hipblasLtMatmul(g_lt_handle[dev], p2->desc, &alpha, w2, p2->la, x, p2->lb, &beta, y2,
                         p2->lc, y2, p2->lc, &p2->algo, ws, ws_bytes, hs);
  }
  if (st != HIPBLAS_STATUS_SUCCESS) return static_cast<int>(hipErrorLaunchFailure);
  return static_cast<int>(hipGetLastError());
}
