// hipBLASLt GEMMs as the benchmark's yardstick for the hand-written MFMA
// kernels (gemm.hip, gemm_fp8.hip). Built into its own library,
// libsh_blaslt_yardstick.so, which bench.py and the yardstick parity tests
// load; libstrict_hip.so neither links nor loads it, and sh_gemm_bf16 /
// sh_gemm_fp8 always run the hand-written kernels.
//
// C ABI (status 0 = ok, 7 = hipBLASLt has no algorithm for the shape, 3 = a
// hipBLASLt / HIP call failed; shy_last_error() has the text):
//   shy_gemm_bf16(stream, A, B, C, M, N, K, lda, ldb, ldc)
//   shy_gemm_fp8(stream, A, sa, Bt, sb, C, M, N, K, lda, ldb, ldc)
//   shy_release()   destroys every handle, plan and workspace
// with the operand conventions of sh_gemm_bf16 / sh_gemm_fp8
// (include/strict_hip.h): device pointers, row-major, enqueued on `stream`.
//
// Row-major C = A B is the column-major product C^T = B^T A^T, so the
// hipBLASLt call's first operand is B (bf16: B row-major [K][N] is B^T in
// column-major, no transpose; fp8: Bt row-major [N][K] is a column-major
// K x N matrix, transposed) and its second is A (row-major [M][K] is A^T in
// column-major). For fp8 the call's row scale vector (OUTER_VEC_32F on its
// first operand, N values) is sb and its column scale vector sa.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <map>
#include <mutex>
#include <tuple>

#define SHY_API extern "C" __attribute__((visibility("default")))

namespace {

constexpr int kOk = 0, kErrHip = 3, kUnsupported = 7;
constexpr size_t kWorkspaceBytes = 64ull << 20;

thread_local char g_error[512];

int fail(int status, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof g_error, fmt, ap);
  va_end(ap);
  return status;
}

struct Plan {
  hipblasLtMatmulDesc_t op = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  bool ok = false;  // an algorithm exists for this shape
};

// (device, kind, M, N, K, lda, ldb, ldc)
typedef std::tuple<int, int, int, int, int, int, int, int> PlanKey;

struct State {
  hipblasLtHandle_t handle = nullptr;
  void *workspace = nullptr;
};

std::mutex g_mu;
std::map<int, State> g_states;  // per device
std::map<PlanKey, Plan> g_plans;

void destroy_plan(Plan &p) {
  if (p.a) hipblasLtMatrixLayoutDestroy(p.a);
  if (p.b) hipblasLtMatrixLayoutDestroy(p.b);
  if (p.c) hipblasLtMatrixLayoutDestroy(p.c);
  if (p.op) hipblasLtMatmulDescDestroy(p.op);
  p = Plan{};
}

State *state_for(int device) {
  State &st = g_states[device];
  if (!st.handle) {
    if (hipblasLtCreate(&st.handle) != HIPBLAS_STATUS_SUCCESS) return nullptr;
    if (hipMalloc(&st.workspace, kWorkspaceBytes) != hipSuccess) {
      hipblasLtDestroy(st.handle);
      st.handle = nullptr;
      return nullptr;
    }
  }
  return &st;
}

// The plan for kind 0 (bf16) or 1 (fp8 with vector scales).
Plan *plan_for(int device, State &st, int kind, int M, int N, int K, int lda, int ldb, int ldc) {
  const PlanKey key{device, kind, M, N, K, lda, ldb, ldc};
  auto it = g_plans.find(key);
  if (it != g_plans.end()) return &it->second;
  Plan &p = g_plans[key];
  const hipDataType in = kind == 0 ? HIP_R_16BF : HIP_R_8F_E4M3;
  const hipblasOperation_t opa = kind == 0 ? HIPBLAS_OP_N : HIPBLAS_OP_T, opb = HIPBLAS_OP_N;
  bool ok = hipblasLtMatmulDescCreate(&p.op, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSA, &opa, sizeof opa) ==
                 HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSB, &opb, sizeof opb) ==
                 HIPBLAS_STATUS_SUCCESS;
  if (kind == 1) {
    const hipblasLtMatmulMatrixScale_t vec = HIPBLASLT_MATMUL_MATRIX_SCALE_OUTER_VEC_32F;
    ok = ok && hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_A_SCALE_MODE, &vec,
                                               sizeof vec) == HIPBLAS_STATUS_SUCCESS;
    ok = ok && hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_B_SCALE_MODE, &vec,
                                               sizeof vec) == HIPBLAS_STATUS_SUCCESS;
    // the scale pointers are set per call; a placeholder lets the heuristic
    // see that vector scales are in use
    const void *dummy = st.workspace;
    ok = ok && hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_A_SCALE_POINTER, &dummy,
                                               sizeof dummy) == HIPBLAS_STATUS_SUCCESS;
    ok = ok && hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_B_SCALE_POINTER, &dummy,
                                               sizeof dummy) == HIPBLAS_STATUS_SUCCESS;
  }
  // first operand: bf16 B^T (N x K, ld ldb); fp8 Bt stored K x N (ld ldb), transposed
  if (kind == 0)
    ok = ok && hipblasLtMatrixLayoutCreate(&p.a, in, N, K, ldb) == HIPBLAS_STATUS_SUCCESS;
  else
    ok = ok && hipblasLtMatrixLayoutCreate(&p.a, in, K, N, ldb) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&p.b, in, K, M, lda) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&p.c, HIP_R_16BF, N, M, ldc) == HIPBLAS_STATUS_SUCCESS;
  if (ok) {
    hipblasLtMatmulPreference_t pref = nullptr;
    if (hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS) {
      const uint64_t ws = kWorkspaceBytes;
      hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws,
                                            sizeof ws);
      hipblasLtMatmulHeuristicResult_t res[1];
      int n = 0;
      if (hipblasLtMatmulAlgoGetHeuristic(st.handle, p.op, p.a, p.b, p.c, p.c, pref, 1, res, &n) ==
              HIPBLAS_STATUS_SUCCESS &&
          n > 0 && res[0].state == HIPBLAS_STATUS_SUCCESS) {
        p.algo = res[0].algo;
        p.ok = true;
      }
      hipblasLtMatmulPreferenceDestroy(pref);
    }
  }
  return &p;
}

int run(hipStream_t s, int kind, const void *first, const void *second, const float *first_scale,
        const float *second_scale, void *C, int M, int N, int K, int lda, int ldb, int ldc) {
  if (M <= 0 || N <= 0 || K <= 0) return fail(kUnsupported, "empty GEMM");
  std::lock_guard<std::mutex> lock(g_mu);
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return fail(kErrHip, "hipGetDevice failed");
  State *st = state_for(device);
  if (!st) return fail(kErrHip, "creating the hipBLASLt handle / workspace failed");
  Plan *p = plan_for(device, *st, kind, M, N, K, lda, ldb, ldc);
  if (!p->ok) return fail(kUnsupported, "hipBLASLt has no algorithm for this shape");
  if (kind == 1) {
    if (hipblasLtMatmulDescSetAttribute(p->op, HIPBLASLT_MATMUL_DESC_A_SCALE_POINTER, &first_scale,
                                        sizeof first_scale) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatmulDescSetAttribute(p->op, HIPBLASLT_MATMUL_DESC_B_SCALE_POINTER, &second_scale,
                                        sizeof second_scale) != HIPBLAS_STATUS_SUCCESS)
      return fail(kErrHip, "hipBLASLt: setting the scale vectors failed");
  }
  const float alpha = 1.0f, beta = 0.0f;
  const hipblasStatus_t r = hipblasLtMatmul(st->handle, p->op, &alpha, first, p->a, second, p->b,
                                            &beta, C, p->c, C, p->c, &p->algo, st->workspace,
                                            kWorkspaceBytes, s);
  if (r != HIPBLAS_STATUS_SUCCESS) return fail(kErrHip, "hipblasLtMatmul failed (status %d)", (int)r);
  return kOk;
}

}  // namespace

SHY_API const char *shy_last_error(void) { return g_error; }

SHY_API int shy_gemm_bf16(void *stream, const uint16_t *A, const uint16_t *B, uint16_t *C, int M,
                          int N, int K, int lda, int ldb, int ldc) {
  return run(static_cast<hipStream_t>(stream), 0, B, A, nullptr, nullptr, C, M, N, K, lda, ldb, ldc);
}

SHY_API int shy_gemm_fp8(void *stream, const uint8_t *A, const float *sa, const uint8_t *Bt,
                         const float *sb, uint16_t *C, int M, int N, int K, int lda, int ldb,
                         int ldc) {
  return run(static_cast<hipStream_t>(stream), 1, Bt, A, sb, sa, C, M, N, K, lda, ldb, ldc);
}

SHY_API void shy_release(void) {
  std::lock_guard<std::mutex> lock(g_mu);
  for (auto &kv : g_plans) destroy_plan(kv.second);
  g_plans.clear();
  for (auto &kv : g_states) {
    if (kv.second.handle) hipblasLtDestroy(kv.second.handle);
    if (kv.second.workspace) (void)hipFree(kv.second.workspace);
  }
  g_states.clear();
}
