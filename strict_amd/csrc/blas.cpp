// Plain GEMMs through hipBLASLt: the counterpart of the cuBLAS handle the
// reference keeps in Kernel.Handle (Kernel.cs:10-11, :16). The hand-written
// MFMA kernels (gemm.hip, gemm_fp8.hip) are the default; STRICT_HIP_GEMM=blaslt
// routes sh_gemm_bf16 / sh_gemm_fp8 here for the shapes hipBLASLt's heuristic
// has a gfx950 algorithm for (the others still take the hand-written kernels).
// The bench times both, so the library's figure is the yardstick for ours.
//
// Row-major C = A B is the column-major product C^T = B^T A^T, so the
// hipBLASLt call's first operand is B (bf16: B row-major [K][N] is B^T in
// column-major, no transpose; fp8: Bt row-major [N][K] is a column-major
// K x N matrix, transposed) and its second is A (row-major [M][K] is A^T in
// column-major). For fp8 the call's row scale vector (OUTER_VEC_32F on its
// first operand, N values) is sb and its column scale vector sa.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <tuple>

#include "common.h"

namespace sh {
namespace {

constexpr size_t kWorkspaceBytes = 64ull << 20;

struct Plan {
  hipblasLtMatmulDesc_t op = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  bool ok = false;  // an algorithm exists for this shape
};

// (kind, M, N, K, lda, ldb, ldc)
typedef std::tuple<int, int, int, int, int, int, int> PlanKey;

struct State {
  hipblasLtHandle_t handle = nullptr;
  void *workspace = nullptr;
  std::map<PlanKey, Plan> plans;
};

std::mutex g_mu;
std::map<const sh_ctx *, State> g_states;

bool enabled() {
  const char *e = getenv("STRICT_HIP_GEMM");
  return e && std::strcmp(e, "blaslt") == 0;
}

void destroy_plan(Plan &p) {
  if (p.a) hipblasLtMatrixLayoutDestroy(p.a);
  if (p.b) hipblasLtMatrixLayoutDestroy(p.b);
  if (p.c) hipblasLtMatrixLayoutDestroy(p.c);
  if (p.op) hipblasLtMatmulDescDestroy(p.op);
  p = Plan{};
}

// The plan for kind 0 (bf16) or 1 (fp8 with vector scales); nullptr when the
// state cannot be created.
Plan *plan_for(sh_ctx *ctx, int kind, int M, int N, int K, int lda, int ldb, int ldc) {
  State &st = g_states[ctx];
  if (!st.handle) {
    if (hipblasLtCreate(&st.handle) != HIPBLAS_STATUS_SUCCESS) return nullptr;
    if (hipMalloc(&st.workspace, kWorkspaceBytes) != hipSuccess) {
      hipblasLtDestroy(st.handle);
      st.handle = nullptr;
      return nullptr;
    }
  }
  const PlanKey key{kind, M, N, K, lda, ldb, ldc};
  auto it = st.plans.find(key);
  if (it != st.plans.end()) return &it->second;
  Plan &p = st.plans[key];
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

int run(sh_ctx *ctx, hipStream_t s, int kind, const void *first, const void *second,
        const float *first_scale, const float *second_scale, void *C, int M, int N, int K,
        int lda, int ldb, int ldc) {
  if (!enabled()) return SH_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_mu);
  Plan *p = plan_for(ctx, kind, M, N, K, lda, ldb, ldc);
  if (!p || !p->ok) return SH_ERR_UNSUPPORTED;
  State &st = g_states[ctx];
  if (kind == 1) {
    if (hipblasLtMatmulDescSetAttribute(p->op, HIPBLASLT_MATMUL_DESC_A_SCALE_POINTER, &first_scale,
                                        sizeof first_scale) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatmulDescSetAttribute(p->op, HIPBLASLT_MATMUL_DESC_B_SCALE_POINTER, &second_scale,
                                        sizeof second_scale) != HIPBLAS_STATUS_SUCCESS)
      return fail(SH_ERR_HIP, "hipBLASLt: setting the scale vectors failed");
  }
  const float alpha = 1.0f, beta = 0.0f;
  const hipblasStatus_t r = hipblasLtMatmul(st.handle, p->op, &alpha, first, p->a, second, p->b,
                                            &beta, C, p->c, C, p->c, &p->algo, st.workspace,
                                            kWorkspaceBytes, s);
  if (r != HIPBLAS_STATUS_SUCCESS) return fail(SH_ERR_HIP, "hipblasLtMatmul failed (status %d)", (int)r);
  return SH_OK;
}

}  // namespace

int blaslt_gemm_bf16(sh_ctx *ctx, hipStream_t s, const uint16_t *A, const uint16_t *B, uint16_t *C,
                     int M, int N, int K, int lda, int ldb, int ldc) {
  return run(ctx, s, 0, B, A, nullptr, nullptr, C, M, N, K, lda, ldb, ldc);
}

int blaslt_gemm_fp8(sh_ctx *ctx, hipStream_t s, const uint8_t *A, const float *sa,
                    const uint8_t *Bt, const float *sb, uint16_t *C, int M, int N, int K, int lda,
                    int ldb, int ldc) {
  return run(ctx, s, 1, Bt, A, sb, sa, C, M, N, K, lda, ldb, ldc);
}

void blaslt_release(sh_ctx *ctx) {
  std::lock_guard<std::mutex> lock(g_mu);
  auto it = g_states.find(ctx);
  if (it == g_states.end()) return;
  for (auto &kv : it->second.plans) destroy_plan(kv.second);
  if (it->second.handle) hipblasLtDestroy(it->second.handle);
  if (it->second.workspace) (void)hipFree(it->second.workspace);
  g_states.erase(it);
}

}  // namespace sh
