// Plain library GEMM of the prefill: out = heads . o_proj^T (fp16 operands, fp32 accumulate and
// output, no epilogue) through hipBLASLt. The epilogue-fused GEMMs stay hand-written
// (mla_prefill.hip). One plan per (M, N, K), built on first use with the heuristic's first
// algorithm (deterministic choice, no workspace).
#include <hipblaslt/hipblaslt.h>

#include <vector>

#include "mla_internal.h"

namespace kvl {
namespace {

struct LtPlan {
    int M = 0, N = 0, K = 0, lda = 0, ldw = 0, ldc = 0;
    bool ok = false;
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
    hipblasLtMatmulAlgo_t algo{};
};

hipblasLtHandle_t g_lt = nullptr;
int g_lt_state = 0;  // 0 untried, 1 ready, -1 unavailable
std::vector<LtPlan> g_plans;

bool lt_ready() {
    if (g_lt_state == 0) g_lt_state = hipblasLtCreate(&g_lt) == HIPBLAS_STATUS_SUCCESS ? 1 : -1;
    return g_lt_state == 1;
}

// Row-major C[M, N] = A[M, K] . W[N, K]^T is column-major C^T[N, M] = W^T(op T of W as
// col-major [K, N]) . A^T (A as col-major [K, M]).
bool build(LtPlan &p) {
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    if (hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS) return false;
    if (hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof ta) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof tb) != HIPBLAS_STATUS_SUCCESS)
        return false;
    if (hipblasLtMatrixLayoutCreate(&p.la, HIP_R_16F, p.K, p.N, p.ldw) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&p.lb, HIP_R_16F, p.K, p.M, p.lda) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&p.lc, HIP_R_32F, p.N, p.M, p.ldc) != HIPBLAS_STATUS_SUCCESS)
        return false;
    hipblasLtMatmulPreference_t pref = nullptr;
    if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return false;
    uint64_t wmax = 0;
    hipblasLtMatmulHeuristicResult_t res[1];
    int n = 0;
    const bool got =
        hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wmax, sizeof wmax) ==
            HIPBLAS_STATUS_SUCCESS &&
        hipblasLtMatmulAlgoGetHeuristic(g_lt, p.desc, p.la, p.lb, p.lc, p.lc, pref, 1, res, &n) ==
            HIPBLAS_STATUS_SUCCESS &&
        n > 0;
    hipblasLtMatmulPreferenceDestroy(pref);
    if (!got) return false;
    p.algo = res[0].algo;
    return true;
}

}  // namespace

hipError_t lt_gemm_f16(hipStream_t st, float *C, int ldc, const _Float16 *A, int lda, const _Float16 *W,
                       int ldw, int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0 || !lt_ready()) return hipErrorNotSupported;
    LtPlan *p = nullptr;
    for (auto &q : g_plans)
        if (q.M == M && q.N == N && q.K == K && q.lda == lda && q.ldw == ldw && q.ldc == ldc) p = &q;
    if (!p) {
        LtPlan q;
        q.M = M, q.N = N, q.K = K, q.lda = lda, q.ldw = ldw, q.ldc = ldc;
        q.ok = build(q);
        g_plans.push_back(q);
        p = &g_plans.back();
    }
    if (!p->ok) return hipErrorNotSupported;
    const float alpha = 1.f, beta = 0.f;
    if (hipblasLtMatmul(g_lt, p->desc, &alpha, W, p->la, A, p->lb, &beta, C, p->lc, C, p->lc, &p->algo, nullptr, 0,
                        st) != HIPBLAS_STATUS_SUCCESS)
        return hipErrorLaunchFailure;
    return hipSuccess;
}

}  // namespace kvl
