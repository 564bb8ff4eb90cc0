// BF16 matrix product of the model projections through hipBLASLt:
// out[tokens][rows] = BF16(in[tokens][inner] . weight[rows][inner]^T), fp32
// accumulation, rounded once.  The role of tv_hip_matrix_multiply
// (hipblaslt_bridge.cpp:203-233): a plain library GEMM, not part of the
// attention kernels, kept behind the same context so a caller binds one
// library.  Plans (descriptor, layouts, algorithm, workspace) are cached per
// (rows, tokens, inner) like the reference's make_plan.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <memory>
#include <string>
#include <tuple>

#include "kernels.hpp"

namespace mslim {

namespace {

struct GemmPlan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    size_t workspace_bytes = 0;
    void *workspace = nullptr;
    ~GemmPlan() {
        if (workspace) (void)hipFree(workspace);
        if (a) hipblasLtMatrixLayoutDestroy(a);
        if (b) hipblasLtMatrixLayoutDestroy(b);
        if (c) hipblasLtMatrixLayoutDestroy(c);
        if (desc) hipblasLtMatmulDescDestroy(desc);
    }
};

constexpr size_t kMaxWorkspace = 32ull << 20;

}  // namespace

struct GemmState {
    hipblasLtHandle_t handle = nullptr;
    std::map<std::tuple<int, int, int>, std::unique_ptr<GemmPlan>> plans;
    ~GemmState() {
        plans.clear();
        if (handle) hipblasLtDestroy(handle);
    }
};

void gemm_state_destroy(GemmState *state) { delete state; }

namespace {

int lt_status(hipblasStatus_t s, const char *what, std::string &err) {
    if (s == HIPBLAS_STATUS_SUCCESS) return 0;
    err = std::string(what) + " hipBLASLt status=" + std::to_string((int)s);
    return 200 + (int)s;
}

// Column-major view: C (rows x tokens, ld rows) = op_T(A) . B, where A is the
// row-major weight seen as inner x rows (ld inner) and B the row-major input
// seen as inner x tokens (ld inner).
GemmPlan *make_plan(GemmState &st, int rows, int tokens, int inner, std::string &err, int &code) {
    auto key = std::make_tuple(rows, tokens, inner);
    auto it = st.plans.find(key);
    if (it != st.plans.end()) return it->second.get();
    auto plan = std::make_unique<GemmPlan>();
    code = lt_status(hipblasLtMatmulDescCreate(&plan->desc, HIPBLAS_COMPUTE_32F, HIP_R_32F), "matmul desc", err);
    if (code) return nullptr;
    const hipblasOperation_t op_t = HIPBLAS_OP_T, op_n = HIPBLAS_OP_N;
    code = lt_status(hipblasLtMatmulDescSetAttribute(plan->desc, HIPBLASLT_MATMUL_DESC_TRANSA, &op_t, sizeof op_t),
                     "matmul transA", err);
    if (code) return nullptr;
    code = lt_status(hipblasLtMatmulDescSetAttribute(plan->desc, HIPBLASLT_MATMUL_DESC_TRANSB, &op_n, sizeof op_n),
                     "matmul transB", err);
    if (code) return nullptr;
    code = lt_status(hipblasLtMatrixLayoutCreate(&plan->a, HIP_R_16BF, inner, rows, inner), "layout A", err);
    if (code) return nullptr;
    code = lt_status(hipblasLtMatrixLayoutCreate(&plan->b, HIP_R_16BF, inner, tokens, inner), "layout B", err);
    if (code) return nullptr;
    code = lt_status(hipblasLtMatrixLayoutCreate(&plan->c, HIP_R_16BF, rows, tokens, rows), "layout C", err);
    if (code) return nullptr;
    hipblasLtMatmulPreference_t pref = nullptr;
    code = lt_status(hipblasLtMatmulPreferenceCreate(&pref), "preference", err);
    if (code) return nullptr;
    uint64_t ws = kMaxWorkspace;
    hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof ws);
    hipblasLtMatmulHeuristicResult_t result[1];
    int found = 0;
    const hipblasStatus_t hs = hipblasLtMatmulAlgoGetHeuristic(st.handle, plan->desc, plan->a, plan->b, plan->c,
                                                               plan->c, pref, 1, result, &found);
    hipblasLtMatmulPreferenceDestroy(pref);
    code = lt_status(hs, "algorithm heuristic", err);
    if (code) return nullptr;
    if (found < 1) {
        err = "hipBLASLt found no BF16 algorithm for rows=" + std::to_string(rows) +
              " tokens=" + std::to_string(tokens) + " inner=" + std::to_string(inner);
        code = 403;
        return nullptr;
    }
    plan->algo = result[0].algo;
    plan->workspace_bytes = result[0].workspaceSize;
    if (plan->workspace_bytes) {
        const hipError_t e = hipMalloc(&plan->workspace, plan->workspace_bytes);
        if (e != hipSuccess) {
            err = std::string("hipMalloc GEMM workspace: ") + hipGetErrorString(e);
            code = 100 + (int)e;
            return nullptr;
        }
    }
    GemmPlan *raw = plan.get();
    st.plans.emplace(key, std::move(plan));
    code = 0;
    return raw;
}

}  // namespace

int gemm_bf16(GemmState *&state, const void *weight, const void *input, void *output, int inner, int rows,
              int tokens, hipStream_t stream, std::string &err) {
    if (!state) {
        auto *st = new (std::nothrow) GemmState;
        if (!st) {
            err = "Out of memory for the GEMM state";
            return -1;
        }
        if (int code = lt_status(hipblasLtCreate(&st->handle), "hipblasLtCreate", err)) {
            delete st;
            return code;
        }
        state = st;
    }
    int code = 0;
    GemmPlan *plan = make_plan(*state, rows, tokens, inner, err, code);
    if (!plan) return code ? code : 403;
    const float alpha = 1.0f, beta = 0.0f;
    return lt_status(hipblasLtMatmul(state->handle, plan->desc, &alpha, weight, plan->a, input, plan->b, &beta,
                                     output, plan->c, output, plan->c, &plan->algo, plan->workspace,
                                     plan->workspace_bytes, stream),
                     "BF16 matmul", err)
               ? 404
               : 0;
}

}  // namespace mslim
