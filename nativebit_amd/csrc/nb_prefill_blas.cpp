// Prefill through a dequantized weight: the packed W is expanded to bf16 in
// the caller's workspace by the format kernel (nb_dequant's chunk kernel),
// then y = x . W^T is one plain hipBLASLt GEMM (bf16 operands, fp32
// accumulation, bf16 or fp32 y).  This is the reference's own prefill
// semantics -- gather W, cast to bf16, dense matmul (inference/eval_ppl.py:
// 149-174) -- with the gather on the GPU; for many activation rows the
// library GEMM outruns the fused dequant-GEMM kernel, whose MFMA loop also
// decodes the stream.
//
// Row-major y (M x N) = x (M x K) . W^T, W row-major N x K, is the
// column-major product y^T (N x M) = op(A) . B with A = W viewed as K x N
// (op = transpose) and B = x^T viewed as K x M.
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "nb_internal.h"

namespace nb {
namespace {

struct GemmPlan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    bool ok = false;  // an algorithm exists for this shape
};

using PlanKey = std::tuple<int, int, int, int64_t, int64_t, int, int64_t>;

struct DeviceBlas {
    hipblasLtHandle_t handle = nullptr;
    std::map<PlanKey, GemmPlan> plans;
};

constexpr int kMaxDevices = 64;
constexpr size_t kMaxPlans = 512;  // per device; shapes past this are planned per call
std::mutex g_mu;
DeviceBlas g_dev[kMaxDevices];

void destroy(GemmPlan& p) {
    if (p.a) hipblasLtMatrixLayoutDestroy(p.a);
    if (p.b) hipblasLtMatrixLayoutDestroy(p.b);
    if (p.c) hipblasLtMatrixLayoutDestroy(p.c);
    if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
    p = GemmPlan{};
}

// Descriptors and the heuristic's first algorithm for one shape.
GemmPlan make_plan(hipblasLtHandle_t h, int M, int N, int K, int64_t ldx, int64_t ldy,
                   int y_dtype, int64_t blas_ws) {
    GemmPlan p;
    const hipDataType yt = y_dtype == NB_BF16 ? HIP_R_16BF : HIP_R_32F;
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    const uint64_t ws = (uint64_t)blas_ws;
    hipblasLtMatmulPreference_t pref = nullptr;
    hipblasLtMatmulHeuristicResult_t res{};
    int found = 0;
    bool good = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS &&
                hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) == HIPBLAS_STATUS_SUCCESS &&
                hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) == HIPBLAS_STATUS_SUCCESS &&
                hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16BF, K, N, K) == HIPBLAS_STATUS_SUCCESS &&
                hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16BF, K, M, ldx) == HIPBLAS_STATUS_SUCCESS &&
                hipblasLtMatrixLayoutCreate(&p.c, yt, N, M, ldy) == HIPBLAS_STATUS_SUCCESS &&
                hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS &&
                hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                                      &ws, sizeof(ws)) == HIPBLAS_STATUS_SUCCESS &&
                hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.a, p.b, p.c, p.c, pref, 1, &res,
                                                &found) == HIPBLAS_STATUS_SUCCESS &&
                found > 0 && res.state == HIPBLAS_STATUS_SUCCESS;
    if (pref) hipblasLtMatmulPreferenceDestroy(pref);
    if (good) {
        p.algo = res.algo;
        p.ok = true;
    }
    return p;
}

}  // namespace

int64_t prefill_ws_weight_bytes(int N, int K) {
    return (((int64_t)N * K * 2) + 255) / 256 * 256;
}

int launch_prefill_ws(const void* x, int64_t ldx, const uint8_t* packed, const float* codebook,
                      void* y, int y_dtype, int64_t ldy, int M, int N, int K, void* workspace,
                      int64_t ws_bytes, hipStream_t stream) {
    const int64_t wbytes = prefill_ws_weight_bytes(N, K);
    void* w = workspace;
    void* blas_ws = static_cast<unsigned char*>(workspace) + wbytes;
    const int64_t blas_bytes = ws_bytes - wbytes;

    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        return fail(NB_ELAUNCH, "nb_gemm_prefill_ws: no current device");
    }
    GemmPlan local;
    bool cached = false;
    GemmPlan plan;
    hipblasLtHandle_t handle;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        DeviceBlas& d = g_dev[dev];
        if (!d.handle && hipblasLtCreate(&d.handle) != HIPBLAS_STATUS_SUCCESS) {
            d.handle = nullptr;
            return fail(NB_ELAUNCH, "nb_gemm_prefill_ws: hipblasLtCreate failed");
        }
        handle = d.handle;
        const PlanKey key{M, N, K, ldx, ldy, y_dtype, blas_bytes};
        auto it = d.plans.find(key);
        if (it != d.plans.end()) {
            plan = it->second;
            cached = true;
        } else if (d.plans.size() < kMaxPlans) {
            plan = d.plans[key] = make_plan(handle, M, N, K, ldx, ldy, y_dtype, blas_bytes);
            cached = true;
        }
    }
    if (!cached) plan = local = make_plan(handle, M, N, K, ldx, ldy, y_dtype, blas_bytes);
    if (!plan.ok) {
        // no library algorithm for this shape: the fused kernel computes it
        if (!cached) destroy(local);
        return launch_prefill2(x, ldx, packed, codebook, y, y_dtype, ldy, M, N, K, nullptr, 0,
                               stream);
    }
    const int64_t total = (int64_t)N * K;
    int st = launch_dequant(packed, codebook, w, NB_BF16, total, total / 128, 3, 8, 128, stream);
    if (st) {
        if (!cached) destroy(local);
        return st;
    }
    const float alpha = 1.f, beta = 0.f;
    const hipblasStatus_t s = hipblasLtMatmul(handle, plan.desc, &alpha, w, plan.a, x, plan.b, &beta,
                                              y, plan.c, y, plan.c, &plan.algo, blas_ws,
                                              (size_t)blas_bytes, stream);
    if (!cached) destroy(local);
    if (s != HIPBLAS_STATUS_SUCCESS) {
        return fail(NB_ELAUNCH, "nb_gemm_prefill_ws: hipblasLtMatmul status %d", (int)s);
    }
    return check_launch("nb_gemm_prefill_ws");
}

}  // namespace nb
