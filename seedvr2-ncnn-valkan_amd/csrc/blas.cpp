// Matrix products of the InnerProduct layers.
//
// fp16 (the fast mode): hipBLASLt with fp32 accumulation.  The first product
// of a shape on a device plans it: the library's best-ranked kernel that needs
// no workspace, kept for the rest of the process.  The choice depends on the
// shape alone, so a shape is computed with the same kernel (and rounds the
// same way) in every process, and planning neither runs nor synchronises
// anything.  (Timing the library's 16 best-ranked kernels instead and keeping
// the fastest changed the 720p DiT step by less than its run-to-run spread.)
// Without a workspace, products on different streams share nothing.  The
// gated form carries the block's gated residual in the library's epilogue
// (per-channel alpha, beta 1, optional bias), planned per shape in the same
// way.
// fp32 (the parity mode): gemm_f32_exact (gemm_exact.hip), double
// accumulation in the order of the CPU oracle, the bias added in double; bit
// for bit the oracle's W x + b, and against ncnn's float InnerProduct (whose
// summation order is unknown here) equal only up to its rounding.
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <set>
#include <string>
#include <tuple>

#include "sv2_internal.h"

namespace sv2
{
namespace
{

std::mutex g_mutex;

int current_device(int* rc)
{
    int device = 0;
    const hipError_t err = hipGetDevice(&device);
    if (err != hipSuccess)
    {
        *rc = hip_error(err, "gemm: hipGetDevice");
        return -1;
    }
    return device;
}

// One hipBLASLt handle per device (caller holds g_mutex).
hipblasLtHandle_t lt_for(int device, int* rc)
{
    static std::map<int, hipblasLtHandle_t> handles;
    auto it = handles.find(device);
    if (it != handles.end())
        return it->second;
    hipblasLtHandle_t h = nullptr;
    if (hipblasLtCreate(&h) != HIPBLAS_STATUS_SUCCESS)
    {
        *rc = set_error(SV2_EDEVICE, "gemm: hipblasLtCreate failed");
        return nullptr;
    }
    handles[device] = h;
    return h;
}

// A tuned fp16 product: column-major D[out x rows] = op(A) B with A = W
// stored [out][in] row-major (in x out, transposed), B = X [rows][in]
// row-major (in x rows), D = Y [rows][out] row-major (out x rows).
struct LtPlan
{
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr;
    hipblasLtMatrixLayout_t b = nullptr;
    hipblasLtMatrixLayout_t d = nullptr;
    hipblasLtMatmulAlgo_t algo{};
};

using PlanKey = std::tuple<int, int, int, int, int>; // device, rows, in, out, gated

// The gated form: D = gate[c] * (X W^T)[r][c] + R[r][c] (+ bias[c]) (alpha a
// device vector over the output channels, beta 1, C = the residual R, the
// library's bias epilogue added after the alpha scaling).
struct Gated
{
    const float* gate = nullptr;
    const void* residual = nullptr;
    const float* bias = nullptr;
};

void destroy_plan(LtPlan* plan)
{
    if (plan->d)
        hipblasLtMatrixLayoutDestroy(plan->d);
    if (plan->b)
        hipblasLtMatrixLayoutDestroy(plan->b);
    if (plan->a)
        hipblasLtMatrixLayoutDestroy(plan->a);
    if (plan->desc)
        hipblasLtMatmulDescDestroy(plan->desc);
    *plan = LtPlan();
}

int describe(int rows, int in, int out, const Gated* gated, LtPlan* plan)
{
    if (hipblasLtMatmulDescCreate(&plan->desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS)
        return set_error(SV2_EDEVICE, "gemm: hipblasLtMatmulDescCreate failed");
    if (gated)
    {
        const int32_t mode = HIPBLASLT_POINTER_MODE_ALPHA_DEVICE_VECTOR_BETA_HOST;
        if (hipblasLtMatmulDescSetAttribute(plan->desc, HIPBLASLT_MATMUL_DESC_POINTER_MODE, &mode, sizeof(mode)) !=
            HIPBLAS_STATUS_SUCCESS)
            return set_error(SV2_EUNSUPPORTED, "gemm: hipBLASLt has no per-channel alpha");
        if (gated->bias)
        {
            const hipblasLtEpilogue_t epi = HIPBLASLT_EPILOGUE_BIAS;
            const int32_t bias_type = HIP_R_32F;
            if (hipblasLtMatmulDescSetAttribute(plan->desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi)) !=
                    HIPBLAS_STATUS_SUCCESS ||
                hipblasLtMatmulDescSetAttribute(plan->desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bias_type,
                                                sizeof(bias_type)) != HIPBLAS_STATUS_SUCCESS ||
                hipblasLtMatmulDescSetAttribute(plan->desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &gated->bias,
                                                sizeof(gated->bias)) != HIPBLAS_STATUS_SUCCESS)
                return set_error(SV2_EUNSUPPORTED, "gemm: hipBLASLt has no fp32 bias epilogue");
        }
    }
    const hipblasOperation_t ta = HIPBLAS_OP_T;
    const hipblasOperation_t tb = HIPBLAS_OP_N;
    if (hipblasLtMatmulDescSetAttribute(plan->desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) !=
            HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatmulDescSetAttribute(plan->desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) !=
            HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&plan->a, HIP_R_16F, in, out, in) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&plan->b, HIP_R_16F, in, rows, in) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&plan->d, HIP_R_16F, out, rows, out) != HIPBLAS_STATUS_SUCCESS)
        return set_error(SV2_EDEVICE, "gemm: hipBLASLt descriptor setup failed");
    return SV2_OK;
}

// Plans one product shape: the library's best-ranked kernel that needs no
// workspace.  The choice depends on the shape alone (no timing), so every
// process computes a shape with the same kernel and the same rounding, and
// planning never touches the stream.
int make_plan(hipblasLtHandle_t h, int rows, int in, int out, const Gated* gated, LtPlan* plan)
{
    int rc = describe(rows, in, out, gated, plan);
    if (rc != SV2_OK)
    {
        destroy_plan(plan);
        return rc;
    }
    hipblasLtMatmulPreference_t pref = nullptr;
    if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS)
    {
        destroy_plan(plan);
        return set_error(SV2_EDEVICE, "gemm: hipblasLtMatmulPreferenceCreate failed");
    }
    const uint64_t no_workspace = 0;
    hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &no_workspace,
                                          sizeof(no_workspace));
    constexpr int kCandidates = 16;
    hipblasLtMatmulHeuristicResult_t res[kCandidates];
    int got = 0;
    const hipblasStatus_t hs =
        hipblasLtMatmulAlgoGetHeuristic(h, plan->desc, plan->a, plan->b, plan->d, plan->d, pref, kCandidates, res, &got);
    hipblasLtMatmulPreferenceDestroy(pref);
    for (int i = 0; hs == HIPBLAS_STATUS_SUCCESS && i < got; i++)
        if (res[i].state == HIPBLAS_STATUS_SUCCESS && res[i].workspaceSize == 0)
        {
            plan->algo = res[i].algo;
            return SV2_OK;
        }
    destroy_plan(plan);
    return set_error(SV2_EUNSUPPORTED, "gemm: hipBLASLt has no workspace-free kernel for an fp16 product of this shape");
}

int gemm_f16(hipStream_t stream, int rows, int in, int out, const void* x, const void* w, void* y,
             const Gated* gated = nullptr)
{
    int rc = SV2_OK;
    LtPlan plan;
    hipblasLtHandle_t h = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_mutex);
        const int device = current_device(&rc);
        if (device < 0)
            return rc;
        h = lt_for(device, &rc);
        if (!h)
            return rc;
        static std::map<PlanKey, LtPlan> plans;
        static std::set<PlanKey> unsupported; // gated shapes the library has no kernel for
        const PlanKey key{device, rows, in, out, gated ? (gated->bias ? 2 : 1) : 0};
        if (unsupported.count(key))
            return set_error(SV2_EUNSUPPORTED, "gemm: hipBLASLt has no gated kernel for this shape");
        auto it = plans.find(key);
        if (it == plans.end())
        {
            LtPlan fresh;
            if ((rc = make_plan(h, rows, in, out, gated, &fresh)) != SV2_OK)
            {
                if (gated && rc == SV2_EUNSUPPORTED)
                    unsupported.insert(key);
                return rc;
            }
            it = plans.emplace(key, fresh).first;
        }
        plan = it->second;
        // the bias pointer is a property of the shared descriptor: set it for
        // this call while the lock is held, and enqueue under the lock
        if (gated && gated->bias)
        {
            if (hipblasLtMatmulDescSetAttribute(plan.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &gated->bias,
                                                sizeof(gated->bias)) != HIPBLAS_STATUS_SUCCESS)
                return set_error(SV2_EDEVICE, "gemm: hipBLASLt bias pointer");
            const float one = 1.f;
            if (hipblasLtMatmul(h, plan.desc, gated->gate, w, plan.a, x, plan.b, &one, gated->residual, plan.d, y,
                                plan.d, &plan.algo, nullptr, 0, stream) != HIPBLAS_STATUS_SUCCESS)
                return set_error(SV2_EDEVICE, "gemm: hipblasLtMatmul failed");
            return SV2_OK;
        }
    }
    const float one = 1.f;
    const float zero = 0.f;
    const void* alpha = gated ? static_cast<const void*>(gated->gate) : &one;
    const float* beta = gated ? &one : &zero;
    const void* c = gated ? gated->residual : y;
    if (hipblasLtMatmul(h, plan.desc, alpha, w, plan.a, x, plan.b, beta, c, plan.d, y, plan.d, &plan.algo, nullptr,
                        0, stream) != HIPBLAS_STATUS_SUCCESS)
        return set_error(SV2_EDEVICE, "gemm: hipblasLtMatmul failed");
    return SV2_OK;
}

} // namespace

int gemm_rows_gated(hipStream_t stream, int dtype, int rows, int in, int out, const void* x, const void* w, void* y,
                    const float* gate, const void* residual, const float* bias)
{
    if (dtype != SV2_F16)
        return set_error(SV2_EUNSUPPORTED, "gemm: the gated product runs on fp16 only");
    if (rows == 0)
        return SV2_OK;
    const Gated g{gate, residual, bias};
    return gemm_f16(stream, rows, in, out, x, w, y, &g);
}

int gemm_rows(hipStream_t stream, int dtype, int rows, int in, int out, const void* x, const void* w, void* y)
{
    return gemm_rows_bias(stream, dtype, rows, in, out, x, w, nullptr, y);
}

int gemm_rows_bias(hipStream_t stream, int dtype, int rows, int in, int out, const void* x, const void* w,
                   const float* bias, void* y)
{
    if (rows == 0)
        return SV2_OK;
    if (dtype == SV2_F32)
        return gemm_f32_exact(stream, rows, in, out, static_cast<const float*>(x), static_cast<const float*>(w), bias,
                              static_cast<float*>(y));
    if (dtype != SV2_F16)
        return set_error(SV2_EINVAL, "gemm: compute dtype must be fp32 or fp16");
    const int rc = gemm_f16(stream, rows, in, out, x, w, y);
    return (rc != SV2_OK || !bias) ? rc : launch_bias_rows(y, bias, SV2_F16, rows, out, stream);
}

} // namespace sv2
