// Matrix products of the InnerProduct layers on rocBLAS, one handle per
// device for the whole process.
#include <rocblas/rocblas.h>

#include <map>
#include <mutex>
#include <string>

#include "sv2_internal.h"

namespace sv2
{
namespace
{

// One rocBLAS handle per device, shared by every layer of the process.
rocblas_handle blas_handle(int* rc)
{
    static std::mutex mutex;
    static std::map<int, rocblas_handle> handles;
    int device = 0;
    hipError_t err = hipGetDevice(&device);
    if (err != hipSuccess)
    {
        *rc = sv2::hip_error(err, "gemm: hipGetDevice");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(mutex);
    auto it = handles.find(device);
    if (it != handles.end())
        return it->second;
    rocblas_handle h = nullptr;
    if (rocblas_create_handle(&h) != rocblas_status_success)
    {
        *rc = sv2::set_error(SV2_EDEVICE, "gemm: rocblas_create_handle failed");
        return nullptr;
    }
    handles[device] = h;
    return h;
}

} // namespace

int gemm_rows(hipStream_t stream, int dtype, int rows, int in, int out, const void* x, const void* w, void* y)
{
    if (rows == 0)
        return SV2_OK;
    int rc = SV2_OK;
    rocblas_handle h = blas_handle(&rc);
    if (!h)
        return rc;
    const rocblas_datatype t = dtype == SV2_F32 ? rocblas_datatype_f32_r : rocblas_datatype_f16_r;
    const float alpha = 1.f;
    const float beta = 0.f;
    rocblas_set_stream(h, stream);
    // column-major view: Y^T [out x rows] = W [out x in] * X^T [in x rows]
    const rocblas_status st = rocblas_gemm_ex(h, rocblas_operation_transpose, rocblas_operation_none, out, rows, in,
                                              &alpha, w, t, in, x, t, in, &beta, y, t, out, y, t, out,
                                              rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
    if (st != rocblas_status_success)
        return sv2::set_error(SV2_EDEVICE, std::string("gemm: rocblas_gemm_ex failed: ") + rocblas_status_to_string(st));
    return SV2_OK;
}

} // namespace sv2
