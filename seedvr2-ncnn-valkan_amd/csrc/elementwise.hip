// Row-wise and element-wise kernels around the attention of the SeedVR2-3B DiT
// block: token RMSNorm fused with ada input modulation, gated residual, and
// the SwiGLU gate.  All three are HBM-bound; they move 16 bytes per lane per
// access (8 halfs or 4+4 floats) and read every element once.
#include "sv2_internal.h"

#include <cmath>

namespace sv2
{
namespace
{

struct F32
{
};
struct F16
{
};
struct BF16
{
};

template <typename T>
__device__ inline void ld8(const void* base, long long i, float x[8]);
template <typename T>
__device__ inline void st8(void* base, long long i, const float x[8]);

template <>
__device__ inline void ld8<F32>(const void* base, long long i, float x[8])
{
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + i);
    const float4 a = p[0];
    const float4 b = p[1];
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}
template <>
__device__ inline void st8<F32>(void* base, long long i, const float x[8])
{
    float4* p = reinterpret_cast<float4*>(static_cast<float*>(base) + i);
    p[0] = make_float4(x[0], x[1], x[2], x[3]);
    p[1] = make_float4(x[4], x[5], x[6], x[7]);
}

typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;

template <>
__device__ inline void ld8<F16>(const void* base, long long i, float x[8])
{
    const f16x8 v = *reinterpret_cast<const f16x8*>(static_cast<const _Float16*>(base) + i);
#pragma unroll
    for (int e = 0; e < 8; e++)
        x[e] = static_cast<float>(v[e]);
}
template <>
__device__ inline void st8<F16>(void* base, long long i, const float x[8])
{
    f16x8 v;
#pragma unroll
    for (int e = 0; e < 8; e++)
        v[e] = static_cast<_Float16>(x[e]);
    *reinterpret_cast<f16x8*>(static_cast<_Float16*>(base) + i) = v;
}

// float -> bf16 with round-to-nearest-even (NaN kept quiet).
__device__ inline uint32_t to_bf16_bits(float f)
{
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7fffffffu) > 0x7f800000u)
        return 0x7fc0u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

template <>
__device__ inline void ld8<BF16>(const void* base, long long i, float x[8])
{
    const uint4 v = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + i);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; e++)
    {
        x[2 * e] = __builtin_bit_cast(float, w[e] << 16);
        x[2 * e + 1] = __builtin_bit_cast(float, w[e] & 0xffff0000u);
    }
}
template <>
__device__ inline void st8<BF16>(void* base, long long i, const float x[8])
{
    uint4 v;
    v.x = to_bf16_bits(x[0]) | (to_bf16_bits(x[1]) << 16);
    v.y = to_bf16_bits(x[2]) | (to_bf16_bits(x[3]) << 16);
    v.z = to_bf16_bits(x[4]) | (to_bf16_bits(x[5]) << 16);
    v.w = to_bf16_bits(x[6]) | (to_bf16_bits(x[7]) << 16);
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(base) + i) = v;
}

// Most 8-element vectors one lane keeps in registers per row (dim <= 8*64*kMaxVec).
constexpr int kMaxVec = 8;

// One wave per row.  Follows apply_rmsnorm + apply_ada_input
// (seedvr2_dit_block.cpp:770-805): a double sum of squares, inv =
// 1/sqrtf(float(ss/dim) + eps), x *= inv, then
// x = x*(emb[c*6+slot+1] + scale[c]) + emb[c*6+slot] + shift[c] evaluated left
// to right in fp32 with no fused multiply-add.  The row stays in registers
// between the reduction and the write, so HBM sees one read and one write.
template <typename T>
__global__ __launch_bounds__(256) void rmsnorm_ada_kernel(const void* x, void* y, int rows, int dim, float eps,
                                                          const float* emb, const float* shift, const float* scale,
                                                          int slot, int has_ada)
{
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows)
        return;
    const int nvec = dim / 8;
    const long long base = static_cast<long long>(row) * dim;
    float v[kMaxVec][8];
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < kMaxVec; k++)
    {
        const int vi = lane + 64 * k;
        if (vi < nvec)
        {
            ld8<T>(x, base + vi * 8, v[k]);
#pragma unroll
            for (int e = 0; e < 8; e++)
                ss += static_cast<double>(v[k][e]) * static_cast<double>(v[k][e]);
        }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1)
        ss += __shfl_xor(ss, m);
    const float inv = 1.f / sqrtf(static_cast<float>(ss / dim) + eps);
#pragma unroll
    for (int k = 0; k < kMaxVec; k++)
    {
        const int vi = lane + 64 * k;
        if (vi < nvec)
        {
            float out[8];
#pragma unroll
            for (int e = 0; e < 8; e++)
            {
                const int c = vi * 8 + e;
                float t = v[k][e] * inv;
                if (has_ada)
                {
                    const float mul = emb[c * 6 + slot + 1] + scale[c];
                    const float add1 = t * mul;
                    const float add2 = add1 + emb[c * 6 + slot];
                    t = add2 + shift[c];
                }
                out[e] = t;
            }
            st8<T>(y, base + vi * 8, out);
        }
    }
}

// seedvr2_dit_block.cpp:807-825 (mode 0), :1198-1209 (mode 1), :1225-1246 (mode 2).
template <typename T>
__global__ __launch_bounds__(256) void ada_residual_kernel(void* x, const void* residual, long long count, int dim,
                                                           const float* emb, const float* gate, int slot, int mode)
{
#pragma clang fp contract(off)
    const long long i = (static_cast<long long>(blockIdx.x) * 256 + threadIdx.x) * 8;
    if (i >= count)
        return;
    float a[8];
    ld8<T>(x, i, a);
    float out[8];
    if (mode == 2)
    {
#pragma unroll
        for (int e = 0; e < 8; e++)
            out[e] = a[e] * 2.f;
    }
    else
    {
        float r[8];
        ld8<T>(residual, i, r);
        if (mode == 1)
        {
#pragma unroll
            for (int e = 0; e < 8; e++)
                out[e] = a[e] + r[e];
        }
        else
        {
            const int c0 = static_cast<int>(i % dim);
#pragma unroll
            for (int e = 0; e < 8; e++)
            {
                const int c = c0 + e;
                const float mul = emb[c * 6 + slot] + gate[c];
                const float t = a[e] * mul;
                out[e] = t + r[e];
            }
        }
    }
    st8<T>(x, i, out);
}

// silu(g) * v with silu(g) = g / (1 + exp(-g)) (seedvr2_dit_block.cpp:58-61, :1103-1109).
template <typename T>
__global__ __launch_bounds__(256) void swiglu_kernel(void* gate, const void* value, long long count)
{
#pragma clang fp contract(off)
    const long long i = (static_cast<long long>(blockIdx.x) * 256 + threadIdx.x) * 8;
    if (i >= count)
        return;
    float g[8];
    float v[8];
    ld8<T>(gate, i, g);
    ld8<T>(value, i, v);
#pragma unroll
    for (int e = 0; e < 8; e++)
    {
        const float den = 1.f + expf(-g[e]);
        g[e] = (g[e] / den) * v[e];
    }
    st8<T>(gate, i, g);
}

bool dtype_ok(int t)
{
    return t == SV2_F32 || t == SV2_F16 || t == SV2_BF16;
}

} // namespace
} // namespace sv2

extern "C" {

int sv2_rmsnorm_ada(const void* x, void* y, int io_dtype, int rows, int dim, float eps, const float* emb,
                    const float* shift, const float* scale, int slot_base, int has_ada, void* stream_ptr)
{
    using namespace sv2;
    if (!dtype_ok(io_dtype) || rows < 0 || dim <= 0)
        return set_error(SV2_EINVAL, "rmsnorm_ada: bad dtype or shape");
    if (dim % 8 != 0 || dim > 8 * 64 * kMaxVec)
        return set_error(SV2_EUNSUPPORTED, "rmsnorm_ada: dim must be a multiple of 8 and <= 4096");
    if (rows == 0)
        return SV2_OK;
    if (!x || !y || (has_ada && (!emb || !shift || !scale)))
        return set_error(SV2_EINVAL, "rmsnorm_ada: null pointer");
    if (slot_base != 0 && slot_base != 3)
        return set_error(SV2_EINVAL, "rmsnorm_ada: slot_base must be 0 or 3");
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    const dim3 grid((rows + 3) / 4);
    if (io_dtype == SV2_F32)
        hipLaunchKernelGGL(rmsnorm_ada_kernel<F32>, grid, dim3(256), 0, stream, x, y, rows, dim, eps, emb, shift, scale,
                           slot_base, has_ada);
    else if (io_dtype == SV2_F16)
        hipLaunchKernelGGL(rmsnorm_ada_kernel<F16>, grid, dim3(256), 0, stream, x, y, rows, dim, eps, emb, shift, scale,
                           slot_base, has_ada);
    else
        hipLaunchKernelGGL(rmsnorm_ada_kernel<BF16>, grid, dim3(256), 0, stream, x, y, rows, dim, eps, emb, shift,
                           scale, slot_base, has_ada);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? SV2_OK : hip_error(err, "rmsnorm_ada_kernel launch");
}

int sv2_ada_residual(void* x, const void* residual, int io_dtype, int rows, int dim, const float* emb,
                     const float* gate, int slot_base, int mode, void* stream_ptr)
{
    using namespace sv2;
    if (!dtype_ok(io_dtype) || rows < 0 || dim <= 0 || mode < 0 || mode > 2)
        return set_error(SV2_EINVAL, "ada_residual: bad dtype, shape or mode");
    if (dim % 8 != 0)
        return set_error(SV2_EUNSUPPORTED, "ada_residual: dim must be a multiple of 8");
    if (rows == 0)
        return SV2_OK;
    if (!x || (mode != 2 && !residual) || (mode == 0 && (!emb || !gate)))
        return set_error(SV2_EINVAL, "ada_residual: null pointer");
    if (slot_base != 0 && slot_base != 3)
        return set_error(SV2_EINVAL, "ada_residual: slot_base must be 0 or 3");
    const long long count = static_cast<long long>(rows) * dim;
    const dim3 grid(static_cast<unsigned>((count / 8 + 255) / 256));
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    const int slot = slot_base + 2;
    if (io_dtype == SV2_F32)
        hipLaunchKernelGGL(ada_residual_kernel<F32>, grid, dim3(256), 0, stream, x, residual, count, dim, emb, gate,
                           slot, mode);
    else if (io_dtype == SV2_F16)
        hipLaunchKernelGGL(ada_residual_kernel<F16>, grid, dim3(256), 0, stream, x, residual, count, dim, emb, gate,
                           slot, mode);
    else
        hipLaunchKernelGGL(ada_residual_kernel<BF16>, grid, dim3(256), 0, stream, x, residual, count, dim, emb, gate,
                           slot, mode);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? SV2_OK : hip_error(err, "ada_residual_kernel launch");
}

int sv2_swiglu(void* gate, const void* value, int io_dtype, int64_t count, void* stream_ptr)
{
    using namespace sv2;
    if (!dtype_ok(io_dtype) || count < 0)
        return set_error(SV2_EINVAL, "swiglu: bad dtype or count");
    if (count % 8 != 0)
        return set_error(SV2_EUNSUPPORTED, "swiglu: count must be a multiple of 8");
    if (count == 0)
        return SV2_OK;
    if (!gate || !value)
        return set_error(SV2_EINVAL, "swiglu: null pointer");
    const dim3 grid(static_cast<unsigned>((count / 8 + 255) / 256));
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    if (io_dtype == SV2_F32)
        hipLaunchKernelGGL(swiglu_kernel<F32>, grid, dim3(256), 0, stream, gate, value, static_cast<long long>(count));
    else if (io_dtype == SV2_F16)
        hipLaunchKernelGGL(swiglu_kernel<F16>, grid, dim3(256), 0, stream, gate, value, static_cast<long long>(count));
    else
        hipLaunchKernelGGL(swiglu_kernel<BF16>, grid, dim3(256), 0, stream, gate, value, static_cast<long long>(count));
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? SV2_OK : hip_error(err, "swiglu_kernel launch");
}

} // extern "C"
