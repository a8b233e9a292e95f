// 8-element vector loads and stores of fp32 / fp16 / bf16 device tensors,
// converting to and from fp32 registers (16 bytes per lane for the half
// types, 2 x 16 bytes for fp32).  Offsets are in elements and must be
// multiples of 8.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sv2
{
namespace vec
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
// The raw bytes of 8 elements (16 for fp16 / bf16, 32 for fp32), for kernels
// that keep data in flight in registers before converting it.
template <typename T>
struct Raw8
{
    uint4 r[1];
};
template <>
struct Raw8<F32>
{
    uint4 r[2];
};

template <typename T>
__device__ inline void ld_raw8(const void* base, long long i, Raw8<T>& v)
{
    constexpr int n = sizeof(Raw8<T>) / sizeof(uint4);
    const uint4* p = reinterpret_cast<const uint4*>(static_cast<const char*>(base) + i * 2 * n);
#pragma unroll
    for (int k = 0; k < n; k++)
        v.r[k] = p[k];
}

__device__ inline void raw8_float(const Raw8<F32>& v, float x[8])
{
#pragma unroll
    for (int k = 0; k < 2; k++)
    {
        x[4 * k] = __builtin_bit_cast(float, v.r[k].x);
        x[4 * k + 1] = __builtin_bit_cast(float, v.r[k].y);
        x[4 * k + 2] = __builtin_bit_cast(float, v.r[k].z);
        x[4 * k + 3] = __builtin_bit_cast(float, v.r[k].w);
    }
}
__device__ inline void raw8_float(const Raw8<F16>& v, float x[8])
{
    const f16x8 h = __builtin_bit_cast(f16x8, v.r[0]);
#pragma unroll
    for (int e = 0; e < 8; e++)
        x[e] = static_cast<float>(h[e]);
}
__device__ inline void raw8_float(const Raw8<BF16>& v, float x[8])
{
    const uint32_t w[4] = {v.r[0].x, v.r[0].y, v.r[0].z, v.r[0].w};
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

} // namespace vec
} // namespace sv2
