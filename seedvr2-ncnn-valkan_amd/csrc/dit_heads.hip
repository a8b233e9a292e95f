// Data-movement kernels of the DiT input and output heads
// (src/layers/seedvr2_dit_input.cpp, src/layers/seedvr2_dit_output.cpp of the
// reference): the 1x2x2 patchify gather, the timestep sinusoid, the
// unpatchify scatter and an fp32 -> compute-dtype conversion.  All are
// HBM-bound permutations; one thread writes one output element so that
// writes are coalesced along the channel (or token) axis they run on.
#include "sv2_internal.h"
#include "vec_io.h"

#include <cmath>

namespace sv2
{
namespace
{

using namespace vec;

template <typename T>
__device__ inline void store1(void* base, long long i, float v);
template <>
__device__ inline void store1<F32>(void* base, long long i, float v)
{
    static_cast<float*>(base)[i] = v;
}
template <>
__device__ inline void store1<F16>(void* base, long long i, float v)
{
    static_cast<_Float16*>(base)[i] = static_cast<_Float16>(v);
}
template <>
__device__ inline void store1<BF16>(void* base, long long i, float v)
{
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    if ((u & 0x7fffffffu) > 0x7f800000u)
        u = 0x7fc00000u;
    else
        u += 0x7fffu + ((u >> 16) & 1u);
    static_cast<uint16_t*>(base)[i] = static_cast<uint16_t>(u >> 16);
}

template <typename T>
__device__ inline float load1(const void* base, long long i);
template <>
__device__ inline float load1<F32>(const void* base, long long i)
{
    return static_cast<const float*>(base)[i];
}
template <>
__device__ inline float load1<F16>(const void* base, long long i)
{
    return static_cast<float>(static_cast<const _Float16*>(base)[i]);
}
template <>
__device__ inline float load1<BF16>(const void* base, long long i)
{
    return __builtin_bit_cast(float, static_cast<uint32_t>(static_cast<const uint16_t*>(base)[i]) << 16);
}

// patches[p][(dy*2 + dx)*C + c] = video[token (t, 2y+dy, 2x+dx)][c]
// (seedvr2_dit_input.cpp:336-352), for the patched grid T x h x w.  The
// source is token-major [T*H*W, C] (the layer's vid blob) or channel-major
// [C][T][H][W] (the DiT's latent, flattened by dit.cpp:66-80 on the host in
// the reference).
template <typename TO>
__global__ __launch_bounds__(256) void patchify_kernel(const float* video, void* patches, int T, int h, int w, int C,
                                                       int channel_major)
{
    const long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    const long long cols = 4LL * C;
    const long long total = static_cast<long long>(T) * h * w * cols;
    if (i >= total)
        return;
    const long long p = i / cols;
    const int j = static_cast<int>(i - p * cols);
    const int q = j / C;
    const int c = j - q * C;
    const int dy = q >> 1;
    const int dx = q & 1;
    const int x = static_cast<int>(p % w);
    const int y = static_cast<int>((p / w) % h);
    const int t = static_cast<int>(p / (static_cast<long long>(w) * h));
    const int H = 2 * h;
    const int W = 2 * w;
    const long long token = (static_cast<long long>(t) * H + 2 * y + dy) * W + 2 * x + dx;
    const long long src = channel_major ? static_cast<long long>(c) * T * H * W + token : token * C + c;
    store1<TO>(patches, i, video[src]);
}

// output[token (t, 2y+dy, 2x+dx)][c] = projected[p][(dy*2 + dx)*OC + c]
// (seedvr2_dit_output.cpp:394-413); token-major [T*H*W, OC] or channel-major
// [OC][T][H][W] (dit.cpp:82-95) fp32 output.
template <typename TI>
__global__ __launch_bounds__(256) void unpatchify_kernel(const void* projected, float* output, int T, int h, int w,
                                                         int OC, int channel_major)
{
    const long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    const int H = 2 * h;
    const int W = 2 * w;
    const long long tokens = static_cast<long long>(T) * H * W;
    if (i >= tokens * OC)
        return;
    long long token;
    int c;
    if (channel_major)
    {
        c = static_cast<int>(i / tokens);
        token = i - static_cast<long long>(c) * tokens;
    }
    else
    {
        token = i / OC;
        c = static_cast<int>(i - token * OC);
    }
    const int X = static_cast<int>(token % W);
    const int Y = static_cast<int>((token / W) % H);
    const int t = static_cast<int>(token / (static_cast<long long>(W) * H));
    const long long p = (static_cast<long long>(t) * h + (Y >> 1)) * w + (X >> 1);
    const int q = (Y & 1) * 2 + (X & 1);
    output[i] = load1<TI>(projected, p * 4 * OC + q * OC + c);
}

// The timestep sinusoid (seedvr2_dit_input.cpp:365-374), fp32:
// f_i = exp(-log(10000) * i / half), out[i] = sin(t f_i), out[i + half] = cos(t f_i).
__global__ __launch_bounds__(256) void sinusoid_kernel(float* out, float timestep, int half)
{
#pragma clang fp contract(off)
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= half)
        return;
    const float neg_log = -logf(10000.f);
    const float frequency = expf(neg_log * static_cast<float>(i) / static_cast<float>(half));
    const float value = timestep * frequency;
    out[i] = sinf(value);
    out[i + half] = cosf(value);
}

template <typename TO>
__global__ __launch_bounds__(256) void from_f32_kernel(void* dst, const float* src, long long count)
{
    const long long i = (static_cast<long long>(blockIdx.x) * 256 + threadIdx.x) * 8;
    if (i >= count)
        return;
    float a[8];
    ld8<F32>(src, i, a);
    st8<TO>(dst, i, a);
}

unsigned blocks_for(long long n)
{
    return static_cast<unsigned>((n + 255) / 256);
}

int launch_status(const char* what)
{
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? SV2_OK : hip_error(err, what);
}

} // namespace

int launch_patchify(const float* video, void* patches, int dtype, int T, int h, int w, int C, int channel_major,
                    hipStream_t stream)
{
    const long long total = static_cast<long long>(T) * h * w * 4 * C;
    if (total <= 0 || total / 256 >= (1LL << 31))
        return set_error(SV2_EINVAL, "patchify: bad shape");
    const dim3 grid(blocks_for(total));
    if (dtype == SV2_F32)
        hipLaunchKernelGGL(patchify_kernel<F32>, grid, dim3(256), 0, stream, video, patches, T, h, w, C, channel_major);
    else if (dtype == SV2_F16)
        hipLaunchKernelGGL(patchify_kernel<F16>, grid, dim3(256), 0, stream, video, patches, T, h, w, C, channel_major);
    else
        hipLaunchKernelGGL(patchify_kernel<BF16>, grid, dim3(256), 0, stream, video, patches, T, h, w, C,
                           channel_major);
    return launch_status("patchify_kernel launch");
}

int launch_unpatchify(const void* projected, float* output, int dtype, int T, int h, int w, int OC, int channel_major,
                      hipStream_t stream)
{
    const long long total = static_cast<long long>(T) * h * w * 4 * OC;
    if (total <= 0 || total / 256 >= (1LL << 31))
        return set_error(SV2_EINVAL, "unpatchify: bad shape");
    const dim3 grid(blocks_for(total));
    if (dtype == SV2_F32)
        hipLaunchKernelGGL(unpatchify_kernel<F32>, grid, dim3(256), 0, stream, projected, output, T, h, w, OC,
                           channel_major);
    else if (dtype == SV2_F16)
        hipLaunchKernelGGL(unpatchify_kernel<F16>, grid, dim3(256), 0, stream, projected, output, T, h, w, OC,
                           channel_major);
    else
        hipLaunchKernelGGL(unpatchify_kernel<BF16>, grid, dim3(256), 0, stream, projected, output, T, h, w, OC,
                           channel_major);
    return launch_status("unpatchify_kernel launch");
}

int launch_sinusoid(float* out, float timestep, int dim, hipStream_t stream)
{
    if (dim <= 0 || dim % 2 != 0)
        return set_error(SV2_EINVAL, "sinusoid: dim must be even and positive");
    hipLaunchKernelGGL(sinusoid_kernel, dim3(blocks_for(dim / 2)), dim3(256), 0, stream, out, timestep, dim / 2);
    return launch_status("sinusoid_kernel launch");
}

int launch_from_f32(void* dst, const float* src, int dtype, long long count, hipStream_t stream)
{
    if (count < 0 || count % 8 != 0)
        return set_error(SV2_EINVAL, "from_f32: count must be a multiple of 8");
    if (count == 0)
        return SV2_OK;
    if (dtype == SV2_F32)
    {
        const hipError_t err = hipMemcpyAsync(dst, src, count * sizeof(float), hipMemcpyDeviceToDevice, stream);
        return err == hipSuccess ? SV2_OK : hip_error(err, "from_f32 copy");
    }
    const dim3 grid(blocks_for(count / 8));
    if (dtype == SV2_F16)
        hipLaunchKernelGGL(from_f32_kernel<F16>, grid, dim3(256), 0, stream, dst, src, count);
    else
        hipLaunchKernelGGL(from_f32_kernel<BF16>, grid, dim3(256), 0, stream, dst, src, count);
    return launch_status("from_f32_kernel launch");
}

} // namespace sv2
