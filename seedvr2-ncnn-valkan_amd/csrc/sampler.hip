// The Euler sampler around the DiT on the device (src/model/sampler.cpp and
// the latent preparation of src/core/engine.cpp of the reference): the
// condition latent, the 33-channel DiT input, classifier-free guidance with
// the standard-deviation rescale, and the Euler / v-lerp update.  Latents are
// fp32 [C][T][H][W] arrays; every operation is elementwise, in fp32 with the
// reference's operation order and no fused multiply-add, so the outputs equal
// the reference's bit for bit (the guidance rescale factor comes from double
// sums whose order differs from the reference's, within an ulp of it).
#include "sv2_internal.h"

#include <cmath>

// Every float expression here is evaluated as written: no contraction into
// fused multiply-adds, on the device and on the host.
#pragma clang fp contract(off)

namespace sv2
{
namespace
{

constexpr int kThreads = 256;
constexpr int kReduceBlocks = 1024; // partial sums of the guidance statistics

unsigned blocks_for(long long n)
{
    return static_cast<unsigned>((n + kThreads - 1) / kThreads);
}

int launch_status(const char* what)
{
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? SV2_OK : hip_error(err, what);
}

// engine.cpp:106-122: (1 - ratio) * encoded + ratio * noise
__global__ __launch_bounds__(kThreads) void condition_kernel(const float* a, const float* b, float* out,
                                                             long long count, float ratio)
{
    const long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= count)
        return;
    const float wa = 1.0f - ratio;
    const float left = wa * a[i];
    const float right = ratio * b[i];
    out[i] = left + right;
}

// engine.cpp:125-149: channels 0-15 the latent, 16-31 the condition, 32 ones.
// Channel-major: [16][tokens] sources into [33][tokens] (the CPU engine);
// token-major: [tokens][16] sources into [tokens][33] (sampler.cpp:337-357).
__global__ __launch_bounds__(kThreads) void dit_input_kernel(const float* latent, const float* condition, float* out,
                                                             long long tokens, int channel_major)
{
    const long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= 33 * tokens)
        return;
    long long c, t;
    if (channel_major)
    {
        c = i / tokens;
        t = i - c * tokens;
        out[i] = c < 16 ? latent[c * tokens + t] : (c < 32 ? condition[(c - 16) * tokens + t] : 1.0f);
    }
    else
    {
        t = i / 33;
        c = i - t * 33;
        out[i] = c < 16 ? latent[t * 16 + c] : (c < 32 ? condition[t * 16 + c - 16] : 1.0f);
    }
}

// sampler.cpp:217-218: neg + scale * (pos - neg); with `partial` (the
// rescale), each block also writes its double sums of pos, pos^2, out, out^2
// (grid-stride over the elements, fixed order per block).
__global__ __launch_bounds__(kThreads) void cfg_kernel(const float* pos, const float* neg, float* out,
                                                       long long count, float scale, double* partial)
{
    double sp = 0.0, spp = 0.0, so = 0.0, soo = 0.0;
    const long long stride = static_cast<long long>(gridDim.x) * kThreads;
    for (long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; i < count; i += stride)
    {
        const float p = pos[i];
        const float n = neg[i];
        const float diff = p - n;
        const float scaled = scale * diff;
        const float o = n + scaled;
        out[i] = o;
        if (partial)
        {
            sp += p;
            spp += static_cast<double>(p) * p;
            so += o;
            soo += static_cast<double>(o) * o;
        }
    }
    if (!partial)
        return;
    __shared__ double red[4][kThreads];
    red[0][threadIdx.x] = sp;
    red[1][threadIdx.x] = spp;
    red[2][threadIdx.x] = so;
    red[3][threadIdx.x] = soo;
    __syncthreads();
    for (int s = kThreads / 2; s > 0; s >>= 1)
    {
        if (static_cast<int>(threadIdx.x) < s)
            for (int k = 0; k < 4; k++)
                red[k][threadIdx.x] += red[k][threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x < 4)
        partial[blockIdx.x * 4 + threadIdx.x] = red[threadIdx.x][0];
}

// sampler.cpp:41-62 (unbiased standard deviation from the sums) and :219-235:
// factor = rescale * std(pos) / std(out) + (1 - rescale) when std(out) > 0.
// One block: thread t adds the partials of blocks t, t + 256, ... in that
// order, then a fixed tree over the threads, so the factor does not depend
// on scheduling.  factor_out[0] = factor, [1] = 1 when it applies.
__global__ __launch_bounds__(kThreads) void cfg_factor_kernel(const double* partial, int nblocks, long long count,
                                                              float rescale, float* factor_out)
{
    __shared__ double red[4][kThreads];
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    for (int b = threadIdx.x; b < nblocks; b += kThreads)
        for (int k = 0; k < 4; k++)
            acc[k] += partial[4 * b + k];
    for (int k = 0; k < 4; k++)
        red[k][threadIdx.x] = acc[k];
    __syncthreads();
    for (int s = kThreads / 2; s > 0; s >>= 1)
    {
        if (static_cast<int>(threadIdx.x) < s)
            for (int k = 0; k < 4; k++)
                red[k][threadIdx.x] += red[k][threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x != 0)
        return;
    const double sp = red[0][0], spp = red[1][0], so = red[2][0], soo = red[3][0];
    double std_pos = 0.0, std_out = 0.0;
    if (count > 1)
    {
        const double n = static_cast<double>(count);
        std_pos = sqrt(fmax(0.0, (spp - sp * sp / n) / (n - 1)));
        std_out = sqrt(fmax(0.0, (soo - so * so / n) / (n - 1)));
    }
    if (std_out > 0.0)
    {
        factor_out[0] = static_cast<float>(static_cast<double>(rescale) * std_pos / std_out +
                                           static_cast<double>(1.0f - rescale));
        factor_out[1] = 1.0f;
    }
    else
    {
        factor_out[0] = 1.0f;
        factor_out[1] = 0.0f;
    }
}

__global__ __launch_bounds__(kThreads) void cfg_scale_kernel(float* out, long long count, const float* factor)
{
    const long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= count || factor[1] == 0.0f)
        return;
    out[i] *= factor[0];
}

// sampler.cpp:253-263: x0 = x - bt * pred, xT = x + at * pred,
// out = as * x0 + bs * xT (endpoint: bs = 0, as = 1 gives out = x0 exactly).
__global__ __launch_bounds__(kThreads) void euler_kernel(const float* pred, const float* cur, float* out,
                                                         long long count, float bt, float at, float as, float bs,
                                                         int endpoint)
{
    const long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= count)
        return;
    const float x = cur[i];
    const float p = pred[i];
    const float x0 = x - bt * p;
    if (endpoint)
    {
        out[i] = x0;
        return;
    }
    const float xT = x + at * p;
    const float left = as * x0;
    const float right = bs * xT;
    out[i] = left + right;
}

int check_count(long long count, const char* what)
{
    if (count < 0 || count / kThreads >= (1LL << 31))
        return set_error(SV2_EINVAL, std::string(what) + ": bad element count");
    return SV2_OK;
}

} // namespace
} // namespace sv2

extern "C" {

int sv2_euler_timesteps(int steps, float* out)
try
{
    if (!out)
        return sv2::set_error(SV2_EINVAL, "sv2_euler_timesteps: null output");
    // EulerSampler::EulerSampler (sampler.cpp:181-187): at least one step
    const int n = steps < 1 ? 1 : steps;
    for (int i = 0; i < n; i++)
        out[i] = 1000.0f * (1.0f - static_cast<float>(i) / n);
    return n;
}
catch (...)
{
    return sv2::caught_exception("sv2_euler_timesteps");
}

float sv2_condition_ratio(float noise_scale, int frames, int height, int width)
{
    // transformed_condition_timestep (engine.cpp:79-92) over the encoded
    // latent's [T][H][W], divided by 1000 as make_condition_latent does
    // (engine.cpp:110): the resolution-dependent shift of the noise level.
    const float timestep = noise_scale * 1000.0f;
    if (timestep == 0.0f)
        return 0.0f;
    const float f = static_cast<float>((frames - 1) * 4 + 1);
    const float h = static_cast<float>(height * 8);
    const float w = static_cast<float>(width * 8);
    const float x1 = 256.0f * 256.0f * 37.0f;
    const float x2 = 1280.0f * 720.0f * 145.0f;
    const float shift = 1.0f + (h * w * f - x1) * (5.0f - 1.0f) / (x2 - x1);
    const float normalized = timestep / 1000.0f;
    return 1000.0f * shift * normalized / (1.0f + (shift - 1.0f) * normalized) / 1000.0f;
}

int sv2_make_condition(const float* encoded, const float* noise, float* out, int64_t count, float ratio,
                       void* stream)
try
{
    using namespace sv2;
    int rc = check_count(count, "sv2_make_condition");
    if (rc != SV2_OK)
        return rc;
    if (count == 0)
        return SV2_OK;
    if (!encoded || !noise || !out)
        return set_error(SV2_EINVAL, "sv2_make_condition: null pointer");
    hipLaunchKernelGGL(condition_kernel, dim3(blocks_for(count)), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                       encoded, noise, out, static_cast<long long>(count), ratio);
    return launch_status("condition_kernel launch");
}
catch (...)
{
    return sv2::caught_exception("sv2_make_condition");
}

int sv2_make_dit_input(const float* latent, const float* condition, float* out, int64_t tokens, int channel_major,
                       void* stream)
try
{
    using namespace sv2;
    int rc = check_count(33 * tokens, "sv2_make_dit_input");
    if (rc != SV2_OK)
        return rc;
    if (tokens == 0)
        return SV2_OK;
    if (!latent || !condition || !out)
        return set_error(SV2_EINVAL, "sv2_make_dit_input: null pointer");
    hipLaunchKernelGGL(dit_input_kernel, dim3(blocks_for(33 * tokens)), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), latent, condition, out, static_cast<long long>(tokens),
                       channel_major ? 1 : 0);
    return launch_status("dit_input_kernel launch");
}
catch (...)
{
    return sv2::caught_exception("sv2_make_dit_input");
}

int64_t sv2_cfg_workspace_size(int64_t count)
try
{
    (void)count;
    // partial sums of every reduction block + the factor
    return static_cast<int64_t>(sv2::kReduceBlocks) * 4 * sizeof(double) + 256;
}
catch (...)
{
    return sv2::caught_exception("sv2_cfg_workspace_size");
}

int sv2_apply_cfg(const float* positive, const float* negative, float* out, int64_t count, float scale,
                  float rescale, void* workspace, size_t workspace_bytes, void* stream_ptr)
try
{
    using namespace sv2;
    int rc = check_count(count, "sv2_apply_cfg");
    if (rc != SV2_OK)
        return rc;
    if (count == 0)
        return SV2_OK;
    if (!positive || !negative || !out)
        return set_error(SV2_EINVAL, "sv2_apply_cfg: null pointer");
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    if (rescale == 0.0f)
    {
        const int nb = static_cast<int>(std::min<long long>(blocks_for(count), 1LL << 20));
        hipLaunchKernelGGL(cfg_kernel, dim3(nb), dim3(kThreads), 0, stream, positive, negative, out,
                           static_cast<long long>(count), scale, static_cast<double*>(nullptr));
        return launch_status("cfg_kernel launch");
    }
    if (!workspace || static_cast<int64_t>(workspace_bytes) < sv2_cfg_workspace_size(count))
        return set_error(SV2_EINVAL, "sv2_apply_cfg: the rescale needs sv2_cfg_workspace_size bytes of workspace");
    double* partial = static_cast<double*>(workspace);
    float* factor = reinterpret_cast<float*>(static_cast<char*>(workspace) + kReduceBlocks * 4 * sizeof(double));
    const int nb = static_cast<int>(std::min<long long>(blocks_for(count), kReduceBlocks));
    hipLaunchKernelGGL(cfg_kernel, dim3(nb), dim3(kThreads), 0, stream, positive, negative, out,
                       static_cast<long long>(count), scale, partial);
    if ((rc = launch_status("cfg_kernel launch")) != SV2_OK)
        return rc;
    hipLaunchKernelGGL(cfg_factor_kernel, dim3(1), dim3(kThreads), 0, stream, partial, nb,
                       static_cast<long long>(count), rescale, factor);
    if ((rc = launch_status("cfg_factor_kernel launch")) != SV2_OK)
        return rc;
    hipLaunchKernelGGL(cfg_scale_kernel, dim3(blocks_for(count)), dim3(kThreads), 0, stream, out,
                       static_cast<long long>(count), factor);
    return launch_status("cfg_scale_kernel launch");
}
catch (...)
{
    return sv2::caught_exception("sv2_apply_cfg");
}

int sv2_euler_step(const float* prediction, const float* current, float* out, int64_t count, float timestep,
                   float next_timestep, void* stream)
try
{
    using namespace sv2;
    int rc = check_count(count, "sv2_euler_step");
    if (rc != SV2_OK)
        return rc;
    if (count == 0)
        return SV2_OK;
    if (!prediction || !current || !out)
        return set_error(SV2_EINVAL, "sv2_euler_step: null pointer");
    // EulerSampler::step_to (sampler.cpp:253-256)
    const float bt = timestep / 1000.0f;
    const float at = 1.0f - bt;
    const float bs = std::fmin(std::fmax(next_timestep / 1000.0f, 0.0f), 1.0f);
    const float as = 1.0f - bs;
    hipLaunchKernelGGL(euler_kernel, dim3(blocks_for(count)), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                       prediction, current, out, static_cast<long long>(count), bt, at, as, bs, 0);
    return launch_status("euler_kernel launch");
}
catch (...)
{
    return sv2::caught_exception("sv2_euler_step");
}

int sv2_euler_endpoint(const float* prediction, const float* current, float* out, int64_t count, float timestep,
                       void* stream)
try
{
    using namespace sv2;
    int rc = check_count(count, "sv2_euler_endpoint");
    if (rc != SV2_OK)
        return rc;
    if (count == 0)
        return SV2_OK;
    if (!prediction || !current || !out)
        return set_error(SV2_EINVAL, "sv2_euler_endpoint: null pointer");
    // EulerSampler::endpoint (sampler.cpp:280-282)
    const float bt = timestep / 1000.0f;
    hipLaunchKernelGGL(euler_kernel, dim3(blocks_for(count)), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                       prediction, current, out, static_cast<long long>(count), bt, 0.0f, 1.0f, 0.0f, 1);
    return launch_status("euler_kernel launch");
}
catch (...)
{
    return sv2::caught_exception("sv2_euler_endpoint");
}

} // extern "C"
