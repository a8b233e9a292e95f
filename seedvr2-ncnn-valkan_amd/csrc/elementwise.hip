// Row-wise and element-wise kernels around the attention of the SeedVR2-3B DiT
// block: token RMSNorm fused with ada input modulation, gated residual, and
// the SwiGLU gate.  All three are HBM-bound; they move 16 bytes per lane per
// access (8 halfs or 4+4 floats) and read every element once.
#include "sv2_internal.h"
#include "vec_io.h"

#include <cmath>
#include <type_traits>

namespace sv2
{
namespace
{

using namespace vec;

// 1.f / std::sqrt(float(ss / n) + eps) as the reference evaluates it
// (seedvr2_dit_block.cpp:770-782) from the double sum of squares: the
// double quotient rounded to float, then a correctly rounded float sqrt and
// divide (each formed in double and rounded once, which for float operands is
// the correctly rounded float result).
__device__ inline float reference_inv_rms(double ss, int n, float eps)
{
    const float mean = static_cast<float>(ss / static_cast<double>(n));
    const float root = static_cast<float>(__builtin_sqrt(static_cast<double>(mean + eps)));
    return static_cast<float>(1.0 / static_cast<double>(root));
}

// std::exp of a float as the fp32 parity mode evaluates it: correctly rounded
// (exp in double, rounded once); the 16-bit modes use the single-precision
// library exp.
template <typename T>
__device__ inline float exp_of(float x)
{
    if constexpr (std::is_same_v<T, F32>)
        return static_cast<float>(exp(static_cast<double>(x)));
    else
        return expf(x);
}

// Most 8-element vectors one lane keeps in registers per row (dim <= 8*64*kMaxVec).
constexpr int kMaxVec = 8;
// The same for rows of up to 2560 channels (fewer registers, more waves).
constexpr int kNarrowVec = 5;

// Operands of the ada modulation for 8 consecutive channels c0..c0+7.
//   input:  mul[c] = emb[c*6+slot+1] + scale[c], e0[c] = emb[c*6+slot], sh[c] = shift[c]
//   output: g[c]   = emb[c*6+slot+2] + gate[c]
// The reference's emb blob interleaves the six slots per channel ([dim][6]);
// EmbInput / EmbGate read it as it is (4-byte loads at a 24-byte stride).
// TableInput / TableGate read per-layer vectors precomputed by ada_table_kernel
// with the same fp32 additions, as 16-byte loads: the results are identical.
struct EmbInput
{
    const float* emb;
    const float* shift;
    const float* scale;
    int slot;
    __device__ void load(int c0, float mul[8], float e0[8], float sh[8]) const
    {
#pragma clang fp contract(off)
#pragma unroll
        for (int e = 0; e < 8; e++)
        {
            const int c = c0 + e;
            mul[e] = emb[c * 6 + slot + 1] + scale[c];
            e0[e] = emb[c * 6 + slot];
            sh[e] = shift[c];
        }
    }
};

struct TableInput
{
    const float* mul;
    const float* e0;
    const float* shift;
    __device__ void load(int c0, float m[8], float e[8], float sh[8]) const
    {
        ld8<F32>(mul, c0, m);
        ld8<F32>(e0, c0, e);
        ld8<F32>(shift, c0, sh);
    }
};

struct EmbGate
{
    const float* emb;
    const float* gate;
    int slot;
    __device__ void load(int c0, float g[8]) const
    {
#pragma clang fp contract(off)
#pragma unroll
        for (int e = 0; e < 8; e++)
            g[e] = emb[(c0 + e) * 6 + slot] + gate[c0 + e];
    }
};

struct TableGate
{
    const float* g;
    __device__ void load(int c0, float out[8]) const
    {
        ld8<F32>(g, c0, out);
    }
};

// Rows of one workgroup (4 waves, one row at a time per wave): 16 when the
// launch still fills the chip with them, else 4 (one per wave).
constexpr int kNormRowsPerBlock = 16;
constexpr int kNormRowsPerBlockFew = 4;

// Follows apply_rmsnorm + apply_ada_input (seedvr2_dit_block.cpp:770-805): a
// double sum of squares, inv = 1/sqrtf(float(ss/dim) + eps), x *= inv, then
// x = x*(emb[c*6+slot+1] + scale[c]) + emb[c*6+slot] + shift[c] evaluated left
// to right in fp32 with no fused multiply-add.  With `gamma` (the DiT output
// head's norm weight, seedvr2_dit_output.cpp:372-384) x = (x * inv) * gamma[c]
// before the modulation.  A row stays in registers between the reduction and
// the write, so HBM sees one read and one write.  The workgroup stages the
// modulation vectors (and gamma) in LDS once for its `rpb` rows (16 on large
// launches), so they are read from L2 once per 16 rows rather than once per
// row.  LDS: `tables`
// floats [mul | e0 | shift | gamma] of dim each (the ones in use).
template <typename T, typename Mod, int kVec, int rpb>
__global__ __launch_bounds__(256) void rmsnorm_ada_kernel(const void* x, void* y, int rows, int dim, float eps,
                                                          Mod mod, const float* gamma, int has_ada)
{
#pragma clang fp contract(off)
    extern __shared__ __attribute__((aligned(16))) float tab[];
    float* t_mul = tab;
    float* t_e0 = tab + dim;
    float* t_sh = tab + 2 * dim;
    float* t_gm = tab + (has_ada ? 3 * dim : 0);
    for (int c0 = threadIdx.x * 8; c0 < dim; c0 += 256 * 8)
    {
        if (has_ada)
        {
            float mul[8], e0[8], sh[8];
            mod.load(c0, mul, e0, sh);
            st8<F32>(t_mul, c0, mul);
            st8<F32>(t_e0, c0, e0);
            st8<F32>(t_sh, c0, sh);
        }
        if (gamma)
        {
            float gm[8];
            ld8<F32>(gamma, c0, gm);
            st8<F32>(t_gm, c0, gm);
        }
    }
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nvec = dim / 8;
    // each wave's next row is loaded while the current one is reduced and
    // written, so two rows per wave are in flight
    Raw8<T> cur[kVec];
    Raw8<T> nxt[kVec];
    int row = blockIdx.x * rpb + wave;
    if (row >= rows)
        return;
#pragma unroll
    for (int k = 0; k < kVec; k++)
        if (lane + 64 * k < nvec)
            ld_raw8<T>(x, static_cast<long long>(row) * dim + (lane + 64 * k) * 8, cur[k]);
    for (int r = 0; r < rpb / 4; r++, row += 4)
    {
        const bool more = r + 1 < rpb / 4 && row + 4 < rows;
        if (more)
        {
#pragma unroll
            for (int k = 0; k < kVec; k++)
                if (lane + 64 * k < nvec)
                    ld_raw8<T>(x, static_cast<long long>(row + 4) * dim + (lane + 64 * k) * 8, nxt[k]);
        }
        const long long base = static_cast<long long>(row) * dim;
        float v[kVec][8];
        double ss = 0.0;
#pragma unroll
        for (int k = 0; k < kVec; k++)
        {
            const int vi = lane + 64 * k;
            if (vi < nvec)
            {
                raw8_float(cur[k], v[k]);
#pragma unroll
                for (int e = 0; e < 8; e++)
                    ss += static_cast<double>(v[k][e]) * static_cast<double>(v[k][e]);
            }
        }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1)
            ss += __shfl_xor(ss, m);
        const float inv = reference_inv_rms(ss, dim, eps);
#pragma unroll
        for (int k = 0; k < kVec; k++)
        {
            const int vi = lane + 64 * k;
            if (vi < nvec)
            {
                const int c0 = vi * 8;
                float out[8];
#pragma unroll
                for (int e = 0; e < 8; e++)
                    out[e] = v[k][e] * inv;
                if (gamma)
                {
                    float gm[8];
                    ld8<F32>(t_gm, c0, gm);
#pragma unroll
                    for (int e = 0; e < 8; e++)
                        out[e] = out[e] * gm[e];
                }
                if (has_ada)
                {
                    float mul[8], e0[8], sh[8];
                    ld8<F32>(t_mul, c0, mul);
                    ld8<F32>(t_e0, c0, e0);
                    ld8<F32>(t_sh, c0, sh);
#pragma unroll
                    for (int e = 0; e < 8; e++)
                    {
                        const float add1 = out[e] * mul[e];
                        const float add2 = add1 + e0[e];
                        out[e] = add2 + sh[e];
                    }
                }
                st8<T>(y, base + c0, out);
            }
        }
        if (!more)
            return;
#pragma unroll
        for (int k = 0; k < kVec; k++)
            cur[k] = nxt[k];
    }
}

// seedvr2_dit_block.cpp:807-825 (mode 0), :1198-1209 (mode 1), :1225-1246
// (mode 2).  With `bias`, x = x + bias[c] first (the bias of the preceding
// InnerProduct, fused here instead of a pass of its own).
template <typename T, typename Gate>
__global__ __launch_bounds__(256) void ada_residual_kernel(void* x, const void* residual, long long count, int dim,
                                                           Gate gate, const float* bias, int mode)
{
#pragma clang fp contract(off)
    const long long i = (static_cast<long long>(blockIdx.x) * 256 + threadIdx.x) * 8;
    if (i >= count)
        return;
    const int c0 = static_cast<int>(i % dim);
    float a[8];
    ld8<T>(x, i, a);
    if (bias)
    {
        float b[8];
        ld8<F32>(bias, c0, b);
#pragma unroll
        for (int e = 0; e < 8; e++)
            a[e] = a[e] + b[e];
    }
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
            float g[8];
            gate.load(c0, g);
#pragma unroll
            for (int e = 0; e < 8; e++)
            {
                const float t = a[e] * g[e];
                out[e] = t + r[e];
            }
        }
    }
    st8<T>(x, i, out);
}

// Per-layer modulation vectors from the emb blob (see EmbInput / EmbGate):
// out[0][c] = emb[c*6+slot+1] + scale[c], out[1][c] = emb[c*6+slot],
// out[2][c] = emb[c*6+slot+2] + gate[c] (skipped when gate is NULL), for dim
// channels.
__global__ __launch_bounds__(256) void ada_table_kernel(const float* emb, const float* scale, const float* gate,
                                                        int slot, int dim, float* out)
{
#pragma clang fp contract(off)
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= dim)
        return;
    out[c] = emb[c * 6 + slot + 1] + scale[c];
    out[dim + c] = emb[c * 6 + slot];
    if (gate)
        out[2 * dim + c] = emb[c * 6 + slot + 2] + gate[c];
}

// Every modulation table of one block in one launch (each a
// ada_table_kernel table, in the same float operations): tables t = 0 .. n-1
// of [3][dim] at out + 3 * dim * t, slot 0 for even t (attention) and 3 for
// odd t (MLP), from scale[t] / gate[t]; then, when bias is not NULL,
// out[12 * dim + c] = (emb[c*6+2] + gate[0][c]) * bias[c], the video
// projection's bias moved past its gate (an InnerProduct bias for a product that adds it after its per-channel scaling).
struct BlockAda
{
    const float* scale[4];
    const float* gate[4];
    const float* bias;
    int tables;
};

__global__ __launch_bounds__(256) void block_tables_kernel(const float* emb, BlockAda a, int dim, float* out)
{
#pragma clang fp contract(off)
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= dim)
        return;
    for (int t = 0; t < a.tables; t++)
    {
        const int slot = (t & 1) ? 3 : 0;
        float* o = out + static_cast<long long>(3 * t) * dim;
        o[c] = emb[c * 6 + slot + 1] + a.scale[t][c];
        o[dim + c] = emb[c * 6 + slot];
        if (a.gate[t])
            o[2 * dim + c] = emb[c * 6 + slot + 2] + a.gate[t][c];
    }
    if (a.bias)
    {
        const float g = emb[c * 6 + 2] + a.gate[0][c];
        out[12LL * dim + c] = g * a.bias[c];
    }
}

// silu(g) * v with silu(g) = g / (1 + exp(-g)) (seedvr2_dit_block.cpp:58-61, :1103-1109).
// fp32 (the parity mode): the correctly rounded exp and an IEEE division, as
// the CPU layer.  fp16 / bf16: the hardware exp2 and reciprocal (each within
// about an fp32 ulp), which the 16-bit rounding of the result absorbs except
// at a rounding boundary (within one ulp of the output type); at 21600 x
// 6912 fp16 this took the launch from 141 to 137 us (6.5 TB/s of its 6 bytes
// per element).
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
        if constexpr (std::is_same_v<T, F32>)
        {
            const float den = 1.f + exp_of<T>(-g[e]);
            g[e] = (g[e] / den) * v[e];
        }
        else
        {
            const float den = 1.f + __builtin_amdgcn_exp2f(g[e] * -1.4426950408889634f);
            g[e] = (g[e] * __builtin_amdgcn_rcpf(den)) * v[e];
        }
    }
    st8<T>(gate, i, g);
}

// y[r][c] += b[c] (the bias of an InnerProduct whose matrix product ran
// without one; none when b is NULL), optionally followed by silu(v) = v / (1 +
// exp(-v)) (the time MLP of the DiT input head, seedvr2_dit_input.cpp:377-388).
template <typename T>
__global__ __launch_bounds__(256) void bias_rows_kernel(void* y, const float* b, long long count, int cols,
                                                        int silu)
{
#pragma clang fp contract(off)
    const long long i = (static_cast<long long>(blockIdx.x) * 256 + threadIdx.x) * 8;
    if (i >= count)
        return;
    float a[8];
    ld8<T>(y, i, a);
    const int c0 = static_cast<int>(i % cols);
#pragma unroll
    for (int e = 0; e < 8; e++)
    {
        if (b)
            a[e] += b[c0 + e];
        if (silu)
            a[e] = a[e] / (1.f + exp_of<T>(-a[e]));
    }
    st8<T>(y, i, a);
}

// dst (fp32) = src (dtype), 8 elements per lane.
template <typename T>
__global__ __launch_bounds__(256) void to_f32_kernel(float* dst, const void* src, long long count)
{
    const long long i = (static_cast<long long>(blockIdx.x) * 256 + threadIdx.x) * 8;
    if (i >= count)
        return;
    float a[8];
    ld8<T>(src, i, a);
    st8<F32>(dst, i, a);
}

// x = bf16(x), round to nearest even on the bits (seedvr2_dit_block.cpp:68-79).
__global__ __launch_bounds__(256) void bf16_round_kernel(float* x, long long count)
{
    const long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    if (i < count)
        x[i] = bf16_round(x[i]);
}

bool dtype_ok(int t)
{
    return t == SV2_F32 || t == SV2_F16 || t == SV2_BF16;
}

} // namespace

int launch_bias_rows(void* y, const float* b, int dtype, int rows, int cols, hipStream_t stream)
{
    return launch_bias_act(y, b, dtype, rows, cols, 0, stream);
}

int launch_bias_act(void* y, const float* b, int dtype, int rows, int cols, int silu, hipStream_t stream)
{
    if (!dtype_ok(dtype) || rows < 0 || cols <= 0 || cols % 8 != 0)
        return set_error(SV2_EINVAL, "bias_rows: bad dtype or shape");
    const long long count = static_cast<long long>(rows) * cols;
    if (count == 0)
        return SV2_OK;
    const dim3 grid(static_cast<unsigned>((count / 8 + 255) / 256));
    if (dtype == SV2_F32)
        hipLaunchKernelGGL(bias_rows_kernel<F32>, grid, dim3(256), 0, stream, y, b, count, cols, silu);
    else if (dtype == SV2_F16)
        hipLaunchKernelGGL(bias_rows_kernel<F16>, grid, dim3(256), 0, stream, y, b, count, cols, silu);
    else
        hipLaunchKernelGGL(bias_rows_kernel<BF16>, grid, dim3(256), 0, stream, y, b, count, cols, silu);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? SV2_OK : hip_error(err, "bias_rows_kernel launch");
}
int launch_bf16_round(float* x, long long count, hipStream_t stream)
{
    if (count <= 0)
        return SV2_OK;
    const long long blocks = (count + 255) / 256;
    if (blocks > 0x7fffffffLL)
        return set_error(SV2_EUNSUPPORTED, "bf16_round: too many elements");
    hipLaunchKernelGGL(bf16_round_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, x, count);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? SV2_OK : hip_error(err, "bf16_round_kernel launch");
}

int launch_to_f32(float* dst, const void* src, int dtype, long long count, hipStream_t stream)
{
    if (!dtype_ok(dtype) || count < 0 || count % 8 != 0)
        return set_error(SV2_EINVAL, "to_f32: bad dtype or count");
    if (count == 0)
        return SV2_OK;
    if (dtype == SV2_F32)
    {
        const hipError_t err = hipMemcpyAsync(dst, src, count * sizeof(float), hipMemcpyDeviceToDevice, stream);
        return err == hipSuccess ? SV2_OK : hip_error(err, "to_f32 copy");
    }
    const dim3 grid(static_cast<unsigned>((count / 8 + 255) / 256));
    if (dtype == SV2_F16)
        hipLaunchKernelGGL(to_f32_kernel<F16>, grid, dim3(256), 0, stream, dst, src, count);
    else
        hipLaunchKernelGGL(to_f32_kernel<BF16>, grid, dim3(256), 0, stream, dst, src, count);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? SV2_OK : hip_error(err, "to_f32_kernel launch");
}
template <typename Mod, int kVec, int rpb>
void launch_rmsnorm_rows(const void* x, void* y, int dtype, int rows, int dim, float eps, Mod mod, const float* gamma,
                         int has_ada, size_t lds, hipStream_t stream)
{
    const dim3 grid((rows + rpb - 1) / rpb);
    if (dtype == SV2_F32)
        hipLaunchKernelGGL((rmsnorm_ada_kernel<F32, Mod, kVec, rpb>), grid, dim3(256), lds, stream, x, y, rows, dim,
                           eps, mod, gamma, has_ada);
    else if (dtype == SV2_F16)
        hipLaunchKernelGGL((rmsnorm_ada_kernel<F16, Mod, kVec, rpb>), grid, dim3(256), lds, stream, x, y, rows, dim,
                           eps, mod, gamma, has_ada);
    else
        hipLaunchKernelGGL((rmsnorm_ada_kernel<BF16, Mod, kVec, rpb>), grid, dim3(256), lds, stream, x, y, rows, dim,
                           eps, mod, gamma, has_ada);
}

template <typename Mod>
int launch_rmsnorm(const void* x, void* y, int dtype, int rows, int dim, float eps, Mod mod, const float* gamma,
                   int has_ada, hipStream_t stream)
{
    if (rows == 0)
        return SV2_OK;
    if (dim <= 0 || dim % 8 != 0 || dim > 8 * 64 * kMaxVec)
        return set_error(SV2_EUNSUPPORTED, "rmsnorm_ada: dim must be a multiple of 8 and <= 4096");
    const size_t lds = static_cast<size_t>((has_ada ? 3 : 0) + (gamma ? 1 : 0)) * dim * sizeof(float);
    // rows of up to 2560 channels (the 3B model's width) keep 5 vectors per
    // lane in registers, wider ones up to kMaxVec; launches too small to fill
    // the chip with 16-row workgroups take one row per wave
    const bool narrow = dim <= 8 * 64 * kNarrowVec;
    const bool many = rows >= 256 * kNormRowsPerBlock;
    if (narrow && many)
        launch_rmsnorm_rows<Mod, kNarrowVec, kNormRowsPerBlock>(x, y, dtype, rows, dim, eps, mod, gamma, has_ada, lds,
                                                                stream);
    else if (narrow)
        launch_rmsnorm_rows<Mod, kNarrowVec, kNormRowsPerBlockFew>(x, y, dtype, rows, dim, eps, mod, gamma, has_ada,
                                                                   lds, stream);
    else if (many)
        launch_rmsnorm_rows<Mod, kMaxVec, kNormRowsPerBlock>(x, y, dtype, rows, dim, eps, mod, gamma, has_ada, lds,
                                                             stream);
    else
        launch_rmsnorm_rows<Mod, kMaxVec, kNormRowsPerBlockFew>(x, y, dtype, rows, dim, eps, mod, gamma, has_ada, lds,
                                                                stream);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? SV2_OK : hip_error(err, "rmsnorm_ada_kernel launch");
}

// Mode 0 with the gate read from emb (the sv2_ada_residual entry point):
// x = x * (emb[c*6+slot] + gate[c]) + residual.  emb's gate column is strided
// (6 floats per channel), so the workgroup forms the channel gates once in
// LDS for kResidualRows rows instead of every lane reading them from L2 per
// element; the rows then stream through with 16-byte accesses.
constexpr int kResidualRows = 16;
constexpr int kResidualMaxDim = 16384; // LDS for the staged gates: dim floats

template <typename T>
__global__ __launch_bounds__(256) void ada_residual_emb_kernel(void* x, const void* residual, int rows, int dim,
                                                               const float* emb, const float* gate, int slot)
{
#pragma clang fp contract(off)
    extern __shared__ __attribute__((aligned(16))) float g[];
    for (int c = threadIdx.x; c < dim; c += 256)
        g[c] = emb[c * 6 + slot] + gate[c];
    __syncthreads();
    const int r0 = blockIdx.x * kResidualRows;
    const int nr = min(kResidualRows, rows - r0);
    const int chunks = dim / 8;
    // item j of the workgroup: row r0 + rr, channels cc * 8 ..; walked with
    // the row and chunk stepped incrementally (no division per item)
    int rr = 0;
    int cc = threadIdx.x;
    while (cc >= chunks)
    {
        cc -= chunks;
        rr++;
    }
    while (rr < nr)
    {
        const int c0 = cc * 8;
        const long long i = static_cast<long long>(r0 + rr) * dim + c0;
        float a[8];
        float r[8];
        ld8<T>(x, i, a);
        ld8<T>(residual, i, r);
        const float4 g0 = *reinterpret_cast<const float4*>(&g[c0]);
        const float4 g1 = *reinterpret_cast<const float4*>(&g[c0 + 4]);
        const float gg[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
        float out[8];
#pragma unroll
        for (int e = 0; e < 8; e++)
        {
            const float t = a[e] * gg[e];
            out[e] = t + r[e];
        }
        st8<T>(x, i, out);
        cc += 256;
        while (cc >= chunks)
        {
            cc -= chunks;
            rr++;
        }
    }
}

int launch_residual_emb(void* x, const void* residual, int dtype, int rows, int dim, const float* emb,
                        const float* gate, int slot, hipStream_t stream)
{
    const dim3 grid(static_cast<unsigned>((rows + kResidualRows - 1) / kResidualRows));
    const size_t lds = static_cast<size_t>(dim) * sizeof(float);
    if (dtype == SV2_F32)
        hipLaunchKernelGGL((ada_residual_emb_kernel<F32>), grid, dim3(256), lds, stream, x, residual, rows, dim, emb,
                           gate, slot);
    else if (dtype == SV2_F16)
        hipLaunchKernelGGL((ada_residual_emb_kernel<F16>), grid, dim3(256), lds, stream, x, residual, rows, dim, emb,
                           gate, slot);
    else
        hipLaunchKernelGGL((ada_residual_emb_kernel<BF16>), grid, dim3(256), lds, stream, x, residual, rows, dim, emb,
                           gate, slot);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? SV2_OK : hip_error(err, "ada_residual_emb_kernel launch");
}

template <typename Gate>
int launch_residual(void* x, const void* residual, int dtype, int rows, int dim, Gate gate, const float* bias,
                    int mode, hipStream_t stream)
{
    const long long count = static_cast<long long>(rows) * dim;
    if (count == 0)
        return SV2_OK;
    const dim3 grid(static_cast<unsigned>((count / 8 + 255) / 256));
    if (dtype == SV2_F32)
        hipLaunchKernelGGL((ada_residual_kernel<F32, Gate>), grid, dim3(256), 0, stream, x, residual, count, dim,
                           gate, bias, mode);
    else if (dtype == SV2_F16)
        hipLaunchKernelGGL((ada_residual_kernel<F16, Gate>), grid, dim3(256), 0, stream, x, residual, count, dim,
                           gate, bias, mode);
    else
        hipLaunchKernelGGL((ada_residual_kernel<BF16, Gate>), grid, dim3(256), 0, stream, x, residual, count, dim,
                           gate, bias, mode);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? SV2_OK : hip_error(err, "ada_residual_kernel launch");
}

int launch_block_tables(const float* emb, const float* const* scale, const float* const* gate, int tables,
                        const float* bias, int dim, float* out, hipStream_t stream)
{
    if (dim <= 0 || dim % 8 != 0 || tables < 1 || tables > 4 || (bias && !gate[0]))
        return set_error(SV2_EINVAL, "block_tables: bad dim, table count or bias");
    BlockAda a{};
    for (int t = 0; t < tables; t++)
    {
        a.scale[t] = scale[t];
        a.gate[t] = gate[t];
    }
    a.bias = bias;
    a.tables = tables;
    hipLaunchKernelGGL(block_tables_kernel, dim3((dim + 255) / 256), dim3(256), 0, stream, emb, a, dim, out);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? SV2_OK : hip_error(err, "block_tables_kernel launch");
}

int launch_ada_table(const float* emb, const float* scale, const float* gate, int slot, int dim, float* out,
                     hipStream_t stream)
{
    if (dim <= 0 || dim % 8 != 0 || (slot != 0 && slot != 3))
        return set_error(SV2_EINVAL, "ada_table: bad dim or slot");
    hipLaunchKernelGGL(ada_table_kernel, dim3((dim + 255) / 256), dim3(256), 0, stream, emb, scale, gate, slot, dim,
                       out);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? SV2_OK : hip_error(err, "ada_table_kernel launch");
}

int launch_rmsnorm_table(const void* x, void* y, int dtype, int rows, int dim, float eps, const float* table,
                         const float* shift, const float* gamma, int has_ada, hipStream_t stream)
{
    const TableInput mod{table, table ? table + dim : nullptr, shift};
    return launch_rmsnorm(x, y, dtype, rows, dim, eps, mod, gamma, has_ada, stream);
}

int launch_residual_table(void* x, const void* residual, int dtype, int rows, int dim, const float* table,
                          const float* bias, int mode, hipStream_t stream)
{
    const TableGate gate{table ? table + 2 * dim : nullptr};
    return launch_residual(x, residual, dtype, rows, dim, gate, bias, mode, stream);
}
} // namespace sv2

extern "C" {

int sv2_rmsnorm_ada(const void* x, void* y, int io_dtype, int rows, int dim, float eps, const float* emb,
                    const float* shift, const float* scale, int slot_base, int has_ada, void* stream_ptr)
try
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
    const EmbInput mod{emb, shift, scale, slot_base};
    return launch_rmsnorm(x, y, io_dtype, rows, dim, eps, mod, nullptr, has_ada, static_cast<hipStream_t>(stream_ptr));
}
catch (...)
{
    return sv2::caught_exception("sv2_rmsnorm_ada");
}

int sv2_ada_residual(void* x, const void* residual, int io_dtype, int rows, int dim, const float* emb,
                     const float* gate_vec, int slot_base, int mode, void* stream_ptr)
try
{
    using namespace sv2;
    if (!dtype_ok(io_dtype) || rows < 0 || dim <= 0 || mode < 0 || mode > 2)
        return set_error(SV2_EINVAL, "ada_residual: bad dtype, shape or mode");
    if (dim % 8 != 0)
        return set_error(SV2_EUNSUPPORTED, "ada_residual: dim must be a multiple of 8");
    if (rows == 0)
        return SV2_OK;
    if (!x || (mode != 2 && !residual) || (mode == 0 && (!emb || !gate_vec)))
        return set_error(SV2_EINVAL, "ada_residual: null pointer");
    if (slot_base != 0 && slot_base != 3)
        return set_error(SV2_EINVAL, "ada_residual: slot_base must be 0 or 3");
    if (mode == 0 && dim <= kResidualMaxDim)
        return launch_residual_emb(x, residual, io_dtype, rows, dim, emb, gate_vec, slot_base + 2,
                                   static_cast<hipStream_t>(stream_ptr));
    const EmbGate gate{emb, gate_vec, slot_base + 2};
    return launch_residual(x, residual, io_dtype, rows, dim, gate, nullptr, mode, static_cast<hipStream_t>(stream_ptr));
}
catch (...)
{
    return sv2::caught_exception("sv2_ada_residual");
}

int sv2_swiglu(void* gate, const void* value, int io_dtype, int64_t count, void* stream_ptr)
try
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
catch (...)
{
    return sv2::caught_exception("sv2_swiglu");
}

} // extern "C"
