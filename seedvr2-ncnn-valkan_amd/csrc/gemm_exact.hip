// The fp32 InnerProduct of the parity mode: y = float(sum_i double(x_i) *
// double(w_i) + double(b)), every output's products added one after another
// in increasing i, then the bias, then one rounding to float.
//
// The products of two floats are exact in double, so each step rounds only
// the running sum, and the result is the same bit for bit as any evaluation
// that adds the same exact products in the same order and rounds the same
// way: the CPU oracle's double-accumulated y = W x + b, W [out][in] row-major.
// The reference's InnerProduct is ncnn's (seedvr2_dit_block.cpp:28-56 creates
// it), which accumulates in float in an order not known here (ncnn is not in
// the reference tree): against it this product is pinned by the closed form
// y = W x + b only, not bit for bit.
//
// On the VALU in fp64 (an fp64 MFMA would sum four products per step in its
// own order).  Two forms of the same arithmetic:
//   * tiled (rows > 16): one 256-thread workgroup per 64 x 128 tile of y;
//     each thread keeps an 8 x 4 block of double accumulators; k moves
//     through LDS in stages of 8, held as double, two stages in flight;
//   * few rows (rows <= 16, e.g. the DiT's one-row time MLP): one one-wave
//     workgroup per 16 output columns, so a wide product spreads over many
//     CUs and several workgroups share each; W moves through LDS in chunks of
//     64 k, transposed, the next chunk loaded into registers meanwhile.
#include "sv2_internal.h"

namespace sv2
{
namespace
{

constexpr int kBM = 64;   // rows of y per workgroup
constexpr int kBN = 128;  // output columns per workgroup
constexpr int kBK = 8;    // k per LDS stage
constexpr int kTM = 8;    // rows per thread
constexpr int kTN = 4;    // columns per thread

__global__ __launch_bounds__(256) void gemm_f32_exact_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                             const float* __restrict__ bias, float* __restrict__ y,
                                                             int rows, int in, int out)
{
    __shared__ double xs[2][kBK][kBM];
    __shared__ double ws[2][kBK][kBN];
    const int tid = threadIdx.x;
    const int tx = tid & 31; // columns 4 tx .. 4 tx + 3
    const int ty = tid >> 5; // rows 8 ty .. 8 ty + 7
    const int row0 = blockIdx.y * kBM;
    const int col0 = blockIdx.x * kBN;

    // staging assignment: x tile 64 rows x 8 k (2 per thread), w tile 128
    // columns x 8 k (4 per thread); values past the edges are zero (their
    // products are +0 and leave the sums unchanged)
    const int xr = tid >> 2;
    const int xk = (tid & 3) * 2;
    const int wc = tid >> 1;
    const int wk = (tid & 1) * 4;
    const bool x_row_ok = row0 + xr < rows;
    const bool w_col_ok = col0 + wc < out;
    const float* xp = x + static_cast<long long>(x_row_ok ? row0 + xr : 0) * in;
    const float* wp = w + static_cast<long long>(w_col_ok ? col0 + wc : 0) * in;

    auto stage = [&](int buf, int k0) {
#pragma unroll
        for (int e = 0; e < 2; e++)
        {
            const int k = k0 + xk + e;
            xs[buf][xk + e][xr] = (x_row_ok && k < in) ? static_cast<double>(xp[k]) : 0.0;
        }
#pragma unroll
        for (int e = 0; e < 4; e++)
        {
            const int k = k0 + wk + e;
            ws[buf][wk + e][wc] = (w_col_ok && k < in) ? static_cast<double>(wp[k]) : 0.0;
        }
    };

    double acc[kTM][kTN];
#pragma unroll
    for (int i = 0; i < kTM; i++)
#pragma unroll
        for (int j = 0; j < kTN; j++)
            acc[i][j] = 0.0;

    const int nk = (in + kBK - 1) / kBK;
    stage(0, 0);
    __syncthreads();
    for (int s = 0; s < nk; s++)
    {
        const int buf = s & 1;
        if (s + 1 < nk)
            stage(buf ^ 1, (s + 1) * kBK);
#pragma unroll
        for (int k = 0; k < kBK; k++)
        {
            double a[kTM];
            double b[kTN];
#pragma unroll
            for (int i = 0; i < kTM; i++)
                a[i] = xs[buf][k][ty * kTM + i];
#pragma unroll
            for (int j = 0; j < kTN; j++)
                b[j] = ws[buf][k][tx * kTN + j];
#pragma unroll
            for (int i = 0; i < kTM; i++)
#pragma unroll
                for (int j = 0; j < kTN; j++)
                    acc[i][j] = __builtin_fma(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }

    double bv[kTN];
#pragma unroll
    for (int j = 0; j < kTN; j++)
    {
        const int c = col0 + tx * kTN + j;
        bv[j] = (bias && c < out) ? static_cast<double>(bias[c]) : 0.0;
    }
#pragma unroll
    for (int i = 0; i < kTM; i++)
    {
        const int r = row0 + ty * kTM + i;
        if (r >= rows)
            break;
        float* yr = y + static_cast<long long>(r) * out;
#pragma unroll
        for (int j = 0; j < kTN; j++)
        {
            const int c = col0 + tx * kTN + j;
            if (c < out)
                yr[c] = static_cast<float>(acc[i][j] + bv[j]);
        }
    }
}

constexpr int kRowsSmall = 16; // the few-rows form handles up to this many rows
constexpr int kCols = 16;      // output columns per few-rows workgroup (one wave)
constexpr int kChunk = 64;     // k per LDS chunk of the few-rows form

// One wave: lane (c, s) = (lane % 16, lane / 16) owns column col0 + c for
// rows s, s + 4, s + 8, s + 12.  Lane l stages 16 consecutive k of W row
// col0 + l / 4, and loads the next chunk's into registers while the current
// chunk is summed; several of these small workgroups share a CU and hide
// each other's loads.
__global__ __launch_bounds__(64) void gemv_f32_exact_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                            const float* __restrict__ bias, float* __restrict__ y,
                                                            int rows, int in, int out)
{
    __shared__ float wt[kChunk][kCols];      // wt[k][c] = W[col0 + c][k0 + k]
    __shared__ float xs[kRowsSmall][kChunk]; // xs[r][k] = x[r][k0 + k]
    const int lane = threadIdx.x;
    const int c = lane & (kCols - 1);
    const int slot = lane >> 4;
    const int col0 = blockIdx.x * kCols;
    const int wr = lane >> 2;
    const int wk = (lane & 3) * 16;
    const bool w_ok = col0 + wr < out;
    const float* wp = w + static_cast<long long>(w_ok ? col0 + wr : 0) * in;

    // values past the edges are zero: their products are +0 and the running
    // sums, which start at +0, stay what they were
    float wv[16];
    auto load_w = [&](int k0) {
#pragma unroll
        for (int e = 0; e < 16; e++)
        {
            const int k = k0 + wk + e;
            wv[e] = (w_ok && k < in) ? wp[k] : 0.f;
        }
    };

    double acc[kRowsSmall / 4];
#pragma unroll
    for (int i = 0; i < kRowsSmall / 4; i++)
        acc[i] = 0.0;

    load_w(0);
    for (int k0 = 0; k0 < in; k0 += kChunk)
    {
#pragma unroll
        for (int e = 0; e < 16; e++)
            wt[wk + e][wr] = wv[e];
#pragma unroll
        for (int j = 0; j < kRowsSmall * kChunk / 64; j++)
        {
            const int i = lane + 64 * j;
            const int r = i / kChunk;
            const int k = k0 + i % kChunk;
            xs[r][i % kChunk] = (r < rows && k < in) ? x[static_cast<long long>(r) * in + k] : 0.f;
        }
        __syncthreads();
        if (k0 + kChunk < in)
            load_w(k0 + kChunk);
#pragma unroll
        for (int i = 0; i < kRowsSmall / 4; i++)
        {
            if (slot + 4 * i >= rows) // rows past the input: nothing to sum
                break;
#pragma unroll 16
            for (int k = 0; k < kChunk; k++)
                acc[i] = __builtin_fma(static_cast<double>(xs[slot + 4 * i][k]), static_cast<double>(wt[k][c]), acc[i]);
        }
        __syncthreads();
    }
    if (col0 + c >= out)
        return;
    const double bv = bias ? static_cast<double>(bias[col0 + c]) : 0.0;
#pragma unroll
    for (int i = 0; i < kRowsSmall / 4; i++)
    {
        const int r = slot + 4 * i;
        if (r < rows)
            y[static_cast<long long>(r) * out + col0 + c] = static_cast<float>(acc[i] + bv);
    }
}

} // namespace

int gemm_f32_exact(hipStream_t stream, int rows, int in, int out, const float* x, const float* w, const float* bias,
                   float* y)
{
    if (rows < 0 || in <= 0 || out <= 0)
        return set_error(SV2_EINVAL, "inner product (fp32): bad shape");
    if (rows == 0)
        return SV2_OK;
    if (!x || !w || !y)
        return set_error(SV2_EINVAL, "inner product (fp32): null pointer");
    if (rows <= kRowsSmall)
    {
        hipLaunchKernelGGL(gemv_f32_exact_kernel, dim3(static_cast<unsigned>((out + kCols - 1) / kCols)), dim3(64), 0,
                           stream, x, w, bias, y, rows, in, out);
        const hipError_t err = hipGetLastError();
        return err == hipSuccess ? SV2_OK : hip_error(err, "gemv_f32_exact_kernel launch");
    }
    const dim3 grid(static_cast<unsigned>((out + kBN - 1) / kBN), static_cast<unsigned>((rows + kBM - 1) / kBM));
    if (grid.y > 65535u)
        return set_error(SV2_EUNSUPPORTED, "inner product (fp32): too many rows");
    hipLaunchKernelGGL(gemm_f32_exact_kernel, grid, dim3(256), 0, stream, x, w, bias, y, rows, in, out);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? SV2_OK : hip_error(err, "gemm_f32_exact_kernel launch");
}

} // namespace sv2

extern "C" int sv2_inner_product_f32(const float* x, const float* w, const float* bias, float* y, int rows, int in,
                                     int out, void* stream)
try
{
    return sv2::gemm_f32_exact(static_cast<hipStream_t>(stream), rows, in, out, x, w, bias, y);
}
catch (...)
{
    return sv2::caught_exception("sv2_inner_product_f32");
}
