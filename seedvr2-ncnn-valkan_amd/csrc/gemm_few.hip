// fp16 InnerProducts of a few rows (the text branch's 58 tokens): the
// reference runs them as ncnn InnerProduct on the text rows
// (seedvr2_dit_block.cpp:28-56, :668-674; called at :1155-1156, :1180-1181,
// :1101 and :1111), followed by the ada-residual and SwiGLU passes
// (:807-825, :1198-1209, :1093-1112).  With at most 64 rows a product is a
// stream of its weight matrix: every weight is used by few rows, so the
// kernel is built to read W once at HBM rate and fold the passes that follow
// it into its epilogue.
//
//   Y[m][n] = epilogue(sum_k X[m][k] * W[n][k])   X [M][K], W [N][K] fp16, M <= 64
//
// A 256-thread workgroup (4 waves) owns 64 columns of Y (SwiGLU: 32 columns,
// whose 32 gate rows and 32 value rows make up its 64 W rows) and a range of
// K.  K moves in blocks of 64 (one whole 128-byte line of every row) through
// a 4-slot LDS ring, three blocks ahead.  Both operands arrive by
// global_load_lds_dwordx4 in whole lines: eight adjacent lanes fetch one
// row's line, which keeps each request a full cache line (operand-ordered
// 16-byte loads, one row per lane, stream W at about 0.7 of this rate).
// Chunk c of row r sits in slot c ^ (r & 7), so the MFMA operand reads of 16
// rows at one chunk spread over the LDS banks.  Each wave multiplies its 16
// W rows by the 64 X rows on v_mfma_f32_16x16x32_f16 (4 row tiles, two
// k-steps per block).
//
// K is split over gridDim.y workgroups when the column tiles alone give too
// few workgroups (2560 output columns are 40 tiles): each writes its fp32
// partial sums, and a second kernel adds them in split order and applies the
// epilogue, so the result does not depend on timing.  Epilogues, every fp32
// step in the unfused passes' order without fused multiply-adds:
//   kGemmStore     Y = fp16(fp16(acc) + bias)  (bias optional: Y = fp16(acc))
//   kGemmResidual  Y = fp16((fp16(acc) + bias) * gate + R)  (bias, gate optional)
//   kGemmSwiGLU    Y = fp16((g / (1 + exp(-g))) * u), g, u = fp16 of the gate
//                  and value sums (never split)
#include "sv2_internal.h"
#include <algorithm>

#pragma clang fp contract(off)

namespace sv2
{
namespace
{

typedef __attribute__((ext_vector_type(8))) _Float16 h8;
typedef __attribute__((ext_vector_type(4))) _Float16 h4;
typedef __attribute__((ext_vector_type(4))) float f4;

constexpr int kMaxRows = 64;
constexpr int kSlots = 4;                     // LDS ring slots (8, seven blocks ahead, measured slower)
constexpr int kAhead = kSlots - 1;            // blocks in flight ahead of the one multiplied
constexpr int kRowBytes = 128;                // 64 halfs of K per row and block
constexpr int kOperandBytes = 64 * kRowBytes; // 64 rows of one operand
constexpr int kStageBytes = 2 * kOperandBytes;
constexpr int kLds = kSlots * kStageBytes;    // 64 KB: two workgroups per CU
constexpr int kThreads = 256;
constexpr int kTargetGroups = 240;            // about one workgroup per CU
constexpr int kMinBlocks = 4;                 // K blocks per workgroup at least, when split
constexpr int kDmaPerBlock = 4;               // fetches per wave and K block (2 W, 2 X)
constexpr int kMaxSplits = 8;                 // K splits at most (the reduction loads them all at once)

struct FewArgs
{
    const _Float16* x;
    const _Float16* w;
    const _Float16* w2;
    _Float16* y;
    const _Float16* r;
    const float* bias;
    const float* gate;
    float* part; // [splits][m][n]
    int m;
    int n;
    int k;
    int epi;
};

// One 16-byte piece per lane from global memory straight into LDS at
// lds + 16 * lane (the LDS base is wave-uniform, passed in M0).  The
// compiler does not count these loads in its vmcnt waits; the loop below
// waits for them itself.
__device__ inline void dma16(const void* g, char* lds)
{
    const unsigned base = __builtin_amdgcn_readfirstlane(static_cast<unsigned>(reinterpret_cast<size_t>(lds)));
    unsigned saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %2, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "s"(base), "v"(g)
                 : "memory");
}

// s_waitcnt vmcnt(n) for the n fetches of the blocks younger than the one
// about to be multiplied (n a multiple of kDmaPerBlock below kAhead blocks'
// worth; the counter's high bits sit at 14-15)
template <int N>
__device__ inline void wait_vm()
{
    static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

__device__ inline void wait_younger(int younger)
{
    switch (younger)
    {
    case 6: wait_vm<6 * kDmaPerBlock>(); break;
    case 5: wait_vm<5 * kDmaPerBlock>(); break;
    case 4: wait_vm<4 * kDmaPerBlock>(); break;
    case 3: wait_vm<3 * kDmaPerBlock>(); break;
    case 2: wait_vm<2 * kDmaPerBlock>(); break;
    case 1: wait_vm<kDmaPerBlock>(); break;
    default: wait_vm<0>(); break;
    }
}
static_assert(kAhead - 1 <= 6, "wait_younger covers at most 6 younger blocks");
static_assert(kLds <= 160 * 1024, "LDS of one gfx950 CU");

__device__ inline float h2f(_Float16 v)
{
    return static_cast<float>(v);
}

__device__ inline float round16(float v)
{
    return static_cast<float>(static_cast<_Float16>(v));
}

// The store / gated-residual epilogue of one output element from its fp32 sum.
__device__ inline _Float16 finish(const FewArgs& a, float acc, int row, int col)
{
    float v = round16(acc);
    if (a.bias)
        v = v + a.bias[col];
    if (a.epi == kGemmResidual)
    {
        if (a.gate)
            v = v * a.gate[col];
        v = v + h2f(a.r[static_cast<long long>(row) * a.n + col]);
    }
    return static_cast<_Float16>(v);
}

template <bool SW>
__global__ __launch_bounds__(kThreads) void gemm_few_kernel(FewArgs a)
{
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n0 = blockIdx.x * (SW ? 32 : 64);
    const int nb = a.k / 64;
    const int splits = gridDim.y;
    const int b0 = static_cast<int>(static_cast<long long>(blockIdx.y) * nb / splits);
    const int b1 = static_cast<int>(static_cast<long long>(blockIdx.y + 1) * nb / splits);
    const int nblk = b1 - b0;

    // fetch rows of this wave: tile rows 16 wave + 8 i + lane / 8 of W and X,
    // lane & 7 the LDS slot, (lane & 7) ^ (row & 7) the chunk it holds
    const _Float16* wsrc[2];
    const _Float16* xsrc[2];
#pragma unroll
    for (int i = 0; i < 2; i++)
    {
        const int tr = 16 * wave + 8 * i + (lane >> 3);
        const int chunk = (lane & 7) ^ (tr & 7);
        const _Float16* wrow;
        if (SW)
            wrow = tr < 32 ? a.w + static_cast<long long>(n0 + tr) * a.k
                           : a.w2 + static_cast<long long>(n0 + tr - 32) * a.k;
        else
            wrow = a.w + static_cast<long long>(n0 + tr) * a.k;
        wsrc[i] = wrow + 8 * chunk;
        // X rows past the last are fetched from the last row; their sums are
        // never stored
        xsrc[i] = a.x + static_cast<long long>(min(tr, a.m - 1)) * a.k + 8 * chunk;
    }
    auto fetch = [&](int b) {
        char* st = smem + (b % kSlots) * kStageBytes;
        const long long koff = static_cast<long long>(b0 + b) * 64;
#pragma unroll
        for (int i = 0; i < 2; i++)
        {
            dma16(wsrc[i] + koff, st + (16 * wave + 8 * i) * kRowBytes);
            dma16(xsrc[i] + koff, st + kOperandBytes + (16 * wave + 8 * i) * kRowBytes);
        }
    };

    f4 acc[4];
#pragma unroll
    for (int t = 0; t < 4; t++)
        acc[t] = f4{0.f, 0.f, 0.f, 0.f};
    const int lr = lane & 15;
    const int lq = lane >> 4;
    for (int b = 0; b < kAhead && b < nblk; b++)
        fetch(b);
    for (int b = 0; b < nblk; b++)
    {
        // block b has landed once only the younger blocks' fetches are outstanding
        wait_younger(min(nblk - 1 - b, kAhead - 1));
        // every wave's part of block b is in LDS, and every wave is done
        // with block b - 1, whose slot the next fetch reuses
        __syncthreads();
        if (b + kAhead < nblk)
            fetch(b + kAhead);
        const char* st = smem + (b % kSlots) * kStageBytes;
#pragma unroll
        for (int s = 0; s < 2; s++)
        {
            // lane: operand row lr, k = 32 s + 8 lq .. + 7 (chunk 4 s + lq)
            const int c = 4 * s + lq;
            const int wr = 16 * wave + lr;
            const h8 wv = *reinterpret_cast<const h8*>(st + wr * kRowBytes + 16 * (c ^ (wr & 7)));
            h8 xv[4];
#pragma unroll
            for (int t = 0; t < 4; t++)
            {
                const int xr = 16 * t + lr;
                xv[t] = *reinterpret_cast<const h8*>(st + kOperandBytes + xr * kRowBytes + 16 * (c ^ (xr & 7)));
            }
#pragma unroll
            for (int t = 0; t < 4; t++)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wv, xv[t], acc[t], 0, 0, 0);
        }
    }

    // acc[t][i] is the sum of Y row 16 t + lr, tile column 16 wave + 4 lq + i
    if (splits > 1)
    {
#pragma unroll
        for (int t = 0; t < 4; t++)
        {
            const int row = 16 * t + lr;
            if (row < a.m)
                *reinterpret_cast<f4*>(a.part + (static_cast<long long>(blockIdx.y) * a.m + row) * a.n + n0 +
                                       16 * wave + 4 * lq) = acc[t];
        }
        return;
    }
    if constexpr (SW)
    {
        // the value waves (2, 3) hand their sums to the gate waves of the
        // same columns through LDS (free: every fetch has landed and every
        // wave has passed the loop's last barrier once this one is passed)
        __syncthreads();
        f4* xch = reinterpret_cast<f4*>(smem);
        if (wave >= 2)
        {
#pragma unroll
            for (int t = 0; t < 4; t++)
                xch[((wave - 2) * 4 + t) * 64 + lane] = acc[t];
        }
        __syncthreads();
        if (wave >= 2)
            return;
        const int col = n0 + 16 * wave + 4 * lq;
#pragma unroll
        for (int t = 0; t < 4; t++)
        {
            const int row = 16 * t + lr;
            if (row >= a.m)
                continue;
            const f4 u = xch[(wave * 4 + t) * 64 + lane];
            h4 o;
#pragma unroll
            for (int i = 0; i < 4; i++)
            {
                const float gf = round16(acc[t][i]);
                const float den = 1.f + expf(-gf);
                o[i] = static_cast<_Float16>((gf / den) * round16(u[i]));
            }
            *reinterpret_cast<h4*>(a.y + static_cast<long long>(row) * a.n + col) = o;
        }
        return;
    }
    else
    {
        const int col = n0 + 16 * wave + 4 * lq;
#pragma unroll
        for (int t = 0; t < 4; t++)
        {
            const int row = 16 * t + lr;
            if (row >= a.m)
                continue;
            h4 o;
#pragma unroll
            for (int i = 0; i < 4; i++)
                o[i] = finish(a, acc[t][i], row, col + i);
            *reinterpret_cast<h4*>(a.y + static_cast<long long>(row) * a.n + col) = o;
        }
    }
}

// Y = epilogue(sum over the splits' partials in split order); one thread per
// four consecutive outputs of a row.
__global__ __launch_bounds__(256) void gemm_few_reduce_kernel(FewArgs a, int splits)
{
    const long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    const int quads = a.n / 4;
    if (i >= static_cast<long long>(a.m) * quads)
        return;
    const int row = static_cast<int>(i / quads);
    const int col = static_cast<int>(i - static_cast<long long>(row) * quads) * 4;
    // every split's load is issued before the first add, then the sums are
    // added in split order
    f4 v[kMaxSplits];
#pragma unroll
    for (int p = 0; p < kMaxSplits; p++)
        if (p < splits)
            v[p] = *reinterpret_cast<const f4*>(a.part + (static_cast<long long>(p) * a.m + row) * a.n + col);
    f4 s = v[0];
#pragma unroll
    for (int p = 1; p < kMaxSplits; p++)
        if (p < splits)
            s += v[p];
    h4 o;
#pragma unroll
    for (int e = 0; e < 4; e++)
        o[e] = finish(a, s[e], row, col + e);
    *reinterpret_cast<h4*>(a.y + static_cast<long long>(row) * a.n + col) = o;
}

} // namespace

bool gemm_few_supported(int rows, int in, int out, int epi)
{
    if (rows < 1 || rows > kMaxRows || in <= 0 || in % 64 != 0 || out <= 0)
        return false;
    if (epi == kGemmSwiGLU)
        return out % 32 == 0;
    return (epi == kGemmStore || epi == kGemmResidual) && out % 64 == 0;
}

int gemm_few_splits(int rows, int in, int out, int epi)
{
    if (!gemm_few_supported(rows, in, out, epi) || epi == kGemmSwiGLU)
        return 1;
    const int tiles = out / 64;
    const int blocks = in / 64;
    const int want = (kTargetGroups + tiles / 2) / tiles;
    return std::max(1, std::min({want, blocks / kMinBlocks, kMaxSplits}));
}

size_t gemm_few_workspace(int rows, int in, int out, int epi)
{
    const int splits = gemm_few_splits(rows, in, out, epi);
    return splits > 1 ? static_cast<size_t>(splits) * rows * out * sizeof(float) : 0;
}

int gemm_few(hipStream_t stream, int rows, int in, int out, const void* x, const void* w, const void* w2, void* y,
             int epi, const float* bias, const float* gate, const void* residual, void* work, size_t work_bytes)
{
    if (epi != kGemmStore && epi != kGemmResidual && epi != kGemmSwiGLU)
        return set_error(SV2_EINVAL, "few-row inner product: unknown epilogue");
    if (rows == 0 && in > 0 && out > 0)
        return SV2_OK;
    if (!gemm_few_supported(rows, in, out, epi))
        return set_error(SV2_EUNSUPPORTED, "few-row inner product: needs 1-64 rows, in % 64 == 0 and out % 64 == 0 "
                                           "(SwiGLU: out % 32 == 0)");
    if (!x || !w || !y || (epi == kGemmResidual && !residual) || (epi == kGemmSwiGLU && !w2))
        return set_error(SV2_EINVAL, "few-row inner product: null pointer");
    if (epi == kGemmSwiGLU && (bias || gate))
        return set_error(SV2_EINVAL, "few-row inner product: SwiGLU takes no bias or gate");
    if (misaligned(x, 16) || misaligned(w, 16) || misaligned(w2, 16) || misaligned(y, 8) || misaligned(residual, 8) ||
        misaligned(work, 16))
        return set_error(SV2_EINVAL, "few-row inner product: x, W and the workspace must be 16-byte aligned, y and "
                                     "residual 8-byte aligned");
    const int splits = gemm_few_splits(rows, in, out, epi);
    const size_t need = gemm_few_workspace(rows, in, out, epi);
    if (need > 0 && (!work || work_bytes < need))
        return set_error(SV2_EINVAL, "few-row inner product: workspace too small");
    const int rc = set_dynamic_lds(reinterpret_cast<const void*>(epi == kGemmSwiGLU ? &gemm_few_kernel<true>
                                                                                    : &gemm_few_kernel<false>),
                                   kLds, "gemm_few: dynamic LDS attribute");
    if (rc != SV2_OK)
        return rc;
    FewArgs a;
    a.x = static_cast<const _Float16*>(x);
    a.w = static_cast<const _Float16*>(w);
    a.w2 = static_cast<const _Float16*>(w2);
    a.y = static_cast<_Float16*>(y);
    a.r = static_cast<const _Float16*>(residual);
    a.bias = bias;
    a.gate = gate;
    a.part = static_cast<float*>(work);
    a.m = rows;
    a.n = out;
    a.k = in;
    a.epi = epi;
    const dim3 grid(static_cast<unsigned>(out / (epi == kGemmSwiGLU ? 32 : 64)), static_cast<unsigned>(splits));
    if (epi == kGemmSwiGLU)
        hipLaunchKernelGGL(gemm_few_kernel<true>, grid, dim3(kThreads), kLds, stream, a);
    else
        hipLaunchKernelGGL(gemm_few_kernel<false>, grid, dim3(kThreads), kLds, stream, a);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return hip_error(err, "gemm_few_kernel launch");
    if (splits > 1)
    {
        const long long quads = static_cast<long long>(rows) * (out / 4);
        hipLaunchKernelGGL(gemm_few_reduce_kernel, dim3(static_cast<unsigned>((quads + 255) / 256)), dim3(256), 0,
                           stream, a, splits);
        err = hipGetLastError();
        if (err != hipSuccess)
            return hip_error(err, "gemm_few_reduce_kernel launch");
    }
    return SV2_OK;
}

} // namespace sv2

extern "C" int64_t sv2_inner_product_f16_few_workspace(int rows, int in, int out, int epilogue)
try
{
    if (epilogue != SV2_EPI_STORE && epilogue != SV2_EPI_RESIDUAL && epilogue != SV2_EPI_SWIGLU)
        return sv2::set_error(SV2_EINVAL, "sv2_inner_product_f16_few_workspace: unknown epilogue");
    if (rows == 0 && in > 0 && out > 0)
        return 0;
    if (!sv2::gemm_few_supported(rows, in, out, epilogue))
        return sv2::set_error(SV2_EUNSUPPORTED, "sv2_inner_product_f16_few_workspace: unsupported shape");
    return static_cast<int64_t>(sv2::gemm_few_workspace(rows, in, out, epilogue));
}
catch (...)
{
    return sv2::caught_exception("sv2_inner_product_f16_few_workspace");
}

extern "C" int sv2_inner_product_f16_few(const void* x, const void* w, const void* w_value, void* y, int rows, int in,
                                         int out, int epilogue, const float* bias, const float* gate,
                                         const void* residual, void* workspace, size_t workspace_bytes, void* stream)
try
{
    if (epilogue != SV2_EPI_SWIGLU && w_value)
        return sv2::set_error(SV2_EINVAL, "sv2_inner_product_f16_few: w_value is only read by SV2_EPI_SWIGLU");
    return sv2::gemm_few(static_cast<hipStream_t>(stream), rows, in, out, x, w, w_value, y, epilogue, bias, gate,
                         residual, workspace, workspace_bytes);
}
catch (...)
{
    return sv2::caught_exception("sv2_inner_product_f16_few");
}
