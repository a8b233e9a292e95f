// fp16 matrix products of the block's InnerProducts on gfx950 MFMA with the
// epilogues that follow them in the block fused in (the reference runs ncnn
// InnerProduct, seedvr2_dit_block.cpp:28-56 and :668-674, then separate
// SwiGLU and ada-residual passes, :1093-1112 and :807-825).
//
//   Y[m][n] = epilogue(sum_k X[m][k] * W[n][k])      X [M][K], W [N][K] fp16
//
// One 512-thread workgroup computes a 256 x 256 tile of Y, two waves per
// SIMD (one hides the other's barrier and LDS waits), each wave a 128 x 64
// block as 4 x 2 MFMA tiles of 32 x 32 (v_mfma_f32_32x32x16_f16, fp32
// accumulators).  K advances in stages of 64 (whole 128-byte lines of every
// row) through two LDS stages (32 KB of W rows + 32 KB of X rows each),
// the next filled by global_load_lds while the current one is multiplied:
// one barrier per stage and no staging registers.
// The products are computed transposed (W as the A operand), so a lane holds
// four consecutive columns of one output row; the tile is rounded to fp16
// (the InnerProduct's output), staged in LDS, and leaves in 16-byte row
// segments with the epilogue applied in fp32:
//   kStore     Y = fp16(acc)
//   kResidual  Y = fp16((fp16(acc) + bias) * gate + R), the gated residual
//              (bias and gate optional: without gate, Y = fp16(acc) + bias + R)
//   kSwiGLU    two weight matrices, gate W and value W2, both [N][K]: a
//              workgroup's 256 W rows are 128 gate rows and the same 128
//              value rows, its output tile 256 x 128 of Y [M][N] =
//              fp16((g / (1 + exp(-g))) * u), g, u = fp16(acc) of the halves.
// Every fp32 operation follows the unfused kernels' order without fused
// multiply-adds, so the epilogue adds no rounding of its own.
#include "sv2_internal.h"

#pragma clang fp contract(off)

namespace sv2
{
namespace
{

typedef __attribute__((ext_vector_type(8))) _Float16 h8;
typedef __attribute__((ext_vector_type(4))) _Float16 h4;
typedef __attribute__((ext_vector_type(16))) float f16acc;

constexpr int kBM = 256;                      // rows of Y per workgroup
constexpr int kBN = 256;                      // columns of Y (rows of W) per workgroup
constexpr int kBK = 64;                       // K per stage
constexpr int kStages = 2;                    // LDS stages (one in flight)
constexpr int kKSteps = kBK / 16;             // MFMA k-steps per stage
constexpr int kRowBytes = kBK * 2;            // 128
constexpr int kTileBytes = kBM * kRowBytes;   // 32 KB: one operand tile of a stage
constexpr int kStageBytes = 2 * kTileBytes;   // W tile + X tile
constexpr int kThreads = 512;
constexpr int kGroupM = 4;                    // row bands per tile group (see the tile order)
constexpr int kEpiStride = 144;               // bytes per staged output row (128 + 16: bank spread)
constexpr int kEpiBytes = 128 * kEpiStride;   // one wave's 128 x 64 fp16 block
constexpr int kLds = (kStages * kStageBytes > 8 * kEpiBytes) ? kStages * kStageBytes : 8 * kEpiBytes;
static_assert(kLds <= 160 * 1024, "LDS of one gfx950 CU");

// s_waitcnt immediates: vmcnt(N) with expcnt / lgkmcnt unconstrained (gfx9
// encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14).
constexpr int kWaitVm0 = 0x0F70;

constexpr int kStore = kGemmStore;
constexpr int kResidual = kGemmResidual;
constexpr int kSwiGLU = kGemmSwiGLU;

struct GemmArgs
{
    const _Float16* x;  // [M][K]
    const _Float16* w;  // [N][K]
    const _Float16* w2; // kSwiGLU: the value projection [N][K]
    _Float16* y;        // [M][N]
    const _Float16* r; // kResidual: [M][N]
    const float* bias; // [N] or null
    const float* gate; // [N] or null
    int m, n, k;
    int epi;
    int tiles_n;        // N / 256 (kSwiGLU: N / 128)
};

// Stage tiles are 256 rows of 128 bytes (64 fp16 of K); 16-byte chunk c
// (k = 8c..8c+7) of row r sits in slot c ^ (r & 7), so the operand reads of
// 8 consecutive rows hit all 32 banks.

// One 16-byte global -> LDS copy per lane (global_load_lds_dwordx4): lane i
// writes LDS bytes [lds + 16 i, lds + 16 i + 16), lds wave-uniform.  Inline
// assembly keeps the compiler from waiting on it before unrelated LDS reads;
// the loop places the vmcnt waits.  M0 is saved and restored.
__device__ inline void dma16(const void* g, char* lds)
{
    const unsigned base = __builtin_amdgcn_readfirstlane(static_cast<unsigned>(reinterpret_cast<size_t>(lds)));
    unsigned saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %2, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "s"(base), "v"(g)
                 : "memory");
}

// Stage kt of the workgroup's tile: wave w fetches rows 32w..32w+31 of the W
// tile and of the X tile, 8 rows (1 KB) per instruction, lane l taking row
// l / 8 of the 8 and the chunk that lands in slot l % 8 (8 fetches per lane).
// W tile row r is row wbase + r of W, or for kSwiGLU row wbase + r % 128 of
// W (r < 128, waves 0-3) or W2 (waves 4-7).  X rows past M repeat row M - 1
// (their outputs are not stored).
__device__ inline void fetch_stage(const GemmArgs& a, char* stage, int m0, int wbase, int kt, int wave, int lane)
{
    const int k0 = kt * kBK;
    const bool swiglu = a.epi == kSwiGLU;
    const _Float16* wsrc = swiglu && wave >= 4 ? a.w2 : a.w;
    const int wrow0 = swiglu ? wbase - 128 * (wave >> 2) : wbase;
#pragma unroll
    for (int i = 0; i < 4; i++)
    {
        const int r0 = 32 * wave + 8 * i;
        const int r = r0 + (lane >> 3);
        const int c = (lane & 7) ^ (r & 7);
        dma16(wsrc + static_cast<long long>(wrow0 + r) * a.k + k0 + 8 * c, stage + r0 * kRowBytes);
        const int xr = min(m0 + r, a.m - 1);
        dma16(a.x + static_cast<long long>(xr) * a.k + k0 + 8 * c, stage + kTileBytes + r0 * kRowBytes);
    }
}

__device__ inline float h2f(_Float16 v)
{
    return static_cast<float>(v);
}

// Per-column epilogue operands of a lane's 8 output columns (the same for
// every row the lane stores): bias and gate, read once.
struct EpiCols
{
    float b[8];
    float g[8];
};

__device__ inline EpiCols epi_cols(const GemmArgs& a, int col)
{
    EpiCols c;
#pragma unroll
    for (int e = 0; e < 8; e++)
    {
        c.b[e] = 0.f;
        c.g[e] = 1.f;
    }
    if (a.epi == kResidual)
    {
#pragma unroll
        for (int e = 0; e < 8; e++)
        {
            if (a.bias)
                c.b[e] = a.bias[col + e];
            if (a.gate)
                c.g[e] = a.gate[col + e];
        }
    }
    return c;
}

// Epilogue of one 16-byte segment (8 columns) of an output row.
__device__ inline h8 finish_segment(const GemmArgs& a, const EpiCols& c, const h8 p, long long row, int col)
{
    h8 out;
    if (a.epi == kStore)
        return p;
    // kResidual
    const h8 res = *reinterpret_cast<const h8*>(a.r + row * a.n + col);
#pragma unroll
    for (int e = 0; e < 8; e++)
    {
        float v = h2f(p[e]);
        if (a.bias)
            v = v + c.b[e];
        if (a.gate)
            v = v * c.g[e];
        v = v + h2f(res[e]);
        out[e] = static_cast<_Float16>(v);
    }
    return out;
}

__global__ __launch_bounds__(kThreads) void gemm_f16_kernel(GemmArgs a)
{
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int lr = lane & 31;
    const int g = lane >> 5;
    const int wm = wave >> 2; // 128-row half of the tile (X rows)
    const int wn = wave & 3;  // 64-column quarter (W rows)

    // workgroup ids go round-robin over the 8 XCDs; each XCD takes a
    // contiguous run of tiles (whole row bands, sharing their X rows in the
    // XCD's L2): XCD x owns tiles [x q + min(x, r), ...) for total = 8 q + r
    const int total = static_cast<int>(gridDim.x);
    const int xcd = blockIdx.x & 7;
    const int q8 = total >> 3;
    const int r8 = total & 7;
    const int id = xcd * q8 + min(xcd, r8) + static_cast<int>(blockIdx.x >> 3);
    // grouped order: consecutive ids walk kGroupM row bands of one column of
    // tiles before the next column, so the workgroups an XCD runs at once
    // cover about 4 row bands x 8 column tiles and share both operands in L2
    const int tiles_m = (a.m + kBM - 1) / kBM;
    const int per_group = kGroupM * a.tiles_n;
    const int grp = id / per_group;
    const int first_m = grp * kGroupM;
    const int group_rows = min(kGroupM, tiles_m - first_m);
    const int in_group = id - grp * per_group;
    const int tm = first_m + in_group % group_rows;
    const int tn = in_group / group_rows;
    const int m0 = tm * kBM;
    const bool swiglu = a.epi == kSwiGLU;
    const int n0 = swiglu ? tn * 128 : tn * kBN; // first Y column of the tile, first W row fetched
    const int nk = a.k / kBK;

    // per-lane operand offsets: row 64 * wn (W) / 128 * wm (X) + lr of a
    // tile, chunk 2 ks + g; the 32-row blocks add 4096 bytes each
    const int swz = lr & 7;
    int offw[kKSteps];
    int offx[kKSteps];
#pragma unroll
    for (int ks = 0; ks < kKSteps; ks++)
    {
        offw[ks] = (64 * wn + lr) * kRowBytes + (((2 * ks + g) ^ swz) << 4);
        offx[ks] = kTileBytes + (128 * wm + lr) * kRowBytes + (((2 * ks + g) ^ swz) << 4);
    }

    f16acc acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
            acc[i][j] = f16acc{};

#pragma unroll
    for (int s = 0; s < kStages - 1; s++)
        if (s < nk)
            fetch_stage(a, smem + s * kStageBytes, m0, n0, s, wave, lane);

    for (int kt = 0; kt < nk; kt++)
    {
        // stage kt, the only one in flight, has landed; after the barrier
        // every wave's part is visible and every wave has finished reading
        // stage kt - 1, whose buffer the fetch of stage kt + 1 reuses
        __builtin_amdgcn_s_waitcnt(kWaitVm0);
        __syncthreads();
        if (kt + kStages - 1 < nk)
            fetch_stage(a, smem + ((kt + kStages - 1) % kStages) * kStageBytes, m0, n0, kt + kStages - 1, wave,
                        lane);
        const char* st = smem + (kt % kStages) * kStageBytes;
        // the operands of two k-steps are read at a time (12 reads), pinned
        // ahead of their MFMAs: left to itself the scheduler reads each
        // operand right before its MFMAs and waits for it
#pragma unroll
        for (int kp = 0; kp < kKSteps; kp += 2)
        {
            h8 fw[2][2];
            h8 fx[2][4];
#pragma unroll
            for (int h = 0; h < 2; h++)
            {
#pragma unroll
                for (int b = 0; b < 2; b++)
                    fw[h][b] = *reinterpret_cast<const h8*>(st + offw[kp + h] + b * 4096);
#pragma unroll
                for (int b = 0; b < 4; b++)
                    fx[h][b] = *reinterpret_cast<const h8*>(st + offx[kp + h] + b * 4096);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fw[h][j], fx[h][i], acc[i][j], 0, 0, 0);
        }
    }

    // acc[i][j] register 4q + e holds Y row m0 + 128 wm + 32 i + lr, column
    // n0 + 64 wn + 32 j + 8 q + 4 g + e.  Round to fp16 (the InnerProduct's
    // output) and stage the wave's 128 x 64 block row-major in LDS.
    __syncthreads(); // every wave is done with the stage buffers
    char* mine = smem + wave * kEpiBytes;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int q = 0; q < 4; q++)
            {
                h4 v;
#pragma unroll
                for (int e = 0; e < 4; e++)
                    v[e] = static_cast<_Float16>(acc[i][j][4 * q + e]);
                *reinterpret_cast<h4*>(mine + (32 * i + lr) * kEpiStride + (32 * j + 8 * q + 4 * g) * 2) = v;
            }

    if (swiglu)
    {
        // the gate columns 64 c..64 c + 63 of the tile sit in the block of
        // wave (wm, c), the matching value columns in wave (wm, c + 2); wave
        // (wm, wn) writes rows 64 (wn >> 1)..+63 of the 128-row half wm,
        // columns n0 + 64 c.. with c = wn & 1
        __syncthreads();
        const int c = wn & 1;
        const char* gate_blk = smem + (4 * wm + c) * kEpiBytes;
        const char* val_blk = smem + (4 * wm + c + 2) * kEpiBytes;
        const int chunk = lane & 7;
        const int ycol = n0 + 64 * c + 8 * chunk;
        const int ncols = a.n;
#pragma unroll 4
        for (int it = 0; it < 8; it++)
        {
            const int rl = 64 * (wn >> 1) + 8 * it + (lane >> 3);
            const long long row = m0 + 128 * wm + rl;
            if (row >= a.m)
                continue;
            const h8 gv = *reinterpret_cast<const h8*>(gate_blk + rl * kEpiStride + chunk * 16);
            const h8 uv = *reinterpret_cast<const h8*>(val_blk + rl * kEpiStride + chunk * 16);
            h8 out;
#pragma unroll
            for (int e = 0; e < 8; e++)
            {
                const float gf = h2f(gv[e]);
                const float den = 1.f + expf(-gf);
                out[e] = static_cast<_Float16>((gf / den) * h2f(uv[e]));
            }
            *reinterpret_cast<h8*>(a.y + row * ncols + ycol) = out;
        }
        return;
    }

    // the block was written and is read back by this wave only: LDS
    // operations of a wave complete in order, the wait keeps the compiler
    // from reordering them
    __builtin_amdgcn_s_waitcnt(0xC07F); // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
    const int chunk = lane & 7;
    const int col = n0 + 64 * wn + 8 * chunk;
    const EpiCols ec = epi_cols(a, col);
#pragma unroll 4
    for (int it = 0; it < 16; it++)
    {
        const int rl = 8 * it + (lane >> 3);
        const long long row = m0 + 128 * wm + rl;
        if (row >= a.m)
            continue;
        const h8 p = *reinterpret_cast<const h8*>(mine + rl * kEpiStride + chunk * 16);
        *reinterpret_cast<h8*>(a.y + row * a.n + col) = finish_segment(a, ec, p, row, col);
    }
}

} // namespace

bool gemm_mfma_supported(int in, int out, int epi)
{
    if (in <= 0 || in % kBK != 0 || out <= 0)
        return false;
    return epi == kSwiGLU ? out % 128 == 0 : out % kBN == 0;
}

int gemm_mfma(hipStream_t stream, int rows, int in, int out, const void* x, const void* w, const void* w2, void* y,
              int epi, const float* bias, const float* gate, const void* residual)
{
    if (rows == 0)
        return SV2_OK;
    if (epi != kStore && epi != kResidual && epi != kSwiGLU)
        return set_error(SV2_EINVAL, "inner product: unknown epilogue");
    if (rows < 0 || !gemm_mfma_supported(in, out, epi))
        return set_error(SV2_EUNSUPPORTED,
                         "inner product: needs in a multiple of 64 and out a multiple of 256 (SwiGLU: 128)");
    if (!x || !w || !y || (epi == kResidual && !residual) || (epi == kSwiGLU && !w2))
        return set_error(SV2_EINVAL, "inner product: null pointer");
    const int rc = set_dynamic_lds(reinterpret_cast<const void*>(&gemm_f16_kernel), kLds,
                                   "gemm_mfma: dynamic LDS attribute");
    if (rc != SV2_OK)
        return rc;
    GemmArgs a;
    a.x = static_cast<const _Float16*>(x);
    a.w = static_cast<const _Float16*>(w);
    a.w2 = static_cast<const _Float16*>(w2);
    a.y = static_cast<_Float16*>(y);
    a.r = static_cast<const _Float16*>(residual);
    a.bias = bias;
    a.gate = gate;
    a.m = rows;
    a.n = out;
    a.k = in;
    a.epi = epi;
    a.tiles_n = epi == kSwiGLU ? out / 128 : out / kBN;
    const long long tiles = static_cast<long long>((rows + kBM - 1) / kBM) * a.tiles_n;
    if (tiles >= (1LL << 31))
        return set_error(SV2_EUNSUPPORTED, "gemm_mfma: too many tiles");
    hipLaunchKernelGGL(gemm_f16_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kThreads), kLds, stream, a);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? SV2_OK : hip_error(err, "gemm_f16_kernel launch");
}

} // namespace sv2

extern "C" int sv2_inner_product_f16(const void* x, const void* w, const void* w_value, void* y, int rows, int in,
                                     int out, int epilogue, const float* bias, const float* gate,
                                     const void* residual, void* stream)
{
    static_assert(SV2_EPI_STORE == sv2::kGemmStore && SV2_EPI_RESIDUAL == sv2::kGemmResidual &&
                      SV2_EPI_SWIGLU == sv2::kGemmSwiGLU,
                  "epilogue codes of the C ABI and the kernel agree");
    if (epilogue != SV2_EPI_SWIGLU && w_value)
        return sv2::set_error(SV2_EINVAL, "sv2_inner_product_f16: w_value is only read by SV2_EPI_SWIGLU");
    return sv2::gemm_mfma(static_cast<hipStream_t>(stream), rows, in, out, x, w, w_value, y, epilogue, bias, gate,
                          residual);
}

