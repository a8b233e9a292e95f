// fp16 matrix products of the block's InnerProducts on gfx950 MFMA with the
// epilogues that follow them in the block fused in (the reference runs ncnn
// InnerProduct, seedvr2_dit_block.cpp:28-56 and :668-674, then separate
// SwiGLU and ada-residual passes, :1093-1112 and :807-825).
//
//   Y[m][n] = epilogue(sum_k X[m][k] * W[n][k])      X [M][K], W [N][K] fp16
//
// One 256-thread workgroup computes a 256 x 256 tile of Y, one wave per
// SIMD, each wave a 128 x 128 block as 4 x 4 MFMA tiles of 32 x 32
// (v_mfma_f32_32x32x16_f16, 256 fp32 accumulators per lane).  K advances in
// stages of 64 (whole 128-byte lines of every row: half-line stages halve the
// fetch rate) through two 64 KB LDS slots.  A stage goes global -> registers
// -> LDS: buffer loads two iterations ahead into one of two register sets,
// then ds_write_b128 in four parts spread over the iteration before it is
// multiplied, so the LDS writes share the bandwidth evenly with the operand
// reads.  One barrier per stage, three quarters through it.
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
#include <climits>

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
constexpr int kBK = 64;                       // K per stage: whole 128-byte lines of every row
constexpr int kKSteps = kBK / 16;             // MFMA k-steps per stage
constexpr int kRowBytes = kBK * 2;            // 128
constexpr int kTileBytes = kBM * kRowBytes;   // 32 KB: one operand tile of a stage
constexpr int kStageBytes = 2 * kTileBytes;   // 64 KB: W tile + X tile
constexpr int kThreads = 256;                 // 4 waves, one per SIMD, 128 x 128 of Y each
constexpr int kGroupM = 4;                    // row bands per tile group (see the tile order)
constexpr int kEpiStride = 272;               // bytes per staged output row (256 + 16: bank spread)
constexpr int kEpiBytes = 128 * kEpiStride;   // one wave's 128 x 128 fp16 block
constexpr int kLds = (2 * kStageBytes > 4 * kEpiBytes) ? 2 * kStageBytes : 4 * kEpiBytes;
static_assert(kLds <= 160 * 1024, "LDS of one gfx950 CU");

constexpr int kStore = kGemmStore;
constexpr int kResidual = kGemmResidual;
constexpr int kSwiGLU = kGemmSwiGLU;

struct GemmArgs
{
    const _Float16* x;  // [M][K]
    const _Float16* w;  // [N][K]
    const _Float16* w2; // kSwiGLU: the value projection [N][K]
    _Float16* y;        // [M][N]
    const _Float16* r;  // kResidual: [M][N]
    const float* bias;  // [N] or null
    const float* gate;  // [N] or null
    int m, n, k;
    int epi;
    int tiles_n;        // N / 256 (kSwiGLU: N / 128)
};

// Global -> register -> LDS staging.  Lane l of wave w loads rows
// 64 w + 8 i + l / 8 (i = 0..7) of the W tile and of the X tile, 16-byte
// chunk l % 8 of the stage's 128 bytes, and writes it to slot
// (l % 8) ^ (row % 8) of its row.  Buffer loads: the lane's part of the
// offset is one VGPR per operand, the row and stage parts are uniform (SGPR
// offset); X rows past M lie past the buffer's end and read as zero.
struct Operands
{
    __amdgpu_buffer_rsrc_t w;
    __amdgpu_buffer_rsrc_t x;
    int vw;   // lane's byte offset in W: (wrow0 + 64 wave + lane / 8) * 2K + 16 (lane % 8)
    int vx;   // lane's byte offset in X: (m0 + 64 wave + lane / 8) * 2K + 16 (lane % 8)
    int row8; // bytes of 8 rows: 16 K
};

struct StageRegs
{
    uint4 w[8];
    uint4 x[8];
};

__device__ inline Operands make_operands(const GemmArgs& a, int m0, int wbase, int wave, int lane)
{
    Operands o;
    const bool swiglu = a.epi == kSwiGLU;
    const _Float16* wsrc = swiglu && wave >= 2 ? a.w2 : a.w;
    const int wrow0 = swiglu ? wbase - 128 * (wave >> 1) : wbase;
    o.w = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(wsrc), static_cast<short>(0), a.n * a.k * 2,
                                            0x00020000);
    o.x = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(a.x), static_cast<short>(0), a.m * a.k * 2,
                                            0x00020000);
    // byte offsets in 32-bit unsigned arithmetic: the rows of the last, padded
    // X tile reach round_up(m, kBM) - 1, whose offset can pass INT_MAX when m *
    // k * 2 is just under it; it stays below 2^32 (k < 2^22), and the buffer
    // resource returns zeros for any offset past the operand
    const uint32_t row = 64u * static_cast<uint32_t>(wave) + static_cast<uint32_t>(lane >> 3);
    const uint32_t kb = 2u * static_cast<uint32_t>(a.k);
    o.vw = static_cast<int>((static_cast<uint32_t>(wrow0) + row) * kb + 16u * static_cast<uint32_t>(lane & 7));
    o.vx = static_cast<int>((static_cast<uint32_t>(m0) + row) * kb + 16u * static_cast<uint32_t>(lane & 7));
    o.row8 = 16 * a.k;
    return o;
}

__device__ inline void load_stage(const Operands& o, StageRegs& r, int kt)
{
    const int k0 = kt * kRowBytes;
#pragma unroll
    for (int i = 0; i < 8; i++)
    {
        const int so = __builtin_amdgcn_readfirstlane(i * o.row8 + k0);
        r.w[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(o.w, o.vw, so, 0));
        r.x[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(o.x, o.vx, so, 0));
    }
}

__device__ inline void store_stage(const StageRegs& r, char* stage, int wave, int lane)
{
#pragma unroll
    for (int i = 0; i < 8; i++)
    {
        const int row = 64 * wave + 8 * i + (lane >> 3);
        const int off = row * kRowBytes + (((lane & 7) ^ (row & 7)) << 4);
        *reinterpret_cast<uint4*>(stage + off) = r.w[i];
        *reinterpret_cast<uint4*>(stage + kTileBytes + off) = r.x[i];
    }
}

// part p of a stage: the lane's W and X rows of groups i = 2p, 2p + 1
__device__ inline void load_part(const Operands& o, StageRegs& r, int kt, int p)
{
    const int k0 = kt * kRowBytes;
#pragma unroll
    for (int i = 2 * p; i < 2 * p + 2; i++)
    {
        const int so = __builtin_amdgcn_readfirstlane(i * o.row8 + k0);
        r.w[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(o.w, o.vw, so, 0));
        r.x[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(o.x, o.vx, so, 0));
    }
}

__device__ inline void store_part(const StageRegs& r, char* stage, int wave, int lane, int p)
{
#pragma unroll
    for (int i = 2 * p; i < 2 * p + 2; i++)
    {
        const int row = 64 * wave + 8 * i + (lane >> 3);
        const int off = row * kRowBytes + (((lane & 7) ^ (row & 7)) << 4);
        *reinterpret_cast<uint4*>(stage + off) = r.w[i];
        *reinterpret_cast<uint4*>(stage + kTileBytes + off) = r.x[i];
    }
}

__device__ inline float h2f(_Float16 v)
{
    return static_cast<float>(v);
}

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

__device__ inline h8 finish_segment(const GemmArgs& a, const EpiCols& c, const h8 p, long long row, int col)
{
    h8 out;
    if (a.epi == kStore)
        return p;
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
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 31;
    const int g = lane >> 5;
    const int wm = wave >> 1; // 128-row half of the tile (X rows)
    const int wn = wave & 1;  // 128-column half (W rows)

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
    const int n0 = swiglu ? tn * 128 : tn * kBN;
    const int nk = a.k / kBK;

    // per-lane operand offsets: row 128 * wn (W) / 128 * wm (X) + lr of a
    // tile, chunk 2 ks + g; the 32-row blocks add 4096 bytes each
    const int swz = lr & 7;
    int offw[kKSteps];
    int offx[kKSteps];
#pragma unroll
    for (int ks = 0; ks < kKSteps; ks++)
    {
        offw[ks] = (128 * wn + lr) * kRowBytes + (((2 * ks + g) ^ swz) << 4);
        offx[ks] = kTileBytes + (128 * wm + lr) * kRowBytes + (((2 * ks + g) ^ swz) << 4);
    }

    f16acc acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
            acc[i][j] = f16acc{};

    const Operands ops = make_operands(a, m0, n0, wave, lane);
    // Stage s: loaded into register set s % 2 two iterations ahead, written
    // to LDS slot s % 2 in four parts (part 0 after the barrier of iteration
    // s - 2, parts 1-3 during the first three k-steps of iteration s - 1,
    // each part's registers reloaded with stage s + 2 right after), read
    // after the barrier of iteration s - 1.  Every iteration writes and
    // loads (stages past the last load stage nk - 1 again and are never
    // multiplied), so the loop body has no branches and the compiler's waits
    // for the loads are exact.
    StageRegs ra, rb;
    const int last = nk - 1;
    load_stage(ops, ra, 0);
    load_stage(ops, rb, min(1, last));
    store_stage(ra, smem, wave, lane);
    load_stage(ops, ra, min(2, last));
    store_part(rb, smem + kStageBytes, wave, lane, 0);
    load_part(ops, rb, min(3, last), 0);
    __syncthreads();

    h8 fw[2][4], fx[2][4];
    auto read_ops = [&](h8 (&w4)[4], h8 (&x4)[4], const char* st, int ks) {
#pragma unroll
        for (int b = 0; b < 4; b++)
        {
            w4[b] = *reinterpret_cast<const h8*>(st + offw[ks] + b * 4096);
            x4[b] = *reinterpret_cast<const h8*>(st + offx[ks] + b * 4096);
        }
    };
    auto mfmas = [&](const h8 (&w4)[4], const h8 (&x4)[4]) {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(w4[j], x4[i], acc[i][j], 0, 0, 0);
    };
    // scheduling groups (masks: 0x100 LDS read, 0x008 MFMA, 0x200 LDS write,
    // 0x020 global read): a phase's eight operand reads first, then its 16
    // MFMAs in groups of four, each group's first MFMA followed by one write
    // and one load
    auto interleave = [&]() {
#pragma unroll
        for (int m = 0; m < 4; m++)
        {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);
        }
    };
    read_ops(fw[0], fx[0], smem, 0);

    // Iteration kt (stage kt in slot kt % 2, its k-step 0 operands in
    // fw/fx[0]; `nx` holds stage kt + 1's parts 1-3, `cur` stage kt + 2):
    // k-steps 0-2 each with the next k-step's reads and one part of stage
    // kt + 1; the barrier (the slot's reads are done, stage kt + 1 is
    // visible); k-step 3 with stage kt + 1's first reads and part 0 of stage
    // kt + 2 into this slot.
    auto iter = [&](int kt, StageRegs& cur, StageRegs& nx) {
        char* st = smem + (kt & 1) * kStageBytes;
        char* sn = smem + ((kt + 1) & 1) * kStageBytes;
#pragma unroll
        for (int ks = 0; ks < kKSteps - 1; ks++)
        {
            read_ops(fw[(ks + 1) & 1], fx[(ks + 1) & 1], st, ks + 1);
            mfmas(fw[ks & 1], fx[ks & 1]);
            store_part(nx, sn, wave, lane, ks + 1);
            load_part(ops, nx, min(kt + 3, last), ks + 1);
            __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
            interleave();
            __builtin_amdgcn_sched_barrier(0);
        }
        __syncthreads();
        read_ops(fw[0], fx[0], sn, 0);
        mfmas(fw[1], fx[1]);
        store_part(cur, st, wave, lane, 0);
        load_part(ops, cur, min(kt + 4, last), 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
        interleave();
        __builtin_amdgcn_sched_barrier(0);
    };
    int kt = 0;
    for (; kt + 1 < nk; kt += 2)
    {
        iter(kt, ra, rb);
        iter(kt + 1, rb, ra);
    }
    if (kt < nk)
        iter(kt, ra, rb);

    // acc[i][j] register 4q + e holds Y row m0 + 128 wm + 32 i + lr, column
    // n0 + 128 wn + 32 j + 8 q + 4 g + e.
    __syncthreads();
    char* mine = smem + wave * kEpiBytes;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
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
        // gate block: wave (wm, 0), value block: wave (wm, 1); wave (wm, wn)
        // writes rows 64 wn..64 wn + 63 of the 128-row half wm
        __syncthreads();
        const char* gate_blk = smem + (2 * wm) * kEpiBytes;
        const char* val_blk = smem + (2 * wm + 1) * kEpiBytes;
        const int chunk = lane & 15;
        const int ycol = n0 + 8 * chunk;
#pragma unroll 4
        for (int it = 0; it < 16; it++)
        {
            const int rl = 64 * wn + 4 * it + (lane >> 4);
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
            *reinterpret_cast<h8*>(a.y + row * a.n + ycol) = out;
        }
        return;
    }

    __builtin_amdgcn_s_waitcnt(0xC07F); // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
    const int chunk = lane & 15;
    const int col = n0 + 128 * wn + 8 * chunk;
    const EpiCols ec = epi_cols(a, col);
#pragma unroll 4
    for (int it = 0; it < 32; it++)
    {
        const int rl = 4 * it + (lane >> 4);
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
    if (misaligned(x, 16) || misaligned(w, 16) || misaligned(w2, 16) || misaligned(y, 16) || misaligned(residual, 16))
        return set_error(SV2_EINVAL, "inner product: x, W, y and residual must be 16-byte aligned");
    // the operands are read through buffer resources with 32-bit byte offsets
    // (the kernel forms them unsigned, so padded tile rows past `rows` stay
    // exact; see make_operands)
    if (static_cast<long long>(rows) * in * 2 > INT_MAX || static_cast<long long>(out) * in * 2 > INT_MAX)
        return set_error(SV2_EUNSUPPORTED, "inner product: an operand exceeds 2 GiB");
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
try
{
    static_assert(SV2_EPI_STORE == sv2::kGemmStore && SV2_EPI_RESIDUAL == sv2::kGemmResidual &&
                      SV2_EPI_SWIGLU == sv2::kGemmSwiGLU,
                  "epilogue codes of the C ABI and the kernel agree");
    if (epilogue != SV2_EPI_SWIGLU && w_value)
        return sv2::set_error(SV2_EINVAL, "sv2_inner_product_f16: w_value is only read by SV2_EPI_SWIGLU");
    return sv2::gemm_mfma(static_cast<hipStream_t>(stream), rows, in, out, x, w, w_value, y, epilogue, bias, gate,
                          residual);
}
catch (...)
{
    return sv2::caught_exception("sv2_inner_product_f16");
}

