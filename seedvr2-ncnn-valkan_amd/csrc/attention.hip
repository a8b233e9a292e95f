// Windowed joint video + text attention of the SeedVR2-3B DiT block on gfx950.
//
// Replaces SeedVR2DiTBlock::attention (seedvr2_dit_block.cpp:870-1091) and the
// reference's per-window qkv_prepare / attention / zero_buffer / window_sum
// shader chain (:192-330, :339-457, :541-572) with one fused kernel plus a
// small text reduction:
//
//   * no materialised window copies: every query and key row is located by
//     index arithmetic on the closed-form window plan and read straight from
//     the [tokens, 3*D] qkv rows;
//   * the per-head RMSNorm * gamma, the RoPE rotation and the bf16 rounding of
//     q and k (and the bf16 rounding of v) run in registers while a tile is
//     staged into LDS;
//   * S^T = K Q^T on bf16 MFMA (q, k are bf16 values, so the operands are
//     exact), online softmax in fp32 with one cross-lane exchange per row,
//     O^T += V^T P^T on fp16 MFMA with fp32 accumulation;
//   * ragged windows are handled by masking keys and padding query rows, never
//     by padding the tensors;
//   * video outputs are written once (the windows partition the grid); text
//     outputs go to per-window bf16 partials which a second kernel sums in
//     window order and scales by 1/nW, exactly as the reference does.
#include "sv2_internal.h"

#include <algorithm>
#include <cmath>
#include <cstring>

namespace sv2
{
namespace
{

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;

constexpr int kBlockM = 128;   // query rows per workgroup (4 waves x 32)
constexpr int kBlockN = 64;    // keys per iteration
constexpr int kThreads = 256;
constexpr int kQkStride = 136; // halfs per LDS row of the q and k tiles (128 + 8 pad)
constexpr int kVtStride = 64;  // halfs per LDS row of the transposed v tile (swizzled)
constexpr float kLog2e = 1.4426950408889634f;

// Element types of the qkv input and of the outputs.
struct F32
{
    using storage = float;
};
struct F16
{
    using storage = _Float16;
};
struct BF16
{
    using storage = uint16_t;
};

template <typename T>
__device__ inline void load8(const void* base, long long offset, float x[8]);

template <>
__device__ inline void load8<F32>(const void* base, long long offset, float x[8])
{
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + offset);
    const float4 a = p[0];
    const float4 b = p[1];
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}

template <>
__device__ inline void load8<F16>(const void* base, long long offset, float x[8])
{
    const f16x8 v = *reinterpret_cast<const f16x8*>(static_cast<const _Float16*>(base) + offset);
#pragma unroll
    for (int e = 0; e < 8; e++)
        x[e] = static_cast<float>(v[e]);
}

template <>
__device__ inline void load8<BF16>(const void* base, long long offset, float x[8])
{
    const uint4 v = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + offset);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; e++)
    {
        x[2 * e] = __builtin_bit_cast(float, w[e] << 16);
        x[2 * e + 1] = __builtin_bit_cast(float, w[e] & 0xffff0000u);
    }
}

template <typename T>
__device__ inline void store4(void* base, long long offset, const float v[4]);

template <>
__device__ inline void store4<F32>(void* base, long long offset, const float v[4])
{
    *reinterpret_cast<float4*>(static_cast<float*>(base) + offset) = make_float4(v[0], v[1], v[2], v[3]);
}

template <>
__device__ inline void store4<F16>(void* base, long long offset, const float v[4])
{
    typedef __attribute__((ext_vector_type(4))) _Float16 f16x4;
    f16x4 h;
    h[0] = static_cast<_Float16>(v[0]);
    h[1] = static_cast<_Float16>(v[1]);
    h[2] = static_cast<_Float16>(v[2]);
    h[3] = static_cast<_Float16>(v[3]);
    *reinterpret_cast<f16x4*>(static_cast<_Float16*>(base) + offset) = h;
}

// bf16 outputs, rounded to nearest even (identity on attention outputs, which
// are bf16 values already; the text averages are not).
template <>
__device__ inline void store4<BF16>(void* base, long long offset, const float v[4])
{
    uint32_t h[4];
#pragma unroll
    for (int e = 0; e < 4; e++)
        h[e] = __builtin_bit_cast(uint32_t, bf16_round(v[e])) >> 16;
    uint2 packed;
    packed.x = h[0] | (h[1] << 16);
    packed.y = h[2] | (h[3] << 16);
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(base) + offset) = packed;
}

struct AttnParams
{
    PlanArgs plan;
    const void* vid_qkv;
    const void* txt_qkv;
    long long row_stride; // elements per qkv row (3*D)
    int heads;
    int dim;              // D = heads * 128
    int text_len;
    int npairs;           // windows * heads
    int nqb;              // query blocks per (window, head)
    int qk_norm;
    int rope_mode;
    int rope_npos;
    float eps;
    float scale;          // 1/sqrt(128) in fp32, as the reference computes it
    const float* gq_vid;
    const float* gk_vid;
    const float* gq_txt;
    const float* gk_txt;
    const float2* rope_tab; // [3][npos][24] (cos, sin)
    void* vid_out;
    uint16_t* partial;      // [nwin][text_len][D] bf16 bits
    float* dbg_pre;         // optional [sum S][D]
};

// Where the window-sequence row j of a window lives and how it is rotated.
struct RowRef
{
    const void* base;  // tensor holding the row
    long long offset;  // element offset of the row start
    bool valid;
    bool text;
    bool rotate;
    int pos[3];
};

__device__ inline RowRef resolve_row(const AttnParams& p, const WindowBox& b, int j)
{
    RowRef r;
    r.valid = j < b.vlen + p.text_len;
    r.text = false;
    r.rotate = false;
    r.pos[0] = r.pos[1] = r.pos[2] = 0;
    r.base = p.vid_qkv;
    r.offset = 0;
    if (!r.valid)
        return r;
    if (j < b.vlen)
    {
        int lt, ly, lx;
        const int row = window_video_row(p.plan, b, j, &lt, &ly, &lx);
        r.offset = static_cast<long long>(row) * p.row_stride;
        if (p.rope_mode == SV2_ROPE_REFERENCE)
        {
            // window-local positions, time offset by the text length (:988, :994)
            r.rotate = true;
            r.pos[0] = p.text_len + lt;
            r.pos[1] = ly;
            r.pos[2] = lx;
        }
        else if (p.rope_mode == SV2_ROPE_ABSOLUTE)
        {
            r.rotate = true;
            r.pos[0] = b.t0 + lt;
            r.pos[1] = b.h0 + ly;
            r.pos[2] = b.w0 + lx;
        }
    }
    else
    {
        const int l = j - b.vlen;
        r.base = p.txt_qkv;
        r.text = true;
        r.offset = static_cast<long long>(l) * p.row_stride;
        if (p.rope_mode == SV2_ROPE_REFERENCE)
        {
            // text token l rotated at (l, l, l) (:1004-1020)
            r.rotate = true;
            r.pos[0] = r.pos[1] = r.pos[2] = l;
        }
    }
    return r;
}

// RoPE axis and pair of an even head dim, or -1 when the dim is not rotated.
__device__ inline int rope_slot(int mode, int d, int* pair)
{
    if (mode == SV2_ROPE_REFERENCE)
    {
        if (d >= 126)
            return -1;
        const int axis = d / 42;
        *pair = (d - axis * 42) >> 1;
        return axis;
    }
    if (mode == SV2_ROPE_ABSOLUTE)
    {
        if (d < 32)
        {
            *pair = d >> 1;
            return 0;
        }
        if (d < 80)
        {
            *pair = (d - 32) >> 1;
            return 1;
        }
        *pair = (d - 80) >> 1;
        return 2;
    }
    return -1;
}

// The q/k prologue for the 8 dims [d0, d0+8) of one row held by one lane;
// the 16 lanes of a row group hold its 128 dims (lanes 16g .. 16g+15, all
// active).  Follows normalize_and_rotate (seedvr2_dit_block.cpp:942-974):
// double sum of squares, inv = 1/sqrtf(float(ss/128) + eps), y = x*inv*gamma,
// rotation of adjacent pairs with (cos, sin) of float(pos)*freq, bf16 RNE.
// Multiplies and adds are kept separate (no contraction), as in the reference.
__device__ inline void qk_prologue8(float x[8], const float* gamma, int d0, const RowRef& row,
                                    const AttnParams& p)
{
#pragma clang fp contract(off)
    if (p.qk_norm)
    {
        double ss = 0.0;
#pragma unroll
        for (int e = 0; e < 8; e++)
            ss += static_cast<double>(x[e]) * static_cast<double>(x[e]);
        ss += __shfl_xor(ss, 1);
        ss += __shfl_xor(ss, 2);
        ss += __shfl_xor(ss, 4);
        ss += __shfl_xor(ss, 8);
        const float inv = 1.f / sqrtf(static_cast<float>(ss / 128.0) + p.eps);
#pragma unroll
        for (int e = 0; e < 8; e++)
            x[e] = x[e] * inv * gamma[d0 + e];
    }
    if (row.rotate)
    {
#pragma unroll
        for (int q = 0; q < 4; q++)
        {
            int pair = 0;
            const int axis = rope_slot(p.rope_mode, d0 + 2 * q, &pair);
            if (axis >= 0)
            {
                const float2 cs = p.rope_tab[(axis * p.rope_npos + row.pos[axis]) * kRopePairSlots + pair];
                const float first = x[2 * q];
                const float second = x[2 * q + 1];
                const float a = first * cs.x;
                const float b = second * cs.y;
                const float c = second * cs.x;
                const float d = first * cs.y;
                x[2 * q] = a - b;
                x[2 * q + 1] = c + d;
            }
        }
    }
#pragma unroll
    for (int e = 0; e < 8; e++)
        x[e] = bf16_round(x[e]);
}

// 8 bf16-exact floats -> 8 bf16 bit patterns packed in a uint4.
__device__ inline uint4 pack_bf16x8(const float x[8])
{
    uint4 v;
    v.x = (__builtin_bit_cast(uint32_t, x[0]) >> 16) | (__builtin_bit_cast(uint32_t, x[1]) & 0xffff0000u);
    v.y = (__builtin_bit_cast(uint32_t, x[2]) >> 16) | (__builtin_bit_cast(uint32_t, x[3]) & 0xffff0000u);
    v.z = (__builtin_bit_cast(uint32_t, x[4]) >> 16) | (__builtin_bit_cast(uint32_t, x[5]) & 0xffff0000u);
    v.w = (__builtin_bit_cast(uint32_t, x[6]) >> 16) | (__builtin_bit_cast(uint32_t, x[7]) & 0xffff0000u);
    return v;
}

// Row permutation of a 32-key S^T tile: swapping bits 2 and 3 of the row makes
// each lane's 16 accumulator registers hold keys 8g..8g+7 and 16+8g..16+8g+7
// (g = lane / 32), which is exactly the k-slice the lane supplies as the B
// operand of the following P*V MFMA.
__device__ inline int key_perm(int i)
{
    return (i & ~12) | ((i & 4) << 1) | ((i & 8) >> 1);
}

// Swizzled offset (in halfs) of key group `grp` (8 keys) in row d of the
// transposed v tile; spreads the 16-byte reads of consecutive rows over banks.
__device__ inline int vt_offset(int d, int grp)
{
    return d * kVtStride + ((grp ^ ((d ^ (d >> 3)) & 7)) << 3);
}

template <typename TI, typename TO>
__global__ __launch_bounds__(kThreads) void window_attention_kernel(AttnParams p)
{
    __shared__ __attribute__((aligned(16))) uint16_t q_tile[kBlockM * kQkStride];
    __shared__ __attribute__((aligned(16))) uint16_t k_tile[kBlockN * kQkStride];
    __shared__ __attribute__((aligned(16))) uint16_t vt_tile[kHeadDim * kVtStride];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    // XCD-aware decode: workgroup ids go round-robin over the 8 XCDs, so
    // ids x, x+8, x+16 ... share an XCD (and its L2).  The query blocks of one
    // (window, head) pair are consecutive on one XCD, so the K/V rows they all
    // read come from that XCD's L2 after the first read from HBM.
    const int id = blockIdx.x;
    const int xcd = id & 7;
    const int slot = id >> 3;
    const int pair = (slot / p.nqb) * 8 + xcd;
    const int qb = slot - (slot / p.nqb) * p.nqb;
    if (pair >= p.npairs)
        return;
    const int wi = pair / p.heads;
    const int head = pair - wi * p.heads;
    const WindowBox box = window_box(p.plan, wi);
    const int seq = box.vlen + p.text_len;
    const int q0 = qb * kBlockM;
    if (q0 >= seq)
        return;

    const int rsub = tid >> 4;  // row within a 16-row pass
    const int chunk = tid & 15; // 8-dim slice of the row
    const int d0 = chunk * 8;
    const long long q_col = static_cast<long long>(head) * kHeadDim;
    const long long k_col = q_col + p.dim;
    const long long v_col = q_col + 2LL * p.dim;

    // ---- query tile: prologue in registers, bf16 into LDS
    for (int pass = 0; pass < kBlockM / 16; pass++)
    {
        const int r = pass * 16 + rsub;
        const RowRef row = resolve_row(p, box, q0 + r);
        float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (row.valid)
            load8<TI>(row.base, row.offset + q_col + d0, x);
        qk_prologue8(x, row.text ? p.gq_txt : p.gq_vid, d0, row, p);
        *reinterpret_cast<uint4*>(&q_tile[r * kQkStride + d0]) = pack_bf16x8(x);
    }
    __syncthreads();

    const int g = lane >> 5;
    const int lr = lane & 31;
    // B operand of S^T = K Q^T: lane holds query lr, dims 16c + 8g .. +7
    bf16x8 qf[8];
#pragma unroll
    for (int c = 0; c < 8; c++)
        qf[c] = *reinterpret_cast<const bf16x8*>(&q_tile[(wave * 32 + lr) * kQkStride + 16 * c + 8 * g]);
    const bool wave_active = q0 + wave * 32 < seq;

    f32x16 o[4];
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
        o[dt] = f32x16{};
    float m_run = -INFINITY;
    float l_run = 0.f;

    const int nkb = (seq + kBlockN - 1) / kBlockN;
    for (int kb = 0; kb < nkb; kb++)
    {
        __syncthreads(); // previous tile fully consumed

        // ---- key tile: prologue in registers, bf16 into LDS
#pragma unroll
        for (int pass = 0; pass < kBlockN / 16; pass++)
        {
            const int r = pass * 16 + rsub;
            const RowRef row = resolve_row(p, box, kb * kBlockN + r);
            float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            if (row.valid)
                load8<TI>(row.base, row.offset + k_col + d0, x);
            qk_prologue8(x, row.text ? p.gk_txt : p.gk_vid, d0, row, p);
            *reinterpret_cast<uint4*>(&k_tile[r * kQkStride + d0]) = pack_bf16x8(x);
        }
        // ---- value tile: bf16 rounding, fp16 operands, transposed into LDS;
        // thread = 4 consecutive keys x one 8-dim slice
        {
            const int kg = tid >> 4;
            float v[4][8];
#pragma unroll
            for (int i = 0; i < 4; i++)
            {
                const RowRef row = resolve_row(p, box, kb * kBlockN + 4 * kg + i);
#pragma unroll
                for (int e = 0; e < 8; e++)
                    v[i][e] = 0.f;
                if (row.valid)
                    load8<TI>(row.base, row.offset + v_col + d0, v[i]);
            }
            typedef __attribute__((ext_vector_type(4))) _Float16 f16x4;
#pragma unroll
            for (int e = 0; e < 8; e++)
            {
                f16x4 h;
#pragma unroll
                for (int i = 0; i < 4; i++)
                    h[i] = static_cast<_Float16>(bf16_round(v[i][e]));
                const int d = d0 + e;
                *reinterpret_cast<f16x4*>(&vt_tile[vt_offset(d, kg >> 1) + (kg & 1) * 4]) = h;
            }
        }
        __syncthreads();

        if (wave_active)
        {
            // ---- S^T for two 32-key subtiles
            f32x16 s[2];
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
            {
                s[kt] = f32x16{};
                const uint16_t* krow = &k_tile[(kt * 32 + key_perm(lr)) * kQkStride + 8 * g];
#pragma unroll
                for (int c = 0; c < 8; c++)
                {
                    const bf16x8 a = *reinterpret_cast<const bf16x8*>(krow + 16 * c);
                    s[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[c], s[kt], 0, 0, 0);
                }
            }
            // ---- scale, mask, online softmax (row = this lane's query)
            float smax = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                {
                    const int i = 8 * (r >> 2) + 4 * g + (r & 3);
                    const int key = kb * kBlockN + kt * 32 + key_perm(i);
                    const float val = key < seq ? s[kt][r] * p.scale : -INFINITY;
                    s[kt][r] = val;
                    smax = fmaxf(smax, val);
                }
            smax = fmaxf(smax, __shfl_xor(smax, 32));
            const float m_new = fmaxf(m_run, smax);
            const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * kLog2e);
            const float bias = m_new * kLog2e;
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
                o[dt] *= alpha;
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                {
                    const float e = __builtin_amdgcn_exp2f(s[kt][r] * kLog2e - bias);
                    s[kt][r] = e;
                    l_run += e;
                }
            // ---- O^T += V^T P^T
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
#pragma unroll
                for (int c2 = 0; c2 < 2; c2++)
                {
                    f16x8 b;
#pragma unroll
                    for (int e = 0; e < 8; e++)
                        b[e] = static_cast<_Float16>(s[kt][8 * c2 + e]);
                    const int grp = kt * 4 + c2 * 2 + g;
#pragma unroll
                    for (int dt = 0; dt < 4; dt++)
                    {
                        const f16x8 a = *reinterpret_cast<const f16x8*>(&vt_tile[vt_offset(dt * 32 + lr, grp)]);
                        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, o[dt], 0, 0, 0);
                    }
                }
        }
    }

    if (!wave_active)
        return;
    const float l_tot = l_run + __shfl_xor(l_run, 32);
    const int j = q0 + wave * 32 + lr;
    if (j >= seq)
        return;
    const float inv_l = 1.f / l_tot;
    const long long pre_row = p.dbg_pre
                                  ? (static_cast<long long>(box.vprefix) + static_cast<long long>(wi) * p.text_len + j) * p.dim
                                  : 0;
    long long out_off;
    bool text = j >= box.vlen;
    if (!text)
    {
        int lt, ly, lx;
        out_off = static_cast<long long>(window_video_row(p.plan, box, j, &lt, &ly, &lx)) * p.dim + q_col;
    }
    else
    {
        out_off = (static_cast<long long>(wi) * p.text_len + (j - box.vlen)) * p.dim + q_col;
    }
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int rq = 0; rq < 4; rq++)
        {
            const int d = dt * 32 + 8 * rq + 4 * g;
            float pre[4];
            float rounded[4];
#pragma unroll
            for (int e = 0; e < 4; e++)
            {
                pre[e] = o[dt][4 * rq + e] * inv_l;
                rounded[e] = bf16_round(pre[e]);
            }
            if (p.dbg_pre)
                store4<F32>(p.dbg_pre, pre_row + q_col + d, pre);
            if (!text)
                store4<TO>(p.vid_out, out_off + d, rounded);
            else
                store4<BF16>(p.partial, out_off + d, rounded);
        }
}

// Text outputs: sum of the per-window bf16 partials in window order, then a
// multiply by 1/nW (seedvr2_dit_block.cpp:1074-1075, :1081-1088).
template <typename TO>
__global__ __launch_bounds__(256) void text_window_reduce_kernel(const uint16_t* partial, void* out, int nwin,
                                                                 long long count, float inv_nw)
{
    const long long i = (static_cast<long long>(blockIdx.x) * 256 + threadIdx.x) * 4;
    if (i >= count)
        return;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int w = 0; w < nwin; w++)
    {
        const uint2 v = *reinterpret_cast<const uint2*>(partial + static_cast<long long>(w) * count + i);
        acc[0] += __builtin_bit_cast(float, v.x << 16);
        acc[1] += __builtin_bit_cast(float, v.x & 0xffff0000u);
        acc[2] += __builtin_bit_cast(float, v.y << 16);
        acc[3] += __builtin_bit_cast(float, v.y & 0xffff0000u);
    }
    float r[4];
#pragma unroll
    for (int e = 0; e < 4; e++)
        r[e] = acc[e] * inv_nw;
    store4<TO>(out, i, r);
}

// Debug / test: the prologue alone, 16 rows per workgroup, fp32 outputs in
// window-sequence order.  Same row resolution and prologue code as above.
template <typename TI>
__global__ __launch_bounds__(256) void qk_prologue_kernel(AttnParams p, int nrb, float* q_out, float* k_out,
                                                          float* v_out)
{
    const int blk = blockIdx.x;
    const int rb = blk % nrb;
    const int rest = blk / nrb;
    const int head = rest % p.heads;
    const int wi = rest / p.heads;
    const WindowBox box = window_box(p.plan, wi);
    const int seq = box.vlen + p.text_len;
    if (rb * 16 >= seq)
        return;
    const int tid = threadIdx.x;
    const int j = rb * 16 + (tid >> 4);
    const int d0 = (tid & 15) * 8;
    const RowRef row = resolve_row(p, box, j);
    const long long q_col = static_cast<long long>(head) * kHeadDim;
    float q[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float k[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (row.valid)
    {
        load8<TI>(row.base, row.offset + q_col + d0, q);
        load8<TI>(row.base, row.offset + q_col + p.dim + d0, k);
        load8<TI>(row.base, row.offset + q_col + 2LL * p.dim + d0, v);
    }
    qk_prologue8(q, row.text ? p.gq_txt : p.gq_vid, d0, row, p);
    qk_prologue8(k, row.text ? p.gk_txt : p.gk_vid, d0, row, p);
    if (!row.valid)
        return;
    const long long base = (static_cast<long long>(box.vprefix) + static_cast<long long>(wi) * p.text_len + j) * p.dim + q_col + d0;
#pragma unroll
    for (int e = 0; e < 8; e++)
    {
        q_out[base + e] = q[e];
        k_out[base + e] = k[e];
        v_out[base + e] = bf16_round(v[e]);
    }
}

__global__ __launch_bounds__(256) void window_index_map_kernel(PlanArgs plan, int32_t* out)
{
    const WindowBox box = window_box(plan, blockIdx.x);
    for (int j = threadIdx.x; j < box.vlen; j += 256)
    {
        int lt, ly, lx;
        out[box.vprefix + j] = window_video_row(plan, box, j, &lt, &ly, &lx);
    }
}

int dtype_ok(int t)
{
    return t == SV2_F32 || t == SV2_F16 || t == SV2_BF16;
}

// Validates the attention arguments and fills the kernel parameters.
int prepare(const sv2_attn_args* a, AttnParams* p, int* smax_out)
{
    if (!a)
        return set_error(SV2_EINVAL, "attention: null args");
    if (a->head_dim != kHeadDim)
        return set_error(SV2_EUNSUPPORTED, "attention: head_dim must be 128");
    if (a->heads <= 0 || a->text_len < 0)
        return set_error(SV2_EINVAL, "attention: heads must be > 0 and text_len >= 0");
    if (!dtype_ok(a->qkv_dtype) || !dtype_ok(a->out_dtype))
        return set_error(SV2_EINVAL, "attention: unknown dtype");
    if (a->rope_mode < SV2_ROPE_REFERENCE || a->rope_mode > SV2_ROPE_NONE)
        return set_error(SV2_EINVAL, "attention: unknown rope mode");
    if (!a->vid_qkv || (a->text_len > 0 && !a->txt_qkv))
        return set_error(SV2_EINVAL, "attention: null qkv pointer");
    if (a->qk_norm && (!a->gamma_q_vid || !a->gamma_k_vid || (a->text_len > 0 && (!a->gamma_q_txt || !a->gamma_k_txt))))
        return set_error(SV2_EINVAL, "attention: qk_norm needs all four gamma vectors");
    std::memset(p, 0, sizeof(*p));
    int rc = build_plan(a->rule, &p->plan);
    if (rc != SV2_OK)
        return rc;
    if (a->rope_mode != SV2_ROPE_NONE)
    {
        const int need = sv2_rope_positions_needed(&a->rule, a->text_len, a->rope_mode);
        if (need < 0)
            return need;
        if (!a->rope_table || a->rope_npos < need)
            return set_error(SV2_EINVAL, "attention: rope table missing or covering too few positions");
    }
    int smax = 0;
    for (int wi = 0; wi < p->plan.nwin; wi++)
        smax = std::max(smax, window_box(p->plan, wi).vlen + a->text_len);
    p->vid_qkv = a->vid_qkv;
    p->txt_qkv = a->txt_qkv;
    p->dim = a->heads * kHeadDim;
    p->row_stride = 3LL * p->dim;
    p->heads = a->heads;
    p->text_len = a->text_len;
    p->npairs = p->plan.nwin * a->heads;
    p->nqb = (smax + kBlockM - 1) / kBlockM;
    p->qk_norm = a->qk_norm ? 1 : 0;
    p->rope_mode = a->rope_mode;
    p->rope_npos = a->rope_npos;
    p->eps = a->eps;
    p->scale = 1.f / std::sqrt(static_cast<float>(kHeadDim));
    p->gq_vid = a->gamma_q_vid;
    p->gk_vid = a->gamma_k_vid;
    p->gq_txt = a->gamma_q_txt ? a->gamma_q_txt : a->gamma_q_vid;
    p->gk_txt = a->gamma_k_txt ? a->gamma_k_txt : a->gamma_k_vid;
    p->rope_tab = reinterpret_cast<const float2*>(a->rope_table);
    p->vid_out = a->vid_out;
    p->dbg_pre = a->debug_pre;
    *smax_out = smax;
    return SV2_OK;
}

int64_t workspace_bytes(const AttnParams& p)
{
    const int64_t bytes = static_cast<int64_t>(p.plan.nwin) * p.text_len * p.dim * 2;
    return (bytes + 255) & ~int64_t(255);
}

template <typename TI, typename TO>
void launch_attention(const AttnParams& p, hipStream_t stream)
{
    const int groups = (p.npairs + 7) / 8;
    const unsigned grid = static_cast<unsigned>(groups) * 8u * static_cast<unsigned>(p.nqb);
    hipLaunchKernelGGL((window_attention_kernel<TI, TO>), dim3(grid), dim3(kThreads), 0, stream, p);
}

template <typename TI>
void launch_attention_in(const AttnParams& p, int out_dtype, hipStream_t stream)
{
    if (out_dtype == SV2_F32)
        launch_attention<TI, F32>(p, stream);
    else if (out_dtype == SV2_F16)
        launch_attention<TI, F16>(p, stream);
    else
        launch_attention<TI, BF16>(p, stream);
}

} // namespace
} // namespace sv2

extern "C" {

int64_t sv2_window_attention_workspace(const sv2_attn_args* args)
{
    using namespace sv2;
    AttnParams p;
    int smax = 0;
    const int rc = prepare(args, &p, &smax);
    if (rc != SV2_OK)
        return rc;
    return workspace_bytes(p);
}

int sv2_window_attention(const sv2_attn_args* args, void* stream_ptr)
{
    using namespace sv2;
    AttnParams p;
    int smax = 0;
    int rc = prepare(args, &p, &smax);
    if (rc != SV2_OK)
        return rc;
    if (!args->vid_out || (args->text_len > 0 && !args->txt_out))
        return set_error(SV2_EINVAL, "attention: null output pointer");
    const int64_t need = workspace_bytes(p);
    if (need > 0 && (!args->workspace || static_cast<int64_t>(args->workspace_bytes) < need))
        return set_error(SV2_EINVAL, "attention: workspace missing or too small");
    p.partial = static_cast<uint16_t*>(args->workspace);
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);

    if (args->qkv_dtype == SV2_F32)
        launch_attention_in<F32>(p, args->out_dtype, stream);
    else if (args->qkv_dtype == SV2_F16)
        launch_attention_in<F16>(p, args->out_dtype, stream);
    else
        launch_attention_in<BF16>(p, args->out_dtype, stream);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return hip_error(err, "window_attention_kernel launch");

    if (p.text_len > 0)
    {
        const long long count = static_cast<long long>(p.text_len) * p.dim;
        const unsigned grid = static_cast<unsigned>((count / 4 + 255) / 256);
        const float inv_nw = 1.f / static_cast<float>(p.plan.nwin);
        if (args->out_dtype == SV2_F32)
            hipLaunchKernelGGL(text_window_reduce_kernel<F32>, dim3(grid), dim3(256), 0, stream, p.partial,
                               args->txt_out, p.plan.nwin, count, inv_nw);
        else if (args->out_dtype == SV2_F16)
            hipLaunchKernelGGL(text_window_reduce_kernel<F16>, dim3(grid), dim3(256), 0, stream, p.partial,
                               args->txt_out, p.plan.nwin, count, inv_nw);
        else
            hipLaunchKernelGGL(text_window_reduce_kernel<BF16>, dim3(grid), dim3(256), 0, stream, p.partial,
                               args->txt_out, p.plan.nwin, count, inv_nw);
        err = hipGetLastError();
        if (err != hipSuccess)
            return hip_error(err, "text_window_reduce_kernel launch");
    }
    return SV2_OK;
}

int sv2_qk_prologue(const sv2_attn_args* args, float* q_out, float* k_out, float* v_out, void* stream_ptr)
{
    using namespace sv2;
    AttnParams p;
    int smax = 0;
    const int rc = prepare(args, &p, &smax);
    if (rc != SV2_OK)
        return rc;
    if (!q_out || !k_out || !v_out)
        return set_error(SV2_EINVAL, "qk_prologue: null output pointer");
    const int nrb = (smax + 15) / 16;
    const unsigned grid = static_cast<unsigned>(p.plan.nwin) * p.heads * nrb;
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    if (args->qkv_dtype == SV2_F32)
        hipLaunchKernelGGL(qk_prologue_kernel<F32>, dim3(grid), dim3(256), 0, stream, p, nrb, q_out, k_out, v_out);
    else if (args->qkv_dtype == SV2_F16)
        hipLaunchKernelGGL(qk_prologue_kernel<F16>, dim3(grid), dim3(256), 0, stream, p, nrb, q_out, k_out, v_out);
    else
        hipLaunchKernelGGL(qk_prologue_kernel<BF16>, dim3(grid), dim3(256), 0, stream, p, nrb, q_out, k_out, v_out);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return hip_error(err, "qk_prologue_kernel launch");
    return SV2_OK;
}

int sv2_window_index_map(const sv2_window_rule* rule, int32_t* out, void* stream_ptr)
{
    using namespace sv2;
    if (!rule || !out)
        return set_error(SV2_EINVAL, "sv2_window_index_map: null argument");
    PlanArgs plan;
    const int rc = build_plan(*rule, &plan);
    if (rc != SV2_OK)
        return rc;
    hipLaunchKernelGGL(window_index_map_kernel, dim3(plan.nwin), dim3(256), 0,
                       static_cast<hipStream_t>(stream_ptr), plan, out);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return hip_error(err, "window_index_map_kernel launch");
    return SV2_OK;
}

} // extern "C"
