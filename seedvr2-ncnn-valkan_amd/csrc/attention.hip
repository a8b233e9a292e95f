// Windowed joint video + text attention of the SeedVR2-3B DiT block on gfx950.
//
// Replaces SeedVR2DiTBlock::attention (seedvr2_dit_block.cpp:870-1091) and the
// reference's per-window qkv_prepare / attention / zero_buffer / window_sum
// shader chain (:192-330, :339-457, :541-572):
//
//   text_prepare_kernel   the q/k prologue of the L_txt text tokens, once per
//                         layer (their RoPE positions (l, l, l) do not depend
//                         on the window): bf16 q/k and transposed v (in the
//                         P*V operand type) into the workspace;
//   window_attention_kernel
//                         one 12-wave workgroup per (window, head) and up to
//                         384 query rows (windows with more rows split them
//                         evenly over several workgroups).  Every video row of
//                         the window is located through a per-window row table
//                         built in LDS from the closed-form plan (no
//                         materialised window copies).  Key and value tiles of
//                         64 keys move from global memory straight into LDS
//                         (global_load_lds, no staging registers), two tiles
//                         ahead: waves 0-7 fetch the key tile and run the k
//                         prologue (RMSNorm * gamma, RoPE, bf16) in place,
//                         waves 8-11 fetch the value tile and write v, rounded
//                         to bf16, transposed.  Each wave
//                         owns 32 query rows whose q prologue runs in
//                         registers.  S^T = K Q^T on bf16 MFMA (exact
//                         operands), online softmax per 32-key subtile in fp32
//                         with lazy rescaling (row max / sum exchanged between
//                         half-waves with v_permlane32_swap), O^T += V^T P^T on
//                         fp16 MFMA (fp16 inputs: P and V as fp16) or bf16 MFMA
//                         (fp32 / bf16 inputs: exact bf16 V, P split into 3 / 2
//                         bf16 terms).  Ragged windows: keys past the window are
//                         masked, query rows past it are not stored.  Video
//                         outputs are written once (the windows partition the
//                         grid), text outputs to per-window bf16 partials;
//   text_window_reduce_kernel
//                         text outputs: partials summed in window order, times
//                         1/nW, as the reference accumulates them.
#include "sv2_internal.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>

namespace sv2
{
namespace
{

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(4))) _Float16 f16x4;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kWaves = 12;
constexpr int kThreads = kWaves * 64;        // 768
constexpr int kLoaderThreads = 512;          // fp32 inputs: waves 0-7 load and prepare key/value tiles
constexpr int kRowsPerGroup = kWaves * 32;   // query rows per workgroup
constexpr int kBlockN = 64;                  // keys per tile
constexpr int kTileBytes = kBlockN * kHeadDim * 2; // one K, V or V^T tile of 16-bit values
constexpr int kVtStride = 64;                // halfs per row of the transposed value tile (swizzled)
constexpr int kTextPad = 64;                 // text rows of the prepared workspace are padded to this
constexpr int kDirectTextTiles = 2;          // text tiles fetched before the loop come as finished V^T tiles
constexpr int kMaxVideoRows = 4096;          // video tokens per window (local coordinates fit 10 bits)
constexpr int kPrepRows = 16;                // text rows per text_prepare workgroup
constexpr int kMaxLds = 160 * 1024;          // LDS of one gfx950 CU
constexpr int kMaxOrdered = 256;             // plans with at most this many windows run largest-first
// s_waitcnt immediates for vmcnt(0) / vmcnt(4) with expcnt and lgkmcnt left
// unconstrained (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] |
// vmcnt[5:4] << 14).
constexpr int kWaitVmcnt0 = 0x0F70;
constexpr int kWaitVmcnt2 = 0x0F72;
constexpr int kWaitVmcnt4 = 0x0F74;
constexpr float kRescaleLog2 = 8.f;          // O is rescaled only when a row max grows by more than 2^8
constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------- element types

// kPTerms: how P enters O^T += V^T P^T.  1: P rounded to fp16 against V held
// as fp16 (the bf16-rounded values, exact in fp16 within its range) on the
// fp16 MFMA.  2 or 3: V held as its exact bf16 value and P split into that
// many bf16 terms (hi + mid [+ lo], each the rounded remainder of the last),
// one bf16 MFMA per term: 16 or 24 significant bits of P and no fp16 range
// limit on V.  The fp32 input mode is the parity mode and takes 3 terms.
//
// kExact: the q/k prologue follows the reference's arithmetic step for step
// (double sum of squares, float(sum / 128), correctly rounded fp32 sqrt and
// divide, unfused products): the fp32 and bf16 input modes.  The fp16 mode
// keeps an fp32 sum, the hardware reciprocal square root and fused RoPE
// products (each may move a q/k element by one bf16 ulp, rarely).
struct F32
{
    static constexpr int kVec = 2; // uint4 per 8 elements
    static constexpr bool kDma = false;
    static constexpr int kPTerms = 3;
    static constexpr bool kExact = true;
};
struct F16
{
    static constexpr int kVec = 1;
    static constexpr bool kDma = true;
    static constexpr int kPTerms = 1;
    static constexpr bool kExact = false;
};
struct BF16
{
    static constexpr int kVec = 1;
    static constexpr bool kDma = true;
    static constexpr int kPTerms = 2;
    static constexpr bool kExact = true;
};

template <typename T>
__device__ inline void load_raw8(const void* base, long long offset, uint4 (&r)[T::kVec])
{
    if constexpr (T::kVec == 2)
    {
        const uint4* src = reinterpret_cast<const uint4*>(static_cast<const float*>(base) + offset);
        r[0] = src[0];
        r[1] = src[1];
    }
    else
    {
        r[0] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + offset);
    }
}

template <typename T>
__device__ inline void raw8_to_float(const uint4 (&r)[T::kVec], float x[8]);

template <>
__device__ inline void raw8_to_float<F32>(const uint4 (&r)[2], float x[8])
{
    const uint32_t w[8] = {r[0].x, r[0].y, r[0].z, r[0].w, r[1].x, r[1].y, r[1].z, r[1].w};
#pragma unroll
    for (int e = 0; e < 8; e++)
        x[e] = __builtin_bit_cast(float, w[e]);
}

template <>
__device__ inline void raw8_to_float<F16>(const uint4 (&r)[1], float x[8])
{
    const f16x8 v = __builtin_bit_cast(f16x8, r[0]);
#pragma unroll
    for (int e = 0; e < 8; e++)
        x[e] = static_cast<float>(v[e]);
}

template <>
__device__ inline void raw8_to_float<BF16>(const uint4 (&r)[1], float x[8])
{
    const uint32_t w[4] = {r[0].x, r[0].y, r[0].z, r[0].w};
#pragma unroll
    for (int e = 0; e < 4; e++)
    {
        x[2 * e] = __builtin_bit_cast(float, w[e] << 16);
        x[2 * e + 1] = __builtin_bit_cast(float, w[e] & 0xffff0000u);
    }
}

template <typename T>
__device__ inline void load8(const void* base, long long offset, float x[8])
{
    uint4 r[T::kVec];
    load_raw8<T>(base, offset, r);
    raw8_to_float<T>(r, x);
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
    f16x4 h;
    h[0] = static_cast<_Float16>(v[0]);
    h[1] = static_cast<_Float16>(v[1]);
    h[2] = static_cast<_Float16>(v[2]);
    h[3] = static_cast<_Float16>(v[3]);
    *reinterpret_cast<f16x4*>(static_cast<_Float16*>(base) + offset) = h;
}

// Two floats rounded to bf16 (nearest even) in one v_cvt_pk_bf16_f32; a
// pair converted element by element costs a second conversion and a pack.
__device__ inline uint32_t bf16_pair_bits(float a, float b)
{
    typedef __attribute__((ext_vector_type(2))) float f32x2;
    typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
}

// bf16 rounded to nearest even (identity on attention outputs, which are
// bf16 values already; the text averages are not).
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

// 8 floats -> 8 bf16 (round to nearest even, v_cvt_pk_bf16_f32).  For finite
// values this is the reference's rounding (seedvr2_dit_block.cpp:68-79).
__device__ inline uint4 to_bf16x8(const float x[8])
{
    bf16x8 v;
#pragma unroll
    for (int e = 0; e < 8; e++)
        v[e] = static_cast<__bf16>(x[e]);
    return __builtin_bit_cast(uint4, v);
}

template <typename T>
__device__ inline void store2(void* base, long long offset, float a, float b);

template <>
__device__ inline void store2<F32>(void* base, long long offset, float a, float b)
{
    *reinterpret_cast<float2*>(static_cast<float*>(base) + offset) = make_float2(a, b);
}

template <>
__device__ inline void store2<F16>(void* base, long long offset, float a, float b)
{
    f16x2 h;
    h[0] = static_cast<_Float16>(a);
    h[1] = static_cast<_Float16>(b);
    *reinterpret_cast<f16x2*>(static_cast<_Float16*>(base) + offset) = h;
}

template <>
__device__ inline void store2<BF16>(void* base, long long offset, float a, float b)
{
    const uint32_t lo = __builtin_bit_cast(uint32_t, bf16_round(a)) >> 16;
    const uint32_t hi = __builtin_bit_cast(uint32_t, bf16_round(b)) & 0xffff0000u;
    *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(base) + offset) = lo | hi;
}

// ---------------------------------------------------------------- parameters

// Byte offsets of the dynamic LDS regions of one workgroup.
struct LdsLayout
{
    int k;       // [3][64 rows][16 slots] x 16 B: key tiles, swizzled; bf16 after the prologue
    int vraw;    // [2] x 16 KB: fetched value tiles, rows by 32-dim quarters (vq_offset)
    int vt;      // [2][128 rows][64 keys]: transposed value tiles in the P*V operand type, swizzled
    int rows;    // int2 [vmax]: global video row, packed local (t | y << 10 | x << 20)
    int rope;    // float2 [rope_rows][24]: cos/sin rows t..., y..., x... of the window
    int gamma;   // float [2][128]: q, k gammas of the video branch
    int krope;   // int2 [16 chunks][4 pairs]: a key lane's RoPE table offset and position shift
    int total;
};

struct AttnParams
{
    PlanArgs plan;
    LdsLayout lds;
    const void* vid_qkv;
    const void* txt_qkv;
    long long row_stride; // elements per qkv row (3*D)
    int heads;
    int dim;              // D = heads * 128
    int text_len;
    int text_pad;         // text_len rounded up to a multiple of kTextPad
    int npairs;           // windows * heads
    int nqb;              // query blocks per (window, head)
    int qk_norm;
    int rope_npos;
    int out_dtype;
    float eps;
    float score_log2;     // (1/sqrt(128)) * log2(e): exp(s*scale - m) = exp2(s*score_log2 - m')
    const float* gq_vid;
    const float* gk_vid;
    const float* gq_txt;
    const float* gk_txt;
    const float2* rope_tab; // [3][npos][24] (cos, sin)
    void* vid_out;
    uint16_t* partial;      // [nwin][text_len][D] bf16
    float* dbg_pre;         // optional [sum S][D]
    uint16_t* txt_q;        // [heads][text_len][128] bf16, prepared
    uint16_t* txt_k;        // [heads][text_len][128] bf16, prepared
    uint16_t* txt_vt;       // [heads][text_pad][128] P*V operand type, prepared
    uint16_t* txt_vlds;     // [heads][kDirectTextTiles][64 * 128]: the first text tiles' V^T
                            // in the byte order of an LDS V^T tile (16-bit inputs)
    float* nq_txt;          // optional debug captures [text_len][D]: text q, k after the norm, before RoPE
    float* nk_txt;
    int ordered;            // windows dispatched in the order of `order` (else in plan order)
    int exact;              // the reference-order fp64 kernel (fp32 inputs)
    long long seq_rows;     // sum over windows of S_w (window-sequence rows)
    int16_t order[kMaxOrdered]; // window indices by decreasing video length
};

// ---------------------------------------------------------------- lane helpers

// Sum over the 16 lanes of a row group: quad xor 1, quad xor 2, half-row
// mirror, row mirror (DPP), every lane ends with the full sum.
__device__ inline float row16_sum(float v)
{
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
    return v;
}

// The values of lanes l % 32 and l % 32 + 32 (v_permlane32_swap, a VALU op
// exchanging the upper half-wave of one register with the lower half-wave of
// another): starting from two copies of v, one register ends up holding the
// lower half-wave's values in every lane and the other the upper half-wave's,
// so both lanes of a pair receive the two operands in the same order and the
// reductions below agree bit for bit.  Written as inline assembly (with the
// wait states a VALU write needs before a permlane read): the compiler's
// builtin for this instruction treats its two results as one value.
__device__ inline void with_partner(float v, float* a, float* b)
{
    float x = v;
    float y = v;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(x), "+v"(y));
    *a = x;
    *b = y;
}

__device__ inline float partner_max(float v)
{
    float a, b;
    with_partner(v, &a, &b);
    return fmaxf(a, b);
}

__device__ inline float partner_sum(float v)
{
    float a, b;
    with_partner(v, &a, &b);
    return a + b;
}

// The double versions: the two 32-bit halves move through the same lane
// exchanges.
template <int kCtrl>
__device__ inline double dpp_f64(double v)
{
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(u)), kCtrl, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(u >> 32)), kCtrl, 0xF, 0xF,
                                               false);
    return __builtin_bit_cast(double, (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
                                          static_cast<uint32_t>(lo));
}

__device__ inline double row16_sum_f64(double v)
{
    v += dpp_f64<0xB1>(v);
    v += dpp_f64<0x4E>(v);
    v += dpp_f64<0x141>(v);
    v += dpp_f64<0x140>(v);
    return v;
}

__device__ inline double partner_sum_f64(double v)
{
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    float lo_a, lo_b, hi_a, hi_b;
    with_partner(__builtin_bit_cast(float, static_cast<uint32_t>(u)), &lo_a, &lo_b);
    with_partner(__builtin_bit_cast(float, static_cast<uint32_t>(u >> 32)), &hi_a, &hi_b);
    const double a = __builtin_bit_cast(double, (static_cast<uint64_t>(__builtin_bit_cast(uint32_t, hi_a)) << 32) |
                                                    __builtin_bit_cast(uint32_t, lo_a));
    const double b = __builtin_bit_cast(double, (static_cast<uint64_t>(__builtin_bit_cast(uint32_t, hi_b)) << 32) |
                                                    __builtin_bit_cast(uint32_t, lo_b));
    return a + b;
}

// ---------------------------------------------------------------- prologue

// RoPE axis and table slot of an even head dim.  Dims a variant leaves
// unrotated (126, 127 of the reference layout) read slot 23, which the table
// fills with (cos, sin) = (1, 0).
template <int RM>
__device__ inline void rope_axis_slot(int d, int* axis, int* slot)
{
    if constexpr (RM == SV2_ROPE_ABSOLUTE)
    {
        if (d < 32)
        {
            *axis = 0;
            *slot = d >> 1;
        }
        else if (d < 80)
        {
            *axis = 1;
            *slot = (d - 32) >> 1;
        }
        else
        {
            *axis = 2;
            *slot = (d - 80) >> 1;
        }
    }
    else
    {
        if (d < 126)
        {
            const int a = d / 42;
            *axis = a;
            *slot = (d - 42 * a) >> 1;
        }
        else
        {
            *axis = 2;
            *slot = kRopePairSlots - 1;
        }
    }
}

__device__ inline float inv_rms(float ss, float eps)
{
    return __builtin_amdgcn_rsqf(ss * (1.f / 128.f) + eps);
}

// 1.f / std::sqrt(float(ss / 128) + eps) as the reference evaluates it
// (seedvr2_dit_block.cpp:947-950) from the double sum of squares ss.  The
// float sqrt and divide are correctly rounded: each is formed in double and
// rounded once to float, which for float operands gives the correctly
// rounded float result (53 >= 2 * 24 + 2 bits).
__device__ inline float inv_rms_exact(double ss, float eps)
{
    const float mean = static_cast<float>(ss * (1.0 / 128.0));
    const float root = static_cast<float>(__builtin_sqrt(static_cast<double>(mean + eps)));
    return static_cast<float>(1.0 / static_cast<double>(root));
}

// Partial double sum of squares of n values (the products are exact in
// double, so a fused multiply-add rounds as the reference's multiply then add).
template <int N>
__device__ inline double square_sum_f64(const float* x)
{
    double ss = 0.0;
#pragma unroll
    for (int e = 0; e < N; e++)
        ss = __builtin_fma(static_cast<double>(x[e]), static_cast<double>(x[e]), ss);
    return ss;
}

// (a, b) -> (a c - b s, b c + a s), each product rounded before the add as in
// the reference's float expression.
__device__ inline float2 rotate_unfused(float first, float second, float2 c)
{
#pragma clang fp contract(off)
    return make_float2(first * c.x - second * c.y, second * c.x + first * c.y);
}

// y = x * inv * gamma, then the rotation of the 4 adjacent pairs of the 8
// dims (seedvr2_dit_block.cpp:950-971): (a, b) -> (a c - b s, b c + a s).
// cs(q) gives the (cos, sin) of pair q.  kExact: unfused products (the
// reference's rounding); else one product fused into the add.  norm_out (the
// debug captures only): the 8 values after the norm, before the rotation.
template <bool kRotate, bool kExact, typename CosSin>
__device__ inline void scale_rotate8(float x[8], const float* gamma8, float inv, bool norm, CosSin cs,
                                     float* norm_out = nullptr)
{
    if (norm)
    {
#pragma unroll
        for (int e = 0; e < 8; e++)
            x[e] = x[e] * inv * gamma8[e];
    }
    if (norm_out)
    {
#pragma unroll
        for (int e = 0; e < 8; e++)
            norm_out[e] = x[e];
    }
    if constexpr (kRotate)
    {
#pragma unroll
        for (int q = 0; q < 4; q++)
        {
            const float2 c = cs(q);
            const float first = x[2 * q];
            const float second = x[2 * q + 1];
            if constexpr (kExact)
            {
                const float2 r = rotate_unfused(first, second, c);
                x[2 * q] = r.x;
                x[2 * q + 1] = r.y;
            }
            else
            {
                x[2 * q] = __builtin_fmaf(first, c.x, -(second * c.y));
                x[2 * q + 1] = __builtin_fmaf(second, c.x, first * c.y);
            }
        }
    }
}

// ---------------------------------------------------------------- layout helpers

// Row permutation of a 32-key S^T tile: swapping bits 2 and 3 of the row makes
// each lane's 16 accumulator registers hold keys 8g..8g+7 and 16+8g..16+8g+7
// (g = lane / 32), which is exactly the k-slice the lane supplies as the B
// operand of the following P*V MFMA.
__device__ inline int key_perm(int i)
{
    return (i & ~12) | ((i & 4) << 1) | ((i & 8) >> 1);
}

// Byte offset of chunk c (dims 8c..8c+7) of row r in a key tile.  The tile is
// split into two 8 KB halves (dims 0-63, 64-127); in a half, row r holds 8
// 16-byte slots at r * 128 and chunk c & 7 sits in slot (c & 7) ^ ((r >> 1) & 7).
// The MFMA operand reads of 16 consecutive rows then hit 16 different slot
// positions, and a lane's eight reads of one row are four per-lane bases plus
// immediate offsets (half * 8192).
__device__ inline int k_slot_offset(int r, int c)
{
    return (c >> 3) * 8192 + r * 128 + (((c & 7) ^ ((r >> 1) & 7)) << 4);
}

// Byte offset of chunk c (dims 8c..8c+7) of key row r in a fetched value
// tile: four 4 KB quarters (dims 32q..32q+31), 64 bytes per row within a
// quarter.  The transposing reads of the V^T transpose (below) touch eight
// rows of one quarter, 64 bytes each: every bank at most twice per wave and
// once per half-wave, with no swizzle.
__device__ inline int vq_offset(int r, int c)
{
    return (c >> 2) * 4096 + r * 64 + ((c & 3) << 4);
}

// Swizzled offset (in halfs) of key group `grp` (8 keys, 0..7) in row d of the
// transposed value tile; spreads the 16-byte operand reads of 8 consecutive
// rows and the 16-byte writes of 16 consecutive rows over the banks.
__device__ inline int vt_offset(int d, int grp)
{
    return d * kVtStride + ((grp ^ ((d ^ (d >> 3)) & 7)) << 3);
}

// Two values rounded to bf16 (the reference's rounding of v) and handed to the
// fp16 MFMA: the bf16 values are exact in fp16 within its range.
__device__ inline f16x2 bf16_pair_as_f16(float a, float b)
{
    const uint32_t u = bf16_pair_bits(a, b);
    return __builtin_bit_cast(f16x2, __builtin_amdgcn_cvt_pkrtz(__builtin_bit_cast(float, u << 16),
                                                                __builtin_bit_cast(float, u & 0xffff0000u)));
}

// Two values of v rounded to bf16, packed in the operand type of the P*V MFMA
// of input type TI: fp16 of the bf16 values (one P term) or the bf16 bits.
template <typename TI>
__device__ inline uint32_t v_pair_operand(float a, float b)
{
    if constexpr (TI::kPTerms == 1)
        return __builtin_bit_cast(uint32_t, bf16_pair_as_f16(a, b));
    else
        return bf16_pair_bits(a, b);
}

// Writes the transposed value items of keys 2r, 2r+1 (8 dims at d0) in the
// P*V operand type of input type TI.
template <typename TI>
__device__ inline void store_vt_pair(char* vt, int r, int d0, const float v0[8], const float v1[8])
{
    uint16_t* t = reinterpret_cast<uint16_t*>(vt);
    const int key = 2 * r;
#pragma unroll
    for (int e = 0; e < 8; e++)
        *reinterpret_cast<uint32_t*>(&t[vt_offset(d0 + e, key >> 3) + (key & 7)]) = v_pair_operand<TI>(v0[e], v1[e]);
}

// Eight values of v rounded to bf16, in the P*V operand type of input type TI.
template <typename TI>
__device__ inline uint4 v_operand8(const float x[8])
{
    return make_uint4(v_pair_operand<TI>(x[0], x[1]), v_pair_operand<TI>(x[2], x[3]),
                      v_pair_operand<TI>(x[4], x[5]), v_pair_operand<TI>(x[6], x[7]));
}

// A P*V operand element back in fp32 (for the prologue debug captures).
template <typename TI>
__device__ inline float v_operand_value(uint16_t bits)
{
    if constexpr (TI::kPTerms == 1)
        return static_cast<float>(__builtin_bit_cast(_Float16, bits));
    else
        return __builtin_bit_cast(float, static_cast<uint32_t>(bits) << 16);
}

// A copy of v the compiler cannot see through.  Lane-derived offsets computed
// from it inside the tile loop are recomputed each iteration (two or three
// integer ops each) instead of being hoisted and kept live across the loop,
// which would exceed the 168 VGPRs a 12-wave workgroup allows.
__device__ inline int opaque(int v)
{
    asm volatile("" : "+v"(v));
    return v;
}

// One 16-byte global -> LDS copy per lane (global_load_lds_dwordx4): lane i
// writes LDS bytes [lds + 16 i, lds + 16 i + 16), lds being wave-uniform.
// Issued through inline assembly so that the compiler does not treat later
// LDS reads as possibly depending on it (it would otherwise wait for every
// fetch in flight before any LDS read); the kernel places the vmcnt waits
// itself.  M0 (the LDS base of the copy) is saved and restored.
__device__ inline void dma16(const void* g, char* lds)
{
    const unsigned base = __builtin_amdgcn_readfirstlane(static_cast<unsigned>(reinterpret_cast<size_t>(lds)));
    unsigned saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %2, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "s"(base), "v"(g)
                 : "memory");
}

// ---------------------------------------------------------------- per-window staging

// Row of the staged RoPE table where each axis starts.
struct RopeBase
{
    int b[3];
};

__device__ inline RopeBase rope_base(const WindowBox& box)
{
    RopeBase r;
    r.b[0] = 0;
    r.b[1] = box.lt;
    r.b[2] = box.lt + box.lh;
    return r;
}

struct Staged
{
    const int2* rows;
    const float2* rope;
    const float* gamma;
};

__device__ inline Staged staged(const AttnParams& p, const char* smem)
{
    Staged s;
    s.rows = reinterpret_cast<const int2*>(smem + p.lds.rows);
    s.rope = reinterpret_cast<const float2*>(smem + p.lds.rope);
    s.gamma = reinterpret_cast<const float*>(smem + p.lds.gamma);
    return s;
}

// Fills the gather table, the window's RoPE rows and the gammas (threads
// stride by nthreads; the caller synchronises).
template <int RM>
__device__ inline void stage_window(const AttnParams& p, const WindowBox& box, char* smem, int tid, int nthreads)
{
    int2* rows = reinterpret_cast<int2*>(smem + p.lds.rows);
    float2* rope = reinterpret_cast<float2*>(smem + p.lds.rope);
    float* gamma = reinterpret_cast<float*>(smem + p.lds.gamma);
    for (int j = tid; j < box.vlen; j += nthreads)
    {
        int lt, ly, lx;
        const int row = window_video_row(p.plan, box, j, &lt, &ly, &lx);
        rows[j] = make_int2(row, static_cast<int>(static_cast<uint32_t>(lt) | (static_cast<uint32_t>(ly) << 10) |
                                                  (static_cast<uint32_t>(lx) << 20)));
    }
    if constexpr (RM != SV2_ROPE_NONE)
    {
        const int nrows = box.lt + box.lh + box.lw;
        constexpr bool ref = RM == SV2_ROPE_REFERENCE;
        for (int i = tid; i < nrows * kRopePairSlots; i += nthreads)
        {
            const int r = i / kRopePairSlots;
            const int slot = i - r * kRopePairSlots;
            int axis, gpos;
            if (r < box.lt)
            {
                axis = 0;
                gpos = ref ? p.text_len + r : box.t0 + r; // (L_txt + t - t0) or absolute t
            }
            else if (r < box.lt + box.lh)
            {
                axis = 1;
                gpos = (r - box.lt) + (ref ? 0 : box.h0);
            }
            else
            {
                axis = 2;
                gpos = (r - box.lt - box.lh) + (ref ? 0 : box.w0);
            }
            rope[i] = p.rope_tab[(axis * p.rope_npos + gpos) * kRopePairSlots + slot];
        }
    }
    for (int i = tid; i < 2 * kHeadDim; i += nthreads)
    {
        const float* src = i < kHeadDim ? p.gq_vid : p.gk_vid;
        gamma[i] = p.qk_norm ? src[i % kHeadDim] : 1.f;
    }
}

// Query operand of S^T = K Q^T for window-sequence row qrow (clamped by the
// caller to a valid row): the lane holds dims 16c + 8g .. +7 of the row, the
// partner lane (lane ^ 32) the other half.  Video rows: the raw row is loaded
// by query_load and its prologue runs in query_finish; text rows read the
// prepared workspace.
template <typename TI>
struct QueryRaw
{
    uint4 r[8][TI::kVec];
};

template <typename TI>
__device__ inline void query_load(const AttnParams& p, const Staged& s, const WindowBox& box, int head, int qrow,
                                  int g, QueryRaw<TI>& raw)
{
    if (qrow < box.vlen)
    {
        const long long base = static_cast<long long>(s.rows[qrow].x) * p.row_stride +
                               static_cast<long long>(head) * kHeadDim + 8 * g;
#pragma unroll
        for (int c = 0; c < 8; c++)
            load_raw8<TI>(p.vid_qkv, base + 16 * c, raw.r[c]);
    }
    else
    {
        const uint16_t* src = p.txt_q + (static_cast<long long>(head) * p.text_len + (qrow - box.vlen)) * kHeadDim + 8 * g;
#pragma unroll
        for (int c = 0; c < 8; c++)
        {
            raw.r[c][0] = *reinterpret_cast<const uint4*>(src + 16 * c);
            if constexpr (TI::kVec == 2)
                raw.r[c][1] = make_uint4(0u, 0u, 0u, 0u);
        }
    }
}

// norm_out (the debug captures only): where dims 8g.. of the row's values
// after the norm and before RoPE go (chunk c at norm_out + 16 c); video rows.
template <typename TI, int RM>
__device__ inline void query_finish(const AttnParams& p, const Staged& s, const WindowBox& box, int qrow, int g,
                                    const QueryRaw<TI>& raw, bf16x8 qf[8], float* norm_out = nullptr)
{
    const bool is_video = qrow < box.vlen;
    if (!is_video)
    {
#pragma unroll
        for (int c = 0; c < 8; c++)
            qf[c] = __builtin_bit_cast(bf16x8, raw.r[c][0]);
    }
    // both lanes of a pair take the same branch; the partner exchange below
    // runs on every lane
    float x[64];
#pragma unroll
    for (int c = 0; c < 8; c++)
    {
        if (is_video)
            raw8_to_float<TI>(raw.r[c], &x[8 * c]);
        else
#pragma unroll
            for (int e = 0; e < 8; e++)
                x[8 * c + e] = 0.f;
    }
    float inv = 1.f;
    if (p.qk_norm)
    {
        if constexpr (TI::kExact)
        {
            inv = inv_rms_exact(partner_sum_f64(square_sum_f64<64>(x)), p.eps);
        }
        else
        {
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < 64; i++)
                ss = __builtin_fmaf(x[i], x[i], ss);
            inv = inv_rms(partner_sum(ss), p.eps);
        }
    }
    if (!is_video)
        return;
    // RoPE lookups: the lane's three table rows (t, y, x of its token) are
    // resolved once; the axis and slot of each pair are constants of the
    // unrolled chunk and pair indices for either value of the lane half g, so
    // a lookup is a select between two precomputed offsets
    const uint32_t packed = static_cast<uint32_t>(s.rows[qrow].y);
    const RopeBase rb = rope_base(box);
    const int base0 = (rb.b[0] + static_cast<int>(packed & 1023u)) * kRopePairSlots;
    const int base1 = (rb.b[1] + static_cast<int>((packed >> 10) & 1023u)) * kRopePairSlots;
    const int base2 = (rb.b[2] + static_cast<int>((packed >> 20) & 1023u)) * kRopePairSlots;
#pragma unroll
    for (int c = 0; c < 8; c++)
    {
        const int d0 = 16 * c + 8 * g;
        scale_rotate8<RM != SV2_ROPE_NONE, TI::kExact>(&x[8 * c], &s.gamma[d0], inv, p.qk_norm != 0, [&](int q) {
            int axis_a, slot_a, axis_b, slot_b;
            rope_axis_slot<RM>(16 * c + 2 * q, &axis_a, &slot_a);
            rope_axis_slot<RM>(16 * c + 2 * q + 8, &axis_b, &slot_b);
            const int ia = (axis_a == 0 ? base0 : (axis_a == 1 ? base1 : base2)) + slot_a;
            const int ib = (axis_b == 0 ? base0 : (axis_b == 1 ? base1 : base2)) + slot_b;
            return s.rope[g ? ib : ia];
        }, norm_out ? norm_out + 16 * c : nullptr);
        qf[c] = __builtin_bit_cast(bf16x8, to_bf16x8(&x[8 * c]));
    }
}

// Makes the query operand's loads complete here rather than at its first use
// in the tile loop: the compiler's wait for them counts only its own memory
// operations (not the key/value fetches, issued through inline assembly), so
// a wait inside the loop would also hold the fetches in flight there.
__device__ inline void settle(bf16x8 qf[8])
{
#pragma unroll
    for (int c = 0; c < 8; c++)
        asm volatile("" : "+v"(qf[c]));
}

// Per-thread RoPE lookup of a key chunk: the chunk (8 dims) is fixed per
// thread, so the table offset of each of its 4 pairs is too; only the row's
// local position varies.
struct KeyRope
{
    int off[4];
    int shift[4];
};

template <int RM>
__device__ inline KeyRope key_rope(const RopeBase& rb, int d0)
{
    KeyRope k;
#pragma unroll
    for (int q = 0; q < 4; q++)
    {
        int axis, slot;
        rope_axis_slot<RM>(d0 + 2 * q, &axis, &slot);
        // selects rather than rb.b[axis]: a runtime index would put the
        // array in scratch memory
        const int row0 = axis == 0 ? rb.b[0] : (axis == 1 ? rb.b[1] : rb.b[2]);
        k.off[q] = row0 * kRopePairSlots + slot;
        k.shift[q] = 10 * axis;
    }
    return k;
}

// The window's KeyRope of every key chunk, staged once so the tile loop reads
// a lane's four (table offset, position shift) pairs with two LDS loads: the
// per-pair axis selection, recomputed each tile, costs divergent branches.
// Threads 0-63 write one pair each (chunk = tid / 4, pair tid % 4); the
// caller synchronises.
template <int RM>
__device__ inline void stage_key_rope(const AttnParams& p, const WindowBox& box, char* smem, int tid)
{
    if constexpr (RM != SV2_ROPE_NONE)
    {
        if (tid < 64)
        {
            const KeyRope k = key_rope<RM>(rope_base(box), 8 * (tid >> 2));
            const int q = tid & 3;
            const int off = q == 0 ? k.off[0] : (q == 1 ? k.off[1] : (q == 2 ? k.off[2] : k.off[3]));
            const int shift = q == 0 ? k.shift[0] : (q == 1 ? k.shift[1] : (q == 2 ? k.shift[2] : k.shift[3]));
            reinterpret_cast<int2*>(smem + p.lds.krope)[tid] = make_int2(off, shift);
        }
    }
}

// A key lane's KeyRope from the staged table (stage_key_rope).
template <int RM>
__device__ inline KeyRope staged_key_rope(const AttnParams& p, const char* smem, int chunk)
{
    KeyRope k;
    if constexpr (RM != SV2_ROPE_NONE)
    {
        const int4* t = reinterpret_cast<const int4*>(smem + p.lds.krope) + 2 * chunk;
        const int4 a = t[0];
        const int4 b = t[1];
        k.off[0] = a.x;
        k.shift[0] = a.y;
        k.off[1] = a.z;
        k.shift[1] = a.w;
        k.off[2] = b.x;
        k.shift[2] = b.y;
        k.off[3] = b.z;
        k.shift[3] = b.w;
    }
    else
    {
#pragma unroll
        for (int q = 0; q < 4; q++)
        {
            k.off[q] = 0;
            k.shift[q] = 0;
        }
    }
    return k;
}

// Prologue of one key chunk (8 dims of a row whose 128 dims are spread over
// 16 consecutive lanes, all active): per-head RMSNorm (fp32 sum of squares),
// gamma, RoPE, bf16 rounding.
template <int RM, bool kExact>
__device__ inline uint4 key_chunk(const AttnParams& p, const Staged& s, const KeyRope& kr, float x[8], int d0,
                                  uint32_t packed, float* norm_out = nullptr)
{
    float inv = 1.f;
    if (p.qk_norm)
    {
        if constexpr (kExact)
        {
            inv = inv_rms_exact(row16_sum_f64(square_sum_f64<8>(x)), p.eps);
        }
        else
        {
            float ss = 0.f;
#pragma unroll
            for (int e = 0; e < 8; e++)
                ss = __builtin_fmaf(x[e], x[e], ss);
            inv = inv_rms(row16_sum(ss), p.eps);
        }
    }
    scale_rotate8<RM != SV2_ROPE_NONE, kExact>(x, &s.gamma[kHeadDim + d0], inv, p.qk_norm != 0, [&](int q) {
        const int local = static_cast<int>((packed >> kr.shift[q]) & 1023u);
        return s.rope[kr.off[q] + local * kRopePairSlots];
    }, norm_out);
    return to_bf16x8(x);
}

// ---------------------------------------------------------------- text prepare

// Text tokens: q/k prologue with the text branch's gammas and positions
// (l, l, l) in the reference RoPE mode (text is not rotated in the absolute
// mode), v rounded to bf16 and stored in the P*V operand type, [heads][text_pad][128]
// with zero rows up to text_pad so masked keys multiply finite values.
template <typename TI, int RM>
__global__ __launch_bounds__(256) void text_prepare_kernel(AttnParams p)
{
    const int head = blockIdx.y;
    const int l = blockIdx.x * kPrepRows + (threadIdx.x >> 4);
    const int chunk = threadIdx.x & 15;
    const int d0 = chunk * 8;
    const bool valid = l < p.text_len;
    const long long row = static_cast<long long>(valid ? l : 0) * p.row_stride + static_cast<long long>(head) * kHeadDim;
    float q[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float k[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (valid)
    {
        load8<TI>(p.txt_qkv, row + d0, q);
        load8<TI>(p.txt_qkv, row + p.dim + d0, k);
        load8<TI>(p.txt_qkv, row + 2LL * p.dim + d0, v);
    }
    const int pos = valid ? l : 0;
    auto cs = [&](int qq) {
        int axis, slot;
        rope_axis_slot<RM>(d0 + 2 * qq, &axis, &slot);
        return p.rope_tab[(axis * p.rope_npos + pos) * kRopePairSlots + slot];
    };
    float gq[8];
    float gk[8];
#pragma unroll
    for (int e = 0; e < 8; e++)
    {
        gq[e] = p.qk_norm ? p.gq_txt[d0 + e] : 1.f;
        gk[e] = p.qk_norm ? p.gk_txt[d0 + e] : 1.f;
    }
    float iq = 1.f;
    float ik = 1.f;
    if (p.qk_norm)
    {
        if constexpr (TI::kExact)
        {
            iq = inv_rms_exact(row16_sum_f64(square_sum_f64<8>(q)), p.eps);
            ik = inv_rms_exact(row16_sum_f64(square_sum_f64<8>(k)), p.eps);
        }
        else
        {
            float sq = 0.f;
            float sk = 0.f;
#pragma unroll
            for (int e = 0; e < 8; e++)
            {
                sq = __builtin_fmaf(q[e], q[e], sq);
                sk = __builtin_fmaf(k[e], k[e], sk);
            }
            iq = inv_rms(row16_sum(sq), p.eps);
            ik = inv_rms(row16_sum(sk), p.eps);
        }
    }
    constexpr bool rotate = RM == SV2_ROPE_REFERENCE;
    const long long cap = (static_cast<long long>(valid ? l : 0) * p.dim) + static_cast<long long>(head) * kHeadDim + d0;
    scale_rotate8<rotate, TI::kExact>(q, gq, iq, p.qk_norm != 0, cs, (p.nq_txt && valid) ? p.nq_txt + cap : nullptr);
    scale_rotate8<rotate, TI::kExact>(k, gk, ik, p.qk_norm != 0, cs, (p.nk_txt && valid) ? p.nk_txt + cap : nullptr);
    const uint4 qb = to_bf16x8(q);
    const uint4 kb = to_bf16x8(k);
    if (l >= p.text_pad)
        return;
    if (valid)
    {
        const long long o = (static_cast<long long>(head) * p.text_len + l) * kHeadDim + d0;
        *reinterpret_cast<uint4*>(p.txt_q + o) = qb;
        *reinterpret_cast<uint4*>(p.txt_k + o) = kb;
    }
    // rows past text_len are zero (+0.0 is the all-zero pattern in fp16 and
    // bf16 alike): masked keys then multiply finite values
    const uint4 vop = valid ? v_operand8<TI>(v) : make_uint4(0u, 0u, 0u, 0u);
    *reinterpret_cast<uint4*>(p.txt_vt + (static_cast<long long>(head) * p.text_pad + l) * kHeadDim + d0) = vop;
    if constexpr (TI::kDma)
    {
        // the first text tiles also as V^T tiles in LDS byte order: dim d of
        // key j sits at element vt_offset(d, j / 8) + j % 8 of its tile, the
        // layout the value waves' transpose writes, so the attention kernel
        // copies these tiles into LDS unchanged
        if (l < kDirectTextTiles * kBlockN)
        {
            uint16_t* tile = p.txt_vlds + (static_cast<long long>(head) * kDirectTextTiles + l / kBlockN) *
                                              (kBlockN * kHeadDim);
            const int j = l % kBlockN;
            const uint32_t w[4] = {vop.x, vop.y, vop.z, vop.w};
#pragma unroll
            for (int e = 0; e < 8; e++)
                tile[vt_offset(d0 + e, j >> 3) + (j & 7)] = static_cast<uint16_t>(w[e >> 1] >> (16 * (e & 1)));
        }
    }
}

// ---------------------------------------------------------------- key/value tiles

struct Geometry
{
    int vlen;   // video keys / queries of the window
    int seq;    // vlen + text_len
    int ntb;    // text key tiles (processed first)
    int nkb;    // all key tiles
};

__device__ inline char* k_tile(char* smem, const AttnParams& p, int kb)
{
    return smem + p.lds.k + (kb % 3) * kTileBytes;
}

__device__ inline char* vraw_tile(char* smem, const AttnParams& p, int kb)
{
    return smem + p.lds.vraw + (kb & 1) * kTileBytes;
}

__device__ inline char* vt_tile(char* smem, const AttnParams& p, int kb)
{
    return smem + p.lds.vt + (kb & 1) * kTileBytes;
}

// 16-bit inputs: tile kb moves from global memory straight into LDS, one 1 KB
// wave-instruction at a time (the lane order fixes where each 16-byte chunk
// lands).  Waves 0-7 fetch the key tile, wave w rows 8w..8w+7, one half (64
// dims) per instruction, lane l taking row 8w + l / 8; waves 8-11 fetch the
// value tile, wave 8+v rows 16v..16v+15, one 32-dim quarter per instruction,
// lane l taking row 16v + l / 4 (text value rows come prepared from the
// workspace in the same layout).  Each wave prepares exactly the chunks it
// fetched, so no barrier separates the fetch from the prologue.  Rows past the end of a ragged tile repeat the last
// valid row: their scores are masked and their values multiply p = 0.
// Fetches per lane and tile: 2 (key waves), 4 (value waves).
template <typename TI>
__device__ inline void dma_tile(const AttnParams& p, const Geometry& gm, const Staged& s, char* smem, int head,
                                int kb, int wave, int lane)
{
    const int sl = lane & 7;
    if (wave < 8)
    {
        char* kt = k_tile(smem, p, kb);
        const int r = 8 * wave + (lane >> 3);
        const int ksl = sl ^ ((r >> 1) & 7); // chunk (within the half) the swizzled slot holds
        const uint16_t* krow;
        if (kb < gm.ntb)
            krow = p.txt_k + (static_cast<long long>(head) * p.text_len + min(kb * kBlockN + r, p.text_len - 1)) *
                                 kHeadDim;
        else
            krow = static_cast<const uint16_t*>(p.vid_qkv) +
                   static_cast<long long>(s.rows[min((kb - gm.ntb) * kBlockN + r, gm.vlen - 1)].x) * p.row_stride +
                   p.dim + head * kHeadDim;
#pragma unroll
        for (int i = 0; i < 2; i++)
            dma16(krow + 8 * (8 * i + ksl), kt + i * 8192 + 8 * wave * 128);
        return;
    }
    const int v = wave - 8;
    if (kb < gm.ntb && kb < kDirectTextTiles)
    {
        // the first text tiles come as finished V^T tiles: a straight copy
        // into the V^T slot (free: these tiles are fetched before the loop)
        const uint16_t* src = p.txt_vlds + (static_cast<long long>(head) * kDirectTextTiles + kb) *
                                               (kBlockN * kHeadDim);
        char* dst = vt_tile(smem, p, kb);
#pragma unroll
        for (int q = 0; q < 4; q++)
            dma16(src + (q * 4096 + 1024 * v) / 2 + 8 * lane, dst + q * 4096 + 1024 * v);
        return;
    }
    // value rows: instruction q writes LDS bytes q * 4096 + 1024 v + 16 lane,
    // i.e. chunk 4q + (lane & 3) of row 16v + lane / 4 (vq_offset)
    char* vt = vraw_tile(smem, p, kb);
    const int r = 16 * v + (lane >> 2);
    const uint16_t* vrow;
    if (kb < gm.ntb)
        vrow = p.txt_vt + (static_cast<long long>(head) * p.text_pad + kb * kBlockN + r) * kHeadDim;
    else
        vrow = static_cast<const uint16_t*>(p.vid_qkv) +
               static_cast<long long>(s.rows[min((kb - gm.ntb) * kBlockN + r, gm.vlen - 1)].x) * p.row_stride +
               2LL * p.dim + head * kHeadDim;
#pragma unroll
    for (int q = 0; q < 4; q++)
        dma16(vrow + 8 * (4 * q + (lane & 3)), vt + q * 4096 + 1024 * v);
}

// Waits until this lane's fetches of the older of the (at most) two tiles in
// flight have landed: key waves issue 2 fetches per tile, value waves 4.
__device__ inline void wait_tile_fetch(int wave, bool newer_in_flight)
{
    if (!newer_in_flight)
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    else if (wave < 8)
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt2);
    else
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt4);
}

// Eight keys of one dim from a fetched value tile with two transposing LDS
// reads (ds_read_b64_tr_b16).  Within each 16-lane group such a read hands
// lane i element i % 4 of the 8-byte pieces addressed by group lanes
// i / 4 + 4 j, j = 0..3; when group lane k addresses key row r0 + k / 4 at
// dims d0 + 4 (k % 4), lane i receives keys r0 .. r0 + 3 of dim d0 + i.  The
// second read is four rows (256 bytes) further.
__device__ inline uint4 v_keys8_tr(const char* vr, int off)
{
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vr + off));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vr + off + 256));
    const uint2 a = __builtin_bit_cast(uint2, lo);
    const uint2 b = __builtin_bit_cast(uint2, hi);
    return make_uint4(a.x, a.y, b.x, b.y);
}

// 16-bit inputs: the prologue of tile kb, run by the waves that fetched it
// (after their own fetches have landed), so no barrier separates the fetch
// from the prologue.  Video: waves 0-7 run the k prologue (RMSNorm * gamma,
// RoPE, bf16) in place.  Waves 8-11 write the V^T tile from the rows they
// fetched: wave 8+v's 16-lane groups read the 8-key columns of key groups 2v,
// 2v+1 (16 dims per group and read) with transposing reads, round fp16 values
// to bf16 (bf16 inputs and the prepared text rows are rounded already;
// rounding them again changes nothing) and store each column as one 16-byte
// chunk.
template <typename TI, int RM>
__device__ inline void prepare_tile(const AttnParams& p, const Geometry& gm, const Staged& s, char* smem, int kb,
                                    int wave, int lane)
{
    const int chunk = lane & 15;
    const int d0 = chunk * 8;
    if (wave < 8)
    {
        if (kb < gm.ntb)
            return;
        char* kt = k_tile(smem, p, kb);
        const int base = (kb - gm.ntb) * kBlockN;
        const int last = gm.vlen - 1;
        const KeyRope kr = staged_key_rope<RM>(p, smem, chunk);
#pragma unroll
        for (int i = 0; i < 2; i++)
        {
            const int r = 8 * wave + 4 * i + (lane >> 4);
            uint4* slot = reinterpret_cast<uint4*>(kt + k_slot_offset(r, chunk));
            uint4 raw[1] = {*slot};
            float x[8];
            raw8_to_float<TI>(raw, x);
            const uint32_t packed = static_cast<uint32_t>(s.rows[min(base + r, last)].y);
            *slot = key_chunk<RM, TI::kExact>(p, s, kr, x, d0, packed);
        }
        return;
    }
    if (kb < gm.ntb && kb < kDirectTextTiles)
        return; // copied in finished (dma_tile)
    const char* vr = vraw_tile(smem, p, kb);
    char* vt = vt_tile(smem, p, kb);
    const int q = lane >> 4;
    const int i = lane & 15;
#pragma unroll
    for (int it = 0; it < 4; it++)
    {
        // key groups 2v, 2v+1 (the rows this wave fetched) x 8 blocks of 16 dims
        const int blk = 4 * it + q;
        const int db = blk & 7;
        const int grp = 2 * (wave - 8) + (blk >> 3);
        uint4 u = v_keys8_tr(vr, vq_offset(8 * grp + (i >> 2), 2 * db + ((i & 3) >> 1)) + 8 * (i & 1));
        if constexpr (TI::kPTerms == 1)
        {
            float x[8];
            uint4 raw[1] = {u};
            raw8_to_float<TI>(raw, x);
            u = v_operand8<TI>(x);
        }
        *reinterpret_cast<uint4*>(vt + 2 * vt_offset(16 * db + i, grp)) = u;
    }
}

// fp32 inputs: waves 0-7 load tile kb into registers and prepare it into the
// same LDS tiles (no raw copy in LDS).
template <int RM>
__device__ inline void load_prepare_tile_f32(const AttnParams& p, const Geometry& gm, const Staged& s, char* smem,
                                             int head, int kb, int tid)
{
    char* kt = k_tile(smem, p, kb);
    char* vt = vt_tile(smem, p, kb);
    const int r = tid >> 4;
    const int chunk = tid & 15;
    const int d0 = chunk * 8;
    const KeyRope kr = staged_key_rope<RM>(p, smem, chunk);
    if (kb < gm.ntb)
    {
        const int base = kb * kBlockN;
        const long long kbase = static_cast<long long>(head) * p.text_len;
#pragma unroll
        for (int i = 0; i < 2; i++)
        {
            const int rr = r + 32 * i;
            const int l = min(base + rr, p.text_len - 1);
            *reinterpret_cast<uint4*>(kt + k_slot_offset(rr, chunk)) =
                *reinterpret_cast<const uint4*>(p.txt_k + (kbase + l) * kHeadDim + d0);
        }
        // the prepared text rows (bf16 bits), transposed: keys 2r, 2r+1
        const uint16_t* vs = p.txt_vt + (static_cast<long long>(head) * p.text_pad + base + 2 * r) * kHeadDim + d0;
        uint16_t* t = reinterpret_cast<uint16_t*>(vt);
        const int key = 2 * r;
#pragma unroll
        for (int e = 0; e < 8; e++)
            *reinterpret_cast<uint32_t*>(&t[vt_offset(d0 + e, key >> 3) + (key & 7)]) =
                static_cast<uint32_t>(vs[e]) | (static_cast<uint32_t>(vs[e + kHeadDim]) << 16);
        return;
    }
    const int base = (kb - gm.ntb) * kBlockN;
    const int last = gm.vlen - 1;
    const long long k_col = static_cast<long long>(p.dim) + static_cast<long long>(head) * kHeadDim + d0;
    const long long v_col = k_col + p.dim;
#pragma unroll
    for (int i = 0; i < 2; i++)
    {
        const int rr = r + 32 * i;
        const int2 a = s.rows[min(base + rr, last)];
        float x[8];
        load8<F32>(p.vid_qkv, static_cast<long long>(a.x) * p.row_stride + k_col, x);
        *reinterpret_cast<uint4*>(kt + k_slot_offset(rr, chunk)) =
            key_chunk<RM, F32::kExact>(p, s, kr, x, d0, static_cast<uint32_t>(a.y));
    }
    float v0[8];
    float v1[8];
    load8<F32>(p.vid_qkv, static_cast<long long>(s.rows[min(base + 2 * r, last)].x) * p.row_stride + v_col, v0);
    load8<F32>(p.vid_qkv, static_cast<long long>(s.rows[min(base + 2 * r + 1, last)].x) * p.row_stride + v_col, v1);
    store_vt_pair<F32>(vt, r, d0, v0, v1);
}

// ---------------------------------------------------------------- attention step

// Per-lane byte offsets of the MFMA operand reads, fixed for the whole loop:
// kb4[j] = row key_perm(lr) of the key tile, chunk 2j + g (dims 16j + 8g),
// half 0; chunk 2c + g is kb4[c & 3] + (c >> 2) * 8192, subtile kt adds
// kt * 4096.  vb4[m] = row lr of the V^T tile, key group
// (g ^ f(lr)) ^ 2m with f(d) = (d ^ (d >> 3)) & 7; the read of rows
// dt * 32 + lr, key group 4 kt + 2 c2 + g is vb4[c2 + 2 (kt ^ (dt & 1))] +
// dt * 4096 (the swizzle of row dt * 32 + lr is f(lr) ^ 4 (dt & 1)).
struct ReadBases
{
    int k[4];
    int v[4];
};

__device__ inline ReadBases read_bases(int lane)
{
    const int lr = lane & 31;
    const int g = lane >> 5;
    ReadBases b;
    const int r = key_perm(lr);
    const int y = (r >> 1) & 7;
#pragma unroll
    for (int j = 0; j < 4; j++)
        b.k[j] = r * 128 + (((2 * j + g) ^ y) << 4);
    const int u = g ^ ((lr ^ (lr >> 3)) & 7);
#pragma unroll
    for (int m = 0; m < 4; m++)
        b.v[m] = lr * 128 + ((u ^ (2 * m)) << 4);
    return b;
}

// One 32-key subtile of the online softmax for the wave's 32 query rows.  NT
// is the input type's kPTerms (how P enters the P*V product).
template <int KT, int NT>
__device__ inline void attend_subtile(const AttnParams& p, const char* kt, const char* vt, const ReadBases& rb,
                                      const bf16x8 qf[8], int nvalid, int g, f32x16 o[4], float& m_run,
                                      float& l_run)
{
    // ---- S^T = K Q^T for 32 keys; K fragments are read four at a time ahead
    // of the MFMAs that consume them
    f32x16 s = f32x16{};
#pragma unroll
    for (int h = 0; h < 2; h++)
    {
        bf16x8 a[4];
#pragma unroll
        for (int c = 0; c < 4; c++)
            a[c] = *reinterpret_cast<const bf16x8*>(kt + rb.k[c] + h * 8192 + KT * 4096);
#pragma unroll
        for (int c = 0; c < 4; c++)
            s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[c], qf[4 * h + c], s, 0, 0, 0);
    }
    // ---- mask a ragged subtile.  Register r of lane group g holds S^T row
    // 8(r/4) + 4g + r%4, i.e. key 16((r/4)/2) + 8g + 4((r/4)%2) + r%4; the
    // per-register part is a constant, so only one limit is live.
    if (nvalid < 32)
    {
        const int lim = nvalid - 8 * g;
#pragma unroll
        for (int r = 0; r < 16; r++)
        {
            const int kconst = 16 * ((r >> 2) >> 1) + 4 * ((r >> 2) & 1) + (r & 3);
            if (kconst >= lim)
                s[r] = -INFINITY;
        }
    }
    float smax = s[0];
#pragma unroll
    for (int r = 1; r < 16; r++)
        smax = fmaxf(smax, s[r]);
    const float m_new = fmaxf(m_run, partner_max(smax));
    // lazy rescale: keep the old reference max unless it is exceeded by more
    // than 2^8 (p stays <= 256, exact in fp16 and fp32); O / l does not depend
    // on the reference max
    const bool grow = (m_new - m_run) * p.score_log2 > kRescaleLog2;
    if (__any(grow))
    {
        if (grow)
        {
            const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * p.score_log2);
            l_run *= alpha;
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
                o[dt] *= alpha;
            m_run = m_new;
        }
    }
    const float bias = m_run * p.score_log2;
    if constexpr (NT > 1)
    {
        // ---- P as NT bf16 terms against exact bf16 V.  Each term is the
        // bf16 rounding of what the terms before it left over (the remainders
        // are exact in fp32: a value and its rounding are within a factor of
        // two), so the terms sum to p within 2^-18 (NT = 2) or 2^-27 (NT = 3)
        // of p.  The row sum adds the same terms.
#pragma unroll
        for (int c2 = 0; c2 < 2; c2++)
        {
            bf16x8 va[4];
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
                va[dt] = *reinterpret_cast<const bf16x8*>(vt + rb.v[c2 + 2 * (KT ^ (dt & 1))] + dt * 4096);
            uint32_t bw[NT][4];
#pragma unroll
            for (int e = 0; e < 8; e += 2)
            {
                float r0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[8 * c2 + e], p.score_log2, -bias));
                float r1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[8 * c2 + e + 1], p.score_log2, -bias));
#pragma unroll
                for (int t = 0; t < NT; t++)
                {
                    const uint32_t u = bf16_pair_bits(r0, r1);
                    const float h0 = __builtin_bit_cast(float, u << 16);
                    const float h1 = __builtin_bit_cast(float, u & 0xffff0000u);
                    bw[t][e >> 1] = u;
                    l_run += h0;
                    l_run += h1;
                    r0 -= h0;
                    r1 -= h1;
                }
            }
#pragma unroll
            for (int t = 0; t < NT; t++)
            {
                const bf16x8 b = __builtin_bit_cast(bf16x8, make_uint4(bw[t][0], bw[t][1], bw[t][2], bw[t][3]));
#pragma unroll
                for (int dt = 0; dt < 4; dt++)
                    o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[dt], b, o[dt], 0, 0, 0);
            }
        }
        return;
    }
    // ---- P (fp16), row sums from the same fp16 values, O^T += V^T P^T
#pragma unroll
    for (int c2 = 0; c2 < 2; c2++)
    {
        f16x8 va[4];
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
            va[dt] = *reinterpret_cast<const f16x8*>(vt + rb.v[c2 + 2 * (KT ^ (dt & 1))] + dt * 4096);
        f16x8 b;
#pragma unroll
        for (int e = 0; e < 8; e += 2)
        {
            const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[8 * c2 + e], p.score_log2, -bias));
            const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[8 * c2 + e + 1], p.score_log2, -bias));
            f16x2 h;
            h[0] = static_cast<_Float16>(p0); // round to nearest even (v_cvt_pk_f16_f32)
            h[1] = static_cast<_Float16>(p1);
            b[e] = h[0];
            b[e + 1] = h[1];
            l_run = __builtin_amdgcn_fdot2(h, f16x2{static_cast<_Float16>(1.f), static_cast<_Float16>(1.f)}, l_run,
                                           false);
        }
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
            o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[dt], b, o[dt], 0, 0, 0);
    }
}

// Query rows of one workgroup: a window of S rows is split into
// ceil(S / 384) blocks of equal size (rounded up to 32 rows).
struct QueryBlock
{
    int q0;
    int q1;
};

__device__ inline QueryBlock query_block(int seq, int qb)
{
    const int nqb = (seq + kRowsPerGroup - 1) / kRowsPerGroup;
    const int per = ((seq + nqb - 1) / nqb + 31) / 32 * 32;
    QueryBlock b;
    b.q0 = qb * per;
    b.q1 = min(b.q0 + per, seq);
    return b;
}

// Four outputs already rounded to bf16 (two packed pairs) in the output type.
__device__ inline void store_rounded(int out_dtype, void* base, long long offset, uint32_t lo, uint32_t hi)
{
    const float v[4] = {__builtin_bit_cast(float, lo << 16), __builtin_bit_cast(float, lo & 0xffff0000u),
                        __builtin_bit_cast(float, hi << 16), __builtin_bit_cast(float, hi & 0xffff0000u)};
    if (out_dtype == SV2_BF16)
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(base) + offset) = make_uint2(lo, hi);
    else if (out_dtype == SV2_F16)
        store4<F16>(base, offset, v);
    else
        store4<F32>(base, offset, v);
}

// Epilogue of one wave: O / l, rounded to bf16 where the reference rounds each
// output element (seedvr2_dit_block.cpp:1074; v_cvt_pk_bf16_f32 rounds to
// nearest even), video rows scattered to their grid rows, text rows to this
// window's bf16 partials.
__device__ inline void write_outputs(const AttnParams& p, const Staged& s, const WindowBox& box, int wi, int head,
                                     int qrow, int g, const f32x16 o[4], float inv_l)
{
    const long long q_col = static_cast<long long>(head) * kHeadDim;
    const bool text = qrow >= box.vlen;
    long long out_off;
    if (!text)
        out_off = static_cast<long long>(s.rows[qrow].x) * p.dim + q_col;
    else
        out_off = (static_cast<long long>(wi) * p.text_len + (qrow - box.vlen)) * p.dim + q_col;
    const long long pre_row =
        (static_cast<long long>(box.vprefix) + static_cast<long long>(wi) * p.text_len + qrow) * p.dim + q_col;
    void* dst = text ? static_cast<void*>(p.partial) : p.vid_out;
    const int dt_out = text ? SV2_BF16 : p.out_dtype;
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int rq = 0; rq < 4; rq++)
        {
            const int d = dt * 32 + 8 * rq + 4 * g;
            float pre[4];
#pragma unroll
            for (int e = 0; e < 4; e++)
                pre[e] = o[dt][4 * rq + e] * inv_l;
            if (p.dbg_pre)
                store4<F32>(p.dbg_pre, pre_row + d, pre);
            store_rounded(dt_out, dst, out_off + d, bf16_pair_bits(pre[0], pre[1]), bf16_pair_bits(pre[2], pre[3]));
        }
}

// Bytes per row of the epilogue staging area: 256 B of outputs + 16 B, so the
// rows of one store wave start on different LDS banks.
constexpr int kEpiStride = 272;

// Epilogue of one wave for 16-bit outputs: the wave's 32 x 128 tile of
// rounded outputs (as write_outputs rounds them) is staged in LDS, then every
// 256-byte output row segment is stored by 16 lanes with one 16-byte store
// each, instead of sixteen 8-byte pieces from two lanes.  Every lane of the
// wave takes part (rows at or past q_end are staged but not stored).
__device__ inline void write_outputs_lds(const AttnParams& p, const Staged& s, const WindowBox& box, int wi,
                                         int head, int q_wave0, int q_end, int lane, const f32x16 o[4],
                                         float inv_l, char* stage)
{
    const int lr = lane & 31;
    const int g = lane >> 5;
    const int qrow = q_wave0 + lr;
    const bool text = qrow >= box.vlen;
    const bool f16_out = !text && p.out_dtype == SV2_F16;
    const long long pre_row =
        (static_cast<long long>(box.vprefix) + static_cast<long long>(wi) * p.text_len + qrow) * p.dim +
        static_cast<long long>(head) * kHeadDim;
    char* my_row = stage + lr * kEpiStride;
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int rq = 0; rq < 4; rq++)
        {
            const int d = dt * 32 + 8 * rq + 4 * g;
            float pre[4];
#pragma unroll
            for (int e = 0; e < 4; e++)
                pre[e] = o[dt][4 * rq + e] * inv_l;
            if (p.dbg_pre && qrow < q_end)
                store4<F32>(p.dbg_pre, pre_row + d, pre);
            uint32_t lo = bf16_pair_bits(pre[0], pre[1]);
            uint32_t hi = bf16_pair_bits(pre[2], pre[3]);
            if (f16_out)
            {
                // the bf16 values are exact in fp16 within its range
                f16x2 fa, fb;
                fa[0] = static_cast<_Float16>(__builtin_bit_cast(float, lo << 16));
                fa[1] = static_cast<_Float16>(__builtin_bit_cast(float, lo & 0xffff0000u));
                fb[0] = static_cast<_Float16>(__builtin_bit_cast(float, hi << 16));
                fb[1] = static_cast<_Float16>(__builtin_bit_cast(float, hi & 0xffff0000u));
                lo = __builtin_bit_cast(uint32_t, fa);
                hi = __builtin_bit_cast(uint32_t, fb);
            }
            *reinterpret_cast<uint2*>(my_row + 2 * d) = make_uint2(lo, hi);
        }
    // the rows are read back by other lanes of this wave: LDS operations of a
    // wave complete in order, and the wait makes the compiler keep it so
    __builtin_amdgcn_s_waitcnt(0xC07F); // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
    const int chunk = lane & 15;
    const long long col = static_cast<long long>(head) * kHeadDim + chunk * 8;
#pragma unroll
    for (int it = 0; it < 8; it++)
    {
        const int rl = it * 4 + (lane >> 4);
        const int q = q_wave0 + rl;
        if (q < q_end)
        {
            const uint4 v = *reinterpret_cast<const uint4*>(stage + rl * kEpiStride + chunk * 16);
            uint16_t* dst;
            if (q < box.vlen)
                dst = static_cast<uint16_t*>(p.vid_out) + static_cast<long long>(s.rows[q].x) * p.dim + col;
            else
                dst = p.partial + (static_cast<long long>(wi) * p.text_len + (q - box.vlen)) * p.dim + col;
            *reinterpret_cast<uint4*>(dst) = v;
        }
    }
}

template <typename TI, int RM>
__global__ __launch_bounds__(kThreads) void window_attention_kernel(AttnParams p)
{
    extern __shared__ __attribute__((aligned(16))) char smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // wave-uniform: wave-derived offsets live in scalar registers
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool loader = tid < kLoaderThreads;

    // XCD-aware decode: workgroup ids go round-robin over the 8 XCDs; the query
    // blocks of one (window, head) pair are consecutive ids of one XCD and
    // share its L2 for the key/value rows they both read.
    const int id = blockIdx.x;
    const int xcd = id & 7;
    const int slot = id >> 3;
    const int grp = slot / p.nqb;
    const int pair = grp * 8 + xcd;
    const int qb = slot - grp * p.nqb;
    if (pair >= p.npairs)
        return;
    // largest windows first, so the last workgroups of the launch are short
    const int wslot = pair / p.heads;
    const int head = pair - wslot * p.heads;
    const int wi = p.ordered ? static_cast<int>(p.order[wslot]) : wslot;
    const WindowBox box = window_box(p.plan, wi);
    Geometry gm;
    gm.vlen = box.vlen;
    gm.seq = box.vlen + p.text_len;
    gm.ntb = (p.text_len + kBlockN - 1) / kBlockN;
    gm.nkb = gm.ntb + (box.vlen + kBlockN - 1) / kBlockN;
    const QueryBlock qbk = query_block(gm.seq, qb);
    if (qbk.q0 >= gm.seq)
        return;

    stage_window<RM>(p, box, smem, tid, kThreads);
    stage_key_rope<RM>(p, box, smem, tid);
    __syncthreads();
    const Staged s = staged(p, smem);

    const int lr = lane & 31;
    const int g = lane >> 5;
    const bool wave_active = qbk.q0 + wave * 32 < qbk.q1;
    const int qrow = qbk.q0 + wave * 32 + lr;
    const int qrow_c = min(qrow, gm.seq - 1);
    const ReadBases rdb = read_bases(lane);

    // the fetches of tiles 0 and 1 and the query loads are in flight together
    const int last_tile = gm.nkb - 1;
    if constexpr (TI::kDma)
    {
        dma_tile<TI>(p, gm, s, smem, head, 0, wave, lane);
        if (last_tile >= 1)
            dma_tile<TI>(p, gm, s, smem, head, 1, wave, lane);
    }
    QueryRaw<TI> qraw;
    query_load<TI>(p, s, box, head, qrow_c, g, qraw);
    bf16x8 qf[8];
    query_finish<TI, RM>(p, s, box, qrow_c, g, qraw, qf);
    settle(qf);

    f32x16 o[4];
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
        o[dt] = f32x16{};
    float m_run = -INFINITY;
    float l_run = 0.f;

    if constexpr (TI::kDma)
    {
        // tile 0 has landed once at most tile 1's fetches are outstanding
        wait_tile_fetch(wave, last_tile >= 1);
        prepare_tile<TI, RM>(p, gm, s, smem, 0, wave, lane);
    }
    else if (loader)
    {
        load_prepare_tile_f32<RM>(p, gm, s, smem, head, 0, tid);
    }
    __syncthreads();

    auto valid_keys = [&](int kb) {
        return kb < gm.ntb ? p.text_len - kb * kBlockN : gm.vlen - (kb - gm.ntb) * kBlockN;
    };
    for (int kb = 0; kb < gm.nkb; kb++)
    {
        // fetch tile kb+2 into the buffers tile kb-1 used (all reads of them
        // ended before the last barrier), attend tile kb, prepare tile kb+1
        // (fetched one step earlier)
        const int ln = opaque(lane);
        const bool fetch = kb + 2 <= last_tile;
        const bool value_wave = wave >= 8;
        if constexpr (TI::kDma)
        {
            // the value waves prepare tile kb+1 before they attend, while the
            // key waves attend first: one group's VALU work meets the other's
            // MFMAs.  Tile kb+1 has landed once nothing is outstanding (its
            // fetches are the value waves' only ones in flight here).
            if (value_wave && kb + 1 < gm.nkb)
            {
                __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
                prepare_tile<TI, RM>(p, gm, s, smem, kb + 1, wave, ln);
            }
            if (fetch)
                dma_tile<TI>(p, gm, s, smem, head, kb + 2, wave, ln);
        }
        if (wave_active)
        {
            const char* kt = k_tile(smem, p, kb);
            const char* vt = vt_tile(smem, p, kb);
            const int nv = valid_keys(kb);
            attend_subtile<0, TI::kPTerms>(p, kt, vt, rdb, qf, nv, g, o, m_run, l_run);
            if (nv > 32)
                attend_subtile<1, TI::kPTerms>(p, kt, vt, rdb, qf, nv - 32, g, o, m_run, l_run);
        }
        if (kb + 1 < gm.nkb)
        {
            if constexpr (TI::kDma)
            {
                // key waves: tile kb+1 has landed once only tile kb+2's
                // fetches (if any) are outstanding
                if (!value_wave)
                {
                    wait_tile_fetch(wave, fetch);
                    prepare_tile<TI, RM>(p, gm, s, smem, kb + 1, wave, ln);
                }
            }
            else if (loader)
            {
                load_prepare_tile_f32<RM>(p, gm, s, smem, head, kb + 1, opaque(tid));
            }
        }
        __syncthreads();
    }

    if (!wave_active)
        return;
    const float l_tot = partner_sum(l_run);
    if constexpr (TI::kDma)
    {
        // 16-bit outputs leave through LDS (the tile buffers are free: every
        // wave passed the loop's last barrier and every fetch has landed)
        if (p.out_dtype != SV2_F32)
        {
            write_outputs_lds(p, s, box, wi, head, qbk.q0 + wave * 32, qbk.q1, lane, o, 1.f / l_tot,
                              smem + p.lds.k + wave * 32 * kEpiStride);
            return;
        }
    }
    if (qrow >= qbk.q1)
        return;
    write_outputs(p, s, box, wi, head, qrow, g, o, 1.f / l_tot);
}

// Text outputs: sum of the per-window bf16 partials in window order, then a
// multiply by 1/nW (seedvr2_dit_block.cpp:1074-1075, :1081-1088).  Each thread
// owns two elements; the loads of 16 windows are issued before their adds so
// the sequential sum does not serialise on memory latency.
template <typename TO>
__global__ __launch_bounds__(256) void text_window_reduce_kernel(const uint32_t* partial, void* out, int nwin,
                                                                 long long pairs, float inv_nw)
{
    const long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= pairs)
        return;
    float a0 = 0.f;
    float a1 = 0.f;
    int w = 0;
    for (; w + 16 <= nwin; w += 16)
    {
        uint32_t v[16];
#pragma unroll
        for (int u = 0; u < 16; u++)
            v[u] = partial[static_cast<long long>(w + u) * pairs + i];
#pragma unroll
        for (int u = 0; u < 16; u++)
        {
            a0 += __builtin_bit_cast(float, v[u] << 16);
            a1 += __builtin_bit_cast(float, v[u] & 0xffff0000u);
        }
    }
    for (; w < nwin; w++)
    {
        const uint32_t v = partial[static_cast<long long>(w) * pairs + i];
        a0 += __builtin_bit_cast(float, v << 16);
        a1 += __builtin_bit_cast(float, v & 0xffff0000u);
    }
    store2<TO>(out, 2 * i, a0 * inv_nw, a1 * inv_nw);
}

// Outputs of qk_prologue_kernel (each may be NULL): q, k, v after the
// prologue in window-sequence order [sum S][D]; video q, k after the norm and
// before RoPE in grid row order [T*H*W][D].
struct PrologueOut
{
    float* q;
    float* k;
    float* v;
    float* nq_vid;
    float* nk_vid;
};

// Debug / test: q, k, v after the prologue, fp32, window-sequence order, from
// the device functions the attention kernel runs: queries through the MFMA
// operand-layout path, keys 16 lanes per row, values as the P*V operands;
// text rows from the prepared workspace.  One workgroup (4 waves) per
// (window, head, 32 rows).
template <typename TI, int RM>
__global__ __launch_bounds__(256) void qk_prologue_kernel(AttnParams p, int nrb, PrologueOut out)
{
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int blk = blockIdx.x;
    const int rb = blk % nrb;
    const int rest = blk / nrb;
    const int head = rest % p.heads;
    const int wi = rest / p.heads;
    const WindowBox box = window_box(p.plan, wi);
    const int seq = box.vlen + p.text_len;
    if (rb * 32 >= seq)
        return;
    const int tid = threadIdx.x;
    stage_window<RM>(p, box, smem, tid, 256);
    __syncthreads();
    const Staged s = staged(p, smem);
    const long long q_col = static_cast<long long>(head) * kHeadDim;
    const long long seq_base = static_cast<long long>(box.vprefix) + static_cast<long long>(wi) * p.text_len;

    if (tid < 64)
    {
        const int lr = tid & 31;
        const int g = tid >> 5;
        const int j = rb * 32 + lr;
        QueryRaw<TI> raw;
        query_load<TI>(p, s, box, head, min(j, seq - 1), g, raw);
        bf16x8 qf[8];
        float* nq = (out.nq_vid && j < box.vlen)
                        ? out.nq_vid + static_cast<long long>(s.rows[j].x) * p.dim + q_col + 8 * g
                        : nullptr;
        query_finish<TI, RM>(p, s, box, min(j, seq - 1), g, raw, qf, nq);
        if (j < seq && out.q)
        {
#pragma unroll
            for (int c = 0; c < 8; c++)
#pragma unroll
                for (int e = 0; e < 8; e++)
                    out.q[(seq_base + j) * p.dim + q_col + 16 * c + 8 * g + e] = static_cast<float>(qf[c][e]);
        }
    }
    const int d0 = (tid & 15) * 8;
    const KeyRope kr = key_rope<RM>(rope_base(box), d0);
    for (int pass = 0; pass < 2; pass++)
    {
        const int j = rb * 32 + pass * 16 + (tid >> 4);
        const bool valid = j < seq;
        const int jc = min(j, seq - 1);
        const long long o = (seq_base + j) * p.dim + q_col + d0;
        if (jc < box.vlen)
        {
            const int2 vr = s.rows[jc];
            float k[8];
            float v[8];
            load8<TI>(p.vid_qkv, static_cast<long long>(vr.x) * p.row_stride + q_col + p.dim + d0, k);
            load8<TI>(p.vid_qkv, static_cast<long long>(vr.x) * p.row_stride + q_col + 2LL * p.dim + d0, v);
            float* nk = (out.nk_vid && valid) ? out.nk_vid + static_cast<long long>(vr.x) * p.dim + q_col + d0 : nullptr;
            const bf16x8 kb =
                __builtin_bit_cast(bf16x8, key_chunk<RM, TI::kExact>(p, s, kr, k, d0, static_cast<uint32_t>(vr.y), nk));
            if (valid && out.k)
            {
#pragma unroll
                for (int e = 0; e < 8; e++)
                    out.k[o + e] = static_cast<float>(kb[e]);
            }
            if (valid && out.v)
            {
#pragma unroll
                for (int e = 0; e < 8; e += 2)
                {
                    const uint32_t h = v_pair_operand<TI>(v[e], v[e + 1]);
                    out.v[o + e] = v_operand_value<TI>(static_cast<uint16_t>(h & 0xffffu));
                    out.v[o + e + 1] = v_operand_value<TI>(static_cast<uint16_t>(h >> 16));
                }
            }
        }
        else if (valid)
        {
            const int l = jc - box.vlen;
            const uint16_t* ks = p.txt_k + (static_cast<long long>(head) * p.text_len + l) * kHeadDim + d0;
            const uint16_t* vs = p.txt_vt + (static_cast<long long>(head) * p.text_pad + l) * kHeadDim + d0;
#pragma unroll
            for (int e = 0; e < 8; e++)
            {
                if (out.k)
                    out.k[o + e] = __builtin_bit_cast(float, static_cast<uint32_t>(ks[e]) << 16);
                if (out.v)
                    out.v[o + e] = v_operand_value<TI>(vs[e]);
            }
        }
    }
}

// ---------------------------------------------------------------- exact mode

constexpr int kExactWaves = 4; // query rows per exact_attention_kernel workgroup, one per wave

// The reference CPU layer's attention core step for step
// (seedvr2_dit_block.cpp:1045-1079), for the fp32 parity mode.  Inputs are
// q, k, v after the prologue in window-sequence order ([sum_w S_w][D] fp32
// holding bf16 values, written by qk_prologue_kernel).  One wave per query
// row; per query, in the reference's order and rounding:
//   scores    s_j = float(sum_d double(q_d) * k_jd) * scale, the double sum in
//             increasing d (lanes split the keys; each lane sums its own);
//   maximum   m = max_j s_j;
//   exp       e_j = exp(s_j - m), correctly rounded (formed in double and
//             rounded once to float);
//   sum       den = sum_j e_j in float, in increasing j (sequence order:
//             video keys, then text keys) by one lane;
//   weights   w_j = e_j / den, correctly rounded (formed in double);
//   outputs   out_d = bf16(float(sum_j double(w_j) * v_jd)), the double sum in
//             increasing j (lanes split the dims).
// The products of two floats are exact in double, so the double sums round
// exactly as the reference's.  Video outputs go to their grid rows, text
// outputs to the window's bf16 partials.  LDS: q [4][128], scores [4][sstride]
// (sstride: the longest window sequence rounded up to a multiple of 4, so
// every wave's scores start 16-byte aligned).
__global__ __launch_bounds__(256) void exact_attention_kernel(AttnParams p, const float* __restrict__ q,
                                                              const float* __restrict__ k,
                                                              const float* __restrict__ v, int nqg, int sstride,
                                                              float scale)
{
    extern __shared__ __attribute__((aligned(16))) float xsm[];
    const int blk = blockIdx.x;
    const int qg = blk % nqg;
    const int rest = blk / nqg;
    const int head = rest % p.heads;
    const int wi = rest / p.heads;
    const WindowBox box = window_box(p.plan, wi);
    const int seq = box.vlen + p.text_len;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int query = qg * kExactWaves + wave;
    if (query >= seq)
        return; // wave-uniform; the kernel has no workgroup barrier
    float* qs = xsm + wave * kHeadDim;
    float* sc = xsm + kExactWaves * kHeadDim + wave * sstride;
    const long long seq_base = static_cast<long long>(box.vprefix) + static_cast<long long>(wi) * p.text_len;
    const long long hc = static_cast<long long>(head) * kHeadDim;
    const float* qrow = q + (seq_base + query) * p.dim + hc;
    qs[lane] = qrow[lane];
    qs[lane + 64] = qrow[lane + 64];
    __builtin_amdgcn_s_waitcnt(0xC07F); // lgkmcnt(0): the row is read back by every lane of this wave
    __builtin_amdgcn_wave_barrier();

    float mloc = -INFINITY;
    for (int j = lane; j < seq; j += 64)
    {
        const float* krow = k + (seq_base + j) * p.dim + hc;
        double dot = 0.0;
        for (int d = 0; d < kHeadDim; d += 4)
        {
            const float4 qa = *reinterpret_cast<const float4*>(qs + d);
            const float4 ka = *reinterpret_cast<const float4*>(krow + d);
            dot = __builtin_fma(static_cast<double>(qa.x), static_cast<double>(ka.x), dot);
            dot = __builtin_fma(static_cast<double>(qa.y), static_cast<double>(ka.y), dot);
            dot = __builtin_fma(static_cast<double>(qa.z), static_cast<double>(ka.z), dot);
            dot = __builtin_fma(static_cast<double>(qa.w), static_cast<double>(ka.w), dot);
        }
        const float sj = static_cast<float>(dot) * scale;
        sc[j] = sj;
        mloc = fmaxf(mloc, sj);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
        mloc = fmaxf(mloc, __shfl_xor(mloc, o));
    for (int j = lane; j < seq; j += 64)
        sc[j] = static_cast<float>(exp(static_cast<double>(sc[j] - mloc)));
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_wave_barrier();
    float den = 0.f;
    if (lane == 0)
    {
        int j = 0;
        for (; j + 4 <= seq; j += 4)
        {
            const float4 e4 = *reinterpret_cast<const float4*>(sc + j);
            den += e4.x;
            den += e4.y;
            den += e4.z;
            den += e4.w;
        }
        for (; j < seq; j++)
            den += sc[j];
    }
    den = __shfl(den, 0);
    __builtin_amdgcn_wave_barrier();
    const double dden = static_cast<double>(den);
    for (int j = lane; j < seq; j += 64)
        sc[j] = static_cast<float>(static_cast<double>(sc[j]) / dden);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_wave_barrier();

    const bool text = query >= box.vlen;
    long long out_off;
    if (!text)
    {
        int lt, ly, lx;
        out_off = static_cast<long long>(window_video_row(p.plan, box, query, &lt, &ly, &lx)) * p.dim + hc;
    }
    else
    {
        out_off = (static_cast<long long>(wi) * p.text_len + (query - box.vlen)) * p.dim + hc;
    }
    const float* vcol = v + seq_base * p.dim + hc;
#pragma unroll
    for (int h = 0; h < 2; h++)
    {
        const int d = lane + 64 * h;
        double sum = 0.0;
        for (int j = 0; j < seq; j++)
            sum = __builtin_fma(static_cast<double>(sc[j]), static_cast<double>(vcol[static_cast<long long>(j) * p.dim + d]),
                                sum);
        const float pre = static_cast<float>(sum);
        const float rounded = bf16_round(pre);
        if (p.dbg_pre)
            p.dbg_pre[(seq_base + query) * p.dim + hc + d] = pre;
        const uint32_t bits = __builtin_bit_cast(uint32_t, rounded);
        if (text)
            p.partial[out_off + d] = static_cast<uint16_t>(bits >> 16);
        else if (p.out_dtype == SV2_F32)
            static_cast<float*>(p.vid_out)[out_off + d] = rounded;
        else if (p.out_dtype == SV2_F16)
            static_cast<_Float16*>(p.vid_out)[out_off + d] = static_cast<_Float16>(rounded);
        else
            static_cast<uint16_t*>(p.vid_out)[out_off + d] = static_cast<uint16_t>(bits >> 16);
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

// ---------------------------------------------------------------- host side

int dtype_ok(int t)
{
    return t == SV2_F32 || t == SV2_F16 || t == SV2_BF16;
}

struct Workspace
{
    int64_t partial;
    int64_t txt_q;
    int64_t txt_k;
    int64_t txt_vt;
    int64_t txt_vlds;
    int64_t seq_q; // exact mode: q, k, v after the prologue, window-sequence order, fp32
    int64_t seq_k;
    int64_t seq_v;
    int64_t total;
};

int64_t align256(int64_t v)
{
    return (v + 255) & ~int64_t(255);
}

Workspace workspace_layout(const AttnParams& p)
{
    Workspace w;
    int64_t off = 0;
    w.partial = off;
    off = align256(off + static_cast<int64_t>(p.plan.nwin) * p.text_len * p.dim * 2);
    w.txt_q = off;
    off = align256(off + static_cast<int64_t>(p.heads) * p.text_len * kHeadDim * 2);
    w.txt_k = off;
    off = align256(off + static_cast<int64_t>(p.heads) * p.text_len * kHeadDim * 2);
    w.txt_vt = off;
    off = align256(off + static_cast<int64_t>(p.heads) * kHeadDim * p.text_pad * 2);
    w.txt_vlds = off;
    off = align256(off + static_cast<int64_t>(p.heads) * kDirectTextTiles * kBlockN * kHeadDim * 2);
    if (p.text_len == 0)
        off = 0;
    w.seq_q = w.seq_k = w.seq_v = off;
    if (p.exact)
    {
        const int64_t bytes = align256(p.seq_rows * p.dim * 4);
        w.seq_q = off;
        w.seq_k = off + bytes;
        w.seq_v = off + 2 * bytes;
        off += 3 * bytes;
    }
    w.total = off;
    return w;
}

int align16(int v)
{
    return (v + 15) & ~15;
}

// LDS of the attention kernel for a plan: the staged row table of the largest
// window, then the key/value tiles, RoPE rows and gammas; after the tile loop
// the 16-bit epilogue stages its outputs over those last three (the row table
// is still read there).
LdsLayout lds_layout(int vmax, int rope_rows)
{
    LdsLayout l;
    int off = 0;
    l.rows = off;
    off = align16(off + vmax * 8);
    l.k = off;
    off += 3 * kTileBytes;
    l.vraw = off;
    off += 2 * kTileBytes;
    l.vt = off;
    off += 2 * kTileBytes;
    l.rope = off;
    off = align16(off + rope_rows * kRopePairSlots * 8);
    l.gamma = off;
    off += 2 * kHeadDim * 4;
    l.krope = off;
    off += 16 * 4 * 8;
    l.total = std::max(off, l.k + kWaves * 32 * kEpiStride);
    return l;
}

// LDS of the prologue debug kernel (no tiles).
LdsLayout lds_layout_staging(int vmax, int rope_rows)
{
    LdsLayout l;
    l.k = l.vraw = l.vt = 0;
    int off = 0;
    l.rows = off;
    off = align16(off + vmax * 8);
    l.rope = off;
    off = align16(off + rope_rows * kRopePairSlots * 8);
    l.gamma = off;
    off += 2 * kHeadDim * 4;
    l.krope = off;
    off += 16 * 4 * 8;
    l.total = off;
    return l;
}

// Validates the attention arguments and fills the kernel parameters.
int prepare(const sv2_attn_args* a, AttnParams* p, int* smax_out, int* vmax_out, int* rope_rows_out)
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
    if (misaligned(a->vid_qkv, 16) || (a->text_len > 0 && misaligned(a->txt_qkv, 16)) ||
        misaligned(a->vid_out, 16) || (a->text_len > 0 && misaligned(a->txt_out, 16)))
        return set_error(SV2_EINVAL, "attention: qkv and output pointers must be 16-byte aligned");
    if (a->qk_norm && (!a->gamma_q_vid || !a->gamma_k_vid))
        return set_error(SV2_EINVAL, "attention: qk_norm needs the video gamma vectors");
    if (a->exact && a->qkv_dtype != SV2_F32)
        return set_error(SV2_EINVAL, "attention: the exact mode takes fp32 qkv");
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
    int vmax = 0;
    int rope_rows = 0;
    for (int wi = 0; wi < p->plan.nwin; wi++)
    {
        const WindowBox b = window_box(p->plan, wi);
        if (b.vlen > kMaxVideoRows)
            return set_error(SV2_EUNSUPPORTED, "attention: a window holds more than 4096 video tokens");
        if (b.lt > 1023 || b.lh > 1023 || b.lw > 1023)
            return set_error(SV2_EUNSUPPORTED, "attention: window extent beyond 1023 on an axis");
        smax = std::max(smax, b.vlen + a->text_len);
        vmax = std::max(vmax, b.vlen);
        rope_rows = std::max(rope_rows, b.lt + b.lh + b.lw);
    }
    if (a->rope_mode == SV2_ROPE_NONE)
        rope_rows = 0;
    // dispatch order: windows by decreasing video length (stable), so that a
    // plan's ragged small windows form the tail of the launch
    p->ordered = p->plan.nwin <= kMaxOrdered ? 1 : 0;
    if (p->ordered)
    {
        int idx[kMaxOrdered];
        int len[kMaxOrdered];
        for (int wi = 0; wi < p->plan.nwin; wi++)
        {
            idx[wi] = wi;
            len[wi] = window_box(p->plan, wi).vlen;
        }
        std::stable_sort(idx, idx + p->plan.nwin, [&](int x, int y) { return len[x] > len[y]; });
        for (int wi = 0; wi < p->plan.nwin; wi++)
            p->order[wi] = static_cast<int16_t>(idx[wi]);
    }
    const int64_t qkv_elems = static_cast<int64_t>(a->rule.frames) * a->rule.height * a->rule.width * 3 * a->heads * kHeadDim;
    if (qkv_elems >= (int64_t(1) << 40))
        return set_error(SV2_EUNSUPPORTED, "attention: qkv tensor too large");
    p->lds = lds_layout(vmax, rope_rows);
    if (p->lds.total > kMaxLds)
        return set_error(SV2_EUNSUPPORTED, "attention: the window's staged tables exceed the LDS of a CU");
    p->vid_qkv = a->vid_qkv;
    p->txt_qkv = a->txt_qkv;
    p->dim = a->heads * kHeadDim;
    p->row_stride = 3LL * p->dim;
    p->heads = a->heads;
    p->text_len = a->text_len;
    p->text_pad = (a->text_len + kTextPad - 1) / kTextPad * kTextPad;
    p->npairs = p->plan.nwin * a->heads;
    p->nqb = (smax + kRowsPerGroup - 1) / kRowsPerGroup;
    p->qk_norm = a->qk_norm ? 1 : 0;
    p->rope_npos = a->rope_npos;
    p->out_dtype = a->out_dtype;
    p->eps = a->eps;
    p->score_log2 = (1.f / std::sqrt(static_cast<float>(kHeadDim))) * kLog2e;
    p->gq_vid = a->gamma_q_vid;
    p->gk_vid = a->gamma_k_vid;
    p->gq_txt = a->gamma_q_txt ? a->gamma_q_txt : a->gamma_q_vid;
    p->gk_txt = a->gamma_k_txt ? a->gamma_k_txt : a->gamma_k_vid;
    p->rope_tab = reinterpret_cast<const float2*>(a->rope_table);
    p->vid_out = a->vid_out;
    p->dbg_pre = a->debug_pre;
    p->exact = a->exact ? 1 : 0;
    p->seq_rows = static_cast<long long>(a->rule.frames) * a->rule.height * a->rule.width +
                  static_cast<long long>(p->plan.nwin) * a->text_len;
    *smax_out = smax;
    *vmax_out = vmax;
    *rope_rows_out = rope_rows;
    return SV2_OK;
}

int bind_workspace(const sv2_attn_args* a, AttnParams* p)
{
    const Workspace w = workspace_layout(*p);
    if (w.total > 0 && (!a->workspace || static_cast<int64_t>(a->workspace_bytes) < w.total))
        return set_error(SV2_EINVAL, "attention: workspace missing or too small");
    if (w.total > 0 && misaligned(a->workspace, 16))
        return set_error(SV2_EINVAL, "attention: workspace must be 16-byte aligned");
    char* base = static_cast<char*>(a->workspace);
    p->partial = reinterpret_cast<uint16_t*>(base + w.partial);
    p->txt_q = reinterpret_cast<uint16_t*>(base + w.txt_q);
    p->txt_k = reinterpret_cast<uint16_t*>(base + w.txt_k);
    p->txt_vt = reinterpret_cast<uint16_t*>(base + w.txt_vt);
    p->txt_vlds = reinterpret_cast<uint16_t*>(base + w.txt_vlds);
    return SV2_OK;
}

template <typename TI, int RM>
void launch_text_prepare(const AttnParams& p, hipStream_t stream)
{
    const dim3 grid((p.text_pad + kPrepRows - 1) / kPrepRows, p.heads);
    hipLaunchKernelGGL((text_prepare_kernel<TI, RM>), grid, dim3(256), 0, stream, p);
}

// stages: SV2_ATTN_STAGE_TEXT_PREPARE and / or SV2_ATTN_STAGE_WINDOWS.
template <typename TI, int RM>
int launch_attention(const AttnParams& p, int stages, hipStream_t stream)
{
    const int rc = set_dynamic_lds(reinterpret_cast<const void*>(&window_attention_kernel<TI, RM>), p.lds.total,
                                   "window attention: dynamic LDS attribute");
    if (rc != SV2_OK)
        return rc;
    if (p.text_len > 0 && (stages & SV2_ATTN_STAGE_TEXT_PREPARE))
        launch_text_prepare<TI, RM>(p, stream);
    if (!(stages & SV2_ATTN_STAGE_WINDOWS))
    {
        const hipError_t err = hipGetLastError();
        return err == hipSuccess ? SV2_OK : hip_error(err, "text_prepare_kernel launch");
    }
    const int groups = (p.npairs + 7) / 8;
    const unsigned grid = static_cast<unsigned>(groups) * 8u * static_cast<unsigned>(p.nqb);
    hipLaunchKernelGGL((window_attention_kernel<TI, RM>), dim3(grid), dim3(kThreads), p.lds.total, stream, p);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? SV2_OK : hip_error(err, "window attention launch");
}

template <typename TI>
int launch_rope(const AttnParams& p, int rope_mode, int stages, hipStream_t stream)
{
    if (rope_mode == SV2_ROPE_REFERENCE)
        return launch_attention<TI, SV2_ROPE_REFERENCE>(p, stages, stream);
    if (rope_mode == SV2_ROPE_ABSOLUTE)
        return launch_attention<TI, SV2_ROPE_ABSOLUTE>(p, stages, stream);
    return launch_attention<TI, SV2_ROPE_NONE>(p, stages, stream);
}

template <typename TO>
void launch_reduce(const AttnParams& p, void* out, hipStream_t stream)
{
    const long long pairs = static_cast<long long>(p.text_len) * p.dim / 2;
    const unsigned grid = static_cast<unsigned>((pairs + 255) / 256);
    const float inv_nw = 1.f / static_cast<float>(p.plan.nwin);
    hipLaunchKernelGGL(text_window_reduce_kernel<TO>, dim3(grid), dim3(256), 0, stream,
                       reinterpret_cast<const uint32_t*>(p.partial), out, p.plan.nwin, pairs, inv_nw);
}

template <typename TI, int RM>
int launch_prologue(const AttnParams& p, int nrb, const PrologueOut& out, hipStream_t stream)
{
    if (p.text_len > 0)
        launch_text_prepare<TI, RM>(p, stream);
    const unsigned grid = static_cast<unsigned>(p.plan.nwin) * p.heads * nrb;
    hipLaunchKernelGGL((qk_prologue_kernel<TI, RM>), dim3(grid), dim3(256), p.lds.total, stream, p, nrb, out);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? SV2_OK : hip_error(err, "qk_prologue launch");
}

template <typename TI>
int launch_prologue_rope(const AttnParams& p, int rope_mode, int nrb, const PrologueOut& out, hipStream_t stream)
{
    if (rope_mode == SV2_ROPE_REFERENCE)
        return launch_prologue<TI, SV2_ROPE_REFERENCE>(p, nrb, out, stream);
    if (rope_mode == SV2_ROPE_ABSOLUTE)
        return launch_prologue<TI, SV2_ROPE_ABSOLUTE>(p, nrb, out, stream);
    return launch_prologue<TI, SV2_ROPE_NONE>(p, nrb, out, stream);
}

// The prologue alone with any of its captures (PrologueOut, and the text
// norms through p.nq_txt / p.nk_txt): the debug entry points.
int run_prologue(const sv2_attn_args* args, const PrologueOut& out, float* nq_txt, float* nk_txt,
                 hipStream_t stream)
{
    AttnParams p;
    int smax = 0, vmax = 0, rope_rows = 0;
    int rc = prepare(args, &p, &smax, &vmax, &rope_rows);
    if (rc != SV2_OK)
        return rc;
    if ((rc = bind_workspace(args, &p)) != SV2_OK)
        return rc;
    p.lds = lds_layout_staging(vmax, rope_rows);
    p.nq_txt = nq_txt;
    p.nk_txt = nk_txt;
    const int nrb = (smax + 31) / 32;
    if (args->qkv_dtype == SV2_F32)
        return launch_prologue_rope<F32>(p, args->rope_mode, nrb, out, stream);
    if (args->qkv_dtype == SV2_F16)
        return launch_prologue_rope<F16>(p, args->rope_mode, nrb, out, stream);
    return launch_prologue_rope<BF16>(p, args->rope_mode, nrb, out, stream);
}

// Exact mode: the prologue into the workspace's window-sequence buffers, then
// exact_attention_kernel (the text reduction follows as in the flash path).
int launch_exact(const AttnParams& p, const Workspace& w, char* base, int rope_mode, int smax, int vmax,
                 int rope_rows, hipStream_t stream)
{
    AttnParams ps = p;
    ps.lds = lds_layout_staging(vmax, rope_rows);
    float* q = reinterpret_cast<float*>(base + w.seq_q);
    float* k = reinterpret_cast<float*>(base + w.seq_k);
    float* v = reinterpret_cast<float*>(base + w.seq_v);
    int rc = launch_prologue_rope<F32>(ps, rope_mode, (smax + 31) / 32, PrologueOut{q, k, v, nullptr, nullptr}, stream);
    if (rc != SV2_OK)
        return rc;
    const int sstride = (smax + 3) & ~3;
    const int lds = (kExactWaves * kHeadDim + kExactWaves * sstride) * static_cast<int>(sizeof(float));
    if (lds > kMaxLds)
        return set_error(SV2_EUNSUPPORTED, "attention (exact): window too long for the LDS of a CU");
    if ((rc = set_dynamic_lds(reinterpret_cast<const void*>(&exact_attention_kernel), lds,
                              "attention (exact): dynamic LDS attribute")) != SV2_OK)
        return rc;
    const int nqg = (smax + kExactWaves - 1) / kExactWaves;
    const long long grid = static_cast<long long>(p.plan.nwin) * p.heads * nqg;
    if (grid >= (1LL << 31))
        return set_error(SV2_EUNSUPPORTED, "attention (exact): grid too large");
    const float scale = 1.f / std::sqrt(static_cast<float>(kHeadDim)); // seedvr2_dit_block.cpp:896
    hipLaunchKernelGGL(exact_attention_kernel, dim3(static_cast<unsigned>(grid)), dim3(kExactWaves * 64), lds, stream,
                       p, q, k, v, nqg, sstride, scale);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? SV2_OK : hip_error(err, "exact_attention_kernel launch");
}

} // namespace

// Scratch of the no-allocation entry point (sv2_window_attention_no_alloc):
// the per-window bf16 text partials, the prepared text q, k, v^T and the
// first text tiles' v^T in LDS order of one attention call.  48 MiB covers the
// 720p x 21f workload (144 windows x 58 text tokens x 2560 channels of
// partials, 44.3 MB in all).  Each device that
// loads the library holds its own copy until the process ends.  Every byte a
// call reads is written earlier in the same call (all text rows of every
// window and head, the whole prepared text), so nothing is cleared between
// calls; calls that overlap on one device share it and race.
constexpr int64_t kStaticScratchBytes = int64_t(48) << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace
{

// The device address of `scratch` on the current device, looked up once per
// device (the array's name in host code is a host-side stand-in, not a
// device address).
int static_scratch_address(void** out)
{
    static std::mutex lock;
    static std::map<int, void*> address;
    int device = 0;
    hipError_t err = hipGetDevice(&device);
    if (err != hipSuccess)
        return hip_error(err, "attention (no alloc): hipGetDevice");
    std::lock_guard<std::mutex> guard(lock);
    auto it = address.find(device);
    if (it == address.end())
    {
        void* ptr = nullptr;
        err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (err != hipSuccess || !ptr)
            return hip_error(err != hipSuccess ? err : hipErrorInvalidSymbol,
                             "attention (no alloc): address of the static scratch");
        it = address.emplace(device, ptr).first;
    }
    *out = it->second;
    return SV2_OK;
}

} // namespace

int attention_captures(const sv2_attn_args* args, float* q, float* k, float* v, float* nq_vid, float* nk_vid,
                       float* nq_txt, float* nk_txt, hipStream_t stream)
{
    if (!q && !k && !v && !nq_vid && !nk_vid && !nq_txt && !nk_txt)
        return SV2_OK;
    return run_prologue(args, PrologueOut{q, k, v, nq_vid, nk_vid}, nq_txt, nk_txt, stream);
}

} // namespace sv2

extern "C" {

int64_t sv2_window_attention_workspace(const sv2_attn_args* args)
try
{
    using namespace sv2;
    AttnParams p;
    int smax = 0, vmax = 0, rope_rows = 0;
    const int rc = prepare(args, &p, &smax, &vmax, &rope_rows);
    if (rc != SV2_OK)
        return rc;
    return workspace_layout(p).total;
}
catch (...)
{
    return sv2::caught_exception("sv2_window_attention_workspace");
}

int sv2_window_attention_stages(const sv2_attn_args* args, int stages, void* stream_ptr)
try
{
    using namespace sv2;
    if (stages <= 0 || (stages & ~SV2_ATTN_STAGE_ALL) != 0)
        return set_error(SV2_EINVAL, "attention: stages must be a non-empty set of SV2_ATTN_STAGE_* bits");
    AttnParams p;
    int smax = 0, vmax = 0, rope_rows = 0;
    int rc = prepare(args, &p, &smax, &vmax, &rope_rows);
    if (rc != SV2_OK)
        return rc;
    if (!args->vid_out || (args->text_len > 0 && !args->txt_out))
        return set_error(SV2_EINVAL, "attention: null output pointer");
    if (p.exact && stages != SV2_ATTN_STAGE_ALL)
        return set_error(SV2_EUNSUPPORTED, "attention: the exact mode runs its stages together (SV2_ATTN_STAGE_ALL)");
    if ((rc = bind_workspace(args, &p)) != SV2_OK)
        return rc;
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);

    const int launch_stages = stages & (SV2_ATTN_STAGE_TEXT_PREPARE | SV2_ATTN_STAGE_WINDOWS);
    if (p.exact)
        rc = launch_exact(p, workspace_layout(p), static_cast<char*>(args->workspace), args->rope_mode, smax, vmax,
                          rope_rows, stream);
    else if (launch_stages == 0)
        rc = SV2_OK;
    else if (args->qkv_dtype == SV2_F32)
        rc = launch_rope<F32>(p, args->rope_mode, launch_stages, stream);
    else if (args->qkv_dtype == SV2_F16)
        rc = launch_rope<F16>(p, args->rope_mode, launch_stages, stream);
    else
        rc = launch_rope<BF16>(p, args->rope_mode, launch_stages, stream);
    if (rc != SV2_OK)
        return rc;

    if (p.text_len > 0 && (stages & SV2_ATTN_STAGE_TEXT_REDUCE))
    {
        if (args->out_dtype == SV2_F32)
            launch_reduce<F32>(p, args->txt_out, stream);
        else if (args->out_dtype == SV2_F16)
            launch_reduce<F16>(p, args->txt_out, stream);
        else
            launch_reduce<BF16>(p, args->txt_out, stream);
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess)
            return hip_error(err, "text_window_reduce_kernel launch");
    }
    return SV2_OK;
}
catch (...)
{
    return sv2::caught_exception("sv2_window_attention_stages");
}

int sv2_window_attention(const sv2_attn_args* args, void* stream_ptr)
{
    return sv2_window_attention_stages(args, SV2_ATTN_STAGE_ALL, stream_ptr);
}

int sv2_window_attention_no_alloc(const sv2_attn_args* args, void* stream_ptr)
try
{
    using namespace sv2;
    if (!args)
        return set_error(SV2_EINVAL, "attention (no alloc): null args");
    if (args->exact)
        return set_error(SV2_EUNSUPPORTED,
                         "attention (no alloc): the exact mode's window-sequence buffers exceed the static scratch");
    const int64_t need = sv2_window_attention_workspace(args);
    if (need < 0)
        return static_cast<int>(need);
    if (need > kStaticScratchBytes)
    {
        char msg[160];
        std::snprintf(msg, sizeof(msg), "attention (no alloc): needs %lld bytes of scratch, the static scratch holds %lld",
                      static_cast<long long>(need), static_cast<long long>(kStaticScratchBytes));
        return set_error(SV2_EUNSUPPORTED, msg);
    }
    void* ptr = nullptr;
    const int rc = static_scratch_address(&ptr);
    if (rc != SV2_OK)
        return rc;
    sv2_attn_args a = *args;
    a.workspace = ptr;
    a.workspace_bytes = static_cast<size_t>(kStaticScratchBytes);
    return sv2_window_attention(&a, stream_ptr);
}
catch (...)
{
    return sv2::caught_exception("sv2_window_attention_no_alloc");
}

int sv2_qk_prologue(const sv2_attn_args* args, float* q_out, float* k_out, float* v_out, void* stream_ptr)
try
{
    using namespace sv2;
    if (!args)
        return set_error(SV2_EINVAL, "qk_prologue: null args");
    if (!q_out || !k_out || !v_out)
        return set_error(SV2_EINVAL, "qk_prologue: null output pointer");
    return run_prologue(args, PrologueOut{q_out, k_out, v_out, nullptr, nullptr}, nullptr, nullptr,
                        static_cast<hipStream_t>(stream_ptr));
}
catch (...)
{
    return sv2::caught_exception("sv2_qk_prologue");
}

int sv2_window_index_map(const sv2_window_rule* rule, int32_t* out, void* stream_ptr)
try
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
catch (...)
{
    return sv2::caught_exception("sv2_window_index_map");
}

} // extern "C"
