// Internal declarations shared by the host launch layer and the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <vector>

#include "seedvr2_hip.h"

namespace sv2
{

// Head dimension the MFMA tiling is written for (SeedVR2-3B: 20 heads x 128).
constexpr int kHeadDim = 128;

// Most non-empty window intervals one axis may have; the per-axis boundary
// lists travel to the kernels by value in the kernel arguments.
constexpr int kMaxAxisIntervals = 48;

// Pairs per RoPE axis slot in the cos/sin table (reference: 21, absolute: 16/24/24).
constexpr int kRopePairSlots = 24;

// The non-empty intervals of one axis of a window plan, as boundaries:
// interval i is [b[i], b[i+1]).  They partition [0, extent).
struct AxisPlan
{
    int n;
    int b[kMaxAxisIntervals + 1];
};

// A window plan in closed form.  The reference enumerates windows w-outer,
// h-middle, t-inner and skips empty ones (seedvr2_dit_block.cpp:853-866);
// an axis interval is empty independently of the other axes, so the kept
// windows are exactly the product of the per-axis non-empty intervals in that
// order, and window index wi decodes as it = wi % nt, ih = (wi / nt) % nh,
// iw = wi / (nt * nh).
struct PlanArgs
{
    AxisPlan t, h, w;
    int T, H, W;
    int nwin;
};

struct WindowBox
{
    int t0, t1, h0, h1, w0, w1;
    int lt, lh, lw;
    int vlen;    // video tokens in the window
    int vprefix; // video tokens of all earlier windows (window-sequence offset)
};

__host__ __device__ inline WindowBox window_box(const PlanArgs& p, int wi)
{
    const int it = wi % p.t.n;
    const int rest = wi / p.t.n;
    const int ih = rest % p.h.n;
    const int iw = rest / p.h.n;
    WindowBox b;
    b.t0 = p.t.b[it];
    b.t1 = p.t.b[it + 1];
    b.h0 = p.h.b[ih];
    b.h1 = p.h.b[ih + 1];
    b.w0 = p.w.b[iw];
    b.w1 = p.w.b[iw + 1];
    b.lt = b.t1 - b.t0;
    b.lh = b.h1 - b.h0;
    b.lw = b.w1 - b.w0;
    b.vlen = b.lt * b.lh * b.lw;
    // earlier windows: every full w-column before iw, then the full h-rows
    // before ih within column iw, then the t-slices before it
    b.vprefix = b.w0 * p.H * p.T + b.lw * b.h0 * p.T + b.lw * b.lh * b.t0;
    return b;
}

// Global video row of local token j (t -> y -> x order) of a window.
__host__ __device__ inline int window_video_row(const PlanArgs& p, const WindowBox& b, int j,
                                                int* lt_out, int* ly_out, int* lx_out)
{
    const int plane = b.lh * b.lw;
    const int t = j / plane;
    const int rem = j - t * plane;
    const int y = rem / b.lw;
    const int x = rem - y * b.lw;
    *lt_out = t;
    *ly_out = y;
    *lx_out = x;
    return ((b.t0 + t) * p.H + (b.h0 + y)) * p.W + (b.w0 + x);
}

// bf16 round-to-nearest-even on the raw bits, kept in an fp32 container
// (the arithmetic of seedvr2_dit_block.cpp:68-79).
__host__ __device__ inline float bf16_round(float value)
{
    uint32_t bits = __builtin_bit_cast(uint32_t, value);
    bits += 0x7fffu + ((bits >> 16) & 1u);
    bits &= 0xffff0000u;
    return __builtin_bit_cast(float, bits);
}

// Thread-local error message plumbing for the C ABI.
int set_error(int code, const std::string& message);
// True for a non-null pointer that is not `bytes`-aligned (bytes a power of
// two): operands fetched by 16-byte vector loads or straight into LDS are
// refused rather than read at the wrong address.
inline bool misaligned(const void* ptr, uintptr_t bytes)
{
    return ptr && (reinterpret_cast<uintptr_t>(ptr) & (bytes - 1)) != 0;
}
int hip_error(hipError_t err, const char* what);
// Called from the catch clause of an entry point of the C ABI, which lets no
// C++ exception out (std::bad_alloc of a host container, std::system_error
// of a thread): records what was caught and returns SV2_EDEVICE, the
// allocation-failure code.
int caught_exception(const char* entry) noexcept;
// Raises a kernel's dynamic LDS limit to at least `bytes` on the current
// device.  The attribute is per device; it is set once per (kernel, device)
// and size, under a lock, not on every launch.
int set_dynamic_lds(const void* kernel, int bytes, const char* what);

// The attention prologue's debug captures for these attention arguments
// (each output may be NULL): q, k, v after the prologue in window-sequence
// order [sum S][D]; q, k after the norm and before RoPE, video rows in grid
// order [T*H*W][D] and text rows [L_txt][D].  Enqueued on `stream`.
int attention_captures(const sv2_attn_args* args, float* q, float* k, float* v, float* nq_vid, float* nk_vid,
                       float* nq_txt, float* nk_txt, hipStream_t stream);
// Rounds count fp32 values to bf16 (nearest even) in place.
int launch_bf16_round(float* x, long long count, hipStream_t stream);

// Builds the closed-form plan; returns SV2_OK or an error code.
int build_plan(const sv2_window_rule& rule, PlanArgs* plan);

// y[r][c] += b[c] for a [rows, cols] tensor of dtype (cols a multiple of 8).
int launch_bias_rows(void* y, const float* b, int dtype, int rows, int cols, hipStream_t stream);
// The same, then y = silu(y) when `silu` is non-zero.
int launch_bias_act(void* y, const float* b, int dtype, int rows, int cols, int silu, hipStream_t stream);

// Per-layer ada modulation table [3][dim] from the emb blob [dim][6]:
// row 0 emb[c*6+slot+1] + scale[c], row 1 emb[c*6+slot], row 2
// emb[c*6+slot+2] + gate[c] (slot 0 attention, 3 MLP).
int launch_ada_table(const float* emb, const float* scale, const float* gate, int slot, int dim, float* out,
                     hipStream_t stream);
// A block's tables in one launch: `tables` (1-4) of them at out + 3 * dim * t,
// slot 0 for even t and 3 for odd t, from scale[t] and gate[t]; with `bias`,
// out + 12 * dim gets (table 0's gate row) * bias, the gated bias.
int launch_block_tables(const float* emb, const float* const* scale, const float* const* gate, int tables,
                        const float* bias, int dim, float* out, hipStream_t stream);
// Token RMSNorm (times gamma[c] when gamma is not NULL), then when has_ada
// the input modulation with rows 0-1 of `table` and `shift`.  Arguments
// already validated (dim a multiple of 8, <= 4096).
int launch_rmsnorm_table(const void* x, void* y, int dtype, int rows, int dim, float eps, const float* table,
                         const float* shift, const float* gamma, int has_ada, hipStream_t stream);
// x = (x [+ bias]) * table[2] + residual (mode 0), x + residual (mode 1),
// 2x (mode 2); bias may be NULL.
int launch_residual_table(void* x, const void* residual, int dtype, int rows, int dim, const float* table,
                          const float* bias, int mode, hipStream_t stream);

// y[rows, out] = x[rows, in] W^T, W [out][in] row-major (an InnerProduct
// without its bias), in dtype (SV2_F32 or SV2_F16); enqueued on `stream`.
// fp16 runs on hipBLASLt with fp32 accumulation (the first product of a
// shape times the library's candidate kernels and synchronises the stream
// once); fp32 on gemm_f32_exact.
int gemm_rows(hipStream_t stream, int dtype, int rows, int in, int out, const void* x, const void* w, void* y);
// The same with the InnerProduct's bias (may be NULL): fp32 adds it to the
// double sum before the one rounding; fp16 adds it in a pass after the product.
int gemm_rows_bias(hipStream_t stream, int dtype, int rows, int in, int out, const void* x, const void* w,
                   const float* bias, void* y);
// fp32 y = float(sum_i double(x_i) double(w_i) + double(bias)): products added
// in increasing i, one rounding (gemm_exact.hip); bias may be NULL.
int gemm_f32_exact(hipStream_t stream, int rows, int in, int out, const float* x, const float* w, const float* bias,
                   float* y);
// fp16 only: y = gate[c] * (x W^T)[r][c] + residual[r][c] (+ bias[c] when
// bias is not null), the gated residual of seedvr2_dit_block.cpp:807-825 in
// the product's epilogue (fp32, one rounding to fp16); -2 when hipBLASLt has
// no kernel for it.  A preceding InnerProduct bias b enters as bias = gate * b.
int gemm_rows_gated(hipStream_t stream, int dtype, int rows, int in, int out, const void* x, const void* w, void* y,
                    const float* gate, const void* residual, const float* bias = nullptr);

// fp16 y = epilogue(x W^T) on the hand-written MFMA kernel (gemm.hip), x
// [rows][in], W (and w2) [out][in].  Epilogues: store; the gated residual
// y = fp16((fp16(x W^T) + bias) * gate + residual) (bias, gate optional);
// SwiGLU y = silu(fp16(x W^T)) * fp16(x W2^T).  Needs in % 64 == 0 and
// out % 256 == 0 (SwiGLU: out % 128 == 0).
constexpr int kGemmStore = 0;
constexpr int kGemmResidual = 1;
constexpr int kGemmSwiGLU = 2;
bool gemm_mfma_supported(int in, int out, int epi);
int gemm_mfma(hipStream_t stream, int rows, int in, int out, const void* x, const void* w, const void* w2, void* y,
              int epi, const float* bias, const float* gate, const void* residual);

// fp16 y = epilogue(x W^T) for 1-64 rows on the weight-streaming kernel
// (gemm_few.hip), the same epilogues as gemm_mfma (kGemmStore also takes an
// optional bias: y = fp16(fp16(x W^T) + bias)).  Needs in % 64 == 0 and
// out % 64 == 0 (SwiGLU: out % 32 == 0).  K may be split over workgroups:
// `work` then holds gemm_few_workspace() bytes of fp32 partial sums.
bool gemm_few_supported(int rows, int in, int out, int epi);
int gemm_few_splits(int rows, int in, int out, int epi);
size_t gemm_few_workspace(int rows, int in, int out, int epi);
int gemm_few(hipStream_t stream, int rows, int in, int out, const void* x, const void* w, const void* w2, void* y,
             int epi, const float* bias, const float* gate, const void* residual, void* work, size_t work_bytes);

// Allocates device memory for `count` host fp32 values, stores them as dtype
// (SV2_F32 or SV2_F16, round to nearest) and records the allocation in *owned.
int upload_weights(std::vector<void*>* owned, const float* host, size_t count, int dtype, const void** dev);

// The compute dtype a block was created with.
int block_compute_dtype(const sv2_block* block);

// Head kernels (dit_heads.hip).
int launch_patchify(const float* video, void* patches, int dtype, int T, int h, int w, int C, int channel_major,
                    hipStream_t stream);
int launch_unpatchify(const void* projected, float* output, int dtype, int T, int h, int w, int OC, int channel_major,
                      hipStream_t stream);
int launch_sinusoid(float* out, float timestep, int dim, hipStream_t stream);
int launch_from_f32(void* dst, const float* src, int dtype, long long count, hipStream_t stream);

// dst (fp32) = src (dtype); count a multiple of 8.
int launch_to_f32(float* dst, const void* src, int dtype, long long count, hipStream_t stream);

} // namespace sv2
