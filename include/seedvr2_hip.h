/*
 * seedvr2_hip.h — C ABI of the MI355X (gfx950) windowed multimodal attention
 * path of the SeedVR2-3B DiT block.
 *
 * The reference has no C ABI: its path lives inside the ncnn custom layer
 * SeedVR2DiTBlock (src/layers/seedvr2_dit_block.{h,cpp} of
 * czwdysj/seedvr2-ncnn-valkan).  Each entry point below replaces one piece of
 * that layer, cited per function.  The ncnn-compatible C++ layer in this
 * library is the production caller; tests and foreign-language bindings call
 * these functions directly.
 *
 * Conventions
 *   - plain pointers and sizes; every tensor pointer is device memory unless a
 *     parameter says "host";
 *   - row-major 2-D tensors [rows, cols]; qkv rows hold q at column h*128,
 *     k at D + h*128, v at 2D + h*128 (the InnerProduct output layout of the
 *     reference, seedvr2_dit_block.cpp:984-999);
 *   - launchers only enqueue work on `stream` (a hipStream_t; NULL = the null
 *     stream) and never synchronise;
 *   - return codes: SV2_OK (0), SV2_EINVAL (-1, bad argument, the reference's
 *     invalid-input code), SV2_EUNSUPPORTED (-2, valid but unsupported shape),
 *     SV2_EDEVICE (-100, a HIP error, the reference's allocation/sublayer
 *     failure code).  sv2_last_error() returns a message for the last failure
 *     on the calling thread.
 */
#ifndef SEEDVR2_HIP_H
#define SEEDVR2_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SV2_OK 0
#define SV2_EINVAL (-1)
#define SV2_EUNSUPPORTED (-2)
#define SV2_EDEVICE (-100)

/* Element types of device tensors. */
typedef enum sv2_dtype {
    SV2_F32 = 0,
    SV2_F16 = 1,
    SV2_BF16 = 2
} sv2_dtype;

/* RoPE variants of the q/k prologue. */
typedef enum sv2_rope_mode {
    /* dit_v2 mmrope3d as the reference computes it (seedvr2_dit_block.cpp:956-971,
     * :988, :994, :1004-1020): 3 axes x 21 adjacent pairs over dims 0..125,
     * window-local positions (L_txt + t - t0, y - h0, x - w0) for video, and
     * (l, l, l) for text token l. */
    SV2_ROPE_REFERENCE = 0,
    /* head_dim split 32/48/48 over t/h/w, freq_i = theta^(-2i/d_axis),
     * absolute grid positions (t, y, x), text tokens not rotated. */
    SV2_ROPE_ABSOLUTE = 1,
    SV2_ROPE_NONE = 2
} sv2_rope_mode;

/* Which windows a grid is split into.  Replaces the inputs of
 * SeedVR2DiTBlock::make_windows (seedvr2_dit_block.cpp:827-868): the patched
 * grid comes from set_runtime_shape / the vid_shape blob, `shifted` from
 * param 3.  wt/wh/ww == 0 select the reference's adaptive size on that axis
 * (:832-838); a positive value fixes the window extent on that axis. */
typedef struct sv2_window_rule {
    int frames;  /* T */
    int height;  /* H */
    int width;   /* W */
    int shifted; /* half-window shift on axes whose window is smaller than the extent */
    int wt, wh, ww;
} sv2_window_rule;

/* One window: [t0,t1) x [h0,h1) x [w0,w1).  Same fields as
 * SeedVR2DiTBlock::Window (seedvr2_dit_block.h:98-106). */
typedef struct sv2_window {
    int t0, t1, h0, h1, w0, w1;
} sv2_window;

/* Host.  Computes the window plan in the reference order (w outer, h, t inner,
 * empty windows skipped), seedvr2_dit_block.cpp:827-868.  Writes up to `cap`
 * windows to `out` (host memory; may be NULL when cap == 0) and returns the
 * window count, or a negative error code. */
int sv2_window_plan(const sv2_window_rule* rule, sv2_window* out, int cap);

/* Device.  Writes the gather index map the attention kernel uses: for each
 * window in plan order and each video token of it in t -> y -> x order, the
 * global video row (t*H + y)*W + x (seedvr2_dit_block.cpp:976-981).
 * `out` is int32 [T*H*W]. */
int sv2_window_index_map(const sv2_window_rule* rule, int32_t* out, void* stream);

/* Host.  Size in floats of the RoPE cos/sin table of a mode for positions
 * 0..npos-1: 3 axes x npos x 24 pairs x (cos, sin). */
size_t sv2_rope_table_floats(int npos);

/* Host.  Fills `host_table` (sv2_rope_table_floats(npos) floats) with
 * cos/sin of float(pos) * freq per axis and pair, evaluated with the host C
 * library's cosf/sinf exactly as the reference's CPU layer evaluates them
 * (seedvr2_dit_block.cpp:963-965).  `freqs` (host, 21 floats) is the
 * rope_freqs weight for SV2_ROPE_REFERENCE; `theta` is used by
 * SV2_ROPE_ABSOLUTE.  The caller uploads the table to device memory. */
int sv2_rope_table_build(int rope_mode, const float* freqs, float theta, int npos,
                         float* host_table);

/* Host.  Smallest npos a table must cover for this rule, text length and mode. */
int sv2_rope_positions_needed(const sv2_window_rule* rule, int text_len, int rope_mode);

/* Arguments of the joint video-window + text attention.  Replaces
 * SeedVR2DiTBlock::attention (seedvr2_dit_block.cpp:870-1091) and, on the
 * device, the qkv_prepare / attention / zero_buffer / window_sum shaders
 * (:192-330, :339-438, :442-457, :541-572). */
typedef struct sv2_attn_args {
    sv2_window_rule rule;
    int heads;          /* H; head_dim is 128 */
    int head_dim;       /* must be 128 */
    int text_len;       /* L_txt (>= 0) */
    float eps;          /* RMSNorm eps of the q/k norm (param 8, default 1e-5) */
    int qk_norm;        /* 1: per-head RMSNorm * gamma on q, k (reference); 0: none */
    int rope_mode;      /* sv2_rope_mode */
    const float* rope_table; /* device, from sv2_rope_table_build; unused for NONE */
    int rope_npos;      /* positions covered by rope_table */
    const void* vid_qkv;     /* [T*H*W, 3*heads*128] */
    const void* txt_qkv;     /* [text_len, 3*heads*128] */
    int qkv_dtype;           /* sv2_dtype */
    const float* gamma_q_vid; /* [128] fp32 norm_q of the video branch */
    const float* gamma_k_vid;
    const float* gamma_q_txt; /* [128] norm_q of the text branch (= video branch when shared) */
    const float* gamma_k_txt;
    void* vid_out;           /* [T*H*W, heads*128] */
    void* txt_out;           /* [text_len, heads*128] */
    int out_dtype;           /* sv2_dtype */
    void* workspace;         /* device scratch, sv2_window_attention_workspace() bytes */
    size_t workspace_bytes;
    float* debug_pre;        /* optional [sum_w S_w, heads*128] fp32: every query's
                                output before its bf16 rounding, window-sequence order
                                (video t->y->x then text), NULL to skip */
} sv2_attn_args;

/* Host.  Bytes of device workspace sv2_window_attention needs for these args
 * (the per-window text partial outputs), or a negative error code. */
int64_t sv2_window_attention_workspace(const sv2_attn_args* args);

/* Device.  Fused per-head QK-RMSNorm + RoPE + bf16 prologue and online-softmax
 * flash attention of every video window jointly with all text tokens, on
 * gfx950 MFMA; video outputs written once per token (windows partition the
 * grid), text outputs averaged over windows in window order.  Every output
 * element is rounded to bf16 as the reference rounds it (:1074). */
int sv2_window_attention(const sv2_attn_args* args, void* stream);

/* Device.  Debug/test entry: the prologue alone.  Writes q, k, v after
 * normalisation, rotation and bf16 rounding, fp32, each [sum_w S_w, heads*128]
 * in window-sequence order; the same device code the attention kernel runs
 * (the reference's attention_q/k/v debug captures, seedvr2_dit_block.cpp:1030-1043). */
int sv2_qk_prologue(const sv2_attn_args* args, float* q_out, float* k_out, float* v_out,
                    void* stream);

/* Device.  Token RMSNorm over `dim` (no gamma) fused with ada input
 * modulation.  Replaces apply_rmsnorm + apply_ada_input
 * (seedvr2_dit_block.cpp:770-805) and the rmsnorm_reduce / rmsnorm_apply
 * shaders (:89-179).  y = (x * inv_rms) * (emb[c*6+slot+1] + scale[c])
 *                         + emb[c*6+slot] + shift[c]
 * when has_ada, else y = x * inv_rms.  x, y: [rows, dim] of io_dtype; emb
 * [6*dim], shift, scale [dim]: fp32.  slot_base is 0 (attention) or 3 (MLP). */
int sv2_rmsnorm_ada(const void* x, void* y, int io_dtype, int rows, int dim, float eps,
                    const float* emb, const float* shift, const float* scale, int slot_base,
                    int has_ada, void* stream);

/* Device.  Output modulation and residual, in place on `x`.  Replaces
 * apply_ada_output_and_residual (seedvr2_dit_block.cpp:807-825), the last-layer
 * text variants (:1198-1209, :1225-1246) and the ada_residual shader (:465-508):
 *   mode 0: x = x * (emb[c*6+slot_base+2] + gate[c]) + residual
 *   mode 1: x = x + residual
 *   mode 2: x = 2 * x                                                     */
int sv2_ada_residual(void* x, const void* residual, int io_dtype, int rows, int dim,
                     const float* emb, const float* gate, int slot_base, int mode,
                     void* stream);

/* Device.  SwiGLU gate in place: gate = silu(gate) * value.  Replaces the
 * loop in apply_mlp (seedvr2_dit_block.cpp:1093-1112) and the silu shader
 * (:514-533). */
int sv2_swiglu(void* gate, const void* value, int io_dtype, int64_t count, void* stream);

/* Message of the last failure on the calling thread (never NULL). */
const char* sv2_last_error(void);

/* Library version string. */
const char* sv2_version(void);

#ifdef __cplusplus
}
#endif

#endif
