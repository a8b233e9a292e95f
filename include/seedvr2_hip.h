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
 *     SV2_EDEVICE (-100, a HIP error or a failed host allocation, the
 *     reference's allocation/sublayer failure code).  sv2_last_error()
 *     returns a message for the last failure on the calling thread.  No C++
 *     exception leaves an entry point.
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
    int exact;               /* 0: the MFMA flash kernel.  1 (fp32 qkv only): the
                                reference CPU layer's arithmetic step for step
                                (seedvr2_dit_block.cpp:942-1088: double dot products
                                and output sums in the reference's order, float
                                scores, correctly rounded exp and weights, the
                                denominator summed in key order), the fp32 parity
                                mode; its workspace also holds q, k, v after the
                                prologue, 3 x [sum_w S_w, heads*128] fp32 */
} sv2_attn_args;

/* Host.  Bytes of device workspace sv2_window_attention needs for these args
 * (the per-window text partial outputs), or a negative error code. */
int64_t sv2_window_attention_workspace(const sv2_attn_args* args);

/* Device.  Fused per-head QK-RMSNorm + RoPE + bf16 prologue and online-softmax
 * flash attention of every video window jointly with all text tokens, on
 * gfx950 MFMA; video outputs written once per token (windows partition the
 * grid), text outputs averaged over windows in window order.  Every output
 * element is rounded to bf16 as the reference rounds it (:1074).  qkv, output
 * and workspace pointers must be 16-byte aligned (SV2_EINVAL otherwise): the
 * kernel fetches rows straight into LDS in 16-byte pieces. */
int sv2_window_attention(const sv2_attn_args* args, void* stream);

/* The three launches of sv2_window_attention, selectable (a bit set of the
 * values below; SV2_ATTN_STAGE_ALL is sv2_window_attention):
 *   SV2_ATTN_STAGE_TEXT_PREPARE  the text rows' q/k prologue and V, once per
 *                                layer, into the workspace;
 *   SV2_ATTN_STAGE_WINDOWS       the window attention kernel (video outputs,
 *                                per-window text partials in the workspace);
 *   SV2_ATTN_STAGE_TEXT_REDUCE   the text outputs from those partials.
 * Each stage reads what the earlier ones left in the same workspace, so stages
 * run in this order on one stream with the same args.  No counterpart in the
 * reference (its Vulkan path records the three as one sequence): for callers
 * that time or schedule the launches one at a time.  The exact mode accepts
 * SV2_ATTN_STAGE_ALL only (SV2_EUNSUPPORTED otherwise). */
enum sv2_attn_stage {
    SV2_ATTN_STAGE_TEXT_PREPARE = 1,
    SV2_ATTN_STAGE_WINDOWS = 2,
    SV2_ATTN_STAGE_TEXT_REDUCE = 4,
    SV2_ATTN_STAGE_ALL = 7
};
int sv2_window_attention_stages(const sv2_attn_args* args, int stages, void* stream);

/* Device.  sv2_window_attention for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc); it has no counterpart in the reference.  args->workspace
 * and workspace_bytes are ignored: the scratch is a static device array of
 * the library, 48 MiB per device (the 720p x 21f workload needs 44.3 MB), held
 * until the process ends.  Calls whose sv2_window_attention_workspace exceeds
 * it, and the exact mode, return SV2_EUNSUPPORTED.  Calls that overlap on one
 * device share the array and race; calls on one stream are ordered.
 * Allocates nothing (no hipMalloc / hipFree). */
int sv2_window_attention_no_alloc(const sv2_attn_args* args, void* stream);

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

/* ------------------------------------------------------------------------
 * The SeedVR2DiTBlock layer (seedvr2_dit_block.h:38-172): one MM-DiT block
 * of SeedVR2-3B on the device.  Same parameters (ids 0-8 of the layer's
 * ParamDict, seedvr2_dit_block.cpp:643-655), the same weight order
 * (load_branch / load_model, :657-688) and the same blob layouts (bottoms
 * vid [L_v, dim], txt [L_txt, dim], emb [6*dim], the patched (T, H, W);
 * tops vid_out, txt_out).  Optional ids 9-13 select variants the reference
 * does not have (fixed window extents, absolute 3-D RoPE, no q/k norm); their
 * defaults are the reference semantics.
 * ------------------------------------------------------------------------ */

typedef struct sv2_block_config {
    int block_index;     /* param 0 */
    int shared_weights;  /* param 1: one weight branch for video and text (blocks >= 10) */
    int last_layer;      /* param 2: text skips ada input / gate, txt_out = 2 * txt_proj */
    int shifted_window;  /* param 3 */
    int dim;             /* param 4 (2560) */
    int heads;           /* param 5 (20) */
    int head_dim;        /* param 6 (128) */
    int mlp_hidden;      /* param 7 (6912) */
    float norm_eps;      /* param 8 (1e-5) */
    int window_t;        /* param 9: window extent on t, 0 = the reference's adaptive rule */
    int window_h;        /* param 10 */
    int window_w;        /* param 11 */
    int rope_mode;       /* param 12: sv2_rope_mode (default SV2_ROPE_REFERENCE) */
    int qk_norm;         /* param 13: 1 (default) = per-head RMSNorm * gamma on q, k */
    int fused_gemm;      /* param 14: 1 = the video branch's InnerProducts on the hand-written
                            MFMA kernel with their passes fused (sv2_inner_product_f16: qkv;
                            proj_out + gated residual; gate/in + SwiGLU; out + gated residual),
                            fp16 compute only (ignored for fp32) and not while debug captures
                            are set; needs dim % 256 == 0 and mlp_hidden % 128 == 0.
                            0 (default) = library GEMMs and separate passes. */
} sv2_block_config;

/* Weights of one branch ("vid", "txt" or the shared "all"), in the order the
 * exporter writes them (tools/export_seedvr2_dit_ncnn.py:222-235).  Matrices
 * are [out][in] row-major (InnerProduct layout). */
typedef struct sv2_block_branch {
    const void* ada[6];  /* [dim] each: attn shift, scale, gate, mlp shift, scale, gate (fp32) */
    const void* w_qkv;   /* [3*dim][dim] */
    const void* w_proj;  /* [dim][dim] */
    const void* b_proj;  /* [dim] fp32 */
    const void* norm_q;  /* [head_dim] fp32 */
    const void* norm_k;  /* [head_dim] fp32 */
    const void* w_gate;  /* [mlp_hidden][dim] */
    const void* w_in;    /* [mlp_hidden][dim] */
    const void* w_out;   /* [dim][mlp_hidden] */
} sv2_block_branch;

typedef struct sv2_block sv2_block;

/* Host.  Fills `config` with the reference defaults (the exporter's block 0). */
void sv2_block_config_default(sv2_block_config* config);

/* Loads one exported block: the SeedVR2DiTBlock layer of `param_path` and
 * its weights from `bin_path` (replaces ncnn's Net::load_param / load_model
 * driving SeedVR2DiTBlock::load_param / load_model, seedvr2_dit_block.cpp:
 * 643-688), then uploads the weights: matrices in `compute_dtype` (SV2_F32 or
 * SV2_F16), vectors in fp32.  Returns SV2_OK, SV2_EINVAL (-1) for a file that
 * does not parse or whose layer parameters are invalid (dim != heads *
 * head_dim, as load_param), SV2_EDEVICE (-100) for a weight stream that ends
 * early or an allocation failure (load_model's code). */
int sv2_block_load(const char* param_path, const char* bin_path, int compute_dtype, sv2_block** out);

/* Creates a block from weights already in memory.  weights_on_device == 0:
 * host fp32 arrays, converted and uploaded (owned by the block).
 * weights_on_device == 1: device arrays, matrices in compute_dtype and
 * vectors in fp32, borrowed (they must outlive the block).  `txt` is ignored
 * when config->shared_weights.  rope_freqs: host, 21 fp32 (the block's
 * rope.freqs), may be NULL unless rope_mode is SV2_ROPE_REFERENCE. */
int sv2_block_create(const sv2_block_config* config, const sv2_block_branch* vid, const sv2_block_branch* txt,
                     const float* rope_freqs, int weights_on_device, int compute_dtype, sv2_block** out);

/* Host.  The parameters the block was created with. */
int sv2_block_get_config(const sv2_block* block, sv2_block_config* config);

/* The patched grid (T, H, W) of the next forward
 * (SeedVR2DiTBlock::set_runtime_shape, seedvr2_dit_block.cpp:609-615). */
int sv2_block_set_runtime_shape(sv2_block* block, int frames, int height, int width);

/* Bytes of device workspace a forward of text_len text tokens needs at the
 * current runtime shape. */
int64_t sv2_block_workspace_size(const sv2_block* block, int text_len);

/* Device.  One block forward (SeedVR2DiTBlock::forward, seedvr2_dit_block.cpp:
 * 1114-1267): vid [T*H*W, dim] and txt [text_len, dim] in the compute dtype,
 * emb [6*dim] fp32; writes vid_out, txt_out (same shapes, compute dtype).
 * Enqueues on `stream` only.  workspace may be NULL (the block then keeps
 * its own, grown on demand; forwards of one block that may run at the same
 * time, on different streams, must then each pass their own workspace).
 * Returns SV2_EINVAL when the runtime shape was not set (as the layer's
 * device forward, :1320-1321). */
int sv2_block_forward(sv2_block* block, const void* vid, const void* txt, int text_len, const float* emb,
                      void* vid_out, void* txt_out, void* workspace, size_t workspace_bytes, void* stream);

void sv2_block_destroy(sv2_block* block);

/* Host.  A diagnostic with no counterpart in the reference: 1 when the last
 * sv2_block_forward ran its row-wise steps (RMSNorm + ada, the InnerProducts,
 * gated residuals, SwiGLU) once over the video and text rows together (shared
 * weights outside the last layer, no debug captures, text rows right after the
 * video rows in the caller's buffers and in the workspace), 0 when it ran
 * them per branch, a negative error code for a null block. */
int sv2_block_last_forward_merged(const sv2_block* block);

/* Host.  Rows of the window-sequence order at the current runtime shape:
 * the sum over the windows of (window video tokens + text_len), the row
 * count of the attention_q/k/v/output captures (seedvr2_dit_block.cpp:
 * 1030-1043). */
int64_t sv2_block_window_rows(const sv2_block* block, int text_len);

/* Host buffers.  One block forward from and to host memory, as the layer's
 * CPU forward over ncnn::Mat blobs (SeedVR2DiTBlock::forward,
 * seedvr2_dit_block.cpp:1114-1267): vid [T*H*W, dim], txt [text_len, dim],
 * emb [6*dim] and the outputs are fp32 host arrays, whatever the compute
 * dtype.  host_debug (may be NULL): fp32 host arrays of the captures wanted
 * for this call (the sizes of sv2_block_debug).  Stages everything through
 * device memory the block keeps (grown on demand), runs on the null stream
 * and returns when the outputs are on the host.  This is the entry point of
 * the ncnn layer adapter; device callers use sv2_block_forward.  The staging
 * memory and the workspace belong to the block: calls on one block must not
 * overlap (different blocks are independent). */
int sv2_block_forward_host(sv2_block* block, const float* vid, const float* txt, int text_len, const float* emb,
                           float* vid_out, float* txt_out, const struct sv2_block_debug* host_debug);

/* Intermediate captures of one forward, fp32 device arrays (any may be NULL).
 * Replaces SeedVR2DiTBlockDebugTensors (seedvr2_dit_block.h:20-36): its 14
 * fields in the reference's row orders, plus the attention outputs as
 * proj_out reads them.  S_sum = sum over the windows of (window video tokens
 * + L_txt): the window-sequence rows (each window's video tokens t -> y -> x,
 * then the text tokens), in plan order. */
typedef struct sv2_block_debug {
    float* qkv_vid;       /* [L_v, 3*dim] */
    float* qkv_txt;       /* [L_txt, 3*dim] */
    float* attention_vid; /* [L_v, dim]: bf16-rounded attention outputs, the input of proj_out */
    float* attention_txt; /* [L_txt, dim]: text outputs averaged over windows (:1081-1088) */
    float* projected_vid; /* [L_v, dim]: proj_out + bias before the gate (:1188-1192) */
    float* projected_txt; /* [L_txt, dim] */
    float* output_vid;    /* [L_v, dim] */
    float* output_txt;    /* [L_txt, dim] */
    float* norm_q_vid;    /* [L_v, dim]: q after RMSNorm * gamma, before RoPE (:908-918, :986-990) */
    float* norm_q_txt;    /* [L_txt, dim] (:1007-1012) */
    float* norm_k_vid;    /* [L_v, dim] */
    float* norm_k_txt;    /* [L_txt, dim] */
    float* attention_q;   /* [S_sum, dim]: q after norm, RoPE and bf16, window-sequence order (:1030-1043) */
    float* attention_k;   /* [S_sum, dim] */
    float* attention_v;   /* [S_sum, dim]: v rounded to bf16 (in the fp16 mode: as the fp16 operand) */
    float* attention_output; /* [S_sum, dim]: each query's bf16-rounded output per window (:1074-1077) */
} sv2_block_debug;

/* Enables captures for the following forwards (NULL disables them), as
 * SeedVR2DiTBlock::set_debug_tensors (seedvr2_dit_block.cpp:617-620).  The
 * struct is copied; the arrays must stay valid while captures are enabled. */
int sv2_block_set_debug(sv2_block* block, const sv2_block_debug* debug);

/* ------------------------------------------------------------------------
 * The DiT input and output heads and the 32-block DiT forward
 * (SeedVR2DiTInput, seedvr2_dit_input.{h,cpp}; SeedVR2DiTOutput,
 * seedvr2_dit_output.{h,cpp}; SeedVR2DiT::forward, src/model/dit.cpp:
 * 281-383).  Same parameters, weight order and blob layouts; latent, text
 * and the DiT output are fp32 device arrays, the hidden streams between the
 * heads and the blocks are in the compute dtype.
 * ------------------------------------------------------------------------ */

typedef struct sv2_dit_input_config {
    int dim;             /* param 0 (2560) */
    int video_channels;  /* param 1 (33) */
    int text_channels;   /* param 2 (5120) */
    int sinusoidal_dim;  /* param 3 (256) */
    int embedding_dim;   /* param 4 (15360 = 6 * dim) */
} sv2_dit_input_config;

/* Weights of the input head in the exporter's order
 * (tools/export_seedvr2_dit_ncnn.py:259-276).  Matrices [out][in]; biases fp32. */
typedef struct sv2_dit_input_weights {
    const void* w_vid;      /* [dim][4 * video_channels] */
    const void* b_vid;      /* [dim] */
    const void* w_txt;      /* [dim][text_channels] */
    const void* b_txt;      /* [dim] */
    const void* w_time_in;  /* [dim][sinusoidal_dim] */
    const void* b_time_in;  /* [dim] */
    const void* w_time_hid; /* [dim][dim] */
    const void* b_time_hid; /* [dim] */
    const void* w_time_out; /* [embedding_dim][dim] */
    const void* b_time_out; /* [embedding_dim] */
} sv2_dit_input_weights;

typedef struct sv2_dit_input sv2_dit_input;

/* Loads the SeedVR2DiTInput layer of an exported .param/.bin pair
 * (seedvr2_dit_input.cpp:207-227).  Returns SV2_EINVAL when the parameters
 * fail load_param's check (odd sinusoidal_dim, embedding_dim != 6 * dim). */
int sv2_dit_input_load(const char* param_path, const char* bin_path, int compute_dtype, sv2_dit_input** out);
/* Creates the head from host fp32 (weights_on_device 0, converted and owned)
 * or borrowed device weights (1): w_vid, w_txt in the compute dtype, the time
 * MLP matrices and every bias fp32. */
int sv2_dit_input_create(const sv2_dit_input_config* config, const sv2_dit_input_weights* weights,
                         int weights_on_device, int compute_dtype, sv2_dit_input** out);
int sv2_dit_input_get_config(const sv2_dit_input* head, sv2_dit_input_config* config);
/* Device workspace bytes of a forward on the grid T x H x W (before the 2x2
 * patchify) with text_len text tokens. */
int64_t sv2_dit_input_workspace_size(const sv2_dit_input* head, int frames, int height, int width, int text_len);
/* SeedVR2DiTInput::forward (seedvr2_dit_input.cpp:311-403): video fp32
 * [T*H*W, video_channels] token-major (channel_major 0) or [video_channels][T][H][W]
 * (channel_major 1), text fp32 [text_len, text_channels], timestep (the raw
 * value, 1000 at the first Euler step).  Writes vid_out [T*(H/2)*(W/2), dim]
 * and txt_out [text_len, dim] in the compute dtype and emb fp32 [embedding_dim].
 * H and W must be even (:328-330). */
int sv2_dit_input_forward(sv2_dit_input* head, const float* video, int channel_major, const float* text,
                          int text_len, float timestep, int frames, int height, int width, void* vid_out,
                          void* txt_out, float* emb, void* workspace, size_t workspace_bytes, void* stream);
void sv2_dit_input_destroy(sv2_dit_input* head);

typedef struct sv2_dit_output_config {
    int dim;             /* param 0 (2560) */
    int output_channels; /* param 1 (16) */
    float norm_eps;      /* param 2 (1e-5) */
} sv2_dit_output_config;

/* Weights of the output head in the exporter's order
 * (tools/export_seedvr2_dit_ncnn.py:289-293). */
typedef struct sv2_dit_output_weights {
    const void* norm_weight; /* [dim] fp32 */
    const void* shift;       /* [dim] fp32 */
    const void* scale;       /* [dim] fp32 */
    const void* w_proj;      /* [4 * output_channels][dim] */
    const void* b_proj;      /* [4 * output_channels] fp32 */
} sv2_dit_output_weights;

typedef struct sv2_dit_output sv2_dit_output;

/* Loads the SeedVR2DiTOutput layer (seedvr2_dit_output.cpp:256-273). */
int sv2_dit_output_load(const char* param_path, const char* bin_path, int compute_dtype, sv2_dit_output** out);
int sv2_dit_output_create(const sv2_dit_output_config* config, const sv2_dit_output_weights* weights,
                          int weights_on_device, int compute_dtype, sv2_dit_output** out);
int sv2_dit_output_get_config(const sv2_dit_output* head, sv2_dit_output_config* config);
/* Workspace bytes of a forward over the patched grid T x h x w. */
int64_t sv2_dit_output_workspace_size(const sv2_dit_output* head, int frames, int height, int width);
/* SeedVR2DiTOutput::forward (seedvr2_dit_output.cpp:349-428): vid [T*h*w, dim]
 * in the compute dtype and emb fp32 [6 * dim] give output fp32 on the grid
 * T x 2h x 2w: token-major [T*2h*2w, output_channels] (channel_major 0) or
 * [output_channels][T][2h][2w] (channel_major 1). */
int sv2_dit_output_forward(sv2_dit_output* head, const void* vid, const float* emb, int frames, int height,
                           int width, float* output, int channel_major, void* workspace, size_t workspace_bytes,
                           void* stream);
void sv2_dit_output_destroy(sv2_dit_output* head);

typedef struct sv2_dit sv2_dit;

/* Loads a whole exported DiT from `model_dir` (SeedVR2DiT::load, dit.cpp:
 * 120-174, resident mode): seedvr2_dit_input.ncnn.{param,bin},
 * seedvr2_dit_block_NN.ncnn.{param,bin} for NN = 00..31 and
 * seedvr2_dit_output.ncnn.{param,bin}.  Every block is uploaded once.
 * When model_dir holds a SHA256SUMS manifest, every file it lists is checked
 * first (sv2_verify_checksums) and a failed check fails the load with
 * SV2_EINVAL before any weight is read. */
int sv2_dit_load(const char* model_dir, int compute_dtype, sv2_dit** out);
/* sv2_dit_load with the check chosen: SV2_VERIFY_NONE hashes nothing (the
 * reference's loader, src/model/dit.cpp:120-174, never does; about 7 GB of
 * hashing is saved), SV2_VERIFY_IF_PRESENT is sv2_dit_load, SV2_VERIFY_STRICT
 * also fails without a SHA256SUMS (sv2_verify_checksums_strict).  The check
 * reads the files in a pass of its own before the load reads them. */
enum sv2_verify_mode { SV2_VERIFY_NONE = 0, SV2_VERIFY_IF_PRESENT = 1, SV2_VERIFY_STRICT = 2 };
int sv2_dit_load_ex(const char* model_dir, int compute_dtype, int verify, sv2_dit** out);
/* Assembles a DiT from existing heads and blocks (borrowed; they must outlive
 * the DiT and share its compute dtype). */
int sv2_dit_create(sv2_dit_input* input, sv2_block* const* blocks, int block_count, sv2_dit_output* output,
                   sv2_dit** out);
/* Host.  The heads' parameters and the block count of a DiT. */
int sv2_dit_get_config(const sv2_dit* dit, sv2_dit_input_config* input, sv2_dit_output_config* output,
                       int* block_count);
/* Workspace bytes of a forward on the latent grid T x H x W (H, W even) with
 * text_len text tokens; sets every block's runtime shape to (T, H/2, W/2). */
int64_t sv2_dit_workspace_size(sv2_dit* dit, int frames, int height, int width, int text_len);
/* One DiT forward (SeedVR2DiT::forward, dit.cpp:281-383): latent fp32
 * [video_channels][T][H][W], text fp32 [text_len, text_channels], the raw
 * timestep; output fp32 [output_channels][T][H][W].  The input head, every
 * block and the output head are enqueued on `stream` with no host
 * synchronisation between them; the hidden streams stay in device memory. */
int sv2_dit_forward(sv2_dit* dit, const float* latent, const float* text, int text_len, float timestep, int frames,
                    int height, int width, float* output, void* workspace, size_t workspace_bytes, void* stream);
void sv2_dit_destroy(sv2_dit* dit);

/* ---- fp16 InnerProduct with the pass that follows it fused in, on a
 * hand-written gfx950 MFMA kernel.  Replaces the block's ncnn InnerProduct
 * layers (load_inner_product, seedvr2_dit_block.cpp:27-55; the five per
 * branch, :668-674) together with the elementwise pass after each:
 *   SV2_EPI_STORE     y [rows, out] = fp16(x W^T)                      (qkv)
 *   SV2_EPI_RESIDUAL  y [rows, out] = fp16((fp16(x W^T) + bias) * gate
 *                     + residual), bias and gate optional (NULL): the
 *                     gated residual after proj_out and mlp_out_proj
 *                     (apply_ada_output_and_residual, :807-825)
 *   SV2_EPI_SWIGLU    y [rows, out] = fp16(silu(g) * u), g = fp16(x W^T),
 *                     u = fp16(x W_value^T): mlp_gate_proj, mlp_in_proj and
 *                     the gate of apply_mlp (:1093-1112)
 * x fp16 [rows, in]; W, W_value fp16 [out, in] row-major (the InnerProduct
 * weight layout); residual fp16 [rows, out]; bias, gate fp32 [out].  Every
 * fp32 step follows the unfused kernels' order.  Requires in % 64 == 0 and
 * out % 256 == 0 (SV2_EPI_SWIGLU: out % 128 == 0); SV2_EUNSUPPORTED
 * otherwise.  x, W, W_value, y and residual must be 16-byte aligned
 * (SV2_EINVAL otherwise).  y may not alias x, W or residual. */
#define SV2_EPI_STORE 0
#define SV2_EPI_RESIDUAL 1
#define SV2_EPI_SWIGLU 2
int sv2_inner_product_f16(const void* x, const void* w, const void* w_value, void* y, int rows, int in, int out,
                          int epilogue, const float* bias, const float* gate, const void* residual, void* stream);

/* ---- The same InnerProducts and fused passes for 1-64 rows (the text
 * branch's tokens: seedvr2_dit_block.cpp:1155-1156, :1180-1181, :1101,
 * :1111 on the text rows), on a weight-streaming kernel: each weight is read
 * once, whole 128-byte lines straight into LDS, K split over workgroups when
 * the output columns alone give too few.  Epilogues as sv2_inner_product_f16;
 * SV2_EPI_STORE also takes an optional bias: y = fp16(fp16(x W^T) + bias).
 * Requires 1 <= rows <= 64, in % 64 == 0 and out % 64 == 0 (SV2_EPI_SWIGLU:
 * out % 32 == 0, no bias or gate); SV2_EUNSUPPORTED otherwise.  When K is
 * split the partial sums go to `workspace` (device memory of at least
 * sv2_inner_product_f16_few_workspace() bytes; 0 bytes: none needed, NULL
 * allowed); they are added in a fixed order, so results do not depend on
 * timing.  Calls that share a workspace must not overlap.  x, W, W_value
 * and the workspace must be 16-byte aligned, y and residual 8-byte aligned
 * (SV2_EINVAL otherwise).  y may not alias x, W, residual or the
 * workspace. */
int64_t sv2_inner_product_f16_few_workspace(int rows, int in, int out, int epilogue);
int sv2_inner_product_f16_few(const void* x, const void* w, const void* w_value, void* y, int rows, int in, int out,
                              int epilogue, const float* bias, const float* gate, const void* residual,
                              void* workspace, size_t workspace_bytes, void* stream);

/* ---- fp32 InnerProduct of the parity mode.  Replaces the block's ncnn
 * InnerProduct layers (load_inner_product, seedvr2_dit_block.cpp:27-55) and
 * the heads' (seedvr2_dit_input.cpp:354-392, seedvr2_dit_output.cpp:388-390)
 * in fp32: y [rows, out] = float(sum_i double(x_i) * double(w_i) + double(b)),
 * the exact products of each output added in increasing i, then the bias
 * (NULL: none), one rounding to float.  x fp32 [rows, in], W fp32 [out, in]
 * row-major, bias fp32 [out].  Any shape; y may not alias x or W. */
int sv2_inner_product_f32(const float* x, const float* w, const float* bias, float* y, int rows, int in, int out,
                          void* stream);

/* ---- Euler sampler (src/model/sampler.h:18-78) and the latent preparation
 * of the engine loop (src/core/engine.cpp:79-149, :306-350).  Latents are
 * fp32 device arrays treated as flat element sequences except where a layout
 * is named.  Every operation evaluates the reference's float expression in
 * the same order without fused multiply-adds, so outputs are bit-identical
 * to the reference's CPU sampler; the guidance rescale factor is formed from
 * double sums in a fixed order and can differ from the reference's by an
 * ulp of the factor. */

/* Host.  The schedule of EulerSampler::EulerSampler (sampler.cpp:181-187):
 * steps <= 0 counts as 1; out[i] = 1000 * (1 - i / steps).  `out` holds
 * max(1, steps) floats; returns that count, or SV2_EINVAL. */
int sv2_euler_timesteps(int steps, float* out);
/* Host.  The condition noise ratio of make_condition_latent (engine.cpp:79-92
 * and :110): transformed_condition_timestep(noise_scale) / 1000 for an
 * encoded latent of frames x height x width. */
float sv2_condition_ratio(float noise_scale, int frames, int height, int width);
/* out = (1 - ratio) * encoded + ratio * noise, elementwise over `count`
 * floats (make_condition_latent, engine.cpp:106-122;
 * EulerSampler::make_condition_vulkan, sampler.h:45-51). */
int sv2_make_condition(const float* encoded, const float* noise, float* out, int64_t count, float ratio,
                       void* stream);
/* The 33-channel DiT input: channels 0-15 the latent, 16-31 the condition,
 * 32 ones.  channel_major != 0: [16][tokens] sources, [33][tokens] output
 * (make_dit_input, engine.cpp:125-149); 0: [tokens][16] sources,
 * [tokens][33] output (EulerSampler::make_dit_input_vulkan,
 * sampler.cpp:337-357). */
int sv2_make_dit_input(const float* latent, const float* condition, float* out, int64_t tokens, int channel_major,
                       void* stream);
/* Workspace bytes of sv2_apply_cfg with a non-zero rescale (a few KiB). */
int64_t sv2_cfg_workspace_size(int64_t count);
/* Classifier-free guidance (EulerSampler::apply_cfg, sampler.cpp:201-236;
 * apply_cfg_vulkan, sampler.h:58-65): out = neg + scale * (pos - neg); when
 * rescale != 0 and the unbiased standard deviation of out is positive, out is
 * multiplied by float(rescale * std(pos) / std(out) + (1 - rescale)).  The
 * statistics are reduced on the device (no host synchronisation); the
 * workspace is needed only when rescale != 0.  `out` may alias either
 * input (each element is read before it is written, by the same thread). */
int sv2_apply_cfg(const float* positive, const float* negative, float* out, int64_t count, float scale,
                  float rescale, void* workspace, size_t workspace_bytes, void* stream);
/* The Euler / v-lerp update (EulerSampler::step_to, sampler.cpp:239-265):
 * with bt = t / 1000, at = 1 - bt, bs = clamp(t_next / 1000, 0, 1),
 * as = 1 - bs: out = as * (x - bt * pred) + bs * (x + at * pred). */
int sv2_euler_step(const float* prediction, const float* current, float* out, int64_t count, float timestep,
                   float next_timestep, void* stream);
/* The last step (EulerSampler::endpoint, sampler.cpp:267-285):
 * out = x - (t / 1000) * pred. */
int sv2_euler_endpoint(const float* prediction, const float* current, float* out, int64_t count, float timestep,
                       void* stream);

/* Message of the last failure on the calling thread (never NULL). */
/* ------------------------------------------------------------------------
 * Model integrity (scripts/verify-models.sh:17-24; download-models.sh:
 * 93-97, :140-148).  Host only.
 * ------------------------------------------------------------------------ */

/* SHA-256 (FIPS 180-4) of `bytes` bytes at `data` into digest[32]. */
int sv2_sha256(const void* data, size_t bytes, unsigned char digest[32]);

/* SHA-256 of a whole file. */
int sv2_sha256_file(const char* path, unsigned char digest[32]);

/* `sha256sum --check --strict SHA256SUMS` in `dir`: parses the manifest
 * (lines "<64 hex digits> <name>" or "<digest> *<name>"; blank lines skipped;
 * names must not be empty, start with '.' or contain '/'; no extra fields)
 * and hashes every listed file on `threads` threads (<= 0: up to 16).
 * Returns the number of files verified, 0 when `dir` has no SHA256SUMS, or
 * SV2_EINVAL for a malformed manifest, a listed file that is missing, or a
 * digest that does not match (sv2_last_error names the line or file). */
int sv2_verify_checksums(const char* dir, int threads);

/* sv2_verify_checksums, but a directory without a non-empty SHA256SUMS fails
 * with SV2_EINVAL, as scripts/verify-models.sh:22 fails a component without
 * one.  A file that cannot be hashed for lack of host memory gives
 * SV2_EDEVICE (both functions). */
int sv2_verify_checksums_strict(const char* dir, int threads);

/* scripts/verify-models.sh for the parts this library loads: under
 * `model_root`, default_pos_emb.bin and default_neg_emb.bin present and, when
 * `bundled_embeddings` is not NULL, byte-identical to the copies in that
 * directory (:27-31); dit_full_fp16/SHA256SUMS required and every listed file
 * intact (:33-34); all 68 files of the DiT present and non-empty (:36-47).
 * The VAE component is not checked (the library has no VAE).  Returns the
 * number of DiT files hashed, or a negative error code naming the file. */
int sv2_verify_model_set(const char* model_root, const char* bundled_embeddings, int threads);

const char* sv2_last_error(void);

/* Library version string. */
const char* sv2_version(void);

#ifdef __cplusplus
}
#endif

#endif
