/*
 * refcpu — CPU oracle for the SeedVR2 DiT windowed multimodal attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference
 * SeedVR2DiTBlock fp32 CPU layer (src/layers/seedvr2_dit_block.cpp:58-79,
 * :643-688, :770-1267 of czwdysj/seedvr2-ncnn-valkan).  It is the checker the
 * parity tests, the smoke check and the CPU-baseline leg of the benchmark
 * compare the HIP path against.  Nothing in the product links or calls it.
 *
 * Each function cites the reference lines it follows.  Arithmetic follows the
 * reference op for op: double accumulations where the reference uses double,
 * float casts at the same points, bf16 round-to-nearest-even at the same
 * points, window order w -> h -> t, text outputs averaged over windows in
 * window order.  Build with -ffp-contract=off so no multiply-add is fused
 * (the reference is built for baseline x86-64, which has no FMA).
 *
 * exp: the reference calls std::exp on floats (softmax :1059, silu :58-61),
 * i.e. the platform libm's expf, whose last bit depends on the libm (glibc
 * 2.35's expf differs from the correctly rounded value for 6.3e-4 of the
 * arguments in [-32, 8], by one ulp).  The oracle evaluates the correctly
 * rounded value, orc_expf(x) = (float)exp((double)x), the libm-independent
 * result every conforming expf approximates; it is pinned against float64
 * numpy and against the host libm's expf (at most one ulp apart).
 *
 * Pinning status (what checks each function beyond its own formula):
 *   orc_bf16            exhaustive-by-class test against torch's bfloat16 cast
 *   orc_make_windows    hand-derived known-answer plans, partition invariants,
 *                       exact-rational brute force over small grids
 *   orc_window_attention textbook softmax attention in float64 on tiny shapes,
 *                       S=1 / identical-key / one-hot special cases, RoPE as
 *                       complex rotation, norm preservation, window-masked
 *                       global attention formulation
 *   orc_rmsnorm_rows, orc_ada_input, orc_ada_output_residual, orc_swiglu
 *                       closed forms in float64 numpy
 *   orc_inner_product   y = W x + b in float64 (summation order of ncnn's
 *                       InnerProduct is not available here: parity unpinned
 *                       for GEMM summation order, values pinned by closed form)
 *   orc_block_forward   a float64 numpy statement of the block from the model's
 *                       definitions with its own window plan, on weights
 *                       designed so that a wrong branch, modulation slot or
 *                       residual source fails (each planted and shown to
 *                       fail); the algebra's identities bit for bit (W_out = 0
 *                       leaves the gated projection plus the input; zero
 *                       projections return the inputs); one window over the
 *                       grid equals global joint attention
 *   dit_forward (oracle.py) input head -> blocks -> output head against the
 *                       same numpy statement with numpy heads
 *   orc_dit_input_forward, orc_dit_output_forward
 *                       patchify / unpatchify against an einops-style numpy
 *                       reshape, the sinusoid and time MLP against a float64
 *                       numpy evaluation, timestep 0 special case, identity
 *                       projections that expose the permutations exactly
 *   orc_euler_timesteps, orc_make_condition, orc_make_dit_input,
 *   orc_apply_cfg, orc_euler_step, orc_euler_endpoint, orc_condition_ratio
 *                       the reference's own known answers (runtime_unit_test
 *                       CFG 3.0 and endpoint 0.75; sampler_vulkan_runner's
 *                       condition, 33-channel layout, CFG 2.5/0.4 and step
 *                       1000->500 cases), float64 closed forms, numpy std
 *                       with ddof=1, and identities (scale 1 gives pos,
 *                       rescale 1 matches std(pos), endpoint = step to 0,
 *                       step to t gives x, the ratio at 1280x720x145 is
 *                       5t/(1+4t), at 256x256x37 it is t)
 */
#ifndef SEEDVR2_REFCPU_H
#define SEEDVR2_REFCPU_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct orc_window {
    int t0, t1, h0, h1, w0, w1;
} orc_window;

/* RoPE variants. */
enum {
    ORC_ROPE_REFERENCE = 0, /* 3 axes x 21 adjacent pairs, window-local positions, text rotated at (l,l,l) */
    ORC_ROPE_ABSOLUTE = 1,  /* head_dim split 32/48/48 over t/h/w, absolute grid positions, text not rotated */
    ORC_ROPE_NONE = 2
};

/* bf16 round-to-nearest-even kept in an fp32 container (seedvr2_dit_block.cpp:68-79). */
float orc_bf16(float value);

/* std::exp of a float, correctly rounded: (float)exp((double)x). */
float orc_expf(float x);

/* orc_bf16 over an array (for exhaustive tests of the rounding rule). */
void orc_bf16_array(const float* in, float* out, int64_t count);

/* Adaptive window size rule (seedvr2_dit_block.cpp:832-838). */
void orc_adaptive_window(int T, int H, int W, int* wt, int* wh, int* ww);

/* Window plan (seedvr2_dit_block.cpp:827-868).  wt/wh/ww == 0 selects the
 * reference adaptive size on that axis.  Returns the number of windows, or
 * -1 if it exceeds cap (out may be NULL with cap 0 to query the count). */
int orc_make_windows(int T, int H, int W, int shifted, int wt, int wh, int ww,
                     orc_window* out, int cap);

typedef struct orc_attn_cfg {
    int heads;
    int head_dim;
    float eps;
    int qk_norm;            /* 1: per-head RMSNorm * gamma on q and k (reference); 0: none */
    int rope_mode;          /* ORC_ROPE_* */
    const float* freqs;     /* [21] rope frequencies (reference mode) */
    float rope_theta;       /* absolute mode */
    const float* gq_vid;    /* [head_dim] norm_q of the video branch */
    const float* gk_vid;
    const float* gq_txt;    /* [head_dim] norm_q of the text branch (vid branch if shared) */
    const float* gk_txt;
    int shifted;
    int wt, wh, ww;         /* 0 = adaptive */
    int threads;            /* OpenMP threads over heads; <= 0 uses the default */
} orc_attn_cfg;

/* Windowed joint video+text attention (seedvr2_dit_block.cpp:870-1091).
 * vid_qkv [Lv, 3D] and txt_qkv [Lt, 3D] rows, q at column h*hd, k at D+h*hd,
 * v at 2D+h*hd.  Outputs vid_out [Lv, D], txt_out [Lt, D].
 * Optional captures (NULL to skip), each [sum_w S_w, D] in window-sequence
 * order (video tokens t->y->x, then text): q/k/v after the prologue, and the
 * attention output before its bf16 rounding.
 * video_mask (optional, [nW]): video queries of window w are evaluated only if
 * video_mask[w] != 0 (text queries always are, since the text output averages
 * over every window); skipped video rows of vid_out are left untouched.
 * Returns 0, or -1 on a shape mismatch. */
int orc_window_attention(const orc_attn_cfg* cfg, int T, int H, int W, int Lt,
                         const float* vid_qkv, const float* txt_qkv,
                         float* vid_out, float* txt_out,
                         float* cap_q, float* cap_k, float* cap_v, float* cap_pre,
                         const unsigned char* video_mask);

/* q and k of every head after RMSNorm * gamma, before RoPE: the reference's
 * norm_q/k_vid (grid row order) and norm_q/k_txt debug captures
 * (seedvr2_dit_block.h:20-36, :908-918, :989-1016).  Outputs may be NULL. */
int orc_qk_norms(const orc_attn_cfg* cfg, int Lv, int Lt, const float* vid_qkv, const float* txt_qkv,
                 float* nq_vid, float* nk_vid, float* nq_txt, float* nk_txt);

/* Token RMSNorm over the last dim, no gamma (seedvr2_dit_block.cpp:770-782). */
void orc_rmsnorm_rows(float* x, int rows, int dim, float eps);

/* Ada input modulation (seedvr2_dit_block.cpp:784-805); slot_base 0 (attn) or 3 (mlp). */
void orc_ada_input(float* x, int rows, int dim, const float* emb, const float* shift,
                   const float* scale, int slot_base);

/* Gated residual (seedvr2_dit_block.cpp:807-825); gate slot = slot_base + 2. */
void orc_ada_output_residual(float* x, const float* residual, int rows, int dim,
                             const float* emb, const float* gate, int slot_base);

/* SwiGLU gate g <- silu(g) * v (seedvr2_dit_block.cpp:58-61, :1093-1112). */
void orc_swiglu(float* gate, const float* value, int64_t count);

/* ncnn InnerProduct semantics: y[r][o] = b[o] + sum_i W[o][i] * x[r][i],
 * W row-major [out][in].  Accumulated in double. */
void orc_inner_product(const float* x, int rows, int in, const float* weight,
                       const float* bias, int out, float* y, int threads);

typedef struct orc_branch {
    const float* attn_shift;
    const float* attn_scale;
    const float* attn_gate;
    const float* mlp_shift;
    const float* mlp_scale;
    const float* mlp_gate;
    const float* w_qkv;   /* [3D][D] */
    const float* w_proj;  /* [D][D] */
    const float* b_proj;  /* [D] */
    const float* norm_q;  /* [hd] */
    const float* norm_k;  /* [hd] */
    const float* w_gate;  /* [F][D] */
    const float* w_in;    /* [F][D] */
    const float* w_out;   /* [D][F] */
} orc_branch;

typedef struct orc_block {
    int dim, heads, head_dim, mlp_hidden;
    float eps;
    int shared, last_layer, shifted;
    int wt, wh, ww;
    int rope_mode;
    float rope_theta;
    int qk_norm;
    orc_branch vid;
    orc_branch txt;       /* ignored when shared */
    const float* freqs;   /* [21] */
    int threads;
} orc_block;

/* One block forward (seedvr2_dit_block.cpp:1114-1267).  vid [Lv, D], txt [Lt, D],
 * emb [6D].  Returns 0, -1 on invalid shapes, -100 on allocation failure. */
int orc_block_head(const orc_block* blk, const float* vid, int Lv, const float* txt, int Lt, const float* emb,
                   float* qkv_v, float* qkv_t);
int orc_block_attention(const orc_block* blk, int T, int H, int W, int Lt, const float* qkv_v, const float* qkv_t,
                        float* att_v, float* att_t);
int orc_block_tail(const orc_block* blk, const float* att_v, int Lv, const float* att_t, int Lt, const float* vid,
                   const float* txt, const float* emb, float* vid_out, float* txt_out, float* proj_v, float* proj_t);
int orc_block_forward(const orc_block* blk, const float* vid, int Lv, const float* txt, int Lt,
                      const float* emb, int T, int H, int W, float* vid_out, float* txt_out);

/* The DiT input head (seedvr2_dit_input.cpp:311-403).  Matrices [out][in]. */
typedef struct orc_dit_input {
    int dim, video_channels, text_channels, sinusoidal_dim, embedding_dim;
    const float *w_vid, *b_vid, *w_txt, *b_txt;
    const float *w_tin, *b_tin, *w_thid, *b_thid, *w_tout, *b_tout;
    int threads;
} orc_dit_input;

/* video [T*H*W, video_channels] token-major, text [L, text_channels];
 * writes vid_out [T*(H/2)*(W/2), dim], txt_out [L, dim], emb [embedding_dim].
 * Returns -1 for an odd H or W or a bad config (:317-330). */
int orc_dit_input_forward(const orc_dit_input* in, const float* video, const float* text, int L, float timestep,
                          int T, int H, int W, float* vid_out, float* txt_out, float* emb);

/* The DiT output head (seedvr2_dit_output.cpp:349-428). */
typedef struct orc_dit_output {
    int dim, output_channels;
    float eps;
    const float *norm, *shift, *scale, *w_proj, *b_proj;
    int threads;
} orc_dit_output;

/* vid [T*h*w, dim], emb [6*dim]; writes out [T*2h*2w, output_channels]
 * token-major. */
int orc_dit_output_forward(const orc_dit_output* o, const float* vid, const float* emb, int T, int h, int w,
                           float* out);

/* ---- Euler sampler and latent preparation (src/model/sampler.cpp:27-62,
 * :181-285; src/core/engine.cpp:79-149).  Latents are flat fp32 arrays in
 * the reference's [C][T][H][W] order unless a layout is named. */

/* Timesteps of EulerSampler(steps) (sampler.cpp:181-187); returns the count. */
int orc_euler_timesteps(int steps, float* out);
/* transformed_condition_timestep(noise_scale, latent) / 1000
 * (engine.cpp:79-92, :110) for a T x H x W latent. */
float orc_condition_ratio(float noise_scale, int T, int H, int W);
/* make_condition_latent (engine.cpp:106-122). */
void orc_make_condition(const float* encoded, const float* noise, float* out, int64_t count, float ratio);
/* make_dit_input (engine.cpp:125-149), channel-major, or the token-major
 * [tokens][33] layout of make_dit_input_vulkan (sampler.cpp:337-357). */
void orc_make_dit_input(const float* latent, const float* condition, float* out, int64_t tokens, int channel_major);
/* standard_deviation (sampler.cpp:41-62): double sums in element order. */
double orc_standard_deviation(const float* x, int64_t count);
/* EulerSampler::apply_cfg (sampler.cpp:201-236). */
void orc_apply_cfg(const float* pos, const float* neg, float* out, int64_t count, float scale, float rescale);
/* EulerSampler::step_to (sampler.cpp:239-265). */
void orc_euler_step(const float* pred, const float* x, float* out, int64_t count, float t, float t_next);
/* EulerSampler::endpoint (sampler.cpp:267-285). */
void orc_euler_endpoint(const float* pred, const float* x, float* out, int64_t count, float t);

#ifdef __cplusplus
}
#endif

#endif
