/*
 * refcpu.c — CPU oracle (test infrastructure only; see refcpu.h).
 *
 * Restates the reference SeedVR2DiTBlock fp32 CPU path
 * (czwdysj/seedvr2-ncnn-valkan, src/layers/seedvr2_dit_block.cpp).
 * Compile with -ffp-contract=off and without -march flags that enable FMA.
 */
#include "refcpu.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* seedvr2_dit_block.cpp:68-79 — add 0x7fff plus the lowest kept bit, then
 * clear the low half: round to nearest, ties to even, on the raw bits. */
float orc_bf16(float value)
{
    uint32_t bits;
    memcpy(&bits, &value, sizeof(bits));
    bits += 0x7fffu + ((bits >> 16) & 1u);
    bits &= 0xffff0000u;
    memcpy(&value, &bits, sizeof(value));
    return value;
}

/* The reference's std::exp(float) (seedvr2_dit_block.cpp:58-61, :1059),
 * correctly rounded: exp in double (error well below 2^-29 of the float
 * rounding step) rounded once to float. */
float orc_expf(float x)
{
    return (float)exp((double)x);
}

void orc_bf16_array(const float* in, float* out, int64_t count)
{
    for (int64_t i = 0; i < count; i++)
        out[i] = orc_bf16(in[i]);
}

static int ceil_div_i(int value, int divisor) { return (value + divisor - 1) / divisor; }
static int min_i(int a, int b) { return a < b ? a : b; }
static int max_i(int a, int b) { return a > b ? a : b; }

/* seedvr2_dit_block.cpp:832-838: about 3600 latent pixels per window group,
 * three windows per spatial axis, frames grouped by four (capped at 30). */
void orc_adaptive_window(int T, int H, int W, int* wt, int* wh, int* ww)
{
    const double scale = sqrt(3600.0 / (double)(H * W));
    const int resized_h = (int)nearbyint(H * scale); /* ties-to-even in the default mode */
    const int resized_w = (int)nearbyint(W * scale);
    *wh = ceil_div_i(resized_h, 3);
    *ww = ceil_div_i(resized_w, 3);
    *wt = ceil_div_i(min_i(T, 30), 4);
}

/* seedvr2_dit_block.cpp:840-866 — half-window shift only on axes whose window
 * is smaller than the extent; truncating casts; empty windows skipped; loop
 * order w (outer) -> h -> t (inner). */
int orc_make_windows(int T, int H, int W, int shifted, int wt, int wh, int ww,
                     orc_window* out, int cap)
{
    int at, ah, aw;
    orc_adaptive_window(T, H, W, &at, &ah, &aw);
    const int window_frames = wt > 0 ? wt : at;
    const int window_height = wh > 0 ? wh : ah;
    const int window_width = ww > 0 ? ww : aw;

    const double shift_t = shifted && window_frames < T ? 0.5 : 0.0;
    const double shift_h = shifted && window_height < H ? 0.5 : 0.0;
    const double shift_w = shifted && window_width < W ? 0.5 : 0.0;
    const int count_t = shifted ? (shift_t > 0.0 ? (int)ceil((T - shift_t) / window_frames) + 1 : 1)
                                : ceil_div_i(T, window_frames);
    const int count_h = shifted ? (shift_h > 0.0 ? (int)ceil((H - shift_h) / window_height) + 1 : 1)
                                : ceil_div_i(H, window_height);
    const int count_w = shifted ? (shift_w > 0.0 ? (int)ceil((W - shift_w) / window_width) + 1 : 1)
                                : ceil_div_i(W, window_width);

    int n = 0;
    for (int iw = 0; iw < count_w; iw++)
        for (int ih = 0; ih < count_h; ih++)
            for (int it = 0; it < count_t; it++)
            {
                const int t0 = max_i((int)((it - shift_t) * window_frames), 0);
                const int t1 = min_i((int)((it - shift_t + 1.0) * window_frames), T);
                const int h0 = max_i((int)((ih - shift_h) * window_height), 0);
                const int h1 = min_i((int)((ih - shift_h + 1.0) * window_height), H);
                const int w0 = max_i((int)((iw - shift_w) * window_width), 0);
                const int w1 = min_i((int)((iw - shift_w + 1.0) * window_width), W);
                if (t1 > t0 && h1 > h0 && w1 > w0)
                {
                    if (out)
                    {
                        if (n >= cap)
                            return -1;
                        out[n].t0 = t0; out[n].t1 = t1;
                        out[n].h0 = h0; out[n].h1 = h1;
                        out[n].w0 = w0; out[n].w1 = w1;
                    }
                    n++;
                }
            }
    return n;
}

/* Rotation layout of one RoPE variant: per axis, the first dim, the pair
 * count and the frequency of each pair. */
typedef struct rope_layout {
    int offset[3];
    int pairs[3];
    float freq[3][64];
} rope_layout;

static void make_rope_layout(const orc_attn_cfg* cfg, rope_layout* r)
{
    memset(r, 0, sizeof(*r));
    if (cfg->rope_mode == ORC_ROPE_REFERENCE)
    {
        /* seedvr2_dit_block.cpp:956-971: 3 axes x 21 adjacent pairs, dims 0..125 */
        for (int a = 0; a < 3; a++)
        {
            r->offset[a] = a * 42;
            r->pairs[a] = 21;
            for (int p = 0; p < 21; p++)
                r->freq[a][p] = cfg->freqs[p];
        }
    }
    else if (cfg->rope_mode == ORC_ROPE_ABSOLUTE)
    {
        /* head_dim split 32/48/48 over t/h/w, freq_i = theta^(-2i/d_axis) */
        const int dims[3] = {32, 48, 48};
        int off = 0;
        for (int a = 0; a < 3; a++)
        {
            r->offset[a] = off;
            r->pairs[a] = dims[a] / 2;
            for (int p = 0; p < dims[a] / 2; p++)
                r->freq[a][p] = (float)(1.0 / pow((double)cfg->rope_theta, (2.0 * p) / dims[a]));
            off += dims[a];
        }
    }
}

/* The per-head RMSNorm * gamma step of normalize_and_rotate
 * (seedvr2_dit_block.cpp:947-951): a double sum, float mean, then x * inv * g.
 * Without the q/k norm the values pass through. */
static void normalize_head(const float* source, const float* gamma, float* destination, int head_dim, float eps,
                           int qk_norm)
{
    if (qk_norm)
    {
        double square_sum = 0.0;
        for (int d = 0; d < head_dim; d++)
            square_sum += (double)source[d] * source[d];
        const float inverse_rms = 1.f / sqrtf((float)(square_sum / head_dim) + eps);
        for (int d = 0; d < head_dim; d++)
            destination[d] = source[d] * inverse_rms * gamma[d];
    }
    else
    {
        for (int d = 0; d < head_dim; d++)
            destination[d] = source[d];
    }
}

/* seedvr2_dit_block.cpp:942-974 (normalize_and_rotate): per-head RMSNorm with
 * a double sum, gamma, adjacent-pair rotation, then bf16 of every dim. */
static void normalize_and_rotate(const float* source, const float* gamma, float* destination,
                                 int head_dim, float eps, int qk_norm, const rope_layout* rope,
                                 int rotate, const int positions[3])
{
    normalize_head(source, gamma, destination, head_dim, eps, qk_norm);
    if (rotate)
    {
        for (int axis = 0; axis < 3; axis++)
            for (int pair = 0; pair < rope->pairs[axis]; pair++)
            {
                const int d = rope->offset[axis] + pair * 2;
                const float angle = (float)positions[axis] * rope->freq[axis][pair];
                const float cosine = cosf(angle);
                const float sine = sinf(angle);
                const float first = destination[d];
                const float second = destination[d + 1];
                destination[d] = first * cosine - second * sine;
                destination[d + 1] = second * cosine + first * sine;
            }
    }
    for (int d = 0; d < head_dim; d++)
        destination[d] = orc_bf16(destination[d]);
}

/* The debug captures norm_q/k_vid and norm_q/k_txt of the reference
 * (seedvr2_dit_block.h:20-36, filled at :908-918 and :989-1016): q and k of
 * every head after RMSNorm * gamma and before RoPE, video rows in grid order
 * [Lv][dim], text rows [Lt][dim]; any output may be NULL. */
int orc_qk_norms(const orc_attn_cfg* cfg, int Lv, int Lt, const float* vid_qkv, const float* txt_qkv,
                 float* nq_vid, float* nk_vid, float* nq_txt, float* nk_txt)
{
    const int hd = cfg->head_dim;
    const int dim = cfg->heads * hd;
    if (Lv < 0 || Lt < 0)
        return -1;
    for (int head = 0; head < cfg->heads; head++)
    {
        for (int r = 0; r < Lv; r++)
        {
            const float* row = vid_qkv + (size_t)r * 3 * dim;
            if (nq_vid)
                normalize_head(row + head * hd, cfg->gq_vid, nq_vid + (size_t)r * dim + head * hd, hd, cfg->eps,
                               cfg->qk_norm);
            if (nk_vid)
                normalize_head(row + dim + head * hd, cfg->gk_vid, nk_vid + (size_t)r * dim + head * hd, hd,
                               cfg->eps, cfg->qk_norm);
        }
        for (int l = 0; l < Lt; l++)
        {
            const float* row = txt_qkv + (size_t)l * 3 * dim;
            if (nq_txt)
                normalize_head(row + head * hd, cfg->gq_txt, nq_txt + (size_t)l * dim + head * hd, hd, cfg->eps,
                               cfg->qk_norm);
            if (nk_txt)
                normalize_head(row + dim + head * hd, cfg->gk_txt, nk_txt + (size_t)l * dim + head * hd, hd,
                               cfg->eps, cfg->qk_norm);
        }
    }
    return 0;
}

/* seedvr2_dit_block.cpp:870-1091 */
int orc_window_attention(const orc_attn_cfg* cfg, int T, int H, int W, int Lt,
                         const float* vid_qkv, const float* txt_qkv,
                         float* vid_out, float* txt_out,
                         float* cap_q, float* cap_k, float* cap_v, float* cap_pre,
                         const unsigned char* video_mask)
{
    const int heads = cfg->heads;
    const int hd = cfg->head_dim;
    const int dim = heads * hd;
    const int Lv = T * H * W;
    if (T <= 0 || H <= 0 || W <= 0 || Lt < 0)
        return -1;
    if (cfg->rope_mode == ORC_ROPE_REFERENCE && hd < 126)
        return -1;
    if (cfg->rope_mode == ORC_ROPE_ABSOLUTE && hd != 128)
        return -1;

    const int nw = orc_make_windows(T, H, W, cfg->shifted, cfg->wt, cfg->wh, cfg->ww, NULL, 0);
    if (nw <= 0)
        return -1;
    orc_window* windows = (orc_window*)malloc(sizeof(orc_window) * (size_t)nw);
    int* seq_off = (int*)malloc(sizeof(int) * (size_t)nw);
    if (!windows || !seq_off)
    {
        free(windows);
        free(seq_off);
        return -100;
    }
    orc_make_windows(T, H, W, cfg->shifted, cfg->wt, cfg->wh, cfg->ww, windows, nw);
    int total_seq = 0;
    int max_seq = 0;
    for (int i = 0; i < nw; i++)
    {
        const orc_window* w = &windows[i];
        const int s = (w->t1 - w->t0) * (w->h1 - w->h0) * (w->w1 - w->w0) + Lt;
        seq_off[i] = total_seq;
        total_seq += s;
        if (s > max_seq)
            max_seq = s;
    }

    /* reference fills both outputs with zeros (:894-895) before accumulating */
    for (int i = 0; i < nw; i++)
    {
        if (video_mask && !video_mask[i])
            continue;
        const orc_window* w = &windows[i];
        for (int t = w->t0; t < w->t1; t++)
            for (int y = w->h0; y < w->h1; y++)
                memset(vid_out + ((size_t)(t * H + y) * W + w->w0) * dim, 0,
                       sizeof(float) * (size_t)(w->w1 - w->w0) * dim);
    }
    (void)Lv;

    rope_layout rope;
    make_rope_layout(cfg, &rope);
    const int rotate_video = cfg->rope_mode != ORC_ROPE_NONE;
    const int rotate_text = cfg->rope_mode == ORC_ROPE_REFERENCE;
    const float attention_scale = 1.f / sqrtf((float)hd);
    const float inverse_window_count = 1.f / (float)nw;
    int failed = 0;

#ifdef _OPENMP
    const int nt = cfg->threads > 0 ? cfg->threads : omp_get_max_threads();
#pragma omp parallel for num_threads(nt) schedule(dynamic, 1)
#endif
    for (int head = 0; head < heads; head++)
    {
        float* text_acc = (float*)calloc((size_t)(Lt > 0 ? Lt : 1) * hd, sizeof(float));
        float* q = (float*)malloc(sizeof(float) * (size_t)max_seq * hd);
        float* k = (float*)malloc(sizeof(float) * (size_t)max_seq * hd);
        float* v = (float*)malloc(sizeof(float) * (size_t)max_seq * hd);
        float* scores = (float*)malloc(sizeof(float) * (size_t)max_seq);
        int* video_index = (int*)malloc(sizeof(int) * (size_t)max_seq);
        double* acc = (double*)malloc(sizeof(double) * (size_t)hd);
        if (!text_acc || !q || !k || !v || !scores || !video_index || !acc)
        {
#ifdef _OPENMP
#pragma omp atomic write
#endif
            failed = 1;
        }
        else
        {
            for (int wi = 0; wi < nw; wi++)
            {
                const orc_window* w = &windows[wi];
                const int video_length = (w->t1 - w->t0) * (w->h1 - w->h0) * (w->w1 - w->w0);
                const int seq = video_length + Lt;
                const int do_video = !video_mask || video_mask[wi];

                /* gather: video tokens t -> y -> x, row (t*H+y)*W+x (:976-1003) */
                int token = 0;
                for (int t = w->t0; t < w->t1; t++)
                    for (int y = w->h0; y < w->h1; y++)
                        for (int x = w->w0; x < w->w1; x++, token++)
                        {
                            const int index = (t * H + y) * W + x;
                            video_index[token] = index;
                            const float* row = vid_qkv + (size_t)index * 3 * dim;
                            int pos[3];
                            if (cfg->rope_mode == ORC_ROPE_ABSOLUTE)
                            {
                                pos[0] = t; pos[1] = y; pos[2] = x;
                            }
                            else
                            {
                                pos[0] = Lt + (t - w->t0); pos[1] = y - w->h0; pos[2] = x - w->w0;
                            }
                            normalize_and_rotate(row + head * hd, cfg->gq_vid, q + (size_t)token * hd,
                                                 hd, cfg->eps, cfg->qk_norm, &rope, rotate_video, pos);
                            normalize_and_rotate(row + dim + head * hd, cfg->gk_vid, k + (size_t)token * hd,
                                                 hd, cfg->eps, cfg->qk_norm, &rope, rotate_video, pos);
                            const float* vs = row + 2 * dim + head * hd;
                            float* vd = v + (size_t)token * hd;
                            for (int d = 0; d < hd; d++)
                                vd[d] = orc_bf16(vs[d]);
                        }
                /* text tokens appended after the video tokens (:1004-1028) */
                for (int l = 0; l < Lt; l++, token++)
                {
                    const float* row = txt_qkv + (size_t)l * 3 * dim;
                    const int pos[3] = {l, l, l};
                    normalize_and_rotate(row + head * hd, cfg->gq_txt, q + (size_t)token * hd,
                                         hd, cfg->eps, cfg->qk_norm, &rope, rotate_text, pos);
                    normalize_and_rotate(row + dim + head * hd, cfg->gk_txt, k + (size_t)token * hd,
                                         hd, cfg->eps, cfg->qk_norm, &rope, rotate_text, pos);
                    const float* vs = row + 2 * dim + head * hd;
                    float* vd = v + (size_t)token * hd;
                    for (int d = 0; d < hd; d++)
                        vd[d] = orc_bf16(vs[d]);
                }

                if (cap_q || cap_k || cap_v)
                    for (int s = 0; s < seq; s++)
                    {
                        const size_t dst = (size_t)(seq_off[wi] + s) * dim + (size_t)head * hd;
                        if (cap_q) memcpy(cap_q + dst, q + (size_t)s * hd, sizeof(float) * hd);
                        if (cap_k) memcpy(cap_k + dst, k + (size_t)s * hd, sizeof(float) * hd);
                        if (cap_v) memcpy(cap_v + dst, v + (size_t)s * hd, sizeof(float) * hd);
                    }

                /* attention core (:1045-1079) */
                for (int query = do_video ? 0 : video_length; query < seq; query++)
                {
                    const float* qd = q + (size_t)query * hd;
                    float maximum = -INFINITY;
                    for (int key = 0; key < seq; key++)
                    {
                        const float* kd = k + (size_t)key * hd;
                        double dot = 0.0;
                        for (int d = 0; d < hd; d++)
                            dot += (double)qd[d] * kd[d];
                        scores[key] = (float)dot * attention_scale;
                        if (scores[key] > maximum)
                            maximum = scores[key];
                    }
                    float denominator = 0.f;
                    for (int key = 0; key < seq; key++)
                    {
                        scores[key] = orc_expf(scores[key] - maximum);
                        denominator += scores[key];
                    }
                    /* per output dim the sum runs over keys in key order, exactly
                     * as the reference's d-outer / key-inner loop; only the loop
                     * nest is swapped so V is read contiguously */
                    for (int d = 0; d < hd; d++)
                        acc[d] = 0.0;
                    for (int key = 0; key < seq; key++)
                    {
                        const double p = (double)(scores[key] / denominator);
                        const float* vd = v + (size_t)key * hd;
                        for (int d = 0; d < hd; d++)
                            acc[d] += p * vd[d];
                    }
                    float* destination;
                    if (query < video_length)
                        destination = vid_out + (size_t)video_index[query] * dim + (size_t)head * hd;
                    else
                        destination = text_acc + (size_t)(query - video_length) * hd;
                    for (int d = 0; d < hd; d++)
                    {
                        const float pre = (float)acc[d];
                        destination[d] += orc_bf16(pre);
                        if (cap_pre)
                            cap_pre[(size_t)(seq_off[wi] + query) * dim + (size_t)head * hd + d] = pre;
                    }
                }
            }
            /* text average over windows (:1081-1088) */
            for (int l = 0; l < Lt; l++)
                for (int d = 0; d < hd; d++)
                    txt_out[(size_t)l * dim + (size_t)head * hd + d] = text_acc[(size_t)l * hd + d] * inverse_window_count;
        }
        free(text_acc);
        free(q);
        free(k);
        free(v);
        free(scores);
        free(video_index);
        free(acc);
    }
    free(windows);
    free(seq_off);
    return failed ? -100 : 0;
}

/* seedvr2_dit_block.cpp:770-782 */
void orc_rmsnorm_rows(float* x, int rows, int dim, float eps)
{
    for (int r = 0; r < rows; r++)
    {
        float* data = x + (size_t)r * dim;
        double square_sum = 0.0;
        for (int c = 0; c < dim; c++)
            square_sum += (double)data[c] * data[c];
        const float inverse_rms = 1.f / sqrtf((float)(square_sum / dim) + eps);
        for (int c = 0; c < dim; c++)
            data[c] *= inverse_rms;
    }
}

/* seedvr2_dit_block.cpp:784-805: x*(emb[c*6+slot+1]+scale) + emb[c*6+slot] + shift */
void orc_ada_input(float* x, int rows, int dim, const float* emb, const float* shift,
                   const float* scale, int slot_base)
{
    for (int r = 0; r < rows; r++)
    {
        float* data = x + (size_t)r * dim;
        for (int c = 0; c < dim; c++)
        {
            const int offset = c * 6 + slot_base;
            data[c] = data[c] * (emb[offset + 1] + scale[c]) + emb[offset] + shift[c];
        }
    }
}

/* seedvr2_dit_block.cpp:807-825: x*(emb[c*6+slot+2]+gate) + residual */
void orc_ada_output_residual(float* x, const float* residual, int rows, int dim,
                             const float* emb, const float* gate, int slot_base)
{
    const int slot = slot_base + 2;
    for (int r = 0; r < rows; r++)
    {
        float* data = x + (size_t)r * dim;
        const float* skip = residual + (size_t)r * dim;
        for (int c = 0; c < dim; c++)
            data[c] = data[c] * (emb[c * 6 + slot] + gate[c]) + skip[c];
    }
}

/* seedvr2_dit_block.cpp:58-61 and :1103-1109 */
void orc_swiglu(float* gate, const float* value, int64_t count)
{
    for (int64_t i = 0; i < count; i++)
    {
        const float g = gate[i];
        gate[i] = (g / (1.f + orc_expf(-g))) * value[i];
    }
}

/* ncnn InnerProduct (seedvr2_dit_block.cpp:28-56 creates it): W [out][in] row
 * major.  Tiled 4 rows x 8 outputs; every output keeps its own double
 * accumulator summed in input order, so the result equals a plain dot product
 * per output (the tiling only interleaves independent chains). */
void orc_inner_product(const float* x, int rows, int in, const float* weight,
                       const float* bias, int out, float* y, int threads)
{
    enum { RB = 4, OB = 8 };
    const int rb_count = (rows + RB - 1) / RB;
    const int ob_count = (out + OB - 1) / OB;
    const long long tasks = (long long)rb_count * ob_count;
#ifdef _OPENMP
    const int nt = threads > 0 ? threads : omp_get_max_threads();
#pragma omp parallel for num_threads(nt) schedule(static)
#else
    (void)threads;
#endif
    for (long long task = 0; task < tasks; task++)
    {
        const int r0 = (int)(task / ob_count) * RB;
        const int o0 = (int)(task % ob_count) * OB;
        const int rn = rows - r0 < RB ? rows - r0 : RB;
        const int on = out - o0 < OB ? out - o0 : OB;
        double acc[RB][OB];
        const float* xr[RB];
        const float* wr[OB];
        for (int a = 0; a < RB; a++)
        {
            xr[a] = x + (size_t)(r0 + (a < rn ? a : 0)) * in;
            for (int b = 0; b < OB; b++)
                acc[a][b] = 0.0;
        }
        for (int b = 0; b < OB; b++)
            wr[b] = weight + (size_t)(o0 + (b < on ? b : 0)) * in;
        for (int i = 0; i < in; i++)
        {
            double xv[RB];
            for (int a = 0; a < RB; a++)
                xv[a] = xr[a][i];
            for (int b = 0; b < OB; b++)
            {
                const double wv = wr[b][i];
                for (int a = 0; a < RB; a++)
                    acc[a][b] += wv * xv[a];
            }
        }
        for (int a = 0; a < rn; a++)
            for (int b = 0; b < on; b++)
                y[(size_t)(r0 + a) * out + o0 + b] = (float)(acc[a][b] + (bias ? (double)bias[o0 + b] : 0.0));
    }
}

static float* clone_rows(const float* src, size_t count)
{
    float* dst = (float*)malloc(sizeof(float) * (count ? count : 1));
    if (dst && count)
        memcpy(dst, src, sizeof(float) * count);
    return dst;
}

/* seedvr2_dit_block.cpp:1093-1112 */
static int apply_mlp(const orc_block* blk, const orc_branch* br, const float* input, int rows, float* output)
{
    const int D = blk->dim, F = blk->mlp_hidden;
    float* gate = (float*)malloc(sizeof(float) * (size_t)rows * F + 4);
    float* value = (float*)malloc(sizeof(float) * (size_t)rows * F + 4);
    if (!gate || !value)
    {
        free(gate);
        free(value);
        return -100;
    }
    orc_inner_product(input, rows, D, br->w_gate, NULL, F, gate, blk->threads);
    orc_inner_product(input, rows, D, br->w_in, NULL, F, value, blk->threads);
    orc_swiglu(gate, value, (int64_t)rows * F);
    orc_inner_product(gate, rows, F, br->w_out, NULL, D, output, blk->threads);
    free(gate);
    free(value);
    return 0;
}

/* Steps before the attention (seedvr2_dit_block.cpp:1141-1156): token
 * RMSNorm + ada input (text skips the ada on the last layer), then the QKV
 * InnerProducts.  qkv_v [Lv, 3D], qkv_t [Lt, 3D]. */
int orc_block_head(const orc_block* blk, const float* vid, int Lv, const float* txt, int Lt, const float* emb,
                   float* qkv_v, float* qkv_t)
{
    const int D = blk->dim;
    if (blk->heads * blk->head_dim != D || Lv < 0 || Lt < 0)
        return -1;
    const orc_branch* vb = &blk->vid;
    const orc_branch* tb = blk->shared ? &blk->vid : &blk->txt; /* :1139 */
    const size_t nv = (size_t)Lv * D, nt = (size_t)Lt * D;
    float* xa_v = clone_rows(vid, nv);
    float* xa_t = clone_rows(txt, nt);
    if (!xa_v || !xa_t)
    {
        free(xa_v);
        free(xa_t);
        return -100;
    }
    orc_rmsnorm_rows(xa_v, Lv, D, blk->eps);
    orc_rmsnorm_rows(xa_t, Lt, D, blk->eps);
    orc_ada_input(xa_v, Lv, D, emb, vb->attn_shift, vb->attn_scale, 0);
    if (!blk->last_layer)
        orc_ada_input(xa_t, Lt, D, emb, tb->attn_shift, tb->attn_scale, 0);
    orc_inner_product(xa_v, Lv, D, vb->w_qkv, NULL, 3 * D, qkv_v, blk->threads);
    orc_inner_product(xa_t, Lt, D, tb->w_qkv, NULL, 3 * D, qkv_t, blk->threads);
    free(xa_v);
    free(xa_t);
    return 0;
}

/* The block's attention (seedvr2_dit_block.cpp:870-1091) with the block's
 * parameters and the per-branch q/k norm weights. */
int orc_block_attention(const orc_block* blk, int T, int H, int W, int Lt, const float* qkv_v, const float* qkv_t,
                        float* att_v, float* att_t)
{
    const orc_branch* vb = &blk->vid;
    const orc_branch* tb = blk->shared ? &blk->vid : &blk->txt;
    orc_attn_cfg cfg;
    memset(&cfg, 0, sizeof(cfg));
    cfg.heads = blk->heads;
    cfg.head_dim = blk->head_dim;
    cfg.eps = blk->eps;
    cfg.qk_norm = blk->qk_norm;
    cfg.rope_mode = blk->rope_mode;
    cfg.freqs = blk->freqs;
    cfg.rope_theta = blk->rope_theta;
    cfg.gq_vid = vb->norm_q;
    cfg.gk_vid = vb->norm_k;
    cfg.gq_txt = tb->norm_q;
    cfg.gk_txt = tb->norm_k;
    cfg.shifted = blk->shifted;
    cfg.wt = blk->wt;
    cfg.wh = blk->wh;
    cfg.ww = blk->ww;
    cfg.threads = blk->threads;
    return orc_window_attention(&cfg, T, H, W, Lt, qkv_v, qkv_t, att_v, att_t, NULL, NULL, NULL, NULL, NULL);
}

/* Steps after the attention (seedvr2_dit_block.cpp:1180-1260): output
 * projections with bias, gated residuals, the MLPs, and the last layer's
 * text rule.  proj_v / proj_t (optional, may be NULL) receive the projected
 * values before the gate, as the reference's debug capture (:1188-1192). */
int orc_block_tail(const orc_block* blk, const float* att_v, int Lv, const float* att_t, int Lt, const float* vid,
                   const float* txt, const float* emb, float* vid_out, float* txt_out, float* proj_v, float* proj_t)
{
    const int D = blk->dim;
    const orc_branch* vb = &blk->vid;
    const orc_branch* tb = blk->shared ? &blk->vid : &blk->txt;
    const size_t nv = (size_t)Lv * D, nt = (size_t)Lt * D;
    int rc = -100;
    float* p_v = (float*)malloc(sizeof(float) * (nv ? nv : 1));
    float* p_t = (float*)malloc(sizeof(float) * (nt ? nt : 1));
    float* m_in = (float*)malloc(sizeof(float) * (nv > nt ? nv : (nt ? nt : 1)));
    if (!p_v || !p_t || !m_in)
        goto done;

    /* :1180-1209 */
    orc_inner_product(att_v, Lv, D, vb->w_proj, vb->b_proj, D, p_v, blk->threads);
    orc_inner_product(att_t, Lt, D, tb->w_proj, tb->b_proj, D, p_t, blk->threads);
    if (proj_v)
        memcpy(proj_v, p_v, sizeof(float) * nv);
    if (proj_t && nt)
        memcpy(proj_t, p_t, sizeof(float) * nt);
    orc_ada_output_residual(p_v, vid, Lv, D, emb, vb->attn_gate, 0);
    if (!blk->last_layer)
        orc_ada_output_residual(p_t, txt, Lt, D, emb, tb->attn_gate, 0);
    else
        for (size_t i = 0; i < nt; i++)
            p_t[i] += txt[i];

    /* video MLP (:1211-1223) */
    memcpy(m_in, p_v, sizeof(float) * nv);
    orc_rmsnorm_rows(m_in, Lv, D, blk->eps);
    orc_ada_input(m_in, Lv, D, emb, vb->mlp_shift, vb->mlp_scale, 3);
    if (apply_mlp(blk, vb, m_in, Lv, vid_out) != 0)
        goto done;
    orc_ada_output_residual(vid_out, p_v, Lv, D, emb, vb->mlp_gate, 3);

    if (blk->last_layer)
    {
        /* :1225-1246: the text result of the last block is twice txt_proj */
        for (size_t i = 0; i < nt; i++)
            txt_out[i] = p_t[i] * 2.f;
    }
    else if (Lt > 0)
    {
        /* :1248-1260 */
        memcpy(m_in, p_t, sizeof(float) * nt);
        orc_rmsnorm_rows(m_in, Lt, D, blk->eps);
        orc_ada_input(m_in, Lt, D, emb, tb->mlp_shift, tb->mlp_scale, 3);
        if (apply_mlp(blk, tb, m_in, Lt, txt_out) != 0)
            goto done;
        orc_ada_output_residual(txt_out, p_t, Lt, D, emb, tb->mlp_gate, 3);
    }
    rc = 0;
done:
    free(p_v);
    free(p_t);
    free(m_in);
    return rc;
}

/* seedvr2_dit_block.cpp:1114-1267 */
int orc_block_forward(const orc_block* blk, const float* vid, int Lv, const float* txt, int Lt,
                      const float* emb, int T, int H, int W, float* vid_out, float* txt_out)
{
    const int D = blk->dim;
    if (blk->heads * blk->head_dim != D || T * H * W != Lv || Lv <= 0 || Lt < 0)
        return -1;
    const size_t nv = (size_t)Lv * D, nt = (size_t)Lt * D;
    int rc = -100;
    float* qkv_v = (float*)malloc(sizeof(float) * nv * 3);
    float* qkv_t = (float*)malloc(sizeof(float) * (nt ? nt : 1) * 3);
    float* att_v = (float*)malloc(sizeof(float) * nv);
    float* att_t = (float*)malloc(sizeof(float) * (nt ? nt : 1));
    if (!qkv_v || !qkv_t || !att_v || !att_t)
        goto done;
    if ((rc = orc_block_head(blk, vid, Lv, txt, Lt, emb, qkv_v, qkv_t)) != 0)
        goto done;
    rc = orc_block_attention(blk, T, H, W, Lt, qkv_v, qkv_t, att_v, att_t);
    if (rc != 0)
    {
        rc = rc == -1 ? -1 : -100;
        goto done;
    }
    rc = orc_block_tail(blk, att_v, Lv, att_t, Lt, vid, txt, emb, vid_out, txt_out, NULL, NULL);
done:
    free(qkv_v);
    free(qkv_t);
    free(att_v);
    free(att_t);
    return rc;
}

static float silu_f(float v)
{
    return v / (1.f + orc_expf(-v));
}

/* seedvr2_dit_input.cpp:311-403 */
int orc_dit_input_forward(const orc_dit_input* in, const float* video, const float* text, int L, float timestep,
                          int T, int H, int W, float* vid_out, float* txt_out, float* emb)
{
    const int C = in->video_channels, D = in->dim, S = in->sinusoidal_dim;
    if (T <= 0 || H <= 0 || W <= 0 || H % 2 != 0 || W % 2 != 0 || L < 0 || S % 2 != 0 ||
        in->embedding_dim != 6 * D)
        return -1;
    const int h = H / 2, w = W / 2, rows = T * h * w;
    float* patches = (float*)malloc(sizeof(float) * (size_t)rows * 4 * C);
    float* sinus = (float*)malloc(sizeof(float) * (size_t)S);
    float* h1 = (float*)malloc(sizeof(float) * (size_t)D);
    float* h2 = (float*)malloc(sizeof(float) * (size_t)D);
    if (!patches || !sinus || !h1 || !h2)
    {
        free(patches);
        free(sinus);
        free(h1);
        free(h2);
        return -100;
    }
    /* :336-352 patch p = (t, y, x) on the patched grid; its 4 source
     * positions in (dy, dx) order, video_channels values each */
    for (int p = 0; p < rows; p++)
    {
        const int x = p % w, y = (p / w) % h, t = p / (w * h);
        float* dst = patches + (size_t)p * 4 * C;
        for (int dy = 0; dy < 2; dy++)
            for (int dx = 0; dx < 2; dx++)
            {
                const size_t src = ((size_t)(t * H + y * 2 + dy) * W + x * 2 + dx) * C;
                memcpy(dst, video + src, sizeof(float) * C);
                dst += C;
            }
    }
    orc_inner_product(patches, rows, 4 * C, in->w_vid, in->b_vid, D, vid_out, in->threads);
    orc_inner_product(text, L, in->text_channels, in->w_txt, in->b_txt, D, txt_out, in->threads);
    /* :360-392 */
    const int half = S / 2;
    for (int i = 0; i < half; i++)
    {
        const float frequency = expf(-logf(10000.f) * (float)i / (float)half);
        const float value = timestep * frequency;
        sinus[i] = sinf(value);
        sinus[i + half] = cosf(value);
    }
    orc_inner_product(sinus, 1, S, in->w_tin, in->b_tin, D, h1, in->threads);
    for (int i = 0; i < D; i++)
        h1[i] = silu_f(h1[i]);
    orc_inner_product(h1, 1, D, in->w_thid, in->b_thid, D, h2, in->threads);
    for (int i = 0; i < D; i++)
        h2[i] = silu_f(h2[i]);
    orc_inner_product(h2, 1, D, in->w_tout, in->b_tout, in->embedding_dim, emb, in->threads);
    free(patches);
    free(sinus);
    free(h1);
    free(h2);
    return 0;
}

/* seedvr2_dit_output.cpp:349-428 */
int orc_dit_output_forward(const orc_dit_output* o, const float* vid, const float* emb, int T, int h, int w,
                           float* out)
{
    const int D = o->dim, OC = o->output_channels, rows = T * h * w;
    if (T <= 0 || h <= 0 || w <= 0 || D <= 0 || OC <= 0)
        return -1;
    float* normed = (float*)calloc((size_t)rows * D, sizeof(float));
    float* proj = (float*)malloc(sizeof(float) * (size_t)rows * 4 * OC);
    if (!normed || !proj)
    {
        free(normed);
        free(proj);
        return -100;
    }
    for (int r = 0; r < rows; r++)
    {
        const float* x = vid + (size_t)r * D;
        float* y = normed + (size_t)r * D;
        double ss = 0.0;
        for (int c = 0; c < D; c++)
            ss += (double)x[c] * x[c];
        const float inv = 1.f / sqrtf((float)(ss / D) + o->eps);
        for (int c = 0; c < D; c++)
        {
            const float value = x[c] * inv * o->norm[c];
            y[c] = value * (emb[c * 6 + 1] + o->scale[c]) + emb[c * 6] + o->shift[c];
        }
    }
    orc_inner_product(normed, rows, D, o->w_proj, o->b_proj, 4 * OC, proj, o->threads);
    const int H = 2 * h, W = 2 * w;
    for (int p = 0; p < rows; p++)
    {
        const int x = p % w, y = (p / w) % h, t = p / (w * h);
        const float* src = proj + (size_t)p * 4 * OC;
        for (int dy = 0; dy < 2; dy++)
            for (int dx = 0; dx < 2; dx++)
            {
                float* dst = out + ((size_t)(t * H + y * 2 + dy) * W + x * 2 + dx) * OC;
                memcpy(dst, src, sizeof(float) * OC);
                src += OC;
            }
    }
    free(normed);
    free(proj);
    return 0;
}

/* ---- Euler sampler ---------------------------------------------------- */

int orc_euler_timesteps(int steps, float* out)
{
    /* sampler.cpp:181-187 */
    const int n = steps < 1 ? 1 : steps;
    for (int i = 0; i < n; i++)
        out[i] = 1000.0f * (1.0f - (float)i / n);
    return n;
}

float orc_condition_ratio(float noise_scale, int T, int H, int W)
{
    /* engine.cpp:79-92: latent frames/height/width mapped back to pixels */
    const float timestep = noise_scale * 1000.0f;
    if (timestep == 0.0f)
        return 0.0f;
    const float frames = (float)((T - 1) * 4 + 1);
    const float height = (float)(H * 8);
    const float width = (float)(W * 8);
    const float x1 = 256.0f * 256.0f * 37.0f;
    const float x2 = 1280.0f * 720.0f * 145.0f;
    const float shift = 1.0f + (height * width * frames - x1) * (5.0f - 1.0f) / (x2 - x1);
    const float normalized = timestep / 1000.0f;
    const float transformed = 1000.0f * shift * normalized / (1.0f + (shift - 1.0f) * normalized);
    return transformed / 1000.0f; /* engine.cpp:110 */
}

void orc_make_condition(const float* encoded, const float* noise, float* out, int64_t count, float ratio)
{
    /* engine.cpp:117-118 */
    for (int64_t i = 0; i < count; i++)
        out[i] = (1.0f - ratio) * encoded[i] + ratio * noise[i];
}

void orc_make_dit_input(const float* latent, const float* condition, float* out, int64_t tokens, int channel_major)
{
    for (int64_t t = 0; t < tokens; t++)
        for (int c = 0; c < 33; c++)
        {
            float v;
            if (channel_major) /* engine.cpp:127-147 */
                v = c < 16 ? latent[c * tokens + t] : c < 32 ? condition[(c - 16) * tokens + t] : 1.0f;
            else /* [tokens][16] -> [tokens][33] */
                v = c < 16 ? latent[t * 16 + c] : c < 32 ? condition[t * 16 + c - 16] : 1.0f;
            out[channel_major ? c * tokens + t : t * 33 + c] = v;
        }
}

double orc_standard_deviation(const float* x, int64_t count)
{
    /* sampler.cpp:41-62 */
    double sum = 0.0, square_sum = 0.0;
    for (int64_t i = 0; i < count; i++)
    {
        sum += x[i];
        square_sum += (double)x[i] * x[i];
    }
    if (count <= 1)
        return 0.0;
    double variance = (square_sum - sum * sum / count) / (count - 1);
    if (variance < 0.0)
        variance = 0.0;
    return sqrt(variance);
}

void orc_apply_cfg(const float* pos, const float* neg, float* out, int64_t count, float scale, float rescale)
{
    /* sampler.cpp:217-235 */
    for (int64_t i = 0; i < count; i++)
        out[i] = neg[i] + scale * (pos[i] - neg[i]);
    if (rescale == 0.0f)
        return;
    const double cfg_std = orc_standard_deviation(out, count);
    if (!(cfg_std > 0.0))
        return;
    const float factor = (float)(rescale * orc_standard_deviation(pos, count) / cfg_std + (1.0f - rescale));
    for (int64_t i = 0; i < count; i++)
        out[i] *= factor;
}

void orc_euler_step(const float* pred, const float* x, float* out, int64_t count, float t, float t_next)
{
    /* sampler.cpp:253-263 */
    const float bt = t / 1000.0f;
    const float at = 1.0f - bt;
    float bs = t_next / 1000.0f;
    bs = bs < 0.0f ? 0.0f : (bs > 1.0f ? 1.0f : bs);
    const float as = 1.0f - bs;
    for (int64_t i = 0; i < count; i++)
    {
        const float x0 = x[i] - bt * pred[i];
        const float xT = x[i] + at * pred[i];
        out[i] = as * x0 + bs * xT;
    }
}

void orc_euler_endpoint(const float* pred, const float* x, float* out, int64_t count, float t)
{
    /* sampler.cpp:280-282 */
    const float bt = t / 1000.0f;
    for (int64_t i = 0; i < count; i++)
        out[i] = x[i] - bt * pred[i];
}
