// The DiT around the blocks: the SeedVR2DiTInput and SeedVR2DiTOutput heads
// (src/layers/seedvr2_dit_input.cpp, seedvr2_dit_output.cpp of the
// reference) and the 32-block forward of SeedVR2DiT (src/model/dit.cpp).
// Every weight is uploaded once; a forward enqueues the input head, all
// blocks and the output head on one stream with no host synchronisation, and
// the hidden streams ping-pong between two device buffers.
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "ncnn_format.h"
#include "sv2_internal.h"

namespace
{

size_t esize(int dtype)
{
    return dtype == SV2_F32 ? 4 : 2;
}

size_t align256(size_t v)
{
    return (v + 255) & ~static_cast<size_t>(255);
}

void free_all(std::vector<void*>* owned)
{
    for (void* p : *owned)
        (void)hipFree(p);
    owned->clear();
}

// A block-owned scratch buffer for callers that pass no workspace.  Growing it
// waits for the stream first: queued work may still read the old one.
int own_workspace(void** ws, size_t* ws_bytes, size_t need, hipStream_t stream, char** out)
{
    if (*ws_bytes < need)
    {
        if (*ws)
        {
            hipError_t err = hipStreamSynchronize(stream);
            if (err != hipSuccess)
                return sv2::hip_error(err, "synchronize before workspace resize");
            (void)hipFree(*ws);
            *ws = nullptr;
            *ws_bytes = 0;
        }
        hipError_t err = hipMalloc(ws, need);
        if (err != hipSuccess)
        {
            *ws = nullptr;
            return sv2::hip_error(err, "workspace allocation");
        }
        *ws_bytes = need;
    }
    *out = static_cast<char*>(*ws);
    return SV2_OK;
}

const sv2::ParamLayer* find_layer(const std::vector<sv2::ParamLayer>& layers, const char* type)
{
    for (const sv2::ParamLayer& l : layers)
        if (l.type == type)
            return &l;
    return nullptr;
}

} // namespace

struct sv2_dit_input
{
    sv2_dit_input_config cfg{};
    int dtype = SV2_F32;
    const void* w_vid = nullptr;
    const float* b_vid = nullptr;
    const void* w_txt = nullptr;
    const float* b_txt = nullptr;
    const float* w_tin = nullptr;
    const float* b_tin = nullptr;
    const float* w_thid = nullptr;
    const float* b_thid = nullptr;
    const float* w_tout = nullptr;
    const float* b_tout = nullptr;
    std::vector<void*> owned;
    void* ws = nullptr;
    size_t ws_bytes = 0;

    ~sv2_dit_input()
    {
        free_all(&owned);
        if (ws)
            (void)hipFree(ws);
    }
};

struct sv2_dit_output
{
    sv2_dit_output_config cfg{};
    int dtype = SV2_F32;
    const float* norm = nullptr;
    const float* shift = nullptr;
    const float* scale = nullptr;
    const void* w_proj = nullptr;
    const float* b_proj = nullptr;
    std::vector<void*> owned;
    void* ws = nullptr;
    size_t ws_bytes = 0;

    ~sv2_dit_output()
    {
        free_all(&owned);
        if (ws)
            (void)hipFree(ws);
    }
};

struct sv2_dit
{
    sv2_dit_input* input = nullptr;
    std::vector<sv2_block*> blocks;
    sv2_dit_output* output = nullptr;
    bool owns = false;
    int dtype = SV2_F32;
    void* ws = nullptr;
    size_t ws_bytes = 0;

    ~sv2_dit()
    {
        if (owns)
        {
            sv2_dit_input_destroy(input);
            for (sv2_block* b : blocks)
                sv2_block_destroy(b);
            sv2_dit_output_destroy(output);
        }
        if (ws)
            (void)hipFree(ws);
    }
};

namespace
{

// Workspace of the input head: patches [T*h*w, 4C], the text converted to the
// compute dtype [L, text_channels] (fp16 mode only), the sinusoid [S] and the
// two hidden vectors [dim] of the time MLP (fp32).
struct InputWs
{
    size_t patches, text, sin, h1, h2, total;
};

InputWs input_layout(const sv2_dit_input* in, int T, int H, int W, int L)
{
    const sv2_dit_input_config& c = in->cfg;
    const size_t es = esize(in->dtype);
    const size_t Lp = static_cast<size_t>(T) * (H / 2) * (W / 2);
    InputWs w{};
    size_t off = 0;
    w.patches = off;
    off = align256(off + Lp * 4 * c.video_channels * es);
    w.text = off;
    off = align256(off + (in->dtype == SV2_F32 ? 0 : static_cast<size_t>(L) * c.text_channels * es));
    w.sin = off;
    off = align256(off + c.sinusoidal_dim * sizeof(float));
    w.h1 = off;
    off = align256(off + c.dim * sizeof(float));
    w.h2 = off;
    off = align256(off + c.dim * sizeof(float));
    w.total = off;
    return w;
}

struct OutputWs
{
    size_t table, normed, projected, total;
};

OutputWs output_layout(const sv2_dit_output* out, int T, int h, int w)
{
    const size_t es = esize(out->dtype);
    const size_t Lp = static_cast<size_t>(T) * h * w;
    OutputWs o{};
    size_t off = 0;
    o.table = off;
    off = align256(off + 3 * static_cast<size_t>(out->cfg.dim) * sizeof(float));
    o.normed = off;
    off = align256(off + Lp * out->cfg.dim * es);
    o.projected = off;
    off = align256(off + Lp * 4 * out->cfg.output_channels * es);
    o.total = off;
    return o;
}

int validate_input_config(const sv2_dit_input_config& c)
{
    // load_param's check (seedvr2_dit_input.cpp:214)
    if (c.dim <= 0 || c.video_channels <= 0 || c.text_channels <= 0 || c.sinusoidal_dim <= 0 ||
        c.sinusoidal_dim % 2 != 0 || c.embedding_dim != c.dim * 6)
        return sv2::set_error(SV2_EINVAL, "dit input: sinusoidal_dim must be even and embedding_dim = 6 * dim");
    if (c.dim % 8 != 0 || c.text_channels % 8 != 0)
        return sv2::set_error(SV2_EUNSUPPORTED, "dit input: dim and text_channels must be multiples of 8");
    return SV2_OK;
}

int validate_output_config(const sv2_dit_output_config& c)
{
    // load_param's check (seedvr2_dit_output.cpp:261)
    if (c.dim <= 0 || c.output_channels <= 0)
        return sv2::set_error(SV2_EINVAL, "dit output: dim and output_channels must be positive");
    if (c.dim % 8 != 0 || c.dim > 4096 || (4 * c.output_channels) % 8 != 0)
        return sv2::set_error(SV2_EUNSUPPORTED,
                              "dit output: dim must be a multiple of 8 up to 4096, output_channels even");
    return SV2_OK;
}

} // namespace

extern "C" {

int sv2_dit_input_create(const sv2_dit_input_config* config, const sv2_dit_input_weights* w, int weights_on_device,
                         int compute_dtype, sv2_dit_input** out)
try
{
    using namespace sv2;
    if (!config || !w || !out)
        return set_error(SV2_EINVAL, "sv2_dit_input_create: null argument");
    *out = nullptr;
    int rc = validate_input_config(*config);
    if (rc != SV2_OK)
        return rc;
    if (compute_dtype != SV2_F32 && compute_dtype != SV2_F16)
        return set_error(SV2_EINVAL, "sv2_dit_input_create: compute dtype must be SV2_F32 or SV2_F16");
    if (!w->w_vid || !w->b_vid || !w->w_txt || !w->b_txt || !w->w_time_in || !w->b_time_in || !w->w_time_hid ||
        !w->b_time_hid || !w->w_time_out || !w->b_time_out)
        return set_error(SV2_EINVAL, "sv2_dit_input_create: missing weight");
    sv2_dit_input* in = new sv2_dit_input();
    in->cfg = *config;
    in->dtype = compute_dtype;
    const sv2_dit_input_config& c = *config;
    const size_t D = c.dim;
    if (weights_on_device)
    {
        in->w_vid = w->w_vid;
        in->b_vid = static_cast<const float*>(w->b_vid);
        in->w_txt = w->w_txt;
        in->b_txt = static_cast<const float*>(w->b_txt);
        in->w_tin = static_cast<const float*>(w->w_time_in);
        in->b_tin = static_cast<const float*>(w->b_time_in);
        in->w_thid = static_cast<const float*>(w->w_time_hid);
        in->b_thid = static_cast<const float*>(w->b_time_hid);
        in->w_tout = static_cast<const float*>(w->w_time_out);
        in->b_tout = static_cast<const float*>(w->b_time_out);
        *out = in;
        return SV2_OK;
    }
    struct Item
    {
        const void* src;
        size_t count;
        int dtype;
        const void** dst;
    };
    const void* p[10];
    const Item items[] = {
        {w->w_vid, D * 4 * c.video_channels, compute_dtype, &in->w_vid},
        {w->b_vid, D, SV2_F32, &p[1]},
        {w->w_txt, D * c.text_channels, compute_dtype, &in->w_txt},
        {w->b_txt, D, SV2_F32, &p[3]},
        {w->w_time_in, D * c.sinusoidal_dim, SV2_F32, &p[4]},
        {w->b_time_in, D, SV2_F32, &p[5]},
        {w->w_time_hid, D * D, SV2_F32, &p[6]},
        {w->b_time_hid, D, SV2_F32, &p[7]},
        {w->w_time_out, static_cast<size_t>(c.embedding_dim) * D, SV2_F32, &p[8]},
        {w->b_time_out, static_cast<size_t>(c.embedding_dim), SV2_F32, &p[9]},
    };
    for (const Item& it : items)
    {
        if ((rc = upload_weights(&in->owned, static_cast<const float*>(it.src), it.count, it.dtype, it.dst)) !=
            SV2_OK)
        {
            delete in;
            return rc;
        }
    }
    in->b_vid = static_cast<const float*>(p[1]);
    in->b_txt = static_cast<const float*>(p[3]);
    in->w_tin = static_cast<const float*>(p[4]);
    in->b_tin = static_cast<const float*>(p[5]);
    in->w_thid = static_cast<const float*>(p[6]);
    in->b_thid = static_cast<const float*>(p[7]);
    in->w_tout = static_cast<const float*>(p[8]);
    in->b_tout = static_cast<const float*>(p[9]);
    *out = in;
    return SV2_OK;
}
catch (...)
{
    return sv2::caught_exception("sv2_dit_input_create");
}

int sv2_dit_input_load(const char* param_path, const char* bin_path, int compute_dtype, sv2_dit_input** out)
try
{
    using namespace sv2;
    if (!param_path || !bin_path || !out)
        return set_error(SV2_EINVAL, "sv2_dit_input_load: null argument");
    *out = nullptr;
    std::vector<ParamLayer> layers;
    std::string err;
    if (read_param_file(param_path, &layers, &err) != 0)
        return set_error(SV2_EINVAL, "sv2_dit_input_load: " + err);
    const ParamLayer* l = find_layer(layers, "SeedVR2DiTInput");
    if (!l)
        return set_error(SV2_EINVAL, std::string("sv2_dit_input_load: no SeedVR2DiTInput layer in ") + param_path);
    if (l->bottoms.size() != 4 || l->tops.size() != 4)
        return set_error(SV2_EINVAL, "sv2_dit_input_load: SeedVR2DiTInput needs 4 bottoms and 4 tops");
    sv2_dit_input_config c;
    c.dim = l->get_int(0, 2560);
    c.video_channels = l->get_int(1, 33);
    c.text_channels = l->get_int(2, 5120);
    c.sinusoidal_dim = l->get_int(3, 256);
    c.embedding_dim = l->get_int(4, 15360);
    int rc = validate_input_config(c);
    if (rc != SV2_OK)
        return rc;
    // weight order of load_model (seedvr2_dit_input.cpp:217-227): each
    // InnerProduct reads its tagged matrix, then its raw bias
    BinReader bin;
    if (bin.open(bin_path, &err) != 0)
        return set_error(SV2_EDEVICE, "sv2_dit_input_load: " + err);
    const size_t D = c.dim;
    const size_t ins[5] = {static_cast<size_t>(4 * c.video_channels), static_cast<size_t>(c.text_channels),
                           static_cast<size_t>(c.sinusoidal_dim), D, D};
    const size_t outs[5] = {D, D, D, D, static_cast<size_t>(c.embedding_dim)};
    std::vector<float> mats[5], biases[5];
    for (int i = 0; i < 5; i++)
        if (bin.load_tagged(ins[i] * outs[i], &mats[i], &err) != 0 || bin.load_raw(outs[i], &biases[i], &err) != 0)
            return set_error(SV2_EDEVICE, std::string("sv2_dit_input_load: ") + bin_path + ": " + err);
    sv2_dit_input_weights w;
    w.w_vid = mats[0].data();
    w.b_vid = biases[0].data();
    w.w_txt = mats[1].data();
    w.b_txt = biases[1].data();
    w.w_time_in = mats[2].data();
    w.b_time_in = biases[2].data();
    w.w_time_hid = mats[3].data();
    w.b_time_hid = biases[3].data();
    w.w_time_out = mats[4].data();
    w.b_time_out = biases[4].data();
    return sv2_dit_input_create(&c, &w, 0, compute_dtype, out);
}
catch (...)
{
    return sv2::caught_exception("sv2_dit_input_load");
}

int sv2_dit_input_get_config(const sv2_dit_input* head, sv2_dit_input_config* config)
try
{
    if (!head || !config)
        return sv2::set_error(SV2_EINVAL, "sv2_dit_input_get_config: null argument");
    *config = head->cfg;
    return SV2_OK;
}
catch (...)
{
    return sv2::caught_exception("sv2_dit_input_get_config");
}

int64_t sv2_dit_input_workspace_size(const sv2_dit_input* head, int frames, int height, int width, int text_len)
try
{
    if (!head || frames <= 0 || height <= 0 || width <= 0 || height % 2 != 0 || width % 2 != 0 || text_len < 0)
        return sv2::set_error(SV2_EINVAL, "sv2_dit_input_workspace_size: bad argument");
    return static_cast<int64_t>(input_layout(head, frames, height, width, text_len).total);
}
catch (...)
{
    return sv2::caught_exception("sv2_dit_input_workspace_size");
}

int sv2_dit_input_forward(sv2_dit_input* in, const float* video, int channel_major, const float* text, int text_len,
                          float timestep, int frames, int height, int width, void* vid_out, void* txt_out, float* emb,
                          void* workspace, size_t workspace_bytes, void* stream_ptr)
try
{
    using namespace sv2;
    if (!in || !video || !vid_out || !emb || text_len < 0 || (text_len > 0 && (!text || !txt_out)))
        return set_error(SV2_EINVAL, "sv2_dit_input_forward: null argument");
    // the reference's shape checks (seedvr2_dit_input.cpp:317-330)
    if (frames <= 0 || height <= 0 || width <= 0 || height % 2 != 0 || width % 2 != 0)
        return set_error(SV2_EINVAL, "sv2_dit_input_forward: the grid must be positive with even height and width");
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    const InputWs lay = input_layout(in, frames, height, width, text_len);
    char* ws = static_cast<char*>(workspace);
    int rc;
    if (ws)
    {
        if (workspace_bytes < lay.total)
            return set_error(SV2_EINVAL, "sv2_dit_input_forward: workspace too small");
    }
    else if ((rc = own_workspace(&in->ws, &in->ws_bytes, lay.total, stream, &ws)) != SV2_OK)
        return rc;
    const sv2_dit_input_config& c = in->cfg;
    const int dt = in->dtype;
    const int h = height / 2, w = width / 2;
    const int Lp = frames * h * w;
    void* patches = ws + lay.patches;
    float* sin = reinterpret_cast<float*>(ws + lay.sin);
    float* h1 = reinterpret_cast<float*>(ws + lay.h1);
    float* h2 = reinterpret_cast<float*>(ws + lay.h2);
    // video: patchify (:336-352), vid_in InnerProduct with bias (:354-358)
    if ((rc = launch_patchify(video, patches, dt, frames, h, w, c.video_channels, channel_major, stream)) != SV2_OK ||
        (rc = gemm_rows_bias(stream, dt, Lp, 4 * c.video_channels, c.dim, patches, in->w_vid, in->b_vid, vid_out)) !=
            SV2_OK)
        return rc;
    // text: txt_in InnerProduct with bias
    if (text_len > 0)
    {
        const void* x = text;
        if (dt != SV2_F32)
        {
            if ((rc = launch_from_f32(ws + lay.text, text, dt, static_cast<long long>(text_len) * c.text_channels,
                                      stream)) != SV2_OK)
                return rc;
            x = ws + lay.text;
        }
        if ((rc = gemm_rows_bias(stream, dt, text_len, c.text_channels, c.dim, x, in->w_txt, in->b_txt, txt_out)) !=
            SV2_OK)
            return rc;
    }
    // timestep: sinusoid, proj_in + silu, proj_hid + silu, proj_out (:360-392), fp32
    if ((rc = launch_sinusoid(sin, timestep, c.sinusoidal_dim, stream)) != SV2_OK ||
        (rc = gemm_rows_bias(stream, SV2_F32, 1, c.sinusoidal_dim, c.dim, sin, in->w_tin, in->b_tin, h1)) != SV2_OK ||
        (rc = launch_bias_act(h1, nullptr, SV2_F32, 1, c.dim, 1, stream)) != SV2_OK ||
        (rc = gemm_rows_bias(stream, SV2_F32, 1, c.dim, c.dim, h1, in->w_thid, in->b_thid, h2)) != SV2_OK ||
        (rc = launch_bias_act(h2, nullptr, SV2_F32, 1, c.dim, 1, stream)) != SV2_OK ||
        (rc = gemm_rows_bias(stream, SV2_F32, 1, c.dim, c.embedding_dim, h2, in->w_tout, in->b_tout, emb)) != SV2_OK)
        return rc;
    return SV2_OK;
}
catch (...)
{
    return sv2::caught_exception("sv2_dit_input_forward");
}

void sv2_dit_input_destroy(sv2_dit_input* head)
{
    delete head;
}

int sv2_dit_output_create(const sv2_dit_output_config* config, const sv2_dit_output_weights* w,
                          int weights_on_device, int compute_dtype, sv2_dit_output** out)
try
{
    using namespace sv2;
    if (!config || !w || !out)
        return set_error(SV2_EINVAL, "sv2_dit_output_create: null argument");
    *out = nullptr;
    int rc = validate_output_config(*config);
    if (rc != SV2_OK)
        return rc;
    if (compute_dtype != SV2_F32 && compute_dtype != SV2_F16)
        return set_error(SV2_EINVAL, "sv2_dit_output_create: compute dtype must be SV2_F32 or SV2_F16");
    if (!w->norm_weight || !w->shift || !w->scale || !w->w_proj || !w->b_proj)
        return set_error(SV2_EINVAL, "sv2_dit_output_create: missing weight");
    sv2_dit_output* o = new sv2_dit_output();
    o->cfg = *config;
    o->dtype = compute_dtype;
    const size_t D = config->dim, P = 4 * static_cast<size_t>(config->output_channels);
    if (weights_on_device)
    {
        o->norm = static_cast<const float*>(w->norm_weight);
        o->shift = static_cast<const float*>(w->shift);
        o->scale = static_cast<const float*>(w->scale);
        o->w_proj = w->w_proj;
        o->b_proj = static_cast<const float*>(w->b_proj);
        *out = o;
        return SV2_OK;
    }
    const void* p[4];
    if ((rc = upload_weights(&o->owned, static_cast<const float*>(w->norm_weight), D, SV2_F32, &p[0])) != SV2_OK ||
        (rc = upload_weights(&o->owned, static_cast<const float*>(w->shift), D, SV2_F32, &p[1])) != SV2_OK ||
        (rc = upload_weights(&o->owned, static_cast<const float*>(w->scale), D, SV2_F32, &p[2])) != SV2_OK ||
        (rc = upload_weights(&o->owned, static_cast<const float*>(w->w_proj), P * D, compute_dtype, &o->w_proj)) !=
            SV2_OK ||
        (rc = upload_weights(&o->owned, static_cast<const float*>(w->b_proj), P, SV2_F32, &p[3])) != SV2_OK)
    {
        delete o;
        return rc;
    }
    o->norm = static_cast<const float*>(p[0]);
    o->shift = static_cast<const float*>(p[1]);
    o->scale = static_cast<const float*>(p[2]);
    o->b_proj = static_cast<const float*>(p[3]);
    *out = o;
    return SV2_OK;
}
catch (...)
{
    return sv2::caught_exception("sv2_dit_output_create");
}

int sv2_dit_output_load(const char* param_path, const char* bin_path, int compute_dtype, sv2_dit_output** out)
try
{
    using namespace sv2;
    if (!param_path || !bin_path || !out)
        return set_error(SV2_EINVAL, "sv2_dit_output_load: null argument");
    *out = nullptr;
    std::vector<ParamLayer> layers;
    std::string err;
    if (read_param_file(param_path, &layers, &err) != 0)
        return set_error(SV2_EINVAL, "sv2_dit_output_load: " + err);
    const ParamLayer* l = find_layer(layers, "SeedVR2DiTOutput");
    if (!l)
        return set_error(SV2_EINVAL, std::string("sv2_dit_output_load: no SeedVR2DiTOutput layer in ") + param_path);
    if (l->bottoms.size() != 3 || l->tops.size() != 2)
        return set_error(SV2_EINVAL, "sv2_dit_output_load: SeedVR2DiTOutput needs 3 bottoms and 2 tops");
    sv2_dit_output_config c;
    c.dim = l->get_int(0, 2560);
    c.output_channels = l->get_int(1, 16);
    c.norm_eps = l->get_float(2, 1e-5f);
    int rc = validate_output_config(c);
    if (rc != SV2_OK)
        return rc;
    // load_model (seedvr2_dit_output.cpp:264-273)
    BinReader bin;
    if (bin.open(bin_path, &err) != 0)
        return set_error(SV2_EDEVICE, "sv2_dit_output_load: " + err);
    const size_t D = c.dim, P = 4 * static_cast<size_t>(c.output_channels);
    std::vector<float> norm, shift, scale, wp, bp;
    if (bin.load_raw(D, &norm, &err) != 0 || bin.load_raw(D, &shift, &err) != 0 || bin.load_raw(D, &scale, &err) != 0 ||
        bin.load_tagged(P * D, &wp, &err) != 0 || bin.load_raw(P, &bp, &err) != 0)
        return set_error(SV2_EDEVICE, std::string("sv2_dit_output_load: ") + bin_path + ": " + err);
    sv2_dit_output_weights w;
    w.norm_weight = norm.data();
    w.shift = shift.data();
    w.scale = scale.data();
    w.w_proj = wp.data();
    w.b_proj = bp.data();
    return sv2_dit_output_create(&c, &w, 0, compute_dtype, out);
}
catch (...)
{
    return sv2::caught_exception("sv2_dit_output_load");
}

int sv2_dit_output_get_config(const sv2_dit_output* head, sv2_dit_output_config* config)
try
{
    if (!head || !config)
        return sv2::set_error(SV2_EINVAL, "sv2_dit_output_get_config: null argument");
    *config = head->cfg;
    return SV2_OK;
}
catch (...)
{
    return sv2::caught_exception("sv2_dit_output_get_config");
}

int64_t sv2_dit_output_workspace_size(const sv2_dit_output* head, int frames, int height, int width)
try
{
    if (!head || frames <= 0 || height <= 0 || width <= 0)
        return sv2::set_error(SV2_EINVAL, "sv2_dit_output_workspace_size: bad argument");
    return static_cast<int64_t>(output_layout(head, frames, height, width).total);
}
catch (...)
{
    return sv2::caught_exception("sv2_dit_output_workspace_size");
}

int sv2_dit_output_forward(sv2_dit_output* o, const void* vid, const float* emb, int frames, int height, int width,
                           float* output, int channel_major, void* workspace, size_t workspace_bytes,
                           void* stream_ptr)
try
{
    using namespace sv2;
    if (!o || !vid || !emb || !output)
        return set_error(SV2_EINVAL, "sv2_dit_output_forward: null argument");
    if (frames <= 0 || height <= 0 || width <= 0)
        return set_error(SV2_EINVAL, "sv2_dit_output_forward: bad grid");
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    const OutputWs lay = output_layout(o, frames, height, width);
    char* ws = static_cast<char*>(workspace);
    int rc;
    if (ws)
    {
        if (workspace_bytes < lay.total)
            return set_error(SV2_EINVAL, "sv2_dit_output_forward: workspace too small");
    }
    else if ((rc = own_workspace(&o->ws, &o->ws_bytes, lay.total, stream, &ws)) != SV2_OK)
        return rc;
    const sv2_dit_output_config& c = o->cfg;
    const int dt = o->dtype;
    const int Lp = frames * height * width;
    const int P = 4 * c.output_channels;
    void* normed = ws + lay.normed;
    void* projected = ws + lay.projected;
    // RMSNorm * norm_weight + ada with emb slot 0 (:368-386), vid_out.proj
    // with bias (:388-390), unpatchify (:391-413)
    float* table = reinterpret_cast<float*>(ws + lay.table);
    if ((rc = launch_ada_table(emb, o->scale, nullptr, 0, c.dim, table, stream)) != SV2_OK ||
        (rc = launch_rmsnorm_table(vid, normed, dt, Lp, c.dim, c.norm_eps, table, o->shift, o->norm, 1, stream)) !=
            SV2_OK ||
        (rc = gemm_rows_bias(stream, dt, Lp, c.dim, P, normed, o->w_proj, o->b_proj, projected)) != SV2_OK ||
        (rc = launch_unpatchify(projected, output, dt, frames, height, width, c.output_channels, channel_major,
                                stream)) != SV2_OK)
        return rc;
    return SV2_OK;
}
catch (...)
{
    return sv2::caught_exception("sv2_dit_output_forward");
}

void sv2_dit_output_destroy(sv2_dit_output* head)
{
    delete head;
}

int sv2_dit_create(sv2_dit_input* input, sv2_block* const* blocks, int block_count, sv2_dit_output* output,
                   sv2_dit** out)
try
{
    using namespace sv2;
    if (!input || !output || !out || block_count < 0 || (block_count > 0 && !blocks))
        return set_error(SV2_EINVAL, "sv2_dit_create: null argument");
    *out = nullptr;
    const int dt = input->dtype;
    if (output->dtype != dt)
        return set_error(SV2_EINVAL, "sv2_dit_create: the heads use different compute dtypes");
    for (int i = 0; i < block_count; i++)
    {
        sv2_block_config bc;
        if (!blocks[i] || sv2_block_get_config(blocks[i], &bc) != SV2_OK)
            return set_error(SV2_EINVAL, "sv2_dit_create: null block");
        if (block_compute_dtype(blocks[i]) != dt)
            return set_error(SV2_EINVAL, "sv2_dit_create: a block uses another compute dtype than the heads");
        if (bc.dim != input->cfg.dim || bc.dim != output->cfg.dim || bc.dim * 6 != input->cfg.embedding_dim)
            return set_error(SV2_EINVAL, "sv2_dit_create: block width differs from the heads");
    }
    sv2_dit* d = new sv2_dit();
    d->input = input;
    d->blocks.assign(blocks, blocks + block_count);
    d->output = output;
    d->dtype = dt;
    *out = d;
    return SV2_OK;
}
catch (...)
{
    return sv2::caught_exception("sv2_dit_create");
}

int sv2_dit_load(const char* model_dir, int compute_dtype, sv2_dit** out)
{
    return sv2_dit_load_ex(model_dir, compute_dtype, SV2_VERIFY_IF_PRESENT, out);
}

int sv2_dit_load_ex(const char* model_dir, int compute_dtype, int verify, sv2_dit** out)
try
{
    using namespace sv2;
    if (!model_dir || !out)
        return set_error(SV2_EINVAL, "sv2_dit_load: null argument");
    if (verify < SV2_VERIFY_NONE || verify > SV2_VERIFY_STRICT)
        return set_error(SV2_EINVAL, "sv2_dit_load: unknown verify mode");
    *out = nullptr;
    const std::string root(model_dir);
    auto path = [&](const std::string& stem, const char* ext) { return root + "/" + stem + ".ncnn" + ext; };
    // every file is checked before anything is loaded (dit.cpp:122-134)
    std::vector<std::string> stems = {"seedvr2_dit_input", "seedvr2_dit_output"};
    for (int i = 0; i < 32; i++)
    {
        char stem[64];
        std::snprintf(stem, sizeof(stem), "seedvr2_dit_block_%02d", i);
        stems.push_back(stem);
    }
    for (const std::string& s : stems)
        for (const char* ext : {".param", ".bin"})
        {
            std::FILE* f = std::fopen(path(s, ext).c_str(), "rb");
            if (!f)
                return set_error(SV2_EINVAL, "sv2_dit_load: DiT model file is missing: " + path(s, ext));
            std::fclose(f);
        }
    // the directory's SHA256SUMS (scripts/verify-models.sh:17-24): when it
    // has one, or required
    const int checked = verify == SV2_VERIFY_NONE     ? 0
                        : verify == SV2_VERIFY_STRICT ? sv2_verify_checksums_strict(model_dir, 0)
                                                      : sv2_verify_checksums(model_dir, 0);
    if (checked < 0)
        return checked;
    sv2_dit* d = new sv2_dit();
    d->owns = true;
    d->dtype = compute_dtype;
    int rc = sv2_dit_input_load(path(stems[0], ".param").c_str(), path(stems[0], ".bin").c_str(), compute_dtype,
                                &d->input);
    if (rc == SV2_OK)
        rc = sv2_dit_output_load(path(stems[1], ".param").c_str(), path(stems[1], ".bin").c_str(), compute_dtype,
                                 &d->output);
    for (int i = 0; i < 32 && rc == SV2_OK; i++)
    {
        sv2_block* b = nullptr;
        rc = sv2_block_load(path(stems[2 + i], ".param").c_str(), path(stems[2 + i], ".bin").c_str(), compute_dtype,
                            &b);
        if (rc == SV2_OK)
            d->blocks.push_back(b);
    }
    if (rc == SV2_OK && (d->input->cfg.dim != d->output->cfg.dim))
        rc = set_error(SV2_EINVAL, "sv2_dit_load: the heads have different widths");
    if (rc != SV2_OK)
    {
        delete d;
        return rc;
    }
    *out = d;
    return SV2_OK;
}
catch (...)
{
    return sv2::caught_exception("sv2_dit_load");
}

} // extern "C"

namespace
{

struct DitWs
{
    size_t vid[2], txt[2], emb, scratch, total;
};

int dit_layout(sv2_dit* d, int T, int H, int W, int L, DitWs* out)
{
    using namespace sv2;
    if (T <= 0 || H <= 0 || W <= 0 || H % 2 != 0 || W % 2 != 0 || L < 0)
        return set_error(SV2_EINVAL, "dit: the latent grid must be positive with even height and width");
    const int h = H / 2, w = W / 2;
    const size_t es = esize(d->dtype);
    const size_t D = d->input->cfg.dim;
    const size_t Lp = static_cast<size_t>(T) * h * w;
    size_t scratch = input_layout(d->input, T, H, W, L).total;
    scratch = std::max(scratch, output_layout(d->output, T, h, w).total);
    for (sv2_block* b : d->blocks)
    {
        int rc = sv2_block_set_runtime_shape(b, T, h, w);
        if (rc != SV2_OK)
            return rc;
        const int64_t need = sv2_block_workspace_size(b, L);
        if (need < 0)
            return static_cast<int>(need);
        scratch = std::max(scratch, static_cast<size_t>(need));
    }
    size_t off = 0;
    for (int i = 0; i < 2; i++)
    {
        out->vid[i] = off;
        off = align256(off + Lp * D * es);
        out->txt[i] = off;
        off = align256(off + static_cast<size_t>(L) * D * es);
    }
    out->emb = off;
    off = align256(off + 6 * D * sizeof(float));
    out->scratch = off;
    off = align256(off + scratch);
    out->total = off;
    return SV2_OK;
}

} // namespace

extern "C" {

int sv2_dit_get_config(const sv2_dit* dit, sv2_dit_input_config* input, sv2_dit_output_config* output,
                       int* block_count)
try
{
    if (!dit)
        return sv2::set_error(SV2_EINVAL, "sv2_dit_get_config: null dit");
    if (input)
        *input = dit->input->cfg;
    if (output)
        *output = dit->output->cfg;
    if (block_count)
        *block_count = static_cast<int>(dit->blocks.size());
    return SV2_OK;
}
catch (...)
{
    return sv2::caught_exception("sv2_dit_get_config");
}

int64_t sv2_dit_workspace_size(sv2_dit* dit, int frames, int height, int width, int text_len)
try
{
    if (!dit)
        return sv2::set_error(SV2_EINVAL, "sv2_dit_workspace_size: null dit");
    DitWs lay;
    const int rc = dit_layout(dit, frames, height, width, text_len, &lay);
    return rc == SV2_OK ? static_cast<int64_t>(lay.total) : rc;
}
catch (...)
{
    return sv2::caught_exception("sv2_dit_workspace_size");
}

int sv2_dit_forward(sv2_dit* d, const float* latent, const float* text, int text_len, float timestep, int frames,
                    int height, int width, float* output, void* workspace, size_t workspace_bytes, void* stream_ptr)
try
{
    using namespace sv2;
    if (!d || !latent || !output || text_len < 0 || (text_len > 0 && !text))
        return set_error(SV2_EINVAL, "sv2_dit_forward: null argument");
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    DitWs lay;
    int rc = dit_layout(d, frames, height, width, text_len, &lay);
    if (rc != SV2_OK)
        return rc;
    char* ws = static_cast<char*>(workspace);
    if (ws)
    {
        if (workspace_bytes < lay.total)
            return set_error(SV2_EINVAL, "sv2_dit_forward: workspace too small");
    }
    else if ((rc = own_workspace(&d->ws, &d->ws_bytes, lay.total, stream, &ws)) != SV2_OK)
        return rc;
    const int h = height / 2, w = width / 2;
    void* vid[2] = {ws + lay.vid[0], ws + lay.vid[1]};
    void* txt[2] = {ws + lay.txt[0], ws + lay.txt[1]};
    float* emb = reinterpret_cast<float*>(ws + lay.emb);
    char* scratch = ws + lay.scratch;
    const size_t scratch_bytes = lay.total - lay.scratch;
    void* tx0 = text_len > 0 ? txt[0] : nullptr;
    if ((rc = sv2_dit_input_forward(d->input, latent, 1, text, text_len, timestep, frames, height, width, vid[0], tx0,
                                    emb, scratch, scratch_bytes, stream)) != SV2_OK)
        return rc;
    int cur = 0;
    for (sv2_block* b : d->blocks)
    {
        void* tin = text_len > 0 ? txt[cur] : nullptr;
        void* tout = text_len > 0 ? txt[cur ^ 1] : nullptr;
        if ((rc = sv2_block_forward(b, vid[cur], tin, text_len, emb, vid[cur ^ 1], tout, scratch, scratch_bytes,
                                    stream)) != SV2_OK)
            return rc;
        cur ^= 1;
    }
    return sv2_dit_output_forward(d->output, vid[cur], emb, frames, h, w, output, 1, scratch, scratch_bytes, stream);
}
catch (...)
{
    return sv2::caught_exception("sv2_dit_forward");
}

void sv2_dit_destroy(sv2_dit* dit)
{
    delete dit;
}

} // extern "C"
