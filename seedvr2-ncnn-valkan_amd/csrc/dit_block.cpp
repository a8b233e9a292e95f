// The SeedVR2DiTBlock layer on the device (src/layers/seedvr2_dit_block.{h,cpp}
// of the reference): parameters, weight loading from the exported
// .param/.bin pair, and the block forward as a chain of the library's kernels
// on one stream — token RMSNorm + ada, the QKV / proj / MLP InnerProducts
// (hipBLASLt in fp16, the fp64-accumulating exact GEMM in the fp32 parity
// mode, or the fused MFMA kernel under param 14), the windowed attention,
// gated residuals and SwiGLU.
#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "ncnn_format.h"
#include "sv2_internal.h"

using sv2::gemm_few;
using sv2::gemm_mfma;
using sv2::gemm_rows;
using sv2::gemm_rows_bias;
using sv2::kGemmResidual;
using sv2::kGemmStore;
using sv2::kGemmSwiGLU;

namespace
{

struct DevBranch
{
    const float* ada[6] = {};
    const void* w_qkv = nullptr;
    const void* w_proj = nullptr;
    const float* b_proj = nullptr;
    const float* norm_q = nullptr;
    const float* norm_k = nullptr;
    const void* w_gate = nullptr;
    const void* w_in = nullptr;
    const void* w_out = nullptr;
};

size_t dtype_size(int dtype)
{
    return dtype == SV2_F32 ? 4 : 2;
}

} // namespace

struct sv2_block
{
    sv2_block_config cfg{};
    int dtype = SV2_F32;
    DevBranch vid;
    DevBranch txt;
    std::vector<void*> owned;
    float freqs[21] = {};
    bool has_freqs = false;
    int T = 0, H = 0, W = 0;
    bool shape_valid = false;
    // RoPE cos/sin table on the device, covering rope_npos positions; grown
    // only.  Tables it replaced (queued work may still read them) and the
    // pinned host copies of every upload stay allocated until the block goes.
    float* rope = nullptr;
    int rope_npos = 0;
    std::vector<float*> rope_retired;
    std::vector<float*> rope_host;
    // workspace kept by the block when the caller passes none
    void* ws = nullptr;
    size_t ws_bytes = 0;
    bool debug_on = false;
    sv2_block_debug debug{};
    // whether the last forward ran the row-wise steps over the video and
    // text rows at once (sv2_block_last_forward_merged)
    int last_merged = 0;
    // device staging of sv2_block_forward_host, grown on demand
    void* stage = nullptr;
    size_t stage_bytes = 0;

    ~sv2_block()
    {
        if (stage)
            (void)hipFree(stage);
        for (void* p : owned)
            (void)hipFree(p);
        if (rope)
            (void)hipFree(rope);
        for (float* t : rope_retired)
            (void)hipFree(t);
        for (float* h : rope_host)
            (void)hipHostFree(h);
        if (ws)
            (void)hipFree(ws);
    }
};

namespace
{

int validate_config(const sv2_block_config& c)
{
    if (c.dim <= 0 || c.heads <= 0 || c.head_dim <= 0 || c.mlp_hidden <= 0 || c.dim != c.heads * c.head_dim)
        return sv2::set_error(SV2_EINVAL, "block: dim must equal heads * head_dim (SeedVR2DiTBlock::load_param)");
    if (c.head_dim != 128)
        return sv2::set_error(SV2_EUNSUPPORTED, "block: head_dim must be 128");
    if (c.dim % 8 != 0 || c.mlp_hidden % 8 != 0 || c.dim > 4096)
        return sv2::set_error(SV2_EUNSUPPORTED, "block: dim and mlp_hidden must be multiples of 8, dim <= 4096");
    if (c.window_t < 0 || c.window_h < 0 || c.window_w < 0)
        return sv2::set_error(SV2_EINVAL, "block: window extents must be >= 0");
    if (c.rope_mode < SV2_ROPE_REFERENCE || c.rope_mode > SV2_ROPE_NONE)
        return sv2::set_error(SV2_EINVAL, "block: unknown rope mode");
    if (c.fused_gemm && (!sv2::gemm_mfma_supported(c.dim, 3 * c.dim, sv2::kGemmStore) ||
                         !sv2::gemm_mfma_supported(c.dim, c.mlp_hidden, sv2::kGemmSwiGLU) ||
                         !sv2::gemm_mfma_supported(c.mlp_hidden, c.dim, sv2::kGemmResidual)))
        return sv2::set_error(SV2_EUNSUPPORTED,
                              "block: fused InnerProducts need dim % 256 == 0 and mlp_hidden % 128 == 0");
    return SV2_OK;
}

// Uploads `count` elements: fp32 host values converted to `dtype` (matrices)
// or kept fp32 (vectors, dtype SV2_F32).
int upload(sv2_block* b, const float* host, size_t count, int dtype, const void** dev)
{
    return sv2::upload_weights(&b->owned, host, count, dtype, dev);
}

int bind_branch(sv2_block* b, const sv2_block_branch& in, bool on_device, DevBranch* out)
{
    const sv2_block_config& c = b->cfg;
    const size_t D = c.dim, F = c.mlp_hidden, hd = c.head_dim;
    for (int i = 0; i < 6; i++)
        if (!in.ada[i])
            return sv2::set_error(SV2_EINVAL, "block: missing ada vector");
    if (!in.w_qkv || !in.w_proj || !in.b_proj || !in.norm_q || !in.norm_k || !in.w_gate || !in.w_in || !in.w_out)
        return sv2::set_error(SV2_EINVAL, "block: missing branch weight");
    if (on_device)
    {
        for (int i = 0; i < 6; i++)
            out->ada[i] = static_cast<const float*>(in.ada[i]);
        out->w_qkv = in.w_qkv;
        out->w_proj = in.w_proj;
        out->b_proj = static_cast<const float*>(in.b_proj);
        out->norm_q = static_cast<const float*>(in.norm_q);
        out->norm_k = static_cast<const float*>(in.norm_k);
        out->w_gate = in.w_gate;
        out->w_in = in.w_in;
        out->w_out = in.w_out;
        return SV2_OK;
    }
    int rc;
    const void* p;
    for (int i = 0; i < 6; i++)
    {
        if ((rc = upload(b, static_cast<const float*>(in.ada[i]), D, SV2_F32, &p)) != SV2_OK)
            return rc;
        out->ada[i] = static_cast<const float*>(p);
    }
    if ((rc = upload(b, static_cast<const float*>(in.w_qkv), 3 * D * D, b->dtype, &out->w_qkv)) != SV2_OK ||
        (rc = upload(b, static_cast<const float*>(in.w_proj), D * D, b->dtype, &out->w_proj)) != SV2_OK ||
        (rc = upload(b, static_cast<const float*>(in.w_gate), F * D, b->dtype, &out->w_gate)) != SV2_OK ||
        (rc = upload(b, static_cast<const float*>(in.w_in), F * D, b->dtype, &out->w_in)) != SV2_OK ||
        (rc = upload(b, static_cast<const float*>(in.w_out), D * F, b->dtype, &out->w_out)) != SV2_OK)
        return rc;
    if ((rc = upload(b, static_cast<const float*>(in.b_proj), D, SV2_F32, &p)) != SV2_OK)
        return rc;
    out->b_proj = static_cast<const float*>(p);
    if ((rc = upload(b, static_cast<const float*>(in.norm_q), hd, SV2_F32, &p)) != SV2_OK)
        return rc;
    out->norm_q = static_cast<const float*>(p);
    if ((rc = upload(b, static_cast<const float*>(in.norm_k), hd, SV2_F32, &p)) != SV2_OK)
        return rc;
    out->norm_k = static_cast<const float*>(p);
    return SV2_OK;
}

sv2_window_rule block_rule(const sv2_block* b)
{
    sv2_window_rule r;
    r.frames = b->T;
    r.height = b->H;
    r.width = b->W;
    r.shifted = b->cfg.shifted_window ? 1 : 0;
    r.wt = b->cfg.window_t;
    r.wh = b->cfg.window_h;
    r.ww = b->cfg.window_w;
    return r;
}

// Makes the block's RoPE table cover the positions this forward needs.  A
// position's row depends only on the rope mode and the block's frequencies,
// and the attention indexes the table with the table's own position count,
// so a table built for more positions serves every smaller need: CFG
// forwards that alternate text lengths reuse it.  Growing enqueues the upload
// of a pinned host copy into a new buffer and retires the old one; nothing
// waits for the stream, so a forward whose table already covers its shape
// launches kernels only (and can be captured in a HIP graph).
int ensure_rope(sv2_block* b, int text_len, hipStream_t stream)
{
    if (b->cfg.rope_mode == SV2_ROPE_NONE)
        return SV2_OK;
    const sv2_window_rule rule = block_rule(b);
    const int npos = sv2_rope_positions_needed(&rule, text_len, b->cfg.rope_mode);
    if (npos < 0)
        return npos;
    if (b->rope && npos <= b->rope_npos)
        return SV2_OK;
    if (b->cfg.rope_mode == SV2_ROPE_REFERENCE && !b->has_freqs)
        return sv2::set_error(SV2_EINVAL, "block: the reference RoPE needs rope_freqs");
    const size_t floats = sv2_rope_table_floats(npos);
    float* host = nullptr;
    hipError_t err = hipHostMalloc(reinterpret_cast<void**>(&host), floats * sizeof(float), hipHostMallocDefault);
    if (err != hipSuccess || !host)
        return sv2::hip_error(err != hipSuccess ? err : hipErrorOutOfMemory, "block: pinned RoPE table");
    b->rope_host.push_back(host);
    int rc = sv2_rope_table_build(b->cfg.rope_mode, b->freqs, 10000.f, npos, host);
    if (rc != SV2_OK)
        return rc;
    float* dev = nullptr;
    err = hipMalloc(reinterpret_cast<void**>(&dev), floats * sizeof(float));
    if (err != hipSuccess || !dev)
        return sv2::hip_error(err != hipSuccess ? err : hipErrorOutOfMemory, "block: hipMalloc of the RoPE table");
    err = hipMemcpyAsync(dev, host, floats * sizeof(float), hipMemcpyHostToDevice, stream);
    if (err != hipSuccess)
    {
        (void)hipFree(dev);
        return sv2::hip_error(err, "block: RoPE table upload");
    }
    if (b->rope)
        b->rope_retired.push_back(b->rope);
    b->rope = dev;
    b->rope_npos = npos;
    return SV2_OK;
}

sv2_attn_args attention_args(const sv2_block* b, int text_len)
{
    sv2_attn_args a;
    std::memset(&a, 0, sizeof(a));
    a.rule = block_rule(b);
    a.heads = b->cfg.heads;
    a.head_dim = b->cfg.head_dim;
    a.text_len = text_len;
    a.eps = b->cfg.norm_eps;
    a.qk_norm = b->cfg.qk_norm;
    a.rope_mode = b->cfg.rope_mode;
    a.rope_table = b->rope;
    a.rope_npos = b->rope_npos;
    a.qkv_dtype = b->dtype;
    a.out_dtype = b->dtype;
    // the fp32 compute mode is the parity mode: the attention in the
    // reference's own order and rounding
    a.exact = b->dtype == SV2_F32 ? 1 : 0;
    const DevBranch& tb = b->cfg.shared_weights ? b->vid : b->txt;
    a.gamma_q_vid = b->vid.norm_q;
    a.gamma_k_vid = b->vid.norm_k;
    a.gamma_q_txt = tb.norm_q;
    a.gamma_k_txt = tb.norm_k;
    return a;
}

// Workspace regions (bytes, 256-aligned): xa / m [R, D], qkv [R, 3D], att [R, D],
// p_v [Lv, D], p_t [Lt, D], g and u [R, F], the few-row InnerProducts' partial
// sums (fp16 text rows), attention workspace; R = max(Lv, Lt).
struct BlockWorkspace
{
    size_t tables, xa, qkv_v, qkv_t, att_v, att_t, p_v, p_t, g, u, few, few_bytes, attn, total;
};

// The text branch's InnerProducts run on the few-row kernel (gemm_few.hip)
// when the compute type is fp16 and every one of its shapes fits it.
bool few_text_products(const sv2_block* b, int text_len)
{
    using namespace sv2;
    const int D = b->cfg.dim, F = b->cfg.mlp_hidden;
    return b->dtype == SV2_F16 && gemm_few_supported(text_len, D, 3 * D, kGemmStore) &&
           gemm_few_supported(text_len, D, D, kGemmResidual) && gemm_few_supported(text_len, D, F, kGemmSwiGLU) &&
           gemm_few_supported(text_len, F, D, kGemmResidual);
}

size_t align256(size_t v)
{
    return (v + 255) & ~static_cast<size_t>(255);
}

int workspace_layout(const sv2_block* b, int text_len, BlockWorkspace* w)
{
    const size_t es = dtype_size(b->dtype);
    const size_t D = b->cfg.dim, F = b->cfg.mlp_hidden;
    const size_t Lv = static_cast<size_t>(b->T) * b->H * b->W, Lt = text_len;
    // rows of the normalised input and of the MLP's gate / value: the video
    // and text rows together when the row-wise steps run merged
    const size_t R = Lv + Lt;
    sv2_attn_args a = attention_args(b, text_len);
    a.vid_qkv = reinterpret_cast<const void*>(16); // placeholders: the size query reads no memory
    a.txt_qkv = reinterpret_cast<const void*>(16);
    if (a.rope_mode != SV2_ROPE_NONE)
    {
        a.rope_table = reinterpret_cast<const float*>(16);
        const sv2_window_rule rule = block_rule(b);
        a.rope_npos = sv2_rope_positions_needed(&rule, text_len, a.rope_mode);
        if (a.rope_npos < 0)
            return a.rope_npos;
    }
    if (a.qk_norm && (!a.gamma_q_vid || !a.gamma_k_vid))
        return sv2::set_error(SV2_EINVAL, "block: missing norm weights");
    const int64_t attn = sv2_window_attention_workspace(&a);
    if (attn < 0)
        return static_cast<int>(attn);
    size_t off = 0;
    // four ada tables [3][D] fp32 (video attention, video MLP, text attention,
    // text MLP), then the video projection's bias times its gate [D]
    w->tables = off;
    off = align256(off + 13 * D * sizeof(float));
    w->xa = off;
    off = align256(off + R * D * es);
    w->qkv_v = off;
    off = align256(off + Lv * 3 * D * es);
    w->qkv_t = off;
    off = align256(off + Lt * 3 * D * es);
    w->att_v = off;
    off = align256(off + Lv * D * es);
    w->att_t = off;
    off = align256(off + Lt * D * es);
    w->p_v = off;
    off = align256(off + Lv * D * es);
    w->p_t = off;
    off = align256(off + Lt * D * es);
    w->g = off;
    off = align256(off + R * F * es);
    w->u = off;
    off = align256(off + R * F * es);
    w->few = off;
    w->few_bytes = 0;
    if (few_text_products(b, text_len))
    {
        const int d = b->cfg.dim, f = b->cfg.mlp_hidden;
        w->few_bytes = std::max({sv2::gemm_few_workspace(text_len, d, 3 * d, sv2::kGemmStore),
                                 sv2::gemm_few_workspace(text_len, d, d, sv2::kGemmResidual),
                                 sv2::gemm_few_workspace(text_len, f, d, sv2::kGemmResidual)});
    }
    off = align256(off + w->few_bytes);
    w->attn = off;
    off = align256(off + static_cast<size_t>(attn));
    w->total = off;
    return SV2_OK;
}

// The MLP of one branch on rows [rows, D]: RMSNorm + ada (mlp shift/scale),
// gate and in InnerProducts, SwiGLU, out InnerProduct, gated residual with x
// (seedvr2_dit_block.cpp:1093-1112, :1211-1223, :1248-1260).  `table` is the
// branch's MLP modulation table.  `fused`: the hand-written MFMA products
// with their passes fused in; `few` (text rows): the few-row kernel, the
// same fusion, partial sums in few_ws.
int branch_mlp(const sv2_block* b, hipStream_t stream, const DevBranch& br, const float* table, const void* x,
               int rows, void* out, char* m, char* g, char* u, bool fused, bool few = false, char* few_ws = nullptr,
               size_t few_bytes = 0)
{
    using namespace sv2;
    if (rows == 0)
        return SV2_OK;
    const int D = b->cfg.dim, F = b->cfg.mlp_hidden, dt = b->dtype;
    int rc;
    if ((rc = launch_rmsnorm_table(x, m, dt, rows, D, b->cfg.norm_eps, table, br.ada[3], nullptr, 1, stream)) !=
        SV2_OK)
        return rc;
    if (fused)
    {
        // gate/in products with the SwiGLU gate, then the out product with
        // the gated residual (mlp_gate is the table's third row)
        if ((rc = gemm_mfma(stream, rows, D, F, m, br.w_gate, br.w_in, g, kGemmSwiGLU, nullptr, nullptr,
                            nullptr)) != SV2_OK)
            return rc;
        return gemm_mfma(stream, rows, F, D, g, br.w_out, nullptr, out, kGemmResidual, nullptr, table + 2 * D, x);
    }
    if (few)
    {
        if ((rc = gemm_few(stream, rows, D, F, m, br.w_gate, br.w_in, g, kGemmSwiGLU, nullptr, nullptr, nullptr,
                           few_ws, few_bytes)) != SV2_OK)
            return rc;
        return gemm_few(stream, rows, F, D, g, br.w_out, nullptr, out, kGemmResidual, nullptr, table + 2 * D, x,
                        few_ws, few_bytes);
    }
    if ((rc = gemm_rows(stream, dt, rows, D, F, m, br.w_gate, g)) != SV2_OK ||
        (rc = gemm_rows(stream, dt, rows, D, F, m, br.w_in, u)) != SV2_OK)
        return rc;
    if ((rc = sv2_swiglu(g, u, dt, static_cast<int64_t>(rows) * F, stream)) != SV2_OK)
        return rc;
    if (dt == SV2_F16)
    {
        // the gated residual in the out product's epilogue
        rc = gemm_rows_gated(stream, dt, rows, F, D, g, br.w_out, out, table + 2 * D, x);
        if (rc != SV2_EUNSUPPORTED)
            return rc;
    }
    if ((rc = gemm_rows(stream, dt, rows, F, D, g, br.w_out, out)) != SV2_OK)
        return rc;
    return launch_residual_table(out, x, dt, rows, D, table, nullptr, 0, stream);
}

} // namespace

int sv2::upload_weights(std::vector<void*>* owned, const float* host, size_t count, int dtype, const void** dev)
{
    void* p = nullptr;
    const size_t bytes = count * (dtype == SV2_F32 ? 4 : 2);
    hipError_t err = hipMalloc(&p, bytes ? bytes : 4);
    if (err != hipSuccess)
        return sv2::hip_error(err, "hipMalloc of weights");
    owned->push_back(p);
    if (dtype == SV2_F32)
    {
        err = hipMemcpy(p, host, bytes, hipMemcpyHostToDevice);
    }
    else
    {
        std::vector<_Float16> half(count);
        for (size_t i = 0; i < count; i++)
            half[i] = static_cast<_Float16>(host[i]);
        err = hipMemcpy(p, half.data(), bytes, hipMemcpyHostToDevice);
    }
    if (err != hipSuccess)
        return sv2::hip_error(err, "hipMemcpy of weights");
    *dev = p;
    return SV2_OK;
}

int sv2::block_compute_dtype(const sv2_block* block)
{
    return block->dtype;
}

extern "C" {

void sv2_block_config_default(sv2_block_config* c)
{
    if (!c)
        return;
    std::memset(c, 0, sizeof(*c));
    c->dim = 2560;
    c->heads = 20;
    c->head_dim = 128;
    c->mlp_hidden = 6912;
    c->norm_eps = 1e-5f;
    c->rope_mode = SV2_ROPE_REFERENCE;
    c->qk_norm = 1;
    c->fused_gemm = 0;
}

int sv2_block_create(const sv2_block_config* config, const sv2_block_branch* vid, const sv2_block_branch* txt,
                     const float* rope_freqs, int weights_on_device, int compute_dtype, sv2_block** out)
try
{
    using namespace sv2;
    if (!config || !vid || !out || (!config->shared_weights && !txt))
        return set_error(SV2_EINVAL, "sv2_block_create: null argument");
    *out = nullptr;
    int rc = validate_config(*config);
    if (rc != SV2_OK)
        return rc;
    if (compute_dtype != SV2_F32 && compute_dtype != SV2_F16)
        return set_error(SV2_EINVAL, "sv2_block_create: compute dtype must be SV2_F32 or SV2_F16");
    sv2_block* b = new sv2_block();
    b->cfg = *config;
    b->dtype = compute_dtype;
    if (rope_freqs)
    {
        std::memcpy(b->freqs, rope_freqs, sizeof(b->freqs));
        b->has_freqs = true;
    }
    if ((rc = bind_branch(b, *vid, weights_on_device != 0, &b->vid)) == SV2_OK && !config->shared_weights)
        rc = bind_branch(b, *txt, weights_on_device != 0, &b->txt);
    if (rc != SV2_OK)
    {
        delete b;
        return rc;
    }
    if (config->shared_weights)
        b->txt = b->vid;
    *out = b;
    return SV2_OK;
}
catch (...)
{
    return sv2::caught_exception("sv2_block_create");
}

int sv2_block_load(const char* param_path, const char* bin_path, int compute_dtype, sv2_block** out)
try
{
    using namespace sv2;
    if (!param_path || !bin_path || !out)
        return set_error(SV2_EINVAL, "sv2_block_load: null argument");
    *out = nullptr;
    std::vector<ParamLayer> layers;
    std::string err;
    if (read_param_file(param_path, &layers, &err) != 0)
        return set_error(SV2_EINVAL, "sv2_block_load: " + err);
    const ParamLayer* layer = nullptr;
    for (const ParamLayer& l : layers)
        if (l.type == "SeedVR2DiTBlock")
            layer = &l;
    if (!layer)
        return set_error(SV2_EINVAL, std::string("sv2_block_load: no SeedVR2DiTBlock layer in ") + param_path);
    if (layer->bottoms.size() != 4 || layer->tops.size() != 2)
        return set_error(SV2_EINVAL, "sv2_block_load: SeedVR2DiTBlock needs 4 bottoms and 2 tops");
    sv2_block_config c;
    sv2_block_config_default(&c);
    c.block_index = layer->get_int(0, 0);
    c.shared_weights = layer->get_int(1, 0) != 0;
    c.last_layer = layer->get_int(2, 0) != 0;
    c.shifted_window = layer->get_int(3, 0) != 0;
    c.dim = layer->get_int(4, 2560);
    c.heads = layer->get_int(5, 20);
    c.head_dim = layer->get_int(6, 128);
    c.mlp_hidden = layer->get_int(7, 6912);
    c.norm_eps = layer->get_float(8, 1e-5f);
    c.window_t = layer->get_int(9, 0);
    c.window_h = layer->get_int(10, 0);
    c.window_w = layer->get_int(11, 0);
    c.rope_mode = layer->get_int(12, SV2_ROPE_REFERENCE);
    c.qk_norm = layer->get_int(13, 1) != 0;
    c.fused_gemm = layer->get_int(14, 0) != 0;
    int rc = validate_config(c);
    if (rc != SV2_OK)
        return rc;

    // weight order of load_branch / load_model (seedvr2_dit_block.cpp:657-688)
    BinReader bin;
    if (bin.open(bin_path, &err) != 0)
        return set_error(SV2_EDEVICE, "sv2_block_load: " + err);
    const size_t D = c.dim, F = c.mlp_hidden, hd = c.head_dim;
    struct HostBranch
    {
        std::vector<float> ada[6], w_qkv, w_proj, b_proj, norm_q, norm_k, w_gate, w_in, w_out;
    };
    HostBranch hb[2];
    const int nbranch = c.shared_weights ? 1 : 2;
    for (int bi = 0; bi < nbranch; bi++)
    {
        HostBranch& h = hb[bi];
        bool ok = true;
        for (int i = 0; i < 6 && ok; i++)
            ok = bin.load_raw(D, &h.ada[i], &err) == 0;
        ok = ok && bin.load_tagged(3 * D * D, &h.w_qkv, &err) == 0;
        ok = ok && bin.load_tagged(D * D, &h.w_proj, &err) == 0;
        ok = ok && bin.load_raw(D, &h.b_proj, &err) == 0;
        ok = ok && bin.load_raw(hd, &h.norm_q, &err) == 0;
        ok = ok && bin.load_raw(hd, &h.norm_k, &err) == 0;
        ok = ok && bin.load_tagged(F * D, &h.w_gate, &err) == 0;
        ok = ok && bin.load_tagged(F * D, &h.w_in, &err) == 0;
        ok = ok && bin.load_tagged(D * F, &h.w_out, &err) == 0;
        if (!ok)
            return set_error(SV2_EDEVICE, std::string("sv2_block_load: ") + bin_path + ": " + err);
    }
    std::vector<float> freqs;
    if (bin.load_raw(21, &freqs, &err) != 0)
        return set_error(SV2_EDEVICE, std::string("sv2_block_load: ") + bin_path + ": rope freqs: " + err);
    auto view = [](const HostBranch& h) {
        sv2_block_branch v;
        for (int i = 0; i < 6; i++)
            v.ada[i] = h.ada[i].data();
        v.w_qkv = h.w_qkv.data();
        v.w_proj = h.w_proj.data();
        v.b_proj = h.b_proj.data();
        v.norm_q = h.norm_q.data();
        v.norm_k = h.norm_k.data();
        v.w_gate = h.w_gate.data();
        v.w_in = h.w_in.data();
        v.w_out = h.w_out.data();
        return v;
    };
    const sv2_block_branch vb = view(hb[0]);
    const sv2_block_branch tb = view(hb[nbranch - 1]);
    return sv2_block_create(&c, &vb, &tb, freqs.data(), 0, compute_dtype, out);
}
catch (...)
{
    return sv2::caught_exception("sv2_block_load");
}

int sv2_block_get_config(const sv2_block* block, sv2_block_config* config)
try
{
    if (!block || !config)
        return sv2::set_error(SV2_EINVAL, "sv2_block_get_config: null argument");
    *config = block->cfg;
    return SV2_OK;
}
catch (...)
{
    return sv2::caught_exception("sv2_block_get_config");
}

int sv2_block_set_runtime_shape(sv2_block* block, int frames, int height, int width)
try
{
    if (!block)
        return sv2::set_error(SV2_EINVAL, "sv2_block_set_runtime_shape: null block");
    block->T = frames;
    block->H = height;
    block->W = width;
    block->shape_valid = frames > 0 && height > 0 && width > 0;
    return block->shape_valid ? SV2_OK : sv2::set_error(SV2_EINVAL, "sv2_block_set_runtime_shape: bad shape");
}
catch (...)
{
    return sv2::caught_exception("sv2_block_set_runtime_shape");
}

int64_t sv2_block_workspace_size(const sv2_block* block, int text_len)
try
{
    using namespace sv2;
    if (!block || text_len < 0)
        return set_error(SV2_EINVAL, "sv2_block_workspace_size: bad argument");
    if (!block->shape_valid)
        return set_error(SV2_EINVAL, "sv2_block_workspace_size: runtime shape not set");
    BlockWorkspace w;
    const int rc = workspace_layout(block, text_len, &w);
    return rc == SV2_OK ? static_cast<int64_t>(w.total) : rc;
}
catch (...)
{
    return sv2::caught_exception("sv2_block_workspace_size");
}

int sv2_block_forward(sv2_block* b, const void* vid, const void* txt, int text_len, const float* emb, void* vid_out,
                      void* txt_out, void* workspace, size_t workspace_bytes, void* stream_ptr)
try
{
    using namespace sv2;
    if (!b || !vid || !emb || !vid_out || text_len < 0 || (text_len > 0 && (!txt || !txt_out)))
        return set_error(SV2_EINVAL, "sv2_block_forward: null argument or bad text length");
    if (!b->shape_valid)
        return set_error(SV2_EINVAL, "sv2_block_forward: set_runtime_shape was not called");
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    BlockWorkspace w;
    int rc = workspace_layout(b, text_len, &w);
    if (rc != SV2_OK)
        return rc;
    char* ws = static_cast<char*>(workspace);
    if (ws)
    {
        if (workspace_bytes < w.total)
            return set_error(SV2_EINVAL, "sv2_block_forward: workspace too small");
    }
    else
    {
        if (b->ws_bytes < w.total)
        {
            if (b->ws)
            {
                hipError_t err = hipStreamSynchronize(stream); // queued work may still use the old buffer
                if (err != hipSuccess)
                    return hip_error(err, "sv2_block_forward: synchronize before workspace resize");
                (void)hipFree(b->ws);
                b->ws = nullptr;
                b->ws_bytes = 0;
            }
            hipError_t err = hipMalloc(&b->ws, w.total);
            if (err != hipSuccess)
            {
                b->ws = nullptr;
                return hip_error(err, "sv2_block_forward: workspace allocation");
            }
            b->ws_bytes = w.total;
        }
        ws = static_cast<char*>(b->ws);
    }
    if ((rc = ensure_rope(b, text_len, stream)) != SV2_OK)
        return rc;

    const sv2_block_config& c = b->cfg;
    const int D = c.dim, dt = b->dtype;
    const int Lv = b->T * b->H * b->W, Lt = text_len;
    const DevBranch& vb = b->vid;
    const DevBranch& tb = c.shared_weights ? b->vid : b->txt;
    char* xa = ws + w.xa;
    char* qkv_v = ws + w.qkv_v;
    char* qkv_t = ws + w.qkv_t;
    char* att_v = ws + w.att_v;
    char* att_t = ws + w.att_t;
    char* p_v = ws + w.p_v;
    char* p_t = ws + w.p_t;
    char* g = ws + w.g;
    char* u = ws + w.u;
    const size_t es = dtype_size(dt);

    // ada modulation tables of this layer: the emb blob's slots combined with
    // the branch vectors once, read as contiguous rows by the kernels below
    float* tables = reinterpret_cast<float*>(ws + w.tables);
    float* tab_va = tables;
    float* tab_vm = tables + 3 * D;
    float* tab_ta = tables + 6 * D;
    float* tab_tm = tables + 9 * D;
    const sv2_block_debug* dbg = b->debug_on ? &b->debug : nullptr;
    // With shared weights outside the last layer the text rows get the video
    // rows' treatment in every step but the attention: the same branch (:1139)
    // and the same ada slots of the same emb, so the same tables.  When the
    // caller's text rows follow its video rows in memory (as the DiT lays its
    // hidden streams out) and this layout's text regions follow the video
    // ones, each row-wise step (RMSNorm + ada, the InnerProducts, the gated
    // residuals, SwiGLU) runs once over all Lv + Lt rows.
    const size_t row_bytes = static_cast<size_t>(D) * es;
    const bool merged = c.shared_weights && !c.last_layer && Lt > 0 && !dbg &&
                        static_cast<const char*>(txt) == static_cast<const char*>(vid) + Lv * row_bytes &&
                        static_cast<const char*>(txt_out) == static_cast<const char*>(vid_out) + Lv * row_bytes &&
                        qkv_t == qkv_v + 3 * Lv * row_bytes && att_t == att_v + Lv * row_bytes &&
                        p_t == p_v + Lv * row_bytes;
    const int Lr = merged ? Lv + Lt : Lv; // rows of the video branch's row-wise steps
    b->last_merged = merged ? 1 : 0;
    // unmerged fp16 text rows (at most 64) take the few-row InnerProducts
    // with their passes fused; debug captures need the separate passes
    const bool few = Lt > 0 && !merged && !dbg && few_text_products(b, Lt);
    // the video branch on the fused MFMA InnerProducts (param 14)
    const bool fused = c.fused_gemm && dt == SV2_F16 && !dbg;
    // the library path's gated projection adds the bias after the gate
    const bool gated_bias = !fused && dt == SV2_F16 && !dbg && Lv > 0 && vb.b_proj;
    // the layer's tables in one launch: video attention and MLP, then the
    // unmerged text rows' (tab_ta, tab_tm), then the gated bias
    {
        const float* scales[4] = {vb.ada[1], vb.ada[4], tb.ada[1], tb.ada[4]};
        const float* gates[4] = {vb.ada[2], vb.ada[5], tb.ada[2], tb.ada[5]};
        if ((rc = launch_block_tables(emb, scales, gates, (Lt > 0 && !merged) ? 4 : 2,
                                      gated_bias ? vb.b_proj : nullptr, D, tables, stream)) != SV2_OK)
            return rc;
    }
    // token RMSNorm + ada input; text skips the ada on the last layer (:1141-1151)
    if ((rc = launch_rmsnorm_table(vid, xa, dt, Lr, D, c.norm_eps, tab_va, vb.ada[0], nullptr, 1, stream)) != SV2_OK)
        return rc;
    if ((rc = fused ? gemm_mfma(stream, Lr, D, 3 * D, xa, vb.w_qkv, nullptr, qkv_v, kGemmStore, nullptr, nullptr,
                                nullptr)
                    : gemm_rows(stream, dt, Lr, D, 3 * D, xa, vb.w_qkv, qkv_v)) != SV2_OK)
        return rc;
    auto capture = [&](float* dst, const void* src, int rows, int cols) {
        return dst ? launch_to_f32(dst, src, dt, static_cast<long long>(rows) * cols, stream) : SV2_OK;
    };
    // the projection before the gate: proj_out + bias, in fp32 (bias NULL:
    // the product already holds it)
    auto capture_projected = [&](float* dst, const void* src, const float* bias, int rows) {
        if (!dst)
            return SV2_OK;
        const int r = launch_to_f32(dst, src, dt, static_cast<long long>(rows) * D, stream);
        return (r != SV2_OK || !bias) ? r : launch_bias_rows(dst, bias, SV2_F32, rows, D, stream);
    };
    // fp32: the proj_out bias enters the product's double sum before its one
    // rounding, as in the InnerProduct; fp16: the gated residual pass adds it
    const float* vbias_in_product = dt == SV2_F32 ? vb.b_proj : nullptr;
    const float* vbias_in_residual = dt == SV2_F32 ? nullptr : vb.b_proj;
    const float* tbias_in_product = dt == SV2_F32 ? tb.b_proj : nullptr;
    const float* tbias_in_residual = dt == SV2_F32 ? nullptr : tb.b_proj;
    if (dbg && (rc = capture(dbg->qkv_vid, qkv_v, Lv, 3 * D)) != SV2_OK)
        return rc;
    if (Lt > 0 && !merged)
    {
        if ((rc = launch_rmsnorm_table(txt, xa, dt, Lt, D, c.norm_eps, tab_ta, tb.ada[0], nullptr,
                                       c.last_layer ? 0 : 1, stream)) != SV2_OK)
            return rc;
        if ((rc = few ? gemm_few(stream, Lt, D, 3 * D, xa, tb.w_qkv, nullptr, qkv_t, kGemmStore, nullptr, nullptr,
                                 nullptr, ws + w.few, w.few_bytes)
                      : gemm_rows(stream, dt, Lt, D, 3 * D, xa, tb.w_qkv, qkv_t)) != SV2_OK)
            return rc;
        if (dbg && (rc = capture(dbg->qkv_txt, qkv_t, Lt, 3 * D)) != SV2_OK)
            return rc;
    }
    // windowed joint attention (:870-1091)
    sv2_attn_args a = attention_args(b, text_len);
    a.vid_qkv = qkv_v;
    a.txt_qkv = Lt > 0 ? qkv_t : nullptr;
    a.vid_out = att_v;
    a.txt_out = Lt > 0 ? att_t : nullptr;
    a.workspace = ws + w.attn;
    a.workspace_bytes = w.total - w.attn;
    if (dbg)
    {
        // the prologue's captures from this forward's own qkv: norm_q/k before
        // RoPE, attention_q/k/v in window-sequence order (:908-918, :1030-1043)
        if ((rc = sv2::attention_captures(&a, dbg->attention_q, dbg->attention_k, dbg->attention_v,
                                          dbg->norm_q_vid, dbg->norm_k_vid, Lt > 0 ? dbg->norm_q_txt : nullptr,
                                          Lt > 0 ? dbg->norm_k_txt : nullptr, stream)) != SV2_OK)
            return rc;
        a.debug_pre = dbg->attention_output;
    }
    if ((rc = sv2_window_attention(&a, stream)) != SV2_OK)
        return rc;
    if (dbg && dbg->attention_output)
    {
        // every query's output per window, rounded to bf16 where the kernel
        // (and the reference, :1074) rounds it
        const int nwin = sv2_window_plan(&a.rule, nullptr, 0);
        if (nwin < 0)
            return nwin;
        const long long seq_rows = static_cast<long long>(Lv) + static_cast<long long>(nwin) * Lt;
        if ((rc = sv2::launch_bf16_round(dbg->attention_output, seq_rows * D, stream)) != SV2_OK)
            return rc;
    }
    if (dbg && ((rc = capture(dbg->attention_vid, att_v, Lv, D)) != SV2_OK ||
                (Lt > 0 && (rc = capture(dbg->attention_txt, att_t, Lt, D)) != SV2_OK)))
        return rc;
    // output projections; their bias is added in the gated residual (:1180-1209)
    if (fused)
    {
        if ((rc = gemm_mfma(stream, Lr, D, D, att_v, vb.w_proj, nullptr, p_v, kGemmResidual, vb.b_proj,
                            tab_va + 2 * D, vid)) != SV2_OK)
            return rc;
    }
    else
    {
        // fp16 without debug captures: the gated residual (bias moved past the
        // gate) in the product's epilogue
        rc = SV2_EUNSUPPORTED;
        if (dt == SV2_F16 && !dbg && Lv > 0)
        {
            rc = gemm_rows_gated(stream, dt, Lr, D, D, att_v, vb.w_proj, p_v, tab_va + 2 * D, vid,
                                 gated_bias ? tables + 12 * D : nullptr);
            if (rc != SV2_OK && rc != SV2_EUNSUPPORTED)
                return rc;
        }
        if (rc == SV2_EUNSUPPORTED)
        {
            if ((rc = gemm_rows_bias(stream, dt, Lr, D, D, att_v, vb.w_proj, vbias_in_product, p_v)) != SV2_OK)
                return rc;
            if (dbg && (rc = capture_projected(dbg->projected_vid, p_v, vbias_in_residual, Lv)) != SV2_OK)
                return rc;
            if ((rc = launch_residual_table(p_v, vid, dt, Lr, D, tab_va, vbias_in_residual, 0, stream)) != SV2_OK)
                return rc;
        }
    }
    if (Lt > 0 && !merged && few)
    {
        // proj_out of the text rows with its bias and the (gated, or on the
        // last layer plain) residual in the epilogue (:1180-1209)
        if ((rc = gemm_few(stream, Lt, D, D, att_t, tb.w_proj, nullptr, p_t, kGemmResidual, tb.b_proj,
                           c.last_layer ? nullptr : tab_ta + 2 * D, txt, ws + w.few, w.few_bytes)) != SV2_OK)
            return rc;
    }
    else if (Lt > 0 && !merged)
    {
        if ((rc = gemm_rows_bias(stream, dt, Lt, D, D, att_t, tb.w_proj, tbias_in_product, p_t)) != SV2_OK)
            return rc;
        if (dbg && (rc = capture_projected(dbg->projected_txt, p_t, tbias_in_residual, Lt)) != SV2_OK)
            return rc;
        // the last layer adds the plain residual (:1198-1209)
        if ((rc = launch_residual_table(p_t, txt, dt, Lt, D, tab_ta, tbias_in_residual, c.last_layer ? 1 : 0,
                                        stream)) != SV2_OK)
            return rc;
    }
    // MLPs (:1211-1260); the last layer's text output is 2 * txt_proj (:1225-1246)
    if ((rc = branch_mlp(b, stream, vb, tab_vm, p_v, Lr, vid_out, xa, g, u, fused)) != SV2_OK)
        return rc;
    if (Lt > 0 && !merged)
    {
        if (c.last_layer)
        {
            hipError_t err = hipMemcpyAsync(txt_out, p_t, static_cast<size_t>(Lt) * D * es, hipMemcpyDeviceToDevice,
                                            stream);
            if (err != hipSuccess)
                return hip_error(err, "sv2_block_forward: text copy");
            if ((rc = launch_residual_table(txt_out, nullptr, dt, Lt, D, nullptr, nullptr, 2, stream)) != SV2_OK)
                return rc;
        }
        else if ((rc = branch_mlp(b, stream, tb, tab_tm, p_t, Lt, txt_out, xa, g, u, false, few, ws + w.few,
                                  w.few_bytes)) != SV2_OK)
        {
            return rc;
        }
    }
    if (dbg && ((rc = capture(dbg->output_vid, vid_out, Lv, D)) != SV2_OK ||
                (Lt > 0 && (rc = capture(dbg->output_txt, txt_out, Lt, D)) != SV2_OK)))
        return rc;
    return SV2_OK;
}
catch (...)
{
    return sv2::caught_exception("sv2_block_forward");
}

int sv2_block_last_forward_merged(const sv2_block* block)
{
    if (!block)
        return sv2::set_error(SV2_EINVAL, "sv2_block_last_forward_merged: null block");
    return block->last_merged;
}

int64_t sv2_block_window_rows(const sv2_block* block, int text_len)
try
{
    using namespace sv2;
    if (!block || text_len < 0)
        return set_error(SV2_EINVAL, "sv2_block_window_rows: bad argument");
    if (!block->shape_valid)
        return set_error(SV2_EINVAL, "sv2_block_window_rows: runtime shape not set");
    const sv2_window_rule rule = block_rule(block);
    const int n = sv2_window_plan(&rule, nullptr, 0);
    if (n < 0)
        return n;
    std::vector<sv2_window> wins(n);
    if (sv2_window_plan(&rule, wins.data(), n) != n)
        return set_error(SV2_EINVAL, "sv2_block_window_rows: window plan changed");
    int64_t rows = 0;
    for (const sv2_window& w : wins)
        rows += int64_t(w.t1 - w.t0) * (w.h1 - w.h0) * (w.w1 - w.w0) + text_len;
    return rows;
}
catch (...)
{
    return sv2::caught_exception("sv2_block_window_rows");
}

int sv2_block_forward_host(sv2_block* b, const float* vid, const float* txt, int text_len, const float* emb,
                           float* vid_out, float* txt_out, const sv2_block_debug* host_debug)
try
{
    using namespace sv2;
    if (!b || !vid || !emb || !vid_out || text_len < 0 || (text_len > 0 && (!txt || !txt_out)))
        return set_error(SV2_EINVAL, "sv2_block_forward_host: null argument or bad text length");
    if (!b->shape_valid)
        return set_error(SV2_EINVAL, "sv2_block_forward_host: set_runtime_shape was not called");
    const int64_t D = b->cfg.dim, Lv = int64_t(b->T) * b->H * b->W, Lt = text_len;
    const int64_t S = host_debug ? sv2_block_window_rows(b, text_len) : 0;
    if (S < 0)
        return static_cast<int>(S);
    const int dt = b->dtype;
    const size_t es = dtype_size(dt);

    // staging layout: fp32 inputs and outputs, their compute-dtype copies
    // (fp16 mode only) and the captures the caller asked for, each 256-byte aligned
    size_t total = 0;
    auto take = [&total](size_t bytes) {
        const size_t at = total;
        total += (bytes + 255) & ~size_t(255);
        return at;
    };
    const size_t o_vid = take(Lv * D * 4), o_txt = take(Lt * D * 4), o_emb = take(6 * D * 4);
    const size_t o_vout = take(Lv * D * 4), o_tout = take(Lt * D * 4);
    const bool cast = dt != SV2_F32;
    const size_t o_vc = cast ? take(Lv * D * es) : 0, o_tc = cast ? take(Lt * D * es) : 0;
    const size_t o_voc = cast ? take(Lv * D * es) : 0, o_toc = cast ? take(Lt * D * es) : 0;
    // the captures: host pointer, device offset, element count (field order of sv2_block_debug)
    struct Capture
    {
        float* host;
        size_t offset;
        int64_t count;
    };
    float* sv2_block_debug::*const fields[16] = {
        &sv2_block_debug::qkv_vid,       &sv2_block_debug::qkv_txt,       &sv2_block_debug::attention_vid,
        &sv2_block_debug::attention_txt, &sv2_block_debug::projected_vid, &sv2_block_debug::projected_txt,
        &sv2_block_debug::output_vid,    &sv2_block_debug::output_txt,    &sv2_block_debug::norm_q_vid,
        &sv2_block_debug::norm_q_txt,    &sv2_block_debug::norm_k_vid,    &sv2_block_debug::norm_k_txt,
        &sv2_block_debug::attention_q,   &sv2_block_debug::attention_k,   &sv2_block_debug::attention_v,
        &sv2_block_debug::attention_output};
    const int64_t counts[16] = {Lv * 3 * D, Lt * 3 * D, Lv * D, Lt * D, Lv * D, Lt * D, Lv * D, Lt * D,
                                Lv * D,     Lt * D,     Lv * D, Lt * D, S * D,  S * D,  S * D,  S * D};
    std::vector<Capture> caps;
    for (int i = 0; host_debug && i < 16; i++)
        if (host_debug->*fields[i] && counts[i] > 0)
            caps.push_back({host_debug->*fields[i], take(size_t(counts[i]) * 4), counts[i]});

    if (b->stage_bytes < total)
    {
        if (b->stage)
            (void)hipFree(b->stage);
        b->stage = nullptr;
        b->stage_bytes = 0;
        hipError_t err = hipMalloc(&b->stage, total);
        if (err != hipSuccess)
        {
            b->stage = nullptr;
            return hip_error(err, "sv2_block_forward_host: staging allocation");
        }
        b->stage_bytes = total;
    }
    char* st = static_cast<char*>(b->stage);
    auto dev = [st](size_t off) { return reinterpret_cast<float*>(st + off); };
    hipStream_t stream = nullptr;
    hipError_t err = hipMemcpy(dev(o_vid), vid, Lv * D * 4, hipMemcpyHostToDevice);
    if (err == hipSuccess && Lt > 0)
        err = hipMemcpy(dev(o_txt), txt, Lt * D * 4, hipMemcpyHostToDevice);
    if (err == hipSuccess)
        err = hipMemcpy(dev(o_emb), emb, 6 * D * 4, hipMemcpyHostToDevice);
    if (err != hipSuccess)
        return hip_error(err, "sv2_block_forward_host: upload");
    int rc = SV2_OK;
    void* vin = dev(o_vid);
    void* tin = dev(o_txt);
    void* vout = dev(o_vout);
    void* tout = dev(o_tout);
    if (cast)
    {
        vin = st + o_vc;
        tin = st + o_tc;
        vout = st + o_voc;
        tout = st + o_toc;
        if ((rc = launch_from_f32(vin, dev(o_vid), dt, Lv * D, stream)) != SV2_OK ||
            (Lt > 0 && (rc = launch_from_f32(tin, dev(o_txt), dt, Lt * D, stream)) != SV2_OK))
            return rc;
    }

    // the captures go to the staging copies for this call only
    const bool saved_on = b->debug_on;
    const sv2_block_debug saved = b->debug;
    if (host_debug)
    {
        sv2_block_debug d{};
        for (const Capture& c : caps)
            for (int i = 0; i < 16; i++)
                if (host_debug->*fields[i] == c.host)
                    d.*fields[i] = dev(c.offset);
        b->debug = d;
        b->debug_on = true;
    }
    rc = sv2_block_forward(b, vin, Lt > 0 ? tin : nullptr, text_len, dev(o_emb), vout, Lt > 0 ? tout : nullptr,
                           nullptr, 0, stream);
    b->debug_on = saved_on;
    b->debug = saved;
    if (rc != SV2_OK)
        return rc;
    if (cast && ((rc = launch_to_f32(dev(o_vout), vout, dt, Lv * D, stream)) != SV2_OK ||
                 (Lt > 0 && (rc = launch_to_f32(dev(o_tout), tout, dt, Lt * D, stream)) != SV2_OK)))
        return rc;
    err = hipMemcpy(vid_out, dev(o_vout), Lv * D * 4, hipMemcpyDeviceToHost);
    if (err == hipSuccess && Lt > 0)
        err = hipMemcpy(txt_out, dev(o_tout), Lt * D * 4, hipMemcpyDeviceToHost);
    for (size_t i = 0; err == hipSuccess && i < caps.size(); i++)
        err = hipMemcpy(caps[i].host, dev(caps[i].offset), size_t(caps[i].count) * 4, hipMemcpyDeviceToHost);
    return err == hipSuccess ? SV2_OK : hip_error(err, "sv2_block_forward_host: download");
}
catch (...)
{
    return sv2::caught_exception("sv2_block_forward_host");
}

int sv2_block_set_debug(sv2_block* block, const sv2_block_debug* debug)
try
{
    if (!block)
        return sv2::set_error(SV2_EINVAL, "sv2_block_set_debug: null block");
    block->debug_on = debug != nullptr;
    if (debug)
        block->debug = *debug;
    return SV2_OK;
}
catch (...)
{
    return sv2::caught_exception("sv2_block_set_debug");
}

void sv2_block_destroy(sv2_block* block)
{
    delete block;
}

} // extern "C"
