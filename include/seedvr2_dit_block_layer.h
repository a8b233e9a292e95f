/* The library's DiT block presented as the reference's ncnn custom layer
 * SeedVR2DiTBlock (src/layers/seedvr2_dit_block.h:38-172).
 *
 * sv2::DiTBlockLayer<Api> derives from Api::Layer and overrides the layer's
 * virtual interface with ncnn's signatures; Api names the five ncnn types:
 *
 *   struct NcnnApi {
 *       using Layer = ncnn::Layer;  using ParamDict = ncnn::ParamDict;
 *       using ModelBin = ncnn::ModelBin;  using Mat = ncnn::Mat;
 *       using Option = ncnn::Option;
 *   };
 *   class SeedVR2DiTBlock : public sv2::DiTBlockLayer<NcnnApi> {};
 *   DEFINE_LAYER_CREATOR(SeedVR2DiTBlock)
 *
 * which is what seedvr2-ncnn-valkan_amd/ncnn/seedvr2_dit_block.cpp holds: a
 * translation unit that replaces src/layers/seedvr2_dit_block.cpp in an ncnn
 * build, so that net.register_custom_layer("SeedVR2DiTBlock",
 * SeedVR2DiTBlock_layer_creator) (src/model/dit.cpp:59) loads the block into
 * this library.  Of the Api types it uses only what ncnn declares:
 *   ParamDict::get(int id, int default), ParamDict::get(int id, float default)
 *   ModelBin::load(int w, int type) -> Mat (type 1 raw fp32, 0 tagged; fp32 data)
 *   Mat: w, h, dims, empty(), create(w, h, elemsize, allocator),
 *        create(w, elemsize, allocator), data
 *   Option: blob_allocator, use_fp16_arithmetic
 *   Layer: one_blob_only, support_inplace and the virtuals overridden below.
 *
 * Semantics, as the reference layer:
 *   load_param   ids 0-8 (seedvr2_dit_block.cpp:643-655) and this library's
 *                ids 9-14 (sv2_block_config); -1 when dim != heads * head_dim.
 *   load_model   the branch weights in ModelBin order (:657-688): 6 ada
 *                vectors, qkv, proj_out + bias, norm_q, norm_k, mlp gate, in,
 *                out; the text branch unless shared; then the 21 RoPE
 *                frequencies.  -100 for a record that fails to load.
 *   create_pipeline  uploads the weights (sv2_block_create), fp16 compute
 *                when opt.use_fp16_arithmetic, else fp32 (the parity mode,
 *                the reference's CPU arithmetic); host copies are released.
 *   forward      bottoms vid [L_v, dim], txt [L_t, dim], emb [6*dim],
 *                vid_shape int32 [3] (T, H, W); tops vid_out, txt_out
 *                (fp32 Mats from opt.blob_allocator); -1 for blob counts or
 *                shapes that do not match (:1119-1138), -100 for a failure
 *                of the device forward.  The forward is staged through device
 *                memory (sv2_block_forward_host).
 *   set_runtime_shape / set_debug_tensors  as the reference (:609-620).
 *
 * The device side, in place of the reference's Vulkan path (upload_model
 * :1271-1300, forward over VkMat :1302-1677), with sv2::DeviceMat blobs and an
 * sv2::DeviceCompute (the HIP stream and the device allocators, the roles of
 * VkCompute and opt.blob_vkallocator / opt.workspace_vkallocator):
 *   upload_model the device block from the loaded weights, when
 *                create_pipeline has not made it (a no-op otherwise).
 *   forward      bottoms vid [L_v, dim] and txt [L_t, dim] in the compute
 *                dtype (4-byte elements for fp32, 2-byte for fp16), emb
 *                [6*dim] fp32, vid_shape [3] (checked for size only: the grid
 *                is the one set_runtime_shape injected, as the reference's
 *                Vulkan forward reads it, :1317-1324); tops from
 *                cmd.blob_allocator in the compute dtype.  It only enqueues on
 *                cmd.stream: no host wait, no host copy of any blob.  The
 *                scratch comes from cmd.workspace_allocator and goes back to
 *                it when forward returns, while the enqueued work may still
 *                use it: the allocators must hand a freed buffer only to
 *                work enqueued later on the same stream (a caching pool used
 *                with one stream does).  -1 for blob counts, shapes or
 *                element sizes that do not match or a missing runtime shape,
 *                -100 for a failed allocation or launch.
 */
#pragma once

#include <cstdio>
#include <memory>
#include <vector>

#include "seedvr2_hip.h"

/* hipStream_t as the HIP runtime declares it, so this header needs no HIP
 * headers. */
struct ihipStream_t;
typedef struct ihipStream_t* hipStream_t;

namespace sv2
{

/* Device memory for DeviceMat blobs (ncnn::VkAllocator's role): fastMalloc
 * returns device memory or NULL, fastFree takes it back. */
class DeviceAllocator
{
  public:
    virtual ~DeviceAllocator() = default;
    virtual void* fastMalloc(size_t bytes) = 0;
    virtual void fastFree(void* ptr) = 0;
};

/* A blob in device memory, pack 1, rows of w elements of elemsize bytes
 * (ncnn::VkMat's role for this layer).  Copies share the buffer; the last
 * copy to go returns it to its allocator.  borrow() wraps memory the caller
 * owns. */
struct DeviceMat
{
    int dims = 0;
    int w = 0;
    int h = 0;
    size_t elemsize = 0;
    void* data = nullptr;
    std::shared_ptr<void> mem;

    void create(int w_, size_t es, DeviceAllocator* allocator)
    {
        allocate(1, w_, 1, es, allocator);
    }
    void create(int w_, int h_, size_t es, DeviceAllocator* allocator)
    {
        allocate(2, w_, h_, es, allocator);
    }
    bool empty() const
    {
        return data == nullptr || size_t(w) * size_t(h) == 0;
    }
    void release()
    {
        mem.reset();
        data = nullptr;
        dims = w = h = 0;
        elemsize = 0;
    }
    static DeviceMat borrow(void* ptr, int w_, int h_, size_t es, int dims_ = 2)
    {
        DeviceMat m;
        m.dims = dims_;
        m.w = w_;
        m.h = h_;
        m.elemsize = es;
        m.data = ptr;
        return m;
    }

  private:
    void allocate(int d, int w_, int h_, size_t es, DeviceAllocator* allocator)
    {
        release();
        dims = d;
        w = w_;
        h = h_;
        elemsize = es;
        const size_t bytes = size_t(w_ > 0 ? w_ : 0) * size_t(h_ > 0 ? h_ : 0) * es;
        if (!bytes || !allocator)
            return;
        void* p = allocator->fastMalloc(bytes);
        if (!p)
            return;
        mem = std::shared_ptr<void>(p, [allocator](void* q) { allocator->fastFree(q); });
        data = p;
    }
};

/* Where a device forward records its work (ncnn::VkCompute's role): the HIP
 * stream (NULL: the null stream) and the allocators of the tops and of the
 * scratch. */
struct DeviceCompute
{
    hipStream_t stream = nullptr;
    DeviceAllocator* blob_allocator = nullptr;
    DeviceAllocator* workspace_allocator = nullptr;
};

/* The captures of SeedVR2DiTBlockDebugTensors (seedvr2_dit_block.h:20-36),
 * over the caller's Mat type; forward sizes and fills each one. */
template <class Mat>
struct BlockDebugTensors
{
    Mat qkv_vid;
    Mat qkv_txt;
    Mat norm_q_vid;
    Mat norm_q_txt;
    Mat norm_k_vid;
    Mat norm_k_txt;
    Mat attention_q;
    Mat attention_k;
    Mat attention_v;
    Mat attention_output;
    Mat projected_vid;
    Mat projected_txt;
    Mat output_vid;
    Mat output_txt;
};

template <class Api>
class DiTBlockLayer : public Api::Layer
{
  public:
    using Mat = typename Api::Mat;
    using ParamDict = typename Api::ParamDict;
    using ModelBin = typename Api::ModelBin;
    using Option = typename Api::Option;
    using DebugTensors = BlockDebugTensors<Mat>;

    DiTBlockLayer()
    {
        this->one_blob_only = false;
        this->support_inplace = false;
        sv2_block_config_default(&config_);
    }
    ~DiTBlockLayer() override
    {
        sv2_block_destroy(block_);
    }
    DiTBlockLayer(const DiTBlockLayer&) = delete;
    DiTBlockLayer& operator=(const DiTBlockLayer&) = delete;

    int load_param(const ParamDict& pd) override
    {
        sv2_block_config& c = config_;
        c.block_index = pd.get(0, 0);
        c.shared_weights = pd.get(1, 0) != 0;
        c.last_layer = pd.get(2, 0) != 0;
        c.shifted_window = pd.get(3, 0) != 0;
        c.dim = pd.get(4, 2560);
        c.heads = pd.get(5, 20);
        c.head_dim = pd.get(6, 128);
        c.mlp_hidden = pd.get(7, 6912);
        c.norm_eps = pd.get(8, 1e-5f);
        c.window_t = pd.get(9, 0);
        c.window_h = pd.get(10, 0);
        c.window_w = pd.get(11, 0);
        c.rope_mode = pd.get(12, static_cast<int>(SV2_ROPE_REFERENCE));
        c.qk_norm = pd.get(13, 1) != 0;
        c.fused_gemm = pd.get(14, 0) != 0;
        return c.dim == c.heads * c.head_dim ? 0 : -1;
    }

    int load_model(const ModelBin& mb) override
    {
        const int D = config_.dim, F = config_.mlp_hidden, hd = config_.head_dim;
        const int nbranch = config_.shared_weights ? 1 : 2;
        for (int b = 0; b < nbranch; b++)
        {
            Branch& br = branch_[b];
            for (int i = 0; i < 6; i++)
                if (!load(mb, D, 1, &br.ada[i]))
                    return -100;
            // InnerProduct::load_model: weights type 0, then the bias type 1
            if (!load(mb, 3 * D * D, 0, &br.w_qkv) || !load(mb, D * D, 0, &br.w_proj) || !load(mb, D, 1, &br.b_proj) ||
                !load(mb, hd, 1, &br.norm_q) || !load(mb, hd, 1, &br.norm_k) || !load(mb, F * D, 0, &br.w_gate) ||
                !load(mb, F * D, 0, &br.w_in) || !load(mb, D * F, 0, &br.w_out))
                return -100;
        }
        return load(mb, 21, 1, &freqs_) ? 0 : -100;
    }

    int create_pipeline(const Option& opt) override
    {
        sv2_block_destroy(block_);
        block_ = nullptr;
        const sv2_block_branch vid = view(branch_[0]);
        const sv2_block_branch txt = view(branch_[config_.shared_weights ? 0 : 1]);
        const int dtype = opt.use_fp16_arithmetic ? SV2_F16 : SV2_F32;
        compute_dtype_ = dtype;
        const int rc = sv2_block_create(&config_, &vid, &txt, static_cast<const float*>(freqs_.data), 0, dtype, &block_);
        if (rc != SV2_OK)
        {
            std::fprintf(stderr, "SeedVR2DiTBlock[%d]: %s\n", config_.block_index, sv2_last_error());
            block_ = nullptr;
            return -100;
        }
        if (shape_valid_)
            sv2_block_set_runtime_shape(block_, frames_, height_, width_);
        branch_[0] = Branch();
        branch_[1] = Branch();
        return 0;
    }

    int destroy_pipeline(const Option&) override
    {
        sv2_block_destroy(block_);
        block_ = nullptr;
        return 0;
    }

    int forward(const std::vector<Mat>& bottom_blobs, std::vector<Mat>& top_blobs, const Option& opt) const override
    {
        if (bottom_blobs.size() != 4 || top_blobs.size() != 2)
        {
            std::fprintf(stderr, "SeedVR2DiTBlock[%d]: blob count mismatch (bottom=%zu top=%zu)\n",
                         config_.block_index, bottom_blobs.size(), top_blobs.size());
            return -1;
        }
        const Mat& vid = bottom_blobs[0];
        const Mat& txt = bottom_blobs[1];
        const Mat& emb = bottom_blobs[2];
        const Mat& shape = bottom_blobs[3];
        const int D = config_.dim;
        if (vid.dims != 2 || txt.dims != 2 || vid.w != D || txt.w != D || emb.w != 6 * D || shape.dims != 1 ||
            shape.w != 3)
        {
            std::fprintf(stderr, "SeedVR2DiTBlock[%d]: invalid input vid=(dims=%d w=%d h=%d) txt=(dims=%d w=%d h=%d) "
                                 "emb=%d shape=%d expected_dim=%d\n",
                         config_.block_index, vid.dims, vid.w, vid.h, txt.dims, txt.w, txt.h, emb.w, shape.w, D);
            return -1;
        }
        if (!block_)
            return -100;
        const int* thw = static_cast<const int*>(shape.data);
        if (int64_t(thw[0]) * thw[1] * thw[2] != vid.h ||
            sv2_block_set_runtime_shape(block_, thw[0], thw[1], thw[2]) != SV2_OK)
        {
            std::fprintf(stderr, "SeedVR2DiTBlock[%d]: vid_shape (%d, %d, %d) does not match %d video rows\n",
                         config_.block_index, thw[0], thw[1], thw[2], vid.h);
            return -1;
        }
        const int Lv = vid.h, Lt = txt.h;
        Mat& vid_out = top_blobs[0];
        Mat& txt_out = top_blobs[1];
        vid_out.create(D, Lv, size_t(4u), opt.blob_allocator);
        txt_out.create(D, Lt, size_t(4u), opt.blob_allocator);
        if (vid_out.empty() || (Lt > 0 && txt_out.empty()))
            return -100;
        sv2_block_debug host{};
        if (debug_ && !size_debug(Lv, Lt, &host))
            return -100;
        const int rc = sv2_block_forward_host(block_, static_cast<const float*>(vid.data),
                                              Lt > 0 ? static_cast<const float*>(txt.data) : nullptr, Lt,
                                              static_cast<const float*>(emb.data), static_cast<float*>(vid_out.data),
                                              Lt > 0 ? static_cast<float*>(txt_out.data) : nullptr,
                                              debug_ ? &host : nullptr);
        if (rc != SV2_OK)
        {
            std::fprintf(stderr, "SeedVR2DiTBlock[%d]: %s\n", config_.block_index, sv2_last_error());
            return -100;
        }
        return 0;
    }

    /* The device block from the loaded weights, when create_pipeline has not
     * made it (SeedVR2DiTBlock::upload_model, seedvr2_dit_block.cpp:1271). */
    int upload_model(DeviceCompute&, const Option& opt)
    {
        return block_ ? 0 : create_pipeline(opt);
    }

    /* The block forward over device blobs: enqueued on cmd.stream only
     * (SeedVR2DiTBlock::forward over VkMat, seedvr2_dit_block.cpp:1302-1324
     * for the checks). */
    int forward(const std::vector<DeviceMat>& bottom_blobs, std::vector<DeviceMat>& top_blobs, DeviceCompute& cmd,
                const Option&) const
    {
        if (bottom_blobs.size() != 4 || top_blobs.size() != 2)
            return -1;
        const DeviceMat& vid = bottom_blobs[0];
        const DeviceMat& txt = bottom_blobs[1];
        const DeviceMat& emb = bottom_blobs[2];
        const DeviceMat& shape = bottom_blobs[3];
        const int D = config_.dim;
        if (vid.dims != 2 || vid.w != D || txt.dims != 2 || txt.w != D || emb.w != 6 * D || shape.w != 3)
            return -1;
        if (!block_ || !shape_valid_ || int64_t(frames_) * height_ * width_ != vid.h)
            return -1;
        const size_t es = dtype_bytes();
        if (vid.elemsize != es || (txt.h > 0 && txt.elemsize != es) || emb.elemsize != 4 || vid.empty() ||
            emb.empty() || (txt.h > 0 && txt.empty()))
            return -1;
        const int Lv = vid.h, Lt = txt.h;
        DeviceMat& vid_out = top_blobs[0];
        DeviceMat& txt_out = top_blobs[1];
        vid_out.create(D, Lv, es, cmd.blob_allocator);
        txt_out.create(D, Lt, es, cmd.blob_allocator);
        if (vid_out.empty() || (Lt > 0 && txt_out.empty()))
            return -100;
        const int64_t need = sv2_block_workspace_size(block_, Lt);
        if (need < 0)
            return -100;
        // rows of 1 MiB: a workspace past 2 GiB (large grids) keeps its byte
        // count out of the blob's int extents
        const int64_t row = int64_t(1) << 20;
        const int64_t rows = need > 0 ? (need + row - 1) / row : 1;
        if (rows > int64_t(0x7fffffff))
            return -100;
        DeviceMat ws;
        ws.create(static_cast<int>(row), static_cast<int>(rows), size_t(1u), cmd.workspace_allocator);
        if (ws.empty())
            return -100;
        const int rc = sv2_block_forward(block_, vid.data, Lt > 0 ? txt.data : nullptr, Lt,
                                         static_cast<const float*>(emb.data), vid_out.data,
                                         Lt > 0 ? txt_out.data : nullptr, ws.data, size_t(need),
                                         static_cast<void*>(cmd.stream));
        if (rc != SV2_OK)
        {
            std::fprintf(stderr, "SeedVR2DiTBlock[%d]: %s\n", config_.block_index, sv2_last_error());
            return -100;
        }
        return 0;
    }

    /* Bytes per element of the device blobs: 2 in the fp16 compute mode, 4
     * in fp32 (0 before create_pipeline). */
    size_t dtype_bytes() const
    {
        return block_ ? (compute_dtype_ == SV2_F16 ? 2u : 4u) : 0u;
    }

    /* The patched grid of the next device forward (the ncnn CPU forward reads
     * it from the vid_shape blob instead). */
    void set_runtime_shape(int frames, int height, int width)
    {
        frames_ = frames;
        height_ = height;
        width_ = width;
        shape_valid_ = frames > 0 && height > 0 && width > 0;
        if (block_ && shape_valid_)
            sv2_block_set_runtime_shape(block_, frames, height, width);
    }

    /* Captures of the following forwards; the caller keeps `tensors` alive. */
    void set_debug_tensors(DebugTensors* tensors)
    {
        debug_ = tensors;
    }

    /* The device block, for callers that run sv2_block_forward on device
     * buffers themselves (NULL before create_pipeline). */
    sv2_block* block() const
    {
        return block_;
    }
    const sv2_block_config& config() const
    {
        return config_;
    }

  private:
    struct Branch
    {
        Mat ada[6], w_qkv, w_proj, b_proj, norm_q, norm_k, w_gate, w_in, w_out;
    };

    static bool load(const ModelBin& mb, int count, int type, Mat* out)
    {
        *out = mb.load(count, type);
        return !out->empty() && out->w == count;
    }

    static sv2_block_branch view(const Branch& b)
    {
        sv2_block_branch v;
        for (int i = 0; i < 6; i++)
            v.ada[i] = b.ada[i].data;
        v.w_qkv = b.w_qkv.data;
        v.w_proj = b.w_proj.data;
        v.b_proj = b.b_proj.data;
        v.norm_q = b.norm_q.data;
        v.norm_k = b.norm_k.data;
        v.w_gate = b.w_gate.data;
        v.w_in = b.w_in.data;
        v.w_out = b.w_out.data;
        return v;
    }

    // Sizes the caller's capture Mats ([rows, cols] fp32) and points `host` at them.
    bool size_debug(int Lv, int Lt, sv2_block_debug* host) const
    {
        const int D = config_.dim;
        const int64_t S = sv2_block_window_rows(block_, Lt);
        if (S < 0)
            return false;
        DebugTensors& t = *debug_;
        bool ok = true;
        auto make = [&ok](Mat& m, int cols, int64_t rows, float** dst) {
            m.create(cols, static_cast<int>(rows), size_t(4u), nullptr);
            ok = ok && (rows == 0 || !m.empty());
            *dst = rows > 0 ? static_cast<float*>(m.data) : nullptr;
        };
        make(t.qkv_vid, 3 * D, Lv, &host->qkv_vid);
        make(t.qkv_txt, 3 * D, Lt, &host->qkv_txt);
        make(t.norm_q_vid, D, Lv, &host->norm_q_vid);
        make(t.norm_q_txt, D, Lt, &host->norm_q_txt);
        make(t.norm_k_vid, D, Lv, &host->norm_k_vid);
        make(t.norm_k_txt, D, Lt, &host->norm_k_txt);
        make(t.attention_q, D, S, &host->attention_q);
        make(t.attention_k, D, S, &host->attention_k);
        make(t.attention_v, D, S, &host->attention_v);
        make(t.attention_output, D, S, &host->attention_output);
        make(t.projected_vid, D, Lv, &host->projected_vid);
        make(t.projected_txt, D, Lt, &host->projected_txt);
        make(t.output_vid, D, Lv, &host->output_vid);
        make(t.output_txt, D, Lt, &host->output_txt);
        return ok;
    }

    sv2_block_config config_{};
    Branch branch_[2];
    Mat freqs_;
    sv2_block* block_ = nullptr;
    int compute_dtype_ = SV2_F32;
    int frames_ = 0, height_ = 0, width_ = 0;
    bool shape_valid_ = false;
    DebugTensors* debug_ = nullptr;
};

} // namespace sv2
