// A C++ consumer of the library's layer boundary: the command line of the
// reference's block runner (tests/dit_block_runner.cpp), with the block
// registered as the custom layer "SeedVR2DiTBlock" through
// SeedVR2DiTBlock_layer_creator and driven through the ncnn layer interface
// (load_param, load_model, create_pipeline, forward) of sv2::DiTBlockLayer.
//
//   block_runner model.param model.bin vid.f32 vid_rows txt.f32 txt_rows
//                emb.f32 T H W vid_out.f32 txt_out.f32 [debug_prefix]
//       inputs raw fp32 ([rows, dim], emb [6*dim]); outputs and captures fp32
//       with an int32 [rows, cols] header.  SEEDVR2_FP16=1 selects fp16
//       arithmetic (Option::use_fp16_arithmetic), else fp32.
//   block_runner --load-only model.param model.bin
//       parses and loads the block without a device and prints its
//       parameters and the bytes of the .bin left unread.
//   block_runner --device-chain N b0.param b0.bin ... vid.f32 vid_rows
//                txt.f32 txt_rows emb.f32 T H W vid_out.f32 txt_out.f32
//       N blocks chained on device blobs (sv2::DeviceMat) through the
//       adapter's upload_model and device forward, as the reference DiT
//       drives its blocks on VkMat (src/model/dit.cpp:545-581): the inputs
//       are uploaded once, each block's tops are the next block's bottoms,
//       every forward enqueues on one HIP stream, and the host waits and
//       downloads once, after the last block.  Blobs come from a caching
//       device pool (freed buffers reused by later allocations on the same
//       stream).
//
// Exit codes as the reference runner: 2 usage, 3 inputs, 4 model load,
// 6 inference, 7 outputs, 8 captures.
#include <hip/hip_runtime_api.h>

#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <map>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "host_half.h"
#include "layer_types.h"
#include "seedvr2_dit_block_layer.h"

class SeedVR2DiTBlock : public sv2::DiTBlockLayer<host::Api>
{
};
typedef sv2::BlockDebugTensors<host::Mat> SeedVR2DiTBlockDebugTensors;

host::Layer* SeedVR2DiTBlock_layer_creator(void*)
{
    return new SeedVR2DiTBlock;
}

namespace
{
bool read_matrix(const std::string& path, int rows, int cols, host::Mat& out)
{
    out.create(cols, rows, size_t(4u));
    if (rows > 0 && out.empty())
        return false;
    std::ifstream in(path, std::ios::binary);
    if (!in)
        return false;
    const std::streamsize bytes = std::streamsize(rows) * cols * 4;
    in.read(static_cast<char*>(out.data), bytes);
    return in.gcount() == bytes;
}

bool write_matrix(const std::string& path, const host::Mat& m)
{
    if (m.dims != 2 || m.elemsize != 4u)
        return false;
    std::ofstream out(path, std::ios::binary);
    if (!out)
        return false;
    const int32_t shape[2] = {m.h, m.w};
    out.write(reinterpret_cast<const char*>(shape), sizeof(shape));
    if (m.data)
        out.write(static_cast<const char*>(m.data), std::streamsize(m.h) * m.w * 4);
    return bool(out);
}

// A caching pool of device buffers (a blob allocator in ncnn's sense): a
// freed buffer goes back to the pool and serves a later request of at most
// its size.  With one stream, stream order makes the reuse safe: work that
// reads a freed buffer was enqueued before the work that writes its reuse.
class DevicePool : public sv2::DeviceAllocator
{
  public:
    ~DevicePool() override
    {
        for (auto& kv : size_)
            (void)hipFree(kv.first);
    }
    void* fastMalloc(size_t bytes) override
    {
        auto it = free_.lower_bound(bytes);
        if (it != free_.end() && it->first <= 2 * bytes + 4096)
        {
            void* p = it->second;
            free_.erase(it);
            return p;
        }
        void* p = nullptr;
        if (hipMalloc(&p, bytes) != hipSuccess)
            return nullptr;
        size_[p] = bytes;
        return p;
    }
    void fastFree(void* ptr) override
    {
        if (ptr)
            free_.emplace(size_[ptr], ptr);
    }

  private:
    std::map<void*, size_t> size_;
    std::multimap<size_t, void*> free_;
};

SeedVR2DiTBlock* find_block(host::Net& net);

// Host fp32 values -> a device blob in the compute dtype (elements of es = 2
// or 4 bytes), [h][w] (dims 2) or [w] (dims 1).
bool upload(const host::Mat& m, size_t es, DevicePool& pool, sv2::DeviceMat* out)
{
    if (m.dims == 1)
        out->create(m.w, es, &pool);
    else
        out->create(m.w, m.h, es, &pool);
    const size_t n = size_t(m.w) * size_t(m.h);
    if (n == 0)
        return true;
    if (out->empty())
        return false;
    const float* src = static_cast<const float*>(m.data);
    if (es == 4)
        return hipMemcpy(out->data, src, n * 4, hipMemcpyHostToDevice) == hipSuccess;
    std::vector<uint16_t> half(n);
    for (size_t i = 0; i < n; i++)
        half[i] = host_half::from_float(src[i]);
    return hipMemcpy(out->data, half.data(), n * 2, hipMemcpyHostToDevice) == hipSuccess;
}

// A device blob in the compute dtype -> host fp32 rows.
bool download(const sv2::DeviceMat& d, host::Mat* out)
{
    out->create(d.w, d.h, size_t(4u));
    const size_t n = size_t(d.w) * size_t(d.h);
    if (n == 0)
        return true;
    if (out->empty() || d.empty())
        return false;
    float* dst = static_cast<float*>(out->data);
    if (d.elemsize == 4)
        return hipMemcpy(dst, d.data, n * 4, hipMemcpyDeviceToHost) == hipSuccess;
    std::vector<uint16_t> half(n);
    if (hipMemcpy(half.data(), d.data, n * 2, hipMemcpyDeviceToHost) != hipSuccess)
        return false;
    for (size_t i = 0; i < n; i++)
        dst[i] = host::half_to_float(half[i]);
    return true;
}

// --device-chain: argv[2] = N, then N (param, bin) pairs, then the inputs and
// outputs of the single-block form.
int device_chain(int argc, char** argv)
{
    const int n = argc > 2 ? std::atoi(argv[2]) : 0;
    if (n < 1 || argc != 3 + 2 * n + 10)
    {
        std::fprintf(stderr, "usage: %s --device-chain N b0.param b0.bin ... vid.f32 vid_rows txt.f32 txt_rows "
                             "emb.f32 T H W vid_out.f32 txt_out.f32\n", argv[0]);
        return 2;
    }
    char** a = argv + 3 + 2 * n;
    const int vid_rows = std::atoi(a[1]);
    const int txt_rows = std::atoi(a[3]);
    const int frames = std::atoi(a[5]), height = std::atoi(a[6]), width = std::atoi(a[7]);
    const char* fp16 = std::getenv("SEEDVR2_FP16");
    std::vector<std::unique_ptr<host::Net>> nets;
    std::vector<SeedVR2DiTBlock*> layers;
    DevicePool pool;
    hipStream_t stream = nullptr;
    if (hipStreamCreate(&stream) != hipSuccess)
        return 6;
    sv2::DeviceCompute cmd;
    cmd.stream = stream;
    cmd.blob_allocator = &pool;
    cmd.workspace_allocator = &pool;
    for (int i = 0; i < n; i++)
    {
        auto net = std::make_unique<host::Net>();
        net->opt.use_fp16_arithmetic = fp16 && std::string(fp16) == "1";
        net->register_custom_layer("SeedVR2DiTBlock", SeedVR2DiTBlock_layer_creator);
        if (net->load_param(argv[3 + 2 * i]) != 0 || net->load_model(argv[4 + 2 * i]) != 0)
        {
            std::fprintf(stderr, "failed to load block %d\n", i);
            return 4;
        }
        SeedVR2DiTBlock* layer = find_block(*net);
        if (!layer || layer->upload_model(cmd, net->opt) != 0)
            return 4;
        layers.push_back(layer);
        nets.push_back(std::move(net));
    }
    const int dim = layers[0]->config().dim;
    const size_t es = layers[0]->dtype_bytes();
    host::Mat vid, txt, emb;
    if (!read_matrix(a[0], vid_rows, dim, vid) || !read_matrix(a[2], txt_rows, dim, txt) ||
        !read_matrix(a[4], 1, 6 * dim, emb))
    {
        std::fprintf(stderr, "failed to read input matrices\n");
        return 3;
    }
    emb.dims = 1; // a [6*dim] vector, as the emb blob
    host::Mat shape(3, size_t(4u));
    static_cast<int*>(shape.data)[0] = frames;
    static_cast<int*>(shape.data)[1] = height;
    static_cast<int*>(shape.data)[2] = width;
    std::vector<sv2::DeviceMat> bottoms(4);
    if (!upload(vid, es, pool, &bottoms[0]) || !upload(txt, es, pool, &bottoms[1]) ||
        !upload(emb, 4, pool, &bottoms[2]) || !upload(shape, 4, pool, &bottoms[3]))
    {
        std::fprintf(stderr, "failed to upload the inputs\n");
        return 3;
    }
    const auto start = std::chrono::steady_clock::now();
    for (int i = 0; i < n; i++)
    {
        layers[i]->set_runtime_shape(frames, height, width);
        std::vector<sv2::DeviceMat> tops(2);
        const int rc = layers[i]->forward(bottoms, tops, cmd, nets[i]->opt);
        if (rc != 0)
        {
            std::fprintf(stderr, "block %d inference failed (%d)\n", i, rc);
            return 6;
        }
        // the next block reads these tops; the previous bottoms go back to the pool
        bottoms[0] = tops[0];
        bottoms[1] = tops[1];
    }
    const double enqueue_ms =
        std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - start).count();
    if (hipStreamSynchronize(stream) != hipSuccess)
    {
        std::fprintf(stderr, "device chain failed on the stream\n");
        return 6;
    }
    const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - start).count();
    std::printf("device_chain blocks=%d enqueue_ms=%.3f total_ms=%.3f\n", n, enqueue_ms, ms);
    host::Mat vo, to;
    if (!download(bottoms[0], &vo) || !download(bottoms[1], &to) || !write_matrix(a[8], vo) ||
        !write_matrix(a[9], to))
    {
        std::fprintf(stderr, "failed to write block outputs\n");
        return 7;
    }
    bottoms.clear();
    (void)hipStreamDestroy(stream);
    return 0;
}

SeedVR2DiTBlock* find_block(host::Net& net)
{
    for (host::Layer* l : net.mutable_layers())
        if (auto* b = dynamic_cast<SeedVR2DiTBlock*>(l))
            return b;
    return nullptr;
}
} // namespace

int main(int argc, char** argv)
{
    if (argc > 1 && std::string(argv[1]) == "--device-chain")
        return device_chain(argc, argv);
    if (argc == 4 && std::string(argv[1]) == "--load-only")
    {
        host::Net net;
        net.create_pipelines = false;
        net.register_custom_layer("SeedVR2DiTBlock", SeedVR2DiTBlock_layer_creator);
        if (net.load_param(argv[2]) != 0)
        {
            std::fprintf(stderr, "failed to load block param\n");
            return 4;
        }
        if (net.load_model(argv[3]) != 0)
        {
            std::fprintf(stderr, "failed to load block model\n");
            return 4;
        }
        SeedVR2DiTBlock* b = find_block(net);
        if (!b)
            return 4;
        const sv2_block_config& c = b->config();
        std::printf("params 0=%d 1=%d 2=%d 3=%d 4=%d 5=%d 6=%d 7=%d 8=%.9g 9=%d 10=%d 11=%d 12=%d 13=%d 14=%d\n",
                    c.block_index, c.shared_weights, c.last_layer, c.shifted_window, c.dim, c.heads, c.head_dim,
                    c.mlp_hidden, double(c.norm_eps), c.window_t, c.window_h, c.window_w, c.rope_mode, c.qk_norm,
                    c.fused_gemm);
        std::printf("trailing_bytes=%lld\n", static_cast<long long>(net.trailing_bytes));
        return 0;
    }
    if (argc != 13 && argc != 14)
    {
        std::fprintf(stderr,
                     "usage: %s model.param model.bin vid.f32 vid_rows txt.f32 txt_rows emb.f32 T H W "
                     "vid_out.f32 txt_out.f32 [debug_prefix]\n       %s --load-only model.param model.bin\n",
                     argv[0], argv[0]);
        return 2;
    }
    const int vid_rows = std::atoi(argv[4]);
    const int txt_rows = std::atoi(argv[6]);
    const int frames = std::atoi(argv[8]);
    const int height = std::atoi(argv[9]);
    const int width = std::atoi(argv[10]);
    const char* fp16 = std::getenv("SEEDVR2_FP16");

    host::Net net;
    net.opt.use_fp16_arithmetic = fp16 && std::string(fp16) == "1";
    net.register_custom_layer("SeedVR2DiTBlock", SeedVR2DiTBlock_layer_creator);
    if (net.load_param(argv[1]) != 0 || net.load_model(argv[2]) != 0)
    {
        std::fprintf(stderr, "failed to load block model\n");
        return 4;
    }
    SeedVR2DiTBlock* layer = find_block(net);
    if (!layer)
        return 4;
    const int dim = layer->config().dim;
    host::Mat vid, txt, emb;
    if (!read_matrix(argv[3], vid_rows, dim, vid) || !read_matrix(argv[5], txt_rows, dim, txt) ||
        !read_matrix(argv[7], 1, 6 * dim, emb))
    {
        std::fprintf(stderr, "failed to read input matrices\n");
        return 3;
    }
    host::Mat shape(3, size_t(4u));
    static_cast<int*>(shape.data)[0] = frames;
    static_cast<int*>(shape.data)[1] = height;
    static_cast<int*>(shape.data)[2] = width;

    SeedVR2DiTBlockDebugTensors debug;
    if (argc == 14)
        layer->set_debug_tensors(&debug);
    std::vector<host::Mat> bottoms = {vid, txt, emb, shape};
    std::vector<host::Mat> tops(2);
    const auto start = std::chrono::steady_clock::now();
    const int rc = layer->forward(bottoms, tops, net.opt);
    const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - start).count();
    if (rc != 0)
    {
        std::fprintf(stderr, "block inference failed (%d)\n", rc);
        return 6;
    }
    std::printf("block_forward_ms=%.3f\n", ms);
    if (!write_matrix(argv[11], tops[0]) || !write_matrix(argv[12], tops[1]))
    {
        std::fprintf(stderr, "failed to write block outputs\n");
        return 7;
    }
    if (argc == 14)
    {
        const std::string prefix = argv[13];
        const std::pair<const char*, const host::Mat*> captures[] = {
            {"qkv_vid", &debug.qkv_vid},
            {"qkv_txt", &debug.qkv_txt},
            {"norm_q_vid", &debug.norm_q_vid},
            {"norm_q_txt", &debug.norm_q_txt},
            {"norm_k_vid", &debug.norm_k_vid},
            {"norm_k_txt", &debug.norm_k_txt},
            {"attention_q", &debug.attention_q},
            {"attention_k", &debug.attention_k},
            {"attention_v", &debug.attention_v},
            {"attention_output", &debug.attention_output},
            {"projected_vid", &debug.projected_vid},
            {"projected_txt", &debug.projected_txt},
            {"output_vid", &debug.output_vid},
            {"output_txt", &debug.output_txt},
        };
        for (const auto& c : captures)
            if (!write_matrix(prefix + "_" + c.first + ".f32", *c.second))
            {
                std::fprintf(stderr, "failed to write debug capture %s\n", c.first);
                return 8;
            }
    }
    std::printf("vid=%dx%d txt=%dx%d\n", tops[0].h, tops[0].w, tops[1].h, tops[1].w);
    return 0;
}
