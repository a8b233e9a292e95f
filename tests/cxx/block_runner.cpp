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
//
// Exit codes as the reference runner: 2 usage, 3 inputs, 4 model load,
// 6 inference, 7 outputs, 8 captures.
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <string>
#include <utility>

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
