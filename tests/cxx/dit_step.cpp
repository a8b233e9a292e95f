// The SeedVR2-3B DiT forward of one Euler step, driven from C++ through the C
// ABI alone: no torch and no Python in the process, so the GEMM library it
// maps is the one a C++ ncnn integration loads (the library's own link to
// ROCm's libhipblaslt), not a copy bundled with a Python framework.
//
// The DiT is assembled as SeedVR2DiT::load holds it resident (src/model/
// dit.cpp:120-174): the input head, 32 blocks and the output head, created
// from device weights (sv2_dit_input_create, sv2_block_create,
// sv2_dit_output_create with weights_on_device = 1) and joined with
// sv2_dit_create; the blocks carry the exporter's flags (shared weights from
// block 10, the last block's text rule, odd blocks shifted;
// tools/export_seedvr2_dit_ncnn.py:204-206) and 2x9x16 windows.  Weights are
// N(0, 0.02^2) (q/k norm and output norm weights U(0.5, 1.5)), fp16 matrices
// and fp32 vectors; the latent N(0, 1) with its last channel all ones, the
// text N(0, 1).
//
//   dit_step [--frames T] [--height H] [--width W] [--text L] [--steps K]
//            [--warmup W] [--fused 0|1]
//       defaults: the 1280x720x21 latent grid 6 x 90 x 160, 58 text tokens,
//       3 timed forwards after 1 warm-up, library InnerProducts.
//
// Prints one JSON line: the mean forward time over the timed forwards (HIP
// events on the forward's stream), whether the output is finite, and the
// path of the libhipblaslt the process mapped.  Exit codes: 2 usage,
// 4 creation, 6 forward, 7 output.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <string>
#include <vector>

#include "host_half.h"
#include "seedvr2_hip.h"

namespace
{
constexpr int kDim = 2560;
constexpr int kHeads = 20;
constexpr int kMlp = 6912;
constexpr int kBlocks = 32;
constexpr int kLatentC = 33;
constexpr int kTextC = 5120;
constexpr int kOutC = 16;
constexpr size_t kPool = size_t(1) << 24; // random values reused, from a rotating start, by every array

struct Rng
{
    uint64_t s;
    uint64_t next()
    {
        uint64_t z = (s += 0x9e3779b97f4a7c15ull);
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        return z ^ (z >> 31);
    }
    double uniform() { return (double(next() >> 11) + 0.5) * (1.0 / 9007199254740992.0); }
    double normal()
    {
        const double u = uniform(), v = uniform();
        return std::sqrt(-2.0 * std::log(u)) * std::cos(6.283185307179586 * v);
    }
};

[[noreturn]] void fail(int code, const char* what)
{
    std::fprintf(stderr, "dit_step: %s: %s\n", what, sv2_last_error());
    std::exit(code);
}

void check_hip(hipError_t e, const char* what)
{
    if (e != hipSuccess)
    {
        std::fprintf(stderr, "dit_step: %s: %s\n", what, hipGetErrorString(e));
        std::exit(4);
    }
}

// Device arrays filled from pinned pools of random values: N(0, 1) fp32,
// N(0, 0.02^2) as fp16, U(0.5, 1.5) fp32.  Each array starts at its own
// offset into the pool.
class Weights
{
  public:
    explicit Weights(hipStream_t stream) : stream_(stream)
    {
        Rng rng{1234};
        check_hip(hipHostMalloc(reinterpret_cast<void**>(&normal_), kPool * 4, hipHostMallocDefault), "host pool");
        check_hip(hipHostMalloc(reinterpret_cast<void**>(&small_), kPool * 2, hipHostMallocDefault), "host pool");
        check_hip(hipHostMalloc(reinterpret_cast<void**>(&unit_), kPool * 4, hipHostMallocDefault), "host pool");
        for (size_t i = 0; i < kPool; i++)
        {
            const double n = rng.normal();
            normal_[i] = float(n);
            small_[i] = host_half::from_float(float(0.02 * n));
            unit_[i] = float(0.5 + rng.uniform());
        }
    }
    ~Weights()
    {
        for (void* p : owned_)
            (void)hipFree(p);
        (void)hipHostFree(normal_);
        (void)hipHostFree(small_);
        (void)hipHostFree(unit_);
    }
    enum Kind
    {
        kMatrix,   // fp16 N(0, 0.02^2)
        kVector,   // fp32 N(0, 0.02^2)
        kUnit,     // fp32 U(0.5, 1.5)
        kNormal,   // fp32 N(0, 1)
        kMatrix32, // fp32 N(0, 0.02^2) (the time MLP of the input head)
    };
    void* make(size_t count, Kind kind)
    {
        const size_t es = kind == kMatrix ? 2 : 4;
        void* dev = nullptr;
        check_hip(hipMalloc(&dev, count * es), "weights");
        owned_.push_back(dev);
        if (kind == kMatrix32 || kind == kVector)
            scaled(count);
        const char* pool = kind == kMatrix ? reinterpret_cast<const char*>(small_)
                           : kind == kUnit ? reinterpret_cast<const char*>(unit_)
                           : kind == kNormal ? reinterpret_cast<const char*>(normal_)
                                             : reinterpret_cast<const char*>(scaled_.data());
        size_t start = (next_start_ += 7919) % kPool;
        size_t done = 0;
        while (done < count)
        {
            const size_t n = std::min(count - done, kPool - start);
            check_hip(hipMemcpyAsync(static_cast<char*>(dev) + done * es, pool + start * es, n * es,
                                     hipMemcpyHostToDevice, stream_),
                      "weight upload");
            done += n;
            start = 0;
        }
        // the scaled copy is pageable and rewritten by the next array
        if (kind == kMatrix32 || kind == kVector)
            check_hip(hipStreamSynchronize(stream_), "weight upload");
        return dev;
    }
  private:
    void scaled(size_t count)
    {
        if (scaled_.size() < std::min(count, kPool))
        {
            scaled_.resize(kPool);
            for (size_t i = 0; i < kPool; i++)
                scaled_[i] = 0.02f * normal_[i];
        }
    }
    hipStream_t stream_;
    float* normal_ = nullptr;
    uint16_t* small_ = nullptr;
    float* unit_ = nullptr;
    std::vector<float> scaled_;
    std::vector<void*> owned_;
    size_t next_start_ = 0;
};

sv2_block_branch make_branch(Weights& w)
{
    sv2_block_branch b;
    for (auto& a : b.ada)
        a = w.make(kDim, Weights::kVector);
    b.w_qkv = w.make(size_t(3) * kDim * kDim, Weights::kMatrix);
    b.w_proj = w.make(size_t(kDim) * kDim, Weights::kMatrix);
    b.b_proj = w.make(kDim, Weights::kVector);
    b.norm_q = w.make(128, Weights::kUnit);
    b.norm_k = w.make(128, Weights::kUnit);
    b.w_gate = w.make(size_t(kMlp) * kDim, Weights::kMatrix);
    b.w_in = w.make(size_t(kMlp) * kDim, Weights::kMatrix);
    b.w_out = w.make(size_t(kDim) * kMlp, Weights::kMatrix);
    return b;
}

std::string mapped(const char* fragment)
{
    std::ifstream maps("/proc/self/maps");
    std::string line;
    while (std::getline(maps, line))
    {
        const size_t slash = line.find('/');
        if (slash != std::string::npos && line.find(fragment, slash) != std::string::npos)
            return line.substr(slash);
    }
    return "";
}

int arg_int(int argc, char** argv, const char* name, int def)
{
    for (int i = 1; i + 1 < argc; i++)
        if (std::strcmp(argv[i], name) == 0)
            return std::atoi(argv[i + 1]);
    return def;
}
} // namespace

int main(int argc, char** argv)
{
    for (int i = 1; i < argc; i += 2)
    {
        static const char* known[] = {"--frames", "--height", "--width", "--text", "--steps", "--warmup", "--fused"};
        bool ok = i + 1 < argc;
        bool found = false;
        for (const char* k : known)
            found = found || std::strcmp(argv[i], k) == 0;
        if (!ok || !found)
        {
            std::fprintf(stderr, "usage: dit_step [--frames T] [--height H] [--width W] [--text L] [--steps K] "
                                 "[--warmup W] [--fused 0|1]\n");
            return 2;
        }
    }
    const int T = arg_int(argc, argv, "--frames", 6);
    const int H = arg_int(argc, argv, "--height", 90);
    const int W = arg_int(argc, argv, "--width", 160);
    const int L = arg_int(argc, argv, "--text", 58);
    const int steps = arg_int(argc, argv, "--steps", 3);
    const int warmup = arg_int(argc, argv, "--warmup", 1);
    const int fused = arg_int(argc, argv, "--fused", 0);
    if (T < 1 || H < 2 || W < 2 || H % 2 || W % 2 || L < 1 || steps < 1 || warmup < 0)
    {
        std::fprintf(stderr, "dit_step: invalid shape or counts\n");
        return 2;
    }

    hipStream_t stream = nullptr;
    check_hip(hipStreamCreate(&stream), "stream");
    Weights w(stream);

    float freqs[21];
    for (int i = 0; i < 21; i++)
        freqs[i] = float(1.0 / std::pow(10000.0, (2.0 * i) / 42.0));

    std::vector<sv2_block*> blocks(kBlocks, nullptr);
    for (int i = 0; i < kBlocks; i++)
    {
        sv2_block_config c;
        sv2_block_config_default(&c);
        c.block_index = i;
        c.shared_weights = i >= 10;
        c.last_layer = i == kBlocks - 1;
        c.shifted_window = i % 2;
        c.dim = kDim;
        c.heads = kHeads;
        c.head_dim = 128;
        c.mlp_hidden = kMlp;
        c.window_t = 2;
        c.window_h = 9;
        c.window_w = 16;
        c.fused_gemm = fused;
        const sv2_block_branch vid = make_branch(w);
        sv2_block_branch txt = vid;
        if (!c.shared_weights)
            txt = make_branch(w);
        if (sv2_block_create(&c, &vid, &txt, freqs, 1, SV2_F16, &blocks[i]) != SV2_OK)
            fail(4, "sv2_block_create");
    }

    sv2_dit_input_config ic{kDim, kLatentC, kTextC, 256, 6 * kDim};
    sv2_dit_input_weights iw;
    iw.w_vid = w.make(size_t(kDim) * 4 * kLatentC, Weights::kMatrix);
    iw.b_vid = w.make(kDim, Weights::kVector);
    iw.w_txt = w.make(size_t(kDim) * kTextC, Weights::kMatrix);
    iw.b_txt = w.make(kDim, Weights::kVector);
    iw.w_time_in = w.make(size_t(kDim) * 256, Weights::kMatrix32);
    iw.b_time_in = w.make(kDim, Weights::kVector);
    iw.w_time_hid = w.make(size_t(kDim) * kDim, Weights::kMatrix32);
    iw.b_time_hid = w.make(kDim, Weights::kVector);
    iw.w_time_out = w.make(size_t(6) * kDim * kDim, Weights::kMatrix32);
    iw.b_time_out = w.make(size_t(6) * kDim, Weights::kVector);
    sv2_dit_input* input = nullptr;
    if (sv2_dit_input_create(&ic, &iw, 1, SV2_F16, &input) != SV2_OK)
        fail(4, "sv2_dit_input_create");

    sv2_dit_output_config oc{kDim, kOutC, 1e-5f};
    sv2_dit_output_weights ow;
    ow.norm_weight = w.make(kDim, Weights::kUnit);
    ow.shift = w.make(kDim, Weights::kVector);
    ow.scale = w.make(kDim, Weights::kVector);
    ow.w_proj = w.make(size_t(4) * kOutC * kDim, Weights::kMatrix);
    ow.b_proj = w.make(4 * kOutC, Weights::kVector);
    sv2_dit_output* output = nullptr;
    if (sv2_dit_output_create(&oc, &ow, 1, SV2_F16, &output) != SV2_OK)
        fail(4, "sv2_dit_output_create");

    sv2_dit* dit = nullptr;
    if (sv2_dit_create(input, blocks.data(), kBlocks, output, &dit) != SV2_OK)
        fail(4, "sv2_dit_create");

    // latent N(0, 1) with the last channel all ones (the condition mask), text N(0, 1)
    const size_t plane = size_t(T) * H * W;
    float* latent = static_cast<float*>(w.make(size_t(kLatentC) * plane, Weights::kNormal));
    std::vector<float> ones(plane, 1.f);
    check_hip(hipMemcpyAsync(latent + size_t(kLatentC - 1) * plane, ones.data(), plane * 4, hipMemcpyHostToDevice,
                             stream),
              "latent");
    float* text = static_cast<float*>(w.make(size_t(L) * kTextC, Weights::kNormal));
    float* out = nullptr;
    check_hip(hipMalloc(reinterpret_cast<void**>(&out), size_t(kOutC) * plane * 4), "output");
    const int64_t ws_bytes = sv2_dit_workspace_size(dit, T, H, W, L);
    if (ws_bytes < 0)
        fail(4, "sv2_dit_workspace_size");
    void* ws = nullptr;
    check_hip(hipMalloc(&ws, size_t(ws_bytes)), "workspace");
    check_hip(hipStreamSynchronize(stream), "setup");

    for (int i = 0; i < warmup; i++)
        if (sv2_dit_forward(dit, latent, text, L, 1000.f, T, H, W, out, ws, size_t(ws_bytes), stream) != SV2_OK)
            fail(6, "sv2_dit_forward");
    check_hip(hipStreamSynchronize(stream), "warm-up");
    std::vector<hipEvent_t> ev(2 * size_t(steps));
    for (auto& e : ev)
        check_hip(hipEventCreate(&e), "event");
    for (int i = 0; i < steps; i++)
    {
        check_hip(hipEventRecord(ev[2 * i], stream), "event");
        if (sv2_dit_forward(dit, latent, text, L, 1000.f, T, H, W, out, ws, size_t(ws_bytes), stream) != SV2_OK)
            fail(6, "sv2_dit_forward");
        check_hip(hipEventRecord(ev[2 * i + 1], stream), "event");
    }
    check_hip(hipStreamSynchronize(stream), "forward");
    double total = 0.0;
    for (int i = 0; i < steps; i++)
    {
        float ms = 0.f;
        check_hip(hipEventElapsedTime(&ms, ev[2 * i], ev[2 * i + 1]), "event time");
        total += ms;
    }
    std::vector<float> host(size_t(kOutC) * plane);
    if (hipMemcpy(host.data(), out, host.size() * 4, hipMemcpyDeviceToHost) != hipSuccess)
    {
        std::fprintf(stderr, "dit_step: output download failed\n");
        return 7;
    }
    bool finite = true;
    for (float v : host)
        finite = finite && std::isfinite(v);

    const std::string blaslt = mapped("libhipblaslt");
    std::printf("{\"ms\": %.3f, \"steps\": %d, \"warmup\": %d, \"finite\": %s, \"fused_gemm\": %d, "
                "\"grid\": [%d, %d, %d], \"text_len\": %d, \"hipblaslt\": \"%s\"}\n",
                total / steps, steps, warmup, finite ? "true" : "false", fused, T, H, W, L, blaslt.c_str());

    for (auto& e : ev)
        (void)hipEventDestroy(e);
    sv2_dit_destroy(dit);
    for (sv2_block* b : blocks)
        sv2_block_destroy(b);
    sv2_dit_input_destroy(input);
    sv2_dit_output_destroy(output);
    (void)hipFree(ws);
    (void)hipFree(out);
    (void)hipStreamDestroy(stream);
    return finite ? 0 : 7;
}
