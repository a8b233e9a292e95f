// Host-side types with the members of ncnn's Layer, ParamDict, ModelBin, Mat
// and Option that sv2::DiTBlockLayer uses, so that the adapter compiles, loads
// exported blocks and runs without an ncnn build:
//   ParamDict  the id=value pairs of one .param layer line (ints; a value with
//              '.', 'e' or 'E' is a float, as ncnn's ParamDict::load_param)
//   ModelBin   a .bin stream of ModelBin::load(w, type) records: type 1 raw
//              fp32; type 0 a 4-byte flag, then fp16 (0x01306B47), fp32
//              (0x0002C056 or flag 0) or a 256-entry fp32 table + uint8
//              indices (any other non-zero flag), decoded to fp32
//   Net        load_param / load_model of a .param + .bin pair through
//              registered layer creators (ncnn::Net::register_custom_layer)
#pragma once

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <sstream>
#include <string>
#include <vector>

namespace host
{

struct Mat
{
    int dims = 0;
    int w = 0;
    int h = 0;
    size_t elemsize = 4;
    void* data = nullptr;
    std::shared_ptr<std::vector<unsigned char>> store;

    Mat() = default;
    Mat(int w_, size_t es, void* allocator = nullptr)
    {
        create(w_, es, allocator);
    }
    void create(int w_, size_t es, void* = nullptr)
    {
        allocate(1, w_, 1, es);
    }
    void create(int w_, int h_, size_t es, void* = nullptr)
    {
        allocate(2, w_, h_, es);
    }
    bool empty() const
    {
        return data == nullptr || size_t(w) * h == 0;
    }

  private:
    void allocate(int d, int w_, int h_, size_t es)
    {
        dims = d;
        w = w_;
        h = h_;
        elemsize = es;
        const size_t bytes = size_t(w_ > 0 ? w_ : 0) * size_t(h_ > 0 ? h_ : 0) * es;
        store = bytes ? std::make_shared<std::vector<unsigned char>>(bytes) : nullptr;
        data = store ? store->data() : nullptr;
    }
};

struct Option
{
    void* blob_allocator = nullptr;
    bool use_fp16_arithmetic = false;
};

struct ParamDict
{
    std::map<int, std::string> values;

    int get(int id, int fallback) const
    {
        auto it = values.find(id);
        return it == values.end() ? fallback : std::atoi(it->second.c_str());
    }
    float get(int id, float fallback) const
    {
        auto it = values.find(id);
        return it == values.end() ? fallback : std::strtof(it->second.c_str(), nullptr);
    }
};

inline float half_to_float(uint16_t h)
{
    const uint32_t sign = uint32_t(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0x1f)
        bits = sign | 0x7f800000u | (mant << 13);
    else if (exp != 0)
        bits = sign | ((exp + 112u) << 23) | (mant << 13);
    else if (mant == 0)
        bits = sign;
    else
    {
        int e = -1;
        do
        {
            mant <<= 1;
            e++;
        } while (!(mant & 0x400u));
        bits = sign | (uint32_t(112 - e) << 23) | ((mant & 0x3ffu) << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

class ModelBin
{
  public:
    explicit ModelBin(const std::string& path) : in_(path, std::ios::binary)
    {
    }
    bool ok() const
    {
        return bool(in_);
    }
    // bytes after the last record read (a fully consumed file has none)
    int64_t remaining() const
    {
        const std::streampos at = in_.tellg();
        in_.seekg(0, std::ios::end);
        const std::streampos end = in_.tellg();
        in_.seekg(at);
        return int64_t(end - at);
    }
    Mat load(int w, int type) const
    {
        Mat m;
        if (w <= 0)
            return m;
        m.create(w, size_t(4u));
        float* out = static_cast<float*>(m.data);
        if (type == 1)
            return read(out, size_t(w) * 4) ? m : Mat();
        uint32_t flag = 0;
        unsigned char f[4];
        if (!read(f, 4))
            return Mat();
        std::memcpy(&flag, f, 4);
        if (flag == 0x01306B47u)
        {
            std::vector<uint16_t> half(w);
            if (!read(half.data(), size_t(w) * 2) || !skip((4 - (size_t(w) * 2) % 4) % 4))
                return Mat();
            for (int i = 0; i < w; i++)
                out[i] = half_to_float(half[i]);
            return m;
        }
        if (flag == 0x000D4B38u)
            return Mat(); // int8 records are not used by the block
        if (flag == 0x0002C056u || f[0] + f[1] + f[2] + f[3] == 0)
            return read(out, size_t(w) * 4) ? m : Mat();
        float table[256];
        std::vector<unsigned char> idx(w);
        if (!read(table, sizeof(table)) || !read(idx.data(), size_t(w)) || !skip((4 - size_t(w) % 4) % 4))
            return Mat();
        for (int i = 0; i < w; i++)
            out[i] = table[idx[i]];
        return m;
    }

  private:
    bool read(void* dst, size_t bytes) const
    {
        in_.read(static_cast<char*>(dst), static_cast<std::streamsize>(bytes));
        return size_t(in_.gcount()) == bytes;
    }
    bool skip(size_t bytes) const
    {
        char pad[4];
        return bytes == 0 || read(pad, bytes);
    }
    mutable std::ifstream in_;
};

struct Layer
{
    virtual ~Layer() = default;
    bool one_blob_only = false;
    bool support_inplace = false;
    virtual int load_param(const ParamDict&)
    {
        return 0;
    }
    virtual int load_model(const ModelBin&)
    {
        return 0;
    }
    virtual int create_pipeline(const Option&)
    {
        return 0;
    }
    virtual int destroy_pipeline(const Option&)
    {
        return 0;
    }
    virtual int forward(const std::vector<Mat>&, std::vector<Mat>&, const Option&) const
    {
        return -1;
    }
};

struct Api
{
    using Layer = host::Layer;
    using ParamDict = host::ParamDict;
    using ModelBin = host::ModelBin;
    using Mat = host::Mat;
    using Option = host::Option;
};

typedef Layer* (*layer_creator_func)(void* userdata);

// The custom layers of one .param file (Input layers are skipped), loaded in
// file order as ncnn::Net::load_param / load_model do.
class Net
{
  public:
    Option opt;
    bool create_pipelines = true; // false: parse and load only (no device)
    int64_t trailing_bytes = -1;  // bytes of the .bin left after load_model

    ~Net()
    {
        for (auto& l : layers_)
        {
            if (create_pipelines)
                l.layer->destroy_pipeline(opt);
            delete l.layer;
        }
    }
    void register_custom_layer(const std::string& type, layer_creator_func creator)
    {
        creators_[type] = creator;
    }
    int load_param(const std::string& path)
    {
        std::ifstream in(path);
        std::string magic, line;
        int nlayers = 0, nblobs = 0;
        if (!(in >> magic >> nlayers >> nblobs) || magic != "7767517")
            return -1;
        std::getline(in, line);
        for (int i = 0; i < nlayers && std::getline(in, line); i++)
        {
            std::istringstream ls(line);
            std::string type, name;
            int nb = 0, nt = 0;
            ls >> type >> name >> nb >> nt;
            std::string blob;
            for (int k = 0; k < nb + nt; k++)
                ls >> blob;
            if (type == "Input")
                continue;
            auto it = creators_.find(type);
            if (it == creators_.end())
            {
                std::fprintf(stderr, "layer %s not exists or registered\n", type.c_str());
                return -1;
            }
            ParamDict pd;
            std::string kv;
            while (ls >> kv)
            {
                const size_t eq = kv.find('=');
                if (eq != std::string::npos)
                    pd.values[std::atoi(kv.substr(0, eq).c_str())] = kv.substr(eq + 1);
            }
            Layer* layer = it->second(nullptr);
            if (!layer || layer->load_param(pd) != 0)
            {
                delete layer;
                return -1;
            }
            layers_.push_back({type, layer});
        }
        return layers_.empty() ? -1 : 0;
    }
    int load_model(const std::string& path)
    {
        ModelBin mb(path);
        if (!mb.ok())
            return -1;
        for (auto& l : layers_)
            if (l.layer->load_model(mb) != 0)
                return -1;
        trailing_bytes = mb.remaining();
        for (auto& l : layers_)
            if (create_pipelines && l.layer->create_pipeline(opt) != 0)
                return -1;
        return 0;
    }
    std::vector<Layer*> mutable_layers()
    {
        std::vector<Layer*> out;
        for (auto& l : layers_)
            out.push_back(l.layer);
        return out;
    }

  private:
    struct Entry
    {
        std::string type;
        Layer* layer;
    };
    std::map<std::string, layer_creator_func> creators_;
    std::vector<Entry> layers_;
};

} // namespace host
