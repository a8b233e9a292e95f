// Readers of the ncnn .param / .bin formats (see ncnn_format.h).
#include "ncnn_format.h"

#include <cctype>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>

namespace sv2
{

namespace
{
constexpr uint32_t kTagFp16 = 0x01306B47u;
constexpr uint32_t kTagInt8 = 0x000D4B38u;
constexpr uint32_t kTagFp32 = 0x0002C056u;
constexpr int kParamMagic = 7767517;
constexpr int kArrayKeyBase = -23300;

bool is_float_text(const std::string& v)
{
    return v.find_first_of(".eE") != std::string::npos;
}
} // namespace

int ParamLayer::get_int(int id, int fallback) const
{
    const auto it = values.find(id);
    if (it == values.end())
        return fallback;
    if (is_float_text(it->second))
        return static_cast<int>(std::strtof(it->second.c_str(), nullptr));
    return static_cast<int>(std::strtol(it->second.c_str(), nullptr, 10));
}

float ParamLayer::get_float(int id, float fallback) const
{
    const auto it = values.find(id);
    if (it == values.end())
        return fallback;
    return std::strtof(it->second.c_str(), nullptr);
}

int read_param_file(const std::string& path, std::vector<ParamLayer>* layers, std::string* error)
{
    std::ifstream in(path);
    if (!in)
    {
        *error = "cannot open " + path;
        return -1;
    }
    int magic = 0;
    int layer_count = 0;
    int blob_count = 0;
    if (!(in >> magic) || magic != kParamMagic)
    {
        *error = path + ": not an ncnn .param file (magic 7767517 missing)";
        return -1;
    }
    if (!(in >> layer_count >> blob_count) || layer_count < 0 || blob_count < 0)
    {
        *error = path + ": bad layer / blob count line";
        return -1;
    }
    std::string line;
    std::getline(in, line); // rest of the count line
    layers->clear();
    for (int li = 0; li < layer_count; li++)
    {
        do
        {
            if (!std::getline(in, line))
            {
                *error = path + ": fewer layer lines than declared";
                return -1;
            }
        } while (line.find_first_not_of(" \t\r") == std::string::npos);
        std::istringstream ls(line);
        ParamLayer layer;
        int nb = 0;
        int nt = 0;
        if (!(ls >> layer.type >> layer.name >> nb >> nt) || nb < 0 || nt < 0)
        {
            *error = path + ": malformed layer line: " + line;
            return -1;
        }
        layer.bottoms.resize(nb);
        layer.tops.resize(nt);
        for (auto& b : layer.bottoms)
            ls >> b;
        for (auto& t : layer.tops)
            ls >> t;
        if (!ls)
        {
            *error = path + ": layer line lists fewer blobs than declared: " + line;
            return -1;
        }
        std::string kv;
        while (ls >> kv)
        {
            const size_t eq = kv.find('=');
            if (eq == std::string::npos || eq == 0)
            {
                *error = path + ": malformed param '" + kv + "' in: " + line;
                return -1;
            }
            char* end = nullptr;
            const long id = std::strtol(kv.c_str(), &end, 10);
            if (end != kv.c_str() + eq)
            {
                *error = path + ": malformed param id '" + kv + "'";
                return -1;
            }
            const std::string value = kv.substr(eq + 1);
            if (id <= kArrayKeyBase)
            {
                std::vector<std::string> items;
                std::stringstream vs(value);
                std::string item;
                while (std::getline(vs, item, ','))
                    items.push_back(item);
                if (items.empty())
                {
                    *error = path + ": empty array param '" + kv + "'";
                    return -1;
                }
                items.erase(items.begin()); // leading element count
                layer.arrays[static_cast<int>(kArrayKeyBase - id)] = items;
            }
            else
            {
                layer.values[static_cast<int>(id)] = value;
            }
        }
        layers->push_back(std::move(layer));
    }
    return 0;
}

float half_to_float(uint16_t h)
{
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1f;
    uint32_t mant = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0)
    {
        if (mant == 0)
        {
            bits = sign;
        }
        else
        {
            // subnormal: normalise
            int e = -1;
            do
            {
                e++;
                mant <<= 1;
            } while ((mant & 0x400u) == 0);
            mant &= 0x3ffu;
            bits = sign | (static_cast<uint32_t>(127 - 15 - e) << 23) | (mant << 13);
        }
    }
    else if (exp == 31)
    {
        bits = sign | 0x7f800000u | (mant << 13);
    }
    else
    {
        bits = sign | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    float f;
    std::memcpy(&f, &bits, sizeof(f));
    return f;
}

BinReader::~BinReader()
{
    if (file_)
        std::fclose(file_);
}

int BinReader::open(const std::string& path, std::string* error)
{
    if (file_)
        std::fclose(file_);
    file_ = std::fopen(path.c_str(), "rb");
    if (!file_)
    {
        *error = "cannot open " + path;
        return -1;
    }
    std::fseek(file_, 0, SEEK_END);
    size_ = std::ftell(file_);
    std::fseek(file_, 0, SEEK_SET);
    pos_ = 0;
    return 0;
}

int64_t BinReader::remaining() const
{
    return size_ - pos_;
}

int BinReader::read_bytes(void* dst, size_t bytes, std::string* error)
{
    if (!file_ || static_cast<int64_t>(bytes) > size_ - pos_)
    {
        *error = "weight file ended early";
        return -1;
    }
    if (bytes && std::fread(dst, 1, bytes, file_) != bytes)
    {
        *error = "weight file read failed";
        return -1;
    }
    pos_ += static_cast<int64_t>(bytes);
    return 0;
}

int BinReader::load_raw(size_t count, std::vector<float>* out, std::string* error)
{
    out->resize(count);
    return read_bytes(out->data(), count * sizeof(float), error);
}

int BinReader::load_tagged(size_t count, std::vector<float>* out, std::string* error)
{
    unsigned char flag[4];
    if (read_bytes(flag, 4, error) != 0)
        return -1;
    uint32_t tag;
    std::memcpy(&tag, flag, 4);
    out->resize(count);
    if (tag == kTagFp16)
    {
        const size_t bytes = (count * 2 + 3) & ~static_cast<size_t>(3);
        std::vector<uint16_t> half((bytes + 1) / 2);
        if (read_bytes(half.data(), bytes, error) != 0)
            return -1;
        for (size_t i = 0; i < count; i++)
            (*out)[i] = half_to_float(half[i]);
        return 0;
    }
    if (tag == kTagInt8)
    {
        *error = "int8 weight records are not supported";
        return -1;
    }
    if (tag == kTagFp32 || tag == 0)
        return read_bytes(out->data(), count * sizeof(float), error);
    // a non-zero flag without a known tag: quantisation table + indices
    float table[256];
    if (read_bytes(table, sizeof(table), error) != 0)
        return -1;
    const size_t bytes = (count + 3) & ~static_cast<size_t>(3);
    std::vector<unsigned char> index(bytes);
    if (read_bytes(index.data(), bytes, error) != 0)
        return -1;
    for (size_t i = 0; i < count; i++)
        (*out)[i] = table[index[i]];
    return 0;
}

} // namespace sv2
