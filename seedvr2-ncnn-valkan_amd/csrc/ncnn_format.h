// Readers of the ncnn model formats the reference's DiT blocks ship in: the
// text .param graph and the .bin weight stream of ModelBin records.
//
// .param (tools/export_seedvr2_dit_ncnn.py:166-187 writes it):
//   7767517
//   <layer count> <blob count>
//   <type> <name> <bottom count> <top count> <bottoms...> <tops...> <id=value...>
// A value containing '.', 'e' or 'E' is a float, otherwise an int; an id of
// -23300 - k marks an array "n,v1,...,vn" for param k.
//
// .bin: a sequence of ModelBin::load(count, type) records
// (tools/export_seedvr2_dit_ncnn.py:120-150):
//   type 1  raw fp32 values, no header (ada vectors, biases, norms, rope freqs);
//   type 0  a 4-byte tag, then the values (InnerProduct weights):
//             0x01306B47  fp16, padded to a multiple of 4 bytes
//             0x000D4B38  int8 (not supported here)
//             0x0002C056  fp32
//             0x00000000  fp32
//             other       a 256-entry fp32 table followed by count uint8
//                         indices (padded to 4 bytes): value = table[index]
#pragma once

#include <cstdint>
#include <cstdio>
#include <map>
#include <string>
#include <vector>

namespace sv2
{

struct ParamLayer
{
    std::string type;
    std::string name;
    std::vector<std::string> bottoms;
    std::vector<std::string> tops;
    std::map<int, std::string> values; // scalar params by id
    std::map<int, std::vector<std::string>> arrays;

    bool has(int id) const
    {
        return values.count(id) != 0;
    }
    int get_int(int id, int fallback) const;
    float get_float(int id, float fallback) const;
};

// Parses a .param file.  Returns 0, or -1 with a message in *error.
int read_param_file(const std::string& path, std::vector<ParamLayer>* layers, std::string* error);

// Sequential reader of ModelBin records.
class BinReader
{
  public:
    BinReader() = default;
    ~BinReader();
    BinReader(const BinReader&) = delete;
    BinReader& operator=(const BinReader&) = delete;

    int open(const std::string& path, std::string* error);
    // type 1: count raw fp32 values
    int load_raw(size_t count, std::vector<float>* out, std::string* error);
    // type 0: tagged record of count values, decoded to fp32
    int load_tagged(size_t count, std::vector<float>* out, std::string* error);
    // bytes left in the stream (to check that a file was fully consumed)
    int64_t remaining() const;

  private:
    int read_bytes(void* dst, size_t bytes, std::string* error);

    std::FILE* file_ = nullptr;
    int64_t size_ = 0;
    int64_t pos_ = 0;
};

// IEEE half -> float (all finite values, infinities and NaN).
float half_to_float(uint16_t h);

} // namespace sv2
