// SHA-256 (FIPS 180-4) and the SHA256SUMS check of a model directory.
//
// The reference checks a model directory with `sha256sum --check --strict
// SHA256SUMS` (scripts/verify-models.sh:17-24) and parses the manifest as
// lines "<64 hex digits> <file name>", rejecting file names that contain '/',
// are empty or start with '.', and lines with extra fields
// (download-models.sh:93-97, :140-148).  sv2_verify_checksums does the same in
// the library, hashing the listed files on several threads.
#include <algorithm>
#include <atomic>
#include <cctype>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <sstream>
#include <string>
#include <thread>
#include <vector>

#include "sv2_internal.h"

namespace sv2
{
namespace
{

// The first 32 bits of the fractional parts of the cube roots of the first
// 64 primes (FIPS 180-4, 4.2.2).
constexpr uint32_t kRound[64] = {
    0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u, 0x923f82a4u, 0xab1c5ed5u,
    0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u, 0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u,
    0xe49b69c1u, 0xefbe4786u, 0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
    0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u, 0x06ca6351u, 0x14292967u,
    0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u, 0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u,
    0xa2bfe8a1u, 0xa81a664bu, 0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
    0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au, 0x5b9cca4fu, 0x682e6ff3u,
    0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u, 0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};

// The first 32 bits of the fractional parts of the square roots of the first
// 8 primes (FIPS 180-4, 5.3.3).
constexpr uint32_t kInitial[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                                  0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};

inline uint32_t rotr(uint32_t x, int n)
{
    return (x >> n) | (x << (32 - n));
}

class Sha256
{
  public:
    Sha256()
    {
        std::memcpy(h_, kInitial, sizeof(h_));
    }

    void update(const unsigned char* p, size_t n)
    {
        bytes_ += n;
        if (fill_)
        {
            const size_t take = std::min(n, size_t(64) - fill_);
            std::memcpy(block_ + fill_, p, take);
            fill_ += take;
            p += take;
            n -= take;
            if (fill_ < 64)
                return;
            compress(block_);
            fill_ = 0;
        }
        for (; n >= 64; p += 64, n -= 64)
            compress(p);
        std::memcpy(block_, p, n);
        fill_ = n;
    }

    // Padding (5.1.1): a 1 bit, zeros to 56 mod 64 bytes, the message length
    // in bits as a big-endian 64-bit integer.
    void finish(unsigned char digest[32])
    {
        const uint64_t bits = bytes_ * 8;
        unsigned char pad[72] = {0x80};
        const size_t zeros = (fill_ < 56 ? 56 - fill_ : 120 - fill_);
        for (int i = 0; i < 8; i++)
            pad[zeros + i] = static_cast<unsigned char>(bits >> (56 - 8 * i));
        update(pad, zeros + 8);
        for (int i = 0; i < 8; i++)
            for (int j = 0; j < 4; j++)
                digest[4 * i + j] = static_cast<unsigned char>(h_[i] >> (24 - 8 * j));
    }

  private:
    // One 512-bit block (6.2.2).
    void compress(const unsigned char* p)
    {
        uint32_t w[64];
        for (int t = 0; t < 16; t++)
            w[t] = uint32_t(p[4 * t]) << 24 | uint32_t(p[4 * t + 1]) << 16 | uint32_t(p[4 * t + 2]) << 8 |
                   uint32_t(p[4 * t + 3]);
        for (int t = 16; t < 64; t++)
        {
            const uint32_t s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3);
            const uint32_t s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10);
            w[t] = w[t - 16] + s0 + w[t - 7] + s1;
        }
        uint32_t a = h_[0], b = h_[1], c = h_[2], d = h_[3], e = h_[4], f = h_[5], g = h_[6], h = h_[7];
        for (int t = 0; t < 64; t++)
        {
            const uint32_t t1 =
                h + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + kRound[t] + w[t];
            const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
            h = g;
            g = f;
            f = e;
            e = d + t1;
            d = c;
            c = b;
            b = a;
            a = t1 + t2;
        }
        h_[0] += a;
        h_[1] += b;
        h_[2] += c;
        h_[3] += d;
        h_[4] += e;
        h_[5] += f;
        h_[6] += g;
        h_[7] += h;
    }

    uint32_t h_[8];
    unsigned char block_[64];
    size_t fill_ = 0;
    uint64_t bytes_ = 0;
};

// Digest of a file, read in 4 MiB pieces; false when it cannot be read.
bool hash_file(const std::string& path, unsigned char digest[32])
{
    std::FILE* f = std::fopen(path.c_str(), "rb");
    if (!f)
        return false;
    std::vector<unsigned char> buf(size_t(4) << 20);
    Sha256 s;
    size_t got;
    while ((got = std::fread(buf.data(), 1, buf.size(), f)) > 0)
        s.update(buf.data(), got);
    const bool ok = !std::ferror(f);
    std::fclose(f);
    if (ok)
        s.finish(digest);
    return ok;
}

std::string hex(const unsigned char digest[32])
{
    static const char* digits = "0123456789abcdef";
    std::string out(64, '0');
    for (int i = 0; i < 32; i++)
    {
        out[2 * i] = digits[digest[i] >> 4];
        out[2 * i + 1] = digits[digest[i] & 15];
    }
    return out;
}

struct Entry
{
    std::string digest; // 64 lower-case hex digits
    std::string name;
    int line;
};

// Parses SHA256SUMS.  Lines are "<digest> <name>" or "<digest> *<name>" (the
// sha256sum text and binary forms, two characters between the fields);
// blank lines are skipped (download-models.sh:142).
int parse_manifest(const std::string& path, std::vector<Entry>* out)
{
    std::ifstream in(path);
    if (!in)
        return set_error(SV2_EINVAL, "checksums: cannot read " + path);
    std::string line;
    int number = 0;
    while (std::getline(in, line))
    {
        number++;
        if (!line.empty() && line.back() == '\r')
            line.pop_back();
        if (line.find_first_not_of(" \t") == std::string::npos)
            continue;
        std::istringstream fields(line);
        std::string digest, name, extra;
        fields >> digest >> name;
        const bool more = bool(fields >> extra);
        const std::string where = path + ":" + std::to_string(number);
        if (digest.size() != 64 ||
            !std::all_of(digest.begin(), digest.end(), [](unsigned char c) { return std::isxdigit(c) != 0; }))
            return set_error(SV2_EINVAL, "checksums: invalid SHA256 at " + where);
        if (more)
            return set_error(SV2_EINVAL, "checksums: invalid checksum line at " + where);
        if (!name.empty() && name[0] == '*')
            name.erase(0, 1);
        if (name.empty() || name[0] == '.' || name.find('/') != std::string::npos)
            return set_error(SV2_EINVAL, "checksums: unsafe file name at " + where + ": " + name);
        std::transform(digest.begin(), digest.end(), digest.begin(),
                       [](unsigned char c) { return static_cast<char>(std::tolower(c)); });
        out->push_back({digest, name, number});
    }
    if (out->empty())
        return set_error(SV2_EINVAL, "checksums: " + path + " lists no files");
    return SV2_OK;
}

} // namespace
} // namespace sv2

namespace sv2
{
namespace
{

// Size of a file in bytes, -1 when it cannot be opened.
long long file_size(const std::string& path)
{
    std::FILE* f = std::fopen(path.c_str(), "rb");
    if (!f)
        return -1;
    long long n = -1;
    if (std::fseek(f, 0, SEEK_END) == 0)
        n = std::ftell(f);
    std::fclose(f);
    return n;
}

bool read_whole(const std::string& path, std::vector<unsigned char>* out)
{
    std::FILE* f = std::fopen(path.c_str(), "rb");
    if (!f)
        return false;
    out->clear();
    unsigned char buf[1 << 16];
    size_t n;
    while ((n = std::fread(buf, 1, sizeof(buf), f)) > 0)
        out->insert(out->end(), buf, buf + n);
    const bool ok = !std::ferror(f);
    std::fclose(f);
    return ok;
}

// `sha256sum --check --strict SHA256SUMS` in `dir`.  Without a manifest:
// 0 (nothing to check), or an error when `strict` (scripts/verify-models.sh:22
// requires a non-empty one).  Each worker records per file 0 (ok), 1
// (unreadable), 2 (mismatch) or 3 (could not be hashed: an allocation failed
// on its thread), so no exception leaves a thread; when a thread cannot be
// started the threads already running and the calling thread share the
// files, and every started thread is joined before returning.
int verify_manifest(const std::string& root, int threads, bool strict)
{
    const std::string manifest = root + "/SHA256SUMS";
    const long long size = file_size(manifest);
    if (size < 0 || (strict && size == 0))
    {
        if (strict)
            return set_error(SV2_EINVAL, "checksums: " + manifest + " is missing");
        return 0; // nothing to check
    }
    std::vector<Entry> entries;
    int rc = parse_manifest(manifest, &entries);
    if (rc != SV2_OK)
        return rc;
    if (threads <= 0)
        threads = static_cast<int>(std::min(16u, std::max(1u, std::thread::hardware_concurrency())));
    threads = std::min<int>(threads, static_cast<int>(entries.size()));
    // each worker takes the next file; the first failure in list order is reported
    std::atomic<size_t> next{0};
    std::vector<int> status(entries.size(), 0);
    auto work = [&]() noexcept {
        for (size_t i; (i = next.fetch_add(1)) < entries.size();)
        {
            try
            {
                unsigned char digest[32];
                if (!hash_file(root + "/" + entries[i].name, digest))
                    status[i] = 1;
                else if (hex(digest) != entries[i].digest)
                    status[i] = 2;
            }
            catch (...)
            {
                status[i] = 3;
            }
        }
    };
    std::vector<std::thread> pool;
    try
    {
        pool.reserve(static_cast<size_t>(threads));
        for (int t = 1; t < threads; t++)
            pool.emplace_back(work);
    }
    catch (...)
    {
        // fewer threads than asked for: the rest of the files go to the
        // threads already started and to this one
    }
    work();
    for (std::thread& t : pool)
        t.join();
    for (size_t i = 0; i < entries.size(); i++)
    {
        if (status[i] == 3)
            return set_error(SV2_EDEVICE, "checksums: " + root + "/" + entries[i].name +
                                              " could not be hashed (out of host memory)");
        if (status[i])
            return set_error(SV2_EINVAL, "checksums: " + root + "/" + entries[i].name +
                                             (status[i] == 1 ? " is missing or unreadable"
                                                             : " is corrupted (SHA256 mismatch)"));
    }
    return static_cast<int>(entries.size());
}

} // namespace
} // namespace sv2

extern "C" {

int sv2_sha256(const void* data, size_t bytes, unsigned char digest[32])
try
{
    if ((!data && bytes) || !digest)
        return sv2::set_error(SV2_EINVAL, "sv2_sha256: null argument");
    sv2::Sha256 s;
    s.update(static_cast<const unsigned char*>(data), bytes);
    s.finish(digest);
    return SV2_OK;
}
catch (...)
{
    return sv2::caught_exception("sv2_sha256");
}

int sv2_sha256_file(const char* path, unsigned char digest[32])
try
{
    if (!path || !digest)
        return sv2::set_error(SV2_EINVAL, "sv2_sha256_file: null argument");
    return sv2::hash_file(path, digest) ? SV2_OK
                                        : sv2::set_error(SV2_EINVAL, std::string("sv2_sha256_file: cannot read ") + path);
}
catch (...)
{
    return sv2::caught_exception("sv2_sha256_file");
}

int sv2_verify_checksums(const char* dir, int threads)
try
{
    if (!dir)
        return sv2::set_error(SV2_EINVAL, "sv2_verify_checksums: null directory");
    return sv2::verify_manifest(dir, threads, false);
}
catch (...)
{
    return sv2::caught_exception("sv2_verify_checksums");
}

int sv2_verify_checksums_strict(const char* dir, int threads)
try
{
    if (!dir)
        return sv2::set_error(SV2_EINVAL, "sv2_verify_checksums_strict: null directory");
    return sv2::verify_manifest(dir, threads, true);
}
catch (...)
{
    return sv2::caught_exception("sv2_verify_checksums_strict");
}

int sv2_verify_model_set(const char* model_root, const char* bundled_embeddings, int threads)
try
{
    using namespace sv2;
    if (!model_root)
        return set_error(SV2_EINVAL, "sv2_verify_model_set: null model directory");
    const std::string root(model_root);
    // the default text embeddings: present, and equal to the bundled ones
    // (scripts/verify-models.sh:27-31)
    for (const char* name : {"default_pos_emb.bin", "default_neg_emb.bin"})
    {
        std::vector<unsigned char> have;
        if (!read_whole(root + "/" + name, &have) || have.empty())
            return set_error(SV2_EINVAL, std::string("model set: ") + name + " is missing");
        if (bundled_embeddings)
        {
            std::vector<unsigned char> want;
            if (!read_whole(std::string(bundled_embeddings) + "/" + name, &want))
                return set_error(SV2_EINVAL, std::string("model set: the bundled ") + name + " is missing");
            if (have != want)
                return set_error(SV2_EINVAL, std::string("model set: ") + name + " differs from the bundled embedding");
        }
    }
    // the DiT component: its manifest required and every listed file intact
    // (:33-34), then every file the DiT loads present and non-empty (:36-47)
    const std::string dit = root + "/dit_full_fp16";
    const int n = verify_manifest(dit, threads, true);
    if (n < 0)
        return n;
    std::vector<std::string> stems = {"seedvr2_dit_input", "seedvr2_dit_output"};
    for (int i = 0; i < 32; i++)
    {
        char stem[64];
        std::snprintf(stem, sizeof(stem), "seedvr2_dit_block_%02d", i);
        stems.push_back(stem);
    }
    for (const std::string& stem : stems)
        for (const char* ext : {".ncnn.param", ".ncnn.bin"})
            if (file_size(dit + "/" + stem + ext) <= 0)
                return set_error(SV2_EINVAL, "model set: dit_full_fp16/" + stem + ext + " is missing or empty");
    return n;
}
catch (...)
{
    return sv2::caught_exception("sv2_verify_model_set");
}

} // extern "C"
