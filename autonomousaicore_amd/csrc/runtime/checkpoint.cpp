#include "checkpoint.hpp"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <memory>

#include "error.hpp"

namespace aic {

uint32_t adler32(const uint8_t* data, size_t len) {
    constexpr uint32_t kMod = 65521;
    // 5552 bytes is the longest run whose sums cannot overflow 32 bits before the reduction
    uint32_t a = 1, b = 0;
    while (len > 0) {
        const size_t n = std::min<size_t>(len, 5552);
        for (size_t i = 0; i < n; ++i) {
            a += data[i];
            b += a;
        }
        a %= kMod;
        b %= kMod;
        data += n;
        len -= n;
    }
    return (b << 16) | a;
}

namespace {

struct File {
    std::FILE* f = nullptr;
    ~File() {
        if (f) std::fclose(f);
    }
};

template <typename T>
void put(std::FILE* f, const T& v, const std::string& path) {
    AIC_CHECK(std::fwrite(&v, sizeof(T), 1, f) == 1, IOError, "write failed: ", path);
}

void put_bytes(std::FILE* f, const void* p, size_t n, const std::string& path) {
    if (n == 0) return;
    AIC_CHECK(std::fwrite(p, 1, n, f) == n, IOError, "write failed: ", path);
}

template <typename T>
T get(std::FILE* f, const std::string& path) {
    T v{};
    AIC_CHECK(std::fread(&v, sizeof(T), 1, f) == 1, FormatError, "truncated checkpoint: ", path);
    return v;
}

void get_bytes(std::FILE* f, void* p, size_t n, const std::string& path) {
    if (n == 0) return;
    AIC_CHECK(std::fread(p, 1, n, f) == n, FormatError, "truncated checkpoint: ", path);
}

// The registration keys of a parameter's path: "layers.3.attn.q_proj.weight" ->
// {"layers.3", "attn", "q_proj", "weight"}; "layers" and "experts" take their index along.
std::vector<std::string> keys_of(const std::string& name) {
    std::vector<std::string> parts, out;
    size_t start = 0;
    while (true) {
        const size_t dot = name.find('.', start);
        parts.push_back(name.substr(start, dot == std::string::npos ? std::string::npos : dot - start));
        if (dot == std::string::npos) break;
        start = dot + 1;
    }
    for (size_t i = 0; i < parts.size(); ++i) {
        const bool indexed = (parts[i] == "layers" || parts[i] == "experts") && i + 1 < parts.size() &&
                             !parts[i + 1].empty() &&
                             std::all_of(parts[i + 1].begin(), parts[i + 1].end(), [](char c) { return c >= '0' && c <= '9'; });
        if (indexed) {
            out.push_back(parts[i] + "." + parts[i + 1]);
            ++i;
        } else {
            out.push_back(parts[i]);
        }
    }
    return out;
}

}  // namespace

void write_checkpoint(const std::string& path, const CheckpointMeta& meta, const std::vector<CheckpointTensorRef>& ts) {
    File fh;
    fh.f = std::fopen(path.c_str(), "wb");
    AIC_CHECK(fh.f, IOError, "Failed to open checkpoint file for writing: ", path);
    std::FILE* f = fh.f;
    put(f, kCheckpointMagic, path);
    put(f, kCheckpointVersion, path);
    put(f, meta.step, path);
    put(f, meta.epoch, path);
    put(f, meta.best_val_loss, path);
    put(f, static_cast<uint32_t>(meta.description.size()), path);
    put_bytes(f, meta.description.data(), meta.description.size(), path);
    put(f, static_cast<uint64_t>(ts.size()), path);
    for (const auto& t : ts) {
        AIC_CHECK(t.data || t.nbytes == 0, InvalidArgument, "checkpoint tensor without data: ", t.name);
        put(f, static_cast<uint32_t>(t.name.size()), path);
        put_bytes(f, t.name.data(), t.name.size(), path);
        put(f, static_cast<int32_t>(t.dims.size()), path);
        for (int64_t d : t.dims) put(f, d, path);
        put(f, t.dtype, path);
        put(f, t.nbytes, path);
        put_bytes(f, t.data, static_cast<size_t>(t.nbytes), path);
        put(f, adler32(static_cast<const uint8_t*>(t.data), static_cast<size_t>(t.nbytes)), path);
    }
    AIC_CHECK(std::fflush(f) == 0, IOError, "write failed: ", path);
}

void read_checkpoint(const std::string& path, CheckpointMeta& meta, std::vector<CheckpointTensor>& ts) {
    File fh;
    fh.f = std::fopen(path.c_str(), "rb");
    AIC_CHECK(fh.f, IOError, "Failed to open checkpoint file for reading: ", path);
    std::FILE* f = fh.f;
    std::fseek(f, 0, SEEK_END);
    const long fsize = std::ftell(f);
    std::fseek(f, 0, SEEK_SET);
    const uint32_t magic = get<uint32_t>(f, path);
    AIC_CHECK(magic == kCheckpointMagic, FormatError, "Invalid checkpoint magic number in: ", path);
    const uint32_t version = get<uint32_t>(f, path);
    AIC_CHECK(version == kCheckpointVersion, FormatError, "Unsupported checkpoint version: ", version);
    meta.step = get<int64_t>(f, path);
    meta.epoch = get<int64_t>(f, path);
    meta.best_val_loss = get<float>(f, path);
    const uint32_t dlen = get<uint32_t>(f, path);
    AIC_CHECK(static_cast<long>(dlen) <= fsize, FormatError, "corrupt description length in: ", path);
    meta.description.assign(dlen, '\0');
    get_bytes(f, meta.description.data(), dlen, path);
    const uint64_t n = get<uint64_t>(f, path);
    ts.clear();
    for (uint64_t i = 0; i < n; ++i) {
        CheckpointTensor t;
        const uint32_t nl = get<uint32_t>(f, path);
        AIC_CHECK(static_cast<long>(nl) <= fsize, FormatError, "corrupt name length in: ", path);
        t.name.assign(nl, '\0');
        get_bytes(f, t.name.data(), nl, path);
        const int32_t rank = get<int32_t>(f, path);
        AIC_CHECK(rank >= 0 && rank <= 16, FormatError, "corrupt rank for tensor '", t.name, "' in: ", path);
        t.dims.resize(static_cast<size_t>(rank));
        for (auto& d : t.dims) d = get<int64_t>(f, path);
        t.dtype = get<int32_t>(f, path);
        const uint64_t nbytes = get<uint64_t>(f, path);
        AIC_CHECK(nbytes <= static_cast<uint64_t>(fsize), FormatError, "corrupt size for tensor '", t.name, "' in: ",
                  path);
        t.data.resize(static_cast<size_t>(nbytes));
        get_bytes(f, t.data.data(), static_cast<size_t>(nbytes), path);
        const uint32_t stored = get<uint32_t>(f, path);
        AIC_CHECK(stored == adler32(t.data.data(), t.data.size()), FormatError, "Adler-32 checksum mismatch for tensor '",
                  t.name, "' in checkpoint: ", path);
        ts.push_back(std::move(t));
    }
}

std::vector<size_t> module_order(const std::vector<std::string>& names) {
    std::vector<std::vector<std::string>> keys(names.size());
    for (size_t i = 0; i < names.size(); ++i) keys[i] = keys_of(names[i]);
    std::vector<size_t> idx(names.size());
    for (size_t i = 0; i < idx.size(); ++i) idx[i] = i;
    std::stable_sort(idx.begin(), idx.end(), [&](size_t x, size_t y) {
        const auto& a = keys[x];
        const auto& b = keys[y];
        for (size_t l = 0; l < a.size() && l < b.size(); ++l) {
            const bool leaf_a = l + 1 == a.size(), leaf_b = l + 1 == b.size();
            if (a[l] == b[l] && leaf_a == leaf_b) continue;
            if (leaf_a != leaf_b) return leaf_a;  // a module's own parameters come before its submodules
            return a[l] < b[l];
        }
        return a.size() < b.size();
    });
    return idx;
}

}  // namespace aic
