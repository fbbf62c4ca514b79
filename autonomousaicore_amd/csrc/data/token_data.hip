#include "token_data.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <numeric>

#include "../kernels/common.hpp"
#include "../runtime/error.hpp"
#include "../runtime/memory_pool.hpp"

namespace aic::data {

// ---------------------------------------------------------------------------- dataset
TokenDataset::TokenDataset(const std::string& path, int64_t seq_len, int64_t stride)
    : seq_len_(seq_len), stride_(stride) {
    AIC_CHECK(seq_len_ > 0, InvalidArgument, "seq_len must be positive, got ", seq_len_);
    const int fd = ::open(path.c_str(), O_RDONLY);
    AIC_CHECK(fd >= 0, IOError, "Failed to open token file: ", path);
    struct stat st {};
    if (::fstat(fd, &st) != 0) {
        ::close(fd);
        AIC_THROW(IOError, "Failed to stat token file: ", path);
    }
    map_bytes_ = static_cast<size_t>(st.st_size);
    if (map_bytes_ % sizeof(int64_t) != 0) {
        ::close(fd);
        AIC_THROW(InvalidArgument, "File size in bytes (", map_bytes_, ") is not a multiple of sizeof(int64_t)");
    }
    if (map_bytes_ > 0) {
        map_ = ::mmap(nullptr, map_bytes_, PROT_READ, MAP_PRIVATE, fd, 0);
        if (map_ == MAP_FAILED) {
            map_ = nullptr;
            ::close(fd);
            AIC_THROW(IOError, "Failed to map token file: ", path);
        }
    }
    ::close(fd);
    tok_ = static_cast<const int64_t*>(map_);
    total_ = static_cast<int64_t>(map_bytes_ / sizeof(int64_t));
    compute_samples();
}

TokenDataset::TokenDataset(std::vector<int64_t> tokens, int64_t seq_len, int64_t stride)
    : mem_(std::move(tokens)), seq_len_(seq_len), stride_(stride) {
    AIC_CHECK(seq_len_ > 0, InvalidArgument, "seq_len must be positive, got ", seq_len_);
    tok_ = mem_.data();
    total_ = static_cast<int64_t>(mem_.size());
    compute_samples();
}

TokenDataset::~TokenDataset() {
    if (map_) ::munmap(map_, map_bytes_);
}

void TokenDataset::compute_samples() {
    if (stride_ <= 0) stride_ = seq_len_;
    // a sample needs seq_len + 1 tokens (inputs and the next-token targets)
    num_samples_ = total_ >= seq_len_ + 1 ? (total_ - 1 - seq_len_) / stride_ + 1 : 0;
}

void TokenDataset::get_item(int64_t idx, int64_t* input, int64_t* target) const {
    AIC_CHECK(idx >= 0 && idx < num_samples_, OutOfRange, "Dataset index ", idx, " out of range [0, ", num_samples_,
              ")");
    const int64_t start = idx * stride_;
    if (input) std::memcpy(input, tok_ + start, sizeof(int64_t) * static_cast<size_t>(seq_len_));
    if (target) std::memcpy(target, tok_ + start + 1, sizeof(int64_t) * static_cast<size_t>(seq_len_));
}

int64_t TokenDataset::token_at(int64_t i) const {
    AIC_CHECK(i >= 0 && i < total_, OutOfRange, "Token index ", i, " out of bounds for total tokens ", total_);
    return tok_[i];
}

void TokenDataset::write_binary_file(const std::string& path, const int64_t* tokens, int64_t n) {
    std::FILE* f = std::fopen(path.c_str(), "wb");
    AIC_CHECK(f, IOError, "Failed to open output binary token file: ", path);
    const size_t w = n > 0 ? std::fwrite(tokens, sizeof(int64_t), static_cast<size_t>(n), f) : 0;
    const int c = std::fclose(f);
    AIC_CHECK(w == static_cast<size_t>(n > 0 ? n : 0) && c == 0, IOError, "write failed: ", path);
}

// ---------------------------------------------------------------------------- gather kernel
namespace {

// Block b copies the window tokens[start_b, start_b + S] into inputs row b (first S) and
// targets row b (last S); 8-byte elements, grid-stride over the row.
__global__ __launch_bounds__(256) void gather_windows_k(const int64_t* __restrict__ tokens,
                                                        const int64_t* __restrict__ starts, int64_t S,
                                                        int64_t* __restrict__ inputs, int64_t* __restrict__ targets) {
    const int64_t b = blockIdx.x;
    const int64_t* src = tokens + starts[b];
    for (int64_t i = threadIdx.x; i < S; i += 256) {
        inputs[b * S + i] = src[i];
        targets[b * S + i] = src[i + 1];
    }
}

}  // namespace

// ---------------------------------------------------------------------------- loader
TokenLoader::TokenLoader(std::shared_ptr<TokenDataset> ds, int64_t batch_size, bool shuffle, bool drop_last,
                         uint64_t seed, bool resident)
    : ds_(std::move(ds)), batch_(batch_size), shuffle_(shuffle), drop_last_(drop_last), resident_(resident),
      rng_(seed) {
    AIC_CHECK(ds_ != nullptr, InvalidArgument, "DataLoader requires a valid dataset");
    AIC_CHECK(batch_ > 0, InvalidArgument, "batch_size must be positive, got ", batch_);
    const int64_t n = ds_->size();
    idx_.resize(static_cast<size_t>(n));
    std::iota(idx_.begin(), idx_.end(), int64_t{0});
    num_batches_ = drop_last_ ? n / batch_ : (n + batch_ - 1) / batch_;
    reset();
}

TokenLoader::~TokenLoader() {
    for (int i = 0; i < 2; ++i) {
        if (done_[i]) {
            (void)hipEventSynchronize(done_[i]);
            (void)hipEventDestroy(done_[i]);
        }
        if (pinned_[i]) (void)hipHostFree(pinned_[i]);
    }
    if (dev_tokens_) (void)hipFree(dev_tokens_);
}

void TokenLoader::reset() {
    cur_ = 0;
    if (shuffle_ && !idx_.empty()) std::shuffle(idx_.begin(), idx_.end(), rng_);
}

int64_t TokenLoader::take(std::vector<int64_t>& samples) {
    AIC_CHECK(has_next(), OutOfRange, "DataLoader reached end of epoch (current_batch = ", cur_, ", num_batches = ",
              num_batches_, ")");
    const int64_t start = cur_ * batch_;
    const int64_t b = std::min(batch_, ds_->size() - start);
    samples.assign(idx_.begin() + start, idx_.begin() + start + b);
    ++cur_;
    return b;
}

int64_t TokenLoader::next_host(int64_t* inputs, int64_t* targets) {
    std::vector<int64_t> samples;
    const int64_t b = take(samples);
    const int64_t S = ds_->seq_len();
    for (int64_t i = 0; i < b; ++i) ds_->get_item(samples[static_cast<size_t>(i)], inputs + i * S, targets + i * S);
    return b;
}

int64_t TokenLoader::next_device(int64_t* inputs, int64_t* targets, hipStream_t s) {
    AIC_CHECK(inputs && targets, InvalidArgument, "next_device: null output");
    int dev = 0;
    AIC_HIP_CHECK(hipGetDevice(&dev));
    AIC_CHECK(dev_ < 0 || dev_ == dev, DeviceMismatch, "DataLoader: batches go to the device of the first call");
    dev_ = dev;
    const int64_t S = ds_->seq_len();
    // staging: the sample starts (resident) or both windows (streaming), double-buffered
    const size_t need = resident_ ? static_cast<size_t>(batch_) : static_cast<size_t>(2 * batch_ * S);
    if (pinned_elems_ < need) {
        for (int i = 0; i < 2; ++i) {
            if (done_[i]) AIC_HIP_CHECK(hipEventSynchronize(done_[i]));
            if (pinned_[i]) AIC_HIP_CHECK(hipHostFree(pinned_[i]));
            AIC_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&pinned_[i]), need * sizeof(int64_t),
                                        hipHostMallocDefault));
            if (!done_[i]) AIC_HIP_CHECK(hipEventCreateWithFlags(&done_[i], hipEventDisableTiming));
            used_[i] = false;
        }
        pinned_elems_ = need;
    }
    if (resident_ && !dev_tokens_ && ds_->total_tokens() > 0) {
        const size_t bytes = sizeof(int64_t) * static_cast<size_t>(ds_->total_tokens());
        AIC_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&dev_tokens_), bytes));
        AIC_HIP_CHECK(hipMemcpy(dev_tokens_, ds_->tokens(), bytes, hipMemcpyHostToDevice));
    }
    std::vector<int64_t> samples;
    const int64_t b = take(samples);
    const int k = slot_;
    slot_ ^= 1;
    if (used_[k]) AIC_HIP_CHECK(hipEventSynchronize(done_[k]));  // its previous copy has finished
    int64_t* host = pinned_[k];
    if (resident_) {
        for (int64_t i = 0; i < b; ++i) host[i] = samples[static_cast<size_t>(i)] * ds_->stride();
        int64_t* starts = static_cast<int64_t*>(stream_scratch(sizeof(int64_t) * static_cast<size_t>(batch_), s, 6));
        AIC_HIP_CHECK(hipMemcpyAsync(starts, host, sizeof(int64_t) * static_cast<size_t>(b), hipMemcpyHostToDevice, s));
        hipLaunchKernelGGL(gather_windows_k, dim3(static_cast<unsigned>(b)), dim3(256), 0, s, dev_tokens_, starts, S,
                           inputs, targets);
        AIC_LAUNCH_CHECK("gather_windows");
    } else {
        for (int64_t i = 0; i < b; ++i)
            ds_->get_item(samples[static_cast<size_t>(i)], host + i * S, host + (b + i) * S);
        const size_t bytes = sizeof(int64_t) * static_cast<size_t>(b * S);
        AIC_HIP_CHECK(hipMemcpyAsync(inputs, host, bytes, hipMemcpyHostToDevice, s));
        AIC_HIP_CHECK(hipMemcpyAsync(targets, host + b * S, bytes, hipMemcpyHostToDevice, s));
    }
    AIC_HIP_CHECK(hipEventRecord(done_[k], s));
    used_[k] = true;
    return b;
}

}  // namespace aic::data
