#include "token_data.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <memory>

#include "../kernels/common.hpp"
#include "../runtime/error.hpp"
#include "../runtime/memory_pool.hpp"

namespace aic::data {

// ---------------------------------------------------------------------------- dataset
namespace {

// The whole file as a private read-only mapping; the returned pointer unmaps it when the last
// owner lets go.
std::shared_ptr<const int64_t> map_tokens(const std::string& path, int64_t& count) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    AIC_CHECK(fd >= 0, IOError, "cannot open the token file ", path);
    struct stat info {};
    const bool have_size = ::fstat(fd, &info) == 0;
    const size_t bytes = have_size ? static_cast<size_t>(info.st_size) : 0;
    if (!have_size || bytes % sizeof(int64_t) != 0) {
        ::close(fd);
        AIC_CHECK(have_size, IOError, "cannot read the size of the token file ", path);
        AIC_THROW(InvalidArgument, "token file ", path, " holds ", bytes, " bytes, not a whole number of int64 tokens");
    }
    count = static_cast<int64_t>(bytes / sizeof(int64_t));
    if (bytes == 0) {
        ::close(fd);
        return std::shared_ptr<const int64_t>(new int64_t[1](), std::default_delete<int64_t[]>());
    }
    void* base = ::mmap(nullptr, bytes, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);  // the mapping keeps the file open
    AIC_CHECK(base != MAP_FAILED, IOError, "cannot map the token file ", path);
    return std::shared_ptr<const int64_t>(static_cast<const int64_t*>(base),
                                          [bytes](const int64_t* p) { ::munmap(const_cast<int64_t*>(p), bytes); });
}

}  // namespace

TokenDataset::TokenDataset(const std::string& path, int64_t seq_len, int64_t stride) {
    AIC_CHECK(seq_len > 0, InvalidArgument, "window length must be positive (got ", seq_len, ")");
    data_ = map_tokens(path, count_);
    set_geometry(seq_len, stride);
}

TokenDataset::TokenDataset(std::vector<int64_t> tokens, int64_t seq_len, int64_t stride) {
    AIC_CHECK(seq_len > 0, InvalidArgument, "window length must be positive (got ", seq_len, ")");
    auto owner = std::make_shared<std::vector<int64_t>>(std::move(tokens));
    count_ = static_cast<int64_t>(owner->size());
    data_ = std::shared_ptr<const int64_t>(owner, owner->data());  // aliases the vector's storage
    set_geometry(seq_len, stride);
}

void TokenDataset::set_geometry(int64_t seq_len, int64_t stride) {
    seq_len_ = seq_len;
    stride_ = stride > 0 ? stride : seq_len;  // non-positive stride: non-overlapping windows
    // the last window must end at or before the last token: k * stride + seq_len + 1 <= count
    windows_ = count_ > seq_len_ ? (count_ - seq_len_ - 1) / stride_ + 1 : 0;
}

int64_t TokenDataset::window_start(int64_t idx) const {
    AIC_CHECK(idx >= 0 && idx < windows_, OutOfRange, "window ", idx, " requested from a dataset of ", windows_);
    return idx * stride_;
}

void TokenDataset::get_item(int64_t idx, int64_t* input, int64_t* target) const {
    const int64_t* w = data_.get() + window_start(idx);
    const size_t bytes = sizeof(int64_t) * static_cast<size_t>(seq_len_);
    if (input) std::memcpy(input, w, bytes);
    if (target) std::memcpy(target, w + 1, bytes);
}

int64_t TokenDataset::token_at(int64_t i) const {
    AIC_CHECK(i >= 0 && i < count_, OutOfRange, "token ", i, " requested from ", count_, " tokens");
    return data_.get()[i];
}

void TokenDataset::write_binary_file(const std::string& path, const int64_t* tokens, int64_t n) {
    AIC_CHECK(n >= 0 && (n == 0 || tokens), InvalidArgument, "write_binary_file: bad token array");
    std::unique_ptr<std::FILE, int (*)(std::FILE*)> f(std::fopen(path.c_str(), "wb"), &std::fclose);
    AIC_CHECK(f != nullptr, IOError, "cannot create the token file ", path);
    const size_t written = n > 0 ? std::fwrite(tokens, sizeof(int64_t), static_cast<size_t>(n), f.get()) : 0;
    AIC_CHECK(written == static_cast<size_t>(n) && std::fclose(f.release()) == 0, IOError,
              "short write to the token file ", path);
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
    : ds_(std::move(ds)), batch_(batch_size), shuffle_(shuffle), resident_(resident), engine_(seed) {
    AIC_CHECK(ds_, InvalidArgument, "a loader needs a dataset");
    AIC_CHECK(batch_ > 0, InvalidArgument, "batch size must be positive (got ", batch_, ")");
    const int64_t n = ds_->size();
    order_.resize(static_cast<size_t>(n));
    for (int64_t i = 0; i < n; ++i) order_[static_cast<size_t>(i)] = i;
    batches_ = n / batch_ + ((!drop_last && n % batch_ != 0) ? 1 : 0);
    reset();
}

TokenLoader::~TokenLoader() {
    for (Staging& st : stage_) {
        if (st.copied) {
            (void)hipEventSynchronize(st.copied);
            (void)hipEventDestroy(st.copied);
        }
        if (st.host) (void)hipHostFree(st.host);
    }
    if (dev_tokens_) (void)hipFree(dev_tokens_);
}

void TokenLoader::reset() {
    next_ = 0;
    // the next permutation of the same engine: epoch e is the e-th draw
    if (shuffle_) std::shuffle(order_.begin(), order_.end(), engine_);
}

int64_t TokenLoader::take(std::vector<int64_t>& samples) {
    AIC_CHECK(has_next(), OutOfRange, "the epoch's ", batches_, " batches are used up; reset() starts the next epoch");
    const size_t first = static_cast<size_t>(next_ * batch_);
    const size_t last = std::min(first + static_cast<size_t>(batch_), order_.size());
    samples.assign(order_.begin() + static_cast<std::ptrdiff_t>(first),
                   order_.begin() + static_cast<std::ptrdiff_t>(last));
    ++next_;
    return static_cast<int64_t>(last - first);
}

int64_t TokenLoader::next_host(int64_t* inputs, int64_t* targets) {
    std::vector<int64_t> samples;
    const int64_t b = take(samples);
    const int64_t S = ds_->seq_len();
    for (int64_t i = 0; i < b; ++i) ds_->get_item(samples[static_cast<size_t>(i)], inputs + i * S, targets + i * S);
    return b;
}

void TokenLoader::ensure_staging(size_t elems) {
    if (stage_elems_ >= elems) return;
    for (Staging& st : stage_) {
        if (st.copied) AIC_HIP_CHECK(hipEventSynchronize(st.copied));
        if (st.host) AIC_HIP_CHECK(hipHostFree(st.host));
        st.host = nullptr;
        AIC_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&st.host), elems * sizeof(int64_t), hipHostMallocDefault));
        if (!st.copied) AIC_HIP_CHECK(hipEventCreateWithFlags(&st.copied, hipEventDisableTiming));
        st.in_flight = false;
    }
    stage_elems_ = elems;
}

int64_t TokenLoader::next_device(int64_t* inputs, int64_t* targets, hipStream_t s) {
    AIC_CHECK(inputs && targets, InvalidArgument, "next_device: null output");
    int dev = 0;
    AIC_HIP_CHECK(hipGetDevice(&dev));
    AIC_CHECK(dev_ < 0 || dev_ == dev, DeviceMismatch, "a loader feeds the device of its first next_device call");
    dev_ = dev;
    const int64_t S = ds_->seq_len();
    // staging: the window starts (resident) or both windows (streaming), double-buffered
    ensure_staging(resident_ ? static_cast<size_t>(batch_) : static_cast<size_t>(2 * batch_ * S));
    if (resident_ && !dev_tokens_ && ds_->total_tokens() > 0) {
        const size_t bytes = sizeof(int64_t) * static_cast<size_t>(ds_->total_tokens());
        AIC_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&dev_tokens_), bytes));
        AIC_HIP_CHECK(hipMemcpy(dev_tokens_, ds_->tokens(), bytes, hipMemcpyHostToDevice));
    }
    std::vector<int64_t> samples;
    const int64_t b = take(samples);
    Staging& st = stage_[turn_];
    turn_ ^= 1;
    if (st.in_flight) AIC_HIP_CHECK(hipEventSynchronize(st.copied));  // its previous copy has finished
    if (resident_) {
        for (int64_t i = 0; i < b; ++i) st.host[i] = ds_->window_start(samples[static_cast<size_t>(i)]);
        int64_t* starts = static_cast<int64_t*>(stream_scratch(sizeof(int64_t) * static_cast<size_t>(batch_), s, 6));
        AIC_HIP_CHECK(hipMemcpyAsync(starts, st.host, sizeof(int64_t) * static_cast<size_t>(b), hipMemcpyHostToDevice,
                                     s));
        hipLaunchKernelGGL(gather_windows_k, dim3(static_cast<unsigned>(b)), dim3(256), 0, s, dev_tokens_, starts, S,
                           inputs, targets);
        AIC_LAUNCH_CHECK("gather_windows");
    } else {
        for (int64_t i = 0; i < b; ++i)
            ds_->get_item(samples[static_cast<size_t>(i)], st.host + i * S, st.host + (b + i) * S);
        const size_t bytes = sizeof(int64_t) * static_cast<size_t>(b * S);
        AIC_HIP_CHECK(hipMemcpyAsync(inputs, st.host, bytes, hipMemcpyHostToDevice, s));
        AIC_HIP_CHECK(hipMemcpyAsync(targets, st.host + b * S, bytes, hipMemcpyHostToDevice, s));
    }
    AIC_HIP_CHECK(hipEventRecord(st.copied, s));
    st.in_flight = true;
    return b;
}

}  // namespace aic::data
