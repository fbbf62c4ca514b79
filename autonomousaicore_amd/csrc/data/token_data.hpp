// Token data for the training step: BinaryTokenDataset and DataLoader of the reference
// (include/data/dataset.hpp, include/data/dataloader.hpp; src/data/dataset.cpp:155-219,
// src/data/dataloader.cpp:12-78), feeding device buffers.
//
// Same samples and order as the reference: sample i is the window tokens[i*stride, +seq_len]
// with targets shifted by one token; num_samples = (total - 1 - seq_len) / stride + 1; the
// loader shuffles its index list with std::shuffle and a std::mt19937_64(seed) at
// construction and at every reset(), so epoch e sees the e-th successive shuffle.
//
// On the device side a batch is produced two ways:
//   * resident: the whole token array is copied to HBM once (a 1 B-token corpus is 8 GB of
//     the 288 GB), and each batch is one gather kernel over the B window starts -- no
//     per-step host work beyond B start offsets;
//   * streaming: the host assembles the batch into one of two pinned staging buffers and
//     copies it asynchronously on the caller's stream; a buffer is reused only after the
//     event recorded behind its previous copy has completed.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <memory>
#include <random>
#include <string>
#include <vector>

namespace aic::data {

// A sequence of int64 tokens cut into training windows: window i starts at token i * stride
// and holds seq_len inputs followed by their next tokens as targets, so it spans seq_len + 1
// tokens.  The tokens live in memory or in a read-only mapping of a raw little-endian int64
// file; the storage is shared (the loader's resident copy reads it once).
class TokenDataset {
public:
    TokenDataset(const std::string& path, int64_t seq_len, int64_t stride);  // mapped file
    TokenDataset(std::vector<int64_t> tokens, int64_t seq_len, int64_t stride);

    int64_t size() const { return windows_; }
    int64_t seq_len() const { return seq_len_; }
    int64_t stride() const { return stride_; }
    int64_t total_tokens() const { return count_; }
    const int64_t* tokens() const { return data_.get(); }
    // first token of window idx (checked)
    int64_t window_start(int64_t idx) const;
    // input / target windows of sample idx (host, seq_len each; either may be null)
    void get_item(int64_t idx, int64_t* input, int64_t* target) const;
    int64_t token_at(int64_t i) const;
    static void write_binary_file(const std::string& path, const int64_t* tokens, int64_t n);

private:
    void set_geometry(int64_t seq_len, int64_t stride);
    std::shared_ptr<const int64_t> data_;  // releases the mapping or the vector
    int64_t count_ = 0, seq_len_ = 0, stride_ = 0, windows_ = 0;
};

// Batches of windows in epoch order: the identity, or a permutation drawn by std::shuffle from
// one std::mt19937_64(seed) that keeps running across epochs (a new draw at construction and at
// every reset()).  Batch k holds positions [k * batch_size, (k + 1) * batch_size) of the order;
// a short last batch is kept unless drop_last.
class TokenLoader {
public:
    TokenLoader(std::shared_ptr<TokenDataset> ds, int64_t batch_size, bool shuffle, bool drop_last, uint64_t seed,
                bool resident);
    ~TokenLoader();
    TokenLoader(const TokenLoader&) = delete;
    TokenLoader& operator=(const TokenLoader&) = delete;

    int64_t num_batches() const { return batches_; }
    int64_t batch_size() const { return batch_; }
    bool has_next() const { return next_ < batches_; }
    void reset();
    // Sample indices of the next batch (advances); returns the batch's size.
    int64_t take(std::vector<int64_t>& samples);
    // The next batch on the host ([b, seq_len] each).
    int64_t next_host(int64_t* inputs, int64_t* targets);
    // The next batch into device buffers ([b, seq_len] int64 each), ordered on stream s.
    int64_t next_device(int64_t* inputs, int64_t* targets, hipStream_t s);

private:
    void ensure_staging(size_t elems);
    std::shared_ptr<TokenDataset> ds_;
    int64_t batch_, batches_ = 0, next_ = 0;
    bool shuffle_, resident_;
    std::vector<int64_t> order_;
    std::mt19937_64 engine_;
    int dev_ = -1;
    int64_t* dev_tokens_ = nullptr;  // resident copy
    struct Staging {
        int64_t* host = nullptr;  // pinned
        hipEvent_t copied = nullptr;
        bool in_flight = false;
    } stage_[2];
    int turn_ = 0;
    size_t stage_elems_ = 0;
};

}  // namespace aic::data
