// The reference's binary checkpoint format (.aic), host side.
//
// Layout (src/train/checkpoint.cpp:30-95, docs/architecture.md:96-117), little-endian:
//   u32 magic 0x41494330 ('AIC0'), u32 version 1, i64 step, i64 epoch, f32 best_val_loss,
//   u32 desc_len, desc bytes, u64 num_tensors, then per tensor:
//   u32 name_len, name, i32 rank, i64 dims[rank], i32 dtype (the reference's DType enum:
//   0 f32, 1 f16, 2 bf16, 3 i32, 4 i64, 5 u8, 6 u16), u64 nbytes, data, u32 Adler-32 of data.
// The reader rejects a bad magic or version and any tensor whose checksum does not match
// (FormatError), as load_checkpoint does (src/train/checkpoint.cpp:108-168).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace aic {

struct CheckpointMeta {
    int64_t step = 0;
    int64_t epoch = 0;
    float best_val_loss = 0.0f;
    std::string description;
};

struct CheckpointTensor {
    std::string name;
    std::vector<int64_t> dims;
    int32_t dtype = 0;
    std::vector<uint8_t> data;
};

constexpr uint32_t kCheckpointMagic = 0x41494330u;
constexpr uint32_t kCheckpointVersion = 1;

// Adler-32 (RFC 1950): a = 1 + sum of bytes, b = sum of the a's, both mod 65521.
uint32_t adler32(const uint8_t* data, size_t len);

// Writes meta and the tensors in the given order (data pointers are host memory).
struct CheckpointTensorRef {
    std::string name;
    std::vector<int64_t> dims;
    int32_t dtype;
    const void* data;
    uint64_t nbytes;
};
void write_checkpoint(const std::string& path, const CheckpointMeta& meta, const std::vector<CheckpointTensorRef>& ts);
// Reads and verifies the whole file.
void read_checkpoint(const std::string& path, CheckpointMeta& meta, std::vector<CheckpointTensor>& ts);

// Indices of `names` in the order Module::named_parameters() visits them
// (include/nn/module.hpp:63-76): at every module level the module's own parameters first,
// sorted by name, then its submodules sorted by registered key.  Keys that contain a dot
// ("layers.3", "experts.7") are single registrations; every other dot separates levels.
std::vector<size_t> module_order(const std::vector<std::string>& names);

}  // namespace aic
