// Stream-ordered device memory: hipMallocAsync / hipFreeAsync on each device's default
// memory pool, with the pool's release threshold raised to "never" so that freed blocks stay
// cached for reuse instead of going back to the driver.
//
// Replaces the reference's DeviceMemoryPool (include/memory/memory_pool.hpp:90-155,
// src/memory/memory_pool.cpp:174-312), which keeps a best-fit free list of cudaMalloc
// blocks guarded by events.  Here the HIP runtime's stream-ordered allocator provides the
// caching and the cross-stream ordering; this layer adds the configuration, statistics and
// the error policy.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace aic {

struct MemoryStats {
    int64_t allocated_bytes = 0;  // live bytes handed out through the pool
    int64_t peak_bytes = 0;       // high-water mark of allocated_bytes
    int64_t num_allocs = 0;
    int64_t num_frees = 0;
};

// Allocates `bytes` on the current device, ordered on `stream`.  Throws aic::Error
// (OutOfMemory / HipError) on failure.  bytes == 0 returns nullptr.
void* pool_alloc(size_t bytes, hipStream_t stream);
// Frees a pointer from pool_alloc, ordered on `stream`.  nullptr is a no-op.
void pool_free(void* ptr, hipStream_t stream);
MemoryStats pool_stats();

// RAII device buffer from the pool.
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    DeviceBuffer(size_t bytes, hipStream_t s) : ptr_(pool_alloc(bytes, s)), bytes_(bytes), stream_(s) {}
    ~DeviceBuffer() { reset(); }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&& o) noexcept : ptr_(o.ptr_), bytes_(o.bytes_), stream_(o.stream_) { o.ptr_ = nullptr; }
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
        if (this != &o) {
            reset();
            ptr_ = o.ptr_;
            bytes_ = o.bytes_;
            stream_ = o.stream_;
            o.ptr_ = nullptr;
        }
        return *this;
    }
    void reset() noexcept;
    void* get() const { return ptr_; }
    template <typename T>
    T* as() const { return static_cast<T*>(ptr_); }
    size_t bytes() const { return bytes_; }

private:
    void* ptr_ = nullptr;
    size_t bytes_ = 0;
    hipStream_t stream_ = nullptr;
};

// Scratch memory owned by the library, one growing buffer per (device, stream, slot): work
// on one stream runs in order, so a kernel's scratch can be reused by the next call on the
// same stream without a free and a new allocation (each of which costs a few microseconds of
// stream time).  The pointer stays valid until the next call with the same key asks for more
// bytes; callers use it only for the duration of their own launches.  Slots let one call hold
// several buffers at once.
void* stream_scratch(size_t bytes, hipStream_t stream, int slot = 0);
// Returns every scratch buffer cached for `stream` to the pool (stream-ordered on it); called
// before the stream is destroyed, so that the buffers do not outlive it and a later stream at
// the same handle address does not inherit them.
void stream_scratch_release(hipStream_t stream);

}  // namespace aic
