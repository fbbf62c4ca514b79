#include "memory_pool.hpp"

#include <atomic>
#include <map>
#include <tuple>
#include <cstdint>
#include <mutex>
#include <unordered_map>

#include "error.hpp"

namespace aic {

namespace {

std::mutex g_mu;
std::unordered_map<void*, size_t> g_live;  // pointer -> bytes, for the statistics
MemoryStats g_stats;
bool g_configured[64] = {};

void configure_device_pool() {
    int dev = 0;
    AIC_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64 || g_configured[dev]) return;
    hipMemPool_t pool;
    AIC_HIP_CHECK(hipDeviceGetDefaultMemPool(&pool, dev));
    uint64_t threshold = UINT64_MAX;
    AIC_HIP_CHECK(hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &threshold));
    g_configured[dev] = true;
}

}  // namespace

void* pool_alloc(size_t bytes, hipStream_t stream) {
    if (bytes == 0) return nullptr;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        configure_device_pool();
    }
    void* p = nullptr;
    hipError_t st = hipMallocAsync(&p, bytes, stream);
    if (st == hipErrorOutOfMemory) {
        (void)hipGetLastError();
        AIC_THROW(OutOfMemory, "device pool: cannot allocate ", bytes, " bytes");
    }
    AIC_HIP_CHECK(st);
    std::lock_guard<std::mutex> lk(g_mu);
    g_live[p] = bytes;
    g_stats.allocated_bytes += static_cast<int64_t>(bytes);
    g_stats.num_allocs += 1;
    if (g_stats.allocated_bytes > g_stats.peak_bytes) g_stats.peak_bytes = g_stats.allocated_bytes;
    return p;
}

void pool_free(void* ptr, hipStream_t stream) {
    if (!ptr) return;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_live.find(ptr);
        AIC_CHECK(it != g_live.end(), InvalidArgument, "pool_free of a pointer the pool did not allocate");
        g_stats.allocated_bytes -= static_cast<int64_t>(it->second);
        g_stats.num_frees += 1;
        g_live.erase(it);
    }
    AIC_HIP_CHECK(hipFreeAsync(ptr, stream));
}

MemoryStats pool_stats() {
    std::lock_guard<std::mutex> lk(g_mu);
    return g_stats;
}

namespace {
struct ScratchEntry {
    void* ptr = nullptr;
    size_t bytes = 0;
};
std::mutex scratch_mu;
std::map<std::tuple<int, hipStream_t, int>, ScratchEntry>& scratch_cache() {
    static std::map<std::tuple<int, hipStream_t, int>, ScratchEntry> cache;
    return cache;
}
}  // namespace

void stream_scratch_release(hipStream_t stream) {
    std::lock_guard<std::mutex> lk(scratch_mu);
    auto& cache = scratch_cache();
    for (auto it = cache.begin(); it != cache.end();) {
        if (std::get<1>(it->first) == stream) {
            if (it->second.ptr) pool_free(it->second.ptr, stream);
            it = cache.erase(it);
        } else {
            ++it;
        }
    }
}

void* stream_scratch(size_t bytes, hipStream_t stream, int slot) {
    auto& cache = scratch_cache();
    auto& mu = scratch_mu;
    using Entry = ScratchEntry;
    if (bytes == 0) return nullptr;
    int dev = 0;
    AIC_HIP_CHECK(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(mu);
    Entry& e = cache[std::make_tuple(dev, stream, slot)];
    if (e.bytes < bytes) {
        if (e.ptr) pool_free(e.ptr, stream);  // stream-ordered: earlier launches finish first
        e.ptr = nullptr;
        e.bytes = 0;
        const size_t grow = bytes + bytes / 4;  // headroom so slowly growing sizes do not churn
        e.ptr = pool_alloc(grow, stream);
        e.bytes = grow;
    }
    return e.ptr;
}

void DeviceBuffer::reset() noexcept {
    if (ptr_) {
        try {
            pool_free(ptr_, stream_);
        } catch (...) {
        }
        ptr_ = nullptr;
    }
}

}  // namespace aic
