// device.h — HIP device, stream and caching buffer pool under the tape engine.
//
// Replaces the reference's Vulkan runtime (GrillyDevice, BufferPool, CommandBatch:
// cpp/include/grilly/{device,buffer_pool,command_batch}.h).  A buffer id is the device
// pointer cast to uint64 (the reference uses the VkBuffer handle, autograd.cpp:228-233),
// so any device pointer — including a torch tensor's data_ptr() — is a valid buffer id.
// Freed buffers go back to power-of-two size buckets (buffer_pool.h:99-101 uses the same
// bucketing) and are reused without another hipMalloc.  All work is ordered on one
// stream; nothing here synchronises except download() and synchronize().
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

namespace grilly {

// hipError_t -> std::runtime_error (the role of vkCheck, command_batch.cpp:9-14)
void hip_check(hipError_t e, const char* what);

class Device {
public:
    explicit Device(int index = 0);
    ~Device();
    Device(const Device&) = delete;
    Device& operator=(const Device&) = delete;

    int index() const { return index_; }
    std::string name() const { return name_; }
    hipStream_t stream() const { return stream_; }
    // Launch on a caller-owned stream (e.g. torch.cuda.current_stream().cuda_stream).
    // 0 is the null (default) stream, which is what torch reports for its default stream.
    void use_stream(uint64_t handle);
    // Back to the device's own (non-blocking) stream.
    void use_own_stream();

    uint64_t acquire(size_t bytes);  // from the pool; contents undefined
    void release(uint64_t id);       // back to the pool
    size_t buffer_bytes(uint64_t id) const;

    void upload(uint64_t id, const void* host, size_t bytes, size_t offset = 0);
    void download(uint64_t id, void* host, size_t bytes, size_t offset = 0);
    void zero(uint64_t id, size_t bytes);  // fill kernel, stream-ordered
    void synchronize();

    // HIP graph capture (OpGraph): while a sink is set, every buffer acquire() hands out is
    // appended to it and pinned.  release() of a pinned buffer is deferred until unpin(), so
    // memory a captured graph reads or writes is not handed out again while the graph can
    // still be replayed.
    void pin_acquisitions(std::vector<uint64_t>* sink);  // nullptr: stop pinning
    void unpin(const std::vector<uint64_t>& ids);

    struct Stats {
        size_t bytes_live = 0, bytes_cached = 0;
        uint64_t allocs = 0, reuses = 0;
    };
    Stats stats() const;
    void trim();  // return cached blocks to HIP

private:
    static size_t bucket(size_t bytes);
    int index_ = 0;
    std::string name_;
    hipStream_t own_stream_ = nullptr;
    hipStream_t stream_ = nullptr;
    mutable std::mutex mu_;
    std::unordered_map<uint64_t, size_t> live_;            // id -> bucket bytes
    std::multimap<size_t, uint64_t> free_;                 // bucket bytes -> id
    std::vector<uint64_t>* pin_sink_ = nullptr;
    std::unordered_map<uint64_t, bool> pinned_;            // id -> released by its owner
    void release_locked(uint64_t id);
    Stats stats_;
};

}  // namespace grilly
