// device.cpp — HIP device, stream and caching buffer pool (see device.h).
#include "device.h"

#include "gn_bwd.h"

#include <cstring>

namespace grilly {

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess)
        throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

Device::Device(int index) : index_(index) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
        throw std::runtime_error("grilly_core.Device: no HIP device is visible");
    if (index < 0 || index >= n) throw std::runtime_error("grilly_core.Device: bad device index");
    hip_check(hipSetDevice(index), "hipSetDevice");
    hipDeviceProp_t prop;
    hip_check(hipGetDeviceProperties(&prop, index), "hipGetDeviceProperties");
    name_ = std::string(prop.name) + " (" + prop.gcnArchName + ")";
    // default-priority stream (work on streams of different priorities is avoided)
    hip_check(hipStreamCreateWithFlags(&own_stream_, hipStreamNonBlocking), "hipStreamCreate");
    stream_ = own_stream_;
}

Device::~Device() {
    hipSetDevice(index_);
    hipStreamSynchronize(stream_);
    std::lock_guard<std::mutex> g(mu_);
    for (auto& kv : free_) hipFree(reinterpret_cast<void*>(kv.second));
    for (auto& kv : live_) hipFree(reinterpret_cast<void*>(kv.first));
    if (own_stream_) hipStreamDestroy(own_stream_);
}

void Device::use_stream(uint64_t handle) { stream_ = reinterpret_cast<hipStream_t>(handle); }

void Device::use_own_stream() { stream_ = own_stream_; }

size_t Device::bucket(size_t bytes) {
    size_t b = 256;
    while (b < bytes) b <<= 1;
    return b;
}

uint64_t Device::acquire(size_t bytes) {
    const size_t b = bucket(bytes ? bytes : 1);
    std::lock_guard<std::mutex> g(mu_);
    auto it = free_.find(b);
    uint64_t id;
    if (it != free_.end()) {
        id = it->second;
        free_.erase(it);
        stats_.bytes_cached -= b;
        stats_.reuses++;
    } else {
        void* p = nullptr;
        hipError_t e = hipMalloc(&p, b);
        if (e != hipSuccess) {
            // clear the failed call's sticky error so the next launch check does not report
            // it, then give cached blocks back and retry once
            (void)hipGetLastError();
            for (auto& kv : free_) hipFree(reinterpret_cast<void*>(kv.second));
            free_.clear();
            stats_.bytes_cached = 0;
            hip_check(hipMalloc(&p, b), "hipMalloc");
        }
        id = reinterpret_cast<uint64_t>(p);
        stats_.allocs++;
    }
    live_[id] = b;
    stats_.bytes_live += b;
    if (pin_sink_) {
        pin_sink_->push_back(id);
        pinned_[id] = false;
    }
    return id;
}

void Device::release(uint64_t id) {
    std::lock_guard<std::mutex> g(mu_);
    auto p = pinned_.find(id);
    if (p != pinned_.end()) {
        if (p->second) throw std::runtime_error("Device.release: buffer released twice");
        p->second = true;  // back to the pool at unpin()
        return;
    }
    release_locked(id);
}

void Device::pin_acquisitions(std::vector<uint64_t>* sink) {
    std::lock_guard<std::mutex> g(mu_);
    pin_sink_ = sink;
}

void Device::unpin(const std::vector<uint64_t>& ids) {
    std::lock_guard<std::mutex> g(mu_);
    for (uint64_t id : ids) {
        auto p = pinned_.find(id);
        if (p == pinned_.end()) continue;
        const bool released = p->second;
        pinned_.erase(p);
        if (released) release_locked(id);
    }
}

void Device::release_locked(uint64_t id) {
    auto it = live_.find(id);
    if (it == live_.end()) throw std::runtime_error("Device.release: unknown buffer id");
    free_.emplace(it->second, id);
    stats_.bytes_live -= it->second;
    stats_.bytes_cached += it->second;
    live_.erase(it);
}

size_t Device::buffer_bytes(uint64_t id) const {
    std::lock_guard<std::mutex> g(mu_);
    auto it = live_.find(id);
    return it == live_.end() ? 0 : it->second;
}

void Device::upload(uint64_t id, const void* host, size_t bytes, size_t offset) {
    hip_check(hipMemcpyAsync(reinterpret_cast<char*>(id) + offset, host, bytes,
                             hipMemcpyHostToDevice, stream_), "upload");
    hip_check(hipStreamSynchronize(stream_), "upload sync");
}

void Device::download(uint64_t id, void* host, size_t bytes, size_t offset) {
    hip_check(hipMemcpyAsync(host, reinterpret_cast<const char*>(id) + offset, bytes,
                             hipMemcpyDeviceToHost, stream_), "download");
    hip_check(hipStreamSynchronize(stream_), "download sync");
}

void Device::zero(uint64_t id, size_t bytes) {
    // a fill kernel, not hipMemsetAsync: the stream may be under HIP graph capture
    if (gn_zero(reinterpret_cast<void*>(id), (int64_t)bytes, stream_) != GN_OK)
        throw std::runtime_error(std::string("Device.zero: ") + gn_last_error());
}

void Device::synchronize() { hip_check(hipStreamSynchronize(stream_), "synchronize"); }

Device::Stats Device::stats() const {
    std::lock_guard<std::mutex> g(mu_);
    return stats_;
}

void Device::trim() {
    synchronize();
    std::lock_guard<std::mutex> g(mu_);
    for (auto& kv : free_) hipFree(reinterpret_cast<void*>(kv.second));
    free_.clear();
    stats_.bytes_cached = 0;
}

}  // namespace grilly
