// gn_lane.cpp — the per-device side stream of gn_lane.h.
#include "gn_lane.h"

namespace gn {
namespace {

struct Lane {
    std::mutex mu;
    int state = 0;  // 0: not yet created, 1: ready, -1: unavailable
    hipStream_t side = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
};

constexpr int kMaxDevices = 64;
Lane g_lanes[kMaxDevices];

}  // namespace

SideBySide::SideBySide(hipStream_t s, Fork when) : s_(s) {
    if (when == Fork::kNever) return;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess) {
        (void)hipGetLastError();
        return;
    }
    const bool capturing = cs != hipStreamCaptureStatusNone;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();
        return;
    }
    // the lane belongs to the current device: a stream of another device keeps issue order
    hipDevice_t sdev = dev;
    if (hipStreamGetDevice(s, &sdev) != hipSuccess || sdev != dev) {
        (void)hipGetLastError();
        return;
    }
    Lane& L = g_lanes[dev];
    std::unique_lock<std::mutex> lk(L.mu);
    if (L.state == 0) {
        // stream and event creation are kept out of a capture in progress
        if (capturing) return;
        if (hipStreamCreateWithFlags(&L.side, hipStreamNonBlocking) == hipSuccess &&
            hipEventCreateWithFlags(&L.fork, hipEventDisableTiming) == hipSuccess &&
            hipEventCreateWithFlags(&L.join, hipEventDisableTiming) == hipSuccess) {
            L.state = 1;
        } else {
            (void)hipGetLastError();
            L.state = -1;
        }
    }
    if (L.state != 1) return;
    if (when == Fork::kCaptured && !capturing) return;  // the lane is ready for a later capture
    if (hipEventRecord(L.fork, s) != hipSuccess) {
        (void)hipGetLastError();
        return;
    }
    if (hipStreamWaitEvent(L.side, L.fork, 0) != hipSuccess) {
        (void)hipGetLastError();
        return;
    }
    side_ = L.side;
    join_ = L.join;
    lock_ = std::move(lk);
}

int SideBySide::join() {
    if (!side_) return GN_OK;
    hipStream_t side = side_;
    side_ = nullptr;
    const bool ok = hipEventRecord(join_, side) == hipSuccess &&
                    hipStreamWaitEvent(s_, join_, 0) == hipSuccess;
    if (lock_.owns_lock()) lock_.unlock();
    if (!ok) {
        (void)hipGetLastError();
        set_error("side stream join failed");
        return GN_E_HIP;
    }
    return GN_OK;
}

}  // namespace gn
