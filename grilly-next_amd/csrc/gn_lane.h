// gn_lane.h — a second stream per device for the products of one backward call that do not
// depend on each other (a Linear's weight gradient beside its input gradient).  The call forks
// the side stream off the caller's stream with an event and joins it back with another before
// it returns, so to the caller the call stays one stream-ordered operation; under HIP graph
// capture the fork and the join become the graph's edges.  The side stream has the default
// priority and does not synchronise with the null stream (the events order it).
#pragma once

#include <mutex>

#include "gn_common.h"

namespace gn {

// When a call forks: never, only while the caller's stream is being captured into a graph
// (the fork and join are then paid once, at capture), or always.
enum class Fork { kNever, kCaptured, kAlways };

class SideBySide {
public:
    // Without a fork, or when the side stream cannot be had (created on a call outside graph
    // capture, kept for the process), side() is the caller's stream and everything runs in
    // issue order.
    SideBySide(hipStream_t s, Fork when);
    ~SideBySide() { join(); }
    SideBySide(const SideBySide&) = delete;
    SideBySide& operator=(const SideBySide&) = delete;

    hipStream_t side() const { return side_ ? side_ : s_; }
    bool forked() const { return side_ != nullptr; }
    // the caller's stream waits for the side stream's work; GN_OK or GN_E_HIP
    int join();

private:
    hipStream_t s_;
    hipStream_t side_ = nullptr;
    hipEvent_t join_ = nullptr;
    // one fork/join sequence at a time per device: the lane's stream and events are shared
    std::unique_lock<std::mutex> lock_;
};

}  // namespace gn
