// op_graph.h — recorded dispatches replayed as one HIP graph launch.
//
// Replaces the reference's OpGraph (cpp/include/grilly/op_graph.h:84-133,
// cpp/src/op_graph.cpp:123-246), which records Vulkan dispatches with addOp, fuses known
// pairs, drops barriers between dispatches that share no buffer, and submits everything in
// one command buffer.  Here the dispatches are the library's kernel launches: they are
// recorded by HIP stream capture while the tape (or any other caller of the device stream)
// issues them, instantiated once, and replayed with one hipGraphLaunch, which removes the
// per-launch host cost (argument packing, the tape walk, the C-ABI checks) from every step
// after the first.  No entry point of the kernel library allocates, synchronises or calls
// hipMemsetAsync, so a capture holds kernel nodes only.
//
// Same names as the reference: size(), clear(), optimize(device) -> FusionStats,
// execute(device).  Recording differs: begin_capture(device) / end_capture() around the
// launches (one capture per segment; segments replay in order), or capture_backward(tape,
// loss, grad) for a tape's backward pass.  optimize() instantiates the executable graph;
// operator fusion is already in the kernels (bias sums in the weight-gradient GEMM, GLU
// local gradients in the projection's epilogue, norm statistics in one pass), so ops_fused
// and barriers_eliminated report 0 and original_ops == optimized_ops == kernel nodes.
//
// Replay contract (HIP graph semantics): every launch reads and writes the addresses it
// was recorded with.  Tensors the recorded work reads (activations, saved statistics,
// weights, the upstream gradient) must stay allocated at the same addresses while the
// graph is replayed; write new values into them between replays.  Buffers the device pool
// handed out during the capture (the gradients, split-K scratch) are pinned to the graph:
// they survive the tape's end() and go back to the pool at clear() or destruction.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <unordered_map>
#include <vector>

#include "autograd.h"
#include "device.h"

namespace grilly {

struct FusionStats {  // op_graph.h:59-64
    uint32_t opsFused = 0;
    uint32_t barriersEliminated = 0;
    uint32_t originalOps = 0;
    uint32_t optimizedOps = 0;
};

class OpGraph {
public:
    OpGraph() = default;
    ~OpGraph();
    OpGraph(const OpGraph&) = delete;
    OpGraph& operator=(const OpGraph&) = delete;

    // Record every launch issued on `dev` until end_capture().  The device's launches go to a
    // capture stream meanwhile; its previous stream is restored at end_capture().
    void begin_capture(Device& dev);
    void end_capture();
    // Record the backward pass of a recorded tape (TapeContext::backward under capture) and
    // keep its gradient table: get_grad_buffer() answers after the tape has ended.
    void capture_backward(autograd::TapeContext& tape, autograd::Node* loss_node,
                          uint64_t grad_output_buffer);
    bool capturing() const { return capturing_; }

    size_t size() const;  // kernel nodes recorded
    void clear();
    FusionStats optimize(Device& dev);  // instantiate (also done by the first execute)
    void execute(Device& dev);          // one hipGraphLaunch on the device's current stream
    uint64_t get_grad_buffer(uint64_t input_buffer_id) const;

    struct NodeCounts {
        size_t kernel = 0, memcpy = 0, memset = 0, other = 0;
    };
    NodeCounts node_counts() const;
    uint64_t replays() const { return replays_; }

private:
    void check_device(const Device& dev, const char* what) const;
    void abort_capture() noexcept;
    void release_segment_pins() noexcept;

    Device* dev_ = nullptr;
    hipStream_t cap_stream_ = nullptr;
    hipStream_t prev_stream_ = nullptr;
    hipStream_t last_stream_ = nullptr;  // stream of the last replay
    bool capturing_ = false;
    std::vector<hipGraph_t> segments_;
    hipGraph_t whole_ = nullptr;  // the segments chained as child graphs (2+ segments)
    hipGraphExec_t exec_ = nullptr;
    std::vector<uint64_t> pinned_;
    size_t pin_mark_ = 0;  // pinned_ entries before the open capture
    std::unordered_map<uint64_t, uint64_t> grads_;
    uint64_t replays_ = 0;
};

}  // namespace grilly
