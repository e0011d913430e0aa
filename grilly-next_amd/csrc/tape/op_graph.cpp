// op_graph.cpp — HIP graph capture and replay of recorded launches (see op_graph.h).
#include "op_graph.h"

#include <stdexcept>
#include <string>

namespace grilly {

namespace {

void count_nodes(hipGraph_t g, OpGraph::NodeCounts& c) {
    size_t n = 0;
    hip_check(hipGraphGetNodes(g, nullptr, &n), "OpGraph: hipGraphGetNodes");
    if (n == 0) return;
    std::vector<hipGraphNode_t> nodes(n);
    hip_check(hipGraphGetNodes(g, nodes.data(), &n), "OpGraph: hipGraphGetNodes");
    for (size_t i = 0; i < n; ++i) {
        hipGraphNodeType t;
        hip_check(hipGraphNodeGetType(nodes[i], &t), "OpGraph: hipGraphNodeGetType");
        if (t == hipGraphNodeTypeKernel) {
            c.kernel++;
        } else if (t == hipGraphNodeTypeMemcpy) {
            c.memcpy++;
        } else if (t == hipGraphNodeTypeMemset) {
            c.memset++;
        } else if (t == hipGraphNodeTypeGraph) {
            hipGraph_t child = nullptr;
            hip_check(hipGraphChildGraphNodeGetGraph(nodes[i], &child), "OpGraph: child graph");
            count_nodes(child, c);
        } else {
            c.other++;  // empty nodes of a capture that forked and joined, events
        }
    }
}

}  // namespace

OpGraph::~OpGraph() {
    try {
        clear();
    } catch (...) {
    }
}

void OpGraph::check_device(const Device& dev, const char* what) const {
    if (dev_ && dev_ != &dev)
        throw std::invalid_argument(std::string("OpGraph.") + what +
                                    ": the graph was recorded on another device");
}

void OpGraph::begin_capture(Device& dev) {
    if (capturing_) throw std::runtime_error("OpGraph.begin_capture: a capture is already open");
    check_device(dev, "begin_capture");
    dev_ = &dev;
    if (!cap_stream_)
        hip_check(hipStreamCreateWithFlags(&cap_stream_, hipStreamNonBlocking),
                  "OpGraph: capture stream");
    // a new segment changes the graph: the executable one is rebuilt at the next optimize()
    if (exec_) {
        hip_check(hipGraphExecDestroy(exec_), "OpGraph: hipGraphExecDestroy");
        exec_ = nullptr;
    }
    if (whole_) {
        hip_check(hipGraphDestroy(whole_), "OpGraph: hipGraphDestroy");
        whole_ = nullptr;
    }
    // relaxed: a pool miss may still call hipMalloc while the capture is open
    hip_check(hipStreamBeginCapture(cap_stream_, hipStreamCaptureModeRelaxed),
              "OpGraph: hipStreamBeginCapture");
    prev_stream_ = dev.stream();
    dev.use_stream(reinterpret_cast<uint64_t>(cap_stream_));
    pin_mark_ = pinned_.size();
    dev.pin_acquisitions(&pinned_);
    capturing_ = true;
}

void OpGraph::end_capture() {
    if (!capturing_) throw std::runtime_error("OpGraph.end_capture: no capture is open");
    dev_->pin_acquisitions(nullptr);
    dev_->use_stream(reinterpret_cast<uint64_t>(prev_stream_));
    capturing_ = false;
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(cap_stream_, &g);
    if (e != hipSuccess || !g) {
        if (g) hipGraphDestroy(g);
        release_segment_pins();
        hip_check(e == hipSuccess ? hipErrorUnknown : e, "OpGraph: hipStreamEndCapture");
    }
    segments_.push_back(g);
}

void OpGraph::abort_capture() noexcept {
    if (!capturing_) return;
    dev_->pin_acquisitions(nullptr);
    dev_->use_stream(reinterpret_cast<uint64_t>(prev_stream_));
    capturing_ = false;
    hipGraph_t g = nullptr;
    if (hipStreamEndCapture(cap_stream_, &g) == hipSuccess && g) hipGraphDestroy(g);
    (void)hipGetLastError();
    release_segment_pins();
}

// the buffers acquired by a segment that was not kept go back to their owners' control
void OpGraph::release_segment_pins() noexcept {
    if (pin_mark_ >= pinned_.size()) return;
    std::vector<uint64_t> mine(pinned_.begin() + (std::ptrdiff_t)pin_mark_, pinned_.end());
    pinned_.resize(pin_mark_);
    try {
        dev_->unpin(mine);
    } catch (...) {
    }
}

void OpGraph::capture_backward(autograd::TapeContext& tape, autograd::Node* loss_node,
                               uint64_t grad_output_buffer) {
    begin_capture(tape.device());
    try {
        tape.backward(loss_node, grad_output_buffer);
    } catch (...) {
        abort_capture();
        throw;
    }
    end_capture();
    for (const auto& kv : tape.grads()) grads_[kv.first] = kv.second;
}

OpGraph::NodeCounts OpGraph::node_counts() const {
    NodeCounts c;
    for (hipGraph_t g : segments_) count_nodes(g, c);
    return c;
}

size_t OpGraph::size() const { return node_counts().kernel; }

FusionStats OpGraph::optimize(Device& dev) {
    check_device(dev, "optimize");
    if (capturing_) throw std::runtime_error("OpGraph.optimize: end the capture first");
    FusionStats st;
    if (segments_.empty()) return st;
    if (!exec_) {
        hipGraph_t g = segments_[0];
        if (segments_.size() > 1) {
            hip_check(hipGraphCreate(&whole_, 0), "OpGraph: hipGraphCreate");
            hipGraphNode_t prev = nullptr;
            for (hipGraph_t s : segments_) {
                hipGraphNode_t node = nullptr;
                hip_check(hipGraphAddChildGraphNode(&node, whole_, prev ? &prev : nullptr,
                                                    prev ? 1 : 0, s),
                          "OpGraph: hipGraphAddChildGraphNode");
                prev = node;
            }
            g = whole_;
        }
        hip_check(hipGraphInstantiateWithFlags(&exec_, g, 0), "OpGraph: hipGraphInstantiate");
    }
    const uint32_t n = (uint32_t)size();
    st.originalOps = n;
    st.optimizedOps = n;
    return st;
}

void OpGraph::execute(Device& dev) {
    check_device(dev, "execute");
    if (capturing_) throw std::runtime_error("OpGraph.execute: end the capture first");
    if (segments_.empty()) return;
    if (!exec_) optimize(dev);
    last_stream_ = dev.stream();
    hip_check(hipGraphLaunch(exec_, last_stream_), "OpGraph: hipGraphLaunch");
    replays_++;
}

uint64_t OpGraph::get_grad_buffer(uint64_t id) const {
    auto it = grads_.find(id);
    return it == grads_.end() ? 0ULL : it->second;
}

void OpGraph::clear() {
    abort_capture();
    // a replay may still be running: its buffers go back to the pool only after it ends
    if (replays_ && dev_) hip_check(hipStreamSynchronize(last_stream_), "OpGraph: synchronize");
    if (exec_) hipGraphExecDestroy(exec_);
    exec_ = nullptr;
    if (whole_) hipGraphDestroy(whole_);
    whole_ = nullptr;
    for (hipGraph_t g : segments_) hipGraphDestroy(g);
    segments_.clear();
    if (dev_ && !pinned_.empty()) dev_->unpin(pinned_);
    pinned_.clear();
    pin_mark_ = 0;
    grads_.clear();
    if (cap_stream_) hipStreamDestroy(cap_stream_);
    cap_stream_ = nullptr;
    dev_ = nullptr;
    replays_ = 0;
    last_stream_ = nullptr;
}

}  // namespace grilly
