// autograd.h — grilly-next's tape autograd engine, MI355X build.
//
// Field-for-field compatible with the reference types (cpp/include/grilly/autograd/
// autograd.h:46-455): TensorRef, OpType (same numbering), the packed parameter structs,
// Node (a fixed-size arena object, no heap), BackwardEngine and TapeContext.  The backward
// walk is the reference's Wengert-list walk (autograd.cpp:22-93); the per-op handlers call
// libgn_bwd through its C ABI (include/gn_bwd.h) and every launch is ordered on the
// device stream, with no per-dispatch synchronisation.
//
// Differences from the reference, each deliberate:
//   * fan-out gradients are summed (the reference drops the second one, autograd.cpp:78-86);
//   * the gradient table is an open-addressing hash (the reference scans linearly,
//     autograd.cpp:132-166) and overflows with an exception instead of silently;
//   * TensorRef.dtype 4 = bf16 (2 bytes) is added to 0 f32, 1 f16, 2 u32, 3 i32;
//   * RMSNorm, Softmax, ReLU, SiLU, Tanh, Sigmoid, LayerNorm, FlashAttention2 and
//     CrossEntropy have real handlers (stubs or missing in the reference,
//     autograd.cpp:543-711), and FusedGLU (appended after VSACosineBlendLoss) carries the
//     fused SwiGLU/GEGLU/ReGLU projection backward.
#pragma once

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <utility>
#include <vector>

#include "device.h"
#include "gn_bwd.h"
#include "tape_arena.h"

namespace grilly {
namespace autograd {

struct TensorRef {
    uint64_t buffer_id;  // device pointer (0 = none)
    uint32_t ndim;
    uint32_t shape[8];
    uint32_t dtype;  // 0 f32, 1 f16, 2 u32, 3 i32, 4 bf16
    bool requires_grad;

    size_t numel() const {
        size_t n = 1;
        for (uint32_t i = 0; i < ndim; ++i) n *= shape[i];
        return n;
    }
    static size_t elem_size(uint32_t dtype) { return (dtype == 1 || dtype == 4) ? 2 : 4; }
    size_t size_bytes() const { return numel() * elem_size(dtype); }
    static TensorRef none() {
        TensorRef r{};
        return r;
    }
    bool valid() const { return buffer_id != 0ULL; }
    // rows x last-dim view used by the 2-D handlers
    size_t last() const { return ndim ? shape[ndim - 1] : 1; }
    size_t rows() const { return ndim ? numel() / last() : 0; }
};

enum class OpType : uint8_t {
    Add = 0, Sub, Mul, Div, Neg, Pow,
    MatMul, Linear,
    ReLU, GELU, SiLU, Tanh, Sigmoid, Softmax,
    LayerNorm, RMSNorm,
    FlashAttention2,
    Conv2d, Conv1d,
    Sum, Mean, Max, Min,
    Reshape, Transpose, Slice,
    CrossEntropy, MSELoss,
    CubeMindSurprise,
    TemporalSurprise,
    VSAUnpackProject, VSASurrogateLoss, VSALoRAExpand, VSACosineBlendLoss,
    FusedGLU,   // added by this build: fused gate/up projection + GLU backward
    Embedding,  // added by this build: row gather (tied embeddings); backward scatter-adds
    _Count
};
static_assert(static_cast<int>(OpType::VSACosineBlendLoss) == 33, "OpType numbering");

// ---- packed parameter structs (Node::params[64]) -------------------------------------
struct TemporalSurpriseParams {  // autograd.h:151-160
    float avg_coherence, avg_contradiction, temporal_multiplier, alpha;
    uint32_t num_branches, dt;
};
struct VSASurrogateLossParams {  // autograd.h:172-184 (40 bytes; its comment says 44)
    float gamma, delta_margin, lambda;
    uint32_t K, D, winning_k, runner_up_k;
    float loss_value, temperature, diversity_lambda;
};
static_assert(sizeof(VSASurrogateLossParams) == 40, "VSASurrogateLossParams layout");
struct VSALoRAExpandParams { uint32_t K, D, rank; };
struct VSACosineBlendLossParams {
    uint32_t K, D;
    float temperature, lambda_distill, lambda_entropy, loss_value, tau_oracle;
};
// Parameter blocks for the handlers this build adds (all optional: zeros mean defaults).
struct GELUParams { uint32_t erf_form; };                     // 0 = tanh form (GLSL)
struct LayerNormParams { float eps; uint32_t stat_is_var; };  // eps default 1e-5
// RMSNorm: the saved per-row statistic (saved slot 1) is 0 = rstd, 1 = mean(x^2) as
// rms-norm.glsl:52 saves it, 2 = sqrt(mean(x^2) + eps) as snn-rmsnorm.glsl:55 saves it;
// eps (default 1e-6) is used by form 1 only.
struct RMSNormParams { float eps; uint32_t stat_kind; };
struct AttentionParams {
    float scale;        // 0 -> 1/sqrt(D)
    uint32_t causal;    // 1 = causal mask j <= i
    uint32_t rope_mode; // 0 none, 1 interleaved, 2 half
    float rope_theta;   // 0 -> 10000
    uint32_t layout;    // 0: inputs Q, K, V [B,H,S,D]; 1: inputs[0] = fused QKV [B,S,3*H*D],
                        //    output O [B,S,H*D] (the layout a fused QKV projection produces)
    uint32_t heads;     // H, for layout 1
};
struct CrossEntropyParams { float scale; uint32_t has_scale; };  // scale default 1 (no 1/B)
struct FusedGLUParams { uint32_t kind; };                       // GN_GLU_* kind
struct MSELossParams { float scale; uint32_t has_scale; };      // scale default 1/n (mean)

static constexpr uint32_t kMaxNodeIO = 8;

struct Node {
    Node* prev_in_tape;
    OpType op;
    uint32_t seq;
    uint32_t num_inputs;
    uint32_t num_outputs;
    TensorRef inputs[kMaxNodeIO];
    TensorRef outputs[kMaxNodeIO];
    uint32_t num_saved;
    uint64_t saved_buffer_ids[kMaxNodeIO];
    uint64_t grad_output_buffer;
    uint64_t grad_input_buffers[kMaxNodeIO];
    uint8_t params[64];
    uint32_t params_size;
    float emotion[2];  // CubeMind emotion state slot (autograd.h:267), unused here
};

template <typename T, typename... Args>
T* TapeArena::allocate_node(Args&&... args) {
    T* node = allocate<T>(std::forward<Args>(args)...);
    node->prev_in_tape = tail<T>();
    set_tail(node);
    return node;
}

class BackwardEngine {
public:
    explicit BackwardEngine(Device& dev);

    void backward(TapeArena& tape, Node* loss_node, uint64_t grad_output_buffer);
    uint64_t get_grad_buffer(uint64_t input_buffer_id) const;
    void clear_grads();

    struct Stats {
        uint32_t nodes_visited, nodes_with_grad, shaders_dispatched, cpu_fallbacks;
        uint32_t fanout_accumulations;
    };
    Stats last_stats() const { return stats_; }

    // A weight whose surprise-momentum step the Linear backward applies in its own pass over
    // W (gn_linear_bwd_surprise_momentum): the weight's gradient is then never stored and
    // get_grad_buffer(weight) stays 0, so an optimizer that skips gradient-less weights does
    // not apply the step twice.  Taken only when the weight is saved by exactly one Linear
    // node of the tape (its whole gradient comes from that node) and the kernel takes the
    // shape; otherwise the pass stores the gradient as usual.
    struct FusedUpdate {
        uint64_t state;  // s_bar buffer, same shape as the weight
        float eta, alpha, lambda, floor_, wd, clip;
        bool applied;    // set by the pass that applied it
    };
    void set_fused_update(uint64_t weight, const FusedUpdate& u);
    void clear_fused_updates() { fused_.clear(); }
    bool fused_update_applied(uint64_t weight) const;

    // A Linear whose input is the output of the FusedGLU node recorded right before it (the
    // FFN's down projection), with no other gradient for that output: the Linear's backward
    // writes the GLU's local gradients [dGate | dUp] in the epilogue of its input-gradient
    // GEMM (gn_ffn_down_glu_bwd_ws) and the FusedGLU node starts from them
    // (gn_glu_proj_bwd_ws).  The GLU output's own gradient is then never formed:
    // get_grad_buffer() for it stays 0.  bf16 only; off by default, so every gradient the
    // reference's engine keeps is kept unless the caller asks for the fusion.
    void set_glu_epilogue(bool on) { glu_epilogue_ = on; }
    bool glu_epilogue() const { return glu_epilogue_; }

    static constexpr size_t kGradTableSize = 8192;  // power of two

private:
    friend class TapeContext;
    struct GradEntry {
        uint64_t buffer_id;
        uint64_t grad_id;
        uint64_t grad_bytes;
        uint32_t dtype;
        bool owned;  // grad_id was allocated for this tensor alone (safe to add into)
    };

    void dispatch(Node* n);
    // record gradient `g` (dtype, numel) for tensor `id`, summing on fan-out
    void contribute(uint64_t id, uint64_t g, uint32_t dtype, size_t numel, bool owned);
    // record `g` as the gradient of the input version of an in-place tensor (overwrites)
    void replace(uint64_t id, uint64_t g, uint32_t dtype, size_t numel, bool owned);
    static bool writes_in_place(const Node* n, uint64_t id);
    GradEntry* find(uint64_t id) const;
    GradEntry* find_or_insert(uint64_t id);
    uint64_t alloc_grad(size_t bytes);
    // split-K scratch shared by the handlers of one backward pass (every launch is ordered
    // on the engine's stream, so each node may reuse it); grown on demand, 0 bytes -> 0
    uint64_t split_ws(size_t bytes);
    const void* gout(Node* n) const;
    // output buffer of a norm's input gradient, summed with the input's existing gradient
    uint64_t norm_dx(Node* n, const void** add);
    uint64_t bf16_copy_for(Node* n, uint64_t dX);
    Node* glu_before(Node* n) const;

    void bwd_linear(Node* n);
    void bwd_act(Node* n, int kind, bool uses_output);
    void bwd_softmax(Node* n);
    void bwd_layernorm(Node* n);
    void bwd_rmsnorm(Node* n);
    void bwd_attention(Node* n);
    void bwd_cross_entropy(Node* n);
    void bwd_add_sub(Node* n, bool sub);
    void bwd_passthrough(Node* n);
    void bwd_vsa_unpack_project(Node* n);
    void bwd_vsa_surrogate(Node* n);
    void bwd_fused_glu(Node* n);
    void bwd_embedding(Node* n);
    void bwd_binary(Node* n, int op);
    void bwd_reduce(Node* n, int op);
    void bwd_transpose(Node* n);
    void bwd_mse(Node* n);
    void bwd_matmul(Node* n);
    void bwd_vsa_lora_expand(Node* n);
    void bwd_vsa_cosine_blend(Node* n);
    void bwd_surprise_passthrough(Node* n);

    Device& dev_;
    Stats stats_{};
    uint32_t borrowed_ = 0;  // inputs whose gradient is the upstream buffer itself
    uint32_t handled_ = 0;   // inputs whose gradient the handler already summed into the table
    uint64_t ws_id_ = 0;     // split-K scratch of the current pass (owned by backward_bufs_)
    size_t ws_bytes_ = 0;
    std::vector<uint64_t> backward_bufs_;
    mutable std::vector<GradEntry> table_;
    uint32_t count_ = 0;
    struct FusedSlot {
        uint64_t weight;
        FusedUpdate u;
        bool eligible;  // saved by exactly one Linear node of the current tape
    };
    std::vector<FusedSlot> fused_;
    // (fp32 gradient buffer, its bf16 copy) pairs a norm backward wrote in its own pass for the
    // bf16 input of the Add visited next (bwd_layernorm, bwd_add_sub)
    std::vector<std::pair<uint64_t, uint64_t>> bf16_copies_;
    // norm backwards whose parameter gradients are still partial rows in their workspaces,
    // summed by one gn_norm_finish at the end of the pass (or before anything reads them)
    std::vector<GnNormFinish> norm_pending_;
    // set_glu_epilogue: [dGate | dUp] a Linear's backward wrote for the FusedGLU node visited
    // next (bwd_linear -> bwd_fused_glu)
    bool glu_epilogue_ = false;
    const Node* glu_node_ = nullptr;
    uint64_t glu_gu_ = 0;
    bool norm_pending(uint64_t buf) const;
    void flush_norms();
    FusedSlot* fused_for(uint64_t weight);
};

class TapeContext {
public:
    TapeContext(Device& dev, size_t arena_capacity = TapeArena::kDefaultCapacity);

    void begin();
    Node* record_op(OpType op, const TensorRef* inputs, uint32_t num_inputs,
                    const TensorRef* outputs, uint32_t num_outputs, const void* params = nullptr,
                    uint32_t params_size = 0);
    void save_for_backward(Node* node, const uint64_t* ids, uint32_t count);
    void backward(Node* loss_node, uint64_t grad_output_buffer);
    uint64_t get_grad_buffer(uint64_t id) const { return engine_.get_grad_buffer(id); }
    void set_fused_update(uint64_t weight, const BackwardEngine::FusedUpdate& u) {
        engine_.set_fused_update(weight, u);
    }
    void clear_fused_updates() { engine_.clear_fused_updates(); }
    bool fused_update_applied(uint64_t weight) const { return engine_.fused_update_applied(weight); }
    void set_glu_epilogue(bool on) { engine_.set_glu_epilogue(on); }
    bool glu_epilogue() const { return engine_.glu_epilogue(); }
    // every (tensor id, gradient buffer id) pair of the last backward pass
    std::vector<std::pair<uint64_t, uint64_t>> grads() const;
    void end();
    uint64_t acquire_temp(size_t bytes);

    bool is_recording() const { return recording_; }
    TapeArena& arena() { return arena_; }
    Device& device() { return dev_; }
    BackwardEngine::Stats last_backward_stats() const { return engine_.last_stats(); }
    size_t arena_bytes_used() const { return arena_.bytes_used(); }
    float arena_utilization() const { return arena_.utilization(); }

private:
    Device& dev_;
    TapeArena arena_;
    BackwardEngine engine_;
    bool recording_ = false;
    uint32_t seq_ = 0;
    std::vector<uint64_t> step_bufs_;
};

}  // namespace autograd
}  // namespace grilly
