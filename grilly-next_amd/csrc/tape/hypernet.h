// hypernet.h — the VSA hypernetwork, its surprise-momentum optimizer and one training step,
// on the MI355X tape engine.
//
// The reference's only real caller of the tape backward (VSAHypernetwork,
// cpp/include/grilly/models/vsa_hypernetwork.h:21-115 and vsa_hypernetwork.cpp:11-160;
// SurpriseMomentumOptimizer and vsa_training_step, cpp/python/bindings.cpp:3049-3286):
//
//   forward: vsa_state (bitpacked) -> VSAUnpackProject (vsa_dim -> d_model) -> Linear
//            (d_model -> 2 d_model) -> GELU -> Linear (2 d_model -> K vsa_dim), recorded on
//            the tape with the reference's saved slots and run by libgn_bwd's forward kernels
//   loss:    VSASurrogateLoss with the reference's constants (bindings.cpp:3169-3176); its
//            forward (dots, Gumbel top-2, softmax branch weights, hinge + contrastive) runs
//            in one kernel with seeded noise (the reference's noise is unseeded)
//   step:    tape.backward from the loss, the surprise-momentum update of every parameter
//            that received a gradient (one multi-tensor launch), tape.end
//
// Differences from the reference, each deliberate:
//   * the Gumbel noise is reproducible: (gumbel_seed, gumbel_counter) of the model select it,
//     and the counter advances once per loss forward;
//   * for a batch of more than one row the output layer is laid out [batch, K * vsa_dim]
//     (what the tape records and the loss reads); the reference's chunked forward writes
//     [K][batch][vsa_dim], which agrees only for its batch of one (vsa_hypernetwork.cpp:279-306);
//   * the optimizer does not clear the gradients after the update (clear_grad 0): the buffers
//     are the backward pass's own and tape.end() releases them right after, so the zeros of the
//     reference's shader (surprise-momentum.glsl, clear_grad 1) would never be read.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "autograd.h"

namespace grilly {
namespace models {

using autograd::Node;
using autograd::TapeContext;
using autograd::TensorRef;

class VSAHypernetwork {
public:
    VSAHypernetwork(Device& dev, uint32_t d_model = 768, uint32_t vsa_dim = 10240, uint32_t K = 16,
                    uint32_t router_hidden = 32, uint32_t seed = 42);
    ~VSAHypernetwork();
    VSAHypernetwork(const VSAHypernetwork&) = delete;
    VSAHypernetwork& operator=(const VSAHypernetwork&) = delete;

    // Records the four nodes and runs their forward kernels; returns the predictions
    // [batch, K, vsa_dim] (fp32, requires_grad).  vsa_state: u32 words [words] or [batch, words].
    TensorRef forward(TapeContext& tape, TensorRef vsa_state);

    // Order: W_proj, b_proj, W1, b1, W2, b2, W_r1, b_r1, W_r2, b_r2 (bindings.cpp:2973-2984).
    std::vector<uint64_t> parameter_buffer_ids() const;
    std::vector<uint64_t> parameter_sizes() const;

    uint32_t d_model() const { return d_model_; }
    uint32_t vsa_dim() const { return vsa_dim_; }
    uint32_t K() const { return K_; }
    uint32_t router_hidden() const { return router_hidden_; }
    uint32_t num_weight_bufs() const { return 10; }
    TensorRef last_output() const { return last_output_; }
    TensorRef h_t() const { return h_t_; }
    Device& device() { return dev_; }

    // Gumbel noise of the surrogate loss forward: drawn at (gumbel_seed, gumbel_counter); the
    // counter advances after every loss forward run for this model.
    uint64_t gumbel_seed = 0;
    uint64_t gumbel_counter = 0;

private:
    Device& dev_;
    uint32_t d_model_, vsa_dim_, K_, router_hidden_;
    uint64_t w_[10] = {};
    TensorRef last_output_{}, h_t_{};
};

class SurpriseMomentumOptimizer {
public:
    // One zeroed s_bar per parameter of `model` (bindings.cpp:3071-3138).
    SurpriseMomentumOptimizer(Device& dev, const VSAHypernetwork& model, float lr = 1e-3f,
                              float alpha = 0.9f, float clip = 1.0f);
    ~SurpriseMomentumOptimizer();
    SurpriseMomentumOptimizer(const SurpriseMomentumOptimizer&) = delete;
    SurpriseMomentumOptimizer& operator=(const SurpriseMomentumOptimizer&) = delete;

    // Before the backward pass: hand each weight's step to the tape, so a weight that only a
    // Linear node of a few rows uses is updated inside that node's backward pass over W
    // (gn_linear_bwd_surprise_momentum, same result bit for bit) and its gradient is never
    // stored.  A no-op when fuse_linear_updates is false.
    void prepare(TapeContext& tape);
    // The update vsa_training_step applies between backward and end (bindings.cpp:3198-3277):
    // every parameter whose gradient the tape holds, one launch per 24 tensors (the weights
    // prepare() handed over were updated by the backward pass).  Returns the number of
    // parameters updated.
    int apply(TapeContext& tape);

    const std::vector<uint64_t>& s_bar_buffer_ids() const { return s_bar_; }
    const std::vector<uint64_t>& weight_ids() const { return weights_; }
    const std::vector<uint64_t>& sizes() const { return sizes_; }

    float eta_base, alpha_momentum, lambda_recall = 0.0f, surprise_floor = 0.01f,
                                     weight_decay = 0.0f, clip_max;
    uint64_t steps = 0;
    bool fuse_linear_updates = true;

private:
    Device& dev_;
    std::vector<uint64_t> weights_, sizes_, s_bar_;
};

// A step-scoped u32 buffer holding `rows` bitpacked vectors of `words` words (the reference's
// upload_bitpacked, vsa_loss_node.cpp:19-34); [words] for one row, else [rows, words].
TensorRef upload_bitpacked(TapeContext& tape, const uint32_t* data, uint32_t rows, uint32_t words);

// Records the VSASurrogateLoss node of a hypernetwork forward with the reference's constants
// (bindings.cpp:3164-3186): inputs [predicted, true_delta], output a scalar.
Node* record_surrogate_loss(TapeContext& tape, const TensorRef& predicted, const TensorRef& delta);

// The loss node's forward (dispatch_vsa_loss_forward, vsa_loss_node.cpp:36-180): runs the
// fused surrogate forward kernel, appends the results and weights buffers to the node's saved
// slots (where the backward reads them), stores winning_k / runner_up_k / loss_value in its
// params and returns the batch mean of the loss (one small device-to-host copy).
float vsa_loss_forward(TapeContext& tape, Node* node, uint64_t seed, uint64_t counter,
                       bool noise = true);

// begin, upload, forward, loss forward, backward, optimizer (if any), end; returns the loss
// (bindings.cpp:3140-3286).  state, delta: rows x words u32 each.
float vsa_training_step(TapeContext& tape, VSAHypernetwork& model, const uint32_t* state,
                        const uint32_t* delta, uint32_t rows, uint32_t words,
                        SurpriseMomentumOptimizer* optimizer);

}  // namespace models
}  // namespace grilly
