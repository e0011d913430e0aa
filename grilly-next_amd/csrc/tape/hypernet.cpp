// hypernet.cpp — VSAHypernetwork, SurpriseMomentumOptimizer and the training step
// (see hypernet.h for the contract and the reference lines each part follows).
#include "hypernet.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <random>
#include <stdexcept>

#include "gn_bwd.h"

namespace grilly {
namespace models {

using autograd::OpType;
using autograd::VSASurrogateLossParams;

namespace {

void gn_call(int rc, const char* what) {
    if (rc != GN_OK) throw std::runtime_error(std::string(what) + ": " + gn_last_error());
}

void* P(uint64_t id) { return reinterpret_cast<void*>(id); }

TensorRef ref2(uint64_t id, uint32_t rows, uint32_t cols, uint32_t dtype, bool grad) {
    TensorRef r{};
    r.buffer_id = id;
    r.ndim = 2;
    r.shape[0] = rows;
    r.shape[1] = cols;
    r.dtype = dtype;
    r.requires_grad = grad;
    return r;
}

// Element counts in parameter order (bindings.cpp:2973-2984).
std::vector<uint64_t> sizes_of(uint64_t d, uint64_t v, uint64_t K, uint64_t rh) {
    const uint64_t h = 2 * d;
    return {d * v, d, h * d, h, K * v * h, K * v, rh * d, rh, K * rh, K};
}

}  // namespace

// ───────────────────────────────────────────────────────────────────── VSAHypernetwork

// vsa_hypernetwork.cpp:11-49: one std::mt19937(seed) draws, in this order, W_proj ~ N(0,
// sqrt(2/(vsa_dim + d_model))), W1 ~ N(0, sqrt(2/(d_model + hidden))), W2 ~ N(0, 1/sqrt(hidden)),
// W_r1 ~ N(0, 1/sqrt(d_model)), W_r2 ~ N(0, 1/sqrt(router_hidden)); the biases are zero.
VSAHypernetwork::VSAHypernetwork(Device& dev, uint32_t d_model, uint32_t vsa_dim, uint32_t K,
                                 uint32_t router_hidden, uint32_t seed)
    : dev_(dev), d_model_(d_model), vsa_dim_(vsa_dim), K_(K), router_hidden_(router_hidden) {
    if (d_model == 0 || vsa_dim == 0 || K == 0 || router_hidden == 0)
        throw std::invalid_argument("VSAHypernetwork: every dimension must be positive");
    if (vsa_dim % 32 != 0)
        throw std::invalid_argument("VSAHypernetwork: vsa_dim must be a multiple of 32 (bitpacked words)");
    gumbel_seed = seed;
    const auto sizes = sizes_of(d_model, vsa_dim, K, router_hidden);
    for (int i = 0; i < 10; ++i) w_[i] = dev_.acquire(sizes[i] * sizeof(float));
    std::mt19937 rng(seed);
    const uint32_t hidden = 2 * d_model;
    const float scales[5] = {std::sqrt(2.0f / (vsa_dim + d_model)), std::sqrt(2.0f / (d_model + hidden)),
                             1.0f / std::sqrt(float(hidden)), 1.0f / std::sqrt(float(d_model)),
                             1.0f / std::sqrt(float(router_hidden))};
    // stage through a bounded host buffer: W2 alone is K * vsa_dim * hidden floats
    constexpr size_t kChunk = size_t(1) << 24;
    std::vector<float> host(kChunk);
    for (int t = 0; t < 5; ++t) {
        const int slot = 2 * t;
        std::normal_distribution<float> dist(0.0f, scales[t]);
        for (uint64_t off = 0; off < sizes[slot]; off += kChunk) {
            const size_t n = (size_t)std::min<uint64_t>(kChunk, sizes[slot] - off);
            for (size_t i = 0; i < n; ++i) host[i] = dist(rng);
            dev_.upload(w_[slot], host.data(), n * sizeof(float), off * sizeof(float));
        }
        dev_.zero(w_[slot + 1], sizes[slot + 1] * sizeof(float));
    }
    dev_.synchronize();
}

VSAHypernetwork::~VSAHypernetwork() {
    try {
        dev_.synchronize();
        for (uint64_t id : w_)
            if (id) dev_.release(id);
    } catch (...) {
    }
}

std::vector<uint64_t> VSAHypernetwork::parameter_buffer_ids() const {
    return std::vector<uint64_t>(w_, w_ + 10);
}

std::vector<uint64_t> VSAHypernetwork::parameter_sizes() const {
    return sizes_of(d_model_, vsa_dim_, K_, router_hidden_);
}

// vsa_hypernetwork.cpp:52-160: the same four nodes and saved slots, one forward kernel each.
TensorRef VSAHypernetwork::forward(TapeContext& tape, TensorRef vsa_state) {
    const uint32_t batch = vsa_state.ndim >= 2 ? vsa_state.shape[0] : 1;
    const uint32_t words = vsa_state.ndim ? vsa_state.shape[vsa_state.ndim - 1] : 0;
    if (vsa_state.ndim < 1 || vsa_state.ndim > 2 || words * 32 != vsa_dim_ || batch == 0)
        throw std::invalid_argument("VSAHypernetwork.forward: vsa_state must be u32 [" +
                                    std::to_string(vsa_dim_ / 32) + "] or [batch, " +
                                    std::to_string(vsa_dim_ / 32) + "]");
    if (!vsa_state.valid()) throw std::invalid_argument("VSAHypernetwork.forward: vsa_state has no buffer");
    void* s = dev_.stream();
    const uint32_t d = d_model_, hidden = 2 * d_model_, out_dim = K_ * vsa_dim_;

    // 1. unpack + project (bits -> d_model)
    TensorRef h_t = ref2(tape.acquire_temp((size_t)batch * d * 4), batch, d, 0, true);
    {
        TensorRef in[1] = {vsa_state}, out[1] = {h_t};
        Node* n0 = tape.record_op(OpType::VSAUnpackProject, in, 1, out, 1);
        const uint64_t saves[2] = {w_[0], w_[1]};
        tape.save_for_backward(n0, saves, 2);
        const size_t wsb = gn_vsa_fwd_workspace_bytes((int)batch, (int)d, (int)vsa_dim_);
        const uint64_t ws = wsb ? tape.acquire_temp(wsb) : 0;
        gn_call(gn_vsa_unpack_project_fwd((const uint32_t*)P(vsa_state.buffer_id), (const float*)P(w_[0]),
                                          (const float*)P(w_[1]), (float*)P(h_t.buffer_id), (int)batch,
                                          (int)d, (int)vsa_dim_, (int)words, P(ws), wsb, s),
                "VSAHypernetwork unpack-project forward");
    }
    h_t_ = h_t;

    // 2. Linear d_model -> hidden
    TensorRef h_mid = ref2(tape.acquire_temp((size_t)batch * hidden * 4), batch, hidden, 0, true);
    gn_call(gn_linear_fwd(P(h_t.buffer_id), P(w_[2]), P(w_[3]), P(h_mid.buffer_id), (int)batch,
                          (int)hidden, (int)d, GN_F32, s),
            "VSAHypernetwork layer 1 forward");
    {
        TensorRef in[1] = {h_t}, out[1] = {h_mid};
        Node* n1 = tape.record_op(OpType::Linear, in, 1, out, 1);
        const uint64_t saves[2] = {w_[2], w_[3]};
        tape.save_for_backward(n1, saves, 2);
    }

    // 3. GELU (tanh form, activation-gelu.glsl)
    TensorRef h_act = ref2(tape.acquire_temp((size_t)batch * hidden * 4), batch, hidden, 0, true);
    gn_call(gn_act_fwd(GN_ACT_GELU_TANH, P(h_mid.buffer_id), P(h_act.buffer_id),
                       (int64_t)batch * hidden, GN_F32, s),
            "VSAHypernetwork GELU forward");
    {
        TensorRef in[1] = {h_mid}, out[1] = {h_act};
        tape.record_op(OpType::GELU, in, 1, out, 1);
    }

    // 4. Linear hidden -> K * vsa_dim, recorded 2-D (its backward reads shape[1] as N)
    TensorRef pred = ref2(tape.acquire_temp((size_t)batch * out_dim * 4), batch, out_dim, 0, true);
    gn_call(gn_linear_fwd(P(h_act.buffer_id), P(w_[4]), P(w_[5]), P(pred.buffer_id), (int)batch,
                          (int)out_dim, (int)hidden, GN_F32, s),
            "VSAHypernetwork layer 2 forward");
    {
        TensorRef in[1] = {h_act}, out[1] = {pred};
        Node* n3 = tape.record_op(OpType::Linear, in, 1, out, 1);
        const uint64_t saves[2] = {w_[4], w_[5]};
        tape.save_for_backward(n3, saves, 2);
    }

    TensorRef out3 = pred;
    out3.ndim = 3;
    out3.shape[0] = batch;
    out3.shape[1] = K_;
    out3.shape[2] = vsa_dim_;
    last_output_ = out3;
    return out3;
}

// ──────────────────────────────────────────────────────────── SurpriseMomentumOptimizer

SurpriseMomentumOptimizer::SurpriseMomentumOptimizer(Device& dev, const VSAHypernetwork& model,
                                                     float lr, float alpha, float clip)
    : eta_base(lr), alpha_momentum(alpha), clip_max(clip), dev_(dev) {
    weights_ = model.parameter_buffer_ids();
    sizes_ = model.parameter_sizes();
    for (uint64_t n : sizes_) {
        const uint64_t id = dev_.acquire(n * sizeof(float));
        dev_.zero(id, n * sizeof(float));
        s_bar_.push_back(id);
    }
    dev_.synchronize();
}

SurpriseMomentumOptimizer::~SurpriseMomentumOptimizer() {
    try {
        dev_.synchronize();
        for (uint64_t id : s_bar_) dev_.release(id);
    } catch (...) {
    }
}

void SurpriseMomentumOptimizer::prepare(TapeContext& tape) {
    tape.clear_fused_updates();
    if (!fuse_linear_updates) return;
    for (size_t i = 0; i < weights_.size(); ++i)
        tape.set_fused_update(weights_[i], autograd::BackwardEngine::FusedUpdate{
                                               s_bar_[i], eta_base, alpha_momentum, lambda_recall,
                                               surprise_floor, weight_decay, clip_max, false});
}

int SurpriseMomentumOptimizer::apply(TapeContext& tape) {
    std::vector<gn_opt_param> entries;
    int fused = 0;
    for (size_t i = 0; i < weights_.size(); ++i) {
        if (tape.fused_update_applied(weights_[i])) {  // stepped by its Linear backward
            ++fused;
            continue;
        }
        const uint64_t g = tape.get_grad_buffer(weights_[i]);
        if (g == 0) continue;  // no gradient for this parameter (bindings.cpp:3228-3232)
        gn_opt_param p{};
        p.W = (float*)P(weights_[i]);
        p.grad = (float*)P(g);
        p.state0 = (float*)P(s_bar_[i]);
        p.state1 = nullptr;    // the reference's delta scratch is never read back
        p.recalled = nullptr;  // recalled gradient: zero (bindings.cpp:3045-3047)
        p.n = (int64_t)sizes_[i];
        entries.push_back(p);
    }
    if (!entries.empty())
        gn_call(gn_surprise_momentum_step(entries.data(), (int)entries.size(), eta_base, alpha_momentum,
                                          lambda_recall, surprise_floor, weight_decay, clip_max, 0,
                                          dev_.stream()),
                "SurpriseMomentumOptimizer step");
    tape.clear_fused_updates();
    ++steps;
    return (int)entries.size() + fused;
}

// ───────────────────────────────────────────────────────────────────── loss and step

TensorRef upload_bitpacked(TapeContext& tape, const uint32_t* data, uint32_t rows, uint32_t words) {
    const size_t bytes = (size_t)rows * words * sizeof(uint32_t);
    const uint64_t id = tape.acquire_temp(bytes);
    tape.device().upload(id, data, bytes);
    TensorRef r{};
    r.buffer_id = id;
    if (rows <= 1) {
        r.ndim = 1;
        r.shape[0] = words;
    } else {
        r.ndim = 2;
        r.shape[0] = rows;
        r.shape[1] = words;
    }
    r.dtype = 2;  // u32
    r.requires_grad = false;
    return r;
}

Node* record_surrogate_loss(TapeContext& tape, const TensorRef& predicted, const TensorRef& delta) {
    if (predicted.ndim != 3) throw std::invalid_argument("surrogate loss: predictions must be [batch, K, D]");
    VSASurrogateLossParams p{};
    p.gamma = 1.0f;         // hinge margin
    p.delta_margin = 1.0f;  // contrastive branch separation
    p.lambda = 0.3f;        // contrastive weight
    p.K = predicted.shape[1];
    p.D = predicted.shape[2];
    p.temperature = 1.0f;   // Gumbel-softmax temperature
    p.diversity_lambda = 0.01f;
    TensorRef loss{};
    loss.ndim = 1;
    loss.shape[0] = 1;
    loss.dtype = 0;
    TensorRef in[2] = {predicted, delta}, out[1] = {loss};
    return tape.record_op(OpType::VSASurrogateLoss, in, 2, out, 1, &p, sizeof(p));
}

float vsa_loss_forward(TapeContext& tape, Node* node, uint64_t seed, uint64_t counter, bool noise) {
    if (!node || node->op != OpType::VSASurrogateLoss)
        throw std::invalid_argument("vsa_loss_forward: not a VSASurrogateLoss node");
    VSASurrogateLossParams p{};
    std::memcpy(&p, node->params, sizeof(p));
    const TensorRef& preds = node->inputs[0];
    const TensorRef& bits = node->inputs[1];
    const uint32_t B = preds.shape[0], K = p.K, D = p.D, words = (D + 31) / 32;
    if (preds.ndim != 3 || preds.shape[1] != K || preds.shape[2] != D)
        throw std::invalid_argument("vsa_loss_forward: predictions must be [batch, K, D] of the params");
    if (bits.numel() != (size_t)B * words)
        throw std::invalid_argument("vsa_loss_forward: target bits must hold batch x ceil(D/32) words");
    if (node->num_saved + 2 > autograd::kMaxNodeIO)
        throw std::invalid_argument("vsa_loss_forward: the node's saved slots are full");
    Device& dev = tape.device();
    const uint64_t dots = tape.acquire_temp((size_t)B * K * 4);
    const uint64_t results = tape.acquire_temp((size_t)B * 4 * 4);
    const uint64_t weights = tape.acquire_temp((size_t)B * K * 4);
    const uint64_t loss = tape.acquire_temp((size_t)B * 4);
    gn_call(gn_vsa_surrogate_fwd((const float*)P(preds.buffer_id), (const uint32_t*)P(bits.buffer_id),
                                 (float*)P(dots), (uint32_t*)P(results), (float*)P(weights), (float*)P(loss),
                                 (int)B, (int)K, (int)D, (int)words, p.gamma, p.delta_margin, p.lambda,
                                 p.temperature, seed, counter, noise ? 0u : GN_NO_GUMBEL, dev.stream()),
            "VSA surrogate forward");
    // saved slots the backward reads: [n-2] results, [n-1] weights (vsa_loss_node.cpp:156-159)
    node->saved_buffer_ids[node->num_saved++] = results;
    node->saved_buffer_ids[node->num_saved++] = weights;
    std::vector<float> lv(B);
    uint32_t r01[2];
    dev.download(results, r01, sizeof(r01));
    dev.download(loss, lv.data(), (size_t)B * 4);
    double total = 0.0;
    for (float l : lv) total += l;
    p.winning_k = r01[0];
    p.runner_up_k = r01[1];
    p.loss_value = (float)(total / B);
    std::memcpy(node->params, &p, sizeof(p));
    node->params_size = std::max<uint32_t>(node->params_size, sizeof(p));
    return p.loss_value;
}

float vsa_training_step(TapeContext& tape, VSAHypernetwork& model, const uint32_t* state,
                        const uint32_t* delta, uint32_t rows, uint32_t words,
                        SurpriseMomentumOptimizer* optimizer) {
    if (words * 32 != model.vsa_dim())
        throw std::invalid_argument("vsa_training_step: the state holds " + std::to_string(words) +
                                    " words per row; the model needs " + std::to_string(model.vsa_dim() / 32));
    tape.begin();
    try {
        TensorRef s = upload_bitpacked(tape, state, rows, words);
        TensorRef predicted = model.forward(tape, s);
        TensorRef d = upload_bitpacked(tape, delta, rows, words);
        Node* loss_node = record_surrogate_loss(tape, predicted, d);
        const float loss = vsa_loss_forward(tape, loss_node, model.gumbel_seed, model.gumbel_counter++);
        if (optimizer) optimizer->prepare(tape);
        tape.backward(loss_node, 0ULL);
        if (optimizer) optimizer->apply(tape);
        tape.end();
        return loss;
    } catch (...) {
        tape.clear_fused_updates();
        tape.end();
        throw;
    }
}

}  // namespace models
}  // namespace grilly
