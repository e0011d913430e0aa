// autograd.cpp — BackwardEngine and TapeContext (see autograd.h for the contract).
#include "autograd.h"

#include <cmath>
#include <string>

#include "gn_bwd.h"

namespace grilly {
namespace autograd {

namespace {

int gn_dtype(uint32_t d, const char* what) {
    if (d == 0) return GN_F32;
    if (d == 4) return GN_BF16;
    throw std::invalid_argument(std::string(what) + ": tensor dtype must be f32 (0) or bf16 (4)");
}

void gn_call(int rc, const char* what) {
    if (rc != GN_OK) throw std::runtime_error(std::string(what) + ": " + gn_last_error());
}

void* P(uint64_t id) { return reinterpret_cast<void*>(id); }

template <typename T>
T params_of(const Node* n) {
    T p{};
    std::memcpy(&p, n->params, std::min<size_t>(sizeof(T), n->params_size));
    return p;
}

inline uint64_t mix(uint64_t x) {
    x ^= x >> 33;
    x *= 0xff51afd7ed558ccdULL;
    x ^= x >> 33;
    return x;
}

}  // namespace

// ═════════════════════════════════════════════════════════════════════ BackwardEngine

BackwardEngine::BackwardEngine(Device& dev) : dev_(dev), table_(kGradTableSize) { clear_grads(); }

void BackwardEngine::clear_grads() {
    for (auto& e : table_) e = GradEntry{};
    count_ = 0;
}

BackwardEngine::GradEntry* BackwardEngine::find(uint64_t id) const {
    if (id == 0) return nullptr;
    const size_t mask = kGradTableSize - 1;
    for (size_t i = mix(id) & mask, probes = 0; probes < kGradTableSize; i = (i + 1) & mask, ++probes) {
        if (table_[i].buffer_id == id) return &table_[i];
        if (table_[i].buffer_id == 0) return nullptr;
    }
    return nullptr;
}

BackwardEngine::GradEntry* BackwardEngine::find_or_insert(uint64_t id) {
    if (GradEntry* e = find(id)) return e;
    if (count_ >= kGradTableSize * 3 / 4)
        throw std::length_error("BackwardEngine: gradient table full (more than 6144 tensors)");
    const size_t mask = kGradTableSize - 1;
    size_t i = mix(id) & mask;
    while (table_[i].buffer_id != 0) i = (i + 1) & mask;
    table_[i] = GradEntry{id, 0, 0, 0, false};
    ++count_;
    return &table_[i];
}

uint64_t BackwardEngine::get_grad_buffer(uint64_t id) const {
    const GradEntry* e = find(id);
    return e ? e->grad_id : 0ULL;
}

uint64_t BackwardEngine::alloc_grad(size_t bytes) {
    uint64_t id = dev_.acquire(bytes);
    backward_bufs_.push_back(id);
    return id;
}

uint64_t BackwardEngine::split_ws(size_t bytes) {
    if (bytes == 0) return 0;
    if (bytes > ws_bytes_) {
        ws_id_ = alloc_grad(bytes);
        ws_bytes_ = bytes;
    }
    return ws_id_;
}

void BackwardEngine::contribute(uint64_t id, uint64_t g, uint32_t dtype, size_t numel, bool owned) {
    if (id == 0 || g == 0) return;
    GradEntry* e = find_or_insert(id);
    // a fan-out add reads or writes a gradient a deferred norm finish has not written yet
    if (e->grad_id != 0 && (norm_pending(g) || norm_pending(e->grad_id))) flush_norms();
    const size_t bytes = numel * TensorRef::elem_size(dtype);
    if (e->grad_id == 0) {
        *e = GradEntry{id, g, bytes, dtype, owned};
        return;
    }
    // fan-out: the second consumer's gradient is added (autograd.cpp:78-86 drops it).  The
    // same buffer arriving twice is two contributions too (Add(x, x), x + Reshape(x): both
    // borrow the upstream buffer), so it is summed like any other pair.
    if (e->dtype != dtype || e->grad_bytes != bytes)
        throw std::runtime_error("BackwardEngine: fan-out gradients disagree in dtype or size");
    if (!e->owned && owned) {
        // the recorded gradient is borrowed (another node's buffer) but the new one is this
        // contribution's own: add the borrowed one into it and keep it (one kernel, no copy;
        // a single fp add is commutative, so the sum is the same either way round)
        gn_call(gn_add_inplace(P(g), P(e->grad_id), (int64_t)numel, gn_dtype(dtype, "fan-out"),
                               dev_.stream()), "fan-out add");
        e->grad_id = g;
        e->owned = true;
        stats_.fanout_accumulations++;
        stats_.shaders_dispatched++;
        return;
    }
    if (!e->owned) {
        uint64_t fresh = alloc_grad(bytes);
        gn_call(gn_convert(P(e->grad_id), gn_dtype(dtype, "fan-out"), P(fresh),
                           gn_dtype(dtype, "fan-out"), (int64_t)numel, dev_.stream()),
                "fan-out copy");
        stats_.shaders_dispatched++;
        e->grad_id = fresh;
        e->owned = true;
    }
    gn_call(gn_add_inplace(P(e->grad_id), P(g), (int64_t)numel, gn_dtype(dtype, "fan-out"),
                           dev_.stream()), "fan-out add");
    stats_.fanout_accumulations++;
    stats_.shaders_dispatched++;
}

// A node whose output lives in one of its input buffers (an in-place op or a view such as
// Reshape onto the same buffer) shares that buffer id between the two versions of the tensor.
bool BackwardEngine::writes_in_place(const Node* n, uint64_t id) {
    for (uint32_t o = 0; o < n->num_outputs && o < kMaxNodeIO; ++o)
        if (n->outputs[o].buffer_id == id) return true;
    return false;
}

// The gradient of the input version of an in-place tensor: the table entry under its id held
// the gradient of the output version (already summed over that version's consumers, which
// come later on the tape and were visited first); from here on the entry is the earlier
// version's gradient, which the earlier consumers visited next add onto.
void BackwardEngine::replace(uint64_t id, uint64_t g, uint32_t dtype, size_t numel, bool owned) {
    if (id == 0 || g == 0) return;
    GradEntry* e = find_or_insert(id);
    *e = GradEntry{id, g, numel * TensorRef::elem_size(dtype), dtype, owned};
}

const void* BackwardEngine::gout(Node* n) const {
    if (n->grad_output_buffer <= 1)
        throw std::invalid_argument(
            "backward: this node needs an upstream gradient buffer (grad_output_buffer)");
    return P(n->grad_output_buffer);
}

void BackwardEngine::backward(TapeArena& tape, Node* loss_node, uint64_t grad_output_buffer) {
    stats_ = {};
    ws_id_ = 0;
    ws_bytes_ = 0;
    bf16_copies_.clear();
    norm_pending_.clear();
    glu_node_ = nullptr;
    glu_gu_ = 0;
    if (!loss_node) throw std::invalid_argument("backward: loss node is None");
    // autograd.cpp:30-31: 0 means "the loss computes its own gradient" (sentinel 1)
    loss_node->grad_output_buffer = grad_output_buffer ? grad_output_buffer : 1ULL;
    // a fused weight update needs the weight's whole gradient from one Linear node
    for (FusedSlot& f : fused_) {
        int linear_uses = 0, other_uses = 0;
        for (Node* cur = tape.tail<Node>(); cur != nullptr; cur = cur->prev_in_tape) {
            for (uint32_t i = 0; i < cur->num_inputs && i < kMaxNodeIO; ++i)
                other_uses += cur->inputs[i].buffer_id == f.weight;
            for (uint32_t i = 0; i < cur->num_saved && i < kMaxNodeIO; ++i)
                if (cur->saved_buffer_ids[i] == f.weight) {
                    if (cur->op == OpType::Linear && i == 0) ++linear_uses;
                    else ++other_uses;
                }
        }
        f.eligible = linear_uses == 1 && other_uses == 0;
        f.u.applied = false;
    }
    for (Node* cur = tape.tail<Node>(); cur != nullptr; cur = cur->prev_in_tape) {
        stats_.nodes_visited++;
        if (cur->grad_output_buffer == 0) {
            for (uint32_t i = 0; i < cur->num_outputs && i < kMaxNodeIO; ++i) {
                uint64_t g = get_grad_buffer(cur->outputs[i].buffer_id);
                if (g) {
                    cur->grad_output_buffer = g;
                    break;
                }
            }
        }
        // a FusedGLU whose output gradient the down projection's epilogue turned into gu
        if (cur->grad_output_buffer == 0 && cur == glu_node_) cur->grad_output_buffer = 1;
        if (cur->grad_output_buffer == 0) continue;
        stats_.nodes_with_grad++;
        std::memset(cur->grad_input_buffers, 0, sizeof(cur->grad_input_buffers));
        borrowed_ = 0;
        handled_ = 0;
        dispatch(cur);
        for (uint32_t i = 0; i < cur->num_inputs && i < kMaxNodeIO; ++i) {
            const TensorRef& in = cur->inputs[i];
            if (!in.requires_grad || cur->grad_input_buffers[i] == 0 || ((handled_ >> i) & 1u))
                continue;
            const bool own = !((borrowed_ >> i) & 1u);
            // an in-place node's first input with this id replaces the entry (it becomes the
            // input version's gradient); a later input with the same id (Add(x, x) written
            // into x) adds onto it, as the out-of-place form does
            bool first = true;
            for (uint32_t j = 0; j < i && first; ++j)
                first = !(cur->inputs[j].buffer_id == in.buffer_id && cur->inputs[j].requires_grad &&
                          cur->grad_input_buffers[j] != 0 && !((handled_ >> j) & 1u));
            if (first && writes_in_place(cur, in.buffer_id))
                replace(in.buffer_id, cur->grad_input_buffers[i], in.dtype, in.numel(), own);
            else
                contribute(in.buffer_id, cur->grad_input_buffers[i], in.dtype, in.numel(), own);
        }
    }
    flush_norms();
}

bool BackwardEngine::norm_pending(uint64_t buf) const {
    if (!buf) return false;
    for (const GnNormFinish& f : norm_pending_)
        if (reinterpret_cast<uint64_t>(f.dgamma) == buf || reinterpret_cast<uint64_t>(f.dbeta) == buf)
            return true;
    return false;
}

void BackwardEngine::flush_norms() {
    if (norm_pending_.empty()) return;
    gn_call(gn_norm_finish(norm_pending_.data(), (int)norm_pending_.size(), dev_.stream()),
            "norm parameter gradients (deferred finish)");
    stats_.shaders_dispatched++;
    norm_pending_.clear();
}

void BackwardEngine::dispatch(Node* n) {
    switch (n->op) {
        case OpType::Linear: bwd_linear(n); break;
        case OpType::ReLU: bwd_act(n, GN_ACT_RELU, false); break;
        case OpType::GELU:
            bwd_act(n, params_of<GELUParams>(n).erf_form ? GN_ACT_GELU_ERF : GN_ACT_GELU_TANH, false);
            break;
        case OpType::SiLU: bwd_act(n, GN_ACT_SILU, false); break;
        case OpType::Tanh: bwd_act(n, GN_ACT_TANH, true); break;
        case OpType::Sigmoid: bwd_act(n, GN_ACT_SIGMOID, true); break;
        case OpType::Softmax: bwd_softmax(n); break;
        case OpType::LayerNorm: bwd_layernorm(n); break;
        case OpType::RMSNorm: bwd_rmsnorm(n); break;
        case OpType::FlashAttention2: bwd_attention(n); break;
        case OpType::CrossEntropy: bwd_cross_entropy(n); break;
        case OpType::Add: bwd_add_sub(n, false); break;
        case OpType::Reshape: bwd_passthrough(n); break;
        case OpType::VSAUnpackProject: bwd_vsa_unpack_project(n); break;
        case OpType::VSASurrogateLoss: bwd_vsa_surrogate(n); break;
        case OpType::FusedGLU: bwd_fused_glu(n); break;
        case OpType::Embedding: bwd_embedding(n); break;
        case OpType::Sub: bwd_binary(n, GN_BIN_SUB); break;
        case OpType::Mul: bwd_binary(n, GN_BIN_MUL); break;
        case OpType::Div: bwd_binary(n, GN_BIN_DIV); break;
        case OpType::Neg: bwd_binary(n, GN_BIN_NEG); break;
        case OpType::Sum: bwd_reduce(n, GN_RED_SUM); break;
        case OpType::Mean: bwd_reduce(n, GN_RED_MEAN); break;
        case OpType::Transpose: bwd_transpose(n); break;
        case OpType::MSELoss: bwd_mse(n); break;
        case OpType::MatMul: bwd_matmul(n); break;
        case OpType::VSALoRAExpand: bwd_vsa_lora_expand(n); break;
        case OpType::VSACosineBlendLoss: bwd_vsa_cosine_blend(n); break;
        case OpType::CubeMindSurprise:
        case OpType::TemporalSurprise: bwd_surprise_passthrough(n); break;
        default: stats_.cpu_fallbacks++; break;  // no handler (autograd.cpp:126-128)
    }
}

void BackwardEngine::set_fused_update(uint64_t weight, const FusedUpdate& u) {
    if (!weight || !u.state) throw std::invalid_argument("set_fused_update: weight and state buffers required");
    if (FusedSlot* f = fused_for(weight)) {
        f->u = u;
        return;
    }
    fused_.push_back(FusedSlot{weight, u, false});
}

BackwardEngine::FusedSlot* BackwardEngine::fused_for(uint64_t weight) {
    for (FusedSlot& f : fused_)
        if (f.weight == weight) return &f;
    return nullptr;
}

bool BackwardEngine::fused_update_applied(uint64_t weight) const {
    for (const FusedSlot& f : fused_)
        if (f.weight == weight) return f.u.applied;
    return false;
}

// Linear: y = x W^T + b (autograd.cpp:172-305); saved[0] = W [N x K], saved[1] = b or 0.
void BackwardEngine::bwd_linear(Node* n) {
    const TensorRef& x = n->inputs[0];
    const TensorRef& y = n->outputs[0];
    const int M = (int)x.rows(), K = (int)x.last(), N = (int)y.last();
    if ((size_t)M != y.rows()) throw std::invalid_argument("Linear: input/output rows differ");
    const int dt = gn_dtype(x.dtype, "Linear");
    const uint64_t W = n->saved_buffer_ids[0], b = n->num_saved > 1 ? n->saved_buffer_ids[1] : 0;
    if (!W) throw std::invalid_argument("Linear: saved_buffer_ids[0] must hold W");
    FusedSlot* f = fused_for(W);
    if (f && f->eligible && dt == GN_F32 && M > 0 && N > 0) {
        // the weight's optimizer step in this pass over W; dW is never stored
        uint64_t dX = x.requires_grad ? alloc_grad(x.size_bytes()) : 0;
        uint64_t db = b ? alloc_grad((size_t)N * 4) : 0;
        const size_t wsb = gn_linear_workspace_bytes(M, N, K, dt);
        const uint64_t ws = split_ws(wsb);
        const FusedUpdate& u = f->u;
        const int rc = gn_linear_bwd_surprise_momentum(
            gout(n), P(x.buffer_id), P(W), (float*)P(u.state), P(dX), P(db), M, N, K, u.eta,
            u.alpha, u.lambda, u.floor_, u.wd, u.clip, P(ws), wsb, dev_.stream());
        if (rc == GN_OK) {
            f->u.applied = true;
            stats_.shaders_dispatched += 2;
            n->grad_input_buffers[0] = dX;
            if (b) contribute(b, db, 0, (size_t)N, true);
            return;
        }
        if (rc != GN_E_INVALID) gn_call(rc, "Linear backward (fused surprise-momentum)");
        // a shape the fused kernel does not take: the usual backward below
    }
    if (Node* g = glu_before(n)) {
        // x = glu(gate, up) feeds only this node: the GLU's local gradients come out of the
        // input-gradient GEMM's epilogue for the FusedGLU node visited next (dX never formed)
        uint64_t gu = alloc_grad((size_t)2 * M * K * 2);
        uint64_t dW = alloc_grad((size_t)N * K * 4);
        uint64_t db = b ? alloc_grad((size_t)N * 4) : 0;
        const size_t wsb = gn_linear_workspace_bytes(M, N, K, dt);
        const uint64_t ws = split_ws(wsb);
        gn_call(gn_ffn_down_glu_bwd_ws((int)params_of<FusedGLUParams>(g).kind, gout(n),
                                       P(x.buffer_id), P(W), P(g->saved_buffer_ids[2]),
                                       P(g->saved_buffer_ids[3]), P(gu), P(dW), P(db), M, N, K, dt,
                                       0, P(ws), wsb, dev_.stream()),
                "Linear backward (GLU local gradients in the epilogue)");
        stats_.shaders_dispatched += 2;
        glu_node_ = g;
        glu_gu_ = gu;
        contribute(W, dW, 0, (size_t)N * K, true);
        if (b) contribute(b, db, 0, (size_t)N, true);
        return;
    }
    uint64_t dX = x.requires_grad ? alloc_grad(x.size_bytes()) : 0;
    uint64_t dW = alloc_grad((size_t)N * K * 4);
    uint64_t db = b ? alloc_grad((size_t)N * 4) : 0;
    const size_t wsb = gn_linear_workspace_bytes(M, N, K, dt);
    const uint64_t ws = split_ws(wsb);
    gn_call(gn_linear_bwd_ws(gout(n), P(x.buffer_id), P(W), P(dX), P(dW), P(db), M, N, K, dt, 0,
                             P(ws), wsb, dev_.stream()), "Linear backward");
    stats_.shaders_dispatched += db ? 3 : 2;
    n->grad_input_buffers[0] = dX;
    contribute(W, dW, 0, (size_t)N * K, true);
    if (b) contribute(b, db, 0, (size_t)N, true);
}

// Elementwise activations; tanh/sigmoid read the saved output (activation-tanh-backward.glsl:33).
void BackwardEngine::bwd_act(Node* n, int kind, bool uses_output) {
    const TensorRef& x = n->inputs[0];
    if (!x.requires_grad) return;
    const uint64_t src = uses_output ? n->outputs[0].buffer_id : x.buffer_id;
    uint64_t dX = alloc_grad(x.size_bytes());
    gn_call(gn_act_bwd(kind, gout(n), P(src), P(dX), (int64_t)x.numel(), gn_dtype(x.dtype, "activation"),
                       0, dev_.stream()), "activation backward");
    stats_.shaders_dispatched++;
    n->grad_input_buffers[0] = dX;
}

void BackwardEngine::bwd_softmax(Node* n) {
    const TensorRef& x = n->inputs[0];
    const TensorRef& y = n->outputs[0];
    if (!x.requires_grad) return;
    uint64_t dX = alloc_grad(x.size_bytes());
    gn_call(gn_softmax_bwd(gout(n), P(y.buffer_id), P(dX), (int)y.rows(), (int)y.last(),
                           gn_dtype(y.dtype, "Softmax"), dev_.stream()), "Softmax backward");
    stats_.shaders_dispatched++;
    n->grad_input_buffers[0] = dX;
}

// Output buffer of a norm's input gradient.  When the input already holds a gradient of the
// same dtype and size (the residual branch of a pre-norm block, recorded later on the tape and
// so visited first), the norm kernel adds it in its own pass (its dX_add): into that buffer
// when the engine owns it, else into a fresh buffer that replaces it.  The table is then up
// to date and the input is marked handled.  *add receives the addend (nullptr: none).
uint64_t BackwardEngine::norm_dx(Node* n, const void** add) {
    const TensorRef& x = n->inputs[0];
    *add = nullptr;
    GradEntry* e = (x.requires_grad && !writes_in_place(n, x.buffer_id)) ? find(x.buffer_id) : nullptr;
    if (e && e->grad_id && e->dtype == x.dtype && e->grad_bytes == x.size_bytes()) {
        *add = P(e->grad_id);
        if (!e->owned) {
            e->grad_id = alloc_grad(x.size_bytes());
            e->owned = true;
        }
        handled_ |= 1u;
        stats_.fanout_accumulations++;
        return e->grad_id;
    }
    return alloc_grad(x.size_bytes());
}

// A pre-norm block with its residual stream in fp32 records x = Add(x_prev, y_bf16) right
// before Norm(x): in the reverse walk the Add is the next node, and no other consumer of x is
// visited in between, so the norm's dX (with every earlier consumer's gradient summed in by
// norm_dx) is x's whole gradient, and the Add would convert it to bf16 for y.  The norm then
// writes that bf16 copy in its own pass: returns the copy's buffer (0: no copy wanted).
uint64_t BackwardEngine::bf16_copy_for(Node* n, uint64_t dX) {
    const TensorRef& x = n->inputs[0];
    const Node* a = n->prev_in_tape;
    if (!dX || !x.requires_grad || x.dtype != 0 /* f32 */ || !a || a->op != OpType::Add || a->num_outputs < 1 ||
        a->outputs[0].buffer_id != x.buffer_id || writes_in_place(n, x.buffer_id))
        return 0;
    // dX is x's whole gradient only when no earlier contribution is left to add after this node
    const GradEntry* e = find(x.buffer_id);
    if (!(handled_ & 1u) && e && e->grad_id) return 0;
    bool wants = false;
    for (uint32_t i = 0; i < a->num_inputs && i < kMaxNodeIO; ++i) {
        const TensorRef& in = a->inputs[i];
        wants = wants || (in.requires_grad && in.dtype == 4 /* bf16 */ && in.numel() == x.numel());
    }
    if (!wants) return 0;
    const uint64_t c = alloc_grad(x.numel() * 2);
    bf16_copies_.emplace_back(dX, c);
    return c;
}

// The FusedGLU node whose output is this Linear's input, when set_glu_epilogue is on and the
// fusion applies: bf16, the GLU recorded right before the Linear (so every other consumer of
// its output comes later on the tape and was visited first) and no gradient of that output
// in the table yet (no other consumer), so this node's contribution is the whole gradient.
Node* BackwardEngine::glu_before(Node* n) const {
    const TensorRef& x = n->inputs[0];
    Node* g = n->prev_in_tape;
    if (!glu_epilogue_ || !g || g->op != OpType::FusedGLU || !x.requires_grad || x.dtype != 4 /* bf16 */ ||
        g->num_inputs < 1 || g->num_outputs < 1 || g->num_saved < 4 || !g->saved_buffer_ids[2] ||
        !g->saved_buffer_ids[3] || g->outputs[0].buffer_id != x.buffer_id ||
        g->inputs[0].buffer_id == x.buffer_id || g->inputs[0].dtype != 4 ||
        g->outputs[0].numel() != x.numel() || g->outputs[0].last() != x.last() ||
        params_of<FusedGLUParams>(g).kind > GN_GLU_REGLU_UP)
        return nullptr;
    const GradEntry* e = find(x.buffer_id);
    return e && e->grad_id ? nullptr : g;
}

// saved: [0] gamma, [1] beta (or 0), [2] mean, [3] rstd (or var with stat_is_var).  x and its
// gradient may be fp32 under a bf16 output (a residual stream kept in fp32): dy and gamma take
// the output's dtype.
void BackwardEngine::bwd_layernorm(Node* n) {
    const TensorRef& x = n->inputs[0];
    const int rows = (int)x.rows(), F = (int)x.last();
    LayerNormParams p = params_of<LayerNormParams>(n);
    if (p.eps == 0.f) p.eps = 1e-5f;
    const uint64_t gamma = n->saved_buffer_ids[0], beta = n->saved_buffer_ids[1];
    const uint64_t mean = n->saved_buffer_ids[2], rstd = n->saved_buffer_ids[3];
    if (!gamma || !mean || !rstd) throw std::invalid_argument("LayerNorm: saved gamma/mean/rstd missing");
    const int xdt = gn_dtype(x.dtype, "LayerNorm");
    const int ydt = n->num_outputs ? gn_dtype(n->outputs[0].dtype, "LayerNorm output") : xdt;
    const void* add = nullptr;
    uint64_t dX = norm_dx(n, &add);
    uint64_t dG = alloc_grad((size_t)F * 4);
    uint64_t dB = beta ? alloc_grad((size_t)F * 4) : 0;
    const size_t wsb = gn_norm_workspace_bytes(rows, F);
    uint64_t ws = alloc_grad(wsb);
    const uint64_t dX16 = bf16_copy_for(n, dX);
    // the parameter gradients' finish is deferred to one launch for the whole pass (the call
    // refuses shapes off the row-kernel path, which then finish here)
    auto call = [&](unsigned fl) {
        fl |= p.stat_is_var ? GN_LN_STAT_VAR : 0;
        if (dX16)
            return gn_layernorm_bwd_ex16(gout(n), ydt, P(x.buffer_id), xdt, P(gamma), (const float*)P(mean),
                                         (const float*)P(rstd), add, P(dX), P(dX16), (float*)P(dG),
                                         (float*)P(dB), rows, F, p.eps, fl, P(ws), wsb, dev_.stream());
        return gn_layernorm_bwd_ex(gout(n), ydt, P(x.buffer_id), xdt, P(gamma), (const float*)P(mean),
                                   (const float*)P(rstd), add, P(dX), (float*)P(dG), (float*)P(dB), rows,
                                   F, p.eps, fl, P(ws), wsb, dev_.stream());
    };
    int rc = call(GN_NORM_PARTIALS);
    if (rc == GN_OK)
        norm_pending_.push_back(GnNormFinish{P(ws), (float*)P(dG), (float*)P(dB), rows, F, 1, 0});
    else if (rc == GN_E_INVALID)
        rc = call(0);
    gn_call(rc, "LayerNorm backward");
    stats_.shaders_dispatched += 2;
    if (x.requires_grad) n->grad_input_buffers[0] = dX;
    contribute(gamma, dG, 0, F, true);
    if (beta) contribute(beta, dB, 0, F, true);
}

// saved: [0] w, [1] the per-row statistic (fp32; rstd unless RMSNormParams names another
// form); dtypes as LayerNorm
void BackwardEngine::bwd_rmsnorm(Node* n) {
    const TensorRef& x = n->inputs[0];
    const int rows = (int)x.rows(), F = (int)x.last();
    RMSNormParams p = params_of<RMSNormParams>(n);
    if (p.eps == 0.f) p.eps = 1e-6f;
    if (p.stat_kind > 2) throw std::invalid_argument("RMSNorm: stat_kind must be 0, 1 or 2");
    const unsigned stat_flag = p.stat_kind == 1 ? GN_RMS_STAT_MEANSQ : p.stat_kind == 2 ? GN_RMS_STAT_RMS : 0u;
    const uint64_t w = n->saved_buffer_ids[0], rstd = n->saved_buffer_ids[1];
    if (!w || !rstd) throw std::invalid_argument("RMSNorm: saved w/rstd missing");
    const int xdt = gn_dtype(x.dtype, "RMSNorm");
    const int ydt = n->num_outputs ? gn_dtype(n->outputs[0].dtype, "RMSNorm output") : xdt;
    const void* add = nullptr;
    uint64_t dX = norm_dx(n, &add);
    uint64_t dW = alloc_grad((size_t)F * 4);
    const size_t wsb = gn_norm_workspace_bytes(rows, F);
    uint64_t ws = alloc_grad(wsb);
    auto call = [&](unsigned fl) {
        return gn_rmsnorm_bwd_stat(gout(n), ydt, P(x.buffer_id), xdt, P(w), (const float*)P(rstd), add,
                                   P(dX), (float*)P(dW), rows, F, p.eps, stat_flag | fl, P(ws), wsb,
                                   dev_.stream());
    };
    int rc = call(GN_NORM_PARTIALS);
    if (rc == GN_OK)
        norm_pending_.push_back(GnNormFinish{P(ws), (float*)P(dW), nullptr, rows, F, 0, 0});
    else if (rc == GN_E_INVALID)
        rc = call(0);
    gn_call(rc, "RMSNorm backward");
    stats_.shaders_dispatched += 2;
    if (x.requires_grad) n->grad_input_buffers[0] = dX;
    contribute(w, dW, 0, F, true);
}

// layout 0: inputs Q, K, V [B, H, S, D]; outputs[0] = O; saved[0] = LSE fp32 [B*H*S].
// layout 1: inputs[0] = fused QKV [B, S, 3*H*D]; outputs[0] = O [B, S, H*D]; the gradient
// of the fused buffer comes back in one [B, S, 3*H*D] buffer (dQ | dK | dV per row).
// An optional last input (inputs[3] in layout 0, inputs[1] in layout 1) is the reference's
// key-padding mask, fp32 [B, S] (flash-attention2.glsl:150-154); it gets no gradient.
static const float* attention_mask(const Node* n, uint32_t slot, int B, int S) {
    if (n->num_inputs <= slot || n->inputs[slot].buffer_id == 0) return nullptr;
    const TensorRef& m = n->inputs[slot];
    if (m.dtype != 0 || m.numel() != (uint64_t)B * S)
        throw std::invalid_argument("FlashAttention2: the key mask must be fp32 [B, S]");
    return static_cast<const float*>(P(m.buffer_id));
}

void BackwardEngine::bwd_attention(Node* n) {
    AttentionParams pa = params_of<AttentionParams>(n);
    if (pa.layout == 1) {
        const TensorRef& qkv = n->inputs[0];
        const TensorRef& o = n->outputs[0];
        if (qkv.ndim != 3 || o.ndim != 3 || pa.heads == 0)
            throw std::invalid_argument("FlashAttention2 (fused QKV): qkv [B,S,3HD], O [B,S,HD], heads > 0");
        const int B = (int)qkv.shape[0], S = (int)qkv.shape[1], H = (int)pa.heads;
        const int64_t C3 = qkv.shape[2], HD = o.shape[2];
        if (C3 != 3 * HD || HD % H != 0)
            throw std::invalid_argument("FlashAttention2 (fused QKV): qkv width must be 3 x O width");
        const int D = (int)(HD / H);
        const float scale = pa.scale != 0.f ? pa.scale : 1.0f / std::sqrt((float)D);
        const float theta = pa.rope_theta != 0.f ? pa.rope_theta : 10000.f;
        const uint64_t lse = n->saved_buffer_ids[0];
        if (!lse) throw std::invalid_argument("FlashAttention2: saved LSE missing");
        const size_t es = TensorRef::elem_size(qkv.dtype);
        uint64_t dqkv = alloc_grad(qkv.size_bytes());
        const size_t wsb = gn_attn_workspace_bytes_dtype(B, H, S, D, gn_dtype(qkv.dtype, "FlashAttention2"));
        uint64_t ws = alloc_grad(wsb);
        const char* base = static_cast<const char*>(P(qkv.buffer_id));
        char* gbase = static_cast<char*>(P(dqkv));
        const float* mask = attention_mask(n, 1, B, S);
        gn_call(gn_attn_bwd_bshd_mask(base, base + HD * es, base + 2 * HD * es, P(o.buffer_id),
                                      gout(n), (const float*)P(lse), mask, gbase, gbase + HD * es,
                                      gbase + 2 * HD * es, B, H, S, D, C3, HD, C3, scale,
                                      (int)pa.causal, (int)pa.rope_mode, theta,
                                      gn_dtype(qkv.dtype, "FlashAttention2"), P(ws), wsb,
                                      dev_.stream()), "attention backward (fused QKV)");
        stats_.shaders_dispatched += 3;
        n->grad_input_buffers[0] = dqkv;
        return;
    }
    const TensorRef& q = n->inputs[0];
    const TensorRef& k = n->inputs[1];
    const TensorRef& v = n->inputs[2];
    if (q.ndim < 3) throw std::invalid_argument("FlashAttention2: Q must be [B,H,S,D] or [H,S,D]");
    const int D = (int)q.shape[q.ndim - 1], S = (int)q.shape[q.ndim - 2];
    const int H = (int)q.shape[q.ndim - 3], B = q.ndim >= 4 ? (int)q.shape[q.ndim - 4] : 1;
    AttentionParams p = params_of<AttentionParams>(n);
    const float scale = p.scale != 0.f ? p.scale : 1.0f / std::sqrt((float)D);
    const float theta = p.rope_theta != 0.f ? p.rope_theta : 10000.f;
    const uint64_t lse = n->saved_buffer_ids[0];
    if (!lse) throw std::invalid_argument("FlashAttention2: saved LSE missing");
    uint64_t dQ = alloc_grad(q.size_bytes()), dK = alloc_grad(k.size_bytes()), dV = alloc_grad(v.size_bytes());
    const size_t wsb = gn_attn_workspace_bytes_dtype(B, H, S, D, gn_dtype(q.dtype, "FlashAttention2"));
    uint64_t ws = alloc_grad(wsb);
    const float* mask = attention_mask(n, 3, B, S);
    gn_call(gn_attn_bwd_mask(P(q.buffer_id), P(k.buffer_id), P(v.buffer_id),
                             P(n->outputs[0].buffer_id), gout(n), (const float*)P(lse), mask,
                             P(dQ), P(dK), P(dV), B, H, S, D, scale, (int)p.causal,
                             (int)p.rope_mode, theta, gn_dtype(q.dtype, "FlashAttention2"), P(ws),
                             wsb, dev_.stream()), "attention backward");
    stats_.shaders_dispatched += 3;
    n->grad_input_buffers[0] = dQ;
    n->grad_input_buffers[1] = dK;
    n->grad_input_buffers[2] = dV;
}

// cross-entropy-backward.glsl:29-84: softmax - onehot, scaled (default 1: no 1/B).  The
// loss is a root: like the reference shader it takes no upstream gradient.
void BackwardEngine::bwd_cross_entropy(Node* n) {
    const TensorRef& z = n->inputs[0];
    const TensorRef& t = n->inputs[1];
    if (!z.requires_grad) return;
    CrossEntropyParams p = params_of<CrossEntropyParams>(n);
    const float scale = p.has_scale ? p.scale : 1.0f;
    uint64_t dZ = alloc_grad(z.size_bytes());
    gn_call(gn_xent_bwd(P(z.buffer_id), (const int32_t*)P(t.buffer_id), P(dZ), (int)z.rows(),
                        (int)z.last(), scale, gn_dtype(z.dtype, "CrossEntropy"), dev_.stream()),
            "cross-entropy backward");
    stats_.shaders_dispatched++;
    n->grad_input_buffers[0] = dZ;
}

// Add: both inputs receive the upstream gradient itself (borrowed, copied on fan-out).  An
// input stored in another dtype than the sum (a bf16 branch added into an fp32 residual
// stream) receives the upstream gradient converted once to its own dtype.
void BackwardEngine::bwd_add_sub(Node* n, bool /*sub*/) {
    const uint64_t g = reinterpret_cast<uint64_t>(gout(n));
    const TensorRef& out = n->outputs[0];
    for (uint32_t i = 0; i < n->num_inputs && i < 2; ++i) {
        const TensorRef& in = n->inputs[i];
        if (!in.requires_grad) continue;
        if (in.numel() != out.numel())
            throw std::invalid_argument("Add: broadcasting inputs are not supported");
        if (in.dtype != out.dtype) {
            // the bf16 copy the norm visited just before wrote in its pass (bf16_copy_for);
            // taken once, so a second bf16 input gets its own buffer
            uint64_t c = 0;
            if (in.dtype == 4 /* bf16 */)
                for (auto& bc : bf16_copies_)
                    if (bc.first == g && bc.second) {
                        c = bc.second;
                        bc.second = 0;
                        break;
                    }
            if (!c) {
                c = alloc_grad(in.size_bytes());
                gn_call(gn_convert(P(g), gn_dtype(out.dtype, "Add output"), P(c), gn_dtype(in.dtype, "Add input"),
                                   (int64_t)in.numel(), dev_.stream()),
                        "Add backward (dtype conversion)");
                stats_.shaders_dispatched++;
            }
            n->grad_input_buffers[i] = c;
            continue;
        }
        n->grad_input_buffers[i] = g;
        borrowed_ |= 1u << i;
    }
}

void BackwardEngine::bwd_passthrough(Node* n) {
    if (!n->inputs[0].requires_grad) return;
    n->grad_input_buffers[0] = reinterpret_cast<uint64_t>(gout(n));
    borrowed_ |= 1u;
}

// backward_vsa_unpack_project (autograd.cpp:727-815): inputs[0] = bits [Bn, words] (or
// [words] for one row), outputs[0] = y [Bn, O]; saved[0] = W [O x D], saved[1] = b or 0.
void BackwardEngine::bwd_vsa_unpack_project(Node* n) {
    const TensorRef& bits = n->inputs[0];
    const TensorRef& y = n->outputs[0];
    const int words = (int)bits.last();
    const int Bn = bits.ndim >= 2 ? (int)bits.rows() : 1;
    const int O = (int)y.last(), D = words * 32;
    const uint64_t W = n->saved_buffer_ids[0], b = n->num_saved > 1 ? n->saved_buffer_ids[1] : 0;
    uint64_t dW = alloc_grad((size_t)O * D * 4);
    uint64_t db = b ? alloc_grad((size_t)O * 4) : 0;
    const int dt = gn_dtype(y.dtype, "VSAUnpackProject");
    const size_t wsb = gn_vsa_workspace_bytes(Bn, O);
    uint64_t ws = wsb ? alloc_grad(wsb) : 0;
    gn_call(gn_vsa_unpack_project_bwd(gout(n), (const uint32_t*)P(bits.buffer_id), (float*)P(dW),
                                      (float*)P(db), Bn, O, D, words, dt, 0, P(ws), wsb, dev_.stream()),
            "VSA unpack-project backward");
    stats_.shaders_dispatched += db ? 2 : 1;
    n->grad_input_buffers[0] = 0;  // bitpacked input: no gradient
    if (W) contribute(W, dW, 0, (size_t)O * D, true);
    if (b) contribute(b, db, 0, (size_t)O, true);
}

// backward_vsa_surrogate_loss (autograd.cpp:713-725): grad scale 1; saved[n-2] = results,
// saved[n-1] = weights (vsa_loss_node.cpp:156-159, 209-215).
void BackwardEngine::bwd_vsa_surrogate(Node* n) {
    VSASurrogateLossParams p = params_of<VSASurrogateLossParams>(n);
    const TensorRef& preds = n->inputs[0];
    const TensorRef& bits = n->inputs[1];
    if (n->num_saved < 2) throw std::invalid_argument("VSASurrogateLoss: results/weights not saved");
    const int Bn = (int)preds.shape[0];
    const int words = (int)((p.D + 31) / 32);
    uint64_t dP = alloc_grad((size_t)Bn * p.K * p.D * 4);
    gn_call(gn_vsa_surrogate_bwd((const float*)P(preds.buffer_id), (const uint32_t*)P(bits.buffer_id),
                                 (const uint32_t*)P(n->saved_buffer_ids[n->num_saved - 2]),
                                 (const float*)P(n->saved_buffer_ids[n->num_saved - 1]), (float*)P(dP),
                                 Bn, (int)p.K, (int)p.D, words, p.gamma, p.delta_margin, p.lambda,
                                 1.0f, 0, dev_.stream()), "VSA surrogate backward");
    stats_.shaders_dispatched++;
    n->grad_input_buffers[0] = dP;
}

// FusedGLU: inputs[0] = X [M x K]; outputs[0] = glu(gate, up) [M x H];
// saved: [0] Wg, [1] Wu, [2] gate, [3] up, [4] bg or 0, [5] bu or 0.
void BackwardEngine::bwd_fused_glu(Node* n) {
    const TensorRef& x = n->inputs[0];
    const TensorRef& y = n->outputs[0];
    const int M = (int)x.rows(), K = (int)x.last(), H = (int)y.last();
    const uint64_t* s = n->saved_buffer_ids;
    if (!s[0] || !s[1] || !s[2] || !s[3]) throw std::invalid_argument("FusedGLU: saved Wg/Wu/gate/up missing");
    const uint64_t bg = n->num_saved > 4 ? s[4] : 0, bu = n->num_saved > 5 ? s[5] : 0;
    const int dt = gn_dtype(x.dtype, "FusedGLU");
    const size_t es = TensorRef::elem_size(x.dtype);
    uint64_t dX = x.requires_grad ? alloc_grad(x.size_bytes()) : 0;
    uint64_t dWg = alloc_grad((size_t)H * K * 4), dWu = alloc_grad((size_t)H * K * 4);
    uint64_t dbg = bg ? alloc_grad((size_t)H * 4) : 0, dbu = bu ? alloc_grad((size_t)H * 4) : 0;
    const size_t wsb = gn_glu_workspace_bytes(M, K, H, dt);
    const uint64_t ws = split_ws(wsb);
    if (n == glu_node_) {
        // [dGate | dUp] from the down projection's epilogue (bwd_linear, set_glu_epilogue)
        gn_call(gn_glu_proj_bwd_ws(P(glu_gu_), P(x.buffer_id), P(s[0]), P(s[1]), P(dX), P(dWg),
                                   P(dWu), P(dbg), P(dbu), M, K, H, dt, 0, P(ws), wsb,
                                   dev_.stream()),
                "FusedGLU backward (projections)");
        glu_node_ = nullptr;
        glu_gu_ = 0;
        n->grad_output_buffer = 0;  // its output's gradient was never formed
        stats_.shaders_dispatched += 3;
    } else {
        uint64_t gu = alloc_grad((size_t)2 * M * H * es);
        gn_call(gn_glu_linear_bwd_ws((int)params_of<FusedGLUParams>(n).kind, gout(n), P(s[2]),
                                     P(s[3]), P(x.buffer_id), P(s[0]), P(s[1]), P(dX), P(dWg),
                                     P(dWu), P(dbg), P(dbu), P(gu), M, K, H, dt, 0, P(ws), wsb,
                                     dev_.stream()),
                "FusedGLU backward");
        stats_.shaders_dispatched += 4;
    }
    n->grad_input_buffers[0] = dX;
    contribute(s[0], dWg, 0, (size_t)H * K, true);
    contribute(s[1], dWu, 0, (size_t)H * K, true);
    if (bg) contribute(bg, dbg, 0, H, true);
    if (bu) contribute(bu, dbu, 0, H, true);
}

// Embedding: outputs[0] = rows of the table gathered by inputs[0] (int32 ids, T of them);
// saved[0] = the table [V x d].  dTable[id[t]] += dX[t] (fp32).  With a tied LM head the
// table already holds that head's dW in the gradient table: the rows are added into it.
void BackwardEngine::bwd_embedding(Node* n) {
    const TensorRef& ids = n->inputs[0];
    const TensorRef& x = n->outputs[0];
    const uint64_t table = n->saved_buffer_ids[0];
    if (!table) throw std::invalid_argument("Embedding: saved_buffer_ids[0] must hold the table");
    if (n->params_size < 4)
        throw std::invalid_argument("Embedding: params must hold the vocabulary size (uint32)");
    uint32_t V = 0;
    std::memcpy(&V, n->params, sizeof(V));
    const int T = (int)ids.numel(), d = (int)x.last();
    if ((size_t)T != x.rows()) throw std::invalid_argument("Embedding: one id per output row");
    GradEntry* e = find(table);
    const bool into = e && e->grad_id && e->owned && e->dtype == 0 &&
                      e->grad_bytes == (size_t)V * d * 4;
    uint64_t dE = into ? e->grad_id : alloc_grad((size_t)V * d * 4);
    gn_call(gn_embedding_bwd(gout(n), (const int32_t*)P(ids.buffer_id), (float*)P(dE), T, d, (int)V,
                             gn_dtype(x.dtype, "Embedding"), into ? GN_ACCUMULATE : 0u,
                             dev_.stream()), "embedding backward");
    stats_.shaders_dispatched += into ? 1 : 2;
    if (!into) contribute(table, dE, 0, (size_t)V * d, true);
}

// ═════════════════════════════════════════════════════════════════════ TapeContext

TapeContext::TapeContext(Device& dev, size_t arena_capacity)
    : dev_(dev), arena_(arena_capacity), engine_(dev) {}

uint64_t TapeContext::acquire_temp(size_t bytes) {
    uint64_t id = dev_.acquire(bytes);
    step_bufs_.push_back(id);
    return id;
}

void TapeContext::begin() {
    arena_.reset();
    engine_.clear_grads();
    seq_ = 0;
    recording_ = true;
}

// autograd.cpp:884-917
Node* TapeContext::record_op(OpType op, const TensorRef* inputs, uint32_t num_inputs,
                             const TensorRef* outputs, uint32_t num_outputs, const void* params,
                             uint32_t params_size) {
    if (!recording_) return nullptr;
    Node* node = arena_.allocate_node<Node>();
    node->op = op;
    node->seq = seq_++;
    node->num_inputs = std::min(num_inputs, kMaxNodeIO);
    node->num_outputs = std::min(num_outputs, kMaxNodeIO);
    node->num_saved = 0;
    node->grad_output_buffer = 0;
    node->params_size = 0;
    node->emotion[0] = node->emotion[1] = 0.f;
    std::memset(node->inputs, 0, sizeof(node->inputs));
    std::memset(node->outputs, 0, sizeof(node->outputs));
    std::memset(node->saved_buffer_ids, 0, sizeof(node->saved_buffer_ids));
    std::memset(node->grad_input_buffers, 0, sizeof(node->grad_input_buffers));
    std::memset(node->params, 0, sizeof(node->params));
    for (uint32_t i = 0; i < node->num_inputs; ++i) node->inputs[i] = inputs[i];
    for (uint32_t i = 0; i < node->num_outputs; ++i) node->outputs[i] = outputs[i];
    if (params && params_size > 0) {
        if (params_size > sizeof(node->params))
            throw std::invalid_argument("record_op: params larger than 64 bytes");
        std::memcpy(node->params, params, params_size);
        node->params_size = params_size;
    }
    return node;
}

void TapeContext::save_for_backward(Node* node, const uint64_t* ids, uint32_t count) {
    if (!node) return;
    for (uint32_t i = 0; i < count && i < kMaxNodeIO; ++i) node->saved_buffer_ids[i] = ids[i];
    node->num_saved = std::min(count, kMaxNodeIO);
}

void TapeContext::backward(Node* loss_node, uint64_t grad_output_buffer) {
    recording_ = false;
    engine_.backward(arena_, loss_node, grad_output_buffer);
}

std::vector<std::pair<uint64_t, uint64_t>> TapeContext::grads() const {
    std::vector<std::pair<uint64_t, uint64_t>> out;
    for (const auto& e : engine_.table_)
        if (e.buffer_id && e.grad_id) out.emplace_back(e.buffer_id, e.grad_id);
    return out;
}

void TapeContext::end() {
    for (uint64_t b : step_bufs_) dev_.release(b);
    step_bufs_.clear();
    for (uint64_t b : engine_.backward_bufs_) dev_.release(b);
    engine_.backward_bufs_.clear();
    arena_.reset();
    engine_.clear_grads();
    seq_ = 0;
    recording_ = false;
}

}  // namespace autograd
}  // namespace grilly

namespace grilly {
namespace autograd {

// Sub / Mul / Div / Neg (stubs at autograd.cpp:631-654): elementwise, no broadcasting.
// Sub's first input borrows the upstream buffer (backward_sub :632-633 does the same).
void BackwardEngine::bwd_binary(Node* n, int op) {
    const TensorRef& a = n->inputs[0];
    const bool two = op != GN_BIN_NEG;
    if (two && n->num_inputs < 2) throw std::invalid_argument("binary op: two inputs expected");
    const TensorRef* b = two ? &n->inputs[1] : nullptr;
    const size_t numel = n->outputs[0].numel();
    if (a.numel() != numel || (b && b->numel() != numel))
        throw std::invalid_argument("binary op: broadcasting inputs are not supported");
    if (b && b->dtype != a.dtype) throw std::invalid_argument("binary op: inputs differ in dtype");
    const int dt = gn_dtype(a.dtype, "binary op");
    const bool ga = a.requires_grad, gb = b && b->requires_grad;
    if (!ga && !gb) return;
    uint64_t dA = 0, dB = gb ? alloc_grad(b->size_bytes()) : 0;
    if (ga) {
        if (op == GN_BIN_SUB) {
            dA = reinterpret_cast<uint64_t>(gout(n));
            borrowed_ |= 1u;
        } else {
            dA = alloc_grad(a.size_bytes());
        }
    }
    const bool kernel_da = ga && op != GN_BIN_SUB;
    if (kernel_da || gb) {
        gn_call(gn_binary_bwd(op, gout(n), P(a.buffer_id), b ? P(b->buffer_id) : nullptr,
                              kernel_da ? P(dA) : nullptr, gb ? P(dB) : nullptr, (int64_t)numel, dt,
                              0, dev_.stream()),
                "binary op backward");
        stats_.shaders_dispatched++;
    }
    n->grad_input_buffers[0] = dA;
    if (gb) n->grad_input_buffers[1] = dB;
}

// Sum / Mean (stubs at autograd.cpp:695-707): a reduction over the trailing elements of the
// input, outputs[0].numel() rows of input.numel() / outputs[0].numel() each (a scalar output
// is the full reduction).
void BackwardEngine::bwd_reduce(Node* n, int op) {
    const TensorRef& x = n->inputs[0];
    if (!x.requires_grad) return;
    const size_t outer = n->outputs[0].numel(), total = x.numel();
    if (outer == 0 || total % outer != 0)
        throw std::invalid_argument("Sum/Mean: output size must divide the input size");
    uint64_t dX = alloc_grad(x.size_bytes());
    gn_call(gn_reduce_bwd(op, gout(n), P(dX), (int64_t)outer, (int64_t)(total / outer),
                          gn_dtype(x.dtype, "Sum/Mean"), 0, dev_.stream()),
            "Sum/Mean backward");
    stats_.shaders_dispatched++;
    n->grad_input_buffers[0] = dX;
}

// Transpose of the last two dims (stub at autograd.cpp:689-693).
void BackwardEngine::bwd_transpose(Node* n) {
    const TensorRef& x = n->inputs[0];
    if (!x.requires_grad) return;
    if (x.ndim < 2) throw std::invalid_argument("Transpose: input needs two dims or more");
    const int rows = (int)x.shape[x.ndim - 2], cols = (int)x.shape[x.ndim - 1];
    const int64_t batch = (int64_t)(x.numel() / ((size_t)rows * cols));
    uint64_t dX = alloc_grad(x.size_bytes());
    gn_call(gn_transpose_bwd(gout(n), P(dX), batch, rows, cols, gn_dtype(x.dtype, "Transpose"), 0,
                             dev_.stream()),
            "Transpose backward");
    stats_.shaders_dispatched++;
    n->grad_input_buffers[0] = dX;
}

// MSELoss (stub at autograd.cpp:663-667): inputs[0] = pred, inputs[1] = target; the upstream
// gradient is a scalar buffer (or the loss sentinel, read as 1).
void BackwardEngine::bwd_mse(Node* n) {
    const TensorRef& p = n->inputs[0];
    if (!p.requires_grad) return;
    if (n->num_inputs < 2 || n->inputs[1].numel() != p.numel())
        throw std::invalid_argument("MSELoss: target must match the prediction's size");
    MSELossParams mp = params_of<MSELossParams>(n);
    const float scale = mp.has_scale ? mp.scale : (float)(1.0 / (double)p.numel());
    const float* dL = n->grad_output_buffer > 1 ? (const float*)P(n->grad_output_buffer) : nullptr;
    uint64_t dP = alloc_grad(p.size_bytes());
    gn_call(gn_mse_bwd(P(p.buffer_id), P(n->inputs[1].buffer_id), dL, P(dP), (int64_t)p.numel(),
                       scale, gn_dtype(p.dtype, "MSELoss"), 0, dev_.stream()),
            "MSELoss backward");
    stats_.shaders_dispatched++;
    n->grad_input_buffers[0] = dP;
}

// MatMul (stub at autograd.cpp:543-549): C [M x N] = A [M x K] . B [K x N]:
// dA = dC B^T, dB = A^T dC, each in its input's dtype.
void BackwardEngine::bwd_matmul(Node* n) {
    if (n->num_inputs < 2) throw std::invalid_argument("MatMul: two inputs expected");
    const TensorRef& a = n->inputs[0];
    const TensorRef& b = n->inputs[1];
    const int M = (int)a.rows(), K = (int)a.last(), N = (int)b.last();
    if ((int)b.rows() != K || a.dtype != b.dtype)
        throw std::invalid_argument("MatMul: shapes [M x K] . [K x N] of one dtype expected");
    const int dt = gn_dtype(a.dtype, "MatMul");
    if (a.requires_grad) {
        uint64_t dA = alloc_grad(a.size_bytes());
        gn_call(gn_gemm(gout(n), P(b.buffer_id), N, nullptr, nullptr, 0, P(dA), M, K, 0, 1, dt, dt, 0,
                        dev_.stream()),
                "MatMul dA");
        stats_.shaders_dispatched++;
        n->grad_input_buffers[0] = dA;
    }
    if (b.requires_grad) {
        uint64_t dB = alloc_grad(b.size_bytes());
        gn_call(gn_gemm(P(a.buffer_id), gout(n), M, nullptr, nullptr, 0, P(dB), K, N, 1, 0, dt, dt, 0,
                        dev_.stream()),
                "MatMul dB");
        stats_.shaders_dispatched++;
        n->grad_input_buffers[1] = dB;
    }
}

// backward_vsa_lora_expand (autograd.cpp:817-843): inputs[0] = coefficients [Bn, K*rank]
// (or [Bn, K, rank]); saved[0] = basis B [D x rank], saved[1] = coefficients.  The
// coefficient gradient flows to inputs[0]; the basis gradient goes to the table under the
// basis id (for the optimizer), as the reference does.
void BackwardEngine::bwd_vsa_lora_expand(Node* n) {
    VSALoRAExpandParams p = params_of<VSALoRAExpandParams>(n);
    if (n->num_saved < 2 || !n->saved_buffer_ids[0] || !n->saved_buffer_ids[1])
        throw std::invalid_argument("VSALoRAExpand: saved basis/coefficients missing");
    const int Bn = (int)n->inputs[0].shape[0];
    uint64_t dC = alloc_grad((size_t)Bn * p.K * p.rank * 4);
    uint64_t dB = alloc_grad((size_t)p.D * p.rank * 4);
    gn_call(gn_vsa_lora_expand_bwd((const float*)gout(n), (const float*)P(n->saved_buffer_ids[0]),
                                   (const float*)P(n->saved_buffer_ids[1]), (float*)P(dC), (float*)P(dB),
                                   Bn, (int)p.K, (int)p.D, (int)p.rank, 1.0f, 0, dev_.stream()),
            "VSA LoRA-expand backward");
    stats_.shaders_dispatched += 2;
    n->grad_input_buffers[0] = dC;
    contribute(n->saved_buffer_ids[0], dB, 0, (size_t)p.D * p.rank, true);
}

// backward_vsa_cosine_blend_loss (autograd.cpp:845-859): inputs[0] = preds [Bn, K, D],
// inputs[1] = true bits; saved [n-3] = router weights, [n-2] = blended, [n-1] = loss_info;
// grad_scale 10 on a zeroed buffer.
void BackwardEngine::bwd_vsa_cosine_blend(Node* n) {
    VSACosineBlendLossParams p = params_of<VSACosineBlendLossParams>(n);
    if (n->num_saved < 3) throw std::invalid_argument("VSACosineBlendLoss: weights/blended/loss_info not saved");
    const int Bn = (int)n->inputs[0].shape[0];
    const int words = (int)((p.D + 31) / 32);
    uint64_t dP = alloc_grad((size_t)Bn * p.K * p.D * 4);
    const uint64_t* s = n->saved_buffer_ids + n->num_saved - 3;
    gn_call(gn_vsa_cosine_blend_bwd((const uint32_t*)P(n->inputs[1].buffer_id), (const float*)P(s[0]),
                                    (const float*)P(s[1]), (const float*)P(s[2]), (float*)P(dP), Bn,
                                    (int)p.K, (int)p.D, words, 10.0f, 0, dev_.stream()),
            "VSA cosine-blend backward");
    stats_.shaders_dispatched++;
    n->grad_input_buffers[0] = dP;
}

// backward_cubemind_surprise / backward_temporal_surprise (autograd.cpp:669-685): the
// gradient passes through unchanged and the node's params are overwritten with the
// multiplier (1 + alpha surprise, or clamp(temporal_multiplier alpha, -1, 1)) for the caller.
void BackwardEngine::bwd_surprise_passthrough(Node* n) {
    if (!n->inputs[0].requires_grad) return;
    float mult;
    if (n->op == OpType::CubeMindSurprise) {
        float alpha = 0.5f;
        if (n->params_size >= sizeof(float)) std::memcpy(&alpha, n->params, sizeof(float));
        mult = 1.0f + alpha * n->emotion[0];
    } else {
        TemporalSurpriseParams t = params_of<TemporalSurpriseParams>(n);
        mult = std::min(1.0f, std::max(-1.0f, t.temporal_multiplier * t.alpha));
    }
    std::memcpy(n->params, &mult, sizeof(float));
    n->params_size = sizeof(float);
    n->grad_input_buffers[0] = reinterpret_cast<uint64_t>(gout(n));
    borrowed_ |= 1u;
    stats_.shaders_dispatched++;
}

}  // namespace autograd
}  // namespace grilly
