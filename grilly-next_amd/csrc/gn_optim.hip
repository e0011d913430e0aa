// gn_optim.hip — optimizer steps applied between the tape's backward and end: the
// reference's surprise-momentum.glsl (used by vsa_training_step, bindings.cpp:3198-3277) and
// adamw-update.glsl.  Both are pure streams over fp32 parameter state (HBM-bound: 28-34 bytes
// per element), so one launch covers up to kOptMaxT tensors: the host packs the pointers and a
// prefix table of block counts into the kernel argument, each block finds its tensor in that
// table, and each thread moves one 16-byte vector of every stream (a scalar tail covers n % 4
// and unaligned tensors).  The streams are touched once, so loads and stores are
// non-temporal (measured on MI355X over the decoder's 138 M parameters: 4.8 TB/s with
// cached accesses and two vectors per thread, 5.6 TB/s like this).  The reference
// dispatches one pipeline per tensor and 128 MB chunk.
#include <algorithm>

#include "gn_common.h"
#include "gn_sm.h"

namespace gn {
namespace {

constexpr int kOptMaxT = 24;
constexpr int kOptThreads = 256;
constexpr int kOptVec = 4;                                  // elements per vector access
constexpr int kOptChunk = kOptThreads * kOptVec;            // elements per block

struct OptBatch {
    gn_opt_param p[kOptMaxT];
    int bstart[kOptMaxT + 1];  // first block of each tensor; bstart[count] = grid size
    int vec[kOptMaxT];         // 1: every pointer of the tensor is 16-byte aligned
    int count;
};

struct AdamHyper {
    float lr, b1, b2, eps, wd, b1t, b2t;
    int clear;
};

// adamw-update.glsl:41-61 for one element
__device__ __forceinline__ void adamw_elem(const AdamHyper& h, float g, float& m, float& v, float& w) {
    const float m_new = h.b1 * m + (1.0f - h.b1) * g;
    const float v_new = h.b2 * v + (1.0f - h.b2) * g * g;
    m = m_new;
    v = v_new;
    const float m_hat = m_new / fmaxf(1e-12f, 1.0f - h.b1t);
    const float v_hat = v_new / fmaxf(1e-12f, 1.0f - h.b2t);
    const float decayed = w * (1.0f - h.lr * h.wd);
    w = decayed - h.lr * m_hat / (sqrtf(fmaxf(v_hat, 0.0f)) + h.eps);
}

__device__ __forceinline__ int find_tensor(const OptBatch& b) {
    int t = 0;
    while (t + 1 < b.count && (int)blockIdx.x >= b.bstart[t + 1]) ++t;
    return t;
}

typedef float vf4 __attribute__((ext_vector_type(4)));
typedef uint32_t vu2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float4 ld4(const float* p) {
    const vf4 v = __builtin_nontemporal_load(reinterpret_cast<const vf4*>(p));
    return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void st4(float* p, const float (&v)[4]) {
    const vf4 x = {v[0], v[1], v[2], v[3]};
    __builtin_nontemporal_store(x, reinterpret_cast<vf4*>(p));
}
__device__ __forceinline__ void st4_bf16(void* p, int64_t i, const float (&w)[4]) {
    const vu2 x = {pack_bf2(w[0], w[1]), pack_bf2(w[2], w[3])};
    __builtin_nontemporal_store(x, reinterpret_cast<vu2*>(reinterpret_cast<bf16_t*>(p) + i));
}

__global__ __launch_bounds__(kOptThreads) void surprise_momentum_kernel(OptBatch b, SmHyper h) {
    const int t = find_tensor(b);
    const gn_opt_param p = b.p[t];
    const int64_t i = (int64_t)(blockIdx.x - b.bstart[t]) * kOptChunk + (int64_t)threadIdx.x * kOptVec;
    if (i >= p.n) return;
    if (b.vec[t] && i + kOptVec <= p.n) {
        const float4 g4 = ld4(p.grad + i), s4 = ld4(p.state0 + i), w4 = ld4(p.W + i);
        const float4 r4 = p.recalled ? ld4(p.recalled + i) : make_float4(0.f, 0.f, 0.f, 0.f);
        const float g[4] = {g4.x, g4.y, g4.z, g4.w}, r[4] = {r4.x, r4.y, r4.z, r4.w};
        float s[4] = {s4.x, s4.y, s4.z, s4.w}, w[4] = {w4.x, w4.y, w4.z, w4.w}, d[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) sm_elem(h, g[e], r[e], s[e], w[e], d[e]);
        st4(p.state0 + i, s);
        st4(p.W + i, w);
        if (p.state1) st4(p.state1 + i, d);
        if (p.W_bf16) st4_bf16(p.W_bf16, i, w);
        if (h.clear) {
            const float z[4] = {0.f, 0.f, 0.f, 0.f};
            st4(p.grad + i, z);
        }
    } else {
        for (int64_t k = i; k < min(i + (int64_t)kOptVec, p.n); ++k) {
            float s = p.state0[k], w = p.W[k], d;
            sm_elem(h, p.grad[k], p.recalled ? p.recalled[k] : 0.f, s, w, d);
            p.state0[k] = s;
            p.W[k] = w;
            if (p.state1) p.state1[k] = d;
            if (p.W_bf16) reinterpret_cast<bf16_t*>(p.W_bf16)[k] = f2bf(w);
            if (h.clear) p.grad[k] = 0.f;
        }
    }
}

__global__ __launch_bounds__(kOptThreads) void adamw_kernel(OptBatch b, AdamHyper h) {
    const int t = find_tensor(b);
    const gn_opt_param p = b.p[t];
    const int64_t i = (int64_t)(blockIdx.x - b.bstart[t]) * kOptChunk + (int64_t)threadIdx.x * kOptVec;
    if (i >= p.n) return;
    if (b.vec[t] && i + kOptVec <= p.n) {
        const float4 g4 = ld4(p.grad + i), m4 = ld4(p.state0 + i), v4 = ld4(p.state1 + i);
        const float4 w4 = ld4(p.W + i);
        const float g[4] = {g4.x, g4.y, g4.z, g4.w};
        float m[4] = {m4.x, m4.y, m4.z, m4.w}, v[4] = {v4.x, v4.y, v4.z, v4.w};
        float w[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) adamw_elem(h, g[e], m[e], v[e], w[e]);
        st4(p.state0 + i, m);
        st4(p.state1 + i, v);
        st4(p.W + i, w);
        if (p.W_bf16) st4_bf16(p.W_bf16, i, w);
        if (h.clear) {
            const float z[4] = {0.f, 0.f, 0.f, 0.f};
            st4(p.grad + i, z);
        }
    } else {
        for (int64_t k = i; k < min(i + (int64_t)kOptVec, p.n); ++k) {
            float m = p.state0[k], v = p.state1[k], w = p.W[k];
            adamw_elem(h, p.grad[k], m, v, w);
            p.state0[k] = m;
            p.state1[k] = v;
            p.W[k] = w;
            if (p.W_bf16) reinterpret_cast<bf16_t*>(p.W_bf16)[k] = f2bf(w);
            if (h.clear) p.grad[k] = 0.f;
        }
    }
}

inline bool al16p(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Validate and pack up to kOptMaxT tensors per launch; `launch(batch, grid)` issues one kernel.
template <typename L>
int run_batches(const gn_opt_param* params, int count, bool adam, const char* what, hipStream_t s,
                L&& launch) {
    GN_REQUIRE(count >= 0, "%s: count %d", what, count);
    GN_REQUIRE(count == 0 || params, "%s: null parameter array", what);
    for (int i = 0; i < count; ++i) {
        const gn_opt_param& p = params[i];
        GN_REQUIRE(p.n >= 0, "%s: tensor %d has n = %lld", what, i, (long long)p.n);
        if (p.n == 0) continue;
        GN_REQUIRE(p.W && p.grad && p.state0, "%s: tensor %d: W, grad and state0 are required", what, i);
        GN_REQUIRE(!adam || p.state1, "%s: tensor %d: AdamW needs state1 (v)", what, i);
        GN_REQUIRE(p.n <= ((int64_t)1 << 40), "%s: tensor %d too large", what, i);
    }
    OptBatch b{};
    auto flush = [&]() -> int {
        if (b.count == 0) return GN_OK;
        const int grid = b.bstart[b.count];
        if (grid > 0) launch(b, grid);
        GN_LAUNCH_CHECK(what);
        b = OptBatch{};
        return GN_OK;
    };
    for (int i = 0; i < count; ++i) {
        const gn_opt_param& p = params[i];
        if (p.n == 0) continue;
        const int64_t blocks = (p.n + kOptChunk - 1) / kOptChunk;
        if (b.count == kOptMaxT || (int64_t)b.bstart[b.count] + blocks > INT32_MAX / 2) {
            int rc = flush();
            if (rc) return rc;
        }
        const int t = b.count;
        b.p[t] = p;
        b.vec[t] = al16p(p.W) && al16p(p.grad) && al16p(p.state0) &&
                   (!p.state1 || al16p(p.state1)) && (!p.recalled || al16p(p.recalled)) &&
                   (!p.W_bf16 || (reinterpret_cast<uintptr_t>(p.W_bf16) & 7u) == 0);
        b.bstart[t + 1] = b.bstart[t] + (int)blocks;
        b.count = t + 1;
    }
    return flush();
}

}  // namespace
}  // namespace gn

using namespace gn;

extern "C" int gn_surprise_momentum_step(const gn_opt_param* params, int count, float eta_base,
                                         float alpha_momentum, float lambda_recall,
                                         float surprise_floor, float weight_decay, float clip_max,
                                         int clear_grad, void* stream) {
    clear_error();
    hipStream_t s = as_stream(stream);
    const SmHyper h{eta_base, alpha_momentum, lambda_recall, surprise_floor, weight_decay, clip_max,
                    clear_grad ? 1 : 0};
    return run_batches(params, count, false, "gn_surprise_momentum_step", s,
                       [&](const OptBatch& b, int grid) {
                           surprise_momentum_kernel<<<grid, kOptThreads, 0, s>>>(b, h);
                       });
}

extern "C" int gn_adamw_step(const gn_opt_param* params, int count, float lr, float beta1,
                             float beta2, float eps, float weight_decay, float beta1_t,
                             float beta2_t, int clear_grad, void* stream) {
    clear_error();
    hipStream_t s = as_stream(stream);
    const AdamHyper h{lr, beta1, beta2, eps, weight_decay, beta1_t, beta2_t, clear_grad ? 1 : 0};
    return run_batches(params, count, true, "gn_adamw_step", s, [&](const OptBatch& b, int grid) {
        adamw_kernel<<<grid, kOptThreads, 0, s>>>(b, h);
    });
}
