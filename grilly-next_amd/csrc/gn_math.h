// gn_math.h — activation and GLU derivatives shared by the elementwise kernels and the
// GEMM epilogues (formulas from the reference shaders cited at each function).
#pragma once

#include "gn_common.h"

namespace gn {

// ---- activation derivatives --------------------------------------------------------------
constexpr float kSqrt2OverPi = 0.7978845608028654f;
constexpr float kGeluC = 0.044715f;

__device__ __forceinline__ float gelu_tanh_f(float x) {
    return 0.5f * x * (1.0f + tanhf_(kSqrt2OverPi * (x + kGeluC * x * x * x)));
}
// activation-gelu-backward.glsl:38-50: 0.5 (1 + tanh z + x sech^2 z dz/dx)
__device__ __forceinline__ float gelu_tanh_grad_f(float x) {
    float z = kSqrt2OverPi * (x + kGeluC * x * x * x);
    float t = tanhf_(z);
    return 0.5f * (1.0f + t + x * (1.0f - t * t) * kSqrt2OverPi * (1.0f + 3.0f * kGeluC * x * x));
}
// erf form (autograd_core.py:529-542): Phi(x) + x phi(x)
__device__ __forceinline__ float gelu_erf_grad_f(float x) {
    return 0.5f * (1.0f + erff(x * 0.70710678118654752f)) +
           x * 0.3989422804014327f * __expf(-0.5f * x * x);
}
__device__ __forceinline__ float silu_f(float x) { return x * sigmoidf_(x); }
__device__ __forceinline__ float silu_grad_f(float x) {
    float s = sigmoidf_(x);
    return s * (1.0f + x * (1.0f - s));
}

template <int KIND>
__device__ __forceinline__ float act_grad(float x) {
    if constexpr (KIND == GN_ACT_RELU) return x > 0.0f ? 1.0f : 0.0f;
    else if constexpr (KIND == GN_ACT_GELU_TANH) return gelu_tanh_grad_f(x);
    else if constexpr (KIND == GN_ACT_GELU_ERF) return gelu_erf_grad_f(x);
    else if constexpr (KIND == GN_ACT_SILU) return silu_grad_f(x);
    else if constexpr (KIND == GN_ACT_TANH) return 1.0f - x * x;  // x = saved tanh output
    else return x * (1.0f - x);                                    // x = saved sigmoid output
}

// ---- GLU local gradients (fused-{swiglu,geglu,reglu}-backward.glsl local terms) ---------
template <int KIND>
__device__ __forceinline__ void glu_grad(float d, float g, float u, float& dg, float& du) {
    if constexpr (KIND == GN_GLU_SWIGLU_UP) {
        float s = sigmoidf_(u);
        dg = d * u * s;
        du = d * g * s * (1.0f + u * (1.0f - s));
    } else if constexpr (KIND == GN_GLU_SWIGLU_GATE) {
        float s = sigmoidf_(g);
        dg = d * u * s * (1.0f + g * (1.0f - s));
        du = d * g * s;
    } else if constexpr (KIND == GN_GLU_GEGLU_UP) {
        dg = d * gelu_tanh_f(u);
        du = d * g * gelu_tanh_grad_f(u);
    } else if constexpr (KIND == GN_GLU_GEGLU_GATE) {
        dg = d * u * gelu_tanh_grad_f(g);
        du = d * gelu_tanh_f(g);
    } else {  // REGLU_UP
        dg = d * (u > 0.0f ? u : 0.0f);
        du = d * g * (u > 0.0f ? 1.0f : 0.0f);
    }
}

// ---- GLU forward value (fused-swiglu.glsl:78, fused-geglu.glsl:81, fused-reglu.glsl:73) ------
template <int KIND>
__device__ __forceinline__ float glu_val(float g, float u) {
    if constexpr (KIND == GN_GLU_SWIGLU_UP) return g * silu_f(u);
    else if constexpr (KIND == GN_GLU_SWIGLU_GATE) return silu_f(g) * u;
    else if constexpr (KIND == GN_GLU_GEGLU_UP) return g * gelu_tanh_f(u);
    else if constexpr (KIND == GN_GLU_GEGLU_GATE) return gelu_tanh_f(g) * u;
    else return g * (u > 0.0f ? u : 0.0f);  // REGLU_UP
}

}  // namespace gn
