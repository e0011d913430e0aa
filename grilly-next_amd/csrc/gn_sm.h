// gn_sm.h — one element of the reference's surprise-momentum update
// (surprise-momentum.glsl:53-114), shared by the optimizer stream (gn_optim.hip) and the
// skinny Linear backward that applies the update as it forms the weight gradient
// (gn_skinny.hip), so both paths run the same instructions on the same values.
#pragma once

#include "gn_common.h"

namespace gn {

struct SmHyper {
    float eta, alpha, lambda, floor_, wd, clip;
    int clear;
};

__device__ __forceinline__ bool sm_finite(float x) { return !(isnan(x) || isinf(x)); }

// g: gradient, r: recalled gradient (0 when the caller has none); s_bar: surprise state,
// w: weight (both updated in place); d_out: the applied step (the reference's delta scratch)
__device__ __forceinline__ void sm_elem(const SmHyper& h, float g, float r, float& s_bar, float& w,
                                        float& d_out) {
    // every product and sum rounded on its own (no fused multiply-adds): the compiler would
    // otherwise pick contractions per call site, and the two kernels sharing this function
    // must produce the same bits
#pragma clang fp contract(off)
    if (!sm_finite(g) || !sm_finite(r)) {
        d_out = 0.f;
        return;  // W and s_bar unchanged
    }
    const float g_eff = g + h.lambda * r;
    const float pe = fabsf(g - r);
    float s_prev = s_bar;
    if (!sm_finite(s_prev)) s_prev = 0.f;
    float s_new = h.alpha * pe + (1.0f - h.alpha) * s_prev;
    s_new = fminf(s_new, 5.0f);
    s_bar = s_new;
    const float lr = h.eta * (1.0f + fmaxf(s_new, h.floor_));
    float d = lr * g_eff;
    d += h.eta * h.wd * w;
    d = fminf(fmaxf(d, -h.clip), h.clip);
    float w_new = w - d;
    if (!sm_finite(w_new)) w_new = 0.f;
    w = fminf(fmaxf(w_new, -10.0f), 10.0f);
    d_out = d;
}

}  // namespace gn
