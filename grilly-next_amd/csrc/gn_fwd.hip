// gn_fwd.hip — forward kernels that produce the tensors the backward consumes:
//   LayerNorm / RMSNorm forward with their fp32 row statistics, the GLU product, and
//   Linear (X W^T + b) / fused GLU projections on the GEMM core.
//
// Norms: one wave per row, the row held in registers as 8-element chunks (chunk c = lane +
// 64 j), mean and variance from the registers (two reductions, no second read of x), so x
// is read once and y written once: HBM-bound at 2 x rows x F x sizeof(T) bytes.
#include "gn_common.h"
#include "gn_gemm_dma.h"
#include "gn_math.h"

namespace gn {
namespace {

constexpr int kFwdWaves = 4;  // rows per 256-thread block on the register path

// MODE 0 = LayerNorm (fnn-layernorm.glsl:44-102: mean, biased variance, (x-mean)/sqrt(var+eps)
// * gamma + beta), MODE 1 = RMSNorm (rms-norm.glsl:34-70: x * rsqrt(mean(x^2)+eps) * w).
// Row statistics: mean[r] (LayerNorm) and stat[r] by `save_var`: 0 = rstd, 1 = the variance
// (LayerNorm's var_vals) or mean(x^2) (RMSNorm, rms-norm.glsl:52), 2 = sqrt(mean(x^2) + eps)
// (snn-rmsnorm.glsl:55).
// TX: x (a residual stream may be fp32); TY: gamma, beta and y.
template <int MODE, typename TX, typename TY, int NC>
__global__ __launch_bounds__(64 * kFwdWaves) void norm_fwd_rows(
    const TX* __restrict__ X, const TY* __restrict__ gamma, const TY* __restrict__ beta,
    TY* __restrict__ Y, float* __restrict__ mean, float* __restrict__ stat, int rows, int F,
    float eps, int save_var) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * kFwdWaves + (threadIdx.x >> 6);
    if (r >= rows) return;  // whole waves leave together
    const int nchunks = F >> 3;
    const size_t off = (size_t)r * F;
    float x[NC][8];
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int c = lane + 64 * j;
        if (c < nchunks) chunk8<TX>::ld(X + off + 8 * c, x[j]);
        else
#pragma unroll
            for (int e = 0; e < 8; ++e) x[j][e] = 0.f;
    }
    const float invF = 1.0f / (float)F;
    float mu = 0.f;
    if (MODE == 0) {
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < NC; ++j)
#pragma unroll
            for (int e = 0; e < 8; ++e) s += x[j][e];
        mu = wave_sum(s) * invF;
    }
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        if (lane + 64 * j >= nchunks) continue;  // padding chunks hold 0, not mu
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float d = x[j][e] - mu;
            q += d * d;
        }
    }
    const float var = wave_sum(q) * invF;  // RMSNorm: mean(x^2)
    const float rs = rsqrtf(var + eps);
    if (lane == 0) {
        if (MODE == 0 && mean) mean[r] = mu;
        if (stat) stat[r] = save_var == 1 ? var : save_var == 2 ? sqrtf(var + eps) : rs;
    }
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int c = lane + 64 * j;
        if (c >= nchunks) continue;
        float g[8], b[8], y[8];
        if (gamma) chunk8<TY>::ld(gamma + 8 * c, g);
        else
#pragma unroll
            for (int e = 0; e < 8; ++e) g[e] = 1.f;
        if (MODE == 0 && beta) chunk8<TY>::ld(beta + 8 * c, b);
        else
#pragma unroll
            for (int e = 0; e < 8; ++e) b[e] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e)
            y[e] = MODE == 0 ? (x[j][e] - mu) * rs * g[e] + b[e] : g[e] * x[j][e] * rs;
        chunk8<TY>::st(Y + off + 8 * c, y);
    }
}

// Any F / alignment: one 256-thread block per row, two passes over the row in global memory.
template <int MODE, typename TX, typename TY>
__global__ __launch_bounds__(256) void norm_fwd_generic(
    const TX* __restrict__ X, const TY* __restrict__ gamma, const TY* __restrict__ beta,
    TY* __restrict__ Y, float* __restrict__ mean, float* __restrict__ stat, int F, float eps,
    int save_var) {
    __shared__ float sh[4];
    const int r = blockIdx.x;
    const size_t off = (size_t)r * F;
    const float invF = 1.0f / (float)F;
    float mu = 0.f;
    if (MODE == 0) {
        float s = 0.f;
        for (int f = threadIdx.x; f < F; f += 256) s += io<TX>::ld(X, off + f);
        mu = block_sum<4>(s, sh) * invF;
    }
    float q = 0.f;
    for (int f = threadIdx.x; f < F; f += 256) {
        const float d = io<TX>::ld(X, off + f) - mu;
        q += d * d;
    }
    const float var = block_sum<4>(q, sh) * invF;
    const float rs = rsqrtf(var + eps);
    if (threadIdx.x == 0) {
        if (MODE == 0 && mean) mean[r] = mu;
        if (stat) stat[r] = save_var == 1 ? var : save_var == 2 ? sqrtf(var + eps) : rs;
    }
    for (int f = threadIdx.x; f < F; f += 256) {
        const float x = io<TX>::ld(X, off + f);
        const float g = gamma ? io<TY>::ld(gamma, f) : 1.f;
        const float b = (MODE == 0 && beta) ? io<TY>::ld(beta, f) : 0.f;
        io<TY>::st(Y, off + f, MODE == 0 ? (x - mu) * rs * g + b : g * x * rs);
    }
}

inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <int MODE, typename TX, typename TY>
int norm_fwd(const void* X, const void* gamma, const void* beta, void* Y, float* mean,
             float* stat, int rows, int F, float eps, int save_var, hipStream_t s) {
    const bool vec_ok = F % 8 == 0 && F <= 2048 && al16(X) && al16(Y) && (!gamma || al16(gamma)) &&
                        (!beta || al16(beta));
    const TX* x = (const TX*)X;
    const TY* g = (const TY*)gamma;
    const TY* b = (const TY*)beta;
    TY* y = (TY*)Y;
    if (vec_ok) {
        const unsigned grid = (unsigned)((rows + kFwdWaves - 1) / kFwdWaves);
        const int nc = (F / 8 + 63) / 64;
        switch (nc) {
            case 1: norm_fwd_rows<MODE, TX, TY, 1><<<grid, 64 * kFwdWaves, 0, s>>>(x, g, b, y, mean, stat, rows, F, eps, save_var); break;
            case 2: norm_fwd_rows<MODE, TX, TY, 2><<<grid, 64 * kFwdWaves, 0, s>>>(x, g, b, y, mean, stat, rows, F, eps, save_var); break;
            case 3: norm_fwd_rows<MODE, TX, TY, 3><<<grid, 64 * kFwdWaves, 0, s>>>(x, g, b, y, mean, stat, rows, F, eps, save_var); break;
            default: norm_fwd_rows<MODE, TX, TY, 4><<<grid, 64 * kFwdWaves, 0, s>>>(x, g, b, y, mean, stat, rows, F, eps, save_var); break;
        }
    } else {
        norm_fwd_generic<MODE, TX, TY><<<rows, 256, 0, s>>>(x, g, b, y, mean, stat, F, eps, save_var);
    }
    GN_LAUNCH_CHECK(MODE == 0 ? "gn_layernorm_fwd" : "gn_rmsnorm_fwd");
    return GN_OK;
}

// (x, y) dtype pairs: both fp32, both bf16, or fp32 x under a bf16 y
template <int MODE>
int norm_fwd_dispatch(int x_dtype, int y_dtype, const void* X, const void* gamma, const void* beta,
                      void* Y, float* mean, float* stat, int rows, int F, float eps, int save_var,
                      hipStream_t s) {
    if (x_dtype == GN_F32 && y_dtype == GN_F32)
        return norm_fwd<MODE, float, float>(X, gamma, beta, Y, mean, stat, rows, F, eps, save_var, s);
    if (x_dtype == GN_BF16 && y_dtype == GN_BF16)
        return norm_fwd<MODE, bf16_t, bf16_t>(X, gamma, beta, Y, mean, stat, rows, F, eps, save_var, s);
    if (x_dtype == GN_F32 && y_dtype == GN_BF16)
        return norm_fwd<MODE, float, bf16_t>(X, gamma, beta, Y, mean, stat, rows, F, eps, save_var, s);
    set_error("%s: x dtype %d with y dtype %d not supported (f32/f32, bf16/bf16, f32/bf16)",
              MODE == 0 ? "gn_layernorm_fwd" : "gn_rmsnorm_fwd", x_dtype, y_dtype);
    return GN_E_INVALID;
}

// out = glu(gate, up) elementwise; 8 elements per step through 16-byte accesses when VEC.
template <int KIND, typename T, bool VEC>
__global__ __launch_bounds__(256) void glu_fwd_kernel(const T* __restrict__ gate,
                                                      const T* __restrict__ up,
                                                      T* __restrict__ out, int64_t n) {
    const int64_t gid = blockIdx.x * (int64_t)256 + threadIdx.x, stride = (int64_t)gridDim.x * 256;
    int64_t done = 0;
    if constexpr (VEC) {
        const int64_t nvec = n / 8;
        for (int64_t i = gid; i < nvec; i += stride) {
            float g[8], u[8], o[8];
            chunk8<T>::ld(gate + 8 * i, g);
            chunk8<T>::ld(up + 8 * i, u);
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = glu_val<KIND>(g[e], u[e]);
            chunk8<T>::st(out + 8 * i, o);
        }
        done = nvec * 8;
    }
    for (int64_t i = done + gid; i < n; i += stride)
        io<T>::st(out, i, glu_val<KIND>(io<T>::ld(gate, i), io<T>::ld(up, i)));
}

template <typename T, bool VEC>
int launch_glu_fwd(int kind, const void* gate, const void* up, void* out, int64_t n, hipStream_t s) {
    const unsigned grid = grid_for(VEC ? (n + 7) / 8 : n, 256, 16384);
    const T* g = (const T*)gate;
    const T* u = (const T*)up;
    T* o = (T*)out;
    switch (kind) {
        case GN_GLU_SWIGLU_UP: glu_fwd_kernel<GN_GLU_SWIGLU_UP, T, VEC><<<grid, 256, 0, s>>>(g, u, o, n); break;
        case GN_GLU_SWIGLU_GATE: glu_fwd_kernel<GN_GLU_SWIGLU_GATE, T, VEC><<<grid, 256, 0, s>>>(g, u, o, n); break;
        case GN_GLU_GEGLU_UP: glu_fwd_kernel<GN_GLU_GEGLU_UP, T, VEC><<<grid, 256, 0, s>>>(g, u, o, n); break;
        case GN_GLU_GEGLU_GATE: glu_fwd_kernel<GN_GLU_GEGLU_GATE, T, VEC><<<grid, 256, 0, s>>>(g, u, o, n); break;
        default: glu_fwd_kernel<GN_GLU_REGLU_UP, T, VEC><<<grid, 256, 0, s>>>(g, u, o, n); break;
    }
    GN_LAUNCH_CHECK("gn_glu_fwd");
    return GN_OK;
}

int glu_fwd(int kind, const void* gate, const void* up, void* out, int64_t n, int dtype,
            hipStream_t s) {
    const bool vec = al16(gate) && al16(up) && al16(out);
    if (dtype == GN_BF16)
        return vec ? launch_glu_fwd<bf16_t, true>(kind, gate, up, out, n, s)
                   : launch_glu_fwd<bf16_t, false>(kind, gate, up, out, n, s);
    return vec ? launch_glu_fwd<float, true>(kind, gate, up, out, n, s)
               : launch_glu_fwd<float, false>(kind, gate, up, out, n, s);
}

// Y = act(X) elementwise (activation-{relu,gelu,silu,tanh,sigmoid}.glsl forward values).
template <int KIND>
__device__ __forceinline__ float act_val(float x) {
    if constexpr (KIND == GN_ACT_RELU) return x > 0.f ? x : 0.f;
    else if constexpr (KIND == GN_ACT_GELU_TANH) return gelu_tanh_f(x);
    else if constexpr (KIND == GN_ACT_GELU_ERF) return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f));
    else if constexpr (KIND == GN_ACT_SILU) return silu_f(x);
    else if constexpr (KIND == GN_ACT_TANH) return tanhf_(x);
    else return sigmoidf_(x);
}

template <int KIND, typename T>
__global__ __launch_bounds__(256) void act_fwd_kernel(const T* __restrict__ X, T* __restrict__ Y,
                                                      int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        io<T>::st(Y, i, act_val<KIND>(io<T>::ld(X, i)));
}

template <typename T>
int act_fwd(int kind, const void* X, void* Y, int64_t n, hipStream_t s) {
    const unsigned g = grid_for(n, 256, 16384);
    const T* x = (const T*)X;
    T* y = (T*)Y;
    switch (kind) {
        case GN_ACT_RELU: act_fwd_kernel<GN_ACT_RELU, T><<<g, 256, 0, s>>>(x, y, n); break;
        case GN_ACT_GELU_TANH: act_fwd_kernel<GN_ACT_GELU_TANH, T><<<g, 256, 0, s>>>(x, y, n); break;
        case GN_ACT_GELU_ERF: act_fwd_kernel<GN_ACT_GELU_ERF, T><<<g, 256, 0, s>>>(x, y, n); break;
        case GN_ACT_SILU: act_fwd_kernel<GN_ACT_SILU, T><<<g, 256, 0, s>>>(x, y, n); break;
        case GN_ACT_TANH: act_fwd_kernel<GN_ACT_TANH, T><<<g, 256, 0, s>>>(x, y, n); break;
        default: act_fwd_kernel<GN_ACT_SIGMOID, T><<<g, 256, 0, s>>>(x, y, n); break;
    }
    GN_LAUNCH_CHECK("gn_act_fwd");
    return GN_OK;
}

// Y[m][n] = b[n] (or 0): the starting value of a GEMM that then accumulates X W^T.
template <typename T>
__global__ __launch_bounds__(256) void fill_rows(const T* __restrict__ b, T* __restrict__ Y,
                                                 int64_t total, int N) {
    for (int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * 256)
        io<T>::st(Y, i, b ? io<T>::ld(b, i % N) : 0.f);
}

// Y [M x N] = X [M x K] W^T (W [N x K]) + b, all in `dtype` (fp32 accumulation).  The bias
// rides on the GEMM epilogue on the LDS-DMA core; other shapes start Y from the bias and
// accumulate.
int linear_fwd(const void* X, const void* W, const void* b, void* Y, int M, int N, int K,
               int dtype, hipStream_t s) {
    if (dtype == GN_F32 && skinny_fwd_applicable(X, W, Y, M, K))
        return skinny_linear_fwd((const float*)X, (const float*)W, (const float*)b, (float*)Y, M, N,
                                 K, s);
    GemmDesc d{};
    d.nseg = 1;
    d.A[0] = (const bf16_t*)X; d.lda[0] = K; d.Ks[0] = K;
    d.B[0] = (const bf16_t*)W; d.ldb[0] = K;
    d.M = M; d.N = N; d.C = Y; d.C2 = Y; d.Msplit = M; d.ldc = N;
    if (b && dtype == GN_BF16 && K > 0) {
        d.cbias = (const bf16_t*)b;
        if (gemm_dma_applicable(d)) return gemm_run(d, 0, 1, dtype, dtype, s);
        d.cbias = nullptr;
    }
    if (b || K == 0) {
        const int64_t total = (int64_t)M * N;
        if (dtype == GN_BF16)
            fill_rows<bf16_t><<<grid_for(total, 256, 16384), 256, 0, s>>>((const bf16_t*)b, (bf16_t*)Y, total, N);
        else
            fill_rows<float><<<grid_for(total, 256, 16384), 256, 0, s>>>((const float*)b, (float*)Y, total, N);
        GN_LAUNCH_CHECK("gn_linear_fwd (bias)");
        if (K == 0) return GN_OK;
        d.accumulate = 1;
    }
    return gemm_run(d, 0, 1, dtype, dtype, s);
}

}  // namespace
}  // namespace gn

using namespace gn;

extern "C" int gn_layernorm_fwd(const void* X, const void* gamma, const void* beta, void* Y,
                                float* mean, float* rstd, int rows, int F, float eps, int dtype,
                                unsigned flags, void* stream) {
    return gn_layernorm_fwd_ex(X, dtype, gamma, beta, Y, dtype, mean, rstd, rows, F, eps, flags,
                               stream);
}

extern "C" int gn_layernorm_fwd_ex(const void* X, int x_dtype, const void* gamma, const void* beta,
                                   void* Y, int y_dtype, float* mean, float* rstd, int rows, int F,
                                   float eps, unsigned flags, void* stream) {
    clear_error();
    GN_REQUIRE(rows >= 0 && F >= 0, "gn_layernorm_fwd: negative size");
    if (rows == 0) return GN_OK;
    GN_REQUIRE(F > 0, "gn_layernorm_fwd: F = 0 with %d rows", rows);
    GN_REQUIRE(X && Y, "gn_layernorm_fwd: null pointer");
    const int save_var = (flags & GN_LN_STAT_VAR) ? 1 : 0;
    return norm_fwd_dispatch<0>(x_dtype, y_dtype, X, gamma, beta, Y, mean, rstd, rows, F, eps,
                                save_var, as_stream(stream));
}

extern "C" int gn_rmsnorm_fwd(const void* X, const void* w, void* Y, float* rstd, int rows, int F,
                              float eps, int dtype, void* stream) {
    return gn_rmsnorm_fwd_ex(X, dtype, w, Y, dtype, rstd, rows, F, eps, stream);
}

extern "C" int gn_rmsnorm_fwd_stat(const void* X, int x_dtype, const void* w, void* Y, int y_dtype,
                                   float* stat, int rows, int F, float eps, unsigned flags,
                                   void* stream) {
    clear_error();
    GN_REQUIRE(rows >= 0 && F >= 0, "gn_rmsnorm_fwd: negative size");
    if (rows == 0) return GN_OK;
    GN_REQUIRE(F > 0, "gn_rmsnorm_fwd: F = 0 with %d rows", rows);
    GN_REQUIRE(X && Y, "gn_rmsnorm_fwd: null pointer");
    const bool meansq = flags & GN_RMS_STAT_MEANSQ, rms = flags & GN_RMS_STAT_RMS;
    GN_REQUIRE(!(meansq && rms), "gn_rmsnorm_fwd: GN_RMS_STAT_MEANSQ and GN_RMS_STAT_RMS together");
    return norm_fwd_dispatch<1>(x_dtype, y_dtype, X, w, nullptr, Y, nullptr, stat, rows, F, eps,
                                meansq ? 1 : rms ? 2 : 0, as_stream(stream));
}

extern "C" int gn_rmsnorm_fwd_ex(const void* X, int x_dtype, const void* w, void* Y, int y_dtype,
                                 float* rstd, int rows, int F, float eps, void* stream) {
    return gn_rmsnorm_fwd_stat(X, x_dtype, w, Y, y_dtype, rstd, rows, F, eps, 0, stream);
}

extern "C" int gn_glu_fwd(int kind, const void* gate, const void* up, void* out, int64_t n,
                          int dtype, void* stream) {
    clear_error();
    GN_REQUIRE(n >= 0, "gn_glu_fwd: negative size");
    GN_REQUIRE(kind >= GN_GLU_SWIGLU_UP && kind <= GN_GLU_REGLU_UP, "gn_glu_fwd: kind %d", kind);
    GN_REQUIRE(dtype == GN_F32 || dtype == GN_BF16, "gn_glu_fwd: dtype %d (f32, bf16)", dtype);
    if (n == 0) return GN_OK;
    GN_REQUIRE(gate && up && out, "gn_glu_fwd: null pointer");
    return glu_fwd(kind, gate, up, out, n, dtype, as_stream(stream));
}

extern "C" int gn_linear_fwd(const void* X, const void* W, const void* b, void* Y, int M, int N,
                             int K, int dtype, void* stream) {
    clear_error();
    GN_REQUIRE(M >= 0 && N >= 0 && K >= 0, "gn_linear_fwd: negative size");
    GN_REQUIRE(dtype == GN_F32 || dtype == GN_BF16, "gn_linear_fwd: dtype %d (f32, bf16)", dtype);
    if (M == 0 || N == 0) return GN_OK;
    GN_REQUIRE(Y && (K == 0 || (X && W)), "gn_linear_fwd: null pointer");
    return linear_fwd(X, W, b, Y, M, N, K, dtype, as_stream(stream));
}

extern "C" int gn_glu_linear_fwd(int kind, const void* X, const void* Wg, const void* Wu,
                                 const void* bg, const void* bu, void* gate, void* up, void* out,
                                 int M, int H, int K, int dtype, void* stream) {
    clear_error();
    GN_REQUIRE(M >= 0 && H >= 0 && K >= 0, "gn_glu_linear_fwd: negative size");
    GN_REQUIRE(kind >= GN_GLU_SWIGLU_UP && kind <= GN_GLU_REGLU_UP, "gn_glu_linear_fwd: kind %d", kind);
    GN_REQUIRE(dtype == GN_F32 || dtype == GN_BF16, "gn_glu_linear_fwd: dtype %d (f32, bf16)", dtype);
    if (M == 0 || H == 0) return GN_OK;
    GN_REQUIRE(gate && up && out && (K == 0 || (X && Wg && Wu)), "gn_glu_linear_fwd: null pointer");
    hipStream_t s = as_stream(stream);
    int rc = linear_fwd(X, Wg, bg, gate, M, H, K, dtype, s);
    if (rc == GN_OK) rc = linear_fwd(X, Wu, bu, up, M, H, K, dtype, s);
    if (rc == GN_OK) rc = glu_fwd(kind, gate, up, out, (int64_t)M * H, dtype, s);
    return rc;
}

extern "C" int gn_act_fwd(int kind, const void* X, void* Y, int64_t n, int dtype, void* stream) {
    clear_error();
    GN_REQUIRE(n >= 0, "gn_act_fwd: negative size");
    GN_REQUIRE(kind >= GN_ACT_RELU && kind <= GN_ACT_SIGMOID, "gn_act_fwd: kind %d", kind);
    GN_REQUIRE(dtype == GN_F32 || dtype == GN_BF16, "gn_act_fwd: dtype %d (f32, bf16)", dtype);
    if (n == 0) return GN_OK;
    GN_REQUIRE(X && Y, "gn_act_fwd: null pointer");
    if (dtype == GN_BF16) return act_fwd<bf16_t>(kind, X, Y, n, as_stream(stream));
    return act_fwd<float>(kind, X, Y, n, as_stream(stream));
}
