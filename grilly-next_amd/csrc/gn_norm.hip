// gn_norm.hip — row-reduction gradients: LayerNorm, RMSNorm, softmax, cross-entropy.
//
// LayerNorm / RMSNorm: one wave per row, the row held in registers (8-element chunks of
// 16 bytes, chunk c = lane + 64 j), so x and dy are read once and dx written once.  Parameter
// gradients (dgamma/dbeta, dw) are accumulated per lane across the rows a wave owns,
// reduced across the block's waves in LDS, written as one partial row per block to the
// workspace, and summed by a small deterministic finish kernel (no atomics).
#include "gn_common.h"

#include <mutex>

namespace gn {
namespace {

constexpr int kNormBlocks = 512;  // workspace rows reserved (one partial row per block)
constexpr int kNormGrid = 256;    // blocks the row kernel uses at most (one per CU)
constexpr int kNormWaves = 8;     // waves per block (512 threads)

// Register-resident 8-element chunk: bf16 stays packed (4 VGPRs) until it is used.
template <typename T> struct raw8;
template <> struct raw8<float> {
    float v[8];
    __device__ __forceinline__ void load(const float* p) { chunk8<float>::ld(p, v); }
    __device__ __forceinline__ void zero() {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.f;
    }
    __device__ __forceinline__ float operator[](int e) const { return v[e]; }
};
template <> struct raw8<bf16_t> {
    uint32_t w[4];
    __device__ __forceinline__ void load(const bf16_t* p) {
        const uint4 x = *reinterpret_cast<const uint4*>(p);
        w[0] = x.x; w[1] = x.y; w[2] = x.z; w[3] = x.w;
    }
    __device__ __forceinline__ void zero() { w[0] = w[1] = w[2] = w[3] = 0u; }
    __device__ __forceinline__ float operator[](int e) const {
        return __uint_as_float((e & 1) ? (w[e >> 1] & 0xffff0000u) : (w[e >> 1] << 16));
    }
};

// The saved per-row statistic as the row's 1/sqrt(var + eps): kind 0 = rstd itself; 1 = the
// variance (LayerNorm, fnn-layernorm.glsl:77 var_vals) or mean(x^2) (RMSNorm, rms-norm.glsl:52),
// plus eps; 2 = sqrt(mean(x^2) + eps) (snn-rmsnorm.glsl:55).
__device__ __forceinline__ float stat_rstd(float s, int kind, float eps) {
    return kind == 1 ? rsqrtf(s + eps) : kind == 2 ? 1.0f / s : s;
}

// One wave per row; lane l owns 8-element chunks c = l + 64 j (j < NC).  Each wave walks
// rows r, r + stride, ... and requests row r + stride before it works on row r.  gamma / w
// stays in registers.  Parameter-gradient partials live in LDS, one row per wave (each wave
// adds into its own row, so the order of additions is fixed); at the end the block sums
// its waves' rows and writes one partial row to the workspace.
// MODE 0 = LayerNorm (dgamma, dbeta partials), 1 = RMSNorm (dw partials).
// TX: x, dX and the addend (a residual stream kept in fp32); TY: dy and gamma.  `add`
// (nullable, may alias dX) is added to the row's input gradient: the residual branch's
// gradient of a pre-norm block, so the fan-out sum costs no pass of its own.
template <int MODE, typename TX, typename TY, int NC>
__global__ __launch_bounds__(64 * kNormWaves) void norm_bwd_rows(
    const TY* __restrict__ dY, const TX* __restrict__ X, const TY* __restrict__ gamma,
    const float* __restrict__ mean, const float* __restrict__ rstd, TX* dX, const TX* add,
    float* __restrict__ part, int rows, int F, float eps, int stat_kind, bf16_t* __restrict__ dX16) {
    constexpr int NP = MODE == 0 ? 2 : 1;
    extern __shared__ float red[];  // [kNormWaves][NP][F]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nchunks = F >> 3;
    const float invF = 1.0f / (float)F;
    float* my = red + (size_t)wave * NP * F;
    for (int f = 4 * lane; f < NP * F; f += 256) *reinterpret_cast<float4*>(my + f) = make_float4(0.f, 0.f, 0.f, 0.f);

    raw8<TY> gm[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int c = lane + 64 * j;
        if (c < nchunks) gm[j].load(gamma + 8 * c);
        else gm[j].zero();
    }
    // the addend travels with the row too (loaded after the row's reductions it puts a second
    // memory round trip on every row), except for fp32 rows of 4 chunks per lane, where the
    // extra registers would spill
    constexpr bool PRE_ADD = !(sizeof(TX) == 4 && NC == 4);
    auto load_row = [&](int r, raw8<TX> (&x)[NC], raw8<TY> (&dy)[NC], raw8<TX> (&ad)[NC]) {
        const size_t off = (size_t)r * F;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const int c = lane + 64 * j;
            if (c < nchunks) {
                x[j].load(X + off + 8 * c);
                dy[j].load(dY + off + 8 * c);
                if (PRE_ADD && add) ad[j].load(add + off + 8 * c);
                else ad[j].zero();
            } else {
                x[j].zero();
                dy[j].zero();
                ad[j].zero();
            }
        }
    };
    // row statistics travel with the row's loads, so the prefetch of the next row is the
    // only memory traffic in flight while a row is worked on
    auto load_stats = [&](int r, float& mu, float& rs) {
        mu = MODE == 0 ? mean[r] : 0.f;
        rs = rstd[r];
    };
    const int stride = gridDim.x * kNormWaves;
    int r = blockIdx.x * kNormWaves + wave;
    raw8<TX> x[NC], ad[NC];
    raw8<TY> dy[NC];
    float mu = 0.f, rs = 0.f;
    if (r < rows) {
        load_stats(r, mu, rs);
        load_row(r, x, dy, ad);
    }
    while (r < rows) {
        const int rn = r + stride;
        raw8<TX> xn[NC], adn[NC];
        raw8<TY> dyn[NC];
        float mun = 0.f, rsn = 0.f;
        if (rn < rows) {
            load_stats(rn, mun, rsn);
            load_row(rn, xn, dyn, adn);
        }
        const size_t off = (size_t)r * F;
        rs = stat_rstd(rs, stat_kind, eps);
        float s1 = 0.f, s2 = 0.f;
#pragma unroll
        for (int j = 0; j < NC; ++j)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                if (MODE == 0) {
                    const float xh = (x[j][e] - mu) * rs, g = dy[j][e] * gm[j][e];
                    s1 += g;
                    s2 += g * xh;
                } else {
                    s1 += gm[j][e] * dy[j][e] * x[j][e];
                }
            }
        s1 = wave_sum(s1);
        if (MODE == 0) s2 = wave_sum(s2);
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const int c = lane + 64 * j;
            if (c >= nchunks) continue;
            float o[8], pa[8], pb[8];
            if (PRE_ADD) {
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e] = ad[j][e];
            } else if (add) {
                chunk8<TX>::ld(add + off + 8 * c, o);
            }
            float4* qa = reinterpret_cast<float4*>(my + 8 * c);
            float4* qb = reinterpret_cast<float4*>(my + F + 8 * c);
            const float4 a0 = qa[0], a1 = qa[1];
            pa[0] = a0.x; pa[1] = a0.y; pa[2] = a0.z; pa[3] = a0.w;
            pa[4] = a1.x; pa[5] = a1.y; pa[6] = a1.z; pa[7] = a1.w;
            if (MODE == 0) {
                const float4 b0 = qb[0], b1 = qb[1];
                pb[0] = b0.x; pb[1] = b0.y; pb[2] = b0.z; pb[3] = b0.w;
                pb[4] = b1.x; pb[5] = b1.y; pb[6] = b1.z; pb[7] = b1.w;
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float v;
                if (MODE == 0) {
                    const float xh = (x[j][e] - mu) * rs, g = dy[j][e] * gm[j][e];
                    v = rs * (g - s1 * invF - xh * s2 * invF);
                    pa[e] += dy[j][e] * xh;
                    pb[e] += dy[j][e];
                } else {
                    v = rs * gm[j][e] * dy[j][e] - x[j][e] * rs * rs * rs * s1 * invF;
                    pa[e] += dy[j][e] * x[j][e] * rs;
                }
                o[e] = add ? o[e] + v : v;
            }
            chunk8<TX>::st(dX + off + 8 * c, o);
            if (dX16) chunk8<bf16_t>::st(dX16 + off + 8 * c, o);  // the same values, bf16
            qa[0] = make_float4(pa[0], pa[1], pa[2], pa[3]);
            qa[1] = make_float4(pa[4], pa[5], pa[6], pa[7]);
            if (MODE == 0) {
                qb[0] = make_float4(pb[0], pb[1], pb[2], pb[3]);
                qb[1] = make_float4(pb[4], pb[5], pb[6], pb[7]);
            }
        }
#pragma unroll
        for (int j = 0; j < NC; ++j) { x[j] = xn[j]; dy[j] = dyn[j]; ad[j] = adn[j]; }
        mu = mun;
        rs = rsn;
        r = rn;
    }
    // the block's partial rows: waves summed in a fixed order
    __syncthreads();
    for (int p = 0; p < NP; ++p) {
        float* dst = part + ((size_t)p * gridDim.x + blockIdx.x) * F;
        for (int f = 4 * threadIdx.x; f < F; f += 4 * 64 * kNormWaves) {
            float4 s = *reinterpret_cast<const float4*>(red + (size_t)p * F + f);
#pragma unroll
            for (int w = 1; w < kNormWaves; ++w) {
                const float4 v = *reinterpret_cast<const float4*>(red + ((size_t)w * NP + p) * F + f);
                s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
            }
            *reinterpret_cast<float4*>(dst + f) = s;
        }
    }
}

// out[f] (+)= sum_g part[g][f] over G partial rows.  Block: 16 waves x 64 columns (one per
// lane, 256-byte rows); wave w sums rows w, w + 16, ...; the waves' sums are added in a
// fixed order.
// blockIdx.y picks the partial plane: plane 0 (part) -> out0, plane 1 (part + G F) -> out1,
// so the gain and bias sums of a LayerNorm finish in one launch.
__global__ __launch_bounds__(1024) void colsum_partials(const float* __restrict__ part, int G,
                                                        int F, float* __restrict__ out0,
                                                        float* __restrict__ out1, int accumulate) {
    __shared__ float sh[16][64];
    float* __restrict__ out = blockIdx.y ? out1 : out0;
    part += (size_t)blockIdx.y * G * F;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int f = blockIdx.x * 64 + lane;
    float s = 0.f;
    if (f < F) {
#pragma unroll 8
        for (int g = wave; g < G; g += 16) s += part[(size_t)g * F + f];
    }
    sh[wave][lane] = s;
    __syncthreads();
    if (wave == 0 && f < F) {
        float t = sh[0][lane];
#pragma unroll
        for (int w = 1; w < 16; ++w) t += sh[w][lane];
        out[f] = accumulate ? out[f] + t : t;
    }
}

// colsum_partials over a batch of deferred norm calls: blockIdx.z = item, blockIdx.y = plane,
// blockIdx.x = 64-column group; the same sums in the same order as colsum_partials.
struct NormFinishItem {
    const float* part;
    float* out0;
    float* out1;
    int G, F, planes, accumulate;
};
constexpr int kNormFinishBatch = 32;
struct NormFinishBatch {
    NormFinishItem it[kNormFinishBatch];
};
__global__ __launch_bounds__(1024) void colsum_partials_batch(NormFinishBatch b) {
    __shared__ float sh[16][64];
    const NormFinishItem& it = b.it[blockIdx.z];
    if ((int)blockIdx.y >= it.planes || (int)blockIdx.x * 64 >= it.F) return;  // uniform
    float* __restrict__ out = blockIdx.y ? it.out1 : it.out0;
    if (!out) return;
    const float* part = it.part + (size_t)blockIdx.y * it.G * it.F;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int f = blockIdx.x * 64 + lane;
    float s = 0.f;
    if (f < it.F) {
#pragma unroll 8
        for (int g = wave; g < it.G; g += 16) s += part[(size_t)g * it.F + f];
    }
    sh[wave][lane] = s;
    __syncthreads();
    if (wave == 0 && f < it.F) {
        float t = sh[0][lane];
#pragma unroll
        for (int w = 1; w < 16; ++w) t += sh[w][lane];
        out[f] = it.accumulate ? out[f] + t : t;
    }
}

// partial rows the row kernel writes for `rows` (its grid)
inline int norm_grid(int rows) {
    return std::max(1, std::min(kNormGrid, (rows + 2 * kNormWaves - 1) / (2 * kNormWaves)));
}

// Generic fallback (any F): one block per row, two passes over global memory.
template <int MODE, typename TX, typename TY>
__global__ __launch_bounds__(256) void norm_bwd_generic_dx(
    const TY* __restrict__ dY, const TX* __restrict__ X, const TY* __restrict__ gamma,
    const float* __restrict__ mean, const float* __restrict__ rstd, TX* dX, const TX* add, int F,
    float eps, int stat_kind) {
    __shared__ float sh[4];
    const int r = blockIdx.x;
    const size_t off = (size_t)r * F;
    const float mu = MODE == 0 ? mean[r] : 0.f;
    const float rs = stat_rstd(rstd[r], stat_kind, eps);
    float s1 = 0.f, s2 = 0.f;
    for (int f = threadIdx.x; f < F; f += 256) {
        float x = io<TX>::ld(X, off + f), dy = io<TY>::ld(dY, off + f), g = io<TY>::ld(gamma, f);
        if (MODE == 0) {
            float xh = (x - mu) * rs;
            s1 += dy * g;
            s2 += dy * g * xh;
        } else {
            s1 += g * dy * x;
        }
    }
    s1 = block_sum<4>(s1, sh);
    if (MODE == 0) s2 = block_sum<4>(s2, sh);
    const float invF = 1.0f / (float)F;
    for (int f = threadIdx.x; f < F; f += 256) {
        float x = io<TX>::ld(X, off + f), dy = io<TY>::ld(dY, off + f), g = io<TY>::ld(gamma, f);
        float v;
        if (MODE == 0) {
            float xh = (x - mu) * rs;
            v = rs * (dy * g - s1 * invF - xh * s2 * invF);
        } else {
            v = rs * g * dy - x * rs * rs * rs * s1 * invF;
        }
        if (add) v += io<TX>::ld(add, off + f);
        io<TX>::st(dX, off + f, v);
    }
}

// Generic parameter gradients: column sums over all rows (thread per feature).
template <int MODE, typename TX, typename TY>
__global__ __launch_bounds__(256) void norm_bwd_generic_param(
    const TY* __restrict__ dY, const TX* __restrict__ X, const float* __restrict__ mean,
    const float* __restrict__ rstd, float* __restrict__ dA, float* __restrict__ dB, int rows,
    int F, float eps, int stat_kind, int accumulate) {
    const int f = blockIdx.x * 256 + threadIdx.x;
    if (f >= F) return;
    float sa = 0.f, sb = 0.f;
    for (int r = 0; r < rows; ++r) {
        float x = io<TX>::ld(X, (size_t)r * F + f), dy = io<TY>::ld(dY, (size_t)r * F + f);
        const float rs = stat_rstd(rstd[r], stat_kind, eps);
        if (MODE == 0) {
            sa += dy * (x - mean[r]) * rs;
            sb += dy;
        } else {
            sa += dy * x * rs;
        }
    }
    if (dA) dA[f] = accumulate ? dA[f] + sa : sa;
    if (MODE == 0 && dB) dB[f] = accumulate ? dB[f] + sb : sb;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <typename F>
bool allow_lds(F* fn, size_t bytes) {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) == hipSuccess;
}

// add: the input-gradient addend (nullable; dX itself for an in-place accumulation).
// acc: the parameter gradients add onto dA / dB.  dX16 (nullable, fp32 dX only): a bf16 copy
// of dX, written in the row kernel's pass (a conversion pass after the other paths).
template <int MODE, typename TX, typename TY>
int norm_bwd(const void* dY, const void* X, const void* gamma, const float* mean,
             const float* rstd, void* dX, const void* add, float* dA, float* dB, int rows, int F,
             float eps, int stat_var, bool acc, void* ws, size_t ws_bytes, hipStream_t s,
             bf16_t* dX16 = nullptr, bool partials_only = false) {
    if (dX16 && sizeof(TX) != 4) {
        set_error("norm backward: a bf16 copy of dX needs an fp32 dX");
        return GN_E_INVALID;
    }
    // the paths without the row kernel: the copy as a conversion pass after them
    auto copy16 = [&]() -> int {
        if (!dX16) return GN_OK;
        return gn_convert(dX, GN_F32, dX16, GN_BF16, (int64_t)rows * F, s);
    };
    // rows wider than 2048 would not fit in registers: they use the generic path
    const bool vec_ok = (F % 8 == 0) && F <= 2048 && aligned16(dY) && aligned16(X) &&
                        aligned16(dX) && aligned16(gamma) && (!add || aligned16(add));
    const bool need_param = dA || dB;
    const TX* ad = (const TX*)add;
    if (partials_only && !(vec_ok && need_param)) {
        set_error("norm backward: GN_NORM_PARTIALS needs the row kernel (F %% 8 == 0, F <= 2048, "
                  "16-byte aligned tensors) and a parameter gradient");
        return GN_E_INVALID;
    }
    if (vec_ok) {
        // every wave gets two rows or more where the row count allows it
        const int G = norm_grid(rows);
        const size_t need = (size_t)(MODE == 0 ? 2 : 1) * G * F * sizeof(float);
        if (need_param && (!ws || ws_bytes < need)) {
            set_error("norm backward: workspace %zu B < %zu B", ws_bytes, need);
            return GN_E_WORKSPACE;
        }
        float* part = need_param ? (float*)ws : nullptr;
        const int nc = (F / 8 + 63) / 64;
        // without parameter gradients there are no partial rows to write: the generic dx
        // kernel does the input gradient alone
        if (!need_param) {
            norm_bwd_generic_dx<MODE, TX, TY><<<rows, 256, 0, s>>>(
                (const TY*)dY, (const TX*)X, (const TY*)gamma, mean, rstd, (TX*)dX, ad, F, eps, stat_var);
            GN_LAUNCH_CHECK("norm backward (dx only)");
            return copy16();
        }
        const size_t lds = (size_t)kNormWaves * (MODE == 0 ? 2 : 1) * F * sizeof(float);
        if (lds > 64 * 1024) {
            static const bool ok = allow_lds(norm_bwd_rows<MODE, TX, TY, 4>, 160 * 1024) &&
                                   allow_lds(norm_bwd_rows<MODE, TX, TY, 2>, 160 * 1024);
            if (!ok) {
                set_error("norm backward: cannot reserve %zu B of LDS", lds);
                return GN_E_HIP;
            }
        }
#define GN_NORM_LAUNCH(NCV)                                                                    \
    norm_bwd_rows<MODE, TX, TY, NCV><<<G, 64 * kNormWaves, lds, s>>>(                          \
        (const TY*)dY, (const TX*)X, (const TY*)gamma, mean, rstd, (TX*)dX, ad, part, rows, F, \
        eps, stat_var, dX16)
        if (nc <= 1) GN_NORM_LAUNCH(1);
        else if (nc <= 2) GN_NORM_LAUNCH(2);
        else GN_NORM_LAUNCH(4);
#undef GN_NORM_LAUNCH
        GN_LAUNCH_CHECK("norm backward rows");
        if (partials_only) return GN_OK;  // gn_norm_finish adds the partial rows
        const unsigned gf = (F + 63) / 64;
        if (dA && MODE == 0 && dB)
            colsum_partials<<<dim3(gf, 2), 1024, 0, s>>>(part, G, F, dA, dB, acc);
        else if (dA)
            colsum_partials<<<gf, 1024, 0, s>>>(part, G, F, dA, nullptr, acc);
        else if (MODE == 0 && dB)
            colsum_partials<<<gf, 1024, 0, s>>>(part + (size_t)G * F, G, F, dB, nullptr, acc);
        GN_LAUNCH_CHECK("norm backward finish");
        return GN_OK;
    }
    if (dX) {
        norm_bwd_generic_dx<MODE, TX, TY><<<rows, 256, 0, s>>>(
            (const TY*)dY, (const TX*)X, (const TY*)gamma, mean, rstd, (TX*)dX, ad, F, eps, stat_var);
        GN_LAUNCH_CHECK("norm backward generic dx");
        if (int rc = copy16()) return rc;
    }
    if (need_param) {
        norm_bwd_generic_param<MODE, TX, TY><<<(F + 255) / 256, 256, 0, s>>>(
            (const TY*)dY, (const TX*)X, mean, rstd, dA, dB, rows, F, eps, stat_var, acc);
        GN_LAUNCH_CHECK("norm backward generic params");
    }
    return GN_OK;
}

// (TX, TY) pairs the library takes: both fp32, both bf16, or fp32 x / dX with bf16 dy / gamma
// (a residual stream carried in fp32 under a bf16 block).
template <int MODE>
int norm_bwd_dispatch(const char* who, int dy_dtype, int x_dtype, const void* dY, const void* X,
                      const void* gamma, const float* mean, const float* rstd, void* dX,
                      const void* add, float* dA, float* dB, int rows, int F, float eps,
                      int stat_var, bool acc, void* ws, size_t ws_bytes, hipStream_t s,
                      bf16_t* dX16 = nullptr, bool partials_only = false) {
    if (x_dtype == GN_F32 && dy_dtype == GN_F32)
        return norm_bwd<MODE, float, float>(dY, X, gamma, mean, rstd, dX, add, dA, dB, rows, F, eps,
                                            stat_var, acc, ws, ws_bytes, s, dX16, partials_only);
    if (x_dtype == GN_BF16 && dy_dtype == GN_BF16)
        return norm_bwd<MODE, bf16_t, bf16_t>(dY, X, gamma, mean, rstd, dX, add, dA, dB, rows, F,
                                              eps, stat_var, acc, ws, ws_bytes, s, dX16, partials_only);
    if (x_dtype == GN_F32 && dy_dtype == GN_BF16)
        return norm_bwd<MODE, float, bf16_t>(dY, X, gamma, mean, rstd, dX, add, dA, dB, rows, F,
                                             eps, stat_var, acc, ws, ws_bytes, s, dX16, partials_only);
    set_error("%s: x dtype %d with dy dtype %d not supported (f32/f32, bf16/bf16, f32/bf16)", who,
              x_dtype, dy_dtype);
    return GN_E_INVALID;
}

// ---- softmax backward: one block per row (activation-softmax-backward.glsl:36-48) ----
template <typename T>
__global__ __launch_bounds__(256) void softmax_bwd_kernel(const T* __restrict__ dY,
                                                          const T* __restrict__ Y,
                                                          T* __restrict__ dX, int C) {
    __shared__ float sh[4];
    const size_t off = (size_t)blockIdx.x * C;
    float dot = 0.f;
    for (int c = threadIdx.x; c < C; c += 256) dot += io<T>::ld(dY, off + c) * io<T>::ld(Y, off + c);
    dot = block_sum<4>(dot, sh);
    for (int c = threadIdx.x; c < C; c += 256) {
        float y = io<T>::ld(Y, off + c);
        io<T>::st(dX, off + c, y * (io<T>::ld(dY, off + c) - dot));
    }
}

// ---- cross-entropy backward: one block per row (cross-entropy-backward.glsl:41-84) ----
// Single read for the statistics (online max / sum of exp), one more for the gradient.
template <typename T>
__global__ __launch_bounds__(256) void xent_bwd_kernel(const T* __restrict__ Z,
                                                       const int32_t* __restrict__ tgt,
                                                       T* __restrict__ dZ, int C, float scale) {
    __shared__ float shm[4], shs[4];
    const size_t off = (size_t)blockIdx.x * C;
    float m = -INFINITY, s = 0.f;
    for (int c = threadIdx.x; c < C; c += 256) {
        float z = io<T>::ld(Z, off + c);
        if (z > m) {
            s = s * __expf(m - z) + 1.0f;
            m = z;
        } else {
            s += __expf(z - m);
        }
    }
    // combine (m, s) pairs across the block
    float mw = wave_max(m);
    s = (m == -INFINITY) ? 0.f : s * __expf(m - mw);
    s = wave_sum(s);
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    if (l == 0) { shm[w] = mw; shs[w] = s; }
    __syncthreads();
    float M = fmaxf(fmaxf(shm[0], shm[1]), fmaxf(shm[2], shm[3]));
    float S = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) S += (shm[i] == -INFINITY) ? 0.f : shs[i] * __expf(shm[i] - M);
    const float inv = scale / fmaxf(S, 1e-30f);
    const int t = tgt[blockIdx.x];
    for (int c = threadIdx.x; c < C; c += 256) {
        float g = __expf(io<T>::ld(Z, off + c) - M) * inv;
        if (c == t) g -= scale;
        io<T>::st(dZ, off + c, g);
    }
}

// bf16 rows that fit in registers (C % 8 == 0, C <= 2048 NCH): each row is read once with
// 16-byte loads and kept packed in VGPRs through the max, the sum of exp and the gradient
// (cross-entropy-backward.glsl:41-84 does three passes over the row in memory).
template <int NCH>
__global__ __launch_bounds__(256) void xent_bwd_rows_bf16(const bf16_t* __restrict__ Z,
                                                          const int32_t* __restrict__ tgt,
                                                          bf16_t* __restrict__ dZ, int C,
                                                          float scale) {
    __shared__ float sh[4];
    constexpr float kLog2e = 1.4426950408889634f;
    const size_t off = (size_t)blockIdx.x * C;
    const int nch = C >> 3;
    uint4 v[NCH];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
        const int c = threadIdx.x + 256 * j;
        v[j] = c < nch ? *reinterpret_cast<const uint4*>(Z + off + 8 * c) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
        if (threadIdx.x + 256 * j >= nch) continue;
        const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
            m = fmaxf(m, fmaxf(__uint_as_float(w[e] << 16), __uint_as_float(w[e] & 0xffff0000u)));
    }
    const float M = block_max<4>(m, sh);
    const float mb = M * kLog2e;
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
        if (threadIdx.x + 256 * j >= nch) continue;
        const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            s += __builtin_amdgcn_exp2f(__uint_as_float(w[e] << 16) * kLog2e - mb);
            s += __builtin_amdgcn_exp2f(__uint_as_float(w[e] & 0xffff0000u) * kLog2e - mb);
        }
    }
    const float S = block_sum<4>(s, sh);
    const float inv = scale / fmaxf(S, 1e-30f);
    const int t = tgt[blockIdx.x];
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
        const int c = threadIdx.x + 256 * j;
        if (c >= nch) continue;
        const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
        float g[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            g[2 * e] = __builtin_amdgcn_exp2f(__uint_as_float(w[e] << 16) * kLog2e - mb) * inv;
            g[2 * e + 1] = __builtin_amdgcn_exp2f(__uint_as_float(w[e] & 0xffff0000u) * kLog2e - mb) * inv;
        }
        const int rel = t - 8 * c;
        if (rel >= 0 && rel < 8) {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (e == rel) g[e] -= scale;
        }
        *reinterpret_cast<uint4*>(dZ + off + 8 * c) =
            make_uint4(pack_bf2(g[0], g[1]), pack_bf2(g[2], g[3]), pack_bf2(g[4], g[5]), pack_bf2(g[6], g[7]));
    }
}

}  // namespace

// ---- scratch of gn_layernorm_bwd_noalloc --------------------------------------------------
// The row kernel's partial parameter-gradient rows: 2 planes x at most kNormGrid blocks x
// F <= 2048 floats (wider or unaligned rows take the generic kernels, which need none) =
// 4 MiB per device, held until the process ends.  Every call on one device shares it.
constexpr size_t kNoAllocScratchBytes = (size_t)2 * kNormGrid * 2048 * sizeof(float);
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device, looked up once per device (each
// GPU holds its own copy of the array at its own address; the array's name in host code is
// not a device address).
void* scratch_on_current_device() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        set_error("gn_layernorm_bwd_noalloc: no current HIP device (or index >= %d)", kMaxDevices);
        return nullptr;
    }
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            set_error("gn_layernorm_bwd_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s",
                      dev, hipGetErrorString(e));
            return nullptr;
        }
        g_scratch_ptr[dev] = p;
    }
    return g_scratch_ptr[dev];
}
}  // namespace
}  // namespace gn

using namespace gn;

extern "C" size_t gn_norm_workspace_bytes(int rows, int F) {
    if (rows <= 0 || F <= 0) return 0;
    const int G = std::min(kNormBlocks, (rows + kNormWaves - 1) / kNormWaves);
    return (size_t)2 * G * F * sizeof(float);
}

extern "C" int gn_layernorm_bwd(const void* dY, const void* X, const void* gamma,
                                const float* mean, const float* rstd, void* dX, float* dGamma,
                                float* dBeta, int rows, int F, float eps, int dtype,
                                unsigned flags, void* ws, size_t ws_bytes, void* stream) {
    clear_error();
    GN_REQUIRE(rows >= 0 && F > 0, "gn_layernorm_bwd: bad shape rows=%d F=%d", rows, F);
    if (rows == 0) return GN_OK;
    GN_REQUIRE(dY && X && gamma && mean && rstd && dX, "gn_layernorm_bwd: null pointer");
    const bool acc = flags & GN_ACCUMULATE;
    const int sv = (flags & GN_LN_STAT_VAR) ? 1 : 0;
    GN_REQUIRE(dtype == GN_F32 || dtype == GN_BF16, "gn_layernorm_bwd: dtype %d not supported", dtype);
    return norm_bwd_dispatch<0>("gn_layernorm_bwd", dtype, dtype, dY, X, gamma, mean, rstd, dX,
                                acc ? dX : nullptr, dGamma, dBeta, rows, F, eps, sv, acc, ws,
                                ws_bytes, as_stream(stream));
}

extern "C" int gn_layernorm_bwd_ex(const void* dY, int dy_dtype, const void* X, int x_dtype,
                                   const void* gamma, const float* mean, const float* rstd,
                                   const void* dX_add, void* dX, float* dGamma, float* dBeta,
                                   int rows, int F, float eps, unsigned flags, void* ws,
                                   size_t ws_bytes, void* stream) {
    clear_error();
    GN_REQUIRE(rows >= 0 && F > 0, "gn_layernorm_bwd_ex: bad shape rows=%d F=%d", rows, F);
    if (rows == 0) return GN_OK;
    GN_REQUIRE(dY && X && gamma && mean && rstd && dX, "gn_layernorm_bwd_ex: null pointer");
    return norm_bwd_dispatch<0>("gn_layernorm_bwd_ex", dy_dtype, x_dtype, dY, X, gamma, mean, rstd,
                                dX, dX_add, dGamma, dBeta, rows, F, eps,
                                (flags & GN_LN_STAT_VAR) ? 1 : 0, flags & GN_ACCUMULATE, ws,
                                ws_bytes, as_stream(stream), nullptr, flags & GN_NORM_PARTIALS);
}

extern "C" int gn_norm_finish(const GnNormFinish* items, int n, void* stream) {
    clear_error();
    GN_REQUIRE(n >= 0 && (n == 0 || items), "gn_norm_finish: %d items", n);
    hipStream_t s = as_stream(stream);
    for (int i0 = 0; i0 < n; i0 += kNormFinishBatch) {
        NormFinishBatch b{};
        const int m = std::min(kNormFinishBatch, n - i0);
        int maxF = 0;
        for (int i = 0; i < m; ++i) {
            const GnNormFinish& f = items[i0 + i];
            GN_REQUIRE(f.ws && f.rows > 0 && f.F > 0, "gn_norm_finish: item %d: bad workspace or shape", i0 + i);
            b.it[i] = NormFinishItem{(const float*)f.ws, f.dgamma, f.layernorm ? f.dbeta : nullptr,
                                     norm_grid(f.rows), f.F, f.layernorm ? 2 : 1, f.accumulate ? 1 : 0};
            maxF = std::max(maxF, f.F);
        }
        colsum_partials_batch<<<dim3((maxF + 63) / 64, 2, m), 1024, 0, s>>>(b);
        GN_LAUNCH_CHECK("gn_norm_finish");
    }
    return GN_OK;
}

extern "C" int gn_layernorm_bwd_ex16(const void* dY, int dy_dtype, const void* X, int x_dtype,
                                     const void* gamma, const float* mean, const float* rstd,
                                     const void* dX_add, void* dX, void* dX_bf16, float* dGamma,
                                     float* dBeta, int rows, int F, float eps, unsigned flags,
                                     void* ws, size_t ws_bytes, void* stream) {
    clear_error();
    GN_REQUIRE(rows >= 0 && F > 0, "gn_layernorm_bwd_ex16: bad shape rows=%d F=%d", rows, F);
    if (rows == 0) return GN_OK;
    GN_REQUIRE(dY && X && gamma && mean && rstd && dX && dX_bf16, "gn_layernorm_bwd_ex16: null pointer");
    GN_REQUIRE(x_dtype == GN_F32, "gn_layernorm_bwd_ex16: the bf16 copy is of an fp32 dX (x dtype %d)", x_dtype);
    return norm_bwd_dispatch<0>("gn_layernorm_bwd_ex16", dy_dtype, x_dtype, dY, X, gamma, mean, rstd,
                                dX, dX_add, dGamma, dBeta, rows, F, eps,
                                (flags & GN_LN_STAT_VAR) ? 1 : 0, flags & GN_ACCUMULATE, ws,
                                ws_bytes, as_stream(stream), (bf16_t*)dX_bf16, flags & GN_NORM_PARTIALS);
}

extern "C" int gn_layernorm_bwd_noalloc(const void* dY, const void* X, const void* gamma,
                                        const float* mean, const float* rstd, void* dX,
                                        float* dGamma, float* dBeta, int rows, int F, float eps,
                                        int dtype, unsigned flags, void* stream) {
    clear_error();
    GN_REQUIRE(rows >= 0 && F > 0, "gn_layernorm_bwd_noalloc: bad shape rows=%d F=%d", rows, F);
    if (rows == 0) return GN_OK;
    GN_REQUIRE(dY && X && gamma && mean && rstd && dX, "gn_layernorm_bwd_noalloc: null pointer");
    GN_REQUIRE(dtype == GN_F32 || dtype == GN_BF16, "gn_layernorm_bwd_noalloc: dtype %d not supported",
               dtype);
    void* ws = scratch_on_current_device();
    if (!ws) return GN_E_HIP;
    const bool acc = flags & GN_ACCUMULATE;
    const int sv = (flags & GN_LN_STAT_VAR) ? 1 : 0;
    const int rc = norm_bwd_dispatch<0>("gn_layernorm_bwd_noalloc", dtype, dtype, dY, X, gamma, mean,
                                        rstd, dX, acc ? dX : nullptr, dGamma, dBeta, rows, F, eps,
                                        sv, acc, ws, kNoAllocScratchBytes, as_stream(stream));
    if (rc == GN_E_WORKSPACE)
        set_error("gn_layernorm_bwd_noalloc: rows=%d F=%d need more than the %zu B static scratch",
                  rows, F, kNoAllocScratchBytes);
    return rc;
}

extern "C" int gn_rmsnorm_bwd(const void* dY, const void* X, const void* w, const float* rstd,
                              void* dX, float* dW, int rows, int F, int dtype, unsigned flags,
                              void* ws, size_t ws_bytes, void* stream) {
    clear_error();
    GN_REQUIRE(rows >= 0 && F > 0, "gn_rmsnorm_bwd: bad shape rows=%d F=%d", rows, F);
    if (rows == 0) return GN_OK;
    GN_REQUIRE(dY && X && w && rstd && dX, "gn_rmsnorm_bwd: null pointer");
    GN_REQUIRE(dtype == GN_F32 || dtype == GN_BF16, "gn_rmsnorm_bwd: dtype %d not supported", dtype);
    const bool acc = flags & GN_ACCUMULATE;
    return norm_bwd_dispatch<1>("gn_rmsnorm_bwd", dtype, dtype, dY, X, w, nullptr, rstd, dX,
                                acc ? dX : nullptr, dW, nullptr, rows, F, 0.f, 0, acc, ws, ws_bytes,
                                as_stream(stream));
}

extern "C" int gn_rmsnorm_bwd_stat(const void* dY, int dy_dtype, const void* X, int x_dtype,
                                   const void* w, const float* stat, const void* dX_add, void* dX,
                                   float* dW, int rows, int F, float eps, unsigned flags, void* ws,
                                   size_t ws_bytes, void* stream) {
    clear_error();
    GN_REQUIRE(rows >= 0 && F > 0, "gn_rmsnorm_bwd: bad shape rows=%d F=%d", rows, F);
    if (rows == 0) return GN_OK;
    GN_REQUIRE(dY && X && w && stat && dX, "gn_rmsnorm_bwd: null pointer");
    const bool meansq = flags & GN_RMS_STAT_MEANSQ, rms = flags & GN_RMS_STAT_RMS;
    GN_REQUIRE(!(meansq && rms), "gn_rmsnorm_bwd: GN_RMS_STAT_MEANSQ and GN_RMS_STAT_RMS together");
    return norm_bwd_dispatch<1>("gn_rmsnorm_bwd", dy_dtype, x_dtype, dY, X, w, nullptr, stat, dX,
                                dX_add, dW, nullptr, rows, F, eps, meansq ? 1 : rms ? 2 : 0,
                                flags & GN_ACCUMULATE, ws, ws_bytes, as_stream(stream), nullptr,
                                flags & GN_NORM_PARTIALS);
}

extern "C" int gn_rmsnorm_bwd_ex(const void* dY, int dy_dtype, const void* X, int x_dtype,
                                 const void* w, const float* rstd, const void* dX_add, void* dX,
                                 float* dW, int rows, int F, unsigned flags, void* ws,
                                 size_t ws_bytes, void* stream) {
    return gn_rmsnorm_bwd_stat(dY, dy_dtype, X, x_dtype, w, rstd, dX_add, dX, dW, rows, F, 0.f,
                               flags & (GN_ACCUMULATE | GN_NORM_PARTIALS), ws, ws_bytes, stream);
}

extern "C" int gn_softmax_bwd(const void* dY, const void* Y, void* dX, int rows, int C,
                              int dtype, void* stream) {
    clear_error();
    GN_REQUIRE(rows >= 0 && C > 0, "gn_softmax_bwd: bad shape");
    if (rows == 0) return GN_OK;
    GN_REQUIRE(dY && Y && dX, "gn_softmax_bwd: null pointer");
    hipStream_t s = as_stream(stream);
    if (dtype == GN_F32)
        softmax_bwd_kernel<float><<<rows, 256, 0, s>>>((const float*)dY, (const float*)Y, (float*)dX, C);
    else if (dtype == GN_BF16)
        softmax_bwd_kernel<bf16_t><<<rows, 256, 0, s>>>((const bf16_t*)dY, (const bf16_t*)Y, (bf16_t*)dX, C);
    else {
        set_error("gn_softmax_bwd: dtype %d not supported", dtype);
        return GN_E_INVALID;
    }
    GN_LAUNCH_CHECK("gn_softmax_bwd");
    return GN_OK;
}

extern "C" int gn_xent_bwd(const void* logits, const int32_t* targets, void* dLogits, int rows,
                           int C, float scale, int dtype, void* stream) {
    clear_error();
    GN_REQUIRE(rows >= 0 && C > 0, "gn_xent_bwd: bad shape");
    if (rows == 0) return GN_OK;
    GN_REQUIRE(logits && targets && dLogits, "gn_xent_bwd: null pointer");
    hipStream_t s = as_stream(stream);
    if (dtype == GN_F32)
        xent_bwd_kernel<float><<<rows, 256, 0, s>>>((const float*)logits, targets, (float*)dLogits, C, scale);
    else if (dtype == GN_BF16) {
        const bool vec = C % 8 == 0 && ((uintptr_t)logits & 15u) == 0 && ((uintptr_t)dLogits & 15u) == 0;
        const int nch = (C / 8 + 255) / 256;  // 16-byte chunks per thread
        if (vec && nch <= 4)
            xent_bwd_rows_bf16<4><<<rows, 256, 0, s>>>((const bf16_t*)logits, targets, (bf16_t*)dLogits, C, scale);
        else if (vec && nch <= 8)
            xent_bwd_rows_bf16<8><<<rows, 256, 0, s>>>((const bf16_t*)logits, targets, (bf16_t*)dLogits, C, scale);
        else if (vec && nch <= 16)
            xent_bwd_rows_bf16<16><<<rows, 256, 0, s>>>((const bf16_t*)logits, targets, (bf16_t*)dLogits, C, scale);
        else
            xent_bwd_kernel<bf16_t><<<rows, 256, 0, s>>>((const bf16_t*)logits, targets, (bf16_t*)dLogits, C, scale);
    }
    else {
        set_error("gn_xent_bwd: dtype %d not supported", dtype);
        return GN_E_INVALID;
    }
    GN_LAUNCH_CHECK("gn_xent_bwd");
    return GN_OK;
}
