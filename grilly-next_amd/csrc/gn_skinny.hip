// gn_skinny.hip — fp32 Linear forward and backward for a handful of rows (M <= 8).
//
// The reference's hypernetwork runs its Linear layers on one row (vsa_training_step uploads
// one state, bindings.cpp:3152-3160; VSAHypernetwork::forward, vsa_hypernetwork.cpp:52-160).
// With M that small every contraction streams its weight matrix once and does a few flops
// per weight: the bound is HBM, not the matrix cores (the 16 x 10240 x 1536 output layer is
// 1.0 GB of fp32 weights).  These kernels therefore read W and write dW exactly once, with
// 16-byte non-temporal accesses so the streams do not evict the small operands from L2:
//
//   forward  Y[m, n] = sum_k X[m, k] W[n, k] + b[n]          one wave per row n of W
//   backward dW[n, :] (+)= sum_m dY[m, n] X[m, :]            one pass over the rows of W:
//            dX partial += dY[m, n] W[n, :]                  each block owns a row range,
//            db[n] (+)= sum_m dY[m, n]                       X stays in registers
//
// dX = dY W is a reduction over all N rows: each block writes its partial [M x K] plane to
// the caller's workspace and one more pass adds the planes in block order, so the result
// does not depend on scheduling.  Without a workspace the partials are added into dX with
// fp32 atomics (order of additions not fixed).
#include "gn_common.h"
#include "gn_sm.h"

#include <algorithm>

namespace gn {
namespace {

constexpr int kSkinnyMaxM = 8;
constexpr int kSkinnyMaxQ = 4;      // float4 chunks per thread and row: K <= 4 * 256 * 4
constexpr int kSkinnyBlocks = 1024; // row-range blocks of the backward (partial planes)

typedef float f32x4_v __attribute__((ext_vector_type(4)));

// 16-byte loads and stores marked non-temporal (streamed once: kept out of the caches' hot set)
__device__ __forceinline__ float4 ld_nt4(const float* p) {
    const f32x4_v v = __builtin_nontemporal_load(reinterpret_cast<const f32x4_v*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_nt4(float* p, float4 v) {
    f32x4_v w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, reinterpret_cast<f32x4_v*>(p));
}
__device__ __forceinline__ float dot4(float4 a, float4 b) {
    return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
}

// ---- forward: one wave per row n; lane l owns chunks c = l + 64 j of the row ------------
// Up to 8 chunks of a row are loaded before any is used (K <= 2048 in one step), so a wave
// keeps 8 KB of the weight stream in flight; longer rows take several steps.
template <int MT>
__global__ __launch_bounds__(256) void linear_fwd_skinny(const float* __restrict__ X,
                                                         const float* __restrict__ W,
                                                         const float* __restrict__ b,
                                                         float* __restrict__ Y, int M, int N,
                                                         int K) {
    const int lane = threadIdx.x & 63;
    const int nc = K >> 2;
    const float4* X4 = reinterpret_cast<const float4*>(X);
    for (int n = blockIdx.x * 4 + (threadIdx.x >> 6); n < N; n += gridDim.x * 4) {
        const float* Wr = W + (size_t)n * K;
        float acc[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] = 0.f;
        for (int c0 = 0; c0 < nc; c0 += 64 * 8) {
            float4 w[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int c = c0 + lane + 64 * j;
                w[j] = c < nc ? ld_nt4(Wr + 4 * c) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int c = c0 + lane + 64 * j;
                if (c >= nc) continue;
#pragma unroll
                for (int m = 0; m < MT; ++m)
                    if (m < M) acc[m] += dot4(w[j], X4[(size_t)m * nc + c]);
            }
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (m >= M) break;
            const float s = wave_sum(acc[m]);
            if (lane == 0) Y[(size_t)m * N + n] = s + (b ? b[n] : 0.f);
        }
    }
}

// ---- backward: block = 64 * WV threads owning float4 chunks c = t + 64 WV q (q < Q) -----
// Rows [r0, r1) of W, R rows per step, their W chunks loaded before use; with PIPE the next
// step's rows are requested before this step's dW stores, so a wave keeps a step of loads in
// flight behind its stores (one row: R = 8, up to 16 waves, one chunk per thread).
// SM: instead of storing dW, apply the surprise-momentum update to W with it (the chunk of
// dW just formed, the W chunk already loaded for dX, the surprise state s_bar streamed with
// it), writing W and s_bar in place: dW never goes to memory.  dX uses the W loaded before
// the update.
template <int MT, int Q, int R, bool PIPE, bool SM>
__global__ __launch_bounds__(MT == 1 ? 1024 : 256) void linear_bwd_skinny(
    const float* __restrict__ dY, const float* __restrict__ X, const float* W,
    float* __restrict__ dW, float* __restrict__ db, float* __restrict__ part,
    float* __restrict__ dX_atomic, int M, int N, int K, int rows_per_block, int acc_dw,
    int acc_db, int want_dx, float* s_bar, SmHyper h) {
    const int t = threadIdx.x, nthr = blockDim.x;
    const int nc = K >> 2;
    const int r0 = blockIdx.x * rows_per_block, r1 = min(N, r0 + rows_per_block);
    float4 xr[MT][Q], ax[MT][Q];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int c = t + nthr * q;
            xr[m][q] = (m < M && c < nc) ? reinterpret_cast<const float4*>(X)[(size_t)m * nc + c]
                                         : make_float4(0.f, 0.f, 0.f, 0.f);
            ax[m][q] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    float4 w[R][Q], sv[SM ? R : 1][SM ? Q : 1];
    float g[R][MT];
    auto load_rows = [&](int n0) {
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const int n = n0 + i;
#pragma unroll
            for (int m = 0; m < MT; ++m) g[i][m] = (n < r1 && m < M) ? dY[(size_t)m * N + n] : 0.f;
#pragma unroll
            for (int q = 0; q < Q; ++q) {
                const int c = t + nthr * q;
                const bool in = n < r1 && c < nc;
                w[i][q] = ((SM || want_dx) && in) ? ld_nt4(W + (size_t)n * K + 4 * c)
                                                  : make_float4(0.f, 0.f, 0.f, 0.f);
                if constexpr (SM)
                    sv[i][q] = in ? ld_nt4(s_bar + (size_t)n * K + 4 * c) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
    };
    if (PIPE) load_rows(r0);
    for (int n0 = r0; n0 < r1; n0 += R) {
        float4 wc[R][Q], sc[SM ? R : 1][SM ? Q : 1];
        float gc[R][MT];
        if (!PIPE) load_rows(n0);
#pragma unroll
        for (int i = 0; i < R; ++i) {
#pragma unroll
            for (int m = 0; m < MT; ++m) gc[i][m] = g[i][m];
#pragma unroll
            for (int q = 0; q < Q; ++q) {
                wc[i][q] = w[i][q];
                if constexpr (SM) sc[i][q] = sv[i][q];
            }
        }
        if (PIPE && n0 + R < r1) load_rows(n0 + R);
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const int n = n0 + i;
            if (n >= r1) break;
#pragma unroll
            for (int q = 0; q < Q; ++q) {
                const int c = t + nthr * q;
                if (c >= nc) continue;
                float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    o.x += gc[i][m] * xr[m][q].x;
                    o.y += gc[i][m] * xr[m][q].y;
                    o.z += gc[i][m] * xr[m][q].z;
                    o.w += gc[i][m] * xr[m][q].w;
                    ax[m][q].x += gc[i][m] * wc[i][q].x;
                    ax[m][q].y += gc[i][m] * wc[i][q].y;
                    ax[m][q].z += gc[i][m] * wc[i][q].z;
                    ax[m][q].w += gc[i][m] * wc[i][q].w;
                }
                if constexpr (SM) {
                    const float gv[4] = {o.x, o.y, o.z, o.w};
                    float sb[4] = {sc[i][q].x, sc[i][q].y, sc[i][q].z, sc[i][q].w};
                    float wv[4] = {wc[i][q].x, wc[i][q].y, wc[i][q].z, wc[i][q].w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        float d;
                        sm_elem(h, gv[e], 0.f, sb[e], wv[e], d);
                    }
                    st_nt4(const_cast<float*>(W) + (size_t)n * K + 4 * c, make_float4(wv[0], wv[1], wv[2], wv[3]));
                    st_nt4(s_bar + (size_t)n * K + 4 * c, make_float4(sb[0], sb[1], sb[2], sb[3]));
                    continue;
                }
                float* dst = dW + (size_t)n * K + 4 * c;
                if (acc_dw) {
                    const float4 p = *reinterpret_cast<const float4*>(dst);
                    o.x += p.x; o.y += p.y; o.z += p.z; o.w += p.w;
                    *reinterpret_cast<float4*>(dst) = o;
                } else {
                    st_nt4(dst, o);
                }
            }
        }
    }
    if (db) {
        for (int n = r0 + t; n < r1; n += nthr) {
            float s = 0.f;
            for (int m = 0; m < M; ++m) s += dY[(size_t)m * N + n];
            db[n] = acc_db ? db[n] + s : s;
        }
    }
    if (!want_dx) return;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        if (m >= M) break;
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int c = t + nthr * q;
            if (c >= nc) continue;
            if (part) {
                reinterpret_cast<float4*>(part)[((size_t)blockIdx.x * M + m) * nc + c] = ax[m][q];
            } else {
                float* d = dX_atomic + (size_t)m * K + 4 * c;
                atomicAdd(d, ax[m][q].x);
                atomicAdd(d + 1, ax[m][q].y);
                atomicAdd(d + 2, ax[m][q].z);
                atomicAdd(d + 3, ax[m][q].w);
            }
        }
    }
}

// out[f] (+)= sum_g part[g * L + f], g = 0..G-1 in order.  Block: 16 waves x 64 columns;
// wave w sums rows w, w + 16, ...; the waves' sums are added in a fixed order.
__global__ __launch_bounds__(1024) void plane_sum(const float* __restrict__ part, int G, int L,
                                                  float* __restrict__ out, int accumulate) {
    __shared__ float sh[16][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int f = blockIdx.x * 64 + lane;
    float s0 = 0.f, s1 = 0.f;
    if (f < L) {
        // rows g = wave + 16 i: even i into s0, odd i into s1, in order; eight rows' loads go
        // out before their adds (one memory round trip per eight rows)
        for (int g0 = wave; g0 < G; g0 += 128) {
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int g = g0 + 16 * i;
                v[i] = g < G ? part[(size_t)g * L + f] : 0.f;
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (g0 + 16 * i >= G) break;
                if (i % 2 == 0) s0 += v[i];
                else s1 += v[i];
            }
        }
    }
    sh[wave][lane] = s0 + s1;
    __syncthreads();
    if (wave == 0 && f < L) {
        float s = sh[0][lane];
#pragma unroll
        for (int w = 1; w < 16; ++w) s += sh[w][lane];
        out[f] = accumulate ? out[f] + s : s;
    }
}

__global__ void zero_f32(float* __restrict__ p, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        p[i] = 0.f;
}

inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

struct BwdShape {
    int threads, Q, blocks, rows_per_block;
};

// One row (M = 1): one float4 chunk per thread, up to 16 waves (K <= 4096).  More rows: up
// to 4 waves, Q chunks per thread (their X chunks and dX partials stay in registers).
BwdShape bwd_shape(int M, int N, int K) {
    BwdShape s{};
    const int nc = K / 4;
    s.Q = M <= 1 ? 1 : std::max(1, (nc + 255) / 256);
    const int waves = std::max(1, (nc + 64 * s.Q - 1) / (64 * s.Q));
    s.threads = 64 * waves;
    s.blocks = std::max(1, std::min(kSkinnyBlocks, (N + 15) / 16));
    s.rows_per_block = (N + s.blocks - 1) / s.blocks;
    s.rows_per_block = (s.rows_per_block + 3) & ~3;
    s.blocks = (N + s.rows_per_block - 1) / s.rows_per_block;
    return s;
}

template <int MT>
void launch_fwd_mt(const float* X, const float* W, const float* b, float* Y, int M, int N, int K,
                   hipStream_t s) {
    const unsigned grid = (unsigned)std::min<int64_t>((N + 3) / 4, 2048);
    linear_fwd_skinny<MT><<<grid, 256, 0, s>>>(X, W, b, Y, M, N, K);
}

// sm: the fused surprise-momentum update (s_bar, h) instead of the dW store
template <int MT, int Q>
void launch_bwd_mq(const BwdShape& sh, const float* dY, const float* X, const float* W, float* dW,
                   float* db, float* part, float* dXa, int M, int N, int K, int acc, int want_dx,
                   float* s_bar, const SmHyper* sm, hipStream_t s) {
    constexpr int R = MT == 1 ? 8 : 4;
    // the fused update streams s_bar next to W: half the rows per step keeps the prefetched
    // chunks within the 128 registers a 1024-thread block allows (8 rows spill)
    constexpr int RS = MT == 1 ? 4 : R;
    if (sm)
        linear_bwd_skinny<MT, Q, RS, MT == 1, true><<<sh.blocks, sh.threads, 0, s>>>(
            dY, X, W, dW, db, part, dXa, M, N, K, sh.rows_per_block, 0, acc, want_dx, s_bar, *sm);
    else
        linear_bwd_skinny<MT, Q, R, MT == 1, false><<<sh.blocks, sh.threads, 0, s>>>(
            dY, X, W, dW, db, part, dXa, M, N, K, sh.rows_per_block, acc, acc, want_dx, nullptr,
            SmHyper{});
}

template <int MT>
void launch_bwd_m(const BwdShape& sh, const float* dY, const float* X, const float* W, float* dW,
                  float* db, float* part, float* dXa, int M, int N, int K, int acc, int want_dx,
                  float* s_bar, const SmHyper* sm, hipStream_t s) {
    if constexpr (MT == 1) {
        launch_bwd_mq<1, 1>(sh, dY, X, W, dW, db, part, dXa, M, N, K, acc, want_dx, s_bar, sm, s);
    } else {
        switch (sh.Q) {
            case 1: launch_bwd_mq<MT, 1>(sh, dY, X, W, dW, db, part, dXa, M, N, K, acc, want_dx, s_bar, sm, s); break;
            case 2: launch_bwd_mq<MT, 2>(sh, dY, X, W, dW, db, part, dXa, M, N, K, acc, want_dx, s_bar, sm, s); break;
            case 3: launch_bwd_mq<MT, 3>(sh, dY, X, W, dW, db, part, dXa, M, N, K, acc, want_dx, s_bar, sm, s); break;
            default: launch_bwd_mq<MT, 4>(sh, dY, X, W, dW, db, part, dXa, M, N, K, acc, want_dx, s_bar, sm, s); break;
        }
    }
}

}  // namespace

// The skinny kernels take fp32 with M <= 8, K a multiple of 4 (K <= 4096 for the backward)
// and 16-byte aligned operands.
bool skinny_fwd_applicable(const void* X, const void* W, const void* Y, int M, int K) {
    return M >= 1 && M <= kSkinnyMaxM && K > 0 && K % 4 == 0 && al16(X) && al16(W) && al16(Y);
}

// (register budget: the rows' X chunks and dX partials, MT x Q float4 each, stay <= 8 x 2)
// The shapes the skinny backward takes (rows, K and the per-lane register budget mt * q); the
// workspace query and the dispatch share it, so no shape gets a workspace it never uses.
static bool skinny_bwd_shape_ok(int M, int K) {
    if (!(M >= 1 && M <= kSkinnyMaxM && K > 0 && K % 4 == 0 && K <= 4 * 256 * kSkinnyMaxQ))
        return false;
    const int mt = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
    const int q = (K / 4 + 255) / 256;
    return mt * q <= 16;
}

bool skinny_bwd_applicable(const void* dY, const void* X, const void* W, const void* dX,
                           const void* dW, int M, int K) {
    return skinny_bwd_shape_ok(M, K) && al16(X) && al16(W) && al16(dW) && (!dX || al16(dX)) &&
           dY != nullptr;
}

// Workspace for the deterministic dX reduction: one [M x K] fp32 plane per row-range block
// (0 for shapes the skinny kernel does not take).
size_t skinny_bwd_ws_bytes(int M, int N, int K) {
    if (N <= 0 || !skinny_bwd_shape_ok(M, K)) return 0;
    return (size_t)bwd_shape(M, N, K).blocks * M * K * sizeof(float);
}

int skinny_linear_fwd(const float* X, const float* W, const float* b, float* Y, int M, int N,
                      int K, hipStream_t s) {
    if (M <= 1) launch_fwd_mt<1>(X, W, b, Y, M, N, K, s);
    else if (M <= 2) launch_fwd_mt<2>(X, W, b, Y, M, N, K, s);
    else if (M <= 4) launch_fwd_mt<4>(X, W, b, Y, M, N, K, s);
    else launch_fwd_mt<8>(X, W, b, Y, M, N, K, s);
    GN_LAUNCH_CHECK("linear forward (skinny fp32)");
    return GN_OK;
}

// dX (nullable), dW, db (nullable); ws of skinny_bwd_ws_bytes makes dX deterministic.
// sm (nullable): apply the surprise-momentum update to W (s_bar its state) in place of the
// dW store; dW is then not touched.
int skinny_linear_bwd(const float* dY, const float* X, const float* W, float* dX, float* dW,
                      float* db, int M, int N, int K, bool accumulate, void* ws, size_t ws_bytes,
                      hipStream_t s, float* s_bar = nullptr, const SmHyper* sm = nullptr) {
    const BwdShape sh = bwd_shape(M, N, K);
    const size_t need = (size_t)sh.blocks * M * K * sizeof(float);
    float* part = (dX && ws && ws_bytes >= need && al16(ws)) ? (float*)ws : nullptr;
    float* dXa = nullptr;
    if (dX && !part) {
        dXa = dX;
        if (!accumulate) {
            zero_f32<<<grid_for((int64_t)M * K, 256, 1024), 256, 0, s>>>(dX, (int64_t)M * K);
            GN_LAUNCH_CHECK("linear backward (skinny fp32, clear dX)");
        }
    }
    const int acc = accumulate ? 1 : 0, want_dx = dX ? 1 : 0;
    if (M <= 1) launch_bwd_m<1>(sh, dY, X, W, dW, db, part, dXa, M, N, K, acc, want_dx, s_bar, sm, s);
    else if (M <= 2) launch_bwd_m<2>(sh, dY, X, W, dW, db, part, dXa, M, N, K, acc, want_dx, s_bar, sm, s);
    else if (M <= 4) launch_bwd_m<4>(sh, dY, X, W, dW, db, part, dXa, M, N, K, acc, want_dx, s_bar, sm, s);
    else launch_bwd_m<8>(sh, dY, X, W, dW, db, part, dXa, M, N, K, acc, want_dx, s_bar, sm, s);
    GN_LAUNCH_CHECK("linear backward (skinny fp32)");
    if (part) {
        const int L = M * K;
        plane_sum<<<(L + 63) / 64, 1024, 0, s>>>(part, sh.blocks, L, dX, acc);
        GN_LAUNCH_CHECK("linear backward (skinny fp32, dX planes)");
    }
    return GN_OK;
}

}  // namespace gn

// Linear backward of a few fp32 rows with the weight's surprise-momentum step fused in: the
// backward of bwd_linear (autograd.cpp:172-305; dX, db) and the optimizer's per-element
// update (surprise-momentum.glsl:53-114 with no recalled gradient, as vsa_training_step runs
// it: bindings.cpp:3198-3277, 3045-3047) in one pass over W.  W and s_bar are updated in
// place; dW is formed in registers and never stored.
extern "C" int gn_linear_bwd_surprise_momentum(const void* dY, const void* X, void* W, float* s_bar,
                                               void* dX, void* db, int M, int N, int K,
                                               float eta_base, float alpha_momentum,
                                               float lambda_recall, float surprise_floor,
                                               float weight_decay, float clip_max, void* ws,
                                               size_t ws_bytes, void* stream) {
    using namespace gn;
    clear_error();
    GN_REQUIRE(M > 0 && N > 0 && K > 0, "gn_linear_bwd_surprise_momentum: sizes must be positive");
    GN_REQUIRE(dY && X && W && s_bar, "gn_linear_bwd_surprise_momentum: null pointer (dY, X, W, s_bar)");
    GN_REQUIRE(skinny_bwd_applicable(dY, X, W, dX, s_bar, M, K),
               "gn_linear_bwd_surprise_momentum: takes M <= 8 rows, K a multiple of 4 up to 4096 "
               "and 16-byte aligned X, W, s_bar, dX (M=%d K=%d)", M, K);
    const SmHyper h{eta_base, alpha_momentum, lambda_recall, surprise_floor, weight_decay, clip_max, 0};
    return skinny_linear_bwd((const float*)dY, (const float*)X, (const float*)W, (float*)dX, nullptr,
                             (float*)db, M, N, K, false, ws, ws_bytes, as_stream(stream), s_bar, &h);
}
