// gn_attn.hip — attention backward with RoPE and causal masking (plus the forward that
// produces its saved-tensor contract: O and the fp32 row logsumexp).
//
// Semantics follow attention-backward.glsl:73-194 (dV = P^T dO, dP = dO V^T,
// dS = P (dP - rowdot) scale, dQ = dS K, dK = dS^T Q) with RoPE from
// flash-attention2-rope.glsl:73-145 applied to Q and K, so dQ and dK are rotated back with
// R^T, and a causal mask (key j <= query i).  Unlike the reference, P is never
// materialised: it is recomputed per 64x64 tile from the saved LSE, and the row dot
// D_i = sum_j P_ij dP_ij is obtained as rowsum(dO * O) (equal for a consistent forward).
//
// bf16 MFMA path (D = 64 or 128): a pre-pass writes rotated Q, K (bf16) and D_i; then
//   attn_bwd_dkdv: one block per (64-key block, b*h); loops over query blocks,
//                  S = Q K^T and dP = dO V^T (v_mfma_f32_32x32x16_bf16), P and dS written to
//                  LDS transposed, dV += P^T dO, dK += dS^T Q;
//   attn_bwd_dq:   one block per (64-query block, b*h); loops over key blocks,
//                  S^T = K Q^T, dP^T = V dO^T, dQ += dS K.
// Both keep fp32 accumulators in registers and write bf16 through an LDS-staged epilogue
// that applies the inverse rotation.  Two kernels (7 tile products instead of 5) keep the
// dQ reduction free of atomics and deterministic.
// A SIMT path (any D <= 256, fp32 or bf16) serves other shapes and the fp32 dtype.
#include <math.h>

#include "gn_common.h"

namespace gn {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ bf16x8_t afrag(const bf16_t* p) {
    uint4 v = *reinterpret_cast<const uint4*>(p);
    return __builtin_bit_cast(bf16x8_t, v);
}
__device__ __forceinline__ f32x16_t mfma(bf16x8_t a, bf16x8_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ void zero16(f32x16_t& a) {
#pragma unroll
    for (int r = 0; r < 16; ++r) a[r] = 0.f;
}

// RoPE angle for pair i at position p: p * base^(-2i/D), reduced in fp64 then sincos fp32.
__device__ __forceinline__ void rope_cs(int p, int i, int D, float theta, float& c, float& s) {
    const double inv = exp2(-2.0 * (double)i / (double)D * log2((double)theta));
    double a = (double)p * inv;
    a = a - 6.283185307179586 * rint(a * 0.15915494309189535);
    sincosf((float)a, &s, &c);
}
// pair index i and the two element positions of pair i
__device__ __forceinline__ void rope_pair(int mode, int i, int D, int& e0, int& e1) {
    if (mode == GN_ROPE_INTERLEAVED) { e0 = 2 * i; e1 = 2 * i + 1; }
    else { e0 = i; e1 = i + D / 2; }
}

// ---- pre-pass: rotated copies of Q and K, D_i = rowsum(dO * O) ------------------------
template <typename T>
__global__ __launch_bounds__(256) void rope_rotate(const T* __restrict__ X, T* __restrict__ Y,
                                                   int64_t rows, int S, int D, int mode,
                                                   float theta, int inverse) {
    const int half = D / 2;
    for (int64_t idx = blockIdx.x * (int64_t)256 + threadIdx.x; idx < rows * half;
         idx += (int64_t)gridDim.x * 256) {
        const int64_t row = idx / half;
        const int i = (int)(idx % half);
        const int p = (int)(row % S);
        int e0, e1;
        rope_pair(mode, i, D, e0, e1);
        float c, s;
        rope_cs(p, i, D, theta, c, s);
        if (inverse) s = -s;
        const float x0 = io<T>::ld(X, row * D + e0), x1 = io<T>::ld(X, row * D + e1);
        io<T>::st(Y, row * D + e0, x0 * c - x1 * s);
        io<T>::st(Y, row * D + e1, x0 * s + x1 * c);
    }
}

template <typename T>
__global__ __launch_bounds__(256) void row_dot(const T* __restrict__ A, const T* __restrict__ B,
                                               float* __restrict__ out, int64_t rows, int D) {
    const int64_t r = blockIdx.x * (int64_t)4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    float s = 0.f;
    for (int d = lane; d < D; d += 64) s += io<T>::ld(A, r * D + d) * io<T>::ld(B, r * D + d);
    s = wave_sum(s);
    if (lane == 0) out[r] = s;
}

// ---- tile loaders (64 rows x D, bf16) ---------------------------------------------------
// natural: s[row][d] (pitch D+8); rows beyond `nrows` are zero
template <int D>
__device__ __forceinline__ void load_nat(bf16_t* s, const bf16_t* __restrict__ g, int nrows) {
    constexpr int CPR = D / 8;  // 16-byte chunks per row
    for (int c = threadIdx.x; c < 64 * CPR; c += 256) {
        const int r = c / CPR, k = (c % CPR) * 8;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (r < nrows) v = *reinterpret_cast<const uint4*>(g + (size_t)r * D + k);
        *reinterpret_cast<uint4*>(s + r * (D + 8) + k) = v;
    }
}
// transposed: s[d][row] (pitch 72); 4 rows x 8 d per thread, regrouped with v_perm
template <int D>
__device__ __forceinline__ void load_tr(bf16_t* s, const bf16_t* __restrict__ g, int nrows) {
    constexpr int DC = D / 8;  // d chunks
    for (int c = threadIdx.x; c < 16 * DC; c += 256) {
        const int dc = c % DC, rg = c / DC;
        uint32_t w[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = rg * 4 + i;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (r < nrows) v = *reinterpret_cast<const uint4*>(g + (size_t)r * D + dc * 8);
            w[i][0] = v.x; w[i][1] = v.y; w[i][2] = v.z; w[i][3] = v.w;
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint2 lo, hi;
            lo.x = __builtin_amdgcn_perm(w[1][q], w[0][q], 0x05040100u);
            lo.y = __builtin_amdgcn_perm(w[3][q], w[2][q], 0x05040100u);
            hi.x = __builtin_amdgcn_perm(w[1][q], w[0][q], 0x07060302u);
            hi.y = __builtin_amdgcn_perm(w[3][q], w[2][q], 0x07060302u);
            *reinterpret_cast<uint2*>(s + (dc * 8 + 2 * q) * 72 + rg * 4) = lo;
            *reinterpret_cast<uint2*>(s + (dc * 8 + 2 * q + 1) * 72 + rg * 4) = hi;
        }
    }
}

// Store a 64 x D fp32 tile staged in LDS (pitch D+4) to global bf16, applying R^T per row.
template <int D>
__device__ __forceinline__ void store_rotated(const float* st, bf16_t* __restrict__ g, int row0,
                                              int nrows, int mode, float theta) {
    constexpr int H = D / 2;
    for (int idx = threadIdx.x; idx < 64 * H; idx += 256) {
        const int r = idx / H, i = idx % H;
        if (r >= nrows) continue;
        int e0, e1;
        if (mode == GN_ROPE_NONE) { e0 = 2 * i; e1 = 2 * i + 1; }
        else rope_pair(mode, i, D, e0, e1);
        float x0 = st[r * (D + 4) + e0], x1 = st[r * (D + 4) + e1];
        if (mode != GN_ROPE_NONE) {
            float c, s;
            rope_cs(row0 + r, i, D, theta, c, s);
            const float y0 = x0 * c + x1 * s, y1 = -x0 * s + x1 * c;  // R^T
            x0 = y0; x1 = y1;
        }
        g[(size_t)r * D + e0] = f2bf(x0);
        g[(size_t)r * D + e1] = f2bf(x1);
    }
}

// scatter a wave's 32x32 accumulator tile (rows r0.., cols c0..) into an fp32 LDS tile
__device__ __forceinline__ void stage_acc(float* st, int pitch, int r0, int c0, const f32x16_t& a,
                                          float mul) {
    const int lane = threadIdx.x & 63;
    const int col = c0 + (lane & 31), rq = (lane >> 5) * 4;
#pragma unroll
    for (int r = 0; r < 16; ++r) st[(r0 + 8 * (r >> 2) + rq + (r & 3)) * pitch + col] = a[r] * mul;
}

template <int D>
struct DkdvSmem {
    bf16_t K[64 * (D + 8)], V[64 * (D + 8)];
    union {
        struct {
            bf16_t Q[64 * (D + 8)], dO[64 * (D + 8)];
        } n;
        float stage[64 * (D + 4)];
    } u;
    bf16_t Qt[D * 72], dOt[D * 72];
    bf16_t Pt[64 * 72], dSt[64 * 72];
    float L[64], Dr[64];
};

template <int D>
__global__ __launch_bounds__(256) void attn_bwd_dkdv(
    const bf16_t* __restrict__ Qr, const bf16_t* __restrict__ Kr, const bf16_t* __restrict__ V,
    const bf16_t* __restrict__ dO, const float* __restrict__ LSE, const float* __restrict__ Di,
    bf16_t* __restrict__ dK, bf16_t* __restrict__ dV, int S, float scale, int causal,
    int rope_mode, float theta) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    DkdvSmem<D>& sm = *reinterpret_cast<DkdvSmem<D>*>(smem_raw);
    constexpr int NT = D / 64;  // 32-wide d tiles per wave in dK / dV
    const int bh = blockIdx.y, j0 = blockIdx.x * 64;
    const size_t base = (size_t)bh * S * D;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wr = wave >> 1, wc = wave & 1;
    const int fr = lane & 31, fk = (lane >> 5) * 8, rq = (lane >> 5) * 4;

    load_nat<D>(sm.K, Kr + base + (size_t)j0 * D, S - j0);
    load_nat<D>(sm.V, V + base + (size_t)j0 * D, S - j0);

    f32x16_t aV[NT], aK[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) { zero16(aV[t]); zero16(aK[t]); }

    const int nqb = (S + 63) / 64;
    for (int qb = causal ? blockIdx.x : 0; qb < nqb; ++qb) {
        const int q0 = qb * 64;
        __syncthreads();
        load_nat<D>(sm.u.n.Q, Qr + base + (size_t)q0 * D, S - q0);
        load_nat<D>(sm.u.n.dO, dO + base + (size_t)q0 * D, S - q0);
        load_tr<D>(sm.Qt, Qr + base + (size_t)q0 * D, S - q0);
        load_tr<D>(sm.dOt, dO + base + (size_t)q0 * D, S - q0);
        if (threadIdx.x < 64) {
            const int q = q0 + threadIdx.x;
            sm.L[threadIdx.x] = q < S ? LSE[(size_t)bh * S + q] : 0.f;
            sm.Dr[threadIdx.x] = q < S ? Di[(size_t)bh * S + q] : 0.f;
        }
        __syncthreads();
        // S and dP for this wave's 32 (q) x 32 (key) tile
        f32x16_t s, dp;
        zero16(s);
        zero16(dp);
#pragma unroll
        for (int ks = 0; ks < D / 16; ++ks) {
            const int k = ks * 16 + fk;
            s = mfma(afrag(&sm.u.n.Q[(wr * 32 + fr) * (D + 8) + k]), afrag(&sm.K[(wc * 32 + fr) * (D + 8) + k]), s);
            dp = mfma(afrag(&sm.u.n.dO[(wr * 32 + fr) * (D + 8) + k]), afrag(&sm.V[(wc * 32 + fr) * (D + 8) + k]), dp);
        }
        const int keyl = wc * 32 + fr, key = j0 + keyl;
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
            float pv[4], dv[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = g4 * 4 + e;
                const int ql = wr * 32 + 8 * g4 + rq + e, q = q0 + ql;
                const bool ok = q < S && key < S && (!causal || key <= q);
                const float p = ok ? __expf(s[r] * scale - sm.L[ql]) : 0.f;
                pv[e] = p;
                dv[e] = p * (dp[r] - sm.Dr[ql]);
            }
            const int ql0 = wr * 32 + 8 * g4 + rq;
            uint2 pp, dd;
            pp.x = pack_bf2(pv[0], pv[1]); pp.y = pack_bf2(pv[2], pv[3]);
            dd.x = pack_bf2(dv[0], dv[1]); dd.y = pack_bf2(dv[2], dv[3]);
            *reinterpret_cast<uint2*>(&sm.Pt[keyl * 72 + ql0]) = pp;
            *reinterpret_cast<uint2*>(&sm.dSt[keyl * 72 + ql0]) = dd;
        }
        __syncthreads();
        // dV[key][d] += P^T dO ; dK[key][d] += dS^T Q   (contraction over the 64 queries)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int k = ks * 16 + fk;
            const bf16x8_t ap = afrag(&sm.Pt[(wr * 32 + fr) * 72 + k]);
            const bf16x8_t ad = afrag(&sm.dSt[(wr * 32 + fr) * 72 + k]);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const int dcol = wc * 32 + t * 64 + fr;
                aV[t] = mfma(ap, afrag(&sm.dOt[dcol * 72 + k]), aV[t]);
                aK[t] = mfma(ad, afrag(&sm.Qt[dcol * 72 + k]), aK[t]);
            }
        }
    }
    // epilogue: dV (no rotation), then dK * scale with R^T
    __syncthreads();
#pragma unroll
    for (int t = 0; t < NT; ++t) stage_acc(sm.u.stage, D + 4, wr * 32, wc * 32 + t * 64, aV[t], 1.f);
    __syncthreads();
    store_rotated<D>(sm.u.stage, dV + base + (size_t)j0 * D, j0, S - j0, GN_ROPE_NONE, theta);
    __syncthreads();
#pragma unroll
    for (int t = 0; t < NT; ++t) stage_acc(sm.u.stage, D + 4, wr * 32, wc * 32 + t * 64, aK[t], scale);
    __syncthreads();
    store_rotated<D>(sm.u.stage, dK + base + (size_t)j0 * D, j0, S - j0, rope_mode, theta);
}

template <int D>
struct DqSmem {
    bf16_t Q[64 * (D + 8)], dO[64 * (D + 8)];
    union {
        struct {
            bf16_t K[64 * (D + 8)], V[64 * (D + 8)];
        } n;
        float stage[64 * (D + 4)];
    } u;
    bf16_t Kt[D * 72];
    bf16_t dS[64 * 72];
    float L[64], Dr[64];
};

template <int D>
__global__ __launch_bounds__(256) void attn_bwd_dq(
    const bf16_t* __restrict__ Qr, const bf16_t* __restrict__ Kr, const bf16_t* __restrict__ V,
    const bf16_t* __restrict__ dO, const float* __restrict__ LSE, const float* __restrict__ Di,
    bf16_t* __restrict__ dQ, int S, float scale, int causal, int rope_mode, float theta) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    DqSmem<D>& sm = *reinterpret_cast<DqSmem<D>*>(smem_raw);
    constexpr int NT = D / 64;
    const int bh = blockIdx.y, i0 = blockIdx.x * 64;
    const size_t base = (size_t)bh * S * D;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wr = wave >> 1, wc = wave & 1;
    const int fr = lane & 31, fk = (lane >> 5) * 8, rq = (lane >> 5) * 4;

    load_nat<D>(sm.Q, Qr + base + (size_t)i0 * D, S - i0);
    load_nat<D>(sm.dO, dO + base + (size_t)i0 * D, S - i0);
    if (threadIdx.x < 64) {
        const int q = i0 + threadIdx.x;
        sm.L[threadIdx.x] = q < S ? LSE[(size_t)bh * S + q] : 0.f;
        sm.Dr[threadIdx.x] = q < S ? Di[(size_t)bh * S + q] : 0.f;
    }
    f32x16_t aQ[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) zero16(aQ[t]);

    const int nkb = (S + 63) / 64;
    const int kb_end = causal ? (int)blockIdx.x : nkb - 1;
    for (int kb = 0; kb <= kb_end; ++kb) {
        const int k0 = kb * 64;
        __syncthreads();
        load_nat<D>(sm.u.n.K, Kr + base + (size_t)k0 * D, S - k0);
        load_nat<D>(sm.u.n.V, V + base + (size_t)k0 * D, S - k0);
        load_tr<D>(sm.Kt, Kr + base + (size_t)k0 * D, S - k0);
        __syncthreads();
        // S^T and dP^T for this wave's 32 (key) x 32 (q) tile
        f32x16_t st, dpt;
        zero16(st);
        zero16(dpt);
#pragma unroll
        for (int ks = 0; ks < D / 16; ++ks) {
            const int k = ks * 16 + fk;
            st = mfma(afrag(&sm.u.n.K[(wr * 32 + fr) * (D + 8) + k]), afrag(&sm.Q[(wc * 32 + fr) * (D + 8) + k]), st);
            dpt = mfma(afrag(&sm.u.n.V[(wr * 32 + fr) * (D + 8) + k]), afrag(&sm.dO[(wc * 32 + fr) * (D + 8) + k]), dpt);
        }
        const int ql = wc * 32 + fr, q = i0 + ql;
        const float lq = sm.L[ql], dq = sm.Dr[ql];
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
            float dv[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = g4 * 4 + e;
                const int key = k0 + wr * 32 + 8 * g4 + rq + e;
                const bool ok = q < S && key < S && (!causal || key <= q);
                const float p = ok ? __expf(st[r] * scale - lq) : 0.f;
                dv[e] = p * (dpt[r] - dq);
            }
            uint2 dd;
            dd.x = pack_bf2(dv[0], dv[1]);
            dd.y = pack_bf2(dv[2], dv[3]);
            *reinterpret_cast<uint2*>(&sm.dS[ql * 72 + wr * 32 + 8 * g4 + rq]) = dd;
        }
        __syncthreads();
        // dQ[q][d] += dS[q][key] K[key][d]
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int k = ks * 16 + fk;
            const bf16x8_t a = afrag(&sm.dS[(wr * 32 + fr) * 72 + k]);
#pragma unroll
            for (int t = 0; t < NT; ++t)
                aQ[t] = mfma(a, afrag(&sm.Kt[(wc * 32 + t * 64 + fr) * 72 + k]), aQ[t]);
        }
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < NT; ++t) stage_acc(sm.u.stage, D + 4, wr * 32, wc * 32 + t * 64, aQ[t], scale);
    __syncthreads();
    store_rotated<D>(sm.u.stage, dQ + base + (size_t)i0 * D, i0, S - i0, rope_mode, theta);
}

// ---- SIMT path: one wave per query row (dQ, forward) or key row (dK, dV) ----------------
// Each lane owns up to 4 d-values (D <= 256).  Q and K are the already-rotated tensors.
template <typename T>
__device__ __forceinline__ void ld_row(const T* p, int D, float (&v)[4]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int d = lane + 64 * e;
        v[e] = d < D ? io<T>::ld(p, d) : 0.f;
    }
}
__device__ __forceinline__ float dot4(const float (&a)[4], const float (&b)[4]) {
    return wave_sum(a[0] * b[0] + a[1] * b[1] + a[2] * b[2] + a[3] * b[3]);
}

template <typename T>
__global__ __launch_bounds__(256) void attn_fwd_simt(const T* __restrict__ Qr,
                                                     const T* __restrict__ Kr,
                                                     const T* __restrict__ V, T* __restrict__ O,
                                                     float* __restrict__ LSE, int64_t BH, int S,
                                                     int D, float scale, int causal) {
    const int64_t row = blockIdx.x * (int64_t)4 + (threadIdx.x >> 6);
    if (row >= BH * S) return;
    const int64_t bh = row / S;
    const int i = (int)(row % S);
    const size_t base = (size_t)bh * S * D;
    float q[4], o[4] = {0.f, 0.f, 0.f, 0.f};
    ld_row(Qr + base + (size_t)i * D, D, q);
    float m = -INFINITY, l = 0.f;
    const int jn = causal ? i + 1 : S;
    for (int j = 0; j < jn; ++j) {
        float k[4], v[4];
        ld_row(Kr + base + (size_t)j * D, D, k);
        ld_row(V + base + (size_t)j * D, D, v);
        const float s = dot4(q, k) * scale;
        const float mn = fmaxf(m, s);
        const float a = __expf(m - mn), p = __expf(s - mn);
        l = l * a + p;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = o[e] * a + p * v[e];
        m = mn;
    }
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int d = lane + 64 * e;
        if (d < D) io<T>::st(O, base + (size_t)i * D + d, o[e] / l);
    }
    if (lane == 0) LSE[row] = m + __logf(l);
}

template <typename T>
__global__ __launch_bounds__(256) void attn_bwd_dq_simt(
    const T* __restrict__ Qr, const T* __restrict__ Kr, const T* __restrict__ V,
    const T* __restrict__ dO, const float* __restrict__ LSE, const float* __restrict__ Di,
    float* __restrict__ dQacc, int64_t BH, int S, int D, float scale, int causal) {
    const int64_t row = blockIdx.x * (int64_t)4 + (threadIdx.x >> 6);
    if (row >= BH * S) return;
    const int64_t bh = row / S;
    const int i = (int)(row % S);
    const size_t base = (size_t)bh * S * D;
    float q[4], g[4], acc[4] = {0.f, 0.f, 0.f, 0.f};
    ld_row(Qr + base + (size_t)i * D, D, q);
    ld_row(dO + base + (size_t)i * D, D, g);
    const float lse = LSE[row], di = Di[row];
    const int jn = causal ? i + 1 : S;
    for (int j = 0; j < jn; ++j) {
        float k[4], v[4];
        ld_row(Kr + base + (size_t)j * D, D, k);
        ld_row(V + base + (size_t)j * D, D, v);
        const float p = __expf(dot4(q, k) * scale - lse);
        const float ds = p * (dot4(g, v) - di);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] += ds * k[e];
    }
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int d = lane + 64 * e;
        if (d < D) dQacc[base + (size_t)i * D + d] = acc[e] * scale;
    }
}

template <typename T>
__global__ __launch_bounds__(256) void attn_bwd_dkdv_simt(
    const T* __restrict__ Qr, const T* __restrict__ Kr, const T* __restrict__ V,
    const T* __restrict__ dO, const float* __restrict__ LSE, const float* __restrict__ Di,
    float* __restrict__ dKacc, T* __restrict__ dV, int64_t BH, int S, int D, float scale,
    int causal) {
    const int64_t row = blockIdx.x * (int64_t)4 + (threadIdx.x >> 6);
    if (row >= BH * S) return;
    const int64_t bh = row / S;
    const int j = (int)(row % S);
    const size_t base = (size_t)bh * S * D;
    float k[4], v[4], ak[4] = {0.f, 0.f, 0.f, 0.f}, av[4] = {0.f, 0.f, 0.f, 0.f};
    ld_row(Kr + base + (size_t)j * D, D, k);
    ld_row(V + base + (size_t)j * D, D, v);
    for (int i = causal ? j : 0; i < S; ++i) {
        float q[4], g[4];
        ld_row(Qr + base + (size_t)i * D, D, q);
        ld_row(dO + base + (size_t)i * D, D, g);
        const float p = __expf(dot4(q, k) * scale - LSE[bh * S + i]);
        const float ds = p * (dot4(g, v) - Di[bh * S + i]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            av[e] += p * g[e];
            ak[e] += ds * q[e];
        }
    }
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int d = lane + 64 * e;
        if (d < D) {
            dKacc[base + (size_t)j * D + d] = ak[e] * scale;
            io<T>::st(dV, base + (size_t)j * D + d, av[e]);
        }
    }
}

// fp32 rotated-gradient accumulators -> output dtype, applying R^T
template <typename T>
__global__ __launch_bounds__(256) void unrotate_store(const float* __restrict__ acc,
                                                     T* __restrict__ out, int64_t rows, int S,
                                                     int D, int mode, float theta) {
    const int half = D / 2;
    for (int64_t idx = blockIdx.x * (int64_t)256 + threadIdx.x; idx < rows * half;
         idx += (int64_t)gridDim.x * 256) {
        const int64_t row = idx / half;
        const int i = (int)(idx % half);
        int e0, e1;
        if (mode == GN_ROPE_NONE) { e0 = 2 * i; e1 = 2 * i + 1; }
        else rope_pair(mode, i, D, e0, e1);
        float x0 = acc[row * D + e0], x1 = acc[row * D + e1];
        if (mode != GN_ROPE_NONE) {
            float c, s;
            rope_cs((int)(row % S), i, D, theta, c, s);
            const float y0 = x0 * c + x1 * s, y1 = -x0 * s + x1 * c;
            x0 = y0; x1 = y1;
        }
        io<T>::st(out, row * D + e0, x0);
        io<T>::st(out, row * D + e1, x1);
    }
}

struct AttnWs {
    void* Qr;
    void* Kr;
    float* Di;
    float* acc;  // SIMT path only: fp32 [B*H*S*D]
};

inline size_t align_up(size_t x) { return (x + 255) & ~(size_t)255; }

size_t ws_layout(int64_t BHSD, int64_t BHS, size_t esz, bool simt, void* base, AttnWs* w) {
    size_t off = 0;
    auto take = [&](size_t bytes) {
        void* p = base ? (char*)base + off : nullptr;
        off += align_up(bytes);
        return p;
    };
    AttnWs t{};
    t.Qr = take(BHSD * esz);
    t.Kr = take(BHSD * esz);
    t.Di = (float*)take(BHS * 4);
    t.acc = simt ? (float*)take(BHSD * 4) : nullptr;
    if (w) *w = t;
    return off;
}

template <typename F>
bool allow_lds(F* fn, size_t bytes) {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) == hipSuccess;
}

template <int D>
int launch_mfma_bwd(const AttnWs& w, const void* Qp, const void* Kp, const void* V, const void* dO,
                    const float* LSE, void* dQ, void* dK, void* dV, int BH, int S, float scale,
                    int causal, int rope_mode, float theta, hipStream_t s) {
    static const bool ok1 = allow_lds(attn_bwd_dkdv<D>, sizeof(DkdvSmem<D>));
    static const bool ok2 = allow_lds(attn_bwd_dq<D>, sizeof(DqSmem<D>));
    if (!ok1 || !ok2) {
        set_error("gn_attn_bwd: cannot reserve LDS (%zu / %zu B)", sizeof(DkdvSmem<D>), sizeof(DqSmem<D>));
        return GN_E_HIP;
    }
    const int nb = (S + 63) / 64;
    dim3 grid(nb, BH);
    hipLaunchKernelGGL(attn_bwd_dkdv<D>, grid, dim3(256), sizeof(DkdvSmem<D>), s,
                       (const bf16_t*)Qp, (const bf16_t*)Kp, (const bf16_t*)V, (const bf16_t*)dO,
                       LSE, w.Di, (bf16_t*)dK, (bf16_t*)dV, S, scale, causal, rope_mode, theta);
    hipLaunchKernelGGL(attn_bwd_dq<D>, grid, dim3(256), sizeof(DqSmem<D>), s,
                       (const bf16_t*)Qp, (const bf16_t*)Kp, (const bf16_t*)V, (const bf16_t*)dO,
                       LSE, w.Di, (bf16_t*)dQ, S, scale, causal, rope_mode, theta);
    GN_LAUNCH_CHECK("gn_attn_bwd (mfma)");
    return GN_OK;
}

template <typename T>
int attn_bwd_impl(const void* Q, const void* K, const void* V, const void* O, const void* dO,
                  const float* LSE, void* dQ, void* dK, void* dV, int B, int H, int S, int D,
                  float scale, int causal, int rope_mode, float theta, void* ws, size_t ws_bytes,
                  hipStream_t s) {
    const int64_t BH = (int64_t)B * H, rows = BH * S, BHSD = rows * D;
    const bool mfma_ok = sizeof(T) == 2 && (D == 64 || D == 128);
    AttnWs w;
    const size_t need = ws_layout(BHSD, rows, sizeof(T), !mfma_ok, ws, &w);
    if (!ws || ws_bytes < need) {
        set_error("gn_attn_bwd: workspace %zu B < %zu B", ws_bytes, need);
        return GN_E_WORKSPACE;
    }
    const void* Qp = Q;
    const void* Kp = K;
    if (rope_mode != GN_ROPE_NONE) {
        const unsigned g = grid_for(rows * (D / 2), 256, 16384);
        rope_rotate<T><<<g, 256, 0, s>>>((const T*)Q, (T*)w.Qr, rows, S, D, rope_mode, theta, 0);
        rope_rotate<T><<<g, 256, 0, s>>>((const T*)K, (T*)w.Kr, rows, S, D, rope_mode, theta, 0);
        Qp = w.Qr;
        Kp = w.Kr;
    }
    row_dot<T><<<(unsigned)((rows + 3) / 4), 256, 0, s>>>((const T*)dO, (const T*)O, w.Di, rows, D);
    GN_LAUNCH_CHECK("gn_attn_bwd (pre-pass)");
    if (mfma_ok) {
        if (D == 64)
            return launch_mfma_bwd<64>(w, Qp, Kp, V, dO, LSE, dQ, dK, dV, (int)BH, S, scale, causal,
                                       rope_mode, theta, s);
        return launch_mfma_bwd<128>(w, Qp, Kp, V, dO, LSE, dQ, dK, dV, (int)BH, S, scale, causal,
                                    rope_mode, theta, s);
    }
    const unsigned gr = (unsigned)((rows + 3) / 4);
    const unsigned ge = grid_for(rows * (D / 2), 256, 16384);
    attn_bwd_dq_simt<T><<<gr, 256, 0, s>>>((const T*)Qp, (const T*)Kp, (const T*)V, (const T*)dO,
                                           LSE, w.Di, w.acc, BH, S, D, scale, causal);
    unrotate_store<T><<<ge, 256, 0, s>>>(w.acc, (T*)dQ, rows, S, D, rope_mode, theta);
    attn_bwd_dkdv_simt<T><<<gr, 256, 0, s>>>((const T*)Qp, (const T*)Kp, (const T*)V,
                                             (const T*)dO, LSE, w.Di, w.acc, (T*)dV, BH, S, D,
                                             scale, causal);
    unrotate_store<T><<<ge, 256, 0, s>>>(w.acc, (T*)dK, rows, S, D, rope_mode, theta);
    GN_LAUNCH_CHECK("gn_attn_bwd (simt)");
    return GN_OK;
}

}  // namespace
}  // namespace gn

using namespace gn;

extern "C" size_t gn_attn_workspace_bytes(int B, int H, int S, int D) {
    if (B <= 0 || H <= 0 || S <= 0 || D <= 0) return 0;
    const int64_t rows = (int64_t)B * H * S;
    // sized for the larger (SIMT, fp32) layout so one query covers every dtype
    return ws_layout(rows * D, rows, 4, true, nullptr, nullptr);
}

static int attn_check(const void* Q, const void* K, const void* V, int B, int H, int S, int D,
                      int rope_mode, int dtype) {
    GN_REQUIRE(B >= 0 && H >= 0 && S >= 0 && D > 0, "attention: bad shape");
    GN_REQUIRE(Q && K && V, "attention: null pointer");
    GN_REQUIRE(D <= 256 && D % 2 == 0, "attention: D=%d must be even and <= 256", D);
    GN_REQUIRE(rope_mode >= GN_ROPE_NONE && rope_mode <= GN_ROPE_HALF, "attention: rope_mode %d", rope_mode);
    GN_REQUIRE(dtype == GN_F32 || dtype == GN_BF16, "attention: dtype %d", dtype);
    GN_REQUIRE((int64_t)B * H <= 65535, "attention: B*H exceeds grid.y limit");
    return GN_OK;
}

extern "C" int gn_attn_bwd(const void* Q, const void* K, const void* V, const void* O,
                           const void* dO, const float* LSE, void* dQ, void* dK, void* dV, int B,
                           int H, int S, int D, float scale, int causal, int rope_mode,
                           float rope_theta, int dtype, void* ws, size_t ws_bytes,
                           void* stream) {
    clear_error();
    int rc = attn_check(Q, K, V, B, H, S, D, rope_mode, dtype);
    if (rc) return rc;
    if ((int64_t)B * H * S == 0) return GN_OK;
    GN_REQUIRE(O && dO && LSE && dQ && dK && dV, "gn_attn_bwd: null pointer");
    hipStream_t s = as_stream(stream);
    if (dtype == GN_BF16)
        return attn_bwd_impl<bf16_t>(Q, K, V, O, dO, LSE, dQ, dK, dV, B, H, S, D, scale, causal,
                                     rope_mode, rope_theta, ws, ws_bytes, s);
    return attn_bwd_impl<float>(Q, K, V, O, dO, LSE, dQ, dK, dV, B, H, S, D, scale, causal,
                                rope_mode, rope_theta, ws, ws_bytes, s);
}

extern "C" int gn_attn_fwd(const void* Q, const void* K, const void* V, void* O, float* LSE,
                           int B, int H, int S, int D, float scale, int causal, int rope_mode,
                           float rope_theta, int dtype, void* ws, size_t ws_bytes, void* stream) {
    clear_error();
    int rc = attn_check(Q, K, V, B, H, S, D, rope_mode, dtype);
    if (rc) return rc;
    const int64_t rows = (int64_t)B * H * S;
    if (rows == 0) return GN_OK;
    GN_REQUIRE(O && LSE, "gn_attn_fwd: null pointer");
    hipStream_t s = as_stream(stream);
    const size_t esz = dtype == GN_BF16 ? 2 : 4;
    AttnWs w;
    const size_t need = ws_layout(rows * D, rows, esz, false, ws, &w);
    if (rope_mode != GN_ROPE_NONE && (!ws || ws_bytes < need)) {
        set_error("gn_attn_fwd: workspace %zu B < %zu B", ws_bytes, need);
        return GN_E_WORKSPACE;
    }
    const void* Qp = Q;
    const void* Kp = K;
    if (rope_mode != GN_ROPE_NONE) {
        const unsigned g = grid_for(rows * (D / 2), 256, 16384);
        if (dtype == GN_BF16) {
            rope_rotate<bf16_t><<<g, 256, 0, s>>>((const bf16_t*)Q, (bf16_t*)w.Qr, rows, S, D, rope_mode, rope_theta, 0);
            rope_rotate<bf16_t><<<g, 256, 0, s>>>((const bf16_t*)K, (bf16_t*)w.Kr, rows, S, D, rope_mode, rope_theta, 0);
        } else {
            rope_rotate<float><<<g, 256, 0, s>>>((const float*)Q, (float*)w.Qr, rows, S, D, rope_mode, rope_theta, 0);
            rope_rotate<float><<<g, 256, 0, s>>>((const float*)K, (float*)w.Kr, rows, S, D, rope_mode, rope_theta, 0);
        }
        Qp = w.Qr;
        Kp = w.Kr;
    }
    const unsigned gr = (unsigned)((rows + 3) / 4);
    if (dtype == GN_BF16)
        attn_fwd_simt<bf16_t><<<gr, 256, 0, s>>>((const bf16_t*)Qp, (const bf16_t*)Kp, (const bf16_t*)V,
                                                 (bf16_t*)O, LSE, (int64_t)B * H, S, D, scale, causal);
    else
        attn_fwd_simt<float><<<gr, 256, 0, s>>>((const float*)Qp, (const float*)Kp, (const float*)V,
                                                (float*)O, LSE, (int64_t)B * H, S, D, scale, causal);
    GN_LAUNCH_CHECK("gn_attn_fwd");
    return GN_OK;
}
