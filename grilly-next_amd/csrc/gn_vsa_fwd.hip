// gn_vsa_fwd.hip — forward kernels of the VSA hypernetwork's two VSA nodes.
//
// Unpack-project forward (vsa-unpack-project.glsl:40-74,
// dispatch_vsa_unpack_project_forward vsa_loss_node.cpp:476-514):
//     Y[b, o] = sum_j s_b(j) W[o, j] + bias[o],   s_b(j) = bit (j & 31) of X[b, j >> 5] ? +1 : -1
//   * a few rows (Bn <= 8, the hypernetwork's batch of one): HBM-bound, one wave per row o of
//     W (fp32 [O x D]) streaming it once; the signs are applied by flipping the sign bit;
//   * many rows: an MFMA contraction S W^T on the GEMM core.  S = +-1 is exact in bf16 and
//     is expanded from the bits into the workspace; W is split into two bf16 terms
//     (hi = bf16(W), lo = bf16(W - hi), residual ~2^-17 |W|), so the product keeps fp32
//     accuracy: Y = S hi^T + S lo^T as two K segments of one launch, started from the bias.
//
// Surrogate-loss forward (vsa-surrogate-loss-forward.glsl passes 0 and 1 and the host
// top-2 / softmax of dispatch_vsa_loss_forward, vsa_loss_node.cpp:36-180), one block per row:
//     dots[b, k]  = sum_i preds[b, k, i] y_i                                 (pass 0)
//     (win, run)  = top-2 of dots[b, k] + T g_k, g_k Gumbel noise, by strict > in index order
//     weights[b]  = softmax(dots[b, :] / T)
//     results[b]  = {win, run, f32bits(dots[b, win]), f32bits(dots[b, run])}
//     loss[b]     = mean_i max(gamma - y_i preds[b, win, i], 0) + lambda max(0, delta - (dw - dr))
// The reference draws the noise from an unseeded std::mt19937 on the host (vsa_loss_node.cpp:
// 9-14).  Here g_k comes from a counter-based generator keyed by (seed, counter, b, k), so the
// forward is reproducible and the selection runs on the device with no host round trip.
#include "gn_common.h"
#include "gn_gemm_dma.h"

#include <algorithm>

namespace gn {
namespace {

constexpr int kVsaFwdMaxRows = 8;  // rows per pass of the streaming kernel
constexpr int kSurrogateMaxK = 64;

typedef float f32x4_v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 ld_nt4(const float* p) {
    const f32x4_v v = __builtin_nontemporal_load(reinterpret_cast<const f32x4_v*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}

// +w for bit 1, -w for bit 0 (sign-bit flip, exact)
__device__ __forceinline__ float sgn(float w, uint32_t bit) {
    return __uint_as_float(__float_as_uint(w) ^ ((~bit & 1u) << 31));
}

// sum over the four elements of a 16-byte chunk at element j0 = 4c (bits (j0 & 31) .. +3)
__device__ __forceinline__ float signed_sum4(float4 w, uint32_t nib) {
    return sgn(w.x, nib) + sgn(w.y, nib >> 1) + sgn(w.z, nib >> 2) + sgn(w.w, nib >> 3);
}

// ---- unpack-project forward, a few rows: one wave per output row o ------------------------
// Lane l owns chunks c = l + 64 j of the row (4 elements each; D % 32 == 0 so a chunk never
// straddles two words).  Rows b0 .. b0 + nb - 1 of the batch are done in one pass.
template <int MT>
__global__ __launch_bounds__(256) void vsa_fwd_rows(const uint32_t* __restrict__ bits,
                                                    const float* __restrict__ W,
                                                    const float* __restrict__ bias,
                                                    float* __restrict__ Y, int b0, int nb, int O,
                                                    int D, int words) {
    const int lane = threadIdx.x & 63;
    const int nc = D >> 2;
    for (int o = blockIdx.x * 4 + (threadIdx.x >> 6); o < O; o += gridDim.x * 4) {
        const float* Wr = W + (size_t)o * D;
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
                for (int m = 0; m < MT; ++m) {
                    if (m >= nb) break;
                    const uint32_t word = bits[(size_t)(b0 + m) * words + (c >> 3)];
                    acc[m] += signed_sum4(w[j], word >> (4 * (c & 7)));
                }
            }
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (m >= nb) break;
            const float s = wave_sum(acc[m]);
            if (lane == 0) Y[(size_t)(b0 + m) * O + o] = s + (bias ? bias[o] : 0.f);
        }
    }
}

// ---- unpack-project forward, many rows: operand preparation for the MFMA GEMM -------------
// S[b, j] = +-1 in bf16 (0x3F80 / 0xBF80): eight columns (one byte of a word) per thread.
__global__ __launch_bounds__(256) void vsa_expand_bits(const uint32_t* __restrict__ bits,
                                                       bf16_t* __restrict__ S, int64_t nbytes,
                                                       int words) {
    for (int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x; i < nbytes;
         i += (int64_t)gridDim.x * 256) {
        const int64_t wi = i >> 2;  // word index over all rows (row-major [Bn x words])
        const uint32_t byte = (bits[wi] >> (8 * (i & 3))) & 0xffu;
        uint32_t p[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t lo = (byte >> (2 * e)) & 1u ? 0x3F80u : 0xBF80u;
            const uint32_t hi = (byte >> (2 * e + 1)) & 1u ? 0x3F80u : 0xBF80u;
            p[e] = lo | (hi << 16);
        }
        // element j = 32 (wi % words) + 8 (i & 3) of row wi / words: 8 bf16 = 16 bytes
        *reinterpret_cast<uint4*>(S + 8 * i) = make_uint4(p[0], p[1], p[2], p[3]);
        (void)words;
    }
}

// hi = bf16(W), lo = bf16(W - hi), four elements per step
__global__ __launch_bounds__(256) void split_hi_lo(const float* __restrict__ W,
                                                   bf16_t* __restrict__ hi,
                                                   bf16_t* __restrict__ lo, int64_t n4) {
    for (int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x; i < n4;
         i += (int64_t)gridDim.x * 256) {
        const float4 w = ld_nt4(W + 4 * i);
        const float v[4] = {w.x, w.y, w.z, w.w};
        uint32_t h[2], l[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const float a = v[2 * e], b = v[2 * e + 1];
            h[e] = pack_bf2(a, b);
            const float ah = __uint_as_float(h[e] << 16), bh = __uint_as_float(h[e] & 0xffff0000u);
            l[e] = pack_bf2(a - ah, b - bh);
        }
        *reinterpret_cast<uint2*>(hi + 4 * i) = make_uint2(h[0], h[1]);
        *reinterpret_cast<uint2*>(lo + 4 * i) = make_uint2(l[0], l[1]);
    }
}

__global__ __launch_bounds__(256) void fill_bias_rows(const float* __restrict__ bias,
                                                      float* __restrict__ Y, int64_t total,
                                                      int O) {
    for (int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * 256)
        Y[i] = bias ? bias[i % O] : 0.f;
}

// ---- surrogate-loss forward ----------------------------------------------------------------
// splitmix64 finaliser (Steele, Lea & Flood, "Fast splittable pseudorandom number
// generators", 2014) over the Weyl sequence seed + (idx + 1) * golden ratio
__host__ __device__ __forceinline__ uint64_t mix64(uint64_t seed, uint64_t idx) {
    uint64_t x = seed + (idx + 1) * 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// Standard Gumbel sample -log(-log u), u = (23 random bits + 1/2) / 2^23, exactly
// representable in fp32 and inside (0, 1).
__device__ __forceinline__ float gumbel(uint64_t seed, uint64_t idx) {
    const float u = ((float)(uint32_t)(mix64(seed, idx) >> 41) + 0.5f) * 0x1p-23f;
    return -logf(-logf(u));
}

// one block per row, 16 waves: a row's K x D predictions are read once, up to 16 branches'
// loads in flight per thread, so a single row (batch 1) is not held to one wave's round trips
constexpr int kSurThreads = 1024, kSurWaves = kSurThreads / 64;

__global__ __launch_bounds__(kSurThreads) void surrogate_fwd_rows(
    const float* __restrict__ preds, const uint32_t* __restrict__ bits, float* __restrict__ dots,
    uint32_t* __restrict__ results, float* __restrict__ weights, float* __restrict__ loss,
    int Bn, int K, int D, int words, float gamma, float delta, float lambda_c, float temperature,
    uint64_t seed, uint64_t counter, int noise) {
    __shared__ float sh[kSurWaves];
    __shared__ float sd[kSurrogateMaxK], sadj[kSurrogateMaxK];
    __shared__ int swin;
    __shared__ float sdw, sdr;
    const int b = blockIdx.x, t = threadIdx.x;
    const uint32_t* yb = bits + (size_t)b * words;
    const int nc = D >> 2;  // D % 32 == 0
    // the branches' dot products in groups of KG: a thread's loads for all branches of a group
    // go out together (one memory round trip per chunk of D, not one per branch), each branch
    // then reduced as block_sum does (wave sum, the wave sums added in order from zero)
    constexpr int KG = 16;
    __shared__ float shk[KG][kSurWaves];
    const int wv = t >> 6, ln = t & 63;
    for (int k0 = 0; k0 < K; k0 += KG) {
        float s[KG];
#pragma unroll
        for (int j = 0; j < KG; ++j) s[j] = 0.f;
        for (int c = t; c < nc; c += kSurThreads) {
            const uint32_t nib = yb[c >> 3] >> (4 * (c & 7));
            float4 w[KG];
#pragma unroll
            for (int j = 0; j < KG; ++j)
                if (k0 + j < K) w[j] = ld_nt4(preds + ((size_t)b * K + k0 + j) * D + 4 * c);
#pragma unroll
            for (int j = 0; j < KG; ++j)
                if (k0 + j < K) s[j] += signed_sum4(w[j], nib);
        }
#pragma unroll
        for (int j = 0; j < KG; ++j) {
            if (k0 + j >= K) break;
            const float v = wave_sum(s[j]);
            if (ln == 0) shk[j][wv] = v;
        }
        __syncthreads();
        if (t < KG && k0 + t < K) {
            float tt = 0.f;
#pragma unroll
            for (int i = 0; i < kSurWaves; ++i) tt += shk[t][i];
            sd[k0 + t] = tt;
        }
        __syncthreads();
    }
    // the perturbed scores, one branch per thread
    if (t < K)
        sadj[t] = sd[t] + (noise ? gumbel(seed, ((uint64_t)counter * Bn + b) * K + t) : 0.f) *
                              temperature;
    __syncthreads();
    if (t == 0) {
        // top-2 over the perturbed scores, as the reference's host loop (vsa_loss_node.cpp:
        // 102-119): strict >, earlier index kept on ties, both start at index 0
        float max1 = -1e30f, max2 = -1e30f;
        int k1 = 0, k2 = 0;
        for (int k = 0; k < K; ++k) {
            const float adj = sadj[k];
            if (adj > max1) {
                max2 = max1; k2 = k1;
                max1 = adj; k1 = k;
            } else if (adj > max2) {
                max2 = adj; k2 = k;
            }
        }
        float mx = sd[0];
        for (int k = 1; k < K; ++k) mx = fmaxf(mx, sd[k]);
        float se = 0.f;
        for (int k = 0; k < K; ++k) se += expf((sd[k] - mx) / temperature);
        for (int k = 0; k < K; ++k) {
            dots[(size_t)b * K + k] = sd[k];
            weights[(size_t)b * K + k] = expf((sd[k] - mx) / temperature) / se;
        }
        results[(size_t)b * 4 + 0] = (uint32_t)k1;
        results[(size_t)b * 4 + 1] = (uint32_t)k2;
        results[(size_t)b * 4 + 2] = __float_as_uint(sd[k1]);
        results[(size_t)b * 4 + 3] = __float_as_uint(sd[k2]);
        swin = k1;
        sdw = sd[k1];
        sdr = sd[k2];
    }
    __syncthreads();
    const float* pw = preds + ((size_t)b * K + swin) * D;
    float h = 0.f;
    for (int c = t; c < nc; c += kSurThreads) {
        const float4 z = *reinterpret_cast<const float4*>(pw + 4 * c);
        const uint32_t nib = yb[c >> 3] >> (4 * (c & 7));
        // y z = +-z: the hinge term gamma - y z, one per element
        h += fmaxf(gamma - sgn(z.x, nib), 0.f) + fmaxf(gamma - sgn(z.y, nib >> 1), 0.f) +
             fmaxf(gamma - sgn(z.z, nib >> 2), 0.f) + fmaxf(gamma - sgn(z.w, nib >> 3), 0.f);
    }
    h = block_sum<kSurWaves>(h, sh);
    if (t == 0) loss[b] = h / (float)D + lambda_c * fmaxf(0.f, delta - (sdw - sdr));
}

inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct VsaFwdWs {
    bf16_t* S;
    bf16_t* hi;
    bf16_t* lo;
};

size_t vsa_fwd_ws_layout(int Bn, int O, int D, void* base, VsaFwdWs* w) {
    const size_t s = align256((size_t)Bn * D * 2), p = align256((size_t)O * D * 2);
    if (w) {
        char* c = (char*)base;
        w->S = (bf16_t*)c;
        w->hi = (bf16_t*)(c + s);
        w->lo = (bf16_t*)(c + s + p);
    }
    return s + 2 * p;
}

template <int MT>
void launch_rows(const uint32_t* bits, const float* W, const float* bias, float* Y, int b0, int nb,
                 int O, int D, int words, hipStream_t s) {
    const unsigned grid = (unsigned)std::min<int64_t>((O + 3) / 4, 2048);
    vsa_fwd_rows<MT><<<grid, 256, 0, s>>>(bits, W, bias, Y, b0, nb, O, D, words);
}

}  // namespace
}  // namespace gn

using namespace gn;

extern "C" size_t gn_vsa_fwd_workspace_bytes(int Bn, int O, int D) {
    if (Bn <= kVsaFwdMaxRows || O <= 0 || D <= 0) return 0;
    return vsa_fwd_ws_layout(Bn, O, D, nullptr, nullptr);
}

extern "C" int gn_vsa_unpack_project_fwd(const uint32_t* Xbits, const float* W, const float* bias,
                                         float* Y, int Bn, int O, int D, int words, void* ws,
                                         size_t ws_bytes, void* stream) {
    clear_error();
    GN_REQUIRE(Bn >= 0 && O >= 0 && D >= 0, "gn_vsa_unpack_project_fwd: negative size");
    if (Bn == 0 || O == 0) return GN_OK;
    GN_REQUIRE(D > 0 && D % 32 == 0 && words == D / 32,
               "gn_vsa_unpack_project_fwd: D=%d must be a positive multiple of 32 and words=%d = D/32",
               D, words);
    GN_REQUIRE(Xbits && W && Y, "gn_vsa_unpack_project_fwd: null pointer");
    GN_REQUIRE(al16(W), "gn_vsa_unpack_project_fwd: W must be 16-byte aligned");
    hipStream_t s = as_stream(stream);
    const size_t need = vsa_fwd_ws_layout(Bn, O, D, nullptr, nullptr);
    if (Bn > kVsaFwdMaxRows && ws && ws_bytes >= need && al16(ws) && Bn % 8 == 0 && O % 8 == 0 &&
        D % 64 == 0) {
        VsaFwdWs w;
        vsa_fwd_ws_layout(Bn, O, D, ws, &w);
        const int64_t nbytes = (int64_t)Bn * words * 4;
        vsa_expand_bits<<<grid_for(nbytes, 256, 16384), 256, 0, s>>>(Xbits, w.S, nbytes, words);
        const int64_t n4 = (int64_t)O * D / 4;
        split_hi_lo<<<grid_for(n4, 256, 16384), 256, 0, s>>>(W, w.hi, w.lo, n4);
        const int64_t total = (int64_t)Bn * O;
        fill_bias_rows<<<grid_for(total, 256, 16384), 256, 0, s>>>(bias, Y, total, O);
        GN_LAUNCH_CHECK("gn_vsa_unpack_project_fwd (operands)");
        GemmDesc d{};
        d.nseg = 2;
        d.A[0] = w.S; d.lda[0] = D; d.Ks[0] = D;
        d.B[0] = w.hi; d.ldb[0] = D;
        d.A[1] = w.S; d.lda[1] = D; d.Ks[1] = D;
        d.B[1] = w.lo; d.ldb[1] = D;
        d.M = Bn; d.N = O; d.C = Y; d.C2 = Y; d.Msplit = Bn; d.ldc = O;
        d.accumulate = 1;
        return gemm_run(d, 0, 1, GN_BF16, GN_F32, s);
    }
    // streaming kernel, eight rows of the batch per pass over W
    for (int b0 = 0; b0 < Bn; b0 += kVsaFwdMaxRows) {
        const int nb = std::min(kVsaFwdMaxRows, Bn - b0);
        if (nb <= 1) launch_rows<1>(Xbits, W, bias, Y, b0, nb, O, D, words, s);
        else if (nb <= 2) launch_rows<2>(Xbits, W, bias, Y, b0, nb, O, D, words, s);
        else if (nb <= 4) launch_rows<4>(Xbits, W, bias, Y, b0, nb, O, D, words, s);
        else launch_rows<8>(Xbits, W, bias, Y, b0, nb, O, D, words, s);
    }
    GN_LAUNCH_CHECK("gn_vsa_unpack_project_fwd");
    return GN_OK;
}

extern "C" int gn_vsa_surrogate_fwd(const float* preds, const uint32_t* bits, float* dots,
                                    uint32_t* results, float* weights, float* loss, int Bn, int K,
                                    int D, int words, float gamma, float delta, float lambda_c,
                                    float temperature, uint64_t seed, uint64_t counter,
                                    unsigned flags, void* stream) {
    clear_error();
    GN_REQUIRE(Bn >= 0 && K > 0 && D > 0, "gn_vsa_surrogate_fwd: bad shape Bn=%d K=%d D=%d", Bn, K, D);
    if (Bn == 0) return GN_OK;
    GN_REQUIRE(K <= kSurrogateMaxK, "gn_vsa_surrogate_fwd: K=%d > %d", K, kSurrogateMaxK);
    GN_REQUIRE(D % 32 == 0 && words == D / 32,
               "gn_vsa_surrogate_fwd: D=%d must be a multiple of 32 and words=%d = D/32", D, words);
    GN_REQUIRE(preds && bits && dots && results && weights && loss, "gn_vsa_surrogate_fwd: null pointer");
    GN_REQUIRE(al16(preds), "gn_vsa_surrogate_fwd: preds must be 16-byte aligned");
    GN_REQUIRE(temperature > 0.f, "gn_vsa_surrogate_fwd: temperature must be > 0");
    hipStream_t s = as_stream(stream);
    surrogate_fwd_rows<<<Bn, kSurThreads, 0, s>>>(preds, bits, dots, results, weights, loss, Bn, K, D, words,
                                          gamma, delta, lambda_c, temperature, seed, counter,
                                          (flags & GN_NO_GUMBEL) ? 0 : 1);
    GN_LAUNCH_CHECK("gn_vsa_surrogate_fwd");
    return GN_OK;
}
