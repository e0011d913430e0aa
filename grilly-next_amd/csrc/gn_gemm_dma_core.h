// gn_gemm_dma_core.h — gfx950 GEMM core: LDS-DMA staging + transpose reads.  Kernel and
// launch templates (internal linkage); gn_gemm_dma.hip holds the dispatch and the VSA
// weight-gradient launch, and gn_gemm_dma_{f32a,f32b,bf16,glu}.hip instantiate the GEMM
// launches per output type / epilogue (/ A orientation), so the builds run in parallel.
//
//   C[M x N] (+)= sum_s opA(A_s) opB(B_s)        (up to two K-segments, own leading dims)
//
// Block tile BM x BN x 64, 256 threads = 2 x 2 waves, wave tile (BM/2) x (BN/2) built from
// v_mfma_f32_32x32x16_bf16 with fp32 accumulators.  Global -> LDS moves use the 16-byte
// `global_load_lds` DMA (no VGPR staging) into two or three LDS stages, so the DMA of the
// next tiles runs while the MFMAs of the current one execute.  Each operand stays in LDS in its global orientation:
//   * k-contiguous operand (rows of 64 k):   [row][k], 16-byte chunk c of row r stored at
//     chunk c ^ swz(r); MFMA fragments are single ds_read_b128;
//   * k-outer operand (rows of BM/BN columns): [k][col], chunk c of k-row k stored at
//     c ^ fko(k); fragments come from ds_read_b64_tr_b16, which transposes a 4(k) x 16
//     block across each 16-lane group (lane i gets column i, four consecutive k).
// The DMA lane -> global-address map applies the inverse swizzle, so every DMA
// instruction still reads whole 128-byte (or longer) row segments.
// Epilogues: plain store (bf16 or fp32, optional accumulate, optional row split into two
// outputs) or the GLU epilogue, which turns the dA tile of the down projection straight
// into the SwiGLU/GEGLU/ReGLU local gradients (dA never reaches HBM).
#pragma once

#include <cstdlib>
#include <type_traits>
#include <utility>

#include "gn_common.h"
#include "gn_gemm_dma.h"
#include "gn_math.h"
#include "gn_mfma.h"

namespace gn {
namespace {

constexpr int BK = 64;

__device__ __forceinline__ int swz(int r) { return (r ^ (r >> 3)) & 7; }
// k-outer tiles: chunk c of k-row k sits at c ^ fko(k), fko = {0, 6, 10, 12}[k & 3].  A
// transpose read covers 4 consecutive k-rows x 64 bytes per 32 lanes; these four values
// differ in bits 1-2 and in bits 2-3, so the read is conflict-free on a 32-bank and on a
// 64-bank (gfx950) LDS alike (2(k & 3) left 2-way conflicts on 64 banks).
__device__ __forceinline__ int fko(int k) { return ((k & 1) * 6) ^ (((k >> 1) & 1) * 10); }

// Stage one operand tile of R rows/cols (R = BM or BN) into LDS (R*64 bf16 = R*8 chunks,
// R/8 DMA instructions, R/32 per wave).
//   KC (k-contiguous): element (r, k) at P[r*ld + k]; tile stored [r][64], chunk-swizzled
//   else (k-outer):    element (r, k) at P[k*ld + r]; tile stored [64][R], chunk-swizzled
template <int R, bool KC, int NW, int J0 = 0, int J1 = R / (8 * NW)>
__device__ __forceinline__ void stage(const bf16_t* __restrict__ P, int ld, int r0, int rlim,
                                      int k0, uint32_t s) {
    const int lane = threadIdx.x & 63, wave = (threadIdx.x >> 6) & (NW - 1);
    static_assert(R % (8 * NW) == 0, "whole DMA instructions per wave");
#pragma unroll
    for (int j = J0; j < J1; ++j) {
        const int q = wave * (R / (8 * NW)) + j;  // DMA instruction index: slots [64q, 64q+64)
        const int slot = 64 * q + lane;
        const bf16_t* src;
        if (KC) {
            const int r = slot >> 3, p = slot & 7;
            const int c = p ^ swz(r);
            const int rr = min(r0 + r, rlim - 1);  // rows past the edge re-read a valid row
            src = P + (size_t)rr * ld + k0 + c * 8;
        } else {
            constexpr int CPR = R / 8;  // chunks per k-row
            const int k = slot / CPR, p = slot % CPR;
            const int c = p ^ fko(k);
            const int col = min(r0 + c * 8, rlim - 8);
            src = P + (size_t)(k0 + k) * ld + col;
        }
        dma16(src, __builtin_amdgcn_readfirstlane(s + 64 * 16 * q));
    }
}

// Lane byte offsets of the wave's DMA instructions of stage<R, KC, NW> (same element map),
// relative to the tile base stage_base<KC>(P, ld, r0, k0); independent of k0.
template <int R, bool KC, int NW, int NJ = R / (8 * NW)>
__device__ __forceinline__ void stage_offsets(int ld, int r0, int rlim, int wave, uint32_t (&vo)[NJ]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int slot = 64 * (wave * NJ + j) + lane;
        if (KC) {
            const int r = slot >> 3, c = (slot & 7) ^ swz(r);
            const int rr = min(r0 + r, rlim - 1) - r0;  // rows past the edge re-read a valid row
            vo[j] = (uint32_t)(rr * ld + c * 8) * 2u;
        } else {
            constexpr int CPR = R / 8;
            const int k = slot / CPR, c = (slot % CPR) ^ fko(k);
            const int col = min(r0 + c * 8, rlim - 8) - r0;
            vo[j] = (uint32_t)(k * ld + col) * 2u;
        }
    }
}

template <bool KC>
__device__ __forceinline__ const bf16_t* stage_base(const bf16_t* P, int ld, int r0, int k0) {
    return KC ? P + (size_t)r0 * ld + k0 : P + (size_t)k0 * ld + r0;
}

// A-type fragment (32 rows x 16 k) for v_mfma_f32_32x32x16_bf16: lane l -> row l%32,
// k = 8(l/32) .. +7 within k-step ks.
template <int R, bool KC>
__device__ __forceinline__ bf16x8_t frag(const bf16_t* s, int row0, int ks) {
    const int lane = threadIdx.x & 63;
    if (KC) {
        const int r = row0 + (lane & 31);
        const int c = ks * 2 + (lane >> 5);
        uint4 v = *reinterpret_cast<const uint4*>(s + r * BK + ((c ^ swz(r)) * 8));
        return __builtin_bit_cast(bf16x8_t, v);
    } else {
        // 16-lane group g: columns row0 + 16(g%2) .. +15, k = ks*16 + 8(g/2) + {0..3, 4..7}
        const int g = lane >> 4, sl = lane & 15;
        const int col = row0 + 16 * (g & 1) + 4 * (sl & 3);
        const int k = ks * 16 + 8 * (g >> 1) + (sl >> 2);
        const int c = col >> 3, within = col & 7;
        const bf16_t* p0 = s + k * R + ((c ^ fko(k)) * 8) + within;
        const bf16_t* p1 = p0 + 4 * R;  // k + 4 (same swizzle: fko(k+4) == fko(k))
        s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p0));
        s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p1));
        s16x8_t v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        return __builtin_bit_cast(bf16x8_t, v);
    }
}

// GLU local gradients of 8 consecutive elements (gate/up given as 4 packed bf16 pairs).
template <int KIND>
__device__ __forceinline__ void glu8(const float (&v)[8], const uint32_t (&gg)[4],
                                     const uint32_t (&uu)[4], float (&dg)[8], float (&du)[8]) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float gt = __uint_as_float((e & 1) ? (gg[e >> 1] & 0xffff0000u) : (gg[e >> 1] << 16));
        const float up = __uint_as_float((e & 1) ? (uu[e >> 1] & 0xffff0000u) : (uu[e >> 1] << 16));
        glu_grad<KIND>(v[e], gt, up, dg[e], du[e]);
    }
}

// Write one staged 32 x WN strip (LDS, fp32, pitch WN+4) to global memory: lane l owns
// row l/2 and WN/2 consecutive columns, moved 8 at a time with 16-byte accesses.
template <typename CT, int EPI, int WN>
__device__ __forceinline__ void epilogue_rows(const GemmDesc& g, const float* st, int mbase, int nbase,
                                           int lane) {
        const int rr = lane >> 1;
        const int m = mbase + rr;
#pragma unroll
        for (int q = 0; q < WN / 16; ++q) {
            const int c = (lane & 1) * (WN / 2) + q * 8;
            const int n = nbase + c;
            const float4 lo = *reinterpret_cast<const float4*>(st + rr * (WN + 4) + c);
            const float4 hi = *reinterpret_cast<const float4*>(st + rr * (WN + 4) + c + 4);
            float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
            if (m >= g.M || n >= g.N) continue;
            if constexpr (EPI == 0) {
                if (g.cbias) {
                    const uint4 bw = *reinterpret_cast<const uint4*>(g.cbias + n);
                    const uint32_t w[4] = {bw.x, bw.y, bw.z, bw.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        v[2 * e] += __uint_as_float(w[e] << 16);
                        v[2 * e + 1] += __uint_as_float(w[e] & 0xffff0000u);
                    }
                }
                CT* C = reinterpret_cast<CT*>(m < g.Msplit ? g.C : g.C2);
                const size_t idx = (size_t)(m < g.Msplit ? m : m - g.Msplit) * g.ldc + n;
                if constexpr (sizeof(CT) == 4) {
                    float4* p = reinterpret_cast<float4*>(reinterpret_cast<float*>(C) + idx);
                    if (g.accumulate) {
                        const float4 o0 = p[0], o1 = p[1];
                        v[0] += o0.x; v[1] += o0.y; v[2] += o0.z; v[3] += o0.w;
                        v[4] += o1.x; v[5] += o1.y; v[6] += o1.z; v[7] += o1.w;
                    }
                    p[0] = make_float4(v[0], v[1], v[2], v[3]);
                    p[1] = make_float4(v[4], v[5], v[6], v[7]);
                } else {
                    uint4* p = reinterpret_cast<uint4*>(reinterpret_cast<bf16_t*>(C) + idx);
                    if (g.accumulate) {
                        const uint4 o = *p;
                        const uint32_t w[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            v[2 * e] += __uint_as_float(w[e] << 16);
                            v[2 * e + 1] += __uint_as_float(w[e] & 0xffff0000u);
                        }
                    }
                    *p = make_uint4(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]), pack_bf2(v[4], v[5]),
                                    pack_bf2(v[6], v[7]));
                }
            } else {
                const size_t gi = (size_t)m * g.ldg + n;
                const uint4 gw = *reinterpret_cast<const uint4*>(g.gate + gi);
                const uint4 uw = *reinterpret_cast<const uint4*>(g.up + gi);
                const uint32_t gg[4] = {gw.x, gw.y, gw.z, gw.w}, uu[4] = {uw.x, uw.y, uw.z, uw.w};
                float dg[8], du[8];
                switch (g.glu_kind) {
                    case GN_GLU_SWIGLU_UP: glu8<GN_GLU_SWIGLU_UP>(v, gg, uu, dg, du); break;
                    case GN_GLU_SWIGLU_GATE: glu8<GN_GLU_SWIGLU_GATE>(v, gg, uu, dg, du); break;
                    case GN_GLU_GEGLU_UP: glu8<GN_GLU_GEGLU_UP>(v, gg, uu, dg, du); break;
                    case GN_GLU_GEGLU_GATE: glu8<GN_GLU_GEGLU_GATE>(v, gg, uu, dg, du); break;
                    default: glu8<GN_GLU_REGLU_UP>(v, gg, uu, dg, du); break;
                }
                bf16_t* o = g.gu + (size_t)m * g.ldgu + n;
                *reinterpret_cast<uint4*>(o) = make_uint4(pack_bf2(dg[0], dg[1]), pack_bf2(dg[2], dg[3]),
                                                          pack_bf2(dg[4], dg[5]), pack_bf2(dg[6], dg[7]));
                *reinterpret_cast<uint4*>(o + g.H) = make_uint4(pack_bf2(du[0], du[1]), pack_bf2(du[2], du[3]),
                                                                pack_bf2(du[4], du[5]), pack_bf2(du[6], du[7]));
            }
        }
}

template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// GLU epilogue of the four-wave core.  A strip is 32 rows x WN columns of dO; its gate/up
// elements are fetched into registers with a coalesced map (LPR = WN/8 lanes per row, each
// lane 8 consecutive columns = one 16-byte load, so a row segment is one contiguous
// 2*WN-byte run), all loads of a strip issued before any of its math, and (for WN = 64)
// the next strip's loads issued before this strip's math so they overlap it.  Rows and
// columns past the matrix edge load a clamped in-bounds element and are not stored.
template <int WN>
struct GluStrip {
    static constexpr int LPR = WN / 8, RP = 64 / LPR, NP = 32 / RP;
    uint4 g[NP], u[NP];
};

template <int WN>
__device__ __forceinline__ void glu_fetch(const GemmDesc& g, int mbase, int nbase, int lane,
                                          GluStrip<WN>& t) {
    using S = GluStrip<WN>;
    const int n = min(nbase + (lane % S::LPR) * 8, g.N - 8);
#pragma unroll
    for (int p = 0; p < S::NP; ++p) {
        const int m = min(mbase + p * S::RP + lane / S::LPR, g.M - 1);
        const size_t gi = (size_t)m * g.ldg + n;
        t.g[p] = *reinterpret_cast<const uint4*>(g.gate + gi);
        t.u[p] = *reinterpret_cast<const uint4*>(g.up + gi);
    }
}

template <int KIND, int WN>
__device__ __forceinline__ void glu_store(const GemmDesc& g, const float* st, int mbase, int nbase,
                                          int lane, const GluStrip<WN>& t) {
    using S = GluStrip<WN>;
    const int c = (lane % S::LPR) * 8;
    const int n = nbase + c;
#pragma unroll
    for (int p = 0; p < S::NP; ++p) {
        const int rr = p * S::RP + lane / S::LPR;
        const int m = mbase + rr;
        const float4 lo = *reinterpret_cast<const float4*>(st + rr * (WN + 4) + c);
        const float4 hi = *reinterpret_cast<const float4*>(st + rr * (WN + 4) + c + 4);
        const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        if (m >= g.M || n >= g.N) continue;
        const uint32_t gg[4] = {t.g[p].x, t.g[p].y, t.g[p].z, t.g[p].w};
        const uint32_t uu[4] = {t.u[p].x, t.u[p].y, t.u[p].z, t.u[p].w};
        float dg[8], du[8];
        glu8<KIND>(v, gg, uu, dg, du);
        bf16_t* o = g.gu + (size_t)m * g.ldgu + n;
        *reinterpret_cast<uint4*>(o) = make_uint4(pack_bf2(dg[0], dg[1]), pack_bf2(dg[2], dg[3]),
                                                  pack_bf2(dg[4], dg[5]), pack_bf2(dg[6], dg[7]));
        *reinterpret_cast<uint4*>(o + g.H) = make_uint4(pack_bf2(du[0], du[1]), pack_bf2(du[2], du[3]),
                                                        pack_bf2(du[4], du[5]), pack_bf2(du[6], du[7]));
    }
}

// Whole GLU epilogue of one wave's (32 FM) x WN accumulator block, strip by strip through
// the wave's private LDS strip `st` (fp32, pitch WN + 4).
template <int KIND, int FM, int FN, int WN>
__device__ __forceinline__ void glu_epilogue(const GemmDesc& g, const f32x16_t (&acc)[FM][FN], float* st,
                                             int mbase, int nbase, int lane) {
    constexpr bool AHEAD = WN <= 64;  // registers for two strips of gate/up
    GluStrip<WN> t[AHEAD ? 2 : 1];
    const int rq = (lane >> 5) * 4;
    glu_fetch<WN>(g, mbase, nbase, lane, t[0]);
    static_for<FM>([&](auto I_) {
        constexpr int i = decltype(I_)::value;
        constexpr int cur = AHEAD ? (i & 1) : 0;
        if constexpr (!AHEAD) {
            if constexpr (i > 0) glu_fetch<WN>(g, mbase + i * 32, nbase, lane, t[0]);
        }
        wave_lds_sync();  // the previous strip's reads (other lanes) before these writes
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                st[(8 * (r >> 2) + rq + (r & 3)) * (WN + 4) + j * 32 + (lane & 31)] = acc[i][j][r];
        wave_lds_sync();  // these writes before other lanes read them
        if constexpr (AHEAD && i + 1 < FM) glu_fetch<WN>(g, mbase + (i + 1) * 32, nbase, lane, t[cur ^ 1]);
        glu_store<KIND, WN>(g, st, mbase + i * 32, nbase, lane, t[cur]);
    });
}

// Split-K epilogue (fp32 C, cleared beforehand): the strip's rows are added into C with
// hardware fp32 atomics, one row per instruction round (lane = column: 256-byte segments).
template <int WN>
__device__ __forceinline__ void epilogue_atomic(const GemmDesc& g, const float* st, int mbase,
                                                int nbase, int lane) {
#pragma unroll 4
    for (int rr = 0; rr < 32; ++rr) {
        const int m = mbase + rr;
        if (m >= g.M) break;
        float* C = reinterpret_cast<float*>(m < g.Msplit ? g.C : g.C2) +
                   (size_t)(m < g.Msplit ? m : m - g.Msplit) * g.ldc;
#pragma unroll
        for (int c = lane; c < WN; c += 64)
            if (nbase + c < g.N) unsafeAtomicAdd(C + nbase + c, st[rr * (WN + 4) + c]);
    }
}

// C rows (and C2 rows past Msplit) cleared before a split-K launch
__global__ __launch_bounds__(256) void clear_c(GemmDesc g) {
    const int64_t total = (int64_t)g.M * g.N;
    for (int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int m = (int)(i / g.N), n = (int)(i % g.N);
        float* C = reinterpret_cast<float*>(m < g.Msplit ? g.C : g.C2);
        C[(size_t)(m < g.Msplit ? m : m - g.Msplit) * g.ldc + n] = 0.f;
        if (g.bias && n == 0) (m < g.Msplit ? g.bias[m] : g.bias2[m - g.Msplit]) = 0.f;
    }
}

// Split-K through a workspace: the strip's rows go to this split's partial tile (plain
// 16-byte stores, the layout of epilogue_rows; N % 8 == 0 on this core).
template <int WN>
__device__ __forceinline__ void epilogue_part(const GemmDesc& g, const float* st, int mbase,
                                              int nbase, int lane) {
    const int rr = lane >> 1;
    const int m = mbase + rr;
    if (m >= g.M) return;
    float* P = g.part + (size_t)blockIdx.y * g.M * g.N + (size_t)m * g.N;
#pragma unroll
    for (int q = 0; q < WN / 16; ++q) {
        const int c = (lane & 1) * (WN / 2) + q * 8;
        const int n = nbase + c;
        if (n >= g.N) continue;
        const float4 lo = *reinterpret_cast<const float4*>(st + rr * (WN + 4) + c);
        const float4 hi = *reinterpret_cast<const float4*>(st + rr * (WN + 4) + c + 4);
        float4* p = reinterpret_cast<float4*>(P + n);
        p[0] = lo;
        p[1] = hi;
    }
}

// C (+)= the sum over y = 0 .. ksplit-1 of the partial tiles, added in index order (one
// thread per 4 columns of a row), rows below Msplit to C, the rest to C2; then the bias.
// The planes' loads go out together, up to eight per memory round trip (ksplit is uniform,
// so the guards are uniform branches with no wait between the loads), and are then added in
// index order.
__global__ __launch_bounds__(256) void split_reduce(GemmDesc g) {
    const int n4 = g.N / 4;
    const int64_t total = (int64_t)g.M * n4;
    const size_t plane = (size_t)g.M * g.N;
    const int ks = g.ksplit;
    for (int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int m = (int)(i / n4), n = (int)(i % n4) * 4;
        const float* src = g.part + (size_t)m * g.N + n;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int y0 = 0; y0 < ks; y0 += 8) {
            float4 w[8];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (y0 + j < ks) w[j] = *reinterpret_cast<const float4*>(src + (size_t)(y0 + j) * plane);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (y0 + j >= ks) break;
                if (y0 + j == 0) {
                    v = w[0];
                } else {
                    v.x += w[j].x; v.y += w[j].y; v.z += w[j].z; v.w += w[j].w;
                }
            }
        }
        float4* c4 = reinterpret_cast<float4*>(reinterpret_cast<float*>(m < g.Msplit ? g.C : g.C2) +
                                               (size_t)(m < g.Msplit ? m : m - g.Msplit) * g.ldc + n);
        if (g.accumulate) {
            const float4 o = *c4;
            v.x = o.x + v.x; v.y = o.y + v.y; v.z = o.z + v.z; v.w = o.w + v.w;
        }
        *c4 = v;
    }
    if (g.bias) {
        const float* bp = g.part + (size_t)g.ksplit * plane;
        for (int64_t m = blockIdx.x * (int64_t)256 + threadIdx.x; m < g.M; m += (int64_t)gridDim.x * 256) {
            float v = 0.f;
            for (int y0 = 0; y0 < ks; y0 += 8) {
                float w[8];
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (y0 + j < ks) w[j] = bp[(size_t)(y0 + j) * g.M + m];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    if (y0 + j >= ks) break;
                    v = y0 + j == 0 ? w[0] : v + w[j];
                }
            }
            float* dst = m < g.Msplit ? g.bias + m : g.bias2 + (m - g.Msplit);
            *dst = g.accumulate ? *dst + v : v;
        }
    }
}

// ---- GEMM core -------------------------------------------------------------------------
// Four waves (2 x 2, one per SIMD), wave tile (BM/2) x (BN/2), two or three LDS stages.  Every
// MFMA operand is read from LDS two k-steps before its MFMAs run, into one of four register
// sets (set = k-step within the tile, so every index is a compile-time constant).  Per tile t
// (stage S = t & 1):
//   k-step 0: MFMAs of set 0; reads of (t, 2) from S into set 2, spread over the MFMAs;
//   k-step 1: MFMAs of set 1; reads of (t, 3) from S into set 3, all issued in the first
//             half so they have landed by the end of the step;
//             then vmcnt(0) (this wave's DMA of tile t+1) + lgkmcnt(0) + one barrier:
//             tile t+1 is visible to every wave and stage S has no reader left;
//   k-step 2: MFMAs of set 2; DMA of tile t+2 into S and reads of (t+1, 0) from S^1;
//   k-step 3: MFMAs of set 3; reads of (t+1, 1) from S^1 into set 1.
// Each MFMA's operands were requested at least one full k-step earlier, so the wave never
// waits on an LDS read that was issued a couple of MFMAs before.
template <int NM, int NR, bool FRONT>
__host__ __device__ constexpr int reads_before(int q) {
    // number of fragment reads issued after MFMAs 0..q-1 (spread evenly over NM, or over the
    // first half of them when FRONT)
    return FRONT ? (q >= (NM + 1) / 2 ? NR : (NR * q + (NM + 1) / 2 - 1) / ((NM + 1) / 2))
                 : (NR * q + NM - 1) / NM;
}

// BPAR: with BIAS, the two waves of a wave row (wn = 0, 1) hold the same A fragments; the
// wave with wn == BPAR sums the row sums of the fragments i with i % 2 == BPAR only, so each
// row is summed once (-1: no bias).
// PROD = 4: four more waves (one per SIMD) issue every LDS DMA of the block, so the four
// compute waves never stall on a DMA instruction's issue (a wave that issues its share of a
// k-tile's DMA spends ~550 cycles of each ~1800-cycle k-tile there with its matrix pipe idle,
// measured on the dN shape).  The producers mirror the compute waves' barriers: before the
// barrier that publishes tile t+1 they wait for its DMA, after it they issue tile t+STAGES into
// the stage tile t just left.
template <bool TA, bool TB, typename CT, int BM, int BN, int EPI, int STAGES, bool BIAS, int BPAR,
          int PROD = 0>
__device__ __forceinline__ void gemm_body(const GemmDesc& g) {
    static_assert(STAGES == 2 || STAGES == 3, "two or three LDS stages");
    static_assert(PROD == 0 || PROD == 4, "producer waves: 0 or 4");
    static_assert(!BIAS || (BPAR >= 0 && BPAR < 2 && (BM / 64) % 2 == 0), "bias rows split by fragment parity");
    constexpr int NW = 4;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    constexpr int A_ELEMS = BM * BK, B_ELEMS = BN * BK;
    constexpr int STAGE_B = (A_ELEMS + B_ELEMS) * 2;
    constexpr int WM = BM / 2, WN = BN / 2, FM = WM / 32, FN = WN / 32;
    constexpr int NM = FM * FN;
    constexpr int RA = TA ? 2 : 1, RB = TB ? 1 : 2;  // LDS reads per A / B fragment
    constexpr int NR = FM * RA + FN * RB;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void*)smem_raw;

    const int tilesM = (g.M + BM - 1) / BM, tilesN = (g.N + BN - 1) / BN;
    const int nblk = tilesM * tilesN;
    int pid = blockIdx.x;
    if ((nblk & 7) == 0) pid = (pid & 7) * (nblk >> 3) + (pid >> 3);  // XCD-contiguous ranges
    constexpr int GROUP = BM == 2 * BN ? 4 : 8;
    const int group_id = pid / (GROUP * tilesN);
    const int first_m = group_id * GROUP;
    const int gsize = min(tilesM - first_m, GROUP);
    const int in_group = pid % (GROUP * tilesN);
    const int m0 = (first_m + in_group % gsize) * BM;
    const int n0 = (in_group / gsize) * BN;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int wm = wave >> 1, wn = wave & 1;
    const int dw = wave & 3;  // the wave's slice of a tile's DMA (producer or compute wave)
    constexpr bool SELF_DMA = PROD == 0;  // the compute waves issue the DMA themselves

    f32x16_t acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int kt0 = g.Ks[0] / BK;
    const int KTall = kt0 + (g.nseg > 1 ? g.Ks[1] / BK : 0);
    // split y takes the k-tiles [y KTall / ksplit, (y + 1) KTall / ksplit)
    const int nsplit = g.ksplit < 1 ? 1 : g.ksplit;
    const int kt_lo = (int)(((int64_t)blockIdx.y * KTall) / nsplit);
    const int KT = (int)(((int64_t)(blockIdx.y + 1) * KTall) / nsplit) - kt_lo;
    const int last = KT - 1;
    const bf16_t* const A0 = g.A[0];
    const bf16_t* const A1 = g.A[1];
    const bf16_t* const B0 = g.B[0];
    const bf16_t* const B1 = g.B[1];
    const int lda0 = g.lda[0], lda1 = g.lda[1], ldb0 = g.ldb[0], ldb1 = g.ldb[1];

    constexpr int NDA = BM / (8 * NW), NDB = BN / (8 * NW);
    // Lane offsets of the wave's DMA instructions for segment `oseg` (they depend on the
    // segment's leading dimensions only; recomputed once if the two segments differ).  The
    // 256 x 256 bias variant has no 16 VGPRs to spare for them (its accumulators fill the
    // AGPRs): it computes each DMA address as it issues it.
    constexpr bool PRE = !(BM == 256 && BN == 256 && BIAS);
    uint32_t voa[PRE ? NDA : 1], vob[PRE ? NDB : 1];
    int oseg = 0;
    auto set_offsets = [&](int seg) {
        if constexpr (PRE) {
            stage_offsets<BM, !TA, NW>(seg ? lda1 : lda0, m0, g.M, dw, voa);
            stage_offsets<BN, TB, NW>(seg ? ldb1 : ldb0, n0, g.N, dw, vob);
        }
        oseg = seg;
    };
    const bool reoffset = PRE && g.nseg > 1 && (lda0 != lda1 || ldb0 != ldb1);
    auto offsets_for = [&](int tl) {  // before the DMAs of tile tl (tiles are issued in order)
        if (reoffset && oseg == 0 && kt_lo + tl >= kt0) set_offsets(1);
    };
    auto dma_one = [&](auto Q_, int tl, int buf) {
        constexpr int q = decltype(Q_)::value;
        const int t = kt_lo + tl;
        const bool s1 = t >= kt0;
        const int k0 = (s1 ? t - kt0 : t) * BK;
        const uint32_t base = lds0 + (uint32_t)(buf * STAGE_B);
        if constexpr (!PRE) {
            if constexpr (q < NDA)
                stage<BM, !TA, NW, q, q + 1>(s1 ? A1 : A0, s1 ? lda1 : lda0, m0, g.M, k0, base);
            else
                stage<BN, TB, NW, q - NDA, q - NDA + 1>(s1 ? B1 : B0, s1 ? ldb1 : ldb0, n0, g.N, k0,
                                                       base + A_ELEMS * 2);
        } else if constexpr (q < NDA) {
            const bf16_t* src = stage_base<!TA>(s1 ? A1 : A0, s1 ? lda1 : lda0, m0, k0);
            dma16s(src, voa[q], base + 1024u * (uint32_t)(dw * NDA + q));
        } else {
            constexpr int qb = q - NDA;
            const bf16_t* src = stage_base<TB>(s1 ? B1 : B0, s1 ? ldb1 : ldb0, n0, k0);
            dma16s(src, vob[qb], base + A_ELEMS * 2 + 1024u * (uint32_t)(dw * NDB + qb));
        }
    };
    bf16x8_t fa[4][FM], fb[4][FN];
    // BIAS: per-lane partial row sums of op(A): fragment i holds row (lane % 32) of rows
    // wm WM + 32 i, eight k values per lane, summed into four independent accumulators per
    // fragment (one per value pair), so no add waits on another; this wave sums the fragments
    // of parity BPAR (the other wave of its row holds the same fragments and sums the rest)
    float bsum[BIAS ? FM : 1][4];
#pragma unroll
    for (int i = 0; i < (BIAS ? FM : 1); ++i)
#pragma unroll
        for (int d = 0; d < 4; ++d) bsum[i][d] = 0.f;
    // read r of a fragment set: A fragments first, then B (whole fragments per call: a
    // transpose-read fragment is two instructions, issued together)
    auto read_one = [&](auto SET_, auto R_, const bf16_t* sa, int ks) {
        constexpr int set = decltype(SET_)::value, r = decltype(R_)::value;
        if constexpr (r < FM * RA) {
            if constexpr (r % RA == 0) fa[set][r / RA] = frag<BM, !TA>(sa, wm * WM + (r / RA) * 32, ks);
        } else {
            constexpr int rb = r - FM * RA;
            if constexpr (rb % RB == 0) fb[set][rb / RB] = frag<BN, TB>(sa + A_ELEMS, wn * WN + (rb / RB) * 32, ks);
        }
    };
    auto stage_ptr = [&](int buf) { return reinterpret_cast<const bf16_t*>(smem_raw + buf * STAGE_B); };

    // one k-step: MFMAs of set CUR, with the reads of set RSET (k-step rks of stage rbuf) and
    // optionally the DMA of tile dtile into dbuf interleaved
    auto kstep = [&](auto CUR_, auto RSET_, auto FRONT_, auto DMA_, const bf16_t* rsrc, int rks,
                     int dtile, int dbuf) {
        constexpr int cur = decltype(CUR_)::value;
        constexpr bool front = decltype(FRONT_)::value, with_dma = decltype(DMA_)::value;
        constexpr int ND = NDA + NDB;
        static_for<NM>([&](auto Q_) {
            constexpr int q = decltype(Q_)::value;
            acc[q / FN][q % FN] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                fa[cur][q / FN], fb[cur][q % FN], acc[q / FN][q % FN], 0, 0, 0);
            if constexpr (BIAS) {
                // the 4 value pairs of fragment q / FN spread over its FN MFMAs.  With FN >= 4
                // (one pair per MFMA) each pair is widened to fp32 with a shift and a mask
                // (exact) and added on the VALU: 4 VALU ops per MFMA, 128x256 tiles ~10 %
                // faster than v_dot2.  With FN = 2 that would be 8 VALU ops per MFMA, which
                // measured ~10 % slower than one v_dot2c_f32_bf16 against ones per pair
                constexpr int i = q / FN, d0 = (q % FN) * 4 / FN, d1 = (q % FN + 1) * 4 / FN;
                if constexpr (i % 2 != BPAR) {
                    // the other wave of this wave row sums fragment i
                } else if constexpr (FN >= 4) {
                    typedef unsigned u32x4_v __attribute__((ext_vector_type(4)));
                    const u32x4_v w = __builtin_bit_cast(u32x4_v, fa[cur][i]);
                    static_for<4>([&](auto D_) {
                        constexpr int d = decltype(D_)::value;
                        if constexpr (d >= d0 && d < d1)
                            bsum[i][d] += __uint_as_float(w[d] << 16) + __uint_as_float(w[d] & 0xffff0000u);
                    });
                } else {
                    typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
                    const bf16x2_v one = {(__bf16)1.0f, (__bf16)1.0f};
                    static_for<4>([&](auto D_) {
                        constexpr int d = decltype(D_)::value;
                        if constexpr (d >= d0 && d < d1)
                            bsum[i][d] = __builtin_amdgcn_fdot2_f32_bf16(
                                __builtin_shufflevector(fa[cur][i], fa[cur][i], 2 * d, 2 * d + 1), one,
                                bsum[i][d], false);
                    });
                }
            }
            constexpr int r0 = reads_before<NM, NR, front>(q), r1 = reads_before<NM, NR, front>(q + 1);
            static_for<NR>([&](auto R_) {
                constexpr int r = decltype(R_)::value;
                if constexpr (r >= r0 && r < r1) read_one(RSET_, R_, rsrc, rks);
            });
            if constexpr (with_dma) {
                constexpr int d0 = (ND * q + NM - 1) / NM, d1 = (ND * (q + 1) + NM - 1) / NM;
                static_for<ND>([&](auto D_) {
                    constexpr int d = decltype(D_)::value;
                    if constexpr (d >= d0 && d < d1) dma_one(D_, dtile, dbuf);
                });
            }
            __builtin_amdgcn_sched_barrier(0);
        });
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    using BF = std::false_type;
    using BT = std::true_type;

    // STAGES = 3: the DMA of tile t+3 goes into tile t's stage once tile t's last reads are
    // retired (after this tile's barrier), so a tile's DMA has almost two tiles to land; the
    // barrier then waits only for tile t+1 (tile t+2's DMA may still be in flight).
    constexpr int ND = NDA + NDB;
    auto tile = [&](auto BUF_, int t) {
        constexpr int buf = decltype(BUF_)::value;
        const bf16_t* cur = stage_ptr(buf);
        const bf16_t* nxt = stage_ptr((buf + 1) % STAGES);
        kstep(I0{}, I2{}, BF{}, BF{}, cur, 2, 0, 0);
        kstep(I1{}, I3{}, BT{}, BF{}, cur, 3, 0, 0);
        if constexpr (!SELF_DMA)  // lgkmcnt(0): the producers wait for the DMA
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(63) & 0xF0FFu);
        else if constexpr (STAGES == 3)  // vmcnt(ND) and lgkmcnt(0)
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(ND) & 0xF0FFu);
        else  // vmcnt(0) and lgkmcnt(0)
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(0) & 0xF0FFu);
        __syncthreads();
        if constexpr (SELF_DMA) offsets_for(min(t + STAGES, last));
        kstep(I2{}, I0{}, BF{}, std::integral_constant<bool, SELF_DMA>{}, nxt, 0,
              min(t + STAGES, last), buf);
        kstep(I3{}, I1{}, BF{}, BF{}, nxt, 1, 0, 0);
    };
    auto dma_all = [&](int tl, int buf) {
        static_for<ND>([&](auto D_) { dma_one(D_, tl, buf); });
    };
    auto prologue_dma = [&]() {  // tiles 0 .. STAGES-1, then wait for tile 0
        set_offsets(kt_lo >= kt0 ? 1 : 0);
        dma_all(0, 0);
        offsets_for(min(1, last));
        dma_all(min(1, last), 1);
        if constexpr (STAGES == 3) {
            offsets_for(min(2, last));
            dma_all(min(2, last), 2);
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * ND));
        } else {
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(ND));
        }
    };

    if constexpr (PROD > 0) {
        if (wave >= 4) {  // producer: the compute waves' barriers, each with the DMA around it
            if (KT > 0) {
                prologue_dma();
                __syncthreads();
            }
            for (int t = 0; t < KT; ++t) {
                // tile t+1 has landed before the barrier that publishes it (tile t+2 may still
                // be in flight with three stages); tile t's stage is free after it
                if constexpr (STAGES == 3) __builtin_amdgcn_s_waitcnt(vmcnt_imm(ND));
                else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
                __syncthreads();
                offsets_for(min(t + STAGES, last));
                dma_all(min(t + STAGES, last), t % STAGES);
            }
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
            __syncthreads();
            return;
        }
    }

    if (KT > 0) {
        if constexpr (SELF_DMA) prologue_dma();
        __syncthreads();
        static_for<NR>([&](auto R_) { read_one(I0{}, R_, stage_ptr(0), 0); });
        static_for<NR>([&](auto R_) { read_one(I1{}, R_, stage_ptr(0), 1); });
    }
    int t = 0;
    if constexpr (STAGES == 3) {
        for (; t + 2 < KT; t += 3) {
            tile(I0{}, t);
            tile(I1{}, t + 1);
            tile(I2{}, t + 2);
        }
        if (t < KT) tile(I0{}, t);
        if (t + 1 < KT) tile(I1{}, t + 1);
    } else {
        for (; t + 1 < KT; t += 2) {
            tile(I0{}, t);
            tile(I1{}, t + 1);
        }
        if (t < KT) tile(I0{}, t);
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0) & 0xF0FFu);
    __syncthreads();

    if constexpr (BIAS) {
        // lanes l and l ^ 32 hold the two k-halves of one row; the blocks of the first column
        // tile write (or, split over K, add onto the cleared vector: two terms, deterministic)
#pragma unroll
        for (int i = BPAR; i < FM; i += 2) {
            const float p = (bsum[i][0] + bsum[i][1]) + (bsum[i][2] + bsum[i][3]);
            const float v = p + __shfl_xor(p, 32);
            const int m = m0 + wm * WM + i * 32 + lane;
            if (n0 == 0 && lane < 32 && m < g.M) {
                float* dst = m < g.Msplit ? g.bias + m : g.bias2 + (m - g.Msplit);
                if (g.ksplit > 2) g.part[(size_t)g.ksplit * g.M * g.N + (size_t)blockIdx.y * g.M + m] = v;
                else if (g.ksplit > 1) unsafeAtomicAdd(dst, v);
                else *dst = g.accumulate ? *dst + v : v;
            }
        }
    }
    float* st = reinterpret_cast<float*>(smem_raw) + wave * 32 * (WN + 4);
    if constexpr (EPI == 1) {
        const int mb = m0 + wm * WM, nb = n0 + wn * WN;
        switch (g.glu_kind) {
            case GN_GLU_SWIGLU_UP: glu_epilogue<GN_GLU_SWIGLU_UP, FM, FN, WN>(g, acc, st, mb, nb, lane); break;
            case GN_GLU_SWIGLU_GATE: glu_epilogue<GN_GLU_SWIGLU_GATE, FM, FN, WN>(g, acc, st, mb, nb, lane); break;
            case GN_GLU_GEGLU_UP: glu_epilogue<GN_GLU_GEGLU_UP, FM, FN, WN>(g, acc, st, mb, nb, lane); break;
            case GN_GLU_GEGLU_GATE: glu_epilogue<GN_GLU_GEGLU_GATE, FM, FN, WN>(g, acc, st, mb, nb, lane); break;
            default: glu_epilogue<GN_GLU_REGLU_UP, FM, FN, WN>(g, acc, st, mb, nb, lane); break;
        }
        return;
    }
    const int rq = (lane >> 5) * 4;
    // the strip is private to the wave but each lane reads rows other lanes wrote: wave-scope
    // fences around a wave barrier order the accesses (no instructions on a wave64 CU)
    auto strip = [&](auto I_) {
        constexpr int i = decltype(I_)::value;
        wave_lds_sync();
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                st[(8 * (r >> 2) + rq + (r & 3)) * (WN + 4) + j * 32 + (lane & 31)] = acc[i][j][r];
        wave_lds_sync();
        if constexpr (EPI == 0 && sizeof(CT) == 4) {
            if (g.ksplit > 2) {
                epilogue_part<WN>(g, st, m0 + wm * WM + i * 32, n0 + wn * WN, lane);
                return;
            }
            if (g.ksplit > 1) {
                epilogue_atomic<WN>(g, st, m0 + wm * WM + i * 32, n0 + wn * WN, lane);
                return;
            }
        }
        epilogue_rows<CT, EPI, WN>(g, st, m0 + wm * WM + i * 32, n0 + wn * WN, lane);
    };
    static_for<FM>(strip);
}

template <bool TA, bool TB, typename CT, int BM, int BN, int EPI, int STAGES, bool BIAS = false,
          int PROD = 0>
__global__ __launch_bounds__(PROD ? 512 : 256, 1) void gemm_core(GemmDesc g) {
    if constexpr (BIAS) {
        // the fused bias sums are split between the two waves of each wave row: two copies of
        // the body, one per fragment parity (measured 5-10 % faster on the decoder's weight
        // gradients than both waves summing every fragment)
        if ((__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & 1) == 0)
            gemm_body<TA, TB, CT, BM, BN, EPI, STAGES, true, 0, PROD>(g);
        else
            gemm_body<TA, TB, CT, BM, BN, EPI, STAGES, true, 1, PROD>(g);
    } else {
        gemm_body<TA, TB, CT, BM, BN, EPI, STAGES, false, -1, PROD>(g);
    }
}

// ---- VSA unpack-project dW --------------------------------------------------------------
// C[M x N] (+)= (A_hi + A_lo) S over K, one block per 128 x 256 tile, 4 waves (2 x 2) of
// 64 x 128, one wave per SIMD.  Both dY planes (hi and lo, k-contiguous) share one +-1 B tile
// per k-tile, so the bits are expanded once for both and no partial sums cross blocks.
// Per k-tile (64 k):
//   * A_hi, A_lo tiles arrive by LDS DMA two tiles ahead of use (stage = the tile's parity);
//   * each lane loads two raw bit words of the tile after next into registers (plain global
//     loads), and expands the words of the next tile into the B tile of the other stage while
//     the MFMAs of the current tile run (the expansion is interleaved with them);
//   * the barrier that closes k-step 2 publishes the next tile and frees the current stage,
//     whose refill DMA then goes out while k-step 3 runs.
constexpr int kVsaBM = 128, kVsaBN = 256, kVsaNW = 4;

struct VsaK {
    static constexpr int BM = kVsaBM, BN = kVsaBN, NW = kVsaNW;
    static constexpr int WM = BM / 2, WN = BN / 2, FM = WM / 32, FN = WN / 32;
    static constexpr int A_ELEMS = BM * BK, B_ELEMS = BN * BK;
    static constexpr int STAGE_B = (2 * A_ELEMS + B_ELEMS) * 2;  // hi, lo, B
    static constexpr int WPR = BN / 32;                            // bit words per k-row
    static constexpr int WPL = BK * WPR / (64 * NW);               // words expanded per lane
    static constexpr size_t STRIPS = (size_t)NW * 32 * (WN + 4) * sizeof(float);
    static constexpr size_t SMEM = 2 * (size_t)STAGE_B > STRIPS ? 2 * (size_t)STAGE_B : STRIPS;
    static_assert(WPL == 2 && SMEM <= 160 * 1024, "tile shape");
};

// one 16-byte chunk (8 columns) of +-1 bf16 from byte b of the inverted bit word nw:
// column bit 0 -> -1.0 (0xBF80), 1 -> +1.0 (0x3F80).  t2 holds the byte at bits 0-7 and
// again at 15-22, so one shift puts bit 2e at 15 and bit 2e+1 at 31.
__device__ __forceinline__ uint4 vsa_chunk(uint32_t nw, int b) {
    const uint32_t t = (nw >> (8 * b)) & 0xffu;
    const uint32_t t2 = t | (t << 15);
    uint32_t d[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) d[e] = ((t2 << (15 - 2 * e)) & 0x80008000u) | 0x3F803F80u;
    return make_uint4(d[0], d[1], d[2], d[3]);
}

// Interleave: each MFMA followed by up to RD LDS reads, VA VALU, WR LDS writes, VM memory ops.
template <int Q, int NM, int RD, int VA, int WR, int VM>
__device__ __forceinline__ void vsa_sched() {
    if constexpr (Q < NM) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if constexpr (RD > 0) __builtin_amdgcn_sched_group_barrier(0x100, RD, 0);
        if constexpr (VA > 0) __builtin_amdgcn_sched_group_barrier(0x002, VA, 0);
        if constexpr (WR > 0) __builtin_amdgcn_sched_group_barrier(0x200, WR, 0);
        if constexpr (VM > 0) __builtin_amdgcn_sched_group_barrier(0x010, VM, 0);
        vsa_sched<Q + 1, NM, RD, VA, WR, VM>();
    }
}

template <bool TWO>
__global__ __launch_bounds__(64 * kVsaNW, 1) void vsa_dw_dma(VsaDesc v) {
    using C = VsaK;
    constexpr int BM = C::BM, BN = C::BN, NW = C::NW, WM = C::WM, WN = C::WN, FM = C::FM, FN = C::FN;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void*)smem_raw;

    const int tilesM = (v.M + BM - 1) / BM, tilesN = v.N / BN;
    const int nblk = tilesM * tilesN;
    int pid = blockIdx.x;
    if ((nblk & 7) == 0) pid = (pid & 7) * (nblk >> 3) + (pid >> 3);  // XCD-contiguous ranges
    const int m0 = (pid % tilesM) * BM, n0 = (pid / tilesM) * BN;  // the M tiles of one n share bits
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int wm = wave >> 1, wn = wave & 1;

    f32x16_t acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int KT = v.K / BK;
    const bf16_t* const Ahi = v.A[0];
    const bf16_t* const Alo = v.A[1];
    // lane offsets of the wave's A DMAs (the hi and lo planes share lda, hence the offsets)
    constexpr int NJ = BM / (8 * NW);
    uint32_t voa[NJ];
    stage_offsets<BM, true, NW>(v.lda, m0, v.M, wave, voa);
    auto dma_a = [&](int tl, int buf) {
        const uint32_t base = lds0 + (uint32_t)(buf * C::STAGE_B) + 1024u * (uint32_t)(wave * NJ);
        const bf16_t* hi = stage_base<true>(Ahi, v.lda, m0, tl * BK);
#pragma unroll
        for (int j = 0; j < NJ; ++j) dma16s(hi, voa[j], base + 1024u * j);
        if constexpr (TWO) {
            const bf16_t* lo = stage_base<true>(Alo, v.lda, m0, tl * BK);
#pragma unroll
            for (int j = 0; j < NJ; ++j) dma16s(lo, voa[j], base + C::A_ELEMS * 2 + 1024u * j);
        }
    };
    // raw words: lane (wave w, l), slot i -> k-row 16w + 8i + l/8, word l%8 of the tile's 8
    const uint32_t* bits_base = v.bits + n0 / 32 + (lane & 7);
    const int row_l = 16 * wave + (lane >> 3);
    // raw bit words, two register sets used in turn: the set holding tile t+1's words is
    // expanded during tile t and then reloaded with tile t+3's (never indexed dynamically)
    uint32_t rx[2], ry[2];
    auto load_raw = [&](int tl, uint32_t (&dst)[2]) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
            dst[i] = __builtin_nontemporal_load(bits_base + (size_t)(tl * BK + row_l + 8 * i) * v.words);
    };
    // expand word slot i of set src into the B tile of stage buf: 4 chunks; the lanes
    // holding words 4-7 of a row write their chunks rotated by one, so every 16-lane write
    // cycle covers the 16 bank groups once
    auto expand_word = [&](const uint32_t (&src)[2], int i, int buf) {
        bf16_t* sb = reinterpret_cast<bf16_t*>(smem_raw + buf * C::STAGE_B) + 2 * C::A_ELEMS;
        const int r = row_l + 8 * i, wc = lane & 7;
        const uint32_t nw = ~src[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int b = (e + (wc >> 2)) & 3;
            const int c = 4 * wc + b;
            *reinterpret_cast<uint4*>(sb + r * BN + ((c ^ fko(r)) * 8)) = vsa_chunk(nw, b);
        }
    };
    bf16x8_t fh[2][FM], fl[2][FM], fb[2][FN];
    auto load_frags = [&](int buf, int ks, int slot) {
        const bf16_t* sa = reinterpret_cast<const bf16_t*>(smem_raw + buf * C::STAGE_B);
#pragma unroll
        for (int i = 0; i < FM; ++i) fh[slot][i] = frag<BM, true>(sa, wm * WM + i * 32, ks);
        if constexpr (TWO) {
#pragma unroll
            for (int i = 0; i < FM; ++i) fl[slot][i] = frag<BM, true>(sa + C::A_ELEMS, wm * WM + i * 32, ks);
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) fb[slot][j] = frag<BN, false>(sa + 2 * C::A_ELEMS, wn * WN + j * 32, ks);
    };
    auto mfmas = [&](int slot) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fh[slot][i], fb[slot][j], acc[i][j], 0, 0, 0);
        if constexpr (TWO) {
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fl[slot][i], fb[slot][j], acc[i][j], 0, 0, 0);
        }
    };
    constexpr int NM = FM * FN * (TWO ? 2 : 1);         // MFMAs per k-step
    constexpr int NR = FM * (TWO ? 2 : 1) + 2 * FN;     // LDS reads per k-step

    // prologue: tile 0 staged and expanded; tile 1's A DMA and the bits of tiles 1, 2 in
    // flight.  Tail iterations clamp the tile they prefetch to the last one (in-bounds
    // redundant work instead of branches that would split the interleaved schedule).
    // (The DMA instructions are inline assembly that the compiler's wait-count bookkeeping
    // does not see: every bit word is consumed only after an explicit full drain, so the
    // compiler never has to place a vmcnt wait of its own.)
    const int last = KT - 1;
    load_raw(0, ry);
    load_raw(min(1, last), rx);
    dma_a(0, 0);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    expand_word(ry, 0, 0);
    expand_word(ry, 1, 0);
    load_raw(min(2, last), ry);
    dma_a(min(1, last), 1);
    __syncthreads();
    load_frags(0, 0, 0);

    // one k-tile; BUF = t & 1 is a compile-time constant, set holds tile t+1's bits
    auto step = [&](auto BUF_, int t, uint32_t (&set)[2]) {
        constexpr int buf = decltype(BUF_)::value;
        // k-step 0: fragments of step 1, MFMAs of step 0, first word of tile t+1's bits
        // (past the last tile the expansion rewrites the idle stage: harmless)
        load_frags(buf, 1, 1);
        mfmas(0);
        expand_word(set, 0, buf ^ 1);
        vsa_sched<0, NM, 1, 2, 1, 0>();
        __builtin_amdgcn_sched_barrier(0);
        // k-step 1: second word
        load_frags(buf, 2, 0);
        mfmas(1);
        expand_word(set, 1, buf ^ 1);
        vsa_sched<0, NM, 1, 2, 1, 0>();
        __builtin_amdgcn_sched_barrier(0);
        // k-step 2
        load_frags(buf, 3, 1);
        mfmas(0);
        vsa_sched<0, NM, 1, 0, 0, 0>();
        __builtin_amdgcn_sched_barrier(0);
        // tile t+1's A (and the bits of t+2) landed for this wave; the barrier publishes the
        // B tile every wave expanded and retires every read of stage buf
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        __syncthreads();
        load_raw(min(t + 3, last), set);
        dma_a(min(t + 2, last), buf);
        load_frags(buf ^ 1, 0, 0);
        mfmas(1);
        vsa_sched<0, NM, 1, 2, 0, 1>();
        __builtin_amdgcn_sched_barrier(0);
    };
    // pairs of tiles, so every path into the loop head has drained the set it expands next
    int t = 0;
    for (; t + 1 < KT; t += 2) {
        step(std::integral_constant<int, 0>{}, t, rx);
        step(std::integral_constant<int, 1>{}, t + 1, ry);
    }
    if (t < KT) step(std::integral_constant<int, 0>{}, t, rx);
    // the clamped prefetches of the last iterations may still be landing in the stages
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __syncthreads();

    // epilogue: one 32-row strip at a time
    float* st = reinterpret_cast<float*>(smem_raw) + wave * 32 * (WN + 4);
    const int rq = (lane >> 5) * 4;
    GemmDesc g{};
    g.M = v.M; g.N = v.N; g.C = v.C; g.C2 = v.C; g.Msplit = v.M; g.ldc = v.ldc;
    g.accumulate = v.accumulate;
    auto strip = [&](auto I_) {
        constexpr int i = decltype(I_)::value;
        wave_lds_sync();
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                st[(8 * (r >> 2) + rq + (r & 3)) * (WN + 4) + j * 32 + (lane & 31)] = acc[i][j][r];
        wave_lds_sync();
        epilogue_rows<float, 0, WN>(g, st, m0 + wm * WM + i * 32, n0 + wn * WN, lane);
    };
    strip(std::integral_constant<int, 0>{});
    if constexpr (FM > 1) strip(std::integral_constant<int, 1>{});
}

template <typename F>
bool allow_lds(F* fn, size_t bytes) {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) == hipSuccess;
}

template <bool TA, bool TB, typename CT, int BM, int BN, int EPI>
int launch_t(const GemmDesc& g, hipStream_t s) {
    // LDS: the operand stages, or the epilogue's per-wave fp32 strips [32][BN/2 + 4] if larger
    constexpr size_t strips_b = (size_t)4 * 32 * (BN / 2 + 4) * sizeof(float);
    constexpr size_t stage2_b = (size_t)2 * (BM + BN) * BK * sizeof(bf16_t);
    constexpr size_t stage3_b = (size_t)3 * (BM + BN) * BK * sizeof(bf16_t);
    constexpr size_t smem2 = stage2_b > strips_b ? stage2_b : strips_b;
    constexpr size_t smem3 = stage3_b > strips_b ? stage3_b : strips_b;
    constexpr bool fits3 = smem3 <= 160 * 1024;
    static_assert(smem2 <= 160 * 1024, "LDS per CU");
    const int KT = (g.Ks[0] + (g.nseg > 1 ? g.Ks[1] : 0)) / BK;
    // the bias-summing variant exists for weight gradients only (fp32 C, plain epilogue)
    constexpr bool CAN_BIAS = EPI == 0 && sizeof(CT) == 4;
    const bool bias = CAN_BIAS && g.bias;
    // plain-epilogue tiles up to 256 x 128 take four producer waves (two waves per SIMD:
    // 256 x 256's accumulators do not fit beside a second wave)
    constexpr int PR = (EPI == 0 && BM * BN <= 256 * 128) ? 4 : 0;
    constexpr int NT = 256 + 64 * PR;
    // three LDS stages wherever they fit for producer-wave tiles (their block holds the CU
    // alone either way, and the producers issue the extra stage's DMA off the compute waves:
    // the decoder's short k loops, 12-42 k-tiles, took the 12-layer backward 8.37-8.39 ->
    // 8.11-8.12 ms eager, 8.05-8.06 -> 7.89 ms replayed against two stages below 48 k-tiles);
    // for the others three stages pay off on long k loops only (shorter prologue), and the
    // GLU-epilogue 128 x 128 tiles keep two so that two blocks share a CU
    const bool three = fits3 && (PR > 0 || KT / g.ksplit >= 48);
    static const bool ok2 = allow_lds(gemm_core<TA, TB, CT, BM, BN, EPI, 2, false, PR>, smem2);
    static const bool ok3 =
        fits3 ? allow_lds(gemm_core<TA, TB, CT, BM, BN, EPI, fits3 ? 3 : 2, false, PR>, smem3) : false;
    static const bool okb2 = CAN_BIAS ? allow_lds(gemm_core<TA, TB, CT, BM, BN, EPI, 2, CAN_BIAS, PR>, smem2) : false;
    static const bool okb3 = CAN_BIAS && fits3
                                 ? allow_lds(gemm_core<TA, TB, CT, BM, BN, EPI, fits3 ? 3 : 2, CAN_BIAS, PR>, smem3)
                                 : false;
    if (!(three ? (bias ? okb3 : ok3) : (bias ? okb2 : ok2))) {
        set_error("gemm: cannot reserve %zu B of LDS", three ? smem3 : smem2);
        return GN_E_HIP;
    }
    const int tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
    if (g.ksplit == 2)
        clear_c<<<grid_for((int64_t)g.M * g.N, 256, 4096), 256, 0, s>>>(g);
    const dim3 grid(tiles, g.ksplit);
    if (bias && three)
        hipLaunchKernelGGL((gemm_core<TA, TB, CT, BM, BN, EPI, fits3 ? 3 : 2, CAN_BIAS, PR>), grid, dim3(NT), smem3, s, g);
    else if (bias)
        hipLaunchKernelGGL((gemm_core<TA, TB, CT, BM, BN, EPI, 2, CAN_BIAS, PR>), grid, dim3(NT), smem2, s, g);
    else if (three)
        hipLaunchKernelGGL((gemm_core<TA, TB, CT, BM, BN, EPI, fits3 ? 3 : 2, false, PR>), grid, dim3(NT), smem3, s, g);
    else
        hipLaunchKernelGGL((gemm_core<TA, TB, CT, BM, BN, EPI, 2, false, PR>), grid, dim3(NT), smem2, s, g);
    if (g.ksplit > 2)
        split_reduce<<<grid_for((int64_t)g.M * (g.N / 4), 256, 4096), 256, 0, s>>>(g);
    GN_LAUNCH_CHECK("gemm (dma)");
    return GN_OK;
}

// Tile shape and split from a time model fitted to MI355X sweeps of this core over the FFN
// and decoder GEMMs (K from 768 to 32000):
//   block time = KT x t_k[shape] + o[shape] + epilogue, where t_k is the time of one 64-deep
//                k-tile with every CU busy (separate fits for a k-contiguous A and for a
//                k-outer A, i.e. weight gradients with both operands transposed in LDS) and o
//                the fixed cost of a block (DMA prologue, pipeline fill, drain);
//   epilogue     C tile bytes at ~40 KB/us per block (the GLU epilogue moves ~5x that);
//   a last round that fills a fraction f of the 256 CUs costs (0.6 + 0.4 f) of a full round
//                (the blocks of a part-filled round get more L2 / HBM bandwidth each);
//   split-K (two halves, fp32 C only): clear + atomic adds, ~5 us + 0.7 us per MB of C;
//   split-K over 3..8 ranges (fp32 C, workspace given): partial tiles stored, then one
//   reduce pass reading every plane and writing C, ~4 us + bytes at 4 TB/s.
struct TileChoice {
    int shape;    // index into kTileShapes
    int ksplit;
    int m_first;  // > 0: rows [0, m_first) on 256 x 256 tiles, the rest on `shape`
};
constexpr int kTileShapes[4][2] = {{256, 256}, {256, 128}, {128, 256}, {128, 128}};

inline double tile_cost(const GemmDesc& g, bool ta, size_t c_bytes, int epi, int i, int ks,
                        bool filled = false) {
    static constexpr double tk_kc[4] = {1.73, 0.98, 0.98, 0.57};
    static constexpr double tk_ta[4] = {1.60, 0.98, 0.90, 0.52};
    static constexpr double fixed[4] = {16.5, 6.4, 13.0, 6.4};
    const int KT = (g.Ks[0] + (g.nseg > 1 ? g.Ks[1] : 0)) / BK;
    const int bm = kTileShapes[i][0], bn = kTileShapes[i][1];
    const long blocks = (long)((g.M + bm - 1) / bm) * ((g.N + bn - 1) / bn) * ks;
    const long full = blocks / 256;
    const double f = (double)(blocks % 256) / 256.0;
    // filled: a grid under one round costs a whole block time (the blocks are compute-bound),
    // and the bias variant's k-tiles ~25 % more (measured on the decoder's weight gradients)
    const double rounds = filled && full == 0 ? 1.0 : (double)full + (f > 0 ? 0.6 + 0.4 * f : 0.0);
    const double kt = (double)((KT + ks - 1) / ks);
    const double epi_us = (double)bm * bn * (double)c_bytes * (epi ? 5.0 : 1.0) / 40000.0;
    // the producer-wave kernels (plain epilogue, tiles up to 256 x 128) run their
    // k-tiles faster than the sweeps above measured for the self-issuing ones: scaled by the
    // ratio a second sweep (C2 and C5 shapes, every tile forced in turn) picks the fastest or
    // near-fastest tile with
    static constexpr double prod_f[4] = {1.0, 0.88, 0.86, 0.95};
    const double pf = epi == 0 && !g.bias ? prod_f[i] : 1.0;
    const double tk = (ta ? tk_ta[i] : tk_kc[i]) * pf * (filled && g.bias ? 1.25 : 1.0);
    double t = rounds * (kt * tk + fixed[i] + epi_us);
    if (ks == 2) t += 5.0 + 0.7e-6 * (double)g.M * g.N * 4.0;
    if (ks > 2) t += 4.0 + (double)(ks + 1 + (g.accumulate ? 1 : 0)) * g.M * g.N * 4.0 / 4.0e6;
    return t;
}

// workspace bytes of a split over ks ranges into partial planes (ks >= 3)
inline size_t part_bytes(const GemmDesc& g, int ks) {
    return (size_t)ks * g.M * g.N * sizeof(float) + (g.bias ? (size_t)ks * g.M * sizeof(float) : 0);
}

inline TileChoice choose_tile(const GemmDesc& g, bool ta, size_t c_bytes, int epi) {
    const int KT = (g.Ks[0] + (g.nseg > 1 ? g.Ks[1] : 0)) / BK;
    const bool can_split = epi == 0 && c_bytes == 4 && !g.accumulate && !g.cbias && KT >= 32;
    // GLU epilogue over a long k loop: 128 x 128 tiles.  Their two-stage variant holds two
    // blocks per CU (64 KB of LDS, 197 registers), so one block's epilogue (gate/up loads,
    // glu', 16-byte stores) overlaps the other's main loop, which the time model does not
    // describe.  Measured on MI355X, down projection 4096 x 5632 x 2048 with dWd: 225-228 us
    // against 230-236 us for the 256 x 128 / 128 x 256 / 256 x 256 shapes (interleaved runs,
    // one process).  The same holds at 12 k-tiles: the decoder's 8192 x 3072 x 768 down
    // projection (GEGLU in the epilogue) took the 12-layer backward step 8.55 -> 8.39 ms
    // eager, 8.16 -> 8.09 ms replayed, against the model's 256 x 128.  Shorter k loops keep
    // the model's choice.
    if (epi == 1 && KT >= 12) return {3, 1};
    TileChoice best{1, 1};
    double bt = tile_cost(g, ta, c_bytes, epi, 1, 1);
    for (int i = 0; i < 4; ++i) {
        for (int ks = 1; ks <= (can_split ? 2 : 1); ++ks) {
            const double c = tile_cost(g, ta, c_bytes, epi, i, ks);
            if (c < bt) { bt = c; best = {i, ks}; }
        }
    }
    // Partial planes (fp32 C, workspace given; the reduce adds onto C, so accumulation is
    // allowed; each range >= 8 k-tiles) for a choice that leaves the GPU under one round:
    // candidates and that choice compared with the filled-round costs.  Measured on MI355X
    // (dW + db, 8192 rows): 768 x 768 50 -> 33 us (6 ranges), 768 x 3072 86 -> 72 us and
    // 6144 x 768 127 -> 113 us (3 ranges); 2304 x 768 stays with two halves.
    const bool can_part = epi == 0 && c_bytes == 4 && !g.cbias && g.part_cap > 0 && KT >= 48;
    const long tiles = (long)((g.M + kTileShapes[best.shape][0] - 1) / kTileShapes[best.shape][0]) *
                       ((g.N + kTileShapes[best.shape][1] - 1) / kTileShapes[best.shape][1]);
    if (can_part && tiles * best.ksplit < 256) {
        double bf = tile_cost(g, ta, c_bytes, epi, best.shape, best.ksplit, true);
        for (int i = 0; i < 4; ++i) {
            for (int ks : {3, 4, 6, 8}) {
                if (KT / ks < 8 || part_bytes(g, ks) > g.part_cap) continue;
                const double c = tile_cost(g, ta, c_bytes, epi, i, ks, true);
                if (c < bf) { bf = c; best = {i, ks}; }
            }
        }
    }
    // Whole rounds of 256 x 256 tiles over the first rows and the rest on its own best shape,
    // as two launches: a grid whose last round is part-filled then runs most of its work on
    // the tile with the least operand traffic per FLOP.  Each row range is the same product
    // on its rows (every output element's k order is the tile shape's MFMA order), so the
    // result is bit-identical to one launch.  Measured on MI355X (fp32 C, interleaved runs):
    // 11264 x 2048 x 4096 ([dWg;dWu]) 200-204 -> 187-189 us with 8192 rows on 256 x 256;
    // 32000 x 768 x 8192 (LM-head dW) 417-423 -> 377-385 us with 21760 rows.
    if (epi == 0 && best.ksplit == 1 && KT >= 32) {
        const int per_round = 256 / ((g.N + 255) / 256);  // 256 x 256 row tiles per round
        double bs = 0.95 * tile_cost(g, ta, c_bytes, epi, best.shape, 1);
        TileChoice two = best;
        for (int r = 1; per_round > 0 && (long)r * per_round * 256 < g.M; ++r) {
            GemmDesc a = g, b = g;
            a.M = r * per_round * 256;
            b.M = g.M - a.M;
            const double ca = tile_cost(a, ta, c_bytes, epi, 0, 1);
            for (int i = 0; i < 4; ++i) {
                const double c = ca + tile_cost(b, ta, c_bytes, epi, i, 1);
                if (c < bs) { bs = c; two = {i, 1, a.M}; }
            }
        }
        best = two;
    }
    return best;
}

// Rows [m0, m0 + rows) of a plain-epilogue product as a product of its own: op(A)'s rows, the
// C / C2 destination rows and the row-sum vectors offset; the rest shared.
inline GemmDesc row_range(const GemmDesc& g, int m0, int rows, bool ta, size_t c_bytes) {
    GemmDesc r = g;
    for (int s = 0; s < g.nseg; ++s)
        r.A[s] = g.A[s] + (ta ? (size_t)m0 : (size_t)m0 * g.lda[s]);
    r.M = rows;
    if (m0 >= g.Msplit) {
        r.C = static_cast<char*>(g.C2) + (size_t)(m0 - g.Msplit) * g.ldc * c_bytes;
        r.C2 = r.C;
        r.Msplit = rows;
        if (g.bias) r.bias = r.bias2 = g.bias2 + (m0 - g.Msplit);
    } else {
        r.C = static_cast<char*>(g.C) + (size_t)m0 * g.ldc * c_bytes;
        r.Msplit = g.Msplit - m0;  // rows past it still go to C2, at the same C2 rows
        if (g.bias) r.bias = g.bias + m0;
    }
    return r;
}

template <bool TA, bool TB, typename CT, int EPI>
int launch_shape(const GemmDesc& g0, hipStream_t s) {
    GemmDesc g = g0;
    const TileChoice tc = choose_tile(g, TA, sizeof(CT), EPI);
    g.ksplit = tc.ksplit;
    if (tc.m_first > 0) {
        const GemmDesc a = row_range(g, 0, tc.m_first, TA, sizeof(CT));
        const int rc = launch_t<TA, TB, CT, 256, 256, EPI>(a, s);
        if (rc != GN_OK) return rc;
        g = row_range(g, tc.m_first, g.M - tc.m_first, TA, sizeof(CT));
    }
    switch (tc.shape) {
        case 0: return launch_t<TA, TB, CT, 256, 256, EPI>(g, s);
        case 1: return launch_t<TA, TB, CT, 256, 128, EPI>(g, s);
        case 2: return launch_t<TA, TB, CT, 128, 256, EPI>(g, s);
        default: return launch_t<TA, TB, CT, 128, 128, EPI>(g, s);
    }
}

template <typename CT, int EPI>
int launch_trans(const GemmDesc& g, int ta, int tb, hipStream_t s) {
    if (!ta && !tb) return launch_shape<false, false, CT, EPI>(g, s);
    if (!ta && tb) return launch_shape<false, true, CT, EPI>(g, s);
    if (ta && !tb) return launch_shape<true, false, CT, EPI>(g, s);
    return launch_shape<true, true, CT, EPI>(g, s);
}

}  // namespace
}  // namespace gn
