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
// bf16 MFMA path (D = 64 or 128): one pre-pass writes rotated Q, K (bf16), D_i and
// L log2(e); then two kernels, both v_mfma_f32_32x32x16_bf16 with fp32 accumulators in
// registers and operand tiles brought into LDS by DMA while the previous tile computes:
//   attn_dkdv_mfma: one block per (b*h, 128 keys); loops over query tiles of 64;
//   attn_dq_mfma:   one block per (b*h, 128 queries); loops over key tiles of 64.
// P and dS go from the accumulators of one product straight into the operand registers
// of the next (the accumulator row order is matched by the transpose reads of the other
// operand), so neither is ever written to LDS.  Two kernels (7 tile products instead of 5)
// keep the dQ reduction free of atomics and deterministic.  The epilogues stage each
// wave's rows in LDS and apply the inverse rotation from a cos/sin table.
// A SIMT path (any D <= 256, fp32 or bf16) serves other shapes and the fp32 dtype.
//
// Key-padding mask (flash-attention2.glsl:150-154, flash-attention2-rope.glsl:201-205: the
// score of key k in batch b gets (mask[b S + k] - 1) 1e9): a pre-pass turns the mask into a
// per-key additive bias in the kernels' base-2 units (0 for a kept key, -inf where the
// reference's bias is below -1e4, i.e. where exp() of the biased score is 0 in fp32 for any
// row that keeps a key) and one flag per 64-key tile, so tiles without a masked key take the
// unmasked code.  A row whose visible keys are all masked gets O = 0, LSE = -inf and zero
// gradients (the reference's fp32 forward averages such a row uniformly instead).
#include <math.h>

#include <type_traits>

#include "gn_common.h"
#include "gn_lane.h"
#include "gn_mfma.h"

namespace gn {
namespace {

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

// ---- MFMA path (bf16, D = 64 or 128) ---------------------------------------------------
//
// Operand tiles are 64 rows x D bf16 kept in LDS in their global orientation (row pitch
// 2D bytes).  The 16-byte chunk c of tile row r sits at chunk position c ^ tswz<D>(r); for
// the two fragment reads below (ds_read_b128 of one chunk from 32 consecutive rows, and
// the transpose read of 4 consecutive rows x 64 bytes per 32 lanes) this spreads the
// lanes of every LDS pass over distinct banks, for 32- and 64-bank organisations alike.
template <int D> __device__ __forceinline__ int tswz(int r);
template <> __device__ __forceinline__ int tswz<128>(int r) {
    return ((r & 1) * 6) ^ (((r >> 1) & 1) * 10) ^ ((r >> 2) & 1) ^ (((r >> 3) & 1) << 1);
}
template <> __device__ __forceinline__ int tswz<64>(int r) {
    return ((r & 3) << 1) ^ ((r >> 2) & 1) ^ (((r >> 3) & 1) << 1);
}

constexpr int tile_bytes(int D) { return 64 * D * 2; }

// Where the rows of one (batch, head) live: element (b, h, s, d) at p[b sb + h sh + s sr + d]
// (strides in elements).  [B,H,S,D] is {H S D, S D, D}; a [B,S,H,D] buffer whose rows are
// ld elements apart (a fused QKV projection, say) is {S ld, D, ld}.
struct TDesc {
    const void* p;
    int64_t sb, sh, sr;
};
template <typename T = bf16_t>
__device__ __forceinline__ T* head_base(const TDesc& t, int bh, int H) {
    const int b = bh / H, h = bh - b * H;
    return (T*)t.p + b * t.sb + h * t.sh;
}

// DMA rows row0 .. row0+63 of a [S x D] matrix into a swizzled LDS tile (rows past S
// re-read row S-1; the kernels mask them).  D/(8 NW) DMA instructions per wave.
template <int D, int NW = 4>
__device__ __forceinline__ void dma_tile(const bf16_t* __restrict__ g, int64_t sr, int row0,
                                         int S, uint32_t lds) {
    constexpr int CPR = D / 8, RPI = 64 / CPR, PER_WAVE = CPR / NW;
    static_assert(PER_WAVE >= 1, "one DMA instruction per wave at least");
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < PER_WAVE; ++j) {
        const int q = wave * PER_WAVE + j;  // instruction q fills tile bytes [1024q, +1024)
        const int r = q * RPI + lane / CPR;
        const int c = (lane % CPR) ^ tswz<D>(r);
        const int rr = min(row0 + r, S - 1);
        dma16(g + rr * sr + c * 8, __builtin_amdgcn_readfirstlane(lds + q * 1024));
    }
}

// Lane byte offsets of dma_tile's instructions relative to the tile's first row (the
// wave's D/(8 NW) instructions; the row stride sr is below 2^24 elements, checked by the
// entry points).  A tile whose 64 rows all lie before S then moves with a scalar base only.
template <int D, int NW = 4>
struct TileOffsets {
    static constexpr int CPR = D / 8, RPI = 64 / CPR, PER_WAVE = CPR / NW;
    uint32_t v[PER_WAVE];
    __device__ __forceinline__ void init(int64_t sr, int wave) {
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int j = 0; j < PER_WAVE; ++j) {
            const int r = (wave * PER_WAVE + j) * RPI + lane / CPR;
            const int c = (lane % CPR) ^ tswz<D>(r);
            v[j] = (uint32_t)(r * (int)sr + c * 8) * 2u;
        }
    }
};

// dma_tile with precomputed lane offsets (wave: the wave-uniform wave index); the last tile
// of a sequence that is not a multiple of 64 long takes the clamping path
template <int D, int NW = 4>
__device__ __forceinline__ void dma_tile_o(const bf16_t* __restrict__ g, int64_t sr, int row0,
                                           int S, uint32_t lds, int wave,
                                           const TileOffsets<D, NW>& o) {
    using O = TileOffsets<D, NW>;
    if (row0 + 64 <= S) {
        const bf16_t* base = g + (int64_t)row0 * sr;
#pragma unroll
        for (int j = 0; j < O::PER_WAVE; ++j)
            dma16s(base, o.v[j], lds + (uint32_t)((wave * O::PER_WAVE + j) * 1024));
    } else {
        dma_tile<D, NW>(g, sr, row0, S, lds);
    }
}

// Fragment whose 32 rows are tile rows m0 .. m0+31 and whose k runs along d:
// lane l -> row m0 + l%32, d = 16 ks + 8(l/32) .. +7.
template <int D>
__device__ __forceinline__ bf16x8_t frag_rows(const bf16_t* t, int m0, int ks) {
    const int lane = threadIdx.x & 63;
    const int r = m0 + (lane & 31);
    return ld_frag16(t + r * D + (((2 * ks + (lane >> 5)) ^ tswz<D>(r)) << 3));
}

// Fragment whose 32 columns are d = n0 .. n0+31 and whose k runs along tile rows:
// lane l -> column n0 + l%32, rows kb + 4(l/32) + {0..3} then kb + 8 + 4(l/32) + {0..3}.
// With kb = 32i + 16p these are exactly the rows (queries or keys) that elements
// 8p .. 8p+7 of a 32x32 accumulator tile i hold, so a P or dS accumulator converts to an
// MFMA operand in registers, without going through LDS.
template <int D>
__device__ __forceinline__ bf16x8_t frag_cols(const bf16_t* t, int kb, int n0) {
    const int lane = threadIdx.x & 63, s = lane & 15;
    const int col = n0 + 16 * ((lane >> 4) & 1) + 4 * (s & 3);
    const int r0 = kb + 4 * (lane >> 5) + (s >> 2), r1 = r0 + 8;
    const int c = col >> 3, w = col & 7;
    return ld_tr_pair(t + r0 * D + ((c ^ tswz<D>(r0)) << 3) + w,
                      t + r1 * D + ((c ^ tswz<D>(r1)) << 3) + w);
}

// scatter a wave's 32 x D fp32 accumulators (NT tiles of 32 columns) into its LDS strip
template <int D, int NT>
__device__ __forceinline__ void strip_acc(float* st, const f32x16_t (&a)[NT]) {
    const int lane = threadIdx.x & 63, rq = (lane >> 5) * 4;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r)
            st[(8 * (r >> 2) + rq + (r & 3)) * (D + 4) + 32 * t + (lane & 31)] = a[t][r];
}

__device__ __forceinline__ void rot_t(float& x0, float& x1, float2 cs) {
    const float y0 = x0 * cs.x + x1 * cs.y, y1 = x1 * cs.x - x0 * cs.y;  // R^T
    x0 = y0;
    x1 = y1;
}

// Store a wave's 32 staged rows (sequence positions row0 ..) as bf16, times `mul`, with
// the inverse rotation of `mode`.  Each lane moves chunk c and its partner c + D/16
// (8 columns each), which holds every RoPE pair of either layout.
template <int D>
__device__ __forceinline__ void store_rows(const float* st, bf16_t* __restrict__ g, int64_t sr,
                                           int row0, int S, float mul, int mode,
                                           const float2* __restrict__ cs) {
    constexpr int HC = D / 16, P = D + 4;
    const int lane = threadIdx.x & 63;
#pragma unroll 2
    for (int idx = lane; idx < 32 * HC; idx += 64) {
        const int r = idx / HC, c = idx % HC, row = row0 + r;
        if (row >= S) continue;
        float x[8], y[8];
        const float4* sx = reinterpret_cast<const float4*>(st + r * P + 8 * c);
        const float4* sy = reinterpret_cast<const float4*>(st + r * P + 8 * (c + HC));
        const float4 a0 = sx[0], a1 = sx[1], b0 = sy[0], b1 = sy[1];
        x[0] = a0.x; x[1] = a0.y; x[2] = a0.z; x[3] = a0.w;
        x[4] = a1.x; x[5] = a1.y; x[6] = a1.z; x[7] = a1.w;
        y[0] = b0.x; y[1] = b0.y; y[2] = b0.z; y[3] = b0.w;
        y[4] = b1.x; y[5] = b1.y; y[6] = b1.z; y[7] = b1.w;
#pragma unroll
        for (int e = 0; e < 8; ++e) { x[e] *= mul; y[e] *= mul; }
        const float2* t = cs + (size_t)row * (D / 2);
        if (mode == GN_ROPE_INTERLEAVED) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                rot_t(x[2 * e], x[2 * e + 1], t[4 * c + e]);
                rot_t(y[2 * e], y[2 * e + 1], t[4 * (c + HC) + e]);
            }
        } else if (mode == GN_ROPE_HALF) {
#pragma unroll
            for (int e = 0; e < 8; ++e) rot_t(x[e], y[e], t[8 * c + e]);
        }
        bf16_t* o = g + row * sr;
        *reinterpret_cast<bf16x8_t*>(o + 8 * c) = to_bf16x8(x[0], x[1], x[2], x[3], x[4], x[5], x[6], x[7]);
        *reinterpret_cast<bf16x8_t*>(o + 8 * (c + HC)) = to_bf16x8(y[0], y[1], y[2], y[3], y[4], y[5], y[6], y[7]);
    }
}

template <int D, int STAGES, int NW>
struct DkdvCfg {
    static constexpr int TB = tile_bytes(D);
    static constexpr int STAGE = 2 * TB + 512;  // Q tile, dO tile, 64 x L, 64 x D_i
    static constexpr int DMA_PER_TILE = 2 * (D / (8 * NW)) + 1;
    static constexpr int KV = 4 * TB;           // the block's 128 K rows and 128 V rows
    static constexpr int EPI = 4 * 32 * (D + 4) * 4;
    static constexpr int LDS = STAGES * STAGE + KV > EPI ? STAGES * STAGE + KV : EPI;
};

// dK, dV for 128 keys of one (batch, head): wave w owns keys 32 (w % 4) ..; loops over the
// query tiles of 64 that can see those keys.  With NW = 4 each wave takes both 32-query
// halves of a tile in turn (at D = 64, two blocks per CU, K / V fragments in registers); with
// NW = 8 waves w and w + 4 take one half each (two waves per SIMD) and add their partial sums
// at the end.  Per query half and wave:
//   S = Q K^T, dP = dO V^T        (A = Q / dO rows, B = K / V rows, from LDS)
//   P = exp2(S scale log2e - L log2e), dS = P (dP - D_i)    (masked on edge tiles)
//   dV += P^T dO, dK += dS^T Q    (A = P / dS straight from the accumulators,
//                                  B = dO / Q columns by transpose reads)
// The next tiles' Q, dO, L, D_i arrive by LDS DMA while the current one is computed.
template <int D, int STAGES, int NW, bool KB>
__global__ __launch_bounds__(64 * NW) void attn_dkdv_mfma(
    TDesc tQ, TDesc tK, TDesc tV, TDesc tG, const float* __restrict__ Lsc,
    const float* __restrict__ Di, const float2* __restrict__ cs, const float* __restrict__ kb,
    const int* __restrict__ kt, TDesc tdK, TDesc tdV, int H, int S, int Spad, float scale,
    int causal, int rope_mode) {
    static_assert(NW == 4 || NW == 8, "four or eight waves");
    using C = DkdvCfg<D, STAGES, NW>;
    extern __shared__ __align__(1024) unsigned char smem[];
    constexpr int NT = D / 32, KS = D / 16, HALVES = NW == 4 ? 2 : 1;
    const int bh = blockIdx.x, j0 = blockIdx.y * 128;
    const bf16_t* Qr = head_base<const bf16_t>(tQ, bh, H);
    const bf16_t* Kr = head_base<const bf16_t>(tK, bh, H);
    const bf16_t* V = head_base<const bf16_t>(tV, bh, H);
    const bf16_t* dO = head_base<const bf16_t>(tG, bh, H);
    const int lane = threadIdx.x & 63, h = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int kg = wave & 3, half0 = NW == 4 ? 0 : wave >> 2;
    const int kw0 = j0 + kg * 32, key = kw0 + (lane & 31);
    const float c2 = scale * 1.4426950408889634f;
    // key-padding bias of this lane's key; the wave's 32 keys lie in one 64-key tile
    const int bb = bh / H;
    const bool kmask = KB && kw0 < S && kt[bb * (Spad / 64) + kw0 / 64];
    const float kbl = kmask && key < S ? kb[(size_t)bb * Spad + key] : 0.f;

    // the block's K and V rows stay in LDS (after the stages) for the whole block
    const bf16_t* sKb = reinterpret_cast<const bf16_t*>(smem + STAGES * C::STAGE);
    const bf16_t* sVb = sKb + 128 * D;
    f32x16_t aV[NT], aK[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) { zero16(aV[t]); zero16(aK[t]); }

    const uint32_t lds0 = lds_addr(smem);
    const int t0 = causal ? j0 / 64 : 0;
    const int T = (S + 63) / 64 - t0;
    TileOffsets<D, NW> oQ, oG;
    oQ.init(tQ.sr, wave);
    oG.init(tG.sr, wave);
    auto issue = [&](int it) {
        const int q0 = (t0 + it) * 64;
        const uint32_t sb = lds0 + (it % STAGES) * C::STAGE;
        dma_tile_o<D, NW>(Qr, tQ.sr, q0, S, sb, wave, oQ);
        dma_tile_o<D, NW>(dO, tG.sr, q0, S, sb + C::TB, wave, oG);
        // 64 L values then 64 D_i values: one DMA instruction per wave
        constexpr int LANES = 32 / NW;  // 16-byte pieces per wave (32 pieces in all)
        if (lane < LANES) {
            const int piece = wave * LANES + lane;  // 0..15: L, 16..31: D_i
            const float* src = (piece < 16 ? Lsc : Di) + (size_t)bh * Spad + q0 + 4 * (piece & 15);
            dma16(src, __builtin_amdgcn_readfirstlane(sb + 2 * C::TB + 16 * LANES * wave));
        }
    };

    {
        const uint32_t kv = lds0 + STAGES * C::STAGE;
        dma_tile<D, NW>(Kr, tK.sr, j0, S, kv);
        dma_tile<D, NW>(Kr, tK.sr, j0 + 64, S, kv + C::TB);
        dma_tile<D, NW>(V, tV.sr, j0, S, kv + 2 * C::TB);
        dma_tile<D, NW>(V, tV.sr, j0 + 64, S, kv + 3 * C::TB);
    }
    issue(0);
    if (STAGES > 2 && T > 1) issue(1);
    // four waves at D = 64: the wave's K and V fragments (8 per k-step row set, 32 registers)
    // are read from LDS once, after the first tile's barrier, and stay in registers
    constexpr bool KVREG = NW == 4 && D == 64;
    bf16x8_t kr[KVREG ? KS : 1], vr[KVREG ? KS : 1];
    for (int it = 0; it < T; ++it) {
        if (STAGES > 2 && it + 1 < T) __builtin_amdgcn_s_waitcnt(vmcnt_imm(C::DMA_PER_TILE));
        else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        __syncthreads();  // tile `it` is in LDS for every wave; the buffer refilled next is free
        if (it + STAGES - 1 < T) issue(it + STAGES - 1);
        if (KVREG && it == 0) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                kr[ks] = frag_rows<D>(sKb, 32 * kg, ks);
                vr[ks] = frag_rows<D>(sVb, 32 * kg, ks);
            }
        }
        const int q0 = (t0 + it) * 64;
        const unsigned char* sb = smem + (it % STAGES) * C::STAGE;
        const bf16_t* sQ = reinterpret_cast<const bf16_t*>(sb);
        const bf16_t* sG = reinterpret_cast<const bf16_t*>(sb + C::TB);
        const float* sL = reinterpret_cast<const float*>(sb + 2 * C::TB);
        const float* sD = sL + 64;
        if (kw0 >= S || (causal && kw0 > q0 + 63)) continue;  // every key of the wave masked
        const bool full = kw0 + 31 < S && q0 + 63 < S && (!causal || kw0 + 31 <= q0);

        // 32-query halves (keeps S, dP, P, dS of one half live).  Masked entries get
        // S = -inf, hence P = dS = 0 (L and D_i are finite everywhere, padding included);
        // only tiles on the diagonal or the sequence end evaluate the mask (an empty volatile
        // asm keeps the compiler from speculating the mask into every tile as selects).
#pragma unroll
        for (int hh = 0; hh < HALVES; ++hh) {
            const int i = half0 + hh;
            // S, dP: all four fragments of k-step ks+1 (Q, dO, K, V rows) are requested before
            // the MFMAs of ks, so no MFMA waits on a read issued right before it; the
            // scheduling fences keep the compiler from hoisting every LDS read up front
            f32x16_t s, dp;
            zero16(s);
            zero16(dp);
            bf16x8_t fa[2][2], kv[2][2];
            fa[0][0] = frag_rows<D>(sQ, 32 * i, 0);
            fa[0][1] = frag_rows<D>(sG, 32 * i, 0);
            if (!KVREG) {
                kv[0][0] = frag_rows<D>(sKb, 32 * kg, 0);
                kv[0][1] = frag_rows<D>(sVb, 32 * kg, 0);
            }
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                if (ks + 1 < KS) {
                    fa[(ks + 1) & 1][0] = frag_rows<D>(sQ, 32 * i, ks + 1);
                    fa[(ks + 1) & 1][1] = frag_rows<D>(sG, 32 * i, ks + 1);
                    if (!KVREG) {
                        kv[(ks + 1) & 1][0] = frag_rows<D>(sKb, 32 * kg, ks + 1);
                        kv[(ks + 1) & 1][1] = frag_rows<D>(sVb, 32 * kg, ks + 1);
                    }
                }
                const int kk = KVREG ? ks : 0;  // in range for the one-element arrays too
                s = mfma32(fa[ks & 1][0], KVREG ? kr[kk] : kv[ks & 1][0], s);
                dp = mfma32(fa[ks & 1][1], KVREG ? vr[kk] : kv[ks & 1][1], dp);
                __builtin_amdgcn_sched_barrier(0);
            }
            // the first transpose fragments of the dV / dK step are in flight during the exp work
            bf16x8_t fb[2][2];
            fb[0][0] = frag_cols<D>(sG, 32 * i, 0);
            fb[0][1] = frag_cols<D>(sQ, 32 * i, 0);
            if (!full) {
                asm volatile("" ::: "memory");
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int q = q0 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
                    const bool ok = q < S && key < S && (!causal || key <= q);
                    s[r] = ok ? s[r] : -INFINITY;
                }
            }
            float pv[16], dv[16];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int ql = 32 * i + 8 * g + 4 * h;
                const float4 L4 = *reinterpret_cast<const float4*>(sL + ql);
                const float4 D4 = *reinterpret_cast<const float4*>(sD + ql);
                float Lv[4] = {L4.x, L4.y, L4.z, L4.w};
                const float Dv[4] = {D4.x, D4.y, D4.z, D4.w};
                if (KB && kmask) {  // wave-uniform: the bias rides on the L term
#pragma unroll
                    for (int e = 0; e < 4; ++e) Lv[e] -= kbl;
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int r = 4 * g + e;
                    pv[r] = __builtin_amdgcn_exp2f(s[r] * c2 - Lv[e]);
                    dv[r] = pv[r] * (dp[r] - Dv[e]);
                }
            }
            bf16x8_t pa[2], da[2];
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                pa[p] = to_bf16x8(pv[8 * p], pv[8 * p + 1], pv[8 * p + 2], pv[8 * p + 3],
                                  pv[8 * p + 4], pv[8 * p + 5], pv[8 * p + 6], pv[8 * p + 7]);
                da[p] = to_bf16x8(dv[8 * p], dv[8 * p + 1], dv[8 * p + 2], dv[8 * p + 3],
                                  dv[8 * p + 4], dv[8 * p + 5], dv[8 * p + 6], dv[8 * p + 7]);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < 2 * NT; ++j) {  // step j: d tile j/2, query rows 16 (j%2)
                if (j + 1 < 2 * NT) {
                    const int kb = 32 * i + 16 * ((j + 1) & 1), n0 = 32 * ((j + 1) >> 1);
                    fb[(j + 1) & 1][0] = frag_cols<D>(sG, kb, n0);
                    fb[(j + 1) & 1][1] = frag_cols<D>(sQ, kb, n0);
                }
                aV[j >> 1] = mfma32(pa[j & 1], fb[j & 1][0], aV[j >> 1]);
                aK[j >> 1] = mfma32(da[j & 1], fb[j & 1][1], aK[j >> 1]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }

    // epilogue: the key group's 32 x D rows (fp32) go through a private LDS strip; with
    // eight waves the second-half wave deposits its partial sums there first
    float* st = reinterpret_cast<float*>(smem) + kg * 32 * (D + 4);
    auto finish = [&](f32x16_t (&acc)[NT], bf16_t* out, int64_t sr, float mul, int mode) {
        __syncthreads();
        if (NW == 4 || half0 == 1) strip_acc<D, NT>(st, acc);
        __syncthreads();
        if (NW == 8 && half0 == 0) {
            const int rq = (lane >> 5) * 4;
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    st[(8 * (r >> 2) + rq + (r & 3)) * (D + 4) + 32 * t + (lane & 31)] += acc[t][r];
        }
        if (half0 == 0) store_rows<D>(st, out, sr, kw0, S, mul, mode, cs);
    };
    finish(aV, head_base<bf16_t>(tdV, bh, H), tdV.sr, 1.f, GN_ROPE_NONE);
    finish(aK, head_base<bf16_t>(tdK, bh, H), tdK.sr, scale, rope_mode);
}

template <int D, int STAGES>
struct DqCfg {
    static constexpr int TB = tile_bytes(D);
    static constexpr int STAGE = 2 * TB;  // K tile, V tile
    static constexpr int DMA_PER_TILE = 2 * (D / 32);
    static constexpr int EPI = 4 * 32 * (D + 4) * 4;
    static constexpr int LDS = STAGES * STAGE > EPI ? STAGES * STAGE : EPI;
};

// dQ for 128 queries (four waves x 32 queries) of one (batch, head); loops over the key
// tiles of 64 those queries can see.  Per key tile and wave:
//   S^T = K Q^T, dP^T = V dO^T    (A = K / V rows from LDS, B = Q / dO fragments in VGPRs)
//   dS^T = P^T (dP^T - D_i)       (each lane owns one query: its L and D_i are scalars)
//   dQ += dS K                    (A = dS from the accumulators, B = K columns by
//                                  transpose reads)
template <int D, int STAGES>
__global__ __launch_bounds__(256) void attn_dq_mfma(
    TDesc tQ, TDesc tK, TDesc tV, TDesc tG, const float* __restrict__ Lsc,
    const float* __restrict__ Di, const float2* __restrict__ cs, const float* __restrict__ kb,
    const int* __restrict__ kt, TDesc tdQ, int H, int S, int Spad, float scale, int causal,
    int rope_mode) {
    using C = DqCfg<D, STAGES>;
    extern __shared__ __align__(1024) unsigned char smem[];
    constexpr int NT = D / 32, KS = D / 16;
    const int nqb = (S + 127) / 128;
    const int bh = blockIdx.x, i0 = (nqb - 1 - (int)blockIdx.y) * 128;  // longest rows first
    const bf16_t* Qr = head_base<const bf16_t>(tQ, bh, H);
    const bf16_t* Kr = head_base<const bf16_t>(tK, bh, H);
    const bf16_t* V = head_base<const bf16_t>(tV, bh, H);
    const bf16_t* dO = head_base<const bf16_t>(tG, bh, H);
    const int lane = threadIdx.x & 63, h = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int qw0 = i0 + wave * 32, q = qw0 + (lane & 31), qc = min(q, S - 1);
    const float c2 = scale * 1.4426950408889634f;

    bf16x8_t qf[KS], of[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        qf[ks] = ld_frag16(Qr + qc * tQ.sr + 8 * h + 16 * ks);
        of[ks] = ld_frag16(dO + qc * tG.sr + 8 * h + 16 * ks);
    }
    const float lq = Lsc[(size_t)bh * Spad + qc], dq = Di[(size_t)bh * Spad + qc];
    f32x16_t aQ[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) zero16(aQ[t]);

    const uint32_t lds0 = lds_addr(smem);
    const int kend = causal ? min(S, i0 + 128) : S;
    const int T = (kend + 63) / 64;
    TileOffsets<D> oK, oV;
    oK.init(tK.sr, wave);
    oV.init(tV.sr, wave);
    auto issue = [&](int it) {
        const uint32_t sb = lds0 + (it % STAGES) * C::STAGE;
        dma_tile_o<D>(Kr, tK.sr, it * 64, S, sb, wave, oK);
        dma_tile_o<D>(V, tV.sr, it * 64, S, sb + C::TB, wave, oV);
    };

    issue(0);
    if (STAGES > 2 && T > 1) issue(1);
    for (int it = 0; it < T; ++it) {
        if (STAGES > 2 && it + 1 < T) __builtin_amdgcn_s_waitcnt(vmcnt_imm(C::DMA_PER_TILE));
        else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        __syncthreads();
        if (it + STAGES - 1 < T) issue(it + STAGES - 1);
        const int k0 = it * 64;
        const unsigned char* sb = smem + (it % STAGES) * C::STAGE;
        const bf16_t* sK = reinterpret_cast<const bf16_t*>(sb);
        const bf16_t* sV = reinterpret_cast<const bf16_t*>(sb + C::TB);
        if (qw0 >= S || (causal && k0 > qw0 + 31)) continue;  // every key masked for the wave
        const bool full = qw0 + 31 < S && k0 + 63 < S && (!causal || k0 + 63 <= qw0);
        const float* kbt = kb && kt[(bh / H) * (Spad / 64) + it] ? kb + (size_t)(bh / H) * Spad + k0 : nullptr;

        // masked entries get S = -inf, hence dS = 0
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            f32x16_t s, dp;
            zero16(s);
            zero16(dp);
            bf16x8_t fa[2][2];
            fa[0][0] = frag_rows<D>(sK, 32 * i, 0);
            fa[0][1] = frag_rows<D>(sV, 32 * i, 0);
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                if (ks + 1 < KS) {
                    fa[(ks + 1) & 1][0] = frag_rows<D>(sK, 32 * i, ks + 1);
                    fa[(ks + 1) & 1][1] = frag_rows<D>(sV, 32 * i, ks + 1);
                }
                s = mfma32(fa[ks & 1][0], qf[ks], s);
                dp = mfma32(fa[ks & 1][1], of[ks], dp);
                __builtin_amdgcn_sched_barrier(0);
            }
            bf16x8_t fb[2];
            fb[0] = frag_cols<D>(sK, 32 * i, 0);
            if (!full) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int kk = k0 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
                    const bool ok = q < S && kk < S && (!causal || kk <= q);
                    s[r] = ok ? s[r] : -INFINITY;
                }
            }
            float dv[16];
            if (kbt) {  // key-padding biases of the 16 keys this lane holds (masked tiles only),
                        // in score units (scale > 0, checked by the entry points)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const float4 k4 = *reinterpret_cast<const float4*>(kbt + 32 * i + 8 * g + 4 * h);
                    s[4 * g] += k4.x / c2;
                    s[4 * g + 1] += k4.y / c2;
                    s[4 * g + 2] += k4.z / c2;
                    s[4 * g + 3] += k4.w / c2;
                }
            }
#pragma unroll
            for (int r = 0; r < 16; ++r)
                dv[r] = __builtin_amdgcn_exp2f(s[r] * c2 - lq) * (dp[r] - dq);
            bf16x8_t da[2];
#pragma unroll
            for (int p = 0; p < 2; ++p)
                da[p] = to_bf16x8(dv[8 * p], dv[8 * p + 1], dv[8 * p + 2], dv[8 * p + 3],
                                  dv[8 * p + 4], dv[8 * p + 5], dv[8 * p + 6], dv[8 * p + 7]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < 2 * NT; ++j) {
                if (j + 1 < 2 * NT)
                    fb[(j + 1) & 1] = frag_cols<D>(sK, 32 * i + 16 * ((j + 1) & 1), 32 * ((j + 1) >> 1));
                aQ[j >> 1] = mfma32(da[j & 1], fb[j & 1], aQ[j >> 1]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }

    __syncthreads();
    float* st = reinterpret_cast<float*>(smem) + wave * 32 * (D + 4);
    strip_acc<D, NT>(st, aQ);
    __syncthreads();
    store_rows<D>(st, head_base<bf16_t>(tdQ, bh, H), tdQ.sr, qw0, S, scale, rope_mode, cs);
}

// Forward producing the backward's saved tensors: O and the fp32 row logsumexp (natural
// log, S scaled), flash-attention2-rope.glsl:165-247 semantics with the causal mask.  One
// block per (b*h, 128 queries), four waves x 32 queries; K and V tiles of 64 keys arrive by
// LDS DMA (two stages).  Per key tile and wave:
//   S^T = K Q^T      (A = K rows from LDS, B = Q fragments kept in VGPRs): lane = query, so
//                    the running max m and sum l are per-lane scalars (plus one exchange
//                    with lane ^ 32, which holds the other 16 keys of each 32-key half);
//   P^T = exp2(S^T scale log2e - m)  (m in the same base-2 units), O^T = alpha O^T;
//   O^T += V^T P^T   (A = V columns by transpose reads, whose key order is the
//                    accumulator's row order, B = P^T converted in registers).
// The epilogue scales by 1/l, transposes each wave's 32 x D block through LDS and writes
// bf16 rows; LSE = (m + log2 l) ln 2.
template <int D, int STAGES>
__global__ __launch_bounds__(256) void attn_fwd_mfma(TDesc tQ, TDesc tK, TDesc tV, TDesc tO,
                                                     float* __restrict__ LSE,
                                                     const float* __restrict__ kb,
                                                     const int* __restrict__ kt, int H, int S,
                                                     int Spad, float scale, int causal) {
    using C = DqCfg<D, STAGES>;
    extern __shared__ __align__(1024) unsigned char smem[];
    constexpr int NT = D / 32, KS = D / 16;
    const int nqb = (S + 127) / 128;
    const int bh = blockIdx.x, i0 = (nqb - 1 - (int)blockIdx.y) * 128;  // longest rows first
    const bf16_t* Qr = head_base<const bf16_t>(tQ, bh, H);
    const bf16_t* Kr = head_base<const bf16_t>(tK, bh, H);
    const bf16_t* V = head_base<const bf16_t>(tV, bh, H);
    const int lane = threadIdx.x & 63, h = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int qw0 = i0 + wave * 32, q = qw0 + (lane & 31), qc = min(q, S - 1);
    const float c2 = scale * 1.4426950408889634f;

    bf16x8_t qf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = ld_frag16(Qr + qc * tQ.sr + 8 * h + 16 * ks);
    f32x16_t aO[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) zero16(aO[t]);
    float m = -INFINITY, l = 0.f;

    const uint32_t lds0 = lds_addr(smem);
    const int kend = causal ? min(S, i0 + 128) : S;
    const int T = (kend + 63) / 64;
    TileOffsets<D> oK, oV;
    oK.init(tK.sr, wave);
    oV.init(tV.sr, wave);
    auto issue = [&](int it) {
        const uint32_t sb = lds0 + (it % STAGES) * C::STAGE;
        dma_tile_o<D>(Kr, tK.sr, it * 64, S, sb, wave, oK);
        dma_tile_o<D>(V, tV.sr, it * 64, S, sb + C::TB, wave, oV);
    };

    issue(0);
    if (STAGES > 2 && T > 1) issue(1);
    for (int it = 0; it < T; ++it) {
        if (STAGES > 2 && it + 1 < T) __builtin_amdgcn_s_waitcnt(vmcnt_imm(C::DMA_PER_TILE));
        else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        __syncthreads();
        if (it + STAGES - 1 < T) issue(it + STAGES - 1);
        const int k0 = it * 64;
        const unsigned char* sb = smem + (it % STAGES) * C::STAGE;
        const bf16_t* sK = reinterpret_cast<const bf16_t*>(sb);
        const bf16_t* sV = reinterpret_cast<const bf16_t*>(sb + C::TB);
        if (qw0 >= S || (causal && k0 > qw0 + 31)) continue;  // every key masked for the wave
        const bool full = qw0 + 31 < S && k0 + 63 < S && (!causal || k0 + 63 <= qw0);
        const float* kbt = kb && kt[(bh / H) * (Spad / 64) + it] ? kb + (size_t)(bh / H) * Spad + k0 : nullptr;

        f32x16_t sc[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            zero16(sc[i]);
            bf16x8_t fa[2];
            fa[0] = frag_rows<D>(sK, 32 * i, 0);
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                if (ks + 1 < KS) fa[(ks + 1) & 1] = frag_rows<D>(sK, 32 * i, ks + 1);
                sc[i] = mfma32(fa[ks & 1], qf[ks], sc[i]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // scores in base-2 units; masked entries are -inf (P = 0)
        float mt = -INFINITY;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float v = sc[i][r] * c2;
                if (kbt) v += kbt[32 * i + 8 * (r >> 2) + 4 * h + (r & 3)];
                if (!full) {
                    const int kk = k0 + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
                    const bool ok = q < S && kk < S && (!causal || kk <= q);
                    v = ok ? v : -INFINITY;
                }
                sc[i][r] = v;
                mt = fmaxf(mt, v);
            }
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float mn = fmaxf(m, mt);
        const float ms = mn == -INFINITY ? 0.f : mn;  // a row with no visible key yet stays empty
        const float alpha = __builtin_amdgcn_exp2f(m - ms);
        float ps = 0.f;
        bf16x8_t pb[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            float pv[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                pv[e] = __builtin_amdgcn_exp2f(sc[p >> 1][8 * (p & 1) + e] - ms);
                ps += pv[e];
            }
            pb[p] = to_bf16x8(pv[0], pv[1], pv[2], pv[3], pv[4], pv[5], pv[6], pv[7]);
        }
        ps += __shfl_xor(ps, 32);
        l = l * alpha + ps;
        m = mn;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) aO[t][r] *= alpha;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            bf16x8_t fv[2];
            fv[0] = frag_cols<D>(sV, 0, 32 * t);
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                if (p + 1 < 4) fv[(p + 1) & 1] = frag_cols<D>(sV, 16 * (p + 1), 32 * t);
                aO[t] = mfma32(fv[p & 1], pb[p], aO[t]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }

    __syncthreads();
    float* st = reinterpret_cast<float*>(smem) + wave * 32 * (D + 4);
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    // O^T accumulators: lane = query (column), rows = d; transpose into the wave's strip
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r)
            st[(lane & 31) * (D + 4) + 32 * t + 8 * (r >> 2) + 4 * h + (r & 3)] = aO[t][r] * inv;
    __syncthreads();
    store_rows<D>(st, head_base<bf16_t>(tO, bh, H), tO.sr, qw0, S, 1.0f, GN_ROPE_NONE, nullptr);
    if (h == 0 && q < S)
        LSE[(size_t)bh * S + q] = (m + __log2f(l)) * 0.6931471805599453f;
}

// cos/sin table [S][D/2] of the RoPE angles (pair i at position p)
__global__ __launch_bounds__(256) void rope_table(float2* __restrict__ cs, int S, int D,
                                                  float theta) {
    const int half = D / 2;
    for (int64_t idx = blockIdx.x * (int64_t)256 + threadIdx.x; idx < (int64_t)S * half;
         idx += (int64_t)gridDim.x * 256) {
        float c, s;
        rope_cs((int)(idx / half), (int)(idx % half), D, theta, c, s);
        cs[idx] = make_float2(c, s);
    }
}

// The cos/sin entries chunk c of a row at position pos needs: 4 pairs (interleaved mode,
// pairs 4c .. 4c+3) or 8 (half mode, pairs 8 (c mod D/16) .. +7), as 16-byte loads, issued
// with the row's own loads so a lane waits on one memory round trip.
template <int D>
struct RopeTab {
    float4 w[4];  // pair e: (w[e / 2].x, .y) for even e, (.z, .w) for odd e
    __device__ __forceinline__ float2 operator[](int e) const {
        const float4 v = w[e >> 1];
        return (e & 1) ? make_float2(v.z, v.w) : make_float2(v.x, v.y);
    }
};
template <int D>
__device__ __forceinline__ void load_rope_tab(const float2* __restrict__ cs, int pos, int c, int mode,
                                              RopeTab<D>& tab) {
    constexpr int LPR = D / 8;
    const float4* t = reinterpret_cast<const float4*>(cs + (size_t)pos * (D / 2));
    const bool inter = mode == GN_ROPE_INTERLEAVED;  // uniform: a kernel argument
    const int base = inter ? 2 * c : 4 * (c % (LPR / 2));
    // four unconditional loads from in-row addresses (the interleaved mode re-reads its second
    // vector for the unused pairs 4..7), so no load hides behind a branch or a pointer select
    tab.w[0] = t[base];
    tab.w[1] = t[base + 1];
    tab.w[2] = t[inter ? base + 1 : base + 2];
    tab.w[3] = t[inter ? base + 1 : base + 3];
}

// Rotate chunk c (8 elements) of one row of Q and of K (qk4[0], qk4[1], bf16) with the
// chunk's cos/sin entries (load_rope_tab), into Qout / Kout.  Lanes c of one row are D/8
// consecutive lanes (the half mode pairs chunk c with chunk c ^ D/16 across lanes).
template <int D>
__device__ __forceinline__ void rotate_qk_chunk(const uint4 (&qk4)[2], int c, const RopeTab<D>& tab,
                                                int mode, bf16_t* __restrict__ Qout,
                                                bf16_t* __restrict__ Kout) {
    constexpr int LPR = D / 8;
#pragma unroll
    for (int which = 0; which < 2; ++which) {
        const uint4 v4 = qk4[which];
        const uint32_t vw[4] = {v4.x, v4.y, v4.z, v4.w};
        float x[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[2 * e] = __uint_as_float(vw[e] << 16);
            x[2 * e + 1] = __uint_as_float(vw[e] & 0xffff0000u);
        }
        if (mode == GN_ROPE_INTERLEAVED) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float2 r = tab[e];
                const float x0 = x[2 * e], x1 = x[2 * e + 1];
                x[2 * e] = x0 * r.x - x1 * r.y;
                x[2 * e + 1] = x0 * r.y + x1 * r.x;
            }
        } else {  // GN_ROPE_HALF: element e pairs with the same element of chunk c ^ LPR/2
            const bool lo = c < LPR / 2;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float xp = __shfl_xor(x[e], LPR / 2);
                const float2 r = tab[e];
                x[e] = lo ? x[e] * r.x - xp * r.y : xp * r.y + x[e] * r.x;
            }
        }
        *reinterpret_cast<bf16x8_t*>(which ? Kout : Qout) =
            to_bf16x8(x[0], x[1], x[2], x[3], x[4], x[5], x[6], x[7]);
    }
}

// Forward pre-pass (RoPE on): rotated bf16 copies of Q and K from the cos/sin table, D/8
// lanes per row, both tensors in one launch.
template <int D>
__global__ __launch_bounds__(256) void rope_qk_prep(TDesc tQ, TDesc tK, bf16_t* __restrict__ Qr,
                                                    bf16_t* __restrict__ Kr,
                                                    const float2* __restrict__ cs, int64_t rows,
                                                    int H, int S, int mode) {
    constexpr int LPR = D / 8;
    const unsigned gid = blockIdx.x * 256u + threadIdx.x;  // rows * LPR < 2^31 (host check)
    const unsigned row = gid / LPR;
    const int c = (int)(gid % LPR);
    if (row >= (unsigned)rows) return;  // LPR divides 256: whole row groups leave together
    const int pos = (int)(row % (unsigned)S);
    const unsigned bh = row / (unsigned)S;
    const uint4 qk4[2] = {
        *reinterpret_cast<const uint4*>(head_base<const bf16_t>(tQ, (int)bh, H) + pos * tQ.sr + 8 * c),
        *reinterpret_cast<const uint4*>(head_base<const bf16_t>(tK, (int)bh, H) + pos * tK.sr + 8 * c)};
    RopeTab<D> tab;
    load_rope_tab<D>(cs, pos, c, mode, tab);
    const size_t off = (size_t)row * D + 8 * c;
    rotate_qk_chunk<D>(qk4, c, tab, mode, Qr + off, Kr + off);
}

// Pre-pass of the MFMA path, D/8 lanes per row: rotated Q and K (bf16), D_i = rowsum(dO*O)
// and L log2(e), both into [B*H][Spad] arrays whose padding the kernels never unmask.
template <int D>
__global__ __launch_bounds__(256) void attn_prep(
    TDesc tQ, TDesc tK, TDesc tG, TDesc tO, const float* __restrict__ LSE, bf16_t* __restrict__ Qr,
    bf16_t* __restrict__ Kr, float* __restrict__ Lsc, float* __restrict__ Di,
    const float2* __restrict__ cs, int64_t rows, int H, int S, int Spad, int mode) {
    constexpr int LPR = D / 8;
    const unsigned gid = blockIdx.x * 256u + threadIdx.x;  // rows * LPR < 2^31 (host check)
    const unsigned row = gid / LPR;
    const int c = (int)(gid % LPR);
    if (row >= (unsigned)rows) return;  // LPR divides 256: whole row groups leave together
    const int pos = (int)(row % (unsigned)S);
    const unsigned bh = row / (unsigned)S;
    const size_t off = (size_t)row * D + 8 * c;  // in the [B,H,S,D] Qr, Kr copies
    // every global load up front, so one round trip covers them all
    const uint4 o4 = *reinterpret_cast<const uint4*>(head_base<const bf16_t>(tO, (int)bh, H) + pos * tO.sr + 8 * c);
    const uint4 g4 = *reinterpret_cast<const uint4*>(head_base<const bf16_t>(tG, (int)bh, H) + pos * tG.sr + 8 * c);
    uint4 qk4[2] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
    RopeTab<D> tab;
    if (mode != GN_ROPE_NONE) {
        qk4[0] = *reinterpret_cast<const uint4*>(head_base<const bf16_t>(tQ, (int)bh, H) + pos * tQ.sr + 8 * c);
        qk4[1] = *reinterpret_cast<const uint4*>(head_base<const bf16_t>(tK, (int)bh, H) + pos * tK.sr + 8 * c);
        load_rope_tab<D>(cs, pos, c, mode, tab);
    }
    const float lse = LSE[row];  // every lane of the row (one address)
    const uint32_t ow[4] = {o4.x, o4.y, o4.z, o4.w}, gw[4] = {g4.x, g4.y, g4.z, g4.w};
    float dot = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        dot += __uint_as_float(ow[e] << 16) * __uint_as_float(gw[e] << 16);
        dot += __uint_as_float(ow[e] & 0xffff0000u) * __uint_as_float(gw[e] & 0xffff0000u);
    }
#pragma unroll
    for (int m = LPR / 2; m >= 1; m >>= 1) dot += __shfl_xor(dot, m);
    // every lane of the row holds the full dot (butterfly) and stores the row's two values
    // (same address and value across the row's lanes): no branch, so the LSE load stays with
    // the others instead of being sunk behind their wait
    Di[(size_t)bh * Spad + pos] = dot;
    // a row with every visible key masked (LSE = -inf, O = 0) gets P = 0 through L = +inf
    Lsc[(size_t)bh * Spad + pos] = lse == -INFINITY ? INFINITY : lse * 1.4426950408889634f;
    if (c == 0 && pos == S - 1)  // finite padding: masked entries compute exp2(-inf - 0) * (dP - 0)
        for (int p = S; p < Spad; ++p) Di[(size_t)bh * Spad + p] = Lsc[(size_t)bh * Spad + p] = 0.f;
    if (mode == GN_ROPE_NONE) return;
    rotate_qk_chunk<D>(qk4, c, tab, mode, Qr + off, Kr + off);
}

// Key-padding pre-pass: kb[b][k] = the reference's score bias (mask[b S + k] - 1) 1e9 in
// base-2 units, -inf where that bias is below -1e4 (exp() of the biased score is then 0 in fp32
// for any row that keeps a key), 0 past S; kt[b][t] = 1 when 64-key tile t holds a nonzero
// bias.  One wave per tile.
__global__ __launch_bounds__(256) void attn_key_bias(const float* __restrict__ mask,
                                                     float* __restrict__ kb, int* __restrict__ kt,
                                                     int B, int S, int Spad) {
    const int tile = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int tiles = Spad / 64;
    if (tile >= B * tiles) return;  // whole waves leave together
    const int b = tile / tiles, k = (tile % tiles) * 64 + lane;
    float v = 0.f;
    if (k < S) {
        const float bias = (mask[(size_t)b * S + k] - 1.0f) * 1e9f;
        v = bias < -1e4f ? -INFINITY : bias * 1.4426950408889634f;
    }
    kb[(size_t)b * Spad + k] = v;
    const unsigned long long any = __ballot(v != 0.f);
    if (lane == 0) kt[tile] = any != 0ull;
}

// ---- generic MFMA path: D a multiple of 32 up to 256, bf16 or fp32 ---------------------
//
// For the head dims and dtypes the tuned kernels above do not take: bf16 with D = 32, 96, 192
// or 256, and fp32 at any of those D and at 64 and 128.  fp32 operands run on the bf16 matrix
// cores as NP = 2 pieces x = hi + lo (hi = bf16(x), lo = bf16(x - hi), |x - hi - lo| <=
// 2^-17 |x|); a product takes lo.hi + hi.lo + hi.hi (the dropped lo.lo is below 2^-16 of
// |a b|), and P and dS are split the same way in registers.  One template serves both passes:
//   ROLE 0 (dK, dV): wave rows = 32 keys, tiles = 32 queries;
//       S = Q K^T, dP = dO V^T  (A = tile rows, B = the wave's rows),
//       P = exp2(S scale log2e + bias - L log2e), dS = P (dP - D_i),
//       dV += P^T dO, dK += dS^T Q  (A = P / dS from the accumulators, B = tile columns);
//   ROLE 1 (dQ): wave rows = 32 queries, tiles = 32 keys;
//       S^T = K Q^T, dP^T = V dO^T, then dQ += dS K.
// The wave's own operand rows (K, V or Q, dO) stay in registers when D NP <= 256, else they are
// re-read per tile (L2); a tile (both tensors, every piece) is staged through registers into
// LDS (row pitch D + 8 elements), double-buffered, one barrier per tile.  The dK/dV pass
// accumulates DC <= 128 columns per block (gridDim.z column groups for D > 128; S and dP are
// then formed once per group).  Gradients leave as fp32 rows, dQ and dK times scale in the
// rotated space, for the un-rotating conversion pass.
struct GenIn {
    const bf16_t* t[4][2];  // [Q (rotated), K (rotated), V, dO][piece], each [B*H][S][D]
};

template <int NP>
__device__ __forceinline__ f32x16_t mma_np(const bf16x8_t (&a)[NP], const bf16x8_t (&b)[NP],
                                           f32x16_t c) {
    if constexpr (NP == 2) {
        c = mfma32(a[1], b[0], c);
        c = mfma32(a[0], b[1], c);
    }
    return mfma32(a[0], b[0], c);
}

// 8 accumulator values -> NP bf16 operand pieces (hi, then the rounding residual)
template <int NP>
__device__ __forceinline__ void split8(const float* v, bf16x8_t (&o)[NP]) {
    o[0] = to_bf16x8(v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]);
    if constexpr (NP == 2) {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[NP - 1][e] = (__bf16)(v[e] - (float)o[0][e]);
    }
}

template <int D, int NP>
struct GenCfg {
    static constexpr int P = D + 8;                       // LDS row pitch (elements)
    static constexpr int TILE = 2 * NP * 32 * P * 2;      // both tensors, all pieces (bytes)
    static constexpr int STAGE = TILE + 256;              // + 64 floats of per-row data
    static constexpr int LDS = 2 * STAGE;
    static constexpr int CHUNKS = 2 * NP * 32 * (D / 8);  // 16-byte pieces per tile
    static constexpr int NCH = CHUNKS / 256;              // per thread
    static_assert(CHUNKS % 256 == 0, "every thread stages the same number of pieces");
    static constexpr bool RES = D * NP <= 256;            // wave rows held in registers
};

// A tile's register staging: thread tid holds 16-byte pieces j = tid + 256 u of the tile
// (tensor-piece group tp = j / (32 D/8), row, chunk), plus one float4 of per-row data.
template <int D, int NP>
struct GenStage {
    uint4 v[GenCfg<D, NP>::NCH];
    float4 r;
};
struct GenSrc {
    const bf16_t *p0, *p1, *p2, *p3;  // tile planes by group tp (NP = 1: p0, p2)
    const float *r0, *r1;             // row data: r0 then r1 (r1 null: r0 only, 32 floats)
    const float* any;                 // a readable float array (stands in for a null r0 / r1)
    size_t roff, hb;                  // row-data offset of the head / batch; head offset
};

template <int D, int NP>
__device__ __forceinline__ void gen_load(GenStage<D, NP>& st, const GenSrc& g, int t0, int S, int tid) {
    using C = GenCfg<D, NP>;
    constexpr int CR = D / 8;
    // unconditional loads (a conditional one would make the staging array a memory object)
#pragma unroll
    for (int u = 0; u < C::NCH; ++u) {
        const int j = tid + 256 * u;
        const int ch = j % CR, row = (j / CR) % 32, tp = j / (CR * 32);
        const bf16_t* p = NP == 1 ? (tp == 0 ? g.p0 : g.p2)
                                  : (tp == 0 ? g.p0 : tp == 1 ? g.p1 : tp == 2 ? g.p2 : g.p3);
        st.v[u] = *reinterpret_cast<const uint4*>(p + g.hb + (size_t)min(t0 + row, S - 1) * D + 8 * ch);
    }
    // 32 floats from r0 (threads 0-7) then 32 from r1 (threads 8-15); zeros elsewhere
    const float* rp = tid < 8 ? g.r0 : g.r1;
    const bool ok = tid < 16 && rp;
    const float4 v = *reinterpret_cast<const float4*>(ok ? rp + g.roff + t0 + 4 * (tid & 7) : g.any);
    st.r = ok ? v : make_float4(0.f, 0.f, 0.f, 0.f);
}

template <int D, int NP>
__device__ __forceinline__ void gen_store(const GenStage<D, NP>& st, unsigned char* sb, int tid) {
    using C = GenCfg<D, NP>;
    constexpr int CR = D / 8;
#pragma unroll
    for (int u = 0; u < C::NCH; ++u) {
        const int j = tid + 256 * u;
        const int ch = j % CR, row = (j / CR) % 32, tp = j / (CR * 32);
        *reinterpret_cast<uint4*>(sb + ((tp * 32 + row) * C::P + 8 * ch) * 2) = st.v[u];
    }
    if (tid < 16) reinterpret_cast<float4*>(sb + C::TILE)[tid] = st.r;
}

template <int ROLE, int D, int NP, int DC>
__global__ __launch_bounds__(256) void attn_bwd_gen(GenIn in, const float* __restrict__ L2,
                                                    const float* __restrict__ Di,
                                                    const float* __restrict__ kb,
                                                    float* __restrict__ outA,
                                                    float* __restrict__ outB, int H, int S,
                                                    int Spad, float scale, int causal) {
    using C = GenCfg<D, NP>;
    constexpr int KS = D / 16, NT = DC / 32, CR = D / 8;
    extern __shared__ __align__(16) unsigned char smem[];
    const int bh = blockIdx.x, bb = bh / H;
    const int lane = threadIdx.x & 63, h = lane >> 5, tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int blk = ROLE == 0 ? (int)blockIdx.y : (S + 127) / 128 - 1 - (int)blockIdx.y;
    const int w0 = blk * 128 + 32 * wave, wrow = w0 + (lane & 31);
    const int dcol0 = blockIdx.z * DC;
    const float c2 = scale * 1.4426950408889634f;
    const size_t hb = (size_t)bh * S * D;
    // tensors by role: W = the wave's rows, T = the tiles
    constexpr int w_t0 = ROLE == 0 ? 1 : 0, w_t1 = ROLE == 0 ? 2 : 3;
    constexpr int t_t0 = ROLE == 0 ? 0 : 1, t_t1 = ROLE == 0 ? 3 : 2;
    // the tile planes as scalars (a per-thread index into the argument array would put it in
    // scratch memory): tile chunk group tp = tensor * NP + piece
    const bf16_t* tp0 = in.t[t_t0][0];
    const bf16_t* tp1 = in.t[t_t0][NP - 1];
    const bf16_t* tp2 = in.t[t_t1][0];
    const bf16_t* tp3 = in.t[t_t1][NP - 1];

    // the wave's operand rows: B fragments (lane -> row wrow, k = d)
    const size_t wr = hb + (size_t)min(wrow, S - 1) * D + 8 * h;
    auto wfrag = [&](int which, int ks, int p) {
        return ld_frag16((which ? in.t[w_t1][p] : in.t[w_t0][p]) + wr + 16 * ks);
    };
    bf16x8_t wres[C::RES ? 2 : 1][C::RES ? KS : 1][NP];
    if constexpr (C::RES) {
#pragma unroll
        for (int which = 0; which < 2; ++which)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                for (int p = 0; p < NP; ++p) wres[which][ks][p] = wfrag(which, ks, p);
    }
    // per-lane row data of the wave's rows: key bias (ROLE 0), L log2e and D_i (ROLE 1)
    float lb = 0.f, lL = 0.f, lD = 0.f;
    if (ROLE == 0) {
        lb = kb && wrow < S ? kb[(size_t)bb * Spad + wrow] : 0.f;
    } else {
        lL = L2[(size_t)bh * Spad + min(wrow, S - 1)];
        lD = Di[(size_t)bh * Spad + min(wrow, S - 1)];
    }

    f32x16_t accA[ROLE == 0 ? NT : 1], accB[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        zero16(accB[t]);
        if (ROLE == 0) zero16(accA[t]);
    }

    // tiles of 32 rows: ROLE 0 queries from the block's first key (causal) to S; ROLE 1 keys
    // from 0 to the block's last query (causal) or S
    const int tbeg = ROLE == 0 && causal ? blk * 128 : 0;
    const int tend = ROLE == 1 && causal ? min(S, blk * 128 + 128) : S;
    const int T = tbeg < tend ? (tend - tbeg + 31) / 32 : 0;
    GenStage<D, NP> stg;
    const GenSrc src{tp0, tp1, tp2, tp3, ROLE == 0 ? L2 : kb, ROLE == 0 ? Di : nullptr, L2,
                     ROLE == 0 ? (size_t)bh * Spad : (size_t)bb * Spad, hb};
    // T >= 1 (the causal ranges always hold the block's own rows).  The loads and stores run
    // unconditionally (the last iteration re-stages its own tile into the unused buffer), so the
    // staging registers stay registers.
    gen_load<D, NP>(stg, src, tbeg, S, tid);
    gen_store<D, NP>(stg, smem, tid);
    for (int it = 0; it < T; ++it) {
        __syncthreads();  // tile it is in LDS; the other buffer's readers are done
        gen_load<D, NP>(stg, src, tbeg + 32 * min(it + 1, T - 1), S, tid);
        const int t0 = tbeg + 32 * it;
        const unsigned char* sb = smem + (it & 1) * C::STAGE;
        const bf16_t* tT[2][NP];
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            tT[0][p] = reinterpret_cast<const bf16_t*>(sb) + (size_t)p * 32 * C::P;
            tT[1][p] = reinterpret_cast<const bf16_t*>(sb) + (size_t)(NP + p) * 32 * C::P;
        }
        const float* srow = reinterpret_cast<const float*>(sb + C::TILE);
        // tile rows t0 .. t0+31 against the wave's rows w0 .. w0+31
        const int q_lo = ROLE == 0 ? t0 : w0, k_lo = ROLE == 0 ? w0 : t0;
        const bool skip = w0 >= S || (causal && k_lo > q_lo + 31);
        if (!skip) {
            const bool full = t0 + 31 < S && w0 + 31 < S && (!causal || k_lo + 31 <= q_lo);
            f32x16_t s, dp;
            zero16(s);
            zero16(dp);
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                bf16x8_t a0[NP], a1[NP], b0[NP], b1[NP];
#pragma unroll
                for (int p = 0; p < NP; ++p) {
                    a0[p] = ld_frag16(tT[0][p] + (lane & 31) * C::P + 16 * ks + 8 * h);
                    a1[p] = ld_frag16(tT[1][p] + (lane & 31) * C::P + 16 * ks + 8 * h);
                    if constexpr (C::RES) {
                        b0[p] = wres[0][ks][p];
                        b1[p] = wres[1][ks][p];
                    } else {
                        b0[p] = wfrag(0, ks, p);
                        b1[p] = wfrag(1, ks, p);
                    }
                }
                s = mma_np<NP>(a0, b0, s);
                dp = mma_np<NP>(a1, b1, dp);
            }
            // element r: tile row t0 + 8(r/4) + 4h + r%4, wave row wrow
            float pv[16], dv[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int tr = 8 * (r >> 2) + 4 * h + (r & 3);
                float Lr, Dr, br;
                if (ROLE == 0) { Lr = srow[tr]; Dr = srow[32 + tr]; br = lb; }
                else { Lr = lL; Dr = lD; br = kb ? srow[tr] : 0.f; }
                float x = s[r] * c2 + br - Lr;
                if (!full) {
                    const int q = ROLE == 0 ? t0 + tr : wrow, k = ROLE == 0 ? wrow : t0 + tr;
                    x = (q < S && k < S && (!causal || k <= q)) ? x : -INFINITY;
                }
                pv[r] = __builtin_amdgcn_exp2f(x);
                dv[r] = pv[r] * (dp[r] - Dr);
            }
            bf16x8_t pa[2][NP], da[2][NP];
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                if (ROLE == 0) split8<NP>(pv + 8 * p, pa[p]);
                split8<NP>(dv + 8 * p, da[p]);
            }
            // k-step p: tile rows 16p + {4h, 8 + 4h} + 0..3 in both operands
#pragma unroll
            for (int p = 0; p < 2; ++p)
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const int n0 = dcol0 + 32 * t;
                    bf16x8_t c0[NP], c1[NP];
#pragma unroll
                    for (int q = 0; q < NP; ++q) {
                        const int lan = lane & 15;
                        const int col = n0 + 16 * ((lane >> 4) & 1) + 4 * (lan & 3);
                        const int r0 = 16 * p + 4 * h + (lan >> 2);
                        c0[q] = ld_tr_pair(tT[0][q] + r0 * C::P + col, tT[0][q] + (r0 + 8) * C::P + col);
                        if (ROLE == 0)
                            c1[q] = ld_tr_pair(tT[1][q] + r0 * C::P + col, tT[1][q] + (r0 + 8) * C::P + col);
                    }
                    if (ROLE == 0) accA[t] = mma_np<NP>(pa[p], c1, accA[t]);
                    accB[t] = mma_np<NP>(da[p], c0, accB[t]);
                }
        }
        gen_store<D, NP>(stg, smem + ((it + 1) & 1) * C::STAGE, tid);
    }

    // fp32 rows out: column dcol0 + 32t + lane%32, wave rows w0 + 8(r/4) + 4h + r%4
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = w0 + 8 * (r >> 2) + 4 * h + (r & 3);
            if (row < S) {
                const size_t o = hb + (size_t)row * D + dcol0 + 32 * t + (lane & 31);
                outB[o] = accB[t][r] * scale;
                if (ROLE == 0) outA[o] = accA[t][r];
            }
        }
}

// Generic forward (same D, dtypes and operand pieces as attn_bwd_gen): one block per (b*h, 128
// queries), four waves x 32 queries, key tiles of 32 staged into LDS.  Per tile and wave:
//   S^T = K Q^T (A = K tile rows, B = the wave's Q rows, in registers or re-read): lane = query,
//   so the running max m and sum l are per-lane (one exchange with lane ^ 32 per tile);
//   P^T = exp2(S^T scale log2e + bias - m), O^T = alpha O^T + V^T P^T (A = V tile columns by
//   transpose reads, B = P^T from the accumulator, both in the accumulator's key order).
// O = O^T / l leaves in the input dtype, LSE = (m + log2 l) ln 2 (-inf for a row with no visible
// kept key, whose O is 0).
template <typename T, int D, int NP>
__global__ __launch_bounds__(256) void attn_fwd_gen(GenIn in, const float* __restrict__ kb,
                                                    T* __restrict__ O, float* __restrict__ LSE,
                                                    int H, int S, int Spad, float scale, int causal) {
    using C = GenCfg<D, NP>;
    constexpr int KS = D / 16, NT = D / 32;
    extern __shared__ __align__(16) unsigned char smem[];
    const int bh = blockIdx.x, bb = bh / H;
    const int lane = threadIdx.x & 63, h = lane >> 5, tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int blk = (S + 127) / 128 - 1 - (int)blockIdx.y;  // longest rows first
    const int w0 = blk * 128 + 32 * wave, q = w0 + (lane & 31);
    const float c2 = scale * 1.4426950408889634f;
    const size_t hb = (size_t)bh * S * D;
    const size_t wr = hb + (size_t)min(q, S - 1) * D + 8 * h;
    bf16x8_t qres[C::RES ? KS : 1][NP];
    if constexpr (C::RES) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int p = 0; p < NP; ++p) qres[ks][p] = ld_frag16(in.t[0][p] + wr + 16 * ks);
    }
    f32x16_t aO[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) zero16(aO[t]);
    float m = -INFINITY, l = 0.f;

    const int tend = causal ? min(S, blk * 128 + 128) : S;
    const int Tn = (tend + 31) / 32;
    GenStage<D, NP> stg;
    const GenSrc src{in.t[1][0], in.t[1][NP - 1], in.t[2][0], in.t[2][NP - 1], kb, nullptr, LSE,
                     (size_t)bb * Spad, hb};
    gen_load<D, NP>(stg, src, 0, S, tid);
    gen_store<D, NP>(stg, smem, tid);
    for (int it = 0; it < Tn; ++it) {
        __syncthreads();
        gen_load<D, NP>(stg, src, 32 * min(it + 1, Tn - 1), S, tid);
        const int k0 = 32 * it;
        const unsigned char* sb = smem + (it & 1) * C::STAGE;
        const bf16_t* tK[NP];
        const bf16_t* tV[NP];
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            tK[p] = reinterpret_cast<const bf16_t*>(sb) + (size_t)p * 32 * C::P;
            tV[p] = reinterpret_cast<const bf16_t*>(sb) + (size_t)(NP + p) * 32 * C::P;
        }
        const float* sbias = reinterpret_cast<const float*>(sb + C::TILE);
        if (!(w0 >= S || (causal && k0 > w0 + 31))) {
            const bool full = k0 + 31 < S && w0 + 31 < S && (!causal || k0 + 31 <= w0);
            f32x16_t s;
            zero16(s);
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                bf16x8_t a[NP], b[NP];
#pragma unroll
                for (int p = 0; p < NP; ++p) {
                    a[p] = ld_frag16(tK[p] + (lane & 31) * C::P + 16 * ks + 8 * h);
                    if constexpr (C::RES) b[p] = qres[ks][p];
                    else b[p] = ld_frag16(in.t[0][p] + wr + 16 * ks);
                }
                s = mma_np<NP>(a, b, s);
            }
            // element r: key k0 + 8(r/4) + 4h + r%4, query q (scores in base-2 units)
            float x[16], mt = -INFINITY;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int kr = 8 * (r >> 2) + 4 * h + (r & 3);
                float v = s[r] * c2 + (kb ? sbias[kr] : 0.f);
                if (!full) {
                    const int k = k0 + kr;
                    v = (q < S && k < S && (!causal || k <= q)) ? v : -INFINITY;
                }
                x[r] = v;
                mt = fmaxf(mt, v);
            }
            mt = fmaxf(mt, __shfl_xor(mt, 32));
            const float mn = fmaxf(m, mt);
            const float ms = mn == -INFINITY ? 0.f : mn;  // no visible key yet: the row stays empty
            const float alpha = __builtin_amdgcn_exp2f(m - ms);
            float ps = 0.f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                x[r] = __builtin_amdgcn_exp2f(x[r] - ms);
                ps += x[r];
            }
            ps += __shfl_xor(ps, 32);
            l = l * alpha + ps;
            m = mn;
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) aO[t][r] *= alpha;
            bf16x8_t pb[2][NP];
            split8<NP>(x, pb[0]);
            split8<NP>(x + 8, pb[1]);
#pragma unroll
            for (int p = 0; p < 2; ++p)
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    bf16x8_t va[NP];
#pragma unroll
                    for (int u = 0; u < NP; ++u) {
                        const int lan = lane & 15;
                        const int col = 32 * t + 16 * ((lane >> 4) & 1) + 4 * (lan & 3);
                        const int r0 = 16 * p + 4 * h + (lan >> 2);
                        va[u] = ld_tr_pair(tV[u] + r0 * C::P + col, tV[u] + (r0 + 8) * C::P + col);
                    }
                    aO[t] = mma_np<NP>(va, pb[p], aO[t]);
                }
        }
        gen_store<D, NP>(stg, smem + ((it + 1) & 1) * C::STAGE, tid);
    }
    // O^T accumulators: lane = query, element r of tile t: d = 32t + 8(r/4) + 4h + r%4
    if (q < S) {
        const float inv = l > 0.f ? 1.0f / l : 0.f;
        T* orow = O + hb + (size_t)q * D;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = 32 * t + 8 * g + 4 * h;
#pragma unroll
                for (int e = 0; e < 4; ++e) io<T>::st(orow, d + e, aO[t][4 * g + e] * inv);
            }
        if (h == 0) LSE[(size_t)bh * S + q] = l > 0.f ? (m + __log2f(l)) * 0.6931471805599453f : -INFINITY;
    }
}

// Generic path pre-pass: NP bf16 pieces of one [B*H*S, D] tensor (rotated when `mode` is
// set), one thread per element pair.
template <typename T, int NP>
__global__ __launch_bounds__(256) void gen_split(const T* __restrict__ X, bf16_t* __restrict__ y0,
                                                 bf16_t* __restrict__ y1, int64_t rows, int S,
                                                 int D, int mode, float theta) {
    const int half = D / 2;
    for (int64_t idx = blockIdx.x * (int64_t)256 + threadIdx.x; idx < rows * half;
         idx += (int64_t)gridDim.x * 256) {
        const int64_t row = idx / half;
        const int i = (int)(idx % half);
        int e0 = 2 * i, e1 = 2 * i + 1;
        if (mode != GN_ROPE_NONE) rope_pair(mode, i, D, e0, e1);
        float x0 = io<T>::ld(X, row * D + e0), x1 = io<T>::ld(X, row * D + e1);
        if (mode != GN_ROPE_NONE) {
            float c, sn;
            rope_cs((int)(row % S), i, D, theta, c, sn);
            const float r0 = x0 * c - x1 * sn, r1 = x0 * sn + x1 * c;
            x0 = r0;
            x1 = r1;
        }
        const bf16_t h0 = f2bf(x0), h1 = f2bf(x1);
        y0[row * D + e0] = h0;
        y0[row * D + e1] = h1;
        if (NP == 2) {
            y1[row * D + e0] = f2bf(x0 - bf2f(h0));
            y1[row * D + e1] = f2bf(x1 - bf2f(h1));
        }
    }
}

// Generic path row data: D_i = rowsum(dO O) (fp32) and L log2(e) (+inf for a row with no
// visible kept key) into [B*H][Spad], padding zero.  One wave per row.
template <typename T>
__global__ __launch_bounds__(256) void gen_rows(const T* __restrict__ dO, const T* __restrict__ O,
                                                const float* __restrict__ LSE, float* __restrict__ L2,
                                                float* __restrict__ Di, int64_t BH, int S, int Spad,
                                                int D) {
    const int64_t r = blockIdx.x * (int64_t)4 + (threadIdx.x >> 6);  // padded row index
    const int lane = threadIdx.x & 63;
    if (r >= BH * Spad) return;
    const int64_t bh = r / Spad;
    const int pos = (int)(r % Spad);
    float dot = 0.f;
    if (pos < S) {
        const size_t off = ((size_t)bh * S + pos) * D;
        for (int d = lane; d < D; d += 64) dot += io<T>::ld(dO, off + d) * io<T>::ld(O, off + d);
    }
    dot = wave_sum(dot);
    if (lane == 0) {
        const float lse = pos < S ? LSE[(size_t)bh * S + pos] : 0.f;
        Di[r] = dot;
        L2[r] = pos >= S ? 0.f : lse == -INFINITY ? INFINITY : lse * 1.4426950408889634f;
    }
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

// key-padding bias in natural-log units (kb holds base-2 units; -inf stays -inf)
__device__ __forceinline__ float kbias_nat(const float* kbb, int j) {
    return kbb ? kbb[j] * 0.6931471805599453f : 0.f;
}

template <typename T>
__global__ __launch_bounds__(256) void attn_fwd_simt(const T* __restrict__ Qr,
                                                     const T* __restrict__ Kr,
                                                     const T* __restrict__ V, T* __restrict__ O,
                                                     float* __restrict__ LSE,
                                                     const float* __restrict__ kb, int H,
                                                     int64_t BH, int S, int Spad, int D,
                                                     float scale, int causal) {
    const int64_t row = blockIdx.x * (int64_t)4 + (threadIdx.x >> 6);
    if (row >= BH * S) return;
    const int64_t bh = row / S;
    const int i = (int)(row % S);
    const size_t base = (size_t)bh * S * D;
    const float* kbb = kb ? kb + (size_t)(bh / H) * Spad : nullptr;
    float q[4], o[4] = {0.f, 0.f, 0.f, 0.f};
    ld_row(Qr + base + (size_t)i * D, D, q);
    float m = -INFINITY, l = 0.f;
    const int jn = causal ? i + 1 : S;
    for (int j = 0; j < jn; ++j) {
        float k[4], v[4];
        ld_row(Kr + base + (size_t)j * D, D, k);
        ld_row(V + base + (size_t)j * D, D, v);
        const float s = dot4(q, k) * scale + kbias_nat(kbb, j);
        if (s == -INFINITY) continue;  // a masked key (uniform across the wave)
        const float mn = fmaxf(m, s);
        const float a = __expf(m - mn), p = __expf(s - mn);
        l = l * a + p;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = o[e] * a + p * v[e];
        m = mn;
    }
    const int lane = threadIdx.x & 63;
    const float inv = l > 0.f ? 1.0f / l : 0.f;  // no visible kept key: O = 0, LSE = -inf
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int d = lane + 64 * e;
        if (d < D) io<T>::st(O, base + (size_t)i * D + d, o[e] * inv);
    }
    if (lane == 0) LSE[row] = l > 0.f ? m + __logf(l) : -INFINITY;
}

// LSE of a row with no visible kept key is -inf: +inf here makes its P (and dS) 0
__device__ __forceinline__ float lse_eff(float lse) { return lse == -INFINITY ? INFINITY : lse; }

template <typename T>
__global__ __launch_bounds__(256) void attn_bwd_dq_simt(
    const T* __restrict__ Qr, const T* __restrict__ Kr, const T* __restrict__ V,
    const T* __restrict__ dO, const float* __restrict__ LSE, const float* __restrict__ Di,
    const float* __restrict__ kb, float* __restrict__ dQacc, int H, int64_t BH, int S,
    int Spad, int D, float scale, int causal) {
    const int64_t row = blockIdx.x * (int64_t)4 + (threadIdx.x >> 6);
    if (row >= BH * S) return;
    const int64_t bh = row / S;
    const int i = (int)(row % S);
    const size_t base = (size_t)bh * S * D;
    const float* kbb = kb ? kb + (size_t)(bh / H) * Spad : nullptr;
    float q[4], g[4], acc[4] = {0.f, 0.f, 0.f, 0.f};
    ld_row(Qr + base + (size_t)i * D, D, q);
    ld_row(dO + base + (size_t)i * D, D, g);
    const float lse = lse_eff(LSE[row]), di = Di[row];
    const int jn = causal ? i + 1 : S;
    for (int j = 0; j < jn; ++j) {
        float k[4], v[4];
        ld_row(Kr + base + (size_t)j * D, D, k);
        ld_row(V + base + (size_t)j * D, D, v);
        const float p = __expf(dot4(q, k) * scale + kbias_nat(kbb, j) - lse);
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
    const float* __restrict__ kb, float* __restrict__ dKacc, T* __restrict__ dV, int H,
    int64_t BH, int S, int Spad, int D, float scale, int causal) {
    const int64_t row = blockIdx.x * (int64_t)4 + (threadIdx.x >> 6);
    if (row >= BH * S) return;
    const int64_t bh = row / S;
    const int j = (int)(row % S);
    const size_t base = (size_t)bh * S * D;
    const float kbj = kb ? kbias_nat(kb + (size_t)(bh / H) * Spad, j) : 0.f;
    float k[4], v[4], ak[4] = {0.f, 0.f, 0.f, 0.f}, av[4] = {0.f, 0.f, 0.f, 0.f};
    ld_row(Kr + base + (size_t)j * D, D, k);
    ld_row(V + base + (size_t)j * D, D, v);
    for (int i = causal ? j : 0; i < S; ++i) {
        float q[4], g[4];
        ld_row(Qr + base + (size_t)i * D, D, q);
        ld_row(dO + base + (size_t)i * D, D, g);
        const float p = __expf(dot4(q, k) * scale + kbj - lse_eff(LSE[bh * S + i]));
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
    bf16_t* plane[4][2];  // generic path: [Q, K, V, dO][piece] bf16 [B*H][S][D]
    float* L2;            // generic path: L log2(e) [B*H][Spad]
    float* accB;          // generic path: fp32 dK (dQ after it) and dV rows
    float* accA;
    float* Di;
    float* Lsc;   // MFMA path: L log2(e), [B*H][Spad]
    float2* cs;   // MFMA path: RoPE cos/sin table [S][D/2]
    float* acc;   // SIMT path: fp32 [B*H*S*D]
    float* kb;    // key-padding bias (base 2) [B][Spad] (sized for B*H rows)
    int* kt;      // per 64-key tile: any key biased [B][Spad/64]
};



inline size_t align_up(size_t x) { return (x + 255) & ~(size_t)255; }
inline int spad_of(int S) { return (S + 63) / 64 * 64; }

// mfma: bf16 Qr, Kr; Di, Lsc padded to Spad per (b, h); cos/sin table.
// simt: esz-sized Qr, Kr; Di; fp32 accumulator.
enum WsKind { kWsSimt = 0, kWsMfma = 1, kWsGen1 = 2, kWsGen2 = 3 };  // Gen: NP = 1, 2

size_t ws_layout(int64_t BH, int S, int D, size_t esz, int kind, void* base, AttnWs* w) {
    size_t off = 0;
    auto take = [&](size_t bytes) {
        void* p = base ? (char*)base + off : nullptr;
        off += align_up(bytes);
        return p;
    };
    const int64_t BHSD = BH * S * D;
    AttnWs t{};
    if (kind == kWsGen1 || kind == kWsGen2) {
        const int np = kind == kWsGen2 ? 2 : 1;
        for (int i = 0; i < 4; ++i)
            for (int p = 0; p < np; ++p) t.plane[i][p] = (bf16_t*)take(BHSD * 2);
        t.L2 = (float*)take(BH * spad_of(S) * 4);
        t.Di = (float*)take(BH * spad_of(S) * 4);
        t.accA = (float*)take(BHSD * 4);
        t.accB = (float*)take(BHSD * 4);
        t.kb = (float*)take(BH * spad_of(S) * 4);
        t.kt = (int*)take(BH * (spad_of(S) / 64) * 4);
        if (w) *w = t;
        return off;
    }
    const bool mfma = kind == kWsMfma;
    t.Qr = take(BHSD * esz);
    t.Kr = take(BHSD * esz);
    if (mfma) {
        t.Di = (float*)take(BH * spad_of(S) * 4);
        t.Lsc = (float*)take(BH * spad_of(S) * 4);
        t.cs = (float2*)take((size_t)S * (D / 2) * 8);
    } else {
        t.Di = (float*)take(BH * S * 4);
        t.acc = (float*)take(BHSD * 4);
    }
    t.kb = (float*)take(BH * spad_of(S) * 4);
    t.kt = (int*)take(BH * (spad_of(S) / 64) * 4);
    if (w) *w = t;
    return off;
}

// key bias and tile flags from a [B][S] mask (nothing without one); returns the kb / kt
// pointers the kernels take (null: no mask)
void key_bias(const float* mask, const AttnWs& w, int B, int S, hipStream_t s, const float** kb,
              const int** kt) {
    *kb = nullptr;
    *kt = nullptr;
    if (!mask) return;
    const int tiles = B * (spad_of(S) / 64);
    attn_key_bias<<<(tiles + 3) / 4, 256, 0, s>>>(mask, w.kb, w.kt, B, S, spad_of(S));
    *kb = w.kb;
    *kt = w.kt;
}

template <typename F>
bool allow_lds(F* fn, size_t bytes) {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) == hipSuccess;
}

constexpr int kStagesDkdv = 2, kStagesDq = 2;
// dK/dV waves per block: eight (two per SIMD, one block per CU) at D = 128, where the block's
// 128 K and V rows and two stages fill the LDS; four at D = 64 (65 KB of LDS, 207 registers),
// so two blocks share a CU and each wave keeps its K and V fragments in registers
template <int D> constexpr int dkdv_waves() { return D == 64 ? 4 : 8; }

// The eight tensors of one backward call (Q, K: un-rotated inputs).
struct AttnIO {
    TDesc Q, K, V, O, dO, dQ, dK, dV;
};

inline TDesc bhsd(const void* p, int H, int S, int D) {
    return TDesc{p, (int64_t)H * S * D, (int64_t)S * D, (int64_t)D};
}
inline TDesc bshd(const void* p, int S, int D, int64_t ld) {
    return TDesc{p, (int64_t)S * ld, (int64_t)D, ld};
}

template <int D>
int launch_mfma_bwd(const AttnWs& w, const AttnIO& io, const float* LSE, const float* mask,
                    int BH, int H, int S, float scale, int causal, int rope_mode, float theta,
                    hipStream_t s) {
    constexpr int NWK = dkdv_waves<D>();
    using C1 = DkdvCfg<D, kStagesDkdv, NWK>;
    using C2 = DqCfg<D, kStagesDq>;
    static const bool ok1 = allow_lds(attn_dkdv_mfma<D, kStagesDkdv, NWK, false>, C1::LDS) &&
                            allow_lds(attn_dkdv_mfma<D, kStagesDkdv, NWK, true>, C1::LDS);
    static const bool ok2 = allow_lds(attn_dq_mfma<D, kStagesDq>, C2::LDS);
    if (!ok1 || !ok2) {
        set_error("gn_attn_bwd: cannot reserve LDS (%d / %d B)", C1::LDS, C2::LDS);
        return GN_E_HIP;
    }
    const int64_t rows = (int64_t)BH * S;
    const int Spad = spad_of(S);
    if (rows * (D / 8) >= ((int64_t)1 << 31)) {
        set_error("gn_attn_bwd: B*H*S = %lld rows exceeds the bf16 path's 32-bit indexing", (long long)rows);
        return GN_E_INVALID;
    }
    if (rope_mode != GN_ROPE_NONE)
        rope_table<<<grid_for((int64_t)S * (D / 2), 256, 4096), 256, 0, s>>>(w.cs, S, D, theta);
    const float* kb;
    const int* kt;
    key_bias(mask, w, BH / H, S, s, &kb, &kt);
    const int64_t threads = rows * (D / 8);
    attn_prep<D><<<(unsigned)((threads + 255) / 256), 256, 0, s>>>(
        io.Q, io.K, io.dO, io.O, LSE, (bf16_t*)w.Qr, (bf16_t*)w.Kr, w.Lsc, w.Di, w.cs, rows, H, S,
        Spad, rope_mode);
    // rotated copies when RoPE is on, else the inputs in their own layout
    const TDesc tQ = rope_mode != GN_ROPE_NONE ? bhsd(w.Qr, H, S, D) : io.Q;
    const TDesc tK = rope_mode != GN_ROPE_NONE ? bhsd(w.Kr, H, S, D) : io.K;
    const int nb = (S + 127) / 128;
    auto dkdv = kb ? attn_dkdv_mfma<D, kStagesDkdv, NWK, true>
                   : attn_dkdv_mfma<D, kStagesDkdv, NWK, false>;
    // dQ does not depend on dK/dV: under graph capture at D = 64 it runs beside it on the
    // device's side stream (a dK/dV and a dQ block fit one CU together, 65 + 35 KB of LDS, so
    // dQ blocks fill the CUs dK/dV's last round leaves idle; C5 replayed 7.95 -> 7.88 ms).
    // Eagerly the fork's host cost outweighs it (C5 8.27 -> 8.33 ms), and at D = 128 the
    // blocks do not share a CU (C3 eager 0.365 -> 0.374 ms), so both run in issue order.
    SideBySide sb(s, D == 64 ? Fork::kCaptured : Fork::kNever);
    hipLaunchKernelGGL(dkdv, dim3(BH, nb), dim3(64 * NWK), C1::LDS, s, tQ, tK, io.V,
                       io.dO, w.Lsc, w.Di, w.cs, kb, kt, io.dK, io.dV, H, S, Spad, scale, causal,
                       rope_mode);
    hipLaunchKernelGGL((attn_dq_mfma<D, kStagesDq>), dim3(BH, nb), dim3(256), C2::LDS, sb.side(),
                       tQ, tK, io.V, io.dO, w.Lsc, w.Di, w.cs, kb, kt, io.dQ, H, S, Spad, scale,
                       causal, rope_mode);
    GN_LAUNCH_CHECK("gn_attn_bwd (mfma)");
    return sb.join();
}

// head dims of the generic MFMA path (multiples of 32 whose dK/dV column groups of <= 128
// divide D)
inline bool gen_dim(int D) { return D == 32 || D == 64 || D == 96 || D == 128 || D == 192 || D == 256; }

template <typename F>
bool allow_gen_lds(F* fn, size_t bytes) {
    return bytes <= 64 * 1024 || allow_lds(fn, bytes);
}

template <typename T, int D, int NP>
int launch_gen_bwd(const AttnWs& w, const void* Q, const void* K, const void* V, const void* O,
                   const void* dO, const float* LSE, const float* mask, void* dQ, void* dK,
                   void* dV, int B, int H, int S, float scale, int causal, int rope_mode,
                   float theta, hipStream_t s) {
    using C = GenCfg<D, NP>;
    constexpr int DC = D > 128 ? D / 2 : D;
    static const bool ok0 = allow_gen_lds(attn_bwd_gen<0, D, NP, DC>, C::LDS);
    static const bool ok1 = allow_gen_lds(attn_bwd_gen<1, D, NP, D>, C::LDS);
    if (!ok0 || !ok1) {
        set_error("gn_attn_bwd: cannot reserve %d B of LDS (generic path)", C::LDS);
        return GN_E_HIP;
    }
    const int64_t BH = (int64_t)B * H, rows = BH * S;
    const int Spad = spad_of(S);
    const float* kb;
    const int* kt;
    key_bias(mask, w, B, S, s, &kb, &kt);
    GenIn in{};
    const void* src[4] = {Q, K, V, dO};
    gen_planes<T, NP>(w, src, 4, in, rows, S, D, rope_mode, theta, s);
    gen_rows<T><<<(unsigned)((BH * Spad + 3) / 4), 256, 0, s>>>((const T*)dO, (const T*)O, LSE, w.L2,
                                                                 w.Di, BH, S, Spad, D);
    const unsigned nb = (unsigned)((S + 127) / 128);
    hipLaunchKernelGGL((attn_bwd_gen<0, D, NP, DC>), dim3((unsigned)BH, nb, D / DC), dim3(256), C::LDS,
                       s, in, w.L2, w.Di, kb, w.accA, w.accB, H, S, Spad, scale, causal);
    const unsigned ge = grid_for(rows * (D / 2), 256, 16384);
    unrotate_store<T><<<ge, 256, 0, s>>>(w.accB, (T*)dK, rows, S, D, rope_mode, theta);
    unrotate_store<T><<<ge, 256, 0, s>>>(w.accA, (T*)dV, rows, S, D, GN_ROPE_NONE, theta);
    hipLaunchKernelGGL((attn_bwd_gen<1, D, NP, D>), dim3((unsigned)BH, nb, 1), dim3(256), C::LDS, s,
                       in, w.L2, w.Di, kb, nullptr, w.accB, H, S, Spad, scale, causal);
    unrotate_store<T><<<ge, 256, 0, s>>>(w.accB, (T*)dQ, rows, S, D, rope_mode, theta);
    GN_LAUNCH_CHECK("gn_attn_bwd (generic mfma)");
    return GN_OK;
}

// operand planes of the generic path: rotated Q, K; V, dO as they are (bf16 inputs without
// rotation are used in place).  n = 3 for the forward (Q, K, V), 4 for the backward.
template <typename T, int NP>
void gen_planes(const AttnWs& w, const void* const* src, int n, GenIn& in, int64_t rows, int S,
                int D, int rope_mode, float theta, hipStream_t s) {
    const unsigned g = grid_for(rows * (D / 2), 256, 16384);
    for (int i = 0; i < n; ++i) {
        const int mode = i < 2 ? rope_mode : GN_ROPE_NONE;
        if (NP == 1 && mode == GN_ROPE_NONE) {
            in.t[i][0] = in.t[i][1] = (const bf16_t*)src[i];
            continue;
        }
        gen_split<T, NP><<<g, 256, 0, s>>>((const T*)src[i], w.plane[i][0], w.plane[i][NP - 1], rows,
                                           S, D, mode, theta);
        for (int p = 0; p < 2; ++p) in.t[i][p] = w.plane[i][p < NP ? p : 0];
    }
}

template <typename T, int D, int NP>
int launch_gen_fwd(const AttnWs& w, const void* Q, const void* K, const void* V, const float* kb,
                   void* O, float* LSE, int B, int H, int S, float scale, int causal,
                   int rope_mode, float theta, hipStream_t s) {
    using C = GenCfg<D, NP>;
    static const bool ok = allow_gen_lds(attn_fwd_gen<T, D, NP>, C::LDS);
    if (!ok) {
        set_error("gn_attn_fwd: cannot reserve %d B of LDS (generic path)", C::LDS);
        return GN_E_HIP;
    }
    const int64_t BH = (int64_t)B * H;
    GenIn in{};
    const void* src[3] = {Q, K, V};
    gen_planes<T, NP>(w, src, 3, in, BH * S, S, D, rope_mode, theta, s);
    hipLaunchKernelGGL((attn_fwd_gen<T, D, NP>), dim3((unsigned)BH, (unsigned)((S + 127) / 128)),
                       dim3(256), C::LDS, s, in, kb, (T*)O, LSE, H, S, spad_of(S), scale, causal);
    GN_LAUNCH_CHECK("gn_attn_fwd (generic mfma)");
    return GN_OK;
}

template <typename T, int NP>
int gen_fwd_dispatch(const AttnWs& w, const void* Q, const void* K, const void* V, const float* kb,
                     void* O, float* LSE, int B, int H, int S, int D, float scale, int causal,
                     int rope_mode, float theta, hipStream_t s) {
    switch (D) {
        case 32: return launch_gen_fwd<T, 32, NP>(w, Q, K, V, kb, O, LSE, B, H, S, scale, causal, rope_mode, theta, s);
        case 64: return launch_gen_fwd<T, 64, NP>(w, Q, K, V, kb, O, LSE, B, H, S, scale, causal, rope_mode, theta, s);
        case 96: return launch_gen_fwd<T, 96, NP>(w, Q, K, V, kb, O, LSE, B, H, S, scale, causal, rope_mode, theta, s);
        case 128: return launch_gen_fwd<T, 128, NP>(w, Q, K, V, kb, O, LSE, B, H, S, scale, causal, rope_mode, theta, s);
        case 192: return launch_gen_fwd<T, 192, NP>(w, Q, K, V, kb, O, LSE, B, H, S, scale, causal, rope_mode, theta, s);
        case 256: return launch_gen_fwd<T, 256, NP>(w, Q, K, V, kb, O, LSE, B, H, S, scale, causal, rope_mode, theta, s);
    }
    set_error("gn_attn_fwd: generic path has no D=%d", D);
    return GN_E_INVALID;
}

template <typename T, int NP>
int gen_bwd_dispatch(const AttnWs& w, const void* Q, const void* K, const void* V, const void* O,
                     const void* dO, const float* LSE, const float* mask, void* dQ, void* dK,
                     void* dV, int B, int H, int S, int D, float scale, int causal, int rope_mode,
                     float theta, hipStream_t s) {
#define GN_GEN(DV)                                                                              \
    case DV:                                                                                    \
        return launch_gen_bwd<T, DV, NP>(w, Q, K, V, O, dO, LSE, mask, dQ, dK, dV, B, H, S, scale, \
                                         causal, rope_mode, theta, s);
    switch (D) {
        GN_GEN(32)
        GN_GEN(96)
        GN_GEN(192)
        GN_GEN(256)
        GN_GEN(64)
        GN_GEN(128)
    }
#undef GN_GEN
    set_error("gn_attn_bwd: generic path has no D=%d", D);
    return GN_E_INVALID;
}

template <typename T>
int attn_bwd_impl(const void* Q, const void* K, const void* V, const void* O, const void* dO,
                  const float* LSE, const float* mask, void* dQ, void* dK, void* dV, int B, int H,
                  int S, int D, float scale, int causal, int rope_mode, float theta, void* ws,
                  size_t ws_bytes, hipStream_t s) {
    const int64_t BH = (int64_t)B * H, rows = BH * S, BHSD = rows * D;
    // the MFMA kernels move 16-byte chunks (LDS DMA, vector stores) from and to every tensor
    // and the workspace: an offset view takes the SIMT kernels instead
    const void* ptrs[9] = {Q, K, V, O, dO, dQ, dK, dV, ws};
    bool al16 = true;
    for (const void* p : ptrs) al16 = al16 && ((reinterpret_cast<uintptr_t>(p) & 15u) == 0);
    const bool mfma_ok = sizeof(T) == 2 && (D == 64 || D == 128) && al16;
    // the generic matrix-core path for the other D and for fp32
    const bool gen_ok = !mfma_ok && gen_dim(D) && al16 && BH * S * (int64_t)D < ((int64_t)1 << 31);
    if (gen_ok) {
        AttnWs w;
        const int kind = sizeof(T) == 4 ? kWsGen2 : kWsGen1;
        const size_t need = ws_layout(BH, S, D, sizeof(T), kind, ws, &w);
        if (!ws || ws_bytes < need) {
            set_error("gn_attn_bwd: workspace %zu B < %zu B", ws_bytes, need);
            return GN_E_WORKSPACE;
        }
        if (sizeof(T) == 4)
            return gen_bwd_dispatch<T, 2>(w, Q, K, V, O, dO, LSE, mask, dQ, dK, dV, B, H, S, D, scale,
                                          causal, rope_mode, theta, s);
        return gen_bwd_dispatch<T, 1>(w, Q, K, V, O, dO, LSE, mask, dQ, dK, dV, B, H, S, D, scale,
                                      causal, rope_mode, theta, s);
    }
    AttnWs w;
    const size_t need = ws_layout(BH, S, D, sizeof(T), mfma_ok ? kWsMfma : kWsSimt, ws, &w);
    if (!ws || ws_bytes < need) {
        set_error("gn_attn_bwd: workspace %zu B < %zu B", ws_bytes, need);
        return GN_E_WORKSPACE;
    }
    if (mfma_ok) {
        const AttnIO io{bhsd(Q, H, S, D),  bhsd(K, H, S, D),  bhsd(V, H, S, D),  bhsd(O, H, S, D),
                        bhsd(dO, H, S, D), bhsd(dQ, H, S, D), bhsd(dK, H, S, D), bhsd(dV, H, S, D)};
        if (D == 64)
            return launch_mfma_bwd<64>(w, io, LSE, mask, (int)BH, H, S, scale, causal, rope_mode, theta, s);
        return launch_mfma_bwd<128>(w, io, LSE, mask, (int)BH, H, S, scale, causal, rope_mode, theta, s);
    }
    const float* kb;
    const int* kt;
    key_bias(mask, w, B, S, s, &kb, &kt);
    const int Spad = spad_of(S);
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
    const unsigned gr = (unsigned)((rows + 3) / 4);
    const unsigned ge = grid_for(rows * (D / 2), 256, 16384);
    attn_bwd_dq_simt<T><<<gr, 256, 0, s>>>((const T*)Qp, (const T*)Kp, (const T*)V, (const T*)dO,
                                           LSE, w.Di, kb, w.acc, H, BH, S, Spad, D, scale, causal);
    unrotate_store<T><<<ge, 256, 0, s>>>(w.acc, (T*)dQ, rows, S, D, rope_mode, theta);
    attn_bwd_dkdv_simt<T><<<gr, 256, 0, s>>>((const T*)Qp, (const T*)Kp, (const T*)V,
                                             (const T*)dO, LSE, w.Di, kb, w.acc, (T*)dV, H, BH, S,
                                             Spad, D, scale, causal);
    unrotate_store<T><<<ge, 256, 0, s>>>(w.acc, (T*)dK, rows, S, D, rope_mode, theta);
    GN_LAUNCH_CHECK("gn_attn_bwd (simt)");
    (void)BHSD;
    return GN_OK;
}

}  // namespace
}  // namespace gn

using namespace gn;

extern "C" size_t gn_attn_workspace_bytes_dtype(int B, int H, int S, int D, int dtype) {
    if (B <= 0 || H <= 0 || S <= 0 || D <= 0) return 0;
    const int64_t BH = (int64_t)B * H;
    const size_t esz = dtype == GN_BF16 ? 2 : 4;
    // the path a call takes depends on D, the dtype and the pointers' alignment (unaligned
    // views fall back to the SIMT kernels): the largest layout among the candidates
    size_t need = ws_layout(BH, S, D, esz, kWsSimt, nullptr, nullptr);
    size_t alt = 0;
    if (dtype == GN_BF16 && (D == 64 || D == 128)) alt = ws_layout(BH, S, D, 2, kWsMfma, nullptr, nullptr);
    else if (gen_dim(D)) alt = ws_layout(BH, S, D, esz, dtype == GN_BF16 ? kWsGen1 : kWsGen2, nullptr, nullptr);
    return need > alt ? need : alt;
}

extern "C" size_t gn_attn_workspace_bytes(int B, int H, int S, int D) {
    if (B <= 0 || H <= 0 || S <= 0 || D <= 0) return 0;
    // the larger of the two layouts, so one query covers every dtype and path
    return gn_attn_workspace_bytes_dtype(B, H, S, D, GN_F32) > gn_attn_workspace_bytes_dtype(B, H, S, D, GN_BF16)
               ? gn_attn_workspace_bytes_dtype(B, H, S, D, GN_F32)
               : gn_attn_workspace_bytes_dtype(B, H, S, D, GN_BF16);
}

static int attn_check(const void* Q, const void* K, const void* V, int B, int H, int S, int D,
                      int rope_mode, int dtype, float scale) {
    GN_REQUIRE(B >= 0 && H >= 0 && S >= 0 && D > 0, "attention: bad shape");
    GN_REQUIRE(scale > 0.f && scale < INFINITY, "attention: scale %g must be positive and finite", scale);
    GN_REQUIRE(Q && K && V, "attention: null pointer");
    GN_REQUIRE(D <= 256 && D % 2 == 0, "attention: D=%d must be even and <= 256", D);
    GN_REQUIRE(rope_mode >= GN_ROPE_NONE && rope_mode <= GN_ROPE_HALF, "attention: rope_mode %d", rope_mode);
    GN_REQUIRE(dtype == GN_F32 || dtype == GN_BF16, "attention: dtype %d", dtype);
    GN_REQUIRE((int64_t)B * H <= 65535, "attention: B*H exceeds grid.y limit");
    return GN_OK;
}

extern "C" int gn_attn_bwd_mask(const void* Q, const void* K, const void* V, const void* O,
                                const void* dO, const float* LSE, const float* key_mask, void* dQ,
                                void* dK, void* dV, int B, int H, int S, int D, float scale,
                                int causal, int rope_mode, float rope_theta, int dtype, void* ws,
                                size_t ws_bytes, void* stream) {
    clear_error();
    int rc = attn_check(Q, K, V, B, H, S, D, rope_mode, dtype, scale);
    if (rc) return rc;
    if ((int64_t)B * H * S == 0) return GN_OK;
    GN_REQUIRE(O && dO && LSE && dQ && dK && dV, "gn_attn_bwd: null pointer");
    hipStream_t s = as_stream(stream);
    if (dtype == GN_BF16)
        return attn_bwd_impl<bf16_t>(Q, K, V, O, dO, LSE, key_mask, dQ, dK, dV, B, H, S, D, scale,
                                     causal, rope_mode, rope_theta, ws, ws_bytes, s);
    return attn_bwd_impl<float>(Q, K, V, O, dO, LSE, key_mask, dQ, dK, dV, B, H, S, D, scale,
                                causal, rope_mode, rope_theta, ws, ws_bytes, s);
}

extern "C" int gn_attn_bwd(const void* Q, const void* K, const void* V, const void* O,
                           const void* dO, const float* LSE, void* dQ, void* dK, void* dV, int B,
                           int H, int S, int D, float scale, int causal, int rope_mode,
                           float rope_theta, int dtype, void* ws, size_t ws_bytes,
                           void* stream) {
    return gn_attn_bwd_mask(Q, K, V, O, dO, LSE, nullptr, dQ, dK, dV, B, H, S, D, scale, causal,
                            rope_mode, rope_theta, dtype, ws, ws_bytes, stream);
}

extern "C" int gn_attn_bwd_bshd_mask(const void* Q, const void* K, const void* V, const void* O,
                                     const void* dO, const float* LSE, const float* key_mask,
                                     void* dQ, void* dK, void* dV, int B, int H, int S, int D,
                                     int64_t ld_qkv, int64_t ld_o, int64_t ld_dqkv, float scale,
                                     int causal, int rope_mode, float rope_theta, int dtype,
                                     void* ws, size_t ws_bytes, void* stream) {
    clear_error();
    int rc = attn_check(Q, K, V, B, H, S, D, rope_mode, dtype, scale);
    if (rc) return rc;
    if ((int64_t)B * H * S == 0) return GN_OK;
    GN_REQUIRE(O && dO && LSE && dQ && dK && dV, "gn_attn_bwd_bshd: null pointer");
    GN_REQUIRE(dtype == GN_BF16 && (D == 64 || D == 128),
               "gn_attn_bwd_bshd: bf16 with D = 64 or 128 only (D=%d, dtype %d)", D, dtype);
    GN_REQUIRE(ld_qkv >= (int64_t)H * D && ld_o >= (int64_t)H * D && ld_dqkv >= (int64_t)H * D,
               "gn_attn_bwd_bshd: row strides must cover H*D = %d elements", H * D);
    GN_REQUIRE(ld_qkv % 8 == 0 && ld_o % 8 == 0 && ld_dqkv % 8 == 0,
               "gn_attn_bwd_bshd: row strides must be multiples of 8 elements");
    GN_REQUIRE(ld_qkv < (1 << 24) && ld_o < (1 << 24) && ld_dqkv < (1 << 24),
               "gn_attn_bwd_bshd: row strides must be below 2^24 elements");
    const void* ptrs[9] = {Q, K, V, O, dO, dQ, dK, dV, ws};
    for (const void* p : ptrs)
        GN_REQUIRE(((uintptr_t)p & 15u) == 0,
                   "gn_attn_bwd_bshd: pointers (and the workspace) must be 16-byte aligned");
    AttnWs w;
    const int64_t BH = (int64_t)B * H;
    const size_t need = ws_layout(BH, S, D, 2, kWsMfma, ws, &w);
    if (!ws || ws_bytes < need) {
        set_error("gn_attn_bwd_bshd: workspace %zu B < %zu B", ws_bytes, need);
        return GN_E_WORKSPACE;
    }
    const AttnIO io{bshd(Q, S, D, ld_qkv),  bshd(K, S, D, ld_qkv),  bshd(V, S, D, ld_qkv),
                    bshd(O, S, D, ld_o),    bshd(dO, S, D, ld_o),   bshd(dQ, S, D, ld_dqkv),
                    bshd(dK, S, D, ld_dqkv), bshd(dV, S, D, ld_dqkv)};
    hipStream_t s = as_stream(stream);
    if (D == 64)
        return launch_mfma_bwd<64>(w, io, LSE, key_mask, (int)BH, H, S, scale, causal, rope_mode,
                                   rope_theta, s);
    return launch_mfma_bwd<128>(w, io, LSE, key_mask, (int)BH, H, S, scale, causal, rope_mode,
                                rope_theta, s);
}

extern "C" int gn_attn_bwd_bshd(const void* Q, const void* K, const void* V, const void* O,
                                const void* dO, const float* LSE, void* dQ, void* dK, void* dV,
                                int B, int H, int S, int D, int64_t ld_qkv, int64_t ld_o,
                                int64_t ld_dqkv, float scale, int causal, int rope_mode,
                                float rope_theta, int dtype, void* ws, size_t ws_bytes,
                                void* stream) {
    return gn_attn_bwd_bshd_mask(Q, K, V, O, dO, LSE, nullptr, dQ, dK, dV, B, H, S, D, ld_qkv,
                                 ld_o, ld_dqkv, scale, causal, rope_mode, rope_theta, dtype, ws,
                                 ws_bytes, stream);
}

extern "C" int gn_attn_fwd_mask(const void* Q, const void* K, const void* V, const float* key_mask,
                                void* O, float* LSE, int B, int H, int S, int D, float scale,
                                int causal, int rope_mode, float rope_theta, int dtype, void* ws,
                                size_t ws_bytes, void* stream) {
    clear_error();
    int rc = attn_check(Q, K, V, B, H, S, D, rope_mode, dtype, scale);
    if (rc) return rc;
    const int64_t rows = (int64_t)B * H * S;
    if (rows == 0) return GN_OK;
    GN_REQUIRE(O && LSE, "gn_attn_fwd: null pointer");
    hipStream_t s = as_stream(stream);
    auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    const bool mfma = dtype == GN_BF16 && (D == 64 || D == 128) && al16(Q) && al16(K) && al16(V) &&
                      al16(O) && ((rope_mode == GN_ROPE_NONE && !key_mask) || al16(ws)) &&
                      (rope_mode == GN_ROPE_NONE || rows * (D / 8) < ((int64_t)1 << 31));
    const size_t esz = dtype == GN_BF16 ? 2 : 4;
    AttnWs w;
    // MFMA path: rotated bf16 Q, K, the cos/sin table (the backward's layout) and the key
    // bias; SIMT path: rotated Q, K and the key bias
    const size_t need = mfma ? ws_layout((int64_t)B * H, S, D, 2, kWsMfma, ws, &w)
                             : ws_layout((int64_t)B * H, S, D, esz, kWsSimt, ws, &w);
    if ((rope_mode != GN_ROPE_NONE || key_mask) && (!ws || ws_bytes < need)) {
        set_error("gn_attn_fwd: workspace %zu B < %zu B", ws_bytes, need);
        return GN_E_WORKSPACE;
    }
    // the generic matrix-core forward for the other D and fp32, when a workspace is given
    const bool gen = !mfma && gen_dim(D) && al16(Q) && al16(K) && al16(V) && al16(O) && al16(ws) &&
                     rows * D < ((int64_t)1 << 31) &&
                     ws_bytes >= ws_layout((int64_t)B * H, S, D, esz, dtype == GN_BF16 ? kWsGen1 : kWsGen2,
                                           nullptr, nullptr);
    if (gen) {
        ws_layout((int64_t)B * H, S, D, esz, dtype == GN_BF16 ? kWsGen1 : kWsGen2, ws, &w);
        const float* kbg;
        const int* ktg;
        key_bias(key_mask, w, B, S, s, &kbg, &ktg);
        if (dtype == GN_BF16)
            return gen_fwd_dispatch<bf16_t, 1>(w, Q, K, V, kbg, O, LSE, B, H, S, D, scale, causal,
                                               rope_mode, rope_theta, s);
        return gen_fwd_dispatch<float, 2>(w, Q, K, V, kbg, O, LSE, B, H, S, D, scale, causal,
                                          rope_mode, rope_theta, s);
    }
    const float* kb;
    const int* kt;
    key_bias(key_mask, w, B, S, s, &kb, &kt);
    const int Spad = spad_of(S);
    const void* Qp = Q;
    const void* Kp = K;
    if (rope_mode != GN_ROPE_NONE && mfma) {
        // one table pass (S * D/2 angles) and one rotation pass over Q and K together
        rope_table<<<grid_for((int64_t)S * (D / 2), 256, 4096), 256, 0, s>>>(w.cs, S, D, rope_theta);
        const unsigned g = (unsigned)((rows * (D / 8) + 255) / 256);
        if (D == 64)
            rope_qk_prep<64><<<g, 256, 0, s>>>(bhsd(Q, H, S, D), bhsd(K, H, S, D), (bf16_t*)w.Qr,
                                               (bf16_t*)w.Kr, w.cs, rows, H, S, rope_mode);
        else
            rope_qk_prep<128><<<g, 256, 0, s>>>(bhsd(Q, H, S, D), bhsd(K, H, S, D), (bf16_t*)w.Qr,
                                                (bf16_t*)w.Kr, w.cs, rows, H, S, rope_mode);
        Qp = w.Qr;
        Kp = w.Kr;
    } else if (rope_mode != GN_ROPE_NONE) {
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
    if (mfma) {
        const int BH = B * H;
        const TDesc tQ = bhsd(Qp, H, S, D), tK = bhsd(Kp, H, S, D), tV = bhsd(V, H, S, D),
                    tO = bhsd(O, H, S, D);
        const dim3 grid(BH, (S + 127) / 128);
        if (D == 64) {
            using C = DqCfg<64, kStagesDq>;
            static const bool ok = allow_lds(attn_fwd_mfma<64, kStagesDq>, C::LDS);
            GN_REQUIRE(ok, "gn_attn_fwd: cannot reserve %d B of LDS", C::LDS);
            hipLaunchKernelGGL((attn_fwd_mfma<64, kStagesDq>), grid, dim3(256), C::LDS, s, tQ, tK, tV, tO,
                               LSE, kb, kt, H, S, Spad, scale, causal);
        } else {
            using C = DqCfg<128, kStagesDq>;
            static const bool ok = allow_lds(attn_fwd_mfma<128, kStagesDq>, C::LDS);
            GN_REQUIRE(ok, "gn_attn_fwd: cannot reserve %d B of LDS", C::LDS);
            hipLaunchKernelGGL((attn_fwd_mfma<128, kStagesDq>), grid, dim3(256), C::LDS, s, tQ, tK, tV, tO,
                               LSE, kb, kt, H, S, Spad, scale, causal);
        }
        GN_LAUNCH_CHECK("gn_attn_fwd (mfma)");
        return GN_OK;
    }
    const unsigned gr = (unsigned)((rows + 3) / 4);
    if (dtype == GN_BF16)
        attn_fwd_simt<bf16_t><<<gr, 256, 0, s>>>((const bf16_t*)Qp, (const bf16_t*)Kp, (const bf16_t*)V,
                                                 (bf16_t*)O, LSE, kb, H, (int64_t)B * H, S, Spad, D,
                                                 scale, causal);
    else
        attn_fwd_simt<float><<<gr, 256, 0, s>>>((const float*)Qp, (const float*)Kp, (const float*)V,
                                                (float*)O, LSE, kb, H, (int64_t)B * H, S, Spad, D,
                                                scale, causal);
    GN_LAUNCH_CHECK("gn_attn_fwd");
    return GN_OK;
}

extern "C" int gn_attn_fwd(const void* Q, const void* K, const void* V, void* O, float* LSE,
                           int B, int H, int S, int D, float scale, int causal, int rope_mode,
                           float rope_theta, int dtype, void* ws, size_t ws_bytes, void* stream) {
    return gn_attn_fwd_mask(Q, K, V, nullptr, O, LSE, B, H, S, D, scale, causal, rope_mode,
                            rope_theta, dtype, ws, ws_bytes, stream);
}
