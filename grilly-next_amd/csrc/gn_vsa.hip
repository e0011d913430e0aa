// gn_vsa.hip — VSA unpack-project backward (vsa-unpack-project-backward.glsl:42-74):
//
//   dW[o, j] = sum_b dY[b, o] * s_b(j),   s_b(j) = bit (j & 31) of X[b, j >> 5] ? +1 : -1
//
// A bf16 MFMA contraction over the batch (M = O, N = D, K = Bn).  The +-1 operand is
// produced from the packed bits while staging the LDS tile (never materialised in HBM).
// +-1 is exact in bf16; fp32 dY keeps fp32 accuracy by splitting it into two bf16 terms
// dY = hi + lo (hi = bf16(dY), lo = bf16(dY - hi), residual ~2^-17 |dY|), both multiplied
// against the same +-1 fragment with fp32 accumulation.
//
// Tile 128 (o) x 128 (j) x 32 (b), 4 waves of 64 x 64 (2 x 2 v_mfma_f32_32x32x16_bf16).
#include "gn_common.h"
#include "gn_gemm_dma.h"

namespace gn {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int VBM = 128, VBN = 128, VBK = 32;
constexpr int VP = VBK + 8;  // LDS pitch in bf16 (80 bytes)
constexpr int VT = 128 * VP;

__device__ __forceinline__ bf16x8_t frag(const bf16_t* p) {
    uint4 v = *reinterpret_cast<const uint4*>(p);
    return __builtin_bit_cast(bf16x8_t, v);
}

// SPLIT = true: dY fp32, two-term bf16 split.  SPLIT = false: dY bf16.
template <bool SPLIT>
__global__ __launch_bounds__(256, 2) void vsa_dw_kernel(const void* __restrict__ dYv,
                                                        const uint32_t* __restrict__ bits,
                                                        float* __restrict__ dW, int Bn, int O,
                                                        int D, int words, int accumulate,
                                                        int vec_ok) {
    __shared__ __align__(16) bf16_t sAh[2][VT];
    __shared__ __align__(16) bf16_t sAl[SPLIT ? 2 : 1][SPLIT ? VT : 8];
    __shared__ __align__(16) bf16_t sB[2][VT];

    const int tilesN = (D + VBN - 1) / VBN;
    const int tm = blockIdx.x / tilesN, tn = blockIdx.x % tilesN;
    const int o0 = tm * VBM, j0 = tn * VBN;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    f32x16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // loader mapping: 16 column chunks of 8 (o for A, j for B) x 16 groups of 2 b-rows
    const int cc = t & 15, bg = t >> 4;
    float av[2][8];
    uint32_t bw[2];
    auto gload = [&](int kt) {
        const int b0 = kt * VBK + bg * 2;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int b = b0 + r;
            const int o = o0 + cc * 8;
            if (!vec_ok) {  // any O: scalar loads with per-element bounds
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const size_t idx = (size_t)b * O + o + e;
                    float v = 0.f;
                    if (b < Bn && o + e < O)
                        v = SPLIT ? reinterpret_cast<const float*>(dYv)[idx]
                                  : bf2f(reinterpret_cast<const bf16_t*>(dYv)[idx]);
                    av[r][e] = v;
                }
            } else if (SPLIT) {
                const float* p = reinterpret_cast<const float*>(dYv) + (size_t)b * O + o;
                if (b < Bn && o < O) {
                    float4 x = *reinterpret_cast<const float4*>(p);
                    float4 y = *reinterpret_cast<const float4*>(p + 4);
                    av[r][0] = x.x; av[r][1] = x.y; av[r][2] = x.z; av[r][3] = x.w;
                    av[r][4] = y.x; av[r][5] = y.y; av[r][6] = y.z; av[r][7] = y.w;
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) av[r][e] = 0.f;
                }
            } else {
                const bf16_t* p = reinterpret_cast<const bf16_t*>(dYv) + (size_t)b * O + o;
                if (b < Bn && o < O) {
                    uint4 x = *reinterpret_cast<const uint4*>(p);
                    uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        av[r][2 * e] = __uint_as_float(w[e] << 16);
                        av[r][2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) av[r][e] = 0.f;
                }
            }
            const int j = j0 + cc * 8;
            // rows past Bn contribute nothing: their A values are zero, any bits will do
            bw[r] = (b < Bn && j < D) ? bits[(size_t)b * words + (j >> 5)] : 0u;
        }
    };
    auto sstore = [&](int buf) {
        // A: column o = cc*8+e gets the b-pair (bg*2, bg*2+1) as one dword
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float x0 = av[0][e], x1 = av[1][e];
            const bf16_t h0 = f2bf(x0), h1 = f2bf(x1);
            *reinterpret_cast<uint32_t*>(&sAh[buf][(cc * 8 + e) * VP + bg * 2]) =
                (uint32_t)h0 | ((uint32_t)h1 << 16);
            if (SPLIT) {
                const float l0 = x0 - bf2f(h0), l1 = x1 - bf2f(h1);
                *reinterpret_cast<uint32_t*>(&sAl[buf][(cc * 8 + e) * VP + bg * 2]) = pack_bf2(l0, l1);
            }
        }
        // B: column j = cc*8+e gets (s_b0(j), s_b1(j)); bf16 +1 = 0x3F80, -1 = 0xBF80
        const int sh = (cc * 8) & 31;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t v0 = ((bw[0] >> (sh + e)) & 1u) ? 0x3F80u : 0xBF80u;
            const uint32_t v1 = ((bw[1] >> (sh + e)) & 1u) ? 0x3F80u : 0xBF80u;
            *reinterpret_cast<uint32_t*>(&sB[buf][(cc * 8 + e) * VP + bg * 2]) = v0 | (v1 << 16);
        }
    };

    const int KT = (Bn + VBK - 1) / VBK;
    if (KT > 0) {
        gload(0);
        sstore(0);
    }
    __syncthreads();
    const int frow = lane & 31, fk = (lane >> 5) * 8;
    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < KT) gload(kt + 1);
#pragma unroll
        for (int ks = 0; ks < VBK / 16; ++ks) {
            const int ka = ks * 16 + fk;
            bf16x8_t b0 = frag(&sB[cur][(wn * 64 + frow) * VP + ka]);
            bf16x8_t b1 = frag(&sB[cur][(wn * 64 + 32 + frow) * VP + ka]);
            bf16x8_t a0 = frag(&sAh[cur][(wm * 64 + frow) * VP + ka]);
            bf16x8_t a1 = frag(&sAh[cur][(wm * 64 + 32 + frow) * VP + ka]);
            acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0, acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b1, acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b0, acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b1, acc[1][1], 0, 0, 0);
            if (SPLIT) {
                bf16x8_t l0 = frag(&sAl[cur][(wm * 64 + frow) * VP + ka]);
                bf16x8_t l1 = frag(&sAl[cur][(wm * 64 + 32 + frow) * VP + ka]);
                acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(l0, b0, acc[0][0], 0, 0, 0);
                acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(l0, b1, acc[0][1], 0, 0, 0);
                acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(l1, b0, acc[1][0], 0, 0, 0);
                acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(l1, b1, acc[1][1], 0, 0, 0);
            }
        }
        if (kt + 1 < KT) sstore(cur ^ 1);
        __syncthreads();
    }

    const int col_l = lane & 31, rq = (lane >> 5) * 4;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = j0 + wn * 64 + j * 32 + col_l;
            if (n >= D) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = o0 + wm * 64 + i * 32 + 8 * (r >> 2) + rq + (r & 3);
                if (m >= O) continue;
                const size_t idx = (size_t)m * D + n;
                dW[idx] = accumulate ? dW[idx] + acc[i][j][r] : acc[i][j][r];
            }
        }
}

// dY [Bn x O] -> its transposed bf16 planes [O x Bn] for the MFMA path: hi = bf16(dY) and,
// for fp32 dY, lo = bf16(dY - hi) (the same two-term split vsa_dw_kernel forms in LDS).
// The transpose makes the batch (the contraction index) contiguous, so the dW kernel reads
// its dY fragments with plain 16-byte LDS reads.  64 x 64 tiles through LDS; Bn % 64 == 0.
template <typename T>
__global__ __launch_bounds__(256) void vsa_split_dy_t(const T* __restrict__ dY, bf16_t* __restrict__ hi,
                                                      bf16_t* __restrict__ lo, int Bn, int O) {
    __shared__ float tile[64][65];
    const int b0 = blockIdx.y * 64, o0 = blockIdx.x * 64, t = threadIdx.x;
    // load: 64 rows (b) x 64 columns (o), 16 threads per row, 4 consecutive o per thread
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = (t >> 4) + 16 * i, c = (t & 15) * 4;
        const int o = o0 + c;
        float v[4] = {0.f, 0.f, 0.f, 0.f};
        const size_t base = (size_t)(b0 + r) * O + o;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (o + e < O) {
                if constexpr (sizeof(T) == 4) v[e] = dY[base + e];
                else v[e] = bf2f(dY[base + e]);
            }
#pragma unroll
        for (int e = 0; e < 4; ++e) tile[r][c + e] = v[e];
    }
    __syncthreads();
    // store: row o of the transposed planes, 8 consecutive b (one 16-byte chunk) per thread
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int orow = (t >> 3) + 32 * i, c = (t & 7) * 8;
        const int o = o0 + orow;
        if (o >= O) continue;
        uint32_t h[4], l[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float x0 = tile[c + 2 * e][orow], x1 = tile[c + 2 * e + 1][orow];
            h[e] = pack_bf2(x0, x1);
            l[e] = pack_bf2(x0 - __uint_as_float(h[e] << 16), x1 - __uint_as_float(h[e] & 0xffff0000u));
        }
        const size_t dst = (size_t)o * Bn + b0 + c;
        *reinterpret_cast<uint4*>(hi + dst) = make_uint4(h[0], h[1], h[2], h[3]);
        if (sizeof(T) == 4) *reinterpret_cast<uint4*>(lo + dst) = make_uint4(l[0], l[1], l[2], l[3]);
    }
}

inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

}  // namespace

int colsum_dispatch(const void* in, float* out, int M, int N, int dtype, unsigned flags,
                    hipStream_t s, int ld, float* scratch = nullptr, size_t scratch_floats = 0);

}  // namespace gn

using namespace gn;

// Workspace of the MFMA-DMA path: the transposed bf16 planes of dY (hi and lo for fp32 dY,
// one plane for bf16).  Without it (or when the shape does not fit that path) the
// LDS-staging kernel runs instead.
extern "C" size_t gn_vsa_workspace_bytes(int Bn, int O) {
    if (Bn <= 0 || O <= 0) return 0;
    return 2 * align256((size_t)Bn * O * sizeof(bf16_t));
}

extern "C" int gn_vsa_unpack_project_bwd(const void* dY, const uint32_t* Xbits, float* dW,
                                         float* db, int Bn, int O, int D, int words, int dtype,
                                         unsigned flags, void* ws, size_t ws_bytes,
                                         void* stream) {
    clear_error();
    GN_REQUIRE(Bn >= 0 && O >= 0 && D >= 0, "gn_vsa_unpack_project_bwd: negative size");
    if (O == 0 || D == 0) return GN_OK;
    GN_REQUIRE(dY && Xbits && dW, "gn_vsa_unpack_project_bwd: null pointer");
    GN_REQUIRE(D % 32 == 0 && words >= D / 32,
               "gn_vsa_unpack_project_bwd: D=%d must be a multiple of 32 with words >= D/32", D);
    GN_REQUIRE(dtype == GN_F32 || dtype == GN_BF16, "gn_vsa_unpack_project_bwd: dtype %d", dtype);
    hipStream_t s = as_stream(stream);
    const int tiles = ((O + VBM - 1) / VBM) * ((D + VBN - 1) / VBN);
    const int acc = (flags & GN_ACCUMULATE) ? 1 : 0;
    // db first, with dW (overwritten next unless accumulating) as its scratch
    if (db) {
        const int rc = colsum_dispatch(dY, db, Bn, O, dtype, flags, s, O, acc ? nullptr : dW,
                                       (size_t)O * D);
        if (rc) return rc;
    }
    // MFMA-DMA path: dY as transposed bf16 planes (hi, and lo for fp32), bits expanded in
    // LDS once per block and k-tile
    {
        const size_t plane = align256((size_t)Bn * O * sizeof(bf16_t));
        VsaDesc v{};
        v.bits = Xbits;
        v.words = words;
        v.K = Bn; v.M = O; v.N = D;
        v.C = dW; v.ldc = D; v.lda = Bn;
        v.accumulate = acc;
        v.nseg = dtype == GN_F32 ? 2 : 1;
        v.A[0] = static_cast<const bf16_t*>(ws);
        v.A[1] = reinterpret_cast<const bf16_t*>(static_cast<const unsigned char*>(ws) + plane);
        const bool have = ws && ws_bytes >= (size_t)v.nseg * plane && al16(ws);
        if (have && Bn > 0 && vsa_dma_applicable(v)) {
            const dim3 grid((O + 63) / 64, Bn / 64);
            bf16_t* hi = const_cast<bf16_t*>(v.A[0]);
            bf16_t* lo = const_cast<bf16_t*>(v.A[1]);
            if (dtype == GN_F32)
                vsa_split_dy_t<float><<<grid, 256, 0, s>>>(static_cast<const float*>(dY), hi, lo, Bn, O);
            else
                vsa_split_dy_t<bf16_t><<<grid, 256, 0, s>>>(static_cast<const bf16_t*>(dY), hi, lo, Bn, O);
            GN_LAUNCH_CHECK("gn_vsa_unpack_project_bwd (transpose)");
            return vsa_dma_launch(v, s);
        }
    }
    const int vec_ok = (O % 8 == 0) && al16(dY);
    if (dtype == GN_F32)
        vsa_dw_kernel<true><<<tiles, 256, 0, s>>>(dY, Xbits, dW, Bn, O, D, words, acc, vec_ok);
    else
        vsa_dw_kernel<false><<<tiles, 256, 0, s>>>(dY, Xbits, dW, Bn, O, D, words, acc, vec_ok);
    GN_LAUNCH_CHECK("gn_vsa_unpack_project_bwd");
    return GN_OK;
}
