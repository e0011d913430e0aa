// gn_gemm_dma.h — descriptor of the LDS-DMA GEMM core (gn_gemm_dma.hip).
#pragma once

#include "gn_common.h"
#include "gn_math.h"

namespace gn {

struct GemmDesc {
    // transA = 0: A_s[m * lda + k];  transA = 1: A_s[k * lda + m]
    // transB = 0: B_s[k * ldb + n];  transB = 1: B_s[n * ldb + k]
    const bf16_t* A[2];
    int lda[2];
    const bf16_t* B[2];
    int ldb[2];
    int Ks[2];
    int nseg;
    int M, N;
    // plain epilogue (epi 0): rows < Msplit -> C, rows >= Msplit -> C2 (row m - Msplit)
    void* C;
    void* C2;
    int Msplit;
    int ldc;
    int accumulate;
    // GLU epilogue (epi 1): the GEMM result is dO of glu(gate, up); writes
    // gu[m * ldgu + n] = dGate, gu[m * ldgu + H + n] = dUp (bf16)
    int epi;
    const bf16_t* gate;
    const bf16_t* up;
    int ldg;
    bf16_t* gu;
    int ldgu;
    int H;
    int glu_kind;
    // split-K (plain fp32 epilogue only): blockIdx.y picks one of ksplit k-ranges and the
    // partial tiles are added into C with fp32 atomics after C is cleared; with two splits
    // the result is exactly a + b whichever lands first, so it stays deterministic
    int ksplit;
    // row sums of op(A) (the bias gradient of a weight-gradient GEMM, db = sum_rows dY when
    // A = dY^T): rows < Msplit -> bias[m], rows >= Msplit -> bias2[m - Msplit], fp32, added
    // to the existing values when accumulate; nullptr: none (plain fp32 epilogue only)
    float* bias;
    float* bias2;
    // column bias of the plain epilogue (a forward Linear's b): C[m][n] = acc + cbias[n],
    // bf16, LDS-DMA core only, no split-K; nullptr: none
    const bf16_t* cbias;
    // split-K through a workspace (plain fp32 epilogue, ksplit >= 3): split y stores its
    // partial tile at part + y*M*N (row-major, pitch N) and, with a bias, its row sums at
    // part + ksplit*M*N + y*M; split_reduce then adds the splits in index order into C and
    // the bias, so the result does not depend on which block finishes first.  part_cap: bytes
    // available at part (0: no workspace; splits of two then add into C with atomics)
    float* part;
    size_t part_cap;
};

// Store one accumulated element (m, n) according to the descriptor's epilogue.
template <typename CT, int EPI>
__device__ __forceinline__ void gemm_store(const GemmDesc& g, int m, int n, float v);

// VSA unpack-project weight gradient on the same core:
//   C[M x N] (+)= sum_s A_s S,   A_s bf16 [M x K] (the transposed hi / lo bf16 planes of dY,
//   k-contiguous), S[k][n] = bit n % 32 of bits[k * words + n / 32] ? +1 : -1 (expanded in LDS).
struct VsaDesc {
    const bf16_t* A[2];
    int nseg;       // 1 (bf16 dY) or 2 (fp32 dY as hi + lo)
    int lda;        // row pitch of A_s (>= K)
    const uint32_t* bits;
    int words;
    int K, M, N;    // K = rows (batch), M = out_dim, N = vsa_dim
    float* C;
    int ldc;
    int accumulate;
};
bool vsa_dma_applicable(const VsaDesc& v);
int vsa_dma_launch(const VsaDesc& v, hipStream_t s);

bool gemm_dma_applicable(const GemmDesc& g);
// Workspace bytes the launch of g would use for its split-K partials if part_cap were
// unbounded (0: none).
size_t gemm_dma_part_bytes(const GemmDesc& g, int transA, int c_dtype);
int gemm_dma_launch(const GemmDesc& g, int transA, int transB, int c_dtype, hipStream_t s);
// Its instantiation units (gn_gemm_dma_{f32a,f32b,bf16,glu}.hip): fp32 C with A k-contiguous /
// k-outer, bf16 C, and the GLU epilogue (untransposed operands only).
int gemm_dma_f32_ta0(const GemmDesc& g, int transB, hipStream_t s);
int gemm_dma_f32_ta1(const GemmDesc& g, int transB, hipStream_t s);
int gemm_dma_bf16(const GemmDesc& g, int transA, int transB, hipStream_t s);
int gemm_dma_glu(const GemmDesc& g, int transA, int transB, hipStream_t s);
// C (+)= sum over y < g.ksplit of the planes at g.part (index order); N % 4 == 0, C and ldc
// 16-byte aligned.
void launch_split_reduce(const GemmDesc& g, hipStream_t s);

// fp32 operands on the bf16 MFMA pipe through a six-product three-piece split (gn_gemm_f32.hip)
bool gemm_f32_applicable(const GemmDesc& g);
// workspace bytes the launch would use for split-K partial planes (0: none)
size_t gemm_f32_part_bytes(const GemmDesc& g);
int gemm_f32_launch(const GemmDesc& g, int transA, int transB, hipStream_t s);

template <typename CT, int EPI>
__device__ __forceinline__ void gemm_store(const GemmDesc& g, int m, int n, float v) {
    if constexpr (EPI == 0) {
        CT* C = reinterpret_cast<CT*>(m < g.Msplit ? g.C : g.C2);
        const size_t idx = (size_t)(m < g.Msplit ? m : m - g.Msplit) * g.ldc + n;
        io<CT>::st(C, idx, g.accumulate ? v + io<CT>::ld(C, idx) : v);
    } else {
        const size_t gi = (size_t)m * g.ldg + n;
        const float gt = bf2f(g.gate[gi]), up = bf2f(g.up[gi]);
        float dg, du;
        switch (g.glu_kind) {
            case GN_GLU_SWIGLU_UP: glu_grad<GN_GLU_SWIGLU_UP>(v, gt, up, dg, du); break;
            case GN_GLU_SWIGLU_GATE: glu_grad<GN_GLU_SWIGLU_GATE>(v, gt, up, dg, du); break;
            case GN_GLU_GEGLU_UP: glu_grad<GN_GLU_GEGLU_UP>(v, gt, up, dg, du); break;
            case GN_GLU_GEGLU_GATE: glu_grad<GN_GLU_GEGLU_GATE>(v, gt, up, dg, du); break;
            default: glu_grad<GN_GLU_REGLU_UP>(v, gt, up, dg, du); break;
        }
        g.gu[(size_t)m * g.ldgu + n] = f2bf(dg);
        g.gu[(size_t)m * g.ldgu + g.H + n] = f2bf(du);
    }
}

// Epilogue of one 32x32 MFMA accumulator tile (lane layout: col = lane%32, row =
// 8(r/4) + 4(lane/32) + r%4) at (m0, n0).  For the GLU epilogue all 32 gate/up loads of
// the tile are issued before any store, so their latencies overlap.
template <typename CT, int EPI, typename ACC>
__device__ __forceinline__ void gemm_store_tile(const GemmDesc& g, int m0, int n0, const ACC& a) {
    const int lane = threadIdx.x & 63;
    const int n = n0 + (lane & 31), rq = (lane >> 5) * 4;
    if (n >= g.N) return;
    if constexpr (EPI == 0) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = m0 + 8 * (r >> 2) + rq + (r & 3);
            if (m < g.M) gemm_store<CT, 0>(g, m, n, a[r]);
        }
    } else {
        const bf16_t* __restrict__ gp = g.gate;
        const bf16_t* __restrict__ upp = g.up;
        bf16_t* __restrict__ gu = g.gu;
        bf16_t gv[16], uv[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = min(m0 + 8 * (r >> 2) + rq + (r & 3), g.M - 1);
            gv[r] = gp[(size_t)m * g.ldg + n];
            uv[r] = upp[(size_t)m * g.ldg + n];
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = m0 + 8 * (r >> 2) + rq + (r & 3);
            if (m >= g.M) continue;
            float dg, du;
            const float v = a[r], gt = bf2f(gv[r]), up = bf2f(uv[r]);
            switch (g.glu_kind) {
                case GN_GLU_SWIGLU_UP: glu_grad<GN_GLU_SWIGLU_UP>(v, gt, up, dg, du); break;
                case GN_GLU_SWIGLU_GATE: glu_grad<GN_GLU_SWIGLU_GATE>(v, gt, up, dg, du); break;
                case GN_GLU_GEGLU_UP: glu_grad<GN_GLU_GEGLU_UP>(v, gt, up, dg, du); break;
                case GN_GLU_GEGLU_GATE: glu_grad<GN_GLU_GEGLU_GATE>(v, gt, up, dg, du); break;
                default: glu_grad<GN_GLU_REGLU_UP>(v, gt, up, dg, du); break;
            }
            gu[(size_t)m * g.ldgu + n] = f2bf(dg);
            gu[(size_t)m * g.ldgu + g.H + n] = f2bf(du);
        }
    }
}

// fp32 Linear on a handful of rows (M <= 8; gn_skinny.hip): HBM-bound passes over W.
bool skinny_fwd_applicable(const void* X, const void* W, const void* Y, int M, int K);
bool skinny_bwd_applicable(const void* dY, const void* X, const void* W, const void* dX,
                           const void* dW, int M, int K);
size_t skinny_bwd_ws_bytes(int M, int N, int K);
int skinny_linear_fwd(const float* X, const float* W, const float* b, float* Y, int M, int N,
                      int K, hipStream_t s);
struct SmHyper;
int skinny_linear_bwd(const float* dY, const float* X, const float* W, float* dX, float* dW,
                      float* db, int M, int N, int K, bool accumulate, void* ws, size_t ws_bytes,
                      hipStream_t s, float* s_bar = nullptr, const SmHyper* sm = nullptr);

// Run C (+)= sum_s op(A_s) op(B_s) described by `d`: the LDS-DMA kernel when the shape
// allows it, else the register-staged MFMA kernel, else the SIMT kernel.
int gemm_run(const GemmDesc& d, int transA, int transB, int dtype, int c_dtype, hipStream_t s);

}  // namespace gn
