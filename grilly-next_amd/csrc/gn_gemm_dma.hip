// gn_gemm_dma.hip — dispatch of the LDS-DMA GEMM core (gn_gemm_dma_core.h) and the VSA
// unpack-project weight-gradient launch.  The GEMM launches themselves are instantiated in
// gn_gemm_dma_{f32a,f32b,bf16,glu}.hip.
#include "gn_gemm_dma_core.h"

namespace gn {

bool vsa_dma_applicable(const VsaDesc& v) {
    auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (v.K % BK || v.N % kVsaBN || v.lda % 8 || v.ldc % 8) return false;
    if (!al(v.C) || !al(v.A[0]) || (v.nseg > 1 && !al(v.A[1]))) return false;
    return v.K > 0 && v.M > 0 && v.N > 0;
}

int vsa_dma_launch(const VsaDesc& v, hipStream_t s) {
    const int tiles = ((v.M + kVsaBM - 1) / kVsaBM) * (v.N / kVsaBN);
    if (v.nseg > 1) {
        static const bool ok = allow_lds(vsa_dw_dma<true>, VsaK::SMEM);
        if (!ok) {
            set_error("vsa dW: cannot reserve %zu B of LDS", VsaK::SMEM);
            return GN_E_HIP;
        }
        hipLaunchKernelGGL(vsa_dw_dma<true>, dim3(tiles), dim3(64 * kVsaNW), VsaK::SMEM, s, v);
    } else {
        static const bool ok = allow_lds(vsa_dw_dma<false>, VsaK::SMEM);
        if (!ok) {
            set_error("vsa dW: cannot reserve %zu B of LDS", VsaK::SMEM);
            return GN_E_HIP;
        }
        hipLaunchKernelGGL(vsa_dw_dma<false>, dim3(tiles), dim3(64 * kVsaNW), VsaK::SMEM, s, v);
    }
    GN_LAUNCH_CHECK("vsa dW (dma)");
    return GN_OK;
}

bool gemm_dma_applicable(const GemmDesc& g) {
    auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (g.M % 8 || g.N % 8 || g.M < 8 || g.N < 8) return false;
    if (g.epi == 0 && (!al(g.C) || !al(g.C2) || g.ldc % 8 || (g.cbias && !al(g.cbias)))) return false;
    if (g.epi == 1 && (!al(g.gate) || !al(g.up) || !al(g.gu) || g.ldg % 8 || g.ldgu % 8 || g.H % 8))
        return false;
    for (int s = 0; s < g.nseg; ++s) {
        if (g.Ks[s] % BK || !al(g.A[s]) || !al(g.B[s]) || g.lda[s] % 8 || g.ldb[s] % 8) return false;
    }
    return true;
}

size_t gemm_dma_part_bytes(const GemmDesc& g0, int transA, int c_dtype) {
    if (g0.epi != 0 || c_dtype != GN_F32) return 0;
    GemmDesc g = g0;
    g.part_cap = ~(size_t)0;
    const TileChoice tc = choose_tile(g, transA != 0, sizeof(float), 0);
    return tc.ksplit > 2 ? part_bytes(g, tc.ksplit) : 0;
}

void launch_split_reduce(const GemmDesc& g, hipStream_t s) {
    split_reduce<<<grid_for((int64_t)g.M * (g.N / 4), 256, 4096), 256, 0, s>>>(g);
}

int gemm_dma_launch(const GemmDesc& g, int transA, int transB, int c_dtype, hipStream_t s) {
    if (g.epi == 1) return gemm_dma_glu(g, transA, transB, s);
    if (c_dtype == GN_F32) return transA ? gemm_dma_f32_ta1(g, transB, s) : gemm_dma_f32_ta0(g, transB, s);
    return gemm_dma_bf16(g, transA, transB, s);
}

}  // namespace gn
