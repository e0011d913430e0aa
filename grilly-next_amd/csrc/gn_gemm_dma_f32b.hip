// gn_gemm_dma_f32b.hip — LDS-DMA GEMM launches with fp32 output, k-outer A (transA = 1: the weight gradients), instantiated in a
// compilation unit of their own (gn_gemm_dma_core.h).
#include "gn_gemm_dma_core.h"

namespace gn {

int gemm_dma_f32_ta1(const GemmDesc& g, int transB, hipStream_t s) {
    return transB ? launch_shape<true, true, float, 0>(g, s) : launch_shape<true, false, float, 0>(g, s);
}

}  // namespace gn
