// gn_gemm_dma_f32a.hip — LDS-DMA GEMM launches with fp32 output, k-contiguous A (transA = 0), instantiated in a
// compilation unit of their own (gn_gemm_dma_core.h).
#include "gn_gemm_dma_core.h"

namespace gn {

int gemm_dma_f32_ta0(const GemmDesc& g, int transB, hipStream_t s) {
    return transB ? launch_shape<false, true, float, 0>(g, s) : launch_shape<false, false, float, 0>(g, s);
}

}  // namespace gn
