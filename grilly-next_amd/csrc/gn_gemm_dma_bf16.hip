// gn_gemm_dma_bf16.hip — LDS-DMA GEMM launches with bf16 output, every operand orientation, instantiated in a
// compilation unit of their own (gn_gemm_dma_core.h).
#include "gn_gemm_dma_core.h"

namespace gn {

int gemm_dma_bf16(const GemmDesc& g, int transA, int transB, hipStream_t s) {
    return launch_trans<bf16_t, 0>(g, transA, transB, s);
}

}  // namespace gn
