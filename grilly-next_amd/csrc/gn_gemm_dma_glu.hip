// gn_gemm_dma_glu.hip — LDS-DMA GEMM launches with the GLU epilogue (down projection dA = dY Wd: both operands untransposed, the
// only orientation it is called with), instantiated in a
// compilation unit of their own (gn_gemm_dma_core.h).
#include "gn_gemm_dma_core.h"

namespace gn {

int gemm_dma_glu(const GemmDesc& g, int transA, int transB, hipStream_t s) {
    if (transA || transB) {
        set_error("gemm: the GLU epilogue takes untransposed operands only");
        return GN_E_INVALID;
    }
    return launch_shape<false, false, bf16_t, 1>(g, s);
}

}  // namespace gn
