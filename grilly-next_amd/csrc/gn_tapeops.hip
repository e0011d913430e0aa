// gn_tapeops.hip — backward kernels of the tape ops the reference leaves as stubs
// (autograd.cpp:543-711: Sub, Mul, Div, Sum, Mean, Transpose, MSE set a sentinel gradient
// id) and of its two VSA heads (LoRA expand, cosine blend: autograd.cpp:817-859).
// Elementwise ops are single-pass HBM streams (grid-stride, one element per thread per
// step); the transpose goes through a 64 x 65 LDS tile so both sides stay coalesced; the
// LoRA-expand gradients are two GEMMs on the GEMM core's dispatch.
#include "gn_common.h"

namespace gn {

int gemm_dispatch(const void* A0, const void* B0, int K0, const void* A1, const void* B1, int K1,
                  void* C, int M, int N, int transA, int transB, int dtype, int c_dtype,
                  unsigned flags, hipStream_t s, void* ws, size_t ws_bytes);

namespace {

// One instantiation per op: the first version switched on a runtime op inside the loop and
// its Neg path stored a register that only the Sub/Mul/Div paths assigned (read in the
// generated ISA: the -dy value never reached the store); straight-line kernels avoid that.
template <typename T, int OP>
__global__ __launch_bounds__(256) void binary_bwd_kernel(const T* __restrict__ dY,
                                                         const T* __restrict__ A,
                                                         const T* __restrict__ B, T* __restrict__ dA,
                                                         T* __restrict__ dB, int64_t n, int acc) {
    for (int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const float g = io<T>::ld(dY, i);
        float da, db = 0.f;
        if constexpr (OP == GN_BIN_SUB) {
            da = g;
            db = -g;
        } else if constexpr (OP == GN_BIN_MUL) {
            da = dA ? g * io<T>::ld(B, i) : 0.f;
            db = dB ? g * io<T>::ld(A, i) : 0.f;
        } else if constexpr (OP == GN_BIN_DIV) {
            const float b = io<T>::ld(B, i);
            da = g / b;
            db = dB ? -g * io<T>::ld(A, i) / (b * b) : 0.f;
        } else {
            da = -g;
        }
        if (dA) io<T>::st(dA, i, acc ? io<T>::ld(dA, i) + da : da);
        if constexpr (OP != GN_BIN_NEG) {
            if (dB) io<T>::st(dB, i, acc ? io<T>::ld(dB, i) + db : db);
        }
    }
}

template <typename T>
int launch_binary(int op, const void* dY, const void* A, const void* B, void* dA, void* dB,
                  int64_t n, int acc, hipStream_t s) {
    const unsigned g = grid_for(n, 256);
    auto y = (const T*)dY;
    auto a = (const T*)A;
    auto b = (const T*)B;
    switch (op) {
        case GN_BIN_SUB: binary_bwd_kernel<T, GN_BIN_SUB><<<g, 256, 0, s>>>(y, a, b, (T*)dA, (T*)dB, n, acc); break;
        case GN_BIN_MUL: binary_bwd_kernel<T, GN_BIN_MUL><<<g, 256, 0, s>>>(y, a, b, (T*)dA, (T*)dB, n, acc); break;
        case GN_BIN_DIV: binary_bwd_kernel<T, GN_BIN_DIV><<<g, 256, 0, s>>>(y, a, b, (T*)dA, (T*)dB, n, acc); break;
        default: binary_bwd_kernel<T, GN_BIN_NEG><<<g, 256, 0, s>>>(y, a, b, (T*)dA, (T*)dB, n, acc); break;
    }
    GN_LAUNCH_CHECK("gn_binary_bwd");
    return GN_OK;
}

template <typename T>
__global__ __launch_bounds__(256) void reduce_bwd_kernel(const T* __restrict__ dY, T* __restrict__ dX,
                                                         int64_t outer, int64_t inner, float mul,
                                                         int acc) {
    const int64_t n = outer * inner;
    for (int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const float v = io<T>::ld(dY, i / inner) * mul;
        io<T>::st(dX, i, acc ? io<T>::ld(dX, i) + v : v);
    }
}

// dX[b, r, c] = dY[b, c, r]: block = one 64 x 64 tile of dX (rows r0.., cols c0..), 256
// threads; the tile is read from dY row-wise (coalesced along r) into LDS and written to dX
// row-wise (coalesced along c).  Pitch 65 keeps the column reads conflict-free.
template <typename T>
__global__ __launch_bounds__(256) void transpose_bwd_kernel(const T* __restrict__ dY, T* __restrict__ dX,
                                                            int rows, int cols, int acc) {
    __shared__ float tile[64][65];
    const int b = blockIdx.z;
    const int r0 = blockIdx.x * 64, c0 = blockIdx.y * 64;
    const T* src = dY + (size_t)b * rows * cols;  // [cols][rows]
    T* dst = dX + (size_t)b * rows * cols;        // [rows][cols]
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int j = ty; j < 64; j += 4) {
        const int c = c0 + j, r = r0 + tx;
        tile[j][tx] = (c < cols && r < rows) ? io<T>::ld(src, (size_t)c * rows + r) : 0.f;
    }
    __syncthreads();
    for (int j = ty; j < 64; j += 4) {
        const int r = r0 + j, c = c0 + tx;
        if (r < rows && c < cols) {
            const size_t o = (size_t)r * cols + c;
            const float v = tile[tx][j];
            io<T>::st(dst, o, acc ? io<T>::ld(dst, o) + v : v);
        }
    }
}

template <typename T>
__global__ __launch_bounds__(256) void mse_bwd_kernel(const T* __restrict__ P, const T* __restrict__ Tg,
                                                      const float* __restrict__ dL, T* __restrict__ dP,
                                                      int64_t n, float scale, int acc) {
    const float g = 2.0f * scale * (dL ? dL[0] : 1.0f);
    for (int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const float v = g * (io<T>::ld(P, i) - io<T>::ld(Tg, i));
        io<T>::st(dP, i, acc ? io<T>::ld(dP, i) + v : v);
    }
}

// vsa-cosine-blend-backward.glsl:37-70; block (x, b): 256 elements i of row b, all K branches
__global__ __launch_bounds__(256) void cosine_blend_bwd_kernel(
    const uint32_t* __restrict__ bits, const float* __restrict__ weights,
    const float* __restrict__ blended, const float* __restrict__ info, float* __restrict__ dP,
    int K, int D, int words, float scale, int acc) {
    const int b = blockIdx.y;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= D) return;
    const float dot_bt = info[(size_t)b * 3 + 1], norm_sq = info[(size_t)b * 3 + 2];
    const float norm_b = sqrtf(fmaxf(norm_sq, 1e-8f));
    const float sqrt_D = sqrtf((float)D);
    const float cosine = dot_bt / (norm_b * sqrt_D);
    const float y = ((bits[(size_t)b * words + (i >> 5)] >> (i & 31)) & 1u) ? 1.0f : -1.0f;
    const float bi = blended[(size_t)b * D + i];
    const float gb = -(y / (norm_b * sqrt_D) - cosine * bi / fmaxf(norm_sq, 1e-8f));
    for (int k = 0; k < K; ++k) {
        const size_t idx = ((size_t)b * K + k) * D + i;
        const float g = fminf(fmaxf(gb * weights[(size_t)b * K + k] * scale, -1.0f), 1.0f);
        dP[idx] = acc ? dP[idx] + g : g;
    }
}

}  // namespace
}  // namespace gn

using namespace gn;

extern "C" int gn_binary_bwd(int op, const void* dY, const void* A, const void* B, void* dA,
                             void* dB, int64_t n, int dtype, unsigned flags, void* stream) {
    clear_error();
    GN_REQUIRE(op >= GN_BIN_SUB && op <= GN_BIN_NEG, "gn_binary_bwd: op %d", op);
    GN_REQUIRE(n >= 0, "gn_binary_bwd: negative size");
    if (n == 0 || (!dA && !dB)) return GN_OK;
    GN_REQUIRE(dY, "gn_binary_bwd: null dY");
    GN_REQUIRE(op != GN_BIN_NEG || !dB, "gn_binary_bwd: negation has one input");
    GN_REQUIRE(op != GN_BIN_MUL || ((!dA || B) && (!dB || A)), "gn_binary_bwd: mul needs the other operand");
    GN_REQUIRE(op != GN_BIN_DIV || (B && (!dB || A)), "gn_binary_bwd: div needs b (and a for db)");
    GN_REQUIRE(dtype == GN_F32 || dtype == GN_BF16, "gn_binary_bwd: dtype %d", dtype);
    hipStream_t s = as_stream(stream);
    const int acc = (flags & GN_ACCUMULATE) ? 1 : 0;
    if (dtype == GN_F32) return launch_binary<float>(op, dY, A, B, dA, dB, n, acc, s);
    return launch_binary<bf16_t>(op, dY, A, B, dA, dB, n, acc, s);
}

extern "C" int gn_reduce_bwd(int op, const void* dY, void* dX, int64_t outer, int64_t inner,
                             int dtype, unsigned flags, void* stream) {
    clear_error();
    GN_REQUIRE(op == GN_RED_SUM || op == GN_RED_MEAN, "gn_reduce_bwd: op %d", op);
    GN_REQUIRE(outer >= 0 && inner >= 0, "gn_reduce_bwd: negative size");
    if (outer == 0 || inner == 0) return GN_OK;
    GN_REQUIRE(dY && dX, "gn_reduce_bwd: null pointer");
    GN_REQUIRE(dtype == GN_F32 || dtype == GN_BF16, "gn_reduce_bwd: dtype %d", dtype);
    hipStream_t s = as_stream(stream);
    const float mul = op == GN_RED_MEAN ? (float)(1.0 / (double)inner) : 1.0f;
    const unsigned g = grid_for(outer * inner, 256);
    const int acc = (flags & GN_ACCUMULATE) ? 1 : 0;
    if (dtype == GN_F32)
        reduce_bwd_kernel<float><<<g, 256, 0, s>>>((const float*)dY, (float*)dX, outer, inner, mul, acc);
    else
        reduce_bwd_kernel<bf16_t><<<g, 256, 0, s>>>((const bf16_t*)dY, (bf16_t*)dX, outer, inner, mul, acc);
    GN_LAUNCH_CHECK("gn_reduce_bwd");
    return GN_OK;
}

extern "C" int gn_transpose_bwd(const void* dY, void* dX, int64_t batch, int rows, int cols,
                                int dtype, unsigned flags, void* stream) {
    clear_error();
    GN_REQUIRE(batch >= 0 && rows >= 0 && cols >= 0, "gn_transpose_bwd: negative size");
    if (batch == 0 || rows == 0 || cols == 0) return GN_OK;
    GN_REQUIRE(dY && dX, "gn_transpose_bwd: null pointer");
    GN_REQUIRE(batch <= 65535, "gn_transpose_bwd: batch %lld > 65535", (long long)batch);
    GN_REQUIRE(dtype == GN_F32 || dtype == GN_BF16, "gn_transpose_bwd: dtype %d", dtype);
    hipStream_t s = as_stream(stream);
    dim3 grid((rows + 63) / 64, (cols + 63) / 64, (unsigned)batch);
    const int acc = (flags & GN_ACCUMULATE) ? 1 : 0;
    if (dtype == GN_F32)
        transpose_bwd_kernel<float><<<grid, 256, 0, s>>>((const float*)dY, (float*)dX, rows, cols, acc);
    else
        transpose_bwd_kernel<bf16_t><<<grid, 256, 0, s>>>((const bf16_t*)dY, (bf16_t*)dX, rows, cols, acc);
    GN_LAUNCH_CHECK("gn_transpose_bwd");
    return GN_OK;
}

extern "C" int gn_mse_bwd(const void* pred, const void* target, const float* dLoss, void* dPred,
                          int64_t n, float scale, int dtype, unsigned flags, void* stream) {
    clear_error();
    GN_REQUIRE(n >= 0, "gn_mse_bwd: negative size");
    if (n == 0) return GN_OK;
    GN_REQUIRE(pred && target && dPred, "gn_mse_bwd: null pointer");
    GN_REQUIRE(dtype == GN_F32 || dtype == GN_BF16, "gn_mse_bwd: dtype %d", dtype);
    hipStream_t s = as_stream(stream);
    const unsigned g = grid_for(n, 256);
    const int acc = (flags & GN_ACCUMULATE) ? 1 : 0;
    if (dtype == GN_F32)
        mse_bwd_kernel<float><<<g, 256, 0, s>>>((const float*)pred, (const float*)target, dLoss,
                                               (float*)dPred, n, scale, acc);
    else
        mse_bwd_kernel<bf16_t><<<g, 256, 0, s>>>((const bf16_t*)pred, (const bf16_t*)target, dLoss,
                                                (bf16_t*)dPred, n, scale, acc);
    GN_LAUNCH_CHECK("gn_mse_bwd");
    return GN_OK;
}

extern "C" int gn_vsa_lora_expand_bwd(const float* dPreds, const float* basis, const float* coeffs,
                                      float* dCoeffs, float* dBasis, int Bn, int K, int D, int rank,
                                      float scale, unsigned flags, void* stream) {
    clear_error();
    GN_REQUIRE(Bn >= 0 && K >= 0 && D >= 0 && rank >= 0, "gn_vsa_lora_expand_bwd: negative size");
    const int rowsBK = Bn * K;
    if (rowsBK == 0 || D == 0 || rank == 0) return GN_OK;
    GN_REQUIRE(dPreds, "gn_vsa_lora_expand_bwd: null dPreds");
    GN_REQUIRE(!dCoeffs || basis, "gn_vsa_lora_expand_bwd: dCoeffs needs the basis");
    GN_REQUIRE(!dBasis || coeffs, "gn_vsa_lora_expand_bwd: dBasis needs the coefficients");
    GN_REQUIRE(scale == 1.0f, "gn_vsa_lora_expand_bwd: grad_scale other than 1 is not supported "
                              "(the reference handler passes 1, autograd.cpp:834)");
    hipStream_t s = as_stream(stream);
    int rc;
    // dCoeffs [Bn*K x rank] = dPreds [Bn*K x D] . basis [D x rank]
    if (dCoeffs && (rc = gemm_dispatch(dPreds, basis, D, nullptr, nullptr, 0, dCoeffs, rowsBK, rank,
                                       0, 0, GN_F32, GN_F32, flags, s, nullptr, 0)))
        return rc;
    // dBasis [D x rank] (+)= dPreds^T . coeffs  (A stored [Bn*K x D] = transposed)
    if (dBasis && (rc = gemm_dispatch(dPreds, coeffs, rowsBK, nullptr, nullptr, 0, dBasis, D, rank,
                                      1, 0, GN_F32, GN_F32, flags, s, nullptr, 0)))
        return rc;
    return GN_OK;
}

extern "C" int gn_vsa_cosine_blend_bwd(const uint32_t* true_bits, const float* weights,
                                       const float* blended, const float* loss_info, float* dPreds,
                                       int Bn, int K, int D, int words, float grad_scale,
                                       unsigned flags, void* stream) {
    clear_error();
    GN_REQUIRE(Bn >= 0 && K >= 0 && D >= 0, "gn_vsa_cosine_blend_bwd: negative size");
    if (Bn == 0 || K == 0 || D == 0) return GN_OK;
    GN_REQUIRE(true_bits && weights && blended && loss_info && dPreds,
               "gn_vsa_cosine_blend_bwd: null pointer");
    GN_REQUIRE(words * 32 >= D, "gn_vsa_cosine_blend_bwd: %d words cannot hold D = %d", words, D);
    GN_REQUIRE(Bn <= 65535, "gn_vsa_cosine_blend_bwd: batch %d > 65535", Bn);
    hipStream_t s = as_stream(stream);
    cosine_blend_bwd_kernel<<<dim3((D + 255) / 256, Bn), 256, 0, s>>>(
        true_bits, weights, blended, loss_info, dPreds, K, D, words, grad_scale,
        (flags & GN_ACCUMULATE) ? 1 : 0);
    GN_LAUNCH_CHECK("gn_vsa_cosine_blend_bwd");
    return GN_OK;
}
