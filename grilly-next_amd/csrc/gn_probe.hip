// gn_probe.hip — two measurement kernels for the roofline ceilings on the device itself:
// an MFMA-only loop (no memory traffic) and a streaming 16-byte copy.  They carry no part of
// the backward pass; bench.py --ceilings times them next to the spec figures.
#include "gn_common.h"
#include "gn_mfma.h"

namespace gn {
namespace {

// Each wave keeps 8 independent 32x32 accumulators busy: iters x 8 MFMAs of 32x32x16 bf16.
__global__ __launch_bounds__(256) void probe_mfma(float* __restrict__ out, int iters) {
    const int lane = threadIdx.x & 63;
    bf16x8_t a, b;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        a[e] = (__bf16)(0.001f * (lane + e));
        b[e] = (__bf16)(0.002f * (lane - e));
    }
    f32x16_t acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) zero16(acc[j]);
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = mfma32(a, b, acc[j]);
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[j][r];
    out[blockIdx.x * 256 + threadIdx.x] = s;
}

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// Streaming copy, grid-stride over 16-byte vectors, NV vectors loaded per thread before any
// of them is stored.  NT: non-temporal (streaming) loads and stores, else plain ones.
template <int NV, bool NT>
__global__ __launch_bounds__(256) void probe_copy(u32x4* __restrict__ dst, const u32x4* __restrict__ src,
                                                  int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x;
    for (; i + (NV - 1) * stride < n; i += NV * stride) {
        u32x4 v[NV];
#pragma unroll
        for (int k = 0; k < NV; ++k)
            v[k] = NT ? __builtin_nontemporal_load(src + i + k * stride) : src[i + k * stride];
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            if (NT) __builtin_nontemporal_store(v[k], dst + i + k * stride);
            else dst[i + k * stride] = v[k];
        }
    }
    for (; i < n; i += stride) dst[i] = src[i];
}

// Read-only stream: 8 vectors in flight per thread, one xor-folded word per thread written
// so the loads cannot be dropped (4 bytes per thread of writes: negligible traffic).
__global__ __launch_bounds__(256) void probe_read(unsigned* __restrict__ out, const u32x4* __restrict__ src,
                                                  int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x;
    u32x4 acc = {0u, 0u, 0u, 0u};
    for (; i + 7 * stride < n; i += 8 * stride) {
        u32x4 v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = __builtin_nontemporal_load(src + i + k * stride);
#pragma unroll
        for (int k = 0; k < 8; ++k) acc ^= v[k];
    }
    for (; i < n; i += stride) acc ^= src[i];
    out[blockIdx.x * 256 + threadIdx.x] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

}  // namespace
}  // namespace gn

using namespace gn;

extern "C" int gn_probe_mfma(float* out, int blocks, int iters, void* stream) {
    clear_error();
    GN_REQUIRE(out && blocks > 0 && iters > 0, "gn_probe_mfma: bad arguments");
    probe_mfma<<<blocks, 256, 0, as_stream(stream)>>>(out, iters);
    GN_LAUNCH_CHECK("gn_probe_mfma");
    return GN_OK;
}

extern "C" int gn_probe_copy(void* dst, const void* src, size_t bytes, int mode, void* stream) {
    clear_error();
    GN_REQUIRE(dst && src && bytes % 16 == 0, "gn_probe_copy: 16-byte multiples only");
    GN_REQUIRE(((uintptr_t)dst & 15u) == 0 && ((uintptr_t)src & 15u) == 0,
               "gn_probe_copy: 16-byte aligned pointers only");
    GN_REQUIRE(mode >= 0 && mode <= 3, "gn_probe_copy: mode %d (0..3)", mode);
    const int64_t n = (int64_t)(bytes / 16);
    hipStream_t s = as_stream(stream);
    const unsigned grid = grid_for(n, 256, 4096);
    u32x4* d = (u32x4*)dst;
    const u32x4* sv = (const u32x4*)src;
    switch (mode) {
        case 0: probe_copy<4, true><<<grid, 256, 0, s>>>(d, sv, n); break;
        case 1: probe_copy<4, false><<<grid, 256, 0, s>>>(d, sv, n); break;
        case 2: probe_copy<8, false><<<grid, 256, 0, s>>>(d, sv, n); break;
        default:
            GN_REQUIRE(bytes >= (size_t)grid * 256 * 4, "gn_probe_copy: read mode needs dst >= %u B",
                       grid * 256 * 4);
            probe_read<<<grid, 256, 0, s>>>((unsigned*)dst, sv, n);
            break;
    }
    GN_LAUNCH_CHECK("gn_probe_copy");
    return GN_OK;
}
