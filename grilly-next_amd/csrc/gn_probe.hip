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

// Four independent 16-byte loads in flight per thread before their stores.
__global__ __launch_bounds__(256) void probe_copy(uint4* __restrict__ dst, const uint4* __restrict__ src,
                                                  int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x;
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    const u32x4* s4 = reinterpret_cast<const u32x4*>(src);
    u32x4* d4 = reinterpret_cast<u32x4*>(dst);
    for (; i + 3 * stride < n; i += 4 * stride) {  // streaming (non-temporal) accesses
        const u32x4 a = __builtin_nontemporal_load(s4 + i), b = __builtin_nontemporal_load(s4 + i + stride);
        const u32x4 c = __builtin_nontemporal_load(s4 + i + 2 * stride);
        const u32x4 d = __builtin_nontemporal_load(s4 + i + 3 * stride);
        __builtin_nontemporal_store(a, d4 + i);
        __builtin_nontemporal_store(b, d4 + i + stride);
        __builtin_nontemporal_store(c, d4 + i + 2 * stride);
        __builtin_nontemporal_store(d, d4 + i + 3 * stride);
    }
    for (; i < n; i += stride) dst[i] = src[i];
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

extern "C" int gn_probe_copy(void* dst, const void* src, size_t bytes, void* stream) {
    clear_error();
    GN_REQUIRE(dst && src && bytes % 16 == 0, "gn_probe_copy: 16-byte multiples only");
    GN_REQUIRE(((uintptr_t)dst & 15u) == 0 && ((uintptr_t)src & 15u) == 0,
               "gn_probe_copy: 16-byte aligned pointers only");
    const int64_t n = (int64_t)(bytes / 16);
    probe_copy<<<grid_for(n, 256, 4096), 256, 0, as_stream(stream)>>>((uint4*)dst, (const uint4*)src, n);
    GN_LAUNCH_CHECK("gn_probe_copy");
    return GN_OK;
}
