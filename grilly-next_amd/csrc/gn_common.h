// gn_common.h — shared device/host helpers for libgn_bwd (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include <cstdio>
#include <string>

#include "gn_bwd.h"

namespace gn {

// ---- error reporting (thread-local message behind gn_last_error) --------------------
void set_error(const char* fmt, ...);
void clear_error();

#define GN_REQUIRE(cond, ...)                  \
    do {                                       \
        if (!(cond)) {                         \
            ::gn::set_error(__VA_ARGS__);      \
            return GN_E_INVALID;               \
        }                                      \
    } while (0)

#define GN_LAUNCH_CHECK(what)                                                          \
    do {                                                                               \
        hipError_t e_ = hipGetLastError();                                             \
        if (e_ != hipSuccess) {                                                        \
            ::gn::set_error("%s: launch failed: %s", what, hipGetErrorString(e_));       \
            return GN_E_HIP;                                                           \
        }                                                                              \
    } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ---- bf16 storage helpers -------------------------------------------------------------
typedef uint16_t bf16_t;  // raw bf16 bits in memory

__device__ __forceinline__ float bf2f(bf16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

// round-to-nearest-even float -> bf16 (NaN stays NaN): gfx950's v_cvt_pk_bf16_f32
__device__ __forceinline__ bf16_t f2bf(float f) { return __builtin_bit_cast(bf16_t, (__bf16)f); }

// pack two floats into one dword of bf16 (lo = a, hi = b), one v_cvt_pk_bf16_f32
__device__ __forceinline__ uint32_t pack_bf2(float a, float b) {
    typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
    bf16x2_v v;
    v[0] = (__bf16)a;
    v[1] = (__bf16)b;
    return __builtin_bit_cast(uint32_t, v);
}

template <typename T> struct io;
template <> struct io<float> {
    static __device__ __forceinline__ float ld(const float* p, size_t i) { return p[i]; }
    static __device__ __forceinline__ void st(float* p, size_t i, float v) { p[i] = v; }
};
template <> struct io<bf16_t> {
    static __device__ __forceinline__ float ld(const bf16_t* p, size_t i) { return bf2f(p[i]); }
    static __device__ __forceinline__ void st(bf16_t* p, size_t i, float v) { p[i] = f2bf(v); }
};

// ---- small math (fast hardware exp; formulas from the op definitions) ----------------
__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }
__device__ __forceinline__ float tanhf_(float z) {
    // tanh(z) = 1 - 2 / (exp(2z) + 1); saturates cleanly for |z| large
    float e = __expf(2.0f * z);
    return 1.0f - 2.0f / (e + 1.0f);
}

// ---- wave / block reductions (wave64) -------------------------------------------------
// Within each row of 16 lanes by DPP moves (quad_perm [1,0,3,2] and [2,3,0,1], then
// row_half_mirror and row_mirror, which act as xor 4 and xor 8 once quads and half-rows hold
// equal values), then the four row results read with v_readlane and combined in a fixed
// order: every lane gets the same value, a few cycles per step instead of an LDS-crossbar
// round trip per step.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_mov<0x141>(v);  // row_half_mirror
    v += dpp_mov<0x140>(v);  // row_mirror
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_mov<0xB1>(v));
    v = fmaxf(v, dpp_mov<0x4E>(v));
    v = fmaxf(v, dpp_mov<0x141>(v));
    v = fmaxf(v, dpp_mov<0x140>(v));
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

// Sum over a block of NW waves; `sh` must hold NW floats. Result broadcast to all threads.
template <int NW>
__device__ __forceinline__ float block_sum(float v, float* sh) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    __syncthreads();
    if (l == 0) sh[w] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < NW; ++i) t += sh[i];
    return t;
}
template <int NW>
__device__ __forceinline__ float block_max(float v, float* sh) {
    v = wave_max(v);
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    __syncthreads();
    if (l == 0) sh[w] = v;
    __syncthreads();
    float t = -INFINITY;
#pragma unroll
    for (int i = 0; i < NW; ++i) t = fmaxf(t, sh[i]);
    return t;
}

// Eight consecutive elements as float through one or two 16-byte accesses (16-byte aligned).
template <typename T> struct chunk8;
template <> struct chunk8<float> {
    static __device__ __forceinline__ void ld(const float* p, float (&v)[8]) {
        const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
    static __device__ __forceinline__ void st(float* p, const float (&v)[8]) {
        reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
        reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
};
template <> struct chunk8<bf16_t> {
    static __device__ __forceinline__ void ld(const bf16_t* p, float (&v)[8]) {
        const uint4 x = *reinterpret_cast<const uint4*>(p);
        const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = __uint_as_float(w[i] << 16);
            v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    }
    static __device__ __forceinline__ void st(bf16_t* p, const float (&v)[8]) {
        *reinterpret_cast<uint4*>(p) = make_uint4(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]),
                                                  pack_bf2(v[4], v[5]), pack_bf2(v[6], v[7]));
    }
};

// Orders one wave's LDS accesses across its lanes (writes of some lanes before reads of
// others, or reads before the next overwrite) without a block barrier: wave-scope release and
// acquire fences around a wave barrier.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

inline unsigned grid_for(int64_t n, int per_block, unsigned cap = 65535u * 16u) {
    int64_t g = (n + per_block - 1) / per_block;
    if (g < 1) g = 1;
    if (g > (int64_t)cap) g = cap;
    return (unsigned)g;
}

// Zero `bytes` bytes at p with a fill kernel (gn_elementwise.hip).  The library clears memory
// this way, never with hipMemsetAsync, so that every entry point records only kernel nodes
// when a caller captures it into a HIP graph.
hipError_t launch_zero(void* p, size_t bytes, hipStream_t s);

}  // namespace gn
