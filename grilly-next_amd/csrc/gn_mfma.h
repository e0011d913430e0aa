// gn_mfma.h — gfx950 building blocks shared by the MFMA kernels: operand vector types, the
// 32x32x16 bf16 MFMA, the LDS transpose read and the 16-byte global->LDS DMA.
#pragma once

#include "gn_common.h"

namespace gn {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef short s16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4;

// D(32x32) += A(32x16) B(16x32).  Lane l supplies A row l%32 / B column l%32 with
// k = 8(l/32) .. +7 (any k order works as long as A and B use the same one); the result
// holds column l%32, rows 8(r/4) + 4(l/32) + r%4 in element r.
__device__ __forceinline__ f32x16_t mfma32(bf16x8_t a, bf16x8_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ void zero16(f32x16_t& a) {
#pragma unroll
    for (int r = 0; r < 16; ++r) a[r] = 0.f;
}

__device__ __forceinline__ bf16x8_t ld_frag16(const bf16_t* p) {
    return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(p));
}

// Two ds_read_b64_tr_b16: within each 16-lane group lane i receives column i of the
// 4 (rows) x 16 (columns) block addressed by the group, four consecutive rows.
__device__ __forceinline__ bf16x8_t ld_tr_pair(const bf16_t* p0, const bf16_t* p1) {
    s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p0));
    s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p1));
    s16x8_t v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(bf16x8_t, v);
}

// eight floats -> eight bf16 (v_cvt_pk_bf16_f32, round to nearest even)
__device__ __forceinline__ bf16x8_t to_bf16x8(float a0, float a1, float a2, float a3, float a4,
                                              float a5, float a6, float a7) {
    bf16x8_t v;
    v[0] = (__bf16)a0; v[1] = (__bf16)a1; v[2] = (__bf16)a2; v[3] = (__bf16)a3;
    v[4] = (__bf16)a4; v[5] = (__bf16)a5; v[6] = (__bf16)a6; v[7] = (__bf16)a7;
    return v;
}

// LDS byte address of a pointer into __shared__ memory (the DMA's M0 operand)
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(lds_void*)p;
}

// One 16-byte DMA per lane: lane l's bytes land at LDS byte address lds_base + 16*l.
// Issued from inline assembly so the compiler does not order later LDS reads of *other*
// buffers behind it (it cannot tell buffers apart); callers wait for their own DMA
// explicitly (s_waitcnt vmcnt + barrier) before reading the buffer it fills.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds_base) {
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, off"
        :
        : "s"(lds_base), "v"(g)
        : "memory", "m0");
}

// The same DMA from a wave-uniform base (SGPRs) plus a per-lane 32-bit byte offset.  A
// tile's base moves with k on the scalar unit while the lane offsets (row and swizzled
// chunk within the tile) are computed once per kernel, so a tile's DMA costs no vector
// instructions; 64-bit per-lane address arithmetic per tile takes ~8 VALU instructions
// per DMA, most of them multi-pass, and stretches the MFMA step that issues them.
__device__ __forceinline__ void dma16s(const void* sbase, uint32_t voff, uint32_t lds_base) {
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %2"
        :
        : "s"(lds_base), "v"(voff), "s"(sbase)
        : "memory", "m0");
}

// s_waitcnt immediate that waits until at most N vector-memory operations are
// outstanding (vmcnt bits [3:0] and [15:14]; expcnt and lgkmcnt left at their maxima)
constexpr unsigned vmcnt_imm(unsigned n) { return 0x0F70u | (n & 15u) | ((n >> 4) << 14); }

}  // namespace gn
