// gn_gemm.hip — the contraction core of the backward pass.
//
//   C[M x N] (+)= sum_s opA(A_s) opB(B_s)      (s = up to two K-segments)
//
// bf16 path: 128x128 block tile, BK = 64, 256 threads = 4 waves (2 x 2), each wave a
// 64 x 64 sub-tile made of 2 x 2 v_mfma_f32_32x32x16_bf16 (fp32 accumulation).  Both
// operands are staged in LDS as [row][k] (k contiguous, 16-byte padded rows) so every MFMA
// fragment is one ds_read_b128.  Operands whose k index is the *outer* (row) dimension
// in global memory (dY^T in dW = dY^T X, W in dX = dY W, X in dW) are transposed in
// registers on the way into LDS: a thread loads 4 k-rows x 8 columns (four 16-byte loads)
// and v_perm_b32 regroups them into eight 4-element k-runs.  Global->LDS traffic for tile
// t+1 is issued before the MFMAs of tile t (register prefetch + double-buffered LDS).
// Blocks are remapped so each XCD (8 per MI355X, round-robin dispatch) owns a contiguous
// range of tiles, grouped 8 tile-rows high for L2 reuse.
//
// fp32 path (and bf16 shapes that are not multiples of 8): a 64x64 SIMT tile kernel.
#include <algorithm>

#include "gn_common.h"

namespace gn {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int LDS_PITCH = BK;  // bf16 elements per LDS row (128 bytes, XOR-swizzled chunks)
constexpr int TILE_ELEMS = 128 * LDS_PITCH;

// 16-byte chunk c of row r lives at chunk c ^ swz(r).  Fragment reads (32 consecutive rows,
// one chunk) and the transposed stores (rows 8 apart) both spread over all 8 chunk slots.
__device__ __forceinline__ int swz(int r) { return (r ^ (r >> 3)) & 7; }

struct GemmArgs {
    const bf16_t* A[2];
    const bf16_t* B[2];
    int Ks[2];
    int nseg;
    void* C;
    int M, N;
    int accumulate;
};

// Load one 128-row x 64-k operand tile into registers (4 x 16 bytes per thread).
//   KCONTIG: element (r, k) at P[r * ld + k]    (r = row of the tile: m for A, n for B)
//   else   : element (r, k) at P[k * ld + r]
template <bool KCONTIG>
__device__ __forceinline__ void load_tile(const bf16_t* __restrict__ P, int ld, int r0,
                                          int rlim, int k0, int klim, uint4 (&reg)[4]) {
    const int t = threadIdx.x;
    if (KCONTIG) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = t + 256 * i;
            const int r = r0 + (c >> 3), k = k0 + (c & 7) * 8;
            if (r < rlim && k < klim)
                reg[i] = *reinterpret_cast<const uint4*>(P + (size_t)r * ld + k);
            else
                reg[i] = make_uint4(0, 0, 0, 0);
        }
    } else {
        const int rc = t & 15, kg = t >> 4;  // 16 column chunks of 8, 16 groups of 4 k-rows
        const int r = r0 + rc * 8;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int k = k0 + kg * 4 + i;
            if (r < rlim && k < klim)
                reg[i] = *reinterpret_cast<const uint4*>(P + (size_t)k * ld + r);
            else
                reg[i] = make_uint4(0, 0, 0, 0);
        }
    }
}

template <bool KCONTIG>
__device__ __forceinline__ void store_tile(bf16_t* __restrict__ s, const uint4 (&reg)[4]) {
    const int t = threadIdx.x;
    if (KCONTIG) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = t + 256 * i;
            const int r = c >> 3;
            *reinterpret_cast<uint4*>(s + r * LDS_PITCH + (((c & 7) ^ swz(r)) * 8)) = reg[i];
        }
    } else {
        // reg[i] holds row k = kg*4+i, columns rc*8 .. rc*8+7 (two bf16 per dword).
        // Output for column j: the 4 k-values (reg[0..3] element j) as two dwords.
        const int rc = t & 15, kg = t >> 4;
        const uint32_t w0[4] = {reg[0].x, reg[0].y, reg[0].z, reg[0].w};
        const uint32_t w1[4] = {reg[1].x, reg[1].y, reg[1].z, reg[1].w};
        const uint32_t w2[4] = {reg[2].x, reg[2].y, reg[2].z, reg[2].w};
        const uint32_t w3[4] = {reg[3].x, reg[3].y, reg[3].z, reg[3].w};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            // low halves -> column 2d, high halves -> column 2d+1
            uint2 lo, hi;
            lo.x = __builtin_amdgcn_perm(w1[d], w0[d], 0x05040100u);
            lo.y = __builtin_amdgcn_perm(w3[d], w2[d], 0x05040100u);
            hi.x = __builtin_amdgcn_perm(w1[d], w0[d], 0x07060302u);
            hi.y = __builtin_amdgcn_perm(w3[d], w2[d], 0x07060302u);
            const int r0 = rc * 8 + 2 * d, r1 = r0 + 1;
            *reinterpret_cast<uint2*>(s + r0 * LDS_PITCH + (((kg >> 1) ^ swz(r0)) * 8) + (kg & 1) * 4) = lo;
            *reinterpret_cast<uint2*>(s + r1 * LDS_PITCH + (((kg >> 1) ^ swz(r1)) * 8) + (kg & 1) * 4) = hi;
        }
    }
}

__device__ __forceinline__ bf16x8_t lds_frag(const bf16_t* p) {
    uint4 v = *reinterpret_cast<const uint4*>(p);
    return __builtin_bit_cast(bf16x8_t, v);
}

template <bool TA, bool TB, typename CT>
__global__ __launch_bounds__(256, 2) void gemm_bf16_mfma(GemmArgs g) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    bf16_t* sA = reinterpret_cast<bf16_t*>(smem_raw);  // [2][128][LDS_PITCH]
    bf16_t* sB = sA + 2 * TILE_ELEMS;                   // [2][128][LDS_PITCH]

    // ---- tile coordinates: XCD-contiguous ranges, then 8-tall groups ----
    const int tilesM = (g.M + BM - 1) / BM, tilesN = (g.N + BN - 1) / BN;
    const int nblk = tilesM * tilesN;
    int pid = blockIdx.x;
    if ((nblk & 7) == 0) pid = (pid & 7) * (nblk >> 3) + (pid >> 3);
    const int GROUP = 8;
    const int group_id = pid / (GROUP * tilesN);
    const int first_m = group_id * GROUP;
    const int gsize = min(tilesM - first_m, GROUP);
    const int in_group = pid % (GROUP * tilesN);
    const int tm = first_m + (in_group % gsize);
    const int tn = in_group / gsize;
    const int m0 = tm * BM, n0 = tn * BN;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    f32x16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int kt0 = (g.Ks[0] + BK - 1) / BK;
    const int kt1 = g.nseg > 1 ? (g.Ks[1] + BK - 1) / BK : 0;
    const int KT = kt0 + kt1;

    uint4 ra[4], rb[4];
    auto gload = [&](int t) {
        const int s = t < kt0 ? 0 : 1;
        const int k0 = (t < kt0 ? t : t - kt0) * BK;
        const int Ks = g.Ks[s];
        // A: TA=0 -> [M x Ks] (k contiguous); TA=1 -> stored [Ks x M]
        if (!TA) load_tile<true>(g.A[s], Ks, m0, g.M, k0, Ks, ra);
        else load_tile<false>(g.A[s], g.M, m0, g.M, k0, Ks, ra);
        // B: TB=1 -> stored [N x Ks] (k contiguous); TB=0 -> [Ks x N]
        if (TB) load_tile<true>(g.B[s], Ks, n0, g.N, k0, Ks, rb);
        else load_tile<false>(g.B[s], g.N, n0, g.N, k0, Ks, rb);
    };
    auto sstore = [&](int buf) {
        store_tile<!TA>(sA + buf * TILE_ELEMS, ra);
        store_tile<TB>(sB + buf * TILE_ELEMS, rb);
    };

    if (KT > 0) {
        gload(0);
        sstore(0);
    }
    __syncthreads();

    const int frow = lane & 31, fhalf = lane >> 5;
    // fragment rows: a rows wm*64 + {0,32} + frow, b rows wn*64 + {0,32} + frow
    const int ra0 = wm * 64 + frow, ra1 = ra0 + 32, rb0 = wn * 64 + frow, rb1 = rb0 + 32;
    const int sa0 = swz(ra0), sa1 = swz(ra1), sb0 = swz(rb0), sb1 = swz(rb1);
    for (int t = 0; t < KT; ++t) {
        const int cur = t & 1;
        if (t + 1 < KT) gload(t + 1);
        const bf16_t* As = sA + cur * TILE_ELEMS;
        const bf16_t* Bs = sB + cur * TILE_ELEMS;
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const int ch = ks * 2 + fhalf;
            bf16x8_t a0 = lds_frag(As + ra0 * LDS_PITCH + ((ch ^ sa0) * 8));
            bf16x8_t a1 = lds_frag(As + ra1 * LDS_PITCH + ((ch ^ sa1) * 8));
            bf16x8_t b0 = lds_frag(Bs + rb0 * LDS_PITCH + ((ch ^ sb0) * 8));
            bf16x8_t b1 = lds_frag(Bs + rb1 * LDS_PITCH + ((ch ^ sb1) * 8));
            acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0, acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b1, acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b0, acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b1, acc[1][1], 0, 0, 0);
        }
        if (t + 1 < KT) sstore(cur ^ 1);
        __syncthreads();
    }

    // ---- epilogue: 32x32 accumulator layout: col = lane%32, row = 8*(r/4) + 4*(lane/32) + r%4
    CT* C = reinterpret_cast<CT*>(g.C);
    const int col_l = lane & 31, rq = (lane >> 5) * 4;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + wn * 64 + j * 32 + col_l;
            if (n >= g.N) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + rq + (r & 3);
                if (m >= g.M) continue;
                const size_t idx = (size_t)m * g.N + n;
                float v = acc[i][j][r];
                if (g.accumulate) v += io<CT>::ld(C, idx);
                io<CT>::st(C, idx, v);
            }
        }
}

// ---- SIMT fallback: 64x64 tile, BK 16, 4x4 outputs per thread -------------------------
template <typename TI, typename CT, bool TA, bool TB>
__global__ __launch_bounds__(256) void gemm_simt(const TI* A0, const TI* B0, int K0,
                                                 const TI* A1, const TI* B1, int K1, CT* C,
                                                 int M, int N, int accumulate) {
    __shared__ float sA[16][64 + 4];
    __shared__ float sB[16][64 + 4];
    const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    float acc[4][4] = {};
    for (int s = 0; s < 2; ++s) {
        const TI* A = s ? A1 : A0;
        const TI* B = s ? B1 : B0;
        const int Ks = s ? K1 : K0;
        if (!A || Ks <= 0) continue;
        for (int k0 = 0; k0 < Ks; k0 += 16) {
            for (int e = threadIdx.x; e < 16 * 64; e += 256) {
                const int kk = e / 64, mm = e % 64;
                const int m = m0 + mm, k = k0 + kk;
                float va = 0.f;
                if (m < M && k < Ks) va = TA ? io<TI>::ld(A, (size_t)k * M + m) : io<TI>::ld(A, (size_t)m * Ks + k);
                sA[kk][mm] = va;
                const int n = n0 + mm;
                float vb = 0.f;
                if (n < N && k < Ks) vb = TB ? io<TI>::ld(B, (size_t)n * Ks + k) : io<TI>::ld(B, (size_t)k * N + n);
                sB[kk][mm] = vb;
            }
            __syncthreads();
#pragma unroll
            for (int kk = 0; kk < 16; ++kk) {
                float a[4], b[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) a[i] = sA[kk][ty + 16 * i];
#pragma unroll
                for (int j = 0; j < 4; ++j) b[j] = sB[kk][tx + 16 * j];
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[i][j] += a[i] * b[j];
            }
            __syncthreads();
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int m = m0 + ty + 16 * i, n = n0 + tx + 16 * j;
            if (m < M && n < N) {
                const size_t idx = (size_t)m * N + n;
                float v = acc[i][j];
                if (accumulate) v += io<CT>::ld(C, idx);
                io<CT>::st(C, idx, v);
            }
        }
}

// ---- column sums (db): thread per column, rows split over grid.y with fp32 atomics ------
template <typename TI>
__global__ __launch_bounds__(256) void colsum_kernel(const TI* __restrict__ in, float* out,
                                                     int M, int N, int rows_per) {
    const int n = blockIdx.x * 256 + threadIdx.x;
    if (n >= N) return;
    const int r0 = blockIdx.y * rows_per, r1 = min(M, r0 + rows_per);
    float s = 0.f;
    for (int r = r0; r < r1; ++r) s += io<TI>::ld(in, (size_t)r * N + n);
    if (gridDim.y == 1) out[n] += s;
    else atomicAdd(out + n, s);
}

__global__ void zero_kernel(float* p, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0.f;
}

inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

constexpr size_t kMfmaSmem = (size_t)4 * TILE_ELEMS * sizeof(bf16_t);

// LDS above 64 KiB per workgroup must be requested explicitly (gfx950 has 160 KiB per CU).
template <typename F>
bool allow_big_lds(F* fn, size_t bytes) {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) == hipSuccess;
}

template <bool TA, bool TB>
int launch_mfma(const GemmArgs& g, int c_dtype, hipStream_t s) {
    const int tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
    static const bool ok_f = allow_big_lds(gemm_bf16_mfma<TA, TB, float>, kMfmaSmem);
    static const bool ok_b = allow_big_lds(gemm_bf16_mfma<TA, TB, bf16_t>, kMfmaSmem);
    if (!(c_dtype == GN_F32 ? ok_f : ok_b)) {
        set_error("gn_gemm: cannot reserve %zu B of LDS", kMfmaSmem);
        return GN_E_HIP;
    }
    if (c_dtype == GN_F32)
        hipLaunchKernelGGL((gemm_bf16_mfma<TA, TB, float>), dim3(tiles), dim3(256), kMfmaSmem, s, g);
    else
        hipLaunchKernelGGL((gemm_bf16_mfma<TA, TB, bf16_t>), dim3(tiles), dim3(256), kMfmaSmem, s, g);
    GN_LAUNCH_CHECK("gn_gemm (mfma)");
    return GN_OK;
}

template <typename TI, typename CT>
int launch_simt_t(const void* A0, const void* B0, int K0, const void* A1, const void* B1, int K1,
                  void* C, int M, int N, int ta, int tb, bool acc, hipStream_t s) {
    dim3 grid((N + 63) / 64, (M + 63) / 64);
#define GN_SIMT(TAV, TBV)                                                                     \
    gemm_simt<TI, CT, TAV, TBV><<<grid, 256, 0, s>>>((const TI*)A0, (const TI*)B0, K0,        \
                                                      (const TI*)A1, (const TI*)B1, K1, (CT*)C, \
                                                      M, N, acc ? 1 : 0)
    if (!ta && !tb) GN_SIMT(false, false);
    else if (!ta && tb) GN_SIMT(false, true);
    else if (ta && !tb) GN_SIMT(true, false);
    else GN_SIMT(true, true);
#undef GN_SIMT
    GN_LAUNCH_CHECK("gn_gemm (simt)");
    return GN_OK;
}

}  // namespace

// Internal entry shared by the linear / GLU handlers (no error clearing).
int gemm_dispatch(const void* A0, const void* B0, int K0, const void* A1, const void* B1, int K1,
                  void* C, int M, int N, int transA, int transB, int dtype, int c_dtype,
                  unsigned flags, hipStream_t s) {
    GN_REQUIRE(M >= 0 && N >= 0 && K0 >= 0 && K1 >= 0, "gn_gemm: negative size");
    if (M == 0 || N == 0) return GN_OK;
    GN_REQUIRE(C, "gn_gemm: null C");
    const bool acc = flags & GN_ACCUMULATE;
    const bool seg1 = A1 && B1 && K1 > 0;
    if (K0 + (seg1 ? K1 : 0) == 0) {
        if (acc) return GN_OK;
        GN_REQUIRE(c_dtype == GN_F32 || c_dtype == GN_BF16, "gn_gemm: bad c_dtype");
        hipError_t e = hipMemsetAsync(C, 0, (size_t)M * N * (c_dtype == GN_F32 ? 4 : 2), s);
        if (e != hipSuccess) { set_error("gn_gemm: memset failed"); return GN_E_HIP; }
        return GN_OK;
    }
    GN_REQUIRE(A0 && B0, "gn_gemm: null operand");
    if (dtype == GN_BF16) {
        GN_REQUIRE(c_dtype == GN_F32 || c_dtype == GN_BF16, "gn_gemm: c_dtype %d", c_dtype);
        const bool mfma_ok = (M % 8 == 0) && (N % 8 == 0) && (K0 % 8 == 0) &&
                             (!seg1 || K1 % 8 == 0) && al16(A0) && al16(B0) &&
                             (!seg1 || (al16(A1) && al16(B1)));
        if (mfma_ok) {
            GemmArgs g{};
            g.A[0] = (const bf16_t*)A0; g.B[0] = (const bf16_t*)B0; g.Ks[0] = K0;
            g.A[1] = (const bf16_t*)(seg1 ? A1 : A0); g.B[1] = (const bf16_t*)(seg1 ? B1 : B0);
            g.Ks[1] = seg1 ? K1 : 0;
            g.nseg = seg1 ? 2 : 1;
            g.C = C; g.M = M; g.N = N; g.accumulate = acc ? 1 : 0;
            if (!transA && !transB) return launch_mfma<false, false>(g, c_dtype, s);
            if (!transA && transB) return launch_mfma<false, true>(g, c_dtype, s);
            if (transA && !transB) return launch_mfma<true, false>(g, c_dtype, s);
            return launch_mfma<true, true>(g, c_dtype, s);
        }
        if (c_dtype == GN_F32)
            return launch_simt_t<bf16_t, float>(A0, B0, K0, seg1 ? A1 : nullptr, B1, K1, C, M, N,
                                                transA, transB, acc, s);
        return launch_simt_t<bf16_t, bf16_t>(A0, B0, K0, seg1 ? A1 : nullptr, B1, K1, C, M, N,
                                             transA, transB, acc, s);
    }
    if (dtype == GN_F32) {
        GN_REQUIRE(c_dtype == GN_F32, "gn_gemm: fp32 path writes fp32 C");
        return launch_simt_t<float, float>(A0, B0, K0, seg1 ? A1 : nullptr, B1, K1, C, M, N,
                                           transA, transB, acc, s);
    }
    set_error("gn_gemm: dtype %d not supported (f32, bf16)", dtype);
    return GN_E_INVALID;
}

int colsum_dispatch(const void* in, float* out, int M, int N, int dtype, unsigned flags,
                    hipStream_t s) {
    GN_REQUIRE(M >= 0 && N >= 0, "gn_colsum: negative size");
    if (N == 0) return GN_OK;
    GN_REQUIRE(in && out, "gn_colsum: null pointer");
    if (!(flags & GN_ACCUMULATE)) zero_kernel<<<(N + 255) / 256, 256, 0, s>>>(out, N);
    if (M == 0) { GN_LAUNCH_CHECK("gn_colsum"); return GN_OK; }
    // enough (column-block x row-split) work items to occupy the GPU
    const int cb = (N + 255) / 256;
    int splits = std::max(1, std::min(1024 / cb, (M + 63) / 64));
    if (M <= 4096 && cb >= 8) splits = 1;
    const int rows_per = (M + splits - 1) / splits;
    splits = (M + rows_per - 1) / rows_per;
    dim3 grid(cb, splits);
    if (dtype == GN_F32) colsum_kernel<float><<<grid, 256, 0, s>>>((const float*)in, out, M, N, rows_per);
    else if (dtype == GN_BF16) colsum_kernel<bf16_t><<<grid, 256, 0, s>>>((const bf16_t*)in, out, M, N, rows_per);
    else { set_error("gn_colsum: dtype %d", dtype); return GN_E_INVALID; }
    GN_LAUNCH_CHECK("gn_colsum");
    return GN_OK;
}

}  // namespace gn

using namespace gn;

extern "C" int gn_gemm(const void* A0, const void* B0, int K0, const void* A1, const void* B1,
                       int K1, void* C, int M, int N, int transA, int transB, int dtype,
                       int c_dtype, unsigned flags, void* stream) {
    clear_error();
    return gemm_dispatch(A0, B0, K0, A1, B1, K1, C, M, N, transA, transB, dtype, c_dtype, flags,
                         as_stream(stream));
}

extern "C" int gn_colsum(const void* in, float* out, int M, int N, int dtype, unsigned flags,
                         void* stream) {
    clear_error();
    return colsum_dispatch(in, out, M, N, dtype, flags, as_stream(stream));
}

// Linear backward (autograd.cpp:172-305): three stream-ordered launches, no host sync.
extern "C" int gn_linear_bwd(const void* dY, const void* X, const void* W, void* dX, void* dW,
                             void* db, int M, int N, int K, int dtype, unsigned flags,
                             void* stream) {
    clear_error();
    GN_REQUIRE(M >= 0 && N >= 0 && K >= 0, "gn_linear_bwd: negative size");
    GN_REQUIRE(dY && X && W && dW, "gn_linear_bwd: null pointer (dY, X, W, dW are required)");
    GN_REQUIRE(dtype == GN_F32 || dtype == GN_BF16, "gn_linear_bwd: dtype %d", dtype);
    hipStream_t s = as_stream(stream);
    int rc;
    if (dX) {  // dX[M x K] = dY[M x N] . W[N x K]
        rc = gemm_dispatch(dY, W, N, nullptr, nullptr, 0, dX, M, K, 0, 0, dtype, dtype, flags, s);
        if (rc) return rc;
    }
    // dW[N x K] = dY^T . X  (A = dY stored [M x N] = [Ks x Mout], transposed)
    rc = gemm_dispatch(dY, X, M, nullptr, nullptr, 0, dW, N, K, 1, 0, dtype, GN_F32, flags, s);
    if (rc) return rc;
    if (db) return colsum_dispatch(dY, (float*)db, M, N, dtype, flags, s);
    return GN_OK;
}

extern "C" int gn_glu_linear_bwd(int kind, const void* dO, const void* gate, const void* up,
                                 const void* X, const void* Wg, const void* Wu, void* dX,
                                 void* dWg, void* dWu, void* dbg, void* dbu, void* gu_ws, int M,
                                 int K, int H, int dtype, unsigned flags, void* stream) {
    clear_error();
    GN_REQUIRE(M >= 0 && K >= 0 && H >= 0, "gn_glu_linear_bwd: negative size");
    GN_REQUIRE(dO && gate && up && X && Wg && Wu && dWg && dWu && gu_ws,
               "gn_glu_linear_bwd: null pointer");
    GN_REQUIRE(dtype == GN_F32 || dtype == GN_BF16, "gn_glu_linear_bwd: dtype %d", dtype);
    hipStream_t s = as_stream(stream);
    const size_t esz = dtype == GN_F32 ? 4 : 2;
    void* dG = gu_ws;
    void* dU = (char*)gu_ws + (size_t)M * H * esz;
    int rc = gn_glu_bwd(kind, dO, gate, up, dG, dU, (int64_t)M * H, dtype, stream);
    if (rc) return rc;
    if (dX) {  // dX = dG Wg + dU Wu : one GEMM over the concatenated K = 2H
        rc = gemm_dispatch(dG, Wg, H, dU, Wu, H, dX, M, K, 0, 0, dtype, dtype, flags, s);
        if (rc) return rc;
    }
    rc = gemm_dispatch(dG, X, M, nullptr, nullptr, 0, dWg, H, K, 1, 0, dtype, GN_F32, flags, s);
    if (rc) return rc;
    rc = gemm_dispatch(dU, X, M, nullptr, nullptr, 0, dWu, H, K, 1, 0, dtype, GN_F32, flags, s);
    if (rc) return rc;
    if (dbg && (rc = colsum_dispatch(dG, (float*)dbg, M, H, dtype, flags, s))) return rc;
    if (dbu && (rc = colsum_dispatch(dU, (float*)dbu, M, H, dtype, flags, s))) return rc;
    return GN_OK;
}
