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
#include "gn_gemm_dma.h"
#include "gn_lane.h"

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

template <bool TA, bool TB, typename CT, int EPI>
__global__ __launch_bounds__(256, 2) void gemm_bf16_mfma(GemmDesc g) {
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
        // A: TA=0 -> A[m*lda + k] (k contiguous); TA=1 -> A[k*lda + m]
        if (!TA) load_tile<true>(g.A[s], g.lda[s], m0, g.M, k0, Ks, ra);
        else load_tile<false>(g.A[s], g.lda[s], m0, g.M, k0, Ks, ra);
        // B: TB=1 -> B[n*ldb + k] (k contiguous); TB=0 -> B[k*ldb + n]
        if (TB) load_tile<true>(g.B[s], g.ldb[s], n0, g.N, k0, Ks, rb);
        else load_tile<false>(g.B[s], g.ldb[s], n0, g.N, k0, Ks, rb);
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
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
            gemm_store_tile<CT, EPI>(g, m0 + wm * 64 + i * 32, n0 + wn * 64 + j * 32, acc[i][j]);
}

// ---- SIMT fallback: 64x64 tile, BK 16, 4x4 outputs per thread (any shape, f32 or bf16) ----
template <typename TI, typename CT, bool TA, bool TB, int EPI>
__global__ __launch_bounds__(256) void gemm_simt(GemmDesc g) {
    __shared__ float sA[16][64 + 4];
    __shared__ float sB[16][64 + 4];
    const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    float acc[4][4] = {};
    for (int s = 0; s < g.nseg; ++s) {
        const TI* A = reinterpret_cast<const TI*>(g.A[s]);
        const TI* B = reinterpret_cast<const TI*>(g.B[s]);
        const int Ks = g.Ks[s], lda = g.lda[s], ldb = g.ldb[s];
        for (int k0 = 0; k0 < Ks; k0 += 16) {
            for (int e = threadIdx.x; e < 16 * 64; e += 256) {
                const int kk = e / 64, mm = e % 64;
                const int m = m0 + mm, k = k0 + kk;
                float va = 0.f;
                if (m < g.M && k < Ks) va = TA ? io<TI>::ld(A, (size_t)k * lda + m) : io<TI>::ld(A, (size_t)m * lda + k);
                sA[kk][mm] = va;
                const int n = n0 + mm;
                float vb = 0.f;
                if (n < g.N && k < Ks) vb = TB ? io<TI>::ld(B, (size_t)n * ldb + k) : io<TI>::ld(B, (size_t)k * ldb + n);
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
            if (m < g.M && n < g.N) gemm_store<CT, EPI>(g, m, n, acc[i][j]);
        }
}

// ---- small products: one thread per output, the whole k loop in registers ---------------
// For products whose tiles would leave the GPU nearly idle (an MLP layer of a few hundred
// units over a batch of 64, the 10-wide output layer): every load of the k loop is issued
// without a barrier or an LDS round trip, so the kernel costs about one memory latency.
// Sequential k order per output (deterministic); fp32 FMA, so fp32 operands get full fp32
// precision.
constexpr int kSmallMaxK = 128;
constexpr int64_t kSmallMaxMac = (int64_t)1 << 24;

template <typename TI, typename CT, bool TA, bool TB>
__global__ __launch_bounds__(256) void gemm_small(GemmDesc g) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)g.M * g.N) return;
    const int m = (int)(idx / g.N), n = (int)(idx % g.N);
    float acc = 0.f;
    for (int s = 0; s < g.nseg; ++s) {
        const TI* A = reinterpret_cast<const TI*>(g.A[s]);
        const TI* B = reinterpret_cast<const TI*>(g.B[s]);
        const int Ks = g.Ks[s], lda = g.lda[s], ldb = g.ldb[s];
#pragma unroll 16
        for (int k = 0; k < Ks; ++k) {
            const float a = TA ? io<TI>::ld(A, (size_t)k * lda + m) : io<TI>::ld(A, (size_t)m * lda + k);
            const float b = TB ? io<TI>::ld(B, (size_t)n * ldb + k) : io<TI>::ld(B, (size_t)k * ldb + n);
            acc = fmaf(a, b, acc);
        }
    }
    gemm_store<CT, 0>(g, m, n, acc);
}

inline bool small_applicable(const GemmDesc& d) {
    const int64_t K = (int64_t)d.Ks[0] + (d.nseg > 1 ? d.Ks[1] : 0);
    return d.epi == 0 && !d.bias && !d.cbias && d.ksplit <= 1 && K <= kSmallMaxK &&
           (int64_t)d.M * d.N * K <= kSmallMaxMac;
}

template <typename TI, typename CT>
int launch_small(const GemmDesc& g, int ta, int tb, hipStream_t s) {
    const unsigned grid = (unsigned)(((int64_t)g.M * g.N + 255) / 256);
    if (!ta && !tb) gemm_small<TI, CT, false, false><<<grid, 256, 0, s>>>(g);
    else if (!ta && tb) gemm_small<TI, CT, false, true><<<grid, 256, 0, s>>>(g);
    else if (ta && !tb) gemm_small<TI, CT, true, false><<<grid, 256, 0, s>>>(g);
    else gemm_small<TI, CT, true, true><<<grid, 256, 0, s>>>(g);
    GN_LAUNCH_CHECK("gemm (small)");
    return GN_OK;
}

// ---- small fp32 Linear backward in one launch -------------------------------------------
// dX = dY W, dW = dY^T X and db = column sums of dY for an fp32 Linear whose two products
// gemm_small takes (an MLP layer over a batch of <= 128 rows): block ranges pick the output.
// A dX or dW element runs gemm_small's sequential k loop, and a db column follows
// colsum_small's order (16 interleaved row subsets summed from zero, then added in subset
// order), so the results are bit-identical to the three launches this replaces.
struct SmallLinearBwd {
    const float* dY;  // [M x N]
    const float* X;   // [M x K]
    const float* W;   // [N x K]
    float *dX, *dW, *db;
    int M, N, K, accumulate;
    int bx, bw;  // blocks of the dX range, of the dW range (db follows)
};

__global__ __launch_bounds__(256) void linear_bwd_small(SmallLinearBwd p) {
    const int b = blockIdx.x;
    if (b < p.bx) {  // dX[m][k] = sum_n dY[m][n] W[n][k]
        const int64_t idx = (int64_t)b * 256 + threadIdx.x;
        if (idx >= (int64_t)p.M * p.K) return;
        const int m = (int)(idx / p.K), k = (int)(idx % p.K);
        float a = 0.f;
#pragma unroll 16
        for (int n = 0; n < p.N; ++n) a = fmaf(p.dY[(size_t)m * p.N + n], p.W[(size_t)n * p.K + k], a);
        p.dX[idx] = p.accumulate ? a + p.dX[idx] : a;
        return;
    }
    if (b < p.bx + p.bw) {  // dW[n][k] = sum_m dY[m][n] X[m][k]
        const int64_t idx = (int64_t)(b - p.bx) * 256 + threadIdx.x;
        if (idx >= (int64_t)p.N * p.K) return;
        const int n = (int)(idx / p.K), k = (int)(idx % p.K);
        float a = 0.f;
#pragma unroll 16
        for (int m = 0; m < p.M; ++m) a = fmaf(p.dY[(size_t)m * p.N + n], p.X[(size_t)m * p.K + k], a);
        p.dW[idx] = p.accumulate ? a + p.dW[idx] : a;
        return;
    }
    // db[n] = sum_m dY[m][n]: 16 columns per block, thread (j, c) sums rows j, j + 16, ...
    // of column c (its <= 8 loads issued together), then thread j = 0 adds the 16 subsets in
    // order
    __shared__ float sh[16][17];
    const int c = threadIdx.x & 15, j = threadIdx.x >> 4;
    const int n = (b - p.bx - p.bw) * 16 + c;
    float v[kSmallMaxK / 16];
#pragma unroll
    for (int i = 0; i < kSmallMaxK / 16; ++i) {
        const int r = j + 16 * i;
        v[i] = (n < p.N && r < p.M) ? p.dY[(size_t)r * p.N + n] : 0.f;
    }
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kSmallMaxK / 16; ++i)
        if (j + 16 * i < p.M) s += v[i];
    sh[j][c] = s;
    __syncthreads();
    if (j == 0 && n < p.N) {
        float t = sh[0][c];
#pragma unroll
        for (int w = 1; w < 16; ++w) t += sh[w][c];
        p.db[n] = p.accumulate ? p.db[n] + t : t;
    }
}

// ---- column sums over few rows: one pass, deterministic ---------------------------------
// Block: 16 waves x 64 columns (lane = column); wave w adds rows w, w + 16, ... (all of its
// loads issued together), the waves' sums are added in a fixed order.  No clear, no second
// launch.
constexpr int kColsumSmallRows = 1024;

template <typename TI>
__global__ __launch_bounds__(1024) void colsum_small(const TI* __restrict__ in, float* __restrict__ out,
                                                     int M, int N, int ld, int accumulate) {
    __shared__ float sh[16][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = blockIdx.x * 64 + lane;
    float s = 0.f;
    if (n < N) {
#pragma unroll 8
        for (int r = wave; r < M; r += 16) s += io<TI>::ld(in, (size_t)r * ld + n);
    }
    sh[wave][lane] = s;
    __syncthreads();
    if (wave == 0 && n < N) {
        float t = sh[0][lane];
#pragma unroll
        for (int w = 1; w < 16; ++w) t += sh[w][lane];
        out[n] = accumulate ? out[n] + t : t;
    }
}

// colsum_small's sums (wave w adds rows w, w + 16, ... from zero; the 16 wave sums are added in
// wave order) for four adjacent columns per lane: 16-byte (fp32) or 8-byte (bf16) loads, for
// N and ld multiples of 4 and aligned rows.  Bit-identical to colsum_small.
template <typename TI>
__device__ __forceinline__ float4 ld_col4(const TI* p);
template <>
__device__ __forceinline__ float4 ld_col4<float>(const float* p) {
    return *reinterpret_cast<const float4*>(p);
}
template <>
__device__ __forceinline__ float4 ld_col4<bf16_t>(const bf16_t* p) {
    const uint2 w = *reinterpret_cast<const uint2*>(p);
    return make_float4(__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u),
                       __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xffff0000u));
}

template <typename TI>
__global__ __launch_bounds__(1024) void colsum_small4(const TI* __restrict__ in,
                                                      float* __restrict__ out, int M, int N,
                                                      int ld, int accumulate) {
    __shared__ float4 sh[16][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = (blockIdx.x * 64 + lane) * 4;
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    if (n < N) {
#pragma unroll 8
        for (int r = wave; r < M; r += 16) {
            const float4 v = ld_col4<TI>(in + (size_t)r * ld + n);
            s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
        }
    }
    sh[wave][lane] = s;
    __syncthreads();
    if (wave == 0 && n < N) {
        float4 t = sh[0][lane];
#pragma unroll
        for (int w = 1; w < 16; ++w) {
            const float4 u = sh[w][lane];
            t.x += u.x; t.y += u.y; t.z += u.z; t.w += u.w;
        }
        float4* o = reinterpret_cast<float4*>(out + n);
        if (accumulate) {
            const float4 p = *o;
            t = make_float4(p.x + t.x, p.y + t.y, p.z + t.z, p.w + t.w);
        }
        *o = t;
    }
}

// ---- column sums (db): thread per column, rows split over grid.y with fp32 atomics ------
template <typename TI>
__global__ __launch_bounds__(256) void colsum_kernel(const TI* __restrict__ in, float* out,
                                                     int M, int N, int ld, int rows_per) {
    const int n = blockIdx.x * 256 + threadIdx.x;
    if (n >= N) return;
    const int r0 = blockIdx.y * rows_per, r1 = min(M, r0 + rows_per);
    float s = 0.f;
    for (int r = r0; r < r1; ++r) s += io<TI>::ld(in, (size_t)r * ld + n);
    if (gridDim.y == 1) out[n] += s;
    else atomicAdd(out + n, s);
}

// Deterministic two-pass column sums through a scratch array of R partial rows:
//   pass 1 (grid: 512-column strips x R row ranges, 4 waves): lane l adds 8 consecutive
//           columns over its wave's rows, the 4 waves combine in LDS in a fixed order;
//   pass 2: out[n] (+)= sum_r part[r][n], r in order.
template <typename TI>
__global__ __launch_bounds__(256) void colsum_part(const TI* __restrict__ in, float* __restrict__ part,
                                                   int M, int N, int ld, int rows_per) {
    __shared__ float sh[4][512];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c0 = blockIdx.x * 512 + 8 * lane;
    const int r0 = blockIdx.y * rows_per, r1 = min(M, r0 + rows_per);
    float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (c0 < N) {
#pragma unroll 4
        for (int r = r0 + wave; r < r1; r += 4) {
            const TI* p = in + (size_t)r * ld + c0;
            if constexpr (sizeof(TI) == 2) {
                const uint4 v = *reinterpret_cast<const uint4*>(p);
                const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    s[2 * e] += __uint_as_float(w[e] << 16);
                    s[2 * e + 1] += __uint_as_float(w[e] & 0xffff0000u);
                }
            } else {
                const float4 a = reinterpret_cast<const float4*>(p)[0];
                const float4 b = reinterpret_cast<const float4*>(p)[1];
                s[0] += a.x; s[1] += a.y; s[2] += a.z; s[3] += a.w;
                s[4] += b.x; s[5] += b.y; s[6] += b.z; s[7] += b.w;
            }
        }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) sh[wave][8 * lane + e] = s[e];
    __syncthreads();
    for (int i = threadIdx.x; i < 512; i += 256) {
        const int c = blockIdx.x * 512 + i;
        if (c < N) part[(size_t)blockIdx.y * N + c] = ((sh[0][i] + sh[1][i]) + sh[2][i]) + sh[3][i];
    }
}

// 64 columns x 16 row groups per block; the groups combine in LDS in a fixed order
__global__ __launch_bounds__(1024) void colsum_finish(const float* __restrict__ part, int R, int N,
                                                      float* __restrict__ out, int accumulate) {
    __shared__ float sh[16][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int n = blockIdx.x * 64 + lane;
    float s = 0.f;
    if (n < N)
        for (int r = w; r < R; r += 16) s += part[(size_t)r * N + n];
    sh[w][lane] = s;
    __syncthreads();
    if (w == 0 && n < N) {
        float t = sh[0][lane];
#pragma unroll
        for (int i = 1; i < 16; ++i) t += sh[i][lane];
        out[n] = accumulate ? out[n] + t : t;
    }
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

template <bool TA, bool TB, typename CT, int EPI>
int launch_mfma_t(const GemmDesc& g, hipStream_t s) {
    static const bool ok = allow_big_lds(gemm_bf16_mfma<TA, TB, CT, EPI>, kMfmaSmem);
    if (!ok) {
        set_error("gn_gemm: cannot reserve %zu B of LDS", kMfmaSmem);
        return GN_E_HIP;
    }
    const int tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
    hipLaunchKernelGGL((gemm_bf16_mfma<TA, TB, CT, EPI>), dim3(tiles), dim3(256), kMfmaSmem, s, g);
    GN_LAUNCH_CHECK("gn_gemm (mfma)");
    return GN_OK;
}

template <typename CT, int EPI>
int launch_mfma(const GemmDesc& g, int ta, int tb, hipStream_t s) {
    if (!ta && !tb) return launch_mfma_t<false, false, CT, EPI>(g, s);
    if (!ta && tb) return launch_mfma_t<false, true, CT, EPI>(g, s);
    if (ta && !tb) return launch_mfma_t<true, false, CT, EPI>(g, s);
    return launch_mfma_t<true, true, CT, EPI>(g, s);
}

template <typename TI, typename CT, int EPI>
int launch_simt(const GemmDesc& g, int ta, int tb, hipStream_t s) {
    dim3 grid((g.N + 63) / 64, (g.M + 63) / 64);
    if (!ta && !tb) gemm_simt<TI, CT, false, false, EPI><<<grid, 256, 0, s>>>(g);
    else if (!ta && tb) gemm_simt<TI, CT, false, true, EPI><<<grid, 256, 0, s>>>(g);
    else if (ta && !tb) gemm_simt<TI, CT, true, false, EPI><<<grid, 256, 0, s>>>(g);
    else gemm_simt<TI, CT, true, true, EPI><<<grid, 256, 0, s>>>(g);
    GN_LAUNCH_CHECK("gn_gemm (simt)");
    return GN_OK;
}

bool mfma_applicable(const GemmDesc& g) {
    if (g.M % 8 || g.N % 8) return false;
    for (int s = 0; s < g.nseg; ++s)
        if (g.Ks[s] % 8 || !al16(g.A[s]) || !al16(g.B[s]) || g.lda[s] % 8 || g.ldb[s] % 8) return false;
    return true;
}

}  // namespace

int gemm_run(const GemmDesc& d, int transA, int transB, int dtype, int c_dtype, hipStream_t s) {
    if (d.M == 0 || d.N == 0) return GN_OK;
    if (d.bias && !(dtype == GN_BF16 && c_dtype == GN_F32 && d.epi == 0 && gemm_dma_applicable(d))) {
        set_error("gemm: fused row sums need the LDS-DMA core (bf16 operands, fp32 C)");
        return GN_E_INVALID;
    }
    if (d.cbias && !(dtype == GN_BF16 && d.epi == 0 && gemm_dma_applicable(d))) {
        set_error("gemm: the fused column bias needs the LDS-DMA core (bf16 operands)");
        return GN_E_INVALID;
    }
    if (dtype == GN_BF16) {
        if (gemm_dma_applicable(d)) return gemm_dma_launch(d, transA, transB, c_dtype, s);
        if (mfma_applicable(d)) {
            if (d.epi == 1) return launch_mfma<bf16_t, 1>(d, transA, transB, s);
            if (c_dtype == GN_F32) return launch_mfma<float, 0>(d, transA, transB, s);
            return launch_mfma<bf16_t, 0>(d, transA, transB, s);
        }
        if (d.epi == 1) return launch_simt<bf16_t, bf16_t, 1>(d, transA, transB, s);
        if (c_dtype == GN_F32) return launch_simt<bf16_t, float, 0>(d, transA, transB, s);
        return launch_simt<bf16_t, bf16_t, 0>(d, transA, transB, s);
    }
    if (dtype == GN_F32) {
        if (d.epi == 1) {
            set_error("gemm: the GLU epilogue needs bf16 operands");
            return GN_E_INVALID;
        }
        if (small_applicable(d)) return launch_small<float, float>(d, transA, transB, s);
        if (gemm_f32_applicable(d)) return gemm_f32_launch(d, transA, transB, s);
        return launch_simt<float, float, 0>(d, transA, transB, s);
    }
    set_error("gn_gemm: dtype %d not supported (f32, bf16)", dtype);
    return GN_E_INVALID;
}

int colsum_dispatch(const void* in, float* out, int M, int N, int dtype, unsigned flags,
                    hipStream_t s, int ld, float* scratch, size_t scratch_floats);

// Weight gradient dW[N x Kin] (+)= dY^T X over M rows (dY [M x N] row pitch ldy, X [M x Kin]
// pitch ldx), rows of dW below Msplit to dW, the rest to dW2 (row - Msplit), and the bias
// gradient db = column sums of dY (db for rows < Msplit, db2 beyond) when db != nullptr.
// The bias rides on the GEMM (row sums of its A fragments) when the LDS-DMA core takes the
// shape; otherwise a two-pass column sum runs first, staged in dW (which the GEMM then
// overwrites) unless accumulating.
int weight_grad(const void* dY, int ldy, const void* X, int ldx, int M, int N, int Kin, void* dW,
                void* dW2, int Msplit, float* db, float* db2, int dtype, unsigned flags,
                hipStream_t s, void* ws = nullptr, size_t ws_bytes = 0) {
    GemmDesc d{};
    // split-K partial planes need 16-byte aligned storage; a misaligned workspace is unused
    if (ws && (reinterpret_cast<uintptr_t>(ws) & 15u) == 0) {
        d.part = (float*)ws;
        d.part_cap = ws_bytes;
    }
    d.nseg = 1;
    d.A[0] = (const bf16_t*)dY; d.lda[0] = ldy; d.Ks[0] = M;
    d.B[0] = (const bf16_t*)X; d.ldb[0] = ldx;
    d.M = N; d.N = Kin; d.C = dW; d.C2 = dW2; d.Msplit = Msplit; d.ldc = Kin;
    d.accumulate = (flags & GN_ACCUMULATE) ? 1 : 0;
    if (M == 0 || N == 0 || Kin == 0) {
        if (M == 0 && !d.accumulate && N > 0 && Kin > 0) {
            // no rows: the gradients are zero
            hipError_t e = launch_zero(dW, (size_t)std::min(N, Msplit) * Kin * 4, s);
            if (e == hipSuccess && N > Msplit) e = launch_zero(dW2, (size_t)(N - Msplit) * Kin * 4, s);
            if (e == hipSuccess && db) e = launch_zero(db, (size_t)std::min(N, Msplit) * 4, s);
            if (e == hipSuccess && db2 && N > Msplit) e = launch_zero(db2, (size_t)(N - Msplit) * 4, s);
            if (e != hipSuccess) { set_error("weight gradient: clear failed"); return GN_E_HIP; }
        }
        return GN_OK;
    }
    // The fused row sums make the GEMM ~25 % slower (dot2 on the MFMA pipe), yet measured
    // end to end (12-layer decoder, one box, interleaved runs) fusing every bias beat both the
    // two-pass column sum everywhere (9.73 vs 10.01 ms per step) and fusing only GEMMs under
    // 48 us (9.94 ms): the two extra launches per bias cost more than their kernel time.
    if (db && dtype == GN_BF16 && gemm_dma_applicable(d)) {
        d.bias = db;
        d.bias2 = db2 ? db2 : db + Msplit;
        return gemm_dma_launch(d, 1, 0, GN_F32, s);
    }
    int rc;
    const bool acc = flags & GN_ACCUMULATE;
    const char* dy = (const char*)dY;
    const size_t esz = dtype == GN_F32 ? 4 : 2;
    if (db) {
        const int n1 = std::min(N, Msplit);
        if ((rc = colsum_dispatch(dy, db, M, n1, dtype, flags, s, ldy, acc ? nullptr : (float*)dW,
                                  (size_t)n1 * Kin)))
            return rc;
        if (N > Msplit &&
            (rc = colsum_dispatch(dy + (size_t)Msplit * esz, db2 ? db2 : db + Msplit, M, N - Msplit,
                                  dtype, flags, s, ldy, acc ? nullptr : (float*)dW,
                                  (size_t)n1 * Kin)))
            return rc;
    }
    return gemm_run(d, 1, 0, dtype, GN_F32, s);
}

// Workspace bytes for the split-K partials of weight_grad's GEMM (dW [N x Kin] over M rows),
// as the launch would choose them with an unbounded workspace: the largest over the four
// launches a caller can make (with or without a bias, overwrite or GN_ACCUMULATE; an
// accumulating launch cannot take the two-way atomic split and may want planes instead).
size_t weight_grad_ws_bytes(int M, int N, int Kin, int dtype) {
    if (dtype != GN_BF16 || M <= 0 || N <= 0 || Kin <= 0) return 0;
    const bf16_t* al = reinterpret_cast<const bf16_t*>((uintptr_t)256);  // aligned stand-in
    float* alf = reinterpret_cast<float*>((uintptr_t)256);
    size_t best = 0;
    for (int has_bias = 0; has_bias < 2; ++has_bias)
        for (int acc = 0; acc < 2; ++acc) {
            GemmDesc d{};
            d.nseg = 1;
            d.A[0] = al; d.lda[0] = N; d.Ks[0] = M;
            d.B[0] = al; d.ldb[0] = Kin;
            d.M = N; d.N = Kin; d.C = alf; d.C2 = alf; d.Msplit = N; d.ldc = Kin;
            d.bias = has_bias ? alf : nullptr;
            d.bias2 = has_bias ? alf : nullptr;
            d.accumulate = acc;
            if (!gemm_dma_applicable(d)) continue;
            best = std::max(best, gemm_dma_part_bytes(d, 1, GN_F32));
        }
    return best;
}

// Plain-argument form used by the C entry points.
// ws: split-K partial planes of the fp32 path (may be NULL / short: the split is then
// limited to what fits).
int gemm_dispatch(const void* A0, const void* B0, int K0, const void* A1, const void* B1, int K1,
                  void* C, int M, int N, int transA, int transB, int dtype, int c_dtype,
                  unsigned flags, hipStream_t s, void* ws = nullptr, size_t ws_bytes = 0) {
    GN_REQUIRE(M >= 0 && N >= 0 && K0 >= 0 && K1 >= 0, "gn_gemm: negative size");
    if (M == 0 || N == 0) return GN_OK;
    GN_REQUIRE(C, "gn_gemm: null C");
    GN_REQUIRE(c_dtype == GN_F32 || c_dtype == GN_BF16, "gn_gemm: c_dtype %d", c_dtype);
    GN_REQUIRE(dtype == GN_BF16 || c_dtype == GN_F32, "gn_gemm: fp32 path writes fp32 C");
    const bool acc = flags & GN_ACCUMULATE;
    const bool seg1 = A1 && B1 && K1 > 0;
    if (K0 + (seg1 ? K1 : 0) == 0) {
        if (acc) return GN_OK;
        hipError_t e = launch_zero(C, (size_t)M * N * (c_dtype == GN_F32 ? 4 : 2), s);
        if (e != hipSuccess) { set_error("gn_gemm: clear failed"); return GN_E_HIP; }
        return GN_OK;
    }
    GN_REQUIRE(A0 && B0, "gn_gemm: null operand");
    GemmDesc d{};
    d.A[0] = (const bf16_t*)A0; d.B[0] = (const bf16_t*)B0; d.Ks[0] = K0;
    d.lda[0] = transA ? M : K0; d.ldb[0] = transB ? K0 : N;
    d.nseg = seg1 ? 2 : 1;
    if (seg1) {
        d.A[1] = (const bf16_t*)A1; d.B[1] = (const bf16_t*)B1; d.Ks[1] = K1;
        d.lda[1] = transA ? M : K1; d.ldb[1] = transB ? K1 : N;
    }
    d.M = M; d.N = N; d.C = C; d.C2 = C; d.Msplit = M; d.ldc = N;
    d.accumulate = acc ? 1 : 0;
    if (ws && al16(ws)) {
        d.part = (float*)ws;
        d.part_cap = ws_bytes;
    }
    return gemm_run(d, transA, transB, dtype, c_dtype, s);
}

// Split-K workspace bytes of the fp32 Linear backward's two GEMMs (dX = dY W over N,
// dW = dY^T X over M rows) on the six-product bf16 MFMA path: the larger of the two (they run
// one after the other on the stream and share it).
static size_t linear_f32_ws_bytes(int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    const bf16_t* al = reinterpret_cast<const bf16_t*>((uintptr_t)256);  // aligned stand-in
    float* alf = reinterpret_cast<float*>((uintptr_t)256);
    GemmDesc x{};
    x.nseg = 1;
    x.A[0] = al; x.lda[0] = N; x.Ks[0] = N;
    x.B[0] = al; x.ldb[0] = K;
    x.M = M; x.N = K; x.C = alf; x.C2 = alf; x.Msplit = M; x.ldc = K;
    GemmDesc w = x;
    w.A[0] = al; w.lda[0] = N; w.Ks[0] = M;
    w.B[0] = al; w.ldb[0] = K;
    w.M = N; w.N = K; w.Msplit = N; w.ldc = K;
    size_t b = 0;
    if (gemm_f32_applicable(x)) b = std::max(b, gemm_f32_part_bytes(x));
    if (gemm_f32_applicable(w)) b = std::max(b, gemm_f32_part_bytes(w));
    return b;
}

int colsum_dispatch(const void* in, float* out, int M, int N, int dtype, unsigned flags,
                    hipStream_t s, int ld, float* scratch, size_t scratch_floats) {
    if (ld <= 0) ld = N;
    GN_REQUIRE(M >= 0 && N >= 0, "gn_colsum: negative size");
    if (N == 0) return GN_OK;
    GN_REQUIRE(in && out, "gn_colsum: null pointer");
    const size_t es = dtype == GN_F32 ? 4 : 2;
    if (M > 0 && M <= kColsumSmallRows && (dtype == GN_F32 || dtype == GN_BF16)) {
        const int acc = (flags & GN_ACCUMULATE) ? 1 : 0;
        const size_t row_b = (size_t)ld * es;
        if (N % 4 == 0 && row_b % (4 * es) == 0 && al16(out) &&
            (reinterpret_cast<uintptr_t>(in) & (4 * es - 1)) == 0) {
            const unsigned g = (unsigned)((N / 4 + 63) / 64);
            if (dtype == GN_F32)
                colsum_small4<float><<<g, 1024, 0, s>>>((const float*)in, out, M, N, ld, acc);
            else
                colsum_small4<bf16_t><<<g, 1024, 0, s>>>((const bf16_t*)in, out, M, N, ld, acc);
        } else {
            const unsigned g = (unsigned)((N + 63) / 64);
            if (dtype == GN_F32) colsum_small<float><<<g, 1024, 0, s>>>((const float*)in, out, M, N, ld, acc);
            else colsum_small<bf16_t><<<g, 1024, 0, s>>>((const bf16_t*)in, out, M, N, ld, acc);
        }
        GN_LAUNCH_CHECK("gn_colsum (few rows)");
        return GN_OK;
    }
    const bool vec = N % 8 == 0 && ld % 8 == 0 && al16(in) && (dtype == GN_F32 || dtype == GN_BF16);
    if (scratch && vec && M > 0 && scratch_floats >= (size_t)N) {
        const int cb = (N + 511) / 512;
        int R = std::max(1, std::min({(M + 31) / 32, 512 / cb, (int)std::min<size_t>(scratch_floats / N, 4096)}));
        const int rows_per = (M + R - 1) / R;
        R = (M + rows_per - 1) / rows_per;
        if (dtype == GN_F32)
            colsum_part<float><<<dim3(cb, R), 256, 0, s>>>((const float*)in, scratch, M, N, ld, rows_per);
        else
            colsum_part<bf16_t><<<dim3(cb, R), 256, 0, s>>>((const bf16_t*)in, scratch, M, N, ld, rows_per);
        colsum_finish<<<(N + 63) / 64, 1024, 0, s>>>(scratch, R, N, out, (flags & GN_ACCUMULATE) ? 1 : 0);
        GN_LAUNCH_CHECK("gn_colsum (two-pass)");
        return GN_OK;
    }
    (void)es;
    if (!(flags & GN_ACCUMULATE)) zero_kernel<<<(N + 255) / 256, 256, 0, s>>>(out, N);
    if (M == 0) { GN_LAUNCH_CHECK("gn_colsum"); return GN_OK; }
    // enough (column-block x row-split) work items to occupy the GPU
    const int cb = (N + 255) / 256;
    int splits = std::max(1, std::min(1024 / cb, (M + 63) / 64));
    if (M <= 4096 && cb >= 8) splits = 1;
    const int rows_per = (M + splits - 1) / splits;
    splits = (M + rows_per - 1) / rows_per;
    dim3 grid(cb, splits);
    if (dtype == GN_F32) colsum_kernel<float><<<grid, 256, 0, s>>>((const float*)in, out, M, N, ld, rows_per);
    else if (dtype == GN_BF16) colsum_kernel<bf16_t><<<grid, 256, 0, s>>>((const bf16_t*)in, out, M, N, ld, rows_per);
    else { set_error("gn_colsum: dtype %d", dtype); return GN_E_INVALID; }
    GN_LAUNCH_CHECK("gn_colsum");
    return GN_OK;
}

// An fp32 Linear backward whose products gemm_small takes (batch <= kSmallMaxK rows, dX's
// k loop over the N outputs <= kSmallMaxK, each product <= kSmallMaxMac multiply-adds) runs
// as one launch of linear_bwd_small: same results as the dX GEMM, the db column sums and
// the dW GEMM launched one after another, a third of the launches.
bool small_linear_applicable(int M, int N, int K, bool with_dx) {
    if (M < 1 || N < 1 || K < 1 || M > kSmallMaxK) return false;
    if ((int64_t)N * K * M > kSmallMaxMac) return false;
    return !with_dx || (N <= kSmallMaxK && (int64_t)M * K * N <= kSmallMaxMac);
}

int small_linear_launch(const float* dY, const float* X, const float* W, float* dX, float* dW,
                        float* db, int M, int N, int K, bool acc, hipStream_t s) {
    SmallLinearBwd p{dY, X, W, dX, dW, db, M, N, K, acc ? 1 : 0, 0, 0};
    p.bx = dX ? (int)(((int64_t)M * K + 255) / 256) : 0;
    p.bw = (int)(((int64_t)N * K + 255) / 256);
    const int bb = db ? (N + 15) / 16 : 0;
    linear_bwd_small<<<p.bx + p.bw + bb, 256, 0, s>>>(p);
    GN_LAUNCH_CHECK("linear backward (small, one launch)");
    return GN_OK;
}

// Whether a call's input-gradient product runs beside its weight-gradient product (on the
// device's side stream, gn_lane.h), both on the LDS-DMA core (bf16).  The weight gradient is
// issued first, on the caller's stream: its grid takes the compute units it needs and the
// input gradient's blocks fill the rest, which pays where a grid leaves part of the GPU idle
// in its last round (the decoder's 192-tile input gradients, the FFN's 176-tile dWd).  The
// two outputs do not alias and each product's k order is unchanged, so the results are
// those of the two products run one after the other.
// Measured on the C5 decoder (12 layers, eager step / graph replay, ms): no fork 9.07 / 9.07;
// fork from 2 GFLOP per product 9.06 / 8.64; from 50 GFLOP 8.97-8.99 / 8.82.  Eagerly, each
// fork/join costs ~40 us of host time (two event records, two cross-stream waits) and
// cross-queue latency on the GPU that the smaller pairs do not win back; a captured graph
// pays the host part once.  Hence: forked from kSideBySideFlop under capture, from
// kSideBySideEagerFlop otherwise.
// Only where one of the two grids is under one round: two grids that each fill the GPU (the
// FFN's dN, 256 tiles, beside its [dWg;dWu], 704) gain nothing from sharing it, and the
// long blocks of the second one then start late (measured 0.363 -> 0.40 ms for that pair).
// Grid sizes are estimated on the usual tiles: 256 x 128 for the bf16 input gradient,
// 256 x 256 for the fp32 weight gradient.
constexpr double kSideBySideFlop = 2.0e9;
constexpr double kSideBySideEagerFlop = 5.0e10;

inline long grid_est(long rows, long cols, int bm, int bn) {
    return ((rows + bm - 1) / bm) * ((cols + bn - 1) / bn);
}

// dx: the input gradient's output [xr x xc]; dw: the weight gradient's [wr x wc]
Fork side_by_side(int dtype, double flop_dx, double flop_dw, long xr, long xc, long wr, long wc) {
    const double lo = std::min(flop_dx, flop_dw);
    if (dtype != GN_BF16 || lo < kSideBySideFlop) return Fork::kNever;
    if (std::min(grid_est(xr, xc, 256, 128), grid_est(wr, wc, 256, 256)) >= 256) return Fork::kNever;
    return lo >= kSideBySideEagerFlop ? Fork::kAlways : Fork::kCaptured;
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
    return colsum_dispatch(in, out, M, N, dtype, flags, as_stream(stream), N, nullptr, 0);
}

// Linear backward (autograd.cpp:172-305): three stream-ordered launches, no host sync.
extern "C" int gn_linear_bwd(const void* dY, const void* X, const void* W, void* dX, void* dW,
                             void* db, int M, int N, int K, int dtype, unsigned flags,
                             void* stream) {
    return gn_linear_bwd_ws(dY, X, W, dX, dW, db, M, N, K, dtype, flags, nullptr, 0, stream);
}

extern "C" size_t gn_linear_workspace_bytes(int M, int N, int K, int dtype) {
    if (dtype == GN_F32) return std::max(skinny_bwd_ws_bytes(M, N, K), linear_f32_ws_bytes(M, N, K));
    return weight_grad_ws_bytes(M, N, K, dtype);
}

// Same, with a workspace for the weight gradient's split-K partials (may be NULL / short:
// the split is then limited to what fits).
extern "C" int gn_linear_bwd_ws(const void* dY, const void* X, const void* W, void* dX, void* dW,
                                void* db, int M, int N, int K, int dtype, unsigned flags,
                                void* ws, size_t ws_bytes, void* stream) {
    clear_error();
    GN_REQUIRE(M >= 0 && N >= 0 && K >= 0, "gn_linear_bwd: negative size");
    GN_REQUIRE(dY && X && W && dW, "gn_linear_bwd: null pointer (dY, X, W, dW are required)");
    GN_REQUIRE(dtype == GN_F32 || dtype == GN_BF16, "gn_linear_bwd: dtype %d", dtype);
    hipStream_t s = as_stream(stream);
    if (dtype == GN_F32 && M > 0 && N > 0 && skinny_bwd_applicable(dY, X, W, dX, dW, M, K))
        return skinny_linear_bwd((const float*)dY, (const float*)X, (const float*)W, (float*)dX,
                                 (float*)dW, (float*)db, M, N, K, flags & GN_ACCUMULATE, ws,
                                 ws_bytes, s);
    if (dtype == GN_F32 && small_linear_applicable(M, N, K, dX != nullptr))
        return small_linear_launch((const float*)dY, (const float*)X, (const float*)W, (float*)dX,
                                   (float*)dW, (float*)db, M, N, K, flags & GN_ACCUMULATE, s);
    const double mac = (double)M * N * K;
    SideBySide sb(s, dX ? side_by_side(dtype, 2.0 * mac, 2.0 * mac, M, K, N, K) : Fork::kNever);
    // dW[N x K] = dY^T . X  (A = dY stored [M x N] = [Ks x Mout], transposed), db fused
    int rc = weight_grad(dY, N, X, K, M, N, K, dW, dW, N, (float*)db, nullptr, dtype, flags, s, ws,
                         ws_bytes);
    if (rc == GN_OK && dX)  // dX[M x K] = dY[M x N] . W[N x K]
        rc = gemm_dispatch(dY, W, N, nullptr, nullptr, 0, dX, M, K, 0, 0, dtype, dtype, flags,
                           sb.side(), dtype == GN_F32 ? ws : nullptr, ws_bytes);
    const int jr = sb.join();
    return rc ? rc : jr;
}

namespace gn {
int glu_bwd_to_gu(int kind, const void* dO, const void* gate, const void* up, void* gu, int M,
                  int H, int dtype, hipStream_t s);
}

// Projection part of the fused GLU backward, from the local gradients gu = [dGate | dUp]
// ([M x 2H], row pitch 2H): dX = dGate Wg + dUp Wu (one GEMM over K = 2H), dWg and dWu from
// one GEMM over the 2H rows of gu^T X (rows < H -> dWg, rows >= H -> dWu), bias sums.
static int glu_proj_impl(const void* gu, const void* X, const void* Wg, const void* Wu,
                         void* dX, void* dWg, void* dWu, void* dbg, void* dbu, int M, int K,
                         int H, int dtype, unsigned flags, void* ws, size_t ws_bytes,
                         void* stream);

extern "C" int gn_glu_proj_bwd(const void* gu, const void* X, const void* Wg, const void* Wu,
                               void* dX, void* dWg, void* dWu, void* dbg, void* dbu, int M, int K,
                               int H, int dtype, unsigned flags, void* stream) {
    clear_error();
    return glu_proj_impl(gu, X, Wg, Wu, dX, dWg, dWu, dbg, dbu, M, K, H, dtype, flags, nullptr, 0,
                         stream);
}

extern "C" int gn_glu_proj_bwd_ws(const void* gu, const void* X, const void* Wg, const void* Wu,
                                  void* dX, void* dWg, void* dWu, void* dbg, void* dbu, int M,
                                  int K, int H, int dtype, unsigned flags, void* ws,
                                  size_t ws_bytes, void* stream) {
    clear_error();
    return glu_proj_impl(gu, X, Wg, Wu, dX, dWg, dWu, dbg, dbu, M, K, H, dtype, flags, ws,
                         ws_bytes, stream);
}

static int glu_proj_impl(const void* gu, const void* X, const void* Wg, const void* Wu,
                         void* dX, void* dWg, void* dWu, void* dbg, void* dbu, int M, int K,
                         int H, int dtype, unsigned flags, void* ws, size_t ws_bytes,
                         void* stream) {
    GN_REQUIRE(M >= 0 && K >= 0 && H >= 0, "gn_glu_proj_bwd: negative size");
    GN_REQUIRE(gu && X && Wg && Wu, "gn_glu_proj_bwd: null pointer");
    GN_REQUIRE((dWg == nullptr) == (dWu == nullptr) && (dWg || (!dbg && !dbu)),
               "gn_glu_proj_bwd: dWg and dWu go together (both NULL: frozen weights, no biases)");
    GN_REQUIRE(dtype == GN_F32 || dtype == GN_BF16, "gn_glu_proj_bwd: dtype %d", dtype);
    hipStream_t s = as_stream(stream);
    const size_t esz = dtype == GN_F32 ? 4 : 2;
    const char* g0 = (const char*)gu;
    const bool acc = flags & GN_ACCUMULATE;
    if (M == 0 || K == 0 || H == 0) return GN_OK;
    const double mac = 2.0 * (double)M * K * H;
    SideBySide sb(s, dX && dWg ? side_by_side(dtype, 2.0 * mac, 2.0 * mac, M, K, 2L * H, K) : Fork::kNever);
    int rc = GN_OK;
    if (dWg) {
        // dWg / dWu from one GEMM over the 2H rows of gu^T X, with the bias sums fused
        if ((dbg == nullptr) != (dbu == nullptr)) {
            // one bias only: sum it separately, the GEMM carries none
            float* scr = acc ? nullptr : (float*)dWg;
            if (dbg)
                rc = colsum_dispatch(g0, (float*)dbg, M, H, dtype, flags, s, 2 * H, scr, (size_t)H * K);
            if (rc == GN_OK && dbu)
                rc = colsum_dispatch(g0 + (size_t)H * esz, (float*)dbu, M, H, dtype, flags, s, 2 * H,
                                     scr, (size_t)H * K);
            if (rc == GN_OK)
                rc = weight_grad(g0, 2 * H, X, K, M, 2 * H, K, dWg, dWu, H, nullptr, nullptr, dtype,
                                 flags, s, ws, ws_bytes);
        } else {
            rc = weight_grad(g0, 2 * H, X, K, M, 2 * H, K, dWg, dWu, H, (float*)dbg, (float*)dbu,
                             dtype, flags, s, ws, ws_bytes);
        }
    }
    if (rc == GN_OK && dX) {
        GemmDesc d{};
        d.nseg = 2;
        d.A[0] = (const bf16_t*)g0; d.lda[0] = 2 * H; d.B[0] = (const bf16_t*)Wg; d.ldb[0] = K; d.Ks[0] = H;
        d.A[1] = (const bf16_t*)(g0 + (size_t)H * esz); d.lda[1] = 2 * H;
        d.B[1] = (const bf16_t*)Wu; d.ldb[1] = K; d.Ks[1] = H;
        d.M = M; d.N = K; d.C = dX; d.C2 = dX; d.Msplit = M; d.ldc = K; d.accumulate = acc;
        rc = gemm_run(d, 0, 0, dtype, dtype, sb.side());
    }
    const int jr = sb.join();
    return rc ? rc : jr;
}

extern "C" int gn_glu_linear_bwd(int kind, const void* dO, const void* gate, const void* up,
                                 const void* X, const void* Wg, const void* Wu, void* dX,
                                 void* dWg, void* dWu, void* dbg, void* dbu, void* gu_ws, int M,
                                 int K, int H, int dtype, unsigned flags, void* stream) {
    return gn_glu_linear_bwd_ws(kind, dO, gate, up, X, Wg, Wu, dX, dWg, dWu, dbg, dbu, gu_ws, M, K,
                                H, dtype, flags, nullptr, 0, stream);
}

extern "C" size_t gn_glu_workspace_bytes(int M, int K, int H, int dtype) {
    return weight_grad_ws_bytes(M, 2 * H, K, dtype);
}

extern "C" int gn_glu_linear_bwd_ws(int kind, const void* dO, const void* gate, const void* up,
                                    const void* X, const void* Wg, const void* Wu, void* dX,
                                    void* dWg, void* dWu, void* dbg, void* dbu, void* gu_ws,
                                    int M, int K, int H, int dtype, unsigned flags, void* ws,
                                    size_t ws_bytes, void* stream) {
    clear_error();
    GN_REQUIRE(M >= 0 && K >= 0 && H >= 0, "gn_glu_linear_bwd: negative size");
    GN_REQUIRE(dO && gate && up && X && Wg && Wu && dWg && dWu && gu_ws,
               "gn_glu_linear_bwd: null pointer");
    GN_REQUIRE(dtype == GN_F32 || dtype == GN_BF16, "gn_glu_linear_bwd: dtype %d", dtype);
    int rc = glu_bwd_to_gu(kind, dO, gate, up, gu_ws, M, H, dtype, as_stream(stream));
    if (rc) return rc;
    return glu_proj_impl(gu_ws, X, Wg, Wu, dX, dWg, dWu, dbg, dbu, M, K, H, dtype, flags, ws,
                         ws_bytes, stream);
}

// Down projection backward with the GLU local gradient fused into the dA epilogue:
//   gu = [dGate | dUp] of glu(gate, up) at dO = dA = dY Wd   (dA never written)
//   dWd = dY^T A (fp32),  dbd = column sums of dY (optional).
static int ffn_down_glu_impl(int kind, const void* dY, const void* A, const void* Wd,
                             const void* gate, const void* up, void* gu, void* dWd, void* dbd,
                             int M, int N, int H, int dtype, unsigned flags, void* ws,
                             size_t ws_bytes, void* stream) {
    GN_REQUIRE(M >= 0 && N >= 0 && H >= 0, "gn_ffn_down_glu_bwd: negative size");
    GN_REQUIRE(dY && A && Wd && gate && up && gu, "gn_ffn_down_glu_bwd: null pointer");
    GN_REQUIRE(dWd || !dbd, "gn_ffn_down_glu_bwd: dbd without dWd");
    GN_REQUIRE(dtype == GN_BF16, "gn_ffn_down_glu_bwd: bf16 only (fp32: gn_linear_bwd + gn_glu_linear_bwd)");
    GN_REQUIRE(kind >= GN_GLU_SWIGLU_UP && kind <= GN_GLU_REGLU_UP, "gn_ffn_down_glu_bwd: kind %d", kind);
    if (M == 0 || H == 0) return GN_OK;
    hipStream_t s = as_stream(stream);
    const double mac = (double)M * N * H;
    SideBySide sb(s, dWd ? side_by_side(dtype, 2.0 * mac, 2.0 * mac, M, H, N, H) : Fork::kNever);
    int rc = GN_OK;
    // frozen down projection (dWd NULL): the local gradients only
    if (dWd)
        rc = weight_grad(dY, N, A, H, M, N, H, dWd, dWd, N, (float*)dbd, nullptr, dtype, flags, s, ws,
                         ws_bytes);
    if (rc == GN_OK) {
        GemmDesc d{};
        d.nseg = 1;
        d.A[0] = (const bf16_t*)dY; d.lda[0] = N; d.Ks[0] = N;
        d.B[0] = (const bf16_t*)Wd; d.ldb[0] = H;
        d.M = M; d.N = H; d.Msplit = M;
        d.epi = 1; d.gate = (const bf16_t*)gate; d.up = (const bf16_t*)up; d.ldg = H;
        d.gu = (bf16_t*)gu; d.ldgu = 2 * H; d.H = H; d.glu_kind = kind;
        rc = gemm_run(d, 0, 0, dtype, GN_BF16, sb.side());
    }
    const int jr = sb.join();
    return rc ? rc : jr;
}

extern "C" int gn_ffn_down_glu_bwd(int kind, const void* dY, const void* A, const void* Wd,
                                   const void* gate, const void* up, void* gu, void* dWd,
                                   void* dbd, int M, int N, int H, int dtype, unsigned flags,
                                   void* stream) {
    clear_error();
    return ffn_down_glu_impl(kind, dY, A, Wd, gate, up, gu, dWd, dbd, M, N, H, dtype, flags,
                             nullptr, 0, stream);
}

// Same, with a workspace for dWd's split-K partials: gn_linear_workspace_bytes(M, N, H, dtype).
extern "C" int gn_ffn_down_glu_bwd_ws(int kind, const void* dY, const void* A, const void* Wd,
                                      const void* gate, const void* up, void* gu, void* dWd,
                                      void* dbd, int M, int N, int H, int dtype, unsigned flags,
                                      void* ws, size_t ws_bytes, void* stream) {
    clear_error();
    return ffn_down_glu_impl(kind, dY, A, Wd, gate, up, gu, dWd, dbd, M, N, H, dtype, flags, ws,
                             ws_bytes, stream);
}
