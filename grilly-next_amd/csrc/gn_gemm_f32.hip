// gn_gemm_f32.hip — fp32 contractions on the bf16 matrix cores (six-product split).
//
//   C[M x N] (+)= sum_s op(A_s) op(B_s),   A_s, B_s and C fp32
//
// Each fp32 operand element x is split on its way from registers into LDS into three bf16
// pieces,  x0 = bf16(x),  x1 = bf16(x - x0),  x2 = bf16(x - x0 - x1)  (each difference is
// exact in fp32), and every product is accumulated as
//   a2 b0 + a1 b1 + a0 b2 + a1 b0 + a0 b1 + a0 b0
// with v_mfma_f32_32x32x16_bf16 (products of bf16 pieces are exact, sums in fp32): the
// "bf16x6" scheme of Henry, Tang & Heinecke (ARITH 2019).  x0 + x1 + x2 carries x to
// |x - x0 - x1 - x2| <= 2^-25 |x|, and the dropped products a1 b2, a2 b1, a2 b2 are each below
// 2^-24 |a b|, so a product is fp32-grade: per-element results match an fp32 FMA chain to
// within the fp32 accumulation error, which an optimizer that divides by a running gradient
// magnitude (AdamW) needs.  The three-product variant (a0 b0 + a0 b1 + a1 b0) is good only to
// ~2^-16 per product and visibly moved AdamW updates of small gradients.  Six bf16 MFMAs per
// product keep ~415 TFLOP/s of fp32 work on MI355X, against 157 TFLOP/s for
// v_mfma_f32_32x32x2_f32.  Non-finite inputs give NaN (inf - inf in the split).
//
// Block tile TM x TN (128 x 128, or 64 x 256 for M <= 64), 16 fp32 k per stage, 256 threads =
// 4 waves, each wave 64 x 64 of 2 x 2 accumulators.  LDS holds, per operand and stage, three
// planes (x0, x1, x2) in the operand's own orientation: [rows][16] for operands with k
// contiguous in memory (a fragment is one ds_read_b128), [16][rows] for operands with rows
// contiguous (a fragment is two transposing ds_read_b64_tr_b16), so every thread writes its
// global loads to LDS as contiguous runs and a wave's writes do not collide in the banks.  Software pipeline with two LDS
// stages, two register sets and one barrier per stage: while the MFMAs read stage t, the
// registers holding k-tile t+1 are split into the other stage and take the loads of k-tile
// t+3, so each load has two stages of MFMAs to arrive.  Long-K shapes with few tiles split K
// over blockIdx.y into fp32 partial planes that split_reduce adds in index order
// (deterministic).  (A persistent grid streaming (tile, k-range) items through the pipeline
// was measured slower: 445 against 350 us on the 1 GB weight gradient below.)
#include <algorithm>

#include "gn_common.h"
#include "gn_gemm_dma.h"
#include "gn_mfma.h"

namespace gn {
namespace {

constexpr int TK = 16;     // fp32 k per stage
constexpr int PITCH = TK;  // bf16 per LDS row of one plane (32 bytes)

__device__ __forceinline__ int swz(int r) { return (r >> 2) & 1; }

typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

// (a, b) -> their three bf16 pieces as packed pairs (one v_cvt_pk_bf16_f32 per piece; the
// pieces widen back to fp32 with a shift or a mask)
__device__ __forceinline__ void split2(float a, float b, uint32_t& p0, uint32_t& p1, uint32_t& p2) {
    p0 = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v){a, b}, bf16x2v));
    const float ra = a - __uint_as_float(p0 << 16), rb = b - __uint_as_float(p0 & 0xffff0000u);
    p1 = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v){ra, rb}, bf16x2v));
    const float sa = ra - __uint_as_float(p1 << 16), sb = rb - __uint_as_float(p1 & 0xffff0000u);
    p2 = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v){sa, sb}, bf16x2v));
}

// Operand tile of ROWS rows x TK k, three planes (x0, x1, x2) of ROWS * TK bf16 in LDS.
//   KCONTIG (element (r, k) at P[r * ld + k]): planes are [ROWS][TK] (32-byte rows, the two
//     16-byte chunks swapped every four rows); float4 i of thread t holds row c / 4,
//     k 4 (c % 4) .. +3 with c = t + 256 i; a fragment is one ds_read_b128.
//   else (element (r, k) at P[k * ld + r]): planes are [TK][ROWS] (row r of k-row k in 16-byte
//     chunk (r / 8) ^ kxor(k)); thread t holds rows 4 (t % RG) .. +3 (RG = ROWS / 4 row groups)
//     at NV = ROWS / 64 consecutive k from (t / RG) NV, float4 i being k-row i, and writes them
//     as 8-byte runs along the rows (the lanes of a wave cover whole k-rows: no bank
//     conflicts); a fragment is two ds_read_b64_tr_b16, which transpose 4 k-rows x 16 rows.
template <int ROWS, bool KCONTIG>
struct Tile {
    static constexpr int NV = ROWS / 64;  // float4 registers per thread
    static constexpr int RG = ROWS / 4;
    static constexpr int FRAG_READS = KCONTIG ? 1 : 2;  // LDS reads per fragment
    static constexpr int PLANE = ROWS * PITCH;

    static __device__ __forceinline__ int kxor(int k) {
        // even values keep the two chunks a 16-row half of a transposed read spans adjacent
        if constexpr (ROWS >= 128) return ((k & 1) * 6) ^ (((k >> 1) & 1) * 10);
        else return 2 * (k & 3);
    }

    // Rows >= rlim and k >= klim read as zero (rlim and klim are multiples of 4, and so is
    // every 4-run start along the contiguous index, so a 16-byte load is entirely in or out).
    // Out-of-range loads read a clamped in-range address and are zeroed afterwards, so the
    // loads carry no branches and the wait for them can count outstanding loads.
    // ok: bit i set when float4 i is in range (the store zeroes the others; testing here would
    // wait for the load).
    static __device__ __forceinline__ void load(const float* __restrict__ P, int ld, int r0,
                                                int rlim, int k0, int klim, float4 (&v)[NV],
                                                uint32_t& ok) {
        const int t = threadIdx.x;
        ok = 0;
        if (KCONTIG) {
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int c = t + 256 * i;
                const int r = r0 + (c >> 2), k = k0 + (c & 3) * 4;
                ok |= (uint32_t)(r < rlim && k < klim) << i;
                v[i] = *reinterpret_cast<const float4*>(P + (size_t)min(r, rlim - 1) * ld + min(k, klim - 4));
            }
        } else {
            const int r = r0 + (t % RG) * 4, kb = k0 + (t / RG) * NV;
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int k = kb + i;
                ok |= (uint32_t)(r < rlim && k < klim) << i;
                v[i] = *reinterpret_cast<const float4*>(P + (size_t)min(k, klim - 1) * ld + min(r, rlim - 4));
            }
        }
    }

    // four values -> the three planes, 8 bytes each at element offset off
    static __device__ __forceinline__ void put4(bf16_t* __restrict__ s, int off, float a, float b,
                                                float c, float d) {
        uint32_t lo[3], hi[3];
        split2(a, b, lo[0], lo[1], lo[2]);
        split2(c, d, hi[0], hi[1], hi[2]);
#pragma unroll
        for (int j = 0; j < 3; ++j) *reinterpret_cast<uint2*>(s + j * PLANE + off) = make_uint2(lo[j], hi[j]);
    }

    // The registers of load() as the three planes at s (out-of-range float4s as zeros).
    static __device__ __forceinline__ void store(bf16_t* __restrict__ s, const float4 (&v)[NV],
                                                 uint32_t ok) {
        const int t = threadIdx.x;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const bool in = (ok >> i) & 1u;
            const float a = in ? v[i].x : 0.f, b = in ? v[i].y : 0.f;
            const float c = in ? v[i].z : 0.f, d = in ? v[i].w : 0.f;
            if (KCONTIG) {
                const int e = t + 256 * i;
                const int r = e >> 2, q = e & 3;  // k = 4q .. 4q+3
                put4(s, r * PITCH + (((q >> 1) ^ swz(r)) * 8) + (q & 1) * 4, a, b, c, d);
            } else {
                const int r = (t % RG) * 4, k = (t / RG) * NV + i;
                put4(s, k * ROWS + (((r >> 3) ^ kxor(k)) * 8) + (r & 7), a, b, c, d);
            }
        }
    }

    // MFMA operand of rows row0 .. row0+31 (lane l: row row0 + l % 32, k 8 (l / 32) .. +7) from
    // plane p of the tile at s
    static __device__ __forceinline__ bf16x8_t frag(const bf16_t* s, int p, int row0) {
        const int lane = threadIdx.x & 63;
        const bf16_t* pl = s + p * PLANE;
        if (KCONTIG) {
            const int r = row0 + (lane & 31);
            return __builtin_bit_cast(
                bf16x8_t,
                *reinterpret_cast<const uint4*>(pl + r * PITCH + (((lane >> 5) ^ swz(r)) * 8)));
        } else {
            // 16-lane group g: rows row0 + 16 (g % 2) .. +15, k-rows 8 (g / 2) + {0..3, 4..7}
            const int g = lane >> 4, sl = lane & 15;
            const int r = row0 + 16 * (g & 1) + 4 * (sl & 3);
            const int k = 8 * (g >> 1) + (sl >> 2);
            const bf16_t* p0 = pl + k * ROWS + (((r >> 3) ^ kxor(k)) * 8) + (r & 7);
            return ld_tr_pair(p0, p0 + 4 * ROWS);  // kxor(k + 4) == kxor(k)
        }
    }
};

template <int TM, int TN, bool TA, bool TB>
struct Cfg {
    using TileA = Tile<TM, !TA>;
    using TileB = Tile<TN, TB>;
    static constexpr int STAGE = 3 * (TM + TN) * PITCH;  // bf16 per stage (A then B planes)
    static constexpr size_t SMEM = (size_t)2 * STAGE * sizeof(bf16_t);
    static constexpr int WN = TN / 64;  // waves along N (4 waves of 64 x 64)
};

template <int TM, int TN, bool TA, bool TB>
__global__ __launch_bounds__(256, 2) void gemm_f32x6(GemmDesc g) {
    using C = Cfg<TM, TN, TA, TB>;
    using LA = typename C::TileA;
    using LB = typename C::TileB;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    bf16_t* smem = reinterpret_cast<bf16_t*>(smem_raw);  // [2][A planes | B planes]

    // tile coordinates: XCD-contiguous ranges (blocks are dispatched round-robin over the
    // 8 XCDs), then 8-tall groups
    const int tilesM = (g.M + TM - 1) / TM, tilesN = (g.N + TN - 1) / TN;
    const int tiles = tilesM * tilesN;
    int pid = blockIdx.x;
    if ((tiles & 7) == 0) pid = (pid & 7) * (tiles >> 3) + (pid >> 3);
    const int group_id = pid / (8 * tilesN);
    const int first_m = group_id * 8;
    const int gsize = min(tilesM - first_m, 8);
    const int in_group = pid % (8 * tilesN);
    const int m0 = (first_m + in_group % gsize) * TM, n0 = (in_group / gsize) * TN;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / C::WN, wn = wave % C::WN;
    const int ra0 = wm * 64, rb0 = wn * 64;

    f32x16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) zero16(acc[i][j]);

    // this block's k-tiles (split blockIdx.y) over the concatenated segments
    const int kt0 = (g.Ks[0] + TK - 1) / TK;
    const int KT = kt0 + (g.nseg > 1 ? (g.Ks[1] + TK - 1) / TK : 0);
    const int splits = g.ksplit > 1 ? g.ksplit : 1;
    const int per = (KT + splits - 1) / splits;
    const int tb = blockIdx.y * per, te = min(KT, tb + per);

    // two register sets in flight: when the MFMAs run k-tile t, set X holds k-tile t+1 and
    // the other set k-tile t+2 (loads issued two iterations before they are needed)
    struct Regs {
        float4 a[LA::NV], b[LB::NV];
        uint32_t oka, okb;
    };
    Regs r0s, r1s;
    auto gload = [&](int t, Regs& R) {
        const int sg = t < kt0 ? 0 : 1;
        const int k0 = (t < kt0 ? t : t - kt0) * TK;
        // A: TA = 0 -> A[m * lda + k] (k contiguous); TA = 1 -> A[k * lda + m]
        LA::load(reinterpret_cast<const float*>(g.A[sg]), g.lda[sg], m0, g.M, k0, g.Ks[sg], R.a, R.oka);
        // B: TB = 1 -> B[n * ldb + k] (k contiguous); TB = 0 -> B[k * ldb + n]
        LB::load(reinterpret_cast<const float*>(g.B[sg]), g.ldb[sg], n0, g.N, k0, g.Ks[sg], R.b, R.okb);
    };
    auto sstore = [&](int buf, const Regs& R) {
        bf16_t* st = smem + buf * C::STAGE;
        LA::store(st, R.a, R.oka);
        LB::store(st + 3 * LA::PLANE, R.b, R.okb);
    };

    auto iter = [&](int t, Regs& R) {
        // stage (t - tb) & 1 holds k-tile t (split last iteration); every wave has finished
        // reading the other stage, which the split below overwrites
        __syncthreads();
        const bf16_t* As = smem + ((t - tb) & 1) * C::STAGE;
        const bf16_t* Bs = As + 3 * LA::PLANE;
        bf16x8_t a[3][2], b[3][2];
#pragma unroll
        for (int p = 0; p < 3; ++p) {
            a[p][0] = LA::frag(As, p, ra0);
            a[p][1] = LA::frag(As, p, ra0 + 32);
            b[p][0] = LB::frag(Bs, p, rb0);
            b[p][1] = LB::frag(Bs, p, rb0 + 32);
        }
        // The next k-tile's split goes into the other stage while the MFMAs below run; its
        // registers then take the loads of k-tile t+3 (clamped into this split's range: past
        // its end the last tile is loaded again and its split lands in a stage nothing reads).
        sstore(((t - tb) & 1) ^ 1, R);
        gload(min(t + 3, te - 1), R);
        // smallest terms first: (2,0) (1,1) (0,2) (1,0) (0,1) (0,0)
        constexpr int PA[6] = {2, 1, 0, 1, 0, 0}, PB[6] = {0, 1, 2, 0, 1, 0};
#pragma unroll
        for (int q = 0; q < 6; ++q)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = mfma32(a[PA[q]][i], b[PB[q]][j], acc[i][j]);
        // issue order: the fragment reads, then each MFMA followed by a share of the split's
        // VALU work, LDS writes and loads, so the split runs while the matrix pipe is busy
        __builtin_amdgcn_sched_group_barrier(0x100, 6 * (LA::FRAG_READS + LB::FRAG_READS), 0);
#pragma unroll
        for (int q = 0; q < 24; ++q) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // VALU
            __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // DS write
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
        }
    };

    if (tb < te) {
        // the first two k-tiles' loads go out together, so only one load latency precedes the
        // first split (short k loops, e.g. K = 64, are all prologue)
        gload(tb, r0s);
        gload(min(tb + 1, te - 1), r1s);
        sstore(0, r0s);
        gload(min(tb + 2, te - 1), r0s);
        for (int t = tb; t < te; t += 2) {
            iter(t, r1s);
            if (t + 1 < te) iter(t + 1, r0s);
        }
    }

    // epilogue: accumulator element r of lane l is (row 8(r/4) + 4(l/32) + r%4, col l%32);
    // a split's partial tile goes to its plane
    if (splits > 1) {
        float* P = g.part + (size_t)blockIdx.y * g.M * g.N;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int n = n0 + rb0 + j * 32 + (lane & 31);
                if (n >= g.N) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m0 + ra0 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    if (m < g.M) P[(size_t)m * g.N + n] = acc[i][j][r];
                }
            }
    } else if ((((uintptr_t)g.C | (uintptr_t)g.C2) & 15) == 0 && (g.ldc & 3) == 0) {
        // 16-byte stores: each wave stages one 32 x 32 accumulator at a time in its own LDS
        // strip (pitch 40 floats, so the two row groups of a staging write fall in disjoint
        // banks) and writes it back as whole row segments, lane l taking rows l / 8 + 8 q and
        // columns 4 (l % 8) .. +3 (N % 4 == 0, so a vector is entirely in or out).  Overwritten
        // outputs are stored non-temporally (the 1 GB weight gradient of the hypernetwork's
        // output layer at batch 64: 0.675 -> 0.631-0.641 ms for its Linear backward); the
        // same hint on the loads of an operand no other block reads made it slower.
        __syncthreads();  // every wave is done reading the operand stages
        float* strip = reinterpret_cast<float*>(smem_raw) + wave * (32 * 40);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                // the strip is private to the wave, but its lanes read what other lanes wrote:
                // wave-scope release/acquire around a wave barrier order the writes before the
                // reads (and the reads before the next tile's writes, below); no instruction
                // is emitted for them on a wave64 CU
                wave_lds_sync();
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    strip[(8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * 40 + (lane & 31)] = acc[i][j][r];
                wave_lds_sync();
                const int n = n0 + rb0 + j * 32 + 4 * (lane & 7);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int row = (lane >> 3) + 8 * q;
                    float4 v = *reinterpret_cast<const float4*>(strip + row * 40 + 4 * (lane & 7));
                    const int m = m0 + ra0 + i * 32 + row;
                    if (m >= g.M || n >= g.N) continue;
                    float* dst = reinterpret_cast<float*>(m < g.Msplit ? g.C : g.C2) +
                                 (size_t)(m < g.Msplit ? m : m - g.Msplit) * g.ldc + n;
                    if (g.accumulate) {
                        const float4 o = *reinterpret_cast<const float4*>(dst);
                        v.x += o.x; v.y += o.y; v.z += o.z; v.w += o.w;
                        *reinterpret_cast<float4*>(dst) = v;
                    } else {
                        const f32x4v w = {v.x, v.y, v.z, v.w};
                        __builtin_nontemporal_store(w, reinterpret_cast<f32x4v*>(dst));
                    }
                }
            }
    } else {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                gemm_store_tile<float, 0>(g, m0 + ra0 + i * 32, n0 + rb0 + j * 32, acc[i][j]);
    }
}

inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }


inline int k_tiles(const GemmDesc& g) {
    return (g.Ks[0] + TK - 1) / TK + (g.nseg > 1 ? (g.Ks[1] + TK - 1) / TK : 0);
}

// 64 x 256 tiles when the output has at most 64 rows (a batch of rows against a wide weight),
// else 128 x 128 (also measured for wide outputs: 256-column tiles were no faster)
inline bool wide(const GemmDesc& g) { return g.M <= 64; }

// Blocks that run at once: two per CU (the kernel's VGPRs allow two waves per SIMD).
int resident_blocks() {
    static const int n = [] {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0)
            cus = 256;
        return 2 * cus;
    }();
    return n;
}

// Splits of K for shapes with fewer tiles than the GPU runs blocks at once: as many ranges as
// fill it once (tiles x splits <= blocks, no half-empty second round), each
// at least 16 k-tiles (256 k), the partial planes within cap.  Returns the number of
// non-empty ranges (1: no split).
int choose_split(const GemmDesc& g, size_t cap) {
    if (cap == 0 || g.N % 4 || g.ldc % 4 || !al16(g.C) || (g.C2 && !al16(g.C2))) return 1;
    const int tm = wide(g) ? 64 : 128, tn = wide(g) ? 256 : 128;
    const long tiles = (long)((g.M + tm - 1) / tm) * ((g.N + tn - 1) / tn);
    const int KT = k_tiles(g);
    const long blocks = resident_blocks();
    if (2 * tiles > blocks || KT < 32) return 1;
    int ks = (int)std::min<long>({(long)KT / 16, blocks / tiles, 128L});
    while (ks > 1 && (size_t)ks * g.M * g.N * sizeof(float) > cap) --ks;
    if (ks < 2) return 1;
    const int per = (KT + ks - 1) / ks;
    return (KT + per - 1) / per;
}

template <int TM, int TN, bool TA, bool TB>
int launch_t(const GemmDesc& g, hipStream_t s) {
    constexpr size_t smem = Cfg<TM, TN, TA, TB>::SMEM;
    static const bool ok =
        hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_f32x6<TM, TN, TA, TB>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) == hipSuccess;
    if (!ok) {
        set_error("gn_gemm (fp32): cannot reserve %zu B of LDS", smem);
        return GN_E_HIP;
    }
    const int tiles = ((g.M + TM - 1) / TM) * ((g.N + TN - 1) / TN);
    hipLaunchKernelGGL((gemm_f32x6<TM, TN, TA, TB>), dim3(tiles, g.ksplit > 1 ? g.ksplit : 1),
                       dim3(256), smem, s, g);
    if (g.ksplit > 1) launch_split_reduce(g, s);
    GN_LAUNCH_CHECK("gn_gemm (fp32 bf16x6)");
    return GN_OK;
}

template <int TM, int TN>
int launch_tiles(const GemmDesc& g, int transA, int transB, hipStream_t s) {
    if (!transA && !transB) return launch_t<TM, TN, false, false>(g, s);
    if (!transA && transB) return launch_t<TM, TN, false, true>(g, s);
    if (transA && !transB) return launch_t<TM, TN, true, false>(g, s);
    return launch_t<TM, TN, true, true>(g, s);
}

}  // namespace

bool gemm_f32_applicable(const GemmDesc& g) {
    if (g.epi != 0 || g.bias || g.cbias || g.M <= 0 || g.N <= 0 || g.M % 4 || g.N % 4) return false;
    for (int s = 0; s < g.nseg; ++s)
        if (g.Ks[s] % 4 || !al16(g.A[s]) || !al16(g.B[s]) || g.lda[s] % 4 || g.ldb[s] % 4)
            return false;
    return true;
}

size_t gemm_f32_part_bytes(const GemmDesc& g) {
    const int ks = choose_split(g, ~(size_t)0);
    return ks > 1 ? (size_t)ks * g.M * g.N * sizeof(float) : 0;
}

int gemm_f32_launch(const GemmDesc& g0, int transA, int transB, hipStream_t s) {
    GemmDesc g = g0;
    g.ksplit = choose_split(g, g.part ? g.part_cap : 0);
    if (wide(g)) return launch_tiles<64, 256>(g, transA, transB, s);
    return launch_tiles<128, 128>(g, transA, transB, s);
}

}  // namespace gn
