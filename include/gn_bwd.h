/*
 * gn_bwd.h — C ABI of the MI355X (gfx950) backward-kernel library libgn_bwd.so.
 *
 * This is the drop-in boundary between grilly-next's tape engine and the
 * gradient kernels.  In the reference every per-op handler
 * `BackwardEngine::backward_<op>(Node*)` (cpp/include/grilly/autograd/autograd.h:340-373,
 * selected by the switch at cpp/src/autograd.cpp:95-130) binds descriptor sets and
 * dispatches GLSL passes with a fence wait per pass.  Here the same handlers call one
 * entry point per op, below.  Every entry point:
 *
 *   - takes raw device pointers (row-major, contiguous), sizes, a dtype code and a
 *     hipStream_t passed as `void*` (NULL = the legacy default stream);
 *   - enqueues its kernels on that stream and returns without synchronising;
 *   - allocates nothing: scratch space is passed in by the caller (`ws`, sized by the
 *     matching *_workspace_bytes query);
 *   - returns GN_OK (0) or a negative GN_E* code; gn_last_error() then gives a
 *     message (thread-local).  The library throws no C++ exceptions across this ABI.
 *
 * Shapes follow the reference: X [M x K], W [N x K] (y = X W^T + b), dY [M x N],
 * dW [N x K], attention tensors [B, H, S, D], VSA dW [O x D].
 *
 * dtype codes extend TensorRef.dtype (autograd.h:50): 0 = f32, 1 = f16, 2 = u32,
 * 3 = i32, 4 = bf16.  "bf16 path" below means bf16 activations/weights, fp32
 * accumulation, bf16 activation gradients and fp32 parameter gradients.
 */
#ifndef GN_BWD_H
#define GN_BWD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------------------- */
#define GN_OK 0
#define GN_E_INVALID (-1)   /* bad size, null pointer, unsupported dtype/kind */
#define GN_E_HIP (-2)       /* a HIP runtime call or kernel launch failed */
#define GN_E_WORKSPACE (-3) /* workspace missing or too small */

/* ---- dtype codes (TensorRef.dtype, autograd.h:50, plus bf16) ------------------------ */
#define GN_F32 0
#define GN_F16 1
#define GN_U32 2
#define GN_I32 3
#define GN_BF16 4

/* ---- flags ------------------------------------------------------------------------ */
#define GN_ACCUMULATE 1u  /* add into existing gradients (fan-out) instead of overwriting */
#define GN_LN_STAT_VAR 2u /* layernorm: `rstd` argument holds the biased variance */
#define GN_NO_GUMBEL 4u   /* surrogate forward: top-2 of the plain dot products (no noise) */
#define GN_RMS_STAT_MEANSQ 8u /* rmsnorm: the statistic is mean(x^2) (rms-norm.glsl:52); eps added */
#define GN_RMS_STAT_RMS 16u   /* rmsnorm: the statistic is sqrt(mean(x^2)+eps) (snn-rmsnorm.glsl:55) */
#define GN_NORM_PARTIALS 32u  /* norm backward: leave the parameter gradients as partial rows in
                                 the workspace, for a later gn_norm_finish (see there) */

/* ---- activation kinds (gn_act_bwd) ------------------------------------------------- */
#define GN_ACT_RELU 0      /* dx = dy*[x>0]            activation-relu-backward.glsl:33-37 */
#define GN_ACT_GELU_TANH 1 /* tanh-form GELU'(x)        activation-gelu-backward.glsl:38-50 */
#define GN_ACT_GELU_ERF 2  /* erf-form GELU'(x)         autograd_core.py:529-542 */
#define GN_ACT_SILU 3      /* sig(x)(1+x(1-sig(x)))     activation-silu-backward.glsl:25-42 */
#define GN_ACT_TANH 4      /* input = saved tanh output t: dy*(1-t^2)  activation-tanh-backward.glsl:33 */
#define GN_ACT_SIGMOID 5   /* input = saved sigmoid output s: dy*s*(1-s) */

/* ---- GLU kinds (gn_glu_bwd, gn_glu_linear_bwd) -------------------------------------- */
#define GN_GLU_SWIGLU_UP 0   /* out = gate*SiLU(up)     fused-swiglu-backward.glsl:99-100 */
#define GN_GLU_SWIGLU_GATE 1 /* out = SiLU(gate)*up     swiglu-fused.glsl:60-64 */
#define GN_GLU_GEGLU_UP 2    /* out = gate*GELU_tanh(up) fused-geglu-backward.glsl:101-103 */
#define GN_GLU_GEGLU_GATE 3  /* out = GELU_tanh(gate)*up */
#define GN_GLU_REGLU_UP 4    /* out = gate*ReLU(up)     fused-reglu-backward.glsl:83-86 */

/* ---- RoPE modes (gn_attn_bwd) ------------------------------------------------------- */
#define GN_ROPE_NONE 0
#define GN_ROPE_INTERLEAVED 1 /* pairs (2i,2i+1)         flash-attention2-rope.glsl:101-141 */
#define GN_ROPE_HALF 2        /* pairs (i, i+D/2)        rope.glsl:74-125 */

/* Message for the last failing call on this thread ("" if none). */
const char* gn_last_error(void);

/* Library version string and the gfx target it was built for. */
const char* gn_version(void);

/* ---- linear ----------------------------------------------------------------------- */
/* Replaces BackwardEngine::backward_linear / backward_linear_chunked
 * (cpp/src/autograd.cpp:172-483) and fnn-linear-backward.glsl:43-89.  fp32 products follow
 * gn_gemm's fp32 rules below (matrix-core split above the small-product sizes: fp32-grade per
 * element, NaN where an operand is inf).
 *   dX = dY W      [M x K]  (skipped when dX == NULL: input needs no grad, autograd.cpp:259)
 *   dW = dY^T X    [N x K]
 *   db = sum_rows dY [N]    (skipped when db == NULL)
 * dtype GN_F32: all fp32.  GN_BF16: dY, X, W, dX bf16; dW, db fp32.
 * flags: GN_ACCUMULATE adds into dX, dW, db. */
int gn_linear_bwd(const void* dY, const void* X, const void* W, void* dX, void* dW, void* db,
                  int M, int N, int K, int dtype, unsigned flags, void* stream);

/* gn_linear_bwd with a workspace for the weight gradient's split-K partials (same
 * reference interface: BackwardEngine::backward_linear, autograd.cpp:172-305).  With
 * gn_linear_workspace_bytes(M, N, K, dtype) bytes (16-byte aligned) a weight gradient whose
 * few output tiles would leave most CUs idle is split over 3..8 ranges of the M rows; each
 * range stores its partial tile and one reduce pass adds them in a fixed order, so the result
 * does not depend on scheduling.  ws may be NULL or shorter (the split then stays within it);
 * the query returns the largest size over the four launches of a shape (with or without db,
 * overwrite or GN_ACCUMULATE), and 0 bytes means none of them uses one. */
int gn_linear_bwd_ws(const void* dY, const void* X, const void* W, void* dX, void* dW, void* db,
                     int M, int N, int K, int dtype, unsigned flags, void* ws, size_t ws_bytes,
                     void* stream);
size_t gn_linear_workspace_bytes(int M, int N, int K, int dtype);

/* Plain GEMM entry used by the linear handler and exported for tests/benchmarks:
 *   C[M x N] (+)= sum_s op(A_s) op(B_s), with up to two K-segments s (the second may be NULL).
 *   transA = 0: A_s is [M x Ks] row-major;  transA = 1: A_s is stored [Ks x M] (i.e. A_s^T).
 *   transB = 0: B_s is [Ks x N] row-major;  transB = 1: B_s is stored [N x Ks].
 * dtype GN_BF16: A, B bf16, fp32 accumulation, C is bf16 (c_dtype GN_BF16) or fp32 (GN_F32).
 * dtype GN_F32: all fp32.  Small products (k <= 128 and M*N*k <= 2^24) are plain fp32 FMA
 * chains.  Larger ones with M, N, K multiples of 4 and 16-byte aligned operands run on the
 * bf16 matrix cores: each element x is split into three bf16 pieces (|x - x0 - x1 - x2| <=
 * 2^-25 |x|) and six piece products are accumulated in fp32, so each product term is within
 * ~2^-24 |a b| (fp32-grade: the sum carries fp32 accumulation error on top).  That path has
 * two documented limits: an inf operand, or one above the bf16 maximum (|x| > 3.3895e38),
 * makes every output it feeds NaN (inf - inf in the split) where fp32 FMA gives inf; and
 * operands below the fp32 normal range (|x| < 2^-126) may lose their pieces to denormal
 * flushing on the matrix cores (relative accuracy holds down to about 2^-100 |x|max). */
int gn_gemm(const void* A0, const void* B0, int K0, const void* A1, const void* B1, int K1,
            void* C, int M, int N, int transA, int transB, int dtype, int c_dtype,
            unsigned flags, void* stream);

/* Column sums: out[N] (+)= sum_rows in[M x N] (fp32 out; in is f32 or bf16).  Up to 1024 rows
 * in one pass with a fixed summation order (bit-identical reruns); more rows are split over
 * row blocks added with fp32 atomics. */
int gn_colsum(const void* in, float* out, int M, int N, int dtype, unsigned flags, void* stream);

/* ---- activations ------------------------------------------------------------------ */
/* Replaces backward_gelu (autograd.cpp:485-537) and the relu/silu/tanh/sigmoid stubs
 * (autograd.cpp:551-575); shaders activation-{relu,gelu,silu,tanh}-backward.glsl.
 * dX = dY * act'(X) elementwise over n elements (dtype f32 or bf16 for all three). */
int gn_act_bwd(int kind, const void* dY, const void* X, void* dX, int64_t n, int dtype,
               unsigned flags, void* stream);

/* ---- GLU ---------------------------------------------------------------------------- */
/* Elementwise GLU gradient (the local-gradient part of fused-{swiglu,geglu,reglu}-
 * backward.glsl, e.g. fused-swiglu-backward.glsl:93-100):
 *   dGate = dO * d(out)/d(gate),  dUp = dO * d(out)/d(up),  n elements. */
int gn_glu_bwd(int kind, const void* dO, const void* gate, const void* up, void* dGate,
               void* dUp, int64_t n, int dtype, void* stream);

/* Full fused GLU-projection backward (fused-swiglu-backward.glsl:82-160 and the GEGLU/
 * ReGLU twins): with gate = X Wg^T (+bg), up = X Wu^T (+bu), out = glu(gate, up) [M x H]:
 *   gu_ws = [dGate | dUp], one row of 2H per token  [M x 2H] (dtype of the path)
 *   dX  = dGate Wg + dUp Wu    [M x K]  (skipped when dX == NULL)
 *   dWg = dGate^T X, dWu = dUp^T X  [H x K] (fp32 on the bf16 path)
 *   dbg, dbu = column sums      [H]     (skipped when NULL)
 * gu_ws must hold 2*M*H elements of `dtype`. */
int gn_glu_linear_bwd(int kind, const void* dO, const void* gate, const void* up,
                      const void* X, const void* Wg, const void* Wu, void* dX, void* dWg,
                      void* dWu, void* dbg, void* dbu, void* gu_ws, int M, int K, int H,
                      int dtype, unsigned flags, void* stream);

/* gn_glu_linear_bwd with a workspace for the dWg / dWu GEMM's split-K partials, sized by
 * gn_glu_workspace_bytes(M, K, H, dtype); semantics as gn_linear_bwd_ws. */
int gn_glu_linear_bwd_ws(int kind, const void* dO, const void* gate, const void* up,
                         const void* X, const void* Wg, const void* Wu, void* dX, void* dWg,
                         void* dWu, void* dbg, void* dbu, void* gu_ws, int M, int K, int H,
                         int dtype, unsigned flags, void* ws, size_t ws_bytes, void* stream);
size_t gn_glu_workspace_bytes(int M, int K, int H, int dtype);

/* The projection half of gn_glu_linear_bwd, starting from gu = [dGate | dUp] ([M x 2H])
 * already computed (e.g. by gn_ffn_down_glu_bwd). Same outputs as gn_glu_linear_bwd; dX may be
 * NULL (input needs no gradient) and dWg = dWu = NULL skips the weight gradients (frozen
 * projections; dbg, dbu must then be NULL too), so the two GEMMs can also run as two calls. */
int gn_glu_proj_bwd(const void* gu, const void* X, const void* Wg, const void* Wu, void* dX,
                    void* dWg, void* dWu, void* dbg, void* dbu, int M, int K, int H, int dtype,
                    unsigned flags, void* stream);
/* gn_glu_proj_bwd with a workspace for the dWg / dWu GEMM's split-K partials, sized by
 * gn_glu_workspace_bytes(M, K, H, dtype); semantics as gn_linear_bwd_ws. */
int gn_glu_proj_bwd_ws(const void* gu, const void* X, const void* Wg, const void* Wu, void* dX,
                       void* dWg, void* dWu, void* dbg, void* dbu, int M, int K, int H,
                       int dtype, unsigned flags, void* ws, size_t ws_bytes, void* stream);

/* Down-projection backward with the GLU backward fused into its epilogue (a two-node
 * fusion of backward_linear and the fused-*-backward.glsl local gradients):
 *   dA = dY Wd is never stored; gu = [dGate | dUp] of glu(gate, up) at dO = dA ([M x 2H])
 *   dWd = dY^T A [N x H] fp32;  dbd = column sums of dY [N] (skipped when NULL)
 * dY [M x N], A = glu(gate, up) [M x H], Wd [N x H], gate/up [M x H]. bf16 only.  dWd = NULL
 * (with dbd = NULL) skips the weight gradient: a frozen projection, or the two GEMMs as two
 * calls (the weight gradient is then gn_linear_bwd with dX = NULL on the same operands). */
int gn_ffn_down_glu_bwd(int kind, const void* dY, const void* A, const void* Wd,
                        const void* gate, const void* up, void* gu, void* dWd, void* dbd, int M,
                        int N, int H, int dtype, unsigned flags, void* stream);
/* gn_ffn_down_glu_bwd with a workspace for dWd's split-K partials, sized by
 * gn_linear_workspace_bytes(M, N, H, dtype) (dWd is the weight gradient of the Linear
 * y = A Wd^T); semantics as gn_linear_bwd_ws. */
int gn_ffn_down_glu_bwd_ws(int kind, const void* dY, const void* A, const void* Wd,
                           const void* gate, const void* up, void* gu, void* dWd, void* dbd,
                           int M, int N, int H, int dtype, unsigned flags, void* ws,
                           size_t ws_bytes, void* stream);

/* ---- normalisation ---------------------------------------------------------------- */
/* LayerNorm backward, textbook form (autograd_core.py:591-609; fnn-layernorm-backward.glsl
 * :58-159 restructured, with its gamma placement corrected).  mean/rstd fp32 [rows];
 * with GN_LN_STAT_VAR the `rstd` array holds the biased variance and eps is applied.
 * dGamma, dBeta fp32 [F] (either may be NULL). ws: gn_norm_workspace_bytes(rows, F). */
int gn_layernorm_bwd(const void* dY, const void* X, const void* gamma, const float* mean,
                     const float* rstd, void* dX, float* dGamma, float* dBeta, int rows,
                     int F, float eps, int dtype, unsigned flags, void* ws, size_t ws_bytes,
                     void* stream);

/* gn_layernorm_bwd without a workspace argument, for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  It has no
 * counterpart in the reference.  The partial parameter-gradient rows go to a static device
 * array of the library (4 MiB per GPU, held until the process ends; every row shape fits:
 * F <= 2048 uses at most 2 x 256 x F floats, wider rows need none).  The call allocates
 * nothing and computes exactly what gn_layernorm_bwd computes.  All calls on one GPU share
 * that array: calls that overlap on one GPU (e.g. on two streams at once) race. */
int gn_layernorm_bwd_noalloc(const void* dY, const void* X, const void* gamma, const float* mean,
                             const float* rstd, void* dX, float* dGamma, float* dBeta, int rows,
                             int F, float eps, int dtype, unsigned flags, void* stream);

/* RMSNorm backward (no handler in the reference, autograd.cpp:126-128; forward
 * rms-norm.glsl:34-70): y = x * r * w with r = rsqrt(mean(x^2)+eps) given as rstd [rows].
 *   dx = r*w*dy - x * r^3 * mean_j(w_j dy_j x_j);  dw = sum_rows dy * x * r. */
int gn_rmsnorm_bwd(const void* dY, const void* X, const void* w, const float* rstd, void* dX,
                   float* dW, int rows, int F, int dtype, unsigned flags, void* ws,
                   size_t ws_bytes, void* stream);

size_t gn_norm_workspace_bytes(int rows, int F);

/* Mixed-precision forms of the two norm backwards (same reference formulas as above) for a
 * residual stream kept in fp32 under a bf16 block: x, dX and dX_add in x_dtype; dY and
 * gamma / w in dy_dtype; pairs (f32, f32), (bf16, bf16) and (x f32, dy bf16).
 *   dX = norm_grad + dX_add    (dX_add nullable; it may alias dX for an in-place sum)
 * so a pre-norm block's two input gradients (the residual branch and the norm) are summed in
 * the norm's own pass: the fan-out the reference drops (autograd.cpp:78-86) costs no extra
 * read or write.  GN_ACCUMULATE here applies to the parameter gradients only; GN_LN_STAT_VAR
 * as above.  ws: gn_norm_workspace_bytes(rows, F). */
int gn_layernorm_bwd_ex(const void* dY, int dy_dtype, const void* X, int x_dtype,
                        const void* gamma, const float* mean, const float* rstd,
                        const void* dX_add, void* dX, float* dGamma, float* dBeta, int rows,
                        int F, float eps, unsigned flags, void* ws, size_t ws_bytes,
                        void* stream);
/* Deferred parameter gradients of the norm backwards.  A gn_layernorm_bwd_ex / _ex16 /
 * gn_rmsnorm_bwd_ex call with GN_NORM_PARTIALS writes dX as usual but leaves dGamma / dBeta
 * (dW) as the row kernel's per-block partial rows in its workspace, which must then stay
 * untouched until gn_norm_finish sums them (in the same fixed order, so the results are bit
 * for bit those of the undeferred call).  It takes the row-kernel path only (F % 8 == 0,
 * F <= 2048, 16-byte aligned tensors) and returns GN_E_INVALID otherwise, before any launch.
 * gn_norm_finish sums any number of such calls' partials in one launch: what a tape's backward
 * does once at its end instead of one small launch per norm.  No counterpart in the reference
 * (its LayerNorm backward finishes the parameter gradients itself, ops/layernorm.cpp). */
typedef struct GnNormFinish {
    const void* ws;   /* the workspace of the deferred call */
    float* dgamma;    /* its dGamma (LayerNorm) or dW (RMSNorm); NULL: not wanted */
    float* dbeta;     /* its dBeta (LayerNorm only); NULL: not wanted */
    int rows, F;      /* the deferred call's shape */
    int layernorm;    /* 1: LayerNorm (two planes of partials), 0: RMSNorm (one) */
    int accumulate;   /* add onto dgamma / dbeta instead of overwriting */
} GnNormFinish;
int gn_norm_finish(const GnNormFinish* items, int n, void* stream);

/* gn_layernorm_bwd_ex that also writes dX rounded to bf16 into dX_bf16 in the same pass
 * (x_dtype GN_F32): in a residual stream kept in fp32, the gradient of the Add that produced
 * x reaches its bf16 branch as this copy, where the reference's Add backward
 * (autograd.cpp:611-616) would hand on the fp32 gradient and a conversion pass would follow.
 * No counterpart in the reference; bit-identical to gn_convert(dX -> bf16). */
int gn_layernorm_bwd_ex16(const void* dY, int dy_dtype, const void* X, int x_dtype,
                          const void* gamma, const float* mean, const float* rstd,
                          const void* dX_add, void* dX, void* dX_bf16, float* dGamma,
                          float* dBeta, int rows, int F, float eps, unsigned flags, void* ws,
                          size_t ws_bytes, void* stream);
int gn_rmsnorm_bwd_ex(const void* dY, int dy_dtype, const void* X, int x_dtype, const void* w,
                      const float* rstd, const void* dX_add, void* dX, float* dW, int rows,
                      int F, unsigned flags, void* ws, size_t ws_bytes, void* stream);

/* gn_rmsnorm_bwd_ex for a forward that saved another per-row statistic than rstd: the
 * reference's rms-norm.glsl:52 leaves mean(x^2) in its rms_vals buffer (flag
 * GN_RMS_STAT_MEANSQ: r = rsqrt(stat + eps)) and snn-rmsnorm.glsl:55 leaves sqrt(mean(x^2) +
 * eps) (flag GN_RMS_STAT_RMS: r = 1/stat); with neither flag `stat` is rstd and eps is unused.
 * Same replaced interface as gn_rmsnorm_bwd (no RMSNorm handler in the reference,
 * autograd.cpp:126-128). */
int gn_rmsnorm_bwd_stat(const void* dY, int dy_dtype, const void* X, int x_dtype, const void* w,
                        const float* stat, const void* dX_add, void* dX, float* dW, int rows,
                        int F, float eps, unsigned flags, void* ws, size_t ws_bytes,
                        void* stream);

/* ---- softmax / cross-entropy --------------------------------------------------------- */
/* activation-softmax-backward.glsl:27-49: dX = Y * (dY - sum_c dY*Y), per row of C. */
int gn_softmax_bwd(const void* dY, const void* Y, void* dX, int rows, int C, int dtype,
                   void* stream);

/* cross-entropy-backward.glsl:29-84: dLogits = scale * (softmax(logits) - onehot(target)).
 * targets int32 [rows]; scale = 1 reproduces the reference (no 1/B). A target outside
 * [0, C) contributes no one-hot term (the row gets scale*softmax). */
int gn_xent_bwd(const void* logits, const int32_t* targets, void* dLogits, int rows, int C,
                float scale, int dtype, void* stream);

/* ---- attention ------------------------------------------------------------------------ */
/* Attention backward (attention-backward.glsl:73-194 semantics; RoPE of
 * flash-attention2-rope.glsl:73-145 applied to Q and K inside; causal mask j <= i).
 * Q, K, V, O, dO, dQ, dK, dV: [B, H, S, D]; LSE fp32 [B*H*S] = log sum_j exp(scale*q.k_j).
 * Q and K are the *pre-rotation* tensors; dQ, dK are gradients w.r.t. them.
 * rope_theta = base (10000); positions are 0..S-1.
 * ws: gn_attn_workspace_bytes(B, H, S, D) (or gn_attn_workspace_bytes_dtype).  D even, <= 256. */
int gn_attn_bwd(const void* Q, const void* K, const void* V, const void* O, const void* dO,
                const float* LSE, void* dQ, void* dK, void* dV, int B, int H, int S, int D,
                float scale, int causal, int rope_mode, float rope_theta, int dtype,
                void* ws, size_t ws_bytes, void* stream);

size_t gn_attn_workspace_bytes(int B, int H, int S, int D);

/* The attention workspace for one dtype (GN_F32 or GN_BF16): the largest layout among the
 * paths a call of that dtype and shape can take.  gn_attn_workspace_bytes is the larger of
 * the two.  Paths: bf16 with D = 64 or 128 runs the tuned matrix-core kernels; bf16 with
 * D = 32, 96, 192 or 256 and fp32 with D = 32, 64, 96, 128, 192 or 256 run the generic
 * matrix-core kernels (fp32 as a two-piece bf16 split with three products, fp32-grade);
 * other D (even, <= 256) and views that are not 16-byte aligned run SIMT kernels. */
size_t gn_attn_workspace_bytes_dtype(int B, int H, int S, int D, int dtype);

/* Same backward on the [B, S, H, D] layout with row strides, so a fused QKV projection
 * output [B*S, 3*H*D] feeds it (and its gradient buffer receives dQ, dK, dV) without head
 * transposes: element (b, h, s, d) of Q is Q[(b*S + s)*ld_qkv + h*D + d], K and V likewise
 * from their own base pointers with ld_qkv; O, dO use ld_o; dQ, dK, dV use ld_dqkv.  LSE
 * stays [B, H, S].  The reference binds attention on [B,H,S,D] only
 * (cpp/python/bindings.cpp:425-432); its FA2 forward runs on [B,S,H,D]
 * (flash-attention2.glsl:9,136-143), which is the layout accepted here.
 * bf16, D = 64 or 128; strides multiples of 8 and below 2^24 elements, pointers 16-byte
 * aligned; ws: gn_attn_workspace_bytes(B, H, S, D). */
int gn_attn_bwd_bshd(const void* Q, const void* K, const void* V, const void* O, const void* dO,
                     const float* LSE, void* dQ, void* dK, void* dV, int B, int H, int S, int D,
                     int64_t ld_qkv, int64_t ld_o, int64_t ld_dqkv, float scale, int causal,
                     int rope_mode, float rope_theta, int dtype, void* ws, size_t ws_bytes,
                     void* stream);

/* Attention forward producing the saved-tensor contract of the backward (O and the fp32
 * row logsumexp; flash-attention2-rope.glsl:165-247 semantics plus the causal mask).
 * Same arguments as gn_attn_bwd; ws as sized by gn_attn_workspace_bytes (needed only
 * when rope_mode != GN_ROPE_NONE or a key mask is given). */
int gn_attn_fwd(const void* Q, const void* K, const void* V, void* O, float* LSE, int B,
                int H, int S, int D, float scale, int causal, int rope_mode,
                float rope_theta, int dtype, void* ws, size_t ws_bytes, void* stream);

/* The three attention entries above with the reference's key-padding mask
 * (flash-attention2.glsl:150-154, flash-attention2-rope.glsl:201-205, bound with its mask by
 * flash_attention2 in cpp/python/bindings.cpp:415-450): key_mask fp32 [B, S], 1.0 = keep,
 * 0.0 = masked; the score of key k in batch b gets (key_mask[b*S + k] - 1) * 1e9, applied as
 * -inf where that bias is below -1e4 (so a masked key has P = dS = 0 exactly).  A row whose
 * visible keys are all masked gets O = 0, LSE = -inf and zero gradients (the reference's fp32
 * forward averages such a row uniformly instead).  key_mask NULL: no mask (the entries
 * above).  ws: gn_attn_workspace_bytes(B, H, S, D), 16-byte aligned. */
int gn_attn_fwd_mask(const void* Q, const void* K, const void* V, const float* key_mask, void* O,
                     float* LSE, int B, int H, int S, int D, float scale, int causal,
                     int rope_mode, float rope_theta, int dtype, void* ws, size_t ws_bytes,
                     void* stream);
int gn_attn_bwd_mask(const void* Q, const void* K, const void* V, const void* O, const void* dO,
                     const float* LSE, const float* key_mask, void* dQ, void* dK, void* dV, int B,
                     int H, int S, int D, float scale, int causal, int rope_mode,
                     float rope_theta, int dtype, void* ws, size_t ws_bytes, void* stream);
int gn_attn_bwd_bshd_mask(const void* Q, const void* K, const void* V, const void* O,
                          const void* dO, const float* LSE, const float* key_mask, void* dQ,
                          void* dK, void* dV, int B, int H, int S, int D, int64_t ld_qkv,
                          int64_t ld_o, int64_t ld_dqkv, float scale, int causal, int rope_mode,
                          float rope_theta, int dtype, void* ws, size_t ws_bytes, void* stream);

/* ---- VSA ------------------------------------------------------------------------------ */
/* backward_vsa_unpack_project (autograd.cpp:727-815), vsa-unpack-project-backward.glsl:42-74:
 *   s_b(j) = bit (j&31) of word X[b, j>>5] ? +1 : -1
 *   dW[o, j] (+)= sum_b dY[b, o] * s_b(j)   [O x D] fp32
 *   db[o]    (+)= sum_b dY[b, o]            [O] fp32 (skipped if NULL)
 * dY fp32 [Bn x O] (dtype GN_F32, fp32-accurate via a two-term bf16 split of dY) or bf16.
 * words = D/32 (D must be a multiple of 32).  ws (optional, 16-byte aligned):
 * gn_vsa_workspace_bytes(Bn, O) bytes (the transposed bf16 planes of dY).  The MFMA path runs
 * when the workspace is given and D % 128 == 0, Bn % 64 == 0, words % 4 == 0;
 * other calls take an LDS-staging kernel. */
int gn_vsa_unpack_project_bwd(const void* dY, const uint32_t* Xbits, float* dW, float* db,
                              int Bn, int O, int D, int words, int dtype, unsigned flags,
                              void* ws, size_t ws_bytes, void* stream);

size_t gn_vsa_workspace_bytes(int Bn, int O);

/* vsa-surrogate-loss-backward.glsl:50-88 (dispatch_vsa_loss_backward_with_buf,
 * vsa_loss_node.cpp:182-228):
 *   for each k, i: if gamma - y_i z[b,k,i] > 0: g[b,k,i] += -y_i/D * w[b,k] * scale
 *   if win != run and delta - (dot_win - dot_run) > 0: g[b,run,i] += y_i/D * lambda * scale
 * preds fp32 [Bn x K x D]; bits [Bn x words]; results u32 [Bn x 4] =
 * {win, run, f32bits(dot_win), f32bits(dot_run)}; weights fp32 [Bn x K].
 * Without GN_ACCUMULATE the output is overwritten (no memset needed). */
int gn_vsa_surrogate_bwd(const float* preds, const uint32_t* bits, const uint32_t* results,
                         const float* weights, float* dPreds, int Bn, int K, int D, int words,
                         float gamma, float delta, float lambda_c, float scale, unsigned flags,
                         void* stream);

/* VSA unpack-project forward (vsa-unpack-project.glsl:40-74; dispatch_vsa_unpack_project_forward,
 * vsa_loss_node.cpp:476-514): Y[b, o] = sum_j s_b(j) W[o, j] + bias[o], s_b(j) as in the
 * backward above.  Xbits [Bn x words] u32, W fp32 [O x D] (16-byte aligned), bias fp32 [O] or
 * NULL, Y fp32 [Bn x O]; D a multiple of 32, words = D/32.  Up to 8 rows per pass stream W
 * once (HBM-bound); with more rows and gn_vsa_fwd_workspace_bytes(Bn, O, D) bytes of ws
 * (16-byte aligned; Bn, O multiples of 8, D of 64) the contraction runs on the matrix cores
 * (+-1 exact in bf16, W as two bf16 terms: fp32 accuracy); otherwise one streaming pass per 8
 * rows. */
int gn_vsa_unpack_project_fwd(const uint32_t* Xbits, const float* W, const float* bias, float* Y,
                              int Bn, int O, int D, int words, void* ws, size_t ws_bytes,
                              void* stream);
size_t gn_vsa_fwd_workspace_bytes(int Bn, int O, int D);

/* VSA surrogate-loss forward (vsa-surrogate-loss-forward.glsl passes 0 and 1 and the top-2 /
 * softmax of dispatch_vsa_loss_forward, vsa_loss_node.cpp:36-180), per row b of preds fp32
 * [Bn x K x D] against the bipolar target bits [Bn x words]:
 *   dots[b, k] = sum_i preds[b, k, i] y_i                                   fp32 [Bn x K]
 *   win, run   = top-2 of dots[b, k] + temperature * g(seed, counter, b, k) (strict >, lower
 *                index kept on ties), g a standard Gumbel sample from a counter-based generator
 *                (splitmix64 of seed + ((counter * Bn + b) * K + k + 1) * 0x9E3779B97F4A7C15;
 *                u = (top 23 bits + 1/2) / 2^23; g = -log(-log u)); GN_NO_GUMBEL: g = 0
 *   results[b] = {win, run, f32bits(dots[b, win]), f32bits(dots[b, run])}  u32 [Bn x 4]
 *   weights[b] = softmax(dots[b, :] / temperature)                          fp32 [Bn x K]
 *   loss[b]    = mean_i max(gamma - y_i preds[b, win, i], 0)
 *                + lambda_c * max(0, delta - (dots[b, win] - dots[b, run]))  fp32 [Bn]
 * results and weights are the saved slots gn_vsa_surrogate_bwd reads.  K <= 64; D multiple
 * of 32; preds 16-byte aligned.  The reference draws the noise from an unseeded host RNG
 * (vsa_loss_node.cpp:9-14); here it is reproducible from (seed, counter). */
int gn_vsa_surrogate_fwd(const float* preds, const uint32_t* bits, float* dots, uint32_t* results,
                         float* weights, float* loss, int Bn, int K, int D, int words, float gamma,
                         float delta, float lambda_c, float temperature, uint64_t seed,
                         uint64_t counter, unsigned flags, void* stream);

/* ---- embedding ------------------------------------------------------------------------- */
/* Backward of a row gather X[t] = E[ids[t]] (token embeddings, tied with the LM head in the
 * decoder workload).  The reference tape has no embedding op; this entry serves the
 * Embedding node this build adds next to its OpTypes (autograd.h:81-141).
 *   dE[ids[t], :] (+)= dX[t, :]   dE fp32 [V x d]; dX [T x d] f32 or bf16; ids int32.
 * Without GN_ACCUMULATE dE is cleared first.  Rows with ids outside [0, V) are skipped.
 * Repeated ids are summed with fp32 atomics (order of additions not fixed). */
int gn_embedding_bwd(const void* dX, const int32_t* ids, float* dE, int T, int d, int V,
                     int dtype, unsigned flags, void* stream);

/* ---- the remaining tape ops ------------------------------------------------------------ */
/* The reference leaves these handlers as stubs that set a sentinel gradient id
 * (autograd.cpp:543-711); the formulas here are the textbook ones. */
#define GN_BIN_SUB 0 /* y = a - b: da = dy, db = -dy          (backward_sub :631-638) */
#define GN_BIN_MUL 1 /* y = a * b: da = dy b, db = dy a       (backward_mul :640-646) */
#define GN_BIN_DIV 2 /* y = a / b: da = dy / b, db = -dy a/b^2 (backward_div :648-654) */
#define GN_BIN_NEG 3 /* y = -a:    da = -dy */
/* Elementwise binary backward over n elements (no broadcasting); dA / dB nullable. */
int gn_binary_bwd(int op, const void* dY, const void* A, const void* B, void* dA, void* dB,
                  int64_t n, int dtype, unsigned flags, void* stream);

#define GN_RED_SUM 0  /* backward_sum  :695-700 */
#define GN_RED_MEAN 1 /* backward_mean :702-707 */
/* Backward of a reduction over the trailing `inner` elements of each of `outer` rows:
 * dX[o, i] (+)= dY[o] (x 1/inner for the mean). */
int gn_reduce_bwd(int op, const void* dY, void* dX, int64_t outer, int64_t inner, int dtype,
                  unsigned flags, void* stream);

/* Backward of a transpose of the last two dims (backward_transpose :689-693):
 * Y [batch, cols, rows] = X^T per batch, dX[b, r, c] (+)= dY[b, c, r]. */
int gn_transpose_bwd(const void* dY, void* dX, int64_t batch, int rows, int cols, int dtype,
                     unsigned flags, void* stream);

/* MSE loss backward (backward_mse :663-667): loss = scale * sum (pred - target)^2, so
 * dPred (+)= 2 scale (pred - target) g, g = dLoss[0] (dLoss NULL: g = 1). */
int gn_mse_bwd(const void* pred, const void* target, const float* dLoss, void* dPred, int64_t n,
               float scale, int dtype, unsigned flags, void* stream);

/* VSA LoRA-expand backward (backward_vsa_lora_expand autograd.cpp:817-843,
 * vsa-lora-expand-backward.glsl:38-63): forward preds[b,k,:] = B coeffs[b,k,:] with B [D x rank];
 *   dCoeffs [Bn*K x rank] = scale dPreds B,   dBasis [D x rank] (+)= scale dPreds^T coeffs.
 * All fp32; scale must be 1, the value the reference handler passes (autograd.cpp:834).
 * GN_ACCUMULATE adds into dBasis (the shader's grad_B +=) and dCoeffs. */
int gn_vsa_lora_expand_bwd(const float* dPreds, const float* basis, const float* coeffs,
                           float* dCoeffs, float* dBasis, int Bn, int K, int D, int rank,
                           float scale, unsigned flags, void* stream);

/* VSA cosine-blend loss backward (backward_vsa_cosine_blend_loss autograd.cpp:845-859,
 * vsa-cosine-blend-backward.glsl:37-70): with b = blended[b,:], y = +-1 from true_bits,
 * loss_info[b] = {loss, dot(b, y), |b|^2}:
 *   gb_i = -(y_i / (|b| sqrt(D)) - cos b_i / max(|b|^2, 1e-8)),  |b| = sqrt(max(|b|^2, 1e-8))
 *   dPreds[b,k,i] (+)= clamp(gb_i weights[b,k] grad_scale, -1, 1)
 * (the reference handler uses grad_scale 10 on a zeroed buffer). */
int gn_vsa_cosine_blend_bwd(const uint32_t* true_bits, const float* weights,
                            const float* blended, const float* loss_info, float* dPreds, int Bn,
                            int K, int D, int words, float grad_scale, unsigned flags,
                            void* stream);

/* ---- optimizer steps (between TapeContext.backward and end) ---------------------------- */
/* One parameter tensor of a multi-tensor optimizer step (all fp32, n elements). */
typedef struct gn_opt_param {
    float* W;              /* weights, updated in place */
    float* grad;           /* gradient; zeroed afterwards when clear_grad != 0 */
    float* state0;         /* AdamW: first moment m;  surprise-momentum: s_bar */
    float* state1;         /* AdamW: second moment v; surprise-momentum: delta output (may be NULL) */
    const float* recalled; /* surprise-momentum: recalled gradient (NULL reads as zero) */
    void* W_bf16;          /* optional bf16 copy of the updated W (NULL: none) */
    int64_t n;
} gn_opt_param;

/* Surprise-momentum update of `count` tensors: replaces the per-parameter, per-128 MB-chunk
 * dispatches of surprise-momentum.glsl in vsa_training_step (bindings.cpp:3198-3277) with
 * one launch per 24 tensors.  Per element (surprise-momentum.glsl:53-114):
 *   g, r non-finite -> delta = 0, W and s_bar unchanged;  else
 *   s = min(alpha |g - r| + (1 - alpha) s_bar (non-finite s_bar read as 0), 5);
 *   d = clamp(eta (1 + max(s, floor)) (g + lambda r) + eta wd W, -clip, clip);
 *   W = clamp(W - d (non-finite -> 0), -10, 10);  s_bar = s;  delta = d;
 *   grad = 0 when clear_grad.  params is a host array (read before the call returns). */
int gn_surprise_momentum_step(const gn_opt_param* params, int count, float eta_base,
                              float alpha_momentum, float lambda_recall, float surprise_floor,
                              float weight_decay, float clip_max, int clear_grad, void* stream);

/* fp32 Linear backward of M <= 8 rows with the weight's surprise-momentum step fused into the
 * same pass over W: the backward of bwd_linear (autograd.cpp:172-305: dX = dY W, db = sum of
 * dY's rows) and, in place of storing dW = dY^T X, the update above with that dW as g and no
 * recalled gradient (r = 0, as vsa_training_step runs the optimizer: bindings.cpp:3045-3047,
 * 3198-3277), applied to W and s_bar [N x K] in place.  dX is computed from W before its
 * update; dW is never written (the pass moves 16 bytes per weight instead of the 8 of the
 * backward plus the 20 of the optimizer).  The result equals gn_linear_bwd_ws followed by
 * gn_surprise_momentum_step on the produced dW, bit for bit.  dX and db may be NULL.  Takes K a
 * multiple of 4 up to 4096 and 16-byte aligned X, W, s_bar, dX; other shapes return
 * GN_E_INVALID (run the two calls instead).  ws: gn_linear_workspace_bytes(M, N, K, GN_F32)
 * makes dX deterministic, as for gn_linear_bwd_ws. */
int gn_linear_bwd_surprise_momentum(const void* dY, const void* X, void* W, float* s_bar, void* dX,
                                    void* db, int M, int N, int K, float eta_base,
                                    float alpha_momentum, float lambda_recall, float surprise_floor,
                                    float weight_decay, float clip_max, void* ws, size_t ws_bytes,
                                    void* stream);

/* AdamW update of `count` tensors (adamw-update.glsl:41-61; adam-update.glsl is weight_decay
 * 0).  beta1_t, beta2_t = beta^t for bias correction at step t >= 1, as the shader's push
 * constants.  Per element: m = b1 m + (1-b1) g;  v = b2 v + (1-b2) g^2;
 *   W = W (1 - lr wd) - lr (m / max(1e-12, 1-b1t)) / (sqrt(max(v / max(1e-12, 1-b2t), 0)) + eps)
 * grad = 0 when clear_grad; W_bf16 (if given) receives the rounded new W. */
int gn_adamw_step(const gn_opt_param* params, int count, float lr, float beta1, float beta2,
                  float eps, float weight_decay, float beta1_t, float beta2_t, int clear_grad,
                  void* stream);

/* ---- forward kernels producing the saved tensors the backward consumes ----------------- */
/* LayerNorm forward (fnn-layernorm.glsl:44-102): Y = (X - mean)/sqrt(var + eps) * gamma + beta
 * with the biased variance; mean, rstd fp32 [rows] (the `rstd` array gets the variance, as
 * the reference's var_vals buffer, with GN_LN_STAT_VAR).  gamma/beta NULL: 1/0; mean/rstd
 * NULL: not saved.  Feeds gn_layernorm_bwd with the same flags. */
int gn_layernorm_fwd(const void* X, const void* gamma, const void* beta, void* Y, float* mean,
                     float* rstd, int rows, int F, float eps, int dtype, unsigned flags,
                     void* stream);

/* RMSNorm forward (rms-norm.glsl:34-70): Y = w * X * rsqrt(mean(X^2) + eps); rstd fp32 [rows]
 * (the reference saves mean(X^2); the backward here takes rstd).  w NULL: 1. */
int gn_rmsnorm_fwd(const void* X, const void* w, void* Y, float* rstd, int rows, int F, float eps,
                   int dtype, void* stream);

/* The two norm forwards with X in x_dtype and gamma / beta / w and Y in y_dtype (pairs as the
 * _ex backwards: a residual stream kept in fp32 normalised into a bf16 block). */
int gn_layernorm_fwd_ex(const void* X, int x_dtype, const void* gamma, const void* beta, void* Y,
                        int y_dtype, float* mean, float* rstd, int rows, int F, float eps,
                        unsigned flags, void* stream);
int gn_rmsnorm_fwd_ex(const void* X, int x_dtype, const void* w, void* Y, int y_dtype, float* rstd,
                      int rows, int F, float eps, void* stream);
/* gn_rmsnorm_fwd_ex saving the statistic in the reference's forms: GN_RMS_STAT_MEANSQ writes
 * mean(x^2) (rms-norm.glsl:52), GN_RMS_STAT_RMS writes sqrt(mean(x^2) + eps)
 * (snn-rmsnorm.glsl:55), neither writes rstd.  Feeds gn_rmsnorm_bwd_stat with the same flag. */
int gn_rmsnorm_fwd_stat(const void* X, int x_dtype, const void* w, void* Y, int y_dtype,
                        float* stat, int rows, int F, float eps, unsigned flags, void* stream);

/* Activation forward Y = act(X) over n elements (activation-{relu,gelu,silu}.glsl forward
 * values; the GN_ACT_* kinds: tanh-form GELU by default, erf form, SiLU, tanh, sigmoid).  The
 * backward of GN_ACT_TANH / GN_ACT_SIGMOID then takes this Y, the others take X. */
int gn_act_fwd(int kind, const void* X, void* Y, int64_t n, int dtype, void* stream);

/* GLU product out = glu_kind(gate, up) over n elements (fused-swiglu.glsl:78,
 * fused-geglu.glsl:81, fused-reglu.glsl:73; kinds GN_GLU_*). */
int gn_glu_fwd(int kind, const void* gate, const void* up, void* out, int64_t n, int dtype,
               void* stream);

/* Linear forward (fnn-linear.glsl:33-55): Y [M x N] = X [M x K] W^T + b, W [N x K], b [N] or NULL,
 * all in dtype (fp32 accumulation; bf16 rounds Y once). */
int gn_linear_fwd(const void* X, const void* W, const void* b, void* Y, int M, int N, int K,
                  int dtype, void* stream);

/* Fused GLU projection forward (fused-swiglu.glsl:48-79 and its GEGLU/ReGLU twins):
 * gate = X Wg^T + bg, up = X Wu^T + bu (both kept: the backward's gate/up caches,
 * fused-swiglu-backward.glsl:26-34), out = glu_kind(gate, up).  X [M x K], Wg/Wu [H x K],
 * bg/bu [H] or NULL; gate, up, out [M x H]. */
int gn_glu_linear_fwd(int kind, const void* X, const void* Wg, const void* Wu, const void* bg,
                      const void* bu, void* gate, void* up, void* out, int M, int H, int K,
                      int dtype, void* stream);

/* ---- misc ------------------------------------------------------------------------------ */
/* out[i] (+)= a[i] (f32/bf16): the fan-out accumulation the reference leaves as a TODO
 * (autograd.cpp:78-86). */
int gn_add_inplace(void* out, const void* a, int64_t n, int dtype, void* stream);

/* dst = src in another storage type (f32 -> bf16 rounds to nearest-even; bf16 -> f32 exact):
 * the gradient of a bf16 tensor added into an fp32 stream (an Add node whose inputs differ in
 * dtype) is the fp32 upstream gradient rounded once.  src_dtype == dst_dtype is a bit-exact
 * copy (the tape's fan-out copy of a borrowed gradient). */
int gn_convert(const void* src, int src_dtype, void* dst, int dst_dtype, int64_t n, void* stream);

/* dst[0, bytes) = 0 with a fill kernel.  No entry point of this library calls hipMemsetAsync,
 * hipMalloc or a synchronising HIP call, so any sequence of them (the tape's backward among
 * them) can be captured into a HIP graph and replayed: the graph holds kernel nodes only.
 * Replaces the host memset of a mapped gradient buffer the reference does before each
 * accumulating dispatch (cpp/src/autograd.cpp:223-226, 507, 721), which a device-resident
 * buffer cannot take. */
int gn_zero(void* dst, int64_t bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GN_BWD_H */
