/*
 * oracle.h — CPU restatement of grilly-next's backward formulas.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load liboracle.so, and only as the checker or as the timed CPU
 * baseline; the product path (libgn_bwd.so, grilly_core) never links or calls it.
 *
 * All functions take fp32 host arrays and accumulate in fp64.  Each cites the reference
 * file:line it restates; the pins for each function are listed in tests/test_oracle.py.
 * Parity status: every function below is pinned (golden vectors from an independent
 * torch-fp64 autograd restatement, closed forms, reference known-answer tests).
 */
#ifndef GN_ORACLE_H
#define GN_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* fnn-linear-backward.glsl:47-89; autograd_core.py:511-513 */
void or_linear_bwd(const float* dY, const float* X, const float* W, float* dX, float* dW,
                   float* db, int M, int N, int K);
/* forward y = X W^T + b (fnn-linear.glsl), used to build saved tensors */
void or_linear_fwd(const float* X, const float* W, const float* b, float* Y, int M, int N,
                   int K);

/* activation-*-backward.glsl; kinds as GN_ACT_* in include/gn_bwd.h */
void or_act_bwd(int kind, const float* dY, const float* X, float* dX, int64_t n);
void or_act_fwd(int kind, const float* X, float* Y, int64_t n);

/* fused-{swiglu,geglu,reglu}-backward.glsl local gradients; kinds as GN_GLU_* */
void or_glu_bwd(int kind, const float* dO, const float* gate, const float* up, float* dGate,
                float* dUp, int64_t n);
void or_glu_fwd(int kind, const float* gate, const float* up, float* out, int64_t n);

/* Textbook LayerNorm backward (autograd_core.py:591-609). stat_is_var: rstd holds var. */
void or_layernorm_bwd(const float* dY, const float* X, const float* gamma, const float* mean,
                      const float* rstd, float* dX, float* dGamma, float* dBeta, int rows,
                      int F, float eps, int stat_is_var);
/* The reference GLSL form (fnn-layernorm-backward.glsl:124), kept to pin the gamma==1
 * agreement with the textbook form. */
void or_layernorm_bwd_glsl(const float* dY, const float* X, const float* gamma,
                           const float* mean, const float* rstd, float* dX, int rows, int F);
/* fnn-layernorm.glsl:44-102: biased variance; returns mean and rstd */
void or_layernorm_fwd(const float* X, const float* gamma, const float* beta, float* Y,
                      float* mean, float* rstd, int rows, int F, float eps);

/* RMSNorm (rms-norm.glsl:34-70 forward; backward by closed form) */
void or_rmsnorm_bwd(const float* dY, const float* X, const float* w, const float* rstd,
                    float* dX, float* dW, int rows, int F);
void or_rmsnorm_fwd(const float* X, const float* w, float* Y, float* rstd, int rows, int F,
                    float eps);

/* activation-softmax-backward.glsl:27-49 */
void or_softmax_bwd(const float* dY, const float* Y, float* dX, int rows, int C);
void or_softmax_fwd(const float* X, float* Y, int rows, int C);

/* cross-entropy-backward.glsl:29-84 (targets as int32) */
void or_xent_bwd(const float* logits, const int32_t* targets, float* dLogits, int rows, int C,
                 float scale);

/* RoPE rotation of one [S, D] head in place (flash-attention2-rope.glsl:74-91 interleaved,
 * rope.glsl:74-125 rotate-half); inverse = 1 applies R^T. */
void or_rope(float* X, int S, int D, int mode, float theta, int inverse);

/* attention-backward.glsl:73-194 / autograd_core.py:638-654 with causal mask and RoPE.
 * P is recomputed from LSE; D_i = sum_j P_ij dP_ij as in the reference pass 2. */
void or_attn_bwd(const float* Q, const float* K, const float* V, const float* dO,
                 const float* LSE, float* dQ, float* dK, float* dV, int B, int H, int S, int D,
                 float scale, int causal, int rope_mode, float theta, const float* mask);
void or_attn_fwd(const float* Q, const float* K, const float* V, float* O, float* LSE, int B,
                 int H, int S, int D, float scale, int causal, int rope_mode, float theta,
                 const float* mask);

/* vsa-unpack-project-backward.glsl:42-74 */
void or_unpack_bits(const uint32_t* bits, float* out, int Bn, int D, int words);
void or_vsa_unpack_project_bwd(const float* dY, const uint32_t* bits, float* dW, float* db,
                               int Bn, int O, int D, int words);

/* vsa-surrogate-loss-backward.glsl:50-88; accumulate=0 starts from zero */
void or_vsa_surrogate_bwd(const float* preds, const uint32_t* bits, const uint32_t* results,
                          const float* weights, float* dPreds, int Bn, int K, int D, int words,
                          float gamma, float delta, float lambda_c, float scale,
                          int accumulate);
/* vsa-surrogate-loss-forward.glsl pass 0 (dots) */
void or_vsa_dots(const float* preds, const uint32_t* bits, float* dots, int Bn, int K, int D,
                 int words);

/* vsa-unpack-project.glsl:40-74 (forward): Y[b, o] = sum_j s_b(j) W[o, j] + bias[o] */
void or_vsa_unpack_project_fwd(const uint32_t* bits, const float* W, const float* bias, float* Y,
                               int Bn, int O, int D, int words);
/* counter-based Gumbel noise of the surrogate forward (splitmix64; replaces the reference's
 * unseeded std::mt19937, vsa_loss_node.cpp:9-14) */
uint64_t or_mix64(uint64_t seed, uint64_t idx);
float or_gumbel(uint64_t seed, uint64_t idx);
/* vsa_loss_node.cpp:101-148: top-2 of dots + T g and softmax(dots / T) from given dots */
void or_vsa_select(const float* dots, uint32_t* results, float* weights, int Bn, int K,
                   float temperature, uint64_t seed, uint64_t counter, int noise);
/* vsa-surrogate-loss-forward.glsl pass 1 (hinge on the winner + contrastive margin) */
void or_vsa_surrogate_loss(const float* preds, const uint32_t* bits, const uint32_t* results,
                           float* loss, int Bn, int K, int D, int words, float gamma,
                           float delta, float lambda_c);

/* Sub / Mul / Div / Neg backward (op as GN_BIN_*; stubs at autograd.cpp:631-654) */
void or_binary_bwd(int op, const float* dY, const float* A, const float* B, float* dA, float* dB,
                   int64_t n);
/* Sum / Mean backward over the trailing `inner` elements (stubs at autograd.cpp:695-707) */
void or_reduce_bwd(int op, const float* dY, float* dX, int64_t outer, int64_t inner);
/* Transpose backward of the last two dims: dX[b, r, c] = dY[b, c, r] (autograd.cpp:689-693) */
void or_transpose_bwd(const float* dY, float* dX, int64_t batch, int rows, int cols);
/* MSE backward: dP = 2 scale (P - T) g (autograd.cpp:663-667) */
void or_mse_bwd(const float* P, const float* T, float g, float* dP, int64_t n, float scale);
/* vsa-lora-expand-backward.glsl:38-63 with grad_scale: dC = s dP B, dB = s dP^T C */
void or_lora_expand_bwd(const float* dP, const float* basis, const float* coeffs, float* dC,
                        float* dB, int BK, int D, int rank, float scale);
/* vsa-cosine-blend-backward.glsl:37-70 (dPreds overwritten) */
void or_cosine_blend_bwd(const uint32_t* bits, const float* weights, const float* blended,
                         const float* info, float* dP, int Bn, int K, int D, int words,
                         float grad_scale);

/* surprise-momentum.glsl:53-114, one tensor (recalled / delta may be NULL); updates W, s_bar,
 * delta and (clear_grad) grad in place */
void or_surprise_momentum_step(float* W, float* grad, float* s_bar, float* delta,
                               const float* recalled, int64_t n, float eta_base, float alpha,
                               float lambda_recall, float surprise_floor, float weight_decay,
                               float clip_max, int clear_grad);
/* adamw-update.glsl:41-61 (adam-update.glsl with weight_decay 0), one tensor, in place */
void or_adamw_step(float* W, float* grad, float* m, float* v, int64_t n, float lr, float beta1,
                   float beta2, float eps, float weight_decay, float beta1_t, float beta2_t,
                   int clear_grad);

int or_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
