/*
 * oracle.c — CPU restatement of grilly-next's backward formulas (fp32 in/out, fp64
 * accumulation, OpenMP over rows).
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg, never by the product path.  Each function cites the reference text
 * it restates (paths relative to the grilly-next repository root).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int or_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ---------------------------------------------------------------- linear ---------- */
/* fnn-linear-backward.glsl:47-89 (pass 0: dX = dY W, pass 1: dW = dY^T X, pass 2:
 * db = column sums), autograd_core.py:511-513. */
void or_linear_bwd(const float* dY, const float* X, const float* W, float* dX, float* dW,
                   float* db, int M, int N, int K) {
    if (dX) {
#pragma omp parallel
        {
            double* acc = (double*)malloc(sizeof(double) * (size_t)K);
#pragma omp for schedule(static)
            for (int m = 0; m < M; ++m) {
                for (int k = 0; k < K; ++k) acc[k] = 0.0;
                for (int n = 0; n < N; ++n) {
                    const double a = dY[(size_t)m * N + n];
                    const float* w = W + (size_t)n * K;
                    for (int k = 0; k < K; ++k) acc[k] += a * (double)w[k];
                }
                for (int k = 0; k < K; ++k) dX[(size_t)m * K + k] = (float)acc[k];
            }
            free(acc);
        }
    }
    if (dW) {
#pragma omp parallel
        {
            double* acc = (double*)malloc(sizeof(double) * (size_t)K);
#pragma omp for schedule(static)
            for (int n = 0; n < N; ++n) {
                for (int k = 0; k < K; ++k) acc[k] = 0.0;
                for (int m = 0; m < M; ++m) {
                    const double a = dY[(size_t)m * N + n];
                    const float* x = X + (size_t)m * K;
                    for (int k = 0; k < K; ++k) acc[k] += a * (double)x[k];
                }
                for (int k = 0; k < K; ++k) dW[(size_t)n * K + k] = (float)acc[k];
            }
            free(acc);
        }
    }
    if (db) {
        for (int n = 0; n < N; ++n) {
            double s = 0.0;
            for (int m = 0; m < M; ++m) s += dY[(size_t)m * N + n];
            db[n] = (float)s;
        }
    }
}

void or_linear_fwd(const float* X, const float* W, const float* b, float* Y, int M, int N,
                   int K) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            double s = b ? (double)b[n] : 0.0;
            for (int k = 0; k < K; ++k) s += (double)X[(size_t)m * K + k] * W[(size_t)n * K + k];
            Y[(size_t)m * N + n] = (float)s;
        }
}

/* ---------------------------------------------------------------- activations ----- */
static const double kSqrt2OverPi = 0.7978845608028654;
static const double kGeluCoeff = 0.044715;

static double sigmoid_d(double x) { return 1.0 / (1.0 + exp(-x)); }
static double silu_d(double x) { return x * sigmoid_d(x); }
/* activation-silu-backward.glsl:25-42 */
static double silu_grad_d(double x) {
    double s = sigmoid_d(x);
    return s * (1.0 + x * (1.0 - s));
}
/* fused-geglu-backward.glsl:69-73 */
static double gelu_tanh_d(double x) {
    return 0.5 * x * (1.0 + tanh(kSqrt2OverPi * (x + kGeluCoeff * x * x * x)));
}
/* activation-gelu-backward.glsl:38-50 */
static double gelu_tanh_grad_d(double x) {
    double z = kSqrt2OverPi * (x + kGeluCoeff * x * x * x);
    double t = tanh(z);
    double sech2 = 1.0 - t * t;
    double dz = kSqrt2OverPi * (1.0 + 3.0 * kGeluCoeff * x * x);
    return 0.5 * (1.0 + t + x * sech2 * dz);
}
/* autograd_core.py:529-542 (erf form): Phi(x) + x phi(x) */
static double gelu_erf_grad_d(double x) {
    double phi_cdf = 0.5 * (1.0 + erf(x / sqrt(2.0)));
    double pdf = exp(-0.5 * x * x) / sqrt(2.0 * M_PI);
    return phi_cdf + x * pdf;
}

void or_act_bwd(int kind, const float* dY, const float* X, float* dX, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        double x = X[i], dy = dY[i], g = 0.0;
        switch (kind) {
            case 0: g = (x > 0.0) ? 1.0 : 0.0; break;        /* activation-relu-backward.glsl:33-37 */
            case 1: g = gelu_tanh_grad_d(x); break;
            case 2: g = gelu_erf_grad_d(x); break;
            case 3: g = silu_grad_d(x); break;
            case 4: g = 1.0 - x * x; break;                  /* activation-tanh-backward.glsl:33 */
            case 5: g = x * (1.0 - x); break;                /* sigmoid, x = saved output */
            default: g = 0.0;
        }
        dX[i] = (float)(dy * g);
    }
}

void or_act_fwd(int kind, const float* X, float* Y, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        double x = X[i], y = 0.0;
        switch (kind) {
            case 0: y = x > 0.0 ? x : 0.0; break;
            case 1: y = gelu_tanh_d(x); break;
            case 2: y = 0.5 * x * (1.0 + erf(x / sqrt(2.0))); break;
            case 3: y = silu_d(x); break;
            case 4: y = tanh(x); break;
            case 5: y = sigmoid_d(x); break;
            default: y = 0.0;
        }
        Y[i] = (float)y;
    }
}

/* ---------------------------------------------------------------- GLU ------------- */
/* Local gradients of fused-swiglu-backward.glsl:93-100 (gate*SiLU(up)),
 * fused-geglu-backward.glsl:99-103 (gate*GELU(up)), fused-reglu-backward.glsl:83-86
 * (gate*ReLU(up)); the *_GATE kinds apply the activation to the gate instead
 * (swiglu-fused.glsl:60-64). */
void or_glu_bwd(int kind, const float* dO, const float* gate, const float* up, float* dGate,
                float* dUp, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        double g = gate[i], u = up[i], d = dO[i], dg = 0.0, du = 0.0;
        switch (kind) {
            case 0: dg = d * silu_d(u); du = d * g * silu_grad_d(u); break;
            case 1: dg = d * u * silu_grad_d(g); du = d * silu_d(g); break;
            case 2: dg = d * gelu_tanh_d(u); du = d * g * gelu_tanh_grad_d(u); break;
            case 3: dg = d * u * gelu_tanh_grad_d(g); du = d * gelu_tanh_d(g); break;
            case 4: dg = d * (u > 0.0 ? u : 0.0); du = d * g * (u > 0.0 ? 1.0 : 0.0); break;
            default: break;
        }
        dGate[i] = (float)dg;
        dUp[i] = (float)du;
    }
}

void or_glu_fwd(int kind, const float* gate, const float* up, float* out, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        double g = gate[i], u = up[i], y = 0.0;
        switch (kind) {
            case 0: y = g * silu_d(u); break;
            case 1: y = silu_d(g) * u; break;
            case 2: y = g * gelu_tanh_d(u); break;
            case 3: y = gelu_tanh_d(g) * u; break;
            case 4: y = g * (u > 0.0 ? u : 0.0); break;
            default: break;
        }
        out[i] = (float)y;
    }
}

/* ---------------------------------------------------------------- LayerNorm ------- */
/* Textbook LayerNorm backward: the numpy fallback autograd_core.py:591-609, which is
 * algebraically dx = rstd*(g - mean(g) - xhat*mean(g*xhat)) with g = dy*gamma. */
void or_layernorm_bwd(const float* dY, const float* X, const float* gamma, const float* mean,
                      const float* rstd, float* dX, float* dGamma, float* dBeta, int rows,
                      int F, float eps, int stat_is_var) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const float* x = X + (size_t)r * F;
        const float* dy = dY + (size_t)r * F;
        double mu = mean[r];
        double rs = stat_is_var ? 1.0 / sqrt((double)rstd[r] + eps) : (double)rstd[r];
        double s1 = 0.0, s2 = 0.0;
        for (int f = 0; f < F; ++f) {
            double xh = (x[f] - mu) * rs, g = (double)dy[f] * gamma[f];
            s1 += g;
            s2 += g * xh;
        }
        s1 /= F;
        s2 /= F;
        if (dX)
            for (int f = 0; f < F; ++f) {
                double xh = (x[f] - mu) * rs, g = (double)dy[f] * gamma[f];
                dX[(size_t)r * F + f] = (float)(rs * (g - s1 - xh * s2));
            }
    }
    if (dGamma || dBeta) {
        for (int f = 0; f < F; ++f) {
            double sg = 0.0, sb = 0.0;
            for (int r = 0; r < rows; ++r) {
                double rs = stat_is_var ? 1.0 / sqrt((double)rstd[r] + eps) : (double)rstd[r];
                double xh = (X[(size_t)r * F + f] - (double)mean[r]) * rs;
                double dy = dY[(size_t)r * F + f];
                sg += dy * xh;
                sb += dy;
            }
            if (dGamma) dGamma[f] = (float)sg;
            if (dBeta) dBeta[f] = (float)sb;
        }
    }
}

/* fnn-layernorm-backward.glsl:83-124 as written: gamma multiplies the mean terms too. */
void or_layernorm_bwd_glsl(const float* dY, const float* X, const float* gamma,
                           const float* mean, const float* rstd, float* dX, int rows, int F) {
    for (int r = 0; r < rows; ++r) {
        double mu = mean[r], rs = rstd[r], s1 = 0.0, s2 = 0.0;
        for (int f = 0; f < F; ++f) {
            double xh = (X[(size_t)r * F + f] - mu) * rs;
            double g = (double)dY[(size_t)r * F + f] * gamma[f];
            s1 += g;
            s2 += g * xh;
        }
        for (int f = 0; f < F; ++f) {
            double xh = (X[(size_t)r * F + f] - mu) * rs;
            double dy = dY[(size_t)r * F + f];
            dX[(size_t)r * F + f] = (float)(rs * gamma[f] * (dy - (s1 + xh * s2) / F));
        }
    }
}

/* fnn-layernorm.glsl:44-102: mean, biased variance, y = gamma*(x-mean)*rstd + beta */
void or_layernorm_fwd(const float* X, const float* gamma, const float* beta, float* Y,
                      float* mean, float* rstd, int rows, int F, float eps) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const float* x = X + (size_t)r * F;
        double mu = 0.0, var = 0.0;
        for (int f = 0; f < F; ++f) mu += x[f];
        mu /= F;
        for (int f = 0; f < F; ++f) var += (x[f] - mu) * (x[f] - mu);
        var /= F;
        double rs = 1.0 / sqrt(var + eps);
        mean[r] = (float)mu;
        rstd[r] = (float)rs;
        if (Y)
            for (int f = 0; f < F; ++f)
                Y[(size_t)r * F + f] =
                    (float)(gamma[f] * (x[f] - mu) * rs + (beta ? beta[f] : 0.0f));
    }
}

/* ---------------------------------------------------------------- RMSNorm --------- */
/* Closed form for y = w * x * r, r = (mean(x^2)+eps)^-1/2 (rms-norm.glsl:34-70):
 *   dx_i = r w_i dy_i - x_i r^3 (1/F) sum_j w_j dy_j x_j ;  dw_i = sum_rows dy_i x_i r */
void or_rmsnorm_bwd(const float* dY, const float* X, const float* w, const float* rstd,
                    float* dX, float* dW, int rows, int F) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const float* x = X + (size_t)r * F;
        const float* dy = dY + (size_t)r * F;
        double rs = rstd[r], s = 0.0;
        for (int f = 0; f < F; ++f) s += (double)w[f] * dy[f] * x[f];
        s /= F;
        if (dX)
            for (int f = 0; f < F; ++f)
                dX[(size_t)r * F + f] = (float)(rs * w[f] * dy[f] - x[f] * rs * rs * rs * s);
    }
    if (dW)
        for (int f = 0; f < F; ++f) {
            double s = 0.0;
            for (int r = 0; r < rows; ++r)
                s += (double)dY[(size_t)r * F + f] * X[(size_t)r * F + f] * rstd[r];
            dW[f] = (float)s;
        }
}

void or_rmsnorm_fwd(const float* X, const float* w, float* Y, float* rstd, int rows, int F,
                    float eps) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const float* x = X + (size_t)r * F;
        double ms = 0.0;
        for (int f = 0; f < F; ++f) ms += (double)x[f] * x[f];
        ms /= F;
        double rs = 1.0 / sqrt(ms + eps);
        rstd[r] = (float)rs;
        if (Y)
            for (int f = 0; f < F; ++f) Y[(size_t)r * F + f] = (float)(w[f] * x[f] * rs);
    }
}

/* ---------------------------------------------------------------- softmax / CE ---- */
/* activation-softmax-backward.glsl:36-48 */
void or_softmax_bwd(const float* dY, const float* Y, float* dX, int rows, int C) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        double dot = 0.0;
        for (int c = 0; c < C; ++c) dot += (double)dY[(size_t)r * C + c] * Y[(size_t)r * C + c];
        for (int c = 0; c < C; ++c) {
            size_t i = (size_t)r * C + c;
            dX[i] = (float)(Y[i] * (dY[i] - dot));
        }
    }
}

void or_softmax_fwd(const float* X, float* Y, int rows, int C) {
    for (int r = 0; r < rows; ++r) {
        double mx = -INFINITY, s = 0.0;
        for (int c = 0; c < C; ++c) mx = fmax(mx, X[(size_t)r * C + c]);
        for (int c = 0; c < C; ++c) s += exp(X[(size_t)r * C + c] - mx);
        for (int c = 0; c < C; ++c) Y[(size_t)r * C + c] = (float)(exp(X[(size_t)r * C + c] - mx) / s);
    }
}

/* cross-entropy-backward.glsl:41-84: row max, sum exp, softmax - onehot (no 1/B). */
void or_xent_bwd(const float* logits, const int32_t* targets, float* dLogits, int rows, int C,
                 float scale) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const float* z = logits + (size_t)r * C;
        double mx = -INFINITY, s = 0.0;
        for (int c = 0; c < C; ++c) mx = fmax(mx, z[c]);
        for (int c = 0; c < C; ++c) s += exp(z[c] - mx);
        for (int c = 0; c < C; ++c) {
            double g = exp(z[c] - mx) / s;
            if (c == targets[r]) g -= 1.0;
            dLogits[(size_t)r * C + c] = (float)(scale * g);
        }
    }
}

/* ---------------------------------------------------------------- RoPE ------------ */
/* flash-attention2-rope.glsl:74-91: theta_i(pos) = pos * base^(-2i/D),
 * (x0, x1) -> (x0 c - x1 s, x0 s + x1 c); mode 1 pairs (2i, 2i+1), mode 2 pairs
 * (i, i+D/2) as in rope.glsl. inverse applies the transpose rotation. */
void or_rope(float* X, int S, int D, int mode, float theta, int inverse) {
    if (mode == 0) return;
    for (int p = 0; p < S; ++p)
        for (int i = 0; i < D / 2; ++i) {
            double ang = (double)p * pow((double)theta, -2.0 * i / (double)D);
            double c = cos(ang), s = sin(ang);
            if (inverse) s = -s;
            int i0 = (mode == 1) ? 2 * i : i;
            int i1 = (mode == 1) ? 2 * i + 1 : i + D / 2;
            double x0 = X[(size_t)p * D + i0], x1 = X[(size_t)p * D + i1];
            X[(size_t)p * D + i0] = (float)(x0 * c - x1 * s);
            X[(size_t)p * D + i1] = (float)(x0 * s + x1 * c);
        }
}

static void rope_d(double* X, int S, int D, int mode, double theta, int inverse) {
    if (mode == 0) return;
    for (int p = 0; p < S; ++p)
        for (int i = 0; i < D / 2; ++i) {
            double ang = (double)p * pow(theta, -2.0 * i / (double)D);
            double c = cos(ang), s = sin(ang);
            if (inverse) s = -s;
            int i0 = (mode == 1) ? 2 * i : i;
            int i1 = (mode == 1) ? 2 * i + 1 : i + D / 2;
            double x0 = X[(size_t)p * D + i0], x1 = X[(size_t)p * D + i1];
            X[(size_t)p * D + i0] = x0 * c - x1 * s;
            X[(size_t)p * D + i1] = x0 * s + x1 * c;
        }
}

/* ---------------------------------------------------------------- attention ------- */
/* Key-padding bias of flash-attention2.glsl:150-154 (flash-attention2-rope.glsl:201-205):
 * score += (mask[b*S + k] - 1) * 1e9; 0 without a mask. */
static double key_bias(const float* mask, int b, int S, int k) {
    return mask ? ((double)mask[(size_t)b * S + k] - 1.0) * 1e9 : 0.0;
}

/* Forward with the saved-tensor contract: O and LSE_i = log sum_j exp(scale q_i.k_j + bias_j),
 * RoPE applied to Q and K (flash-attention2-rope.glsl:95-148), causal mask j <= i, key-padding
 * bias from `mask` [B, S] (nullable). */
void or_attn_fwd(const float* Q, const float* K, const float* V, float* O, float* LSE, int B,
                 int H, int S, int D, float scale, int causal, int rope_mode, float theta,
                 const float* mask) {
#pragma omp parallel for schedule(dynamic)
    for (int bh = 0; bh < B * H; ++bh) {
        size_t off = (size_t)bh * S * D;
        const int b = bh / H;
        double* q = (double*)malloc(sizeof(double) * (size_t)S * D);
        double* k = (double*)malloc(sizeof(double) * (size_t)S * D);
        double* p = (double*)malloc(sizeof(double) * (size_t)S);
        for (size_t i = 0; i < (size_t)S * D; ++i) { q[i] = Q[off + i]; k[i] = K[off + i]; }
        rope_d(q, S, D, rope_mode, theta, 0);
        rope_d(k, S, D, rope_mode, theta, 0);
        for (int i = 0; i < S; ++i) {
            int jn = causal ? i + 1 : S;
            double mx = -INFINITY;
            for (int j = 0; j < jn; ++j) {
                double s = 0.0;
                for (int d = 0; d < D; ++d) s += q[(size_t)i * D + d] * k[(size_t)j * D + d];
                p[j] = s * scale + key_bias(mask, b, S, j);
                if (p[j] > mx) mx = p[j];
            }
            double sum = 0.0;
            for (int j = 0; j < jn; ++j) { p[j] = exp(p[j] - mx); sum += p[j]; }
            LSE[(size_t)bh * S + i] = (float)(mx + log(sum));
            for (int d = 0; d < D; ++d) {
                double o = 0.0;
                for (int j = 0; j < jn; ++j) o += p[j] * V[off + (size_t)j * D + d];
                O[off + (size_t)i * D + d] = (float)(o / sum);
            }
        }
        free(q); free(k); free(p);
    }
}

/* attention-backward.glsl:73-194 (dV = P^T dO; dP = dO V^T; dS = P (dP - rowdot) scale;
 * dQ = dS K; dK = dS^T Q), with P recomputed from the saved LSE, the causal mask, and
 * RoPE: the contraction runs on rotated q, k and dQ, dK are rotated back (R^T). */
void or_attn_bwd(const float* Q, const float* K, const float* V, const float* dO,
                 const float* LSE, float* dQ, float* dK, float* dV, int B, int H, int S, int D,
                 float scale, int causal, int rope_mode, float theta, const float* mask) {
#pragma omp parallel for schedule(dynamic)
    for (int bh = 0; bh < B * H; ++bh) {
        size_t off = (size_t)bh * S * D;
        const int b = bh / H;
        size_t SD = (size_t)S * D;
        double* q = (double*)malloc(sizeof(double) * SD);
        double* k = (double*)malloc(sizeof(double) * SD);
        double* dq = (double*)calloc(SD, sizeof(double));
        double* dk = (double*)calloc(SD, sizeof(double));
        double* dv = (double*)calloc(SD, sizeof(double));
        double* p = (double*)malloc(sizeof(double) * (size_t)S);
        double* dp = (double*)malloc(sizeof(double) * (size_t)S);
        for (size_t i = 0; i < SD; ++i) { q[i] = Q[off + i]; k[i] = K[off + i]; }
        rope_d(q, S, D, rope_mode, theta, 0);
        rope_d(k, S, D, rope_mode, theta, 0);
        for (int i = 0; i < S; ++i) {
            int jn = causal ? i + 1 : S;
            double lse = LSE[(size_t)bh * S + i], rowdot = 0.0;
            for (int j = 0; j < jn; ++j) {
                double s = 0.0, t = 0.0;
                for (int d = 0; d < D; ++d) {
                    s += q[(size_t)i * D + d] * k[(size_t)j * D + d];
                    t += (double)dO[off + (size_t)i * D + d] * V[off + (size_t)j * D + d];
                }
                p[j] = exp(s * scale + key_bias(mask, b, S, j) - lse);
                dp[j] = t;
                rowdot += p[j] * t;
            }
            for (int j = 0; j < jn; ++j) {
                double ds = p[j] * (dp[j] - rowdot) * scale;
                for (int d = 0; d < D; ++d) {
                    dv[(size_t)j * D + d] += p[j] * dO[off + (size_t)i * D + d];
                    dq[(size_t)i * D + d] += ds * k[(size_t)j * D + d];
                    dk[(size_t)j * D + d] += ds * q[(size_t)i * D + d];
                }
            }
        }
        rope_d(dq, S, D, rope_mode, theta, 1);
        rope_d(dk, S, D, rope_mode, theta, 1);
        for (size_t i = 0; i < SD; ++i) {
            dQ[off + i] = (float)dq[i];
            dK[off + i] = (float)dk[i];
            dV[off + i] = (float)dv[i];
        }
        free(q); free(k); free(dq); free(dk); free(dv); free(p); free(dp);
    }
}

/* ---------------------------------------------------------------- VSA ------------- */
/* vsa-unpack-project-backward.glsl:50-57, vsa_loop.py:170-175: word j>>5, bit j&31,
 * LSB first, set bit -> +1, clear bit -> -1. */
void or_unpack_bits(const uint32_t* bits, float* out, int Bn, int D, int words) {
    for (int b = 0; b < Bn; ++b)
        for (int j = 0; j < D; ++j)
            out[(size_t)b * D + j] =
                ((bits[(size_t)b * words + (j >> 5)] >> (j & 31)) & 1u) ? 1.0f : -1.0f;
}

/* vsa-unpack-project-backward.glsl:46-74: dW[o,j] = sum_b dY[b,o] s_b(j); db = colsum. */
void or_vsa_unpack_project_bwd(const float* dY, const uint32_t* bits, float* dW, float* db,
                               int Bn, int O, int D, int words) {
#pragma omp parallel
    {
        double* acc = (double*)malloc(sizeof(double) * (size_t)D);
#pragma omp for schedule(static)
        for (int o = 0; o < O; ++o) {
            for (int j = 0; j < D; ++j) acc[j] = 0.0;
            for (int b = 0; b < Bn; ++b) {
                const double g = dY[(size_t)b * O + o];
                const uint32_t* w = bits + (size_t)b * words;
                for (int j = 0; j < D; ++j) acc[j] += ((w[j >> 5] >> (j & 31)) & 1u) ? g : -g;
            }
            for (int j = 0; j < D; ++j) dW[(size_t)o * D + j] = (float)acc[j];
        }
        free(acc);
    }
    if (db)
        for (int o = 0; o < O; ++o) {
            double s = 0.0;
            for (int b = 0; b < Bn; ++b) s += dY[(size_t)b * O + o];
            db[o] = (float)s;
        }
}

/* vsa-surrogate-loss-backward.glsl:50-88 restated per element. */
void or_vsa_surrogate_bwd(const float* preds, const uint32_t* bits, const uint32_t* results,
                          const float* weights, float* dPreds, int Bn, int K, int D, int words,
                          float gamma, float delta, float lambda_c, float scale,
                          int accumulate) {
#pragma omp parallel for schedule(static)
    for (int b = 0; b < Bn; ++b) {
        uint32_t win = results[(size_t)b * 4 + 0], run = results[(size_t)b * 4 + 1];
        float dwin, drun;
        memcpy(&dwin, &results[(size_t)b * 4 + 2], 4);
        memcpy(&drun, &results[(size_t)b * 4 + 3], 4);
        int contrast = (win != run) && ((double)delta - ((double)dwin - (double)drun) > 0.0);
        for (int i = 0; i < D; ++i) {
            double y = ((bits[(size_t)b * words + (i >> 5)] >> (i & 31)) & 1u) ? 1.0 : -1.0;
            for (int k = 0; k < K; ++k) {
                size_t idx = ((size_t)b * K + k) * D + i;
                double g = accumulate ? (double)dPreds[idx] : 0.0;
                if ((double)gamma - y * preds[idx] > 0.0)
                    g += (-y / D) * weights[(size_t)b * K + k] * scale;
                if (contrast && (uint32_t)k == run) g += (y / D) * lambda_c * scale;
                dPreds[idx] = (float)g;
            }
        }
    }
}

/* vsa-surrogate-loss-forward.glsl pass 0: dots[b,k] = sum_i preds[b,k,i] y_i */
void or_vsa_dots(const float* preds, const uint32_t* bits, float* dots, int Bn, int K, int D,
                 int words) {
    for (int b = 0; b < Bn; ++b)
        for (int k = 0; k < K; ++k) {
            double s = 0.0;
            for (int i = 0; i < D; ++i) {
                double y = ((bits[(size_t)b * words + (i >> 5)] >> (i & 31)) & 1u) ? 1.0 : -1.0;
                s += preds[((size_t)b * K + k) * D + i] * y;
            }
            dots[(size_t)b * K + k] = (float)s;
        }
}

/* vsa-unpack-project.glsl:40-74: Y[b, o] = sum_j s_b(j) W[o, j] + bias[o] (fp64 sums). */
void or_vsa_unpack_project_fwd(const uint32_t* bits, const float* W, const float* bias, float* Y,
                               int Bn, int O, int D, int words) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < Bn; ++b)
        for (int o = 0; o < O; ++o) {
            const uint32_t* w = bits + (size_t)b * words;
            const float* Wr = W + (size_t)o * D;
            double s = bias ? (double)bias[o] : 0.0;
            for (int j = 0; j < D; ++j) s += ((w[j >> 5] >> (j & 31)) & 1u) ? Wr[j] : -(double)Wr[j];
            Y[(size_t)b * O + o] = (float)s;
        }
}

/* The counter-based Gumbel source this build uses in place of the reference's unseeded
 * std::mt19937 (vsa_loss_node.cpp:9-14): splitmix64 (Steele, Lea & Flood 2014) of the Weyl
 * value seed + (idx + 1) * 0x9E3779B97F4A7C15, u = (top 23 bits + 1/2) / 2^23 (exact in fp32),
 * g = -log(-log u) in fp32. */
uint64_t or_mix64(uint64_t seed, uint64_t idx) {
    uint64_t x = seed + (idx + 1) * 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

float or_gumbel(uint64_t seed, uint64_t idx) {
    const float u = ((float)(uint32_t)(or_mix64(seed, idx) >> 41) + 0.5f) * 0x1p-23f;
    return -logf(-logf(u));
}

/* dispatch_vsa_loss_forward (vsa_loss_node.cpp:101-148): the top-2 of dots + T g (strict >,
 * earlier index kept on ties, both starting at index 0) and softmax(dots / T) weights, from
 * given fp32 dots [Bn x K]; noise = 0: no Gumbel term. */
void or_vsa_select(const float* dots, uint32_t* results, float* weights, int Bn, int K,
                   float temperature, uint64_t seed, uint64_t counter, int noise) {
    for (int b = 0; b < Bn; ++b) {
        const float* d = dots + (size_t)b * K;
        float max1 = -1e30f, max2 = -1e30f;
        int k1 = 0, k2 = 0;
        for (int k = 0; k < K; ++k) {
            const float g = noise ? or_gumbel(seed, ((uint64_t)counter * Bn + b) * K + k) : 0.0f;
            const float adj = d[k] + g * temperature;
            if (adj > max1) {
                max2 = max1; k2 = k1;
                max1 = adj; k1 = k;
            } else if (adj > max2) {
                max2 = adj; k2 = k;
            }
        }
        double mx = d[0], se = 0.0;
        for (int k = 1; k < K; ++k) mx = d[k] > mx ? d[k] : mx;
        for (int k = 0; k < K; ++k) se += exp((d[k] - mx) / temperature);
        for (int k = 0; k < K; ++k) weights[(size_t)b * K + k] = (float)(exp((d[k] - mx) / temperature) / se);
        uint32_t bw, br;
        memcpy(&bw, &d[k1], 4);
        memcpy(&br, &d[k2], 4);
        results[(size_t)b * 4 + 0] = (uint32_t)k1;
        results[(size_t)b * 4 + 1] = (uint32_t)k2;
        results[(size_t)b * 4 + 2] = bw;
        results[(size_t)b * 4 + 3] = br;
    }
}

/* vsa-surrogate-loss-forward.glsl pass 1: loss[b] = mean_i max(gamma - y_i z[b, win, i], 0)
 * + lambda max(0, delta - (dot_win - dot_run)), with win and the dots from results[b]. */
void or_vsa_surrogate_loss(const float* preds, const uint32_t* bits, const uint32_t* results,
                           float* loss, int Bn, int K, int D, int words, float gamma,
                           float delta, float lambda_c) {
    for (int b = 0; b < Bn; ++b) {
        const int win = (int)results[(size_t)b * 4];
        const float* z = preds + ((size_t)b * K + win) * D;
        const uint32_t* w = bits + (size_t)b * words;
        double h = 0.0;
        for (int i = 0; i < D; ++i) {
            const double y = ((w[i >> 5] >> (i & 31)) & 1u) ? 1.0 : -1.0;
            const double m = gamma - y * z[i];
            h += m > 0.0 ? m : 0.0;
        }
        float dw, dr;
        memcpy(&dw, &results[(size_t)b * 4 + 2], 4);
        memcpy(&dr, &results[(size_t)b * 4 + 3], 4);
        const double c = delta - ((double)dw - dr);
        loss[b] = (float)(h / D + lambda_c * (c > 0.0 ? c : 0.0));
    }
}

/* surprise-momentum.glsl:53-114.  fmin/fmax give the clamps a defined result for a NaN
 * update (the GLSL clamp leaves it undefined); every other branch follows the shader. */
void or_surprise_momentum_step(float* W, float* grad, float* s_bar, float* delta,
                               const float* recalled, int64_t n, float eta_base, float alpha,
                               float lambda_recall, float surprise_floor, float weight_decay,
                               float clip_max, int clear_grad) {
    for (int64_t i = 0; i < n; ++i) {
        const double g = grad[i], r = recalled ? recalled[i] : 0.0;
        if (!isfinite(g) || !isfinite(r)) {  /* shader :71-77 */
            if (delta) delta[i] = 0.0f;
            if (clear_grad) grad[i] = 0.0f;
            continue;
        }
        const double g_eff = g + (double)lambda_recall * r;            /* :80 */
        const double pe = fabs(g - r);                                    /* :83 */
        double sp = s_bar[i];
        if (!isfinite(sp)) sp = 0.0;                                      /* :89 */
        double s = (double)alpha * pe + (1.0 - (double)alpha) * sp;       /* :90 */
        s = fmin(s, 5.0);                                                 /* :92 */
        s_bar[i] = (float)s;
        const double lr = (double)eta_base * (1.0 + fmax(s, (double)surprise_floor)); /* :97 */
        double d = lr * g_eff + (double)eta_base * weight_decay * (double)W[i];       /* :100-104 */
        d = fmin(fmax(d, -(double)clip_max), (double)clip_max);          /* :107 */
        double wn = (double)W[i] - d;                                     /* :110 */
        if (!isfinite(wn)) wn = 0.0;                                      /* :112 */
        W[i] = (float)fmin(fmax(wn, -10.0), 10.0);                        /* :113 */
        if (delta) delta[i] = (float)d;
        if (clear_grad) grad[i] = 0.0f;
    }
}

/* adamw-update.glsl:41-61 */
void or_adamw_step(float* W, float* grad, float* m, float* v, int64_t n, float lr, float beta1,
                   float beta2, float eps, float weight_decay, float beta1_t, float beta2_t,
                   int clear_grad) {
    for (int64_t i = 0; i < n; ++i) {
        const double g = grad[i];
        const double m_new = (double)beta1 * m[i] + (1.0 - (double)beta1) * g;
        const double v_new = (double)beta2 * v[i] + (1.0 - (double)beta2) * g * g;
        m[i] = (float)m_new;
        v[i] = (float)v_new;
        const double m_hat = m_new / fmax(1e-12, 1.0 - (double)beta1_t);
        const double v_hat = v_new / fmax(1e-12, 1.0 - (double)beta2_t);
        const double decayed = (double)W[i] * (1.0 - (double)lr * weight_decay);
        W[i] = (float)(decayed - (double)lr * m_hat / (sqrt(fmax(v_hat, 0.0)) + (double)eps));
        if (clear_grad) grad[i] = 0.0f;
    }
}

void or_binary_bwd(int op, const float* dY, const float* A, const float* B, float* dA, float* dB,
                   int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        const double g = dY[i];
        double da = 0.0, db = 0.0;
        if (op == 0) { da = g; db = -g; }                         /* a - b */
        else if (op == 1) { da = g * B[i]; db = g * A[i]; }       /* a * b */
        else if (op == 2) { da = g / B[i]; db = -g * A[i] / ((double)B[i] * B[i]); } /* a / b */
        else { da = -g; }                                         /* -a */
        if (dA) dA[i] = (float)da;
        if (dB) dB[i] = (float)db;
    }
}

void or_reduce_bwd(int op, const float* dY, float* dX, int64_t outer, int64_t inner) {
    for (int64_t o = 0; o < outer; ++o)
        for (int64_t i = 0; i < inner; ++i)
            dX[o * inner + i] = (float)(op == 1 ? (double)dY[o] / (double)inner : (double)dY[o]);
}

void or_transpose_bwd(const float* dY, float* dX, int64_t batch, int rows, int cols) {
    for (int64_t b = 0; b < batch; ++b)
        for (int r = 0; r < rows; ++r)
            for (int c = 0; c < cols; ++c)
                dX[(b * rows + r) * cols + c] = dY[(b * cols + c) * rows + r];
}

void or_mse_bwd(const float* P, const float* T, float g, float* dP, int64_t n, float scale) {
    for (int64_t i = 0; i < n; ++i) dP[i] = (float)(2.0 * scale * g * ((double)P[i] - T[i]));
}

void or_lora_expand_bwd(const float* dP, const float* basis, const float* coeffs, float* dC,
                        float* dB, int BK, int D, int rank, float scale) {
    for (int row = 0; row < BK; ++row)
        for (int r = 0; r < rank; ++r) {
            double s = 0.0;
            for (int i = 0; i < D; ++i) s += (double)basis[(size_t)i * rank + r] * dP[(size_t)row * D + i];
            dC[(size_t)row * rank + r] = (float)(s * scale);
        }
    for (int i = 0; i < D; ++i)
        for (int r = 0; r < rank; ++r) {
            double s = 0.0;
            for (int row = 0; row < BK; ++row)
                s += (double)dP[(size_t)row * D + i] * coeffs[(size_t)row * rank + r];
            dB[(size_t)i * rank + r] = (float)(s * scale);
        }
}

void or_cosine_blend_bwd(const uint32_t* bits, const float* weights, const float* blended,
                         const float* info, float* dP, int Bn, int K, int D, int words,
                         float grad_scale) {
    for (int b = 0; b < Bn; ++b) {
        const double dot = info[(size_t)b * 3 + 1], nsq = info[(size_t)b * 3 + 2];
        const double nb = sqrt(fmax(nsq, 1e-8)), sd = sqrt((double)D);
        const double cosine = dot / (nb * sd);
        for (int i = 0; i < D; ++i) {
            const double y = ((bits[(size_t)b * words + (i >> 5)] >> (i & 31)) & 1u) ? 1.0 : -1.0;
            const double gb = -(y / (nb * sd) - cosine * blended[(size_t)b * D + i] / fmax(nsq, 1e-8));
            for (int k = 0; k < K; ++k) {
                const double g = gb * weights[(size_t)b * K + k] * grad_scale;
                dP[((size_t)b * K + k) * D + i] = (float)fmin(fmax(g, -1.0), 1.0);
            }
        }
    }
}
