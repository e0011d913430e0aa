"""numpy restatement of the reference's CPU backward path, used as bench.py's CPU baseline.

TEST INFRASTRUCTURE ONLY: imported by bench.py's cpu_baseline leg (and tests); the product
path never imports it.

The reference's runnable CPU path for these ops is the numpy fallback of VulkanBackwardOps
(src/grilly_next/backend/autograd_core.py:486-654): fp32 arrays, BLAS matmuls, elementwise
numpy.  The functions below restate it (same formulas, same fp32 arithmetic); ops the
reference has only as GLSL (cross-entropy, the fused GLU local gradients, RMSNorm, the VSA
kernels, the surprise-momentum update) are written in the same numpy style from their
shaders' formulas.  Every timing runs with the BLAS / OpenMP pools limited to `threads()`.
"""
from __future__ import annotations

import os

import numpy as np


def threads() -> int:
    """Host threads for the baseline: OMP_NUM_THREADS when set (the GPU box sets it to its CPU
    share), else every core."""
    env = os.environ.get("OMP_NUM_THREADS")
    return int(env) if env and env.isdigit() and int(env) > 0 else (os.cpu_count() or 1)


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def limit_threads(n: int):
    """Context manager capping numpy's BLAS and OpenMP pools at n threads."""
    from threadpoolctl import threadpool_limits
    return threadpool_limits(limits=n)


# ---------------------------------------------------------------- autograd_core.py:486-654
def linear_backward(grad_output, x, weight, bias=True):
    """autograd_core.py:511-514: dX = dY W, dW = dY^T X, db = column sums."""
    grad_input = grad_output @ weight
    grad_weight = grad_output.T @ x
    grad_bias = np.sum(grad_output, axis=0) if bias else None
    return grad_input, grad_weight, grad_bias


def relu_backward(grad_output, x):
    """autograd_core.py:545-547"""
    return grad_output * (x > 0).astype(np.float32)


def silu_backward(grad_output, x):
    """autograd_core.py:549-553"""
    sig = 1.0 / (1.0 + np.exp(-x))
    return (grad_output * (sig + x * sig * (1 - sig))).astype(np.float32)


def gelu_tanh(x):
    return 0.5 * x * (1.0 + np.tanh(np.float32(np.sqrt(2.0 / np.pi)) * (x + np.float32(0.044715) * x ** 3)))


def gelu_tanh_backward(grad_output, x):
    """activation-gelu-backward.glsl:38-50 (the tanh form the shaders use)."""
    c = np.float32(np.sqrt(2.0 / np.pi))
    t = np.tanh(c * (x + np.float32(0.044715) * x ** 3))
    return (grad_output * 0.5 * (1 + t + x * (1 - t * t) * c * (1 + 3 * np.float32(0.044715) * x * x))
            ).astype(np.float32)


def softmax_backward(grad_output, softmax_output, dim=-1):
    """autograd_core.py:555-566"""
    sum_term = np.sum(grad_output * softmax_output, axis=dim, keepdims=True)
    return (softmax_output * (grad_output - sum_term)).astype(np.float32)


def layernorm_backward(grad_output, x, gamma, mean, var, eps=1e-5):
    """autograd_core.py:568-615 (the textbook form)"""
    std = np.sqrt(var + eps)
    x_norm = (x - mean) / std
    grad_gamma = np.sum(grad_output * x_norm, axis=0)
    grad_beta = np.sum(grad_output, axis=0)
    N = x.shape[-1]
    dx_norm = grad_output * gamma
    dvar = np.sum(dx_norm * (x - mean) * (-0.5) * (var + eps) ** (-1.5), axis=-1, keepdims=True)
    dmean = np.sum(dx_norm * (-1.0 / std), axis=-1, keepdims=True) + dvar * np.mean(
        -2.0 * (x - mean), axis=-1, keepdims=True)
    grad_input = dx_norm / std + dvar * 2.0 * (x - mean) / N + dmean / N
    return grad_input.astype(np.float32), grad_gamma.astype(np.float32), grad_beta.astype(np.float32)


def attention_backward(grad_output, q, k, v, attn_weights, scale):
    """autograd_core.py:617-654 (attention weights P materialised)"""
    grad_v = np.matmul(attn_weights.swapaxes(-2, -1), grad_output)
    grad_attn = np.matmul(grad_output, v.swapaxes(-2, -1))
    grad_scores = softmax_backward(grad_attn, attn_weights) * scale
    grad_q = np.matmul(grad_scores, k)
    grad_k = np.matmul(grad_scores.swapaxes(-2, -1), q)
    return grad_q.astype(np.float32), grad_k.astype(np.float32), grad_v.astype(np.float32)


# ---------------------------------------------------------------- GLSL-only ops, numpy style
def rmsnorm_backward(grad_output, x, w, rstd):
    """dx = r w dy - x r^3 mean(w dy x); dw = sum_rows dy x r (rms-norm.glsl forward)."""
    r = rstd[:, None]
    s = np.mean(w * grad_output * x, axis=-1, keepdims=True)
    dx = r * w * grad_output - x * r ** 3 * s
    dw = np.sum(grad_output * x * r, axis=0)
    return dx.astype(np.float32), dw.astype(np.float32)


def swiglu_up_local(d, gate, up):
    """fused-swiglu-backward.glsl:93-100 (out = gate * SiLU(up))"""
    sig = 1.0 / (1.0 + np.exp(-up))
    return (d * up * sig).astype(np.float32), (d * gate * sig * (1 + up * (1 - sig))).astype(np.float32)


def cross_entropy_backward(logits, targets, scale=1.0):
    """cross-entropy-backward.glsl:73-84: scale (softmax - onehot)"""
    z = logits - logits.max(axis=-1, keepdims=True)
    e = np.exp(z)
    g = e / e.sum(axis=-1, keepdims=True)
    g[np.arange(len(targets)), targets] -= 1.0
    return (g * scale).astype(np.float32)


def unpack_bits(bits, D):
    """vsa_loop.py:170-175: LSB-first words to +-1"""
    return np.unpackbits(bits.view(np.uint8), axis=1, bitorder="little")[:, :D].astype(np.float32) * 2 - 1


def vsa_unpack_project_backward(grad_output, bits, D):
    """vsa-unpack-project-backward.glsl:46-74: dW = dY^T S, db = column sums"""
    S = unpack_bits(bits, D)
    return grad_output.T @ S, grad_output.sum(axis=0)


def surprise_momentum(W, g, s_bar, eta=1e-3, alpha=0.9, floor=0.01, clip=1.0):
    """surprise-momentum.glsl:53-114 with no recalled gradient and no weight decay"""
    s = np.minimum(alpha * np.abs(g) + (1 - alpha) * s_bar, 5.0)
    d = np.clip(eta * (1 + np.maximum(s, floor)) * g, -clip, clip)
    W -= d
    np.clip(W, -10.0, 10.0, out=W)
    s_bar[...] = s
    return W, s_bar


# ---------------------------------------------------------------- the benchmark steps
def ffn_block_step(x, w, rstd, n, gate, up, a, Wg, Wu, Wd, dY):
    """down projection, SwiGLU local gradients, gate/up projections, RMSNorm."""
    dA, dWd, _ = linear_backward(dY, a, Wd, bias=False)
    dG, dU = swiglu_up_local(dA, gate, up)
    dN1, dWg, _ = linear_backward(dG, n, Wg, bias=False)
    dN2, dWu, _ = linear_backward(dU, n, Wu, bias=False)
    return rmsnorm_backward(dN1 + dN2, x, w, rstd)


def mlp_step(X, y, W1, W2, Z, H, L):
    """CE (scale 1), Linear 2 with dX, ReLU, Linear 1 without dX."""
    dL = cross_entropy_backward(L, y, 1.0)
    dH, dW2, db2 = linear_backward(dL, H, W2)
    dZ = relu_backward(dH, Z)
    return dZ.T @ X, dZ.sum(axis=0), dW2, db2


def attention_step(q, k, v, dO, scale, causal=True):
    """configs[2] per (b, h) batch: P from the forward (recomputed here, as the tape's
    backward would need it), then attention_backward."""
    s = np.matmul(q, k.swapaxes(-2, -1)) * scale
    if causal:
        S = s.shape[-1]
        s = np.where(np.triu(np.ones((S, S), bool), 1), -np.inf, s)
    s = s - s.max(axis=-1, keepdims=True)
    P = np.exp(s)
    P /= P.sum(axis=-1, keepdims=True)
    return attention_backward(dO, q, k, v, P.astype(np.float32), scale)


def hypernet_step(W, state_bits, delta_bits, d, v, K, s_bar, gamma=1.0, delta=1.0, lam=0.3):
    """One VSA hypernetwork training step (vsa_training_step, bindings.cpp:3140-3286) in numpy
    fp32: the forward of vsa_hypernetwork.cpp:52-160, the surrogate loss with a noise-free top-2
    (the selection is K-wide: no time), its backward (vsa-surrogate-loss-backward.glsl:56-88),
    the Linear / GELU / unpack-project backwards and the surprise-momentum update of the six
    parameters that receive gradients.  W: the ten parameters (flat), s_bar: their states."""
    h2 = 2 * d
    Wp, bp = W[0].reshape(d, v), W[1]
    W1, b1 = W[2].reshape(h2, d), W[3]
    W2, b2 = W[4].reshape(K * v, h2), W[5]
    S = unpack_bits(state_bits, v)
    h = S @ Wp.T + bp
    m = h @ W1.T + b1
    a = gelu_tanh(m).astype(np.float32)
    P = (a @ W2.T + b2).reshape(K, v)
    y = unpack_bits(delta_bits, v)[0]
    dots = P @ y
    order = np.argsort(-dots, kind="stable")
    win, run = order[0], order[1]
    e = np.exp(dots - dots.max())
    wts = (e / e.sum()).astype(np.float32)
    g = np.where(gamma - y[None, :] * P > 0, (-y[None, :] / v) * wts[:, None], 0.0).astype(np.float32)
    if delta - (dots[win] - dots[run]) > 0:
        g[run] += y / v * lam
    dP = g.reshape(1, K * v)
    dA, dW2, db2 = linear_backward(dP, a, W2)
    dM = gelu_tanh_backward(dA, m)
    dH, dW1, db1 = linear_backward(dM, h, W1)
    dWp, dbp = vsa_unpack_project_backward(dH, state_bits, v)
    grads = [dWp, dbp, dW1, db1, dW2, db2]
    for i, gr in enumerate(grads):
        surprise_momentum(W[i], gr.reshape(-1), s_bar[i])
    return float(np.mean(np.maximum(gamma - y * P[win], 0)) + lam * max(0.0, delta - (dots[win] - dots[run])))
