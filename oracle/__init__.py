"""numpy front-end of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg as the checker / CPU baseline.  The product path never imports it.
Every function returns fresh fp32 numpy arrays; see oracle.h for the reference file:line
each one restates.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

ACT = {"relu": 0, "gelu_tanh": 1, "gelu_erf": 2, "silu": 3, "tanh": 4, "sigmoid": 5}
GLU = {"swiglu_up": 0, "swiglu_gate": 1, "geglu_up": 2, "geglu_gate": 3, "reglu_up": 4}
ROPE = {"none": 0, "interleaved": 1, "half": 2}


def build() -> None:
    subprocess.check_call(["make", "-s", "-C", _HERE])


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.or_mix64.restype = ctypes.c_uint64
        _lib.or_gumbel.restype = ctypes.c_float
    return _lib


def _f(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a, a.ctypes.data_as(ctypes.c_void_p)


def _u(a):
    a = np.ascontiguousarray(a, dtype=np.uint32)
    return a, a.ctypes.data_as(ctypes.c_void_p)


def _i(a):
    a = np.ascontiguousarray(a, dtype=np.int32)
    return a, a.ctypes.data_as(ctypes.c_void_p)


def _out(shape):
    a = np.empty(shape, dtype=np.float32)
    return a, a.ctypes.data_as(ctypes.c_void_p)


def num_threads() -> int:
    return int(lib().or_num_threads())


def linear_bwd(dY, X, W, need_dx=True, need_db=True):
    M, N = dY.shape
    K = X.shape[1]
    dY, pdy = _f(dY)
    X, px = _f(X)
    W, pw = _f(W)
    dX, pdx = _out((M, K)) if need_dx else (None, None)
    dW, pdw = _out((N, K))
    db, pdb = _out((N,)) if need_db else (None, None)
    lib().or_linear_bwd(pdy, px, pw, pdx, pdw, pdb, M, N, K)
    return dX, dW, db


def linear_fwd(X, W, b=None):
    M, K = X.shape
    N = W.shape[0]
    X, px = _f(X)
    W, pw = _f(W)
    pb = None
    if b is not None:
        b, pb = _f(b)
    Y, py = _out((M, N))
    lib().or_linear_fwd(px, pw, pb, py, M, N, K)
    return Y


def act_bwd(kind, dY, X):
    dY, pdy = _f(dY)
    X, px = _f(X)
    dX, pdx = _out(dY.shape)
    lib().or_act_bwd(ACT[kind], pdy, px, pdx, ctypes.c_int64(dY.size))
    return dX


def act_fwd(kind, X):
    X, px = _f(X)
    Y, py = _out(X.shape)
    lib().or_act_fwd(ACT[kind], px, py, ctypes.c_int64(X.size))
    return Y


def glu_bwd(kind, dO, gate, up):
    dO, pd = _f(dO)
    gate, pg = _f(gate)
    up, pu = _f(up)
    dG, pdg = _out(dO.shape)
    dU, pdu = _out(dO.shape)
    lib().or_glu_bwd(GLU[kind], pd, pg, pu, pdg, pdu, ctypes.c_int64(dO.size))
    return dG, dU


def glu_fwd(kind, gate, up):
    gate, pg = _f(gate)
    up, pu = _f(up)
    out, po = _out(gate.shape)
    lib().or_glu_fwd(GLU[kind], pg, pu, po, ctypes.c_int64(gate.size))
    return out


def layernorm_bwd(dY, X, gamma, mean, rstd, eps=1e-5, stat_is_var=False):
    rows, F = X.shape
    dY, pdy = _f(dY)
    X, px = _f(X)
    gamma, pg = _f(gamma)
    mean, pm = _f(mean)
    rstd, pr = _f(rstd)
    dX, pdx = _out((rows, F))
    dG, pdg = _out((F,))
    dB, pdb = _out((F,))
    lib().or_layernorm_bwd(pdy, px, pg, pm, pr, pdx, pdg, pdb, rows, F,
                           ctypes.c_float(eps), int(stat_is_var))
    return dX, dG, dB


def layernorm_bwd_glsl(dY, X, gamma, mean, rstd):
    rows, F = X.shape
    dY, pdy = _f(dY)
    X, px = _f(X)
    gamma, pg = _f(gamma)
    mean, pm = _f(mean)
    rstd, pr = _f(rstd)
    dX, pdx = _out((rows, F))
    lib().or_layernorm_bwd_glsl(pdy, px, pg, pm, pr, pdx, rows, F)
    return dX


def layernorm_fwd(X, gamma, beta=None, eps=1e-5):
    rows, F = X.shape
    X, px = _f(X)
    gamma, pg = _f(gamma)
    pb = None
    if beta is not None:
        beta, pb = _f(beta)
    Y, py = _out((rows, F))
    mean, pm = _out((rows,))
    rstd, pr = _out((rows,))
    lib().or_layernorm_fwd(px, pg, pb, py, pm, pr, rows, F, ctypes.c_float(eps))
    return Y, mean, rstd


def rmsnorm_bwd(dY, X, w, rstd):
    rows, F = X.shape
    dY, pdy = _f(dY)
    X, px = _f(X)
    w, pw = _f(w)
    rstd, pr = _f(rstd)
    dX, pdx = _out((rows, F))
    dW, pdw = _out((F,))
    lib().or_rmsnorm_bwd(pdy, px, pw, pr, pdx, pdw, rows, F)
    return dX, dW


def rmsnorm_fwd(X, w, eps=1e-6):
    rows, F = X.shape
    X, px = _f(X)
    w, pw = _f(w)
    Y, py = _out((rows, F))
    rstd, pr = _out((rows,))
    lib().or_rmsnorm_fwd(px, pw, py, pr, rows, F, ctypes.c_float(eps))
    return Y, rstd


def softmax_bwd(dY, Y):
    rows, C = Y.shape
    dY, pdy = _f(dY)
    Y, py = _f(Y)
    dX, pdx = _out((rows, C))
    lib().or_softmax_bwd(pdy, py, pdx, rows, C)
    return dX


def softmax_fwd(X):
    rows, C = X.shape
    X, px = _f(X)
    Y, py = _out((rows, C))
    lib().or_softmax_fwd(px, py, rows, C)
    return Y


def xent_bwd(logits, targets, scale=1.0):
    rows, C = logits.shape
    logits, pl = _f(logits)
    targets, pt = _i(targets)
    dL, pdl = _out((rows, C))
    lib().or_xent_bwd(pl, pt, pdl, rows, C, ctypes.c_float(scale))
    return dL


def rope(X, mode="interleaved", theta=10000.0, inverse=False):
    S, D = X.shape
    X = np.array(X, dtype=np.float32, copy=True)
    lib().or_rope(X.ctypes.data_as(ctypes.c_void_p), S, D, ROPE[mode], ctypes.c_float(theta),
                  int(inverse))
    return X


def _mask_arg(mask, B, S):
    """fp32 [B, S] key-padding mask (flash-attention2.glsl:150-154) as a pointer, or None."""
    if mask is None:
        return None, None
    m, pm = _f(np.asarray(mask, dtype=np.float32).reshape(B, S))
    return m, pm


def attn_fwd(Q, K, V, scale=None, causal=True, rope_mode="interleaved", theta=10000.0,
             mask=None):
    B, H, S, D = Q.shape
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    Q, pq = _f(Q)
    K, pk = _f(K)
    V, pv = _f(V)
    m, pm = _mask_arg(mask, B, S)
    O, po = _out((B, H, S, D))
    LSE, pl = _out((B, H, S))
    lib().or_attn_fwd(pq, pk, pv, po, pl, B, H, S, D, ctypes.c_float(scale), int(causal),
                      ROPE[rope_mode], ctypes.c_float(theta), pm)
    return O, LSE


def attn_bwd(Q, K, V, dO, LSE, scale=None, causal=True, rope_mode="interleaved",
             theta=10000.0, mask=None):
    B, H, S, D = Q.shape
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    Q, pq = _f(Q)
    K, pk = _f(K)
    V, pv = _f(V)
    dO, pdo = _f(dO)
    LSE, pl = _f(LSE)
    m, pm = _mask_arg(mask, B, S)
    dQ, pdq = _out((B, H, S, D))
    dK, pdk = _out((B, H, S, D))
    dV, pdv = _out((B, H, S, D))
    lib().or_attn_bwd(pq, pk, pv, pdo, pl, pdq, pdk, pdv, B, H, S, D, ctypes.c_float(scale),
                      int(causal), ROPE[rope_mode], ctypes.c_float(theta), pm)
    return dQ, dK, dV


def unpack_bits(bits, D):
    Bn, words = bits.shape
    bits, pb = _u(bits)
    out, po = _out((Bn, D))
    lib().or_unpack_bits(pb, po, Bn, D, words)
    return out


def vsa_unpack_project_bwd(dY, bits, D):
    Bn, O = dY.shape
    words = bits.shape[1]
    dY, pdy = _f(dY)
    bits, pb = _u(bits)
    dW, pdw = _out((O, D))
    db, pdb = _out((O,))
    lib().or_vsa_unpack_project_bwd(pdy, pb, pdw, pdb, Bn, O, D, words)
    return dW, db


def vsa_surrogate_bwd(preds, bits, results, weights, gamma=1.0, delta=1.0, lambda_c=0.3,
                      scale=1.0, init=None):
    Bn, K, D = preds.shape
    words = bits.shape[1]
    preds, pp = _f(preds)
    bits, pb = _u(bits)
    results, pr = _u(results)
    weights, pw = _f(weights)
    if init is None:
        dP, pdp = _out((Bn, K, D))
        acc = 0
    else:
        dP, pdp = _f(np.array(init, dtype=np.float32, copy=True))
        acc = 1
    lib().or_vsa_surrogate_bwd(pp, pb, pr, pw, pdp, Bn, K, D, words, ctypes.c_float(gamma),
                               ctypes.c_float(delta), ctypes.c_float(lambda_c),
                               ctypes.c_float(scale), acc)
    return dP


def vsa_dots(preds, bits):
    Bn, K, D = preds.shape
    words = bits.shape[1]
    preds, pp = _f(preds)
    bits, pb = _u(bits)
    dots, pd = _out((Bn, K))
    lib().or_vsa_dots(pp, pb, pd, Bn, K, D, words)
    return dots


def vsa_unpack_project_fwd(bits, W, bias=None):
    """Y [Bn x O] = unpack(bits) W^T + bias (vsa-unpack-project.glsl:40-74), fp64 sums."""
    Bn, words = bits.shape
    O, D = W.shape
    bits, pb = _u(bits)
    W, pw = _f(W)
    pbias = None
    if bias is not None:
        bias, pbias = _f(bias)
    Y, py = _out((Bn, O))
    lib().or_vsa_unpack_project_fwd(pb, pw, pbias, py, Bn, O, D, words)
    return Y


def mix64(seed, idx):
    return int(lib().or_mix64(ctypes.c_uint64(seed), ctypes.c_uint64(idx)))


def gumbel(seed, idx):
    return float(lib().or_gumbel(ctypes.c_uint64(seed), ctypes.c_uint64(idx)))


def vsa_select(dots, temperature=1.0, seed=0, counter=0, noise=True):
    """Top-2 + softmax weights of the surrogate forward from given fp32 dots [Bn x K] with
    this build's seeded Gumbel noise (see or_vsa_select).  Returns (results, weights)."""
    Bn, K = dots.shape
    dots, pd = _f(dots)
    results = np.zeros((Bn, 4), dtype=np.uint32)
    weights, pw = _out((Bn, K))
    lib().or_vsa_select(pd, results.ctypes.data_as(ctypes.c_void_p), pw, Bn, K,
                        ctypes.c_float(temperature), ctypes.c_uint64(seed),
                        ctypes.c_uint64(counter), int(noise))
    return results, weights


def vsa_surrogate_loss(preds, bits, results, gamma=1.0, delta=1.0, lambda_c=0.3):
    Bn, K, D = preds.shape
    words = bits.shape[1]
    preds, pp = _f(preds)
    bits, pb = _u(bits)
    results, pr = _u(results)
    loss, pl = _out((Bn,))
    lib().or_vsa_surrogate_loss(pp, pb, pr, pl, Bn, K, D, words, ctypes.c_float(gamma),
                                ctypes.c_float(delta), ctypes.c_float(lambda_c))
    return loss


def vsa_surrogate_fwd(preds, bits, gamma=1.0, delta=1.0, lambda_c=0.3, temperature=1.0, seed=0,
                      counter=0, noise=True):
    """The whole surrogate forward: (dots, results, weights, loss per row)."""
    dots = vsa_dots(preds, bits)
    results, weights = vsa_select(dots, temperature, seed, counter, noise)
    loss = vsa_surrogate_loss(preds, bits, results, gamma, delta, lambda_c)
    return dots, results, weights, loss


def vsa_results_weights(dots, temperature=1.0, rng=None):
    """Seeded restatement of the host top-2 + softmax of vsa_loss_node.cpp:101-148.

    The reference perturbs the dots with unseeded Gumbel noise (vsa_loss_node.cpp:9-14);
    here the noise comes from `rng` (None = no noise), so the backward inputs are
    reproducible.  Returns (results u32 [B,4], weights f32 [B,K]).
    """
    Bn, K = dots.shape
    results = np.zeros((Bn, 4), dtype=np.uint32)
    weights = np.zeros((Bn, K), dtype=np.float32)
    for b in range(Bn):
        adj = dots[b].astype(np.float64)
        if rng is not None:
            u = rng.uniform(1e-8, 1 - 1e-8, size=K)
            adj = adj + (-np.log(-np.log(u))) * temperature
        max1 = max2 = -1e30
        k1 = k2 = 0
        for k in range(K):
            if adj[k] > max1:
                max2, k2 = max1, k1
                max1, k1 = adj[k], k
            elif adj[k] > max2:
                max2, k2 = adj[k], k
        results[b, 0] = k1
        results[b, 1] = k2
        results[b, 2] = np.float32(dots[b, k1]).view(np.uint32)
        results[b, 3] = np.float32(dots[b, k2]).view(np.uint32)
        e = np.exp((dots[b].astype(np.float64) - dots[b].max()) / temperature)
        weights[b] = (e / e.sum()).astype(np.float32)
    return results, weights


def surprise_momentum_step(W, grad, s_bar, recalled=None, eta_base=1e-3, alpha=0.9,
                           lambda_recall=0.0, surprise_floor=0.01, weight_decay=0.0,
                           clip_max=1.0, clear_grad=True):
    """surprise-momentum.glsl:53-114 on copies; returns (W, grad, s_bar, delta) after the step."""
    W, pW = _f(np.array(W, dtype=np.float32, copy=True))
    g, pg = _f(np.array(grad, dtype=np.float32, copy=True))
    s, ps = _f(np.array(s_bar, dtype=np.float32, copy=True))
    d, pd = _out(W.shape)
    r = pr = None
    if recalled is not None:
        r, pr = _f(recalled)
    lib().or_surprise_momentum_step(pW, pg, ps, pd, pr, ctypes.c_int64(W.size),
                                    ctypes.c_float(eta_base), ctypes.c_float(alpha),
                                    ctypes.c_float(lambda_recall), ctypes.c_float(surprise_floor),
                                    ctypes.c_float(weight_decay), ctypes.c_float(clip_max),
                                    int(clear_grad))
    return W, g, s, d


def adamw_step(W, grad, m, v, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.0,
               step=1, clear_grad=True):
    """adamw-update.glsl:41-61 on copies (beta^t from `step`); returns (W, grad, m, v)."""
    W, pW = _f(np.array(W, dtype=np.float32, copy=True))
    g, pg = _f(np.array(grad, dtype=np.float32, copy=True))
    m, pm = _f(np.array(m, dtype=np.float32, copy=True))
    v, pv = _f(np.array(v, dtype=np.float32, copy=True))
    lib().or_adamw_step(pW, pg, pm, pv, ctypes.c_int64(W.size), ctypes.c_float(lr),
                        ctypes.c_float(beta1), ctypes.c_float(beta2), ctypes.c_float(eps),
                        ctypes.c_float(weight_decay), ctypes.c_float(beta1 ** step),
                        ctypes.c_float(beta2 ** step), int(clear_grad))
    return W, g, m, v


BIN = {"sub": 0, "mul": 1, "div": 2, "neg": 3}


def binary_bwd(op, dY, A=None, B=None):
    """Sub / Mul / Div / Neg backward; returns (dA, dB) (dB None for neg)."""
    dY, pY = _f(dY)
    A, pA = _f(A if A is not None else np.zeros_like(dY))
    B, pB = _f(B if B is not None else np.ones_like(dY))
    dA, pdA = _out(dY.shape)
    dB, pdB = _out(dY.shape)
    lib().or_binary_bwd(BIN[op], pY, pA, pB, pdA, pdB, ctypes.c_int64(dY.size))
    return dA, (None if op == "neg" else dB)


def reduce_bwd(op, dY, shape):
    dY, pY = _f(dY)
    dX, pX = _out(shape)
    lib().or_reduce_bwd({"sum": 0, "mean": 1}[op], pY, pX, ctypes.c_int64(dY.size),
                        ctypes.c_int64(dX.size // max(dY.size, 1)))
    return dX


def transpose_bwd(dY):
    dY, pY = _f(dY)
    *lead, cols, rows = dY.shape
    dX, pX = _out((*lead, rows, cols))
    lib().or_transpose_bwd(pY, pX, ctypes.c_int64(dX.size // max(rows * cols, 1)), rows, cols)
    return dX


def mse_bwd(P, T, scale=None, g=1.0):
    P, pP = _f(P)
    T, pT = _f(T)
    dP, pd = _out(P.shape)
    scale = 1.0 / P.size if scale is None else scale
    lib().or_mse_bwd(pP, pT, ctypes.c_float(g), pd, ctypes.c_int64(P.size), ctypes.c_float(scale))
    return dP


def lora_expand_bwd(dP, basis, coeffs, scale=1.0):
    """dP [Bn, K, D], basis [D, rank], coeffs [Bn, K, rank] -> (dCoeffs, dBasis)."""
    dP, pdP = _f(dP)
    basis, pB = _f(basis)
    coeffs, pC = _f(coeffs)
    Bn, K, D = dP.shape
    rank = basis.shape[1]
    dC, pdC = _out((Bn, K, rank))
    dB, pdB = _out((D, rank))
    lib().or_lora_expand_bwd(pdP, pB, pC, pdC, pdB, Bn * K, D, rank, ctypes.c_float(scale))
    return dC, dB


def cosine_blend_bwd(bits, weights, blended, info, K, grad_scale=10.0):
    bits, pb = _u(bits)
    weights, pw = _f(weights)
    blended, pbl = _f(blended)
    info, pi = _f(info)
    Bn, D = blended.shape
    dP, pd = _out((Bn, K, D))
    lib().or_cosine_blend_bwd(pb, pw, pbl, pi, pd, Bn, K, D, bits.shape[1],
                              ctypes.c_float(grad_scale))
    return dP
