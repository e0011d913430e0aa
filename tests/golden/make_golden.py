"""Writes the golden vectors under tests/golden/ (run: python tests/golden/make_golden.py).

The expected outputs come from torch CPU autograd in float64 applied to the FORWARD
definitions of each op — an implementation independent of the oracle's hand-written
backward formulas — so a dropped term, sign or index in the oracle (or the HIP kernels)
disagrees with these files.  Inputs are drawn from numpy.random.default_rng(seed) and
stored as float32; the expected gradients are computed from exactly those float32 values.

Forward definitions used (reference file:line):
  linear        y = x W^T + b                                   fnn-linear.glsl
  activations   relu / gelu(tanh) / gelu(erf) / silu / tanh / sigmoid
                activation-*-backward.glsl, autograd_core.py:529-553
  glu           gate*act(up) / act(gate)*up                     fused-*-backward.glsl
  layernorm     torch layer_norm (biased variance, eps 1e-5)    fnn-layernorm.glsl:44-102
  rmsnorm       w * x * rsqrt(mean(x^2)+eps)                    rms-norm.glsl:34-70
  softmax       softmax over the last axis                      activation-softmax.glsl
  cross-entropy sum over rows of -log softmax[target]           loss-cross-entropy.glsl
  attention     softmax(scale * R(q) R(k)^T, causal) v          flash-attention2-rope.glsl:95-148
  masked attn   the same with (mask - 1) * 1e9 added per key     flash-attention2.glsl:150-154
  rmsnorm stats mean(x^2) and sqrt(mean(x^2) + eps) saved          rms-norm.glsl:52,
                                                                 snn-rmsnorm.glsl:55
  vsa project   y = unpack(bits) W^T + b                        vsa-unpack-project.glsl
  vsa surrogate sum_k w_k mean_i relu(gamma - y_i z_ki) + lambda/D * relu(delta-(dw-dr(z)))
                vsa-surrogate-loss-forward.glsl / -backward.glsl:56-88
  optimizers    torch.optim.AdamW / torch.optim.Adam, three steps  adamw-update.glsl:41-61,
                                                                 adam-update.glsl
  tape ops      a-b, a*b, a/b, -a, sum/mean over trailing dims, transpose, mean((p-t)^2),
                A @ B (autograd.cpp:543-711 stubs); LoRA expand preds = coeffs B^T
                (vsa-lora-expand-forward.glsl); cosine blend loss = -cos(sum_k w_k preds_k, y)
                (vsa-cosine-blend-forward.glsl; the backward's x10 scale and +-1 clamp are applied
                to the autograd gradient)
Run with a list of set names (e.g. `optim`) to write only those files.
"""
import sys
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
torch.set_default_dtype(torch.float64)


def t(a, grad=False):
    x = torch.tensor(np.asarray(a, dtype=np.float64))
    x.requires_grad_(grad)
    return x


def f32(x):
    return np.asarray(x.detach().numpy() if torch.is_tensor(x) else x, dtype=np.float32)


def save(name, **arrays):
    np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrays)


def gen_linear(rng):
    for tag, (M, N, K) in {"small": (5, 7, 11), "c1l2": (64, 10, 256)}.items():
        X = rng.standard_normal((M, K)).astype(np.float32)
        W = (rng.standard_normal((N, K)) * 0.1).astype(np.float32)
        b = rng.standard_normal(N).astype(np.float32)
        dY = rng.standard_normal((M, N)).astype(np.float32)
        x, w, bb = t(X, True), t(W, True), t(b, True)
        ((x @ w.T + bb) * t(dY)).sum().backward()
        save(f"linear_{tag}", X=X, W=W, b=b, dY=dY, dX=f32(x.grad), dW=f32(w.grad),
             db=f32(bb.grad))


def act_forward(kind, x):
    if kind == "relu":
        return torch.relu(x)
    if kind == "gelu_tanh":
        return torch.nn.functional.gelu(x, approximate="tanh")
    if kind == "gelu_erf":
        return torch.nn.functional.gelu(x)
    if kind == "silu":
        return torch.nn.functional.silu(x)
    if kind == "tanh":
        return torch.tanh(x)
    if kind == "sigmoid":
        return torch.sigmoid(x)
    raise ValueError(kind)


def gen_act(rng):
    X = (rng.standard_normal(257) * 3).astype(np.float32)
    X[:4] = [0.0, -0.0, 1e-8, -1e-8]
    dY = rng.standard_normal(257).astype(np.float32)
    out = {"X": X, "dY": dY}
    for kind in ["relu", "gelu_tanh", "gelu_erf", "silu", "tanh", "sigmoid"]:
        x = t(X, True)
        y = act_forward(kind, x)
        (y * t(dY)).sum().backward()
        out["dX_" + kind] = f32(x.grad)
        out["Y_" + kind] = f32(y)
    save("act", **out)


def glu_forward(kind, g, u):
    F = torch.nn.functional
    return {
        "swiglu_up": lambda: g * F.silu(u),
        "swiglu_gate": lambda: F.silu(g) * u,
        "geglu_up": lambda: g * F.gelu(u, approximate="tanh"),
        "geglu_gate": lambda: F.gelu(g, approximate="tanh") * u,
        "reglu_up": lambda: g * torch.relu(u),
    }[kind]()


def gen_glu(rng):
    n = 300
    G = (rng.standard_normal(n) * 2).astype(np.float32)
    U = (rng.standard_normal(n) * 2).astype(np.float32)
    dO = rng.standard_normal(n).astype(np.float32)
    out = {"gate": G, "up": U, "dO": dO}
    for kind in ["swiglu_up", "swiglu_gate", "geglu_up", "geglu_gate", "reglu_up"]:
        g, u = t(G, True), t(U, True)
        (glu_forward(kind, g, u) * t(dO)).sum().backward()
        out["dGate_" + kind] = f32(g.grad)
        out["dUp_" + kind] = f32(u.grad)
    save("glu", **out)


def gen_layernorm(rng):
    rows, F, eps = 9, 33, 1e-5
    X = (rng.standard_normal((rows, F)) * 2 + 0.5).astype(np.float32)
    gamma = rng.standard_normal(F).astype(np.float32)
    beta = rng.standard_normal(F).astype(np.float32)
    dY = rng.standard_normal((rows, F)).astype(np.float32)
    x, g, b = t(X, True), t(gamma, True), t(beta, True)
    y = torch.nn.functional.layer_norm(x, (F,), g, b, eps)
    (y * t(dY)).sum().backward()
    xd = t(X)
    mean = xd.mean(-1)
    var = xd.var(-1, unbiased=False)
    save("layernorm", X=X, gamma=gamma, beta=beta, dY=dY, mean=f32(mean), var=f32(var),
         rstd=f32(1.0 / torch.sqrt(var + eps)), Y=f32(y), dX=f32(x.grad), dGamma=f32(g.grad),
         dBeta=f32(b.grad), eps=np.float32(eps))


def gen_rmsnorm(rng):
    rows, F, eps = 7, 40, 1e-6
    X = rng.standard_normal((rows, F)).astype(np.float32)
    w = (1 + 0.5 * rng.standard_normal(F)).astype(np.float32)
    dY = rng.standard_normal((rows, F)).astype(np.float32)
    x, ww = t(X, True), t(w, True)
    r = torch.rsqrt((x * x).mean(-1, keepdim=True) + eps)
    y = ww * x * r
    (y * t(dY)).sum().backward()
    rd = torch.rsqrt((t(X) ** 2).mean(-1) + eps)
    save("rmsnorm", X=X, w=w, dY=dY, rstd=f32(rd), Y=f32(y), dX=f32(x.grad), dW=f32(ww.grad),
         eps=np.float32(eps))


def gen_softmax_xent(rng):
    rows, C = 6, 19
    Z = (rng.standard_normal((rows, C)) * 3).astype(np.float32)
    dY = rng.standard_normal((rows, C)).astype(np.float32)
    z = t(Z, True)
    y = torch.softmax(z, -1)
    (y * t(dY)).sum().backward()
    save("softmax", X=Z, Y=f32(y), dY=dY, dX=f32(z.grad))
    targets = rng.integers(0, C, size=rows).astype(np.int32)
    z = t(Z, True)
    torch.nn.functional.cross_entropy(z, torch.tensor(targets, dtype=torch.long),
                                      reduction="sum").backward()
    save("xent", logits=Z, targets=targets, dLogits=f32(z.grad))


def rope_t(x, mode, theta):
    """RoPE on [..., S, D] (pos = row index): interleaved pairs (2i,2i+1) or half (i,i+D/2)."""
    S, D = x.shape[-2], x.shape[-1]
    pos = torch.arange(S, dtype=torch.float64)[:, None]
    inv = theta ** (-2.0 * torch.arange(D // 2, dtype=torch.float64) / D)
    ang = pos * inv[None, :]
    c, s = torch.cos(ang), torch.sin(ang)
    if mode == "interleaved":
        x0, x1 = x[..., 0::2], x[..., 1::2]
        y0, y1 = x0 * c - x1 * s, x0 * s + x1 * c
        return torch.stack([y0, y1], dim=-1).reshape(x.shape)
    if mode == "half":
        x0, x1 = x[..., : D // 2], x[..., D // 2:]
        return torch.cat([x0 * c - x1 * s, x0 * s + x1 * c], dim=-1)
    return x


def gen_attention(rng):
    cases = {
        "causal_rope": dict(B=1, H=2, S=13, D=8, causal=True, rope="interleaved"),
        "full_norope": dict(B=2, H=1, S=9, D=16, causal=False, rope="none"),
        "causal_half": dict(B=1, H=1, S=11, D=8, causal=True, rope="half"),
    }
    theta = 10000.0
    for tag, c in cases.items():
        B, H, S, D = c["B"], c["H"], c["S"], c["D"]
        scale = 1.0 / np.sqrt(D)
        Q = rng.standard_normal((B, H, S, D)).astype(np.float32)
        K = rng.standard_normal((B, H, S, D)).astype(np.float32)
        V = rng.standard_normal((B, H, S, D)).astype(np.float32)
        dO = rng.standard_normal((B, H, S, D)).astype(np.float32)
        q, k, v = t(Q, True), t(K, True), t(V, True)
        s = scale * rope_t(q, c["rope"], theta) @ rope_t(k, c["rope"], theta).transpose(-1, -2)
        if c["causal"]:
            s = s.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf"))
        lse = torch.logsumexp(s, -1)
        o = torch.softmax(s, -1) @ v
        (o * t(dO)).sum().backward()
        save(f"attn_{tag}", Q=Q, K=K, V=V, dO=dO, O=f32(o), LSE=f32(lse), dQ=f32(q.grad),
             dK=f32(k.grad), dV=f32(v.grad), scale=np.float32(scale),
             causal=np.int32(c["causal"]), rope=np.array(c["rope"]), theta=np.float32(theta))


def gen_mask_stats(rng):
    """Key-padding-masked attention (flash-attention2.glsl:150-154: score += (mask - 1) * 1e9)
    and the RMSNorm statistic forms the reference's forwards save (rms-norm.glsl:52 mean(x^2),
    snn-rmsnorm.glsl:55 sqrt(mean(x^2) + eps))."""
    cases = {
        "mask_causal_rope": dict(B=2, H=2, S=13, D=8, causal=True, rope="interleaved"),
        "mask_full": dict(B=2, H=1, S=9, D=16, causal=False, rope="none"),
    }
    theta = 10000.0
    for tag, c in cases.items():
        B, H, S, D = c["B"], c["H"], c["S"], c["D"]
        scale = 1.0 / np.sqrt(D)
        Q, K, V, dO = (rng.standard_normal((B, H, S, D)).astype(np.float32) for _ in range(4))
        mask = np.ones((B, S), np.float32)
        mask[1, S - 4:] = 0.0  # a padded tail
        mask[1, 2] = 0.0       # and one key inside the sequence
        q, k, v = t(Q, True), t(K, True), t(V, True)
        s = scale * rope_t(q, c["rope"], theta) @ rope_t(k, c["rope"], theta).transpose(-1, -2)
        s = s + (t(mask)[:, None, None, :] - 1.0) * 1e9
        if c["causal"]:
            s = s.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf"))
        lse = torch.logsumexp(s, -1)
        o = torch.softmax(s, -1) @ v
        (o * t(dO)).sum().backward()
        save(f"attn_{tag}", Q=Q, K=K, V=V, dO=dO, mask=mask, O=f32(o), LSE=f32(lse),
             dQ=f32(q.grad), dK=f32(k.grad), dV=f32(v.grad), scale=np.float32(scale),
             causal=np.int32(c["causal"]), rope=np.array(c["rope"]), theta=np.float32(theta))
    rows, F, eps = 9, 48, 1e-5
    X = rng.standard_normal((rows, F)).astype(np.float32)
    w = (1 + 0.5 * rng.standard_normal(F)).astype(np.float32)
    dY = rng.standard_normal((rows, F)).astype(np.float32)
    x, ww = t(X, True), t(w, True)
    ms = (x * x).mean(-1, keepdim=True)
    y = ww * x * torch.rsqrt(ms + eps)
    (y * t(dY)).sum().backward()
    ms0 = (t(X) ** 2).mean(-1)
    save("rmsnorm_stats", X=X, w=w, dY=dY, meansq=f32(ms0), rms=f32(torch.sqrt(ms0 + eps)),
         rstd=f32(torch.rsqrt(ms0 + eps)), Y=f32(y), dX=f32(x.grad), dW=f32(ww.grad),
         eps=np.float32(eps))


def unpack_t(bits, D):
    b = torch.tensor(bits.astype(np.int64))
    j = torch.arange(D)
    w = b[:, j // 32]
    return ((w >> (j % 32)) & 1).to(torch.float64) * 2 - 1


def gen_vsa(rng):
    Bn, O, D = 6, 5, 96
    words = D // 32
    bits = rng.integers(0, 2**32, size=(Bn, words), dtype=np.uint64).astype(np.uint32)
    bits[0] = 0xFFFFFFFF
    bits[1] = 0
    W = (rng.standard_normal((O, D)) / np.sqrt(D)).astype(np.float32)
    b = rng.standard_normal(O).astype(np.float32)
    dY = rng.standard_normal((Bn, O)).astype(np.float32)
    w, bb = t(W, True), t(b, True)
    y = unpack_t(bits, D) @ w.T + bb
    (y * t(dY)).sum().backward()
    save("vsa_project", bits=bits, W=W, b=b, dY=dY, S=f32(unpack_t(bits, D)), dW=f32(w.grad),
         db=f32(bb.grad))

    # surrogate loss
    Bn, K, D = 4, 3, 64
    words = D // 32
    gamma, delta, lam, scale = 1.0, 1.0, 0.3, 1.0
    preds = rng.standard_normal((Bn, K, D)).astype(np.float32)
    bits = rng.integers(0, 2**32, size=(Bn, words), dtype=np.uint64).astype(np.uint32)
    y = unpack_t(bits, D)
    dots = torch.einsum("bkd,bd->bk", t(preds), y)
    results = np.zeros((Bn, 4), dtype=np.uint32)
    order = torch.argsort(dots, dim=1, descending=True).numpy()
    for bi in range(Bn):
        win, run = int(order[bi, 0]), int(order[bi, 1])
        if bi == 3:
            run = win  # exercises the win == run branch
        results[bi, 0], results[bi, 1] = win, run
        results[bi, 2] = np.float32(dots[bi, win].item()).view(np.uint32)
        results[bi, 3] = np.float32(dots[bi, run].item()).view(np.uint32)
    # make sample 0's contrastive margin active, sample 1's inactive
    wts = torch.softmax(dots, dim=1)
    weights = f32(wts)
    z = t(preds, True)
    wt = t(weights)
    hinge = (wt[:, :, None] * torch.relu(gamma - y[:, None, :] * z)).sum() / D
    con = 0.0
    for bi in range(Bn):
        win, run = int(results[bi, 0]), int(results[bi, 1])
        if win == run:
            continue
        dw = float(np.uint32(results[bi, 2]).view(np.float32))
        dr = (z[bi, run] * y[bi]).sum()
        con = con + torch.relu(delta - (dw - dr))
    loss = hinge + lam / D * con
    loss.backward()
    save("vsa_surrogate", preds=preds, bits=bits, results=results, weights=weights,
         dPreds=f32(z.grad), gamma=np.float32(gamma), delta=np.float32(delta),
         lambda_c=np.float32(lam), scale=np.float32(scale))


def gen_optim(rng):
    """AdamW (decoupled decay) and Adam over three steps with fresh gradients each step;
    torch's update is W(1 - lr wd) - lr/bc1 m / (sqrt(v)/sqrt(bc2) + eps), the shader's
    W(1 - lr wd) - lr m_hat / (sqrt(v_hat) + eps) written differently."""
    n = 37
    W0 = rng.standard_normal(n).astype(np.float32)
    grads = (rng.standard_normal((3, n)) * np.array([1.0, 1e-3, 10.0])[:, None]).astype(np.float32)
    # hyperparameters exactly representable in float32: the shader (and the ABI) take them as
    # fp32 push constants, so e.g. beta2 = 0.999 would differ from torch's double by 1.3e-5
    for tag, cls, kw in (("adamw", torch.optim.AdamW, dict(lr=2.0**-7, betas=(0.875, 1 - 2.0**-10),
                                                           eps=2.0**-26, weight_decay=0.125)),
                         ("adam", torch.optim.Adam, dict(lr=2.0**-8, betas=(0.75, 0.984375),
                                                         eps=2.0**-20, weight_decay=0.0))):
        w = t(W0)
        w.requires_grad_(True)
        opt = cls([w], **kw)
        Ws, ms, vs = [], [], []
        for k in range(3):
            w.grad = t(grads[k])
            opt.step()
            st = opt.state[w]
            Ws.append(f32(w))
            ms.append(f32(st["exp_avg"]))
            vs.append(f32(st["exp_avg_sq"]))
        save("optim_" + tag, W0=W0, grads=grads, W=np.stack(Ws), m=np.stack(ms), v=np.stack(vs),
             lr=np.float32(kw["lr"]), beta1=np.float32(kw["betas"][0]),
             beta2=np.float32(kw["betas"][1]), eps=np.float32(kw["eps"]),
             weight_decay=np.float32(kw["weight_decay"]))


def gen_tapeops(rng):
    n = (5, 7)
    a = rng.standard_normal(n).astype(np.float32)
    b = (rng.standard_normal(n) + np.sign(rng.standard_normal(n)) * 1.5).astype(np.float32)
    dy = rng.standard_normal(n).astype(np.float32)
    out = dict(a=a, b=b, dy=dy)
    for name, fn in (("sub", lambda x, y: x - y), ("mul", lambda x, y: x * y),
                     ("div", lambda x, y: x / y), ("neg", lambda x, y: -x)):
        x, y = t(a, True), t(b, True)
        r = fn(x, y)
        r.backward(t(dy))
        out["d" + name + "_a"] = f32(x.grad)
        out["d" + name + "_b"] = f32(y.grad) if y.grad is not None else np.zeros(n, np.float32)
    X = rng.standard_normal((3, 4, 6)).astype(np.float32)
    for name, fn in (("sum", lambda x: x.sum(-1)), ("mean", lambda x: x.mean(-1)),
                     ("sumall", lambda x: x.sum().reshape(1)), ("meanall", lambda x: x.mean().reshape(1))):
        x = t(X, True)
        r = fn(x)
        g = rng.standard_normal(tuple(r.shape)).astype(np.float32)
        r.backward(t(g))
        out[name + "_dy"], out[name + "_dx"] = g, f32(x.grad)
    x = t(X, True)
    r = x.transpose(-1, -2)
    g = rng.standard_normal(tuple(r.shape)).astype(np.float32)
    r.backward(t(g))
    out["X"], out["tr_dy"], out["tr_dx"] = X, g, f32(x.grad)
    p, tg = rng.standard_normal(11).astype(np.float32), rng.standard_normal(11).astype(np.float32)
    x = t(p, True)
    ((x - t(tg)) ** 2).mean().backward()
    out["mse_p"], out["mse_t"], out["mse_dp"] = p, tg, f32(x.grad)
    A, B = rng.standard_normal((6, 9)).astype(np.float32), rng.standard_normal((9, 4)).astype(np.float32)
    G = rng.standard_normal((6, 4)).astype(np.float32)
    x, y = t(A, True), t(B, True)
    (x @ y).backward(t(G))
    out.update(mm_a=A, mm_b=B, mm_dc=G, mm_da=f32(x.grad), mm_db=f32(y.grad))
    save("tapeops", **out)
    # LoRA expand: preds[b,k,i] = sum_r B[i,r] c[b,k,r]
    Bn, K, D, rank = 3, 2, 40, 5
    basis = rng.standard_normal((D, rank)).astype(np.float32)
    coeffs = rng.standard_normal((Bn, K, rank)).astype(np.float32)
    dP = rng.standard_normal((Bn, K, D)).astype(np.float32)
    cb, cc = t(basis, True), t(coeffs, True)
    torch.einsum("ir,bkr->bki", cb, cc).backward(t(dP))
    save("lora_expand", basis=basis, coeffs=coeffs, dP=dP, dcoeffs=f32(cc.grad), dbasis=f32(cb.grad))
    # cosine blend: blended = sum_k w_k preds_k, loss = -cos(blended, y) per row
    Bn, K, D = 3, 4, 96
    words = D // 32
    bits = rng.integers(0, 2**32, size=(Bn, words), dtype=np.uint64).astype(np.uint32)
    y = np.where((bits[:, np.arange(D) >> 5] >> (np.arange(D) & 31)) & 1, 1.0, -1.0)
    preds = (rng.standard_normal((Bn, K, D)) * 0.05).astype(np.float32)
    w = rng.dirichlet(np.ones(K), size=Bn).astype(np.float32)
    pr = t(preds, True)
    blended = (t(w)[:, :, None] * pr).sum(1)
    cos = (blended * t(y)).sum(1) / (blended.norm(dim=1) * np.sqrt(D))
    (-cos).sum().backward()
    bl = f32(blended)
    info = np.stack([1.0 - f32(cos), (bl * y).sum(1), (bl * bl).sum(1)], 1).astype(np.float32)
    save("cosine_blend", bits=bits, preds=preds, weights=w, blended=bl, info=info,
         dpreds=np.clip(10.0 * f32(pr.grad), -1.0, 1.0).astype(np.float32),
         dpreds_raw=f32(pr.grad))


def main(only=()):
    rng = np.random.default_rng(20261201)
    sets = [("linear", gen_linear), ("act", gen_act), ("glu", gen_glu),
            ("layernorm", gen_layernorm), ("rmsnorm", gen_rmsnorm),
            ("softmax_xent", gen_softmax_xent), ("attention", gen_attention), ("vsa", gen_vsa)]
    for name, fn in sets:
        if not only or name in only:
            fn(rng)
    if not only or "optim" in only:
        gen_optim(np.random.default_rng(20261202))
    if not only or "tapeops" in only:
        gen_tapeops(np.random.default_rng(20261203))
    if not only or "mask" in only:
        gen_mask_stats(np.random.default_rng(20261204))
    print("golden vectors written to", HERE)


if __name__ == "__main__":
    main(tuple(sys.argv[1:]))
