"""The numpy restatement bench.py times as the CPU baseline (oracle/cpu_ref.py) computes the
same gradients as the pinned oracle, so the baseline times the right work (fp32 numpy against
fp64-accumulating C: normwise relative error <= 1e-4)."""
import numpy as np

import oracle
from oracle import cpu_ref
from conftest import rel_err

TOL = 1e-4


def test_ffn_block_step():
    r = np.random.default_rng(1)
    T, DM, H = 64, 96, 160
    x = r.standard_normal((T, DM)).astype(np.float32)
    w = (1 + 0.1 * r.standard_normal(DM)).astype(np.float32)
    Wg, Wu = ((r.standard_normal((H, DM)) * 0.1).astype(np.float32) for _ in range(2))
    Wd = (r.standard_normal((DM, H)) * 0.1).astype(np.float32)
    dY = r.standard_normal((T, DM)).astype(np.float32)
    n, rstd = oracle.rmsnorm_fwd(x, w)
    gate, up = oracle.linear_fwd(n, Wg), oracle.linear_fwd(n, Wu)
    a = oracle.glu_fwd("swiglu_up", gate, up)
    dx, dw = cpu_ref.ffn_block_step(x, w, rstd, n, gate, up, a, Wg, Wu, Wd, dY)
    dA, _, _ = oracle.linear_bwd(dY, a, Wd)
    dG, dU = oracle.glu_bwd("swiglu_up", dA, gate, up)
    dN = oracle.linear_bwd(dG, n, Wg)[0] + oracle.linear_bwd(dU, n, Wu)[0]
    rx, rw = oracle.rmsnorm_bwd(dN, x, w, rstd)
    assert rel_err(dx, rx) < TOL and rel_err(dw, rw) < TOL


def test_attention_and_layernorm():
    r = np.random.default_rng(2)
    BH, S, D = 3, 64, 32
    q, k, v = (r.standard_normal((BH, S, D)).astype(np.float32) for _ in range(3))
    dO = r.standard_normal((BH, S, D)).astype(np.float32)
    got = cpu_ref.attention_step(q, k, v, dO, D ** -0.5)
    _, lse = oracle.attn_fwd(q[None], k[None], v[None], rope_mode="none")
    want = oracle.attn_bwd(q[None], k[None], v[None], dO[None], lse, rope_mode="none")
    for g_, w_ in zip(got, want):
        assert rel_err(g_, w_[0]) < TOL
    x = r.standard_normal((40, 24)).astype(np.float32)
    g = (1 + 0.2 * r.standard_normal(24)).astype(np.float32)
    dy = r.standard_normal((40, 24)).astype(np.float32)
    _, mean, rstd = oracle.layernorm_fwd(x, g)
    var = (1.0 / rstd.astype(np.float64) ** 2 - 1e-5).astype(np.float32)
    got = cpu_ref.layernorm_backward(dy, x, g, mean[:, None], var[:, None])
    for g_, w_ in zip(got, oracle.layernorm_bwd(dy, x, g, mean, rstd)):
        assert rel_err(g_, w_) < TOL


def test_mlp_step():
    r = np.random.default_rng(3)
    X = r.standard_normal((16, 40)).astype(np.float32)
    y = r.integers(0, 10, 16).astype(np.int32)
    W1 = (r.standard_normal((32, 40)) * 0.2).astype(np.float32)
    W2 = (r.standard_normal((10, 32)) * 0.2).astype(np.float32)
    Z = oracle.linear_fwd(X, W1)
    H = np.maximum(Z, 0)
    L = oracle.linear_fwd(H, W2)
    dW1, db1, dW2, db2 = cpu_ref.mlp_step(X, y, W1, W2, Z, H, L)
    dL = oracle.xent_bwd(L, y, 1.0)
    dH, rW2, rb2 = oracle.linear_bwd(dL, H, W2)
    dZ = oracle.act_bwd("relu", dH, Z)
    _, rW1, rb1 = oracle.linear_bwd(dZ, X, W1, need_dx=False)
    for g_, w_ in ((dW1, rW1), (db1, rb1), (dW2, rW2), (db2, rb2)):
        assert rel_err(g_, w_) < TOL


def test_hypernet_step():
    r = np.random.RandomState(4)
    d, v, K, rh = 16, 128, 3, 4
    sizes = [d * v, d, 2 * d * d, 2 * d, K * v * 2 * d, K * v, rh * d, rh, K * rh, K]
    W = [(r.standard_normal(n) * 0.1).astype(np.float32) for n in sizes]
    sb = [np.zeros(n, np.float32) for n in sizes]
    bits_s = r.randint(0, 2 ** 32, size=(1, v // 32), dtype=np.uint32)
    bits_d = r.randint(0, 2 ** 32, size=(1, v // 32), dtype=np.uint32)
    W0 = [w.copy() for w in W]
    loss = cpu_ref.hypernet_step(W, bits_s, bits_d, d, v, K, sb)
    # the oracle composition with the noise-free selection
    Wp, bp, W1, b1, W2, b2 = (W0[0].reshape(d, v), W0[1], W0[2].reshape(2 * d, d), W0[3],
                              W0[4].reshape(K * v, 2 * d), W0[5])
    h = oracle.vsa_unpack_project_fwd(bits_s, Wp, bp)
    m = oracle.linear_fwd(h, W1, b1)
    a = oracle.act_fwd("gelu_tanh", m)
    P = oracle.linear_fwd(a, W2, b2).reshape(1, K, v)
    _, res, wts, lo = oracle.vsa_surrogate_fwd(P, bits_d, noise=False)
    dP = oracle.vsa_surrogate_bwd(P, bits_d, res, wts)
    dA, dW2, db2 = oracle.linear_bwd(dP.reshape(1, -1), a, W2)
    dM = oracle.act_bwd("gelu_tanh", dA, m)
    dH, dW1, db1 = oracle.linear_bwd(dM, h, W1)
    dWp, dbp = oracle.vsa_unpack_project_bwd(dH, bits_s, v)
    assert abs(loss - float(lo[0])) < 1e-4 * abs(float(lo[0]))
    for i, g in enumerate([dWp, dbp, dW1, db1, dW2, db2]):
        Wr, _, sr, _ = oracle.surprise_momentum_step(W0[i], g.reshape(-1), np.zeros(sizes[i], np.float32))
        assert rel_err(W[i] - W0[i], Wr - W0[i]) < 1e-3, i  # the update itself (tiny vs W)
        assert rel_err(sb[i], sr) < TOL, i
    for i in range(6, 10):
        np.testing.assert_array_equal(W[i], W0[i])
