"""Pins the CPU oracle (oracle/) before anything is checked against it.

Each oracle function is checked against
  * golden vectors from torch float64 autograd of the op's forward definition
    (tests/golden/make_golden.py) — independent of the oracle's backward formulas;
  * the reference's own known-answer tests where they exist
    (tests/test_vsa_hypernetwork.py:151-202, tests/test_vsa_training_loop.py:131-148);
  * closed forms and invariants chosen so a dropped term, sign or index fails.
Tolerance: normwise relative error (max|a-b|/max|b|) <= 1e-5 (fp32 output of an fp64
computation).
"""
import numpy as np
import pytest

import oracle
from conftest import golden, rel_err

TOL = 1e-5


def test_linear_golden():
    for tag in ["small", "c1l2"]:
        g = golden(f"linear_{tag}")
        dX, dW, db = oracle.linear_bwd(g["dY"], g["X"], g["W"])
        assert rel_err(dX, g["dX"]) < TOL
        assert rel_err(dW, g["dW"]) < TOL
        assert rel_err(db, g["db"]) < TOL


def test_linear_transpose_identity():
    # dX = dY W must equal (W^T dY^T)^T, and dW for a one-hot dY row picks that X row.
    rng = np.random.default_rng(0)
    X = rng.standard_normal((4, 6)).astype(np.float32)
    W = rng.standard_normal((3, 6)).astype(np.float32)
    dY = np.zeros((4, 3), np.float32)
    dY[2, 1] = 1.0
    dX, dW, db = oracle.linear_bwd(dY, X, W)
    np.testing.assert_array_equal(dX[2], W[1])
    np.testing.assert_array_equal(dW[1], X[2])
    assert np.count_nonzero(dW[[0, 2]]) == 0
    np.testing.assert_array_equal(db, [0, 1, 0])


def test_linear_fwd_matches_numpy_matmul():
    # fnn-linear.glsl:33-55: Y = X W^T + b, against numpy's fp64 matmul (a transposed W or a
    # dropped bias fails; W is not square, so X W would not even have Y's shape)
    for tag in ["small", "c1l2"]:
        g = golden(f"linear_{tag}")
        X, W, b = (g[k].astype(np.float64) for k in ("X", "W", "b"))
        assert rel_err(oracle.linear_fwd(g["X"], g["W"], g["b"]), X @ W.T + b) < TOL
        assert rel_err(oracle.linear_fwd(g["X"], g["W"]), X @ W.T) < TOL


@pytest.mark.parametrize("kind", ["relu", "gelu_tanh", "gelu_erf", "silu", "tanh", "sigmoid"])
def test_act_golden(kind):
    g = golden("act")
    # tanh/sigmoid backward take the saved forward output (activation-tanh-backward.glsl:33)
    inp = g["Y_" + kind] if kind in ("tanh", "sigmoid") else g["X"]
    dX = oracle.act_bwd(kind, g["dY"], inp)
    assert rel_err(dX, g["dX_" + kind]) < TOL


def test_relu_strict_at_zero():
    # activation-relu-backward.glsl:35: derivative is 1 only for x > 0 (0 at x == 0)
    dX = oracle.act_bwd("relu", np.ones(3, np.float32), np.array([0.0, -0.0, 1e-30], np.float32))
    np.testing.assert_array_equal(dX, [0.0, 0.0, 1.0])


@pytest.mark.parametrize("kind", ["swiglu_up", "swiglu_gate", "geglu_up", "geglu_gate", "reglu_up"])
def test_glu_golden(kind):
    g = golden("glu")
    dG, dU = oracle.glu_bwd(kind, g["dO"], g["gate"], g["up"])
    assert rel_err(dG, g["dGate_" + kind]) < TOL
    assert rel_err(dU, g["dUp_" + kind]) < TOL


@pytest.mark.parametrize("kind", ["swiglu_up", "swiglu_gate", "geglu_up", "geglu_gate", "reglu_up"])
def test_glu_fwd_against_torch_activations(kind):
    # fused-swiglu.glsl:78, fused-geglu.glsl:81, fused-reglu.glsl:73, against torch's own
    # float64 SiLU / tanh-GELU / ReLU (library routines, not a retyped formula)
    torch = pytest.importorskip("torch")
    F = torch.nn.functional
    g = golden("glu")
    tg, tu = torch.from_numpy(g["gate"]).double(), torch.from_numpy(g["up"]).double()
    ref = {"swiglu_up": tg * F.silu(tu), "swiglu_gate": F.silu(tg) * tu,
           "geglu_up": tg * F.gelu(tu, approximate="tanh"),
           "geglu_gate": F.gelu(tg, approximate="tanh") * tu, "reglu_up": tg * F.relu(tu)}[kind]
    assert rel_err(oracle.glu_fwd(kind, g["gate"], g["up"]), ref.numpy()) < TOL


def test_glu_orientation_differs():
    # the two SwiGLU conventions (fused-swiglu-backward.glsl vs swiglu-fused.glsl) really differ
    g = golden("glu")
    a = oracle.glu_bwd("swiglu_up", g["dO"], g["gate"], g["up"])[0]
    b = oracle.glu_bwd("swiglu_gate", g["dO"], g["gate"], g["up"])[0]
    assert rel_err(a, b) > 0.1


def test_layernorm_golden():
    g = golden("layernorm")
    dX, dG, dB = oracle.layernorm_bwd(g["dY"], g["X"], g["gamma"], g["mean"], g["rstd"])
    assert rel_err(dX, g["dX"]) < TOL
    assert rel_err(dG, g["dGamma"]) < TOL
    assert rel_err(dB, g["dBeta"]) < TOL
    # the variance form (the reference saves var, fnn-layernorm.glsl:77) gives the same
    dX2, _, _ = oracle.layernorm_bwd(g["dY"], g["X"], g["gamma"], g["mean"], g["var"],
                                     eps=float(g["eps"]), stat_is_var=True)
    assert rel_err(dX2, g["dX"]) < TOL
    # forward restatement reproduces the saved statistics
    Y, mean, rstd = oracle.layernorm_fwd(g["X"], g["gamma"], g["beta"], eps=float(g["eps"]))
    assert rel_err(mean, g["mean"]) < TOL and rel_err(rstd, g["rstd"]) < TOL
    assert rel_err(Y, g["Y"]) < TOL


def test_layernorm_glsl_form_agrees_only_at_unit_gamma():
    # fnn-layernorm-backward.glsl:124 multiplies gamma into the mean terms.  At gamma == 1
    # it coincides with the textbook form; with a random gamma it does not.
    g = golden("layernorm")
    ones = np.ones_like(g["gamma"])
    a = oracle.layernorm_bwd(g["dY"], g["X"], ones, g["mean"], g["rstd"])[0]
    b = oracle.layernorm_bwd_glsl(g["dY"], g["X"], ones, g["mean"], g["rstd"])
    assert rel_err(a, b) < TOL
    c = oracle.layernorm_bwd_glsl(g["dY"], g["X"], g["gamma"], g["mean"], g["rstd"])
    assert rel_err(c, g["dX"]) > 1e-2


def test_rmsnorm_golden():
    g = golden("rmsnorm")
    dX, dW = oracle.rmsnorm_bwd(g["dY"], g["X"], g["w"], g["rstd"])
    assert rel_err(dX, g["dX"]) < TOL
    assert rel_err(dW, g["dW"]) < TOL
    Y, rstd = oracle.rmsnorm_fwd(g["X"], g["w"], eps=float(g["eps"]))
    assert rel_err(rstd, g["rstd"]) < TOL and rel_err(Y, g["Y"]) < TOL


def test_rmsnorm_scale_invariance():
    # y(c x) = y(x) for c > 0 when eps -> 0, so dx . x = 0 for every row (eps = 0 case).
    rng = np.random.default_rng(1)
    X = rng.standard_normal((5, 16)).astype(np.float32)
    w = rng.standard_normal(16).astype(np.float32)
    dY = rng.standard_normal((5, 16)).astype(np.float32)
    _, rstd = oracle.rmsnorm_fwd(X, w, eps=0.0)
    dX, _ = oracle.rmsnorm_bwd(dY, X, w, rstd)
    assert np.max(np.abs(np.sum(dX * X, axis=1))) < 1e-4


def test_softmax_golden_and_invariant():
    g = golden("softmax")
    dX = oracle.softmax_bwd(g["dY"], g["Y"])
    assert rel_err(dX, g["dX"]) < TOL
    assert np.max(np.abs(dX.sum(axis=1))) < 1e-5  # shift invariance: rows sum to zero
    assert rel_err(oracle.softmax_fwd(g["X"]), g["Y"]) < TOL


def test_xent_golden_and_invariant():
    g = golden("xent")
    dL = oracle.xent_bwd(g["logits"], g["targets"], 1.0)
    assert rel_err(dL, g["dLogits"]) < TOL
    assert np.max(np.abs(dL.sum(axis=1))) < 1e-5
    # scale multiplies (the reference uses scale 1: no 1/B, cross-entropy-backward.glsl:77-83)
    assert rel_err(oracle.xent_bwd(g["logits"], g["targets"], 0.25), 0.25 * g["dLogits"]) < TOL
    # the target column is the only negative one
    for r, tgt in enumerate(g["targets"]):
        assert dL[r, tgt] < 0 and np.all(np.delete(dL[r], tgt) > 0)


def test_rope_orthogonal():
    rng = np.random.default_rng(2)
    X = rng.standard_normal((7, 8)).astype(np.float32)
    for mode in ["interleaved", "half"]:
        Y = oracle.rope(X, mode)
        np.testing.assert_allclose(np.linalg.norm(Y, axis=1), np.linalg.norm(X, axis=1), rtol=1e-5)
        np.testing.assert_allclose(oracle.rope(Y, mode, inverse=True), X, atol=1e-5)
        np.testing.assert_array_equal(Y[0], X[0])  # position 0 is the identity
    # interleaved pair 0 at position 1 rotates by exactly 1 radian
    Y = oracle.rope(X, "interleaved")
    c, s = np.cos(1.0), np.sin(1.0)
    np.testing.assert_allclose(Y[1, :2], [X[1, 0] * c - X[1, 1] * s, X[1, 0] * s + X[1, 1] * c],
                               rtol=1e-5)


@pytest.mark.parametrize("tag", ["causal_rope", "full_norope", "causal_half"])
def test_attention_golden(tag):
    g = golden(f"attn_{tag}")
    kw = dict(scale=float(g["scale"]), causal=bool(g["causal"]), rope_mode=str(g["rope"]),
              theta=float(g["theta"]))
    O, LSE = oracle.attn_fwd(g["Q"], g["K"], g["V"], **kw)
    assert rel_err(O, g["O"]) < TOL and rel_err(LSE, g["LSE"]) < TOL
    dQ, dK, dV = oracle.attn_bwd(g["Q"], g["K"], g["V"], g["dO"], g["LSE"], **kw)
    assert rel_err(dQ, g["dQ"]) < TOL
    assert rel_err(dK, g["dK"]) < TOL
    assert rel_err(dV, g["dV"]) < TOL


@pytest.mark.parametrize("tag", ["mask_causal_rope", "mask_full"])
def test_attention_key_mask_golden(tag):
    """The key-padding bias (mask - 1) * 1e9 of flash-attention2.glsl:150-154, against torch
    float64 autograd of the masked forward."""
    g = golden(f"attn_{tag}")
    kw = dict(scale=float(g["scale"]), causal=bool(g["causal"]), rope_mode=str(g["rope"]),
              theta=float(g["theta"]), mask=g["mask"])
    O, LSE = oracle.attn_fwd(g["Q"], g["K"], g["V"], **kw)
    assert rel_err(O, g["O"]) < TOL and rel_err(LSE, g["LSE"]) < TOL
    dQ, dK, dV = oracle.attn_bwd(g["Q"], g["K"], g["V"], g["dO"], g["LSE"], **kw)
    assert rel_err(dQ, g["dQ"]) < TOL
    assert rel_err(dK, g["dK"]) < TOL
    assert rel_err(dV, g["dV"]) < TOL


def test_attention_key_mask_equals_removing_keys():
    """Without the causal mask and RoPE, masking keys is attention over the kept keys alone:
    O, LSE and dQ equal those of the shortened key/value sequence, and the masked keys get
    dK = dV = 0."""
    rng = np.random.default_rng(5)
    B, H, S, D = 1, 2, 12, 8
    Q, K, V, dO = (rng.standard_normal((B, H, S, D)).astype(np.float32) for _ in range(4))
    mask = np.ones((B, S), np.float32)
    drop = [3, 7, 8]
    mask[0, drop] = 0.0
    keep = [j for j in range(S) if j not in drop]
    kw = dict(causal=False, rope_mode="none")
    O, LSE = oracle.attn_fwd(Q, K, V, mask=mask, **kw)
    dQ, dK, dV = oracle.attn_bwd(Q, K, V, dO, LSE, mask=mask, **kw)
    # the shortened problem: queries stay, keys/values are the kept ones (pad queries to the key
    # count is not needed: the oracle takes equal lengths, so run it per query row block)
    Kk, Vk = K[:, :, keep], V[:, :, keep]
    for i in range(S):
        q = np.ascontiguousarray(np.repeat(Q[:, :, i:i + 1], len(keep), axis=2))
        g = np.zeros_like(q)
        g[:, :, 0] = dO[:, :, i]
        o, l = oracle.attn_fwd(q, Kk, Vk, **kw)
        np.testing.assert_allclose(o[:, :, 0], O[:, :, i], rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(l[:, :, 0], LSE[:, :, i], rtol=1e-6, atol=1e-6)
        dq, _, _ = oracle.attn_bwd(q, Kk, Vk, g, l, **kw)
        np.testing.assert_allclose(dq[:, :, 0], dQ[:, :, i], rtol=1e-4, atol=1e-6)
    assert np.all(dK[:, :, drop] == 0.0) and np.all(dV[:, :, drop] == 0.0)


def test_attention_single_key_closed_form():
    # S == 1: P == 1, so dV == dO and dS == P (dP - rowdot) == 0 -> dQ == dK == 0.
    rng = np.random.default_rng(3)
    Q, K, V, dO = (rng.standard_normal((1, 2, 1, 8)).astype(np.float32) for _ in range(4))
    O, LSE = oracle.attn_fwd(Q, K, V)
    dQ, dK, dV = oracle.attn_bwd(Q, K, V, dO, LSE)
    np.testing.assert_allclose(dV, dO, rtol=1e-6)
    assert np.max(np.abs(dQ)) < 1e-6 and np.max(np.abs(dK)) < 1e-6


def test_bitunpack_reference_kat():
    # tests/test_vsa_training_loop.py:131-148: 0xFFFFFFFF -> all +1, 0 -> all -1
    ones = oracle.unpack_bits(np.array([[0xFFFFFFFF, 0xFFFFFFFF]], np.uint32), 64)
    zeros = oracle.unpack_bits(np.array([[0, 0]], np.uint32), 64)
    assert np.all(ones == 1.0) and np.all(zeros == -1.0)
    # LSB-first little-endian order equals np.unpackbits(bitorder="little") (vsa_loop.py:170-175)
    rng = np.random.default_rng(4)
    bits = rng.integers(0, 2**32, size=(3, 5), dtype=np.uint64).astype(np.uint32)
    ref = np.unpackbits(bits.view(np.uint8), axis=1, bitorder="little").astype(np.float32) * 2 - 1
    np.testing.assert_array_equal(oracle.unpack_bits(bits, 160), ref)


def test_vsa_project_golden():
    g = golden("vsa_project")
    D = g["W"].shape[1]
    np.testing.assert_array_equal(oracle.unpack_bits(g["bits"], D), g["S"])
    dW, db = oracle.vsa_unpack_project_bwd(g["dY"], g["bits"], D)
    assert rel_err(dW, g["dW"]) < TOL and rel_err(db, g["db"]) < TOL


def test_vsa_project_popcount_identity():
    # with dY == 1: dW[o, j] = sum_b s_b(j) = 2 * popcount_j - B exactly (integer identity)
    rng = np.random.default_rng(5)
    Bn, O, D = 37, 3, 128
    bits = rng.integers(0, 2**32, size=(Bn, D // 32), dtype=np.uint64).astype(np.uint32)
    dW, db = oracle.vsa_unpack_project_bwd(np.ones((Bn, O), np.float32), bits, D)
    pop = np.unpackbits(bits.view(np.uint8), axis=1, bitorder="little").sum(axis=0).astype(np.int64)
    for o in range(O):
        np.testing.assert_array_equal(dW[o], 2 * pop - Bn)
    np.testing.assert_array_equal(db, Bn)


def test_vsa_surrogate_golden():
    g = golden("vsa_surrogate")
    dP = oracle.vsa_surrogate_bwd(g["preds"], g["bits"], g["results"], g["weights"],
                                  float(g["gamma"]), float(g["delta"]), float(g["lambda_c"]),
                                  float(g["scale"]))
    assert rel_err(dP, g["dPreds"]) < TOL


def _surrogate_case(preds_fn, gamma, dots_win_run=None, K=4, D=256):
    rng = np.random.default_rng(6)
    bits = rng.integers(0, 2**32, size=(1, D // 32), dtype=np.uint64).astype(np.uint32)
    y = oracle.unpack_bits(bits, D)[0]
    preds = np.stack([preds_fn(y) for _ in range(K)])[None].astype(np.float32)
    weights = np.full((1, K), 1.0 / K, np.float32)
    res = np.zeros((1, 4), np.uint32)
    res[0, 0], res[0, 1] = 0, 1
    dw, dr = dots_win_run if dots_win_run else (0.0, 0.0)
    res[0, 2] = np.float32(dw).view(np.uint32)
    res[0, 3] = np.float32(dr).view(np.uint32)
    return preds, bits, res, weights, y


def test_vsa_surrogate_reference_kats():
    K, D = 4, 256
    # perfect prediction (test_vsa_hypernetwork.py:151-165): every hinge inactive; the
    # contrastive margin 0.5 - (100 - 99) < 0 is inactive too -> zero gradient
    p, bits, res, w, y = _surrogate_case(lambda y: 2.0 * y, 0.1, (100.0, 99.0))
    dP = oracle.vsa_surrogate_bwd(p, bits, res, w, gamma=0.1, delta=0.5, lambda_c=0.3)
    assert np.count_nonzero(dP) == 0
    # adversarial (test_vsa_hypernetwork.py:167-178): every hinge active -> -y/D * w_k
    p, bits, res, w, y = _surrogate_case(lambda y: -np.ones_like(y), 0.1, (100.0, 99.0))
    p = -np.abs(p) * 0 - y[None, None, :]  # prediction opposes the target everywhere
    dP = oracle.vsa_surrogate_bwd(p, bits, res, w, gamma=0.1, delta=0.5, lambda_c=0.3)
    np.testing.assert_allclose(dP[0], np.tile(-y / D / K, (K, 1)), rtol=1e-6)
    # contrastive too close (test_vsa_hypernetwork.py:192-202): 0.5 - (100 - 99.8) = 0.3 > 0
    # -> runner-up additionally gets +lambda*y/D
    p, bits, res, w, y = _surrogate_case(lambda y: 2.0 * y, 0.1, (100.0, 99.8))
    dP = oracle.vsa_surrogate_bwd(p, bits, res, w, gamma=0.1, delta=0.5, lambda_c=0.3)
    np.testing.assert_allclose(dP[0, 1], 0.3 * y / D, rtol=1e-6)
    assert np.count_nonzero(dP[0, [0, 2, 3]]) == 0


@pytest.mark.parametrize("kind", ["relu", "gelu_tanh", "gelu_erf", "silu", "tanh", "sigmoid"])
def test_act_fwd_golden(kind):
    # forward values against torch float64 (tests/golden/make_golden.py: Y_* arrays)
    g = golden("act")
    assert rel_err(oracle.act_fwd(kind, g["X"]), g["Y_" + kind]) < TOL


def test_vsa_dots_brute_force():
    # vsa-surrogate-loss-forward.glsl pass 0 against an explicit unpack + fp64 dot per (b, k)
    rng = np.random.default_rng(21)
    Bn, K, D = 3, 5, 96
    bits = rng.integers(0, 2**32, size=(Bn, D // 32), dtype=np.uint64).astype(np.uint32)
    preds = rng.standard_normal((Bn, K, D)).astype(np.float32)
    y = np.unpackbits(bits.view(np.uint8), axis=1, bitorder="little").astype(np.float64) * 2 - 1
    ref = np.array([[float(np.dot(preds[b, k].astype(np.float64), y[b])) for k in range(K)]
                    for b in range(Bn)])
    assert rel_err(oracle.vsa_dots(preds, bits), ref) < TOL
    # all-ones target: the dot is the plain row sum; all-zeros: minus it
    ones = np.full((Bn, D // 32), 0xFFFFFFFF, np.uint32)
    np.testing.assert_allclose(oracle.vsa_dots(preds, ones), preds.sum(-1), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(oracle.vsa_dots(preds, np.zeros_like(ones)), -preds.sum(-1),
                               rtol=1e-5, atol=1e-5)


def test_splitmix64_known_answers():
    # splitmix64 from state 0 (Steele, Lea & Flood 2014): the published first outputs
    assert [oracle.mix64(0, i) for i in range(3)] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4,
                                                      0x06C45D188009454F]


def test_gumbel_moments():
    # standard Gumbel: mean = Euler-Mascheroni gamma, variance = pi^2 / 6 (a sign slip in
    # -log(-log u) moves the mean to -gamma; a dropped log gives an exponential, mean 1)
    g = np.array([oracle.gumbel(11, i) for i in range(60000)])
    se = np.sqrt(np.pi ** 2 / 6 / g.size)
    assert abs(g.mean() - 0.5772156649) < 5 * se
    assert abs(g.var() - np.pi ** 2 / 6) < 0.05
    # quantiles of exp(-exp(-g)) are uniform
    u = np.exp(-np.exp(-g))
    assert abs(np.mean(u < 0.25) - 0.25) < 0.01 and abs(np.mean(u < 0.75) - 0.75) < 0.01


def test_vsa_select_known_answers():
    # noise-free top-2 (vsa_loss_node.cpp:102-119): strict >, the earlier index wins ties,
    # both start at index 0; softmax weights sum to 1 and follow the dots' order
    dots = np.array([[3.0, 1.0, 2.0, -1.0], [1.0, 1.0, 0.0, 0.5], [0.0, 5.0, 5.0, 4.0]], np.float32)
    res, w = oracle.vsa_select(dots, noise=False)
    assert res[:, :2].tolist() == [[0, 2], [0, 1], [1, 2]]
    np.testing.assert_array_equal(res[:, 2].view(np.float32), [3.0, 1.0, 5.0])
    np.testing.assert_array_equal(res[:, 3].view(np.float32), [2.0, 1.0, 5.0])
    np.testing.assert_allclose(w.sum(1), 1.0, rtol=1e-6)
    e = np.exp(dots[0] - 3.0)
    np.testing.assert_allclose(w[0], e / e.sum(), rtol=1e-6)
    # temperature 2 halves the logits
    _, w2 = oracle.vsa_select(dots, temperature=2.0, noise=False)
    e = np.exp((dots[0] - 3.0) / 2)
    np.testing.assert_allclose(w2[0], e / e.sum(), rtol=1e-6)
    # one branch: winner and runner-up are both 0 (no contrastive term)
    res1, w1 = oracle.vsa_select(dots[:, :1], noise=False)
    assert res1[:, :2].tolist() == [[0, 0]] * 3 and np.all(w1 == 1.0)


def test_vsa_select_noise_order():
    # with noise, the winner is the argmax of dots + T g where g is drawn at index
    # (counter * Bn + b) * K + k; the recorded dots stay the unperturbed ones
    rng = np.random.default_rng(22)
    Bn, K, T, seed, ctr = 4, 6, 0.7, 1234, 3
    dots = rng.standard_normal((Bn, K)).astype(np.float32)
    res, _ = oracle.vsa_select(dots, temperature=T, seed=seed, counter=ctr)
    for b in range(Bn):
        adj = [np.float32(dots[b, k]) + np.float32(oracle.gumbel(seed, (ctr * Bn + b) * K + k))
               * np.float32(T) for k in range(K)]
        order = np.argsort(-np.array(adj, np.float64), kind="stable")
        assert res[b, 0] == order[0] and res[b, 1] == order[1]
        assert res[b, 2].view(np.float32) == dots[b, order[0]]


def test_vsa_surrogate_loss_reference_kats():
    # tests/test_vsa_hypernetwork.py:151-202 as losses: perfect prediction -> hinge 0;
    # adversarial -> gamma + 1; contrastive 100 vs 99.8 at margin 0.5 -> 0.3 (times lambda)
    D, K = 256, 2
    rng = np.random.default_rng(23)
    bits = rng.integers(0, 2**32, size=(1, D // 32), dtype=np.uint64).astype(np.uint32)
    y = oracle.unpack_bits(bits, D)[0]
    res = np.zeros((1, 4), np.uint32)
    res[0, 1] = 1
    res[0, 2], res[0, 3] = np.float32(100.0).view(np.uint32), np.float32(99.0).view(np.uint32)
    perfect = np.stack([2 * y, 2 * y])[None]
    assert oracle.vsa_surrogate_loss(perfect, bits, res, gamma=0.1, delta=0.5)[0] == 0.0
    adv = np.stack([-y, -y])[None]
    np.testing.assert_allclose(oracle.vsa_surrogate_loss(adv, bits, res, gamma=0.1, delta=0.5),
                               1.1, rtol=1e-6)
    res[0, 3] = np.float32(99.8).view(np.uint32)
    np.testing.assert_allclose(oracle.vsa_surrogate_loss(perfect, bits, res, gamma=0.1, delta=0.5,
                                                         lambda_c=0.3), 0.3 * 0.3, rtol=1e-4)
    # the loss reads the winner's row only: another row's predictions do not matter
    mixed = np.stack([2 * y, -y])[None]
    res[0, 3] = np.float32(99.0).view(np.uint32)
    assert oracle.vsa_surrogate_loss(mixed, bits, res, gamma=0.1, delta=0.5)[0] == 0.0


def test_vsa_unpack_project_fwd():
    rng = np.random.default_rng(24)
    Bn, O, D = 3, 7, 128
    bits = rng.integers(0, 2**32, size=(Bn, D // 32), dtype=np.uint64).astype(np.uint32)
    W = rng.standard_normal((O, D)).astype(np.float32)
    b = rng.standard_normal(O).astype(np.float32)
    S = oracle.unpack_bits(bits, D).astype(np.float64)
    assert rel_err(oracle.vsa_unpack_project_fwd(bits, W, b), S @ W.T.astype(np.float64) + b) < TOL
    # all bits set: each output is its weight row's sum plus the bias
    ones = np.full((1, D // 32), 0xFFFFFFFF, np.uint32)
    np.testing.assert_allclose(oracle.vsa_unpack_project_fwd(ones, W, b)[0], W.sum(1) + b,
                               rtol=1e-5, atol=1e-5)
    # forward and backward are adjoint: <Y - b, dY> = <W, dW> for dW from the backward
    dY = rng.standard_normal((Bn, O)).astype(np.float32)
    dW, _ = oracle.vsa_unpack_project_bwd(dY, bits, D)
    Y0 = oracle.vsa_unpack_project_fwd(bits, W)
    np.testing.assert_allclose(np.sum(Y0.astype(np.float64) * dY), np.sum(W.astype(np.float64) * dW),
                               rtol=1e-5)


# ---------------------------------------------------------------------------- optimizers
def test_adamw_and_adam_golden_three_steps():
    """torch.optim.AdamW / Adam (float64) over three steps pin adamw-update.glsl's formula
    (and adam-update.glsl = weight_decay 0), including the bias corrections per step."""
    for tag in ["adamw", "adam"]:
        g = golden("optim_" + tag)
        W, m, v = g["W0"], np.zeros_like(g["W0"]), np.zeros_like(g["W0"])
        for k in range(3):
            W, gr, m, v = oracle.adamw_step(W, g["grads"][k], m, v, lr=float(g["lr"]),
                                            beta1=float(g["beta1"]), beta2=float(g["beta2"]),
                                            eps=float(g["eps"]),
                                            weight_decay=float(g["weight_decay"]), step=k + 1)
            assert rel_err(W, g["W"][k]) < TOL and rel_err(m, g["m"][k]) < TOL
            assert rel_err(v, g["v"][k]) < TOL
            assert not gr.any()  # clear_grad zeroes the gradient


def test_adamw_first_step_is_signed_lr():
    # at t = 1, m_hat = g and v_hat = g^2 exactly, so the step is lr * g / (|g| + eps)
    g = np.array([3.0, -0.5, 1e-3], np.float32)
    W, _, _, _ = oracle.adamw_step(np.zeros(3), g, np.zeros(3), np.zeros(3), lr=0.01, eps=0.0)
    assert np.allclose(W, -0.01 * np.sign(g), rtol=1e-6)


def test_surprise_momentum_known_answers():
    """Hand-computed cases of surprise-momentum.glsl:53-114 (eta 0.1, alpha 0.5, lambda 0,
    floor 0.01, clip 1): each exercises one branch."""
    W0 = np.array([1.0, 1.0, 1.0, 10.5, 2.0, -3.0], np.float32)
    g = np.array([0.2, 50.0, np.nan, 0.0, np.inf, 0.1], np.float32)
    s0 = np.array([0.4, 0.0, 0.7, 0.0, 0.2, np.inf], np.float32)
    W, gr, s, d = oracle.surprise_momentum_step(W0, g, s0, eta_base=0.1, alpha=0.5,
                                                weight_decay=0.1, clip_max=1.0)
    # [0] s = 0.5*0.2 + 0.5*0.4 = 0.3; lr = 0.1*1.3 = 0.13; d = 0.026 + 0.1*0.1*1 = 0.036
    # [1] s = min(25, 5) = 5; d = 0.6*50 + 0.01 -> clipped to 1; W = 0
    # [2] NaN gradient: W, s_bar unchanged, delta 0
    # [3] g = 0: s = 0 -> floor 0.01; d = 0.1*0.1*10.5 = 0.105; W = 10.395 -> clamped to 10
    # [4] Inf gradient: skipped like NaN
    # [5] s_bar Inf is read as 0: s = 0.05; d = 0.1*1.05*0.1 + 0.01*(-3) = -0.0195; W = -2.9805
    assert np.allclose(W, [0.964, 0.0, 1.0, 10.0, 2.0, -2.9805], rtol=1e-6, atol=1e-7)
    assert np.allclose(s, [0.3, 5.0, 0.7, 0.0, 0.2, 0.05], rtol=1e-6)
    assert np.allclose(d, [0.036, 1.0, 0.0, 0.105, 0.0, -0.0195], rtol=1e-6, atol=1e-7)
    assert not gr.any()


def test_surprise_momentum_recall_blend():
    # lambda and the recalled gradient enter twice: g_eff = g + lambda r, surprise |g - r|
    W, _, s, d = oracle.surprise_momentum_step(np.zeros(1), np.array([0.3]), np.zeros(1),
                                               recalled=np.array([0.1]), eta_base=1.0,
                                               alpha=1.0, lambda_recall=0.5, clip_max=10.0)
    # s = |0.3 - 0.1| = 0.2; lr = 1.2; d = 1.2 * (0.3 + 0.05) = 0.42
    assert np.allclose(s, [0.2]) and np.allclose(d, [0.42]) and np.allclose(W, [-0.42])


# ---------------------------------------------------------------------------- tape ops
def test_tape_ops_golden():
    g = golden("tapeops")
    for op in ["sub", "mul", "div", "neg"]:
        dA, dB = oracle.binary_bwd(op, g["dy"], g["a"], g["b"])
        assert rel_err(dA, g["d" + op + "_a"]) < TOL, op
        if dB is not None:
            assert rel_err(dB, g["d" + op + "_b"]) < TOL, op
    X = g["X"]
    for name, op in [("sum", "sum"), ("mean", "mean"), ("sumall", "sum"), ("meanall", "mean")]:
        assert rel_err(oracle.reduce_bwd(op, g[name + "_dy"], X.shape), g[name + "_dx"]) < TOL, name
    assert np.array_equal(oracle.transpose_bwd(g["tr_dy"]), g["tr_dx"])
    assert rel_err(oracle.mse_bwd(g["mse_p"], g["mse_t"]), g["mse_dp"]) < TOL
    # MatMul C = A B is Linear with W = B^T: dA = dC B^T, dB = (dC^T A)^T
    dA, dW, _ = oracle.linear_bwd(g["mm_dc"], g["mm_a"], np.ascontiguousarray(g["mm_b"].T),
                                  need_db=False)
    assert rel_err(dA, g["mm_da"]) < TOL and rel_err(dW.T, g["mm_db"]) < TOL


def test_lora_expand_golden():
    g = golden("lora_expand")
    dC, dB = oracle.lora_expand_bwd(g["dP"], g["basis"], g["coeffs"])
    assert rel_err(dC, g["dcoeffs"]) < TOL and rel_err(dB, g["dbasis"]) < TOL


def test_cosine_blend_golden_with_clamp():
    """torch's gradient of -cos(sum_k w_k preds_k, y), times the handler's 10, clamped to +-1
    (a quarter of the entries sit in the clamp)."""
    g = golden("cosine_blend")
    dP = oracle.cosine_blend_bwd(g["bits"], g["weights"], g["blended"], g["info"], K=4)
    assert rel_err(dP, g["dpreds"]) < TOL
    assert 0.1 < np.mean(np.abs(dP) == 1.0) < 0.5
    # without the scale/clamp (grad_scale 1, all |g| < 1) the gradient is torch's exactly
    assert rel_err(oracle.cosine_blend_bwd(g["bits"], g["weights"], g["blended"], g["info"], K=4,
                                           grad_scale=1.0), g["dpreds_raw"]) < TOL
