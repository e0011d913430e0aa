"""GPU parity of the VSA hypernetwork path (the reference's only real caller of the tape
backward): grilly_core.VSAHypernetwork / SurpriseMomentumOptimizer / vsa_training_step /
save|load_hypernetwork_weights under the reference's names (cpp/python/bindings.cpp:2883-3286),
and the forward kernels they run (VSA unpack-project forward, fp32 Linear on one row, GELU,
the fused surrogate-loss forward), each against the CPU oracle.

Tolerances: fp32 paths <= 1e-4 normwise relative error (max|gpu - ref| / max|ref|); the
branch selection and the optimizer update on the same gradient are checked exactly (to an
ulp of the weights)."""
import numpy as np
import pytest

import oracle
from conftest import rel_err

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

FP32_TOL = 1e-4


@pytest.fixture(scope="module")
def env(gpu):
    import grilly_core
    import grilly_bridge as gb
    import gn_bwd
    gn_bwd.lib()
    dev = grilly_core.Device(0)
    gb.attach_torch_stream(dev)
    return grilly_core, gb, gn_bwd, dev


def big_rel(a, b, chunk=1 << 24):
    """rel_err for arrays too large to widen at once (fp32 differences, fp64 maxima)."""
    a = a.reshape(-1)
    b = b.reshape(-1)
    num = den = 0.0
    for i in range(0, a.size, chunk):
        x, y = a[i:i + chunk], b[i:i + chunk]
        num = max(num, float(np.max(np.abs(x - y))))
        den = max(den, float(np.max(np.abs(y))))
    return num / max(den, 1e-30)


def bits_of(rng, rows, words):
    return rng.randint(0, 2 ** 32, size=(rows, words), dtype=np.uint32)


def dev_bits(b):
    return torch.from_numpy(b.view(np.int32)).cuda()


# ------------------------------------------------------------------------------- kernels
@pytest.mark.parametrize("Bn,O,D", [(1, 768, 10240), (3, 40, 256), (8, 96, 512), (13, 64, 1024),
                                    (64, 256, 2048), (256, 768, 10240)])
def test_vsa_unpack_project_fwd(env, Bn, O, D):
    gc, gb, gn, dev = env
    rng = np.random.RandomState(Bn + O)
    bits = bits_of(rng, Bn, D // 32)
    W = (rng.standard_normal((O, D)) / np.sqrt(D)).astype(np.float32)
    b = rng.standard_normal(O).astype(np.float32)
    Y = gn.vsa_unpack_project_fwd(dev_bits(bits), torch.from_numpy(W).cuda(), torch.from_numpy(b).cuda())
    ref = oracle.vsa_unpack_project_fwd(bits, W, b)
    assert rel_err(Y.cpu().numpy(), ref) < FP32_TOL, (Bn, O, D)


def test_vsa_unpack_project_fwd_integer_identity(env):
    # integer weights: every product and sum is exact in fp32 (and in the bf16 hi/lo split),
    # so the result equals the integer identity sum_j s_b(j) W[o, j] bit for bit
    gc, gb, gn, dev = env
    rng = np.random.RandomState(5)
    for Bn in (2, 128):
        O, D = 64, 1024
        bits = bits_of(rng, Bn, D // 32)
        Wi = rng.randint(-100, 100, size=(O, D)).astype(np.int64)
        S = np.unpackbits(bits.view(np.uint8), axis=1, bitorder="little").astype(np.int64) * 2 - 1
        Y = gn.vsa_unpack_project_fwd(dev_bits(bits), torch.from_numpy(Wi.astype(np.float32)).cuda())
        np.testing.assert_array_equal(Y.cpu().numpy(), (S @ Wi.T).astype(np.float32))


@pytest.mark.parametrize("Bn,K,D", [(1, 16, 10240), (5, 4, 1024), (64, 3, 256), (3, 33, 512),
                                    (2, 64, 1024)])
@pytest.mark.parametrize("noise", [True, False])
def test_vsa_surrogate_fwd(env, Bn, K, D, noise):
    gc, gb, gn, dev = env
    rng = np.random.RandomState(7 + K)
    bits = bits_of(rng, Bn, D // 32)
    preds = rng.standard_normal((Bn, K, D)).astype(np.float32) * 0.5
    seed, counter = 99, 4
    dots, res, w, loss = gn.vsa_surrogate_fwd(torch.from_numpy(preds).cuda(), dev_bits(bits),
                                              seed=seed, counter=counter, noise=noise)
    dots_g = dots.cpu().numpy()
    res_g = res.cpu().numpy().view(np.uint32)
    assert rel_err(dots_g, oracle.vsa_dots(preds, bits)) < FP32_TOL
    # selection and weights from the GPU's own dots: exactly the reference's host logic
    res_o, w_o = oracle.vsa_select(dots_g, 1.0, seed, counter, noise)
    np.testing.assert_array_equal(res_g, res_o)
    assert rel_err(w.cpu().numpy(), w_o) < 1e-5
    assert rel_err(loss.cpu().numpy(), oracle.vsa_surrogate_loss(preds, bits, res_o)) < FP32_TOL
    # the oracle's own end-to-end forward agrees unless two perturbed scores nearly tie
    d2, r2, w2, l2 = oracle.vsa_surrogate_fwd(preds, bits, seed=seed, counter=counter, noise=noise)
    assert np.array_equal(r2[:, :2], res_g[:, :2])
    assert rel_err(loss.cpu().numpy(), l2) < FP32_TOL


@pytest.mark.parametrize("M,N,K", [(1, 1536, 768), (2, 777, 1536), (5, 300, 64), (8, 640, 1024),
                                   (1, 10, 256), (4, 4096, 2048), (1, 999, 4096), (1, 5003, 1540)])
def test_linear_fp32_skinny(env, M, N, K):
    gc, gb, gn, dev = env
    rng = np.random.RandomState(M * 31 + N)
    X = rng.standard_normal((M, K)).astype(np.float32)
    W = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    dY = rng.standard_normal((M, N)).astype(np.float32)
    T = lambda a: torch.from_numpy(a).cuda()
    Y = gn.linear_fwd(T(X), T(W), T(b))
    assert rel_err(Y.cpu().numpy(), oracle.linear_fwd(X, W, b)) < FP32_TOL
    rX, rW, rb = oracle.linear_bwd(dY, X, W)
    dX, dW, db = gn.linear_bwd(T(dY), T(X), T(W))
    assert rel_err(dX.cpu().numpy(), rX) < FP32_TOL
    assert rel_err(dW.cpu().numpy(), rW) < FP32_TOL and rel_err(db.cpu().numpy(), rb) < FP32_TOL
    # deterministic with the workspace: a rerun is bit-identical
    dX2, dW2, db2 = gn.linear_bwd(T(dY), T(X), T(W))
    assert torch.equal(dX, dX2) and torch.equal(dW, dW2) and torch.equal(db, db2)
    # without a workspace the dX partials go through atomics: same values to rounding
    dX3, _, _ = gn.linear_bwd(T(dY), T(X), T(W), ws=False)
    assert rel_err(dX3.cpu().numpy(), rX) < FP32_TOL
    # accumulate adds onto what is there
    dXa, dWa, dba = gn.linear_bwd(T(dY), T(X), T(W), dX=dX.clone(), dW=dW.clone(), db=db.clone(),
                                  accumulate=True)
    assert rel_err(dXa.cpu().numpy(), 2 * rX) < FP32_TOL and rel_err(dWa.cpu().numpy(), 2 * rW) < FP32_TOL
    assert rel_err(dba.cpu().numpy(), 2 * rb) < FP32_TOL


@pytest.mark.parametrize("kind", ["relu", "gelu_tanh", "gelu_erf", "silu", "tanh", "sigmoid"])
def test_act_fwd(env, kind):
    gc, gb, gn, dev = env
    x = (np.random.RandomState(3).standard_normal(10007) * 3).astype(np.float32)
    y = gn.act_fwd(kind, torch.from_numpy(x).cuda())
    assert rel_err(y.cpu().numpy(), oracle.act_fwd(kind, x)) < 1e-5
    yb = gn.act_fwd(kind, torch.from_numpy(x).cuda().bfloat16())
    xb = torch.from_numpy(x).bfloat16().float().numpy()
    assert rel_err(yb.float().cpu().numpy(), oracle.act_fwd(kind, xb)) < 1e-2


# ------------------------------------------------------------- the model, reference names
def test_hypernetwork_surface(env):
    # tests/test_vsa_hypernetwork.py:41-65 (the reference test's id count says 6; the model
    # has ten parameters, bindings.cpp:2973-2984)
    gc, gb, gn, dev = env
    m = gc.VSAHypernetwork(dev, d_model=32, vsa_dim=256, K=2, seed=42)
    assert (m.d_model, m.vsa_dim, m.K, m.router_hidden) == (32, 256, 2, 32)
    ids = m.parameter_buffer_ids()
    assert len(ids) == 10 and len(set(ids)) == 10 and all(i != 0 for i in ids)
    assert m.parameter_sizes() == list(gc.hypernetwork_sizes((32, 256, 2, 32)))
    tape = gc.TapeContext(dev)
    state = np.random.RandomState(42).randint(0, 2 ** 32, size=8, dtype=np.uint32)
    out = m.forward_inference(dev, tape, state)
    assert out.shape == (2, 256) and np.all(np.isfinite(out))
    # same seed, same weights; another seed, other weights
    m2 = gc.VSAHypernetwork(dev, d_model=32, vsa_dim=256, K=2, seed=42)
    m3 = gc.VSAHypernetwork(dev, d_model=32, vsa_dim=256, K=2, seed=43)
    w = lambda mm: gb.download(dev, mm.parameter_buffer_ids()[2], (64, 32))
    assert np.array_equal(w(m), w(m2)) and not np.array_equal(w(m), w(m3))
    # the biases start at zero; W1 ~ N(0, sqrt(2 / (d + 2d)))
    assert np.all(gb.download(dev, ids[3], (64,)) == 0)
    big = gc.VSAHypernetwork(dev, d_model=256, vsa_dim=1024, K=2, seed=1)
    W1 = gb.download(dev, big.parameter_buffer_ids()[2], (512, 256))
    assert abs(W1.std() - np.sqrt(2 / 768)) < 0.02 * np.sqrt(2 / 768)
    with pytest.raises(ValueError):
        m.forward(tape, gb.make_tensor_ref(ids[0], (7,), gb.DTYPE_U32))


def test_training_step_small_loss_decreases(env):
    # tests/test_vsa_hypernetwork.py:79-126: a finite non-negative loss, and (xfail in the
    # reference, whose Linear/GELU handlers were scaffolds) a loss that goes down
    gc, gb, gn, dev = env
    m = gc.VSAHypernetwork(dev, d_model=32, vsa_dim=256, K=2, seed=42)
    tape = gc.TapeContext(dev)
    rng = np.random.RandomState(42)
    state = rng.randint(0, 2 ** 32, size=8, dtype=np.uint32)
    delta = state ^ rng.randint(0, 2 ** 32, size=8, dtype=np.uint32)
    loss0 = gc.vsa_training_step(dev, tape, m, state, delta)
    assert np.isfinite(loss0) and loss0 >= 0
    opt = gc.SurpriseMomentumOptimizer(dev, m, lr=0.01)
    losses = [gc.vsa_training_step(dev, tape, m, state, delta, opt) for _ in range(20)]
    assert np.mean(losses[-5:]) < np.mean(losses[:5]), losses
    assert opt.steps == 20 and m.gumbel_counter == 21


def _download_params(gb, dev, m):
    return [gb.download(dev, i, (n,)) for i, n in zip(m.parameter_buffer_ids(), m.parameter_sizes())]


def _oracle_step(W, bits_s, bits_d, d, v, K, seed, counter):
    """The hypernetwork step composed from oracle functions (vsa_hypernetwork.cpp:52-160 and
    the loss/backward of bindings.cpp:3140-3196); W = the ten parameters, flat."""
    h = 2 * d
    Wp, bp, W1, b1, W2, b2 = W[0].reshape(d, v), W[1], W[2].reshape(h, d), W[3], W[4].reshape(K * v, h), W[5]
    x = oracle.vsa_unpack_project_fwd(bits_s, Wp, bp)
    mid = oracle.linear_fwd(x, W1, b1)
    act = oracle.act_fwd("gelu_tanh", mid)
    pred = oracle.linear_fwd(act, W2, b2).reshape(1, K, v)
    dots, res, wts, loss = oracle.vsa_surrogate_fwd(pred, bits_d, seed=seed, counter=counter)
    dP = oracle.vsa_surrogate_bwd(pred, bits_d, res, wts)
    dA, dW2, db2 = oracle.linear_bwd(dP.reshape(1, K * v), act, W2)
    dM = oracle.act_bwd("gelu_tanh", dA, mid)
    dX, dW1, db1 = oracle.linear_bwd(dM, x, W1)
    dWp, dbp = oracle.vsa_unpack_project_bwd(dX, bits_s, v)
    return dict(pred=pred, dots=dots, results=res, loss=float(loss.mean()),
                grads=[dWp, dbp, dW1, db1, dW2, db2])


def test_training_step_reference_defaults_full_size(env):
    """One step at the reference's defaults (d_model 768, vsa_dim 10240, K 16, router 32; W2 is
    16 * 10240 * 1536 fp32 = 1.0 GB): the predictions, dots, branch selection, every gradient
    and the surprise-momentum update against the oracle; then vsa_training_step's loss for the
    next step against the oracle on the updated weights."""
    gc, gb, gn, dev = env
    d, v, K = 768, 10240, 16
    m = gc.VSAHypernetwork(dev)
    assert (m.d_model, m.vsa_dim, m.K, m.router_hidden) == (d, v, K, 32)
    opt = gc.SurpriseMomentumOptimizer(dev, m)
    tape = gc.TapeContext(dev)
    rng = np.random.RandomState(42)
    state = rng.randint(0, 2 ** 32, size=v // 32, dtype=np.uint32)
    delta = rng.randint(0, 2 ** 32, size=v // 32, dtype=np.uint32)
    W0 = _download_params(gb, dev, m)
    ref = _oracle_step(W0, state[None], delta[None], d, v, K, m.gumbel_seed, 0)

    tape.begin()
    s = gc.upload_bitpacked(tape, state)
    pred = m.forward(tape, s)
    assert pred.get_shape() == [1, K, v]
    dl = gc.upload_bitpacked(tape, delta)
    node = gc.record_surrogate_loss(tape, pred, dl)
    loss = gc.vsa_loss_forward(tape, node, m.gumbel_seed, 0)
    P = gb.download(dev, pred.buffer_id, (1, K, v))
    assert rel_err(P, ref["pred"]) < FP32_TOL
    res = gb.download(dev, node.get_saved_buffer(node.num_saved - 2), (1, 4), gb.DTYPE_I32).view(np.uint32)
    assert res[0, :2].tolist() == ref["results"][0, :2].tolist()
    assert abs(loss - ref["loss"]) <= FP32_TOL * abs(ref["loss"])
    tape.backward(node, 0)
    ids = m.parameter_buffer_ids()
    grads = []
    for i, (wid, n) in enumerate(zip(ids, m.parameter_sizes())):
        gid = tape.get_grad_buffer(wid)
        if i >= 6:
            assert gid == 0  # the router gets no gradient from this loss
            continue
        assert gid != 0
        grads.append(gb.download(dev, gid, (n,)))
    for i, (g, r) in enumerate(zip(grads, ref["grads"])):
        assert big_rel(g, r.reshape(-1)) < FP32_TOL, i
    # the optimizer on these gradients: W and s_bar as the oracle's update of the same inputs
    assert opt.apply(tape) == 6
    W1 = _download_params(gb, dev, m)
    sb = [gb.download(dev, i, (n,)) for i, n in zip(opt.s_bar_buffer_ids(), m.parameter_sizes())]
    tape.end()
    for i in range(6):
        Wr, _, sr, _ = oracle.surprise_momentum_step(W0[i], grads[i], np.zeros_like(W0[i]))
        assert np.max(np.abs(W1[i] - Wr)) <= 2 * np.spacing(np.max(np.abs(Wr))), i
        assert big_rel(sb[i], sr) < 1e-6, i
    for i in range(6, 10):
        np.testing.assert_array_equal(W1[i], W0[i])

    # the next step through vsa_training_step (Gumbel draw 1): its loss against the oracle
    m.gumbel_counter = 1
    loss2 = gc.vsa_training_step(dev, tape, m, state, delta, opt)
    ref2 = _oracle_step(W1, state[None], delta[None], d, v, K, m.gumbel_seed, 1)
    assert abs(loss2 - ref2["loss"]) <= FP32_TOL * abs(ref2["loss"])
    assert m.gumbel_counter == 2 and opt.steps == 2


# ------------------------------------------- Linear backward with the optimizer step fused in
@pytest.mark.parametrize("M,N,K", [(1, 4099, 1536), (1, 300, 4096), (3, 1000, 768), (8, 517, 2048)])
def test_linear_bwd_surprise_momentum_matches_two_calls(env, M, N, K):
    """gn_linear_bwd_surprise_momentum against gn_linear_bwd_ws followed by
    gn_surprise_momentum_step on the dW it stored: W, s_bar, dX and db bit for bit, with the
    step's branches exercised (weight decay on, a clip that binds, the +-10 weight bound,
    non-finite s_bar entries, and a column whose gradient is non-finite: an inf in X)."""
    gc, gb, gn, dev = env
    rng = np.random.RandomState(7 * M + K)
    dY = rng.standard_normal((M, N)).astype(np.float32)
    X = rng.standard_normal((M, K)).astype(np.float32)
    X[0, 3] = np.inf
    W = np.clip(rng.standard_normal((N, K)) * 3, -9.99, 9.99).astype(np.float32)
    W[1, :8] = 9.999
    sb = np.abs(rng.standard_normal((N, K))).astype(np.float32)
    sb[2, :4] = np.nan
    sb[3, 4:8] = np.inf
    hyper = dict(eta_base=0.05, alpha=0.7, lambda_recall=0.3, surprise_floor=0.02,
                 weight_decay=0.1, clip_max=0.05)
    t = lambda a: torch.from_numpy(a.copy()).cuda()
    Wa, sa = t(W), t(sb)
    dXa, dWa, dba = gn.linear_bwd(t(dY), t(X), Wa)
    gn.surprise_momentum_step([dict(W=Wa, grad=dWa, state0=sa)], clear_grad=False, **hyper)
    Wb, sbb = t(W), t(sb)
    dXb, dbb = gn.linear_bwd_surprise_momentum(t(dY), t(X), Wb, sbb, **hyper)
    torch.cuda.synchronize()
    for name, a, b in [("W", Wa, Wb), ("s_bar", sa, sbb), ("dX", dXa, dXb), ("db", dba, dbb)]:
        assert torch.equal(a.view(torch.int32), b.view(torch.int32)), name
    # the update did move W (the step is not skipped), and the clamps bound
    assert not torch.equal(Wb, t(W))
    assert float(Wb.abs().max()) <= 10.0


def test_linear_bwd_surprise_momentum_refuses_other_shapes(env):
    gc, gb, gn, dev = env
    dY = torch.zeros((9, 64), device="cuda")  # nine rows: not a skinny shape
    X = torch.zeros((9, 32), device="cuda")
    W = torch.zeros((64, 32), device="cuda")
    with pytest.raises(gn.GnError, match="M <= 8"):
        gn.linear_bwd_surprise_momentum(dY, X, W, torch.zeros_like(W))


@pytest.mark.parametrize("dims", [dict(d_model=64, vsa_dim=512, K=3, router_hidden=8), None])
def test_training_step_fused_update_bit_identical(env, dims):
    """vsa_training_step with the Linear weights stepped inside their backward passes (the
    default) against the separate optimizer pass (fuse_linear_updates = False): losses, all
    ten parameters and their s_bar bit for bit over three steps, at a small shape and at the
    reference's defaults (W2 16 x 10240 x 1536 fp32 = 1.0 GB).  The fused pass stores no
    gradient for the two Linear weights and steps exactly those."""
    gc, gb, gn, dev = env
    dims = dims or {}
    a = gc.VSAHypernetwork(dev, seed=11, **dims)
    b = gc.VSAHypernetwork(dev, seed=11, **dims)
    oa = gc.SurpriseMomentumOptimizer(dev, a, lr=0.01)
    ob = gc.SurpriseMomentumOptimizer(dev, b, lr=0.01)
    assert oa.fuse_linear_updates
    ob.fuse_linear_updates = False
    words = a.vsa_dim // 32
    rng = np.random.RandomState(3)
    tape = gc.TapeContext(dev)
    for step in range(3):
        state = rng.randint(0, 2 ** 32, size=words, dtype=np.uint32)
        delta = rng.randint(0, 2 ** 32, size=words, dtype=np.uint32)
        la = gc.vsa_training_step(dev, tape, a, state, delta, oa)
        lb = gc.vsa_training_step(dev, tape, b, state, delta, ob)
        assert la == lb, step
    for i, (x, y) in enumerate(zip(_download_params(gb, dev, a), _download_params(gb, dev, b))):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32)), i
    sizes = a.parameter_sizes()
    for i, (ia, ib) in enumerate(zip(oa.s_bar_buffer_ids(), ob.s_bar_buffer_ids())):
        x, y = gb.download(dev, ia, (sizes[i],)), gb.download(dev, ib, (sizes[i],))
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32)), i
    # which weights the fused pass steps: W1 and W2 (parameters 2 and 4), by their backward
    tape.begin()
    s = gc.upload_bitpacked(tape, state)
    pred = a.forward(tape, s)
    node = gc.record_surrogate_loss(tape, pred, gc.upload_bitpacked(tape, delta))
    gc.vsa_loss_forward(tape, node, a.gumbel_seed, a.gumbel_counter)
    oa.prepare(tape)
    tape.backward(node, 0)
    ids = a.parameter_buffer_ids()
    no_grad = [i for i in range(6) if tape.get_grad_buffer(ids[i]) == 0]
    assert no_grad == [2, 4], no_grad
    assert oa.apply(tape) == 6
    tape.end()


def test_checkpoint_under_reference_names(env, tmp_path):
    """grilly_core.save/load_hypernetwork_weights(model, path) (bindings.cpp:2965-3039): the
    file is the GRLY v3 layout the Python bridge reads too; with the optimizer, a resumed step
    is bit-identical to the uninterrupted one."""
    gc, gb, gn, dev = env
    dims = dict(d_model=64, vsa_dim=512, K=3, router_hidden=8)
    rng = np.random.RandomState(1)
    state = rng.randint(0, 2 ** 32, size=16, dtype=np.uint32)
    delta = rng.randint(0, 2 ** 32, size=16, dtype=np.uint32)
    tape = gc.TapeContext(dev)
    a = gc.VSAHypernetwork(dev, seed=5, **dims)
    oa = gc.SurpriseMomentumOptimizer(dev, a, lr=0.01)
    gc.vsa_training_step(dev, tape, a, state, delta, oa)
    p = str(tmp_path / "h.grly")
    gc.save_hypernetwork_weights(a, p, oa)
    host, info, _ = gc._grly_read(p, (64, 512, 3, 8), 1)
    for arr, w in zip(host, _download_params(gb, dev, a)):
        np.testing.assert_array_equal(arr, w)
    assert info["kind"] == 0 and info["step"] == 1
    b = gc.VSAHypernetwork(dev, seed=6, **dims)
    ob = gc.SurpriseMomentumOptimizer(dev, b, lr=0.5)
    gc.load_hypernetwork_weights(b, p, ob)
    assert ob.steps == 1 and abs(ob.eta_base - 0.01) < 1e-9
    b.gumbel_seed, b.gumbel_counter = a.gumbel_seed, a.gumbel_counter
    la = gc.vsa_training_step(dev, tape, a, state, delta, oa)
    lb = gc.vsa_training_step(dev, tape, b, state, delta, ob)
    assert la == lb
    for x, y in zip(_download_params(gb, dev, a), _download_params(gb, dev, b)):
        np.testing.assert_array_equal(x, y)
    # weights only, and a dimension mismatch is refused
    c = gc.VSAHypernetwork(dev, seed=7, **dims)
    gc.load_hypernetwork_weights(c, p)
    with pytest.raises(RuntimeError, match="dimension mismatch"):
        gc.load_hypernetwork_weights(gc.VSAHypernetwork(dev, d_model=32, vsa_dim=512, K=3,
                                                        router_hidden=8), p)
