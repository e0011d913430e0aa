"""GPU tests of the tape engine end to end: forward values are built with torch (plumbing),
the ops are recorded on grilly_core.TapeContext exactly as a reference model records them
(cpp/src/models/vsa_hypernetwork.cpp:52-160), backward runs through the C-ABI kernels, and
every gradient is compared with a composition of the CPU oracle.

Tolerances: fp32 paths 1e-4, bf16 paths 2e-2 (normwise relative error)."""
import numpy as np
import pytest

import oracle
from conftest import rel_err

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def env(gpu):
    import grilly_core
    import grilly_bridge as gb
    dev = grilly_core.Device(0)
    gb.attach_torch_stream(dev)
    return grilly_core, gb, dev


def test_tape_runs_on_torchs_stream(env):
    """attach_torch_stream puts the tape's launches on torch's current stream, the default
    (null, handle 0) stream included, so they are ordered with the torch work around them."""
    gc, gb, dev = env
    assert dev.stream_handle() == torch.cuda.current_stream().cuda_stream
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        gb.attach_torch_stream(dev)
        assert dev.stream_handle() == s.cuda_stream
    gb.attach_torch_stream(dev)
    assert dev.stream_handle() == torch.cuda.current_stream().cuda_stream


def T(x, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0").to(dtype).contiguous()


def grad(gb, dev, tape, t, dtype=None):
    gid = tape.get_grad_buffer(t.data_ptr())
    assert gid != 0, "no gradient recorded"
    return gb.download(dev, gid, t.shape, gb.dtype_code(t) if dtype is None else dtype)


def xavier(r, out, inp):
    lim = np.sqrt(6.0 / (inp + out))
    return r.uniform(-lim, lim, size=(out, inp)).astype(np.float32)


def test_mlp_c1_through_tape(env):
    """MLP 784->256->10, fp32, batch 64, ReLU, softmax CE."""
    gc, gb, dev = env
    r = np.random.default_rng(1)
    B = 64
    X = r.standard_normal((B, 784)).astype(np.float32)
    y = r.integers(0, 10, size=B).astype(np.int32)
    W1, W2 = xavier(r, 256, 784), xavier(r, 10, 256)
    b1, b2 = np.zeros(256, np.float32), np.zeros(10, np.float32)
    tX, tW1, tb1, tW2, tb2, ty = T(X), T(W1), T(b1), T(W2), T(b2), T(y, torch.int32)
    Z = (tX @ tW1.t() + tb1).contiguous()
    H = torch.relu(Z).contiguous()
    L = (H @ tW2.t() + tb2).contiguous()
    loss = torch.zeros(1, device="cuda:0")

    tape = gb.create_tape_context(dev)
    tape.begin()
    n1 = tape.record_op(gc.OpType.Linear, [gb.tref(tX)], [gb.tref(Z)])
    tape.save_for_backward(n1, [tW1.data_ptr(), tb1.data_ptr()])
    tape.record_op(gc.OpType.ReLU, [gb.tref(Z, True)], [gb.tref(H)])
    n3 = tape.record_op(gc.OpType.Linear, [gb.tref(H, True)], [gb.tref(L)])
    tape.save_for_backward(n3, [tW2.data_ptr(), tb2.data_ptr()])
    ce = tape.record_op(gc.OpType.CrossEntropy, [gb.tref(L, True), gb.tref(ty)], [gb.tref(loss)],
                        gb.cross_entropy_params(1.0))
    tape.backward(ce, 0)
    stats = tape.last_backward_stats()
    assert stats["nodes_visited"] == 4 and stats["nodes_with_grad"] == 4
    assert stats["cpu_fallbacks"] == 0

    hZ, hH, hL = Z.cpu().numpy(), H.cpu().numpy(), L.cpu().numpy()
    dL = oracle.xent_bwd(hL, y, 1.0)
    dH, dW2, db2 = oracle.linear_bwd(dL, hH, W2)
    dZ = oracle.act_bwd("relu", dH, hZ)
    _, dW1, db1 = oracle.linear_bwd(dZ, X, W1, need_dx=False)
    assert rel_err(grad(gb, dev, tape, L), dL) < 1e-4
    assert rel_err(grad(gb, dev, tape, H), dH) < 1e-4
    assert rel_err(grad(gb, dev, tape, Z), dZ) < 1e-4
    assert rel_err(grad(gb, dev, tape, tW2), dW2) < 1e-4
    assert rel_err(grad(gb, dev, tape, tb2), db2) < 1e-4
    assert rel_err(grad(gb, dev, tape, tW1), dW1) < 1e-4
    assert rel_err(grad(gb, dev, tape, tb1), db1) < 1e-4
    assert tape.get_grad_buffer(tX.data_ptr()) == 0  # input needs no grad (autograd.cpp:259)
    live = dev.pool_stats()["bytes_live"]
    tape.end()
    assert dev.pool_stats()["bytes_live"] < live
    assert not tape.is_recording()


@pytest.mark.parametrize("glu_epilogue", [False, True])
def test_ffn_block_bf16_through_tape(env, glu_epilogue):
    """configs[1] structure at a small size: RMSNorm -> FusedGLU(SwiGLU) -> Linear(down), with
    and without the GLU's local gradients in the down projection's epilogue (then the GLU
    output's gradient is not kept; everything upstream of it is unchanged)."""
    gc, gb, dev = env
    r = np.random.default_rng(2)
    M, Dm, Hd = 96, 256, 384
    bf = torch.bfloat16
    x = T(r.standard_normal((M, Dm)), bf)
    w = T(1 + 0.1 * r.standard_normal(Dm), bf)
    Wg, Wu = (T(r.standard_normal((Hd, Dm)) * 0.05, bf) for _ in range(2))
    Wd = T(r.standard_normal((Dm, Hd)) * 0.05, bf)
    dY = T(r.standard_normal((M, Dm)) * 0.01, bf)
    xf = x.float()
    rstd = torch.rsqrt((xf * xf).mean(-1) + 1e-6).contiguous()
    n = (xf * rstd[:, None] * w.float()).to(bf).contiguous()
    gate, up = (n @ Wg.t()).contiguous(), (n @ Wu.t()).contiguous()
    a = (gate.float() * torch.nn.functional.silu(up.float())).to(bf).contiguous()
    y = (a @ Wd.t()).contiguous()

    tape = gb.create_tape_context(dev)
    tape.set_glu_epilogue(glu_epilogue)
    tape.begin()
    nn_ = tape.record_op(gc.OpType.RMSNorm, [gb.tref(x, True)], [gb.tref(n)])
    tape.save_for_backward(nn_, [w.data_ptr(), rstd.data_ptr()])
    ng = tape.record_op(gc.OpType.FusedGLU, [gb.tref(n, True)], [gb.tref(a)],
                        gb.fused_glu_params("swiglu_up"))
    tape.save_for_backward(ng, [Wg.data_ptr(), Wu.data_ptr(), gate.data_ptr(), up.data_ptr()])
    nd = tape.record_op(gc.OpType.Linear, [gb.tref(a, True)], [gb.tref(y)])
    tape.save_for_backward(nd, [Wd.data_ptr(), 0])
    tape.backward(nd, dY.data_ptr())

    h = lambda t: t.float().cpu().numpy()
    dA, dWd, _ = oracle.linear_bwd(h(dY), h(a), h(Wd))
    dG, dU = oracle.glu_bwd("swiglu_up", dA, h(gate), h(up))
    dN = oracle.linear_bwd(dG, h(n), h(Wg))[0] + oracle.linear_bwd(dU, h(n), h(Wu))[0]
    dWg, dWu = oracle.linear_bwd(dG, h(n), h(Wg))[1], oracle.linear_bwd(dU, h(n), h(Wu))[1]
    dx, dw = oracle.rmsnorm_bwd(dN, h(x), h(w), h(rstd))
    if glu_epilogue:
        assert tape.get_grad_buffer(a.data_ptr()) == 0
        assert ng.grad_output_buffer == 0  # no upstream buffer: it started from [dGate | dUp]
    else:
        assert rel_err(grad(gb, dev, tape, a), dA) < 2e-2
    assert rel_err(grad(gb, dev, tape, Wd, gb.DTYPE_F32), dWd) < 2e-2
    assert rel_err(grad(gb, dev, tape, n), dN) < 2e-2
    assert rel_err(grad(gb, dev, tape, Wg, gb.DTYPE_F32), dWg) < 2e-2
    assert rel_err(grad(gb, dev, tape, Wu, gb.DTYPE_F32), dWu) < 2e-2
    assert rel_err(grad(gb, dev, tape, x), dx) < 2e-2
    assert rel_err(grad(gb, dev, tape, w, gb.DTYPE_F32), dw) < 2e-2
    tape.end()


def test_fanout_is_accumulated(env):
    """Residual z = Linear(x) + x and a weight used twice: both gradients are summed
    (the reference drops the second contribution, autograd.cpp:78-86)."""
    gc, gb, dev = env
    r = np.random.default_rng(3)
    x = T(r.standard_normal((16, 32)))
    W = T(r.standard_normal((32, 32)) * 0.1)
    y = (x @ W.t()).contiguous()
    z = (y + x).contiguous()
    u = (z @ W.t()).contiguous()  # W used a second time
    dU = T(r.standard_normal((16, 32)))
    tape = gb.create_tape_context(dev)
    tape.begin()
    n1 = tape.record_op(gc.OpType.Linear, [gb.tref(x, True)], [gb.tref(y)])
    tape.save_for_backward(n1, [W.data_ptr(), 0])
    tape.record_op(gc.OpType.Add, [gb.tref(y, True), gb.tref(x, True)], [gb.tref(z)])
    n3 = tape.record_op(gc.OpType.Linear, [gb.tref(z, True)], [gb.tref(u)])
    tape.save_for_backward(n3, [W.data_ptr(), 0])
    tape.backward(n3, dU.data_ptr())
    hW, hx, hz, hdU = W.cpu().numpy(), x.cpu().numpy(), z.cpu().numpy(), dU.cpu().numpy()
    dz = hdU @ hW
    dx = dz + dz @ hW
    dW = hdU.T @ hz + dz.T @ hx
    assert rel_err(grad(gb, dev, tape, x), dx) < 1e-4
    assert rel_err(grad(gb, dev, tape, W), dW) < 1e-4
    assert tape.last_backward_stats()["fanout_accumulations"] >= 2
    # the upstream buffer passed through Add must not have been modified
    assert torch.equal(dU.cpu(), torch.from_numpy(hdU))
    tape.end()


def test_same_buffer_contributions_are_summed(env):
    """Add(x, x) and x + Reshape(x): each input borrows the one upstream buffer, so the same
    buffer reaches x twice; both arrivals count (dx = 2 g), checked against float64."""
    gc, gb, dev = env
    r = np.random.default_rng(31)
    x = T(r.standard_normal((8, 16)))
    W = T(r.standard_normal((16, 16)) * 0.1)
    z = (x + x).contiguous()
    u = (z @ W.t()).contiguous()
    dU = T(r.standard_normal((8, 16)))
    tape = gb.create_tape_context(dev)
    tape.begin()
    tape.record_op(gc.OpType.Add, [gb.tref(x, True), gb.tref(x, True)], [gb.tref(z)])
    n = tape.record_op(gc.OpType.Linear, [gb.tref(z, True)], [gb.tref(u)])
    tape.save_for_backward(n, [W.data_ptr(), 0])
    tape.backward(n, dU.data_ptr())
    g = dU.double().cpu().numpy() @ W.double().cpu().numpy()
    assert rel_err(grad(gb, dev, tape, x), 2 * g) < 1e-6
    tape.end()

    # x + Reshape(x), the view in its own buffer: x gets g (through Add) + g (through Reshape)
    v = x.clone().reshape(16, 8).contiguous()  # separate buffer, same elements
    z2 = (x + v.reshape(8, 16)).contiguous()
    u2 = (z2 @ W.t()).contiguous()
    tape.begin()
    tape.record_op(gc.OpType.Reshape, [gb.tref(x, True)], [gb.tref(v, True)])
    vr = gb.make_tensor_ref(v.data_ptr(), (8, 16), gb.DTYPE_F32, True)
    tape.record_op(gc.OpType.Add, [gb.tref(x, True), vr], [gb.tref(z2)])
    n = tape.record_op(gc.OpType.Linear, [gb.tref(z2, True)], [gb.tref(u2)])
    tape.save_for_backward(n, [W.data_ptr(), 0])
    tape.backward(n, dU.data_ptr())
    assert rel_err(grad(gb, dev, tape, x), 2 * g) < 1e-6
    tape.end()

    # an in-place view (Reshape onto x's own buffer) is one tensor, not a fan-out: dx = g + g
    # only through the Add, the view adds nothing of its own
    tape.begin()
    xr = gb.make_tensor_ref(x.data_ptr(), (16, 8), gb.DTYPE_F32, True)
    tape.record_op(gc.OpType.Reshape, [gb.tref(x, True)], [xr])
    xv = gb.make_tensor_ref(x.data_ptr(), (8, 16), gb.DTYPE_F32, True)
    tape.record_op(gc.OpType.Add, [xv, xv], [gb.tref(z)])
    n = tape.record_op(gc.OpType.Linear, [gb.tref(z, True)], [gb.tref(u)])
    tape.save_for_backward(n, [W.data_ptr(), 0])
    tape.backward(n, dU.data_ptr())
    assert rel_err(grad(gb, dev, tape, x), 2 * g) < 1e-6
    tape.end()

    # in-place Add(x, x) written into x itself: both inputs are the input version of x, so its
    # gradient is 2 g as in the out-of-place form (the first input replaces the entry, the
    # second adds onto it)
    y = x.clone().contiguous()
    u3 = ((y + y) @ W.t()).contiguous()
    tape.begin()
    tape.record_op(gc.OpType.Add, [gb.tref(y, True), gb.tref(y, True)], [gb.tref(y)])
    n = tape.record_op(gc.OpType.Linear, [gb.tref(y, True)], [gb.tref(u3)])
    tape.save_for_backward(n, [W.data_ptr(), 0])
    tape.backward(n, dU.data_ptr())
    assert rel_err(grad(gb, dev, tape, y), 2 * g) < 1e-6
    tape.end()


def test_attention_and_layernorm_nodes(env):
    gc, gb, dev = env
    r = np.random.default_rng(4)
    B, H, S, D = 1, 2, 128, 64
    bf = torch.bfloat16
    Q, K, V = (T(r.standard_normal((B, H, S, D)), bf) for _ in range(3))
    dO = T(r.standard_normal((B, H, S, D)) * 0.01, bf)
    h = lambda t: t.float().cpu().numpy()
    O_, LSE_ = oracle.attn_fwd(h(Q), h(K), h(V))
    O, LSE = T(O_, bf), T(LSE_)
    tape = gb.create_tape_context(dev)
    tape.begin()
    na = tape.record_op(gc.OpType.FlashAttention2, [gb.tref(Q, True), gb.tref(K, True), gb.tref(V, True)],
                        [gb.tref(O)], gb.attention_params(causal=True, rope="interleaved"))
    tape.save_for_backward(na, [LSE.data_ptr()])
    tape.backward(na, dO.data_ptr())
    rQ, rK, rV = oracle.attn_bwd(h(Q), h(K), h(V), h(dO), LSE_)
    assert rel_err(grad(gb, dev, tape, Q), rQ) < 2e-2
    assert rel_err(grad(gb, dev, tape, K), rK) < 2e-2
    assert rel_err(grad(gb, dev, tape, V), rV) < 2e-2
    tape.end()

    rows, F = 64, 768
    X = T(r.standard_normal((rows, F)) * 2)
    gamma, beta = T(1 + 0.2 * r.standard_normal(F)), T(r.standard_normal(F))
    Y_, mean_, rstd_ = oracle.layernorm_fwd(h(X), h(gamma), h(beta))
    Y, mean, rstd = T(Y_), T(mean_), T(rstd_)
    dY = T(r.standard_normal((rows, F)))
    tape.begin()
    nl = tape.record_op(gc.OpType.LayerNorm, [gb.tref(X, True)], [gb.tref(Y)], gb.layernorm_params(1e-5))
    tape.save_for_backward(nl, [gamma.data_ptr(), beta.data_ptr(), mean.data_ptr(), rstd.data_ptr()])
    tape.backward(nl, dY.data_ptr())
    rX, rG, rB = oracle.layernorm_bwd(h(dY), h(X), h(gamma), mean_, rstd_)
    assert rel_err(grad(gb, dev, tape, X), rX) < 1e-4
    assert rel_err(grad(gb, dev, tape, gamma), rG) < 1e-4
    assert rel_err(grad(gb, dev, tape, beta), rB) < 1e-4
    tape.end()


def test_vsa_hypernetwork_chain(env):
    """The reference's only taped model (vsa_hypernetwork.cpp:52-160, vsa_training_step
    bindings.cpp:3140-3286): VSAUnpackProject -> Linear -> GELU -> Linear -> VSASurrogateLoss,
    here with a batch of 8 and seeded winner selection."""
    gc, gb, dev = env
    r = np.random.default_rng(5)
    Bn, D, d_model, hidden, K = 8, 1024, 64, 128, 4
    words = D // 32
    bits = r.integers(0, 2**32, size=(Bn, words), dtype=np.uint64).astype(np.uint32)
    target = r.integers(0, 2**32, size=(Bn, words), dtype=np.uint64).astype(np.uint32)
    Wp = (r.standard_normal((d_model, D)) / np.sqrt(D)).astype(np.float32)
    bp = np.zeros(d_model, np.float32)
    W1 = (r.standard_normal((hidden, d_model)) * np.sqrt(2 / (d_model + hidden))).astype(np.float32)
    b1 = np.zeros(hidden, np.float32)
    W2 = (r.standard_normal((K * D, hidden)) * np.sqrt(2 / (hidden + K * D))).astype(np.float32)
    b2 = np.zeros(K * D, np.float32)
    S = oracle.unpack_bits(bits, D)
    h0 = S @ Wp.T + bp
    z1 = h0 @ W1.T + b1
    a1 = oracle.act_fwd("gelu_tanh", z1)
    preds = (a1 @ W2.T + b2).astype(np.float32)
    res, wts = oracle.vsa_results_weights(oracle.vsa_dots(preds.reshape(Bn, K, D), target),
                                          rng=np.random.default_rng(6))
    tb = {k: T(v) for k, v in dict(Wp=Wp, bp=bp, W1=W1, b1=b1, W2=W2, b2=b2, h0=h0, z1=z1,
                                   a1=a1, preds=preds).items()}
    tbits = torch.from_numpy(bits.view(np.int32)).cuda()
    ttarget = torch.from_numpy(target.view(np.int32)).cuda()
    tres = torch.from_numpy(res.view(np.int32)).cuda()
    twts = T(wts)
    loss = torch.zeros(1, device="cuda:0")

    tape = gb.create_tape_context(dev)
    tape.begin()
    bits_ref = gb.make_tensor_ref(tbits.data_ptr(), (Bn, words), gb.DTYPE_U32)
    n0 = tape.record_op(gc.OpType.VSAUnpackProject, [bits_ref], [gb.tref(tb["h0"])])
    tape.save_for_backward(n0, [tb["Wp"].data_ptr(), tb["bp"].data_ptr()])
    n1 = tape.record_op(gc.OpType.Linear, [gb.tref(tb["h0"], True)], [gb.tref(tb["z1"])])
    tape.save_for_backward(n1, [tb["W1"].data_ptr(), tb["b1"].data_ptr()])
    tape.record_op(gc.OpType.GELU, [gb.tref(tb["z1"], True)], [gb.tref(tb["a1"])])
    n3 = tape.record_op(gc.OpType.Linear, [gb.tref(tb["a1"], True)], [gb.tref(tb["preds"])])
    tape.save_for_backward(n3, [tb["W2"].data_ptr(), tb["b2"].data_ptr()])
    preds_ref = gb.make_tensor_ref(tb["preds"].data_ptr(), (Bn, K, D), gb.DTYPE_F32, True)
    tgt_ref = gb.make_tensor_ref(ttarget.data_ptr(), (Bn, words), gb.DTYPE_U32)
    nl = tape.record_op(gc.OpType.VSASurrogateLoss, [preds_ref, tgt_ref], [gb.tref(loss)],
                        gb.vsa_surrogate_params(K, D))
    tape.save_for_backward(nl, [tres.data_ptr(), twts.data_ptr()])
    tape.backward(nl, 0)
    assert tape.last_backward_stats()["cpu_fallbacks"] == 0

    dP = oracle.vsa_surrogate_bwd(preds.reshape(Bn, K, D), target, res, wts).reshape(Bn, K * D)
    da1, dW2, db2 = oracle.linear_bwd(dP, a1, W2)
    dz1 = oracle.act_bwd("gelu_tanh", da1, z1)
    dh0, dW1, db1 = oracle.linear_bwd(dz1, h0, W1)
    dWp, dbp = oracle.vsa_unpack_project_bwd(dh0, bits, D)
    assert rel_err(grad(gb, dev, tape, tb["preds"]), dP) < 1e-5
    assert rel_err(grad(gb, dev, tape, tb["W2"]), dW2) < 1e-4
    assert rel_err(grad(gb, dev, tape, tb["b2"]), db2) < 1e-4
    assert rel_err(grad(gb, dev, tape, tb["W1"]), dW1) < 1e-4
    assert rel_err(grad(gb, dev, tape, tb["b1"]), db1) < 1e-4
    assert rel_err(grad(gb, dev, tape, tb["Wp"]), dWp) < 1e-4
    assert rel_err(grad(gb, dev, tape, tb["bp"]), dbp) < 1e-4
    tape.end()


def test_tape_error_paths(env):
    gc, gb, dev = env
    x = torch.zeros((4, 8), device="cuda:0")
    W = torch.zeros((8, 8), device="cuda:0")
    tape = gb.create_tape_context(dev, arena_capacity=1 << 20)
    assert tape.record_op(gc.OpType.Linear, [gb.tref(x)], [gb.tref(x)]) is None  # not recording
    tape.begin()
    n = tape.record_op(gc.OpType.Linear, [gb.tref(x, True)], [gb.tref(x)])
    tape.save_for_backward(n, [W.data_ptr()])
    with pytest.raises(ValueError, match="upstream gradient"):
        tape.backward(n, 0)  # a Linear root needs dL/dy
    tape.end()
    tape.begin()
    m = tape.record_op(gc.OpType.Conv2d, [gb.tref(x, True)], [gb.tref(x)])
    tape.backward(m, x.data_ptr())
    assert tape.last_backward_stats()["cpu_fallbacks"] == 1  # no handler (autograd.cpp:126-128)
    tape.end()
    small = gb.create_tape_context(dev, arena_capacity=4096)
    small.begin()
    with pytest.raises(MemoryError):
        for _ in range(10):
            small.record_op(gc.OpType.ReLU, [gb.tref(x, True)], [gb.tref(x)])
    small.end()


def _decoder_reference(m):
    """fp32 torch autograd of the same decoder, rounding to bf16 where the GPU run stores
    (straight-through), so both differentiate the same bf16-stored forward; the residual
    stream is fp32 on both sides."""
    import math
    rb = lambda t: t + (t.bfloat16().float() - t).detach()
    leaf = lambda t: t.detach().float().clone().requires_grad_(True)
    B, S, H, d, T = m.B, m.S, m.H, m.d, m.T
    D = d // H
    E = leaf(m.E)
    params = [{k: leaf(v) for k, v in p.items()} for p in m.layers]
    lnf_g, lnf_b = leaf(m.lnf_g), leaf(m.lnf_b)

    def ln(x, g, b):
        mu = x.mean(-1, keepdim=True)
        var = ((x - mu) ** 2).mean(-1, keepdim=True)
        return rb((x - mu) * torch.rsqrt(var + 1e-5) * g + b)

    def gelu(u):
        return 0.5 * u * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (u + 0.044715 * u ** 3)))

    mask = torch.triu(torch.ones(S, S, dtype=torch.bool, device=E.device), 1)
    x = E[m.ids.long()]  # bf16 values, carried in fp32
    for p in params:
        n1 = ln(x, p["ln1_g"], p["ln1_b"])
        qkv = rb(n1 @ p["Wqkv"].t() + p["bqkv"])
        q, k, v = qkv.view(B, S, 3, H, D).permute(2, 0, 3, 1, 4)
        sc = torch.matmul(q, k.transpose(-1, -2).contiguous()) / math.sqrt(D)
        o = torch.matmul(torch.softmax(sc.masked_fill(mask, float("-inf")), -1), v)
        o = rb(o.permute(0, 2, 1, 3).reshape(T, d))
        x2 = x + rb(o @ p["Wo"].t() + p["bo"])
        n2 = ln(x2, p["ln2_g"], p["ln2_b"])
        gate = rb(n2 @ p["Wg"].t() + p["bg"])
        up = rb(n2 @ p["Wu"].t() + p["bu"])
        h = rb(gate * gelu(up))
        x = x2 + rb(h @ p["Wd"].t() + p["bd"])
    logits = rb(ln(x, lnf_g, lnf_b) @ E.t())
    torch.nn.functional.cross_entropy(logits, m.tgt.long()).backward()
    return E, params, lnf_g, lnf_b


@pytest.mark.parametrize("glu_epilogue", [False, True])
def test_decoder_stack_through_tape(env, glu_epilogue):
    """BASELINE configs[4] at a small size: embedding, LN, fused QKV + causal attention on
    the fused layout, residual adds, GEGLU, tied LM head and CE, all through the tape; with
    the GLU's local gradients formed by the down projection's epilogue (set_glu_epilogue) the
    GLU output's own gradient is not kept, and without it it is."""
    gc, gb, dev = env
    import decoder_tape
    m = decoder_tape.Decoder(layers=2, d=128, heads=2, ff=256, vocab=300, batch=2, seq=128, seed=7)
    g = torch.Generator(device="cuda:0")
    g.manual_seed(11)
    for p in m.layers:  # non-trivial norm parameters and biases, so their gradients matter
        for k in ("ln1_g", "ln2_g"):
            p[k].copy_((1 + 0.2 * torch.randn(p[k].shape, device="cuda:0", generator=g)).bfloat16())
        for k in ("ln1_b", "ln2_b", "bqkv", "bo", "bg", "bu", "bd"):
            p[k].copy_((0.05 * torch.randn(p[k].shape, device="cuda:0", generator=g)).bfloat16())
    m.forward()
    tape = gb.create_tape_context(dev)
    tape.set_glu_epilogue(glu_epilogue)
    assert tape.glu_epilogue() == glu_epilogue
    tape.begin()
    loss = m.record(tape)
    tape.backward(loss, 0)
    got = {"E": grad(gb, dev, tape, m.E, gb.DTYPE_F32)}
    for i, p in enumerate(m.layers):
        for k in ("Wqkv", "bqkv", "Wo", "ln1_g", "ln2_b", "Wg", "Wu", "bu", "Wd"):
            got[f"{k}{i}"] = grad(gb, dev, tape, p[k], gb.DTYPE_F32)
        kept = tape.get_grad_buffer(m.acts[i]["h"].data_ptr())
        assert (kept == 0) == glu_epilogue, (i, kept)
    got["lnf_g"] = grad(gb, dev, tape, m.lnf_g, gb.DTYPE_F32)
    tape.end()
    E, params, lnf_g, _ = _decoder_reference(m)
    want = {"E": E.grad, "lnf_g": lnf_g.grad}
    for i, p in enumerate(params):
        for k in ("Wqkv", "bqkv", "Wo", "ln1_g", "ln2_b", "Wg", "Wu", "bu", "Wd"):
            want[f"{k}{i}"] = p[k].grad
    errs = {k: rel_err(got[k], want[k].cpu().numpy()) for k in got}
    bad = {k: v for k, v in errs.items() if not v < 2e-2}
    assert not bad, f"relative errors above 2e-2: {bad} (all: {errs})"


def test_decoder_full_size_through_tape(env):
    """BASELINE configs[4] at its full size (12 layers, d 768, 12 heads, GEGLU 3072, tied
    embedding 32000, B 8 x S 1024): every weight gradient of the first, a middle and the last
    layer, the embedding and the final norm, against fp32 torch autograd of the same
    bf16-stored forward (normwise relative error <= 2e-2 for every tensor).

    The second LayerNorm's gain gradient dgamma = sum_rows dy * xhat cancels heavily (its
    largest entry is ~5 % of sum_rows |dy * xhat| at this size); with the residual stream and
    its gradient in fp32 the error that reaches it stays within the bf16 bound.  The kernel
    itself is also pinned on its own input: dgamma against the oracle's LayerNorm backward fed
    the GPU's own upstream dy (<= 1e-4).  The tape runs as the bench runs it, with the GLU's
    local gradients formed in the down projection's epilogue."""
    gc, gb, dev = env
    import decoder_tape
    m = decoder_tape.Decoder(seed=9)
    g = torch.Generator(device="cuda:0")
    g.manual_seed(13)
    for p in m.layers:
        for k in ("ln1_g", "ln2_g"):
            p[k].copy_((1 + 0.2 * torch.randn(p[k].shape, device="cuda:0", generator=g)).bfloat16())
        for k in ("ln1_b", "ln2_b", "bqkv", "bo", "bg", "bu", "bd"):
            p[k].copy_((0.05 * torch.randn(p[k].shape, device="cuda:0", generator=g)).bfloat16())
    m.forward()
    tape = gb.create_tape_context(dev)
    tape.set_glu_epilogue(m.glu_epilogue)
    tape.begin()
    loss = m.record(tape)
    tape.backward(loss, 0)
    keys = ("Wqkv", "bqkv", "Wo", "bo", "ln1_g", "ln1_b", "ln2_g", "Wg", "Wu", "bg", "Wd", "bd")
    layers = (0, m.L // 2, m.L - 1)
    got = {"E": grad(gb, dev, tape, m.E, gb.DTYPE_F32),
           "lnf_g": grad(gb, dev, tape, m.lnf_g, gb.DTYPE_F32)}
    dn2 = {}
    for i in layers:
        for k in keys:
            got[f"{k}{i}"] = grad(gb, dev, tape, m.layers[i][k], gb.DTYPE_F32)
        dn2[i] = grad(gb, dev, tape, m.acts[i]["n2"])  # the LayerNorm's upstream dy (bf16)
    tape.end()
    for i in layers:  # the LayerNorm backward kernel on its own input: fp32-exact
        a, p = m.acts[i], m.layers[i]
        _, rg, _ = oracle.layernorm_bwd(dn2[i], a["x2"].float().cpu().numpy(),
                                        p["ln2_g"].float().cpu().numpy(),
                                        a["m2"].float().cpu().numpy(), a["r2"].float().cpu().numpy())
        assert rel_err(got[f"ln2_g{i}"], rg) < 1e-4, i
    E, params, lnf_g, _ = _decoder_reference(m)
    want = {"E": E.grad, "lnf_g": lnf_g.grad}
    for i in layers:
        for k in keys:
            want[f"{k}{i}"] = params[i][k].grad
    errs = {k: rel_err(got[k], want[k].cpu().numpy()) for k in got}
    del E, params, lnf_g, want
    torch.cuda.empty_cache()
    bad = {k: v for k, v in errs.items() if not v < 2e-2}
    assert not bad, f"relative errors above the bound: {bad} (all: {errs})"


def test_training_step_with_optimizers(env):
    """BASELINE configs[0] MLP, full training step as vsa_training_step orders it
    (bindings.cpp:3196-3279): backward, optimizer over the tape's gradients, end; then a
    second step on the updated weights.  Weights after each step against oracle grads +
    oracle optimizer; bf16 weights keep an fp32 master and receive the rounded update."""
    gc, gb, dev = env
    r = np.random.default_rng(7)
    B = 64
    X = r.standard_normal((B, 784)).astype(np.float32)
    y = r.integers(0, 10, size=B).astype(np.int32)
    W1, W2 = xavier(r, 256, 784), xavier(r, 10, 256)
    b1, b2 = np.zeros(256, np.float32), np.zeros(10, np.float32)
    tX, ty = T(X), T(y, torch.int32)
    params = [T(W1), T(b1), T(W2), T(b2)]
    for opt_kind in ["adamw", "surprise"]:
        ws = [p.clone() for p in params]
        hw = [p.cpu().numpy() for p in ws]
        if opt_kind == "adamw":
            opt = gb.AdamW(ws, lr=1e-2, weight_decay=0.01)
            st = [[np.zeros_like(h), np.zeros_like(h)] for h in hw]
        else:
            opt = gb.SurpriseMomentumOptimizer(ws, lr=1e-2, alpha=0.9, clip=1.0)
            st = [np.zeros_like(h) for h in hw]
        for step in range(1, 3):
            tW1, tb1, tW2, tb2 = ws
            Z = (tX @ tW1.t() + tb1).contiguous()
            H = torch.relu(Z).contiguous()
            L = (H @ tW2.t() + tb2).contiguous()
            loss = torch.zeros(1, device="cuda:0")
            tape = gb.create_tape_context(dev)
            tape.begin()
            n1 = tape.record_op(gc.OpType.Linear, [gb.tref(tX)], [gb.tref(Z)])
            tape.save_for_backward(n1, [tW1.data_ptr(), tb1.data_ptr()])
            tape.record_op(gc.OpType.ReLU, [gb.tref(Z, True)], [gb.tref(H)])
            n3 = tape.record_op(gc.OpType.Linear, [gb.tref(H, True)], [gb.tref(L)])
            tape.save_for_backward(n3, [tW2.data_ptr(), tb2.data_ptr()])
            ce = tape.record_op(gc.OpType.CrossEntropy, [gb.tref(L, True), gb.tref(ty)],
                                [gb.tref(loss)], gb.cross_entropy_params(1.0 / B))
            tape.backward(ce, 0)
            assert opt.step(tape) == 4
            tape.end()
            torch.cuda.synchronize()
            # oracle: gradients from the same weights, then the same update
            hZ, hH, hL = Z.cpu().numpy(), H.cpu().numpy(), L.cpu().numpy()
            dL = oracle.xent_bwd(hL, y, 1.0 / B)
            _, dW2, db2 = oracle.linear_bwd(dL, hH, hw[2])
            dZ = oracle.act_bwd("relu", oracle.linear_bwd(dL, hH, hw[2])[0], hZ)
            _, dW1, db1 = oracle.linear_bwd(dZ, X, hw[0], need_dx=False)
            for i, g in enumerate([dW1, db1, dW2, db2]):
                if opt_kind == "adamw":
                    hw[i], _, st[i][0], st[i][1] = oracle.adamw_step(
                        hw[i], g, st[i][0], st[i][1], lr=1e-2, weight_decay=0.01, step=step)
                else:
                    hw[i], _, st[i], _ = oracle.surprise_momentum_step(
                        hw[i], g, st[i], eta_base=1e-2, alpha=0.9, clip_max=1.0)
                assert rel_err(ws[i].cpu().numpy(), hw[i]) < 1e-4, (opt_kind, step, i)


def test_remaining_ops_through_tape(env):
    """Sub, Mul, Div, Neg, Transpose, MatMul, Sum/Mean and MSELoss recorded on the tape (the
    reference's stubs, autograd.cpp:543-711) against torch float64 autograd of the same graph:
        d = (x - y) * z / w;  e = -d^T;  f = e @ M;  s = mean(f, -1);  L = mse(s, target)."""
    gc, gb, dev = env
    r = np.random.default_rng(9)
    shp = (6, 10)
    x, y, z = (r.standard_normal(shp).astype(np.float32) for _ in range(3))
    w = (r.standard_normal(shp) + 2.0).astype(np.float32)
    Mm = r.standard_normal((6, 5)).astype(np.float32)
    tgt = r.standard_normal(10).astype(np.float32)
    tx, ty, tz, tw, tM, tt = T(x), T(y), T(z), T(w), T(Mm), T(tgt)
    d1 = (tx - ty).contiguous()
    d2 = (d1 * tz).contiguous()
    d = (d2 / tw).contiguous()
    e0 = d.t().contiguous()
    e = (-e0).contiguous()
    f = (e @ tM).contiguous()
    s = f.mean(-1).contiguous()
    loss = torch.zeros(1, device="cuda:0")
    tape = gb.create_tape_context(dev)
    tape.begin()
    op = gc.OpType
    tape.record_op(op.Sub, [gb.tref(tx, True), gb.tref(ty, True)], [gb.tref(d1)])
    tape.record_op(op.Mul, [gb.tref(d1, True), gb.tref(tz, True)], [gb.tref(d2)])
    tape.record_op(op.Div, [gb.tref(d2, True), gb.tref(tw, True)], [gb.tref(d)])
    tape.record_op(op.Transpose, [gb.tref(d, True)], [gb.tref(e0)])
    tape.record_op(op.Neg, [gb.tref(e0, True)], [gb.tref(e)])
    tape.record_op(op.MatMul, [gb.tref(e, True), gb.tref(tM, True)], [gb.tref(f)])
    tape.record_op(op.Mean, [gb.tref(f, True)], [gb.tref(s)])
    ln = tape.record_op(op.MSELoss, [gb.tref(s, True), gb.tref(tt)], [gb.tref(loss)])
    tape.backward(ln, 0)
    st = tape.last_backward_stats()
    assert st["cpu_fallbacks"] == 0 and st["nodes_with_grad"] == 8

    X = [torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (x, y, z, w, Mm)]
    dd = (X[0] - X[1]) * X[2] / X[3]
    ff = (-dd.t()) @ X[4]
    lref = ((ff.mean(-1) - torch.tensor(tgt, dtype=torch.float64)) ** 2).mean()
    lref.backward()
    for t_, ref in zip([tx, ty, tz, tw, tM], X):
        assert rel_err(grad(gb, dev, tape, t_), ref.grad.numpy()) < 1e-5
    tape.end()


# ---------------------------------------------------------------- GRLY v3 checkpoint
HYPER_DIMS = (64, 256, 4, 32)  # d_model, vsa_dim, K, router_hidden


def test_hypernetwork_checkpoint_device_round_trip(env, tmp_path):
    """save/load_hypernetwork_weights (bindings.cpp:2965-3039) from and into device tensors:
    the file holds the exact fp32 values (bf16 widened), and an fp32 file loaded into bf16
    tensors rounds to nearest-even like torch's conversion, ties and infinities included."""
    gc, gb, dev = env
    sizes = gc.hypernetwork_sizes(HYPER_DIMS)
    g = torch.Generator(device="cuda:0")
    g.manual_seed(3)
    for dt in (torch.float32, torch.bfloat16):
        src = gb.HypernetworkWeights(*HYPER_DIMS, tensors=[
            torch.randn(n, device="cuda:0", generator=g).to(dt) for n in sizes])
        p = tmp_path / f"w_{str(dt)[6:]}.grly"
        gb.save_hypernetwork_weights(src, p)
        host, _, _ = gc._grly_read(str(p), HYPER_DIMS)
        for a, t in zip(host, src.weight_buffers()):
            np.testing.assert_array_equal(a, t.float().cpu().numpy())
        dst = gb.HypernetworkWeights(*HYPER_DIMS, dtype=dt)
        gb.load_hypernetwork_weights(dst, p)
        for a, b in zip(dst.weight_buffers(), src.weight_buffers()):
            assert torch.equal(a, b)
    w32 = [torch.randn(n, device="cuda:0", generator=g) for n in sizes]
    ties = torch.tensor([1 + 2 ** -8, 1 + 3 * 2 ** -8, -(1 + 2 ** -8), 2 ** -130, float("inf"),
                         -float("inf"), 3.0e38, 1e-45], device="cuda:0")
    w32[3][:ties.numel()] = ties
    src = gb.HypernetworkWeights(*HYPER_DIMS, tensors=w32)
    p = tmp_path / "w32.grly"
    gb.save_hypernetwork_weights(src, p)
    dst = gb.HypernetworkWeights(*HYPER_DIMS, dtype=torch.bfloat16)
    gb.load_hypernetwork_weights(dst, p)
    for a, b in zip(dst.weight_buffers(), w32):
        assert torch.equal(a, b.bfloat16())
    with pytest.raises(RuntimeError, match="Model dimension mismatch"):
        gb.load_hypernetwork_weights(gb.HypernetworkWeights(64, 256, 2, 32), p)


class _GradTape:
    """Stands in for a TapeContext after backward: weight id -> gradient buffer id."""

    def __init__(self, weights, grads):
        self.g = {w.data_ptr(): gr for w, gr in zip(weights, grads)}

    def get_grad_buffer(self, wid):
        return self.g[wid].data_ptr()


@pytest.mark.parametrize("opt_kind", ["adamw", "surprise"])
def test_hypernetwork_checkpoint_resumes_training(env, tmp_path, opt_kind):
    """Checkpoint after one optimizer step, reload into a fresh model and optimizer, take the
    next step on both: weights (bf16 copies and fp32 masters) and state agree bit for bit."""
    gc, gb, dev = env
    sizes = gc.hypernetwork_sizes(HYPER_DIMS)
    g = torch.Generator(device="cuda:0")
    g.manual_seed(9)
    A = gb.HypernetworkWeights(*HYPER_DIMS, tensors=[
        (0.1 * torch.randn(n, device="cuda:0", generator=g)).bfloat16() for n in sizes])
    G1, G2 = ([1e-2 * torch.randn(n, device="cuda:0", generator=g) for n in sizes] for _ in range(2))

    def make(model, lr):
        if opt_kind == "adamw":
            return gb.AdamW(model.weight_buffers(), lr=lr, weight_decay=0.01)
        return gb.SurpriseMomentumOptimizer(model.weight_buffers(), lr=lr, alpha=0.9, clip=1.0)

    def state(o):
        return (o.m + o.v) if opt_kind == "adamw" else o.s_bar

    oa = make(A, 1e-2)
    oa.step(_GradTape(A.weight_buffers(), [x.clone() for x in G1]))
    p = tmp_path / "ckpt.grly"
    gb.save_hypernetwork_weights(A, p, optimizer=oa)
    oa.step(_GradTape(A.weight_buffers(), [x.clone() for x in G2]))
    B = gb.HypernetworkWeights(*HYPER_DIMS, dtype=torch.bfloat16)
    ob = make(B, 5e-4)  # hyper-parameters and step come from the file
    gb.load_hypernetwork_weights(B, p, optimizer=ob)
    assert ob.t == 1
    ob.step(_GradTape(B.weight_buffers(), [x.clone() for x in G2]))
    for a, b in zip(A.weight_buffers() + oa.masters + state(oa),
                    B.weight_buffers() + ob.masters + state(ob)):
        assert torch.equal(a, b)
    # a checkpoint without an optimizer section cannot restore one
    q = tmp_path / "plain.grly"
    gb.save_hypernetwork_weights(A, q)
    with pytest.raises(ValueError, match="no"):
        gb.load_hypernetwork_weights(B, q, optimizer=ob)
