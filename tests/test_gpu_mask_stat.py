"""GPU parity of the attention key-padding mask (flash-attention2.glsl:150-154,
flash-attention2-rope.glsl:201-205) and of the RMSNorm saved-statistic forms (rms-norm.glsl:52
mean(x^2), snn-rmsnorm.glsl:55 sqrt(mean(x^2) + eps)), through the C ABI and the tape.

Tolerances (normwise relative error): fp32 <= 1e-4, bf16 <= 2e-2 against the fp32 oracle on
the same bf16-rounded inputs; golden vectors are torch float64 autograd of the forwards."""
import numpy as np
import pytest

import oracle
from conftest import golden, rel_err

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

FP32_TOL = 1e-4
BF16_TOL = 2e-2


@pytest.fixture(scope="module")
def gn(gpu):
    import gn_bwd
    gn_bwd.lib()
    return gn_bwd


def dev(x, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0").to(dtype)


def host(t):
    return t.float().cpu().numpy()


def rnd(x):
    return host(dev(x, torch.bfloat16))


def padded_mask(B, S, lens, holes=()):
    """1 for kept keys: batch b keeps keys < lens[b], minus the (b, k) pairs in `holes`."""
    m = np.zeros((B, S), np.float32)
    for b, n in enumerate(lens):
        m[b, :n] = 1.0
    for b, k in holes:
        m[b, k] = 0.0
    return m


# ---------------------------------------------------------------------------- key mask
@pytest.mark.parametrize("tag", ["mask_causal_rope", "mask_full"])
def test_attention_mask_golden_fp32(gn, tag):
    g = golden(f"attn_{tag}")
    kw = dict(scale=float(g["scale"]), causal=bool(g["causal"]), rope=str(g["rope"]),
              theta=float(g["theta"]), mask=dev(g["mask"]))
    O, LSE = gn.attn_fwd(dev(g["Q"]), dev(g["K"]), dev(g["V"]), **kw)
    assert rel_err(host(O), g["O"]) < FP32_TOL and rel_err(host(LSE), g["LSE"]) < FP32_TOL
    dQ, dK, dV = gn.attn_bwd(dev(g["Q"]), dev(g["K"]), dev(g["V"]), dev(g["O"]), dev(g["dO"]),
                             dev(g["LSE"]), **kw)
    assert rel_err(host(dQ), g["dQ"]) < FP32_TOL
    assert rel_err(host(dK), g["dK"]) < FP32_TOL
    assert rel_err(host(dV), g["dV"]) < FP32_TOL


@pytest.mark.parametrize("S,D,causal,rope", [(320, 128, True, "interleaved"), (320, 64, False, "none"),
                                             (200, 64, True, "half"), (256, 128, False, "interleaved")])
def test_attention_mask_bf16_mfma(gn, S, D, causal, rope):
    """A padded batch on the MFMA kernels: batch 0 unmasked, batch 1 with a ragged padded tail
    (partial 64-key tile) and holes inside the sequence; forward and backward vs the oracle."""
    r = np.random.default_rng(21)
    B, H = 2, 2
    Q, K, V = (rnd(r.standard_normal((B, H, S, D)).astype(np.float32)) for _ in range(3))
    dO = rnd((r.standard_normal((B, H, S, D)) * 0.01).astype(np.float32))
    mask = padded_mask(B, S, [S, S - 57], holes=[(1, 5), (1, 63), (1, 64), (1, 130)])
    kw = dict(causal=causal, rope_mode=rope, mask=mask)
    rO, rL = oracle.attn_fwd(Q, K, V, **kw)
    bf = torch.bfloat16
    O, LSE = gn.attn_fwd(dev(Q, bf), dev(K, bf), dev(V, bf), causal=causal, rope=rope,
                         mask=dev(mask))
    assert rel_err(host(O), rO) < BF16_TOL and rel_err(host(LSE), rL) < 1e-3
    Ob = rnd(rO)
    rQ, rK, rV = oracle.attn_bwd(Q, K, V, dO, rL, **kw)
    dQ, dK, dV = gn.attn_bwd(dev(Q, bf), dev(K, bf), dev(V, bf), dev(Ob, bf), dev(dO, bf), dev(rL),
                             causal=causal, rope=rope, mask=dev(mask))
    assert rel_err(host(dV), rV) < BF16_TOL
    assert rel_err(host(dQ), rQ) < BF16_TOL
    assert rel_err(host(dK), rK) < BF16_TOL
    # masked keys receive no gradient at all
    gone = mask[1] == 0
    assert np.all(host(dK)[1][:, gone] == 0) and np.all(host(dV)[1][:, gone] == 0)


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_attention_mask_fully_masked_rows(gn, dt):
    """A batch whose keys are all masked (no causal mask): O = 0, LSE = -inf and zero
    gradients for it (the documented convention); the other batch matches the oracle."""
    r = np.random.default_rng(22)
    B, H, S, D = 2, 2, 128, 64
    Q, K, V = (rnd(r.standard_normal((B, H, S, D)).astype(np.float32)) for _ in range(3))
    dO = rnd((r.standard_normal((B, H, S, D)) * 0.01).astype(np.float32))
    mask = padded_mask(B, S, [S - 10, 0])
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    tol = BF16_TOL if dt == "bf16" else FP32_TOL
    O, LSE = gn.attn_fwd(dev(Q, tdt), dev(K, tdt), dev(V, tdt), causal=False, rope="none",
                         mask=dev(mask))
    rO, rL = oracle.attn_fwd(Q[:1], K[:1], V[:1], causal=False, rope_mode="none", mask=mask[:1])
    assert rel_err(host(O)[:1], rO) < tol and rel_err(host(LSE)[:1], rL) < 1e-3
    assert np.all(host(O)[1] == 0) and np.all(np.isneginf(host(LSE)[1]))
    dQ, dK, dV = gn.attn_bwd(dev(Q, tdt), dev(K, tdt), dev(V, tdt), O, dev(dO, tdt), LSE,
                             causal=False, rope="none", mask=dev(mask))
    rQ, rK, rV = oracle.attn_bwd(Q[:1], K[:1], V[:1], dO[:1], rL, causal=False, rope_mode="none",
                                 mask=mask[:1])
    for got, ref in ((dQ, rQ), (dK, rK), (dV, rV)):
        g = host(got)
        assert np.all(np.isfinite(g)) and np.all(g[1] == 0)
        assert rel_err(g[:1], ref) < tol


def test_attention_mask_fused_qkv_layout(gn):
    r = np.random.default_rng(23)
    B, H, S, D = 2, 3, 192, 64
    Q, K, V = (rnd(r.standard_normal((B, H, S, D)).astype(np.float32)) for _ in range(3))
    dO = rnd((r.standard_normal((B, H, S, D)) * 0.01).astype(np.float32))
    mask = padded_mask(B, S, [150, S], holes=[(1, 70)])
    O, LSE = oracle.attn_fwd(Q, K, V, causal=True, rope_mode="interleaved", mask=mask)
    O = rnd(O)
    rQ, rK, rV = oracle.attn_bwd(Q, K, V, dO, LSE, causal=True, rope_mode="interleaved", mask=mask)
    bshd = lambda t: np.ascontiguousarray(t.transpose(0, 2, 1, 3).reshape(B, S, H * D))
    qkv = np.concatenate([bshd(Q), bshd(K), bshd(V)], axis=-1)
    dqkv = gn.attn_bwd_qkv(dev(qkv, torch.bfloat16), dev(bshd(O), torch.bfloat16),
                           dev(bshd(dO), torch.bfloat16), dev(LSE), H, causal=True,
                           rope="interleaved", mask=dev(mask))
    got = host(dqkv).reshape(B, S, 3, H, D).transpose(2, 0, 3, 1, 4)
    assert rel_err(got[0], rQ) < BF16_TOL
    assert rel_err(got[1], rK) < BF16_TOL
    assert rel_err(got[2], rV) < BF16_TOL


def test_attention_mask_through_tape(gpu):
    """FlashAttention2 node with the mask as its fourth input (no gradient for it)."""
    import grilly_core as gc
    import grilly_bridge as gb
    d = gc.Device(0)
    gb.attach_torch_stream(d)
    r = np.random.default_rng(24)
    B, H, S, D = 2, 2, 128, 64
    bf = torch.bfloat16
    T = lambda x, t=torch.float32: dev(x, t).contiguous()
    Qn, Kn, Vn = (rnd(r.standard_normal((B, H, S, D)).astype(np.float32)) for _ in range(3))
    dOn = rnd((r.standard_normal((B, H, S, D)) * 0.01).astype(np.float32))
    mask = padded_mask(B, S, [S, 90])
    O_, LSE_ = oracle.attn_fwd(Qn, Kn, Vn, mask=mask)
    Q, K, V, dO, O = T(Qn, bf), T(Kn, bf), T(Vn, bf), T(dOn, bf), T(O_, bf)
    LSE, M = T(LSE_), T(mask)
    tape = gb.create_tape_context(d)
    tape.begin()
    na = tape.record_op(gc.OpType.FlashAttention2,
                        [gb.tref(Q, True), gb.tref(K, True), gb.tref(V, True), gb.tref(M)],
                        [gb.tref(O)], gb.attention_params(causal=True, rope="interleaved"))
    tape.save_for_backward(na, [LSE.data_ptr()])
    tape.backward(na, dO.data_ptr())
    rQ, rK, rV = oracle.attn_bwd(Qn, Kn, Vn, dOn, LSE_, mask=mask)
    g = lambda t: gb.download(d, tape.get_grad_buffer(t.data_ptr()), t.shape, gb.dtype_code(t))
    assert rel_err(g(Q), rQ) < BF16_TOL
    assert rel_err(g(K), rK) < BF16_TOL
    assert rel_err(g(V), rV) < BF16_TOL
    assert tape.get_grad_buffer(M.data_ptr()) == 0
    tape.end()


# ---------------------------------------------------------------------------- RMSNorm stats
@pytest.mark.parametrize("stat", ["rstd", "meansq", "rms"])
def test_rmsnorm_stat_forms_golden(gn, stat):
    """The backward from each saved form against torch float64 autograd; the forward saves
    each form as the reference's shaders define it."""
    g = golden("rmsnorm_stats")
    eps = float(g["eps"])
    X, w = dev(g["X"]), dev(g["w"])
    Y, st = gn.rmsnorm_fwd(X, w, eps=eps, stat=stat)
    assert rel_err(host(Y), g["Y"]) < FP32_TOL
    assert rel_err(host(st), g[stat]) < 1e-6
    dX, dW = gn.rmsnorm_bwd(dev(g["dY"]), X, w, dev(g[stat]), stat=stat, eps=eps)
    assert rel_err(host(dX), g["dX"]) < FP32_TOL and rel_err(host(dW), g["dW"]) < FP32_TOL


@pytest.mark.parametrize("stat", ["meansq", "rms"])
def test_rmsnorm_stat_forms_bf16_c2_width(gn, stat):
    """bf16 at the FFN block's width (d 2048) with an fp32 residual-stream variant: each saved
    form gives the rstd form's gradients."""
    r = np.random.default_rng(25)
    rows, F, eps = 512, 2048, 1e-6
    bf = torch.bfloat16
    x = dev(r.standard_normal((rows, F)), bf)
    w = dev(1 + 0.1 * r.standard_normal(F), bf)
    dY = dev(r.standard_normal((rows, F)) * 0.01, bf)
    _, rstd = gn.rmsnorm_fwd(x, w, eps=eps)
    _, st = gn.rmsnorm_fwd(x, w, eps=eps, stat=stat)
    dX0, dW0 = gn.rmsnorm_bwd(dY, x, w, rstd)
    dX1, dW1 = gn.rmsnorm_bwd(dY, x, w, st, stat=stat, eps=eps)
    assert rel_err(host(dX1), host(dX0)) < 1e-2 and rel_err(host(dW1), host(dW0)) < 1e-5
    ref_x, ref_w = oracle.rmsnorm_bwd(host(dY), host(x), host(w), host(rstd))
    assert rel_err(host(dX1), ref_x) < BF16_TOL and rel_err(host(dW1), ref_w) < BF16_TOL
    xf = x.float().contiguous()
    add = dev(r.standard_normal((rows, F)))
    dX2, _ = gn.rmsnorm_bwd(dY, xf, w, st, stat=stat, eps=eps, dX_add=add)
    assert rel_err(host(dX2), ref_x + host(add)) < BF16_TOL


def test_rmsnorm_stat_form_through_tape(gpu):
    import grilly_core as gc
    import grilly_bridge as gb
    d = gc.Device(0)
    gb.attach_torch_stream(d)
    g = golden("rmsnorm_stats")
    X, w, dY = dev(g["X"]).contiguous(), dev(g["w"]).contiguous(), dev(g["dY"]).contiguous()
    ms, Y = dev(g["meansq"]).contiguous(), dev(g["Y"]).contiguous()
    tape = gb.create_tape_context(d)
    tape.begin()
    n = tape.record_op(gc.OpType.RMSNorm, [gb.tref(X, True)], [gb.tref(Y)],
                       gb.rmsnorm_params(float(g["eps"]), "meansq"))
    tape.save_for_backward(n, [w.data_ptr(), ms.data_ptr()])
    tape.backward(n, dY.data_ptr())
    gX = gb.download(d, tape.get_grad_buffer(X.data_ptr()), X.shape, gb.dtype_code(X))
    gW = gb.download(d, tape.get_grad_buffer(w.data_ptr()), w.shape, gb.dtype_code(w))
    assert rel_err(gX, g["dX"]) < FP32_TOL and rel_err(gW, g["dW"]) < FP32_TOL
    tape.end()
