"""GPU parity of the generic matrix-core attention backward (csrc/gn_attn.hip attn_bwd_gen):
fp32 at D = 32, 64, 96, 128, 192, 256 (two-piece bf16 split, three products) and bf16 at the
head dims the tuned kernels do not take (32, 96, 192, 256), against the oracle restatement of
attention-backward.glsl:73-194 with causal / full masks, both RoPE pairings and the key mask.

Tolerances (normwise relative error): fp32 <= 1e-4, bf16 <= 2e-2 against the fp32 oracle on
the same bf16-rounded inputs."""
import numpy as np
import pytest

import oracle
from conftest import rel_err

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


def _case(gn, dt, B, H, S, D, causal, rope, mask=None, seed=31):
    r = np.random.default_rng(seed)
    Q, K, V = (r.standard_normal((B, H, S, D)).astype(np.float32) for _ in range(3))
    dO = (r.standard_normal((B, H, S, D)) * 0.01).astype(np.float32)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    if dt == "bf16":
        Q, K, V, dO = (rnd(x) for x in (Q, K, V, dO))
    kw = dict(causal=causal, rope_mode=rope, mask=mask)
    O, LSE = oracle.attn_fwd(Q, K, V, **kw)
    if dt == "bf16":
        O = rnd(O)
    rQ, rK, rV = oracle.attn_bwd(Q, K, V, dO, LSE, **kw)
    dQ, dK, dV = gn.attn_bwd(dev(Q, tdt), dev(K, tdt), dev(V, tdt), dev(O, tdt), dev(dO, tdt),
                             dev(LSE), causal=causal, rope=rope,
                             mask=None if mask is None else dev(mask))
    return (host(dQ), host(dK), host(dV)), (rQ, rK, rV)


@pytest.mark.parametrize("D", [32, 64, 96, 128, 192, 256])
@pytest.mark.parametrize("causal,rope", [(True, "interleaved"), (False, "half")])
def test_attention_generic_fp32(gn, D, causal, rope):
    got, ref = _case(gn, "f32", 1, 2, 200, D, causal, rope)
    for g, r in zip(got, ref):
        assert rel_err(g, r) < FP32_TOL


@pytest.mark.parametrize("D", [32, 96, 192, 256])
@pytest.mark.parametrize("causal,rope", [(True, "interleaved"), (False, "none")])
def test_attention_generic_bf16(gn, D, causal, rope):
    got, ref = _case(gn, "bf16", 2, 2, 160, D, causal, rope)
    for g, r in zip(got, ref):
        assert rel_err(g, r) < BF16_TOL


@pytest.mark.parametrize("dt,D", [("f32", 96), ("f32", 128), ("bf16", 256)])
def test_attention_generic_key_mask(gn, dt, D):
    S = 192
    mask = np.ones((2, S), np.float32)
    mask[1, 130:] = 0.0
    mask[1, 17] = 0.0
    got, ref = _case(gn, dt, 2, 2, S, D, True, "interleaved", mask=mask, seed=32)
    tol = FP32_TOL if dt == "f32" else BF16_TOL
    for g, r in zip(got, ref):
        assert rel_err(g, r) < tol
    assert np.all(got[1][1][:, mask[1] == 0] == 0) and np.all(got[2][1][:, mask[1] == 0] == 0)


def test_c3_fp32_full_size_sampled_heads(gn):
    """C3's shape in fp32 (B 4, H 16, S 2048, D 128, causal, interleaved RoPE 1e4): the generic
    matrix-core backward on heads (0, 0), (2, 9), (3, 15) against the oracle (forward and
    backward recomputed from the same inputs), and a second backward bit-identical."""
    r = np.random.default_rng(45)
    B, H, S, D = 4, 16, 2048, 128
    Q, K, V = (r.standard_normal((B, H, S, D)).astype(np.float32) for _ in range(3))
    dO = (r.standard_normal((B, H, S, D)) * 1e-2).astype(np.float32)
    tQ, tK, tV, tdO = dev(Q), dev(K), dev(V), dev(dO)
    O, LSE = gn.attn_fwd(tQ, tK, tV, causal=True, rope="interleaved", theta=10000.0)
    dQ, dK, dV = gn.attn_bwd(tQ, tK, tV, O, tdO, LSE, causal=True, rope="interleaved",
                             theta=10000.0)
    dQ2, dK2, dV2 = gn.attn_bwd(tQ, tK, tV, O, tdO, LSE, causal=True, rope="interleaved",
                                theta=10000.0)
    assert torch.equal(dQ, dQ2) and torch.equal(dK, dK2) and torch.equal(dV, dV2)
    for bi, hi in [(0, 0), (2, 9), (3, 15)]:
        sl = (slice(bi, bi + 1), slice(hi, hi + 1))
        q, k, v, do = (np.ascontiguousarray(t[sl]) for t in (Q, K, V, dO))
        o, lse = oracle.attn_fwd(q, k, v, causal=True, rope_mode="interleaved", theta=10000.0)
        assert rel_err(host(O[bi, hi]), o[0, 0]) < FP32_TOL
        rq, rk, rv = oracle.attn_bwd(q, k, v, do, lse, causal=True, rope_mode="interleaved",
                                     theta=10000.0)
        for got, ref in ((dQ, rq), (dK, rk), (dV, rv)):
            assert rel_err(host(got[bi, hi]), ref[0, 0]) < FP32_TOL, (bi, hi)


@pytest.mark.parametrize("dt,D", [("f32", 32), ("f32", 64), ("f32", 96), ("f32", 128), ("f32", 192),
                                  ("f32", 256), ("bf16", 32), ("bf16", 96), ("bf16", 192),
                                  ("bf16", 256)])
@pytest.mark.parametrize("causal,rope", [(True, "interleaved"), (False, "half")])
def test_attention_generic_forward(gn, dt, D, causal, rope):
    """The generic matrix-core forward: O and the natural-log LSE against the oracle; a key
    mask on the second batch; the backward run on the forward's own O and LSE."""
    r = np.random.default_rng(33)
    B, H, S = 2, 2, 176
    Q, K, V = (r.standard_normal((B, H, S, D)).astype(np.float32) for _ in range(3))
    dO = (r.standard_normal((B, H, S, D)) * 0.01).astype(np.float32)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    if dt == "bf16":
        Q, K, V, dO = (rnd(x) for x in (Q, K, V, dO))
    mask = np.ones((B, S), np.float32)
    mask[1, 120:] = 0.0
    kw = dict(causal=causal, rope_mode=rope, mask=mask)
    rO, rL = oracle.attn_fwd(Q, K, V, **kw)
    O, LSE = gn.attn_fwd(dev(Q, tdt), dev(K, tdt), dev(V, tdt), causal=causal, rope=rope,
                         mask=dev(mask))
    tol = FP32_TOL if dt == "f32" else BF16_TOL
    assert rel_err(host(O), rO) < tol and rel_err(host(LSE), rL) < (FP32_TOL if dt == "f32" else 1e-3)
    rQ, rK, rV = oracle.attn_bwd(Q, K, V, dO, rL, **kw)
    dQ, dK, dV = gn.attn_bwd(dev(Q, tdt), dev(K, tdt), dev(V, tdt), O, dev(dO, tdt), LSE,
                             causal=causal, rope=rope, mask=dev(mask))
    for g, ref in ((dQ, rQ), (dK, rK), (dV, rV)):
        assert rel_err(host(g), ref) < tol
