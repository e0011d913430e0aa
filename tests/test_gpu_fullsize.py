"""GPU parity at the benchmark's full sizes (C3, C4).

The oracle cannot redo a whole full-size workload in test time, so these tests check what a
full-size launch can get wrong (grid shapes, 32-bit offsets, the last heads / rows / tiles)
through properties that do not depend on size:
  * exact integer identities (VSA dW with integer dY: every partial sum is an integer below
    2^24, so the GPU result must equal the integer computation bit for bit);
  * rows, heads or output rows sampled across the whole tensor, recomputed by the oracle from
    the same inputs (each sampled row / head is independent of the others);
  * exact scaling (the surrogate gradient is linear in its scale; doubling is exact in fp32)
    and run-to-run bit-identity.
Tolerances as in test_gpu_kernels.py: bf16 paths 2e-2, fp32 outputs of bf16 products 1e-4.
"""
import numpy as np
import pytest

import oracle
from conftest import rel_err

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

BF16_TOL = 2e-2
FP32_TOL = 1e-4


@pytest.fixture(scope="module")
def gn(gpu):
    import gn_bwd
    gn_bwd.lib()
    return gn_bwd


def dev(x, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0").to(dtype)


def host(t):
    return t.float().cpu().numpy()


def bf16_round(x):
    return host(dev(x, torch.bfloat16))


# ------------------------------------------------------------------- C4: VSA unpack-project
def test_c4_vsa_dw_integer_identity_full_size(gn):
    """C4 at full size (8192 rows x 320 words -> 768 outputs) with dY[b, o] = u_b a_o
    (u in 1..3, a in -2..2): dW[o, j] = a_o (2 sum_b u_b bit_b(j) - sum_b u_b) and
    db[o] = a_o sum_b u_b exactly (bits LSB-first in little-endian words)."""
    r = np.random.default_rng(41)
    Bn, O, D = 8192, 768, 10240
    bits = r.integers(0, 2**32, size=(Bn, D // 32), dtype=np.uint64).astype(np.uint32)
    u = r.integers(1, 4, size=Bn).astype(np.int64)
    a = r.integers(-2, 3, size=O).astype(np.int64)
    dY = (u[:, None] * a[None, :]).astype(np.float32)
    dW, db = gn.vsa_unpack_project_bwd(dev(dY), gn.u32_tensor(bits, "cuda:0"), D)
    unpacked = np.unpackbits(bits.view(np.uint8), axis=1, bitorder="little")
    v = np.zeros(D, np.int64)
    for c in range(0, Bn, 1024):  # sum_b u_b bit_b(j) in int64, 1024 rows at a time
        v += u[c:c + 1024] @ unpacked[c:c + 1024].astype(np.int64)
    v = 2 * v - u.sum()
    np.testing.assert_array_equal(host(dW), (a[:, None] * v[None, :]).astype(np.float32))
    np.testing.assert_array_equal(host(db), (a * u.sum()).astype(np.float32))


def test_c4_vsa_dw_fp32_sampled_outputs_full_size(gn):
    """C4 at full size with N(0, 1) fp32 dY: sampled output rows of dW (first, last and
    random) against the oracle over all 8192 rows, and bit-identical reruns."""
    r = np.random.default_rng(42)
    Bn, O, D = 8192, 768, 10240
    bits = r.integers(0, 2**32, size=(Bn, D // 32), dtype=np.uint64).astype(np.uint32)
    dY = r.standard_normal((Bn, O)).astype(np.float32)
    tb = gn.u32_tensor(bits, "cuda:0")
    tdY = dev(dY)
    dW1, db1 = gn.vsa_unpack_project_bwd(tdY, tb, D)
    dW2, db2 = gn.vsa_unpack_project_bwd(tdY, tb, D)
    assert torch.equal(dW1, dW2) and torch.equal(db1, db2)
    rows = np.unique(np.r_[0, O - 1, r.integers(0, O, 6)])
    rW, rb = oracle.vsa_unpack_project_bwd(np.ascontiguousarray(dY[:, rows]), bits, D)
    assert rel_err(host(dW1)[rows], rW) < FP32_TOL
    assert rel_err(host(db1)[rows], rb) < FP32_TOL


# ------------------------------------------------------------------- C4: surrogate loss
def test_c4_surrogate_full_size_sampled_rows_and_scaling(gn):
    """Surrogate backward at full size (8192 x K=4 x 10240 fp32, 1.3 GB in, 1.3 GB out):
    sampled rows (first, last, random) against the oracle, and scale=2 gives exactly twice
    the scale=1 gradient everywhere."""
    r = np.random.default_rng(43)
    Bn, K, D = 8192, 4, 10240
    g = torch.Generator(device="cuda:0").manual_seed(43)
    preds = torch.randn((Bn, K, D), device="cuda:0", generator=g)
    bits = r.integers(0, 2**32, size=(Bn, D // 32), dtype=np.uint64).astype(np.uint32)
    win = r.integers(0, K, Bn)
    run = np.where(r.random(Bn) < 0.25, win, (win + r.integers(1, K, Bn)) % K)
    dots = r.standard_normal((Bn, 2)).astype(np.float32) * 40
    results = np.stack([win, run, dots[:, 0].view(np.uint32), dots[:, 1].view(np.uint32)],
                       axis=1).astype(np.uint32)
    w = r.random((Bn, K)).astype(np.float32)
    w /= w.sum(1, keepdims=True)
    tb, tr, tw = gn.u32_tensor(bits, "cuda:0"), gn.u32_tensor(results, "cuda:0"), dev(w)
    dP = gn.vsa_surrogate_bwd(preds, tb, tr, tw)
    dP2 = gn.vsa_surrogate_bwd(preds, tb, tr, tw, scale=2.0)
    assert torch.equal(dP2, 2 * dP)
    rows = np.unique(np.r_[0, Bn - 1, r.integers(0, Bn, 4)])
    ref = oracle.vsa_surrogate_bwd(host(preds[torch.from_numpy(rows).to("cuda:0")]),
                                   bits[rows], results[rows], w[rows])
    assert rel_err(host(dP[torch.from_numpy(rows).to("cuda:0")]), ref) < 1e-6


# ------------------------------------------------------------------- C3: attention
def test_c3_attention_full_size_sampled_heads(gn):
    """C3 at full size (B 4, H 16, S 2048, D 128, causal, interleaved RoPE 1e4): the GPU
    forward gives O and LSE, the GPU backward dQ, dK, dV; heads (0, 0), (1, 7) and (3, 15)
    are recomputed by the oracle (forward and backward) from the same bf16 inputs, and a
    second backward is bit-identical."""
    r = np.random.default_rng(44)
    B, H, S, D = 4, 16, 2048, 128
    Q, K, V = (bf16_round(r.standard_normal((B, H, S, D)).astype(np.float32)) for _ in range(3))
    dO = bf16_round((r.standard_normal((B, H, S, D)) * 1e-2).astype(np.float32))
    b = torch.bfloat16
    tQ, tK, tV, tdO = dev(Q, b), dev(K, b), dev(V, b), dev(dO, b)
    O, LSE = gn.attn_fwd(tQ, tK, tV, causal=True, rope="interleaved", theta=10000.0)
    dQ, dK, dV = gn.attn_bwd(tQ, tK, tV, O, tdO, LSE, causal=True, rope="interleaved",
                             theta=10000.0)
    dQ2, dK2, dV2 = gn.attn_bwd(tQ, tK, tV, O, tdO, LSE, causal=True, rope="interleaved",
                                theta=10000.0)
    assert torch.equal(dQ, dQ2) and torch.equal(dK, dK2) and torch.equal(dV, dV2)
    for bi, hi in [(0, 0), (1, 7), (3, 15)]:
        sl = (slice(bi, bi + 1), slice(hi, hi + 1))
        q, k, v, do = (np.ascontiguousarray(t[sl]) for t in (Q, K, V, dO))
        _, lse = oracle.attn_fwd(q, k, v, causal=True, rope_mode="interleaved", theta=10000.0)
        assert rel_err(host(LSE)[bi, hi], lse[0, 0]) < 1e-3
        rq, rk, rv = oracle.attn_bwd(q, k, v, do, lse, causal=True, rope_mode="interleaved",
                                     theta=10000.0)
        for got, ref in ((dQ, rq), (dK, rk), (dV, rv)):
            assert rel_err(host(got[bi, hi]), ref[0, 0]) < BF16_TOL, (bi, hi)


# ------------------------------------------------------------------- C2: FFN block
def test_c2_ffn_block_full_size_sampled(gn):
    """C2 at full size (T 4096, d 2048, h 5632, SwiGLU on up, RMSNorm): the three entry points
    of the headline step; the GLU local gradients and dN on sampled rows, dWd / dWg / dWu on
    sampled output rows (over all 4096 tokens), and the whole RMSNorm backward, against the
    oracle on the same bf16 inputs."""
    r = np.random.default_rng(45)
    T, d, h = 4096, 2048, 5632
    kind = "swiglu_up"
    x = bf16_round(r.standard_normal((T, d)).astype(np.float32))
    w = np.ones(d, np.float32)
    Wg, Wu = (bf16_round((r.standard_normal((h, d)) * 0.02).astype(np.float32)) for _ in range(2))
    Wd = bf16_round((r.standard_normal((d, h)) * 0.02).astype(np.float32))
    dY = bf16_round((r.standard_normal((T, d)) * 1e-2).astype(np.float32))
    n, rstd = oracle.rmsnorm_fwd(x, w)
    n = bf16_round(n)
    b = torch.bfloat16
    tn, tWg, tWu = dev(n, b), dev(Wg, b), dev(Wu, b)
    gate = host(torch.matmul(tn, tWg.t().contiguous()).to(b))
    up = host(torch.matmul(tn, tWu.t().contiguous()).to(b))
    A = bf16_round(oracle.glu_fwd(kind, gate, up))
    gu, dWd, _ = gn.ffn_down_glu_bwd(kind, dev(dY, b), dev(A, b), dev(Wd, b), dev(gate, b),
                                     dev(up, b))
    dN, dWg, dWu, _, _ = gn.glu_proj_bwd(gu, tn, tWg, tWu)
    dx, dw = gn.rmsnorm_bwd(dN, dev(x, b), dev(w, b), dev(rstd))
    torch.cuda.synchronize()
    hgu, hdN = host(gu), host(dN)
    rows = np.unique(np.r_[0, T - 1, r.integers(0, T, 14)])
    dA = oracle.linear_bwd(dY[rows], A[rows], Wd, need_db=False)[0]
    rG, rU = oracle.glu_bwd(kind, dA, gate[rows], up[rows])
    assert rel_err(hgu[rows, :h], rG) < BF16_TOL and rel_err(hgu[rows, h:], rU) < BF16_TOL
    gG, gU = hgu[:, :h], hgu[:, h:]
    rN = gG[rows].astype(np.float64) @ Wg + gU[rows].astype(np.float64) @ Wu
    assert rel_err(hdN[rows], rN) < BF16_TOL
    outs = np.unique(np.r_[0, d - 1, r.integers(0, d, 6)])
    assert rel_err(host(dWd)[outs], dY[:, outs].T.astype(np.float64) @ A) < FP32_TOL
    # dWu rows either side of 2560: [dWg;dWu] row 8192, where its first 256 x 256 launch ends
    outs_h = np.unique(np.r_[0, 2559, 2560, h - 1, r.integers(0, h, 6)])
    assert rel_err(host(dWg)[outs_h], gG[:, outs_h].T.astype(np.float64) @ n) < FP32_TOL
    assert rel_err(host(dWu)[outs_h], gU[:, outs_h].T.astype(np.float64) @ n) < FP32_TOL
    rx, rw = oracle.rmsnorm_bwd(hdN, x, w, rstd)
    assert rel_err(host(dx), rx) < BF16_TOL
    assert rel_err(host(dw), rw) < 1e-3  # fp32 sums over 4096 bf16-rounded rows
