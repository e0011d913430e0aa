"""GPU parity: every libgn_bwd entry point against the CPU oracle on seeded inputs.

Tolerances (normwise relative error max|gpu - ref| / max|ref|):
  fp32 paths   <= 1e-4
  bf16 paths   <= 2e-2 against the fp32 oracle run on the same bf16-rounded inputs
  bit / integer work: exact.
"""
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
    """bf16-round a float32 numpy array (what the kernel actually sees)."""
    return host(dev(x, torch.bfloat16))


def rng_(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------------------- GEMM core
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("shape", [(136, 200, 72), (256, 128, 640), (8, 8, 8), (264, 136, 128),
                                   (520, 392, 256), (1024, 768, 512)])
def test_gemm_bf16_layouts(gn, ta, tb, shape):
    M, N, K = shape
    r = rng_(1)
    A = rnd(r.standard_normal((K, M) if ta else (M, K)).astype(np.float32))
    B = rnd(r.standard_normal((N, K) if tb else (K, N)).astype(np.float32))
    ref = (A.T if ta else A).astype(np.float64) @ (B.T if tb else B).astype(np.float64)
    C = gn.gemm(dev(A, torch.bfloat16), dev(B, torch.bfloat16), bool(ta), bool(tb),
                out_dtype=torch.float32)
    assert rel_err(host(C), ref) < 1e-5
    Cb = gn.gemm(dev(A, torch.bfloat16), dev(B, torch.bfloat16), bool(ta), bool(tb),
                 out_dtype=torch.bfloat16)
    assert rel_err(host(Cb), ref) < 8e-3


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0)])
@pytest.mark.parametrize("shape", [(8192, 768, 768), (8192, 768, 2304), (1000, 384, 192),
                                   (520, 1536, 640)])
def test_gemm_bf16_decoder_input_gradient_shapes(gn, ta, tb, shape):
    """bf16-output products of the decoder's N = 768 input-gradient shapes (192 output tiles of
    256 x 128, under one round of the 256 CUs) and two edge shapes: against fp64, and bit-equal
    to the fp32-output product rounded to bf16 where that one is not split over K (an output
    element's k order does not depend on the tile shape the time model picks)."""
    M, N, K = shape
    r = rng_(2)
    A = rnd(r.standard_normal((K, M) if ta else (M, K)).astype(np.float32))
    B = rnd(r.standard_normal((N, K) if tb else (K, N)).astype(np.float32))
    ref = (A.T if ta else A).astype(np.float64) @ (B.T if tb else B).astype(np.float64)
    Ad, Bd = dev(A, torch.bfloat16), dev(B, torch.bfloat16)
    Cb = gn.gemm(Ad, Bd, bool(ta), bool(tb), out_dtype=torch.bfloat16)
    assert rel_err(host(Cb), ref) < 8e-3
    if K < 2048:
        C = gn.gemm(Ad, Bd, bool(ta), bool(tb), out_dtype=torch.float32)
        assert torch.equal(Cb, C.to(torch.bfloat16))


def test_gemm_two_segments_and_accumulate(gn):
    r = rng_(2)
    M, N, K0, K1 = 64, 96, 40, 24
    A0, A1 = (rnd(r.standard_normal((M, k)).astype(np.float32)) for k in (K0, K1))
    B0, B1 = (rnd(r.standard_normal((k, N)).astype(np.float32)) for k in (K0, K1))
    ref = A0.astype(np.float64) @ B0 + A1.astype(np.float64) @ B1
    C = gn.gemm(dev(A0, torch.bfloat16), dev(B0, torch.bfloat16), A1=dev(A1, torch.bfloat16),
                B1=dev(B1, torch.bfloat16), out_dtype=torch.float32)
    assert rel_err(host(C), ref) < 1e-5
    gn.gemm(dev(A0, torch.bfloat16), dev(B0, torch.bfloat16), C=C, accumulate=True)
    assert rel_err(host(C), ref + A0.astype(np.float64) @ B0) < 1e-5


def test_gemm_two_segments_dma_path(gn):
    # K segments that are multiples of 64 take the LDS-DMA kernel; edge tiles in M and N
    r = rng_(21)
    M, N, K0, K1 = 392, 200, 128, 192
    for ta, tb in [(0, 0), (1, 0), (0, 1)]:
        A0 = rnd(r.standard_normal((K0, M) if ta else (M, K0)).astype(np.float32))
        A1 = rnd(r.standard_normal((K1, M) if ta else (M, K1)).astype(np.float32))
        B0 = rnd(r.standard_normal((N, K0) if tb else (K0, N)).astype(np.float32))
        B1 = rnd(r.standard_normal((N, K1) if tb else (K1, N)).astype(np.float32))
        op = lambda x, t: (x.T if t else x).astype(np.float64)
        ref = op(A0, ta) @ op(B0, tb) + op(A1, ta) @ op(B1, tb)
        C = gn.gemm(dev(A0, torch.bfloat16), dev(B0, torch.bfloat16), bool(ta), bool(tb),
                    A1=dev(A1, torch.bfloat16), B1=dev(B1, torch.bfloat16), out_dtype=torch.float32)
        assert rel_err(host(C), ref) < 1e-5, (ta, tb)


def test_gemm_row_split_whole_rounds(gn):
    """A grid whose last round of tiles would be part-filled (11264 x 2048 x 4096 with a
    k-outer A: the FFN's [dWg;dWu] shape) runs its first 8192 rows as one round of 256 x 256
    tiles and the rest as a second launch: bit-identical to the same rows computed in blocks
    small enough for one launch each, within the fp32 bar of the float64 product on rows
    either side of 8192, and accumulate adds onto what is there.  The weight gradient of a
    Linear of that shape splits its row sums (db) the same way."""
    M, N, K = 11264, 2048, 4096
    g = torch.Generator(device="cuda:0").manual_seed(46)
    A = torch.randn(K, M, device="cuda:0", generator=g).bfloat16()
    B = torch.randn(K, N, device="cuda:0", generator=g).bfloat16()
    C = gn.gemm(A, B, transA=True, out_dtype=torch.float32)
    # the blocks accumulate onto zeros, so none takes a split-K schedule (whose two halves
    # would add in another order)
    zeros = lambda *shape: torch.zeros(shape, device="cuda:0")
    parts = [gn.gemm(A[:, r0:r0 + 1024].contiguous(), B, transA=True, C=zeros(1024, N),
                     accumulate=True) for r0 in range(0, M, 1024)]
    assert torch.equal(C, torch.cat(parts))
    rows = np.r_[0, 255, 8191, 8192, 8193, 10000, M - 1]
    ref = host(A[:, rows]).astype(np.float64).T @ host(B).astype(np.float64)
    assert rel_err(host(C[rows]), ref) < 1e-5
    C2 = C.clone()
    gn.gemm(A, B, transA=True, out_dtype=torch.float32, C=C2, accumulate=True)
    assert torch.equal(C2, C + C)
    # Linear y = x W^T + b with 11264 outputs over 4096 tokens: dW = dY^T X, db = sum_t dY
    dY = torch.randn(K, M, device="cuda:0", generator=g).bfloat16()
    X = torch.randn(K, N, device="cuda:0", generator=g).bfloat16()
    W = (torch.randn(M, N, device="cuda:0", generator=g) * 0.02).bfloat16()
    _, dW, db = gn.linear_bwd(dY, X, W, need_dx=False)
    dWp = [gn.linear_bwd(dY[:, r0:r0 + 1024].contiguous(), X, W[r0:r0 + 1024].contiguous(),
                         need_dx=False, dW=zeros(1024, N), db=zeros(1024), accumulate=True,
                         ws=False)[1] for r0 in range(0, M, 1024)]
    assert torch.equal(dW, torch.cat(dWp))
    hdY = host(dY).astype(np.float64)
    assert rel_err(host(dW[rows]), hdY[:, rows].T @ host(X).astype(np.float64)) < 1e-5
    assert rel_err(host(db), hdY.sum(0)) < 1e-5


def test_gemm_unaligned_falls_back(gn):
    r = rng_(3)
    A = rnd(r.standard_normal((10, 13)).astype(np.float32))
    B = rnd(r.standard_normal((13, 7)).astype(np.float32))
    C = gn.gemm(dev(A, torch.bfloat16), dev(B, torch.bfloat16), out_dtype=torch.float32)
    assert rel_err(host(C), A.astype(np.float64) @ B) < 1e-5


# ---------------------------------------------------------------------------- fp32 on MFMA
# fp32 operands run on the bf16 matrix cores through a three-piece split and six products
# (fp32-grade).  Against float64: normwise <= 1e-4 (the fp32 bar), and, element by element,
# within a few fp32 ulps of the summed magnitudes (what an FMA chain guarantees), which a
# two-piece split (~2^-16 per product) would miss.  A bf16-only product would be off by
# ~2e-3 on these inputs.
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("shape", [(136, 200, 72), (256, 128, 640), (132, 68, 1000), (8, 8, 8),
                                   (10, 13, 7), (1024, 1024, 64)])
def test_gemm_fp32_layouts(gn, ta, tb, shape):
    M, N, K = shape
    r = rng_(31)
    A = (r.standard_normal((K, M) if ta else (M, K)) * 3).astype(np.float32)
    B = r.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    ref = (A.T if ta else A).astype(np.float64) @ (B.T if tb else B).astype(np.float64)
    C = gn.gemm(dev(A), dev(B), bool(ta), bool(tb))
    assert rel_err(host(C), ref) < FP32_TOL
    mag = np.abs(A.T if ta else A).astype(np.float64) @ np.abs(B.T if tb else B)
    bound = 2.0 ** (-20 if K <= 128 else -18)  # fp32 accumulation over K terms, elementwise
    assert np.all(np.abs(host(C) - ref) <= bound * mag + 1e-30)
    bf16_only = (rnd(A).T if ta else rnd(A)).astype(np.float64) @ (rnd(B).T if tb else rnd(B))
    if K >= 64:  # the bound separates the split from a bf16-only product
        assert rel_err(bf16_only, ref) > 10 * FP32_TOL


def test_gemm_fp32_two_segments_and_accumulate(gn):
    r = rng_(32)
    M, N, K0, K1 = 200, 136, 96, 260
    A0, A1 = (r.standard_normal((M, k)).astype(np.float32) for k in (K0, K1))
    B0, B1 = (r.standard_normal((k, N)).astype(np.float32) for k in (K0, K1))
    ref = A0.astype(np.float64) @ B0 + A1.astype(np.float64) @ B1
    C = gn.gemm(dev(A0), dev(B0), A1=dev(A1), B1=dev(B1))
    assert rel_err(host(C), ref) < FP32_TOL
    gn.gemm(dev(A0), dev(B0), C=C, accumulate=True)
    assert rel_err(host(C), ref + A0.astype(np.float64) @ B0) < FP32_TOL


def test_gemm_fp32_split_non_finite_and_tiny_operands(gn):
    """The documented limits of the fp32 matrix-core split (include/gn_bwd.h, gn_gemm): an inf
    in A makes its whole output row NaN (the split forms inf - inf) while every other row stays
    fp32-grade; operands scaled into the low normal range (1e-30) keep the relative bound; the
    small-product FMA path keeps IEEE inf."""
    r = rng_(35)
    M, N, K = 128, 128, 256  # k > 128: the split path
    A = r.standard_normal((M, K)).astype(np.float32)
    B = r.standard_normal((K, N)).astype(np.float32)
    A[3, 5] = np.inf
    C = host(gn.gemm(dev(A), dev(B)))
    assert np.all(np.isnan(C[3]))
    rest = np.arange(M) != 3
    ref = A[rest].astype(np.float64) @ B
    assert rel_err(C[rest], ref) < FP32_TOL
    At = (r.standard_normal((M, K)) * 1e-30).astype(np.float32)
    Ct = host(gn.gemm(dev(At), dev(B)))
    assert rel_err(Ct, At.astype(np.float64) @ B) < FP32_TOL
    # small-product path (k <= 128): IEEE inf, finite elsewhere
    As = r.standard_normal((16, 64)).astype(np.float32)
    As[2, 7] = np.inf
    Bs = np.abs(r.standard_normal((64, 8))).astype(np.float32) + 0.5
    Cs = host(gn.gemm(dev(As), dev(Bs)))
    assert np.all(np.isposinf(Cs[2])) and np.all(np.isfinite(np.delete(Cs, 2, axis=0)))


# Small fp32 products (k <= 128 and M*N*k <= 2^24) take a one-thread-per-output kernel with a
# sequential fp32 k loop; the shapes straddle both limits, so each pair runs on the two paths.
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
@pytest.mark.parametrize("shape", [(40, 52, 128), (40, 52, 129), (2048, 64, 128), (2048, 65, 128),
                                   (10, 256, 64), (64, 256, 10), (1, 1, 1)])
def test_gemm_fp32_small_path_edges(gn, ta, tb, shape):
    M, N, K = shape
    r = rng_(34)
    A = r.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = r.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    a = (A.T if ta else A).astype(np.float64)
    b = (B.T if tb else B).astype(np.float64)
    ref = a @ b
    C0 = r.standard_normal((M, N)).astype(np.float32)
    C = gn.gemm(dev(A), dev(B), bool(ta), bool(tb))
    mag = np.abs(a) @ np.abs(b)
    bound = 2.0 ** (-20 if K <= 128 else -18) * max(1, K // 64)
    assert np.all(np.abs(host(C) - ref) <= bound * mag + 1e-30)
    Cacc = dev(C0)
    gn.gemm(dev(A), dev(B), bool(ta), bool(tb), C=Cacc, accumulate=True)
    assert np.all(np.abs(host(Cacc) - (ref + C0)) <= bound * (mag + np.abs(C0)) + 1e-30)


@pytest.mark.parametrize("shape", [(64, 10, 256), (64, 256, 784), (128, 128, 100), (7, 33, 9),
                                   (128, 129, 3), (129, 10, 20)])
@pytest.mark.parametrize("with_dx", [True, False])
def test_linear_fp32_one_launch_matches_separate(gn, shape, with_dx):
    """An fp32 Linear backward small enough for one launch (batch <= 128, dX's k loop over
    the N outputs <= 128) against the launches it replaces (dX and dW as plain GEMMs, db as
    column sums): bit-identical, overwrite and accumulate.  (128, 129, 3) with dX and
    (129, 10, 20) are past the bounds and run the separate launches inside the entry too.
    Rows above 8 or K % 4 != 0, so the skinny path (batch <= 8) is not the one taken."""
    M, N, K = shape
    r = rng_(36)
    dY = dev(r.standard_normal((M, N)).astype(np.float32))
    X = dev(r.standard_normal((M, K)).astype(np.float32))
    W = dev(r.standard_normal((N, K)).astype(np.float32))
    dX, dW, db = gn.linear_bwd(dY, X, W, need_dx=with_dx, ws=False)
    assert torch.equal(dW, gn.gemm(dY, X, transA=True))
    assert torch.equal(db, gn.colsum(dY))
    if with_dx:
        assert torch.equal(dX, gn.gemm(dY, W))
    base = [dev(r.standard_normal(s).astype(np.float32)) for s in ((M, K), (N, K), (N,))]
    aX, aW, ab = [b.clone() for b in base]
    gn.linear_bwd(dY, X, W, need_dx=with_dx, dX=aX if with_dx else None, dW=aW, db=ab,
                  accumulate=True, ws=False)
    eX, eW, eb = [b.clone() for b in base]
    gn.gemm(dY, X, transA=True, C=eW, accumulate=True)
    gn.colsum(dY, out=eb, accumulate=True)
    assert torch.equal(aW, eW) and torch.equal(ab, eb)
    if with_dx:
        gn.gemm(dY, W, C=eX, accumulate=True)
        assert torch.equal(aX, eX)
    # and against fp64
    y, x, w = (host(t).astype(np.float64) for t in (dY, X, W))
    mag = np.abs(y).T @ np.abs(x)
    assert np.all(np.abs(host(dW) - y.T @ x) <= 2.0 ** -20 * mag + 1e-30)


@pytest.mark.parametrize("M", [1, 7, 64, 1024, 1025])
@pytest.mark.parametrize("N", [10, 300])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_colsum_few_and_many_rows(gn, M, N, dtype):
    """Column sums: up to 1024 rows in one deterministic pass (reruns bit-identical), more
    over row blocks; both against fp64 sums of the same (rounded) values, overwrite and
    accumulate."""
    r = rng_(35)
    x = r.standard_normal((M, N)).astype(np.float32)
    xd = dev(x, dtype)
    ref = host(xd).astype(np.float64).sum(axis=0)
    out = gn.colsum(xd)
    tol = 1e-6 * np.abs(host(xd)).astype(np.float64).sum(axis=0) + 1e-30
    assert np.all(np.abs(host(out) - ref) <= tol)
    if M <= 1024:
        assert torch.equal(out, gn.colsum(xd))
        if N % 4 == 0:
            # four columns per lane (N % 4 == 0, aligned rows) add exactly as one per lane
            for j in (0, 1, N // 2, N - 1):
                assert torch.equal(out[j:j + 1], gn.colsum(xd[:, j:j + 1].contiguous()))
    base = dev(r.standard_normal(N).astype(np.float32))
    acc = base.clone()
    gn.colsum(xd, out=acc, accumulate=True)
    assert np.all(np.abs(host(acc) - (ref + host(base))) <= tol + 1e-6 * np.abs(host(base)))


def test_linear_fp32_c1_first_layer(gn):
    """BASELINE configs[0]'s first Linear (784 -> 256, batch 64, fp32): dW1 [256 x 784] over 64
    rows and db1 on the MFMA path, dX on it too, against the oracle."""
    r = rng_(33)
    X = r.standard_normal((64, 784)).astype(np.float32)
    W = (r.standard_normal((256, 784)) * 0.05).astype(np.float32)
    dY = r.standard_normal((64, 256)).astype(np.float32)
    dX, dW, db = gn.linear_bwd(dev(dY), dev(X), dev(W))
    rdX, rdW, rdb = oracle.linear_bwd(dY, X, W)
    assert rel_err(host(dX), rdX) < FP32_TOL
    assert rel_err(host(dW), rdW) < FP32_TOL
    assert rel_err(host(db), rdb) < FP32_TOL


def test_linear_fp32_hypernetwork_shape(gn):
    """The hypernetwork's output Linear at batch 64 (1536 -> 163840 = K 16 x vsa 10240, fp32,
    W 1.0 GB): dX = dY W runs split-K (K = 163840) through the workspace, dW = dY^T X writes
    the 1 GB gradient.  Checked on samples against float64 (96 columns of dX, 512 rows of dW,
    all of db; normwise <= 1e-4) and bit-identical on a rerun (the planes are reduced in
    index order)."""
    M, N, K = 64, 163840, 1536
    assert gn.linear_workspace_bytes(M, N, K, 0) > 0  # the dX GEMM splits K
    g = torch.Generator(device="cuda:0")
    g.manual_seed(34)
    dY = torch.randn(M, N, device="cuda:0", generator=g)
    X = torch.randn(M, K, device="cuda:0", generator=g)
    W = torch.randn(N, K, device="cuda:0", generator=g) * 0.02
    dX, dW, db = gn.linear_bwd(dY, X, W)
    dX2, _, _ = gn.linear_bwd(dY, X, W, dW=torch.empty_like(dW))
    assert torch.equal(dX, dX2)
    r = rng_(35)
    cols = np.sort(r.choice(K, 96, replace=False))
    rows = np.sort(r.choice(N, 512, replace=False))
    hdY = dY.cpu().numpy().astype(np.float64)
    hX = X.cpu().numpy().astype(np.float64)
    ref_dx = hdY @ W[:, torch.from_numpy(cols).cuda()].cpu().numpy().astype(np.float64)
    assert rel_err(host(dX)[:, cols], ref_dx) < FP32_TOL
    ref_dw = hdY[:, rows].T @ hX
    assert rel_err(host(dW[torch.from_numpy(rows).cuda()]), ref_dw) < FP32_TOL
    assert rel_err(host(db), hdY.sum(axis=0)) < FP32_TOL


# ---------------------------------------------------------------------------- linear
def test_linear_fp32_golden(gn):
    for tag in ["small", "c1l2"]:
        g = golden(f"linear_{tag}")
        dX, dW, db = gn.linear_bwd(dev(g["dY"]), dev(g["X"]), dev(g["W"]))
        assert rel_err(host(dX), g["dX"]) < FP32_TOL
        assert rel_err(host(dW), g["dW"]) < FP32_TOL
        assert rel_err(host(db), g["db"]) < FP32_TOL


@pytest.mark.parametrize("M,N,K", [(256, 384, 320), (512, 256, 1024)])
def test_linear_bf16(gn, M, N, K):
    r = rng_(4)
    X = rnd(r.standard_normal((M, K)).astype(np.float32))
    W = rnd((r.standard_normal((N, K)) * 0.02).astype(np.float32))
    dY = rnd((r.standard_normal((M, N)) * 0.01).astype(np.float32))
    dX, dW, db = gn.linear_bwd(dev(dY, torch.bfloat16), dev(X, torch.bfloat16),
                               dev(W, torch.bfloat16))
    rX, rW, rb = oracle.linear_bwd(dY, X, W)
    assert dX.dtype == torch.bfloat16 and dW.dtype == torch.float32
    assert rel_err(host(dX), rX) < BF16_TOL
    assert rel_err(host(dW), rW) < 1e-4  # fp32 output of bf16 products: only summation order
    assert rel_err(host(db), rb) < 1e-4


@pytest.mark.parametrize("M,N,K", [(8192, 256, 256), (4096, 768, 512), (6144, 136, 200)])
def test_linear_split_k_weight_gradient(gn, M, N, K):
    """Long-K weight gradients with few output tiles take the two-way split-K path (fp32
    atomics onto a cleared dW): same values as the oracle, and bit-identical across runs."""
    r = rng_(14)
    dY = rnd(r.standard_normal((M, N)).astype(np.float32))
    X = rnd(r.standard_normal((M, K)).astype(np.float32))
    W = rnd(r.standard_normal((N, K)).astype(np.float32))
    tdY, tX, tW = dev(dY, torch.bfloat16), dev(X, torch.bfloat16), dev(W, torch.bfloat16)
    _, dW1, db = gn.linear_bwd(tdY, tX, tW)
    _, dW2, _ = gn.linear_bwd(tdY, tX, tW)
    _, rW, rb = oracle.linear_bwd(dY, X, W)
    assert rel_err(host(dW1), rW) < FP32_TOL
    assert rel_err(host(db), rb) < FP32_TOL
    assert torch.equal(dW1, dW2)


@pytest.mark.parametrize("M,N,K", [(8192, 768, 768), (8192, 768, 3072), (8192, 2304, 768)])
def test_linear_split_k_workspace(gn, M, N, K):
    """The decoder's under-filled weight gradients (O-proj, FFN down, QKV shapes) with the
    split-K workspace: partial planes reduced in a fixed order.  Against the oracle, bit-
    identical reruns, accumulation (which may take another split: two-way atomics need a
    cleared C), and without a workspace."""
    r = rng_(16)
    dY = rnd((r.standard_normal((M, N)) * 0.01).astype(np.float32))
    X = rnd(r.standard_normal((M, K)).astype(np.float32))
    W = rnd((r.standard_normal((N, K)) * 0.02).astype(np.float32))
    if (M, N, K) == (8192, 768, 768):
        assert gn.linear_workspace_bytes(M, N, K, 4) > 0  # this shape takes the split
    tdY, tX, tW = dev(dY, torch.bfloat16), dev(X, torch.bfloat16), dev(W, torch.bfloat16)
    _, dW1, db1 = gn.linear_bwd(tdY, tX, tW, need_dx=False)
    _, dW2, db2 = gn.linear_bwd(tdY, tX, tW, need_dx=False)
    _, rW, rb = oracle.linear_bwd(dY, X, W, need_dx=False)
    assert rel_err(host(dW1), rW) < FP32_TOL and rel_err(host(db1), rb) < FP32_TOL
    assert torch.equal(dW1, dW2) and torch.equal(db1, db2)
    dWa, dba = dW1.clone(), db1.clone()
    gn.linear_bwd(tdY, tX, tW, need_dx=False, dW=dWa, db=dba, accumulate=True)
    assert rel_err(host(dWa), 2 * rW) < FP32_TOL and rel_err(host(dba), 2 * rb) < FP32_TOL
    _, dW0, db0 = gn.linear_bwd(tdY, tX, tW, need_dx=False, ws=False)  # no workspace
    assert rel_err(host(dW0), rW) < FP32_TOL and rel_err(host(db0), rb) < FP32_TOL


def test_glu_linear_split_k_workspace(gn):
    """The decoder's GEGLU projection backward (8192 tokens, 768 -> 3072) with the split-K
    workspace: dWg / dWu / biases from partial planes against the path without a workspace
    (fp32 sums of the same bf16 products in another order), dX unchanged, reruns identical."""
    r = rng_(17)
    M, K, H = 8192, 768, 3072
    assert gn.glu_workspace_bytes(M, K, H, 4) > 0  # this shape takes the split
    b = torch.bfloat16
    X = dev(r.standard_normal((M, K)).astype(np.float32), b)
    Wg, Wu = (dev((r.standard_normal((H, K)) * 0.02).astype(np.float32), b) for _ in range(2))
    gate, up = (dev(r.standard_normal((M, H)).astype(np.float32), b) for _ in range(2))
    dO = dev((r.standard_normal((M, H)) * 0.01).astype(np.float32), b)
    args = ("geglu_up", dO, gate, up, X, Wg, Wu)
    ws1 = gn.glu_linear_bwd(*args, need_db=True)
    ws2 = gn.glu_linear_bwd(*args, need_db=True)
    plain = gn.glu_linear_bwd(*args, need_db=True, ws=False)
    assert torch.equal(ws1[0], plain[0])  # dX: same GEMM either way
    for a, c, p in zip(ws1[1:], ws2[1:], plain[1:]):
        assert torch.equal(a, c)
        assert rel_err(host(a), host(p)) < 1e-5


def test_linear_wide_tile_bias_sums(gn):
    """The decoder's gate/up weight-gradient shape (8192 rows, 6144 x 768) takes the 128 x 256
    tile, whose fused bias sums run on the VALU (narrower tiles use v_dot2): dW against an fp32
    BLAS product of the same bf16 values, db against float64 column sums, and bit-identical
    across runs."""
    r = rng_(15)
    M, N, K = 8192, 6144, 768
    dY = rnd((r.standard_normal((M, N)) * 0.01).astype(np.float32))
    X = rnd(r.standard_normal((M, K)).astype(np.float32))
    W = rnd((r.standard_normal((N, K)) * 0.02).astype(np.float32))
    tdY, tX, tW = dev(dY, torch.bfloat16), dev(X, torch.bfloat16), dev(W, torch.bfloat16)
    _, dW1, db1 = gn.linear_bwd(tdY, tX, tW, need_dx=False)
    _, dW2, db2 = gn.linear_bwd(tdY, tX, tW, need_dx=False)
    assert rel_err(host(dW1), dY.T @ X) < 1e-4
    assert rel_err(host(db1), dY.astype(np.float64).sum(axis=0)) < 1e-5
    assert torch.equal(dW1, dW2) and torch.equal(db1, db2)


def test_linear_no_dx_and_accumulate(gn):
    g = golden("linear_small")
    dY, X, W = dev(g["dY"]), dev(g["X"]), dev(g["W"])
    dX, dW, db = gn.linear_bwd(dY, X, W, need_dx=False)
    assert dX is None
    gn.linear_bwd(dY, X, W, need_dx=False, dW=dW, db=db, accumulate=True)
    assert rel_err(host(dW), 2 * g["dW"]) < FP32_TOL
    assert rel_err(host(db), 2 * g["db"]) < FP32_TOL


# ---------------------------------------------------------------------------- activations
@pytest.mark.parametrize("kind", ["relu", "gelu_tanh", "gelu_erf", "silu", "tanh", "sigmoid"])
def test_act_golden_fp32(gn, kind):
    g = golden("act")
    inp = g["Y_" + kind] if kind in ("tanh", "sigmoid") else g["X"]
    dX = gn.act_bwd(kind, dev(g["dY"]), dev(inp))
    assert rel_err(host(dX), g["dX_" + kind]) < FP32_TOL


@pytest.mark.parametrize("kind", ["relu", "gelu_tanh", "silu"])
@pytest.mark.parametrize("n", [4096 * 8 + 3, 1 << 20])
def test_act_bf16(gn, kind, n):
    r = rng_(5)
    X = rnd((r.standard_normal(n) * 3).astype(np.float32))
    dY = rnd(r.standard_normal(n).astype(np.float32))
    dX = gn.act_bwd(kind, dev(dY, torch.bfloat16), dev(X, torch.bfloat16))
    assert rel_err(host(dX), oracle.act_bwd(kind, dY, X)) < BF16_TOL
    gn.act_bwd(kind, dev(dY, torch.bfloat16), dev(X, torch.bfloat16), dX=dX, accumulate=True)
    assert rel_err(host(dX), 2 * oracle.act_bwd(kind, dY, X)) < BF16_TOL


# ---------------------------------------------------------------------------- GLU
@pytest.mark.parametrize("kind", ["swiglu_up", "swiglu_gate", "geglu_up", "geglu_gate", "reglu_up"])
def test_glu_golden_fp32(gn, kind):
    g = golden("glu")
    dG, dU = gn.glu_bwd(kind, dev(g["dO"]), dev(g["gate"]), dev(g["up"]))
    assert rel_err(host(dG), g["dGate_" + kind]) < FP32_TOL
    assert rel_err(host(dU), g["dUp_" + kind]) < FP32_TOL


@pytest.mark.parametrize("kind", ["swiglu_up", "geglu_up"])
def test_glu_linear_bf16(gn, kind):
    r = rng_(6)
    M, K, H = 192, 256, 320
    X = rnd(r.standard_normal((M, K)).astype(np.float32))
    Wg = rnd((r.standard_normal((H, K)) * 0.05).astype(np.float32))
    Wu = rnd((r.standard_normal((H, K)) * 0.05).astype(np.float32))
    gate, up = oracle.linear_fwd(X, Wg), oracle.linear_fwd(X, Wu)
    gate, up = rnd(gate), rnd(up)
    dO = rnd((r.standard_normal((M, H)) * 0.01).astype(np.float32))
    dX, dWg, dWu, dbg, dbu = gn.glu_linear_bwd(kind, dev(dO, torch.bfloat16),
                                               dev(gate, torch.bfloat16), dev(up, torch.bfloat16),
                                               dev(X, torch.bfloat16), dev(Wg, torch.bfloat16),
                                               dev(Wu, torch.bfloat16), need_db=True)
    dG, dU = oracle.glu_bwd(kind, dO, gate, up)
    rX = oracle.linear_bwd(dG, X, Wg)[0] + oracle.linear_bwd(dU, X, Wu)[0]
    assert rel_err(host(dX), rX) < BF16_TOL
    assert rel_err(host(dWg), oracle.linear_bwd(dG, X, Wg)[1]) < BF16_TOL
    assert rel_err(host(dWu), oracle.linear_bwd(dU, X, Wu)[1]) < BF16_TOL
    assert rel_err(host(dbg), dG.sum(0)) < BF16_TOL
    assert rel_err(host(dbu), dU.sum(0)) < BF16_TOL


@pytest.mark.parametrize("M,N,H", [(256, 192, 320), (136, 200, 96), (40, 64, 100)])
@pytest.mark.parametrize("kind", ["swiglu_up", "geglu_up", "reglu_up"])
def test_ffn_down_glu_fused(gn, M, N, H, kind):
    """gn_ffn_down_glu_bwd (GLU epilogue on dA = dY Wd) + gn_glu_proj_bwd against the
    unfused oracle chain; the shapes exercise the DMA, register-staged and SIMT GEMMs."""
    r = rng_(22)
    K = 128
    X = rnd(r.standard_normal((M, K)).astype(np.float32))
    Wg = rnd((r.standard_normal((H, K)) * 0.05).astype(np.float32))
    Wu = rnd((r.standard_normal((H, K)) * 0.05).astype(np.float32))
    gate, up = rnd(oracle.linear_fwd(X, Wg)), rnd(oracle.linear_fwd(X, Wu))
    A = rnd(oracle.glu_fwd(kind, gate, up))
    Wd = rnd((r.standard_normal((N, H)) * 0.05).astype(np.float32))
    dY = rnd((r.standard_normal((M, N)) * 0.01).astype(np.float32))
    b = torch.bfloat16
    gu, dWd, dbd = gn.ffn_down_glu_bwd(kind, dev(dY, b), dev(A, b), dev(Wd, b), dev(gate, b),
                                       dev(up, b), need_db=True)
    dA, rWd, rbd = oracle.linear_bwd(dY, A, Wd)
    dG, dU = oracle.glu_bwd(kind, dA, gate, up)
    hgu = host(gu)
    assert rel_err(hgu[:, :H], dG) < BF16_TOL and rel_err(hgu[:, H:], dU) < BF16_TOL
    assert rel_err(host(dWd), rWd) < 1e-4 and rel_err(host(dbd), rbd) < 1e-4
    dX, dWg, dWu, dbg, dbu = gn.glu_proj_bwd(gu, dev(X, b), dev(Wg, b), dev(Wu, b), need_db=True)
    gG, gU = hgu[:, :H], hgu[:, H:]
    assert rel_err(host(dX), oracle.linear_bwd(gG, X, Wg)[0] + oracle.linear_bwd(gU, X, Wu)[0]) < BF16_TOL
    assert rel_err(host(dWg), oracle.linear_bwd(gG, X, Wg)[1]) < 1e-4
    assert rel_err(host(dWu), oracle.linear_bwd(gU, X, Wu)[1]) < 1e-4
    assert rel_err(host(dbg), gG.sum(0)) < 1e-4 and rel_err(host(dbu), gU.sum(0)) < 1e-4


def test_ffn_down_glu_and_proj_with_workspace(gn):
    """The workspace forms (gn_ffn_down_glu_bwd_ws, gn_glu_proj_bwd_ws) at the C5 decoder's
    FFN shapes, where the weight gradients split K over fp32 planes: the GLU-epilogue GEMM and
    dX are bit-identical to the calls without a workspace (no split on them), the weight and
    bias gradients agree to fp32 rounding and match float64 on sampled rows."""
    import torch
    M, N, H, K = 8192, 768, 3072, 768
    g = torch.Generator(device="cuda:0").manual_seed(31)
    b = torch.bfloat16
    r = lambda *sh, s=1.0: (torch.randn(*sh, device="cuda:0", generator=g) * s).to(b)
    dY, A, Wd, gate, up = r(M, N, s=0.1), r(M, H), r(N, H, s=0.02), r(M, H), r(M, H)
    gu0, dWd0, dbd0 = gn.ffn_down_glu_bwd("geglu_up", dY, A, Wd, gate, up, need_db=True)
    gu1, dWd1, dbd1 = gn.ffn_down_glu_bwd("geglu_up", dY, A, Wd, gate, up, need_db=True, ws=None)
    X, Wg, Wu = r(M, K), r(H, K, s=0.02), r(H, K, s=0.02)
    p0 = gn.glu_proj_bwd(gu0, X, Wg, Wu, need_db=True)
    p1 = gn.glu_proj_bwd(gu0, X, Wg, Wu, need_db=True, ws=None)
    torch.cuda.synchronize()
    assert torch.equal(gu0, gu1) and torch.equal(p0[0], p1[0])
    for a0, a1 in ((dWd0, dWd1), (dbd0, dbd1)) + tuple(zip(p0[1:], p1[1:])):
        assert rel_err(a1.cpu().numpy(), a0.cpu().numpy()) < 1e-5
    rows = torch.tensor([0, N // 2, N - 1], device="cuda:0")
    ref = (dY.t()[rows].double() @ A.double()).cpu().numpy()
    assert rel_err(dWd1[rows].cpu().numpy(), ref) < 1e-5
    rows = torch.tensor([1, H - 1], device="cuda:0")
    ref = (gu0[:, H:].t()[rows].double() @ X.double()).cpu().numpy()
    assert rel_err(p1[2][rows].cpu().numpy(), ref) < 1e-5
    assert rel_err(dbd1.cpu().numpy(), dY.double().sum(0).cpu().numpy()) < 1e-5


# ---------------------------------------------------------------------------- norms
def test_layernorm_golden_fp32(gn):
    g = golden("layernorm")
    dX, dG, dB = gn.layernorm_bwd(dev(g["dY"]), dev(g["X"]), dev(g["gamma"]), dev(g["mean"]),
                                  dev(g["rstd"]))
    assert rel_err(host(dX), g["dX"]) < FP32_TOL
    assert rel_err(host(dG), g["dGamma"]) < FP32_TOL
    assert rel_err(host(dB), g["dBeta"]) < FP32_TOL
    dX2, _, _ = gn.layernorm_bwd(dev(g["dY"]), dev(g["X"]), dev(g["gamma"]), dev(g["mean"]),
                                 dev(g["var"]), eps=float(g["eps"]), stat_is_var=True)
    assert rel_err(host(dX2), g["dX"]) < FP32_TOL


@pytest.mark.parametrize("rows,F,dt", [(8192, 768, "bf16"), (1000, 2048, "f32"), (77, 4096, "bf16"),
                                       (33, 100, "f32"), (5, 6000, "bf16")])
def test_layernorm_shapes(gn, rows, F, dt):
    r = rng_(7)
    X = (r.standard_normal((rows, F)) * 2 + 0.3).astype(np.float32)
    gamma = (1 + 0.3 * r.standard_normal(F)).astype(np.float32)
    dY = r.standard_normal((rows, F)).astype(np.float32)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    if dt == "bf16":
        X, gamma, dY = rnd(X), rnd(gamma), rnd(dY)
    _, mean, rstd = oracle.layernorm_fwd(X, gamma)
    dX, dG, dB = gn.layernorm_bwd(dev(dY, tdt), dev(X, tdt), dev(gamma, tdt), dev(mean), dev(rstd))
    rX, rG, rB = oracle.layernorm_bwd(dY, X, gamma, mean, rstd)
    tol = BF16_TOL if dt == "bf16" else FP32_TOL
    assert rel_err(host(dX), rX) < tol
    assert rel_err(host(dG), rG) < FP32_TOL * 10
    assert rel_err(host(dB), rB) < FP32_TOL * 10


def test_rmsnorm_golden_fp32(gn):
    g = golden("rmsnorm")
    dX, dW = gn.rmsnorm_bwd(dev(g["dY"]), dev(g["X"]), dev(g["w"]), dev(g["rstd"]))
    assert rel_err(host(dX), g["dX"]) < FP32_TOL
    assert rel_err(host(dW), g["dW"]) < FP32_TOL


@pytest.mark.parametrize("rows,F", [(4096, 2048), (300, 768), (17, 50)])
def test_rmsnorm_bf16(gn, rows, F):
    r = rng_(8)
    X = rnd(r.standard_normal((rows, F)).astype(np.float32))
    w = rnd((1 + 0.2 * r.standard_normal(F)).astype(np.float32))
    dY = rnd((r.standard_normal((rows, F)) * 0.01).astype(np.float32))
    _, rstd = oracle.rmsnorm_fwd(X, w)
    dX, dW = gn.rmsnorm_bwd(dev(dY, torch.bfloat16), dev(X, torch.bfloat16),
                            dev(w, torch.bfloat16), dev(rstd))
    rX, rW = oracle.rmsnorm_bwd(dY, X, w, rstd)
    assert rel_err(host(dX), rX) < BF16_TOL
    assert rel_err(host(dW), rW) < 1e-3


@pytest.mark.parametrize("rows,F", [(8192, 768), (300, 2048), (77, 3000)])
@pytest.mark.parametrize("kind", ["layernorm", "rmsnorm"])
def test_norm_bwd_fp32_stream_with_addend(gn, rows, F, kind):
    """x, dX and the addend in fp32 under bf16 dy / gamma (the _ex entries), and the addend
    summed in the same pass: dX = norm_grad(dy) + add, in place (add = dX) too."""
    r = rng_(71)
    X = (r.standard_normal((rows, F)) * 2 + 0.3).astype(np.float32)
    g = rnd((1 + 0.3 * r.standard_normal(F)).astype(np.float32))
    dY = rnd((r.standard_normal((rows, F)) * 0.1).astype(np.float32))
    add = r.standard_normal((rows, F)).astype(np.float32)
    if kind == "layernorm":
        _, mean, rstd = oracle.layernorm_fwd(X, g)
        rX, rG, rB = oracle.layernorm_bwd(dY, X, g, mean, rstd)
        dX, dG, dB = gn.layernorm_bwd(dev(dY, torch.bfloat16), dev(X), dev(g, torch.bfloat16),
                                      dev(mean), dev(rstd), dX_add=dev(add))
        assert rel_err(host(dB), rB) < FP32_TOL
    else:
        _, rstd = oracle.rmsnorm_fwd(X, g)
        rX, rG = oracle.rmsnorm_bwd(dY, X, g, rstd)
        dX, dG = gn.rmsnorm_bwd(dev(dY, torch.bfloat16), dev(X), dev(g, torch.bfloat16), dev(rstd),
                                dX_add=dev(add))
    assert dX.dtype == torch.float32
    assert rel_err(host(dX), rX + add) < FP32_TOL
    assert rel_err(host(dG), rG) < FP32_TOL
    # in place: the addend is the output buffer itself
    buf = dev(add)
    if kind == "layernorm":
        gn.layernorm_bwd(dev(dY, torch.bfloat16), dev(X), dev(g, torch.bfloat16), dev(mean),
                         dev(rstd), dX_add=buf, out=buf)
    else:
        gn.rmsnorm_bwd(dev(dY, torch.bfloat16), dev(X), dev(g, torch.bfloat16), dev(rstd),
                       dX=buf, dX_add=buf)
    assert rel_err(host(buf), rX + add) < FP32_TOL


@pytest.mark.parametrize("rows,F,with_add", [(8192, 768, True), (300, 2048, False), (77, 3000, True),
                                            (64, 100, True)])
def test_layernorm_bwd_bf16_copy_of_dx(gn, rows, F, with_add):
    """gn_layernorm_bwd_ex16: the bf16 copy written in the norm's pass equals dX rounded by
    torch (round to nearest even), and dX, dGamma, dBeta equal the _ex entry's bit for bit
    (F = 100: the generic path, the copy by a conversion pass)."""
    r = rng_(73)
    X = (r.standard_normal((rows, F)) * 2 + 0.3).astype(np.float32)
    g = rnd((1 + 0.3 * r.standard_normal(F)).astype(np.float32))
    dY = rnd((r.standard_normal((rows, F)) * 0.1).astype(np.float32))
    add = dev(r.standard_normal((rows, F)).astype(np.float32)) if with_add else None
    _, mean, rstd = oracle.layernorm_fwd(X, g)
    args = (dev(dY, torch.bfloat16), dev(X), dev(g, torch.bfloat16), dev(mean), dev(rstd))
    c16 = torch.empty((rows, F), dtype=torch.bfloat16, device="cuda:0")
    dX, dG, dB = gn.layernorm_bwd(*args, dX_add=add, dX_bf16=c16)
    dX1, dG1, dB1 = gn.layernorm_bwd(*args, dX_add=add if with_add else torch.zeros_like(dX))
    torch.cuda.synchronize()
    assert torch.equal(dX, dX1) and torch.equal(dG, dG1) and torch.equal(dB, dB1)
    assert torch.equal(c16, dX.to(torch.bfloat16))
    rX, _, _ = oracle.layernorm_bwd(dY, X, g, mean, rstd)
    ref = rX + (host(add) if with_add else 0.0)
    assert rel_err(host(dX), ref) < FP32_TOL


def test_norm_deferred_parameter_finish(gn):
    """GN_NORM_PARTIALS + gn_norm_finish: a LayerNorm and an RMSNorm backward whose parameter
    gradients are summed later in one launch give the immediate calls' dX and parameter
    gradients bit for bit (accumulating form included); a shape off the row-kernel path is
    refused before any launch."""
    r = rng_(74)
    L, P, s = gn.lib(), gn._ptr, gn._stream()
    rows, F = 8192, 768
    X = dev((r.standard_normal((rows, F)) * 2 + 0.3).astype(np.float32))
    g = dev((1 + 0.3 * r.standard_normal(F)).astype(np.float32), torch.bfloat16)
    dY = dev((r.standard_normal((rows, F)) * 0.1).astype(np.float32), torch.bfloat16)
    _, mean, rstd = oracle.layernorm_fwd(host(X), host(g))
    mean, rstd = dev(mean), dev(rstd)
    dX0, dG0, dB0 = gn.layernorm_bwd(dY, X, g, mean, rstd, dX_add=torch.zeros_like(X))
    rows2, F2 = 4096, 2048
    X2 = dev(r.standard_normal((rows2, F2)).astype(np.float32), torch.bfloat16)
    w2 = dev((1 + 0.2 * r.standard_normal(F2)).astype(np.float32), torch.bfloat16)
    dY2 = dev((r.standard_normal((rows2, F2)) * 0.1).astype(np.float32), torch.bfloat16)
    _, rs2 = oracle.rmsnorm_fwd(host(X2), host(w2))
    rs2 = dev(rs2)
    dX20, dW20 = gn.rmsnorm_bwd(dY2, X2, w2, rs2)
    # deferred: both partial sets stay in their workspaces until one finish
    ws1 = gn.workspace(gn.norm_workspace_bytes(rows, F), X.device)
    ws2 = gn.workspace(gn.norm_workspace_bytes(rows2, F2), X.device)
    dX, dG, dB = torch.empty_like(X), torch.full((F,), 7.0, device="cuda:0"), torch.full((F,), 7.0, device="cuda:0")
    dX2, dW2 = torch.empty_like(X2), torch.full((F2,), 7.0, device="cuda:0")
    gn._check(L.gn_layernorm_bwd_ex(P(dY), gn.BF16, P(X), gn.F32, P(g), P(mean), P(rstd), None, P(dX),
                                    P(dG), P(dB), rows, F, 1e-5, gn.NORM_PARTIALS, P(ws1), ws1.numel(), s),
              "layernorm deferred")
    gn._check(L.gn_rmsnorm_bwd_ex(P(dY2), gn.BF16, P(X2), gn.BF16, P(w2), P(rs2), None, P(dX2), P(dW2),
                                  rows2, F2, gn.NORM_PARTIALS, P(ws2), ws2.numel(), s), "rmsnorm deferred")
    torch.cuda.synchronize()
    assert torch.all(dG == 7.0) and torch.all(dW2 == 7.0)  # not written before the finish
    gn.norm_finish([(ws1, dG, dB, rows, F, True, False), (ws2, dW2, None, rows2, F2, False, False)])
    torch.cuda.synchronize()
    assert torch.equal(dX, dX0) and torch.equal(dX2, dX20)
    assert torch.equal(dG, dG0) and torch.equal(dB, dB0) and torch.equal(dW2, dW20)
    # accumulating finish: onto the values already there
    gn.norm_finish([(ws1, dG, dB, rows, F, True, True)])
    torch.cuda.synchronize()
    assert torch.equal(dG, dG0 + dG0) and torch.equal(dB, dB0 + dB0)
    # F = 100 takes the generic path: refused
    Xs = dev(r.standard_normal((64, 100)).astype(np.float32))
    with pytest.raises(gn.GnError):
        gn._check(L.gn_layernorm_bwd_ex(P(Xs), gn.F32, P(Xs), gn.F32, P(Xs[0]), P(Xs[:, 0].contiguous()),
                                        P(Xs[:, 1].contiguous()), None, P(torch.empty_like(Xs)),
                                        P(Xs[1]), P(Xs[2]), 64, 100, 1e-5, gn.NORM_PARTIALS, P(ws1),
                                        ws1.numel(), s), "layernorm deferred (generic)")


@pytest.mark.parametrize("rows,F", [(4096, 768), (50, 3000)])
def test_norm_fwd_fp32_stream_to_bf16(gn, rows, F):
    r = rng_(72)
    X = (r.standard_normal((rows, F)) * 3 - 1).astype(np.float32)
    g = rnd((1 + 0.2 * r.standard_normal(F)).astype(np.float32))
    b = rnd((0.1 * r.standard_normal(F)).astype(np.float32))
    Y, mean, rstd = gn.layernorm_fwd(dev(X), dev(g, torch.bfloat16), dev(b, torch.bfloat16),
                                     out_dtype=torch.bfloat16)
    rY, rm, rr = oracle.layernorm_fwd(X, g, b)
    assert Y.dtype == torch.bfloat16 and rel_err(host(Y), rY) < 1e-2
    assert rel_err(host(mean), rm) < 1e-5 and rel_err(host(rstd), rr) < 1e-5
    Yr, rs = gn.rmsnorm_fwd(dev(X), dev(g, torch.bfloat16), out_dtype=torch.bfloat16)
    rYr, rrs = oracle.rmsnorm_fwd(X, g)
    assert rel_err(host(Yr), rYr) < 1e-2 and rel_err(host(rs), rrs) < 1e-5


def test_convert_f32_bf16(gn):
    r = rng_(73)
    for n in (1 << 20, 1001):
        x = torch.from_numpy((r.standard_normal(n) * 100).astype(np.float32)).cuda()
        x[:4] = torch.tensor([1 + 2 ** -8, 1 + 3 * 2 ** -8, float("inf"), -0.0])  # ties, inf, -0
        b = gn.convert(x, torch.bfloat16)
        assert torch.equal(b, x.bfloat16())  # round to nearest-even, as torch
        assert torch.equal(gn.convert(b, torch.float32), b.float())  # widening is exact


# ---------------------------------------------------------------------------- softmax / CE
def test_softmax_and_xent_golden(gn):
    g = golden("softmax")
    assert rel_err(host(gn.softmax_bwd(dev(g["dY"]), dev(g["Y"]))), g["dX"]) < FP32_TOL
    g = golden("xent")
    dL = gn.xent_bwd(dev(g["logits"]), torch.from_numpy(g["targets"]).cuda(), 1.0)
    assert rel_err(host(dL), g["dLogits"]) < FP32_TOL


@pytest.mark.parametrize("C", [1024, 2048, 4096])
def test_softmax_bwd_bf16_attention_widths(gn, C):
    """Softmax backward on bf16 probability rows as wide as an attention score row (S = 1024 to
    4096 keys; causal rows carry exact zeros past the diagonal), against the oracle on the same
    bf16-rounded inputs (normwise 2e-2)."""
    r = rng_(C)
    rows = 256
    s = (r.standard_normal((rows, C)) * 3).astype(np.float32)
    s[np.triu_indices(rows, 1)[0], np.triu_indices(rows, 1)[1]] = -np.inf  # causal prefix rows
    p = np.exp(s - s.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    Y = dev(p, torch.bfloat16)
    dY = dev(r.standard_normal((rows, C)).astype(np.float32), torch.bfloat16)
    got = host(gn.softmax_bwd(dY, Y))
    want = oracle.softmax_bwd(host(dY), host(Y))
    assert rel_err(got, want) < BF16_TOL
    assert np.all(got[np.triu_indices(rows, 1)] == 0)  # masked keys get no gradient


def test_xent_vocab_bf16(gn):
    r = rng_(9)
    rows, C = 64, 32000
    Z = rnd((r.standard_normal((rows, C)) * 2).astype(np.float32))
    t = r.integers(0, C, size=rows).astype(np.int32)
    dL = gn.xent_bwd(dev(Z, torch.bfloat16), torch.from_numpy(t).cuda(), 1.0 / rows)
    assert rel_err(host(dL), oracle.xent_bwd(Z, t, 1.0 / rows)) < BF16_TOL


# ---------------------------------------------------------------------------- attention
@pytest.mark.parametrize("tag", ["causal_rope", "full_norope", "causal_half"])
def test_attention_golden_fp32(gn, tag):
    g = golden(f"attn_{tag}")
    kw = dict(scale=float(g["scale"]), causal=bool(g["causal"]), rope=str(g["rope"]),
              theta=float(g["theta"]))
    O, LSE = gn.attn_fwd(dev(g["Q"]), dev(g["K"]), dev(g["V"]), **kw)
    assert rel_err(host(O), g["O"]) < FP32_TOL and rel_err(host(LSE), g["LSE"]) < FP32_TOL
    dQ, dK, dV = gn.attn_bwd(dev(g["Q"]), dev(g["K"]), dev(g["V"]), dev(g["O"]), dev(g["dO"]),
                             dev(g["LSE"]), **kw)
    assert rel_err(host(dQ), g["dQ"]) < FP32_TOL
    assert rel_err(host(dK), g["dK"]) < FP32_TOL
    assert rel_err(host(dV), g["dV"]) < FP32_TOL


@pytest.mark.parametrize("S,D,causal,rope", [(256, 128, True, "interleaved"), (130, 64, True, "interleaved"),
                                             (192, 128, False, "none"), (128, 128, True, "half")])
def test_attention_bf16_mfma(gn, S, D, causal, rope):
    r = rng_(10)
    B, H = 2, 3
    Q, K, V = (rnd(r.standard_normal((B, H, S, D)).astype(np.float32)) for _ in range(3))
    dO = rnd((r.standard_normal((B, H, S, D)) * 0.01).astype(np.float32))
    kw = dict(causal=causal, rope_mode=rope)
    O, LSE = oracle.attn_fwd(Q, K, V, **kw)
    O = rnd(O)
    rQ, rK, rV = oracle.attn_bwd(Q, K, V, dO, LSE, **kw)
    dQ, dK, dV = gn.attn_bwd(dev(Q, torch.bfloat16), dev(K, torch.bfloat16), dev(V, torch.bfloat16),
                             dev(O, torch.bfloat16), dev(dO, torch.bfloat16), dev(LSE),
                             causal=causal, rope=rope)
    assert rel_err(host(dV), rV) < BF16_TOL
    assert rel_err(host(dQ), rQ) < BF16_TOL
    assert rel_err(host(dK), rK) < BF16_TOL


def test_attention_bf16_offset_views(gn):
    """Views that start one bf16 element into their storage are not 16-byte aligned: the MFMA
    kernels (16-byte LDS DMA and stores) must not see them; the SIMT path gives the answer."""
    r = rng_(13)
    B, H, S, D = 1, 2, 96, 64
    Q, K, V = (rnd(r.standard_normal((B, H, S, D)).astype(np.float32)) for _ in range(3))
    dO = rnd((r.standard_normal((B, H, S, D)) * 0.01).astype(np.float32))
    O, LSE = oracle.attn_fwd(Q, K, V, causal=True, rope_mode="interleaved")
    O = rnd(O)
    rQ, rK, rV = oracle.attn_bwd(Q, K, V, dO, LSE, causal=True, rope_mode="interleaved")

    def off(x):
        flat = torch.zeros(x.size + 1, dtype=torch.bfloat16, device="cuda")
        v = flat[1:].view(B, H, S, D)
        v.copy_(dev(x, torch.bfloat16))
        return v

    outs = tuple(off(np.zeros_like(Q)) for _ in range(3))
    dQ, dK, dV = gn.attn_bwd(off(Q), off(K), off(V), off(O), off(dO), dev(LSE), causal=True,
                             rope="interleaved", out=outs)
    assert all(t.data_ptr() % 16 == 2 for t in (dQ, dK, dV))
    assert rel_err(host(dV), rV) < BF16_TOL
    assert rel_err(host(dQ), rQ) < BF16_TOL
    assert rel_err(host(dK), rK) < BF16_TOL


@pytest.mark.parametrize("S,D,rope", [(200, 64, "none"), (256, 128, "interleaved"), (96, 64, "half")])
def test_attention_fused_qkv_layout(gn, S, D, rope):
    """[B,S,H,D] rows of a fused QKV buffer in, dQKV in the same layout out; equals the
    [B,H,S,D] oracle after the head permutation."""
    r = rng_(12)
    B, H = 2, 3
    Q, K, V = (rnd(r.standard_normal((B, H, S, D)).astype(np.float32)) for _ in range(3))
    dO = rnd((r.standard_normal((B, H, S, D)) * 0.01).astype(np.float32))
    O, LSE = oracle.attn_fwd(Q, K, V, causal=True, rope_mode=rope)
    O = rnd(O)
    rQ, rK, rV = oracle.attn_bwd(Q, K, V, dO, LSE, causal=True, rope_mode=rope)
    bshd = lambda t: np.ascontiguousarray(t.transpose(0, 2, 1, 3).reshape(B, S, H * D))
    qkv = np.concatenate([bshd(Q), bshd(K), bshd(V)], axis=-1)
    dqkv = gn.attn_bwd_qkv(dev(qkv, torch.bfloat16), dev(bshd(O), torch.bfloat16),
                           dev(bshd(dO), torch.bfloat16), dev(LSE), H, causal=True, rope=rope)
    got = host(dqkv).reshape(B, S, 3, H, D).transpose(2, 0, 3, 1, 4)  # [3, B, H, S, D]
    assert rel_err(got[0], rQ) < BF16_TOL
    assert rel_err(got[1], rK) < BF16_TOL
    assert rel_err(got[2], rV) < BF16_TOL


def test_attention_fused_qkv_rejects_bad_layouts(gn):
    z = torch.zeros(1, 64, 3 * 2 * 64, dtype=torch.bfloat16, device="cuda")
    o = torch.zeros(1, 64, 2 * 64, dtype=torch.bfloat16, device="cuda")
    lse = torch.zeros(1, 2, 64, device="cuda")
    with pytest.raises(gn.GnError):
        gn.attn_bwd_qkv(z.float(), o.float(), o.float(), lse, 2)  # fp32: bf16 only
    L = gn.lib()
    ws = gn.workspace(gn.attn_workspace_bytes(1, 2, 64, 64), z.device)
    zp, op_, lp = z.data_ptr(), o.data_ptr(), lse.data_ptr()
    args = lambda ld, off: (zp, zp + 256, zp + 512, op_, op_, lp, zp + off, zp + 256, zp + 512,
                            1, 2, 64, 64, ld, 128, 384, 0.125, 1, 0, 1e4, gn.BF16,
                            ws.data_ptr(), ws.numel(), gn._stream())
    assert L.gn_attn_bwd_bshd(*args(120, 0)) == -1  # row stride below H*D
    assert L.gn_attn_bwd_bshd(*args(384, 8)) == -1  # dQ not 16-byte aligned
    torch.cuda.synchronize()


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_embedding_scatter_add(gn, dt):
    """dE[ids[t]] += dX[t]: repeated ids sum, ids outside [0, V) are skipped, and
    GN_ACCUMULATE adds onto an existing gradient (the tied LM head's)."""
    r = rng_(13)
    T_, d, V = 1000, 96, 50
    dX = r.standard_normal((T_, d)).astype(np.float32)
    if dt == "bf16":
        dX = rnd(dX)
    ids = r.integers(0, V, size=T_).astype(np.int32)
    ids[::97] = -1
    ids[5] = V + 3
    want = np.zeros((V, d), np.float64)
    ok = (ids >= 0) & (ids < V)
    np.add.at(want, ids[ok], dX[ok].astype(np.float64))
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    tids = torch.from_numpy(ids).cuda()
    dE = gn.embedding_bwd(dev(dX, tdt), tids, V)
    assert rel_err(host(dE), want) < FP32_TOL
    base = r.standard_normal((V, d)).astype(np.float32)
    dE2 = gn.embedding_bwd(dev(dX, tdt), tids, V, dE=dev(base), accumulate=True)
    assert rel_err(host(dE2), want + base) < FP32_TOL


@pytest.mark.parametrize("B,H,S,D,causal,rope", [(1, 2, 96, 64, True, "interleaved"),
                                                 (2, 3, 200, 128, True, "none"),
                                                 (1, 2, 130, 128, False, "half"),
                                                 (1, 1, 64, 64, False, "none"),
                                                 (1, 2, 257, 64, True, "none")])
def test_attention_fwd_bf16_matches_oracle(gn, B, H, S, D, causal, rope):
    """MFMA forward (D 64/128; ragged S, both masks, all RoPE modes) against the oracle: O to
    the bf16 tolerance, the natural-log row LSE to 1e-3, and the LSE consistent with O's
    own normalisation (the backward recomputes P from it)."""
    r = rng_(11)
    Q, K, V = (rnd(r.standard_normal((B, H, S, D)).astype(np.float32)) for _ in range(3))
    O, LSE = gn.attn_fwd(dev(Q, torch.bfloat16), dev(K, torch.bfloat16), dev(V, torch.bfloat16),
                         causal=causal, rope=rope)
    rO, rL = oracle.attn_fwd(Q, K, V, causal=causal, rope_mode=rope)
    assert rel_err(host(O), rO) < BF16_TOL and rel_err(host(LSE), rL) < 1e-3


def test_attention_fwd_then_bwd_round_trip(gn):
    """The backward run on the MFMA forward's own O and LSE matches the oracle backward."""
    r = rng_(12)
    B, H, S, D = 1, 2, 192, 128
    Q, K, V = (rnd(r.standard_normal((B, H, S, D)).astype(np.float32)) for _ in range(3))
    dO = rnd((r.standard_normal((B, H, S, D)) * 0.01).astype(np.float32))
    bf = torch.bfloat16
    O, LSE = gn.attn_fwd(dev(Q, bf), dev(K, bf), dev(V, bf))
    dQ, dK, dV = gn.attn_bwd(dev(Q, bf), dev(K, bf), dev(V, bf), O, dev(dO, bf), LSE)
    _, rL = oracle.attn_fwd(Q, K, V)
    rQ, rK, rV = oracle.attn_bwd(Q, K, V, dO, rL)
    assert rel_err(host(dQ), rQ) < BF16_TOL and rel_err(host(dK), rK) < BF16_TOL
    assert rel_err(host(dV), rV) < BF16_TOL


# ---------------------------------------------------------------------------- VSA
def test_vsa_project_golden(gn):
    g = golden("vsa_project")
    D = g["W"].shape[1]
    bits = gn.u32_tensor(g["bits"], "cuda:0")
    dW, db = gn.vsa_unpack_project_bwd(dev(g["dY"]), bits, D)
    assert rel_err(host(dW), g["dW"]) < FP32_TOL and rel_err(host(db), g["db"]) < FP32_TOL


def test_vsa_project_popcount_exact(gn):
    # integer dY: every partial sum is an exactly representable integer, so the GPU result
    # must equal 2 * popcount - B bit for bit (pins the unpack order)
    r = rng_(12)
    Bn, O, D = 1000, 64, 2048
    bits = r.integers(0, 2**32, size=(Bn, D // 32), dtype=np.uint64).astype(np.uint32)
    dW, _ = gn.vsa_unpack_project_bwd(dev(np.ones((Bn, O), np.float32)), gn.u32_tensor(bits, "cuda:0"), D)
    pop = np.unpackbits(bits.view(np.uint8), axis=1, bitorder="little").sum(0).astype(np.int64)
    np.testing.assert_array_equal(host(dW), np.tile(2 * pop - Bn, (O, 1)).astype(np.float32))


@pytest.mark.parametrize("Bn,O,D", [(512, 768, 1024), (333, 128, 320)])
def test_vsa_project_fp32_split(gn, Bn, O, D):
    r = rng_(13)
    bits = r.integers(0, 2**32, size=(Bn, D // 32), dtype=np.uint64).astype(np.uint32)
    dY = r.standard_normal((Bn, O)).astype(np.float32)
    dW, db = gn.vsa_unpack_project_bwd(dev(dY), gn.u32_tensor(bits, "cuda:0"), D)
    rW, rb = oracle.vsa_unpack_project_bwd(dY, bits, D)
    assert rel_err(host(dW), rW) < FP32_TOL
    assert rel_err(host(db), rb) < FP32_TOL


@pytest.mark.parametrize("dtype,D", [(torch.float32, 1280), (torch.bfloat16, 1280), (torch.float32, 1152)])
def test_vsa_project_mfma_path_popcount_exact(gn, dtype, D):
    # shapes on the MFMA-DMA path (Bn % 64, D % 128; D = 1152 takes the 128-column tiles),
    # an O that leaves a partial 256-row tile, and bit rows padded past D/32 words: dW must
    # equal 2 * popcount - Bn exactly
    r = rng_(21)
    Bn, O, words = 1024, 264, D // 32 + 4
    bits = r.integers(0, 2**32, size=(Bn, words), dtype=np.uint64).astype(np.uint32)
    dW, db = gn.vsa_unpack_project_bwd(dev(np.ones((Bn, O), np.float32), dtype),
                                       gn.u32_tensor(bits, "cuda:0"), D)
    pop = np.unpackbits(bits[:, :D // 32].view(np.uint8), axis=1, bitorder="little").sum(0).astype(np.int64)
    np.testing.assert_array_equal(host(dW), np.tile(2 * pop - Bn, (O, 1)).astype(np.float32))
    np.testing.assert_array_equal(host(db), np.full(O, Bn, np.float32))


@pytest.mark.parametrize("accumulate", [False, True])
def test_vsa_project_mfma_path_fp32(gn, accumulate):
    r = rng_(22)
    Bn, O, D = 2048, 771, 2048  # O: a partial last row tile, not a multiple of 8
    bits = r.integers(0, 2**32, size=(Bn, D // 32), dtype=np.uint64).astype(np.uint32)
    dY = r.standard_normal((Bn, O)).astype(np.float32)
    init = r.standard_normal((O, D)).astype(np.float32)
    dW = dev(init) if accumulate else None
    dW, db = gn.vsa_unpack_project_bwd(dev(dY), gn.u32_tensor(bits, "cuda:0"), D, dW=dW,
                                       accumulate=accumulate)
    rW, rb = oracle.vsa_unpack_project_bwd(dY, bits, D)
    assert rel_err(host(dW), rW + (init if accumulate else 0)) < FP32_TOL
    # the LDS-staging kernel (no workspace) agrees with the MFMA-DMA path
    fW, _ = gn.vsa_unpack_project_bwd(dev(dY), gn.u32_tensor(bits, "cuda:0"), D, ws=False)
    assert rel_err(host(fW), rW) < FP32_TOL
    if not accumulate:
        assert rel_err(host(dW), host(fW)) < FP32_TOL
        # two segments onto a cleared output: the result is bitwise reproducible
        dW2, _ = gn.vsa_unpack_project_bwd(dev(dY), gn.u32_tensor(bits, "cuda:0"), D)
        assert torch.equal(dW, dW2)


def test_vsa_project_mfma_path_bf16(gn):
    r = rng_(23)
    Bn, O, D = 1024, 512, 1024
    bits = r.integers(0, 2**32, size=(Bn, D // 32), dtype=np.uint64).astype(np.uint32)
    dY = rnd(r.standard_normal((Bn, O)).astype(np.float32))  # values exact in bf16
    dW, db = gn.vsa_unpack_project_bwd(dev(dY, torch.bfloat16), gn.u32_tensor(bits, "cuda:0"), D)
    rW, rb = oracle.vsa_unpack_project_bwd(dY, bits, D)
    assert rel_err(host(dW), rW) < FP32_TOL and rel_err(host(db), rb) < FP32_TOL


def test_vsa_surrogate_golden_and_random(gn):
    g = golden("vsa_surrogate")
    dP = gn.vsa_surrogate_bwd(dev(g["preds"]), gn.u32_tensor(g["bits"], "cuda:0"),
                              gn.u32_tensor(g["results"], "cuda:0"), dev(g["weights"]),
                              float(g["gamma"]), float(g["delta"]), float(g["lambda_c"]),
                              float(g["scale"]))
    assert rel_err(host(dP), g["dPreds"]) < 1e-6
    r = rng_(14)
    Bn, K, D = 64, 4, 10240
    preds = r.standard_normal((Bn, K, D)).astype(np.float32)
    bits = r.integers(0, 2**32, size=(Bn, D // 32), dtype=np.uint64).astype(np.uint32)
    res, w = oracle.vsa_results_weights(oracle.vsa_dots(preds, bits), rng=r)
    dP = gn.vsa_surrogate_bwd(dev(preds), gn.u32_tensor(bits, "cuda:0"), gn.u32_tensor(res, "cuda:0"),
                              dev(w))
    ref = oracle.vsa_surrogate_bwd(preds, bits, res, w)
    assert rel_err(host(dP), ref) < 1e-6
    init = r.standard_normal((Bn, K, D)).astype(np.float32)
    dP = gn.vsa_surrogate_bwd(dev(preds), gn.u32_tensor(bits, "cuda:0"), gn.u32_tensor(res, "cuda:0"),
                              dev(w), dPreds=dev(init), accumulate=True)
    assert rel_err(host(dP), oracle.vsa_surrogate_bwd(preds, bits, res, w, init=init)) < 1e-6


def test_add_inplace(gn):
    a = torch.randn(1001, device="cuda:0")
    b = torch.randn(1001, device="cuda:0")
    ref = (a + b).cpu()
    gn.add_inplace(a, b)
    assert torch.equal(a.cpu(), ref)


def test_errors_are_reported(gn):
    x = torch.zeros(4, device="cuda:0")
    rc = gn.lib().gn_act_bwd(99, gn._ptr(x), gn._ptr(x), gn._ptr(x), 4, gn.F32, 0, None)
    assert rc == -1 and "unknown activation" in gn.last_error()
    with pytest.raises(gn.GnError, match="workspace"):
        X = torch.zeros((8, 16), device="cuda:0")
        gn.rmsnorm_bwd(X, X, torch.ones(16, device="cuda:0"), torch.ones(8, device="cuda:0"),
                       ws=torch.empty(1, dtype=torch.uint8, device="cuda:0"))


# ---------------------------------------------------------------------------- optimizers
def _opt_tensors(r, sizes, offset=0):
    """fp32 tensors of the given sizes; offset > 0 makes every tensor a view that starts
    `offset` floats into its storage (misaligned for 16-byte vectors)."""
    def mk(a):
        full = torch.zeros(a.size + offset, device="cuda:0")
        full[offset:] = torch.from_numpy(a.astype(np.float32)).to("cuda:0")
        return full[offset:]
    return [mk(r.standard_normal(n)) for n in sizes]


@pytest.mark.parametrize("offset", [0, 1])
def test_adamw_step_multi_tensor(gn, offset):
    """gn_adamw_step over 30 tensors (two launches of at most 24), ragged sizes (n % 4 != 0)
    and, with offset 1, misaligned storage (scalar path); three steps against the oracle."""
    r = rng_(40)
    sizes = [1, 3, 4, 5, 255, 2049, 4096 + 7] + [int(x) for x in r.integers(1, 3000, 23)]
    W = _opt_tensors(r, sizes, offset)
    m = [torch.zeros_like(w) for w in W]
    v = [torch.zeros_like(w) for w in W]
    W_lp = [torch.empty(w.numel(), dtype=torch.bfloat16, device="cuda:0") for w in W]
    hW, hm, hv = [w.cpu().numpy() for w in W], [np.zeros(n, np.float32) for n in sizes], \
        [np.zeros(n, np.float32) for n in sizes]
    kw = dict(lr=2e-3, beta1=0.9, beta2=0.99, eps=1e-6, weight_decay=0.05)
    for step in range(1, 4):
        G = _opt_tensors(r, sizes, offset)
        hG = [g.cpu().numpy() for g in G]
        gn.adamw_step([dict(W=w, grad=g, state0=a, state1=b, W_bf16=lp)
                       for w, g, a, b, lp in zip(W, G, m, v, W_lp)], step=step, **kw)
        torch.cuda.synchronize()
        for i in range(len(sizes)):
            hW[i], _, hm[i], hv[i] = oracle.adamw_step(hW[i], hG[i], hm[i], hv[i], step=step, **kw)
            assert rel_err(host(W[i]), hW[i]) < 1e-5, (step, i, sizes[i])
            assert rel_err(host(m[i]), hm[i]) < 1e-5 and rel_err(host(v[i]), hv[i]) < 1e-5
            assert not host(G[i]).any()  # clear_grad
            assert np.array_equal(host(W_lp[i]), host(W[i].to(torch.bfloat16)))


def test_surprise_momentum_step_multi_tensor(gn):
    """gn_surprise_momentum_step with non-finite gradients, recalled gradients, an Inf s_bar,
    clipping and the weight clamp, against the oracle over two steps."""
    r = rng_(41)
    sizes = [7, 1000, 4097, 33]
    W = _opt_tensors(r, sizes)
    W[1][:5] = torch.tensor([9.99, -9.99, 0.0, 1.0, -1.0], device="cuda:0")
    S = [torch.zeros_like(w) for w in W]
    S[2][::97] = float("inf")
    D = [torch.empty_like(w) for w in W]
    R = [None, _opt_tensors(r, [1000])[0], None, _opt_tensors(r, [33])[0]]
    hW, hS = [host(w) for w in W], [host(s) for s in S]
    kw = dict(eta_base=0.05, alpha=0.8, lambda_recall=0.3, surprise_floor=0.01,
              weight_decay=0.02, clip_max=0.5)
    for step in range(2):
        G = _opt_tensors(r, sizes)
        for g in G:
            g.mul_(3.0)
        G[0][2] = float("nan")
        G[2][100] = float("-inf")
        hG = [host(g) for g in G]
        gn.surprise_momentum_step([dict(W=w, grad=g, state0=s, state1=d, recalled=rc)
                                   for w, g, s, d, rc in zip(W, G, S, D, R)], **kw)
        torch.cuda.synchronize()
        for i in range(len(sizes)):
            hW[i], _, hS[i], hD = oracle.surprise_momentum_step(
                hW[i], hG[i], hS[i], recalled=None if R[i] is None else host(R[i]), **kw)
            assert rel_err(host(W[i]), hW[i]) < 1e-5, (step, i)
            assert rel_err(host(S[i]), hS[i]) < 1e-5 and rel_err(host(D[i]), hD) < 1e-5
            assert not host(G[i]).any()
    assert np.abs(host(W[1])).max() <= 10.0


def test_optimizer_rejects_bad_entries(gn):
    w = torch.zeros(8, device="cuda:0")
    with pytest.raises(gn.GnError):
        gn.adamw_step([dict(W=w, grad=w, state0=w)])  # AdamW needs v
    with pytest.raises(gn.GnError):
        gn.surprise_momentum_step([dict(W=w, grad=torch.zeros(9, device="cuda:0"), state0=w)])


# ---------------------------------------------------------------------------- tape ops
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_binary_reduce_transpose_mse(gn, dt):
    r = rng_(50)
    n = 4099  # ragged
    a = rnd(r.standard_normal(n).astype(np.float32))
    b = rnd((r.standard_normal(n) + 2.0 * np.sign(r.standard_normal(n))).astype(np.float32))
    dy = rnd(r.standard_normal(n).astype(np.float32))
    tol = 1e-6 if dt == torch.float32 else BF16_TOL
    for op in ["sub", "mul", "div", "neg"]:
        dA, dB = gn.binary_bwd(op, dev(dy, dt), dev(a, dt), dev(b, dt))
        rA, rB = oracle.binary_bwd(op, dy, a, b)
        assert rel_err(host(dA), rA) < tol, op
        if rB is not None:
            assert rel_err(host(dB), rB) < tol, op
    X = r.standard_normal((7, 33, 130)).astype(np.float32)
    for op in ["sum", "mean"]:
        g = rnd(r.standard_normal((7, 33)).astype(np.float32))
        assert rel_err(host(gn.reduce_bwd(op, dev(g, dt), X.shape)), oracle.reduce_bwd(op, g, X.shape)) < tol
        g1 = rnd(r.standard_normal(1).astype(np.float32))
        assert rel_err(host(gn.reduce_bwd(op, dev(g1, dt), X.shape)), oracle.reduce_bwd(op, g1, X.shape)) < tol
    for shape in [(7, 130, 33), (1, 64, 64), (3, 1, 65), (2, 200, 1)]:
        dY = rnd(r.standard_normal(shape).astype(np.float32))
        assert np.array_equal(host(gn.transpose_bwd(dev(dY, dt))), oracle.transpose_bwd(dY))
    p, tg = rnd(r.standard_normal(n).astype(np.float32)), rnd(r.standard_normal(n).astype(np.float32))
    assert rel_err(host(gn.mse_bwd(dev(p, dt), dev(tg, dt))), oracle.mse_bwd(p, tg)) < tol
    assert rel_err(host(gn.mse_bwd(dev(p, dt), dev(tg, dt), scale=0.5,
                                   dLoss=torch.full((1,), 3.0, device="cuda:0"))),
                   oracle.mse_bwd(p, tg, scale=0.5, g=3.0)) < tol


@pytest.mark.parametrize("Bn,K,D,rank", [(3, 2, 40, 5), (64, 4, 1024, 16)])
def test_vsa_lora_expand(gn, Bn, K, D, rank):
    r = rng_(51)
    if Bn == 3:
        gld = golden("lora_expand")
        basis, coeffs, dP = gld["basis"], gld["coeffs"], gld["dP"]
    else:
        basis = r.standard_normal((D, rank)).astype(np.float32)
        coeffs = r.standard_normal((Bn, K, rank)).astype(np.float32)
        dP = r.standard_normal((Bn, K, D)).astype(np.float32)
    dC, dB = gn.vsa_lora_expand_bwd(dev(dP), dev(basis), dev(coeffs))
    rC, rB = oracle.lora_expand_bwd(dP, basis, coeffs)
    assert rel_err(host(dC), rC) < 1e-4 and rel_err(host(dB), rB) < 1e-4


def test_vsa_cosine_blend(gn):
    g = golden("cosine_blend")
    dP = gn.vsa_cosine_blend_bwd(gn.u32_tensor(g["bits"], "cuda:0"), dev(g["weights"]),
                                 dev(g["blended"]), dev(g["info"]), K=4)
    assert rel_err(host(dP), g["dpreds"]) < 1e-5
    r = rng_(52)
    Bn, K, D = 16, 4, 10240
    bits = r.integers(0, 2**32, size=(Bn, D // 32), dtype=np.uint64).astype(np.uint32)
    preds = (r.standard_normal((Bn, K, D)) * 0.05).astype(np.float32)
    w = r.dirichlet(np.ones(K), size=Bn).astype(np.float32)
    bl = (w[:, :, None] * preds).sum(1).astype(np.float32)
    y = oracle.unpack_bits(bits, D)
    info = np.stack([np.zeros(Bn), (bl * y).sum(1), (bl * bl).sum(1)], 1).astype(np.float32)
    dP = gn.vsa_cosine_blend_bwd(gn.u32_tensor(bits, "cuda:0"), dev(w), dev(bl), dev(info), K=K)
    assert rel_err(host(dP), oracle.cosine_blend_bwd(bits, w, bl, info, K)) < 1e-5


# ---------------------------------------------------------------------------- forward kernels
def test_norm_fwd_golden_fp32(gn):
    g = golden("layernorm")
    Y, mean, rstd = gn.layernorm_fwd(dev(g["X"]), dev(g["gamma"]), dev(g["beta"]), eps=float(g["eps"]))
    assert rel_err(host(Y), g["Y"]) < FP32_TOL
    assert rel_err(host(mean), g["mean"]) < FP32_TOL and rel_err(host(rstd), g["rstd"]) < FP32_TOL
    _, _, var = gn.layernorm_fwd(dev(g["X"]), dev(g["gamma"]), dev(g["beta"]), eps=float(g["eps"]),
                                 save_var=True)
    assert rel_err(host(var), g["var"]) < FP32_TOL
    g = golden("rmsnorm")
    Y, rstd = gn.rmsnorm_fwd(dev(g["X"]), dev(g["w"]), eps=float(g["eps"]))
    assert rel_err(host(Y), g["Y"]) < FP32_TOL and rel_err(host(rstd), g["rstd"]) < FP32_TOL


# F: 768 / 520 / 1536 / 2048 take the register path (1-4 chunks per lane, 520 a ragged
# last chunk column), 100 and 4096 the generic one
@pytest.mark.parametrize("rows,F,dt", [(8192, 768, "bf16"), (1000, 2048, "f32"), (256, 1536, "bf16"),
                                       (64, 520, "bf16"), (77, 4096, "bf16"), (33, 100, "f32")])
def test_layernorm_fwd_shapes(gn, rows, F, dt):
    r = rng_(31)
    X = (r.standard_normal((rows, F)) * 2 + 0.3).astype(np.float32)
    gamma = (1 + 0.3 * r.standard_normal(F)).astype(np.float32)
    beta = (0.1 * r.standard_normal(F)).astype(np.float32)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    if dt == "bf16":
        X, gamma, beta = rnd(X), rnd(gamma), rnd(beta)
    Y, mean, rstd = gn.layernorm_fwd(dev(X, tdt), dev(gamma, tdt), dev(beta, tdt))
    rY, rm, rr = oracle.layernorm_fwd(X, gamma, beta)
    assert rel_err(host(Y), rY) < (BF16_TOL if dt == "bf16" else FP32_TOL)
    assert rel_err(host(mean), rm) < FP32_TOL and rel_err(host(rstd), rr) < FP32_TOL
    # no affine parameters: gamma = 1, beta = 0
    Y0, _, _ = gn.layernorm_fwd(dev(X, tdt))
    rY0, _, _ = oracle.layernorm_fwd(X, np.ones(F, np.float32), np.zeros(F, np.float32))
    assert rel_err(host(Y0), rY0) < (BF16_TOL if dt == "bf16" else FP32_TOL)


@pytest.mark.parametrize("rows,F,dt", [(4096, 2048, "bf16"), (300, 768, "f32"), (17, 50, "bf16")])
def test_rmsnorm_fwd_shapes(gn, rows, F, dt):
    r = rng_(32)
    X = r.standard_normal((rows, F)).astype(np.float32)
    w = (1 + 0.2 * r.standard_normal(F)).astype(np.float32)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    if dt == "bf16":
        X, w = rnd(X), rnd(w)
    Y, rstd = gn.rmsnorm_fwd(dev(X, tdt), dev(w, tdt))
    rY, rr = oracle.rmsnorm_fwd(X, w)
    assert rel_err(host(Y), rY) < (BF16_TOL if dt == "bf16" else FP32_TOL)
    assert rel_err(host(rstd), rr) < FP32_TOL


def test_norm_fwd_feeds_backward(gn):
    # the saved statistics of the forward drive the backward exactly as the oracle's do
    r = rng_(33)
    rows, F = 512, 768
    X = rnd((r.standard_normal((rows, F)) + 0.5).astype(np.float32))
    gamma = rnd((1 + 0.3 * r.standard_normal(F)).astype(np.float32))
    dY = rnd(r.standard_normal((rows, F)).astype(np.float32))
    tX, tg, tdY = dev(X, torch.bfloat16), dev(gamma, torch.bfloat16), dev(dY, torch.bfloat16)
    _, mean, var = gn.layernorm_fwd(tX, tg, save_var=True)
    dX, dG, _ = gn.layernorm_bwd(tdY, tX, tg, mean, var, stat_is_var=True)
    _, rm, rr = oracle.layernorm_fwd(X, gamma)
    rX, rG, _ = oracle.layernorm_bwd(dY, X, gamma, rm, rr)
    assert rel_err(host(dX), rX) < BF16_TOL and rel_err(host(dG), rG) < 1e-3


@pytest.mark.parametrize("kind", ["swiglu_up", "swiglu_gate", "geglu_up", "geglu_gate", "reglu_up"])
def test_glu_fwd(gn, kind):
    g = golden("glu")
    out = gn.glu_fwd(kind, dev(g["gate"]), dev(g["up"]))
    assert rel_err(host(out), oracle.glu_fwd(kind, g["gate"], g["up"])) < FP32_TOL
    r = rng_(34)
    n = 8192 * 3 + 5  # a ragged tail after the 8-element vectors
    gate = rnd(r.standard_normal(n + 1).astype(np.float32))
    up = rnd(r.standard_normal(n + 1).astype(np.float32))
    tg, tu = dev(gate, torch.bfloat16), dev(up, torch.bfloat16)
    ref = oracle.glu_fwd(kind, gate[:n], up[:n])
    assert rel_err(host(gn.glu_fwd(kind, tg[:n], tu[:n])), ref) < BF16_TOL
    # views one element in (2-byte aligned) take the scalar path
    ref1 = oracle.glu_fwd(kind, gate[1:], up[1:])
    assert rel_err(host(gn.glu_fwd(kind, tg[1:], tu[1:])), ref1) < BF16_TOL


# (M, N, K): multiples of 64 in K take the LDS-DMA core with the bias in its epilogue;
# K = 40 the register-staged core after a bias fill; K = 0 leaves Y = b
@pytest.mark.parametrize("M,N,K", [(512, 384, 768), (200, 136, 128), (100, 72, 40), (16, 24, 0)])
def test_linear_fwd_bf16(gn, M, N, K):
    r = rng_(35)
    X = rnd(r.standard_normal((M, K)).astype(np.float32))
    W = rnd((r.standard_normal((N, K)) * 0.05).astype(np.float32))
    b = rnd(r.standard_normal(N).astype(np.float32))
    tX, tW, tb = dev(X, torch.bfloat16), dev(W, torch.bfloat16), dev(b, torch.bfloat16)
    Y = gn.linear_fwd(tX, tW, tb)
    assert Y.dtype == torch.bfloat16
    assert rel_err(host(Y), oracle.linear_fwd(X, W, b) if K else np.tile(b, (M, 1))) < 8e-3
    if K:
        assert rel_err(host(gn.linear_fwd(tX, tW)), oracle.linear_fwd(X, W)) < 8e-3


def test_linear_fwd_fp32_golden(gn):
    for tag in ["small", "c1l2"]:
        g = golden(f"linear_{tag}")
        Y = gn.linear_fwd(dev(g["X"]), dev(g["W"]), dev(g["b"]))
        assert rel_err(host(Y), oracle.linear_fwd(g["X"], g["W"], g["b"])) < FP32_TOL


@pytest.mark.parametrize("kind", ["geglu_up", "swiglu_up", "reglu_up"])
def test_glu_linear_fwd(gn, kind):
    r = rng_(36)
    M, H, K = 512, 1024, 768
    X = rnd(r.standard_normal((M, K)).astype(np.float32))
    Wg, Wu = (rnd((r.standard_normal((H, K)) * 0.05).astype(np.float32)) for _ in range(2))
    bg, bu = (rnd((0.1 * r.standard_normal(H)).astype(np.float32)) for _ in range(2))
    gate, up, out = gn.glu_linear_fwd(kind, dev(X, torch.bfloat16), dev(Wg, torch.bfloat16),
                                      dev(Wu, torch.bfloat16), dev(bg, torch.bfloat16),
                                      dev(bu, torch.bfloat16))
    assert rel_err(host(gate), oracle.linear_fwd(X, Wg, bg)) < 8e-3
    assert rel_err(host(up), oracle.linear_fwd(X, Wu, bu)) < 8e-3
    # out is formed from the saved (bf16) gate and up, which the backward then reads
    assert rel_err(host(out), oracle.glu_fwd(kind, host(gate), host(up))) < 8e-3
