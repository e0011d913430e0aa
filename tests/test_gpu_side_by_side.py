"""Linear-type backward calls whose weight and input gradients run side by side (the input
gradient on the library's side stream, forked off the caller's stream and joined before the
call returns): the outputs are bit-identical to the two products launched one call at a time,
eagerly (products of >= 50 GFLOP fork on every call) and replayed from a captured HIP graph
(products of >= 2 GFLOP fork under capture).  The one-at-a-time results are checked against
float64 products on sampled rows, so the comparison is not only between two runs of the same
kernels.
"""
import ctypes

import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def gn(gpu):
    import gn_bwd
    gn_bwd.lib()
    return gn_bwd


def bf(shape, seed, scale=1.0):
    g = torch.Generator(device="cuda:0").manual_seed(seed)
    return (torch.randn(shape, generator=g, device="cuda:0") * scale).to(torch.bfloat16)


def rows_ref(A, B, rows):
    """float64 (A[rows] @ B) for A [M, K], B [K, N]."""
    return (A[rows].double() @ B.double()).cpu().numpy()


def check_rows(out, ref_rows, rows, tol):
    assert rel_err(out[rows].float().cpu().numpy(), ref_rows) < tol


def linear_one_at_a_time(gn, dY, X, W, with_db):
    """dX from gn_gemm and (dW, db) from a dW-only gn_linear_bwd: no fork in either call."""
    dX = gn.gemm(dY, W)
    _, dW, db = gn.linear_bwd(dY, X, W, need_dx=False, need_db=with_db)
    return dX, dW, db


@pytest.mark.parametrize("M,N,K,with_db", [(8192, 3072, 2048, True), (4096, 5632, 2048, False)])
def test_linear_bwd_side_by_side_eager(gn, M, N, K, with_db):
    assert 2.0 * M * N * K >= 5e10  # forks on an eager call
    dY, X, W = bf((M, N), 1, 0.1), bf((M, K), 2), bf((N, K), 3, 0.02)
    dX, dW, db = gn.linear_bwd(dY, X, W, need_db=with_db)
    dX1, dW1, db1 = linear_one_at_a_time(gn, dY, X, W, with_db)
    torch.cuda.synchronize()
    assert torch.equal(dX, dX1) and torch.equal(dW, dW1)
    if with_db:
        assert torch.equal(db, db1)
        ref = dY.double().sum(0).cpu().numpy()
        assert rel_err(db.cpu().numpy(), ref) < 1e-5
    rows = torch.tensor([0, 1, M // 3, M - 1], device="cuda:0")
    check_rows(dX1, rows_ref(dY, W, rows), rows, 8e-3)
    wrows = torch.tensor([0, N // 2, N - 1], device="cuda:0")
    check_rows(dW1, rows_ref(dY.t(), X, wrows), wrows, 1e-5)


def test_glu_proj_bwd_side_by_side_eager(gn):
    M, K, H = 8192, 768, 3072  # the C5 decoder's GEGLU projections: 77 GFLOP per product
    gu, X = bf((M, 2 * H), 4, 0.1), bf((M, K), 5)
    Wg, Wu = bf((H, K), 6, 0.02), bf((H, K), 7, 0.02)
    dX, dWg, dWu, dbg, dbu = gn.glu_proj_bwd(gu, X, Wg, Wu, need_dx=True, need_db=True)
    dX1 = torch.empty_like(dX)
    L, P, s = gn.lib(), gn._ptr, gn._stream()
    gn._check(L.gn_glu_proj_bwd(P(gu), P(X), P(Wg), P(Wu), P(dX1), None, None, None, None, M, K,
                                H, gn.BF16, 0, s), "glu_proj_bwd (dX only)")
    _, dWg1, dWu1, dbg1, dbu1 = gn.glu_proj_bwd(gu, X, Wg, Wu, need_dx=False, need_db=True)
    torch.cuda.synchronize()
    for a, b in ((dX, dX1), (dWg, dWg1), (dWu, dWu1), (dbg, dbg1), (dbu, dbu1)):
        assert torch.equal(a, b)
    rows = torch.tensor([0, M // 2, M - 1], device="cuda:0")
    Wcat = torch.cat([Wg, Wu], 0)
    check_rows(dX1, rows_ref(gu, Wcat, rows), rows, 8e-3)


def test_ffn_down_glu_bwd_side_by_side_eager(gn):
    M, N, H = 4096, 2048, 5632  # C2: 94 GFLOP per product
    dY, A, Wd = bf((M, N), 8, 0.1), bf((M, H), 9), bf((N, H), 10, 0.02)
    gate, up = bf((M, H), 11), bf((M, H), 12)
    gu, dWd, dbd = gn.ffn_down_glu_bwd("swiglu_up", dY, A, Wd, gate, up, need_db=True)
    gu1 = torch.empty_like(gu)
    L, P, s = gn.lib(), gn._ptr, gn._stream()
    gn._check(L.gn_ffn_down_glu_bwd(gn.GLU["swiglu_up"], P(dY), P(A), P(Wd), P(gate), P(up),
                                    P(gu1), None, None, M, N, H, gn.BF16, 0, s),
              "ffn_down_glu_bwd (gu only)")
    _, dWd1, dbd1 = gn.linear_bwd(dY, A, Wd, need_dx=False, need_db=True)
    torch.cuda.synchronize()
    assert torch.equal(gu, gu1) and torch.equal(dWd, dWd1) and torch.equal(dbd, dbd1)
    wrows = torch.tensor([0, N // 2, N - 1], device="cuda:0")
    check_rows(dWd1, rows_ref(dY.t(), A, wrows), wrows, 1e-5)


def test_linear_bwd_side_by_side_graph_replays(gn):
    """The decoder's QKV shape (29 GFLOP per product: forked only under capture).  The eager
    call before the capture also creates the side stream (never created during a capture)."""
    M, N, K = 8192, 2304, 768
    assert 2e9 <= 2.0 * M * N * K < 5e10
    dY, X, W = bf((M, N), 13, 0.1), bf((M, K), 14), bf((N, K), 15, 0.02)
    nb = gn.linear_workspace_bytes(M, N, K, gn.BF16)
    ws = gn.workspace(nb, dY.device) if nb else None
    dX = torch.empty((M, K), dtype=torch.bfloat16, device="cuda:0")
    dW = torch.empty((N, K), dtype=torch.float32, device="cuda:0")
    db = torch.empty((N,), dtype=torch.float32, device="cuda:0")
    L, P = gn.lib(), gn._ptr

    def call():
        wsp, wsb = (None, 0) if ws is None else (P(ws), ws.numel() * ws.element_size())
        gn._check(L.gn_linear_bwd_ws(P(dY), P(X), P(W), P(dX), P(dW), P(db), M, N, K, gn.BF16,
                                     0, wsp, wsb, gn._stream()), "gn_linear_bwd_ws")

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()  # eager on the capture stream first
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    eX, eW, eb = dX.clone(), dW.clone(), db.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    for i in range(4):
        for t in (dX, dW, db):
            t.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(dX, eX) and torch.equal(dW, eW) and torch.equal(db, eb), f"replay {i}"
        _ = (dY.float() * 2).sum().item()  # eager work between the replays
    dX1, dW1, db1 = linear_one_at_a_time(gn, dY, X, W, True)
    torch.cuda.synchronize()
    assert torch.equal(eX, dX1) and torch.equal(eW, dW1) and torch.equal(eb, db1)
    rows = torch.tensor([0, M - 1], device="cuda:0")
    check_rows(dX1, rows_ref(dY, W, rows), rows, 8e-3)
