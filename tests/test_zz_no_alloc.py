"""gn_layernorm_bwd_noalloc (the entry point that allocates nothing) against gn_layernorm_bwd
with a caller-given workspace, both called through the C ABI: the same kernels run, so every
output must be bit-identical.  Two calls in a row, the second on a smaller input (the static
scratch keeps the first call's partial rows; nothing may leak into the second), plus the
accumulate flag and a row width that takes the generic kernels.  Also checked against the
CPU oracle (bf16 path <= 2e-2, fp32 path <= 1e-4, normwise)."""
import numpy as np
import pytest

import oracle
from conftest import rel_err

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def gn(gpu):
    import gn_bwd
    gn_bwd.lib()
    return gn_bwd


def _inputs(r, rows, F, dt):
    x = torch.from_numpy(r.standard_normal((rows, F)).astype(np.float32)).cuda().to(dt)
    dy = torch.from_numpy((r.standard_normal((rows, F)) * 0.1).astype(np.float32)).cuda().to(dt)
    g = torch.from_numpy((1 + 0.1 * r.standard_normal(F)).astype(np.float32)).cuda().to(dt)
    xf = x.float()
    mean = xf.mean(1)
    rstd = torch.rsqrt(xf.var(1, unbiased=False) + 1e-5)
    return dy, x, g, mean.contiguous(), rstd.contiguous()


def _run(gn, noalloc, dy, x, g, mean, rstd, flags=0, out=None):
    L = gn.lib()
    rows, F = x.shape
    dX, dG, dB = out if out is not None else (
        torch.empty_like(x), torch.empty(F, device="cuda"), torch.empty(F, device="cuda"))
    p = lambda t: t.data_ptr()
    if noalloc:
        rc = L.gn_layernorm_bwd_noalloc(p(dy), p(x), p(g), p(mean), p(rstd), p(dX), p(dG), p(dB),
                                        rows, F, 1e-5, gn._dt(x), flags, gn._stream())
    else:
        ws = gn.workspace(gn.norm_workspace_bytes(rows, F), x.device)
        rc = L.gn_layernorm_bwd(p(dy), p(x), p(g), p(mean), p(rstd), p(dX), p(dG), p(dB), rows, F,
                                1e-5, gn._dt(x), flags, p(ws), ws.numel(), gn._stream())
    assert rc == 0, gn.last_error()
    return dX, dG, dB


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_noalloc_matches_workspace_entry(gn, dt):
    r = np.random.default_rng(77)
    for rows, F in [(4096, 2048), (1000, 768)]:  # second call smaller
        args = _inputs(r, rows, F, dt)
        a = _run(gn, True, *args)
        b = _run(gn, False, *args)
        torch.cuda.synchronize()
        for u, v in zip(a, b):
            assert torch.equal(u, v), (rows, F)
        dy, x, g, mean, rstd = (t.float().cpu().numpy() for t in args)
        rx, rg, rb = oracle.layernorm_bwd(dy, x, g, mean, rstd)
        tol = 2e-2 if dt == torch.bfloat16 else 1e-4
        assert rel_err(a[0].float().cpu().numpy(), rx) < tol
        assert rel_err(a[1].cpu().numpy(), rg) < tol and rel_err(a[2].cpu().numpy(), rb) < tol


def test_noalloc_accumulate_and_generic_width(gn):
    r = np.random.default_rng(78)
    dt = torch.bfloat16
    args = _inputs(r, 512, 1024, dt)
    base = tuple(t.clone() for t in _run(gn, False, *args))
    a = _run(gn, True, *args, flags=gn.ACCUMULATE, out=tuple(t.clone() for t in base))
    b = _run(gn, False, *args, flags=gn.ACCUMULATE, out=tuple(t.clone() for t in base))
    torch.cuda.synchronize()
    for u, v in zip(a, b):
        assert torch.equal(u, v)
    # F = 3000 (> 2048, not a multiple of 8): the generic kernels, no scratch used
    args = _inputs(r, 64, 3000, torch.float32)
    a = _run(gn, True, *args)
    b = _run(gn, False, *args)
    torch.cuda.synchronize()
    for u, v in zip(a, b):
        assert torch.equal(u, v)
