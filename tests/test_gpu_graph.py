"""GPU tests of grilly_core.OpGraph, the HIP graph replacement of the reference's OpGraph
(cpp/src/op_graph.cpp:123-246, bindings.cpp:212-235): a tape backward captured once and
replayed gives, replay after replay, the same gradients as the eager tape backward over the
same buffers, with new values written into the recorded tensors and the program's own eager
torch work and synchronisations between replays.  The kernels involved are deterministic
(no atomics), so replay and eager results are compared bit for bit; the embedding's
scatter-add uses fp32 atomics and is compared within 1e-6.  The first replay is also pinned
to the CPU oracle (fp32, normwise relative error <= 1e-4).

The graph holds kernel nodes only: the library clears memory with its own fill kernel
(gn_zero) and copies with a copy kernel, never with hipMemsetAsync / hipMemcpyAsync."""
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


class MLP:
    """BASELINE configs[0]'s MLP (784 -> hidden -> 10, fp32, ReLU, softmax CE) whose tensors
    stay at fixed addresses; refresh() writes a new batch and forward into them in place."""

    def __init__(self, hidden=256, batch=64, seed=1):
        self.r = np.random.default_rng(seed)
        self.B, self.H = batch, hidden
        dev = "cuda:0"
        lim1, lim2 = np.sqrt(6 / (784 + hidden)), np.sqrt(6 / (hidden + 10))
        self.W1 = self._t(self.r.uniform(-lim1, lim1, (hidden, 784)))
        self.W2 = self._t(self.r.uniform(-lim2, lim2, (10, hidden)))
        self.b1 = self._t(0.1 * self.r.standard_normal(hidden))
        self.b2 = self._t(0.1 * self.r.standard_normal(10))
        self.X = torch.empty(batch, 784, device=dev)
        self.y = torch.empty(batch, dtype=torch.int32, device=dev)
        self.Z = torch.empty(batch, hidden, device=dev)
        self.Hh = torch.empty(batch, hidden, device=dev)
        self.L = torch.empty(batch, 10, device=dev)
        self.loss = torch.zeros(1, device=dev)
        self.refresh()

    def _t(self, a):
        return torch.from_numpy(np.asarray(a, np.float32)).to("cuda:0").contiguous()

    def refresh(self):
        self.X.copy_(self._t(self.r.standard_normal((self.B, 784))))
        self.y.copy_(torch.from_numpy(self.r.integers(0, 10, self.B).astype(np.int32)))
        self.Z.copy_(self.X @ self.W1.t() + self.b1)
        self.Hh.copy_(torch.relu(self.Z))
        self.L.copy_(self.Hh @ self.W2.t() + self.b2)

    def record(self, gc, gb, tape):
        n1 = tape.record_op(gc.OpType.Linear, [gb.tref(self.X)], [gb.tref(self.Z)])
        tape.save_for_backward(n1, [self.W1.data_ptr(), self.b1.data_ptr()])
        tape.record_op(gc.OpType.ReLU, [gb.tref(self.Z, True)], [gb.tref(self.Hh)])
        n3 = tape.record_op(gc.OpType.Linear, [gb.tref(self.Hh, True)], [gb.tref(self.L)])
        tape.save_for_backward(n3, [self.W2.data_ptr(), self.b2.data_ptr()])
        return tape.record_op(gc.OpType.CrossEntropy, [gb.tref(self.L, True), gb.tref(self.y)],
                              [gb.tref(self.loss)], gb.cross_entropy_params(1.0))

    def tensors(self):
        return {"L": self.L, "H": self.Hh, "Z": self.Z, "W2": self.W2, "b2": self.b2,
                "W1": self.W1, "b1": self.b1}

    def oracle_grads(self):
        h = lambda t: t.cpu().numpy()
        X, y, W1, W2 = h(self.X), h(self.y), h(self.W1), h(self.W2)
        dL = oracle.xent_bwd(h(self.L), y, 1.0)
        dH, dW2, db2 = oracle.linear_bwd(dL, h(self.Hh), W2)
        dZ = oracle.act_bwd("relu", dH, h(self.Z))
        _, dW1, db1 = oracle.linear_bwd(dZ, X, W1, need_dx=False)
        return {"L": dL, "H": dH, "Z": dZ, "W2": dW2, "b2": db2, "W1": dW1, "b1": db1}


def grads_of(gb, dev, source, tensors, dtype=None):
    """Download the gradient `source` (a tape or a graph) records for each tensor."""
    out = {}
    for k, t in tensors.items():
        gid = source.get_grad_buffer(t.data_ptr())
        assert gid != 0, f"no gradient recorded for {k}"
        out[k] = gb.download(dev, gid, t.shape, gb.dtype_code(t) if dtype is None else dtype)
    return out


def eager_grads(gc, gb, dev, model, tensors, dtype=None, glu_epilogue=False):
    tape = gb.create_tape_context(dev)
    tape.set_glu_epilogue(glu_epilogue)
    tape.begin()
    loss = model.record(gc, gb, tape) if isinstance(model, MLP) else model.record(tape)
    tape.backward(loss, 0)
    out = grads_of(gb, dev, tape, tensors, dtype)
    tape.end()
    return out


def test_zero_and_copy_kernels(env):
    """gn_zero on each store width (16-byte, 4-byte and byte items, chosen by alignment) leaves
    the neighbouring elements alone; a same-dtype gn_convert is a bit-exact word copy (NaN
    payloads included)."""
    import gn_bwd as gn
    for dtype, n, off in ((torch.float32, 4096, 0), (torch.float32, 1003, 1),
                          (torch.bfloat16, 1000, 2), (torch.bfloat16, 777, 1),
                          (torch.bfloat16, 4096, 3)):
        base = torch.randn(n + off + 5, device="cuda:0").to(dtype) + 3.0
        keep = base.clone()
        gn.zero(base[off:off + n])
        torch.cuda.synchronize()
        assert torch.equal(base[:off], keep[:off]) and torch.equal(base[off + n:], keep[off + n:])
        assert torch.count_nonzero(base[off:off + n]).item() == 0
    bits = torch.randint(-2 ** 31, 2 ** 31 - 1, (1004,), dtype=torch.int32, device="cuda:0")
    bits[:8] = torch.tensor([0x7FC00001, 0x7F800001, -0x00400001, 0, -2 ** 31, 1, 0x7F800000, -1],
                            dtype=torch.int32)
    for off in (0, 1):  # 16-byte and 4-byte items
        src = bits[off:].view(torch.float32)
        assert torch.equal(gn.convert(src, torch.float32).view(torch.int32), bits[off:])
    halves = bits.view(torch.int16)
    for off in (0, 2, 1):  # 16-byte, 4-byte and 2-byte items
        hb = halves[off:]
        assert torch.equal(gn.convert(hb.view(torch.bfloat16), torch.bfloat16).view(torch.int16), hb)


def test_mlp_backward_graph_replays_match_eager(env):
    """configs[0] through the tape, captured once: each of three replays, after new data is
    written into the recorded tensors, equals the eager tape backward bit for bit; the first
    is pinned to the oracle.  The gradient buffers stay pinned after the tape has ended."""
    gc, gb, dev = env
    m = MLP(seed=3)
    tape = gb.create_tape_context(dev)
    tape.begin()
    ce = m.record(gc, gb, tape)
    g = gc.OpGraph()
    stream_before = dev.stream_handle()
    g.capture_backward(tape, ce, 0)
    assert dev.stream_handle() == stream_before and not g.is_capturing()
    tape.end()
    counts = g.node_counts()
    assert counts["memset"] == 0 and counts["memcpy"] == 0, counts
    assert counts["kernel"] == g.size() > 0
    st = g.optimize(dev)
    assert st == {"ops_fused": 0, "barriers_eliminated": 0, "original_ops": g.size(),
                  "optimized_ops": g.size()}
    # pinned: still live after the tape's end(), and not handed out again
    gw1 = g.get_grad_buffer(m.W1.data_ptr())
    assert gw1 != 0 and dev.buffer_bytes(gw1) > 0
    other = dev.alloc(dev.buffer_bytes(gw1))
    assert other != gw1
    dev.free(other)

    tensors = m.tensors()
    for rep in range(3):
        m.refresh()
        torch.cuda.synchronize()
        g.execute(dev)
        spare = (m.X @ m.X.t()).sum()  # eager torch work queued behind the replay
        torch.cuda.synchronize()
        got = grads_of(gb, dev, g, tensors)
        want = eager_grads(gc, gb, dev, m, tensors)
        for k in tensors:
            np.testing.assert_array_equal(got[k], want[k], err_msg=f"replay {rep}: {k}")
        if rep == 0:
            ref = m.oracle_grads()
            for k in tensors:
                assert rel_err(got[k], ref[k]) < 1e-4, k
        assert torch.isfinite(spare).item()
    assert g.replays() == 3
    g.clear()
    assert g.size() == 0 and g.get_grad_buffer(m.W1.data_ptr()) == 0


def test_graph_segments_replay_in_order(env):
    """Two captures into one graph (capture_backward, then begin_capture/end_capture around a
    second tape's backward) replay as one launch; both equal their eager results."""
    gc, gb, dev = env
    a, b = MLP(hidden=256, seed=5), MLP(hidden=128, batch=32, seed=6)
    g = gc.OpGraph()
    ta = gb.create_tape_context(dev)
    ta.begin()
    g.capture_backward(ta, a.record(gc, gb, ta), 0)
    ta.end()
    tb = gb.create_tape_context(dev)
    tb.begin()
    loss_b = b.record(gc, gb, tb)
    g.begin_capture(dev)
    assert g.is_capturing()
    tb.backward(loss_b, 0)
    g.end_capture()
    ids_b = {k: tb.get_grad_buffer(t.data_ptr()) for k, t in b.tensors().items()}
    tb.end()
    size_a_b = g.size()
    for m in (a, b):
        m.refresh()
    torch.cuda.synchronize()
    g.execute(dev)
    torch.cuda.synchronize()
    got_a = grads_of(gb, dev, g, a.tensors())
    got_b = {k: gb.download(dev, ids_b[k], t.shape) for k, t in b.tensors().items()}
    want_a = eager_grads(gc, gb, dev, a, a.tensors())
    want_b = eager_grads(gc, gb, dev, b, b.tensors())
    for k in want_a:
        np.testing.assert_array_equal(got_a[k], want_a[k], err_msg=k)
        np.testing.assert_array_equal(got_b[k], want_b[k], err_msg=k)
    assert g.size() == size_a_b and g.node_counts()["memset"] == 0
    g.clear()


def test_capture_errors_leave_the_device_usable(env):
    """A handler that raises during capture ends the capture: the exception reaches the
    caller, the device's stream is restored, nothing was recorded, and an empty graph's
    execute() does nothing.  A second begin_capture and an end_capture with none open raise."""
    gc, gb, dev = env
    m = MLP(seed=8)
    bad = torch.zeros(4, 4, dtype=torch.int32, device="cuda:0")
    tape = gb.create_tape_context(dev)
    tape.begin()
    # an int32 tensor requiring a gradient: the Linear handler rejects its dtype
    n = tape.record_op(gc.OpType.Linear, [gb.tref(bad, True)], [gb.tref(m.L)])
    tape.save_for_backward(n, [m.W1.data_ptr()])
    ce = tape.record_op(gc.OpType.CrossEntropy, [gb.tref(m.L, True), gb.tref(m.y)],
                        [gb.tref(m.loss)], gb.cross_entropy_params(1.0))
    g = gc.OpGraph()
    before = dev.stream_handle()
    with pytest.raises(Exception):
        g.capture_backward(tape, ce, 0)
    tape.end()
    assert not g.is_capturing() and dev.stream_handle() == before
    assert g.size() == 0
    g.execute(dev)
    g.begin_capture(dev)
    with pytest.raises(RuntimeError):
        g.begin_capture(dev)
    g.end_capture()
    with pytest.raises(RuntimeError):
        g.end_capture()
    assert g.size() == 0
    g.clear()
    # the device still runs eager work
    want = eager_grads(gc, gb, dev, m, m.tensors())
    ref = m.oracle_grads()
    assert rel_err(want["W1"], ref["W1"]) < 1e-4


@pytest.mark.parametrize("glu_epilogue", [False, True])
def test_decoder_backward_graph_replays_match_eager(env, glu_epilogue):
    """BASELINE configs[4]'s decoder at a small size (2 layers), captured once: two replays,
    with the logits and targets changed in place between them, equal the eager tape backward
    (bit for bit; the tied embedding's gradient, which sums fp32 atomics, within 1e-6), with
    and without the GLU's local gradients in the down projection's epilogue."""
    gc, gb, dev = env
    import decoder_tape
    m = decoder_tape.Decoder(layers=2, d=256, heads=4, ff=512, vocab=500, batch=2, seq=128, seed=12)
    m.forward()
    tensors = {"E": m.E, "lnf_g": m.lnf_g, "lnf_b": m.lnf_b}
    for i, p in enumerate(m.layers):
        for k in ("Wqkv", "bqkv", "Wo", "bo", "ln1_g", "ln1_b", "ln2_g", "ln2_b", "Wg", "Wu",
                  "bg", "bu", "Wd", "bd"):
            tensors[f"{k}{i}"] = p[k]
    tape = gb.create_tape_context(dev)
    tape.set_glu_epilogue(glu_epilogue)
    tape.begin()
    g = gc.OpGraph()
    g.capture_backward(tape, m.record(tape), 0)
    tape.end()
    assert g.node_counts()["memset"] == 0 and g.node_counts()["memcpy"] == 0
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(3)
    for rep in range(2):
        if rep:
            m.logits.mul_(1.5)
            m.tgt.copy_(torch.randint(0, m.V, m.tgt.shape, device="cuda:0", generator=gen,
                                      dtype=torch.int32))
        torch.cuda.synchronize()
        g.execute(dev)
        torch.cuda.synchronize()
        got = grads_of(gb, dev, g, tensors, gb.DTYPE_F32)
        want = eager_grads(gc, gb, dev, m, tensors, gb.DTYPE_F32, glu_epilogue)
        for k in tensors:
            if k == "E":
                assert rel_err(got[k], want[k]) < 1e-6
            else:
                np.testing.assert_array_equal(got[k], want[k], err_msg=f"replay {rep}: {k}")
    g.clear()
