"""Python helpers around grilly_core, mirroring the reference's
src/grilly_next/backend/_bridge.py (create_tape_context :260, make_tensor_ref :279), plus
packers for the per-op parameter blocks and torch interop.

A buffer id is a device pointer, so a torch tensor on the GPU is wrapped without a copy:
`make_tensor_ref(t.data_ptr(), t.shape, dtype_code(t))`.  Use `attach_torch_stream(device)`
so the tape launches on torch's current stream.
"""
from __future__ import annotations

import struct

import numpy as np

import grilly_core

DTYPE_F32, DTYPE_F16, DTYPE_U32, DTYPE_I32, DTYPE_BF16 = 0, 1, 2, 3, 4
GLU_KIND = {"swiglu_up": 0, "swiglu_gate": 1, "geglu_up": 2, "geglu_gate": 3, "reglu_up": 4}
ROPE_MODE = {"none": 0, "interleaved": 1, "half": 2}


def create_tape_context(device, arena_capacity: int = 64 << 20):
    return grilly_core.TapeContext(device, arena_capacity)


def make_tensor_ref(buffer_id: int, shape, dtype: int = DTYPE_F32, requires_grad: bool = False):
    ref = grilly_core.TensorRef()
    ref.buffer_id = int(buffer_id)
    ref.set_shape([int(s) for s in shape])
    ref.dtype = int(dtype)
    ref.requires_grad = bool(requires_grad)
    return ref


def dtype_code(t) -> int:
    import torch
    return {torch.float32: DTYPE_F32, torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16,
            torch.int32: DTYPE_I32}[t.dtype]


def tref(t, requires_grad: bool = False):
    """TensorRef over a contiguous torch tensor on the GPU (no copy)."""
    assert t.is_cuda and t.is_contiguous()
    return make_tensor_ref(t.data_ptr(), t.shape, dtype_code(t), requires_grad)


def attach_torch_stream(device):
    import torch
    device.use_stream(torch.cuda.current_stream().cuda_stream)


def download(device, buffer_id: int, shape, dtype: int = DTYPE_F32) -> np.ndarray:
    """Copy a device buffer to numpy as float32 (bf16 is widened)."""
    if dtype == DTYPE_BF16:
        raw = device.download(buffer_id, list(shape), np.dtype(np.uint16))
        return (raw.astype(np.uint32) << 16).view(np.float32)
    if dtype == DTYPE_I32:
        return device.download(buffer_id, list(shape), np.dtype(np.int32))
    return device.download(buffer_id, list(shape), np.dtype(np.float32))


# ---- parameter blocks (layouts of the structs in csrc/tape/autograd.h) ------------------
def gelu_params(erf_form: bool = False) -> bytes:
    return struct.pack("<I", int(erf_form))


def layernorm_params(eps: float = 1e-5, stat_is_var: bool = False) -> bytes:
    return struct.pack("<fI", eps, int(stat_is_var))


def rmsnorm_params(eps: float = 1e-6, stat: str = "rstd") -> bytes:
    """RMSNormParams: which per-row statistic saved slot 1 holds: "rstd", "meansq" (mean(x^2),
    rms-norm.glsl:52; eps added in the backward) or "rms" (sqrt(mean(x^2) + eps),
    snn-rmsnorm.glsl:55)."""
    return struct.pack("<fI", eps, {"rstd": 0, "meansq": 1, "rms": 2}[stat])


def attention_params(scale: float = 0.0, causal: bool = True, rope: str = "interleaved",
                     theta: float = 10000.0, fused_qkv_heads: int = 0) -> bytes:
    """AttentionParams.  fused_qkv_heads = H > 0 selects the fused layout: inputs[0] is the
    QKV projection output [B, S, 3*H*D] and the output O is [B, S, H*D]."""
    layout = 1 if fused_qkv_heads else 0
    return struct.pack("<fIIfII", scale, int(causal), ROPE_MODE[rope], theta, layout,
                       int(fused_qkv_heads))


def embedding_params(vocab: int) -> bytes:
    """Embedding node: the table's row count (the table id goes in saved_buffer_ids[0])."""
    return struct.pack("<I", int(vocab))


def cross_entropy_params(scale: float = 1.0) -> bytes:
    return struct.pack("<fI", scale, 1)


def fused_glu_params(kind: str = "swiglu_up") -> bytes:
    return struct.pack("<I", GLU_KIND[kind])


def vsa_surrogate_params(K: int, D: int, gamma: float = 1.0, delta: float = 1.0,
                         lambda_c: float = 0.3, temperature: float = 1.0,
                         winning_k: int = 0, runner_up_k: int = 0) -> bytes:
    """VSASurrogateLossParams (autograd.h:172-184); defaults as in bindings.cpp:3169-3176."""
    return struct.pack("<fffIIIIfff", gamma, delta, lambda_c, K, D, winning_k, runner_up_k,
                       0.0, temperature, 0.01)


# ---------------------------------------------------------------------------- optimizers
class _TapeOptimizer:
    """Optimizer step applied between TapeContext.backward and end, the order the reference's
    vsa_training_step uses (bindings.cpp:3196-3279): each weight's gradient is looked up with
    tape.get_grad_buffer(weight id) (0 = no gradient: the weight is skipped) and every tensor
    is updated by one multi-tensor launch (gn_*_step).  Weights are GPU tensors whose
    data_ptr() is the buffer id the tape recorded; a bf16 weight gets an fp32 master copy and
    receives the rounded update in place, so the next forward sees it."""

    def __init__(self, weights):
        import torch
        self.weights = list(weights)
        self.masters = [w if w.dtype == torch.float32 else w.float().contiguous()
                        for w in self.weights]
        self.t = 0

    def _entries(self, tape, state):
        import torch
        out = []
        for w, mw, st in zip(self.weights, self.masters, state):
            g = tape.get_grad_buffer(w.data_ptr())
            if g == 0:
                continue
            e = dict(W=mw, grad=int(g), **st)
            if w.dtype == torch.bfloat16:
                e["W_bf16"] = w
            out.append(e)
        return out


class SurpriseMomentumOptimizer(_TapeOptimizer):
    """The reference's SurpriseMomentumOptimizer (bindings.cpp:3049-3138: same attribute names
    and defaults; the recalled gradient is zero, as there).  s_bar starts at zero per weight;
    `delta` keeps the last update per element when keep_delta."""

    def __init__(self, weights, lr=1e-3, alpha=0.9, clip=1.0, keep_delta=False):
        import torch
        super().__init__(weights)
        self.eta_base, self.alpha_momentum, self.clip_max = lr, alpha, clip
        self.lambda_recall, self.surprise_floor, self.weight_decay = 0.0, 0.01, 0.0
        self.s_bar = [torch.zeros_like(m) for m in self.masters]
        self.delta = [torch.zeros_like(m) for m in self.masters] if keep_delta else None

    def step(self, tape):
        import gn_bwd
        self.t += 1
        st = [dict(state0=s, state1=(self.delta[i] if self.delta else None))
              for i, s in enumerate(self.s_bar)]
        entries = self._entries(tape, st)
        gn_bwd.surprise_momentum_step(entries, self.eta_base, self.alpha_momentum,
                                      self.lambda_recall, self.surprise_floor, self.weight_decay,
                                      self.clip_max, clear_grad=True)
        return len(entries)


class AdamW(_TapeOptimizer):
    """AdamW over the tape's gradients (adamw-update.glsl:41-61; weight_decay 0 is
    adam-update.glsl)."""

    def __init__(self, weights, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01):
        import torch
        super().__init__(weights)
        self.lr, self.betas, self.eps, self.weight_decay = lr, betas, eps, weight_decay
        self.m = [torch.zeros_like(m) for m in self.masters]
        self.v = [torch.zeros_like(m) for m in self.masters]

    def step(self, tape):
        import gn_bwd
        self.t += 1
        entries = self._entries(tape, [dict(state0=m, state1=v) for m, v in zip(self.m, self.v)])
        gn_bwd.adamw_step(entries, self.lr, self.betas[0], self.betas[1], self.eps,
                          self.weight_decay, step=self.t, clear_grad=True)
        return len(entries)


# ---- GRLY v3 hypernetwork checkpoint (bindings.cpp:2965-3039) -----------------------------
class HypernetworkWeights:
    """The ten weight tensors of the reference's VSAHypernetwork in checkpoint order
    (bindings.cpp:2973-2984), with the model's dimension accessors
    (vsa_hypernetwork.h:39-43).  Tensors are GPU tensors (fp32 or bf16) holding exactly
    grilly_core.hypernetwork_sizes(...) elements each; any shape with that many elements."""

    NAMES = ("W_proj", "b_proj", "W1", "b1", "W2", "b2", "W_r1", "b_r1", "W_r2", "b_r2")

    def __init__(self, d_model, vsa_dim, K, router_hidden=32, tensors=None, device="cuda:0",
                 dtype=None):
        import torch
        self._dims = (int(d_model), int(vsa_dim), int(K), int(router_hidden))
        sizes = grilly_core.hypernetwork_sizes(self._dims)
        if tensors is None:
            tensors = [torch.zeros(n, device=device, dtype=dtype or torch.float32) for n in sizes]
        tensors = list(tensors)
        if len(tensors) != 10 or any(t.numel() != n for t, n in zip(tensors, sizes)):
            raise ValueError(f"HypernetworkWeights: ten tensors of sizes {sizes} expected")
        self.tensors = tensors

    def d_model(self):
        return self._dims[0]

    def vsa_dim(self):
        return self._dims[1]

    def K(self):
        return self._dims[2]

    def router_hidden(self):
        return self._dims[3]

    def num_weight_bufs(self):
        return 10

    def weight_buffers(self):
        return self.tensors

    def dims(self):
        return self._dims


_OPT_KIND = {"SurpriseMomentumOptimizer": 0, "AdamW": 1}


def _dev_list(ts):
    for t in ts:
        if not (t.is_cuda and t.is_contiguous()):
            raise ValueError("checkpoint tensors must be contiguous GPU tensors")
    return [(t.data_ptr(), t.numel(), dtype_code(t)) for t in ts]


def _opt_parts(model, optimizer):
    """(kind, hyper list, state tensors parameter-major, n_states) of an optimizer built over
    model.weight_buffers() in the same order."""
    ws = model.weight_buffers()
    if len(optimizer.weights) != len(ws) or any(a.data_ptr() != b.data_ptr()
                                                for a, b in zip(optimizer.weights, ws)):
        raise ValueError("the optimizer must be built over model.weight_buffers(), in order")
    kind = _OPT_KIND[type(optimizer).__name__]
    if kind == 0:
        per = [[s] + ([optimizer.delta[i]] if optimizer.delta else [])
               for i, s in enumerate(optimizer.s_bar)]
        hyper = [optimizer.eta_base, optimizer.alpha_momentum, optimizer.lambda_recall,
                 optimizer.surprise_floor, optimizer.weight_decay, optimizer.clip_max]
    else:
        per = [[m, v] for m, v in zip(optimizer.m, optimizer.v)]
        hyper = [optimizer.lr, optimizer.betas[0], optimizer.betas[1], optimizer.eps,
                 optimizer.weight_decay]
    return kind, hyper, [t for p in per for t in p], len(per[0])


def save_hypernetwork_weights(model, path, optimizer=None):
    """The reference's save_hypernetwork_weights(model, path) (bindings.cpp:2965-3003): GRLY v3
    header and the ten tensors as fp32.  With an optimizer (SurpriseMomentumOptimizer or AdamW
    over model.weight_buffers()), its fp32 master weights are written in place of the bf16
    copies and its state follows in an optimizer section the reference's loader skips."""
    if optimizer is None:
        grilly_core._grly_save_device(str(path), model.dims(), _dev_list(model.weight_buffers()),
                                      None, [])
        return
    kind, hyper, states, n = _opt_parts(model, optimizer)
    opt = dict(kind=kind, n_states=n, step=int(optimizer.t), hyper=[float(h) for h in hyper])
    grilly_core._grly_save_device(str(path), model.dims(), _dev_list(optimizer.masters), opt,
                                  _dev_list(states))


def load_hypernetwork_weights(model, path, optimizer=None):
    """The reference's load_hypernetwork_weights(model, path) (bindings.cpp:3005-3039): checks
    the magic and dimensions (and, unlike the reference, every tensor's count, so a wrong file
    cannot overrun a buffer).  With an optimizer, the file must hold a section of the same
    kind; masters, state, step and hyper-parameters are restored and bf16 weights receive the
    rounded masters."""
    if optimizer is None:
        grilly_core._grly_load_device(str(path), model.dims(), _dev_list(model.weight_buffers()),
                                      False, [])
        return
    kind, _, states, _ = _opt_parts(model, optimizer)
    _, info = grilly_core._grly_probe(str(path))
    if info is None or info["kind"] != kind:
        raise ValueError(f"{path}: no {type(optimizer).__name__} state in this checkpoint")
    if kind == 0 and info["n_states"] == 2 and not optimizer.delta:
        import torch
        optimizer.delta = [torch.zeros_like(m) for m in optimizer.masters]
        kind, _, states, _ = _opt_parts(model, optimizer)
    opt = grilly_core._grly_load_device(str(path), model.dims(), _dev_list(optimizer.masters),
                                        True, _dev_list(states))
    for w, mw in zip(optimizer.weights, optimizer.masters):
        if w.data_ptr() != mw.data_ptr():
            w.copy_(mw)
    optimizer.t = int(opt["step"])
    h = opt["hyper"]
    if kind == 0:
        (optimizer.eta_base, optimizer.alpha_momentum, optimizer.lambda_recall,
         optimizer.surprise_floor, optimizer.weight_decay, optimizer.clip_max) = h
    else:
        optimizer.lr, b1, b2, optimizer.eps, optimizer.weight_decay = h
        optimizer.betas = (b1, b2)
