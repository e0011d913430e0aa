"""Python front-end of libgn_bwd.so (the C ABI in include/gn_bwd.h).

Device memory and streams come from PyTorch (ROCm build): every function takes torch
tensors that already live on the GPU, passes their raw pointers and the current HIP
stream to the C entry point, and raises GnError on a non-zero status.  There is no CPU
fallback: if the library or a GPU is missing, the call fails loudly.

Function names and argument meaning mirror the reference's backward ops
(src/grilly_next/backend/autograd_core.py:486-654, VulkanBackwardOps) where they exist.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libgn_bwd.so")

F32, F16, U32, I32, BF16 = 0, 1, 2, 3, 4
ACCUMULATE, LN_STAT_VAR, NO_GUMBEL, RMS_STAT_MEANSQ, RMS_STAT_RMS = 1, 2, 4, 8, 16
NORM_PARTIALS = 32
RMS_STAT = {"rstd": 0, "meansq": RMS_STAT_MEANSQ, "rms": RMS_STAT_RMS}
ACT = {"relu": 0, "gelu_tanh": 1, "gelu_erf": 2, "silu": 3, "tanh": 4, "sigmoid": 5}
GLU = {"swiglu_up": 0, "swiglu_gate": 1, "geglu_up": 2, "geglu_gate": 3, "reglu_up": 4}
ROPE = {"none": 0, "interleaved": 1, "half": 2}

# exported symbols, in the order include/gn_bwd.h declares them
SYMBOLS = [
    "gn_last_error", "gn_version", "gn_linear_bwd", "gn_linear_bwd_ws", "gn_linear_workspace_bytes",
    "gn_gemm", "gn_colsum", "gn_act_bwd", "gn_glu_bwd", "gn_glu_linear_bwd", "gn_glu_linear_bwd_ws",
    "gn_glu_workspace_bytes", "gn_glu_proj_bwd", "gn_glu_proj_bwd_ws", "gn_ffn_down_glu_bwd",
    "gn_ffn_down_glu_bwd_ws", "gn_layernorm_bwd",
    "gn_layernorm_bwd_noalloc", "gn_layernorm_bwd_ex", "gn_layernorm_bwd_ex16", "gn_norm_finish", "gn_rmsnorm_bwd", "gn_rmsnorm_bwd_ex",
    "gn_rmsnorm_bwd_stat", "gn_norm_workspace_bytes", "gn_softmax_bwd", "gn_xent_bwd", "gn_attn_bwd",
    "gn_attn_workspace_bytes", "gn_attn_workspace_bytes_dtype", "gn_attn_bwd_bshd", "gn_attn_fwd", "gn_attn_fwd_mask",
    "gn_attn_bwd_mask", "gn_attn_bwd_bshd_mask", "gn_vsa_unpack_project_bwd",
    "gn_vsa_workspace_bytes", "gn_vsa_surrogate_bwd", "gn_vsa_unpack_project_fwd",
    "gn_vsa_fwd_workspace_bytes", "gn_vsa_surrogate_fwd", "gn_embedding_bwd", "gn_binary_bwd",
    "gn_reduce_bwd", "gn_transpose_bwd", "gn_mse_bwd", "gn_vsa_lora_expand_bwd",
    "gn_vsa_cosine_blend_bwd", "gn_surprise_momentum_step", "gn_linear_bwd_surprise_momentum",
    "gn_adamw_step", "gn_layernorm_fwd",
    "gn_rmsnorm_fwd", "gn_layernorm_fwd_ex", "gn_rmsnorm_fwd_ex", "gn_rmsnorm_fwd_stat", "gn_act_fwd", "gn_glu_fwd", "gn_linear_fwd", "gn_glu_linear_fwd", "gn_add_inplace", "gn_convert", "gn_zero",
]
BIN = {"sub": 0, "mul": 1, "div": 2, "neg": 3}
RED = {"sum": 0, "mean": 1}


class GnError(RuntimeError):
    pass


_lib = None
_P = ctypes.c_void_p
_I = ctypes.c_int
_U = ctypes.c_uint
_F = ctypes.c_float
_L = ctypes.c_int64
_Z = ctypes.c_size_t


class OptParam(ctypes.Structure):
    """gn_opt_param (include/gn_bwd.h): one parameter tensor of an optimizer step."""
    _fields_ = [("W", ctypes.c_void_p), ("grad", ctypes.c_void_p), ("state0", ctypes.c_void_p),
                ("state1", ctypes.c_void_p), ("recalled", ctypes.c_void_p),
                ("W_bf16", ctypes.c_void_p), ("n", ctypes.c_int64)]


_OPTP = ctypes.POINTER(OptParam)

_SIGS = {
    "gn_last_error": ([], ctypes.c_char_p),
    "gn_version": ([], ctypes.c_char_p),
    "gn_linear_bwd": ([_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _U, _P], _I),
    "gn_linear_bwd_ws": ([_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _U, _P, _Z, _P], _I),
    "gn_linear_workspace_bytes": ([_I, _I, _I, _I], _Z),
    "gn_gemm": ([_P, _P, _I, _P, _P, _I, _P, _I, _I, _I, _I, _I, _I, _U, _P], _I),
    "gn_colsum": ([_P, _P, _I, _I, _I, _U, _P], _I),
    "gn_act_bwd": ([_I, _P, _P, _P, _L, _I, _U, _P], _I),
    "gn_glu_bwd": ([_I, _P, _P, _P, _P, _P, _L, _I, _P], _I),
    "gn_glu_linear_bwd": ([_I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I,
                           _U, _P], _I),
    "gn_glu_linear_bwd_ws": ([_I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I,
                              _U, _P, _Z, _P], _I),
    "gn_glu_workspace_bytes": ([_I, _I, _I, _I], _Z),
    "gn_glu_proj_bwd": ([_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _U, _P], _I),
    "gn_ffn_down_glu_bwd": ([_I, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _U, _P], _I),
    "gn_glu_proj_bwd_ws": ([_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _U, _P, _Z, _P], _I),
    "gn_ffn_down_glu_bwd_ws": ([_I, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _U, _P, _Z, _P],
                               _I),
    "gn_layernorm_bwd": ([_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _F, _I, _U, _P, _Z, _P], _I),
    "gn_layernorm_bwd_noalloc": ([_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _F, _I, _U, _P], _I),
    "gn_rmsnorm_bwd": ([_P, _P, _P, _P, _P, _P, _I, _I, _I, _U, _P, _Z, _P], _I),
    "gn_layernorm_bwd_ex": ([_P, _I, _P, _I, _P, _P, _P, _P, _P, _P, _P, _I, _I, _F, _U, _P, _Z,
                             _P], _I),
    "gn_norm_finish": ([_P, _I, _P], _I),
    "gn_layernorm_bwd_ex16": ([_P, _I, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _F, _U,
                               _P, _Z, _P], _I),
    "gn_rmsnorm_bwd_ex": ([_P, _I, _P, _I, _P, _P, _P, _P, _P, _I, _I, _U, _P, _Z, _P], _I),
    "gn_rmsnorm_bwd_stat": ([_P, _I, _P, _I, _P, _P, _P, _P, _P, _I, _I, _F, _U, _P, _Z, _P], _I),
    "gn_layernorm_fwd_ex": ([_P, _I, _P, _P, _P, _I, _P, _P, _I, _I, _F, _U, _P], _I),
    "gn_rmsnorm_fwd_ex": ([_P, _I, _P, _P, _I, _P, _I, _I, _F, _P], _I),
    "gn_rmsnorm_fwd_stat": ([_P, _I, _P, _P, _I, _P, _I, _I, _F, _U, _P], _I),
    "gn_convert": ([_P, _I, _P, _I, _L, _P], _I),
    "gn_zero": ([_P, _L, _P], _I),
    "gn_norm_workspace_bytes": ([_I, _I], _Z),
    "gn_softmax_bwd": ([_P, _P, _P, _I, _I, _I, _P], _I),
    "gn_xent_bwd": ([_P, _P, _P, _I, _I, _F, _I, _P], _I),
    "gn_attn_bwd": ([_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _F, _I, _P,
                     _Z, _P], _I),
    "gn_attn_workspace_bytes": ([_I, _I, _I, _I], _Z),
    "gn_attn_workspace_bytes_dtype": ([_I, _I, _I, _I, _I], _Z),
    "gn_attn_bwd_bshd": ([_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _L, _L, _L, _F, _I,
                          _I, _F, _I, _P, _Z, _P], _I),
    "gn_attn_fwd": ([_P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _F, _I, _P, _Z, _P], _I),
    "gn_attn_fwd_mask": ([_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _F, _I, _P, _Z,
                          _P], _I),
    "gn_attn_bwd_mask": ([_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _F,
                          _I, _P, _Z, _P], _I),
    "gn_attn_bwd_bshd_mask": ([_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _L, _L, _L,
                               _F, _I, _I, _F, _I, _P, _Z, _P], _I),
    "gn_vsa_unpack_project_bwd": ([_P, _P, _P, _P, _I, _I, _I, _I, _I, _U, _P, _Z, _P], _I),
    "gn_vsa_workspace_bytes": ([_I, _I], _Z),
    "gn_vsa_surrogate_bwd": ([_P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _F, _F, _F, _U, _P], _I),
    "gn_vsa_unpack_project_fwd": ([_P, _P, _P, _P, _I, _I, _I, _I, _P, _Z, _P], _I),
    "gn_vsa_fwd_workspace_bytes": ([_I, _I, _I], _Z),
    "gn_vsa_surrogate_fwd": ([_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _F, _F, _F,
                              ctypes.c_uint64, ctypes.c_uint64, _U, _P], _I),
    "gn_act_fwd": ([_I, _P, _P, _L, _I, _P], _I),
    "gn_embedding_bwd": ([_P, _P, _P, _I, _I, _I, _I, _U, _P], _I),
    "gn_binary_bwd": ([_I, _P, _P, _P, _P, _P, _L, _I, _U, _P], _I),
    "gn_reduce_bwd": ([_I, _P, _P, _L, _L, _I, _U, _P], _I),
    "gn_transpose_bwd": ([_P, _P, _L, _I, _I, _I, _U, _P], _I),
    "gn_mse_bwd": ([_P, _P, _P, _P, _L, _F, _I, _U, _P], _I),
    "gn_vsa_lora_expand_bwd": ([_P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _U, _P], _I),
    "gn_vsa_cosine_blend_bwd": ([_P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _U, _P], _I),
    "gn_surprise_momentum_step": ([_OPTP, _I, _F, _F, _F, _F, _F, _F, _I, _P], _I),
    "gn_linear_bwd_surprise_momentum": ([_P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _F, _F, _F, _F,
                                         _F, _P, _Z, _P], _I),
    "gn_adamw_step": ([_OPTP, _I, _F, _F, _F, _F, _F, _F, _F, _I, _P], _I),
    "gn_layernorm_fwd": ([_P, _P, _P, _P, _P, _P, _I, _I, _F, _I, _U, _P], _I),
    "gn_rmsnorm_fwd": ([_P, _P, _P, _P, _I, _I, _F, _I, _P], _I),
    "gn_glu_fwd": ([_I, _P, _P, _P, _L, _I, _P], _I),
    "gn_linear_fwd": ([_P, _P, _P, _P, _I, _I, _I, _I, _P], _I),
    "gn_glu_linear_fwd": ([_I, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P], _I),
    "gn_add_inplace": ([_P, _P, _L, _I, _P], _I),
}


def lib():
    """Load libgn_bwd.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise GnError(f"{LIB_PATH} is missing: run python grilly-next_amd/build_native.py")
        l = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGS.items():
            fn = getattr(l, name)
            fn.argtypes = args
            fn.restype = res
        _lib = l
    return _lib


def last_error() -> str:
    return lib().gn_last_error().decode()


def version() -> str:
    return lib().gn_version().decode()


def _check(rc, what):
    if rc != 0:
        raise GnError(f"{what} failed ({rc}): {last_error()}")


# ---------------------------------------------------------------------------------------
import torch  # noqa: E402  (plumbing: device memory and streams)


def _ptr(t):
    if t is None:
        return None
    if not t.is_cuda:
        raise GnError("tensor is not on the GPU")
    if not t.is_contiguous():
        raise GnError("tensor must be contiguous")
    return ctypes.c_void_p(t.data_ptr())


def _off(t, nbytes):
    """Device address nbytes past the start of t (a column block of a row-major buffer)."""
    return ctypes.c_void_p(_ptr(t).value + nbytes)


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dt(t):
    if t.dtype == torch.float32:
        return F32
    if t.dtype == torch.bfloat16:
        return BF16
    raise GnError(f"unsupported dtype {t.dtype}")


def workspace(nbytes, device):
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def linear_workspace_bytes(M, N, K, dtype):
    return int(lib().gn_linear_workspace_bytes(M, N, K, dtype))


def glu_workspace_bytes(M, K, H, dtype):
    return int(lib().gn_glu_workspace_bytes(M, K, H, dtype))


def linear_bwd(dY, X, W, need_dx=True, need_db=True, dX=None, dW=None, db=None, accumulate=False,
               ws=None):
    """(dX, dW, db) for y = X W^T + b.  bf16 inputs give bf16 dX and fp32 dW, db.  ws: the
    split-K workspace (allocated here when None and the shape uses one; False: none)."""
    M, N = dY.shape
    K = X.shape[1]
    dt = _dt(dY)
    if need_dx and dX is None:
        dX = torch.empty((M, K), dtype=dY.dtype, device=dY.device)
    if dW is None:
        dW = torch.empty((N, K), dtype=torch.float32, device=dY.device)
    if need_db and db is None:
        db = torch.empty((N,), dtype=torch.float32, device=dY.device)
    if ws is None:
        nb = linear_workspace_bytes(M, N, K, dt)
        ws = workspace(nb, dY.device) if nb else False
    wsp, wsb = (None, 0) if ws is False else (_ptr(ws), ws.numel() * ws.element_size())
    _check(lib().gn_linear_bwd_ws(_ptr(dY), _ptr(X), _ptr(W), _ptr(dX) if need_dx else None,
                                  _ptr(dW), _ptr(db) if need_db else None, M, N, K, dt,
                                  ACCUMULATE if accumulate else 0, wsp, wsb, _stream()),
           "gn_linear_bwd_ws")
    return (dX if need_dx else None), dW, (db if need_db else None)


def gemm(A0, B0, transA=False, transB=False, A1=None, B1=None, out_dtype=None, C=None,
         accumulate=False):
    K0 = A0.shape[0] if transA else A0.shape[1]
    M = A0.shape[1] if transA else A0.shape[0]
    N = B0.shape[0] if transB else B0.shape[1]
    K1 = 0
    if A1 is not None:
        K1 = A1.shape[0] if transA else A1.shape[1]
    dt = _dt(A0)
    out_dtype = out_dtype or A0.dtype
    if C is None:
        C = torch.empty((M, N), dtype=out_dtype, device=A0.device)
    _check(lib().gn_gemm(_ptr(A0), _ptr(B0), K0, _ptr(A1), _ptr(B1), K1, _ptr(C), M, N,
                         int(transA), int(transB), dt, _dt(C), ACCUMULATE if accumulate else 0,
                         _stream()), "gn_gemm")
    return C


def colsum(x, out=None, accumulate=False):
    M, N = x.shape
    if out is None:
        out = torch.empty((N,), dtype=torch.float32, device=x.device)
    _check(lib().gn_colsum(_ptr(x), _ptr(out), M, N, _dt(x), ACCUMULATE if accumulate else 0,
                           _stream()), "gn_colsum")
    return out


def act_bwd(kind, dY, X, dX=None, accumulate=False):
    if dX is None:
        dX = torch.empty_like(dY)
    _check(lib().gn_act_bwd(ACT[kind], _ptr(dY), _ptr(X), _ptr(dX), dY.numel(), _dt(dY),
                            ACCUMULATE if accumulate else 0, _stream()), "gn_act_bwd")
    return dX


def act_fwd(kind, X, out=None):
    Y = torch.empty_like(X) if out is None else out
    _check(lib().gn_act_fwd(ACT[kind], _ptr(X), _ptr(Y), X.numel(), _dt(X), _stream()), "gn_act_fwd")
    return Y


def glu_bwd(kind, dO, gate, up, dGate=None, dUp=None):
    dGate = torch.empty_like(dO) if dGate is None else dGate
    dUp = torch.empty_like(dO) if dUp is None else dUp
    _check(lib().gn_glu_bwd(GLU[kind], _ptr(dO), _ptr(gate), _ptr(up), _ptr(dGate), _ptr(dUp),
                            dO.numel(), _dt(dO), _stream()), "gn_glu_bwd")
    return dGate, dUp


def glu_linear_bwd(kind, dO, gate, up, X, Wg, Wu, need_dx=True, need_db=False, gu_ws=None,
                   ws=None):
    """Fused GLU-projection backward: (dX, dWg, dWu, dbg, dbu); ws as in linear_bwd."""
    M, H = dO.shape
    K = X.shape[1]
    dev = dO.device
    dX = torch.empty((M, K), dtype=dO.dtype, device=dev) if need_dx else None
    dWg = torch.empty((H, K), dtype=torch.float32, device=dev)
    dWu = torch.empty((H, K), dtype=torch.float32, device=dev)
    dbg = torch.empty((H,), dtype=torch.float32, device=dev) if need_db else None
    dbu = torch.empty((H,), dtype=torch.float32, device=dev) if need_db else None
    if gu_ws is None:
        gu_ws = torch.empty((M, 2 * H), dtype=dO.dtype, device=dev)
    if ws is None:
        nb = glu_workspace_bytes(M, K, H, _dt(dO))
        ws = workspace(nb, dev) if nb else False
    wsp, wsb = (None, 0) if ws is False else (_ptr(ws), ws.numel() * ws.element_size())
    _check(lib().gn_glu_linear_bwd_ws(GLU[kind], _ptr(dO), _ptr(gate), _ptr(up), _ptr(X), _ptr(Wg),
                                      _ptr(Wu), _ptr(dX), _ptr(dWg), _ptr(dWu), _ptr(dbg),
                                      _ptr(dbu), _ptr(gu_ws), M, K, H, _dt(dO), 0, wsp, wsb,
                                      _stream()), "gn_glu_linear_bwd_ws")
    return dX, dWg, dWu, dbg, dbu


def glu_proj_bwd(gu, X, Wg, Wu, need_dx=True, need_db=False, ws=False):
    """Projection half of the GLU backward from gu = [dGate | dUp] ([M, 2H]).  ws: False =
    no workspace (gn_glu_proj_bwd); None = one sized by gn_glu_workspace_bytes, or a uint8
    tensor (gn_glu_proj_bwd_ws)."""
    M, H2 = gu.shape
    H, K = H2 // 2, X.shape[1]
    dev = gu.device
    dX = torch.empty((M, K), dtype=gu.dtype, device=dev) if need_dx else None
    dWg = torch.empty((H, K), dtype=torch.float32, device=dev)
    dWu = torch.empty((H, K), dtype=torch.float32, device=dev)
    dbg = torch.empty((H,), dtype=torch.float32, device=dev) if need_db else None
    dbu = torch.empty((H,), dtype=torch.float32, device=dev) if need_db else None
    args = (_ptr(gu), _ptr(X), _ptr(Wg), _ptr(Wu), _ptr(dX), _ptr(dWg), _ptr(dWu), _ptr(dbg),
            _ptr(dbu), M, K, H, _dt(gu), 0)
    if ws is False:
        _check(lib().gn_glu_proj_bwd(*args, _stream()), "gn_glu_proj_bwd")
    else:
        if ws is None:
            nb = glu_workspace_bytes(M, K, H, _dt(gu))
            ws = workspace(nb, dev) if nb else None
        wsp, wsb = (None, 0) if ws is None else (_ptr(ws), ws.numel() * ws.element_size())
        _check(lib().gn_glu_proj_bwd_ws(*args, wsp, wsb, _stream()), "gn_glu_proj_bwd_ws")
    return dX, dWg, dWu, dbg, dbu


def ffn_down_glu_bwd(kind, dY, A, Wd, gate, up, need_db=False, gu=None, dWd=None, ws=False):
    """Down projection backward with the GLU local gradient fused: (gu, dWd, dbd).  ws as in
    glu_proj_bwd (sized by gn_linear_workspace_bytes(M, N, H); gn_ffn_down_glu_bwd_ws)."""
    M, N = dY.shape
    H = A.shape[1]
    dev = dY.device
    gu = torch.empty((M, 2 * H), dtype=dY.dtype, device=dev) if gu is None else gu
    dWd = torch.empty((N, H), dtype=torch.float32, device=dev) if dWd is None else dWd
    dbd = torch.empty((N,), dtype=torch.float32, device=dev) if need_db else None
    args = (GLU[kind], _ptr(dY), _ptr(A), _ptr(Wd), _ptr(gate), _ptr(up), _ptr(gu), _ptr(dWd),
            _ptr(dbd), M, N, H, _dt(dY), 0)
    if ws is False:
        _check(lib().gn_ffn_down_glu_bwd(*args, _stream()), "gn_ffn_down_glu_bwd")
    else:
        if ws is None:
            nb = linear_workspace_bytes(M, N, H, _dt(dY))
            ws = workspace(nb, dev) if nb else None
        wsp, wsb = (None, 0) if ws is None else (_ptr(ws), ws.numel() * ws.element_size())
        _check(lib().gn_ffn_down_glu_bwd_ws(*args, wsp, wsb, _stream()), "gn_ffn_down_glu_bwd_ws")
    return gu, dWd, dbd


def norm_workspace_bytes(rows, F):
    return int(lib().gn_norm_workspace_bytes(rows, F))


def layernorm_bwd(dY, X, gamma, mean, rstd, eps=1e-5, stat_is_var=False, ws=None,
                  need_param=True, dX_add=None, out=None, dX_bf16=None):
    """(dX, dGamma, dBeta).  dY / gamma may be bf16 under an fp32 X (the _ex entry); dX has
    X's dtype; dX_add (X's dtype, may be `out`) is added to dX in the same pass.  dX_bf16 (fp32
    X): a bf16 tensor that receives dX rounded to bf16 in the same pass (the _ex16 entry)."""
    rows, F = X.shape
    dX = torch.empty_like(X) if out is None else out
    dG = torch.empty((F,), dtype=torch.float32, device=X.device) if need_param else None
    dB = torch.empty((F,), dtype=torch.float32, device=X.device) if need_param else None
    if ws is None:
        ws = workspace(norm_workspace_bytes(rows, F), X.device)
    flags = LN_STAT_VAR if stat_is_var else 0
    if dX_bf16 is not None:
        _check(lib().gn_layernorm_bwd_ex16(_ptr(dY), _dt(dY), _ptr(X), _dt(X), _ptr(gamma), _ptr(mean),
                                           _ptr(rstd), _ptr(dX_add), _ptr(dX), _ptr(dX_bf16), _ptr(dG),
                                           _ptr(dB), rows, F, eps, flags, _ptr(ws), ws.numel(),
                                           _stream()), "gn_layernorm_bwd_ex16")
    elif dX_add is None and dY.dtype == X.dtype:
        _check(lib().gn_layernorm_bwd(_ptr(dY), _ptr(X), _ptr(gamma), _ptr(mean), _ptr(rstd),
                                      _ptr(dX), _ptr(dG), _ptr(dB), rows, F, eps, _dt(X), flags,
                                      _ptr(ws), ws.numel(), _stream()), "gn_layernorm_bwd")
    else:
        _check(lib().gn_layernorm_bwd_ex(_ptr(dY), _dt(dY), _ptr(X), _dt(X), _ptr(gamma), _ptr(mean),
                                         _ptr(rstd), _ptr(dX_add), _ptr(dX), _ptr(dG), _ptr(dB),
                                         rows, F, eps, flags, _ptr(ws), ws.numel(), _stream()),
               "gn_layernorm_bwd_ex")
    return dX, dG, dB


class NormFinish(ctypes.Structure):
    """GnNormFinish (include/gn_bwd.h): one deferred norm backward's parameter gradients."""
    _fields_ = [("ws", ctypes.c_void_p), ("dgamma", ctypes.c_void_p), ("dbeta", ctypes.c_void_p),
                ("rows", ctypes.c_int), ("F", ctypes.c_int), ("layernorm", ctypes.c_int),
                ("accumulate", ctypes.c_int)]


def norm_finish(items):
    """Sum the partial rows of deferred norm backwards (GN_NORM_PARTIALS calls) into their
    parameter gradients, one launch for all: items = [(ws, dgamma, dbeta or None, rows, F,
    layernorm, accumulate), ...]."""
    arr = (NormFinish * max(1, len(items)))()
    for i, (ws, dg, db, rows, F, ln, acc) in enumerate(items):
        arr[i] = NormFinish(_ptr(ws), _ptr(dg), _ptr(db), rows, F, int(ln), int(acc))
    _check(lib().gn_norm_finish(ctypes.cast(arr, ctypes.c_void_p), len(items), _stream()),
           "gn_norm_finish")


def rmsnorm_bwd(dY, X, w, rstd, ws=None, need_param=True, dX=None, dW=None, dX_add=None,
                stat="rstd", eps=1e-6):
    """(dX, dW).  `rstd` holds the per-row statistic named by `stat`: "rstd", "meansq"
    (mean(x^2), rms-norm.glsl:52; eps added) or "rms" (sqrt(mean(x^2) + eps),
    snn-rmsnorm.glsl:55)."""
    rows, F = X.shape
    dX = torch.empty_like(X) if dX is None else dX
    if need_param and dW is None:
        dW = torch.empty((F,), dtype=torch.float32, device=X.device)
    if ws is None:
        ws = workspace(norm_workspace_bytes(rows, F), X.device)
    if stat != "rstd":
        _check(lib().gn_rmsnorm_bwd_stat(_ptr(dY), _dt(dY), _ptr(X), _dt(X), _ptr(w), _ptr(rstd),
                                         _ptr(dX_add), _ptr(dX), _ptr(dW) if need_param else None,
                                         rows, F, eps, RMS_STAT[stat], _ptr(ws), ws.numel(),
                                         _stream()), "gn_rmsnorm_bwd_stat")
    elif dX_add is None and dY.dtype == X.dtype:
        _check(lib().gn_rmsnorm_bwd(_ptr(dY), _ptr(X), _ptr(w), _ptr(rstd), _ptr(dX),
                                    _ptr(dW) if need_param else None, rows, F, _dt(X), 0, _ptr(ws),
                                    ws.numel(), _stream()), "gn_rmsnorm_bwd")
    else:
        _check(lib().gn_rmsnorm_bwd_ex(_ptr(dY), _dt(dY), _ptr(X), _dt(X), _ptr(w), _ptr(rstd),
                                       _ptr(dX_add), _ptr(dX), _ptr(dW) if need_param else None,
                                       rows, F, 0, _ptr(ws), ws.numel(), _stream()),
               "gn_rmsnorm_bwd_ex")
    return dX, (dW if need_param else None)


def zero(t):
    """t[...] = 0 through the library's fill kernel (what it clears with instead of
    hipMemsetAsync); t must be contiguous."""
    assert t.is_contiguous()
    _check(lib().gn_zero(_ptr(t), t.numel() * t.element_size(), _stream()), "gn_zero")
    return t


def convert(src, dtype):
    """src in another storage dtype (f32 <-> bf16, nearest-even; the same dtype copies)."""
    out = torch.empty(src.shape, dtype=dtype, device=src.device)
    _check(lib().gn_convert(_ptr(src), _dt(src), _ptr(out), _dt(out), src.numel(), _stream()),
           "gn_convert")
    return out


def softmax_bwd(dY, Y):
    rows, C = Y.shape
    dX = torch.empty_like(Y)
    _check(lib().gn_softmax_bwd(_ptr(dY), _ptr(Y), _ptr(dX), rows, C, _dt(Y), _stream()),
           "gn_softmax_bwd")
    return dX


def xent_bwd(logits, targets, scale=1.0, dLogits=None):
    rows, C = logits.shape
    dLogits = torch.empty_like(logits) if dLogits is None else dLogits
    t = targets.to(torch.int32).contiguous()
    _check(lib().gn_xent_bwd(_ptr(logits), _ptr(t), _ptr(dLogits), rows, C, scale, _dt(logits),
                             _stream()), "gn_xent_bwd")
    return dLogits


def attn_workspace_bytes(B, H, S, D, dtype=None):
    """Workspace bytes for one dtype (torch dtype or a GN_* code); None: either dtype."""
    if dtype is None:
        return int(lib().gn_attn_workspace_bytes(B, H, S, D))
    code = dtype if isinstance(dtype, int) else (BF16 if dtype == torch.bfloat16 else F32)
    return int(lib().gn_attn_workspace_bytes_dtype(B, H, S, D, code))


def attn_bwd(Q, K, V, O, dO, LSE, scale=None, causal=True, rope="interleaved", theta=10000.0,
             ws=None, out=None, mask=None):
    """(dQ, dK, dV).  mask: fp32 [B, S] key-padding mask (1 keep, 0 masked), or None."""
    B, H, S, D = Q.shape
    scale = D ** -0.5 if scale is None else scale
    dQ, dK, dV = out if out is not None else (torch.empty_like(Q), torch.empty_like(K),
                                              torch.empty_like(V))
    if ws is None:
        ws = workspace(attn_workspace_bytes(B, H, S, D, Q.dtype), Q.device)
    if mask is None:
        _check(lib().gn_attn_bwd(_ptr(Q), _ptr(K), _ptr(V), _ptr(O), _ptr(dO), _ptr(LSE), _ptr(dQ),
                                 _ptr(dK), _ptr(dV), B, H, S, D, scale, int(causal), ROPE[rope],
                                 theta, _dt(Q), _ptr(ws), ws.numel(), _stream()), "gn_attn_bwd")
    else:
        _check(lib().gn_attn_bwd_mask(_ptr(Q), _ptr(K), _ptr(V), _ptr(O), _ptr(dO), _ptr(LSE),
                                      _ptr(mask), _ptr(dQ), _ptr(dK), _ptr(dV), B, H, S, D, scale,
                                      int(causal), ROPE[rope], theta, _dt(Q), _ptr(ws), ws.numel(),
                                      _stream()), "gn_attn_bwd_mask")
    return dQ, dK, dV


def attn_bwd_qkv(qkv, O, dO, LSE, heads, scale=None, causal=True, rope="none", theta=10000.0,
                 ws=None, out=None, mask=None):
    """Backward on a fused QKV projection output qkv [B, S, 3*H*D] (Q | K | V along the last
    axis, each [B, S, H, D]); O, dO [B, S, H*D]; LSE [B, H, S]; mask: fp32 [B, S] key-padding
    mask or None.  Returns dqkv like qkv."""
    B, S, C3 = qkv.shape
    D = C3 // (3 * heads)
    HD = heads * D
    scale = D ** -0.5 if scale is None else scale
    dqkv = out if out is not None else torch.empty_like(qkv)
    if ws is None:
        ws = workspace(attn_workspace_bytes(B, heads, S, D, qkv.dtype), qkv.device)
    e = qkv.element_size()
    _check(lib().gn_attn_bwd_bshd_mask(_ptr(qkv), _off(qkv, HD * e), _off(qkv, 2 * HD * e),
                                       _ptr(O), _ptr(dO), _ptr(LSE), _ptr(mask), _ptr(dqkv),
                                       _off(dqkv, HD * e), _off(dqkv, 2 * HD * e), B, heads, S, D,
                                       C3, O.shape[-1], C3, scale, int(causal), ROPE[rope], theta,
                                       _dt(qkv), _ptr(ws), ws.numel(), _stream()),
           "gn_attn_bwd_bshd")
    return dqkv


def attn_fwd(Q, K, V, scale=None, causal=True, rope="interleaved", theta=10000.0, ws=None,
             mask=None):
    """(O, LSE).  mask: fp32 [B, S] key-padding mask (1 keep, 0 masked), or None."""
    B, H, S, D = Q.shape
    scale = D ** -0.5 if scale is None else scale
    O = torch.empty_like(Q)
    LSE = torch.empty((B, H, S), dtype=torch.float32, device=Q.device)
    if ws is None:
        ws = workspace(attn_workspace_bytes(B, H, S, D, Q.dtype), Q.device)
    _check(lib().gn_attn_fwd_mask(_ptr(Q), _ptr(K), _ptr(V), _ptr(mask), _ptr(O), _ptr(LSE), B,
                                  H, S, D, scale, int(causal), ROPE[rope], theta, _dt(Q), _ptr(ws),
                                  ws.numel(), _stream()), "gn_attn_fwd")
    return O, LSE


def vsa_workspace_bytes(Bn, O):
    return lib().gn_vsa_workspace_bytes(Bn, O)


def vsa_unpack_project_bwd(dY, bits, D, need_db=True, dW=None, db=None, accumulate=False, ws=None):
    """dW[o, j] (+)= sum_b dY[b, o] s_b(j) and db = sum_b dY[b]; the MFMA path uses a
    workspace of vsa_workspace_bytes(Bn, O) (allocated here when not given; ws=False runs
    the LDS-staging kernel without one)."""
    Bn, O = dY.shape
    words = bits.shape[1]
    if dW is None:
        dW = torch.empty((O, D), dtype=torch.float32, device=dY.device)
    if need_db and db is None:
        db = torch.empty((O,), dtype=torch.float32, device=dY.device)
    if ws is None:
        ws = workspace(vsa_workspace_bytes(Bn, O), dY.device)
    ws = ws if ws is not None and ws is not False else None
    _check(lib().gn_vsa_unpack_project_bwd(_ptr(dY), _ptr(bits), _ptr(dW),
                                           _ptr(db) if need_db else None, Bn, O, D, words,
                                           _dt(dY), ACCUMULATE if accumulate else 0,
                                           _ptr(ws) if ws is not None else None,
                                           ws.numel() * ws.element_size() if ws is not None else 0,
                                           _stream()), "gn_vsa_unpack_project_bwd")
    return dW, (db if need_db else None)


def vsa_surrogate_bwd(preds, bits, results, weights, gamma=1.0, delta=1.0, lambda_c=0.3,
                      scale=1.0, dPreds=None, accumulate=False):
    Bn, K, D = preds.shape
    words = bits.shape[1]
    dPreds = torch.empty_like(preds) if dPreds is None else dPreds
    _check(lib().gn_vsa_surrogate_bwd(_ptr(preds), _ptr(bits), _ptr(results), _ptr(weights),
                                      _ptr(dPreds), Bn, K, D, words, gamma, delta, lambda_c,
                                      scale, ACCUMULATE if accumulate else 0, _stream()),
           "gn_vsa_surrogate_bwd")
    return dPreds


def vsa_fwd_workspace_bytes(Bn, O, D):
    return int(lib().gn_vsa_fwd_workspace_bytes(Bn, O, D))


def vsa_unpack_project_fwd(bits, W, bias=None, ws=None):
    """Y [Bn, O] = unpack(bits) W^T + bias (fp32).  ws: the MFMA path's operand workspace
    (allocated here when None and the batch uses one; False: the streaming kernel only)."""
    Bn, words = bits.shape
    O, D = W.shape
    Y = torch.empty((Bn, O), dtype=torch.float32, device=W.device)
    if ws is None:
        nb = vsa_fwd_workspace_bytes(Bn, O, D)
        ws = workspace(nb, W.device) if nb else False
    wsp, wsb = (None, 0) if ws is False else (_ptr(ws), ws.numel())
    _check(lib().gn_vsa_unpack_project_fwd(_ptr(bits), _ptr(W), _ptr(bias), _ptr(Y), Bn, O, D,
                                           words, wsp, wsb, _stream()), "gn_vsa_unpack_project_fwd")
    return Y


def vsa_surrogate_fwd(preds, bits, gamma=1.0, delta=1.0, lambda_c=0.3, temperature=1.0, seed=0,
                      counter=0, noise=True):
    """(dots [Bn,K], results u32 [Bn,4] as int32 storage, weights [Bn,K], loss [Bn])."""
    Bn, K, D = preds.shape
    words = bits.shape[1]
    dev = preds.device
    dots = torch.empty((Bn, K), dtype=torch.float32, device=dev)
    results = torch.empty((Bn, 4), dtype=torch.int32, device=dev)
    weights = torch.empty((Bn, K), dtype=torch.float32, device=dev)
    loss = torch.empty((Bn,), dtype=torch.float32, device=dev)
    _check(lib().gn_vsa_surrogate_fwd(_ptr(preds), _ptr(bits), _ptr(dots), _ptr(results),
                                      _ptr(weights), _ptr(loss), Bn, K, D, words, gamma, delta,
                                      lambda_c, temperature, seed, counter,
                                      0 if noise else NO_GUMBEL, _stream()),
           "gn_vsa_surrogate_fwd")
    return dots, results, weights, loss


def embedding_bwd(dX, ids, V, dE=None, accumulate=False):
    """dE[ids[t]] (+)= dX[t]; dE fp32 [V, d]; ids int32 [T]."""
    T, d = dX.shape
    dE = torch.empty(V, d, device=dX.device) if dE is None else dE
    _check(lib().gn_embedding_bwd(_ptr(dX), _ptr(ids), _ptr(dE), T, d, V, _dt(dX),
                                  ACCUMULATE if accumulate else 0, _stream()), "gn_embedding_bwd")
    return dE


def binary_bwd(op, dY, A=None, B=None, need_da=True, need_db=True):
    """Sub / Mul / Div / Neg backward (no broadcasting); returns (dA, dB)."""
    dA = torch.empty_like(dY) if need_da else None
    dB = torch.empty_like(dY) if (need_db and op != "neg") else None
    _check(lib().gn_binary_bwd(BIN[op], _ptr(dY), _ptr(A), _ptr(B), _ptr(dA), _ptr(dB),
                               dY.numel(), _dt(dY), 0, _stream()), "gn_binary_bwd")
    return dA, dB


def reduce_bwd(op, dY, shape):
    """Sum / Mean over the trailing elements: dY has one value per output row."""
    dX = torch.empty(shape, dtype=dY.dtype, device=dY.device)
    outer = dY.numel()
    _check(lib().gn_reduce_bwd(RED[op], _ptr(dY), _ptr(dX), outer, dX.numel() // max(outer, 1),
                               _dt(dY), 0, _stream()), "gn_reduce_bwd")
    return dX


def transpose_bwd(dY):
    """dY [..., cols, rows] -> dX [..., rows, cols]."""
    *lead, cols, rows = dY.shape
    dX = torch.empty(*lead, rows, cols, dtype=dY.dtype, device=dY.device)
    batch = dX.numel() // max(rows * cols, 1)
    _check(lib().gn_transpose_bwd(_ptr(dY), _ptr(dX), batch, rows, cols, _dt(dY), 0, _stream()),
           "gn_transpose_bwd")
    return dX


def mse_bwd(pred, target, scale=None, dLoss=None):
    dP = torch.empty_like(pred)
    scale = 1.0 / pred.numel() if scale is None else scale
    _check(lib().gn_mse_bwd(_ptr(pred), _ptr(target), _ptr(dLoss), _ptr(dP), pred.numel(), scale,
                            _dt(pred), 0, _stream()), "gn_mse_bwd")
    return dP


def vsa_lora_expand_bwd(dPreds, basis, coeffs):
    """dPreds [Bn, K, D] fp32, basis [D, rank], coeffs [Bn, K, rank] -> (dCoeffs, dBasis)."""
    Bn, K, D = dPreds.shape
    rank = basis.shape[1]
    dC = torch.empty(Bn, K, rank, device=dPreds.device)
    dB = torch.empty(D, rank, device=dPreds.device)
    _check(lib().gn_vsa_lora_expand_bwd(_ptr(dPreds), _ptr(basis), _ptr(coeffs), _ptr(dC), _ptr(dB),
                                        Bn, K, D, rank, 1.0, 0, _stream()), "gn_vsa_lora_expand_bwd")
    return dC, dB


def vsa_cosine_blend_bwd(bits, weights, blended, loss_info, K, grad_scale=10.0):
    """bits [Bn, words] (int32 view of u32), weights [Bn, K], blended [Bn, D], loss_info [Bn, 3]."""
    Bn, D = blended.shape
    dP = torch.empty(Bn, K, D, device=blended.device)
    _check(lib().gn_vsa_cosine_blend_bwd(_ptr(bits), _ptr(weights), _ptr(blended), _ptr(loss_info),
                                         _ptr(dP), Bn, K, D, bits.shape[1], grad_scale, 0, _stream()),
           "gn_vsa_cosine_blend_bwd")
    return dP


def _addr(x):
    """Device address of a tensor (its data pointer) or of a raw buffer id (int); None -> 0."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if not x.is_cuda or not x.is_contiguous():
        raise GnError("optimizer tensors must be contiguous GPU tensors")
    return x.data_ptr()


def _opt_params(entries):
    arr = (OptParam * max(1, len(entries)))()
    for i, e in enumerate(entries):
        W = e["W"]
        if W.dtype != torch.float32:
            raise GnError("optimizer weights (masters) must be float32")
        n = W.numel()
        for key in ("grad", "state0", "state1", "recalled"):
            x = e.get(key)
            if x is not None and not isinstance(x, int) and (x.numel() != n or x.dtype != torch.float32):
                raise GnError(f"optimizer tensor {i}: {key} must be float32 with {n} elements")
        lp = e.get("W_bf16")
        if lp is not None and (lp.numel() != n or lp.dtype != torch.bfloat16):
            raise GnError(f"optimizer tensor {i}: W_bf16 must be bfloat16 with {n} elements")
        arr[i] = OptParam(_addr(W), _addr(e["grad"]), _addr(e["state0"]), _addr(e.get("state1")),
                          _addr(e.get("recalled")), _addr(lp), n)
    return arr


def surprise_momentum_step(entries, eta_base=1e-3, alpha=0.9, lambda_recall=0.0,
                           surprise_floor=0.01, weight_decay=0.0, clip_max=1.0, clear_grad=True):
    """entries: dicts with W, grad, state0 (= s_bar), optional state1 (= delta), recalled,
    W_bf16.  grad may be a raw device address (a tape gradient buffer id)."""
    arr = _opt_params(entries)
    _check(lib().gn_surprise_momentum_step(arr, len(entries), eta_base, alpha, lambda_recall,
                                           surprise_floor, weight_decay, clip_max,
                                           int(clear_grad), _stream()),
           "gn_surprise_momentum_step")


def linear_bwd_surprise_momentum(dY, X, W, s_bar, eta_base=1e-3, alpha=0.9, lambda_recall=0.0,
                                 surprise_floor=0.01, weight_decay=0.0, clip_max=1.0,
                                 need_dx=True, need_db=True, ws=None):
    """fp32 Linear backward of a few rows with W's surprise-momentum step fused in: W and
    s_bar are updated in place, dW is never formed in memory.  Returns (dX, db)."""
    M, N = dY.shape
    K = X.shape[1]
    dX = torch.empty((M, K), dtype=torch.float32, device=dY.device) if need_dx else None
    db = torch.empty((N,), dtype=torch.float32, device=dY.device) if need_db else None
    if ws is None:
        nb = linear_workspace_bytes(M, N, K, F32)
        ws = workspace(nb, dY.device) if nb else False
    wsp, wsb = (None, 0) if ws is False else (_ptr(ws), ws.numel() * ws.element_size())
    _check(lib().gn_linear_bwd_surprise_momentum(_ptr(dY), _ptr(X), _ptr(W), _ptr(s_bar), _ptr(dX),
                                                 _ptr(db), M, N, K, eta_base, alpha, lambda_recall,
                                                 surprise_floor, weight_decay, clip_max, wsp, wsb,
                                                 _stream()),
           "gn_linear_bwd_surprise_momentum")
    return dX, db


def adamw_step(entries, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.0, step=1,
               clear_grad=True):
    """entries: dicts with W, grad, state0 (= m), state1 (= v), optional W_bf16.  The bias
    corrections beta^step are taken from the fp32 betas the kernel receives, so the step
    depends only on fp32 hyper-parameters (a resumed checkpoint continues bit for bit)."""
    arr = _opt_params(entries)
    b1, b2 = ctypes.c_float(beta1).value, ctypes.c_float(beta2).value
    _check(lib().gn_adamw_step(arr, len(entries), lr, beta1, beta2, eps, weight_decay,
                               b1 ** step, b2 ** step, int(clear_grad), _stream()),
           "gn_adamw_step")


# ---- forward kernels (the saved tensors the backward consumes) ------------------------------
def layernorm_fwd(X, gamma=None, beta=None, eps=1e-5, save_var=False, out_dtype=None):
    """Y, mean, rstd (fp32 [rows]; the variance instead of rstd when save_var).  out_dtype:
    Y's dtype (default X's; bf16 under an fp32 X normalises a residual stream into a bf16
    block, gamma / beta then bf16)."""
    rows, F = X.shape
    Y = torch.empty(X.shape, dtype=out_dtype or X.dtype, device=X.device)
    mean = torch.empty((rows,), dtype=torch.float32, device=X.device)
    rstd = torch.empty((rows,), dtype=torch.float32, device=X.device)
    _check(lib().gn_layernorm_fwd_ex(_ptr(X), _dt(X), _ptr(gamma), _ptr(beta), _ptr(Y), _dt(Y),
                                     _ptr(mean), _ptr(rstd), rows, F, eps,
                                     LN_STAT_VAR if save_var else 0, _stream()), "gn_layernorm_fwd")
    return Y, mean, rstd


def rmsnorm_fwd(X, w=None, eps=1e-6, out_dtype=None, stat="rstd"):
    """Y, and the per-row statistic named by `stat` (fp32 [rows]): "rstd", "meansq" or "rms"
    (the reference's saved forms, as rmsnorm_bwd takes them)."""
    rows, F = X.shape
    Y = torch.empty(X.shape, dtype=out_dtype or X.dtype, device=X.device)
    rstd = torch.empty((rows,), dtype=torch.float32, device=X.device)
    _check(lib().gn_rmsnorm_fwd_stat(_ptr(X), _dt(X), _ptr(w), _ptr(Y), _dt(Y), _ptr(rstd), rows,
                                     F, eps, RMS_STAT[stat], _stream()), "gn_rmsnorm_fwd")
    return Y, rstd


def glu_fwd(kind, gate, up, out=None):
    out = torch.empty_like(gate) if out is None else out
    _check(lib().gn_glu_fwd(GLU[kind], _ptr(gate), _ptr(up), _ptr(out), gate.numel(), _dt(gate),
                            _stream()), "gn_glu_fwd")
    return out


def linear_fwd(X, W, b=None, out=None):
    """Y = X W^T + b in X's dtype."""
    M, K = X.shape
    N = W.shape[0]
    Y = torch.empty((M, N), dtype=X.dtype, device=X.device) if out is None else out
    _check(lib().gn_linear_fwd(_ptr(X), _ptr(W), _ptr(b), _ptr(Y), M, N, K, _dt(X), _stream()),
           "gn_linear_fwd")
    return Y


def glu_linear_fwd(kind, X, Wg, Wu, bg=None, bu=None):
    """gate, up (the backward's caches) and out = glu(gate, up)."""
    M, K = X.shape
    H = Wg.shape[0]
    gate = torch.empty((M, H), dtype=X.dtype, device=X.device)
    up = torch.empty_like(gate)
    out = torch.empty_like(gate)
    _check(lib().gn_glu_linear_fwd(GLU[kind], _ptr(X), _ptr(Wg), _ptr(Wu), _ptr(bg), _ptr(bu),
                                   _ptr(gate), _ptr(up), _ptr(out), M, H, K, _dt(X), _stream()),
           "gn_glu_linear_fwd")
    return gate, up, out


def add_inplace(out, a):
    _check(lib().gn_add_inplace(_ptr(out), _ptr(a), out.numel(), _dt(out), _stream()),
           "gn_add_inplace")
    return out


def u32_tensor(arr, device):
    """numpy uint32 -> device tensor holding the same bits (torch has no uint32 kernels)."""
    import numpy as np
    a = np.ascontiguousarray(arr, dtype=np.uint32)
    return torch.from_numpy(a.view(np.int32)).to(device)
