"""CPU checks of the C-ABI boundary: the library loads and exports every entry point that
include/gn_bwd.h declares (no compute calls: this container has no GPU)."""
import ctypes
import os
import re

import pytest

from conftest import ROOT, PKG

HEADER = os.path.join(ROOT, "include", "gn_bwd.h")
LIB = os.path.join(PKG, "libgn_bwd.so")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gn_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared()
    for n in ["gn_linear_bwd", "gn_glu_linear_bwd", "gn_rmsnorm_bwd", "gn_layernorm_bwd",
              "gn_xent_bwd", "gn_attn_bwd", "gn_vsa_unpack_project_bwd", "gn_vsa_surrogate_bwd"]:
        assert n in names


@pytest.mark.skipif(not os.path.exists(LIB), reason="libgn_bwd.so not built")
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(LIB)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


PROBE_LIB = os.path.join(PKG, "libgn_probe.so")


@pytest.mark.skipif(not os.path.exists(PROBE_LIB), reason="libgn_probe.so not built")
def test_probe_library_exports_the_probes():
    """The ceiling probes live in libgn_probe.so, not in the backward library."""
    text = re.sub(r"/\*.*?\*/", "", open(os.path.join(ROOT, "include", "gn_probe.h")).read(), flags=re.S)
    names = sorted(set(re.findall(r"\b(gn_[a-z0-9_]+)\s*\(", text)))
    assert names == ["gn_probe_copy", "gn_probe_mfma"]
    probe = ctypes.CDLL(PROBE_LIB)
    assert all(hasattr(probe, n) for n in names)
    assert not any(hasattr(ctypes.CDLL(LIB), n) for n in names)


@pytest.mark.skipif(not os.path.exists(LIB), reason="libgn_bwd.so not built")
def test_python_frontend_lists_every_symbol():
    import gn_bwd
    assert sorted(gn_bwd.SYMBOLS) == declared()
    lib = gn_bwd.lib()
    assert b"gfx950" in lib.gn_version()
    # size queries are pure host arithmetic
    # two fp32 partial rows per block, one block per 8 rows up to 512 blocks
    assert lib.gn_norm_workspace_bytes(4096, 2048) == 2 * 512 * 2048 * 4
    assert lib.gn_norm_workspace_bytes(100, 64) == 2 * 13 * 64 * 4
    assert lib.gn_attn_workspace_bytes(4, 16, 2048, 128) > 0
    assert lib.gn_attn_workspace_bytes(0, 16, 2048, 128) == 0
    # split-K partial planes: ks fp32 planes of dW [N x K] plus ks bias rows, ks in 3..8,
    # only for bf16 weight gradients that leave the GPU under one round of tiles
    BF16, F32 = 4, 0
    plane = 768 * 768 * 4 + 768 * 4
    o_proj = lib.gn_linear_workspace_bytes(8192, 768, 768, BF16)
    assert o_proj in [ks * plane for ks in (3, 4, 6, 8)]
    # fp32 (six-product bf16 MFMA path): K-split planes of the GEMM that has fewer tiles than
    # the grid has blocks, here dW [768 x 768] over 8192 rows (dX [8192 x 768] has enough)
    f32 = lib.gn_linear_workspace_bytes(8192, 768, 768, F32)
    assert f32 in [ks * 768 * 768 * 4 for ks in range(2, 129)]
    assert lib.gn_linear_workspace_bytes(64, 256, 784, F32) == 0  # short reductions: no split
    # the hypernetwork's output layer at batch 64: dX [64 x 1536] over K = 163840
    hyp = lib.gn_linear_workspace_bytes(64, 163840, 1536, F32)
    assert hyp in [ks * 64 * 1536 * 4 for ks in range(2, 129)]
    assert lib.gn_linear_workspace_bytes(64, 256, 784, BF16) == 0  # short reduction: no split
    assert lib.gn_linear_workspace_bytes(8192, 32000, 768, BF16) == 0  # LM head: many tiles
    glu = lib.gn_glu_workspace_bytes(8192, 768, 3072, BF16)
    assert glu in [ks * (6144 * 768 * 4 + 6144 * 4) for ks in (3, 4, 6, 8)]


@pytest.mark.skipif(not os.path.exists(LIB), reason="libgn_bwd.so not built")
def test_invalid_arguments_rejected_without_gpu():
    # argument validation happens before any HIP call
    import gn_bwd
    lib = gn_bwd.lib()
    assert lib.gn_act_bwd(99, None, None, None, 4, 0, 0, None) == -1  # null pointer first
    assert "null" in gn_bwd.last_error()
    assert lib.gn_act_bwd(0, None, None, None, 0, 0, 0, None) == 0  # empty input is a no-op
    assert lib.gn_vsa_unpack_project_bwd(None, None, None, None, 8, 8, 100, 4, 0, 0, None, 0, None) == -1
    assert lib.gn_attn_bwd(None, None, None, None, None, None, None, None, None, 1, 1, 8, 300,
                           1.0, 1, 1, 1e4, 4, None, 0, None) == -1
    # the workspace forms of the two GLU halves validate like their plain forms
    BF16, F32 = 4, 0
    assert lib.gn_ffn_down_glu_bwd_ws(0, None, None, None, None, None, None, None, None, 8, 8, 8,
                                      BF16, 0, None, 0, None) == -1
    assert "null" in gn_bwd.last_error()
    one = ctypes.c_void_p(16)  # never dereferenced: the checks below fail before any launch
    assert lib.gn_ffn_down_glu_bwd_ws(0, one, one, one, one, one, one, one, one, 8, 8, 8, F32, 0,
                                      None, 0, None) == -1
    assert "bf16" in gn_bwd.last_error()
    assert lib.gn_ffn_down_glu_bwd_ws(9, one, one, one, one, one, one, one, one, 8, 8, 8, BF16, 0,
                                      None, 0, None) == -1
    assert lib.gn_glu_proj_bwd_ws(None, None, None, None, None, None, None, None, None, 8, 8, 8,
                                  BF16, 0, None, 0, None) == -1
    assert lib.gn_glu_proj_bwd_ws(one, one, one, one, None, one, None, None, None, 8, 8, 8, BF16, 0,
                                  None, 0, None) == -1  # dWg and dWu go together
    assert lib.gn_glu_proj_bwd_ws(one, one, one, one, None, None, None, None, None, 0, 8, 8, BF16,
                                  0, None, 0, None) == 0  # no rows: nothing to do


@pytest.mark.skipif(not os.path.exists(LIB), reason="libgn_bwd.so not built")
def test_workspace_query_covers_accumulating_launches():
    # QKV weight gradient (2304 x 768 over 8192 rows): the overwriting launch splits in two
    # atomic halves (no workspace), an accumulating one cannot and takes partial planes; the
    # query must size for the latter
    import gn_bwd
    lib = gn_bwd.lib()
    plane = 2304 * 768 * 4 + 2304 * 4
    assert lib.gn_linear_workspace_bytes(8192, 2304, 768, 4) in [ks * plane for ks in (3, 4, 6, 8)]


@pytest.mark.skipif(not os.path.exists(LIB), reason="libgn_bwd.so not built")
def test_fp32_workspace_query_only_sizes_paths_the_shape_takes():
    # M <= 8 rows but K too wide for the skinny kernel's registers (8 rows x 8192): the call
    # takes the split-K GEMM, whose partial planes are a few MiB; the skinny kernel's planes
    # (one M x K plane per row block, ~256 MiB here) must not be asked for
    import gn_bwd
    lib = gn_bwd.lib()
    wide = lib.gn_linear_workspace_bytes(8, 163840, 8192, 0)
    assert wide < 64 << 20
    # a shape the skinny kernel does take (one row, the hypernetwork's output layer) keeps its
    # deterministic dX planes
    assert lib.gn_linear_workspace_bytes(1, 163840, 1536, 0) > 0


@pytest.mark.skipif(not os.path.exists(LIB), reason="libgn_bwd.so not built")
def test_misaligned_attention_views_rejected_without_gpu():
    # the [B,S,H,D] entry takes only 16-byte aligned tensors (its kernels move 16-byte
    # chunks); the check runs before any HIP call, so it is safe without a device
    import gn_bwd
    lib = gn_bwd.lib()
    base = 1 << 20
    p = lambda off=0: ctypes.c_void_p(base + off)
    args = lambda dq_off: (p(0), p(256), p(512), p(4096), p(8192), p(12288), p(dq_off), p(256),
                           p(512), 1, 2, 64, 64, 384, 128, 384, 0.125, 1, 0, 1e4, 4, p(1 << 16),
                           1 << 24, None)
    assert lib.gn_attn_bwd_bshd(*args(2)) == -1
    assert "16-byte aligned" in gn_bwd.last_error()


@pytest.mark.skipif(not os.path.exists(LIB), reason="libgn_bwd.so not built")
def test_attention_row_strides_bounded_without_gpu():
    # the DMA lane offsets of the attention kernels are 32-bit: a [B,S,H,D] row stride of
    # 2^24 elements or more is refused before any HIP call
    import gn_bwd
    lib = gn_bwd.lib()
    base = 1 << 20
    p = lambda off=0: ctypes.c_void_p(base + off)
    big = 1 << 24
    args = (p(0), p(256), p(512), p(4096), p(8192), p(12288), p(16384), p(256), p(512), 1, 2,
            64, 64, big, 128, 384, 0.125, 1, 0, 1e4, 4, p(1 << 16), 1 << 24, None)
    assert lib.gn_attn_bwd_bshd(*args) == -1
    assert "below 2^24" in gn_bwd.last_error()
