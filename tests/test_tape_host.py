"""Host-side checks of the tape engine module (no GPU needed): the OpType numbering and
TensorRef contract of the reference (cpp/include/grilly/autograd/autograd.h:46-141), the
arena's failure behaviour (tape_arena.h:94-108) and the parameter-block layouts."""
import os
import struct

import pytest

from conftest import PKG

if not any(f.startswith("_grilly_core") and f.endswith(".so") for f in os.listdir(PKG)):
    pytest.skip("_grilly_core (grilly_core's extension) not built", allow_module_level=True)

import grilly_core  # noqa: E402
import grilly_bridge as gb  # noqa: E402

# autograd.h:81-141, in declaration order
REFERENCE_OPS = ["Add", "Sub", "Mul", "Div", "Neg", "Pow", "MatMul", "Linear", "ReLU", "GELU",
                 "SiLU", "Tanh", "Sigmoid", "Softmax", "LayerNorm", "RMSNorm", "FlashAttention2",
                 "Conv2d", "Conv1d", "Sum", "Mean", "Max", "Min", "Reshape", "Transpose", "Slice",
                 "CrossEntropy", "MSELoss", "CubeMindSurprise", "TemporalSurprise",
                 "VSAUnpackProject", "VSASurrogateLoss", "VSALoRAExpand", "VSACosineBlendLoss"]


def test_optype_numbering_matches_reference():
    for i, name in enumerate(REFERENCE_OPS):
        assert getattr(grilly_core.OpType, name).value == i, name
    assert grilly_core.OpType.FusedGLU.value == len(REFERENCE_OPS)


def test_tensor_ref_contract():
    r = grilly_core.TensorRef()
    assert not r.valid() and r.ndim == 0
    r.set_shape([4, 3, 2])
    assert r.get_shape() == [4, 3, 2] and r.numel() == 24
    for dtype, size in [(0, 4), (1, 2), (2, 4), (3, 4), (4, 2)]:
        r.dtype = dtype
        assert r.size_bytes() == 24 * size
    r.buffer_id = 0xDEADBEEF00
    assert r.valid()
    with pytest.raises(ValueError):
        r.set_shape([1] * 9)
    none = grilly_core.TensorRef.none()
    assert none.buffer_id == 0 and not none.requires_grad
    ref = gb.make_tensor_ref(1234, (2, 5), gb.DTYPE_BF16, True)
    assert ref.get_shape() == [2, 5] and ref.dtype == 4 and ref.requires_grad


def test_arena_overflow_raises_memory_error():
    a = grilly_core._TapeArena(4096)
    a.allocate(4000)
    with pytest.raises(MemoryError):
        a.allocate(200)
    a.reset()
    assert a.bytes_used() == 0
    p1 = a.allocate(10, 64)
    assert p1 % 64 == 0
    mark = a.save()
    a.allocate(100)
    a.restore(mark)
    assert a.bytes_used() == mark


def test_node_is_fixed_size():
    # a fixed-size arena object: ~1.1 KiB, so a 12-layer decoder tape fits easily in 64 MiB
    assert 1000 < grilly_core.NODE_BYTES < 1300


def test_param_blocks():
    assert len(gb.vsa_surrogate_params(4, 10240)) == 40
    # AttentionParams: scale, causal, rope_mode, rope_theta, layout, heads
    assert len(gb.attention_params()) == 24
    assert struct.unpack("<fIIfII", gb.attention_params(fused_qkv_heads=12))[4:] == (1, 12)
    assert struct.unpack("<fIIfII", gb.attention_params())[4:] == (0, 0)
    assert len(gb.layernorm_params()) == 8
    assert struct.unpack("<I", gb.embedding_params(32000)) == (32000,)


def test_optype_numbering_extends_the_reference():
    # the reference's values end at VSACosineBlendLoss = 33; this build appends two
    assert int(grilly_core.OpType.FusedGLU) == 34
    assert int(grilly_core.OpType.Embedding) == 35


def test_device_without_gpu_fails_loudly():
    try:
        import torch
        if torch.cuda.is_available():
            pytest.skip("a GPU is present")
    except ImportError:
        pass
    with pytest.raises(RuntimeError, match="no HIP device"):
        grilly_core.Device()


def test_opgraph_api_matches_reference_names():
    """grilly_core.OpGraph carries the reference's Python surface (bindings.cpp:212-235:
    OpGraph(), size, clear, optimize(device) -> dict, execute(device)); an empty graph needs
    no GPU to build, size or clear."""
    g = grilly_core.OpGraph()
    for name in ("size", "clear", "optimize", "execute", "begin_capture", "end_capture",
                 "capture_backward", "get_grad_buffer", "node_counts", "replays"):
        assert callable(getattr(g, name)), name
    assert g.size() == 0 and not g.is_capturing() and g.replays() == 0
    assert g.get_grad_buffer(0x1000) == 0
    assert g.node_counts() == {"kernel": 0, "memcpy": 0, "memset": 0, "other": 0}
    g.clear()
    with pytest.raises(RuntimeError, match="no capture is open"):
        g.end_capture()


def test_library_code_is_capturable():
    """No kernel-library source and no tape source on the backward path clears, copies,
    allocates or synchronises through the HIP runtime: a HIP graph captured from them holds
    kernel nodes only (the runtime's memset nodes are avoided on purpose).  The device pool
    (device.cpp) allocates outside any capture, or relaxed-mode inside one."""
    import glob
    import re
    csrc = os.path.join(PKG, "csrc")
    banned = re.compile(r"\b(hipMemsetAsync|hipMemset|hipMemcpy|hipMemcpyAsync|hipMalloc|hipFree|"
                        r"hipStreamSynchronize|hipDeviceSynchronize)\s*\(")
    files = glob.glob(os.path.join(csrc, "*.hip")) + [os.path.join(csrc, "tape", "autograd.cpp")]
    hits = []
    for f in files:
        for i, line in enumerate(open(f), 1):
            code = line.split("//", 1)[0]
            if banned.search(code):
                hits.append(f"{os.path.relpath(f, PKG)}:{i}: {line.strip()}")
    assert not hits, hits
