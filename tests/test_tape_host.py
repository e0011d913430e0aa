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
