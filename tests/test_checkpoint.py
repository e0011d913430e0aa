"""GRLY v3 hypernetwork checkpoint (bindings.cpp:2965-3039) on the host layer: byte layout,
round trips, the optimizer section, and the loader's checks.  No GPU needed; the device
round trip is in tests/test_gpu_tape.py.

The expected bytes are assembled here with struct from the reference's writer as it reads:
header u32[6] = {0x47524C59, d_model, vsa_dim, K, 10, router_hidden} (bindings.cpp:2994-2995),
then per tensor u32 count + f32 data (bindings.cpp:2997-3000), counts from bindings.cpp:2973-2984.
"""
import struct

import numpy as np
import pytest

import grilly_core

DIMS = (4, 8, 2, 3)  # d_model, vsa_dim, K, router_hidden


def ref_sizes(d, v, K, rh):
    h = 2 * d
    return [d * v, d, h * d, h, K * v * h, K * v, rh * d, rh, K * rh, K]


def tensors(seed, dims=DIMS):
    r = np.random.default_rng(seed)
    return [r.standard_normal(n).astype(np.float32) for n in ref_sizes(*dims)]


def reference_bytes(dims, ws):
    out = struct.pack("<6I", 0x47524C59, dims[0], dims[1], dims[2], 10, dims[3])
    for w in ws:
        out += struct.pack("<I", w.size) + w.astype("<f4").tobytes()
    return out


def test_sizes_match_the_reference_table():
    assert list(grilly_core.hypernetwork_sizes(DIMS)) == ref_sizes(*DIMS)
    # the reference model's defaults (vsa_hypernetwork.h:27-30): 768, 10240, K 16, 32
    assert list(grilly_core.hypernetwork_sizes((768, 10240, 16, 32))) == ref_sizes(768, 10240, 16, 32)
    with pytest.raises(ValueError):  # K * vsa_dim * 2 d_model beyond a 32-bit count
        grilly_core.hypernetwork_sizes((65536, 65536, 4, 32))


def test_writer_produces_the_reference_layout(tmp_path):
    ws = tensors(1)
    p = tmp_path / "a.grly"
    grilly_core._grly_write(str(p), DIMS, ws, None, [])
    assert p.read_bytes() == reference_bytes(DIMS, ws)


def test_reader_reads_a_reference_file(tmp_path):
    ws = tensors(2)
    p = tmp_path / "b.grly"
    p.write_bytes(reference_bytes(DIMS, ws))
    got, opt, st = grilly_core._grly_read(str(p), DIMS)
    assert opt is None and st == []
    for a, b in zip(got, ws):
        np.testing.assert_array_equal(a, b)
    dims, info = grilly_core._grly_probe(str(p))
    assert tuple(dims) == DIMS and info is None


def test_reader_rejects_bad_files(tmp_path):
    ws = tensors(3)
    good = reference_bytes(DIMS, ws)
    p = tmp_path / "c.grly"
    p.write_bytes(b"XXXX" + good[4:])
    with pytest.raises(RuntimeError, match="Invalid checkpoint magic"):
        grilly_core._grly_read(str(p), DIMS)
    p.write_bytes(good)
    with pytest.raises(RuntimeError, match="Model dimension mismatch"):
        grilly_core._grly_read(str(p), (4, 8, 3, 3))
    with pytest.raises(RuntimeError, match="router_hidden"):
        grilly_core._grly_read(str(p), (4, 8, 2, 5))
    p.write_bytes(good[:-5])
    with pytest.raises(RuntimeError, match="truncated"):
        grilly_core._grly_read(str(p), DIMS)
    # a tensor whose stored count differs from the model's (the reference would overrun)
    bad = bytearray(good)
    struct.pack_into("<I", bad, 24, ws[0].size + 1)
    p.write_bytes(bytes(bad))
    with pytest.raises(RuntimeError, match="W_proj"):
        grilly_core._grly_read(str(p), DIMS)
    with pytest.raises(RuntimeError, match="Cannot open"):
        grilly_core._grly_read(str(tmp_path / "missing.grly"), DIMS)


def test_optimizer_section_round_trip_and_reference_prefix(tmp_path):
    ws = tensors(4)
    r = np.random.default_rng(5)
    sizes = ref_sizes(*DIMS)
    states = [r.standard_normal(sizes[i // 2]).astype(np.float32) for i in range(20)]
    opt = dict(kind=1, n_states=2, step=7, hyper=[1e-3, 0.9, 0.999, 1e-8, 0.01])
    p = tmp_path / "d.grly"
    grilly_core._grly_write(str(p), DIMS, ws, opt, states)
    data = p.read_bytes()
    prefix = reference_bytes(DIMS, ws)
    # the reference's loader reads exactly this prefix and stops
    assert data[:len(prefix)] == prefix
    sec = data[len(prefix):]
    assert struct.unpack_from("<4IQI", sec) == (0x54504F47, 1, 1, 2, 7, 5)
    got, info, st = grilly_core._grly_read(str(p), DIMS, opt_states=2)
    assert info["kind"] == 1 and info["n_states"] == 2 and info["step"] == 7
    np.testing.assert_array_equal(np.float32(info["hyper"]), np.float32(opt["hyper"]))
    for a, b in zip(got + st, ws + states):
        np.testing.assert_array_equal(a, b)
    # weights alone still load; the wrong state count and a missing section are errors
    got2, _, _ = grilly_core._grly_read(str(p), DIMS)
    np.testing.assert_array_equal(got2[4], ws[4])
    with pytest.raises(RuntimeError, match="expected 1"):
        grilly_core._grly_read(str(p), DIMS, opt_states=1)
    q = tmp_path / "e.grly"
    q.write_bytes(prefix)
    with pytest.raises(RuntimeError, match="no optimizer section"):
        grilly_core._grly_read(str(q), DIMS, opt_states=2)
    dims, info = grilly_core._grly_probe(str(p))
    assert tuple(dims) == DIMS and info["step"] == 7
