"""safetensors reading / planning on the CPU (the device upload is covered by the GPU test)."""
import numpy as np
import pytest

from sanic_amd import checkpoint
from sanic_amd.backend import to_bf16_bits


def _file(tmp_path, align=16):
    a = np.arange(24, dtype=np.uint16).reshape(4, 6)
    b = np.linspace(-1, 1, 7, dtype=np.float32)
    tensors = {"w.a": ("BF16", (4, 6), a.tobytes()), "w.b": ("F32", (7,), b.tobytes()),
               "w.c": ("BF16", (3,), np.array([1, 2, 3], np.uint16).tobytes())}
    p = str(tmp_path / "m.safetensors")
    checkpoint.write(p, tensors, align=align)
    return p, a, b


def test_header_round_trip(tmp_path):
    p, a, b = _file(tmp_path)
    entries, start, length = checkpoint.read_header(p)
    assert set(entries) == {"w.a", "w.b", "w.c"}
    assert entries["w.a"].shape == (4, 6) and entries["w.a"].dtype == "BF16"
    with open(p, "rb") as f:
        f.seek(start + entries["w.a"].begin)
        assert np.array_equal(np.frombuffer(f.read(48), np.uint16).reshape(4, 6), a)
    assert all(e.begin % 16 == 0 for e in entries.values())


def test_plan_binds_aligned_bf16_in_place_and_converts_the_rest(tmp_path):
    p, _, b = _file(tmp_path, align=2)
    entries, _, _ = checkpoint.read_header(p)
    how = checkpoint.plan(entries, [("w.a", (4, 6)), ("w.b", (7,)), ("w.c", (3,))])
    assert how["w.a"][0] == "slice"           # offset 0
    assert how["w.b"][0] == "convert"         # f32 → bf16
    assert how["w.c"][0] == "convert"         # bf16 at an offset that is not 16-byte aligned
    bits = checkpoint._bf16_bits(memoryview(b.tobytes()), "F32")
    assert np.array_equal(bits, to_bf16_bits(b))


def test_plan_rejects_missing_and_misshaped(tmp_path):
    p, _, _ = _file(tmp_path)
    entries, _, _ = checkpoint.read_header(p)
    with pytest.raises(KeyError):
        checkpoint.plan(entries, [("w.zz", (1,))])
    with pytest.raises(ValueError):
        checkpoint.plan(entries, [("w.a", (6, 4))])


def test_header_rejects_inconsistent_sizes(tmp_path):
    p = str(tmp_path / "bad.safetensors")
    checkpoint.write(p, {"x": ("BF16", (4,), b"\0" * 6)})
    with pytest.raises(ValueError):
        checkpoint.read_header(p)
