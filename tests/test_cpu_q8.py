"""Q8 storage (`Dtype::Q8 { scale }`, /root/reference/src/scalar.rs:190-198): the oracle's
grid rounding pinned to the reference's own known answers (tests/numeric.rs:412-448), the
stored-output and RoundTo paths of the interpreter restatement, the host codec's device rule,
and the library's refusal of scale-less grids. No GPU."""
import ctypes

import numpy as np
import pytest

import oracle
from sanic_amd import abi, backend, ir
from sanic_amd.program import Program


def test_q8_round_trip_known_answers():
    """tests/numeric.rs:414-431: grid points are fixed, off-grid values land on the nearest
    grid point, the ends clamp and ±∞ have homes at ±127·scale."""
    s = 0.5
    for q in (-127, -3, 0, 1, 88, 127):
        assert oracle.round_q8(s, q * s) == q * s
    once = oracle.round_q8(s, 1.23456)
    assert oracle.round_q8(s, once) == once
    assert oracle.round_q8(s, 1.2) == 1.0
    assert oracle.round_q8(s, 1000.0) == 63.5
    assert oracle.round_q8(s, float("inf")) == 63.5
    assert oracle.round_q8(s, float("-inf")) == -63.5


# tests/numeric.rs:433-448 at scale 0.25; the expected grid values worked by hand:
# 0.3/0.25 = 1.2 → 1; −1.7/0.25 = −6.8 → −7; 400 → 127; −0.504 → −1; 0; 126.96 → 127; −127.6 → −127
STORED_X = [0.3, -1.7, 100.0, -0.126, 0.0, 31.74, -31.9]
STORED_WANT = [0.25, -1.75, 31.75, -0.25, 0.0, 31.75, -31.75]


def test_round_to_q8_map_matches_hand_worked_grid():
    p = Program()
    x = p.input("X", (7,), ir.F32)
    p.pointwise("Y", ir.round_to(x, ir.q8(0.25)), ir.F32)
    got = oracle.run_program(p, {"X": np.array(STORED_X)})["Y"]
    assert got.tolist() == STORED_WANT


def test_q8_output_store_matches_hand_worked_grid():
    """The same grid through a stage whose OUTPUT is pinned to Q8 (the narrowing store)."""
    p = Program()
    x = p.input("X", (7,), ir.F32)
    p.pointwise("Y", x * 1.0, ir.q8(0.25))
    got = oracle.run_program(p, {"X": np.array(STORED_X)})["Y"]
    assert got.tolist() == STORED_WANT


def test_host_codec_follows_the_device_store():
    """encode quantizes as the device store does (v/scale in f32, half-to-even, clamp ±127);
    decode is q·scale. Off ties this equals round_to; at a tie the device rule rounds to even
    where the interpreter's f64::round goes away from zero (the reference's Metal store and its
    interpreter differ the same way, emit_metal.rs:182-185 vs scalar.rs:145)."""
    dt = ir.q8(0.25)
    vals = np.array(STORED_X + [0.125, 0.375, -0.125, float("inf"), float("-inf")])
    raw = backend.encode(vals, dt)
    assert np.frombuffer(raw, np.int8).tolist() == [1, -7, 127, -1, 0, 127, -127, 0, 2, 0, 127, -127]
    back = backend.decode(raw, dt, len(vals))
    assert back[:7].tolist() == STORED_WANT
    assert back[7:].tolist() == [0.0, 0.5, 0.0, 31.75, -31.75]
    assert [oracle.round_q8(0.25, v) for v in (0.125, 0.375, -0.125)] == [0.25, 0.5, -0.25]


def test_q8_dtype_carries_its_scale_into_the_descriptor():
    p = Program()
    x = p.input("X", (4, 3), ir.q8(0.03125))
    p.pointwise("Y", ir.round_to(x * 2.0, ir.q8(0.5)), ir.q8(0.5))
    desc, keep = p.pack()
    bufs = keep[3]
    assert bufs[0]["dtype"] == ir.Q8 and bufs[0]["scale"] == np.float32(0.03125)
    assert bufs[1]["dtype"] == ir.Q8 and bufs[1]["scale"] == np.float32(0.5)
    assert ir.dtype_bytes(ir.q8(1.0), 10) == 10
    with pytest.raises(ValueError):
        ir.q8(0.0)
    with pytest.raises(ValueError):
        ir.round_to(x, ir.I8)


def test_library_refuses_a_q8_grid_without_scale():
    """A Q8 buffer or RoundTo(Q8) node with no positive scale is a compile error, not a
    silent zero grid."""
    p = Program()
    x = p.input("X", (8,), ir.F32)
    p.pointwise("Y", ir.Node(ir.MAP, (8,), (x,), op=ir.ROUND_Q8, value=0.0), ir.F32)
    desc, keep = p.pack()
    assert abi.lib().sanic_hip_precompile(ctypes.byref(desc)) != 0
    assert b"scale" in abi.lib().sanic_hip_last_error()

    p = Program()
    x = p.input("X", (8,), ir.q8(1.0))
    p.pointwise("Y", x * 1.0, ir.F32)
    desc, keep = p.pack()
    keep[3][0]["scale"] = 0.0               # a Q8 buffer whose scale was never set
    assert abi.lib().sanic_hip_precompile(ctypes.byref(desc)) != 0
    assert b"scale" in abi.lib().sanic_hip_last_error()


def test_round_f16_matches_numpy_half_conversion():
    """round_to(F16) (scalar.rs:154-178: ties to even, overflow to ±∞, subnormals on the 2^-24
    grid) against numpy's own f32 → f16 conversion, over edge values and a random sweep."""
    edge = [0.0, -0.0, 1.0, 65504.0, 65519.99, 65520.0, 1e6, -1e6, 2.0 ** -24, 2.0 ** -25,
            3 * 2.0 ** -26, 2.0 ** -14, 2.0 ** -14 - 2.0 ** -25, 1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11,
            0.1, -0.3333, float("inf"), float("-inf")]
    rng = np.random.default_rng(5)
    sweep = np.concatenate([rng.standard_normal(4000) * 10.0 ** rng.integers(-9, 6, 4000)])
    for v in edge + sweep.tolist():
        with np.errstate(over="ignore"):
            want = float(np.float32(v).astype(np.float16))
        got = oracle.round_f16(v)
        assert got == want or (np.isnan(got) and np.isnan(want)), (v, got, want)
    assert np.isnan(oracle.round_f16(float("nan")))


def test_f16_output_store_is_narrowed_by_the_oracle():
    p = Program()
    x = p.input("X", (5,), ir.F32)
    p.pointwise("Y", ir.round_to(x, ir.F16) - x, ir.F32)
    p.pointwise("Z", x * 1.0, ir.F16)
    vals = np.array([0.1, 1 + 2.0 ** -11, 70000.0, 2.0 ** -25, -3.3])
    out = oracle.run_program(p, {"X": vals})
    with np.errstate(over="ignore"):
        want = np.float32(vals).astype(np.float16).astype(np.float64)
    assert out["Z"].tolist() == want.tolist()
    np.testing.assert_array_equal(out["Y"], (want - vals).astype(np.float32).astype(np.float64))   # Y is stored f32
