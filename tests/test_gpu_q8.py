"""Narrow storage on the GPU through the C ABI against the oracle: Q8 (the pinned-output grid
of /root/reference/tests/metal.rs:2402-2446, equality, no tolerance; dequantizing loads in a
fold; RoundTo(Q8) inside a stage; a split fold stored to Q8; a Q8 feedback input) and F16
(RoundTo(F16) and an F16-stored output)."""
import numpy as np
import pytest

import oracle
from sanic_amd import carrier as C
from sanic_amd import ir
from sanic_amd.program import STREAM, Program, Sched
from tests.util import run_on_gpu

pytestmark = pytest.mark.gpu


def test_q8_pinned_output_round_trips_the_grid_exactly(dev):
    """tanh of 512 values stored to q8(1/32): the bytes read back ARE the grid the
    interpreter's round_to gives (tests/metal.rs:2402-2446)."""
    q8 = ir.q8(0.03125)
    p = Program()
    x = p.input("X", (512,), ir.F32)
    p.pointwise("Y", ir.map_(ir.TANH, x), q8)
    vals = {"X": oracle.lcg(0x0816, 512)}
    got, exe = run_on_gpu(dev, p, vals)
    want = oracle.run_program(p, vals)["Y"]
    assert got["Y"].tolist() == want.tolist()
    assert len(set(np.round(got["Y"] / 0.03125).tolist())) > 40     # a real spread of grid points


@pytest.mark.parametrize("sched", [None, Sched(lane_stream=True, waves=2), Sched(lane_stream=True, waves=2, split=5)])
def test_q8_input_dequantizes_in_a_fold(dev, sched):
    """Row sums of a q8(1/128) matrix [64, 300]: every term and partial sum is a multiple of
    1/128 below 2^24 of them, so the f32 fold is exact and equals the f64 interpreter."""
    s = 0.0078125
    p = Program()
    x = p.input("X", (64, 300), ir.q8(s))
    p.fused("Y", (64,), 300, [(x, (0, STREAM))], C.plain(ir.M_ADD), sched=sched)
    q = np.round(oracle.lcg(808, 64 * 300) * 127).reshape(64, 300)
    vals = {"X": q * s}
    got, exe = run_on_gpu(dev, p, vals)
    want = oracle.run_program(p, vals)["Y"]
    print(exe.stage_kernel(0))
    np.testing.assert_array_equal(got["Y"], want)


def test_round_to_q8_inside_a_stage(dev):
    """RoundTo(q8(0.1)) of 3·x, then a further map, stored f32: the grid value a store + load
    would give, within f32 rounding of q·0.1 (the oracle forms it in f64)."""
    p = Program()
    x = p.input("X", (1000,), ir.F32)
    p.pointwise("Y", ir.round_to(x * 3.0, ir.q8(0.1)) + 1.0, ir.F32)
    vals = {"X": oracle.lcg(77, 1000)}
    got, _ = run_on_gpu(dev, p, vals)
    want = oracle.run_program(p, vals)["Y"]
    np.testing.assert_allclose(got["Y"], want, rtol=1e-6, atol=0)


def test_split_fold_stored_to_q8(dev):
    """A 7-way split max fold over [16, 5000] stored to q8(0.25): the last workgroup's merge
    narrows through the Q8 store; equality with the interpreter."""
    p = Program()
    x = p.input("X", (16, 5000), ir.F32)
    p.fused("M", (16,), 5000, [(x, (0, STREAM))], C.plain(ir.M_MAX), ir.q8(0.25),
            sched=Sched(lane_stream=True, waves=4, split=7))
    vals = {"X": oracle.lcg(5150, 16 * 5000).reshape(16, 5000) * 20.0}
    got, exe = run_on_gpu(dev, p, vals)
    assert exe.stage_kernel(0).startswith("fold:split")
    want = oracle.run_program(p, vals)["M"]
    assert got["M"].tolist() == want.tolist()


def test_feedback_into_a_q8_input(dev):
    """capture(feedback): an f32 output fed back into a q8(0.25) input through the in-graph
    conversion (the device store rule): x ← grid(x + 0.3) gains exactly one grid step a replay."""
    p = Program()
    x = p.input("x", (8,), ir.q8(0.25))
    p.pointwise("t", x + 0.3, ir.F32)
    exe = dev.prepare(p)
    x0 = np.arange(8) * 0.25 - 1.0
    xb = dev.from_values(x0, p.by_name["x"].dtype)
    rp = exe.capture({"x": xb}, feedback=[("t", "x")])
    for _ in range(3):
        rp.step()
    np.testing.assert_array_equal(xb.read(p.by_name["x"].dtype, 8), x0 + 0.75)


def test_round_to_f16_and_f16_store(dev):
    """RoundTo(F16) inside a stage and an F16-stored output on the GPU against the oracle's
    half rounding (ties to even, overflow to ∞, subnormals): exact."""
    p = Program()
    x = p.input("X", (1024,), ir.F32)
    p.pointwise("Y", ir.round_to(x, ir.F16) * 2.0, ir.F32)
    p.pointwise("Z", x * 1.0, ir.F16)
    v = oracle.lcg(1616, 1024) * 10.0 ** np.repeat(np.arange(-8, 8), 64)
    v[:6] = [65519.0, 65520.0, -1e6, 2.0 ** -25, 3 * 2.0 ** -26, 1 + 2.0 ** -11]
    vals = {"X": v}
    got, _ = run_on_gpu(dev, p, vals)
    want = oracle.run_program(p, vals)
    assert got["Y"].tolist() == want["Y"].tolist()
    assert got["Z"].tolist() == want["Z"].tolist()
