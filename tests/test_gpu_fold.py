"""The generic carrier fold on the GPU against the oracle (scalar, cooperative, split)."""
import numpy as np
import pytest

import oracle
from sanic_amd import carrier as C
from sanic_amd import configs, ir
from sanic_amd.program import BCAST, STREAM, Program, Sched
from tests.util import max_rel_err, run_on_gpu

pytestmark = pytest.mark.gpu

SCHEDS = {
    "auto": None,
    "scalar": Sched(),
    "coop1": Sched(lane_stream=True, waves=1),
    "coop4_chunk2": Sched(lane_stream=True, waves=4, chunk=2),
    "split4": Sched(lane_stream=True, waves=2, split=4),
    "split7_scalar_lanes": Sched(lane_stream=True, waves=1, split=7),
}


@pytest.mark.parametrize("name", list(SCHEDS))
def test_config_a_direct_causal_attention(dev, name):
    """Config A: causal attention f32 [128, 64] within 1e-4 of the interpreter."""
    prog = configs.direct_attention(sched=SCHEDS[name])
    vals = {n: oracle.lcg(s, 128 * 64).reshape(128, 64) for n, s in (("Q", 11), ("K", 12), ("V", 13))}
    got, exe = run_on_gpu(dev, prog, vals)
    graph = ir.attention(prog.node("Q"), prog.node("K"), prog.node("V"), causal=True)
    want = oracle.eval_node(prog, graph, vals)
    err = max_rel_err(got["O"], want)
    print(name, exe.stage_kernel(0), err)
    assert err < 1e-4


def test_direct_attention_known_answer(dev):
    """q = k = I, v = [[2,3],[5,7]], scale 1/√2 (tests/compile.rs:230-263)."""
    prog = configs.direct_attention(S=2, D=2, causal=False)
    vals = {"Q": np.eye(2), "K": np.eye(2), "V": np.array([[2.0, 3.0], [5.0, 7.0]])}
    got, _ = run_on_gpu(dev, prog, vals)
    np.testing.assert_allclose(got["O"].reshape(-1), [2.990715, 4.3209534, 4.009285, 5.6790466],
                               rtol=2e-6)


def test_reduce_rows_known_answer(dev):
    """reduce rows [[1,2],[3,4]] → [3, 7] (lib.rs:10-22)."""
    p = Program()
    x = p.input("X", (2, 2))
    p.fused("Y", (2,), 2, [(x, (0, STREAM))], C.plain(ir.M_ADD))
    got, _ = run_on_gpu(dev, p, {"X": np.array([[1.0, 2.0], [3.0, 4.0]])})
    assert got["Y"].tolist() == [3.0, 7.0]


def test_split_fold_merges_in_last_workgroup(dev):
    """A small split fold (argmax key/tie carrier over 100k elements, 64 workgroups) merges in
    its last-arriving workgroup and matches the first-maximum index exactly, twice in a row
    (the arrival counter re-arms itself)."""
    n = 100_000
    p = Program()
    x = p.input("X", (n,))
    p.fused("I", (1,), n, [(x, (STREAM,)), (ir.iota(n), (STREAM,))], C.first_argmax(), ir.U32,
            sched=Sched(lane_stream=True, waves=4, chunk=4, split=64))
    vals = oracle.lcg(99, n)
    vals[77_777] = 5.0
    vals[88_888] = 5.0          # a tie: the first index wins
    exe = dev.prepare(p)
    assert exe.stage_kernel(0).startswith("fold:split+merge")
    buf = dev.from_values(vals, ir.F32)
    for _ in range(2):
        out = exe.execute({"X": buf})["I"].read(ir.U32, 1)
        assert int(out[0]) == 77_777


@pytest.mark.parametrize("split", [1, 2, 3, 7, 9])
def test_split_attention_equals_one_pass_for_any_block_count(dev, split):
    """A 9-key attention fold split over 1, 2, 3, 7 and 9 workgroups (tests/group.rs:48-84:
    2/3/7 leave uneven remainders, 9 puts one key in each workgroup so the last arriver's merge
    does all of the softmax coupling) equals the one-pass oracle on the GPU."""
    S, D = 9, 5
    prog = configs.direct_attention(S=S, D=D, causal=False,
                                    sched=Sched(lane_stream=True, waves=1, split=split))
    vals = {n: oracle.lcg(seed, S * D).reshape(S, D) * 4.0 - 2.0 for n, seed in (("Q", 31), ("K", 32), ("V", 33))}
    got, exe = run_on_gpu(dev, prog, vals)
    if split > 1:
        assert exe.stage_kernel(0).startswith("fold:split"), exe.stage_kernel(0)
    want = oracle.run_program(prog, vals)["O"]
    # the oracle's own split form agrees with its one pass (interp.rs:555-643)
    split_want, _ = oracle.fold_stage(prog, 0, vals, blocks=split)
    assert np.allclose(split_want, want, rtol=1e-6, atol=1e-7)
    err = max_rel_err(got["O"], want)
    print(exe.stage_kernel(0), split, err)
    assert err < 1e-4


def test_capture_feedback_converts_output_into_input(dev):
    """capture(bindings, feedback): a u32 output fed back into an f32 input inside the graph,
    so each replay sees the previous step's output (compile.rs:869-961, RunError::Feedback on
    mismatched volumes)."""
    p = Program()
    x = p.input("x", (8,), ir.F32)
    p.pointwise("t", ir.map_(ir.ADD, x, ir.const(1.0)), ir.U32)
    exe = dev.prepare(p)
    xb = dev.from_values(np.arange(8, dtype=np.float64), ir.F32)
    rp = exe.capture({"x": xb}, feedback=[("t", "x")])
    for _ in range(3):
        rp.step()
    np.testing.assert_array_equal(xb.read(ir.F32, 8), np.arange(8) + 3.0)
    np.testing.assert_array_equal(rp.buffer("t").read(ir.U32, 8), np.arange(8) + 3)


def test_prefix_scan_fallback_stage_known_answer(dev):
    """The reference's scan known answer through a pointwise (fallback) stage on the GPU
    (tests/laws.rs:715-730): exact."""
    p = Program()
    x = p.input("X", (5,), ir.F32)
    p.pointwise("Y", ir.scan(x, 0, ir.M_ADD), ir.F32)
    got, exe = run_on_gpu(dev, p, {"X": np.array([2.0, -1.0, 3.0, 0.5, 4.0])})
    print(exe.stage_kernel(0))
    np.testing.assert_array_equal(got["Y"], [2.0, 1.0, 4.0, 4.5, 8.5])


@pytest.mark.parametrize("monoid", [ir.M_ADD, ir.M_MAX, ir.M_MIN, ir.M_LSE])
@pytest.mark.parametrize("dim", [0, 1])
def test_prefix_scan_matches_oracle(dev, monoid, dim):
    """[24, 300] scans along either axis against the f64 interpreter: f32 ≤ 1e-4 with the
    reference's metric; Max/Min exact."""
    p = Program()
    x = p.input("X", (24, 300), ir.F32)
    p.pointwise("Y", ir.scan(x, dim, monoid), ir.F32)
    vals = {"X": oracle.lcg(91, 24 * 300).reshape(24, 300)}
    got, _ = run_on_gpu(dev, p, vals)
    want = oracle.run_program(p, vals)["Y"]
    if monoid in (ir.M_MAX, ir.M_MIN):
        np.testing.assert_array_equal(got["Y"], want)
    else:
        assert max_rel_err(got["Y"], want) < 1e-4


@pytest.mark.parametrize("split", [7, 37, 64])
def test_split_merge_butterfly_keeps_first_index(dev, split):
    """The last workgroup's butterfly merge (one lane per partial, identity-padded to a power
    of two) keeps the serial walk's order: of three equal maxima in different partials the
    first index wins, for splits that are and are not powers of two."""
    n = 50_000
    p = Program()
    x = p.input("X", (n,))
    p.fused("I", (1,), n, [(x, (STREAM,)), (ir.iota(n), (STREAM,))], C.first_argmax(), ir.U32,
            sched=Sched(lane_stream=True, waves=4, chunk=4, split=split))
    vals = oracle.lcg(7 + split, n)
    for i in (n - 5, 31_000, 12_345):
        vals[i] = 7.0
    got, exe = run_on_gpu(dev, p, {"X": vals})
    assert exe.stage_kernel(0).startswith("fold:split+merge")
    assert int(got["I"][0]) == 12_345


def test_split_merge_butterfly_small_grid_attention(dev):
    """Config A at 16×8 with a 7-way split: 128 output points merged by butterflies of 8 lanes
    (ExpShifted combine with its −∞ guard), against the interpreter."""
    prog = configs.direct_attention(S=16, D=8, sched=Sched(lane_stream=True, waves=4, split=7))
    vals = {n: oracle.lcg(s, 16 * 8).reshape(16, 8) for n, s in (("Q", 21), ("K", 22), ("V", 23))}
    got, exe = run_on_gpu(dev, prog, vals)
    assert exe.stage_kernel(0).startswith("fold:split+merge")
    want = oracle.run_program(prog, vals)["O"]
    assert max_rel_err(got["O"], want) < 1e-4


@pytest.mark.parametrize("grid,stream", [(1, 1 << 20), (3, 700001), (128, 128256)])
def test_default_schedule_long_stream_small_grid(dev, grid, stream):
    """A stage built without a Sched: the backend prices its schedules (plan.rs:604-850) and
    splits a long stream over a small grid across workgroups; the sums match the oracle."""
    p = Program()
    x = p.input("x", (grid, stream), ir.F32)
    p.fused("y", (grid,), stream, [(x, (0, STREAM))], C.plain(ir.M_ADD))
    vals = {"x": oracle.lcg(grid + stream, grid * stream).reshape(grid, stream)}
    got, exe = run_on_gpu(dev, p, vals)
    assert exe.stage_kernel(0).startswith("fold:split+merge[auto"), exe.stage_kernel(0)
    want = oracle.run_program(p, vals)["y"]
    err = max_rel_err(got["y"], want)
    print(exe.stage_kernel(0), err)
    assert err < 1e-4
