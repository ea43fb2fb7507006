"""The generic stateful machine (sanic_amd.graph: Graph → compile_for → instantiate → step, the
reference's graph.rs:51-345) on a small non-Llama program, stepped on the GPU against the oracle
stepping the same schedule: a running sum with feedback, a fold over it, and a state advanced in
place.

Per step:
  acc.next = acc + x · w            (pointwise; state `acc` takes it by feedback after the step)
  total    = Σ_i acc.next[i] · w[i] (a fused dot fold over the new value)
  count    = where(true, count + 1) (pointwise written into the `count` state in place)
"""
import numpy as np
import pytest

import oracle
from sanic_amd import carrier as C
from sanic_amd import ir
from sanic_amd.graph import Graph, GraphError
from sanic_amd.program import STREAM

pytestmark = pytest.mark.gpu

N = 4096


def _graph():
    g = Graph()
    x = g.input("x", (N,), ir.BF16)
    w = g.input("w", (N,), ir.F32)
    acc = g.state("acc", (N,), ir.F32)
    cnt = g.state("count", (1,), ir.F32)
    p = g.program
    nxt = p.pointwise("acc.next", ir.map_(ir.ADD, acc, ir.map_(ir.MUL, x, w)), ir.F32)
    p.fused("total", (1,), N, [(nxt, (STREAM,)), (w, (STREAM,))], C.dot(2), ir.F32)
    p.pointwise("count.next", ir.map_(ir.ADD, cnt, ir.const(1.0)), ir.F32, grid=(1,),
                where=ir.map_(ir.LT, ir.const(0.0), ir.const(1.0)), into="count")
    g.update("acc", "acc.next")
    g.output("total")
    return g


def test_running_sum_machine_matches_the_oracle_step_by_step(dev):
    g = _graph()
    xv = oracle.synth(901, N, dtype=ir.BF16)
    wv = oracle.lcg(902, N)
    sp = g.compile_for(dev)
    print([sp.exe.stage_kernel(i) for i in range(len(sp.program.stages))], sp.kernel_count())
    m = sp.instantiate({"x": dev.from_values(xv, ir.BF16), "w": dev.from_values(wv, ir.F32)})
    assert np.all(m.read("acc") == 0) and np.all(m.read("count") == 0)     # zeroed at instantiation
    for step in range(5):
        # the oracle steps from the state the GPU holds before the step (an f32 sum may round one
        # ulp away from the f64 oracle's; the states are compared at the f32 tolerance)
        acc, cnt = m.read("acc").reshape(-1), m.read("count").reshape(-1)
        m.step()
        want = oracle.run_program(sp.program, {"x": xv, "w": wv, "acc": acc, "count": cnt})
        got_total, want_total = float(m.read("total")[0]), float(want["total"][0])
        err = abs(got_total - want_total) / (1 + abs(want_total))
        print(step, got_total, want_total, err)
        assert err <= 1e-4
        # the feedback landed in the state: the reference's f32 metric |g − e| / (1 + |e|)
        acc_err = float(np.max(np.abs(m.read("acc") - want["acc.next"]) / (1 + np.abs(want["acc.next"]))))
        assert acc_err <= 1e-6, acc_err
        assert float(m.read("count")[0]) == float(want["count"][0]) == step + 1
    # back-to-back steps with no host in between, then a host write into a state
    m.step_many(3)
    assert float(m.read("count")[0]) == 8.0
    m.write("count", [100.0])
    m.step()
    assert float(m.read("count")[0]) == 101.0


def test_instantiate_refuses_missing_and_unknown_inputs(dev):
    sp = _graph().compile_for(dev)
    with pytest.raises(GraphError, match="missing inputs"):
        sp.instantiate({"x": dev.alloc(N * 2)})
    with pytest.raises(GraphError, match="unknown inputs"):
        sp.instantiate({"x": dev.alloc(N * 2), "w": dev.alloc(N * 4), "y": dev.alloc(4)})
