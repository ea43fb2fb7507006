"""The default schedule of a generic fold (no Sched given): the priced choice among the scalar,
cooperative and split forms (plan.rs:604-850 re-derived for wave64), read off the emitted kernel
kind without a GPU."""
import re

import pytest

from sanic_amd import carrier as C
from sanic_amd import configs, ir
from sanic_amd.program import STREAM, Program, Sched


def _choice(grid, stream, carrier=None, dtype=ir.F32):
    p = Program()
    x = p.input("x", (grid, stream), dtype)
    p.fused("y", (grid,), stream, [(x, (0, STREAM))], carrier or C.plain(ir.M_ADD))
    kind = p.emit(0)[0]
    m = re.search(r"\[auto w(\d+) s(\d+) c(\d+)\]", kind)
    assert m, kind
    return kind, tuple(int(v) for v in m.groups())


def test_long_stream_small_grid_splits_across_workgroups():
    """One output point over 2^20 elements: one lane per point keeps 4 bytes in flight, far
    from Little's law at 8 TB/s; the chosen form spreads the stream over many workgroups."""
    kind, (w, s, c) = _choice(1, 1 << 20)
    assert kind.startswith("fold:split")
    assert w * s * 64 >= 4096 and c >= 2


def test_huge_grid_short_stream_stays_scalar():
    """A million points of 4 elements each: one lane per point already fills the machine and a
    workgroup per point would waste 60 of its 64 lanes (a split unit may not be empty)."""
    kind, (w, s, c) = _choice(1 << 20, 4)
    assert kind.startswith("fold:scalar") and (w, s) == (0, 1)


def test_no_empty_split_units():
    for stream in (64, 100, 300, 5000):
        kind, (w, s, c) = _choice(2, stream, C.plain(ir.M_MAX))
        assert 64 * max(w, 1) * s <= max(stream, 64), (stream, kind)


def test_chunk_divides_the_stream():
    for stream in (4096, 1 << 20, 3 * 4096, 1000):
        kind, (w, s, c) = _choice(1, stream)
        if w:
            assert stream % (64 * w * s * c) == 0 or c == 1, (stream, kind)


def test_argmax_without_sched_is_split():
    V = 128256
    p = Program()
    x = p.input("x", (V,), ir.F32)
    p.fused("token", (1,), V, [(x, (STREAM,)), (ir.iota(V), (STREAM,))], C.first_argmax(), ir.U32)
    assert p.emit(0)[0].startswith("fold:split+merge[auto")


def test_explicit_sched_is_kept():
    p = configs.direct_attention(sched=Sched(lane_stream=True, waves=2, split=4))
    assert p.emit(0)[0] == "fold:split"
    assert configs.direct_attention(sched=Sched()).emit(0)[0] == "fold:scalar"
