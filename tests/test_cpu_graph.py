"""Graph declarations without a GPU: update and output validation (graph.rs:51-160)."""
import pytest

from sanic_amd import ir
from sanic_amd.graph import Graph, GraphError


def test_update_and_output_validation():
    g = Graph()
    x = g.input("x", (8,))
    s = g.state("s", (8,))
    t = g.state("t", (4,))
    g.program.pointwise("s.next", ir.map_(ir.ADD, s, x), ir.F32)
    with pytest.raises(GraphError, match="not a state"):
        g.update("x", "s.next")
    with pytest.raises(GraphError, match="not a stage output"):
        g.update("s", "x")
    with pytest.raises(GraphError, match="volumes differ"):
        g.update("t", "s.next")
    g.update("s", "s.next")
    with pytest.raises(GraphError, match="already has an update"):
        g.update("s", "s.next")
    with pytest.raises(GraphError, match="not a stage output"):
        g.output("s")
    g.output("s.next")
    assert g.states() == ["s", "t"]
    assert g.updates == [("s.next", "s")]
