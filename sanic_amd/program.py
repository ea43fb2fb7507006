"""Schedules as data: buffers, stages and the program descriptor handed across the C ABI.

Restates the backend's input contract: `Stage::{Fused, Elementwise/Gather}` and `Schedule`
(/root/reference/src/partition.rs:44-127), `FoldSched` (/root/reference/src/plan.rs:434-476),
and `Graph::{state, input, update, output}` (/root/reference/src/graph.rs:51-125). A `Program`
is what the reference's partitioner produces for one graph: an ordered list of stages whose
leaves are node trees over program buffers.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

from . import abi, ir
from .carrier import Carrier, ExprTable

INPUT, STATE, OUTPUT, SCRATCH = range(4)
STREAM, BCAST = -1, -2


@dataclass
class Sched:
    """FoldSched re-derived for wave64: `lane_stream` lanes split the stream, `waves`
    wavefronts per workgroup, `chunk` contiguous elements per lane, `split` workgroups per
    output point merged by the carrier's combine (split-K / Flash-Decoding). A stage built
    without a Sched carries `waves = 0` (not lane_stream, split 1): the backend prices its
    candidate schedules and picks one (plan.rs:604-850); `Sched()` itself is the scalar form."""
    lane_stream: bool = False
    waves: int = 1
    chunk: int = 1
    split: int = 1
    variant: int = 0          # tiling variant of the kernel that lowers the stage (the tuner's)


@dataclass
class BufferDecl:
    name: str
    role: int
    dtype: int
    shape: Tuple[int, ...]
    index: int

    @property
    def nbytes(self) -> int:
        return ir.dtype_bytes(self.dtype, int(np.prod(self.shape)) if self.shape else 1)


@dataclass
class Stage:
    kind: int                       # 0 fused, 1 pointwise
    name: str
    out: BufferDecl
    grid: Tuple[int, ...]
    stream: int = 0
    leaves: List[Tuple[ir.Node, Tuple[int, ...]]] = field(default_factory=list)
    carrier: Optional[Carrier] = None
    epilogue: Optional[ir.Node] = None
    sched: Sched = field(default_factory=Sched)
    value: Optional[ir.Node] = None
    where: Optional[ir.Node] = None


class Program:
    """A schedule for the backend: declared buffers plus ordered stages."""

    def __init__(self):
        self.buffers: List[BufferDecl] = []
        self.by_name: Dict[str, BufferDecl] = {}
        self.stages: List[Stage] = []

    # ── buffers ──
    def _decl(self, name, role, shape, dtype) -> BufferDecl:
        if name in self.by_name:
            raise ValueError(f"buffer {name!r} declared twice")
        b = BufferDecl(name, role, dtype, tuple(int(s) for s in shape), len(self.buffers))
        self.buffers.append(b)
        self.by_name[name] = b
        return b

    def node(self, name: str) -> ir.Node:
        """A fresh Input node reading buffer `name`."""
        b = self.by_name[name]
        return ir.input_(name, b.shape, b.dtype)

    def input(self, name: str, shape, dtype=ir.F32) -> ir.Node:
        self._decl(name, INPUT, shape, dtype)
        return self.node(name)

    def state(self, name: str, shape, dtype=ir.F32) -> ir.Node:
        """Graph::state (graph.rs:51-80): caller-bound, rewritten in place by a stage."""
        self._decl(name, STATE, shape, dtype)
        return self.node(name)

    # ── stages ──
    def fused(self, name: str, grid, stream: int, leaves, carrier: Carrier, out_dtype=ir.F32,
              epilogue: Optional[ir.Node] = None, sched: Optional[Sched] = None,
              role: int = OUTPUT) -> ir.Node:
        """Stage::Fused: fold `carrier` over `stream` for every point of `grid`. `leaves` are
        (node, binding) pairs; binding[j] names the grid dim, STREAM or BCAST for leaf dim j."""
        if len(leaves) > abi.MAX_LEAVES:
            raise ValueError("too many leaves")
        out = self._decl(name, role, grid, out_dtype)
        lv = [(n, tuple(b)) for n, b in leaves]
        self.stages.append(Stage(0, name, out, tuple(grid), int(stream), lv, carrier, epilogue,
                                 sched or Sched(waves=0)))
        return self.node(name)

    def pointwise(self, name: str, value: ir.Node, out_dtype=ir.F32, grid=None,
                  where: Optional[ir.Node] = None, into: Optional[str] = None,
                  role: int = OUTPUT) -> ir.Node:
        """Stage::Elementwise / Gather. With `into`, the stage rewrites an existing (state)
        buffer in place and stores only where `where` is nonzero (emit_metal.rs:1103-1178)."""
        grid = tuple(grid if grid is not None else value.shape)
        if into is not None:
            out = self.by_name[into]
            if tuple(out.shape) != grid:
                raise ValueError("in-place grid must equal the state's shape")
        else:
            out = self._decl(name, role, grid, out_dtype)
        self.stages.append(Stage(1, name, out, grid, value=value, where=where))
        return self.node(out.name)

    def repeat_stage(self, i: int, copies: int, fresh_inputs: bool = False) -> List[str]:
        """Append `copies` more instances of stage `i`, each writing its own output buffer
        (for timing one kernel as back-to-back launches inside one captured graph). With
        `fresh_inputs` every copy reads its own copies of the stage's INPUT buffers
        (`<name>.copy<r>`), so back-to-back launches do not find each other's inputs in cache."""
        import copy as _copy
        st = self.stages[i]
        names = []
        for r in range(copies):
            name = f"{st.out.name}.copy{r}"
            out = self._decl(name, OUTPUT, st.out.shape, st.out.dtype)
            dup = _copy.copy(st)
            dup.out = out
            dup.name = name
            if fresh_inputs:
                memo: Dict[int, ir.Node] = {}

                def ren(n: ir.Node) -> ir.Node:
                    if id(n) in memo:
                        return memo[id(n)]
                    if n.kind == ir.INPUT and self.by_name[n.name].role == INPUT:
                        cn = f"{n.name}.copy{r}"
                        if cn not in self.by_name:
                            b = self.by_name[n.name]
                            self._decl(cn, INPUT, b.shape, b.dtype)
                        m = _copy.copy(n)
                        m.name = cn
                    elif n.inputs:
                        m = _copy.copy(n)
                        m.inputs = tuple(ren(c) for c in n.inputs)
                    else:
                        m = n
                    memo[id(n)] = m
                    return m
                if st.kind == 0:
                    dup.leaves = [(ren(nd), b) for nd, b in st.leaves]
                    dup.epilogue = ren(st.epilogue) if st.epilogue is not None else None
                else:
                    dup.value = ren(st.value)
                    dup.where = ren(st.where) if st.where is not None else None
            self.stages.append(dup)
            names.append(name)
        return names

    # ── serialization ──
    def pack(self):
        """Return (ProgramDesc, keepalive) for the C ABI."""
        nt = ir.NodeTable(lambda n: self.by_name[n.name].index)
        et = ExprTable()
        stages = np.zeros(len(self.stages), dtype=abi.STAGE_DT)
        for i, s in enumerate(self.stages):
            r = stages[i]
            r["kind"] = s.kind
            r["out_buffer"] = s.out.index
            r["out_dtype"] = s.out.dtype
            r["rank"] = len(s.grid)
            r["grid"] = list(s.grid) + [0] * (abi.MAX_RANK - len(s.grid))
            r["epilogue"] = -1
            r["value"] = -1
            r["where"] = -1
            if s.kind == 0:
                r["stream"] = s.stream
                r["n_leaves"] = len(s.leaves)
                leaf = [-1] * abi.MAX_LEAVES
                bind = np.full((abi.MAX_LEAVES, abi.MAX_RANK), -3, dtype=np.int32)
                for l, (node, b) in enumerate(s.leaves):
                    leaf[l] = nt.add(node)
                    if len(b) != node.rank:
                        raise ValueError(f"stage {s.name}: leaf {l} binding rank")
                    bind[l, :len(b)] = b
                r["leaf"] = leaf
                r["bind"] = bind
                c = s.carrier
                car = r["carrier"]
                car["slots"] = c.slots
                for k in range(c.slots):
                    car["kind"][k]["kind"] = c.kinds[k].kind
                    car["kind"][k]["monoid"] = c.kinds[k].monoid
                    car["kind"][k]["ref_slot"] = c.kinds[k].ref_slot
                    car["kind"][k]["ties"] = c.kinds[k].ties
                    car["identity"][k] = c.identity[k]
                    car["into"][k] = et.add(c.into[k])
                    car["combine"][k] = et.add(c.combine[k])
                car["project"] = et.add(c.project)
                r["carrier"] = car
                if s.epilogue is not None:
                    r["epilogue"] = nt.add(s.epilogue)
                r["sched"]["lane_stream"] = int(s.sched.lane_stream)
                r["sched"]["waves"] = s.sched.waves
                r["sched"]["chunk"] = s.sched.chunk
                r["sched"]["split"] = s.sched.split
                r["sched"]["variant"] = s.sched.variant
            else:
                r["value"] = nt.add(s.value)
                if s.where is not None:
                    r["where"] = nt.add(s.where)
        nodes = nt.pack()
        exprs = et.pack()
        reindex = np.array(nt.reindex or [0], dtype=np.int64)
        bufs = np.zeros(len(self.buffers), dtype=abi.BUFFER_DT)
        for i, b in enumerate(self.buffers):
            bufs[i]["role"] = b.role
            bufs[i]["dtype"] = b.dtype
            bufs[i]["scale"] = ir.dtype_scale(b.dtype)
            bufs[i]["rank"] = len(b.shape)
            bufs[i]["shape"] = list(b.shape) + [0] * (abi.MAX_RANK - len(b.shape))
        keep = [nodes, exprs, reindex, bufs, stages]
        desc = abi.ProgramDesc(
            len(nodes), nodes.ctypes.data, len(exprs), exprs.ctypes.data,
            len(nt.reindex), reindex.ctypes.data, len(bufs), bufs.ctypes.data,
            len(stages), stages.ctypes.data)
        return desc, keep

    def emit(self, stage: int) -> Tuple[str, str]:
        """(kernel kind, HIP source) of one stage — no GPU needed."""
        desc, keep = self.pack()
        kind = ctypes.create_string_buffer(256)
        cap = 1 << 22
        src = ctypes.create_string_buffer(cap)
        abi.check(abi.lib().sanic_hip_emit_source(ctypes.byref(desc), stage, kind, 256, src, cap))
        return kind.value.decode(), src.value.decode()

    def stage_variants(self, stage: int = -1):
        """Tiling variants the kernel lowering `stage` offers (0: folded into another launch);
        with stage = -1 the list for every stage, from one lowering."""
        desc, keep = self.pack()
        n = (ctypes.c_int * max(1, len(self.stages)))()
        abi.check(abi.lib().sanic_hip_stage_variants(ctypes.byref(desc), stage, n))
        return list(n[:len(self.stages)]) if stage == -1 else n[0]

    def with_variants(self, variants: Dict[int, int]) -> "Program":
        """A copy whose stages carry the given tiling variants (stage index -> variant)."""
        import copy as _copy
        import dataclasses
        p = _copy.copy(self)
        p.stages = list(self.stages)
        for i, v in variants.items():
            st = _copy.copy(p.stages[i])
            st.sched = dataclasses.replace(st.sched or Sched(), variant=int(v))
            p.stages[i] = st
        return p

    def precompile(self):
        desc, keep = self.pack()
        abi.check(abi.lib().sanic_hip_precompile(ctypes.byref(desc)))
