"""Stateful step programs over the HIP backend: the reference's `Graph` (state / input / update /
output, /root/reference/src/graph.rs:51-160) and `Graph::compile_for` → `StepProgram::instantiate`
→ `Machine::step` (graph.rs:231-345), for programs given as stages.

A `Graph` wraps a `Program` (the partitioned schedule the backend receives) and records what the
reference's graph records beside the expression: which buffers are step state and, for every
state, the value it takes at the end of a step. A state is updated one of two ways, as in the
reference:

* in place — a pointwise stage writes the state's own buffer under a `where` (the
  `overwritable_states` law of graph.rs:140-160: `where(c, x, s)` read once by this step). The
  stage itself is the update (`Program.pointwise(..., into=state)`); nothing is recorded;
* by feedback — the state takes the value of a program output after the step
  (`update(state, output)`): the capture converts the output into the state's storage at the end
  of every replay, inside the same graph (compile.rs:869-961).

`Graph.compile_for(dev)` prepares the program (`Backend::prepare`); `StepProgram.instantiate`
allocates and zeroes every state (graph.rs:297-310), binds the caller's inputs and captures one
replay; `Machine.step()` replays it and returns GPU seconds; `Machine.output(name)` reads what the
last step wrote.
"""
from __future__ import annotations

from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

from . import ir
from .backend import Buffer, HipDevice, decode, encode
from .program import INPUT, OUTPUT, SCRATCH, STATE, Program


class GraphError(ValueError):
    """A graph that cannot be instantiated (the reference's `RunError::Feedback` and
    `MissingInput` cases, compile.rs:42-58)."""


class Graph:
    def __init__(self, program: Optional[Program] = None):
        self.program = program if program is not None else Program()
        self.updates: List[Tuple[str, str]] = []      # (output buffer, state buffer)
        self.outputs: List[str] = []

    # ── declarations (graph.rs:51-125) ──
    def input(self, name: str, shape, dtype: int = ir.F32) -> ir.Node:
        return self.program.input(name, shape, dtype)

    def state(self, name: str, shape, dtype: int = ir.F32) -> ir.Node:
        return self.program.state(name, shape, dtype)

    def update(self, state: str, value: str):
        """After every step, `state` takes the value the stage output `value` holds."""
        p = self.program
        if state not in p.by_name or p.by_name[state].role != STATE:
            raise GraphError(f"update target {state!r} is not a state")
        if value not in p.by_name or p.by_name[value].role not in (OUTPUT, SCRATCH):
            raise GraphError(f"update value {value!r} is not a stage output")
        sv, vv = p.by_name[state], p.by_name[value]
        if int(np.prod(sv.shape or (1,))) != int(np.prod(vv.shape or (1,))):
            raise GraphError(f"update {value!r} → {state!r}: volumes differ")
        if any(s == state for _, s in self.updates):
            raise GraphError(f"state {state!r} already has an update")
        self.updates.append((value, state))

    def output(self, name: str):
        """Name a stage output the caller reads after a step."""
        if name not in self.program.by_name or self.program.by_name[name].role not in (OUTPUT, SCRATCH):
            raise GraphError(f"{name!r} is not a stage output")
        self.outputs.append(name)

    def states(self) -> List[str]:
        return [b.name for b in self.program.buffers if b.role == STATE]

    def compile_for(self, dev: HipDevice, variants: Optional[Dict[int, int]] = None) -> "StepProgram":
        prog = self.program.with_variants(variants) if variants else self.program
        return StepProgram(dev, self, prog, dev.prepare(prog))


class StepProgram:
    def __init__(self, dev: HipDevice, graph: Graph, program: Program, exe):
        self.dev, self.graph, self.program, self.exe = dev, graph, program, exe

    def kernel_count(self) -> int:
        """Stages that launch kernels of their own (others are batched into, absorbed by or run
        as the tail of another stage's kernel)."""
        kinds = [self.exe.stage_kernel(i) for i in range(len(self.program.stages))]
        return sum(1 for k in kinds if "-into:" not in k and not k.startswith("tail-of:"))

    def instantiate(self, inputs: Dict[str, Buffer]) -> "Machine":
        """Zeroed states, the caller's inputs bound (borrowed), one captured replay."""
        need = {b.name for b in self.program.buffers if b.role == INPUT}
        missing = sorted(need - set(inputs))
        if missing:
            raise GraphError(f"missing inputs: {missing}")
        unknown = sorted(set(inputs) - need)
        if unknown:
            raise GraphError(f"unknown inputs: {unknown}")
        bind: Dict[str, Buffer] = dict(inputs)
        for b in self.program.buffers:
            if b.role == STATE:
                buf = self.dev.alloc(b.nbytes)
                buf.upload(bytes(b.nbytes))
                bind[b.name] = buf
        return Machine(self, bind)


class Machine:
    def __init__(self, sp: StepProgram, bind: Dict[str, Buffer]):
        self.sp = sp
        self.program = sp.program
        self.bind = bind
        self.replay = sp.exe.capture(bind, self.sp.graph.updates)

    def step(self) -> float:
        """One step (one graph replay, waited for); GPU seconds."""
        return self.replay.step()

    def step_many(self, n: int) -> float:
        """n steps back to back; GPU seconds."""
        return self.replay.step_many(n)

    def buffer(self, name: str) -> Buffer:
        b = self.program.by_name[name]
        return self.bind[name] if b.role in (INPUT, STATE) else self.replay.buffer(name)

    def read(self, name: str) -> np.ndarray:
        """A state's current value or what the last step wrote to an output, as f64."""
        b = self.program.by_name[name]
        n = int(np.prod(b.shape)) if b.shape else 1
        return decode(self.buffer(name).download(b.nbytes), b.dtype, n).reshape(b.shape)

    output = read

    def write(self, name: str, values):
        """Overwrite a state (or a bound input) from the host, in its storage dtype."""
        b = self.program.by_name[name]
        if b.role not in (STATE, INPUT):
            raise GraphError(f"{name!r} is not a state or input")
        arr = np.asarray(values, np.float64).reshape(-1)
        self.bind[name].upload(encode(arr, b.dtype))
