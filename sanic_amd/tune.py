"""Measured tiling tuner: the reference's `SANIC_TUNE=1` (/root/reference/src/compile.rs:1348-1630)
on the HIP backend.

The reference times competing FoldSched candidates of every fold IN CONTEXT: substituted into
the full step and judged by the step's replay wall time, because solo microbenchmarks reward
parallelism a bandwidth-bound step punishes. Here the candidates are the tiling variants the
hand-written kernels offer (`sanic_sched.variant`: rows per GEMV workgroup, threads and chunk
length of decode attention, FlashAttention occupancy); the instrument is the same — the whole
program captured as one hipGraph and replayed.

Rules kept from the reference:
  * isomorphic stages form one FAMILY (keyed on the generated source, which is the same for
    every layer) and swap to a candidate together, judged by one step time;
  * every verdict is a difference of ADJACENT measurements: each candidate is timed next to a
    fresh measurement of the current choice (the clock drifts over a tuning run);
  * overruling the analytic choice needs a 1% margin;
  * the tuned program is re-measured against a fresh analytic baseline at the end, and a tune
    that does not win ships nothing;
  * each measurement is the fastest of a few replays (the min sheds clock ramp).
"""
from __future__ import annotations

import hashlib
import re
from dataclasses import dataclass, field
from typing import Callable, Dict, List, Optional, Tuple

from .program import INPUT, STATE, Program

MARGIN = 0.01
ROUNDS = 3


@dataclass
class Family:
    key: str
    kernel: str
    stages: List[int]
    variants: int


@dataclass
class TuneReport:
    baseline_s: float = 0.0
    tuned_s: float = 0.0
    shipped: bool = False
    choices: Dict[str, int] = field(default_factory=dict)      # family kernel -> variant
    variants: Dict[int, int] = field(default_factory=dict)     # stage -> variant (shipped)
    trials: List[Tuple[str, int, float, float]] = field(default_factory=list)  # (kernel, v, base, cand)


def families(prog: Program) -> List[Family]:
    """Stages whose kernel offers more than one variant, grouped by identical generated source
    (the families of compile.rs:1356-1360)."""
    counts = prog.stage_variants(-1)
    fams: Dict[str, Family] = {}
    for i, n in enumerate(counts):
        if n <= 1:
            continue
        _, src = prog.emit(i)
        key = hashlib.sha1(src.encode()).hexdigest()[:16]
        m = re.search(r'extern "C" __global__ void __launch_bounds__\([^)]*\) (\w+)\(', src)
        f = fams.setdefault(key, Family(key, m.group(1) if m else key, [], n))
        f.stages.append(i)
    return list(fams.values())


def decide(fams: List[Family], measure: Callable[[Dict[int, int]], float],
           margin: float = MARGIN) -> TuneReport:
    """The verdict procedure over any `measure(stage -> variant) -> seconds` instrument."""
    rep = TuneReport()
    chosen: Dict[int, int] = {}
    for f in fams:
        best: Optional[Tuple[float, int]] = None
        for v in range(1, f.variants):
            base = measure(chosen)                     # the current choice, measured adjacently
            cand = dict(chosen)
            cand.update({s: v for s in f.stages})
            t = measure(cand)
            rep.trials.append((f.kernel, v, base, t))
            ratio = t / base
            if ratio < 1.0 - margin and (best is None or ratio < best[0]):
                best = (ratio, v)
        if best is not None:
            chosen.update({s: best[1] for s in f.stages})
            rep.choices[f.kernel] = best[1]
    rep.baseline_s = measure({})
    rep.tuned_s = measure(chosen) if chosen else rep.baseline_s
    rep.shipped = bool(chosen) and rep.tuned_s < rep.baseline_s
    rep.variants = chosen if rep.shipped else {}
    if not rep.shipped:
        rep.choices = {}
    return rep


def zero_bindings(dev, prog: Program):
    """Zero-filled buffers for every input and state (the reference tunes over zeroed scratch
    bindings: the real dispatch list and memory traffic, no data)."""
    out = {}
    for b in prog.buffers:
        if b.role in (INPUT, STATE):
            buf = dev.alloc(max(1, b.nbytes))
            buf.upload(bytes(max(1, b.nbytes)))
            out[b.name] = buf
    return out


def step_instrument(dev, prog: Program, bindings=None, steps: int = 8, rounds: int = ROUNDS,
                    reset: Optional[Callable[[], None]] = None):
    """measure(stage -> variant): the program with those variants captured as one hipGraph
    over `bindings` (zeroed by default), the fastest of `rounds` timings of `steps` back-to-back
    replays, in seconds per step. `reset` runs before every timing (e.g. rewinding a decode
    position state, so that every candidate is timed at the same point of a sequence)."""
    bind = bindings if bindings is not None else zero_bindings(dev, prog)

    def measure(variants: Dict[int, int]) -> float:
        exe = dev.prepare(prog.with_variants(variants))
        rp = exe.capture(bind)
        if reset:
            reset()
        rp.step_many(2)
        times = []
        for _ in range(rounds):
            if reset:
                reset()
            times.append(rp.step_many(steps) / steps)
        del rp, exe
        return min(times)

    return measure


def tune(dev, prog: Program, bindings=None, steps: int = 8, rounds: int = ROUNDS,
         margin: float = MARGIN, reset: Optional[Callable[[], None]] = None) -> TuneReport:
    """SANIC_TUNE for one program on one device: returns the report; `report.variants` is what
    to pass to `Program.with_variants` (empty when the analytic program was not beaten)."""
    return decide(families(prog), step_instrument(dev, prog, bindings, steps, rounds, reset), margin)
