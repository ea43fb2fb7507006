"""SANIC_DEBUG=2/3/4 on the GPU, in child processes (the level is read once per process): the
per-replay line, the frozen-graph dump, and the stage-by-stage first step of level 4, which must
leave the same outputs and states as a plain replay."""
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
pytestmark = pytest.mark.gpu

CHILD = r"""
import numpy as np, struct
from sanic_amd import configs, ir
from sanic_amd.backend import HipDevice
from tests.llama_ref import synth_weights, _upload
from tests.test_cpu_llama_oracle import TINY
from sanic_amd.llama import LlamaMachine
dev = HipDevice(0)
w = synth_weights(TINY, seed=5)
m = LlamaMachine(dev, {k: _upload(dev, a) for k, a in w.items()}, TINY)
m.set_token(3)
m.replay.step_many(3)
print("TOK", m.last_token(), "POS", m.position(), "SUM", float(np.sum(m.last_logits())))
"""


def _run(level):
    env = dict(os.environ)
    env.pop("SANIC_DEBUG", None)
    if level:
        env["SANIC_DEBUG"] = str(level)
    r = subprocess.run([sys.executable, "-c", CHILD], cwd=ROOT, capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    out = [l for l in r.stdout.splitlines() if l.startswith("TOK")][-1]
    return out, r.stderr


def test_debug_levels_report_and_level4_changes_nothing():
    plain, _ = _run(0)
    dbg, err = _run(4)
    assert dbg == plain
    assert re.search(r"\*\*\* hip batched \d+ stages x3 +[\d.]+ms GPU per step", err)
    assert re.search(r"\*\*\* hip graph: \d+ launches", err)
    stage_lines = [l for l in err.splitlines() if re.match(r"\*\*\* hip +\d+ b\d+ +[\d.]+us", l)]
    assert len(stage_lines) >= 5 and any("attn_decode" in l for l in stage_lines)
    assert "stage-by-stage step" in err
