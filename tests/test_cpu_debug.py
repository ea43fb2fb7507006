"""SANIC_DEBUG=1: the compiled schedule dump (the reference's debug level 1, lib.rs:25-46), from
the device-free precompile path, in a child process (the level is read once per process)."""
import os
import re
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_schedule_dump_lists_every_stage_with_its_kernel_and_bytes():
    code = ("from sanic_amd import configs\n"
            "configs.llama_decode(configs.LlamaShape(layers=2, capacity=64)).precompile()\n")
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, capture_output=True, text=True,
                       env=dict(os.environ, SANIC_DEBUG="1"), timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [l for l in r.stderr.splitlines() if l.startswith("***")]
    head = re.match(r"\*\*\* hip schedule: (\d+) stages", lines[0])
    assert head
    n = int(head.group(1))
    rows = [l for l in lines if re.match(r"\*\*\*\s+\d+ b\d+ ", l)]
    assert len(rows) == n
    assert any("skeleton:attn_decode" in l and "block=" in l for l in rows)
    assert any("batched-into" in l and "(in another launch)" in l for l in rows)
    assert re.match(r"\*\*\* hip schedule: ~[\d.]+MB logical", lines[-1])
