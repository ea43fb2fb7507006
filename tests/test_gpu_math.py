"""MapOp::Sin / Cos as the kernels evaluate them (Cody–Waite reduction by π/2, hardware sine /
cosine of the remainder, the library functions beyond |a| ≥ 6400 and for non-finite angles)
against numpy's f64 sin / cos of the same f32 angles. The bound is absolute: the reference
compiles with relaxed math (metal.rs:164-172) and tests its outputs at 2e-3 .. 2e-2 relative; RoPE
angles reach ≈ 4100 rad in config E."""
import numpy as np
import pytest

from sanic_amd import ir
from sanic_amd.program import Program
from tests.util import run_on_gpu

pytestmark = pytest.mark.gpu


def test_sin_cos_against_f64(dev):
    rng = np.random.default_rng(5)
    a = np.concatenate([
        rng.uniform(-4, 4, 4096), rng.uniform(-6400, 6400, 4096),
        np.arange(0, 4096) * np.float32(0.0123),                      # RoPE-like p·invf
        rng.uniform(6400, 1e5, 1024) * rng.choice([-1, 1], 1024),     # the library path
        [0.0, -0.0, np.pi / 2, np.pi, 3 * np.pi / 2, 6399.9, -6399.9, 6400.0, 1e30],
    ]).astype(np.float32)
    a = np.concatenate([a, np.zeros((-a.size) % 8, np.float32)])
    n = a.size
    p = Program()
    x = p.input("x", (n,), ir.F32)
    p.pointwise("s", ir.map_(ir.SIN, x), ir.F32)
    p.pointwise("c", ir.map_(ir.COS, x), ir.F32)
    got, exe = run_on_gpu(dev, p, {"x": a.astype(np.float64)})
    ref_s, ref_c = np.sin(a.astype(np.float64)), np.cos(a.astype(np.float64))
    es = float(np.max(np.abs(got["s"] - ref_s)))
    ec = float(np.max(np.abs(got["c"] - ref_c)))
    print(exe.stage_kernel(0), "max |sin err|", es, "max |cos err|", ec)
    assert es < 4e-6 and ec < 4e-6
    inf = np.array([np.inf, -np.inf, np.nan], np.float32)
    p2 = Program()
    y = p2.input("x", (8,), ir.F32)
    p2.pointwise("s", ir.map_(ir.SIN, y), ir.F32)
    got2, _ = run_on_gpu(dev, p2, {"x": np.concatenate([inf, np.zeros(5, np.float32)]).astype(np.float64)})
    assert np.all(np.isnan(got2["s"][:3]))
