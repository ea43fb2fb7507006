"""Shared helpers for the parity tests."""
import numpy as np


def max_rel_err(got, want) -> float:
    """The reference's metric |got − want| / (1 + |want|) (tests/metal.rs:99-105)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    if got.size == 0:
        return 0.0
    return float(np.max(np.abs(got - want) / (1.0 + np.abs(want))))


def floored_rel_err(got, want, floor: float = 1e-3) -> float:
    """|got − want| / max(|want|, floor): printed beside the reference's metric so that a
    regression on outputs near zero shows even where |g − e| / (1 + |e|) still passes."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    if got.size == 0:
        return 0.0
    return float(np.max(np.abs(got - want) / np.maximum(np.abs(want), floor)))


def run_on_gpu(dev, prog, vals, outputs=None):
    """prepare + execute `prog` with host values; return {output name: f64 values}."""
    exe = dev.prepare(prog)
    bufs = {n: dev.from_values(v, prog.by_name[n].dtype) for n, v in vals.items()}
    outs = exe.execute(bufs)
    res = {}
    for name, buf in outs.items():
        if outputs is None or name in outputs:
            b = prog.by_name[name]
            n = int(np.prod(b.shape)) if b.shape else 1
            res[name] = buf.read(b.dtype, n).reshape(b.shape)
    return res, exe
