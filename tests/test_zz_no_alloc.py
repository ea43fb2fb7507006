"""sanic_hip_execute_static (no device allocation: the intermediates and the split/counter
arena in the library's static scratch) against sanic_hip_execute on the same inputs, bit for
bit, on two calls in a row — the second a smaller program — so the second call runs over
whatever the first left in the shared scratch."""
import numpy as np
import pytest

import oracle
from sanic_amd import carrier as C
from sanic_amd import configs, ir
from sanic_amd.abi import SanicError, lib
from sanic_amd.program import OUTPUT, SCRATCH, STREAM, Program, Sched

pytestmark = pytest.mark.gpu


def _both(dev, prog, vals):
    """(execute's outputs, execute_static's outputs) as raw bytes by name."""
    exe = dev.prepare(prog)
    bufs = {n: dev.from_values(v, prog.by_name[n].dtype) for n, v in vals.items()}
    want = {n: b.download() for n, b in exe.execute(bufs).items()}
    outs = {b.name: dev.alloc(b.nbytes) for b in prog.buffers if b.role == OUTPUT}
    for o in outs.values():
        o.upload(b"\xff" * o.nbytes)             # garbage the call must overwrite
    before = lib().sanic_hip_device_allocations()
    exe.execute_static({**bufs, **outs})
    allocated = lib().sanic_hip_device_allocations() - before
    got = {n: b.download() for n, b in outs.items()}
    assert allocated == 0, f"execute_static made {allocated} device allocations"
    return want, got, exe


def _flash(S):
    NH, NKV = 4, 2
    prog = configs.flash_prefill(NH, NKV, S, window=0).with_variants({2: 2})   # RoPE stages + split flash
    vals = {"Q": oracle.synth(700, NH * S * 64, dtype=ir.BF16).reshape(NH, S, 64),
            "K": oracle.synth(701, NKV * S * 64, dtype=ir.BF16).reshape(NKV, S, 64),
            "V": oracle.synth(702, NKV * S * 64, dtype=ir.BF16).reshape(NKV, S, 64)}
    return prog, vals


def _argmax(V):
    p = Program()
    x = p.input("x", (V,), ir.F32)
    p.fused("token", (1,), V, [(x, (STREAM,)), (ir.iota(V), (STREAM,))], C.first_argmax(), ir.U32,
            sched=Sched(lane_stream=True, waves=4, chunk=4, split=64))
    xv = oracle.lcg(V, V)
    xv[V // 3] = 3.0
    return p, {"x": xv}


@pytest.mark.parametrize("case", ["flash", "argmax"])
def test_execute_static_matches_execute_twice_second_smaller(dev, case):
    sizes = (1024, 256) if case == "flash" else (128256, 5000)
    for n in sizes:
        prog, vals = _flash(n) if case == "flash" else _argmax(n)
        want, got, exe = _both(dev, prog, vals)
        kinds = [exe.stage_kernel(i) for i in range(len(prog.stages))]
        print(case, n, kinds)
        if case == "flash":
            assert "+split2" in kinds[2]           # scratch partials + arrival counters in use
        else:
            assert kinds[0].startswith("fold:split")
        assert want.keys() == got.keys()
        for name in want:
            assert want[name] == got[name], (case, n, name)


def test_execute_static_refuses_programs_beyond_its_scratch(dev):
    """Intermediates larger than the static scratch: a clear error, nothing launched."""
    big = configs.flash_prefill(128, 64, 4096)         # RoPE'd K (32 MiB) and the rotation table (1 MiB)
    exe = dev.prepare(big)
    bufs = {b.name: dev.alloc(b.nbytes) for b in big.buffers if b.role != SCRATCH}
    with pytest.raises(SanicError) as e:
        exe.execute_static(bufs)
    assert "static scratch holds" in str(e.value)
