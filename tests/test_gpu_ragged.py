"""Ragged and edge shapes through whatever kernel the lowering picks (skeleton or generic fold),
against the f64 interpreter: sizes that are not multiples of the skeletons' tiles, tiny output
extents, cache capacities that end inside a chunk or a 16-position run, early/late positions."""
import numpy as np
import pytest

import oracle
from sanic_amd import configs, ir
from tests.test_gpu_skeletons import bf16_rel
from tests.util import floored_rel_err, max_rel_err, run_on_gpu

pytestmark = pytest.mark.gpu


def _vals(prog, seed):
    """Seeded inputs for every input buffer: bf16/f32 values N(0,1); int4 codes U{0..15};
    scales U(0.001, 0.02) with zero points 8·scale; gains N(1, 0.02); weights N(0, 0.02)."""
    out = {}
    for i, b in enumerate(prog.buffers):
        if b.role != 0:
            continue
        n = int(np.prod(b.shape)) if b.shape else 1
        if b.dtype == ir.U4:
            v = np.floor(oracle.lcg(seed + i, n) * 8.0 + 8.0).clip(0, 15)
        elif b.name in ("g",):
            v = oracle.synth(seed + i, n, "normal", 1.0, 0.02, dtype=ir.BF16)
        elif b.name in ("W",):
            v = oracle.synth(seed + i, n, "normal", 0.0, 0.02, dtype=ir.BF16)
        elif b.name == "S":
            v = oracle.synth(seed + i, n, "uniform", 0.001, 0.02, dtype=ir.BF16)
        else:
            v = oracle.synth(seed + i, n, dtype=b.dtype if b.dtype in (ir.BF16, ir.F32) else ir.F32)
        out[b.name] = np.asarray(v, np.float64).reshape(b.shape)
    if "Z" in out and "S" in out:
        out["Z"] = 8.0 * out["S"]
    return out


@pytest.mark.parametrize("M,K,N,kmajor", [
    (1, 1000, 777, False),   # gemv, K not a multiple of 512 (guarded runs), odd N
    (1, 4096, 3, False),     # gemv split-K form with three rows
    (1, 1000, 777, True),    # N-contiguous weights at a ragged size
    (192, 320, 320, True),   # gemm, M not a multiple of 128
    (100, 256, 200, False),  # nothing tile-shaped: generic fold
])
def test_rmsnorm_projection_ragged(dev, M, K, N, kmajor):
    prog = configs.rmsnorm_projection(M=M, K=K, N=N, kmajor=kmajor)
    vals = _vals(prog, 600 + M + K)
    got, exe = run_on_gpu(dev, prog, vals)
    want = oracle.run_program(prog, vals)["y"]
    print(exe.stage_kernel(0), bf16_rel(got["y"], want))
    assert bf16_rel(got["y"], want) < 2e-2


@pytest.mark.parametrize("M,K,N,G", [(1, 1024, 777, 64), (96, 512, 192, 32)])
def test_int4_ragged(dev, M, K, N, G):
    prog = configs.int4_matmul(M=M, K=K, N=N, G=G)
    vals = _vals(prog, 700 + M)
    got, exe = run_on_gpu(dev, prog, vals)
    want = oracle.run_program(prog, vals)["y"]
    print(exe.stage_kernel(0), bf16_rel(got["y"], want))
    assert bf16_rel(got["y"], want) < 2e-2


@pytest.mark.parametrize("cap,pos", [(100, 0), (100, 57), (100, 99), (1000, 999), (1000, 500)])
def test_decode_attention_ragged_capacity(dev, cap, pos):
    """Capacities that end inside a chunk and inside a 16-position value run."""
    NH, NKV, HD = 8, 2, 64
    prog = configs.decode_attention(NH, NKV, HD, cap)
    vals = _vals(prog, 800 + cap)
    vals["position"] = np.array(float(pos))
    got, exe = run_on_gpu(dev, prog, vals)
    want = oracle.run_program(prog, vals)["o"]
    print(exe.stage_kernel(0), cap, pos, max_rel_err(got["o"], want), floored_rel_err(got["o"], want))
    assert exe.stage_kernel(0).startswith("skeleton:attn_decode")
    assert max_rel_err(got["o"], want) < 2e-2


@pytest.mark.parametrize("S,window", [(384, 100), (320, 0), (200, 0)])
def test_flash_prefill_ragged(dev, S, window):
    """Sequence lengths that are not multiples of the 128-row query block (the generic fold
    takes them) and a window that ends mid-tile."""
    prog = configs.flash_prefill(4, 2, S, window=window)
    vals = _vals(prog, 900 + S)
    got, exe = run_on_gpu(dev, prog, vals)
    want = oracle.run_program(prog, vals)["O"]
    print([exe.stage_kernel(i) for i in range(3)], max_rel_err(got["O"], want), floored_rel_err(got["O"], want))
    assert max_rel_err(got["O"], want) < 2e-2


@pytest.mark.parametrize("NH,NKV", [(8, 8), (16, 2), (24, 8), (8, 1)])
def test_decode_attention_head_groupings(dev, NH, NKV):
    """Query heads per KV head 1, 8 and 3 (the workgroup holds all query heads of its KV
    group): every head against the oracle, position past the first chunk."""
    cap, pos = 640, 601
    prog = configs.decode_attention(NH, NKV, 64, cap)
    vals = _vals(prog, 900 + NH + NKV)
    vals["position"] = np.array(float(pos))
    got, exe = run_on_gpu(dev, prog, vals)
    want = oracle.run_program(prog, vals)["o"]
    print(exe.stage_kernel(0), NH, NKV, max_rel_err(got["o"], want), floored_rel_err(got["o"], want))
    assert exe.stage_kernel(0).startswith("skeleton:attn_decode")
    assert max_rel_err(got["o"], want) < 2e-2


def _int4_form(form, M=1, K=2048, N=512, G=64):
    """y = x · dequant(W)ᵀ with the packed 4-bit weight written three ways: q·s − z (the
    reference's grouped W4 graph), q·s (no zero point) and (q − z)·s (zero subtracted first)."""
    from sanic_amd import carrier as C
    from sanic_amd.program import STREAM, Program
    p = Program()
    x = p.input("x", (M, K), ir.BF16)
    wq = p.input("Wq", (N, K // G, G), ir.U4)
    s = ir.unsqueeze(p.input("S", (N, K // G), ir.BF16), 2)
    z = ir.unsqueeze(p.input("Z", (N, K // G), ir.BF16), 2)
    if form == "qs-z":
        deq = ir.map_(ir.SUB, ir.map_(ir.MUL, wq, s), z)
    elif form == "qs":
        deq = ir.map_(ir.MUL, wq, s)
    else:
        deq = ir.map_(ir.MUL, ir.map_(ir.SUB, wq, z), s)
    p.fused("y", (M, N), K, [(x, (0, STREAM)), (ir.flatten(deq, 1, 2), (1, STREAM))], C.dot(2), ir.F32)
    return p


@pytest.mark.parametrize("form", ["qs-z", "qs", "q-z_s"])
def test_int4_gemv_dequant_forms(dev, form):
    """The GEMV folds a run of 8 as s·Σx·q − z·Σx when the weight is q·s ± z or q·s, and
    dequantizes per element otherwise; every form against the oracle at the f32 bound."""
    prog = _int4_form(form)
    vals = _vals(prog, 950)
    got, exe = run_on_gpu(dev, prog, vals)
    want = oracle.run_program(prog, vals)["y"]
    err = max_rel_err(got["y"], want)
    print(exe.stage_kernel(0), form, err)
    assert exe.stage_kernel(0).startswith("skeleton:gemv")
    assert err < 1e-4
