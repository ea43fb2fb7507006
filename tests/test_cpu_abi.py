"""The C-ABI library without a GPU: it loads, exports every declared symbol, its records match
the Python layouts, and it lowers and compiles every shipped configuration (hipRTC needs no GPU).
"""
import ctypes
import os
import re

import numpy as np
import pytest

from sanic_amd import abi, carrier as C, configs, ir
from sanic_amd.program import STREAM, Program, Sched

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "sanic_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sanic_hip_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(abi.LIB_PATH)
    names = declared_functions()
    assert len(names) >= 25
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(abi.SIGNATURES), set(names) ^ set(abi.SIGNATURES)


def test_record_layouts_match():
    want, got = abi.check_layouts()
    assert want == got


def test_open_without_gpu_reports_backend_error():
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is present")
    h = ctypes.c_void_p()
    st = abi.lib().sanic_hip_open(0, ctypes.byref(h))
    assert st == 6 and not h.value   # SANIC_ERR_BACKEND (MetalDevice::open → None)


@pytest.mark.parametrize("name", ["A", "A_scalar", "A_coop", "A_split", "B1", "B1_rows", "B2", "D1", "D2", "C1", "C3",
                                  "E_qkv", "E_attn", "E_gateup"])
def test_lowering_chooses_the_expected_kernel(name):
    progs = {
        # no Sched: the priced default (one wave per point, runs of 2)
        "A": (configs.direct_attention(), 0, "fold:coop[auto w1 s1 c2]"),
        "A_scalar": (configs.direct_attention(sched=Sched()), 0, "fold:scalar"),
        "A_coop": (configs.direct_attention(sched=Sched(lane_stream=True, waves=2)), 0, "fold:coop"),
        "A_split": (configs.direct_attention(sched=Sched(lane_stream=True, waves=2, split=4)), 0, "fold:split"),
        "B1": (configs.rmsnorm_projection(kmajor=True), 0, "skeleton:gemv_kmajor"),
        "B1_rows": (configs.rmsnorm_projection(kmajor=False), 0, "skeleton:gemv"),
        "D1": (configs.int4_matmul(), 0, "skeleton:gemv"),
        "C3": (configs.decode_attention(), 0, "skeleton:attn_decode"),
        "B2": (configs.rmsnorm_projection(M=512), 0, "skeleton:gemm[128x128,a2,kn,pre,"),
        "D2": (configs.int4_matmul(M=128), 0, "skeleton:gemm[128x32,grp,"),
        "C1": (configs.flash_prefill(), 2, "skeleton:flash_prefill"),
        # q/k/v batched into one launch; this step's K/V cache writes done by the attention kernel
        "E_qkv": (configs.llama_decode(), 0, "skeleton:gemv[batched 3]"),
        "E_attn": (configs.llama_decode(), 5, "skeleton:attn_decode[rep 4]+writes2"),
        # gate/up batched with silu(gate)·up computed per row pair
        "E_gateup": (configs.llama_decode(), 7, "skeleton:gemv[batched 2]+paired"),
    }
    p, stage, want = progs[name]
    kind, src = p.emit(stage)
    assert kind.startswith(want), kind
    assert "extern \"C\" __global__" in src


@pytest.mark.parametrize("name,prog,stage,strategy", [
    ("C3", lambda: configs.decode_attention(), 0, "iterative-ilp"),
    ("D2", lambda: configs.int4_matmul(M=128), 0, "iterative-ilp"),
    ("D1", lambda: configs.int4_matmul(), 0, "iterative-ilp"),
    ("B1", lambda: configs.rmsnorm_projection(kmajor=True), 0, "max-memory-clause"),
    ("B1_rows", lambda: configs.rmsnorm_projection(kmajor=False), 0, "max-memory-clause"),
    ("E_gateup", lambda: configs.llama_decode(), 7, "max-memory-clause"),
    ("E_down", lambda: configs.llama_decode(), 10, "iterative-ilp"),
    ("E_o", lambda: configs.llama_decode(), 6, None),
    ("E_qkv", lambda: configs.llama_decode(), 0, None),
    ("E_lm_head", lambda: configs.llama_decode(), 176, "max-memory-clause"),
    ("B2", lambda: configs.rmsnorm_projection(M=512), 0, None),
    ("C1", lambda: configs.flash_prefill(), 2, None),
    ("A", lambda: configs.direct_attention(), 0, None),
])
def test_kernels_carry_their_scheduler_strategy(name, prog, stage, strategy):
    """The lowering marks the kernels measured faster under another machine-scheduler strategy
    with a first source line the compiler step turns into `-amdgpu-sched-strategy=<name>`."""
    kind, src = prog().emit(stage)
    first = src.split("\n", 1)[0]
    if strategy is None:
        assert not first.startswith("// sched-strategy:"), (kind, first)
    else:
        assert first == "// sched-strategy: " + strategy, (kind, first)


def test_precompile_small_program():
    configs.direct_attention(S=16, D=8).precompile()


def test_validation_rejects_bad_programs():
    p = Program()
    x = p.input("X", (4, 4))
    p.fused("Y", (4,), 4, [(x, (0, STREAM))], C.plain(ir.M_ADD))
    p.stages[0].grid = (5,)                 # grid no longer matches the output buffer
    with pytest.raises(abi.SanicError) as e:
        p.emit(0)
    assert e.value.code == 1
    q = Program()
    y = q.input("X", (4, 4))
    q.fused("Y", (4,), 4, [(y, (0, 1))], C.plain(ir.M_ADD))   # binding refers to a grid dim of extent 4? no: dim 1 absent
    with pytest.raises(abi.SanicError):
        q.emit(0)


def test_unpadded_out_of_bounds_reindex_is_rejected():
    p = Program()
    x = p.input("X", (4,))
    shifted = ir.reindex(x, (4,), [(((1, 0),), 1)], padded=False)   # reads X[i + 1]
    p.pointwise("Y", shifted, ir.F32)
    with pytest.raises(abi.SanicError):
        p.emit(0)


def test_int4_gemv_folds_each_run_as_scale_and_zero():
    """A packed 4-bit weight q·s − z with s, z constant over a run of 8 is folded per run
    (s·Σx·q − z·Σx, no per-element dequantization) in the GEMV; a bf16 GEMV and the int4 GEMM
    keep their per-element forms."""
    kind, src = configs.int4_matmul(M=1).emit(0)
    assert kind.startswith("skeleton:gemv")
    assert "rr0_0 = fmaf(" in src and "xs_0 +=" in src and "0x0F0F0F0Fu" in src
    assert "acc0_0 = fmaf(-" in src                       # the zero point enters once per run
    kind, src = configs.rmsnorm_projection(M=1, kmajor=False).emit(0)
    assert kind.startswith("skeleton:gemv") and "rr0_0" not in src
    kind, src = configs.int4_matmul(M=128).emit(0)
    assert kind.startswith("skeleton:gemm") and "0x0F0F0F0Fu" not in src
