"""Python binding of the CPU oracle — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this package, and
only as the checker. It loads oracle/_build/liboracle.so (built by `make -C oracle`), a plain-C
f64 restatement of sanic's interpreter (/root/reference/src/interp.rs) and of the hot-path
graphs; see interp.c and configs.c for the file:line each function follows.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Dict

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "liboracle.so")
_lib = None

D = ctypes.POINTER(ctypes.c_double)
VP = ctypes.c_void_p


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = ctypes.CDLL(LIB)
        L.oracle_round_bf16.restype = ctypes.c_double
        L.oracle_round_bf16.argtypes = [ctypes.c_double]
        L.oracle_round_to.restype = ctypes.c_double
        L.oracle_round_to.argtypes = [ctypes.c_int, ctypes.c_double]
        L.oracle_round_f16.restype = ctypes.c_double
        L.oracle_round_f16.argtypes = [ctypes.c_double]
        L.oracle_round_q8.restype = ctypes.c_double
        L.oracle_round_q8.argtypes = [ctypes.c_double, ctypes.c_double]
        L.oracle_eval.argtypes = [VP, ctypes.c_int, VP, VP]
        L.oracle_fold_stage.argtypes = [VP, ctypes.c_int, VP, ctypes.c_int, VP, VP]
        L.oracle_run_stage.argtypes = [VP, ctypes.c_int, VP, ctypes.c_int]
        L.oracle_run_program.argtypes = [VP, VP, ctypes.c_int]
        L.oracle_lcg_fill.argtypes = [ctypes.c_uint64, ctypes.c_int64, VP]
        L.oracle_synth_uniform.restype = ctypes.c_double
        L.oracle_synth_uniform.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        L.oracle_synth_normal.restype = ctypes.c_double
        L.oracle_synth_normal.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        L.oracle_synth_fill.argtypes = [ctypes.c_uint64, ctypes.c_int64, ctypes.c_int,
                                        ctypes.c_double, ctypes.c_double, ctypes.c_int, VP,
                                        ctypes.c_int]
        L.oracle_synth_fill_bf16.argtypes = [ctypes.c_uint64, ctypes.c_int64, ctypes.c_int,
                                             ctypes.c_double, ctypes.c_double, VP, ctypes.c_int]
        L.oracle_attention.argtypes = [VP, VP, VP, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_double,
                                       ctypes.c_int, ctypes.c_int64, ctypes.c_int64, VP,
                                       ctypes.c_int]
        L.oracle_rope.argtypes = [VP, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int64, VP]
        L.oracle_inv_freq.argtypes = [ctypes.c_double, ctypes.c_int, ctypes.c_int, VP]
        L.oracle_rmsnorm_proj.argtypes = [VP, VP, VP, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_double, VP, ctypes.c_int]
        L.oracle_int4_matmul.argtypes = [VP, VP, VP, VP, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_int, VP, ctypes.c_int]
        L.oracle_llama_step.restype = ctypes.c_int64
        L.oracle_llama_step.argtypes = [VP, ctypes.c_int64, ctypes.c_int64, VP, ctypes.c_int]
        _lib = L
    return _lib


def threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def _p(a: np.ndarray):
    return a.ctypes.data


def f64(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float64)


# ── scalar / generators ──

def round_bf16(v: float) -> float:
    return lib().oracle_round_bf16(float(v))


def round_f16(v: float) -> float:
    """round_to(F16, v) (scalar.rs:124-127, 154-178)."""
    return lib().oracle_round_f16(float(v))


def round_q8(scale: float, v: float) -> float:
    """round_to(Q8 { scale }, v) (scalar.rs:143-147)."""
    return lib().oracle_round_q8(float(scale), float(v))


def lcg(seed: int, n: int) -> np.ndarray:
    """The reference tests' xorshift64* stream, U(-1, 1) (tests/metal.rs:86-96)."""
    out = np.empty(n, np.float64)
    lib().oracle_lcg_fill(seed, n, _p(out))
    return out


def synth(seed: int, n: int, kind: str = "normal", a: float = 0.0, b: float = 1.0,
          dtype: int = 1) -> np.ndarray:
    """Counter-based synthetic values: N(a, b) or U(a, b), rounded through storage dtype."""
    out = np.empty(n, np.float64)
    lib().oracle_synth_fill(seed, n, 1 if kind == "uniform" else 0, a, b, dtype, _p(out),
                            threads())
    return out


def synth_bf16(seed: int, n: int, kind: str = "normal", a: float = 0.0, b: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.uint16)
    lib().oracle_synth_fill_bf16(seed, n, 1 if kind == "uniform" else 0, a, b, _p(out), threads())
    return out


# ── generic interpreter over a Program ──

def _buffers(prog, values: Dict[str, np.ndarray]):
    arrs = []
    for b in prog.buffers:
        n = int(np.prod(b.shape)) if b.shape else 1
        if b.name in values:
            a = f64(values[b.name]).reshape(-1).copy()
            if a.size != n:
                raise ValueError(f"{b.name}: {a.size} values for shape {b.shape}")
        else:
            a = np.zeros(n, np.float64)
        arrs.append(a)
    ptrs = (VP * len(arrs))(*[_p(a) for a in arrs])
    return arrs, ptrs


def run_program(prog, values: Dict[str, np.ndarray], blocks: int = 1) -> Dict[str, np.ndarray]:
    """Schedule::execute_env (partition.rs:2117-2176): every stage, outputs narrowed through
    their storage dtype. Returns every buffer's values by name (states updated in place)."""
    desc, keep = prog.pack()
    arrs, ptrs = _buffers(prog, values)
    if lib().oracle_run_program(ctypes.byref(desc), ptrs, blocks) != 0:
        raise RuntimeError("oracle_run_program failed")
    return {b.name: arrs[b.index].reshape(b.shape) for b in prog.buffers}


def fold_stage(prog, stage: int, values, blocks: int = 1):
    """run_carrier_split (interp.rs:555-643) of one fused stage → (fold values, raw acc)."""
    desc, keep = prog.pack()
    arrs, ptrs = _buffers(prog, values)
    st = prog.stages[stage]
    n = int(np.prod(st.grid))
    out = np.empty(n, np.float64)
    acc = np.empty(n * st.carrier.slots, np.float64)
    if lib().oracle_fold_stage(ctypes.byref(desc), stage, ptrs, blocks, _p(out), _p(acc)) != 0:
        raise RuntimeError("oracle_fold_stage failed (blocks out of range?)")
    return out.reshape(st.grid), acc.reshape(tuple(st.grid) + (st.carrier.slots,))


def eval_node(prog, node, values) -> np.ndarray:
    """interp.rs eval of a graph node (its Input leaves read program buffers by name)."""
    from sanic_amd import ir
    nt = ir.NodeTable(lambda n: prog.by_name[n.name].index)
    root = nt.add(node)
    # pack the program's own tables, then append this node table as a separate descriptor
    import sanic_amd.abi as abi
    nodes = nt.pack()
    reindex = np.array(nt.reindex or [0], dtype=np.int64)
    bufs = np.zeros(len(prog.buffers), dtype=abi.BUFFER_DT)
    for i, b in enumerate(prog.buffers):
        bufs[i]["role"], bufs[i]["dtype"], bufs[i]["rank"] = b.role, b.dtype, len(b.shape)
        bufs[i]["scale"] = ir.dtype_scale(b.dtype)
        bufs[i]["shape"] = list(b.shape) + [0] * (abi.MAX_RANK - len(b.shape))
    desc = abi.ProgramDesc(len(nodes), nodes.ctypes.data, 0, None, len(nt.reindex),
                           reindex.ctypes.data, len(bufs), bufs.ctypes.data, 0, None)
    arrs, ptrs = _buffers(prog, values)
    out = np.empty(int(np.prod(node.shape)) if node.shape else 1, np.float64)
    lib().oracle_eval(ctypes.byref(desc), root, ptrs, _p(out))
    return out.reshape(node.shape)


# ── fused loops ──

def attention(q, k, v, scale, mask=0, q_pos0=0, window=0, v_transposed=False, nthreads=None):
    q, k, v = f64(q), f64(k), f64(v)
    Hq, Sq, Dd = q.shape
    Hkv = k.shape[0]
    Sk = k.shape[1]
    out = np.empty((Hq, Sq, v.shape[1] if v_transposed else v.shape[2]), np.float64)
    lib().oracle_attention(_p(q), _p(k), _p(v), Hq, Hkv, Sq, Sk, Dd, int(v_transposed), scale,
                           mask, q_pos0, window, _p(out), nthreads or threads())
    return out


def inv_freq(theta: float, F: int, llama3: bool = False) -> np.ndarray:
    out = np.empty(F, np.float64)
    lib().oracle_inv_freq(theta, F, int(llama3), _p(out))
    return out


def rope(x, pos0: int, invf) -> np.ndarray:
    x = f64(x).copy()
    H, S, Dd = x.shape
    invf = f64(invf)
    lib().oracle_rope(_p(x), H, S, Dd, pos0, _p(invf))
    return x


def rmsnorm_proj(x, g, w_bits, eps, nthreads=None):
    x, g = f64(x), f64(g)
    w = np.ascontiguousarray(w_bits, dtype=np.uint16)
    M, K = x.shape
    N = w.shape[1]
    y = np.empty((M, N), np.float64)
    lib().oracle_rmsnorm_proj(_p(x), _p(g), _p(w), M, K, N, eps, _p(y), nthreads or threads())
    return y


def int4_matmul(x, packed, s, z, G, nthreads=None):
    x, s, z = f64(x), f64(s), f64(z)
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    M, K = x.shape
    N = s.shape[0]
    y = np.empty((M, N), np.float64)
    lib().oracle_int4_matmul(_p(x), _p(packed), _p(s), _p(z), M, K, N, G, _p(y),
                             nthreads or threads())
    return y
