"""ctypes view of include/sanic_hip.h: record layouts and the library loader.

The record layouts are numpy structured dtypes with C alignment, checked against the library's
own `sizeof`s by `check_layouts()` (tests call it without a GPU).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsanic_hip.so")

MAX_RANK = 8
MAX_SLOTS = 8
MAX_LEAVES = 8

NODE_DT = np.dtype([
    ("kind", "<i4"), ("op", "<i4"), ("dtype", "<i4"), ("buffer", "<i4"), ("n_in", "<i4"),
    ("in", "<i4", 3), ("rank", "<i4"), ("dim", "<i4"), ("shape", "<i8", MAX_RANK),
    ("group", "<i4", MAX_RANK), ("padded", "<i4"), ("map_offset", "<i4"), ("value", "<f8"),
], align=True)

EXPR_DT = np.dtype([
    ("op", "<i4"), ("index", "<i4"), ("a", "<i4"), ("b", "<i4"), ("c", "<i4"), ("value", "<f8"),
], align=True)

SLOT_DT = np.dtype([("kind", "<i4"), ("monoid", "<i4"), ("ref_slot", "<i4"), ("ties", "<i4")],
                   align=True)

CARRIER_DT = np.dtype([
    ("slots", "<i4"), ("kind", SLOT_DT, MAX_SLOTS), ("identity", "<f8", MAX_SLOTS),
    ("into", "<i4", MAX_SLOTS), ("combine", "<i4", MAX_SLOTS), ("project", "<i4"),
], align=True)

SCHED_DT = np.dtype([("lane_stream", "<i4"), ("waves", "<i4"), ("chunk", "<i4"),
                     ("split", "<i4"), ("variant", "<i4")], align=True)

STAGE_DT = np.dtype([
    ("kind", "<i4"), ("out_buffer", "<i4"), ("out_dtype", "<i4"), ("rank", "<i4"),
    ("grid", "<i8", MAX_RANK), ("stream", "<i8"), ("n_leaves", "<i4"),
    ("leaf", "<i4", MAX_LEAVES), ("bind", "<i4", (MAX_LEAVES, MAX_RANK)),
    ("carrier", CARRIER_DT), ("epilogue", "<i4"), ("sched", SCHED_DT), ("value", "<i4"),
    ("where", "<i4"),
], align=True)

BUFFER_DT = np.dtype([("role", "<i4"), ("dtype", "<i4"), ("rank", "<i4"), ("scale", "<f4"),
                      ("shape", "<i8", MAX_RANK)], align=True)


class ProgramDesc(ctypes.Structure):
    _fields_ = [
        ("n_nodes", ctypes.c_int32), ("nodes", ctypes.c_void_p),
        ("n_exprs", ctypes.c_int32), ("exprs", ctypes.c_void_p),
        ("n_reindex", ctypes.c_int32), ("reindex", ctypes.c_void_p),
        ("n_buffers", ctypes.c_int32), ("buffers", ctypes.c_void_p),
        ("n_stages", ctypes.c_int32), ("stages", ctypes.c_void_p),
    ]


class DeviceSpecs(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 64), ("compute_units", ctypes.c_int32),
        ("wave_size", ctypes.c_int32), ("lds_bytes_per_cu", ctypes.c_int32),
        ("hbm_bytes_per_s", ctypes.c_double), ("bf16_mfma_flops", ctypes.c_double),
        ("f32_flops", ctypes.c_double), ("clock_hz", ctypes.c_double),
        ("hbm_bytes", ctypes.c_int64), ("sram_bytes", ctypes.c_double),
        ("regfile_bytes", ctypes.c_double), ("launch_overhead_s", ctypes.c_double),
        ("min_blocks", ctypes.c_double), ("mem_latency_s", ctypes.c_double),
    ]


# every function include/sanic_hip.h declares, with its ctypes signature
VP = ctypes.c_void_p
I = ctypes.c_int
SZ = ctypes.c_size_t
SIGNATURES = {
    "sanic_hip_last_error": (ctypes.c_char_p, []),
    "sanic_hip_open": (I, [I, ctypes.POINTER(VP)]),
    "sanic_hip_close": (None, [VP]),
    "sanic_hip_specs": (I, [VP, ctypes.POINTER(DeviceSpecs)]),
    "sanic_hip_alloc": (I, [VP, SZ, ctypes.POINTER(VP)]),
    "sanic_hip_free": (None, [VP]),
    "sanic_hip_upload": (I, [VP, SZ, VP, SZ]),
    "sanic_hip_download": (I, [VP, SZ, VP, SZ]),
    "sanic_hip_slice": (I, [VP, SZ, SZ, ctypes.POINTER(VP)]),
    "sanic_hip_buffer_bytes": (SZ, [VP]),
    "sanic_hip_buffer_device_ptr": (VP, [VP]),
    "sanic_hip_wrap": (I, [VP, VP, SZ, ctypes.POINTER(VP)]),
    "sanic_hip_prepare": (I, [VP, ctypes.POINTER(ProgramDesc), ctypes.POINTER(VP)]),
    "sanic_hip_exe_free": (None, [VP]),
    "sanic_hip_exe_stage_kernel": (I, [VP, I, ctypes.c_char_p, SZ]),
    "sanic_hip_exe_stage_source": (I, [VP, I, ctypes.c_char_p, SZ]),
    "sanic_hip_execute": (I, [VP, ctypes.POINTER(VP), I, ctypes.POINTER(VP)]),
    "sanic_hip_execute_static": (I, [VP, ctypes.POINTER(VP), I]),
    "sanic_hip_device_allocations": (ctypes.c_uint64, []),
    "sanic_hip_capture": (I, [VP, ctypes.POINTER(VP), I, ctypes.POINTER(ctypes.c_int32), I,
                              ctypes.POINTER(VP)]),
    "sanic_hip_replay_buffer": (I, [VP, I, ctypes.POINTER(VP)]),
    "sanic_hip_step": (I, [VP, ctypes.POINTER(ctypes.c_double)]),
    "sanic_hip_step_many": (I, [VP, I, ctypes.POINTER(ctypes.c_double)]),
    "sanic_hip_replay_free": (None, [VP]),
    "sanic_hip_profile_stages": (I, [VP, ctypes.POINTER(ctypes.c_double), I]),
    "sanic_hip_sync": (I, [VP]),
    "sanic_hip_abi_sizeof": (SZ, [ctypes.c_char_p]),
    "sanic_hip_precompile": (I, [ctypes.POINTER(ProgramDesc)]),
    "sanic_hip_stage_variants": (I, [ctypes.POINTER(ProgramDesc), I, ctypes.POINTER(ctypes.c_int)]),
    "sanic_hip_emit_source": (I, [ctypes.POINTER(ProgramDesc), I, ctypes.c_char_p, SZ,
                                  ctypes.c_char_p, SZ]),
}

_lib = None


class SanicError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[sanic_hip status {code}] {msg}")
        self.code = code


def lib():
    """Load the in-tree HIP library; raise loudly when it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with "
                               "`python -c 'import __graft_entry__ as g; g.build()'`")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status: int):
    if status != 0:
        msg = lib().sanic_hip_last_error()
        raise SanicError(status, msg.decode() if msg else "")


def check_layouts():
    """Compare every record layout with the C compiler's sizeof."""
    L = lib()
    want = {"sanic_node": NODE_DT.itemsize, "sanic_expr": EXPR_DT.itemsize,
            "sanic_slot": SLOT_DT.itemsize, "sanic_carrier": CARRIER_DT.itemsize,
            "sanic_sched": SCHED_DT.itemsize, "sanic_stage": STAGE_DT.itemsize,
            "sanic_buffer_desc": BUFFER_DT.itemsize,
            "sanic_program_desc": ctypes.sizeof(ProgramDesc),
            "sanic_device_specs": ctypes.sizeof(DeviceSpecs)}
    got = {k: L.sanic_hip_abi_sizeof(k.encode()) for k in want}
    return want, got
