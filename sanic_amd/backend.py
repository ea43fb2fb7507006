"""Host mirror of sanic's backend interface over the C ABI.

`HipDevice` mirrors `MetalDevice` (/root/reference/src/metal.rs:148-412) and the `Backend` trait
(`specs`, `prepare`, `execute`, /root/reference/src/compile.rs:87-108); `Executable.capture` and
`Replay.step` mirror `Program::capture` / `MetalReplay::step_timed`
(/root/reference/src/compile.rs:820-1035). Errors surface as `SanicError` carrying the C status
(compile.rs:42-58's RunError / CompileError variants).

The product path has no CPU fallback: without the built library, or without a HIP device,
every entry point raises.
"""
from __future__ import annotations

import ctypes
from typing import Dict, List, Optional, Sequence

import numpy as np

from . import abi, ir
from .program import INPUT, OUTPUT, SCRATCH, STATE, Program

VP = ctypes.c_void_p


# ── host-side encodings of storage dtypes ───────────────────────────────────

def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """f32 → bf16 bits, round to nearest even, NaN kept quiet (scalar.rs:128-135)."""
    f = np.ascontiguousarray(x, dtype=np.float32)
    b = f.view(np.uint32)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(f)
    if nan.any():
        r[nan] = ((b[nan] >> 16) | 0x0040).astype(np.uint16)
    return r


def from_bf16_bits(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def pack_nibbles(u: np.ndarray) -> np.ndarray:
    """Pack unsigned nibbles (0..15) two per byte, low nibble = even index."""
    u = np.asarray(u, dtype=np.uint8).reshape(-1)
    if u.size % 2:
        u = np.concatenate([u, np.zeros(1, np.uint8)])
    return (u[0::2] & 0xF) | ((u[1::2] & 0xF) << 4)


def encode(values: np.ndarray, dtype: int) -> bytes:
    """Values → storage bytes of `dtype` (I4: value + 8 stored; U4: value stored)."""
    v = np.asarray(values)
    if dtype == ir.F32:
        return np.ascontiguousarray(v, dtype=np.float32).tobytes()
    if dtype == ir.BF16:
        return to_bf16_bits(v.astype(np.float32)).tobytes()
    if dtype == ir.F16:
        return np.ascontiguousarray(v, dtype=np.float16).tobytes()
    if dtype == ir.U32:
        return np.ascontiguousarray(v, dtype=np.uint32).tobytes()
    if dtype == ir.I8:
        return np.ascontiguousarray(v, dtype=np.int8).tobytes()
    if dtype == ir.Q8:
        # the device's store rule: v/scale in f32, half-to-even, clamped to ±127
        q = np.rint(np.asarray(v, np.float32) / np.float32(ir.dtype_scale(dtype)))
        return np.clip(np.nan_to_num(q, nan=-127.0), -127, 127).astype(np.int8).tobytes()
    if dtype == ir.I4:
        return pack_nibbles(np.asarray(v, dtype=np.int64) + 8).tobytes()
    if dtype == ir.U4:
        return pack_nibbles(np.asarray(v, dtype=np.int64)).tobytes()
    raise ValueError(f"no device encoding for dtype {dtype}")


def decode(raw: bytes, dtype: int, n: int) -> np.ndarray:
    """Storage bytes → f64 values."""
    if dtype == ir.F32:
        return np.frombuffer(raw, np.float32, n).astype(np.float64)
    if dtype == ir.BF16:
        return from_bf16_bits(np.frombuffer(raw, np.uint16, n)).astype(np.float64)
    if dtype == ir.F16:
        return np.frombuffer(raw, np.float16, n).astype(np.float64)
    if dtype == ir.U32:
        return np.frombuffer(raw, np.uint32, n).astype(np.float64)
    if dtype == ir.Q8:   # q·scale in f32, as the device's load computes it
        return (np.frombuffer(raw, np.int8, n).astype(np.float32) * np.float32(ir.dtype_scale(dtype))).astype(np.float64)
    if dtype == ir.I8:
        return np.frombuffer(raw, np.int8, n).astype(np.float64)
    b = np.frombuffer(raw, np.uint8)
    u = np.empty(b.size * 2, np.int64)
    u[0::2] = b & 0xF
    u[1::2] = b >> 4
    u = u[:n]
    return (u - 8 if dtype == ir.I4 else u).astype(np.float64)


# ── device, buffers ─────────────────────────────────────────────────────────

class Buffer:
    def __init__(self, dev: "HipDevice", handle: int, nbytes: int):
        self.dev = dev
        self.handle = handle
        self.nbytes = nbytes

    def upload(self, data, offset: int = 0):
        mv = memoryview(bytes(data) if not isinstance(data, (bytes, bytearray)) else data)
        abi.check(abi.lib().sanic_hip_upload(self.handle, offset, ctypes.c_char_p(bytes(mv)), len(mv)))

    def upload_array(self, arr: np.ndarray, offset: int = 0):
        a = np.ascontiguousarray(arr)
        abi.check(abi.lib().sanic_hip_upload(self.handle, offset, a.ctypes.data, a.nbytes))

    def download(self, nbytes: Optional[int] = None, offset: int = 0) -> bytes:
        n = self.nbytes - offset if nbytes is None else nbytes
        out = ctypes.create_string_buffer(max(n, 1))
        abi.check(abi.lib().sanic_hip_download(self.handle, offset, out, n))
        return out.raw[:n]

    def read(self, dtype: int, n: int) -> np.ndarray:
        return decode(self.download(ir.dtype_bytes(dtype, n)), dtype, n)

    def slice(self, offset: int, nbytes: int) -> "Buffer":
        h = VP()
        abi.check(abi.lib().sanic_hip_slice(self.handle, offset, nbytes, ctypes.byref(h)))
        return Buffer(self.dev, h.value, nbytes)

    @property
    def device_ptr(self) -> int:
        return abi.lib().sanic_hip_buffer_device_ptr(self.handle)

    def __del__(self):
        try:
            if self.handle:
                abi.lib().sanic_hip_free(self.handle)
                self.handle = None
        except Exception:
            pass


class HipDevice:
    """MetalDevice::open counterpart: raises when no HIP device is present."""

    def __init__(self, ordinal: int = 0):
        h = VP()
        abi.check(abi.lib().sanic_hip_open(ordinal, ctypes.byref(h)))
        self.handle = h.value

    def specs(self) -> abi.DeviceSpecs:
        s = abi.DeviceSpecs()
        abi.check(abi.lib().sanic_hip_specs(self.handle, ctypes.byref(s)))
        return s

    def alloc(self, nbytes: int) -> Buffer:
        h = VP()
        abi.check(abi.lib().sanic_hip_alloc(self.handle, nbytes, ctypes.byref(h)))
        return Buffer(self, h.value, nbytes)

    def from_values(self, values, dtype: int) -> Buffer:
        raw = encode(values, dtype)
        b = self.alloc(len(raw))
        if raw:
            b.upload(raw)
        return b

    def wrap(self, device_ptr: int, nbytes: int) -> Buffer:
        """Borrow caller-owned device memory (from_bytes_nocopy)."""
        h = VP()
        abi.check(abi.lib().sanic_hip_wrap(self.handle, device_ptr, nbytes, ctypes.byref(h)))
        b = Buffer(self, h.value, nbytes)
        return b

    def prepare(self, prog: Program) -> "Executable":
        desc, keep = prog.pack()
        h = VP()
        abi.check(abi.lib().sanic_hip_prepare(self.handle, ctypes.byref(desc), ctypes.byref(h)))
        return Executable(self, prog, h.value)

    def sync(self):
        abi.check(abi.lib().sanic_hip_sync(self.handle))

    def close(self):
        if self.handle:
            abi.lib().sanic_hip_close(self.handle)
            self.handle = None


class Executable:
    def __init__(self, dev: HipDevice, prog: Program, handle: int):
        self.dev = dev
        self.prog = prog
        self.handle = handle

    def stage_kernel(self, i: int) -> str:
        buf = ctypes.create_string_buffer(256)
        abi.check(abi.lib().sanic_hip_exe_stage_kernel(self.handle, i, buf, 256))
        return buf.value.decode()

    def stage_source(self, i: int) -> str:
        buf = ctypes.create_string_buffer(1 << 22)
        abi.check(abi.lib().sanic_hip_exe_stage_source(self.handle, i, buf, 1 << 22))
        return buf.value.decode()

    def _bindings(self, bindings: Dict[str, Buffer]):
        arr = (VP * len(self.prog.buffers))()
        for b in self.prog.buffers:
            if b.name in bindings:
                arr[b.index] = bindings[b.name].handle
        unknown = set(bindings) - set(self.prog.by_name)
        if unknown:
            raise KeyError(f"unknown bindings {sorted(unknown)} (RunError::UnknownInput)")
        return arr

    def execute(self, bindings: Dict[str, Buffer]) -> Dict[str, Buffer]:
        """Backend::execute: run once, return fresh owned output buffers by name."""
        arr = self._bindings(bindings)
        outs = (VP * len(self.prog.buffers))()
        abi.check(abi.lib().sanic_hip_execute(self.handle, arr, len(self.prog.buffers), outs))
        res = {}
        for b in self.prog.buffers:
            if b.role == OUTPUT and outs[b.index]:
                res[b.name] = Buffer(self.dev, outs[b.index], b.nbytes)
        return res

    def execute_static(self, bindings: Dict[str, Buffer]):
        """sanic_hip_execute_static: run once with no device allocation — `bindings` holds the
        caller's buffers for every INPUT, STATE and OUTPUT buffer; intermediates and the
        split/counter arena use the library's static scratch. Returns without waiting."""
        missing = [b.name for b in self.prog.buffers if b.role == OUTPUT and b.name not in bindings]
        if missing:
            raise KeyError(f"outputs must be bound: {missing}")
        arr = self._bindings(bindings)
        abi.check(abi.lib().sanic_hip_execute_static(self.handle, arr, len(self.prog.buffers)))

    def capture(self, bindings: Dict[str, Buffer], feedback: Sequence = ()) -> "Replay":
        """Program::capture: freeze the bindings into one hipGraph; `feedback` pairs
        (output name, input name) copy an output into an input at the end of each step."""
        arr = self._bindings(bindings)
        fb = (ctypes.c_int32 * max(1, 2 * len(feedback)))()
        for i, (o, inp) in enumerate(feedback):
            fb[2 * i] = self.prog.by_name[o].index
            fb[2 * i + 1] = self.prog.by_name[inp].index
        h = VP()
        abi.check(abi.lib().sanic_hip_capture(self.handle, arr, len(self.prog.buffers), fb,
                                              len(feedback), ctypes.byref(h)))
        return Replay(self, h.value, bindings)

    def __del__(self):
        try:
            if self.handle:
                abi.lib().sanic_hip_exe_free(self.handle)
                self.handle = None
        except Exception:
            pass


class Replay:
    def __init__(self, exe: Executable, handle: int, bindings):
        self.exe = exe
        self.handle = handle
        self.bindings = dict(bindings)   # keep borrowed buffers alive

    def buffer(self, name: str) -> Buffer:
        b = self.exe.prog.by_name[name]
        h = VP()
        abi.check(abi.lib().sanic_hip_replay_buffer(self.handle, b.index, ctypes.byref(h)))
        return Buffer(self.exe.dev, h.value, b.nbytes)

    def step(self) -> float:
        """One replay; returns GPU seconds (MetalReplay::step_timed)."""
        s = ctypes.c_double()
        abi.check(abi.lib().sanic_hip_step(self.handle, ctypes.byref(s)))
        return s.value

    def step_many(self, n: int) -> float:
        s = ctypes.c_double()
        abi.check(abi.lib().sanic_hip_step_many(self.handle, n, ctypes.byref(s)))
        return s.value

    def profile_stages(self) -> List[float]:
        n = len(self.exe.prog.stages)
        arr = (ctypes.c_double * n)()
        abi.check(abi.lib().sanic_hip_profile_stages(self.handle, arr, n))
        return list(arr)

    def __del__(self):
        try:
            if self.handle:
                abi.lib().sanic_hip_replay_free(self.handle)
                self.handle = None
        except Exception:
            pass
