"""safetensors checkpoints into device memory for the decode machine.

The reference opens a checkpoint zero-copy on unified memory: one page-aligned host region
holding the whole file, every tensor bound at its in-file offset
(/root/reference/examples/llama3_2.rs:346-380, `open_checkpoint_zero_copy`). On a discrete GPU
the weights have to live in HBM, so the same idea becomes one device arena holding the file's
whole data section, filled by large sequential uploads straight from a memory map, with every
tensor bound as a slice of the arena at its in-file offset (`sanic_hip_slice`). A tensor whose
offset is not 16-byte aligned (the kernels read weights in 128-bit runs) or whose dtype is not
bf16 gets an allocation of its own (f32 / f16 are narrowed to bf16 with round-to-nearest-even,
the storage the decode program reads).

Format (safetensors): 8-byte little-endian header length, a JSON header mapping names to
{"dtype", "shape", "data_offsets": [begin, end]} (offsets relative to the data section) plus an
optional "__metadata__" entry, then the data section.
"""
from __future__ import annotations

import json
import mmap
import struct
from dataclasses import dataclass
from typing import Dict, List, Tuple

import numpy as np

from .backend import Buffer, HipDevice, to_bf16_bits

_ELEM = {"BF16": 2, "F16": 2, "F32": 4}
CHUNK = 256 << 20


@dataclass
class TensorEntry:
    name: str
    dtype: str
    shape: Tuple[int, ...]
    begin: int
    end: int


def read_header(path: str) -> Tuple[Dict[str, TensorEntry], int, int]:
    """(entries, data_start, data_length) of a safetensors file; raises ValueError on a
    malformed header (offsets out of range, sizes that disagree with dtype × shape)."""
    with open(path, "rb") as f:
        raw = f.read(8)
        if len(raw) != 8:
            raise ValueError(f"{path}: shorter than a safetensors header")
        (hlen,) = struct.unpack("<Q", raw)
        header = json.loads(f.read(hlen))
        f.seek(0, 2)
        size = f.tell()
    data_start = 8 + hlen
    data_len = size - data_start
    out = {}
    for name, e in header.items():
        if name == "__metadata__":
            continue
        begin, end = (int(x) for x in e["data_offsets"])
        shape = tuple(int(x) for x in e["shape"])
        dt = e["dtype"]
        if not (0 <= begin <= end <= data_len):
            raise ValueError(f"{path}: {name} offsets {begin}..{end} outside the data section")
        if dt in _ELEM and end - begin != _ELEM[dt] * int(np.prod(shape, dtype=np.int64)):
            raise ValueError(f"{path}: {name} holds {end - begin} bytes, {dt}{list(shape)} needs more or less")
        out[name] = TensorEntry(name, dt, shape, begin, end)
    return out, data_start, data_len


def plan(entries: Dict[str, TensorEntry], wanted: List[Tuple[str, Tuple[int, ...]]]):
    """For each wanted (name, shape): ("slice", entry) when it can bind in place in the arena,
    ("convert", entry) when it needs its own bf16 allocation. Raises KeyError / ValueError for a
    missing tensor or a shape mismatch."""
    out = {}
    for name, shape in wanted:
        e = entries.get(name)
        if e is None:
            raise KeyError(f"checkpoint has no tensor {name!r}")
        if tuple(e.shape) != tuple(shape):
            raise ValueError(f"{name}: checkpoint shape {list(e.shape)}, the model needs {list(shape)}")
        if e.dtype not in _ELEM:
            raise ValueError(f"{name}: unsupported dtype {e.dtype}")
        out[name] = ("slice" if e.dtype == "BF16" and e.begin % 16 == 0 else "convert", e)
    return out


def _bf16_bits(view: memoryview, dtype: str) -> np.ndarray:
    if dtype == "BF16":
        return np.frombuffer(view, np.uint16).copy()
    src = np.frombuffer(view, np.float32 if dtype == "F32" else np.float16).astype(np.float32)
    return to_bf16_bits(src)


def load_weights(dev: HipDevice, path: str, wanted: List[Tuple[str, Tuple[int, ...]]]) -> Dict[str, Buffer]:
    """Device buffers for every wanted tensor: slices of one arena holding the data section,
    or own allocations for tensors that cannot bind in place. The arena stays alive as long as
    any slice does."""
    entries, data_start, data_len = read_header(path)
    how = plan(entries, wanted)
    out: Dict[str, Buffer] = {}
    with open(path, "rb") as f, mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) as mm:
        view = memoryview(mm)
        try:
            if any(k == "slice" for k, _ in how.values()):
                arena = dev.alloc(max(data_len, 1))
                for off in range(0, data_len, CHUNK):
                    n = min(CHUNK, data_len - off)
                    chunk = np.frombuffer(view[data_start + off:data_start + off + n], np.uint8)
                    arena.upload_array(chunk, off)       # straight from the page cache, no copy
                    del chunk
                for name, (kind, e) in how.items():
                    if kind == "slice":
                        out[name] = arena.slice(e.begin, e.end - e.begin)
            for name, (kind, e) in how.items():
                if kind == "convert":
                    bits = _bf16_bits(view[data_start + e.begin:data_start + e.end], e.dtype)
                    b = dev.alloc(bits.nbytes)
                    b.upload(bits.tobytes())
                    out[name] = b
        finally:
            view.release()
    return out


def write(path: str, tensors: Dict[str, Tuple[str, Tuple[int, ...], bytes]], align: int = 16):
    """Write a safetensors file (name -> (dtype, shape, raw bytes)), tensors in the given order,
    each data offset padded to `align` bytes (test fixtures and conversions)."""
    header, blobs, off = {}, [], 0
    for name, (dt, shape, raw) in tensors.items():
        pad = (-off) % align
        if pad:
            blobs.append(b"\0" * pad)
            off += pad
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(header).encode()
    h += b" " * ((-len(h)) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)
