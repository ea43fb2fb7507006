"""Stateful decode over the HIP backend: the `Graph::compile_for` → `instantiate` →
`Machine::step` path (/root/reference/src/graph.rs:231-345) for the Llama-3.2 decode program,
on the generic `sanic_amd.graph` machine.

States (the K/V caches, the position and the current token) are allocated and zeroed at
instantiation (graph.rs:297-310); one step is one hipGraph replay; the greedy token is written
into the `tokens` state by the argmax kernel itself (where the reference feeds `token` back into
an input, compile.rs:869-961), so decode steps launch back to back with no host round trip. Prompt tokens are written by the host
before each prefill step, as the reference's token-by-token prefill does
(/root/reference/examples/llama3_2.rs:587-680).
"""
from __future__ import annotations

import struct
from typing import Dict, List, Optional

import numpy as np

from . import configs, ir
from .backend import Buffer, HipDevice
from .graph import Graph


class LlamaMachine:
    def __init__(self, dev: HipDevice, weights: Dict[str, Buffer],
                 shape: configs.LlamaShape = configs.LLAMA_1B, attn_sched=None,
                 variants: Optional[Dict[int, int]] = None, boundary: int = ir.F32):
        """`variants` (stage -> tiling variant) is what the measured tuner ships
        (`sanic_amd.tune`); none = the analytic choice of every kernel. `boundary` is the
        storage of every materialised intermediate (the reference's `--bf16` policy)."""
        self.dev = dev
        self.shape = shape
        graph = Graph(configs.llama_decode(shape, attn_sched=attn_sched, boundary=boundary))
        graph.output("logits")
        graph.output("token")
        self.step_program = graph.compile_for(dev, variants)
        self.machine = self.step_program.instantiate(weights)
        self.prog = self.step_program.program
        self.exe = self.step_program.exe
        self.bind = self.machine.bind
        self.replay = self.machine.replay
        self.tokens = self.bind["tokens"]
        self.logits = self.replay.buffer("logits")
        self.token = self.replay.buffer("token")

    @classmethod
    def from_checkpoint(cls, dev: HipDevice, path: str, shape: configs.LlamaShape = configs.LLAMA_1B, **kw):
        """A machine over a safetensors checkpoint (HF names; tied embeddings, as
        llama3_2.rs:88-110 reads them): the weights bind as slices of one device arena."""
        from . import checkpoint
        return cls(dev, checkpoint.load_weights(dev, path, shape.weight_shapes()), shape, **kw)

    def set_position(self, pos: int):
        self.bind["position"].upload(struct.pack("<f", float(pos)))

    def position(self) -> int:
        return int(struct.unpack("<f", self.bind["position"].download(4))[0])

    def set_token(self, tok: int):
        self.tokens.upload(struct.pack("<f", float(tok)))

    def step(self, token: Optional[int] = None) -> float:
        """One decode step; `token` overrides the fed-back token (prefill). Returns GPU s."""
        if token is not None:
            self.set_token(token)
        return self.machine.step()

    def prefill(self, prompt: List[int]) -> int:
        """Token-by-token prefill; returns the greedy token after the last prompt token."""
        for t in prompt:
            self.step(t)
        return self.last_token()

    def decode(self, n: int) -> float:
        """n greedy steps back to back (each step's token feeds the next); GPU seconds."""
        return self.machine.step_many(n)

    def last_token(self) -> int:
        return int(np.frombuffer(self.token.download(4), np.uint32)[0])

    def last_logits(self) -> np.ndarray:
        """The last step's logits as stored (f32, or bf16 under the bf16 policy), widened."""
        return self.machine.read("logits").astype(np.float32 if self.prog.by_name["logits"].dtype == ir.F32 else np.float64)

    def cache(self, layer: int, which: str) -> np.ndarray:
        b = self.prog.by_name[f"cache.{layer}.{which}"]
        return np.frombuffer(self.bind[b.name].download(), np.uint16).reshape(b.shape).copy()
