"""The hot-path workloads as programs (schedules), one builder per configuration.

Each builder restates what the reference's partitioner hands its backend for that graph: the
stages, each fused stage's carrier, its leaves as node trees and their axis bindings. The graph
semantics follow /root/reference/src/nn.rs and /root/reference/examples/llama3_2.rs.
"""
from __future__ import annotations

import math

from . import carrier as C
from . import ir
from .program import BCAST, STREAM, Program, Sched


def direct_attention(S: int = 128, D: int = 64, causal: bool = True, dtype: int = ir.F32,
                     sched: Sched = None) -> Program:
    """Config A: single-head softmax(QKᵀ/√d + causal)·V as one FlashAttention carrier fold
    (examples/direct_attention.rs; tests/laws.rs:108-126 carrier). Grid (query, value dim),
    stream = key index; leaves: the masked score (an in-body QKᵀ contraction) and V."""
    p = Program()
    q = p.input("Q", (S, D), dtype)
    k = p.input("K", (S, D), dtype)
    v = p.input("V", (S, D), dtype)
    scores = ir.map_(ir.MUL, ir.matmul(q, ir.transpose(k, 0, 1)), ir.const(1.0 / math.sqrt(D)))
    if causal:
        scores = ir.map_(ir.ADD, scores, ir.causal_mask_like(scores, 0, 1))
    p.fused("O", (S, D), S, [(scores, (0, STREAM)), (v, (STREAM, 1))],
            C.online_softmax_weighted(), ir.F32, sched=sched)
    return p


def precompile_all() -> None:
    """Fill the code-object cache with every shipped configuration's kernels."""
    for s in (None, Sched(lane_stream=True, waves=1), Sched(lane_stream=True, waves=2, split=4)):
        direct_attention(sched=s).precompile()
