"""Positional IR — the node kinds a carrier's leaves are written in.

Restates the node vocabulary of /root/reference/src/ir.rs:72-123 (Input, Const, Iota,
Coordinate, Map, Reduce, Gather, View, Reindex) with purely positional shapes: a node's shape is
a tuple of extents and every operation names dimensions by position. Map broadcasting follows
the interpreter (/root/reference/src/interp.rs Map arm): inputs align to the trailing dimensions
of the output and extent-1 dimensions broadcast.

The frontend compositions below (matmul, softmax, attention, rms_norm, rope, update_cache,
argmax, silu) restate the graph *semantics* of /root/reference/src/ir.rs:1171-1526 and
/root/reference/src/nn.rs:27-212; they build the graphs whose meaning the oracle evaluates.
"""
from __future__ import annotations

import math

import numpy as np
from dataclasses import dataclass, field
from typing import List, Optional, Sequence, Tuple

# storage dtypes (include/sanic_hip.h)
F64, F32, F16, BF16, U32, I8, I4, U4, Q8 = range(9)
DTYPE_NAMES = {F64: "f64", F32: "f32", F16: "f16", BF16: "bf16", U32: "u32", I8: "i8", I4: "i4", U4: "u4",
               Q8: "q8"}


class Q8Dtype(int):
    """`Dtype::Q8 { scale }` (/root/reference/src/scalar.rs:190-198, `Dtype::q8` :276-282): the
    storage code Q8 with its grid step riding along — the scale is part of the type."""

    def __new__(cls, scale: float):
        obj = super().__new__(cls, Q8)
        obj.scale = float(np.float32(scale))
        return obj

    def __repr__(self):
        return f"q8({self.scale})"


def q8(scale: float) -> Q8Dtype:
    if not scale > 0:
        raise ValueError("a Q8 grid needs a positive scale")
    return Q8Dtype(scale)


def dtype_scale(dt: int) -> float:
    """The quantization scale of a dtype that has one (scalar.rs:284-289), else 0."""
    return float(getattr(dt, "scale", 0.0))


def dtype_bytes(dt: int, n: int) -> int:
    """Bytes of `n` packed elements of storage dtype `dt`."""
    if dt in (I4, U4):
        return (n + 1) // 2
    return n * {F64: 8, F32: 4, F16: 2, BF16: 2, U32: 4, I8: 1, Q8: 1}[int(dt)]


# MapOp codes (/root/reference/src/scalar.rs:45-69)
(ADD, SUB, MUL, DIV, MAX, MIN, LT, NEG, RECIP, EXP, LOG, SQRT, TANH, SIN, COS, WHERE,
 ROUND_BF16, ROUND_F32, ROUND_Q8, ROUND_F16) = range(20)
ARITY = {ADD: 2, SUB: 2, MUL: 2, DIV: 2, MAX: 2, MIN: 2, LT: 2, NEG: 1, RECIP: 1, EXP: 1,
         LOG: 1, SQRT: 1, TANH: 1, SIN: 1, COS: 1, WHERE: 3, ROUND_BF16: 1, ROUND_F32: 1,
         ROUND_Q8: 1, ROUND_F16: 1}
OP_NAMES = {ADD: "+", SUB: "-", MUL: "·", DIV: "/", MAX: "max", MIN: "min", LT: "<", NEG: "neg",
            RECIP: "recip", EXP: "exp", LOG: "log", SQRT: "sqrt", TANH: "tanh", SIN: "sin",
            COS: "cos", WHERE: "where", ROUND_BF16: "round_bf16", ROUND_F32: "round_f32",
            ROUND_Q8: "round_q8", ROUND_F16: "round_f16"}

# Monoids (/root/reference/src/scalar.rs:18-41)
M_ADD, M_MUL, M_MAX, M_MIN, M_LSE = range(5)
MONOID_IDENTITY = {M_ADD: 0.0, M_MUL: 1.0, M_MAX: -math.inf, M_MIN: math.inf, M_LSE: -math.inf}

# node kinds
INPUT, CONST, IOTA, COORDINATE, MAP, REDUCE, GATHER, VIEW, REINDEX, FOLD, SCAN = range(11)


@dataclass(eq=False)
class Node:
    kind: int
    shape: Tuple[int, ...]
    inputs: Tuple["Node", ...] = ()
    op: int = 0
    dim: int = 0
    value: float = 0.0
    name: str = ""
    dtype: int = F32
    group: Tuple[int, ...] = ()
    padded: bool = False
    # REINDEX: per source dim (terms=((coef, out_dim), ...), offset)
    rmap: Tuple[Tuple[Tuple[Tuple[int, int], ...], int], ...] = ()

    # operator sugar (Tensor-like, /root/reference/src/tensor.rs)
    def __add__(self, o): return map_(ADD, self, _n(o))
    def __radd__(self, o): return map_(ADD, _n(o), self)
    def __sub__(self, o): return map_(SUB, self, _n(o))
    def __rsub__(self, o): return map_(SUB, _n(o), self)
    def __mul__(self, o): return map_(MUL, self, _n(o))
    def __rmul__(self, o): return map_(MUL, _n(o), self)
    def __truediv__(self, o): return map_(DIV, self, _n(o))
    def __rtruediv__(self, o): return map_(DIV, _n(o), self)
    def __neg__(self): return map_(NEG, self)

    @property
    def rank(self) -> int:
        return len(self.shape)


def _n(x) -> Node:
    return x if isinstance(x, Node) else const(float(x))


# ── node constructors ─────────────────────────────────────────────────────────

def input_(name: str, shape: Sequence[int], dtype: int = F32) -> Node:
    return Node(INPUT, tuple(int(s) for s in shape), name=name, dtype=dtype)


def const(v: float) -> Node:
    return Node(CONST, (), value=float(v))


def iota(n: int) -> Node:
    return Node(IOTA, (int(n),))


def coordinate(src_or_shape, dim: int) -> Node:
    shape = src_or_shape.shape if isinstance(src_or_shape, Node) else tuple(src_or_shape)
    dim = dim % len(shape)
    return Node(COORDINATE, tuple(shape), dim=dim)


def broadcast_shape(shapes: Sequence[Tuple[int, ...]]) -> Tuple[int, ...]:
    r = max((len(s) for s in shapes), default=0)
    out = []
    for i in range(r):
        ext = 1
        for s in shapes:
            j = i - (r - len(s))
            if j < 0:
                continue
            e = s[j]
            if e != 1:
                if ext != 1 and ext != e:
                    raise ValueError(f"map: incompatible extents {shapes}")
                ext = e
        out.append(ext)
    return tuple(out)


def map_(op: int, *ins: Node) -> Node:
    ins = tuple(_n(i) for i in ins)
    if len(ins) != ARITY[op]:
        raise ValueError(f"map op {OP_NAMES[op]} takes {ARITY[op]} inputs")
    return Node(MAP, broadcast_shape([i.shape for i in ins]), ins, op=op)


def round_to(src: Node, dtype: int) -> Node:
    """MapOp::RoundTo(dtype) (scalar.rs:120-152, emit_metal.rs:95-104): the value a store at
    that width followed by a load gives. Q8 carries its scale in the node's `value`."""
    if int(dtype) == Q8:
        return Node(MAP, src.shape, (src,), op=ROUND_Q8, value=dtype_scale(dtype))
    if dtype == BF16:
        return map_(ROUND_BF16, src)
    if dtype == F32:
        return map_(ROUND_F32, src)
    if dtype == F16:
        return map_(ROUND_F16, src)
    if dtype == F64:
        return src
    raise ValueError(f"RoundTo({DTYPE_NAMES.get(int(dtype), dtype)}) needs a scale, not a plain rounding")


def reduce(src: Node, dim: int, monoid: int) -> Node:
    dim = dim % src.rank
    shape = src.shape[:dim] + src.shape[dim + 1:]
    return Node(REDUCE, shape, (src,), op=monoid, dim=dim)


def scan(src: Node, dim: int, monoid: int) -> Node:
    """Inclusive prefix fold along `dim` (ir.rs `scan`; interp.rs `eval_scan`): out[.., i, ..] =
    monoid over src[.., 0..=i, ..]."""
    dim = dim % src.rank
    return Node(SCAN, src.shape, (src,), op=monoid, dim=dim)


def gather(src: Node, index: Node, dim: int) -> Node:
    dim = dim % src.rank
    shape = src.shape[:dim] + index.shape + src.shape[dim + 1:]
    return Node(GATHER, shape, (src, index), dim=dim)


def view(src: Node, group: Sequence[int]) -> Node:
    """Merge consecutive source dims: output dim j flattens `group[j]` source dims."""
    group = tuple(int(g) for g in group)
    if sum(group) != src.rank:
        raise ValueError("view groups must cover the source rank")
    shape, d = [], 0
    for g in group:
        shape.append(math.prod(src.shape[d:d + g]))
        d += g
    return Node(VIEW, tuple(shape), (src,), group=group)


def reindex(src: Node, out_shape: Sequence[int], rmap, padded: bool = False) -> Node:
    """Affine reindex: for each source dim, (terms=((coef, out_dim),...), offset)."""
    rmap = tuple((tuple((int(c), int(d)) for c, d in terms), int(off)) for terms, off in rmap)
    if len(rmap) != src.rank:
        raise ValueError("reindex needs one map entry per source dim")
    return Node(REINDEX, tuple(int(s) for s in out_shape), (src,), padded=padded, rmap=rmap)


def fold_value(shape: Sequence[int]) -> Node:
    """Placeholder for the enclosing fused stage's fold value (epilogue trees only)."""
    return Node(FOLD, tuple(shape))


# ── movement compositions (ir.rs:1004-1363) ───────────────────────────────────

def permute(src: Node, perm: Sequence[int]) -> Node:
    out_shape = [src.shape[p] for p in perm]
    inv = {p: i for i, p in enumerate(perm)}
    return reindex(src, out_shape, [(((1, inv[d]),), 0) for d in range(src.rank)])


def transpose(src: Node, a: int, b: int) -> Node:
    a %= src.rank
    b %= src.rank
    perm = list(range(src.rank))
    perm[a], perm[b] = perm[b], perm[a]
    return permute(src, perm)


def unsqueeze(src: Node, dim: int) -> Node:
    dim = dim % (src.rank + 1)
    out = src.shape[:dim] + (1,) + src.shape[dim:]
    return reindex(src, out, [(((1, d if d < dim else d + 1),), 0) for d in range(src.rank)])


def split(src: Node, dim: int, outer: int, inner: int) -> Node:
    """Split dim into (outer, inner): source index = o·inner + i."""
    dim %= src.rank
    if src.shape[dim] != outer * inner:
        raise ValueError("split extents must multiply to the source extent")
    out = src.shape[:dim] + (outer, inner) + src.shape[dim + 1:]
    m = []
    for d in range(src.rank):
        if d < dim:
            m.append((((1, d),), 0))
        elif d == dim:
            m.append((((inner, dim), (1, dim + 1)), 0))
        else:
            m.append((((1, d + 1),), 0))
    return reindex(src, out, m)


def flatten(src: Node, a: int, b: int) -> Node:
    """Merge dims a..b (inclusive, consecutive) into one."""
    a %= src.rank
    b %= src.rank
    group = [1] * a + [b - a + 1] + [1] * (src.rank - b - 1)
    return view(src, group)


def flip(src: Node, dim: int) -> Node:
    dim %= src.rank
    n = src.shape[dim]
    m = [(((1, d),), 0) if d != dim else (((-1, d),), n - 1) for d in range(src.rank)]
    return reindex(src, src.shape, m)


def expand_heads(src: Node, head_dim: int, repeats: int) -> Node:
    """GQA repeat-interleave of a head dim (/root/reference/src/nn.rs:107-151): output head
    h reads source head h // repeats."""
    if repeats == 1:
        return src
    head_dim %= src.rank
    shape = list(src.shape)
    shape.insert(head_dim + 1, repeats)
    m = [(((1, d if d <= head_dim else d + 1),), 0) for d in range(src.rank)]
    expanded = reindex(src, shape, m)
    return flatten(expanded, head_dim, head_dim + 1)


# ── frontend compositions (ir.rs:1171-1526, nn.rs:27-212) ─────────────────────

def silu(x: Node) -> Node:
    """x · recip(1 + exp(−x)) (ir.rs:1500-1510)."""
    return map_(MUL, x, map_(RECIP, map_(ADD, const(1.0), map_(EXP, map_(NEG, x)))))


def matmul(a: Node, b: Node) -> Node:
    """[..., m, k] @ [..., k, n] via [..., m, k, 1]·[..., 1, k, n] summed over k
    (ir.rs:1171-1223)."""
    left = unsqueeze(a, a.rank)          # [..., m, k, 1]
    right = unsqueeze(b, b.rank - 2)     # [..., 1, k, n]
    prod = map_(MUL, left, right)
    return reduce(prod, prod.rank - 2, M_ADD)


def softmax(x: Node, dim: int) -> Node:
    """exp(x − max) / Σ exp(x − max) (ir.rs:1277-1284)."""
    dim %= x.rank
    m = unsqueeze(reduce(x, dim, M_MAX), dim)
    e = map_(EXP, map_(SUB, x, m))
    return map_(DIV, e, unsqueeze(reduce(e, dim, M_ADD), dim))


def causal_mask_like(scores: Node, qdim: int, kdim: int) -> Node:
    """where(q < k, −1e30, 0) (ir.rs:1511-1526)."""
    return map_(WHERE, map_(LT, coordinate(scores, qdim), coordinate(scores, kdim)),
                const(-1e30), const(0.0))


def attention(q: Node, k: Node, v: Node, mask: Optional[Node] = None, causal: bool = False,
              scale: Optional[float] = None, gqa: bool = False) -> Node:
    """scaled_dot_product_attention (nn.rs:27-105): softmax(Q·Kᵀ·scale + mask)·V, default
    scale 1/√E, GQA by repeat-interleave of the key/value heads."""
    if gqa:
        rep = q.shape[-3] // k.shape[-3]
        k = expand_heads(k, k.rank - 3, rep)
        v = expand_heads(v, v.rank - 3, rep)
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    scores = map_(MUL, matmul(q, transpose(k, -2, -1)), const(scale))
    if causal:
        scores = map_(ADD, scores, causal_mask_like(scores, -2, -1))
    elif mask is not None:
        scores = map_(ADD, scores, mask)
    return matmul(softmax(scores, -1), v)


def rms_norm(x: Node, g: Node, eps: float) -> Node:
    """x·g / √(mean(x², last) + eps) (nn.rs:165-169)."""
    n = x.shape[-1]
    ms = map_(MUL, reduce(map_(MUL, x, x), -1, M_ADD), const(1.0 / n))
    den = unsqueeze(map_(SQRT, map_(ADD, ms, const(eps))), x.rank - 1)
    return map_(DIV, map_(MUL, x, g), den)


def rope_inv_freq(theta: float, freqs: int) -> Node:
    """θ^(−f/F) as exp(f·(−ln θ / F)) (nn.rs:196-199)."""
    return map_(EXP, map_(MUL, iota(freqs), const(-math.log(theta) / freqs)))


def llama3_inv_freq(theta: float, freqs: int, factor=32.0, orig=8192.0, low=1.0, high=4.0) -> Node:
    """Llama-3 wavelength blend (/root/reference/examples/llama3_2.rs:91-107)."""
    inv = rope_inv_freq(theta, freqs)
    wave = map_(DIV, const(2.0 * math.pi), inv)
    low_wave = orig / low
    high_wave = orig / high
    smooth = map_(DIV, map_(SUB, map_(DIV, const(orig), wave), const(low)), const(high - low))
    scaled = map_(DIV, inv, const(factor))
    blended = map_(ADD, map_(MUL, map_(SUB, const(1.0), smooth), scaled), map_(MUL, smooth, inv))
    inner = map_(WHERE, map_(LT, wave, const(high_wave)), inv, blended)
    return map_(WHERE, map_(LT, const(low_wave), wave), scaled, inner)


def rope(x: Node, position: Node, inv_freq: Node) -> Node:
    """Rotate-half RoPE over the trailing head dim (nn.rs:171-194): split the head dim into
    (pair=2, frequency=F); out = x·cos(angle) + flip(x, pair)·sign·sin(angle), sign(pair) =
    2·pair − 1, angle[s, f] = (position + s·0)·inv_freq[f] broadcast over the sequence dim
    x.shape[-2]. A rank-1 `position` gives each row its own position (prefill)."""
    hd = x.shape[-1]
    F = hd // 2
    xs = split(x, -1, 2, F)                     # [..., seq, 2, F]
    seq = x.shape[-2]
    if position.rank == 0:
        # the reference's form: every row of the sequence at `position` (decode)
        pos = map_(ADD, map_(MUL, iota(seq), const(0.0)), position)   # [seq]
    else:
        pos = position                           # per-row positions [seq] (prefill)
    angle = map_(MUL, unsqueeze(pos, 1), unsqueeze(inv_freq, 0))   # [seq, F]
    angle = unsqueeze(angle, 1)                                    # [seq, 1, F]
    sign = unsqueeze(map_(SUB, map_(MUL, iota(2), const(2.0)), const(1.0)), 1)  # [2, 1]
    rotated = map_(MUL, flip(xs, -2), sign)
    out = map_(ADD, map_(MUL, xs, map_(COS, angle)), map_(MUL, rotated, map_(SIN, angle)))
    return flatten(out, -2, -1)


def rope_table(position: Node, inv_freq: Node) -> Node:
    """The rotation rope() applies, as a [seq, 2, F] value: [s, 0, f] = cos(angle[s, f]),
    [s, 1, f] = sin(angle[s, f]), angle[s, f] = position[s]·inv_freq[f] (nn.rs:171-194). It
    depends on the row and the frequency only, so every head that shares the positions can read
    one materialisation of it instead of evaluating cos and sin per element."""
    seq, F = position.shape[0], inv_freq.shape[0]
    angle = unsqueeze(map_(MUL, unsqueeze(position, 1), unsqueeze(inv_freq, 0)), 1)   # [seq, 1, F]
    which = coordinate((seq, 2, F), 1)
    return map_(WHERE, map_(LT, which, const(0.5)), map_(COS, angle), map_(SIN, angle))


def rope_tabled(x: Node, table: Node) -> Node:
    """rope() over x [..., seq, hd] with the rotation read from a rope_table [seq, 2, F]:
    out = x·cos + flip(x, pair)·sign·sin, the same rotate-half form."""
    hd = x.shape[-1]
    F = hd // 2
    seq = x.shape[-2]
    xs = split(x, -1, 2, F)                                         # [..., seq, 2, F]
    cos_t = reindex(table, (seq, 1, F), [(((1, 0),), 0), ((), 0), (((1, 2),), 0)])
    sin_t = reindex(table, (seq, 1, F), [(((1, 0),), 0), ((), 1), (((1, 2),), 0)])
    sign = unsqueeze(map_(SUB, map_(MUL, iota(2), const(2.0)), const(1.0)), 1)  # [2, 1]
    rotated = map_(MUL, flip(xs, -2), sign)
    out = map_(ADD, map_(MUL, xs, cos_t), map_(MUL, rotated, sin_t))
    return flatten(out, -2, -1)


def update_cache(cache: Node, current: Node, position: Node, seq_dim: int) -> Node:
    """where(idx < pos+1 and pos < idx+1, current, cache) (nn.rs:208-212)."""
    idx = coordinate(cache, seq_dim)
    at = map_(MUL, map_(LT, idx, map_(ADD, position, const(1.0))),
              map_(LT, position, map_(ADD, idx, const(1.0))))
    return map_(WHERE, at, current, cache)


def argmax(x: Node, dim: int) -> Node:
    """First index of the maximum (ir.rs:1415-1433)."""
    dim %= x.rank
    m = unsqueeze(reduce(x, dim, M_MAX), dim)
    cand = map_(WHERE, map_(LT, x, m), const(math.inf), coordinate(x, dim))
    return reduce(cand, dim, M_MIN)


# ── serialization to the C ABI's node table ───────────────────────────────────

class NodeTable:
    """Collects nodes (children before parents) and reindex maps into flat tables."""

    def __init__(self, buffer_index):
        self.buffer_index = buffer_index   # callable: Input node -> program buffer index
        self.nodes: List[Node] = []
        self.ids = {}
        self.reindex: List[int] = []

    def add(self, n: Node) -> int:
        key = id(n)
        if key in self.ids:
            return self.ids[key]
        for c in n.inputs:
            self.add(c)
        self.ids[key] = len(self.nodes)
        self.nodes.append(n)
        return self.ids[key]

    def pack(self):
        """numpy structured array matching `sanic_node`."""
        from . import abi
        import numpy as np
        arr = np.zeros(len(self.nodes), dtype=abi.NODE_DT)
        self.reindex = []
        for i, n in enumerate(self.nodes):
            r = arr[i]
            r["kind"] = n.kind
            r["op"] = n.op
            r["dtype"] = n.dtype
            r["buffer"] = self.buffer_index(n) if n.kind == INPUT else -1
            r["n_in"] = len(n.inputs)
            ins = [self.ids[id(c)] for c in n.inputs] + [-1] * (3 - len(n.inputs))
            r["in"] = ins
            r["rank"] = n.rank
            r["dim"] = n.dim
            sh = list(n.shape) + [0] * (8 - n.rank)
            r["shape"] = sh
            gr = list(n.group) + [0] * (8 - len(n.group))
            r["group"] = gr
            r["padded"] = int(n.padded)
            r["value"] = n.value
            if n.kind == REINDEX:
                r["map_offset"] = len(self.reindex)
                for terms, off in n.rmap:
                    self.reindex += [len(terms), off]
                    for c, d in terms:
                        self.reindex += [c, d]
            else:
                r["map_offset"] = -1
        return arr
