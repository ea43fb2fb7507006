"""Carriers: a fold as data — `into`, `combine`, `identity`, `project` over slot scalars.

Restates the data model of /root/reference/src/derive.rs:95-118 (`Expr`), :261-392
(`Carrier`), :518-530 (`SlotKind`) and the combine forms `assemble` builds
(/root/reference/src/derive.rs:1688-1747), including the −∞-guarded rescale of an ExpShifted
slot. `render()` prints the same math notation as the reference's `Carrier::render`
(derive.rs:345-392), so the restated carriers can be checked against the render strings the
reference's own tests pin (/root/reference/tests/laws.rs:108-126).

The reference *derives* carriers from a graph; the rest of its compiler is out of scope here,
so the carriers the hot path needs are restated by constructor (dot, norm-fused projection,
online softmax / FlashAttention, argmax, plain monoid folds). Each constructor names the
derivation rules that produce it in the reference.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

from . import ir

# Expr op codes beyond the MapOp codes (include/sanic_hip.h)
EX_CONST, EX_ITEM, EX_A, EX_B, EX_F = 100, 101, 102, 103, 104

SLOT_PLAIN, SLOT_EXP_SHIFTED, SLOT_AT_EXTREMUM = 0, 1, 2


@dataclass(eq=False)
class Expr:
    op: int
    index: int = 0
    args: tuple = ()
    value: float = 0.0

    def __add__(self, o): return Expr(ir.ADD, args=(self, _e(o)))
    def __sub__(self, o): return Expr(ir.SUB, args=(self, _e(o)))
    def __mul__(self, o): return Expr(ir.MUL, args=(self, _e(o)))
    def __truediv__(self, o): return Expr(ir.DIV, args=(self, _e(o)))


def _e(x) -> Expr:
    return x if isinstance(x, Expr) else cst(float(x))


def cst(v: float) -> Expr: return Expr(EX_CONST, value=float(v))
def item(i: int) -> Expr: return Expr(EX_ITEM, index=i)
def A(i: int) -> Expr: return Expr(EX_A, index=i)
def B(i: int) -> Expr: return Expr(EX_B, index=i)
def F(i: int) -> Expr: return Expr(EX_F, index=i)
def emax(a, b) -> Expr: return Expr(ir.MAX, args=(_e(a), _e(b)))
def emin(a, b) -> Expr: return Expr(ir.MIN, args=(_e(a), _e(b)))
def elt(a, b) -> Expr: return Expr(ir.LT, args=(_e(a), _e(b)))
def eexp(a) -> Expr: return Expr(ir.EXP, args=(_e(a),))
def esqrt(a) -> Expr: return Expr(ir.SQRT, args=(_e(a),))
def ewhere(c, a, b) -> Expr: return Expr(ir.WHERE, args=(_e(c), _e(a), _e(b)))


@dataclass
class Slot:
    kind: int
    monoid: int = ir.M_ADD      # PLAIN: its monoid; AT_EXTREMUM: the key monoid
    ref_slot: int = -1          # EXP_SHIFTED: max slot; AT_EXTREMUM: key slot
    ties: int = ir.M_ADD        # AT_EXTREMUM: the ties monoid


@dataclass
class Carrier:
    into: List[Expr]
    kinds: List[Slot]
    project: Expr
    rules: List[str] = field(default_factory=list)
    combine: List[Expr] = field(default_factory=list)
    identity: List[float] = field(default_factory=list)

    def __post_init__(self):
        if not self.combine:
            self.combine, self.identity = assemble(self.kinds)

    @property
    def slots(self) -> int:
        return len(self.into)

    # ── reference semantics (derive.rs:283-343): f64 evaluation ──
    def lift(self, items: Sequence[float]) -> List[float]:
        return [eval_expr(e, item=items) for e in self.into]

    def merge(self, a, b) -> List[float]:
        return [eval_expr(e, a=a, b=b) for e in self.combine]

    def proj(self, f) -> float:
        return eval_expr(self.project, f=f)

    def fold(self, items) -> float:
        acc = list(self.identity)
        for it in items:
            acc = self.merge(acc, self.lift(it))
        return self.proj(acc)

    def tree_fold(self, items) -> float:
        def rec(xs):
            if not xs:
                return list(self.identity)
            if len(xs) == 1:
                return self.lift(xs[0])
            mid = len(xs) // 2
            return self.merge(rec(xs[:mid]), rec(xs[mid:]))
        return self.proj(rec(list(items)))

    def render(self) -> str:
        """The reference's `Carrier::render` notation (derive.rs:345-392)."""
        row = lambda v: ";  ".join(f"s{i} = {render_expr(e, 0)}" for i, e in enumerate(v))
        return (f"carrier ({self.slots} slots) [{', '.join(self.rules)}]\n"
                f"  into:    {row(self.into)}\n  combine: {row(self.combine)}\n"
                f"  project: {render_expr(self.project, 0)}")


def assemble(kinds: Sequence[Slot]):
    """Combine forms and identities per slot kind (derive.rs:1688-1747)."""
    combine, identity = [], []
    for i, s in enumerate(kinds):
        if s.kind == SLOT_PLAIN:
            m = s.monoid
            if m in (ir.M_ADD, ir.M_LSE):
                combine.append(A(i) + B(i))
            elif m == ir.M_MUL:
                combine.append(A(i) * B(i))
            elif m == ir.M_MAX:
                combine.append(emax(A(i), B(i)))
            else:
                combine.append(emin(A(i), B(i)))
            identity.append(ir.MONOID_IDENTITY[m])
        elif s.kind == SLOT_EXP_SHIFTED:
            mx = s.ref_slot
            big = emax(A(mx), B(mx))
            ra = ewhere(elt(-math.inf, A(mx)), eexp(A(mx) - big), 0.0)
            rb = ewhere(elt(-math.inf, B(mx)), eexp(B(mx) - big), 0.0)
            combine.append(A(i) * ra + B(i) * rb)
            identity.append(0.0)
        else:
            k = s.ref_slot
            tied = {ir.M_ADD: A(i) + B(i), ir.M_MUL: A(i) * B(i), ir.M_MAX: emax(A(i), B(i)),
                    ir.M_MIN: emin(A(i), B(i))}[s.ties]
            if s.monoid == ir.M_MAX:
                combine.append(ewhere(elt(A(k), B(k)), B(i), ewhere(elt(B(k), A(k)), A(i), tied)))
            else:
                combine.append(ewhere(elt(A(k), B(k)), A(i), ewhere(elt(B(k), A(k)), B(i), tied)))
            identity.append(ir.MONOID_IDENTITY[s.ties])
    return combine, identity


# ── f64 evaluation of an Expr (derive.rs `eval`) ──────────────────────────────

def eval_expr(e: Expr, item=None, a=None, b=None, f=None) -> float:
    op = e.op
    if op == EX_CONST:
        return e.value
    if op == EX_ITEM:
        return float(item[e.index])
    if op == EX_A:
        return float(a[e.index])
    if op == EX_B:
        return float(b[e.index])
    if op == EX_F:
        return float(f[e.index])
    v = [eval_expr(x, item, a, b, f) for x in e.args]
    return apply_map(op, v)


def apply_map(op: int, v) -> float:
    """The scalar meaning of each MapOp (interp.rs:472-498)."""
    if op == ir.ADD: return v[0] + v[1]
    if op == ir.SUB: return v[0] - v[1]
    if op == ir.MUL: return v[0] * v[1]
    if op == ir.DIV:
        if v[1] == 0.0:
            if v[0] == 0.0 or math.isnan(v[0]):
                return math.nan
            return math.copysign(math.inf, v[0]) * math.copysign(1.0, v[1])
        return v[0] / v[1]
    if op == ir.MAX: return _fmax(v[0], v[1])
    if op == ir.MIN: return _fmin(v[0], v[1])
    if op == ir.LT: return 1.0 if v[0] < v[1] else 0.0
    if op == ir.NEG: return -v[0]
    if op == ir.RECIP: return apply_map(ir.DIV, [1.0, v[0]])
    if op == ir.EXP:
        try:
            return math.exp(v[0])
        except OverflowError:
            return math.inf
    if op == ir.LOG: return math.log(v[0]) if v[0] > 0 else (-math.inf if v[0] == 0 else math.nan)
    if op == ir.SQRT: return math.sqrt(v[0]) if v[0] >= 0 else math.nan
    if op == ir.TANH: return math.tanh(v[0])
    if op == ir.SIN: return math.sin(v[0])
    if op == ir.COS: return math.cos(v[0])
    if op == ir.WHERE: return v[1] if v[0] != 0.0 else v[2]
    raise ValueError(f"op {op}")


def _fmax(a, b):
    # Rust f64::max ignores NaN
    if math.isnan(a): return b
    if math.isnan(b): return a
    return a if a > b else b


def _fmin(a, b):
    if math.isnan(a): return b
    if math.isnan(b): return a
    return a if a < b else b


# ── rendering (derive.rs:372-470) ────────────────────────────────────────────

def _prec(e: Expr) -> int:
    if e.op == ir.LT: return 1
    if e.op in (ir.ADD, ir.SUB): return 2
    if e.op in (ir.MUL, ir.DIV): return 3
    return 4


def _num(v: float) -> str:
    """Rust's rendering in derive.rs render_expr: −∞ named, integers plain, else `{:e}`."""
    if v == -math.inf: return "-∞"
    if math.isfinite(v) and v == math.trunc(v) and abs(v) < 1e15: return str(int(v))
    if not math.isfinite(v): return "NaN" if math.isnan(v) else "inf"
    mant, exp = f"{v:.17e}".split("e")
    # shortest round-tripping mantissa, as Rust's LowerExp prints
    for digits in range(1, 18):
        m = f"{v:.{digits - 1}e}"
        if float(m) == v:
            mant, exp = m.split("e")
            break
    if "." in mant:
        mant = mant.rstrip("0").rstrip(".")
    return f"{mant}e{int(exp)}"


def render_expr(e: Expr, parent: int) -> str:
    op = e.op
    if op == EX_CONST: return _num(e.value)
    if op == EX_ITEM: return f"x{e.index}"
    if op == EX_A: return f"a{e.index}"
    if op == EX_B: return f"b{e.index}"
    if op == EX_F: return f"s{e.index}"
    p = _prec(e)
    if op in (ir.ADD, ir.SUB, ir.MUL, ir.DIV, ir.LT):
        sym = {ir.ADD: "+", ir.SUB: "-", ir.MUL: "·", ir.DIV: "/", ir.LT: "<"}[op]
        # right operand of a non-commutative op binds tighter; `<` tightens both sides
        lp = p + 1 if op == ir.LT else p
        rp = p + 1 if op in (ir.SUB, ir.DIV, ir.LT) else p
        lhs = render_expr(e.args[0], lp)
        rhs = render_expr(e.args[1], rp)
        joiner = "·" if op == ir.MUL else f" {sym} "
        s = f"{lhs}{joiner}{rhs}"
        return f"({s})" if p < parent else s
    name = {ir.MAX: "max", ir.MIN: "min", ir.EXP: "exp", ir.LOG: "log", ir.SQRT: "sqrt",
            ir.TANH: "tanh", ir.SIN: "sin", ir.COS: "cos", ir.WHERE: "where", ir.NEG: "neg",
            ir.RECIP: "recip"}.get(op, ir.OP_NAMES.get(op, "?"))
    return f"{name}({', '.join(render_expr(x, 0) for x in e.args)})"


# ── restated carriers for the hot path ───────────────────────────────────────

def plain(monoid: int, n_items: int = 1) -> Carrier:
    """`fold` of a plain monoid over the product of the items (rules: fold, fused-map)."""
    body = item(0)
    for i in range(1, n_items):
        body = body * item(i)
    return Carrier([body], [Slot(SLOT_PLAIN, monoid)], F(0),
                   rules=["fold"] + (["fused-map"] if n_items > 1 else []))


def dot(n_items: int = 2) -> Carrier:
    """Σ Πᵢ xᵢ — a contraction (matmul/GEMV/int4 matvec) as one Plain(Add) slot."""
    return plain(ir.M_ADD, n_items)


def norm_fused_projection(n: int, eps: float) -> Carrier:
    """RMSNorm fused into a consuming projection (/root/reference/tests/laws.rs:621-646):
    items (x, g, w); Acc = (Σ x·g·w, Σ x²); project = s0 / √(s1·(1/n) + eps) (defer-div)."""
    into = [item(0) * item(1) * item(2), item(0) * item(0)]
    proj = F(0) / esqrt(F(1) * cst(1.0 / n) + cst(eps))
    return Carrier(into, [Slot(SLOT_PLAIN, ir.M_ADD), Slot(SLOT_PLAIN, ir.M_ADD)], proj,
                   rules=["fold", "fused-map", "tuple", "defer-div"])


def online_softmax_weighted() -> Carrier:
    """The FlashAttention carrier (/root/reference/tests/laws.rs:108-126): items (score,
    value); slots (m, ℓ, o): into s0 = x0, s1 = 1, s2 = x1; m is Plain(Max), ℓ and o are
    ExpShifted on slot 0; project s2 / s1."""
    return Carrier([item(0), cst(1.0), item(1)],
                   [Slot(SLOT_PLAIN, ir.M_MAX), Slot(SLOT_EXP_SHIFTED, ref_slot=0),
                    Slot(SLOT_EXP_SHIFTED, ref_slot=0)],
                   F(2) / F(1), rules=["fold", "tuple", "rescale", "defer-div"])


def first_argmax() -> Carrier:
    """argmax as a key/payload product monoid: items (value, index); s0 = Max key, s1 = Min of
    the index among ties (AtExtremum, derive.rs:1714-1735); project s1."""
    return Carrier([item(0), item(1)],
                   [Slot(SLOT_PLAIN, ir.M_MAX),
                    Slot(SLOT_AT_EXTREMUM, monoid=ir.M_MAX, ref_slot=0, ties=ir.M_MIN)],
                   F(1), rules=["fold", "tuple"])


# ── serialization ────────────────────────────────────────────────────────────

class ExprTable:
    def __init__(self):
        self.exprs: List[Expr] = []
        self.ids = {}

    def add(self, e: Expr) -> int:
        if id(e) in self.ids:
            return self.ids[id(e)]
        kids = [self.add(x) for x in e.args]
        self.ids[id(e)] = len(self.exprs)
        self.exprs.append(e)
        e._kids = kids
        return self.ids[id(e)]

    def pack(self):
        from . import abi
        import numpy as np
        arr = np.zeros(len(self.exprs), dtype=abi.EXPR_DT)
        for i, e in enumerate(self.exprs):
            kids = [self.ids[id(x)] for x in e.args] + [-1] * (3 - len(e.args))
            arr[i]["op"] = e.op
            arr[i]["index"] = e.index
            arr[i]["a"], arr[i]["b"], arr[i]["c"] = kids
            arr[i]["value"] = e.value
        return arr
