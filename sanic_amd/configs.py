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


def flash_prefill(NH: int = 32, NKV: int = 8, S: int = 4096, HD: int = 64, theta: float = 500000.0,
                  window: int = 0, rope_stages: bool = True, v_transposed: bool = False) -> Program:
    """Config C (prefill): GQA causal attention over S tokens, RoPE (rotate-half, plain
    inv_freq, each row at its own position) on Q and K, scale 1/√HD; `window` > 0 adds the
    sliding-window mask (key visible iff q − window + 1 ≤ k ≤ q). The RoPE'd Q and K are
    materialised by two pointwise stages (bf16), then one FlashAttention carrier fold.
    `v_transposed` stores V as [NKV, HD, S] (keys contiguous, the decode cache's layout) and
    reads it through a transposed view.

    With RoPE the rotation of each (row, frequency) is materialised once (`rope_table`, f32
    [S, 2, HD/2]) for every head; K is rotated by a pointwise stage (bf16: every query block
    reads each key row, so it is rotated once, not per reader), and Q's rotation stays inside
    the fold's score leaf (the reference's in-body leaf, nn.rs:176-194), where each query row is
    read once."""
    p = Program()
    q = p.input("Q", (NH, S, HD), ir.BF16)
    k = p.input("K", (NKV, S, HD), ir.BF16)
    v = ir.transpose(p.input("V", (NKV, HD, S), ir.BF16), 1, 2) if v_transposed else p.input("V", (NKV, S, HD), ir.BF16)
    if rope_stages:
        invf = ir.rope_inv_freq(theta, HD // 2)
        table = p.pointwise("rope.table", ir.rope_table(ir.iota(S), invf), ir.F32, role=3)
        q = ir.rope_tabled(q, table)
        k = p.pointwise("Kr", ir.rope_tabled(k, table), ir.BF16, role=3)
    rep = NH // NKV
    scores = ir.reduce(ir.map_(ir.MUL, ir.unsqueeze(q, 2), ir.unsqueeze(ir.expand_heads(k, 0, rep), 1)), 3, ir.M_ADD)
    scores = ir.map_(ir.MUL, scores, ir.const(1.0 / math.sqrt(HD)))            # [NH, S, S]
    scores = ir.map_(ir.ADD, scores, ir.causal_mask_like(scores, 1, 2))
    if window:
        # key visible iff k ≥ q − window + 1:  mask where(k < q − (window − 1), −1e30, 0)
        lo = ir.map_(ir.SUB, ir.coordinate(scores, 1), ir.const(float(window - 1)))
        scores = ir.map_(ir.ADD, scores, ir.map_(ir.WHERE, ir.map_(ir.LT, ir.coordinate(scores, 2), lo),
                                                  ir.const(-1e30), ir.const(0.0)))
    vexp = ir.expand_heads(v, 0, rep)                                            # [NH, S, HD]
    p.fused("O", (NH, S, HD), S, [(scores, (0, 1, STREAM)), (vexp, (0, STREAM, 2))],
            C.online_softmax_weighted(), ir.BF16)
    return p


def precompile_all() -> None:
    """Fill the code-object cache with every shipped configuration's kernels."""
    for s in (None, Sched(lane_stream=True, waves=1), Sched(lane_stream=True, waves=2, split=4)):
        direct_attention(sched=s).precompile()
    for p in (rmsnorm_projection(kmajor=False), rmsnorm_projection(kmajor=True), int4_matmul(),
              decode_attention(), llama_decode(), flash_prefill(), flash_prefill(window=1024)):
        p.precompile()
    # every tiling variant the measured tuner may try (each stage takes variant v when it has
    # more than v; identical sources compile once)
    for p in (llama_decode(), decode_attention(), rmsnorm_projection(kmajor=False),
              flash_prefill(), flash_prefill(window=1024), flash_prefill(4, 2, 256), flash_prefill(4, 2, 256, window=64)):
        counts = p.stage_variants(-1)
        for v in range(1, max(counts) if counts else 1):
            p.with_variants({i: v for i, n in enumerate(counts) if n > v}).precompile()


def rmsnorm_projection(M: int = 1, K: int = 2048, N: int = 8192, eps: float = 1e-5,
                       kmajor: bool = True, sched: Sched = None) -> Program:
    """Config B: (x / rms(x) · g) · W with RMSNorm fused into the projection's fold
    (tests/laws.rs:621-646: Acc = (Σ x·g·w, Σ x²), defer-div). W is [K, N] (K-major, as the
    configuration states) or [N, K] (the reference's [out, in], llama3_2.rs:88)."""
    p = Program()
    x = p.input("x", (M, K), ir.BF16)
    g = p.input("g", (K,), ir.BF16)
    if kmajor:
        w = p.input("W", (K, N), ir.BF16)
        wb = (STREAM, 1)
    else:
        w = p.input("W", (N, K), ir.BF16)
        wb = (1, STREAM)
    p.fused("y", (M, N), K, [(x, (0, STREAM)), (g, (STREAM,)), (w, wb)],
            C.norm_fused_projection(K, eps), ir.BF16, sched=sched)
    return p


def int4_matmul(M: int = 1, K: int = 2048, N: int = 8192, G: int = 64, sched: Sched = None) -> Program:
    """Config D: y = x · dequant(W)ᵀ with W packed uint4 [N, K] (two per byte, low nibble =
    even k), per-group (G along K) bf16 scale s and zero point z: w = u·s − z. The weight leaf
    is the reference's grouped-W4 graph (tests/metal.rs:1179-1273): a [N, K/G, G] product with
    the [N, K/G] scale unsqueezed, flattened back to [N, K]."""
    p = Program()
    x = p.input("x", (M, K), ir.BF16)
    wq = p.input("Wq", (N, K // G, G), ir.U4)
    s = p.input("S", (N, K // G), ir.BF16)
    z = p.input("Z", (N, K // G), ir.BF16)
    deq = ir.map_(ir.SUB, ir.map_(ir.MUL, wq, ir.unsqueeze(s, 2)), ir.unsqueeze(z, 2))
    w = ir.flatten(deq, 1, 2)                      # [N, K]
    p.fused("y", (M, N), K, [(x, (0, STREAM)), (w, (1, STREAM))], C.dot(2), ir.BF16, sched=sched)
    return p


class LlamaShape:
    """Llama-3.2-1B architecture (/root/reference/examples/llama3_2.rs:36-56)."""

    def __init__(self, layers=16, hidden=2048, heads=32, kv_heads=8, head_dim=64, ffn=8192,
                 vocab=128256, capacity=2080, theta=500000.0, eps=1e-5):
        self.layers, self.hidden, self.heads, self.kv_heads = layers, hidden, heads, kv_heads
        self.head_dim, self.ffn, self.vocab, self.capacity = head_dim, ffn, vocab, capacity
        self.theta, self.eps = theta, eps

    def weight_shapes(self):
        """(name, shape) of every bf16 weight, in a fixed order."""
        H, F, hd = self.hidden, self.ffn, self.head_dim
        out = [("model.embed_tokens.weight", (self.vocab, H)), ("model.norm.weight", (H,))]
        for l in range(self.layers):
            pre = f"model.layers.{l}."
            out += [(pre + "input_layernorm.weight", (H,)),
                    (pre + "self_attn.q_proj.weight", (self.heads * hd, H)),
                    (pre + "self_attn.k_proj.weight", (self.kv_heads * hd, H)),
                    (pre + "self_attn.v_proj.weight", (self.kv_heads * hd, H)),
                    (pre + "self_attn.o_proj.weight", (H, self.heads * hd)),
                    (pre + "post_attention_layernorm.weight", (H,)),
                    (pre + "mlp.gate_proj.weight", (F, H)),
                    (pre + "mlp.up_proj.weight", (F, H)),
                    (pre + "mlp.down_proj.weight", (H, F))]
        return out

    def weight_bytes(self) -> int:
        import math as _m
        return sum(2 * _m.prod(s) for _, s in self.weight_shapes())


LLAMA_1B = LlamaShape()


def _split_heads(x, heads, hd):
    """[heads·hd] → [heads, 1, hd] (the q/k/v `.split(-1, heads, head_dim)` with seq = 1)."""
    s = ir.split(x, 0, heads, hd)                  # [heads, hd]
    return ir.unsqueeze(s, 1)


def llama_decode(shape: LlamaShape = LLAMA_1B, attn_sched: Sched = None,
                 argmax_sched: Sched = None, boundary: int = ir.F32) -> Program:
    """One decode step of the Llama-3.2 graph (/root/reference/examples/llama3_2.rs:112-253),
    cut into the stages a carrier partition yields:
      per layer: q/k/v projections with the input RMSNorm fused into their folds (norm-fused
      carrier; layer 0 reads the embedding row through a gather in its leaves) → in-place K/V
      cache row writes (update_cache, RoPE on k) →
      decode attention over the cache (online-softmax carrier; RoPE on q inside its leaf, the
      −∞ prefix mask of positions > pos) → o projection + residual (epilogue) → gate/up with
      the post-attention RMSNorm fused → silu(gate)·up (elementwise) → down projection +
      residual → final RMSNorm fused into the tied lm_head → argmax (key/tie carrier).
    Weights and the K/V caches are bf16; `token` is u32. Every materialised intermediate is
    stored in `boundary` — the reference's boundary-storage policy (`Policy { boundary }`,
    /root/reference/src/cost.rs:16-27): f32 by default, bf16 as its `--bf16` run
    (/root/reference/examples/llama3_2.rs:480-503); arithmetic stays f32 inside every stage."""
    S = shape
    H, hd, NH, NKV, F, V, Cap = S.hidden, S.head_dim, S.heads, S.kv_heads, S.ffn, S.vocab, S.capacity
    rep = NH // NKV
    p = Program()
    # the current token is step state too: the argmax's last workgroup writes the next one in
    # place (the reference feeds `token` back into the `tokens` input, compile.rs:869-961; as a
    # state the conversion runs inside the argmax kernel instead of as one more launch)
    tokens = p.state("tokens", (1,), ir.F32)
    # position is step state advanced on the device at the end of each step (graph.rs:51-125
    # `state` + `update`), so back-to-back replays need no host write
    pos = p.state("position", (), ir.F32)
    for name, shp in S.weight_shapes():
        p.input(name, shp, ir.BF16)
    for l in range(S.layers):
        p.state(f"cache.{l}.key", (NKV, Cap, hd), ir.BF16)
        p.state(f"cache.{l}.value", (NKV, hd, Cap), ir.BF16)
    invf = ir.llama3_inv_freq(S.theta, hd // 2)
    emb = p.node("model.embed_tokens.weight")
    B = boundary
    # the embedding row is read where it is used (layer 0's q/k/v leaves and its residual): a
    # gather is a load, so it is not materialised as a stage of its own
    x = ir.reindex(ir.gather(emb, tokens, 0), (H,), [((), 0), (((1, 0),), 0)])   # [H]
    for l in range(S.layers):
        pre = f"model.layers.{l}."
        g1 = p.node(pre + "input_layernorm.weight")
        proj = {}
        for nm, rows in (("q", NH * hd), ("k", NKV * hd), ("v", NKV * hd)):
            w = p.node(pre + f"self_attn.{nm}_proj.weight")
            proj[nm] = p.fused(f"{pre}{nm}", (rows,), H,
                               [(x, (STREAM,)), (g1, (STREAM,)), (w, (0, STREAM))],
                               C.norm_fused_projection(H, S.eps), B, role=3)
        posn = p.node("position")
        # K cache row: rope(k) at `position` (update_cache along the cache sequence dim)
        kc = p.node(f"cache.{l}.key")
        kr = ir.rope(_split_heads(proj["k"], NKV, hd), posn, invf)            # [kv, 1, hd]
        at_k = ir.map_(ir.MUL, ir.map_(ir.LT, ir.coordinate(kc, 1), ir.map_(ir.ADD, posn, ir.const(1.0))),
                       ir.map_(ir.LT, posn, ir.map_(ir.ADD, ir.coordinate(kc, 1), ir.const(1.0))))
        p.pointwise(f"{pre}kwrite", kr, ir.BF16, grid=kc.shape, where=at_k, into=f"cache.{l}.key")
        vc = p.node(f"cache.{l}.value")
        vt = ir.unsqueeze(ir.split(proj["v"], 0, NKV, hd), 2)                # [kv, hd, 1]
        at_v = ir.map_(ir.MUL, ir.map_(ir.LT, ir.coordinate(vc, 2), ir.map_(ir.ADD, posn, ir.const(1.0))),
                       ir.map_(ir.LT, posn, ir.map_(ir.ADD, ir.coordinate(vc, 2), ir.const(1.0))))
        p.pointwise(f"{pre}vwrite", vt, ir.BF16, grid=vc.shape, where=at_v, into=f"cache.{l}.value")
        # attention over the updated cache (GQA repeat-interleave), q roped in its leaf
        qr = ir.rope(_split_heads(proj["q"], NH, hd), posn, invf)              # [NH, 1, hd]
        kexp = ir.expand_heads(p.node(f"cache.{l}.key"), 0, rep)               # [NH, Cap, hd]
        scores = ir.reduce(ir.map_(ir.MUL, qr, kexp), 2, ir.M_ADD)             # [NH, Cap]
        scores = ir.map_(ir.MUL, scores, ir.const(1.0 / math.sqrt(hd)))
        visible = ir.map_(ir.LT, ir.iota(Cap), ir.map_(ir.ADD, posn, ir.const(1.0)))
        mask = ir.map_(ir.WHERE, visible, ir.const(0.0), ir.const(-math.inf))
        scores = ir.map_(ir.ADD, scores, mask)
        vexp = ir.permute(ir.expand_heads(p.node(f"cache.{l}.value"), 0, rep), (0, 2, 1))  # [NH, Cap, hd]
        att = p.fused(f"{pre}attn", (NH, hd), Cap, [(scores, (0, STREAM)), (vexp, (0, STREAM, 1))],
                      C.online_softmax_weighted(), B, sched=attn_sched, role=3)
        attf = ir.flatten(att, 0, 1)                                            # [NH·hd]
        wo = p.node(pre + "self_attn.o_proj.weight")
        x = p.fused(f"{pre}x_attn", (H,), NH * hd, [(attf, (STREAM,)), (wo, (0, STREAM))], C.dot(2),
                    B, epilogue=ir.map_(ir.ADD, x, ir.fold_value((H,))), role=3)
        g2 = p.node(pre + "post_attention_layernorm.weight")
        gu = {}
        for nm in ("gate", "up"):
            w = p.node(pre + f"mlp.{nm}_proj.weight")
            gu[nm] = p.fused(f"{pre}{nm}", (F,), H, [(x, (STREAM,)), (g2, (STREAM,)), (w, (0, STREAM))],
                             C.norm_fused_projection(H, S.eps), B, role=3)
        # the SwiGLU cone as its own elementwise stage (a cut the partitioner makes so the
        # down projection's leaf is a plain load, not silu recomputed per output row)
        hsw = p.pointwise(f"{pre}mlp.h", ir.map_(ir.MUL, ir.silu(gu["gate"]), gu["up"]), B, role=3)
        wd = p.node(pre + "mlp.down_proj.weight")
        x = p.fused(f"{pre}x_mlp", (H,), F, [(hsw, (STREAM,)), (wd, (0, STREAM))], C.dot(2), B,
                    epilogue=ir.map_(ir.ADD, x, ir.fold_value((H,))), role=3)
    gf = p.node("model.norm.weight")
    logits = p.fused("logits", (V,), H, [(x, (STREAM,)), (gf, (STREAM,)), (emb, (0, STREAM))],
                     C.norm_fused_projection(H, S.eps), B)
    p.fused("token", (1,), V, [(logits, (STREAM,)), (ir.iota(V), (STREAM,))], C.first_argmax(), ir.U32,
            sched=argmax_sched or Sched(lane_stream=True, waves=4, chunk=4, split=64))
    p.pointwise("position.next", ir.map_(ir.ADD, p.node("position"), ir.const(1.0)), ir.F32,
                grid=(), into="position")
    p.pointwise("tokens.next", p.node("token"), ir.F32, grid=(1,), into="tokens")
    return p


def decode_attention(NH: int = 32, NKV: int = 8, HD: int = 64, cap: int = 4096,
                     theta: float = 500000.0, llama3_rope: bool = False, out_dtype: int = ir.BF16,
                     sched: Sched = None, rope: bool = True) -> Program:
    """Config C (decode variant): one query token per head (RoPE at `position` applied in the
    score leaf) against a K cache [NKV, cap, HD] and a V cache stored transposed
    [NKV, HD, cap] (llama3_2.rs:160-173), GQA repeat-interleave, scale 1/√HD, prefix mask
    `iota < position + 1` (−∞ beyond, llama3_2.rs:175-176). `rope=False` takes q as given
    (already rotated), the form a prefill row is compared with."""
    p = Program()
    q = p.input("q", (NH, HD), ir.BF16)
    kc = p.input("k_cache", (NKV, cap, HD), ir.BF16)
    vc = p.input("v_cache", (NKV, HD, cap), ir.BF16)
    pos = p.input("position", (), ir.F32)
    invf = ir.llama3_inv_freq(theta, HD // 2) if llama3_rope else ir.rope_inv_freq(theta, HD // 2)
    qr = ir.rope(ir.unsqueeze(q, 1), pos, invf) if rope else ir.unsqueeze(q, 1)   # [NH, 1, HD]
    rep = NH // NKV
    scores = ir.reduce(ir.map_(ir.MUL, qr, ir.expand_heads(kc, 0, rep)), 2, ir.M_ADD)
    scores = ir.map_(ir.MUL, scores, ir.const(1.0 / math.sqrt(HD)))
    visible = ir.map_(ir.LT, ir.iota(cap), ir.map_(ir.ADD, pos, ir.const(1.0)))
    scores = ir.map_(ir.ADD, scores, ir.map_(ir.WHERE, visible, ir.const(0.0), ir.const(-math.inf)))
    vexp = ir.permute(ir.expand_heads(vc, 0, rep), (0, 2, 1))
    p.fused("o", (NH, HD), cap, [(scores, (0, STREAM)), (vexp, (0, STREAM, 1))],
            C.online_softmax_weighted(), out_dtype, sched=sched)
    return p
