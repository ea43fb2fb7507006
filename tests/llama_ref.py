"""Test helpers for the Llama decode parity checks: synthetic weights and the oracle model."""
import ctypes

import numpy as np

import oracle
from sanic_amd import configs

BF16_ONE = 0x3F80


def synth_weights(shape: configs.LlamaShape, seed: int = 1234):
    """Seeded bf16 weights N(0, 0.02) with norm gains 1 (the configuration's recipe)."""
    out = {}
    for i, (name, shp) in enumerate(shape.weight_shapes()):
        n = int(np.prod(shp))
        if name.endswith("norm.weight"):
            out[name] = np.full(shp, BF16_ONE, np.uint16)
        else:
            out[name] = oracle.synth_bf16(seed * 1000 + i, n, "normal", 0.0, 0.02).reshape(shp)
    return out


class OracleLlama(ctypes.Structure):
    P = ctypes.c_void_p
    _fields_ = [("layers", ctypes.c_int), ("hidden", ctypes.c_int), ("heads", ctypes.c_int),
                ("kv_heads", ctypes.c_int), ("head_dim", ctypes.c_int), ("ffn", ctypes.c_int),
                ("vocab", ctypes.c_int), ("capacity", ctypes.c_int), ("eps", ctypes.c_double),
                ("theta", ctypes.c_double), ("embed", P), ("final_norm", P),
                ("attn_norm", P * 32), ("mlp_norm", P * 32), ("wq", P * 32), ("wk", P * 32),
                ("wv", P * 32), ("wo", P * 32), ("wg", P * 32), ("wu", P * 32), ("wd", P * 32),
                ("kcache", P * 32), ("vcache", P * 32), ("boundary_bf16", ctypes.c_int)]


class OracleModel:
    """oracle_llama_step (oracle/configs.c) over host weights; keeps its own K/V caches."""

    def __init__(self, shape: configs.LlamaShape, w, boundary_bf16: bool = False):
        self.shape = shape
        self.w = w
        S = shape
        self.kc = [np.zeros((S.kv_heads, S.capacity, S.head_dim), np.uint16) for _ in range(S.layers)]
        self.vc = [np.zeros((S.kv_heads, S.head_dim, S.capacity), np.uint16) for _ in range(S.layers)]
        m = OracleLlama()
        m.layers, m.hidden, m.heads, m.kv_heads = S.layers, S.hidden, S.heads, S.kv_heads
        m.head_dim, m.ffn, m.vocab, m.capacity = S.head_dim, S.ffn, S.vocab, S.capacity
        m.eps, m.theta = S.eps, S.theta
        m.boundary_bf16 = int(boundary_bf16)
        p = lambda a: a.ctypes.data
        m.embed = p(w["model.embed_tokens.weight"])
        m.final_norm = p(w["model.norm.weight"])
        for l in range(S.layers):
            pre = f"model.layers.{l}."
            m.attn_norm[l] = p(w[pre + "input_layernorm.weight"])
            m.mlp_norm[l] = p(w[pre + "post_attention_layernorm.weight"])
            m.wq[l] = p(w[pre + "self_attn.q_proj.weight"])
            m.wk[l] = p(w[pre + "self_attn.k_proj.weight"])
            m.wv[l] = p(w[pre + "self_attn.v_proj.weight"])
            m.wo[l] = p(w[pre + "self_attn.o_proj.weight"])
            m.wg[l] = p(w[pre + "mlp.gate_proj.weight"])
            m.wu[l] = p(w[pre + "mlp.up_proj.weight"])
            m.wd[l] = p(w[pre + "mlp.down_proj.weight"])
            m.kcache[l] = p(self.kc[l])
            m.vcache[l] = p(self.vc[l])
        self.m = m

    def load_caches(self, kc, vc):
        for l in range(self.shape.layers):
            self.kc[l][...] = kc[l]
            self.vc[l][...] = vc[l]

    def step(self, token: int, pos: int, nthreads: int = 0):
        logits = np.empty(self.shape.vocab, np.float64)
        tok = oracle.lib().oracle_llama_step(ctypes.byref(self.m), token, pos, logits.ctypes.data,
                                             nthreads or oracle.threads())
        return int(tok), logits


def upload_weights(dev, w):
    return {name: dev.from_values(None, 0) if a is None else _upload(dev, a) for name, a in w.items()}


def _upload(dev, a):
    b = dev.alloc(a.nbytes)
    b.upload_array(a)
    return b
