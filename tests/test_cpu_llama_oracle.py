"""The fused llama loop (oracle_llama_step) pinned against the generic interpreter running the
decode program's schedule — two independent restatements of examples/llama3_2.rs agree."""
import numpy as np

import oracle
from sanic_amd import configs
from tests.llama_ref import OracleModel, synth_weights

TINY = configs.LlamaShape(layers=2, hidden=128, heads=4, kv_heads=2, head_dim=32, ffn=256,
                          vocab=300, capacity=12)


def _values(prog, w, kc, vc, token, pos):
    vals = {}
    for name, a in w.items():
        vals[name] = (a.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    vals["tokens"] = np.array([float(token)])
    vals["position"] = np.array(float(pos))
    for l in range(TINY.layers):
        vals[f"cache.{l}.key"] = (kc[l].astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        vals[f"cache.{l}.value"] = (vc[l].astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return vals


def test_llama_step_oracle_matches_interpreter_schedule():
    w = synth_weights(TINY, seed=5)
    prog = configs.llama_decode(TINY)
    om = OracleModel(TINY, w)
    toks = [3, 17, 250, 9]
    for pos, t in enumerate(toks):
        vals = _values(prog, w, om.kc, om.vc, t, pos)
        res = oracle.run_program(prog, vals)
        tok_ref, logits_ref = om.step(t, pos)
        np.testing.assert_allclose(res["logits"], logits_ref, rtol=1e-6, atol=1e-6)
        assert int(res["token"][0]) == tok_ref
        assert float(res["position"]) == pos + 1
        for l in range(TINY.layers):
            kc = (om.kc[l].astype(np.uint32) << 16).view(np.float32)
            vc = (om.vc[l].astype(np.uint32) << 16).view(np.float32)
            np.testing.assert_array_equal(res[f"cache.{l}.key"].astype(np.float32), kc)
            np.testing.assert_array_equal(res[f"cache.{l}.value"].astype(np.float32), vc)


def test_llama_step_oracle_bf16_boundary_matches_interpreter_schedule():
    """The same pin under the reference's bf16 boundary policy (llama3_2.rs:480-503,
    cost.rs:16-27): every intermediate of the schedule stored bf16, the fused loop rounding at
    the same cuts."""
    from sanic_amd import ir
    w = synth_weights(TINY, seed=5)
    prog = configs.llama_decode(TINY, boundary=ir.BF16)
    om = OracleModel(TINY, w, boundary_bf16=True)
    toks = [3, 17, 250, 9]
    for pos, t in enumerate(toks):
        vals = _values(prog, w, om.kc, om.vc, t, pos)
        res = oracle.run_program(prog, vals)
        tok_ref, logits_ref = om.step(t, pos)
        # bf16-stored logits and caches: bit for bit at this size (measured), the strongest pin
        np.testing.assert_array_equal(res["logits"], logits_ref)
        assert int(res["token"][0]) == tok_ref
        for l in range(TINY.layers):
            kc = (om.kc[l].astype(np.uint32) << 16).view(np.float32)
            vc = (om.vc[l].astype(np.uint32) << 16).view(np.float32)
            np.testing.assert_array_equal(res[f"cache.{l}.key"].astype(np.float32), kc)
            np.testing.assert_array_equal(res[f"cache.{l}.value"].astype(np.float32), vc)
