"""Configuration E end to end on the GPU against the oracle's run of it (tests/golden/llama_e.npz,
written by tests/golden/make_llama_e.py): the full Llama-3.2-1B architecture with seeded bf16
weights, a 2048-token prompt prefilled token by token into the in-place KV cache, then 32 greedy
decode steps (/root/reference/examples/llama3_2.rs:587-680) — the workload bench.py times.

Every step's greedy id is compared (2080 argmaxes). The decode steps are fed the oracle's ids
(teacher forcing), so a step whose top two logits the oracle itself separates by less than the
TIE_GAP — a tie at this precision — is reported, not allowed to derail the steps after it.
"""
import os

import numpy as np
import pytest

from sanic_amd.backend import from_bf16_bits
from sanic_amd.llama import LlamaMachine
from tests.golden import make_llama_e as E
from tests.llama_ref import _upload, synth_weights

pytestmark = pytest.mark.gpu

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "llama_e.npz")
# logits are f32 but sit downstream of 16 layers of bf16 K/V cache entries, each of which an
# f32 evaluation may round one step away from the f64 oracle's: the bf16 bound of the
# reference's metric |g − e| / (1 + |e|) (tests/metal.rs:99-105)
LOGIT_TOL = 2e-2


# a step whose oracle top-2 logits lie closer than this (absolute; the logits are ≈4 in size)
# is a tie at this precision: an f32 path may pick either
TIE_GAP = 1e-2


def test_config_e_prefill_2048_then_32_greedy_steps(dev):
    f = np.load(FIXTURE)
    S = E.shape()
    w = synth_weights(S, seed=E.WEIGHT_SEED)
    m = LlamaMachine(dev, {n: _upload(dev, a) for n, a in w.items()}, S)
    del w
    prompt, ids, gap = f["prompt"], f["ids"], f["gap"]
    assert np.array_equal(prompt, E.prompt_ids(S.vocab))
    check = {int(s): i for i, s in enumerate(f["check_steps"])}
    probe = f["probe_idx"]
    mism, ties, worst = [], 0, 0.0
    for pos in range(E.PROMPT + E.DECODE):
        feed = int(prompt[pos]) if pos < E.PROMPT else int(ids[pos - 1])
        m.step(feed)
        got = m.last_token()
        if pos in check:
            i = check[pos]
            logits = m.last_logits()
            top_idx, top_val = f["top_idx"][i], f["top_val"][i]
            for idx, want in ((top_idx, top_val), (probe, f["probe_val"][i])):
                err = float(np.max(np.abs(logits[idx] - want) / (1 + np.abs(want))))
                worst = max(worst, err)
                assert err < LOGIT_TOL, (pos, err)
        if got != ids[pos]:
            if gap[pos] < TIE_GAP:
                ties += 1
            else:
                mism.append((pos, got, int(ids[pos]), float(gap[pos])))
    print(f"config E: logits max rel err {worst:.3e} at the checked steps; "
          f"{ties} argmax ties (oracle gap within the tolerance), mismatches {mism}")
    assert not mism
    # measured: 0 ties over the 2080 steps
    assert ties <= 2
    # the cache rows at positions 0, 1024, 2047 and 2079 of every layer after the last step:
    # every element within one bf16 rounding step of the oracle's (2^-7 relative to the larger
    # of |e| and a quarter of the row's rms). Not bit-exact: the f32 path and the f64 oracle
    # round an element differently whenever its value lies within their difference of a bf16
    # rounding boundary, and these one-step differences feed forward through 16 layers and
    # 2048 positions until the late layers' hidden states differ by ~1e-3 of their rms (the
    # logits by ~1.4e-3; measured: 5114 of 65536 cache elements differ, none in layer 0's V
    # rows, none by more than one bf16 step of a typical element; the largest absolute
    # difference at a value near zero is 7.5e-4 at rms 0.9)
    total = off = 0
    worst_rel = worst_ref = 0.0
    for l in range(S.layers):
        kc = m.cache(l, "key")[:, f["cache_pos"], :].transpose(1, 0, 2)        # [4, kv, hd]
        vc = m.cache(l, "value")[:, :, f["cache_pos"]].transpose(2, 0, 1)      # [4, kv, hd]
        for got_bits, want_bits in ((kc, f["kcache"][l]), (vc, f["vcache"][l])):
            g = from_bf16_bits(got_bits).astype(np.float64)
            e = from_bf16_bits(want_bits).astype(np.float64)
            rms = np.sqrt(np.mean(e ** 2, axis=-1, keepdims=True))
            rel = np.abs(g - e) / np.maximum(np.abs(e), 0.25 * rms)
            worst_rel = max(worst_rel, float(rel.max()))
            # the reference's own metric (tests/metal.rs:99-105)
            worst_ref = max(worst_ref, float(np.max(np.abs(g - e) / (1.0 + np.abs(e)))))
            total += got_bits.size
            off += int(np.count_nonzero(got_bits != want_bits))
    print(f"cache rows: {off} of {total} bf16 elements differ from the oracle's bits, "
          f"max |g − e| / max(|e|, rms / 4) = {worst_rel:.3e}, max |g − e| / (1 + |e|) = {worst_ref:.3e}")
    # in the reference's metric: within 1e-2 (measured 5.2e-3), half the bf16 bound
    assert worst_ref <= 1e-2
    assert worst_rel <= 2.0 ** -7
    # measured: 5114 of 65536 (7.8%) differ
    assert off <= total * 10 // 100
