"""Configuration E under the reference's bf16 boundary policy (its `--bf16` run,
/root/reference/examples/llama3_2.rs:480-503; `Policy { boundary: BF16 }`, cost.rs:16-27): every
materialised intermediate — projections, attention output, residual stream, SwiGLU product and
the logits — stored bf16, against the oracle's run of the same policy
(tests/golden/llama_e_bf16.npz, written by `tests/golden/make_llama_e.py --bf16`).

The logits themselves are bf16 here, so the top two of a step are often exactly equal or one
bf16 step apart in the oracle's own values; the f32 evaluation may round either of them to the
other side of a bf16 boundary. A step whose oracle top-2 gap is at most two bf16 steps of the top
logit is a tie at this width: reported, not allowed to fail the run (the decode steps are fed
the oracle's ids, so a tie does not derail the steps after it)."""
import os

import numpy as np
import pytest

from sanic_amd import ir
from sanic_amd.llama import LlamaMachine
from tests.golden import make_llama_e as E
from tests.llama_ref import _upload, synth_weights

pytestmark = pytest.mark.gpu

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "llama_e_bf16.npz")
LOGIT_TOL = 2e-2        # the bf16 bound of the reference's metric |g − e| / (1 + |e|)


@pytest.mark.skipif(not os.path.exists(FIXTURE), reason="fixture not generated")
def test_config_e_bf16_policy_prefill_2048_then_32_greedy_steps(dev):
    f = np.load(FIXTURE)
    S = E.shape()
    w = synth_weights(S, seed=E.WEIGHT_SEED)
    m = LlamaMachine(dev, {n: _upload(dev, a) for n, a in w.items()}, S, boundary=ir.BF16)
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
            for idx, want in ((f["top_idx"][i], f["top_val"][i]), (probe, f["probe_val"][i])):
                err = float(np.max(np.abs(logits[idx] - want) / (1 + np.abs(want))))
                worst = max(worst, err)
                assert err < LOGIT_TOL, (pos, err)
        if got != ids[pos]:
            top = float(f["top_val"][check[pos]][0]) if pos in check else None
            bound = 2 * 2.0 ** -7 * (abs(top) if top is not None else 8.0)
            if gap[pos] <= bound:
                ties += 1
            else:
                mism.append((pos, got, int(ids[pos]), float(gap[pos])))
    n_exact = int(np.count_nonzero(gap == 0))
    print(f"config E (bf16 policy): logits max rel err {worst:.3e}; {ties} argmax ties; "
          f"{n_exact} steps whose oracle top two are equal in bf16; mismatches {mism}")
    assert not mism
