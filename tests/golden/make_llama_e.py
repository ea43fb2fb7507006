"""Writes tests/golden/llama_e.npz: the oracle's run of configuration E (BASELINE.json
configs[4]) — the full Llama-3.2-1B architecture with seeded random bf16 weights, a 2048-token
seeded random-id prompt prefilled token by token into the in-place KV cache, then 32 greedy
decode steps — as /root/reference/examples/llama3_2.rs:587-680 runs it (prefill loop, then the
greedy loop feeding each argmax back).

The model is the CPU oracle's fused f64 decode step (oracle_llama_step, oracle/configs.c), whose
agreement with the interpreter running the whole decode schedule is pinned in
tests/test_cpu_llama_oracle.py. Run from the repository root:

    python tests/golden/make_llama_e.py          # ≈25 min on 8 cores
    python tests/golden/make_llama_e.py --bf16   # the same under the bf16 boundary policy
                                                 # → llama_e_bf16.npz

Contents (all arrays; no pickles):
  prompt [2048] i32, ids [2080] i32 (the argmax after every step, prompt and decode),
  gap [2080] f64 (oracle top-1 minus top-2 logit), check_steps [n] i32 (the steps whose logits
  are sampled), top_idx/top_val [n, 16] (the 16 largest logits), probe_idx [64] i32 and
  probe_val [n, 64] (logits at fixed indices), cache_pos [4] i32 and kcache/vcache
  [layers, 4, kv_heads, head_dim] u16 (bf16 bits of the cache rows at those positions after the
  last step).
"""
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from sanic_amd import configs  # noqa: E402
from tests.llama_ref import OracleModel, synth_weights  # noqa: E402

PROMPT = 2048
DECODE = 32
WEIGHT_SEED = 11
PROMPT_SEED = 2048
CACHE_POS = (0, 1024, 2047, 2079)


def shape():
    return configs.LlamaShape(capacity=PROMPT + DECODE)


def prompt_ids(vocab):
    return np.random.default_rng(PROMPT_SEED).integers(0, vocab, size=PROMPT).astype(np.int32)


def check_steps():
    """Every 128th prompt step, the last prompt step and every decode step."""
    s = list(range(0, PROMPT - 1, 128)) + list(range(PROMPT - 1, PROMPT + DECODE))
    return np.array(s, np.int32)


def main(out=os.path.join(os.path.dirname(os.path.abspath(__file__)), "llama_e.npz"), boundary_bf16=False):
    S = shape()
    t0 = time.time()
    w = synth_weights(S, seed=WEIGHT_SEED)
    om = OracleModel(S, w, boundary_bf16=boundary_bf16)
    prompt = prompt_ids(S.vocab)
    probe = np.random.default_rng(7).choice(S.vocab, 64, replace=False).astype(np.int32)
    steps = set(check_steps().tolist())
    n = PROMPT + DECODE
    ids = np.zeros(n, np.int32)
    gap = np.zeros(n, np.float64)
    top_idx, top_val, probe_val = [], [], []
    tok = int(prompt[0])
    for pos in range(n):
        feed = int(prompt[pos]) if pos < PROMPT else tok
        tok, logits = om.step(feed, pos)
        ids[pos] = tok
        part = np.partition(logits, -2)[-2:]
        gap[pos] = part[1] - part[0]
        if pos in steps:
            order = np.argsort(-logits, kind="stable")[:16]
            top_idx.append(order.astype(np.int32))
            top_val.append(logits[order])
            probe_val.append(logits[probe])
        if pos % 64 == 0:
            print(f"step {pos}/{n} {time.time() - t0:.0f}s", flush=True)
    cp = np.array(CACHE_POS, np.int32)
    kc = np.stack([om.kc[l][:, cp, :] for l in range(S.layers)]).transpose(0, 2, 1, 3)  # [L, 4, kv, hd]
    vc = np.stack([om.vc[l][:, :, cp].transpose(0, 2, 1) for l in range(S.layers)]).transpose(0, 2, 1, 3)
    np.savez_compressed(out, prompt=prompt, ids=ids, gap=gap, check_steps=check_steps(),
                        top_idx=np.array(top_idx), top_val=np.array(top_val), probe_idx=probe,
                        probe_val=np.array(probe_val), cache_pos=cp, kcache=kc, vcache=vc)
    print(f"wrote {out} in {time.time() - t0:.0f}s")


if __name__ == "__main__":
    if "--bf16" in sys.argv:
        # the reference's bf16 boundary policy (llama3_2.rs --bf16): every intermediate stored bf16
        main(os.path.join(os.path.dirname(os.path.abspath(__file__)), "llama_e_bf16.npz"), boundary_bf16=True)
    else:
        main()
