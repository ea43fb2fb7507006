"""Attention at score magnitudes where an unshifted softmax overflows (tests/laws.rs:445-476):
planted scores around ±710, 300, 88 and 50, the maximum first or last in the stream. f32 exp
overflows past ≈88.7, so every GPU form of the ExpShifted carrier — the generic fold (scalar,
cooperative, split), the MFMA flash prefill and the split-K decode attention — must shift by
its running maximum and rescale on merge to come out finite and equal to the stable two-pass
result. Expected values come from the f64 oracle over the same (storage-rounded) inputs; the
oracle itself is checked against the closed-form two-pass softmax on the generic case."""
import numpy as np
import pytest

import oracle
from sanic_amd import configs, ir
from sanic_amd.backend import from_bf16_bits
from sanic_amd.program import Sched
from tests.util import max_rel_err, run_on_gpu

pytestmark = pytest.mark.gpu

CENTERS = [50.0, 88.0, 300.0, 710.0, -710.0]


def _noise(n, seed):
    """Offsets in [−4, 4] on a 1/8 grid (exact in bf16 and f32)."""
    return np.round((oracle.lcg(seed, n) * 2.0 - 1.0) * 32.0) / 8.0


def _bf16(a):
    f = np.ascontiguousarray(a, dtype=np.float32)
    b = f.view(np.uint32)
    return from_bf16_bits(((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)).astype(np.float64)


@pytest.mark.parametrize("sched", ["scalar", "coop", "split7"])
@pytest.mark.parametrize("center", CENTERS)
@pytest.mark.parametrize("max_pos", ["first", "last"])
def test_generic_fold_survives_overflow_magnitudes(dev, sched, center, max_pos):
    """Config A's fold (f32, 23 keys, no mask): every query row sees the planted scores
    s_j = K[j][0] / 8 (Q rows = e₀), so O = softmax(s)·V for each row."""
    n, D = 23, 64
    s = center + _noise(n, 42)
    s[0 if max_pos == "first" else n - 1] = center + 5.0
    q = np.zeros((n, D)); q[:, 0] = 1.0
    k = np.zeros((n, D)); k[:, 0] = 8.0 * s
    v = oracle.lcg(7, n * D).reshape(n, D)
    sc = {"scalar": Sched(), "coop": Sched(lane_stream=True, waves=1),
          "split7": Sched(lane_stream=True, waves=1, split=7)}[sched]
    prog = configs.direct_attention(S=n, D=D, causal=False, sched=sc)
    vals = {"Q": q, "K": k, "V": v}
    got, exe = run_on_gpu(dev, prog, vals)
    want = oracle.run_program(prog, vals)["O"]
    # the oracle against the stable two-pass softmax (shift by the true maximum) over the
    # f32-stored V; the oracle's output is narrowed to f32 too
    p = np.exp(s - s.max())
    two_pass = (p @ v.astype(np.float32).astype(np.float64)) / p.sum()
    assert np.allclose(want, two_pass[None, :], rtol=1e-6, atol=1e-7)
    assert np.all(np.isfinite(got["O"]))
    err = max_rel_err(got["O"], want)
    print(exe.stage_kernel(0), center, max_pos, err)
    assert err < 1e-4


@pytest.mark.parametrize("center", CENTERS)
def test_flash_prefill_survives_overflow_magnitudes(dev, center):
    """The MFMA flash skeleton (bf16, 4/2 heads, 256 positions, causal): scores
    s = (Q·K)/8 with Q = (64, 1, 0, …) and K_j = (center/8, c_j, 0, …), so every query row sees
    planted scores around `center` over its causal prefix; the largest key comes first for
    even KV heads and last for odd ones."""
    NH, NKV, S, HD = 4, 2, 256, 64
    q = np.zeros((NH, S, HD)); q[:, :, 0] = 64.0; q[:, :, 1] = 1.0
    k = np.zeros((NKV, S, HD))
    for h in range(NKV):
        k[h, :, 0] = center / 8.0
        k[h, :, 1] = 8.0 * _noise(S, 100 + h)
        k[h, 0 if h % 2 == 0 else S - 1, 1] = 40.0
    v = oracle.synth(9, NKV * S * HD, dtype=ir.BF16).reshape(NKV, S, HD)
    prog = configs.flash_prefill(NH, NKV, S, rope_stages=False)
    vals = {"Q": _bf16(q), "K": _bf16(k), "V": v}
    got, exe = run_on_gpu(dev, prog, vals)
    assert exe.stage_kernel(0).startswith("skeleton:flash_prefill")
    want = oracle.run_program(prog, vals)["O"]
    assert np.all(np.isfinite(got["O"]))
    err = max_rel_err(got["O"], want)
    print(exe.stage_kernel(0), center, err)
    assert err < 2e-2


@pytest.mark.parametrize("center", CENTERS)
def test_decode_attention_survives_overflow_magnitudes(dev, center):
    """The split-K decode skeleton (q given, no RoPE; cache capacity 640, position 600 so the
    stream spans several chunks): planted scores around `center` over the visible prefix, the
    largest at position 0 for even KV groups and at the current position for odd ones."""
    NH, NKV, HD, cap, pos = 32, 8, 64, 640, 600
    q = np.zeros((NH, HD)); q[:, 0] = 64.0; q[:, 1] = 1.0
    k = np.zeros((NKV, cap, HD))
    for g in range(NKV):
        k[g, :, 0] = center / 8.0
        k[g, :, 1] = 8.0 * _noise(cap, 200 + g)
        k[g, 0 if g % 2 == 0 else pos, 1] = 40.0
    v = oracle.synth(10, NKV * HD * cap, dtype=ir.BF16).reshape(NKV, HD, cap)
    prog = configs.decode_attention(NH, NKV, HD, cap, rope=False, out_dtype=ir.F32)
    vals = {"q": _bf16(q), "k_cache": _bf16(k), "v_cache": v, "position": np.array(float(pos))}
    got, exe = run_on_gpu(dev, prog, vals)
    assert exe.stage_kernel(0).startswith("skeleton:attn_decode")
    want = oracle.run_program(prog, vals)["o"]
    assert np.all(np.isfinite(got["o"]))
    err = max_rel_err(got["o"], want)
    print(exe.stage_kernel(0), center, err)
    assert err < 1e-4
