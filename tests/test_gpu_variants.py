"""Every tiling variant the skeletons offer (the measured tuner's candidates) against the oracle,
and one tuning run end to end."""
import numpy as np
import pytest

import oracle
from sanic_amd import configs, ir, tune
from sanic_amd.backend import from_bf16_bits
from tests.test_gpu_skeletons import _bf16_vals, bf16_rel
from tests.util import max_rel_err, run_on_gpu

pytestmark = pytest.mark.gpu


def _c3(dev, prog, pos):
    NH, NKV, HD, CAP = 32, 8, 64, 4096
    q = _bf16_vals(301, NH * HD).reshape(NH, HD)
    kc = _bf16_vals(302, NKV * CAP * HD).reshape(NKV, CAP, HD)
    vc = _bf16_vals(303, NKV * HD * CAP).reshape(NKV, HD, CAP)
    got, exe = run_on_gpu(dev, prog, {"q": q, "k_cache": kc, "v_cache": vc, "position": np.array(float(pos))})
    qr = oracle.rope(q[:, None, :], pos, oracle.inv_freq(500000.0, HD // 2))
    want = oracle.attention(qr, kc, vc, 1.0 / 8.0, mask=3, q_pos0=pos, v_transposed=True)[:, 0, :]
    return bf16_rel(got["o"], want), exe


@pytest.mark.parametrize("variant", range(7))
@pytest.mark.parametrize("pos", [4095, 300])
def test_decode_attention_variants(dev, variant, pos):
    prog = configs.decode_attention().with_variants({0: variant})
    assert prog.stage_variants(0) == 7
    err, exe = _c3(dev, prog, pos)
    print(variant, pos, exe.stage_kernel(0), err)
    assert exe.stage_kernel(0).startswith("skeleton:attn_decode")
    assert err < 2e-2


@pytest.mark.parametrize("variant", range(4))
def test_gemv_rows_per_workgroup_variants(dev, variant):
    K, N = 2048, 8192
    prog = configs.rmsnorm_projection(M=1, K=K, N=N, kmajor=False).with_variants({0: variant})
    x = _bf16_vals(101, K).reshape(1, K)
    g = _bf16_vals(102, K, 1.0, 0.02)
    wbits = oracle.synth_bf16(103, N * K, "normal", 0.0, 0.02).reshape(N, K)
    got, exe = run_on_gpu(dev, prog, {"x": x, "g": g, "W": from_bf16_bits(wbits).astype(np.float64)})
    want = oracle.rmsnorm_proj(x, g, np.ascontiguousarray(wbits.T), 1e-5)
    print(variant, exe.stage_kernel(0), bf16_rel(got["y"], want))
    assert exe.stage_kernel(0).startswith("skeleton:gemv")
    assert bf16_rel(got["y"], want) < 2e-2


@pytest.mark.parametrize("variant", [1, 2])
@pytest.mark.parametrize("window", [0, 64])
def test_flash_occupancy_and_split_variants(dev, window, variant):
    """Variant 1: two workgroups per CU; variant 2: every block's key range split over two
    workgroups whose (m, ℓ, o) partials the later one combines."""
    NH, NKV, S = 4, 2, 256
    prog = configs.flash_prefill(NH, NKV, S, window=window).with_variants({2: variant})
    vals = {"Q": oracle.synth(400, NH * S * 64, dtype=ir.BF16).reshape(NH, S, 64),
            "K": oracle.synth(401, NKV * S * 64, dtype=ir.BF16).reshape(NKV, S, 64),
            "V": oracle.synth(402, NKV * S * 64, dtype=ir.BF16).reshape(NKV, S, 64)}
    got, exe = run_on_gpu(dev, prog, vals)
    assert exe.stage_kernel(2).startswith("skeleton:flash_prefill")
    assert max_rel_err(got["O"], oracle.run_program(prog, vals)["O"]) < 2e-2


def test_tune_decode_attention_end_to_end(dev):
    """One family (the attention stage, seven variants): every candidate timed next to a fresh
    baseline, the shipped choice (if any) beats the analytic program, and it is exact."""
    prog = configs.decode_attention()
    rep = tune.tune(dev, prog, steps=4, rounds=2)
    print(rep)
    assert [t[1] for t in rep.trials] == [1, 2, 3, 4, 5, 6]
    assert rep.baseline_s > 0 and rep.tuned_s > 0
    if rep.shipped:
        assert rep.tuned_s < rep.baseline_s and set(rep.variants) == {0}
    else:
        assert rep.variants == {}
    err, _ = _c3(dev, prog.with_variants(rep.variants), 1000)
    assert err < 2e-2


@pytest.mark.parametrize("variant", range(3))
def test_paired_gemv_variants(dev, variant):
    """The paired gate/up GEMV with the SwiGLU product (rows per workgroup {2, 1, 4}) against
    the oracle's RMSNorm projections."""
    from sanic_amd import carrier as C
    from sanic_amd.program import STREAM, Program
    H, F = 2048, 2048
    p = Program()
    x = p.input("x", (H,), ir.F32)
    g = p.input("g", (H,), ir.BF16)
    ws = {nm: p.input(f"W{nm}", (F, H), ir.BF16) for nm in ("gate", "up")}
    gu = {nm: p.fused(nm, (F,), H, [(x, (STREAM,)), (g, (STREAM,)), (ws[nm], (0, STREAM))],
                      C.norm_fused_projection(H, 1e-5), ir.F32, role=3) for nm in ("gate", "up")}
    p.pointwise("h", ir.map_(ir.MUL, ir.silu(gu["gate"]), gu["up"]), ir.F32)
    counts = p.stage_variants(-1)
    assert counts[0] == 3
    prog = p.with_variants({0: variant})
    xv = _bf16_vals(301, H)
    gv = _bf16_vals(302, H, 1.0, 0.02)
    wg = oracle.synth_bf16(303, F * H, "normal", 0.0, 0.02).reshape(F, H)
    wu = oracle.synth_bf16(304, F * H, "normal", 0.0, 0.02).reshape(F, H)
    got, exe = run_on_gpu(dev, prog, {"x": xv, "g": gv, "Wgate": from_bf16_bits(wg).astype(np.float64),
                                       "Wup": from_bf16_bits(wu).astype(np.float64)})
    assert exe.stage_kernel(0).startswith("skeleton:gemv[batched 2]+paired"), exe.stage_kernel(0)
    want = oracle.run_program(prog, {"x": xv, "g": gv, "Wgate": from_bf16_bits(wg).astype(np.float64),
                                     "Wup": from_bf16_bits(wu).astype(np.float64)})["h"]
    assert max_rel_err(got["h"], want) < 1e-3
