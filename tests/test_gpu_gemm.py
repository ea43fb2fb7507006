"""MFMA GEMM skeleton (configs B2 and D2, plus small ragged shapes) against the oracle."""
import numpy as np
import pytest

import oracle
from sanic_amd import configs, ir
from sanic_amd.backend import from_bf16_bits
from tests.test_gpu_skeletons import bf16_rel, _bf16_vals
from tests.util import run_on_gpu

pytestmark = pytest.mark.gpu


def _report(exe, got, want):
    got = np.asarray(got, np.float64).reshape(want.shape)
    rel = np.abs(got - want) / np.maximum(np.abs(want), 1e-3)
    bad = np.argwhere(rel > 2e-2)
    print(exe.stage_kernel(0), float(rel.max()), "bad", len(bad), bad[:8].tolist(), flush=True)


@pytest.mark.parametrize("variant", [0, 1])
@pytest.mark.parametrize("M,K,N,kmajor", [
    (512, 2048, 8192, True),      # config B2, W [K, N]
    (512, 2048, 8192, False),     # same with the reference's [out, in] layout
    (64, 256, 96, True),
    (192, 128, 160, False),
    (64, 512, 512, True),         # x·g built by the first launch (K % 512 == 0)
    (128, 256, 16384, True),      # 8-wave 128 × 64 tiles, x·g built in-kernel (K % 512 != 0)
    (256, 384, 8192, False),      # 8-wave tiles, [out, in] weights, in-kernel row slots
    (128, 1536, 2048, True),      # operand-building launch with 3 k chunks over 4 waves
])
def test_rmsnorm_gemm(dev, M, K, N, kmajor, variant):
    prog = configs.rmsnorm_projection(M=M, K=K, N=N, kmajor=kmajor).with_variants({0: variant})
    x = _bf16_vals(301, M * K).reshape(M, K)
    g = _bf16_vals(302, K, 1.0, 0.02)
    wbits = oracle.synth_bf16(303, N * K, "normal", 0.0, 0.02)
    wkn = wbits.reshape(K, N) if kmajor else np.ascontiguousarray(wbits.reshape(N, K).T)
    w = from_bf16_bits(wbits).astype(np.float64).reshape((K, N) if kmajor else (N, K))
    got, exe = run_on_gpu(dev, prog, {"x": x, "g": g, "W": w})
    want = oracle.rmsnorm_proj(x, g, np.ascontiguousarray(wkn), 1e-5)
    err = bf16_rel(got["y"], want)
    _report(exe, got["y"], want)
    assert exe.stage_kernel(0).startswith("skeleton:gemm")
    assert err < 2e-2


@pytest.mark.parametrize("M,K,N,kmajor", [(512, 2048, 8192, True), (64, 512, 512, False), (128, 1536, 2048, True)])
def test_rmsnorm_gemm_fragment_order_a(dev, M, K, N, kmajor, monkeypatch):
    """The first launch's x·g planes in MFMA fragment order (each wave loading its A fragments
    directly, 8 × 1 waves) against the row-major planes staged through LDS
    (SANIC_HIP_GEMM_ALDS): both within the bf16 bound of the oracle, and within one output
    rounding of each other (the row slots are summed per K slice in the first form)."""
    x = _bf16_vals(311, M * K).reshape(M, K)
    g = _bf16_vals(312, K, 1.0, 0.02)
    wbits = oracle.synth_bf16(313, N * K, "normal", 0.0, 0.02)
    wkn = wbits.reshape(K, N) if kmajor else np.ascontiguousarray(wbits.reshape(N, K).T)
    w = from_bf16_bits(wbits).astype(np.float64).reshape((K, N) if kmajor else (N, K))
    want = oracle.rmsnorm_proj(x, g, np.ascontiguousarray(wkn), 1e-5)
    outs = {}
    for form in ("fragment", "lds"):
        if form == "lds":
            monkeypatch.setenv("SANIC_HIP_GEMM_ALDS", "1")
        prog = configs.rmsnorm_projection(M=M, K=K, N=N, kmajor=kmajor)
        got, exe = run_on_gpu(dev, prog, {"x": x, "g": g, "W": w})
        kind = exe.stage_kernel(0)
        assert kind.startswith("skeleton:gemm") and ",pre" in kind, kind
        assert (",ad" in kind) == (form == "fragment"), kind
        assert bf16_rel(got["y"], want) < 2e-2
        outs[form] = np.asarray(got["y"], np.float64).reshape(want.shape)
    a, b = outs["fragment"], outs["lds"]
    assert np.max(np.abs(a - b) / np.maximum(np.abs(b), 1e-3)) <= 2.0 ** -7


@pytest.mark.parametrize("M,K,N,G,zk,variant", [
    (128, 2048, 8192, 64, "8s", 0),      # config D2: grouped tiles (q on the MFMA, s/z folded per tile)
    (128, 2048, 8192, 64, "8s", 1),      # the other load depth
    (64, 512, 256, 32, "8s", 0),         # groups narrower than a K tile: hi + lo dequantized B
    (256, 512, 8192, 64, "8s", 0),
    (128, 1024, 512, 128, "any", 0),     # groups of two K tiles, zero points unrelated to s
    (64, 512, 256, 64, "any", 1),
    (128, 2048, 8192, 64, "any", 2),
])
def test_int4_gemm(dev, M, K, N, G, zk, variant):
    """Config D2: packed uint4 [N, K], per-group scale and zero point, w = u·s − z."""
    prog = configs.int4_matmul(M=M, K=K, N=N, G=G).with_variants({0: variant})
    rng = np.random.default_rng(11)
    u = rng.integers(0, 16, size=(N, K))
    s = _bf16_vals(401, N * K // G, 0.001, 0.02, kind="uniform").reshape(N, K // G)
    if zk == "8s":
        z = np.array([oracle.round_bf16(8.0 * v) for v in s.reshape(-1)]).reshape(s.shape)
    else:
        z = _bf16_vals(403, N * K // G, -0.1, 0.1, kind="uniform").reshape(s.shape)
    x = _bf16_vals(402, M * K).reshape(M, K)
    got, exe = run_on_gpu(dev, prog, {"x": x, "Wq": u.reshape(N, K // G, G), "S": s, "Z": z})
    packed = (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8)
    want = oracle.int4_matmul(x, packed, s, z, G)
    err = bf16_rel(got["y"], want)
    _report(exe, got["y"], want)
    assert exe.stage_kernel(0).startswith("skeleton:gemm")
    assert ("grp" in exe.stage_kernel(0)) == (G % 64 == 0)
    assert err < 2e-2
