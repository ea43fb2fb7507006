"""Hand-written skeletons on the GPU against the oracle, at the configurations' full sizes."""
import numpy as np
import pytest

import oracle
from sanic_amd import configs, ir
from sanic_amd.backend import from_bf16_bits
from tests.util import max_rel_err, run_on_gpu

pytestmark = pytest.mark.gpu


def bf16_rel(got, want) -> float:
    """bf16-storage metric of the reference: |g − e| / max(|e|, 1e-3) (tests/metal.rs:2098-2110)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-3)))


def _bf16_vals(seed, n, mean=0.0, std=1.0, kind="normal"):
    return oracle.synth(seed, n, kind, mean, std, dtype=ir.BF16)


@pytest.mark.parametrize("M", [1, 4])
def test_b1_rmsnorm_gemv_rows_layout(dev, M):
    """Config B1 with the reference's [out, in] weight layout: gemv skeleton, bf16 ≤ 2e-2."""
    K, N = 2048, 8192
    prog = configs.rmsnorm_projection(M=M, K=K, N=N, kmajor=False)
    x = _bf16_vals(101, M * K).reshape(M, K)
    g = _bf16_vals(102, K, 1.0, 0.02)
    wbits = oracle.synth_bf16(103, N * K, "normal", 0.0, 0.02).reshape(N, K)
    w = from_bf16_bits(wbits).astype(np.float64)
    got, exe = run_on_gpu(dev, prog, {"x": x, "g": g, "W": w})
    want = oracle.rmsnorm_proj(x, g, np.ascontiguousarray(wbits.T), 1e-5)
    print(exe.stage_kernel(0), bf16_rel(got["y"], want))
    if M == 1:
        assert exe.stage_kernel(0).startswith("skeleton:gemv")
    assert bf16_rel(got["y"], want) < 2e-2


@pytest.mark.parametrize("variant", [0, 1, 2, 3])
@pytest.mark.parametrize("K,N", [(2048, 8192), (256, 1024), (640, 1024)])
def test_b1_rmsnorm_gemv_kmajor(dev, K, N, variant):
    """Config B1 as configured: W bf16 [K, N] (K-major), the N-contiguous gemv skeleton in every
    strip form (0: 128 columns × 4 K slices meeting in scratch; 1: 32-column whole-K strips;
    2: 64 × 2; 3: 256 × 8)."""
    prog = configs.rmsnorm_projection(M=1, K=K, N=N, kmajor=True).with_variants({0: variant})
    x = _bf16_vals(111, K).reshape(1, K)
    g = _bf16_vals(112, K, 1.0, 0.02)
    wbits = oracle.synth_bf16(113, K * N, "normal", 0.0, 0.02).reshape(K, N)
    w = from_bf16_bits(wbits).astype(np.float64)
    got, exe = run_on_gpu(dev, prog, {"x": x, "g": g, "W": w})
    want = oracle.rmsnorm_proj(x, g, wbits, 1e-5)
    print(exe.stage_kernel(0), bf16_rel(got["y"], want))
    assert exe.stage_kernel(0).startswith("skeleton:gemv_kmajor")
    assert bf16_rel(got["y"], want) < 2e-2


def test_d1_int4_gemv(dev):
    """Config D1: packed uint4 [8192, 2048], group 64, s ~ U(0.001, 0.02), z = 8·s."""
    M, K, N, G = 1, 2048, 8192, 64
    prog = configs.int4_matmul(M=M, K=K, N=N, G=G)
    rng = np.random.default_rng(7)
    u = rng.integers(0, 16, size=(N, K))
    s = _bf16_vals(201, N * K // G, 0.001, 0.02, kind="uniform").reshape(N, K // G)
    z = np.array([oracle.round_bf16(8.0 * v) for v in s.reshape(-1)]).reshape(s.shape)
    x = _bf16_vals(202, M * K).reshape(M, K)
    got, exe = run_on_gpu(dev, prog, {"x": x, "Wq": u.reshape(N, K // G, G), "S": s, "Z": z})
    packed = (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8)
    want = oracle.int4_matmul(x, packed, s, z, G)
    print(exe.stage_kernel(0), bf16_rel(got["y"], want))
    assert exe.stage_kernel(0).startswith("skeleton:gemv")
    assert bf16_rel(got["y"], want) < 2e-2


@pytest.mark.parametrize("pos", [4095, 1000, 0, 63, 64])
def test_c3_decode_attention_split(dev, pos):
    """Config C3: 32 query heads / 8 KV heads, 4096-entry cache, split-K combine."""
    NH, NKV, HD, CAP = 32, 8, 64, 4096
    prog = configs.decode_attention(NH, NKV, HD, CAP)
    q = _bf16_vals(301, NH * HD).reshape(NH, HD)
    kc = _bf16_vals(302, NKV * CAP * HD).reshape(NKV, CAP, HD)
    vc = _bf16_vals(303, NKV * HD * CAP).reshape(NKV, HD, CAP)
    got, exe = run_on_gpu(dev, prog, {"q": q, "k_cache": kc, "v_cache": vc, "position": np.array(float(pos))})
    invf = oracle.inv_freq(500000.0, HD // 2)
    qr = oracle.rope(q[:, None, :], pos, invf)
    want = oracle.attention(qr, kc, vc, 1.0 / 8.0, mask=3, q_pos0=pos, v_transposed=True)[:, 0, :]
    print(exe.stage_kernel(0), pos, bf16_rel(got["o"], want))
    assert exe.stage_kernel(0).startswith("skeleton:attn_decode")
    assert bf16_rel(got["o"], want) < 2e-2


def test_device_specs_carry_the_cost_model_fields(dev):
    """Backend::specs (compile.rs:87-108) → DeviceSpecs (cost.rs:33-60): the MI355X figures
    the reference's cost model reads, plus the hardware facts from the runtime."""
    s = dev.specs()
    assert s.compute_units == 256 and s.wave_size == 64
    assert s.hbm_bytes > 250 * 2 ** 30
    assert s.hbm_bytes_per_s == 8.0e12 and s.bf16_mfma_flops == 2.5e15
    assert s.sram_bytes == 160 * 1024 and s.regfile_bytes == 512 * 1024
    assert s.launch_overhead_s == 2.6e-6 and s.min_blocks == 2 * s.compute_units
    # Little's law at these figures: the decode GEMV's 33.5 MB in flight saturates HBM
    assert 33.5e6 / (s.hbm_bytes_per_s * s.mem_latency_s) >= 1.0


@pytest.mark.parametrize("index", [0.0, 299.0, 150.5, 7.4])
def test_gemv_reads_its_activation_through_a_gather(dev, index):
    """The GEMV's activation leaf a gathered row (the decode step's layer 0 reading embed[token]
    with no stage of its own): the index rounded half away from zero, as the interpreter's
    gather (interp.rs, llround); norm-fused, against the oracle running the same program."""
    from sanic_amd import carrier as C
    from sanic_amd.program import STREAM, Program
    V, K, N = 300, 2048, 512
    p = Program()
    emb = p.input("E", (V, K), ir.BF16)
    idx = p.input("idx", (1,), ir.F32)
    g = p.input("g", (K,), ir.BF16)
    w = p.input("W", (N, K), ir.BF16)
    x = ir.reindex(ir.gather(emb, idx, 0), (K,), [((), 0), (((1, 0),), 0)])
    p.fused("y", (N,), K, [(x, (STREAM,)), (g, (STREAM,)), (w, (0, STREAM))], C.norm_fused_projection(K, 1e-5), ir.F32)
    vals = {"E": _bf16_vals(131, V * K).reshape(V, K), "idx": np.array([index]),
            "g": _bf16_vals(132, K, 1.0, 0.02), "W": _bf16_vals(133, N * K, 0.0, 0.02).reshape(N, K)}
    got, exe = run_on_gpu(dev, p, vals)
    want = oracle.run_program(p, vals)["y"]
    err = float(np.max(np.abs(got["y"] - want) / (1 + np.abs(want))))
    print(exe.stage_kernel(0), index, err)
    assert exe.stage_kernel(0).startswith("skeleton:gemv")
    assert err < 1e-4
