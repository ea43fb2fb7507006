"""Exact invariants of the HIP path on the GPU, each against the oracle or against the HIP path
itself: bf16 storage bit for bit, decode attention == the prefill row, the flash edge-tile fast
path == the rendered mask, reserved-cache independence, every decode-attention tiling variant
inside the Llama step, Q8 ties, and replay stability of the cross-workgroup merges."""
import struct

import numpy as np
import pytest

import oracle
from sanic_amd import carrier as C
from sanic_amd import configs, ir
from sanic_amd.backend import from_bf16_bits, to_bf16_bits
from sanic_amd.llama import LlamaMachine
from sanic_amd.program import STREAM, Program, Sched
from tests.llama_ref import OracleModel, _upload, synth_weights
from tests.test_cpu_llama_oracle import TINY
from tests.util import max_rel_err, run_on_gpu

pytestmark = pytest.mark.gpu

# /root/reference/tests/metal.rs:2177-2196, plus two NaNs (a signalling payload and a negative
# quiet one) whose stored bf16 must come out quiet
BF16_VECTORS = [0.0, -0.0, 1.0, 1.0 + 1.0 / 512.0, 1.0 + 3.0 / 512.0, -1.0 - 1.0 / 512.0, 65504.0,
                3.4e38, -3.4e38, float("inf"), float("-inf"), 1e-40, np.pi, -np.e, 0.1, 123456789.0]
NAN_BITS = [0x7F800001, 0xFFC12345]


def test_bf16_store_and_round_to_bit_for_bit(dev):
    """tests/metal.rs:2170-2252: the interpreter's rounding twin, RoundTo(BF16) computed in a
    register (stored f32) and the value written through bf16 storage meet at the same bits —
    ties, ±inf, −0, an f32 subnormal, overflow — and a NaN keeps its sign and payload top and
    comes out quiet."""
    n = len(BF16_VECTORS) + len(NAN_BITS)
    f32 = np.array(BF16_VECTORS, np.float32).view(np.uint32)
    raw = np.concatenate([f32, np.array(NAN_BITS, np.uint32)])
    p = Program()
    x = p.input("X", (n,), ir.F32)
    p.pointwise("R", ir.round_to(x, ir.BF16), ir.F32)
    p.pointwise("S", x * 1.0, ir.BF16)
    exe = dev.prepare(p)
    xb = dev.alloc(4 * n)
    xb.upload_array(raw)
    outs = exe.execute({"X": xb})
    reg = np.frombuffer(outs["R"].download(), np.uint32)
    store = np.frombuffer(outs["S"].download(), np.uint16)
    for i, v in enumerate(BF16_VECTORS):
        want = np.array([oracle.round_bf16(float(np.float32(v)))], np.float32).view(np.uint32)[0]
        assert reg[i] == want, (v, hex(reg[i]), hex(want))
        assert (int(store[i]) << 16) == want, (v, hex(store[i]), hex(want))
    for j, bits in enumerate(NAN_BITS):
        i = len(BF16_VECTORS) + j
        want16 = int(to_bf16_bits(np.array([bits], np.uint32).view(np.float32))[0])
        assert want16 == ((bits >> 16) | 0x40)
        assert int(store[i]) == want16, (hex(bits), hex(store[i]))
        assert reg[i] == want16 << 16, (hex(bits), hex(reg[i]))


def test_q8_store_ties_round_half_to_even(dev):
    """The device's Q8 store rounds v/scale half to even (Metal's rint, emit_metal.rs:182-185):
    exact ties at scale 0.25 land on the even grid point, and ±127 clamps."""
    s = 0.25
    v = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, 126.5, 200.0, -200.0]) * s
    want_q = np.array([0, 2, 2, 0, -2, -2, 4, 126, 127, -127], np.int8)
    p = Program()
    x = p.input("X", (v.size,), ir.F32)
    p.pointwise("Y", x * 1.0, ir.q8(s))
    exe = dev.prepare(p)
    outs = exe.execute({"X": dev.from_values(v, ir.F32)})
    got_q = np.frombuffer(outs["Y"].download(), np.int8)
    np.testing.assert_array_equal(got_q, want_q)


@pytest.mark.parametrize("pos", [0, 1, 63, 64, 127, 128, 1000, 2047, 4095])
def test_decode_attention_equals_prefill_row(dev, pos):
    """tests/metal.rs:864-996 / tests/decode.rs:121-200 on the GPU: the decode attention kernel
    at position p over a cache equals row p of the flash-prefill kernel over the same K/V and
    the same (already rotated) query row — two different kernels, one value."""
    NH, NKV, S, HD = 32, 8, 4096, 64
    q = oracle.synth(610, NH * S * HD, dtype=ir.BF16).reshape(NH, S, HD)
    k = oracle.synth(611, NKV * S * HD, dtype=ir.BF16).reshape(NKV, S, HD)
    v = oracle.synth(612, NKV * S * HD, dtype=ir.BF16).reshape(NKV, S, HD)
    pre = _flash_cached(dev, q, k, v)
    dprog = configs.decode_attention(NH, NKV, HD, S, rope=False, out_dtype=ir.F32)
    got, exe = run_on_gpu(dev, dprog, {"q": q[:, pos, :], "k_cache": k, "v_cache": v.transpose(0, 2, 1),
                                       "position": np.array(float(pos))})
    assert exe.stage_kernel(0).startswith("skeleton:attn_decode"), exe.stage_kernel(0)
    row = pre[:, pos, :]
    err = max_rel_err(row, got["o"])
    print(pos, err)
    # the prefill row is stored bf16 and its PV product takes P in bf16: the bf16 bound
    assert err < 2e-2


_FLASH = {}


def _flash_cached(dev, q, k, v):
    key = (q.shape, k.shape)
    if key not in _FLASH:
        prog = configs.flash_prefill(q.shape[0], k.shape[0], q.shape[1], rope_stages=False)
        got, exe = run_on_gpu(dev, prog, {"Q": q, "K": k, "V": v})
        assert exe.stage_kernel(0).startswith("skeleton:flash_prefill")
        _FLASH.clear()
        _FLASH[key] = got["O"]
    return _FLASH[key]


@pytest.mark.parametrize("shape", [(32, 8, 4096, 0), (32, 8, 4096, 1024), (4, 2, 300, 0), (4, 2, 300, 100)])
def test_flash_edge_fast_path_bit_identical(dev, shape):
    """tests/metal.rs:1773-1833: the honest-window edge tiles scored with the unmasked form
    inside each row's window (the fast path) give the same bits as the rendered mask on every
    element (tiling variant 3 takes the rendered leaf on every edge tile)."""
    NH, NKV, S, W = shape
    vals = {"Q": oracle.synth(620, NH * S * 64, dtype=ir.BF16).reshape(NH, S, 64),
            "K": oracle.synth(621, NKV * S * 64, dtype=ir.BF16).reshape(NKV, S, 64),
            "V": oracle.synth(622, NKV * S * 64, dtype=ir.BF16).reshape(NKV, S, 64)}
    outs = []
    for variant in (0, 3):
        prog = configs.flash_prefill(NH, NKV, S, window=W, rope_stages=False).with_variants({0: variant})
        exe = dev.prepare(prog)
        bufs = {n: dev.from_values(a, ir.BF16) for n, a in vals.items()}
        outs.append(np.frombuffer(exe.execute(bufs)["O"].download(), np.uint16))
    assert np.array_equal(outs[0], outs[1]), int(np.sum(outs[0] != outs[1]))


def _tiny_machine(dev, shape, w, **kw):
    return LlamaMachine(dev, {n: _upload(dev, a) for n, a in w.items()}, shape, **kw)


def _tiny_shape(cap):
    S = TINY
    return configs.LlamaShape(layers=S.layers, hidden=S.hidden, heads=S.heads, kv_heads=S.kv_heads,
                              head_dim=S.head_dim, ffn=S.ffn, vocab=S.vocab, capacity=cap)


def test_reserved_cache_extent_does_not_change_logits(dev):
    """tests/reserved_cache.rs:577: the same prompt through caches of capacity 6, 9, 16 and 22
    gives the same logits — on the GPU bit for bit across capacities, each within 1e-4 of the
    oracle at every step."""
    w = synth_weights(TINY, seed=5)
    prompt = [7, 3, 21, 40, 11, 30]
    first = None
    for cap in (6, 9, 16, 22):
        shape = _tiny_shape(cap)
        m = _tiny_machine(dev, shape, w)
        om = OracleModel(shape, w)
        logits = []
        for pos, t in enumerate(prompt):
            m.step(t)
            tok, want = om.step(t, pos)
            assert m.last_token() == tok
            assert max_rel_err(m.last_logits(), want) < 1e-4, (cap, pos)
            logits.append(m.last_logits())
        if first is None:
            first = logits
        else:
            for a, b in zip(first, logits):
                assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), cap


def _cache_close(got_bits, want_bits):
    """Per element |g − e| / max(|e|, 1e-3) of two arrays of bf16 bits (the reference's bf16
    metric, tests/metal.rs:2098-2110) and the count of elements whose bits differ."""
    g = from_bf16_bits(got_bits).astype(np.float64)
    e = from_bf16_bits(want_bits).astype(np.float64)
    return np.abs(g - e) / np.maximum(np.abs(e), 1e-3), int(np.count_nonzero(got_bits != want_bits))


@pytest.mark.parametrize("variant", range(7))
def test_llama_step_every_attention_variant(dev, variant):
    """Every decode-attention tiling variant (threads × positions per chunk, incl. the row-writer
    workgroup at chunk index NCH) inside the tiny Llama step, over a 300-position cache and past
    several chunk boundaries (64, 128, 256): greedy ids identical, logits within 1e-4, and the
    cache rows the kernel writes within one bf16 rounding step of the oracle's (2^-7 relative,
    floor 1e-3): an f32 evaluation rounds differently from the f64 oracle for an element within
    ~1e-7 of a rounding boundary, so a few cache bits differ; at most 1% of them may."""
    shape = _tiny_shape(300)
    w = synth_weights(shape, seed=9)
    prog = configs.llama_decode(shape)
    attn = [i for i, s in enumerate(prog.stages) if s.name.endswith("attn")]
    m = _tiny_machine(dev, shape, w, variants={i: variant for i in attn})
    om = OracleModel(shape, w)
    rng = np.random.default_rng(variant)
    prompt = rng.integers(0, shape.vocab, 270).tolist()
    tok = None
    for pos in range(275):
        feed = prompt[pos] if pos < len(prompt) else tok
        m.step(feed)
        tok, want = om.step(feed, pos)
        assert m.last_token() == tok, (variant, pos)
        err = max_rel_err(m.last_logits(), want)
        assert err < 1e-4, (variant, pos, err)
    total = off = 0
    for l in range(shape.layers):
        for which, ref in (("key", om.kc[l]), ("value", om.vc[l])):
            rel, n_off = _cache_close(m.cache(l, which), ref)
            assert rel.max() <= 2.0 ** -7, (l, which, float(rel.max()))
            total += rel.size
            off += n_off
    print("variant", variant, "cache elements whose bits differ:", off, "of", total)
    assert off <= total // 100


# ── replay stability of the cross-workgroup merges ──────────────────────────

def _soak(dev, prog, vals, out, n=5000):
    exe = dev.prepare(prog)
    bufs = {k: dev.from_values(v, prog.by_name[k].dtype) for k, v in vals.items()}
    rp = exe.capture(bufs)
    ob = rp.buffer(out)
    rp.step()
    first = ob.download()
    for i in range(n - 1):
        rp.step()
        assert ob.download() == first, f"replay {i + 2} differs from the first"
    return exe


def test_soak_argmax_split(dev):
    """The split argmax (64 workgroups + last-workgroup butterfly merge) over 128256 values with
    planted ties: 5000 replays give the first replay's index every time."""
    V = 128256
    p = Program()
    x = p.input("x", (V,), ir.F32)
    p.fused("token", (1,), V, [(x, (STREAM,)), (ir.iota(V), (STREAM,))], C.first_argmax(), ir.U32,
            sched=Sched(lane_stream=True, waves=4, chunk=4, split=64))
    xv = oracle.lcg(901, V)
    xv[[5000, 70000, 128000]] = 2.0          # a three-way tie for the max: the first index wins
    exe = _soak(dev, p, {"x": xv}, "token")
    assert exe.stage_kernel(0).startswith("fold:split"), exe.stage_kernel(0)


def test_soak_decode_attention(dev):
    """Decode attention's n-way merge in the last workgroup of each KV group: 5000 replays."""
    NH, NKV, HD, CAP = 32, 8, 64, 4096
    vals = {"q": oracle.synth(911, NH * HD, dtype=ir.BF16).reshape(NH, HD),
            "k_cache": oracle.synth(912, NKV * CAP * HD, dtype=ir.BF16).reshape(NKV, CAP, HD),
            "v_cache": oracle.synth(913, NKV * HD * CAP, dtype=ir.BF16).reshape(NKV, HD, CAP),
            "position": np.array(3000.0)}
    exe = _soak(dev, configs.decode_attention(out_dtype=ir.F32), vals, "o")
    assert exe.stage_kernel(0).startswith("skeleton:attn_decode")


def test_soak_kslice_gemv(dev):
    """The K-major GEMV in its K-slice form (K = 16384: the slices' partials meet in scratch
    and the last workgroup of each column group adds them): 5000 replays."""
    K, N = 16384, 512
    prog = configs.rmsnorm_projection(M=1, K=K, N=N, kmajor=True)
    wbits = oracle.synth_bf16(923, K * N, "normal", 0.0, 0.02)
    vals = {"x": oracle.synth(921, K, dtype=ir.BF16).reshape(1, K),
            "g": oracle.synth(922, K, "normal", 1.0, 0.02, dtype=ir.BF16),
            "W": from_bf16_bits(wbits).astype(np.float64).reshape(K, N)}
    exe = _soak(dev, prog, vals, "y")
    assert exe.stage_kernel(0).startswith("skeleton:gemv_kmajor["), exe.stage_kernel(0)


def test_soak_sliced_strip_gemv(dev):
    """The K-major GEMV's 128-column strips over four K slices (the last workgroup of each strip
    adds the slices in slice order): 5000 replays, bit-identical."""
    K, N = 2048, 8192
    prog = configs.rmsnorm_projection(M=1, K=K, N=N, kmajor=True)
    wbits = oracle.synth_bf16(943, K * N, "normal", 0.0, 0.02)
    vals = {"x": oracle.synth(941, K, dtype=ir.BF16).reshape(1, K),
            "g": oracle.synth(942, K, "normal", 1.0, 0.02, dtype=ir.BF16),
            "W": from_bf16_bits(wbits).astype(np.float64).reshape(K, N)}
    exe = _soak(dev, prog, vals, "y")
    assert "x4 slices" in exe.stage_kernel(0), exe.stage_kernel(0)


def test_xcd_local_merge_matches_device_coherent(dev, monkeypatch):
    """The K-major GEMV's slices meet through one XCD's L2 (the runtime found round-robin XCD
    placement at device open) or through device-coherent memory (SANIC_HIP_AGENT_MERGE): the
    same additions in the same order, so bit-identical outputs."""
    K, N = 2048, 8192
    wbits = oracle.synth_bf16(953, K * N, "normal", 0.0, 0.02)
    vals = {"x": oracle.synth(951, K, dtype=ir.BF16).reshape(1, K),
            "g": oracle.synth(952, K, "normal", 1.0, 0.02, dtype=ir.BF16),
            "W": from_bf16_bits(wbits).astype(np.float64).reshape(K, N)}
    got = {}
    for mode in ("xcd", "agent"):
        if mode == "agent":
            monkeypatch.setenv("SANIC_HIP_AGENT_MERGE", "1")
        prog = configs.rmsnorm_projection(M=1, K=K, N=N, kmajor=True)
        out, exe = run_on_gpu(dev, prog, vals)
        kind = exe.stage_kernel(0)
        print(mode, kind, flush=True)
        assert kind.endswith("+xcd") == (mode == "xcd"), kind
        got[mode] = out["y"]
    assert np.array_equal(got["xcd"], got["agent"])


def test_soak_flash_split_variant(dev):
    """The flash split variant (two workgroups per block exchange (m, ℓ, o) partials, the later
    one combines in a fixed operand order): 5000 replays, bit-identical."""
    NH, NKV, S = 4, 2, 512
    vals = {"Q": oracle.synth(930, NH * S * 64, dtype=ir.BF16).reshape(NH, S, 64),
            "K": oracle.synth(931, NKV * S * 64, dtype=ir.BF16).reshape(NKV, S, 64),
            "V": oracle.synth(932, NKV * S * 64, dtype=ir.BF16).reshape(NKV, S, 64)}
    prog = configs.flash_prefill(NH, NKV, S, rope_stages=False).with_variants({0: 2})
    exe = _soak(dev, prog, vals, "O")
    assert "+split2" in exe.stage_kernel(0), exe.stage_kernel(0)
