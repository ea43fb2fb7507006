"""The CPU oracle pinned against the reference's own known answers, laws and closed forms.

Every check here compares the C restatement (oracle/) with something it did not compute
itself: a golden vector from the reference's tests, a textbook closed form, an independent
pure-Python evaluation, or an invariant the mathematics fixes.
"""
import math
import struct

import numpy as np
import pytest

import oracle
from sanic_amd import carrier as C
from sanic_amd import configs, ir
from sanic_amd.program import STREAM, Program, Sched


# ── generators and scalar semantics ─────────────────────────────────────────

def _xorshift_py(seed, n):
    """xorshift64* of /root/reference/tests/metal.rs:86-96, in plain Python integers."""
    x, out = seed, []
    for _ in range(n):
        x ^= x >> 12
        x ^= (x << 25) & 0xFFFFFFFFFFFFFFFF
        x ^= x >> 27
        u = (x * 0x2545F4914F6CDD1D) & 0xFFFFFFFFFFFFFFFF
        out.append(((u >> 11) / float(1 << 53)) * 2.0 - 1.0)
    return out


def test_lcg_matches_reference_xorshift_stream():
    for seed in (1, 0x144A16, 0xBF16, 12345678901234):
        assert oracle.lcg(seed, 64).tolist() == _xorshift_py(seed, 64)


def test_synth_normal_moments():
    v = oracle.synth(7, 200_000, "normal", 0.0, 1.0, dtype=ir.F64)
    assert abs(v.mean()) < 0.01 and abs(v.std() - 1.0) < 0.01
    u = oracle.synth(8, 100_000, "uniform", 0.001, 0.02, dtype=ir.F64)
    assert u.min() >= 0.001 and u.max() <= 0.02 and abs(u.mean() - 0.0105) < 1e-4


BF16_VECTORS = [0.0, -0.0, 1.0, 1.0 + 1.0 / 512.0, 1.0 + 3.0 / 512.0, -1.0 - 1.0 / 512.0, 65504.0,
                3.4e38, -3.4e38, math.inf, -math.inf, 1e-40, math.pi, -math.e, 0.1, 123456789.0]


def _bf16_ref(v):
    """RNE on the high half of the f32 bit pattern, computed with struct (no oracle code)."""
    b = struct.unpack("<I", struct.pack("<f", v))[0]
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) & 0xFFFF
    return struct.unpack("<f", struct.pack("<I", r << 16))[0]


def test_round_bf16_golden_vectors():
    """The bf16 store vectors of /root/reference/tests/metal.rs:2177-2252."""
    for v in BF16_VECTORS:
        got = oracle.round_bf16(v)
        assert struct.pack("<d", got) == struct.pack("<d", _bf16_ref(v)), v
    # the closed forms the vectors were chosen for
    assert oracle.round_bf16(1.0 + 1.0 / 512.0) == 1.0           # a quarter ulp: down
    assert oracle.round_bf16(1.0 + 3.0 / 512.0) == 1.0 + 1.0 / 128  # three quarters: up (ulp 2^-7)
    assert oracle.round_bf16(1.0 + 1.0 / 256.0) == 1.0           # exact tie: to even
    assert oracle.round_bf16(1.0 + 3.0 / 256.0) == 1.0 + 1.0 / 64  # exact tie: to even (up)
    assert oracle.round_bf16(3.4e38) == math.inf
    assert math.copysign(1.0, oracle.round_bf16(-0.0)) == -1.0
    assert math.isnan(oracle.round_bf16(math.nan))


# ── the interpreter on the reference's known answers ────────────────────────

def test_direct_attention_known_answer():
    """q = k = I, v = [[2,3],[5,7]], scale 1/√2 → (tests/compile.rs:230-263)."""
    p = configs.direct_attention(S=2, D=2, causal=False)
    vals = {"Q": np.eye(2), "K": np.eye(2), "V": np.array([[2.0, 3.0], [5.0, 7.0]])}
    out = oracle.run_program(p, vals)["O"].reshape(-1)
    np.testing.assert_allclose(out, [2.990715, 4.3209534, 4.009285, 5.6790466], rtol=1e-6)
    # closed form: p = softmax([1, 0]/√2)
    a = math.exp(1 / math.sqrt(2))
    p0 = a / (a + 1)
    np.testing.assert_allclose(out[0], p0 * 2 + (1 - p0) * 5, rtol=1e-6)
    graph = ir.attention(p.node("Q"), p.node("K"), p.node("V"))
    # the stage output is stored f32; the graph evaluates in f64
    np.testing.assert_allclose(oracle.eval_node(p, graph, vals).reshape(-1), out, rtol=1e-7)


def test_reduce_rows_known_answer():
    """reduce rows [[1,2],[3,4]] → [3, 7] (lib.rs:10-22)."""
    p = Program()
    x = p.input("X", (2, 2))
    p.fused("Y", (2,), 2, [(x, (0, STREAM))], C.plain(ir.M_ADD))
    assert oracle.run_program(p, {"X": np.array([[1.0, 2.0], [3.0, 4.0]])})["Y"].tolist() == [3.0, 7.0]


def test_eval_matches_numpy_on_matmul_softmax_rmsnorm():
    p = Program()
    a = p.input("A", (5, 7))
    b = p.input("B", (7, 3))
    g = p.input("G", (7,))
    vals = {"A": oracle.lcg(1, 35).reshape(5, 7), "B": oracle.lcg(2, 21).reshape(7, 3), "G": oracle.lcg(3, 7)}
    np.testing.assert_allclose(oracle.eval_node(p, ir.matmul(a, b), vals), vals["A"] @ vals["B"], rtol=1e-13)
    sm = oracle.eval_node(p, ir.softmax(a, -1), vals)
    e = np.exp(vals["A"] - vals["A"].max(-1, keepdims=True))
    np.testing.assert_allclose(sm, e / e.sum(-1, keepdims=True), rtol=1e-13)
    rn = oracle.eval_node(p, ir.rms_norm(a, g, 1e-5), vals)
    x = vals["A"]
    np.testing.assert_allclose(rn, x * vals["G"] / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-5), rtol=1e-13)


def test_causal_attention_interpreter_equals_fused_loop_and_carrier():
    """Config A three ways: interp eval of the graph, the carrier fold (run_carrier_split with
    awkward block counts, tests/group.rs:48-116) and the fused f64 loop."""
    p = configs.direct_attention()
    vals = {n: oracle.lcg(s, 128 * 64).reshape(128, 64) for n, s in (("Q", 1), ("K", 2), ("V", 3))}
    graph = ir.attention(p.node("Q"), p.node("K"), p.node("V"), causal=True)
    want = oracle.eval_node(p, graph, vals)
    fused = oracle.attention(vals["Q"][None], vals["K"][None], vals["V"][None], 1 / 8, mask=1)[0]
    np.testing.assert_allclose(fused, want, rtol=1e-12, atol=1e-13)
    for blocks in (1, 2, 3, 7, 9, 128):
        got, _ = oracle.fold_stage(p, 0, vals, blocks)
        np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-13)


# ── carrier laws (tests/laws.rs) ─────────────────────────────────────────────

def test_flash_carrier_render_strings():
    """tests/laws.rs:108-126."""
    r = C.online_softmax_weighted().render()
    assert "into:    s0 = x0;  s1 = 1;  s2 = x1" in r
    assert ("s1 = a1·where(-∞ < a0, exp(a0 - max(a0, b0)), 0) + b1·where(-∞ < b0, exp(b0 - max(a0, b0)), 0)") in r
    assert ("s2 = a2·where(-∞ < a0, exp(a0 - max(a0, b0)), 0) + b2·where(-∞ < b0, exp(b0 - max(a0, b0)), 0)") in r
    assert "project: s2 / s1" in r


def _laws_lcg(seed):
    """tests/laws.rs Lcg: xorshift64* scaled to [-3, 3)."""
    x = max(seed, 1)
    while True:
        x ^= x >> 12
        x ^= (x << 25) & 0xFFFFFFFFFFFFFFFF
        x ^= x >> 27
        u = (x * 0x2545F4914F6CDD1D) & 0xFFFFFFFFFFFFFFFF
        yield ((u >> 11) / float(1 << 53)) * 6.0 - 3.0


def test_norm_fused_carrier_closed_form():
    """tests/laws.rs:621-646: Σ x·g·w / √(Σx²/n + ε), fold == tree_fold == closed form."""
    car = C.norm_fused_projection(16, 1e-5)
    assert car.slots == 2 and "defer-div" in car.rules
    g = _laws_lcg(1234)
    items = [[next(g), next(g), next(g)] for _ in range(16)]
    dot = sum(a * b * c for a, b, c in items)
    ssq = sum(a * a for a, _, _ in items)
    ref = dot / math.sqrt(ssq / 16 + 1e-5)
    assert abs(car.fold(items) - ref) <= 1e-12 * abs(ref)
    assert abs(car.tree_fold(items) - ref) <= 1e-12 * abs(ref)


def _planted_scores(center, n, max_pos, seed):
    g = _laws_lcg(seed)
    s = [center + next(g) for _ in range(n)]
    s[max_pos] = center + 5.0
    return s


@pytest.mark.parametrize("center", [50.0, 88.0, 300.0, 710.0, -710.0])
def test_attention_rescale_survives_overflow_magnitudes(center):
    """tests/laws.rs:445-475: the carrier matches the stable two-pass reference where the naive
    unshifted fold overflows f64."""
    car = C.online_softmax_weighted()
    n = 23
    for max_pos in (0, n - 1):
        scores = _planted_scores(center, n, max_pos, 42)
        g = _laws_lcg(7)
        items = [[s, next(g)] for s in scores]
        mx = max(scores)
        ref = sum(math.exp(a - mx) * b for a, b in items) / sum(math.exp(s - mx) for s in scores)
        assert abs(car.fold(items) - ref) <= 1e-9 * (1 + abs(ref))
        assert abs(car.tree_fold(items) - ref) <= 1e-9 * (1 + abs(ref))
        if center >= 710.0:
            with pytest.raises(OverflowError):
                sum(math.exp(a) * b for a, b in items)


def test_minus_infinity_identity_partial_survives():
    """A partial that folded only masked (−∞) scores is the identity (m = −∞, ℓ = 0): merging it
    on either side leaves the other untouched — no exp(−∞ − −∞) = NaN (derive.rs:1700-1713)."""
    car = C.online_softmax_weighted()
    masked = [[-math.inf, 3.0], [-math.inf, -2.0]]
    live = [[0.5, 1.0], [1.5, -1.0], [-0.25, 2.0]]
    a = list(car.identity)
    for it in masked:
        a = car.merge(a, car.lift(it))
    assert a[0] == -math.inf and a[1] == 0.0 and a[2] == 0.0
    b = list(car.identity)
    for it in live:
        b = car.merge(b, car.lift(it))
    assert car.merge(a, b) == b and car.merge(b, a) == b
    assert not math.isnan(car.proj(car.merge(a, b)))


def test_argmax_carrier_first_index_on_ties():
    car = C.first_argmax()
    vals = [0.3, 2.0, -1.0, 2.0, 1.0]
    items = [[v, float(i)] for i, v in enumerate(vals)]
    assert car.fold(items) == 1.0 and car.tree_fold(items) == 1.0
    assert car.fold(list(reversed([[v, float(i)] for i, v in enumerate(vals)]))) == 1.0


def test_split_fold_equals_one_pass_on_causal_with_identity_partials():
    """tests/group.rs:86-116: causal rows whose early chunks are fully masked."""
    p = configs.direct_attention(S=16, D=8)
    vals = {n: oracle.lcg(s, 16 * 8).reshape(16, 8) for n, s in (("Q", 5), ("K", 6), ("V", 7))}
    one, _ = oracle.fold_stage(p, 0, vals, 1)
    for blocks in (2, 3, 5, 16):
        got, _ = oracle.fold_stage(p, 0, vals, blocks)
        np.testing.assert_allclose(got, one, rtol=1e-12, atol=1e-14)


# ── hot-path graphs: closed forms ────────────────────────────────────────────

def test_rope_is_a_rotation_of_each_pair():
    """rotate-half RoPE = a 2-D rotation of (x_f, x_{f+F}) by pos·inv_freq[f]; norms kept."""
    x = oracle.lcg(11, 3 * 4 * 64).reshape(3, 4, 64)
    invf = oracle.inv_freq(500000.0, 32)
    r = oracle.rope(x, 17, invf)
    for h in range(3):
        for s in range(4):
            for f in range(32):
                th = (17 + s) * invf[f]
                a, b = x[h, s, f], x[h, s, f + 32]
                assert abs(r[h, s, f] - (a * math.cos(th) - b * math.sin(th))) < 1e-12
                assert abs(r[h, s, f + 32] - (b * math.cos(th) + a * math.sin(th))) < 1e-12
    np.testing.assert_allclose(np.linalg.norm(r, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-12)


def test_rope_graph_equals_fused_loop():
    p = Program()
    x = p.input("x", (2, 3, 64))
    pos = p.input("pos", ())
    for llama3 in (False, True):
        invf = ir.llama3_inv_freq(500000.0, 32) if llama3 else ir.rope_inv_freq(500000.0, 32)
        vals = {"x": oracle.lcg(4, 384).reshape(2, 3, 64), "pos": np.array(1000.0)}
        # per-row positions 1000 + s (prefill form)
        rows = ir.map_(ir.ADD, ir.iota(3), pos)
        got = oracle.eval_node(p, ir.rope(x, rows, invf), vals)
        want = oracle.rope(vals["x"], 1000, oracle.inv_freq(500000.0, 32, llama3))
        np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-12)
        # the reference's scalar-position form puts every row at the same position
        got1 = oracle.eval_node(p, ir.rope(x, pos, invf), vals)
        for s in range(3):
            want1 = oracle.rope(vals["x"][:, s:s + 1], 1000, oracle.inv_freq(500000.0, 32, llama3))
            np.testing.assert_allclose(got1[:, s:s + 1], want1, rtol=1e-10, atol=1e-12)


def test_llama3_inv_freq_closed_form():
    """examples/llama3_2.rs:91-107 evaluated in plain Python."""
    got = oracle.inv_freq(500000.0, 32, True)
    for f in range(32):
        inv = 500000.0 ** (-f / 32)
        wave = 2 * math.pi / inv
        if wave > 8192.0:
            want = inv / 32
        elif wave < 2048.0:
            want = inv
        else:
            sm = (8192.0 / wave - 1.0) / 3.0
            want = (1 - sm) * inv / 32 + sm * inv
        assert abs(got[f] - want) <= 1e-14 * want   # exp(f·ln) vs pow: a few ulp


def test_rmsnorm_projection_program_equals_closed_form():
    M, K, N = 3, 64, 40
    p = configs.rmsnorm_projection(M, K, N, kmajor=True)
    x = oracle.synth(1, M * K, dtype=ir.BF16).reshape(M, K)
    g = oracle.synth(2, K, "normal", 1.0, 0.02, dtype=ir.BF16)
    wbits = oracle.synth_bf16(3, K * N, "normal", 0.0, 0.02).reshape(K, N)
    w = (wbits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    got, _ = oracle.fold_stage(p, 0, {"x": x, "g": g, "W": w})
    np.testing.assert_allclose(got, oracle.rmsnorm_proj(x, g, wbits, 1e-5), rtol=1e-12)
    # and against numpy
    ref = (x * g / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-5)) @ w
    np.testing.assert_allclose(got, ref, rtol=1e-10)


def test_int4_program_equals_reference_signed_form():
    """u·s − z with z = 8·s equals the reference's signed I4 load times scale (w4(u) = u − 8)."""
    M, K, N, G = 2, 128, 24, 64
    p = configs.int4_matmul(M, K, N, G)
    rng = np.random.default_rng(3)
    u = rng.integers(0, 16, size=(N, K))
    s = oracle.synth(5, N * K // G, "uniform", 0.001, 0.02, dtype=ir.BF16).reshape(N, K // G)
    z = np.array([oracle.round_bf16(8 * v) for v in s.reshape(-1)]).reshape(s.shape)
    assert np.all(z == 8 * s)
    x = oracle.synth(6, M * K, dtype=ir.BF16).reshape(M, K)
    got, _ = oracle.fold_stage(p, 0, {"x": x, "Wq": u.reshape(N, K // G, G), "S": s, "Z": z})
    signed = (u - 8) * np.repeat(s, G, axis=1)
    np.testing.assert_allclose(got, x @ signed.T, rtol=1e-12, atol=1e-12)
    packed = (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8)
    np.testing.assert_allclose(oracle.int4_matmul(x, packed, s, z, G), got, rtol=1e-12, atol=1e-12)


def test_decode_attention_equals_causal_prefill_row():
    """Incremental decode == causal prefill (tests/decode.rs:121-200): the decode attention at
    position p over a cache equals row p of the causal attention over the same K/V."""
    H, S, D = 2, 12, 16
    q = oracle.lcg(21, H * S * D).reshape(H, S, D)
    k = oracle.lcg(22, H * S * D).reshape(H, S, D)
    v = oracle.lcg(23, H * S * D).reshape(H, S, D)
    full = oracle.attention(q, k, v, 0.25, mask=1)
    for pos in range(S):
        dec = oracle.attention(q[:, pos:pos + 1], k, v, 0.25, mask=3, q_pos0=pos)
        np.testing.assert_allclose(dec[:, 0], full[:, pos], rtol=1e-12, atol=1e-14)
    vt = np.ascontiguousarray(v.transpose(0, 2, 1))
    np.testing.assert_allclose(oracle.attention(q, k, vt, 0.25, mask=1, v_transposed=True), full, rtol=1e-12)


def test_reserved_cache_length_does_not_change_decode():
    """tests/reserved_cache.rs:1-12: unwritten slots past the prefix change nothing."""
    NH, NKV, HD = 4, 2, 16
    prog_s = configs.decode_attention(NH, NKV, HD, 8, out_dtype=ir.F32)
    prog_l = configs.decode_attention(NH, NKV, HD, 40, out_dtype=ir.F32)
    q = oracle.lcg(31, NH * HD).reshape(NH, HD)
    k = oracle.lcg(32, NKV * 8 * HD).reshape(NKV, 8, HD)
    v = oracle.lcg(33, NKV * HD * 8).reshape(NKV, HD, 8)
    kl = np.zeros((NKV, 40, HD)); kl[:, :8] = k
    vl = np.zeros((NKV, HD, 40)); vl[:, :, :8] = v
    a = oracle.run_program(prog_s, {"q": q, "k_cache": k, "v_cache": v, "position": np.array(5.0)})["o"]
    b = oracle.run_program(prog_l, {"q": q, "k_cache": kl, "v_cache": vl, "position": np.array(5.0)})["o"]
    np.testing.assert_allclose(a, b, rtol=1e-12)


def _numpy_attention(q, k, v, scale, visible):
    """Brute-force softmax attention with an explicit visibility matrix (GQA by h // rep)."""
    Hq, Hkv = q.shape[0], k.shape[0]
    rep = Hq // Hkv
    out = np.empty((Hq, q.shape[1], v.shape[2]))
    for h in range(Hq):
        s = q[h] @ k[h // rep].T * scale
        s = np.where(visible, s, -np.inf)
        e = np.exp(s - s.max(-1, keepdims=True))
        out[h] = (e / e.sum(-1, keepdims=True)) @ v[h // rep]
    return out


@pytest.mark.parametrize("window", [0, 1, 5])
def test_fused_attention_masks_against_brute_force(window):
    """oracle.attention's causal (mask 1), sliding-window (mask 2: q − W + 1 ≤ k ≤ q) and
    decode prefix (mask 3: k ≤ q_pos0 for every query row) masks, with GQA, against an explicit mask matrix."""
    Hq, Hkv, S, D = 4, 2, 9, 8
    q = oracle.lcg(41, Hq * S * D).reshape(Hq, S, D)
    k = oracle.lcg(42, Hkv * S * D).reshape(Hkv, S, D)
    v = oracle.lcg(43, Hkv * S * D).reshape(Hkv, S, D)
    qi, ki = np.arange(S)[:, None], np.arange(S)[None, :]
    if window:
        vis = (ki <= qi) & (ki >= qi - window + 1)
        got = oracle.attention(q, k, v, 0.3, mask=2, window=window)
    else:
        vis = ki <= qi
        got = oracle.attention(q, k, v, 0.3, mask=1)
    np.testing.assert_allclose(got, _numpy_attention(q, k, v, 0.3, vis), rtol=1e-12, atol=1e-14)
    pre = oracle.attention(q[:, 2:4], k, v, 0.3, mask=3, q_pos0=4)
    np.testing.assert_allclose(pre, _numpy_attention(q[:, 2:4], k, v, 0.3, np.broadcast_to(ki <= 4, (2, S))),
                               rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("window", [0, 3])
def test_flash_prefill_graph_equals_fused_attention(window):
    """The config-C graph (the rotation table and K-RoPE stages, Q's RoPE inside the score
    leaf, GQA expand, causal and window masks as additive where terms) under the interpreter
    equals the fused attention over RoPE'd inputs."""
    NH, NKV, S, HD = 4, 2, 8, 8
    prog = configs.flash_prefill(NH, NKV, S, HD, theta=10000.0, window=window)
    vals = {"Q": oracle.lcg(51, NH * S * HD).reshape(NH, S, HD),
            "K": oracle.lcg(52, NKV * S * HD).reshape(NKV, S, HD),
            "V": oracle.lcg(53, NKV * S * HD).reshape(NKV, S, HD)}
    rb = np.vectorize(oracle.round_bf16)
    vals = {n: rb(a) for n, a in vals.items()}
    got = oracle.run_program(prog, vals)
    invf = oracle.inv_freq(10000.0, HD // 2)
    qr, kr = oracle.rope(vals["Q"], 0, invf), rb(oracle.rope(vals["K"], 0, invf))
    # the table holds cos and sin rounded to f32: the stored bf16 K rows may sit one rounding
    # step away from those of the f64 rotation
    np.testing.assert_allclose(got["Kr"], kr, rtol=2 ** -8, atol=1e-12)
    want = oracle.attention(qr, got["Kr"], vals["V"], 1 / np.sqrt(HD), mask=2 if window else 1, window=window)
    np.testing.assert_allclose(got["O"], rb(want), rtol=2 ** -7, atol=1e-6)


def _scan_program(shape, dim, monoid):
    p = Program()
    x = p.input("X", shape, ir.F32)
    p.pointwise("Y", ir.scan(x, dim, monoid), ir.F32)
    return p


def test_scan_known_answer():
    """Add-scan of [2, -1, 3, 0.5, 4] (tests/laws.rs:715-730, the reference's fallback stage)."""
    p = _scan_program((5,), 0, ir.M_ADD)
    vals = {"X": np.array([2.0, -1.0, 3.0, 0.5, 4.0])}
    np.testing.assert_array_equal(oracle.eval_node(p, ir.scan(p.node("X"), 0, ir.M_ADD), vals),
                                  [2.0, 1.0, 4.0, 4.5, 8.5])
    np.testing.assert_array_equal(oracle.run_program(p, vals)["Y"], [2.0, 1.0, 4.0, 4.5, 8.5])


@pytest.mark.parametrize("dim", [0, 1])
def test_scan_matches_numpy_cumulative_ops(dim):
    """Every monoid along either axis against numpy's accumulate (inclusive prefix)."""
    x = oracle.lcg(77, 6 * 7).reshape(6, 7) * 2.0
    p = Program()
    p.input("X", (6, 7), ir.F32)
    want = {ir.M_ADD: np.add.accumulate(x, axis=dim), ir.M_MUL: np.multiply.accumulate(x, axis=dim),
            ir.M_MAX: np.maximum.accumulate(x, axis=dim), ir.M_MIN: np.minimum.accumulate(x, axis=dim),
            ir.M_LSE: np.logaddexp.accumulate(x, axis=dim)}
    for m, w in want.items():
        got = oracle.eval_node(p, ir.scan(p.node("X"), dim, m), {"X": x})
        np.testing.assert_allclose(got, w, rtol=1e-12, atol=1e-12)
