"""Headline benchmark: Llama-3.2-1B-shape bf16 decode tokens/s on one MI355X.

Workload (BASELINE.json config E): 16 layers, hidden 2048, 32/8 heads, head_dim 64, SwiGLU 8192,
vocab 128256, tied embeddings, RoPE θ 5e5 (llama-3 schedule), RMSNorm eps 1e-5; bf16 weights
N(0, 0.02) (norm gains 1) generated on the device from a seed; a 2048-token random-id prompt is
prefilled token by token into the in-place bf16 KV cache, then greedy decode steps run as
back-to-back hipGraph replays (token fed back and position advanced on the device). A step is
one decode step; `value` = decode tokens/s over the K timed steps (positions 2048 … 2048+K−1).

Also reported: the roofline of the dominant kernel (the batched gate/up norm-fused GEMV, timed
live with HIP events over back-to-back graph replays of that kernel alone) and the CPU baseline
(the C restatement of the reference's interpreter semantics timed on this host, rank 0 only).
"""
from __future__ import annotations

import argparse
import json
import os
import struct
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PROMPT = 2048
HBM_PEAK = 8.0e12
# Boundary-storage policy of the timed decode step: f32 intermediates (the reference's default
# `Policy`), whose greedy ids match the oracle's exactly; `--bf16-boundary` runs the reference's
# `--bf16` policy (/root/reference/examples/llama3_2.rs:480-503), every materialised
# intermediate stored bf16 — 0.9% faster, but its bf16 logits tie or swap the top two against an
# f64 oracle on ≈5% of steps.
BOUNDARY_BF16 = False


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def device_weights(dev, shape, seed=1234):
    """bf16 N(0, 0.02) weights (norm gains 1) made on the GPU by torch, bound zero-copy."""
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    keep, bufs = [], {}
    for name, shp in shape.weight_shapes():
        if name.endswith("norm.weight"):
            t = torch.ones(shp, dtype=torch.bfloat16, device="cuda")
        else:
            t = (torch.randn(shp, generator=g, device="cuda", dtype=torch.float32) * 0.02).to(torch.bfloat16)
        keep.append(t)
        bufs[name] = dev.wrap(t.data_ptr(), t.numel() * 2)
    torch.cuda.synchronize()
    return bufs, keep


def dominant_kernel_roofline(dev, shape, weights, reps=40, copies=8, boundary=None):
    """The decode step's dominant kernel — the batched gate/up RMSNorm-fused GEMV with the
    SwiGLU product computed per row pair (one launch: N = 2·ffn rows, K = hidden) — `copies`
    launches per hipGraph replay, copy r on layer r's weights (8 × 67 MB overflows the 256 MB
    Infinity Cache, so every launch streams cold weights from HBM as in the decode step), timed
    with HIP events on the library's stream over `reps` back-to-back replays. Per-launch time =
    total / (reps · copies)."""
    from sanic_amd import carrier as C
    from sanic_amd import ir
    from sanic_amd.program import STREAM, Program
    H, F = shape.hidden, shape.ffn
    B = boundary if boundary is not None else (ir.BF16 if BOUNDARY_BF16 else ir.F32)
    bb = 2 if B == ir.BF16 else 4
    p = Program()
    x = p.input("x", (H,), B)
    for r in range(copies):
        g = p.input(f"g{r}", (H,), ir.BF16)
        ws = {nm: p.input(f"W{nm}{r}", (F, H), ir.BF16) for nm in ("gate", "up")}
        gu = {nm: p.fused(f"{nm}{r}", (F,), H, [(x, (STREAM,)), (g, (STREAM,)), (ws[nm], (0, STREAM))],
                          C.norm_fused_projection(H, shape.eps), B) for nm in ("gate", "up")}
        p.pointwise(f"h{r}", ir.map_(ir.MUL, ir.silu(gu["gate"]), gu["up"]), B)
    exe = dev.prepare(p)
    kname = exe.stage_kernel(0)
    assert kname.startswith("skeleton:gemv[batched 2]+paired"), kname
    xb = dev.from_values([0.5] * H, B)
    binds = {"x": xb}
    for r in range(copies):
        pre = f"model.layers.{r % shape.layers}."
        binds.update({f"g{r}": weights[pre + "post_attention_layernorm.weight"],
                      f"Wgate{r}": weights[pre + "mlp.gate_proj.weight"], f"Wup{r}": weights[pre + "mlp.up_proj.weight"]})
    rp = exe.capture(binds)
    rp.step_many(5)
    secs = rp.step_many(reps) / (reps * copies)
    # weights + x + gain (bf16) + gate, up and h outputs (x and the outputs in the boundary dtype)
    nbytes = 2 * F * H * 2 + H * bb + H * 2 + 3 * F * bb
    return {"bound": "hbm", "achieved": nbytes / secs / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
            "frac": nbytes / secs / HBM_PEAK, "traffic": traffic_from_profile(),
            "kernel": f"sanic_gemv_{2 * F}x{H} ({kname})", "bytes_per_launch": nbytes,
            "us_per_launch": secs * 1e6}


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(shape, boundary_bf16, seconds_budget=24.0, interpreter=True):
    """The CPU path on this host, three legs, all outside the GPU's timed region:
      - the oracle's fused f64 decode step (oracle_llama_step: the rustgen-shaped loops over the
        bf16 weights) at positions 2048.. with every thread the host offers us (`value`),
      - the same on one thread,
      - the naive interpreter (oracle_run_program: interp.rs's node-by-node eval of the decode
        schedule) on ONE layer of the model with the vocabulary cut to 16384, labelled as such
        (the full model takes minutes per step this way).
    The decode steps attend over a zero-filled 2048-position cache: the work per step equals a
    real step's (every weight read once, attention over p + 1 positions); only the time is used."""
    import numpy as np
    import oracle
    from sanic_amd import configs, ir
    from tests.llama_ref import OracleModel, synth_weights
    threads = oracle.threads()
    w = synth_weights(shape, seed=99)
    om = OracleModel(shape, w, boundary_bf16=boundary_bf16)

    def timed(nthreads, budget, max_steps):
        n, t0, tok = 0, time.perf_counter(), 1
        while True:
            tok, _ = om.step(tok, PROMPT + n, nthreads)
            n += 1
            el = time.perf_counter() - t0
            if el > budget or n >= max_steps:
                return n, el

    n, el = timed(threads, seconds_budget / 3, 8)
    n1, el1 = timed(1, seconds_budget / 3, 4)
    # the interpreter leg: one layer (same widths, vocabulary 16384), one step (`interpreter`
    # False leaves it out: the leg alone takes tens of seconds)
    one = configs.LlamaShape(layers=1, capacity=PROMPT + 1, vocab=16384)
    prog = configs.llama_decode(one, boundary=ir.BF16 if boundary_bf16 else ir.F32)
    vals = {name: (w[name].reshape(-1)[:int(np.prod(shp))].astype(np.uint32) << 16).view(np.float32)
            .astype(np.float64).reshape(shp) for name, shp in one.weight_shapes()}
    vals["tokens"] = np.array([1.0])
    vals["position"] = np.array(float(PROMPT))
    t0 = time.perf_counter()
    if interpreter:
        oracle.run_program(prog, vals)
    el_i = time.perf_counter() - t0 if interpreter else None
    del om, w, vals
    return {"value": n / el, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{n} decode steps of the full model at positions {PROMPT}..{PROMPT + n - 1} "
                      f"(f64 fused loops over bf16 weights, {threads} threads)",
            "single_thread_tok_s": n1 / el1, "single_thread_steps": n1,
            "interpreter_one_layer_s_per_step": el_i,
            "interpreter_sample": "one decode step of a 1-layer model (hidden 2048, ffn 8192, vocab 16384) "
                                  "through the node-by-node interpreter, single thread",
            "cpu_model": _cpu_model(), "host_cpus": os.cpu_count(), "host": os.uname().nodename}


# ── secondary configurations (BASELINE.json configs B, C, D): one dominant kernel each ──

CONFIGS = {
    # name: (algorithmic unit count, unit, bound)
    "B1": "RMSNorm-fused GEMV M=1, K=2048 → N=8192, W bf16 [K, N] (K-major)",
    "B1rows": "RMSNorm-fused GEMV M=1, K=2048 → N=8192, W bf16 [N, K] (the reference's [out, in])",
    "B2": "RMSNorm-fused GEMM M=512, K=2048 → N=8192, W bf16 [K, N]",
    "C1": "GQA causal FlashAttention prefill, 32/8 heads, d=64, S=4096, RoPE on Q (in the kernel) and K (a stage)",
    "C2": "GQA sliding-window (1024) FlashAttention prefill, 32/8 heads, d=64, S=4096",
    "C3": "GQA decode attention, 1 query vs 4096-entry KV cache, split-K combine",
    "D1": "int4 group-quantized GEMV M=1, [8192, 2048] uint4, group 64",
    "D2": "int4 group-quantized GEMM M=128, [8192, 2048] uint4, group 64",
}


def _bind_random(dev, prog, keep, seed=7):
    """Device-resident synthetic inputs for every INPUT/STATE buffer of `prog` (torch RNG)."""
    import torch
    from sanic_amd import ir
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    binds = {}
    for b in prog.buffers:
        if b.role not in (0, 1):
            continue
        n = int(__import__("math").prod(b.shape)) if b.shape else 1
        base = b.name.split(".copy")[0]
        if b.dtype == ir.BF16:
            t = torch.randn(n, generator=g, device="cuda", dtype=torch.float32).to(torch.bfloat16)
            if base in ("S", "Z"):
                t = (t.float().abs() * 0.005 + 0.001).to(torch.bfloat16)
        elif b.dtype == ir.F32:
            t = torch.zeros(max(n, 1), device="cuda", dtype=torch.float32)
            if base == "position":
                t.fill_(4095.0)
        elif b.dtype in (ir.U4, ir.I4):
            t = torch.randint(0, 256, ((n + 1) // 2,), generator=g, device="cuda", dtype=torch.uint8)
        else:
            t = torch.zeros(b.nbytes, device="cuda", dtype=torch.uint8)
        keep.append(t)
        binds[b.name] = dev.wrap(t.data_ptr(), b.nbytes)
    torch.cuda.synchronize()
    return binds


def _time_program(dev, prog, keep, reps=20):
    exe = dev.prepare(prog)
    binds = _bind_random(dev, prog, keep)
    rp = exe.capture(binds)
    rp.step_many(3)
    return rp.step_many(reps) / reps, exe


COLD_BYTES = 600 << 20      # more than twice the 256 MB Infinity Cache


def config_row(dev, name: str):
    """One secondary configuration's dominant kernel: `copies` launches per graph replay, each
    on its own copy of the inputs (together more than twice the Infinity Cache), so every launch
    reads cold inputs as it would in a real workload; plus the configuration's whole program
    end to end (for C1/C2 with its RoPE stages). Per-launch times include the gap between
    dependent launches inside the graph."""
    from sanic_amd import configs
    keep = []
    if name in ("B1", "B1rows", "B2"):
        M = 512 if name == "B2" else 1
        mk = lambda: configs.rmsnorm_projection(M=M, kmajor=(name != "B1rows"))
        K, N = 2048, 8192
        flops = 2.0 * M * K * N + 2.0 * M * K
        nbytes = K * N * 2 + M * K * 2 + K * 2 + M * N * 2
        bound = "mfma" if name == "B2" else "hbm"
    elif name in ("D1", "D2"):
        M = 128 if name == "D2" else 1
        mk = lambda: configs.int4_matmul(M=M)
        K, N = 2048, 8192
        flops = 2.0 * M * K * N
        nbytes = N * K // 2 + 2 * (N * K // 64) * 2 + M * K * 2 + M * N * 2
        bound = "hbm" if name == "D1" else "both"
    elif name in ("C1", "C2"):
        # as configured: RoPE on Q (inside the flash kernel's score leaf) and K (a pointwise
        # stage), the rotation table shared by every head
        w = 1024 if name == "C2" else 0
        mk = lambda: configs.flash_prefill(window=w)
        S, NH, HD = 4096, 32, 64
        pairs = (w * (w + 1) / 2 + (S - w) * w) if w else S * (S + 1) / 2
        flops = 4.0 * HD * NH * pairs
        nbytes = 2 * (NH * S * HD * 2) + 2 * (8 * S * HD * 2)
        bound = "mfma"
    elif name == "C3":
        mk = lambda: configs.decode_attention()
        flops = 4.0 * 64 * 32 * 4096
        nbytes = 2 * 8 * 4096 * 64 * 2
        bound = "hbm"
    else:
        raise SystemExit(f"unknown config {name}; known: {sorted(CONFIGS)}")
    full = mk()
    t_full, exe_full = _time_program(dev, full, keep)
    prog = mk()
    main = len(prog.stages) - 1          # the configuration's dominant stage (after any RoPE stages)
    in_bytes = sum(b.nbytes for b in prog.buffers if b.role == 0)
    copies = max(8, min(128, -(-COLD_BYTES // max(in_bytes, 1))))

    def timed(n):
        p = mk()
        p.repeat_stage(main, n - 1, fresh_inputs=True)
        os.environ["SANIC_HIP_NO_BATCH"] = "1"
        try:
            return _time_program(dev, p, keep, reps=10)
        finally:
            del os.environ["SANIC_HIP_NO_BATCH"]
    t_k, exe = timed(copies)
    # stages ahead of the main one (C1/C2's rotation table and K-RoPE) run once per replay and
    # are counted in: a conservative per-launch figure (they are ≈10 µs of ≈2.5 ms)
    per = t_k / copies
    row = {"kernel": exe.stage_kernel(main), "us_per_launch": per * 1e6, "bound": bound,
           "launches_per_replay": copies, "inputs_per_launch_bytes": in_bytes,
           "end_to_end_ms": t_full * 1e3, "flops": flops, "bytes": nbytes}
    if bound in ("hbm", "both"):
        row.update({"achieved_GBps": nbytes / per / 1e9, "frac_hbm": nbytes / per / HBM_PEAK})
    if bound in ("mfma", "both"):
        row.update({"achieved_TFLOPs": flops / per / 1e12, "frac_mfma": flops / per / 2.5e15})
    row["frac"] = row["frac_mfma"] if bound == "mfma" else row["frac_hbm"]
    del keep
    return row, exe_full, full


def bench_config(name: str):
    from sanic_amd.backend import HipDevice
    dev = HipDevice(0)
    row, exe_full, full = config_row(dev, name)
    bound = row["bound"]
    t_full = row["end_to_end_ms"] * 1e-3
    out = {"metric": f"{name}: {CONFIGS[name]}",
           "value": (row["flops"] / t_full / 1e12) if bound == "mfma" else (row["bytes"] / t_full / 1e9),
           "unit": "TFLOP/s" if bound == "mfma" else "GB/s", "n_gpus": 1, "config": {"workload": CONFIGS[name]},
           "stages": [exe_full.stage_kernel(i) for i in range(len(full.stages))], "roofline": row, "dtype": "bf16"}
    print(json.dumps(out), flush=True)


def pmc_probe(reps=20):
    """A short program for the rocprofv3 --pmc passes: `reps` launches of the dominant kernel
    (the batched gate/up GEMV, layer-0 shapes) and `reps` plain device copies of 256 MiB, whose
    known byte counts calibrate FETCH_SIZE / WRITE_SIZE."""
    import torch
    from sanic_amd import configs
    from sanic_amd.backend import HipDevice
    torch.cuda.init()
    dev = HipDevice(0)
    shape = configs.LlamaShape(layers=1)
    H, F = shape.hidden, shape.ffn
    keep, weights = [], {}
    pre = "model.layers.0."
    for nm, shp in ((pre + "post_attention_layernorm.weight", (H,)), (pre + "mlp.gate_proj.weight", (F, H)),
                    (pre + "mlp.up_proj.weight", (F, H))):
        t = (torch.randn(shp, device="cuda") * 0.02).to(torch.bfloat16)
        keep.append(t)
        weights[nm] = dev.wrap(t.data_ptr(), t.numel() * 2)
    torch.cuda.synchronize()
    roof = dominant_kernel_roofline(dev, shape, weights, reps=reps)
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"probe": roof["kernel"], "us_per_launch": roof["us_per_launch"],
                      "copy_bytes": 256 << 20}), flush=True)


def traffic_from_profile():
    """HBM bytes per launch of the dominant kernel from the committed PMC summary (the
    `traffic_bytes_per_launch:` line written from two rocprofv3 --pmc passes), or None."""
    path = os.path.join(ROOT, "profiles", "gateup_gemv_16384x2048_hbm_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        return None
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=32)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the per-configuration kernel rows")
    ap.add_argument("--pmc-probe", action="store_true", help="run only the dominant kernel and a calibration copy (for rocprofv3 --pmc)")
    ap.add_argument("--tune", action="store_true",
                    help="run the measured tiling tuner (SANIC_TUNE) on the decode program first and "
                         "bench the tuned program (tuning is outside the timed region)")
    ap.add_argument("--bf16-boundary", action="store_true",
                    help="store the decode step's intermediates bf16 (the reference's --bf16 policy)")
    ap.add_argument("--config", default=None, help="measure a secondary configuration instead: " + ", ".join(CONFIGS))
    args = ap.parse_args()
    if args.pmc_probe:
        pmc_probe()
        return
    if args.config:
        import torch
        torch.cuda.init()
        for name in args.config.split(","):
            bench_config(name)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus above 1 is not supported "
                                   "(see the sharding design note)", "n_gpus": args.gpus}))
        sys.exit(2)

    import torch
    from sanic_amd import configs
    from sanic_amd.backend import HipDevice
    from sanic_amd import ir
    from sanic_amd.llama import LlamaMachine

    boundary = ir.BF16 if args.bf16_boundary or BOUNDARY_BF16 else ir.F32
    cap = PROMPT + max(32, args.steps, args.warmup)
    shape = configs.LlamaShape(capacity=cap)
    torch.cuda.init()
    dev = HipDevice(0)
    t0 = time.perf_counter()
    weights, keep = device_weights(dev, shape)
    tuned = None
    if args.tune:
        from sanic_amd import tune as tuner
        prog = configs.llama_decode(shape, boundary=boundary)
        # zeroed bindings, the decode position rewound to the end of the prompt before every
        # timing: every candidate is judged on the same steps the bench times
        bind = tuner.zero_bindings(dev, prog)
        import struct
        rep = tuner.tune(dev, prog, bind, reset=lambda: bind["position"].upload(struct.pack("<f", float(PROMPT))))
        for kern, v, base, cand in rep.trials:
            log(f"tune {kern} variant {v}: {cand * 1e6:.1f} us vs adjacent {base * 1e6:.1f} us")
        log(f"tune: analytic {rep.baseline_s * 1e6:.1f} us, tuned {rep.tuned_s * 1e6:.1f} us, "
            f"shipped {rep.shipped} {rep.choices}")
        tuned = {"shipped": rep.shipped, "choices": rep.choices,
                 "analytic_us": rep.baseline_s * 1e6, "tuned_us": rep.tuned_s * 1e6}
        m = LlamaMachine(dev, weights, shape, variants=rep.variants, boundary=boundary)
    else:
        m = LlamaMachine(dev, weights, shape, boundary=boundary)
    log(f"prepared in {time.perf_counter() - t0:.1f}s")

    import numpy as np
    rng = np.random.default_rng(2048)
    prompt = rng.integers(0, shape.vocab, size=PROMPT).tolist()
    t0 = time.perf_counter()
    first = m.prefill(prompt)
    prefill_s = time.perf_counter() - t0
    log(f"prefill {PROMPT} tokens token-by-token in {prefill_s:.2f}s; next token {first}")

    # warmup decode steps, then rewind to the end of the prompt and time K steps
    m.decode(args.warmup)
    m.set_position(PROMPT)
    m.set_token(first)
    dev.sync()
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    gpu_s = m.decode(args.steps)
    dev.sync()
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    elapsed = max(wall, gpu_s)
    tok_s = args.steps / elapsed
    ms = elapsed / args.steps * 1e3

    kv_bytes = sum(32768 * (p + 1) for p in range(PROMPT, PROMPT + args.steps)) / args.steps
    step_bytes = shape.weight_bytes() + kv_bytes
    roof = dominant_kernel_roofline(dev, shape, weights, boundary=boundary)
    step_roof = {"bytes_per_step": step_bytes, "achieved_GBps": step_bytes / (ms * 1e-3) / 1e9,
                 "frac_of_8TBps": step_bytes / (ms * 1e-3) / HBM_PEAK}
    rows = {}
    if not args.no_configs:
        for name in CONFIGS:
            rows[name] = config_row(dev, name)[0]
            log(f"{name}: {rows[name]['kernel']} {rows[name]['us_per_launch']:.2f} us/launch, frac {rows[name]['frac']:.3f}")
    cpu = None if args.no_cpu else cpu_baseline(shape, boundary == ir.BF16)
    out = {
        "metric": "tok/s Llama-3.2-1B-shape bf16 decode", "value": tok_s, "unit": "tok/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) bf16 weights, random prompt ids)",
        "config": {"workload": "llama3.2-1b-shape decode, "
                               + ("bf16 boundary storage (the reference's --bf16 policy), " if boundary == ir.BF16 else "f32 intermediates, ")
                               + "2048-token prompt prefilled token-by-token, "
                               f"greedy steps at positions {PROMPT}..{PROMPT + args.steps - 1}",
                   "global_batch": 1, "seq_len": PROMPT, "parallelism": "single-gpu"},
        "roofline": roof, "step_roofline": step_roof, "cpu_baseline": cpu, "configs": rows,
        "gpu_event_seconds": gpu_s, "wall_seconds": wall,
        "prefill_token_by_token_tok_s": PROMPT / prefill_s,
    }
    if tuned is not None:
        out["tuned"] = tuned
    print(json.dumps(out))


if __name__ == "__main__":
    main()
