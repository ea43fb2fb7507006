"""bench.py's contract pieces load without a GPU (a broken default path would only show on the box)."""
import importlib.util
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_bench_defines_every_leg():
    b = _bench()
    for name in ("main", "cpu_baseline", "dominant_kernel_roofline", "bench_config", "pmc_probe", "traffic_from_profile"):
        assert callable(getattr(b, name)), name
    assert set(b.CONFIGS) == {"B1", "B1rows", "B2", "C1", "C2", "C3", "D1", "D2"}


def test_traffic_summary_is_parsed():
    t = _bench().traffic_from_profile()
    assert t is not None and 6.0e7 < t < 8.0e7


def test_cpu_baseline_runs_under_both_policies():
    """The CPU leg of the default bench run, on a one-layer model, under both storage policies."""
    b = _bench()
    from sanic_amd import configs
    shape = configs.LlamaShape(layers=1, capacity=b.PROMPT + 8, vocab=16384)
    for bf16 in (False, True):
        r = b.cpu_baseline(shape, bf16, seconds_budget=0.3, interpreter=False)
        assert r["value"] > 0 and r["kind"] == "port" and r["cores"] >= 1
