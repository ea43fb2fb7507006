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
