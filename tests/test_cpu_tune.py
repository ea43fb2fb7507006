"""The measured tuner's verdict procedure (compile.rs:1348-1630 rules) over a scripted
instrument, and its family grouping over the decode program — no GPU needed."""
from sanic_amd import configs
from sanic_amd.tune import Family, decide, families


class Scripted:
    """measure(stage -> variant): a fixed per-family cost table plus a clock drift per call,
    recording every assignment it was asked to time."""

    def __init__(self, cost, drift=0.0):
        self.cost, self.drift, self.calls = cost, drift, []

    def __call__(self, assign):
        self.calls.append(dict(assign))
        t = 100.0 + self.drift * len(self.calls)
        for (stages, v), c in self.cost.items():
            if all(assign.get(s, 0) == v for s in stages):
                t += c
        return t


def test_winner_needs_the_margin_and_family_swaps_together():
    fams = [Family("a", "ka", [1, 5, 9], 3), Family("b", "kb", [2], 2)]
    # family a: variant 2 saves 3 (3%), variant 1 saves 0.5 (<1%); family b: nothing to gain
    m = Scripted({((1, 5, 9), 2): -3.0, ((1, 5, 9), 1): -0.5})
    rep = decide(fams, m)
    assert rep.shipped and rep.choices == {"ka": 2}
    assert rep.variants == {1: 2, 5: 2, 9: 2}
    # every candidate is timed right after a baseline of the current choice
    for i in range(0, len(rep.trials) * 2, 2):
        base, cand = m.calls[i], m.calls[i + 1]
        assert set(cand) - set(base) or cand != base
    # family b is judged with family a's winner already in place
    b_trial = [i for i, c in enumerate(m.calls) if c.get(2) == 1][0]
    assert m.calls[b_trial].get(1) == 2


def test_adjacent_baselines_absorb_clock_drift():
    # the clock slows down by 0.4 per measurement; a candidate 2% faster than its neighbour
    # still wins, whatever the first baseline read
    fams = [Family("a", "ka", [0], 2)]
    m = Scripted({((0,), 1): -2.0}, drift=0.4)
    rep = decide(fams, m)
    assert rep.choices == {"ka": 1}


def test_a_tune_that_does_not_beat_a_fresh_baseline_ships_nothing():
    fams = [Family("a", "ka", [0], 2)]

    calls = []

    def measure(assign):
        calls.append(dict(assign))
        # the candidate looks 5% faster next to its baseline, but the final comparison
        # (analytic vs tuned, measured fresh) shows no gain
        if len(calls) <= 2:
            return 95.0 if assign else 100.0
        return 100.0
    rep = decide(fams, measure)
    assert not rep.shipped and rep.variants == {} and rep.choices == {}


def test_no_candidates_ships_nothing():
    rep = decide([], lambda a: 1.0)
    assert not rep.shipped and rep.trials == []


def test_decode_program_families():
    """Every per-layer kernel is one family of 16 (15 for the first layer's structural twin),
    each with its variant count; folded stages (batched, absorbed) are not candidates."""
    fams = families(configs.llama_decode())
    by_kernel = {}
    for f in fams:
        by_kernel.setdefault(f.kernel, []).append(f)
    assert any(len(f.stages) == 16 and f.variants == 7 for f in by_kernel["sanic_attn_decode_h32_t2080"])
    assert any(len(f.stages) == 16 and f.variants == 3 for f in by_kernel["sanic_gemv_16384x2048"])
    assert any(len(f.stages) >= 15 and f.variants == 4 for f in by_kernel["sanic_gemv_2048x8192"])
    assert [len(f.stages) for f in by_kernel["sanic_gemv_128256x2048"]] == [1]


def test_flash_edge_tiles_use_the_raw_window():
    """The flash skeleton's edge-tile path needs the row window before an empty window is
    widened: the rendered window_raw has no reset line and the kernel calls it on edge tiles."""
    import re
    from sanic_amd import configs
    for window in (0, 1024):
        kind, src = configs.flash_prefill(window=window).emit(2)
        assert kind.startswith("skeleton:flash_prefill")
        raw = re.search(r"bool window_raw\(.*?\n\}", src, re.S).group(0)
        assert "whi <= wlo" not in raw and "return whi > wlo;" in raw
        assert "window_raw(a, hh, qi, rl, rh)" in src
