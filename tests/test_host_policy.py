"""Host-side policy of the host tier, on the CPU: the adaptive prefetch window
(adaptive_prefetch_controller.py:77-133) against hand-computed traces, and the
chunk -> host-record ranges the prefetcher copies against a brute-force scan."""
from collections import OrderedDict
from types import SimpleNamespace

import numpy as np
import pytest
import torch


def test_adaptive_window_without_signals_stays_at_floor():
    from heterokv.prefetcher import AdaptivePrefetchController
    c = AdaptivePrefetchController()
    assert [c.compute_window() for _ in range(5)] == [2] * 5
    assert c.stats["step"] == 5 and c.stats["miss_rate"] == 0.0


def test_adaptive_window_miss_penalty_moves_one_step_at_a_time():
    from heterokv.prefetcher import AdaptivePrefetchController
    c = AdaptivePrefetchController()
    # miss rate 1: raw = 2 + 0.5 * 1 * 8 = 6, approached by +1 per step
    assert [c.compute_window(cache_miss=True) for _ in range(6)] == [3, 4, 5, 6, 6, 6]


def test_adaptive_window_rounds_half_to_even():
    from heterokv.prefetcher import AdaptivePrefetchController
    c = AdaptivePrefetchController(miss_window_size=8)
    for _ in range(7):
        assert c.compute_window(cache_miss=False) == 2
    # miss rate 1/8: raw = 2 + 0.5 * 0.125 * 8 = 2.5 -> round() gives 2
    assert c.compute_window(cache_miss=True) == 2
    # 2/8: raw = 3 -> 3
    assert c.compute_window(cache_miss=True) == 3


def test_adaptive_window_volatility_trace():
    from heterokv.prefetcher import AdaptivePrefetchController
    c = AdaptivePrefetchController()
    x = torch.tensor([0.0, 1.0, 2.0, 3.0])
    assert c.compute_window(attention_weights=x) == 2          # sigma_ref := sigma_1, deviation 0
    # sigma_2 = 2 s: sigma_ref = 0.9 s + 0.1 * 2 s = 1.1 s, deviation 2/1.1 - 1 = 0.818,
    # raw = 2 + 1.5 * 0.818 = 3.23 -> 3
    assert c.compute_window(attention_weights=2 * x) == 3
    assert abs(c.stats["sigma_ref"] - 1.1 * float(x.std())) < 1e-6
    # sigma_3 = s/4: sigma_ref = 0.99 s + 0.025 s = 1.015 s, deviation 0.25/1.015 - 1 = -0.754,
    # raw = 2 - 1.13 = 0.87 -> clamped to 2
    assert c.compute_window(attention_weights=x / 4) == 2
    # a huge jump is capped at delta_max = 2 and then at one step: 2 -> 3
    assert c.compute_window(attention_weights=100 * x) == 3


def _manager_stub(chunks):
    from heterokv.manager import HeteroKVManager
    m = HeteroKVManager.__new__(HeteroKVManager)
    m._chunks = OrderedDict(chunks)
    m._chunk_eviction_order = list(m._chunks)
    m._chunk_attention_scores = {k: 1.0 / (i + 1) for i, k in enumerate(m._chunks)}
    return m


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_host_runs_match_brute_force(seed):
    rng = np.random.default_rng(seed)
    chunks = [("l0_e0", (0, 0, 448)), ("l0_e1", (0, 448, 1024)), ("l0_e2", (0, 1472, 2048)),
              ("l0_e3", (0, 3520, 900))]
    m = _manager_stub(chunks)
    B = 3
    nb = (3520 + 900 + 15) // 16
    full = (3520 + 900) // 16
    chosen = np.sort(rng.choice(B * full, size=int(0.75 * B * full), replace=False))
    st = SimpleNamespace(n_host=len(chosen), host_lbs=(chosen // B).astype(np.int64), version=0, runs_cache=None)
    assert m._host_runs(st, None) == [(0, len(chosen))]

    def check(sel):
        want = set()
        for k in sel:
            _, start, n = m._chunks[k]
            lbs = set(range(start // 16, (start + n + 15) // 16))
            want |= {i for i, lb in enumerate(st.host_lbs) if lb in lbs}
        runs = m._host_runs(st, sel)
        got = set()
        for k0, k1 in runs:
            assert k1 > k0
            got |= set(range(k0, k1))
        assert got == want, sel
        assert all(runs[i][1] < runs[i + 1][0] for i in range(len(runs) - 1))  # disjoint, merged

    for sel in [("l0_e0",), ("l0_e1", "l0_e3"), ("l0_e0", "l0_e1", "l0_e2", "l0_e3"), ("l0_e2",), ("l0_e2",)]:
        check(sel)
    # the runs are cached per (layer version, selection): a new host placement with a new
    # version is not answered from the cache
    keep = np.sort(rng.choice(len(chosen), size=len(chosen) // 2, replace=False))
    st.host_lbs, st.n_host = st.host_lbs[keep], len(keep)
    st.version += 1
    check(("l0_e2",))
    assert nb >= full


def test_window_selection_follows_score_changes():
    """The cached ranking of a layer's chunks is rebuilt after any score write, and the
    selection stays in eviction order."""
    from heterokv.manager import _Scores
    chunks = [("l0_e%d" % i, (0, 64 * i, 64)) for i in range(6)]
    m = _manager_stub(chunks)
    m._chunk_attention_scores = _Scores({k: 1.0 / (i + 1) for i, k in enumerate(m._chunks)})
    m._ranked, m._sel_cache = {}, {}
    keys = list(m._chunks)
    assert m._top_chunks(0, keys, 2) == ("l0_e0", "l0_e1")
    assert m._top_chunks(0, keys, 2) == ("l0_e0", "l0_e1")          # from the cache
    m._chunk_attention_scores["l0_e4"] = 5.0
    assert m._top_chunks(0, keys, 2) == ("l0_e0", "l0_e4")
    m._chunk_attention_scores.update({"l0_e5": 9.0, "l0_e2": 7.0})
    assert m._top_chunks(0, keys, 3) == ("l0_e2", "l0_e4", "l0_e5")
    # a plain dict put in its place is not cached at all
    m._chunk_attention_scores = {k: float(i) for i, k in enumerate(keys)}
    assert m._top_chunks(0, keys, 2) == ("l0_e4", "l0_e5")
    m._chunk_attention_scores["l0_e0"] = 99.0
    assert m._top_chunks(0, keys, 2) == ("l0_e0", "l0_e5")
