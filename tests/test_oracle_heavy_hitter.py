"""CPU pinning of oracle/heavy_hitter.py (HeavyHitterOracle, heavy_hitter.py:26-101;
compute_block_scores, oracle_triton.py:16-79; the weights the attention patch hands to
the oracle, fused_attention_patch.py:104-107)."""
import math

import numpy as np
import torch

from oracle import heavy_hitter as hh


def test_reference_scenario_cold_blocks():
    """The reference's own check (tests/test_end_to_end_pipeline.py:63-90): 256 tokens,
    ten updates of U[0, 0.1) with tokens 80..111 at 0.001, sink 16, local 32, two blocks
    asked for: the cold blocks 5 and 6, never the sink block."""
    rng = np.random.default_rng(0)
    scores = np.zeros(256, dtype=np.float32)
    for _ in range(10):
        a = (rng.random(256) * 0.1).astype(np.float32)
        a[80:112] = 0.001
        scores = (scores + a).astype(np.float32)
    got = hh.eviction_candidates(scores, 256, 16, 16, 32, 2)
    assert got == [5, 6]
    assert all(c >= 1 for c in got)


def test_block_means_match_float64():
    rng = np.random.default_rng(1)
    for seq_len, bs in [(256, 16), (1000, 16), (777, 7), (64, 128), (5, 16)]:
        ts = rng.random(seq_len + 3).astype(np.float32)
        got = hh.block_scores(ts, seq_len, bs)
        assert got.shape == (-(-seq_len // bs),)
        want = [ts[i:min(i + bs, seq_len)].astype(np.float64).mean() for i in range(0, seq_len, bs)]
        np.testing.assert_allclose(got, want, rtol=2e-6)
    # the last block is a partial one: its mean is over its own tokens only
    ts = np.array([1, 1, 1, 1, 4, 4], dtype=np.float32)
    assert hh.block_scores(ts, 6, 4).tolist() == [1.0, 4.0]


def _brute(ts, seq_len, bs, sink, local, k):
    if seq_len <= sink + local:
        return []
    nb = math.ceil(seq_len / bs)
    sb, lb = math.ceil(sink / bs), math.ceil(local / bs)
    means = np.array([ts[i * bs:min((i + 1) * bs, seq_len)].astype(np.float64).sum() /
                      (min((i + 1) * bs, seq_len) - i * bs) for i in range(nb)])
    means = means.astype(np.float32).astype(np.float64)
    prot = np.zeros(nb, dtype=bool)
    prot[:sb] = True
    prot[max(0, nb - lb):] = True
    means[prot] = np.inf
    order = np.lexsort((np.arange(nb), means))
    return order[:min(k, max(0, nb - sb - lb))].tolist()


def test_candidates_brute_force_and_invariants():
    rng = np.random.default_rng(2)
    for trial in range(60):
        bs = int(rng.choice([1, 4, 16]))
        seq_len = int(rng.integers(1, 600))
        sink = int(rng.integers(0, 80))
        local = int(rng.integers(0, 120))
        k = int(rng.integers(0, 40))
        # quantized values so that equal block means occur
        ts = (rng.integers(0, 4, seq_len) / 4.0).astype(np.float32)
        got = hh.eviction_candidates(ts, seq_len, bs, sink, local, k)
        assert got == _brute(ts, seq_len, bs, sink, local, k), (trial, seq_len, bs, sink, local, k)
        nb = -(-seq_len // bs)
        sb, lb = -(-sink // bs), -(-local // bs)
        assert all(sb <= c < nb - lb for c in got)
        means = hh.block_scores(ts, seq_len, bs)
        assert all((means[a], a) < (means[b], b) for a, b in zip(got, got[1:]))


def test_short_sequences_and_cold_start():
    ts = np.ones(64, dtype=np.float32)
    assert hh.eviction_candidates(ts, 48, 16, 16, 32, 4) == []      # seq_len <= sink + local
    # heavy_hitter.py:63-74: FIFO after the sink while no scores exist
    assert hh.cold_start_candidates(256, 16, 16, 32, 2) == [1, 2]
    assert hh.cold_start_candidates(256, 16, 16, 32, 100) == list(range(1, 14))
    assert hh.cold_start_candidates(40, 16, 16, 32, 2) == []


def test_newest_token_weights():
    rng = np.random.default_rng(3)
    s = rng.normal(size=(6, 50)) * 3
    s[2, 10:20] = -np.inf
    w = hh.newest_token_weights(s)
    assert abs(w.sum() - 1.0) < 1e-12 and (w >= 0).all()
    # independent formula: natural-log softmax of s * ln 2 per head, then the head mean
    want = torch.softmax(torch.tensor(s) * math.log(2.0), dim=-1).mean(dim=0).numpy()
    np.testing.assert_allclose(w, want, rtol=1e-12, atol=1e-15)
    # equal scores: uniform weights; a masked item gets nothing from that head
    assert np.allclose(hh.newest_token_weights(np.zeros((3, 8))), 1.0 / 8)
    assert hh.newest_token_weights(np.array([[0.0, -np.inf]]))[1] == 0.0
