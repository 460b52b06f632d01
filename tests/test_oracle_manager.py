"""Pins the manager restatement (oracle/manager.py) with traces derived by hand from
src/memory/manager.py and src/core/engine_wrapper.py.  CPU only."""
from oracle.manager import CacheOracle, ManagerOracle


def test_reference_stage_bc_parameters():
    # tests/test_end_to_end_pipeline.py:31-56: sink 4, budget 8, 32-token prefill
    m = ManagerOracle(2, sink_tokens=4, hbm_budget_tokens=8)
    out = m.update(0, range(32), "prefill")
    assert out == list(range(32))                       # prefill returns the full input
    assert m.sink[0] == [0, 1, 2, 3]
    assert m.tail[0] == [28, 29, 30, 31]                 # tail budget = 8 - 4
    assert m.dram == {"l0_e0": list(range(4, 28))}
    assert len(m.key_cache[0]) <= 4 + 8
    m.update(1, range(32), "prefill")
    # the eviction counter only moves on layer 0 (manager.py:1292-1294)
    assert list(m.dram) == ["l0_e0", "l1_e1"]
    assert m.chunk_scores == {"l0_e0": 1.0, "l1_e1": 0.5}


def test_short_prefill_has_no_body():
    m = ManagerOracle(1, sink_tokens=64, hbm_budget_tokens=8192)
    m.update(0, range(10), "prefill")
    assert m.sink[0] == list(range(10)) and m.tail[0] == [] and not m.dram


def test_chunked_prefill_128k_keep_tail_4160():
    # 131072 tokens in 2048-token chunks, sink 64, keep_tail 4160 (tail budget 4096):
    # chunk 1 -> sink 64 + tail 1984; chunk 2 -> tail 4032; chunk 3 evicts 1984;
    # chunks 4..64 evict 2048 each: 62 chunks / layer, 1984 + 61*2048 = 126912 tokens,
    # while count_dram_tokens reports 62 * 1984 = 123008.
    m = ManagerOracle(1, sink_tokens=64, hbm_budget_tokens=4160)
    for c in range(64):
        ret = m.update(0, range(2048 * c, 2048 * (c + 1)), "prefill", seq_offset=2048 * c)
        if c == 1:
            assert ret == list(range(64)) + list(range(64, 4096))   # sink + old tail + chunk
    chunks = list(m.dram.values())
    assert len(chunks) == 62
    assert len(chunks[0]) == 1984 and all(len(x) == 2048 for x in chunks[1:])
    assert sum(len(x) for x in chunks) == 126912
    assert m.count_dram_tokens(0) == 123008
    assert m.dram_positions(0) == list(range(64, 64 + 126912))
    assert m.tail[0] == list(range(131072 - 4096, 131072))
    assert m.seq_offsets[0] == 131072


def test_decode_slides_tail_into_heavy_hitters_fifo_then_drops():
    m = ManagerOracle(1, sink_tokens=2, hbm_budget_tokens=6)     # tail 4, hh budget 2048
    m.update(0, range(6), "prefill")                            # sink [0,1], tail [2..5]
    assert m.tail[0] == [2, 3, 4, 5]
    out = m.update(0, [6], "decode")
    assert m.tail[0] == [3, 4, 5, 6] and m.hh[0] == [2]
    assert out == [0, 1, 3, 4, 5, 6, 2]                          # sink + tail + hh
    for p in range(7, 7 + 2047):
        m.update(0, [p], "decode")
    assert len(m.hh[0]) == 2048 and m.hh[0][:3] == [2, 3, 4]
    m.update(0, [7 + 2047], "decode")                           # hh full: evicted token stays queued
    assert len(m.hh[0]) == 2048 and len(m.queue) == 1


def test_competition_queue_top_k_is_fifo_for_any_scores():
    """manager.py:686-715 with attention_competition_queue.py:34-107: the shared queue is
    sorted by score before up to (budget - |hh|) tokens are taken.  With layers updated in
    lockstep the queue holds at most the one token just evicted while a layer has room,
    so whatever the scores, every heavy-hitter zone is the first `budget` tokens its tail
    evicted, in order, and later ones stay queued (never attended).  This is the rule the
    device-side decode step (hkv_zone_step) applies."""
    import random

    class Scored(ManagerOracle):
        def _enqueue(self, layer, position, score):
            super()._enqueue(layer, position, rng.random())

    rng = random.Random(11)
    L, budget = 3, 5
    m = Scored(L, sink_tokens=4, hbm_budget_tokens=12)
    m.hh_budget = budget
    for layer in range(L):
        m.update(layer, range(20), "prefill")
    evicted = [[] for _ in range(L)]
    for p in range(20, 50):
        for layer in range(L):
            if len(m.tail[layer]) == m.tail_budget:
                evicted[layer].append(m.tail[layer][0])
            m.update(layer, [p], "decode", seq_offset=p)
    for layer in range(L):
        assert m.hh[layer] == evicted[layer][:budget], layer
    assert sorted(pos for _, pos, _ in m.queue.values()) == sorted(
        pos for layer in range(L) for pos in evicted[layer][budget:])


def test_decode_before_prefill_and_growing_tail():
    m = ManagerOracle(1, sink_tokens=4, hbm_budget_tokens=8)
    assert m.update(0, [0], "decode") == [0]
    assert m.update(0, [1], "decode") == [0, 1]


def test_cache_path_c_first_decode_skips_layer0():
    c = CacheOracle(2, sink_tokens=4, keep_tail=8)
    for layer in range(2):
        c.update(layer, list(range(32)))
    assert c.real_seq_len == 32
    # decode step 1: layer 0 runs before the swap count is refreshed -> no DRAM tokens
    o0 = c.update(0, [32])
    assert o0 == [0, 1, 2, 3, 29, 30, 31, 32, 28]
    assert c.swap_in_tokens == 24
    o1 = c.update(1, [32])
    assert o1 == list(range(4, 28)) + [0, 1, 2, 3, 29, 30, 31, 32, 28]
    # decode step 2: both layers prepend their DRAM chunk
    o0 = c.update(0, [33])
    assert o0[:24] == list(range(4, 28)) and o0[24:] == [0, 1, 2, 3, 30, 31, 32, 33, 28, 29]
    assert c.get_seq_length(0) == 10 + 24


def test_mask_sizes():
    c = CacheOracle(1, sink_tokens=4, keep_tail=8)
    assert c.get_mask_sizes(5) == (5, 0)          # nothing cached yet
    c.update(0, list(range(6)))                   # sink 4 + tail 2 (tail budget 4)
    assert c.get_mask_sizes(3) == (6 + 3, 0)      # prefill: physical + query
    assert c.get_mask_sizes(1) == (6 + 0 + 1, 0)  # tail still growing
    c.update(0, [6])
    c.update(0, [7])
    assert c.get_mask_sizes(1) == (8, 0)          # tail full: no +1


def test_max_hbm_tokens():
    assert ManagerOracle(1, 64, 8192).max_hbm_tokens() == 64 + 8192 + 4096
    assert ManagerOracle(1, 64, 4160).max_hbm_tokens() == 64 + 4160 + 2080
    assert ManagerOracle(1, 4, 8).max_hbm_tokens() == 4 + 8 + 2048


def test_chunk_selection_and_removal_hand_traces():
    """manager.py:966-978 and :265-278 on hand-built tables: default 1/(c+1) scores keep the
    first w chunks; equal scores keep insertion order (stable sort); the result is in
    eviction order; a removed chunk is no longer gathered or counted."""
    m = ManagerOracle(1, sink_tokens=4, hbm_budget_tokens=8)
    for c in range(4):
        m._evict(0, list(range(10 * c, 10 * c + 5)))
    assert m.select_chunks(0, 2) == ["l0_e0", "l0_e1"]
    assert m.select_chunks(0, 10) == ["l0_e0", "l0_e1", "l0_e2", "l0_e3"]
    assert m.select_chunks(0, 0) == []
    m.chunk_scores.update({"l0_e0": 0.1, "l0_e1": 0.9, "l0_e2": 0.5, "l0_e3": 0.9})
    # ranked: e1 (0.9), e3 (0.9, after e1 by insertion), e2, e0
    assert m.select_chunks(0, 2) == ["l0_e1", "l0_e3"]
    assert m.select_chunks(0, 3) == ["l0_e1", "l0_e2", "l0_e3"]
    assert m.remove_chunk("l0_e1") == [10, 11, 12, 13, 14]
    assert m.dram_positions(0) == [0, 1, 2, 3, 4, 20, 21, 22, 23, 24, 30, 31, 32, 33, 34]
    assert m.count_dram_tokens(0) == 3 * 5
    assert "l0_e1" in m.chunk_order and "l0_e1" in m.chunk_scores
    assert m.select_chunks(0, 2) == ["l0_e2", "l0_e3"]
