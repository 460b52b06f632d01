"""Device-stepped decode (hkv_zone_step) and graph-captured decode (DecodeGraph).

The zone decision of a decode step (manager.py:588-674: append to the recent window
while it has room, else move its oldest token into the heavy-hitter zone while that
has room, else drop it) taken on the GPU must leave the zones, the positions and the
lengths exactly as the host-stepped manager leaves them, across the window-full and
heavy-hitter-full transitions; attention over the device lengths must agree with the
host-stepped launch and with an fp32 reference on the same zones.  A decode step of
a tiny Qwen2 captured once and replayed must give the eager step's logits."""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _kv(seed, B, H, S):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn((B, H, S, 128), generator=g).half(), torch.randn((B, H, S, 128), generator=g).half())


def _ref_attention(q, k, v):
    """fp32 softmax(q k^T / sqrt(128)) v over every token, GQA by head groups."""
    B, Hq = q.shape[:2]
    Hkv = k.shape[1]
    kk = k.float().repeat_interleave(Hq // Hkv, dim=1)
    vv = v.float().repeat_interleave(Hq // Hkv, dim=1)
    s = (q.float().reshape(B, Hq, 1, 128) @ kk.transpose(-1, -2).contiguous()) / math.sqrt(128)
    return (torch.softmax(s, dim=-1) @ vv).reshape(B, Hq, 128)


@pytest.mark.parametrize("prompt,hh_budget,steps", [(30, 24, 70), (200, 24, 60), (200, 0, 40)])
def test_device_step_matches_host_step(prompt, hh_budget, steps):
    print("case: device-stepped decode prompt=%d hh_budget=%d steps=%d" % (prompt, hh_budget, steps), flush=True)
    from heterokv.manager import HeteroKVManager
    L, B, H, HQ, sink, budget = 2, 2, 2, 8, 16, 48
    K, V = _kv(prompt + steps, B, H, prompt + steps)
    mgrs = []
    for dev_mode in (False, True):
        m = HeteroKVManager(L, sink_tokens=sink, hbm_budget_tokens=budget, device=DEV)
        m._heavyhitter_budget = hh_budget
        m.deterministic_decode = True
        for li in range(L):
            m.update(li, K[:, :, :prompt].to(DEV), V[:, :, :prompt].to(DEV), mode="prefill", seq_offset=0)
        if dev_mode:
            m.enable_device_decode(True)
        mgrs.append(m)
    host, dev = mgrs
    queued0 = dev._queued_tokens
    g = torch.Generator().manual_seed(7)
    worst = 0.0
    for step in range(steps):
        pos = prompt + step
        for li in range(L):
            k, v = K[:, :, pos:pos + 1].to(DEV), V[:, :, pos:pos + 1].to(DEV)
            for m in mgrs:
                m.update(li, k, v, mode="decode", seq_offset=pos, materialize=False)
            q = (torch.randn((B, HQ, 1, 128), generator=g)).half().to(DEV)
            oh = host.attend_decode(li, q, include_dram=True).float()
            od = dev.attend_decode(li, q, include_dram=True).float()
            worst = max(worst, (oh - od).abs().max().item())
            assert dev.positions(li, include_dram=True) == host.positions(li, include_dram=True)
            if li == 0 and step % 10 == 0:
                # fp32 reference over the HBM zones alone
                kh, vh = dev.get_hbm_kv(li)
                want = _ref_attention(q, kh, vh)
                got = dev.attend_decode(li, q, include_dram=False).float().reshape(B, HQ, 128)
                err = (got - want).abs().max().item()
                assert err <= 2e-3, (step, err)
    print("  max |device - host| %.2e" % worst, flush=True)
    assert worst <= 2e-3
    torch.cuda.synchronize()
    dropped = 0
    for li in range(L):
        st_h, st_d = host._layers[li], dev._layers[li]
        state = st_d.dev_state.cpu().tolist()
        assert state[:3] == [st_d.tail_head, st_d.tail_len, st_d.hh_len]
        assert [st_d.tail_head, st_d.tail_len, st_d.hh_len] == [st_h.tail_head, st_h.tail_len, st_h.hh_len]
        assert st_d.dev_tail_lens.cpu().tolist() == [st_h.tail_len] * B
        assert st_d.dev_hh_lens.cpu().tolist() == [st_h.hh_len] * B
        dropped += state[3]
        for a, b in zip(dev.get_hbm_kv(li), host.get_hbm_kv(li)):
            assert torch.equal(a, b), li
    assert dropped == dev._queued_tokens - queued0 == host._queued_tokens - queued0
    # every case runs past both transitions: the window and the heavy-hitter zone full
    assert st_h.tail_len == budget - sink and st_h.hh_len == hh_budget and dropped > 0


def test_zone_step_rejects_bad_arguments():
    print("case: hkv_zone_step argument checks", flush=True)
    from heterokv import ops
    from heterokv._lib import HeteroKVError
    tail = ops.F16Zone(1, 2, 32, DEV)
    hh = ops.F16Zone(1, 2, 16, DEV)
    k = torch.zeros((1, 2, 1, 128), dtype=torch.float16, device=DEV)
    state = torch.zeros(4, dtype=torch.int32, device=DEV)
    with pytest.raises(HeteroKVError):
        tail.step(hh, k, k, 33, 8, state)       # ring beyond the zone
    with pytest.raises(HeteroKVError):
        tail.step(hh, k, k, 32, 17, state)      # heavy-hitter budget beyond its zone
    with pytest.raises(HeteroKVError):
        tail.step(hh, k.float(), k.float(), 32, 8, state)


def _tiny_qwen2():
    from transformers import Qwen2Config, Qwen2ForCausalLM
    from heterokv.engine_wrapper import register_attention
    name = register_attention()
    torch.manual_seed(0)
    cfg = Qwen2Config(vocab_size=512, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=4096,
                      attn_implementation=name)
    return Qwen2ForCausalLM(cfg).to(DEV, torch.float16).eval()


@pytest.mark.parametrize("prompt,steps", [(300, 16), (40, 60)])
def test_decode_graph_matches_eager(prompt, steps):
    """Graph replays cross the recent-window-full (prompt 40: window 64 fills at the 40th
    step) and heavy-hitter-full (budget 8) transitions; the INT4 tier (prompt 300) joins
    every replay."""
    print("case: DecodeGraph tiny Qwen2 prompt=%d steps=%d" % (prompt, steps), flush=True)
    from heterokv.engine_wrapper import ChunkedPrefillEngine, DecodeGraph, FusedHeteroCache
    model = _tiny_qwen2()
    ids = torch.randint(0, 512, (1, prompt), generator=torch.Generator().manual_seed(1)).to(DEV)
    caches = []
    for _ in range(2):
        c = FusedHeteroCache(num_layers=2, sink_tokens=16, keep_tail=80, chunk_size=64, device=DEV)
        c._ensure_manager(0)._heavyhitter_budget = 8
        c._manager.deterministic_decode = True
        caches.append(c)
    cache_e, cache_g = caches
    runner = DecodeGraph(model, cache_g)
    with torch.inference_mode():
        for c in caches:
            ChunkedPrefillEngine(model, c, chunk_size=64).prefill(ids)
        assert (len(cache_e.dram_table) > 0) == (prompt > 64)
        tok = ids[:, -1:]
        worst = 0.0
        for step in range(steps):
            p = torch.tensor([[prompt + step]], device=DEV)
            le = model(input_ids=tok, past_key_values=cache_e, position_ids=p, use_cache=True).logits
            lg = runner.step(tok, p)
            assert torch.isfinite(lg).all()
            err = (le.float() - lg.float()).abs().max().item()
            worst = max(worst, err)
            assert err < 5e-2, (step, err)
            tok = le[:, -1:].argmax(-1)
    print("  max |logit diff| %.3e over %d steps (%d replays)" % (worst, steps, steps - 1), flush=True)
    assert runner.graph is not None
    me, mg = cache_e._manager, cache_g._manager
    assert cache_g.real_seq_len == cache_e.real_seq_len == prompt + steps
    assert cache_g._swap_in_tokens == cache_e._swap_in_tokens
    torch.cuda.synchronize()
    for li in range(2):
        assert mg.positions(li, include_dram=True) == me.positions(li, include_dram=True)
        st = mg._layers[li]
        assert st.dev_state.cpu().tolist()[:3] == [st.tail_head, st.tail_len, st.hh_len]
    assert mg._layers[0].hh_len == 8
    # layer 0's K/V depend only on the tokens: the zones hold the same bits
    for a, b in zip(mg.get_hbm_kv(0), me.get_hbm_kv(0)):
        assert torch.equal(a, b)
    runner.close()
    assert not mg.device_decode


def test_decode_graph_rejects_host_work():
    print("case: DecodeGraph argument checks", flush=True)
    from heterokv._lib import HeteroKVError
    from heterokv.engine_wrapper import DecodeGraph, FusedHeteroCache
    with pytest.raises(HeteroKVError):
        DecodeGraph(None, FusedHeteroCache(num_layers=2, device=DEV, fused_decode=False))
    with pytest.raises(HeteroKVError):
        DecodeGraph(None, FusedHeteroCache(num_layers=2, device=DEV, track_attention=True))
    runner = DecodeGraph(None, FusedHeteroCache(num_layers=2, device=DEV))
    with pytest.raises(HeteroKVError):
        runner.step(None, None)      # nothing prefilled yet


def test_decode_graph_reports_replay_errors():
    """A device error raised by a replayed step (here a block-table entry outside the pool,
    which the decode kernel replaces by a valid record and reports as
    HKV_ERR_BIT_BLOCK_ID) reaches the caller at the next step, and the graph is dropped so
    that a later step captures again."""
    print("case: DecodeGraph error word after a replay", flush=True)
    from heterokv._lib import HeteroKVError
    from heterokv.engine_wrapper import ChunkedPrefillEngine, DecodeGraph, FusedHeteroCache
    model = _tiny_qwen2()
    ids = torch.randint(0, 512, (1, 300), generator=torch.Generator().manual_seed(2)).to(DEV)
    cache = FusedHeteroCache(num_layers=2, sink_tokens=16, keep_tail=80, chunk_size=64, device=DEV)
    runner = DecodeGraph(model, cache)
    with torch.inference_mode():
        ChunkedPrefillEngine(model, cache, chunk_size=64).prefill(ids)
        tok = ids[:, -1:]
        for step in range(3):                   # eager, captured, replayed
            runner.step(tok, torch.tensor([[300 + step]], device=DEV))
        torch.cuda.synchronize()
        assert runner.graph is not None
        st = cache._manager._layers[0]
        assert st.bt is not None and st.int4_len > 0
        good = st.bt[0, 0].item()
        st.bt[0, 0] = 1 << 30                   # outside the pool: reported, not read
        runner.step(tok, torch.tensor([[303]], device=DEV))   # this replay sets the bit
        torch.cuda.synchronize()
        st.bt[0, 0] = good
        with pytest.raises(HeteroKVError, match="block table"):
            runner.step(tok, torch.tensor([[304]], device=DEV))
        assert runner.graph is None
        out = runner.step(tok, torch.tensor([[304]], device=DEV))   # captures again
        assert torch.isfinite(out).all() and runner.graph is not None
    runner.close()


@pytest.mark.parametrize("window", [None, 2, "switch"])
def test_decode_graph_with_host_tier(window):
    """75% of the INT4 blocks in pinned host memory: graph replays (the host runs' copies
    captured on a forked stream) give the eager steps' logits, with full retrieval, with a
    two-chunk window, and across a window change (the graph is captured again); after
    close() the native prefetch schedule serves an eager step again."""
    print("case: DecodeGraph with a host tier, window=%s" % window, flush=True)
    from heterokv.engine_wrapper import ChunkedPrefillEngine, DecodeGraph, FusedHeteroCache
    model = _tiny_qwen2()
    prompt, steps = 700, 12
    ids = torch.randint(0, 512, (1, prompt), generator=torch.Generator().manual_seed(3)).to(DEV)
    caches = []
    for _ in range(2):
        c = FusedHeteroCache(num_layers=2, sink_tokens=16, keep_tail=80, chunk_size=64, device=DEV)
        c._ensure_manager(0)._heavyhitter_budget = 8
        c._manager.deterministic_decode = True
        caches.append(c)
    cache_e, cache_g = caches
    runner = DecodeGraph(model, cache_g)
    graphs = set()
    with torch.inference_mode():
        for c in caches:
            ChunkedPrefillEngine(model, c, chunk_size=64).prefill(ids)
            assert c.offload_to_host(0.75, seed=0) > 0
            c.retrieval_window = 2 if window == "switch" else window
        tok = ids[:, -1:]
        worst = 0.0
        for step in range(steps):
            if window == "switch" and step == steps // 2:
                for c in caches:
                    c.retrieval_window = 3
            p = torch.tensor([[prompt + step]], device=DEV)
            le = model(input_ids=tok, past_key_values=cache_e, position_ids=p, use_cache=True).logits
            lg = runner.step(tok, p)
            assert torch.isfinite(lg).all()
            err = (le.float() - lg.float()).abs().max().item()
            worst = max(worst, err)
            assert err < 5e-2, (step, err)
            if runner.graph is not None:
                graphs.add(id(runner.graph))
            tok = le[:, -1:].argmax(-1)
        print("  max |logit diff| %.3e over %d steps, %d graph(s)" % (worst, steps, len(graphs)), flush=True)
        assert len(graphs) == (2 if window == "switch" else 1)
        runner.close()
        p = torch.tensor([[prompt + steps]], device=DEV)
        le = model(input_ids=tok, past_key_values=cache_e, position_ids=p, use_cache=True).logits
        lg = model(input_ids=tok, past_key_values=cache_g, position_ids=p, use_cache=True).logits
        assert (le.float() - lg.float()).abs().max().item() < 5e-2
    cache_e.check_errors()
    cache_g.check_errors()
