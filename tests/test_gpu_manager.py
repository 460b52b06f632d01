"""GPU parity of HeteroKVManager / FusedHeteroCache against the oracle's restatement of
the reference manager (oracle/manager.py): zone contents, eviction ranges, chunk keys,
Path C gather order (bit-exact), INT4 chunk codes (bit-exact), fused decode attention
(2e-3 max-abs against the float64 oracle)."""
import math

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import compressor as oc
from oracle.manager import CacheOracle, ManagerOracle

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _kv(seed, B, H, S, dtype=torch.float16):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn((B, H, S, 128), generator=g)
    k[..., [7, 31, 64, 100]] *= 8
    v = torch.randn((B, H, S, 128), generator=g)
    return k.to(dtype), v.to(dtype)


def _drive(mgr, orc, K, V, layers, chunks, decode_steps):
    """Prefill in `chunks` (sizes), then decode; check every returned tensor."""
    pos = 0
    for n in chunks + [1] * decode_steps:
        mode = "prefill" if n > 1 else "decode"
        for layer in range(layers):
            k = K[:, :, pos:pos + n].to(DEV)
            v = V[:, :, pos:pos + n].to(DEV)
            ok, ov = mgr.update(layer, k, v, mode=mode, seq_offset=pos)
            want = orc.update(layer, range(pos, pos + n), mode, seq_offset=pos)
            assert mgr.positions(layer) == orc.key_cache[layer]
            idx = torch.tensor(want, dtype=torch.long)
            assert torch.equal(ok.cpu(), K.index_select(2, idx)), (layer, pos, mode)
            assert torch.equal(ov.cpu(), V.index_select(2, idx)), (layer, pos, mode)
        pos += n
    return pos


@pytest.mark.parametrize("sink,budget,chunks,steps", [(4, 8, [32], 12), (16, 80, [64, 64, 64, 40], 40),
                                                      (64, 4160, [2048, 2048, 2048, 500], 3)])
def test_manager_index_parity(sink, budget, chunks, steps):
    print("case: manager sink=%d budget=%d chunks=%s decode=%d" % (sink, budget, chunks, steps), flush=True)
    from heterokv.manager import HeteroKVManager
    L, B, H = 2, 1, 2
    total = sum(chunks) + steps
    K, V = _kv(sink + budget, B, H, total)
    mgr = HeteroKVManager(L, sink_tokens=sink, hbm_budget_tokens=budget, device=DEV)
    orc = ManagerOracle(L, sink_tokens=sink, hbm_budget_tokens=budget)
    _drive(mgr, orc, K, V, L, chunks, steps)
    # DRAM chunks: same keys in the same order, same positions, bit-exact codes
    assert list(mgr._dram_table.keys()) == list(orc.dram.keys())
    assert mgr.count_dram_tokens(0) == orc.count_dram_tokens(0)
    assert mgr._chunk_attention_scores == orc.chunk_scores
    for key, posl in orc.dram.items():
        ent = mgr._dram_table[key]
        idx = torch.tensor(posl, dtype=torch.long)
        for name, X in (("k", K), ("v", V)):
            codes, scales, zps = oc.compress(X.index_select(2, idx).numpy(), 128)
            assert np.array_equal(ent[name + "_data"].cpu().numpy(), codes), key
            assert np.array_equal(ent[name + "_scales"].cpu().numpy(), scales), key
            assert np.array_equal(ent[name + "_zps"].cpu().numpy(), zps), key
    for layer in range(L):
        assert mgr.positions(layer, include_dram=True) == orc.dram_positions(layer) + orc.key_cache[layer]
    s = mgr.memory_summary()
    assert s["hbm_tokens"] == sum(len(orc.key_cache[l]) for l in range(L))
    assert s["dram_entries"] == len(orc.dram)
    assert s["max_hbm_tokens"] == orc.max_hbm_tokens()


def _oracle_attention(K, V, q, b, H, positions, dram):
    parts_k = [K[b].index_select(1, torch.tensor(positions)).double().numpy()]
    parts_v = [V[b].index_select(1, torch.tensor(positions)).double().numpy()]
    if dram:
        idx = torch.tensor(dram)
        kc, ks, kz = oc.compress(K[b].index_select(1, idx).numpy(), 128)
        vc, vs, vz = oc.compress(V[b].index_select(1, idx).numpy(), 128)
        parts_k.insert(0, oa.dequant_rows(kc, ks.reshape(H, -1), kz.reshape(H, -1)))
        parts_v.insert(0, oa.dequant_rows(vc, vs.reshape(H, -1), vz.reshape(H, -1)))
    return oa.attend(q[b].double().numpy(), np.concatenate(parts_k, 1), np.concatenate(parts_v, 1))


@pytest.mark.parametrize("hh_budget", [8, 24])
def test_heavy_hitter_zone_fills_then_drops_vs_oracle(hh_budget):
    """A small heavy-hitter budget in both the manager and the oracle (manager.py:686-750,
    attention_competition_queue.py:73-107): decode runs past the recent window filling,
    the heavy-hitter zone filling and the drops after it; at every step the zone contents
    match the oracle's key cache, and fused decode attention over them (and the INT4 tier)
    matches the float64 oracle."""
    print("case: heavy-hitter zone fill then drop, budget %d" % hh_budget, flush=True)
    from heterokv.manager import HeteroKVManager
    L, B, H, HQ = 2, 1, 2, 8
    sink, budget, chunks, steps = 16, 80, [64, 64, 64], 3 * hh_budget + 20
    K, V = _kv(40 + hh_budget, B, H, sum(chunks) + steps)
    mgr = HeteroKVManager(L, sink_tokens=sink, hbm_budget_tokens=budget, device=DEV)
    orc = ManagerOracle(L, sink_tokens=sink, hbm_budget_tokens=budget)
    mgr._heavyhitter_budget = hh_budget     # before any layer's zones are allocated
    orc.hh_budget = hh_budget
    g = torch.Generator().manual_seed(41)
    pos, checked = 0, 0
    for n in chunks + [1] * steps:
        mode = "prefill" if n > 1 else "decode"
        for layer in range(L):
            k, v = K[:, :, pos:pos + n].to(DEV), V[:, :, pos:pos + n].to(DEV)
            mgr.update(layer, k, v, mode=mode, seq_offset=pos)
            orc.update(layer, range(pos, pos + n), mode, seq_offset=pos)
            assert mgr.positions(layer) == orc.key_cache[layer], (layer, pos)
            if mode == "decode" and layer == 1 and pos % 5 == 0:
                q = (torch.randn((B, HQ, 1, 128), generator=g) / math.sqrt(128)).half()
                for include_dram in (False, True):
                    out = mgr.attend_decode(layer, q.to(DEV), include_dram=include_dram).float().cpu().numpy()
                    dram = orc.dram_positions(layer) if include_dram else []
                    ref = _oracle_attention(K, V, q, 0, H, orc.key_cache[layer], dram)
                    assert np.abs(out[0] - ref).max() <= 2e-3, (pos, include_dram)
                checked += 1
        pos += n
    for layer in range(L):
        st = mgr._layers[layer]
        assert st.hh_len == hh_budget                       # filled, then frozen
        assert len(orc.hh[layer]) == hh_budget
    assert checked >= 5
    mgr.check_errors()


def test_manager_decompress_dram_chunks_matches_path_c():
    print("case: decompress_dram_chunks", flush=True)
    from heterokv.manager import HeteroKVManager
    K, V = _kv(3, 1, 2, 200)
    mgr = HeteroKVManager(1, sink_tokens=8, hbm_budget_tokens=40, device=DEV)
    orc = ManagerOracle(1, sink_tokens=8, hbm_budget_tokens=40)
    _drive(mgr, orc, K, V, 1, [100, 100], 0)
    dk, dv, n = mgr.decompress_dram_chunks(0)
    posl = orc.dram_positions(0)
    assert n == len(posl)
    idx = torch.tensor(posl, dtype=torch.long)
    for got, X in ((dk, K), (dv, V)):
        c, s, z = oc.compress(X.index_select(2, idx).numpy(), 128)
        ref = oc.decompress(c, s, z, 128)
        assert np.array_equal(got.cpu().numpy().view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("include_dram", [True, False])
def test_attend_decode_vs_oracle(include_dram):
    print("case: attend_decode include_dram=%s" % include_dram, flush=True)
    from heterokv.manager import HeteroKVManager
    B, H, HQ = 2, 4, 16
    K, V = _kv(5, B, H, 3000)
    mgr = HeteroKVManager(1, sink_tokens=64, hbm_budget_tokens=576, device=DEV)
    orc = ManagerOracle(1, sink_tokens=64, hbm_budget_tokens=576)
    end = _drive(mgr, orc, K, V, 1, [1024, 1024, 900], 40)
    g = torch.Generator().manual_seed(6)
    q = (torch.randn((B, HQ, 1, 128), generator=g) / math.sqrt(128)).half()
    out = mgr.attend_decode(0, q.to(DEV), include_dram=include_dram).float().cpu().numpy()
    hbm = orc.key_cache[0]
    dram = orc.dram_positions(0) if include_dram else []
    for b in range(B):
        parts_k = [K[b].index_select(1, torch.tensor(hbm)).double().numpy()]
        parts_v = [V[b].index_select(1, torch.tensor(hbm)).double().numpy()]
        if dram:
            idx = torch.tensor(dram)
            kc, ks, kz = oc.compress(K[b].index_select(1, idx).numpy(), 128)
            vc, vs, vz = oc.compress(V[b].index_select(1, idx).numpy(), 128)
            parts_k.insert(0, oa.dequant_rows(kc, ks.reshape(H, -1), kz.reshape(H, -1)))
            parts_v.insert(0, oa.dequant_rows(vc, vs.reshape(H, -1), vz.reshape(H, -1)))
        ref = oa.attend(q[b].double().numpy(), np.concatenate(parts_k, 1), np.concatenate(parts_v, 1))
        err = np.abs(out[b] - ref).max()
        print("  b=%d max abs err %.3e (dram tokens %d, hbm tokens %d)" % (b, err, len(dram), len(hbm)), flush=True)
        assert err <= 2e-3
    assert end == 1024 + 1024 + 900 + 40


def test_bf16_inputs_round_trip():
    print("case: bf16 K/V", flush=True)
    from heterokv.manager import HeteroKVManager
    K, V = _kv(8, 1, 2, 90, dtype=torch.bfloat16)
    mgr = HeteroKVManager(1, sink_tokens=4, hbm_budget_tokens=20, device=DEV)
    orc = ManagerOracle(1, sink_tokens=4, hbm_budget_tokens=20)
    _drive(mgr, orc, K, V, 1, [60], 30)
    ent = mgr._dram_table["l0_e0"]
    idx = torch.tensor(orc.dram["l0_e0"])
    c, s, z = oc.compress(K.index_select(2, idx).view(torch.int16).numpy().view(np.uint16), 128)
    assert np.array_equal(ent["k_data"].cpu().numpy(), c) and np.array_equal(ent["k_scales"].cpu().numpy(), s)


def test_cpu_tensors_rejected():
    from heterokv import HeteroKVError
    from heterokv.manager import HeteroKVManager
    mgr = HeteroKVManager(1, device=DEV)
    with pytest.raises(HeteroKVError):
        mgr.update(0, torch.zeros(1, 2, 4, 128), torch.zeros(1, 2, 4, 128))


def test_cache_path_c_semantics_materialized_vs_fused():
    print("case: FusedHeteroCache Path C (materialized) vs fused decode", flush=True)
    from heterokv.engine_wrapper import FusedHeteroCache
    L, B, H, HQ = 2, 1, 2, 8
    K, V = _kv(11, B, H, 400)
    # the reference's length arithmetic, which the oracle restates
    ref_cache = FusedHeteroCache(num_layers=L, sink_tokens=8, keep_tail=40, device=DEV, fused_decode=False,
                                 reference_lengths=True)
    fus_cache = FusedHeteroCache(num_layers=L, sink_tokens=8, keep_tail=40, device=DEV, fused_decode=True,
                                 reference_lengths=True)
    orc = CacheOracle(L, sink_tokens=8, keep_tail=40)
    g = torch.Generator().manual_seed(12)
    pos = 0
    for n in [128, 128, 100] + [1] * 6:
        for layer in range(L):
            k, v = K[:, :, pos:pos + n].to(DEV), V[:, :, pos:pos + n].to(DEV)
            want = orc.update(layer, list(range(pos, pos + n)))
            rk, rv = ref_cache.update(k.clone(), v.clone(), layer)
            assert rk.shape[2] == len(want)
            fk, fv = fus_cache.update(k.clone(), v.clone(), layer)
            assert fus_cache.get_seq_length(layer) == orc.get_seq_length(layer) == ref_cache.get_seq_length(layer)
            assert fus_cache.get_mask_sizes(1, layer) == orc.get_mask_sizes(1, layer)
            if n == 1:
                q = (torch.randn((B, HQ, 1, 128), generator=g) / math.sqrt(128)).half().to(DEV)
                # materialized Path C through plain float32 attention vs the fused route
                rep = HQ // H
                kk = rk.float().repeat_interleave(rep, dim=1)
                vv = rv.float().repeat_interleave(rep, dim=1)
                p = torch.softmax((q.float() @ kk.transpose(-1, -2)) / math.sqrt(128), dim=-1)
                ref = (p @ vv).cpu().numpy()
                route = getattr(fk, "_hkv_route", None)
                assert route is not None
                got = fus_cache._manager.attend_decode(layer, q, include_dram=route[2]).float().cpu().numpy()
                assert np.abs(got - ref).max() <= 2e-3
        pos += n
    assert fus_cache.seen_tokens == pos == orc.real_seq_len


def test_tiny_qwen2_end_to_end_with_registered_attention():
    print("case: tiny random Qwen2 through transformers", flush=True)
    from transformers import Qwen2Config, Qwen2ForCausalLM
    from heterokv.engine_wrapper import ChunkedPrefillEngine, FusedHeteroCache, register_attention
    name = register_attention()
    torch.manual_seed(0)
    cfg = Qwen2Config(vocab_size=512, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=4096,
                      attn_implementation=name)
    model = Qwen2ForCausalLM(cfg).to(DEV, torch.float16).eval()
    ids = torch.randint(0, 512, (1, 300), generator=torch.Generator().manual_seed(1)).to(DEV)
    cache_f = FusedHeteroCache(num_layers=2, sink_tokens=16, keep_tail=80, chunk_size=64, device=DEV)
    cache_r = FusedHeteroCache(num_layers=2, sink_tokens=16, keep_tail=80, chunk_size=64, device=DEV,
                               fused_decode=False)
    with torch.inference_mode():
        ChunkedPrefillEngine(model, cache_f, chunk_size=64).prefill(ids)
        ChunkedPrefillEngine(model, cache_r, chunk_size=64).prefill(ids)
        assert len(cache_f.dram_table) == len(cache_r.dram_table) > 0
        tok = ids[:, -1:]
        for step in range(4):
            p = torch.tensor([[300 + step]], device=DEV)
            lf = model(input_ids=tok, past_key_values=cache_f, position_ids=p, use_cache=True).logits
            lr = model(input_ids=tok, past_key_values=cache_r, position_ids=p, use_cache=True).logits
            assert torch.isfinite(lf).all()
            err = (lf.float() - lr.float()).abs().max().item()
            print("  step %d max |logit diff| %.3e" % (step, err), flush=True)
            assert err < 5e-2
            tok = lf[:, -1:].argmax(-1)


@pytest.mark.parametrize("adaptive", [False, True])
def test_tiny_qwen2_fused_prefill_matches_sdpa(adaptive):
    print("case: tiny Qwen2, fused prefill vs SDPA prefill, adaptive=%s" % adaptive, flush=True)
    from transformers import Qwen2Config, Qwen2ForCausalLM
    from heterokv.engine_wrapper import ChunkedPrefillEngine, FusedHeteroCache, register_attention
    name = register_attention()
    torch.manual_seed(0)
    cfg = Qwen2Config(vocab_size=512, hidden_size=448, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=7, num_key_value_heads=1, head_dim=128, max_position_embeddings=4096,
                      attn_implementation=name)
    model = Qwen2ForCausalLM(cfg).to(DEV, torch.float16).eval()
    ids = torch.randint(0, 512, (1, 352), generator=torch.Generator().manual_seed(1)).to(DEV)
    kw = dict(num_layers=2, sink_tokens=16, keep_tail=80, chunk_size=64, device=DEV, adaptive_self_healing=adaptive)
    cache_f = FusedHeteroCache(fused_prefill=True, **kw)
    cache_s = FusedHeteroCache(**kw)
    with torch.inference_mode():
        lf = ChunkedPrefillEngine(model, cache_f, chunk_size=64).prefill(ids).logits
        ls = ChunkedPrefillEngine(model, cache_s, chunk_size=64).prefill(ids).logits
        err = (lf.float() - ls.float()).abs().max().item()
        print("  last chunk max |logit diff| %.3e" % err, flush=True)
        assert err < 5e-2
        tok = ids[:, -1:]
        for step in range(3):
            p = torch.tensor([[352 + step]], device=DEV)
            a = model(input_ids=tok, past_key_values=cache_f, position_ids=p, use_cache=True).logits
            b = model(input_ids=tok, past_key_values=cache_s, position_ids=p, use_cache=True).logits
            err = (a.float() - b.float()).abs().max().item()
            print("  decode step %d max |logit diff| %.3e" % (step, err), flush=True)
            assert err < 5e-2
            tok = a[:, -1:].argmax(-1)
    if adaptive:
        assert cache_f._manager.retrieval_window == "adaptive"
