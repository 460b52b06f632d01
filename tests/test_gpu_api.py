"""GPU checks of the drop-in surface: device errors surface as HeteroKVError, bf16
activations (checked narrowing), the vectorized zone writes, decode workspaces reused
across geometries, the reference's per-chunk and windowed entry points
(manager.py:233-350, 823-1056; engine_wrapper.py:332-355) against the oracle, and exact
sequence lengths through transformers' generate()."""
import math

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import compressor as oc
from oracle import pool_format as pf
from oracle.manager import ManagerOracle

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _kv(seed, B, H, S, dtype=torch.float16):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn((B, H, S, 128), generator=g)
    k[..., [7, 31, 64, 100]] *= 8
    v = torch.randn((B, H, S, 128), generator=g)
    return k.to(dtype), v.to(dtype)


def _drive(mgr, orc, K, V, layers, chunks, decode_steps=0):
    pos = 0
    for n in chunks + [1] * decode_steps:
        mode = "prefill" if n > 1 else "decode"
        for layer in range(layers):
            mgr.update(layer, K[:, :, pos:pos + n].to(DEV), V[:, :, pos:pos + n].to(DEV), mode=mode, seq_offset=pos)
            orc.update(layer, range(pos, pos + n), mode, seq_offset=pos)
        pos += n
    return pos


def _oracle_codes(X, posl):
    return oc.compress(X.index_select(2, torch.tensor(posl, dtype=torch.long)).numpy(), 128)


# ----------------------------------------------------------------------------- device errors
def test_bad_block_id_through_attend_decode_raises():
    print("case: corrupted block table through HeteroKVManager.attend_decode", flush=True)
    from heterokv import HeteroKVError
    from heterokv.manager import HeteroKVManager
    K, V = _kv(1, 1, 2, 402)
    mgr = HeteroKVManager(1, sink_tokens=16, hbm_budget_tokens=80, device=DEV)
    orc = ManagerOracle(1, sink_tokens=16, hbm_budget_tokens=80)
    _drive(mgr, orc, K, V, 1, [200, 200], 2)
    q = torch.randn((1, 8, 1, 128), generator=torch.Generator().manual_seed(2)).half().to(DEV)
    mgr.attend_decode(0, q)
    mgr.check_errors()                                   # a clean step: nothing reported
    st = mgr._layers[0]
    st.bt[0, 3] = st.pool.num_blocks + 1000              # an id outside the pool
    mgr.attend_decode(0, q)                              # the launch itself does not block
    torch.cuda.synchronize()
    with pytest.raises(HeteroKVError, match="block table"):
        mgr.attend_decode(0, q)                          # the next step's first layer reports it
    mgr.check_errors()                                   # the word was cleared with the report
    mgr.attend_decode(0, q)
    with pytest.raises(HeteroKVError, match="block table"):
        mgr.check_errors()


def test_bf16_out_of_fp16_range_raises():
    print("case: bf16 K beyond the fp16 range", flush=True)
    from heterokv import HeteroKVError
    from heterokv.manager import HeteroKVManager
    K, V = _kv(3, 1, 2, 64, dtype=torch.bfloat16)
    K[0, 1, 50, 9] = 1.0e5                              # lands in the tail zone (fp16)
    mgr = HeteroKVManager(1, sink_tokens=16, hbm_budget_tokens=80, device=DEV)
    mgr.update(0, K.to(DEV), V.to(DEV), mode="prefill")
    with pytest.raises(HeteroKVError, match="bf16"):
        mgr.check_errors()
    K2, V2 = _kv(4, 1, 2, 64, dtype=torch.bfloat16)
    mgr2 = HeteroKVManager(1, sink_tokens=16, hbm_budget_tokens=80, device=DEV)
    mgr2.update(0, (K2 * 100).to(DEV), V2.to(DEV), mode="prefill")   # large but in range: exact
    mgr2.check_errors()
    kk, _ = mgr2.get_hbm_kv(0)
    assert torch.equal(kk.cpu().to(torch.bfloat16), (K2 * 100)[:, :, :kk.shape[2]])


# ----------------------------------------------------------------------------- zone writes
@pytest.mark.parametrize("T,start,ring", [(64, 0, 0), (48, 16, 0), (37, 5, 0), (50, 40, 64), (16, 48, 64),
                                          (100, 3, 100)])
def test_zone_write_layouts(T, start, ring):
    """Whole-tile (LDS transpose) and per-token paths, ring wrap, bf16 sources."""
    print("case: zone write T=%d start=%d ring=%d" % (T, start, ring), flush=True)
    from heterokv import ops
    H = 3
    cap = max(ring, 128)
    for dtype in (torch.float16, torch.bfloat16):
        k, v = _kv(T + start, 2, H, T, dtype=dtype)
        z = ops.F16Zone(2, H, cap, DEV)
        err = ops.ErrorWord(DEV)
        z.write(k.to(DEV), v.to(DEV), start, ring=ring, err=err)
        rk, rv = z.read(cap)
        slots = [((start + t) % ring) if ring else start + t for t in range(T)]
        want_k, want_v = k.to(torch.float16), v.to(torch.float16)   # bf16 -> fp16 is exact here
        assert torch.equal(rk[:, :, slots].cpu(), want_k) and torch.equal(rv[:, :, slots].cpu(), want_v)
        for b in range(2):
            for h in range(H):
                for t0 in range(0, cap, 16):
                    sl = list(range(t0, t0 + 16))
                    if all(s in slots for s in sl):
                        tile = z.v[b, h, t0 // 16].cpu().reshape(4, 16, 8, 4).numpy()
                        assert np.array_equal(tile, pf.v_tile(rv[b, h, t0:t0 + 16].cpu().numpy()))
        err.check()


@pytest.mark.parametrize("src,dst,n", [(0, 16, 32), (16, 0, 16), (3, 40, 21), (20, 7, 1), (0, 0, 48), (32, 64, 17)])
def test_zone_copy_and_read(src, dst, n):
    """hkv_zone_copy (whole-tile 16-byte path for tile-aligned ranges, per-element V moves
    otherwise) and hkv_zone_read of every length (partial last tile) against the slots
    written through hkv_zone_write; the copy leaves every other destination slot alone."""
    print("case: zone copy %d -> %d x %d, reads" % (src, dst, n), flush=True)
    from heterokv import ops
    B, H, cap = 2, 3, 96
    k, v = _kv(7 + src + n, B, H, cap)
    k2, v2 = _kv(8 + dst + n, B, H, cap)
    a = ops.F16Zone(B, H, cap, DEV)
    c = ops.F16Zone(B, H, cap, DEV)
    a.write(k.to(DEV), v.to(DEV), 0)
    c.write(k2.to(DEV), v2.to(DEV), 0)
    for m in (1, 15, 16, 17, 95, 96):
        rk, rv = a.read(m)
        assert torch.equal(rk.cpu(), k[:, :, :m]) and torch.equal(rv.cpu(), v[:, :, :m]), m
    a.copy_to(c, src, dst, n)
    rk, rv = c.read(cap)
    want_k, want_v = k2.clone(), v2.clone()
    want_k[:, :, dst:dst + n] = k[:, :, src:src + n]
    want_v[:, :, dst:dst + n] = v[:, :, src:src + n]
    assert torch.equal(rk.cpu(), want_k) and torch.equal(rv.cpu(), want_v)


def test_zone_write_bf16_conversion_is_exact():
    """bf16 -> fp16 narrowing in the zone kernels equals numpy's round-to-nearest-even
    conversion for every bf16 pattern of magnitude below the fp16 range."""
    print("case: bf16 -> fp16 narrowing, all patterns", flush=True)
    from heterokv import ops
    bits = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    f = oc.bf16_bits_to_f32(bits)
    keep = np.isfinite(f) & (np.abs(f) < 65504.0)
    vals = bits[keep]
    n = (len(vals) + 127) // 128 * 128
    vals = np.concatenate([vals, np.zeros(n - len(vals), dtype=np.uint16)])
    x = torch.from_numpy(vals.view(np.int16)).view(torch.bfloat16).reshape(1, 1, -1, 128)
    T = x.shape[2]
    z = ops.F16Zone(1, 1, (T + 15) // 16 * 16, DEV)
    err = ops.ErrorWord(DEV)
    z.write(x.to(DEV), x.to(DEV), 0, err=err)
    rk, rv = z.read(T)
    want = oc.bf16_bits_to_f32(vals).astype(np.float16).view(np.uint16)
    assert np.array_equal(rk.cpu().numpy().reshape(-1).view(np.uint16), want)
    assert np.array_equal(rv.cpu().numpy().reshape(-1).view(np.uint16), want)
    err.check()


# ----------------------------------------------------------------------------- decode / prefill dtypes
def _decode_case(seed, B, Hq, Hkv, sink, mid, rec, dtype):
    from heterokv import ops
    K, V = _kv(seed, B, Hkv, sink + mid + rec, dtype=dtype)
    g = torch.Generator().manual_seed(seed + 1)
    q = (torch.randn((B, Hq, 128), generator=g) / math.sqrt(128)).to(dtype)
    zs = ops.F16Zone(B, Hkv, max(sink, 16), DEV)
    zs.write(K[:, :, :sink].to(DEV), V[:, :, :sink].to(DEV), 0)
    zr = ops.F16Zone(B, Hkv, rec, DEV)
    zr.write(K[:, :, sink + mid:].to(DEV), V[:, :, sink + mid:].to(DEV), 0)
    nb = (mid + 15) // 16
    pool = ops.Int4Pool(B * nb, Hkv, DEV)
    bt = torch.arange(B * nb, dtype=torch.int32).reshape(B, nb)
    ops.pack_tokens(pool, K[:, :, sink:sink + mid].to(DEV), V[:, :, sink:sink + mid].to(DEV), [0] * B, bt)
    pool.check_errors()
    ref = []
    for b in range(B):
        Kb = K[b].float().numpy() if dtype == torch.float16 else oc.bf16_bits_to_f32(K[b].view(torch.int16).numpy().view(np.uint16))
        Vb = V[b].float().numpy() if dtype == torch.float16 else oc.bf16_bits_to_f32(V[b].view(torch.int16).numpy().view(np.uint16))
        kx = K[b:b + 1, :, sink:sink + mid]
        vx = V[b:b + 1, :, sink:sink + mid]
        to_in = (lambda t: t.numpy()) if dtype == torch.float16 else (lambda t: t.view(torch.int16).numpy().view(np.uint16))
        kc, ks, kz = oc.compress(to_in(kx), 128)
        vc, vs, vz = oc.compress(to_in(vx), 128)
        kk = np.concatenate([Kb[:, :sink].astype(np.float64), oa.dequant_rows(kc[0], ks.reshape(Hkv, -1), kz.reshape(Hkv, -1)),
                             Kb[:, sink + mid:].astype(np.float64)], 1)
        vv = np.concatenate([Vb[:, :sink].astype(np.float64), oa.dequant_rows(vc[0], vs.reshape(Hkv, -1), vz.reshape(Hkv, -1)),
                             Vb[:, sink + mid:].astype(np.float64)], 1)
        qb = q[b].float().numpy().astype(np.float64)
        ref.append(oa.attend(qb[:, None], kk, vv)[:, 0])
    zones = [(zs, None, sink), (zr, None, rec)]
    return q, zones, pool, bt, mid, np.stack(ref)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_dtypes(dtype):
    print("case: decode q/zones %s, out fp16 and q dtype" % dtype, flush=True)
    from heterokv import ops
    q, zones, pool, bt, mid, ref = _decode_case(21, 2, 28, 4, 64, 1500, 700, dtype)
    ws = ops.DecodeWorkspace(DEV)
    out16 = ops.decode_attention(q.to(DEV), zones, pool, bt.to(DEV), int4_max_len=mid, workspace=ws,
                                 out_dtype=torch.float16)
    outq = ops.decode_attention(q.to(DEV), zones, pool, bt.to(DEV), int4_max_len=mid, workspace=ws,
                                deterministic=True)
    out16d = ops.decode_attention(q.to(DEV), zones, pool, bt.to(DEV), int4_max_len=mid, workspace=ws,
                                  deterministic=True, out_dtype=torch.float16)
    torch.cuda.synchronize()
    assert ws.error_flag() == 0
    err = np.abs(out16.float().cpu().numpy() - ref).max()
    print("  max abs err (fp16 out) %.3e" % err, flush=True)
    assert err <= 2e-3
    assert outq.dtype == dtype
    # the q-dtype output is the same fp32 result rounded once: bf16 within half an ulp of it
    a = outq.float().cpu()
    b = out16d.float().cpu()
    assert torch.allclose(a, b.to(dtype).float(), atol=2e-3 if dtype == torch.float16 else 1.6e-2, rtol=0)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_prefill_dtypes(dtype):
    print("case: prefill q/chunk %s" % dtype, flush=True)
    from heterokv import ops
    B, Hq, Hkv, S, P = 1, 8, 2, 96, 40
    K, V = _kv(31, B, Hkv, P + S, dtype=dtype)
    g = torch.Generator().manual_seed(32)
    q = (torch.randn((B, Hq, S, 128), generator=g) / math.sqrt(128)).to(dtype)
    z = ops.F16Zone(B, Hkv, 48, DEV)
    z.write(K[:, :, :P].to(DEV), V[:, :, :P].to(DEV), 0)
    err = ops.ErrorWord(DEV)
    out = ops.prefill_attention(q.to(DEV), zones=[(z, None, P)], chunk_k=K[:, :, P:].to(DEV),
                                chunk_v=V[:, :, P:].to(DEV), err=err, out_dtype=torch.float16)
    err.check()
    f = lambda t: t.float().numpy().astype(np.float64)
    rep = Hq // Hkv
    Kf, Vf, qf = f(K[0]), f(V[0]), f(q[0])
    ref = np.zeros((Hq, S, 128))
    for h in range(Hq):
        kh, vh = Kf[h // rep], Vf[h // rep]
        for i in range(S):
            idx = list(range(P)) + list(range(P, P + i + 1))
            ref[h, i] = oa.attend(qf[h, i][None, None], kh[None, idx], vh[None, idx])[0, 0]
    e = np.abs(out[0].float().cpu().numpy() - ref).max()
    print("  max abs err %.3e" % e, flush=True)
    assert e <= 2e-3
    outq = ops.prefill_attention(q.to(DEV), zones=[(z, None, P)], chunk_k=K[:, :, P:].to(DEV),
                                 chunk_v=V[:, :, P:].to(DEV))
    assert outq.dtype == dtype


def test_decode_workspace_reused_across_geometries():
    """One workspace (sized by the first, larger geometry, so every later call reuses the
    same buffer): 32 pairs at 4K, 8 pairs at 32K, 32 again, 8 again; every output equals a
    fresh workspace's (the ticket area is cleared when the pair count changes)."""
    print("case: decode workspace reuse BH 32 -> 8 -> 32 -> 8", flush=True)
    from heterokv import ops
    big = _decode_case(41, 1, 32, 8, 64, 28608, 4096, torch.float16)
    small = _decode_case(42, 4, 32, 8, 64, 3000, 1000, torch.float16)
    shared = ops.DecodeWorkspace(DEV)
    for q, zones, pool, bt, mid, ref in (small, big, small, big):
        got = ops.decode_attention(q.to(DEV), zones, pool, bt.to(DEV), int4_max_len=mid, workspace=shared,
                                   deterministic=True)
        fresh = ops.decode_attention(q.to(DEV), zones, pool, bt.to(DEV), int4_max_len=mid,
                                     workspace=ops.DecodeWorkspace(DEV), deterministic=True)
        torch.cuda.synchronize()
        assert torch.equal(got, fresh)
        assert np.abs(got.float().cpu().numpy() - ref).max() <= 2e-3
    assert shared.error_flag() == 0


# ----------------------------------------------------------------------------- reference entry points
def test_windowed_gathers_match_oracle():
    print("case: get_dram_chunks_quantized_adaptive / decompress_dram_chunks_adaptive", flush=True)
    from heterokv.manager import HeteroKVManager
    K, V = _kv(51, 1, 2, 400)
    mgr = HeteroKVManager(1, sink_tokens=16, hbm_budget_tokens=80, device=DEV)
    orc = ManagerOracle(1, sink_tokens=16, hbm_budget_tokens=80)
    _drive(mgr, orc, K, V, 1, [64, 64, 64, 64, 40])
    assert len(orc.dram) >= 4
    # window None: the controller's first window is w_min = 2
    got = mgr.get_dram_chunks_quantized_adaptive(0)
    for w, got in ((2, got), (3, mgr.get_dram_chunks_quantized_adaptive(0, window_size=3)),
                   (99, mgr.get_dram_chunks_quantized_adaptive(0, window_size=99))):
        keys = orc.select_chunks(0, w)
        for name, X in (("k", K), ("v", V)):
            codes = [_oracle_codes(X, orc.dram[k]) for k in keys]
            assert np.array_equal(got[name + "_data"].cpu().numpy(), np.concatenate([c[0] for c in codes], 2))
            assert np.array_equal(got[name + "_scales"].cpu().numpy(), np.concatenate([c[1] for c in codes]))
            assert np.array_equal(got[name + "_zps"].cpu().numpy(), np.concatenate([c[2] for c in codes]))
    assert mgr.get_dram_chunks_quantized_adaptive(0, window_size=0) is None
    # scores that do not follow eviction order: the selected chunks, in eviction order
    mgr._chunk_attention_scores.update({"l0_e0": 0.1, "l0_e1": 0.9, "l0_e2": 0.5, "l0_e3": 0.9})
    orc.chunk_scores.update({"l0_e0": 0.1, "l0_e1": 0.9, "l0_e2": 0.5, "l0_e3": 0.9})
    kb, vb, n = mgr.decompress_dram_chunks_adaptive(0, window_size=2)
    keys = orc.select_chunks(0, 2)
    assert keys == ["l0_e1", "l0_e3"]
    posl = sum((orc.dram[k] for k in keys), [])
    assert n == len(posl) and kb.dtype == torch.bfloat16
    for got, X in ((kb, K), (vb, V)):
        c, s, z = _oracle_codes(X, posl)
        want = oc.decompress(c, s, z, 128, out_dtype="bf16")
        assert np.array_equal(got.cpu().view(torch.int16).numpy().view(np.uint16), want)


@pytest.mark.parametrize("aligned", [True, False])
def test_swap_in_and_prefetch(aligned):
    print("case: swap_in / swap_in_quantized / schedule_prefetch aligned=%s" % aligned, flush=True)
    from heterokv.manager import HeteroKVManager
    sink, budget, chunks = (16, 80, [64, 64, 64, 40]) if aligned else (4, 20, [60, 30, 30])
    K, V = _kv(61, 2, 2, 300)
    mgr = HeteroKVManager(1, sink_tokens=sink, hbm_budget_tokens=budget, device=DEV)
    orc = ManagerOracle(1, sink_tokens=sink, hbm_budget_tokens=budget)
    _drive(mgr, orc, K, V, 1, chunks)
    keys = list(orc.dram)
    assert list(mgr._dram_table.keys()) == keys and len(keys) >= 2
    victim = keys[0]
    q = mgr.swap_in_quantized(0, victim)
    c, s, z = _oracle_codes(K, orc.dram[victim])
    assert np.array_equal(q["k_data"].cpu().numpy(), c) and np.array_equal(q["k_scales"].cpu().numpy(), s)
    mgr.schedule_prefetch(victim)
    kb, vb = mgr.swap_in(0, victim)
    for got, X in ((kb, K), (vb, V)):
        c, s, z = _oracle_codes(X, orc.dram[victim])
        want = oc.decompress(c, s, z, 128).astype(np.float32)          # fp16, then .to(bf16)
        want = oc.f32_to_bf16_bits(want)
        assert np.array_equal(got.cpu().view(torch.int16).numpy().view(np.uint16), want)
    orc.remove_chunk(victim)
    assert mgr.swap_in(0, victim) is None
    assert list(mgr._dram_table.keys()) == list(orc.dram)
    assert mgr.count_dram_tokens(0) == orc.count_dram_tokens(0)
    assert mgr.positions(0, include_dram=True) == orc.dram_positions(0) + orc.key_cache[0]
    dk, dv, n = mgr.decompress_dram_chunks(0)
    posl = orc.dram_positions(0)
    assert n == len(posl)
    for got, X in ((dk, K), (dv, V)):
        c, s, z = _oracle_codes(X, posl)
        assert np.array_equal(got.cpu().numpy().view(np.uint16), oc.decompress(c, s, z, 128).view(np.uint16))
    # a second swap without a prefetch takes the synchronous route
    k2 = list(orc.dram)[0]
    kb2, _ = mgr.swap_in(0, k2)
    c, s, z = _oracle_codes(K, orc.dram[k2])
    want = oc.f32_to_bf16_bits(oc.decompress(c, s, z, 128).astype(np.float32))
    assert np.array_equal(kb2.cpu().view(torch.int16).numpy().view(np.uint16), want)
    mgr.check_errors()


# ----------------------------------------------------------------------------- HF lengths
def _tiny_qwen2(layers=2):
    from transformers import Qwen2Config, Qwen2ForCausalLM
    from heterokv.engine_wrapper import register_attention
    name = register_attention()
    torch.manual_seed(0)
    cfg = Qwen2Config(vocab_size=512, hidden_size=512, intermediate_size=1024, num_hidden_layers=layers,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=4096,
                      attn_implementation=name)
    return Qwen2ForCausalLM(cfg).to(DEV, torch.float16).eval()


def test_exact_lengths_and_generate():
    """After a chunked prefill whose last chunk is partial, get_seq_length is the prompt
    length, the materialized route's keys match get_mask_sizes, and generate() -- which
    derives cache_position and RoPE positions from the cache -- produces the tokens of a
    decode loop with explicit positions."""
    print("case: exact lengths + generate()", flush=True)
    from heterokv.engine_wrapper import ChunkedPrefillEngine, FusedHeteroCache
    model = _tiny_qwen2()
    ids = torch.randint(0, 512, (1, 301), generator=torch.Generator().manual_seed(7)).to(DEV)
    kw = dict(num_layers=2, sink_tokens=16, keep_tail=80, chunk_size=64, device=DEV)
    ca, cb = FusedHeteroCache(**kw), FusedHeteroCache(**kw)
    cref = FusedHeteroCache(reference_lengths=True, **kw)
    with torch.inference_mode():
        for c in (ca, cb, cref):
            ChunkedPrefillEngine(model, c, chunk_size=64).prefill(ids[:, :300])
        assert ca.get_seq_length() == 300
        assert ca._manager.dram_tokens(0) + ca._manager.hbm_length(0) == 300
        assert cref.get_seq_length() < 300        # the reference counts no DRAM tokens before decode
        out = model.generate(input_ids=ids, attention_mask=torch.ones_like(ids), past_key_values=ca,
                             max_new_tokens=6, do_sample=False)
        gen = out[0, 301:].tolist()
        tok, want = ids[:, 300:301], []
        for step in range(6):
            p = torch.tensor([[300 + step]], device=DEV)
            lg = model(input_ids=tok, position_ids=p, past_key_values=cb, use_cache=True).logits
            tok = lg[:, -1:].argmax(-1)
            want.append(int(tok))
        print("  generate %s, explicit positions %s" % (gen, want), flush=True)
        assert gen == want
        assert ca.get_seq_length() == cb.get_seq_length() == 306


def test_chunked_prefill_schedules_prefetch():
    """ChunkedPrefillEngine schedules a prefetch of every DRAM chunk after each chunk, as
    the reference does (engine_wrapper.py:484-486): the side stream holds every stored
    chunk dequantized afterwards, a swap_in returns the same bf16 K/V as a direct
    dequantization, and decode logits do not change."""
    print("case: ChunkedPrefillEngine per-chunk prefetch", flush=True)
    from heterokv.engine_wrapper import ChunkedPrefillEngine, FusedHeteroCache
    model = _tiny_qwen2()
    ids = torch.randint(0, 512, (1, 300), generator=torch.Generator().manual_seed(8)).to(DEV)
    kw = dict(num_layers=2, sink_tokens=16, keep_tail=80, chunk_size=64, device=DEV)
    ca, cb = FusedHeteroCache(**kw), FusedHeteroCache(**kw)
    with torch.inference_mode():
        ChunkedPrefillEngine(model, ca, chunk_size=64).prefill(ids)
        ChunkedPrefillEngine(model, cb, chunk_size=64, prefetch_after_chunk=False).prefill(ids)
        torch.cuda.synchronize()
        keys = list(ca.dram_table.keys())
        assert len(keys) >= 4 and keys == list(cb.dram_table.keys())
        pa = ca._manager._async_pf
        assert pa is not None and sorted(pa.buffer) == sorted(keys)
        assert cb._manager._async_pf is None or not cb._manager._async_pf.buffer
        p = torch.tensor([[300]], device=DEV)
        la = model(input_ids=ids[:, -1:], position_ids=p, past_key_values=ca, use_cache=True).logits
        lb = model(input_ids=ids[:, -1:], position_ids=p, past_key_values=cb, use_cache=True).logits
        assert torch.equal(la, lb)
        ka, va = ca.swap_in_chunk(keys[0])
        kb, vb = cb.swap_in_chunk(keys[0])
        assert ka.dtype == torch.bfloat16 and torch.equal(ka, kb) and torch.equal(va, vb)


def test_mask_sizes_match_materialized_keys():
    """get_mask_sizes, asked before each update as transformers does, equals the key length
    the materialized route returns, through prefill, the tail filling, heavy-hitter growth."""
    print("case: exact mask sizes", flush=True)
    from heterokv.engine_wrapper import FusedHeteroCache
    K, V = _kv(71, 1, 2, 500)
    c = FusedHeteroCache(num_layers=2, sink_tokens=8, keep_tail=40, device=DEV, fused_decode=False)
    pos = 0
    for n in [128, 128, 100] + [1] * 60:
        for layer in range(2):
            want, kv_off = c.get_mask_sizes(n, layer)
            q_off = c.get_query_offset(layer)
            if n > 1:
                assert q_off - kv_off == want - n      # query i sees keys [0, prefix + i]
            else:
                assert q_off - kv_off >= want - 1      # the decode query sees every key
            rk, _ = c.update(K[:, :, pos:pos + n].to(DEV), V[:, :, pos:pos + n].to(DEV), layer)
            assert rk.shape[2] == want, (pos, n, layer, rk.shape[2], want)
            assert c.get_seq_length(layer) == pos + n
        pos += n


def _as_hf_view(x):
    """The same values laid out as transformers hands them over: [B, S, H, D] storage seen
    through .transpose(1, 2)."""
    return x.transpose(1, 2).contiguous().transpose(1, 2)


@pytest.mark.parametrize("sink,budget,chunks,hq,hkv,strided", [
    (16, 80, [64, 64, 64, 40], 8, 2, False), (4, 20, [60, 30, 7, 33], 8, 2, False),
    (8, 200, [100, 50, 40, 90, 128], 8, 2, False), (16, 80, [64, 64, 64, 64, 64, 32], 7, 1, True),
    (16, 80, [64, 64, 64, 40], 8, 2, True)])
def test_attend_prefill_vs_oracle(sink, budget, chunks, hq, hkv, strided):
    """update(..., materialize=False) + attend_prefill per chunk against float64 attention
    over the positions the reference hands SDPA (sink + old tail + chunk, causal), then the
    zones and INT4 chunks against the oracle.  strided: inputs laid out as transformers'
    attention modules pass them (transposed views)."""
    print("case: attend_prefill sink=%d budget=%d chunks=%s %d/%d strided=%s" % (sink, budget, chunks, hq, hkv,
                                                                                 strided), flush=True)
    from heterokv.manager import HeteroKVManager
    B, Hkv, Hq = 1, hkv, hq
    K, V = _kv(81, B, Hkv, sum(chunks))
    g = torch.Generator().manual_seed(82)
    Q = (torch.randn((B, Hq, sum(chunks), 128), generator=g) / math.sqrt(128)).half()
    lay = _as_hf_view if strided else (lambda t: t)
    mgr = HeteroKVManager(1, sink_tokens=sink, hbm_budget_tokens=budget, device=DEV)
    orc = ManagerOracle(1, sink_tokens=sink, hbm_budget_tokens=budget)
    pos = 0
    for n in chunks:
        kc, vc = lay(K[:, :, pos:pos + n].to(DEV)), lay(V[:, :, pos:pos + n].to(DEV))
        mgr.update(0, kc, vc, mode="prefill", seq_offset=pos, materialize=False)
        want = orc.update(0, range(pos, pos + n), "prefill", seq_offset=pos)
        out = mgr.attend_prefill(0, lay(Q[:, :, pos:pos + n].to(DEV)), kc, vc).float().cpu().numpy()
        kk = K[0].double().numpy()[:, want]
        vv = V[0].double().numpy()[:, want]
        prefix = len(want) - n
        rep = Hq // Hkv
        err = 0.0
        for h in range(Hq):
            for i in range(n):
                r = oa.attend(Q[0, h, pos + i].double().numpy()[None, None], kk[h // rep][None, :prefix + i + 1],
                              vv[h // rep][None, :prefix + i + 1])[0, 0]
                err = max(err, float(np.abs(out[0, h, i] - r).max()))
        print("  chunk at %d (n=%d, prefix %d): max abs err %.3e" % (pos, n, prefix, err), flush=True)
        assert err <= 2e-3
        pos += n
    assert mgr.positions(0) == orc.key_cache[0]
    kz, vz = mgr.get_hbm_kv(0)
    idx = torch.tensor(orc.key_cache[0], dtype=torch.long)
    assert torch.equal(kz.cpu(), K.index_select(2, idx)) and torch.equal(vz.cpu(), V.index_select(2, idx))
    assert list(mgr._dram_table.keys()) == list(orc.dram)
    for key, posl in orc.dram.items():
        c, s, z = _oracle_codes(K, posl)
        assert np.array_equal(mgr._dram_table[key]["k_data"].cpu().numpy(), c)
    mgr.check_errors()
