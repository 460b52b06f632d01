"""GPU parity at the benchmark configurations' full stated shapes, against the float64 oracle:
C3 (batch 16, the bench's seeded contexts in [8192, 32768] and random-permutation block table),
C4 (one 2048-query prefill launch over 64 + 131072 INT4 + 4096 tokens plus the causal chunk),
C5 (the 28-layer bf16 decoder at 131072 tokens with 75% of the INT4 blocks in host memory,
full and windowed retrieval).  Tolerance 2e-3 max-abs on fp16 outputs."""
import math

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import compressor as oc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
OUTLIERS = [7, 31, 64, 100]
HQ, HKV, D, SINK, RECENT = 32, 8, 128, 64, 4096


def _deq(x_f16, heads):
    """Path C: oracle-compressed rows dequantized to fp16, as float64 [heads, T, 128]."""
    c, s, z = oc.compress(x_f16.numpy(), 128)
    return oa.dequant_rows(c, s.reshape(heads, -1), z.reshape(heads, -1))


def test_c3_full_batch():
    """Batch 16 at the bench's seeded contexts and block table, all 32 heads of every sequence."""
    from heterokv import ops
    gen = torch.Generator().manual_seed(7)
    ctx = torch.randint(8192, 32769, (16,), generator=gen)
    mids = (ctx - SINK - RECENT).tolist()
    nbs = [(m + 15) // 16 for m in mids]
    total, nbmax = sum(nbs), max(nbs)
    perm = torch.randperm(total, generator=gen).to(torch.int32)
    bt = torch.zeros((16, nbmax), dtype=torch.int32)
    off = 0
    for b, nb in enumerate(nbs):
        bt[b, :nb] = perm[off:off + nb]
        off += nb
    print("case: C3 batch 16, contexts %s, %d blocks" % (ctx.tolist(), total), flush=True)
    g = torch.Generator().manual_seed(8)
    pool = ops.Int4Pool(total, HKV, DEV)
    bt_d = bt.to(DEV)
    kv = []
    for b in range(16):
        K = torch.randn((HKV, mids[b], D), generator=g)
        K[..., OUTLIERS] *= 8
        K = K.half()
        V = torch.randn((HKV, mids[b], D), generator=g).half()
        ops.pack_tokens(pool, K[None].to(DEV), V[None].to(DEV), [0], bt_d[b:b + 1])
        kv.append((K, V))
    pool.check_errors()
    sk = torch.randn((16, HKV, SINK, D), generator=g).half()
    sv = torch.randn((16, HKV, SINK, D), generator=g).half()
    rk = torch.randn((16, HKV, RECENT, D), generator=g).half()
    rv = torch.randn((16, HKV, RECENT, D), generator=g).half()
    q = (torch.randn((16, HQ, D), generator=g) / math.sqrt(D)).half()
    sink, rec = ops.F16Zone(16, HKV, SINK, DEV), ops.F16Zone(16, HKV, RECENT, DEV)
    sink.write(sk.to(DEV), sv.to(DEV), 0)
    rec.write(rk.to(DEV), rv.to(DEV), 0)
    ws = ops.DecodeWorkspace(DEV)
    outs = {}
    for det in (False, True):
        outs[det] = ops.decode_attention(q.to(DEV), zones=[(sink, None, SINK), (rec, None, RECENT)], pool=pool,
                                         block_table=bt_d, int4_lens=torch.tensor(mids, dtype=torch.int32).to(DEV),
                                         int4_max_len=max(mids), workspace=ws, deterministic=det).float().cpu().numpy()
    torch.cuda.synchronize()
    assert ws.error_flag() == 0
    worst = 0.0
    for b in range(16):
        K, V = kv[b]
        kk = np.concatenate([_deq(K, HKV), sk[b].double().numpy(), rk[b].double().numpy()], 1)
        vv = np.concatenate([_deq(V, HKV), sv[b].double().numpy(), rv[b].double().numpy()], 1)
        ref = oa.attend(q[b].double().numpy()[:, None], kk, vv)[:, 0]
        for det in (False, True):
            worst = max(worst, float(np.abs(outs[det][b] - ref).max()))
    print("  max abs err over 16 sequences x 32 heads, both schedules: %.3e" % worst, flush=True)
    assert worst <= 2e-3


def test_c4_full_launch():
    """One 2048-query launch over 64 fp16 + 131072 INT4 + 4096 fp16 tokens and the causal chunk;
    72 query rows (both ends, every 64-row tile boundary pair around the 32-row workgroup blocks,
    the last row) x 32 heads against the oracle."""
    from heterokv import ops
    Sq, MID = 2048, 131072
    hist = SINK + MID + RECENT
    print("case: C4 full launch 2048 x (64 + 131072 + 4096 + causal)", flush=True)
    g = torch.Generator().manual_seed(4)
    K = torch.randn((HKV, hist, D), generator=g)
    K[..., OUTLIERS] *= 8
    K = K.half()
    V = torch.randn((HKV, hist, D), generator=g).half()
    CK = torch.randn((HKV, Sq, D), generator=g).half()
    CV = torch.randn((HKV, Sq, D), generator=g).half()
    q = (torch.randn((HQ, Sq, D), generator=g) / math.sqrt(D)).half()
    sink = ops.F16Zone(1, HKV, SINK, DEV)
    sink.write(K[None, :, :SINK].to(DEV), V[None, :, :SINK].to(DEV), 0)
    rec = ops.F16Zone(1, HKV, RECENT, DEV)
    rec.write(K[None, :, SINK + MID:].to(DEV), V[None, :, SINK + MID:].to(DEV), 0)
    nb = MID // 16
    pool = ops.Int4Pool(nb, HKV, DEV)
    bt = torch.randperm(nb, generator=g).to(torch.int32)[None].to(DEV)
    ops.pack_tokens(pool, K[None, :, SINK:SINK + MID].to(DEV), V[None, :, SINK:SINK + MID].to(DEV), [0], bt)
    out = ops.prefill_attention(q[None].to(DEV), zones=[(sink, None, SINK), (rec, None, RECENT)], pool=pool,
                                block_table=bt, int4_max_len=MID, chunk_k=CK[None].to(DEV),
                                chunk_v=CV[None].to(DEV)).float().cpu().numpy()[0]
    pool.check_errors()
    rows = sorted(set([0, 1, 2, 31, 32, 33, 63, 64, 65] + [r for t in range(128, 2048, 256) for r in (t - 1, t)] +
                      [1023, 1024, 1025, 2015, 2016, 2017, 2046, 2047] + list(range(1500, 1532))))
    assert len(rows) >= 64
    kk = np.concatenate([_deq(K[:, SINK:SINK + MID], HKV), K[:, :SINK].double().numpy(),
                         K[:, SINK + MID:].double().numpy(), CK.double().numpy()], 1)
    vv = np.concatenate([_deq(V[:, SINK:SINK + MID], HKV), V[:, :SINK].double().numpy(),
                         V[:, SINK + MID:].double().numpy(), CV.double().numpy()], 1)
    mask = np.arange(hist + Sq)[None, :] <= hist + np.array(rows)[:, None]
    ref = oa.attend(q[:, rows].double().numpy(), kk, vv, mask=mask)
    err = float(np.abs(out[:, rows] - ref).max())
    print("  %d rows x 32 heads: max abs err %.3e" % (len(rows), err), flush=True)
    assert err <= 2e-3


def _c5_model():
    from transformers import Qwen2Config, Qwen2ForCausalLM
    from heterokv.engine_wrapper import register_attention
    cfg = Qwen2Config(vocab_size=152064, hidden_size=3584, intermediate_size=18944, num_hidden_layers=28,
                      num_attention_heads=28, num_key_value_heads=4, max_position_embeddings=135168,
                      rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=False,
                      attn_implementation=register_attention())
    torch.manual_seed(0)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(DEV):
            model = Qwen2ForCausalLM(cfg)
    finally:
        torch.set_default_dtype(prev)
    return model.eval()


def _layer_reference(mgr, layer, q, keys=None):
    """float64 Path C attention of q [Hq, 128] over the layer's INT4 chunks (`keys`, default
    all, in eviction order) from the GPU's stored codes, plus its fp16 zones."""
    keys = mgr._layer_chunks(layer) if keys is None else keys
    H = mgr._layers[layer].H
    ks, vs = [], []
    for key in keys:
        e = mgr.chunk_codes(key)
        ks.append(oa.dequant_rows(e["k_data"][0].cpu().numpy(), e["k_scales"].cpu().numpy().reshape(H, -1),
                                  e["k_zps"].cpu().numpy().reshape(H, -1)))
        vs.append(oa.dequant_rows(e["v_data"][0].cpu().numpy(), e["v_scales"].cpu().numpy().reshape(H, -1),
                                  e["v_zps"].cpu().numpy().reshape(H, -1)))
    zk, zv = mgr.get_hbm_kv(layer)
    kk = np.concatenate(ks + [zk[0].double().cpu().numpy()], 1)
    vv = np.concatenate(vs + [zv[0].double().cpu().numpy()], 1)
    return oa.attend(q.double().numpy()[:, None], kk, vv)[:, 0], kk.shape[1]


def test_c5_tiered_128k_bf16():
    """Two identical caches prefilled with the 131072-token prompt; 75% of one's INT4 blocks
    move to pinned host memory.  Under the fixed decode schedule the offloaded cache's logits
    equal the resident one's bit for bit, in full and windowed retrieval; one layer per step is
    checked against the float64 oracle over its stored INT4 codes and fp16 zones."""
    from heterokv.engine_wrapper import ChunkedPrefillEngine, FusedHeteroCache
    print("case: C5 28-layer bf16, 131072 tokens, 75% host, full + windowed", flush=True)
    model = _c5_model()
    ids = torch.randint(0, 152064, (1, 131072), generator=torch.Generator().manual_seed(1)).to(DEV)
    caches = []
    with torch.inference_mode():
        for i in range(2):
            c = FusedHeteroCache(num_layers=28, sink_tokens=64, keep_tail=4160, chunk_size=2048, device=DEV,
                                 fused_prefill=True)
            eng = ChunkedPrefillEngine(model, c, chunk_size=2048)
            for start in range(0, 131072, 32768):
                eng.prefill(ids[:, start:start + 32768],
                            position_ids=torch.arange(start, start + 32768, device=DEV)[None])
            torch.cuda.synchronize()
            c._manager.deterministic_decode = True
            caches.append(c)
            print("  cache %d prefilled: %d INT4 tokens per layer" % (i, c._manager.dram_tokens(0)), flush=True)
        res, off = caches
        assert res.get_seq_length() == off.get_seq_length() == 131072
        mgr = off._manager
        moved = off.offload_to_host(0.75, seed=0)
        blocks = sum(st.B * st.nb for st in mgr._layers)
        print("  %d of %d INT4 blocks moved to host memory" % (moved, blocks), flush=True)
        assert abs(moved - 0.75 * blocks) <= 28
        tok = ids[:, -1:]
        pos = 131072
        g = torch.Generator().manual_seed(3)
        for mode in ("full", "windowed"):
            if mode == "windowed":
                res.retrieval_window = off.retrieval_window = "adaptive"
            for step in range(2):
                p = torch.tensor([[pos]], device=DEV)
                la = model(input_ids=tok, past_key_values=res, position_ids=p, use_cache=True).logits
                lb = model(input_ids=tok, past_key_values=off, position_ids=p, use_cache=True).logits
                assert torch.isfinite(lb).all()
                assert torch.equal(la, lb), mode
                layer = (7 * step + (0 if mode == "full" else 13)) % 28
                sel = mgr._selection(layer)
                q = (torch.randn((28, D), generator=g) / math.sqrt(D)).half()
                got = mgr.attend_decode(layer, q[None, :, None].to(DEV)).float().cpu().numpy()[0, :, 0]
                ref, n_keys = _layer_reference(mgr, layer, q, None if sel is None else list(sel))
                err = float(np.abs(got - ref).max())
                print("  %s step %d: logits equal; layer %d over %d keys (%s chunks): max abs err %.3e"
                      % (mode, step, layer, n_keys, "all" if sel is None else len(sel), err), flush=True)
                assert err <= 2e-3
                tok = la[:, -1:].argmax(-1)
                pos += 1
        st = off.prefetch_stats()
        assert st["bytes_h2d"] > 0
        res.check_errors()
        off.check_errors()
