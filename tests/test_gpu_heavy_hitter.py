"""GPU parity: heavy-hitter scoring (hkv_attn_weights, hkv_block_scores,
hkv_eviction_candidates; heavy_hitter.py:26-101, oracle_triton.py:16-79) and the decode
kernel's score outputs against oracle/heavy_hitter.py and the float64 attention oracle."""
import math

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import compressor as oc
from oracle import heavy_hitter as hh

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
LOG2E = 1.0 / math.log(2.0)


@pytest.mark.parametrize("seq_len,bs", [(256, 16), (1000, 16), (777, 7), (64, 128), (100000, 16)])
def test_block_scores_bit_exact(seq_len, bs):
    print("case: block scores seq_len=%d bs=%d" % (seq_len, bs), flush=True)
    from heterokv import ops
    g = torch.Generator().manual_seed(seq_len)
    ts = torch.rand(seq_len + 5, generator=g)
    got = ops.block_scores(ts.to(DEV), seq_len, bs).cpu().numpy()
    want = hh.block_scores(ts.numpy(), seq_len, bs)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("seq_len,sink,local,k,quant", [
    (256, 16, 32, 2, False),
    (4096, 64, 512, 17, True),          # equal means: index order
    (130000, 64, 4096, 300, False),     # 8125 blocks, one sort pass
    (16384 * 16 + 5000, 64, 4096, 8, False),   # 16697 blocks: two sorted chunks, then a merge
    (300, 200, 200, 5, False),          # shorter than sink + local: nothing
])
def test_eviction_candidates(seq_len, sink, local, k, quant):
    print("case: eviction seq_len=%d sink=%d local=%d k=%d" % (seq_len, sink, local, k), flush=True)
    from heterokv import ops
    g = torch.Generator().manual_seed(k)
    ts = torch.rand(seq_len, generator=g)
    if quant:
        ts = torch.floor(ts * 4) / 4
    got = ops.eviction_candidates(ts.to(DEV), seq_len, 16, sink, local, k).cpu().tolist()
    want = hh.eviction_candidates(ts.numpy(), seq_len, 16, sink, local, k)
    assert got == want


def test_reference_scenario_on_gpu():
    """tests/test_end_to_end_pipeline.py:63-90 through the HeavyHitterOracle mirror."""
    print("case: HeavyHitterOracle cold blocks", flush=True)
    from heterokv import HeavyHitterOracle, compute_block_scores
    oracle = HeavyHitterOracle(block_size=16, sink_tokens=16, local_window=32)
    assert oracle.get_eviction_candidates(256, 2).tolist() == [1, 2]        # cold start: FIFO
    g = torch.Generator().manual_seed(0)
    for _ in range(10):
        a = torch.rand(256, generator=g) * 0.1
        a[80:112] = 0.001
        oracle.update(a.to(DEV))
    assert oracle.get_eviction_candidates(256, 2).tolist() == [5, 6]
    bsc = compute_block_scores(oracle.token_scores, 256, 16)
    assert bsc.shape[0] == 16
    want = hh.block_scores(oracle.token_scores.cpu().numpy(), 256, 16)
    assert np.array_equal(bsc.cpu().numpy(), want)


def test_decode_scores_and_weights():
    """Decode score outputs: every item's log2-domain score against float64, the row
    statistics, and the head-averaged weights against the oracle; the attention
    output itself is bit-identical with and without the score outputs."""
    print("case: decode scores B=2 32/8 sink 64 + INT4 [900, 500] + recent [300, 200]", flush=True)
    from heterokv import ops
    from test_gpu_decode import Case
    c = Case(21, 2, 32, 8, 64, [900, 500], [300, 200])
    B, Hq, Hkv = 2, 32, 8
    rmax = max(c.recents)
    n = c.maxmid + c.sink + rmax
    scores = torch.full((B, Hq, n), float("-inf"), dtype=torch.float32, device=DEV)
    stats = torch.empty((B, Hq, 2), dtype=torch.float32, device=DEV)
    q = c.q.to(DEV)
    kw = dict(zones=c.zones, pool=c.pool, block_table=c.bt.to(DEV), int4_lens=c.int4_lens.to(DEV),
              int4_max_len=c.maxmid, deterministic=True)
    out_plain = ops.decode_attention(q, **kw)
    out_sc = ops.decode_attention(q, scores=scores, score_stats=stats, **kw)
    torch.cuda.synchronize()
    assert torch.equal(out_plain, out_sc)
    sc = scores.cpu().numpy()
    st = stats.cpu().numpy()
    scale = 1.0 / math.sqrt(128)
    for b in range(B):
        s, m, r = c.sink, c.mids[b], c.recents[b]
        kc, ks, kz = oc.compress(c.K[b, :, s:s + m].numpy(), 128)
        # the kernel applies the K scale to the exact (code - zp) dot product in fp32
        k4 = oa.dequant_rows(kc, ks.reshape(Hkv, m), kz.reshape(Hkv, m), out_fp16=False)
        ksink = c.K[b, :, :s].double().numpy()
        krec = c.K[b, :, s + m:s + m + r].double().numpy()
        qb = c.q[b].double().numpy()
        want = np.full((Hq, n), -np.inf)
        for i in range(Hq):
            kv = i // (Hq // Hkv)
            want[i, :m] = k4[kv] @ qb[i] * scale * LOG2E
            want[i, c.maxmid:c.maxmid + s] = ksink[kv] @ qb[i] * scale * LOG2E
            want[i, c.maxmid + s:c.maxmid + s + r] = krec[kv] @ qb[i] * scale * LOG2E
        fin = np.isfinite(want)
        assert np.array_equal(np.isfinite(sc[b]), fin)
        err = np.abs(sc[b][fin] - want[fin]).max()
        print("  b=%d max score err %.2e" % (b, err), flush=True)
        assert err < 2e-3
        mx = np.where(fin, want, -np.inf).max(axis=1)
        assert np.abs(st[b, :, 0] - mx).max() < 2e-3
        ls = np.exp2(np.where(fin, want - mx[:, None], -np.inf)).sum(axis=1)
        np.testing.assert_allclose(st[b, :, 1], ls, rtol=2e-3)
        w = ops.attn_weights(scores[b:b + 1], stats[b:b + 1]).cpu().numpy()[0]
        np.testing.assert_allclose(w, hh.newest_token_weights(want), rtol=5e-3, atol=1e-7)
        assert abs(w.sum() - 1.0) < 1e-4


def test_manager_feeds_oracle():
    """attend_decode(feed_oracle=True) at every decode step: the oracle board gains one
    probability vector per step (its total grows by exactly one per step) and its
    eviction candidates agree with the numpy oracle on the same board."""
    print("case: manager feed_oracle", flush=True)
    from heterokv.manager import HeteroKVManager
    from heterokv import ops
    L, B, H, HQ = 2, 1, 4, 16
    g = torch.Generator().manual_seed(5)
    T = 1200 + 8
    K = torch.randn((B, H, T, 128), generator=g).half()
    V = torch.randn((B, H, T, 128), generator=g).half()
    mgr = HeteroKVManager(L, sink_tokens=32, hbm_budget_tokens=256, device=DEV)
    for li in range(L):
        mgr.update(li, K[:, :, :1200].to(DEV), V[:, :, :1200].to(DEV), mode="prefill", seq_offset=0)
    steps = 8
    for step in range(steps):
        pos = 1200 + step
        for li in range(L):
            mgr.update(li, K[:, :, pos:pos + 1].to(DEV), V[:, :, pos:pos + 1].to(DEV), mode="decode",
                       seq_offset=pos, materialize=False)
            q = (torch.randn((B, HQ, 1, 128), generator=g) / math.sqrt(128)).half().to(DEV)
            mgr.attend_decode(li, q, feed_oracle=(li == L - 1))
    board = mgr.get_oracle_scores()
    assert board is not None
    torch.cuda.synchronize()
    tot = float(board.double().sum())
    print("  board length %d total %.6f" % (board.numel(), tot), flush=True)
    assert abs(tot - steps) < 1e-3 and float(board.min()) >= 0.0
    n = board.numel()
    got = mgr._oracle.get_eviction_candidates(n, 4).cpu().tolist()
    want = hh.eviction_candidates(board.cpu().numpy(), n, 16, 32, 256, 4)
    assert got == want
    assert ops is not None
