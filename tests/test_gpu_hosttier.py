"""GPU tests of the host tier: staging-addressed block records in the decode and prefill
kernels, the record gather, the native prefetcher (pinned arena, side stream, events), and
HeteroKVManager.offload_to_host with one-layer-ahead prefetch.  Moving records between
HBM and host memory changes no arithmetic, so those outputs must be bit-identical to the
all-resident ones; windowed retrieval (manager.py:931-1056) is checked against the float64
oracle at 2e-3."""
import math

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import compressor as oc
from oracle.manager import ManagerOracle

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _kv(seed, B, H, S):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn((B, H, S, 128), generator=g)
    k[..., [7, 31, 64, 100]] *= 8
    v = torch.randn((B, H, S, 128), generator=g)
    return k.half(), v.half()


def _packed_pool(seed, B, H, T):
    from heterokv import ops
    K, V = _kv(seed, B, H, T)
    nb = (T + 15) // 16
    g = torch.Generator().manual_seed(seed + 1)
    bt = torch.randperm(B * nb, generator=g).to(torch.int32).view(B, nb)
    pool = ops.Int4Pool(B * nb, H, DEV)
    ops.pack_tokens(pool, K.to(DEV), V.to(DEV), [0] * B, bt)
    pool.check_errors()
    return K, V, pool, bt


def _move_to_staging(pool, bt, frac, seed, wipe=True):
    """Gather a random `frac` of the records into a staging pool; the table names them ~k."""
    from heterokv import ops
    B, nb = bt.shape
    rng = np.random.default_rng(seed)
    n = int(round(frac * B * nb))
    flat = np.sort(rng.choice(B * nb, size=n, replace=False))
    ids = bt.view(-1)[torch.from_numpy(flat)]
    staging = ops.Int4Pool(max(n, 1), pool.num_kv_heads, DEV)
    ops.gather_blocks(pool, ids, staging)
    staging.check_errors()
    bt2 = bt.clone().view(-1)
    bt2[torch.from_numpy(flat)] = ~torch.arange(n, dtype=torch.int32)
    if wipe:  # the moved records must now come from staging only
        pool.data[ids.long().to(DEV)] = 0
    return staging, bt2.view(B, nb)


def test_gather_blocks_and_errors():
    print("case: gather_blocks", flush=True)
    from heterokv import ops
    _, _, pool, bt = _packed_pool(1, 2, 4, 300)
    staging = ops.Int4Pool(5, 4, DEV)
    staging.data.copy_(torch.randint(0, 256, staging.data.shape, dtype=torch.uint8, device=DEV))
    ids = torch.tensor([3, ~0, 7, ~4, 0, 12], dtype=torch.int32)
    dst = ops.Int4Pool(8, 4, DEV)
    ops.gather_blocks(pool, ids, dst, staging=staging, dst_offset=1)
    dst.check_errors()
    for i, id_ in enumerate(ids.tolist()):
        want = pool.data[id_] if id_ >= 0 else staging.data[~id_]
        assert torch.equal(dst.data[1 + i], want), i
    bad = ops.Int4Pool(2, 4, DEV)
    ops.gather_blocks(pool, torch.tensor([pool.num_blocks, ~5], dtype=torch.int32), bad, staging=staging)
    with pytest.raises(Exception):
        bad.check_errors()


@pytest.mark.parametrize("frac", [0.6, 1.0])
def test_decode_with_staging_is_bit_identical(frac):
    print("case: decode staging frac=%s" % frac, flush=True)
    from heterokv import ops
    B, H, HQ, T = 2, 8, 32, 3000
    K, V, pool, bt = _packed_pool(2, B, H, T)
    zone = ops.F16Zone(B, H, 64, DEV)
    zone.write(K[:, :, :64].to(DEV), V[:, :, :64].to(DEV), [0] * B)
    g = torch.Generator().manual_seed(3)
    q = (torch.randn((B, HQ, 128), generator=g) / math.sqrt(128)).half().to(DEV)
    ws = ops.DecodeWorkspace(DEV)
    ref = ops.decode_attention(q, zones=[(zone, None, 64)], pool=pool, block_table=bt, int4_max_len=T,
                               workspace=ws, deterministic=True)
    staging, bt2 = _move_to_staging(pool, bt, frac, 4)
    got = ops.decode_attention(q, zones=[(zone, None, 64)], pool=None if frac == 1.0 else pool,
                               block_table=bt2, int4_max_len=T, workspace=ws, staging=staging,
                               deterministic=True)
    torch.cuda.synchronize()
    assert ws.error_flag() == 0
    assert torch.equal(got, ref)


def test_prefill_with_staging_is_bit_identical():
    print("case: prefill staging", flush=True)
    from heterokv import ops
    B, H, HQ, T, SQ = 1, 2, 8, 1000, 70
    K, V, pool, bt = _packed_pool(5, B, H, T)
    g = torch.Generator().manual_seed(6)
    q = (torch.randn((B, HQ, SQ, 128), generator=g) / math.sqrt(128)).half().to(DEV)
    ck, cv = _kv(7, B, H, SQ)
    ref = ops.prefill_attention(q, pool=pool, block_table=bt, int4_max_len=T, chunk_k=ck.to(DEV),
                                chunk_v=cv.to(DEV))
    staging, bt2 = _move_to_staging(pool, bt, 0.5, 8)
    got = ops.prefill_attention(q, pool=pool, block_table=bt2, int4_max_len=T, chunk_k=ck.to(DEV),
                                chunk_v=cv.to(DEV), staging=staging)
    torch.cuda.synchronize()
    pool.check_errors()
    assert torch.equal(got, ref)


def test_prefetcher_copies_events_and_stats():
    print("case: prefetcher", flush=True)
    from heterokv.prefetcher import Prefetcher
    N = 3 << 20
    pf = Prefetcher(DEV, 2 * N, num_slots=3)
    host = pf.host_tensor(0, N)
    host.copy_(torch.randint(0, 256, (N,), dtype=torch.uint8))
    dst = torch.zeros(N, dtype=torch.uint8, device=DEV)
    pf.submit([(dst.data_ptr(), pf.host_ptr(0), N // 2), (dst[N // 2:].data_ptr(), pf.host_ptr(N // 2), N - N // 2)],
              slot=0)
    pf.wait(0)
    assert torch.equal(dst.cpu(), host)
    pf.mark(0)
    # a second copy into the same buffer waits for slot 0's mark
    host2 = pf.host_tensor(N, N)
    host2.copy_(torch.randint(0, 256, (N,), dtype=torch.uint8))
    pf.submit([(dst.data_ptr(), pf.host_ptr(N), N)], slot=1, after_slot=0)
    pf.wait(1)
    assert torch.equal(dst.cpu(), host2)
    assert pf.stall_ms(1) >= 0.0
    # device -> arena
    src = torch.randint(0, 256, (4096,), dtype=torch.uint8, device=DEV)
    pf.stage_out(src, 128)
    torch.cuda.current_stream().synchronize()
    assert torch.equal(pf.host_tensor(128, 4096), src.cpu())
    st = pf.stats()
    assert st["bytes_h2d"] == 2 * N and st["copies_h2d"] == 3 and st["bytes_d2h"] == 4096
    with pytest.raises(Exception):
        pf.host_tensor(2 * N - 10, 20)
    pf.close()


def _feed(mgrs, K, V, layers, chunks):
    """Prefill every manager with the same chunks; returns the next position."""
    pos = 0
    for n in chunks:
        for li in range(layers):
            for m in mgrs:
                m.update(li, K[:, :, pos:pos + n].to(DEV), V[:, :, pos:pos + n].to(DEV), mode="prefill",
                         seq_offset=pos)
        pos += n
    return pos


def _decode_step(mgrs, K, V, layers, pos, q):
    outs = [[] for _ in mgrs]
    for li in range(layers):
        for j, m in enumerate(mgrs):
            m.update(li, K[:, :, pos:pos + 1].to(DEV), V[:, :, pos:pos + 1].to(DEV), mode="decode",
                     seq_offset=pos, materialize=False)
            outs[j].append(m.attend_decode(li, q[li].to(DEV)))
    return outs


@pytest.mark.parametrize("prefetch", [True, False])
def test_manager_offload_bit_identical_to_resident(prefetch):
    print("case: offload_to_host prefetch=%s" % prefetch, flush=True)
    from heterokv.manager import HeteroKVManager
    L, B, H, HQ = 3, 2, 4, 16
    chunks, steps = [1024, 1024, 900], 5
    K, V = _kv(11, B, H, sum(chunks) + steps)
    a = HeteroKVManager(L, sink_tokens=64, hbm_budget_tokens=576, device=DEV, enable_prefetch=prefetch)
    b = HeteroKVManager(L, sink_tokens=64, hbm_budget_tokens=576, device=DEV)
    a.deterministic_decode = b.deterministic_decode = True
    pos = _feed([a, b], K, V, L, chunks)
    key = list(a._dram_table.keys())[1]
    moved = a.offload_to_host(0.75, seed=3)
    nb = (a.dram_tokens(0) + 15) // 16
    assert moved == sum(a.host_blocks(li) for li in range(L))
    assert a.host_blocks(0) == min(round(0.75 * B * nb), B * (a.dram_tokens(0) // 16))
    assert a.memory_summary()["host_bytes"] == moved * 2208 * H
    ca, cb = a.chunk_codes(key), b.chunk_codes(key)
    for name in ca:
        assert torch.equal(ca[name], cb[name]), name
    g = torch.Generator().manual_seed(12)
    for step in range(steps):
        q = [(torch.randn((B, HQ, 1, 128), generator=g) / math.sqrt(128)).half() for _ in range(L)]
        oa_, ob_ = _decode_step([a, b], K, V, L, pos + step, q)
        for li in range(L):
            assert torch.equal(oa_[li], ob_[li]), (step, li)
    st = a.prefetch_stats()
    assert len(st["per_layer"]) == L * steps
    assert all(ms >= 0 for _, ms in st["per_layer"])
    rb = 2208 * H
    per_step = sum(a.host_blocks(li) for li in range(L)) * rb
    # every layer's host records cross once per step (plus at most one look-ahead)
    assert per_step * steps <= st["bytes_h2d"] <= per_step * steps + max(a.host_blocks(li) for li in range(L)) * rb


@pytest.mark.parametrize("window,offload", [(2, False), (2, True), ("adaptive", True)])
def test_windowed_retrieval_vs_oracle(window, offload):
    print("case: windowed retrieval window=%s offload=%s" % (window, offload), flush=True)
    from heterokv.manager import HeteroKVManager
    L, B, H, HQ = 2, 1, 2, 8
    chunks = [1024, 1024, 1024]
    K, V = _kv(21, B, H, sum(chunks) + 1)
    mgr = HeteroKVManager(L, sink_tokens=64, hbm_budget_tokens=576, device=DEV)
    orc = ManagerOracle(L, sink_tokens=64, hbm_budget_tokens=576)
    pos = 0
    for n in chunks:
        for li in range(L):
            mgr.update(li, K[:, :, pos:pos + n].to(DEV), V[:, :, pos:pos + n].to(DEV), mode="prefill",
                       seq_offset=pos)
            orc.update(li, range(pos, pos + n), "prefill", seq_offset=pos)
        pos += n
    if offload:
        mgr.offload_to_host(0.75, seed=1)
    mgr.retrieval_window = window
    g = torch.Generator().manual_seed(22)
    for li in range(L):
        mgr.update(li, K[:, :, pos:pos + 1].to(DEV), V[:, :, pos:pos + 1].to(DEV), mode="decode",
                   seq_offset=pos, materialize=False)
        orc.update(li, [pos], "decode", seq_offset=pos)
        q = (torch.randn((B, HQ, 1, 128), generator=g) / math.sqrt(128)).half()
        out = mgr.attend_decode(li, q.to(DEV)).float().cpu().numpy()
        # reference: the top-2 chunks by score (FIFO fallback 1/(e+1): the two oldest), in
        # eviction order, then the HBM zones
        keys = [k for k in orc.dram if k.startswith("l%d_" % li)]
        ranked = sorted(keys, key=lambda k: orc.chunk_scores[k], reverse=True)[:2]
        sel = [k for k in keys if k in ranked]
        dram = [p for k in sel for p in orc.dram[k]]
        hbm = orc.key_cache[li]
        idx = torch.tensor(dram)
        kc, ks, kz = oc.compress(K[0].index_select(1, idx).numpy(), 128)
        vc, vs, vz = oc.compress(V[0].index_select(1, idx).numpy(), 128)
        kk = np.concatenate([oa.dequant_rows(kc, ks.reshape(H, -1), kz.reshape(H, -1)),
                             K[0].index_select(1, torch.tensor(hbm)).double().numpy()], 1)
        vv = np.concatenate([oa.dequant_rows(vc, vs.reshape(H, -1), vz.reshape(H, -1)),
                             V[0].index_select(1, torch.tensor(hbm)).double().numpy()], 1)
        ref = oa.attend(q[0].double().numpy(), kk, vv)
        err = np.abs(out[0] - ref).max()
        print("  layer %d: %d window tokens, max abs err %.3e" % (li, len(dram), err), flush=True)
        assert len(dram) == 448 + 1024
        assert err <= 2e-3


def test_dram_storage_manager_and_async_prefetcher():
    print("case: DRAMStorageManager / AsyncPrefetcher", flush=True)
    from heterokv import KVCompressor
    from heterokv.prefetcher import AsyncPrefetcher, DRAMStorageManager
    comp = KVCompressor()
    K, V = _kv(31, 1, 2, 64)
    qk, sk, zk = comp.compress(K.to(DEV))
    qv, sv, zv = comp.compress(V.to(DEV))
    entry = {"k_data": qk, "k_scales": sk, "k_zps": zk, "v_data": qv, "v_scales": sv, "v_zps": zv}
    nbytes = sum(t.numel() * t.element_size() for t in entry.values())
    store = DRAMStorageManager(max_entries=2, max_bytes=3 * nbytes)
    assert store.store_entry("l0_e0", entry)
    assert store.store("l0_e1", qk, sk, zk, qv, sv, zv)
    assert not store.store_entry("l0_e2", entry)          # entry cap
    assert store.num_entries == 2 and store.total_bytes == 2 * nbytes
    assert store.keys == ["l0_e0", "l0_e1"]                 # a property, as the reference's
    assert store.memory_summary() == {"num_entries": 2, "total_bytes": 2 * nbytes,
                                      "total_mb": 2 * nbytes / (1024 * 1024)}
    got = store.retrieve("l0_e0")
    assert all(t.device.type == "cpu" and t.is_pinned() for t in got.values())
    for name in entry:
        assert torch.equal(got[name], entry[name].cpu()), name
    dev = store.transfer_to_device("l0_e1", DEV)
    assert torch.equal(dev["v_data"], qv)
    assert store.remove("l0_e1") is not None and store.total_bytes == nbytes
    with pytest.raises(ValueError):
        store.store_entry("bad", {"k_data": qk})
    pf = AsyncPrefetcher(DEV)
    pf.submit_prefetch_task("l0_e0", store.retrieve("l0_e0"), comp)
    assert pf.pending_keys == ["l0_e0"]
    rk, rv = pf.fetch_if_ready("l0_e0")
    assert rk.dtype == torch.bfloat16
    assert torch.equal(rk, comp.decompress(qk, sk, zk).to(torch.bfloat16))
    assert torch.equal(rv, comp.decompress(qv, sv, zv).to(torch.bfloat16))
    assert pf.fetch_if_ready("l0_e0") is None


def test_out_of_order_attends_with_host_tier():
    """attend_decode calls in any layer order (a caller re-attending a layer, skipping one)
    stay bit-identical to an all-resident twin: the look-ahead copy never lands in the
    staging buffer of the layer being attended."""
    print("case: out-of-order attend_decode with a host tier", flush=True)
    from heterokv.manager import HeteroKVManager
    L, B, H, HQ = 4, 1, 4, 16
    K, V = _kv(21, B, H, 2600)
    a = HeteroKVManager(L, sink_tokens=64, hbm_budget_tokens=576, device=DEV)
    b = HeteroKVManager(L, sink_tokens=64, hbm_budget_tokens=576, device=DEV)
    a.deterministic_decode = b.deterministic_decode = True
    pos = _feed([a, b], K, V, L, [1024, 1024, 500])
    a.offload_to_host(0.75, seed=5)
    g = torch.Generator().manual_seed(22)
    order = [0, 1, 2, 3, 0, 0, 1, 3, 2, 1, 2, 3, 0, 2, 1, 0, 3, 3, 1]
    for li in order:
        q = (torch.randn((B, HQ, 1, 128), generator=g) / math.sqrt(128)).half().to(DEV)
        assert torch.equal(a.attend_decode(li, q), b.attend_decode(li, q)), li
    a.check_errors()


def test_window_change_after_lookahead():
    """Switching retrieval_window after full-retrieval steps whose look-ahead already chose
    the next layers' chunks: every later attend uses the new window, as on an all-resident
    twin (which never looks ahead)."""
    print("case: retrieval_window change after look-ahead", flush=True)
    from heterokv.manager import HeteroKVManager
    L, B, H, HQ = 3, 1, 4, 16
    K, V = _kv(23, B, H, 2600)
    a = HeteroKVManager(L, sink_tokens=64, hbm_budget_tokens=576, device=DEV)
    b = HeteroKVManager(L, sink_tokens=64, hbm_budget_tokens=576, device=DEV)
    a.deterministic_decode = b.deterministic_decode = True
    _feed([a, b], K, V, L, [1024, 1024, 500])
    a.offload_to_host(0.75, seed=6)
    g = torch.Generator().manual_seed(24)
    for window in (None, 2, None, "adaptive", 1):
        a.retrieval_window = b.retrieval_window = window
        for li in [0, 1, 2, 0, 1, 2]:
            q = (torch.randn((B, HQ, 1, 128), generator=g) / math.sqrt(128)).half().to(DEV)
            assert torch.equal(a.attend_decode(li, q), b.attend_decode(li, q)), (window, li)
    a.check_errors()
