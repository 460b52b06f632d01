"""GPU parity: split-K INT4/fp16 decode attention (hkv_decode_attn) against the float64
dequantize-then-attend oracle (fused_dequant_attn.py:326-331 + Path C fp16 dequant,
manager.py:806-807), tolerance 2e-3 max-abs on the fp16 output."""
import math

import os

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import compressor as oc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 2e-3  # max-abs on the fp16 output (fp32 accumulation)
OUTLIERS = [7, 31, 64, 100]


def _ceil16(x):
    return max(16, (x + 15) // 16 * 16)


class Case:
    """Three-zone decode inputs: per sequence [sink fp16 | INT4 middle | recent fp16]."""

    def __init__(self, seed, B, Hq, Hkv, sink, mids, recents, q_scale=1.0, sink_cap=None, rec_cap=None):
        from heterokv import ops
        g = torch.Generator().manual_seed(seed)
        self.B, self.Hq, self.Hkv = B, Hq, Hkv
        self.sink, self.mids, self.recents = sink, list(mids), list(recents)
        smax = sink + max(self.mids) + max(self.recents)
        K = torch.randn((B, Hkv, smax, 128), generator=g)
        K[..., OUTLIERS] *= 8
        self.K = K.half()
        self.V = torch.randn((B, Hkv, smax, 128), generator=g).half()
        self.q = (torch.randn((B, Hq, 128), generator=g) * q_scale / math.sqrt(128)).half()
        self.zones = []
        if sink > 0:
            zs = ops.F16Zone(B, Hkv, sink_cap or _ceil16(sink), DEV)
            zs.write(self.K[:, :, :sink].to(DEV), self.V[:, :, :sink].to(DEV), [0] * B)
            self.zones.append((zs, None, sink))
        self.maxmid = max(self.mids)
        nbs = [(m + 15) // 16 for m in self.mids]
        self.nbmax = max(max(nbs), 1)
        total_blocks = sum(nbs) + 2
        perm = torch.randperm(total_blocks, generator=g).to(torch.int32)
        self.bt = torch.zeros((B, self.nbmax), dtype=torch.int32)
        off = 0
        for b, nb in enumerate(nbs):
            self.bt[b, :nb] = perm[off:off + nb]
            off += nb
        self.pool = ops.Int4Pool(total_blocks, Hkv, DEV)
        for b in range(B):
            if self.mids[b]:
                ops.pack_tokens(self.pool, self.K[b:b + 1, :, sink:sink + self.mids[b]].to(DEV),
                                self.V[b:b + 1, :, sink:sink + self.mids[b]].to(DEV), [0], self.bt[b:b + 1])
        self.pool.check_errors()
        if max(self.recents) > 0:
            zr = ops.F16Zone(B, Hkv, rec_cap or _ceil16(max(self.recents)), DEV)
            rmax = max(self.recents)
            kr = torch.zeros((B, Hkv, rmax, 128), dtype=torch.float16)
            vr = torch.zeros((B, Hkv, rmax, 128), dtype=torch.float16)
            for b in range(B):
                s0, r = sink + self.mids[b], self.recents[b]
                kr[b, :, :r] = self.K[b, :, s0:s0 + r]
                vr[b, :, :r] = self.V[b, :, s0:s0 + r]
            zr.write(kr.to(DEV), vr.to(DEV), [0] * B)
            lens = torch.tensor(self.recents, dtype=torch.int32)
            self.zones.append((zr, lens if B > 1 else None, max(self.recents)))
        self.int4_lens = torch.tensor(self.mids, dtype=torch.int32) if B > 1 else None

    def run(self, workspace=None, sm_scale=None, deterministic=False, splits=0):
        from heterokv import ops
        out = ops.decode_attention(self.q.to(DEV), zones=self.zones, pool=self.pool,
                                   block_table=self.bt.to(DEV),
                                   int4_lens=self.int4_lens.to(DEV) if self.int4_lens is not None else None,
                                   int4_max_len=self.maxmid, sm_scale=sm_scale, workspace=workspace,
                                   deterministic=deterministic, splits=splits)
        torch.cuda.synchronize()
        return out.float().cpu().numpy()

    def oracle(self, sm_scale=None):
        outs = []
        for b in range(self.B):
            s, m, r = self.sink, self.mids[b], self.recents[b]
            parts_k, parts_v = [], []
            if m:
                kc, ks, kz = oc.compress(self.K[b, :, s:s + m].numpy(), 128)
                vc, vs, vz = oc.compress(self.V[b, :, s:s + m].numpy(), 128)
                parts_k.append(oa.dequant_rows(kc, ks.reshape(self.Hkv, m), kz.reshape(self.Hkv, m)))
                parts_v.append(oa.dequant_rows(vc, vs.reshape(self.Hkv, m), vz.reshape(self.Hkv, m)))
            parts_k.append(self.K[b, :, :s].double().numpy())
            parts_v.append(self.V[b, :, :s].double().numpy())
            parts_k.append(self.K[b, :, s + m:s + m + r].double().numpy())
            parts_v.append(self.V[b, :, s + m:s + m + r].double().numpy())
            k = np.concatenate(parts_k, axis=1)
            v = np.concatenate(parts_v, axis=1)
            outs.append(oa.attend(self.q[b].double().numpy()[:, None], k, v, sm_scale=sm_scale)[:, 0])
        return np.stack(outs)


def _check(case, **kw):
    """Both block schedules (on-demand and fixed) against the oracle."""
    ref = case.oracle(sm_scale=kw.get("sm_scale"))
    for det in (False, True):
        got = case.run(deterministic=det, **kw)
        err = np.abs(got - ref).max()
        print("  deterministic=%s max abs err %.3e" % (det, err), flush=True)
        assert np.all(np.isfinite(got))
        assert err <= TOL
    return got


def test_small_three_zone():
    print("case: B=1 32/8 sink 64 + INT4 1000 + recent 300", flush=True)
    _check(Case(1, 1, 32, 8, 64, [1000], [300]))


def test_c2_full_geometry():
    print("case: C2 B=1 32/8 ctx 32768 = 64 + 28608 + 4096", flush=True)
    _check(Case(2, 1, 32, 8, 64, [28608], [4096]))


@pytest.mark.parametrize("hq,hkv", [(8, 8), (28, 4), (16, 1), (64, 8)])
def test_gqa_ratios(hq, hkv):
    print("case: GQA %d/%d" % (hq, hkv), flush=True)
    _check(Case(3, 1, hq, hkv, 64, [777], [129]))


def test_int4_only_and_fp16_only():
    print("case: INT4 only", flush=True)
    _check(Case(4, 1, 32, 8, 0, [2000], [0]))
    print("case: fp16 only", flush=True)
    _check(Case(5, 1, 32, 8, 64, [0], [4096]))


def test_ragged_batch_paged():
    print("case: B=4 ragged, random block table", flush=True)
    _check(Case(6, 4, 32, 8, 64, [5000, 17, 1, 3000], [4096, 100, 16, 1]))


def test_sharp_attention_rescaling():
    print("case: large q (sharp softmax)", flush=True)
    _check(Case(7, 1, 32, 8, 64, [3000], [500], q_scale=12.0))


def test_custom_sm_scale():
    print("case: sm_scale 0.3", flush=True)
    _check(Case(8, 1, 32, 8, 16, [500], [64]), sm_scale=0.3)


def test_garbage_beyond_length_is_ignored():
    print("case: NaN in unused zone slots", flush=True)
    c = Case(9, 1, 32, 8, 20, [100], [37])
    for z, _, n in c.zones:
        z.k[:, :, n:] = float("nan")
        vt = z.v.view(1, c.Hkv, -1, 4, 16, 8, 4)
        # slots >= n inside the last tile: token 4g+i
        for s in range(n, z.capacity):
            t, r = divmod(s, 16)
            vt[:, :, t, r // 4, :, :, r % 4] = float("nan")
    _check(c)


def test_deterministic_bitwise():
    print("case: deterministic schedule, run twice, same bits", flush=True)
    from heterokv import ops
    c = Case(10, 2, 32, 8, 64, [9000, 4000], [4096, 2000])
    ws = ops.DecodeWorkspace(DEV)
    a = c.run(workspace=ws, deterministic=True)
    b = c.run(workspace=ws, deterministic=True)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert ws.error_flag() == 0


@pytest.mark.parametrize("hq,hkv,handoff", [(32, 8, False), (32, 8, True), (28, 4, False)])
@pytest.mark.parametrize("splits", [0, 8, 31])
def test_slice_merge_and_its_fallback(monkeypatch, splits, hq, hkv, handoff):
    """One sequence, every range of a pair resident (the grid fits the CUs): each range
    merges one slice of the output once all have arrived.  Eight kv heads take the
    XCD-local hand-off (atomics and loads in the XCD's L2) unless the workspace asks for
    the device-scope one; four kv heads (a pair's ranges on two XCDs) always take the
    device-scope one.  With HKV_DECODE_MERGE_WAIT_TICKS=0 a range stops waiting at its
    first poll that does not find every range arrived, and the last arrival merges every
    slice instead.  Both paths against the oracle on one workspace, alternating, so that
    each launch starts from the counters the previous one left; the error word stays
    clear."""
    from heterokv import ops
    print("case: slice merge, B=1 %d/%d, 64 + 8000 + 1000, splits=%d, agent_handoff=%s" % (hq, hkv, splits, handoff),
          flush=True)
    c = Case(16, 1, hq, hkv, 64, [8000], [1000])
    ref = c.oracle()
    ws = ops.DecodeWorkspace(DEV, agent_handoff=handoff)
    for wait in ("0", None, "0", None, "0", "0", None):
        if wait is None:
            monkeypatch.delenv("HKV_DECODE_MERGE_WAIT_TICKS", raising=False)
        else:
            monkeypatch.setenv("HKV_DECODE_MERGE_WAIT_TICKS", wait)
        got = c.run(workspace=ws, splits=splits)
        err = np.abs(got - ref).max()
        print("  wait=%s max abs err %.3e" % (wait, err), flush=True)
        assert np.all(np.isfinite(got)) and err <= TOL
        assert ws.error_flag() == 0


@pytest.mark.parametrize("hq,hkv", [(32, 8), (28, 4)])
def test_decode_beside_a_concurrent_kernel(hq, hkv):
    """Decode launches while GEMMs on another stream hold many CUs, so the ranges of a pair
    need not all be resident at once: the slice merge's bounded wait hands the merge to the
    last arrival when ranges give up waiting.  Eight kv heads merge in the XCD's L2, four
    (a pair's ranges on two XCDs) at device scope.  Outputs stay within the bound, the
    placement check stays clear (the error word is zero), and the other stream is still
    busy when each decode has finished."""
    from heterokv import ops
    print("case: decode beside a concurrent GEMM stream, B=1 %d/%d, 64 + 8000 + 1000" % (hq, hkv), flush=True)
    c = Case(16, 1, hq, hkv, 64, [8000], [1000])
    ref = c.oracle()
    ws = ops.DecodeWorkspace(DEV)
    side = torch.cuda.Stream(device=DEV)          # default priority
    a = torch.randn(8192, 8192, device=DEV, dtype=torch.bfloat16) / 90
    b = torch.randn(8192, 8192, device=DEV, dtype=torch.bfloat16) / 90
    o = torch.empty_like(a)
    q, bt = c.q.to(DEV), c.bt.to(DEV)
    torch.cuda.synchronize()
    main = torch.cuda.current_stream(DEV)
    overlapped = 0
    for i in range(5):
        with torch.cuda.stream(side):
            for _ in range(3):
                torch.matmul(a, b, out=o)
        side_done = torch.cuda.Event()
        side_done.record(side)
        out = ops.decode_attention(q, zones=c.zones, pool=c.pool, block_table=bt, int4_max_len=c.maxmid,
                                   workspace=ws)
        done = torch.cuda.Event()
        done.record(main)
        done.synchronize()
        overlapped += int(not side_done.query())
        err = np.abs(out.float().cpu().numpy() - ref).max()
        print("  launch %d: max abs err %.3e" % (i, err), flush=True)
        assert err <= TOL
        assert ws.error_flag() == 0
    torch.cuda.synchronize()
    assert overlapped >= 1


def test_schedules_agree_on_long_windows():
    """Ranges longer than one block-id window (1024 INT4 blocks) restage the ids
    between windows: one range per pair (splits=1) over 40000 INT4 tokens = 2500
    blocks = 3 windows, against the oracle in both schedules."""
    print("case: splits=1, 2500 INT4 blocks, B=2", flush=True)
    c = Case(12, 2, 16, 2, 64, [40000, 17000], [300, 4096])
    _check(c, splits=1)


def test_long_ragged_contexts():
    """Long and short sequences in one batch: 140000 INT4 tokens (8750 blocks, many id
    windows per range) beside 33 (an odd block count), one kv head."""
    print("case: B=2 1/4 heads, 140000 and 33 INT4 tokens", flush=True)
    c = Case(14, 2, 4, 1, 16, [140000, 33], [64, 1])
    _check(c)


def test_very_long_context():
    """270000 INT4 tokens (16875 blocks) in one sequence."""
    print("case: B=1 4/1 heads, 270000 INT4 tokens", flush=True)
    c = Case(15, 1, 4, 1, 16, [270000], [64])
    _check(c)


@pytest.mark.parametrize("seed", range(int(os.environ.get("HKV_DECODE_RANDOM_CASES", "24"))))
def test_random_geometries(seed):
    """Seeded random geometries against the float64 oracle in both schedules: batch 1-4,
    1-8 kv heads, n_rep 1-16, sink 0-100, ragged INT4 (0-6000) and recent (0-700) lengths,
    and forced range counts, so that single-kind and mixed ranges, partial blocks,
    empty zones and several placements of the XCD-local hand-off all occur."""
    from heterokv import ops
    rng = np.random.default_rng(1000 + seed)
    B = int(rng.integers(1, 5))
    hkv = int(rng.choice([1, 2, 4, 8]))
    nrep = int(rng.choice([1, 2, 4, 7, 8, 16]))
    sink = int(rng.choice([0, 16, 64, 100]))
    mids = [int(x) for x in rng.integers(0, 6001, B)]
    recents = [int(x) for x in rng.integers(0, 701, B)]
    for b in range(B):
        if sink + mids[b] + recents[b] == 0:
            recents[b] = 1
    splits = int(rng.choice([0, 0, 1, 3, 7, 64]))
    print("case: seed %d B=%d hkv=%d nrep=%d sink=%d mids=%s recents=%s splits=%d"
          % (seed, B, hkv, nrep, sink, mids, recents, splits), flush=True)
    c = Case(2000 + seed, B, hkv * nrep, hkv, sink, mids, recents)
    ws = ops.DecodeWorkspace(DEV)
    _check(c, splits=splits, workspace=ws)
    assert ws.error_flag() == 0


def test_reference_api_fused_dequant_attn_decode():
    """fused_dequant_attn_decode with the reference harness's inputs
    (unified_benchmark.py:142-164: per-head compress, float zero points)."""
    print("case: fused_dequant_attn_decode drop-in, 32 heads x 2000 tokens", flush=True)
    from heterokv import fused_dequant_attn_decode
    g = torch.Generator().manual_seed(12)
    H, S = 32, 2000
    q = torch.randn((1, H, 1, 128), generator=g).half()
    K = torch.randn((1, H, S, 128), generator=g).half()
    V = torch.randn((1, H, S, 128), generator=g).half()
    kc, ks, kz = oc.compress(K.numpy(), 128)
    vc, vs, vz = oc.compress(V.numpy(), 128)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV)  # noqa: E731
    out = fused_dequant_attn_decode(q.to(DEV), t(kc), t(ks).reshape(1, H, S), t(kz).reshape(1, H, S).float(),
                                    t(vc), t(vs).reshape(1, H, S), t(vz).reshape(1, H, S).float())
    assert out.shape == (1, H, 1, 128) and out.dtype == torch.float16
    kd = oa.dequant_rows(kc[0], ks.reshape(H, S), kz.reshape(H, S))
    vd = oa.dequant_rows(vc[0], vs.reshape(H, S), vz.reshape(H, S))
    ref = oa.attend(q[0].double().numpy(), kd, vd)
    err = np.abs(out[0].float().cpu().numpy() - ref).max()
    print("  max abs err %.3e" % err, flush=True)
    assert err <= TOL


def test_reference_api_fp32_q():
    """An fp32 q is rounded to fp16 for the kernel; in range it attends as its fp16
    rounding does, and a finite value beyond the fp16 range is reported (HKV_ERR_BIT_RANGE
    through the API's error word at the next call's check) instead of becoming inf
    silently."""
    print("case: fused_dequant_attn_decode with an fp32 q", flush=True)
    from heterokv import HeteroKVError, fused_dequant_attn_decode
    from heterokv import fused_dequant_attn as fda
    g = torch.Generator().manual_seed(14)
    H, S = 8, 300
    q = torch.randn((1, H, 1, 128), generator=g)
    K = torch.randn((1, H, S, 128), generator=g).half()
    V = torch.randn((1, H, S, 128), generator=g).half()
    kc, ks, kz = oc.compress(K.numpy(), 128)
    vc, vs, vz = oc.compress(V.numpy(), 128)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV)  # noqa: E731
    args = (t(kc), t(ks).reshape(1, H, S), t(kz).reshape(1, H, S), t(vc), t(vs).reshape(1, H, S),
            t(vz).reshape(1, H, S))
    out32 = fused_dequant_attn_decode(q.to(DEV), *args)
    out16 = fused_dequant_attn_decode(q.half().to(DEV), *args)
    assert out32.dtype == torch.float32
    assert (out32 - out16.float()).abs().max().item() <= 1e-3   # on-demand schedule: last-bit differences
    fda._errword(torch.device(DEV)).check()
    big = q.clone()
    big[0, 3, 0, 5] = 1e6
    fused_dequant_attn_decode(big.to(DEV), *args)
    with pytest.raises(HeteroKVError, match="fp16 range"):
        fda._errword(torch.device(DEV)).check()


def test_bad_block_id_sets_flag():
    print("case: decode with an out-of-range block id", flush=True)
    from heterokv import ops
    c = Case(13, 1, 32, 8, 16, [64], [16])
    ws = ops.DecodeWorkspace(DEV)
    c.bt[0, 1] = 10 ** 6
    c.run(workspace=ws)
    assert ws.error_flag() == 1
