"""GPU parity: MFMA chunked-prefill attention (hkv_prefill_attn) against the float64
oracle over [INT4 (Path C fp16 dequant) | fp16 zones | causal chunk]; 2e-3 max-abs."""
import math
import os

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import compressor as oc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 2e-3


def _poison_tails(pool, bt, mids, Hkv):
    """Writes NaN / inf scales and zero point 255 into the unused token slots of each
    sequence's last INT4 block (slots past its length), which the kernels must ignore."""
    from oracle import pool_format as pf
    data = pool.data.cpu().numpy()
    f32 = np.array([np.nan, np.inf, -np.inf], dtype=np.float32).view(np.uint8).reshape(3, 4)
    for b, m in enumerate(mids):
        if m % 16 == 0:
            continue
        rec = data[int(bt[b, (m - 1) // 16])]
        for h in range(Hkv):
            o = pf.offsets(h)
            for t in range(m % 16, 16):
                rec[o["ks"] + 4 * t:o["ks"] + 4 * t + 4] = f32[t % 3]
                rec[o["vs"] + 4 * t:o["vs"] + 4 * t + 4] = f32[(t + 1) % 3]
                rec[o["kz"] + t] = 255
                rec[o["vz"] + t] = 255
    pool.data.copy_(torch.from_numpy(data))


def _ulp16(x):
    """fp16 unit in the last place at |x| (subnormal spacing below 2^-14)."""
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -24)))
    return 2.0 ** np.maximum(e - 10, -24)


def _case(seed, B, Hq, Hkv, Sq, sink, mids, recents, causal=True, q_scale=1.0, poison=False, io_dtype=torch.float16,
          k_scale=1.0, v_scale=1.0):
    from heterokv import ops
    g = torch.Generator().manual_seed(seed)
    hist = sink + max(mids) + max(recents)
    K = torch.randn((B, Hkv, hist, 128), generator=g)
    K[..., [7, 31, 64, 100]] *= 8
    K = (K * k_scale).half()
    V = (torch.randn((B, Hkv, hist, 128), generator=g) * v_scale).half()
    # q, the chunk and the output in io_dtype (bf16 q/chunk values are exact in fp16 here)
    CK = torch.randn((B, Hkv, Sq, 128), generator=g).to(io_dtype)
    CV = torch.randn((B, Hkv, Sq, 128), generator=g).to(io_dtype)
    q = (torch.randn((B, Hq, Sq, 128), generator=g) * q_scale / math.sqrt(128)).to(io_dtype)
    zones = []
    if sink:
        zs = ops.F16Zone(B, Hkv, sink, DEV)
        zs.write(K[:, :, :sink].to(DEV), V[:, :, :sink].to(DEV), [0] * B)
        zones.append((zs, None, sink))
    if max(recents):
        rmax = max(recents)
        zr = ops.F16Zone(B, Hkv, rmax, DEV)
        kr = torch.zeros((B, Hkv, rmax, 128), dtype=torch.float16)
        vr = torch.zeros_like(kr)
        for b in range(B):
            s0 = sink + mids[b]
            kr[b, :, :recents[b]] = K[b, :, s0:s0 + recents[b]]
            vr[b, :, :recents[b]] = V[b, :, s0:s0 + recents[b]]
        zr.write(kr.to(DEV), vr.to(DEV), [0] * B)
        zones.append((zr, torch.tensor(recents, dtype=torch.int32).to(DEV), rmax))
    nbs = [(m + 15) // 16 for m in mids]
    nbmax = max(max(nbs), 1)
    pool = ops.Int4Pool(sum(nbs) + 1, Hkv, DEV)
    perm = torch.randperm(sum(nbs) + 1, generator=g).to(torch.int32)
    bt = torch.zeros((B, nbmax), dtype=torch.int32)
    off = 0
    for b in range(B):
        bt[b, :nbs[b]] = perm[off:off + nbs[b]]
        off += nbs[b]
        if mids[b]:
            ops.pack_tokens(pool, K[b:b + 1, :, sink:sink + mids[b]].to(DEV), V[b:b + 1, :, sink:sink + mids[b]].to(DEV),
                            [0], bt[b:b + 1])
    if poison:
        _poison_tails(pool, bt, mids, Hkv)
    out = ops.prefill_attention(q.to(DEV), zones=zones, pool=pool, block_table=bt.to(DEV),
                                int4_lens=torch.tensor(mids, dtype=torch.int32).to(DEV), int4_max_len=max(mids),
                                chunk_k=CK.to(DEV) if causal else None, chunk_v=CV.to(DEV) if causal else None)
    torch.cuda.synchronize()
    pool.check_errors()
    got = out.float().cpu().numpy()
    for b in range(B):
        m, r = mids[b], recents[b]
        ks = [K[b, :, :sink].double().numpy()]
        vs = [V[b, :, :sink].double().numpy()]
        if m:
            kc, kss, kz = oc.compress(K[b, :, sink:sink + m].numpy(), 128)
            vc, vss, vz = oc.compress(V[b, :, sink:sink + m].numpy(), 128)
            ks.append(oa.dequant_rows(kc, kss.reshape(Hkv, m), kz.reshape(Hkv, m)))
            vs.append(oa.dequant_rows(vc, vss.reshape(Hkv, m), vz.reshape(Hkv, m)))
        ks.append(K[b, :, sink + m:sink + m + r].double().numpy())
        vs.append(V[b, :, sink + m:sink + m + r].double().numpy())
        nh = sum(x.shape[1] for x in ks)
        mask = np.ones((Sq, nh), dtype=bool)
        if causal:
            ks.append(CK[b].double().numpy())
            vs.append(CV[b].double().numpy())
            mask = np.concatenate([mask, np.tril(np.ones((Sq, Sq), dtype=bool))], axis=1)
        ref = oa.attend(q[b].double().numpy(), np.concatenate(ks, 1), np.concatenate(vs, 1), mask=mask)
        # a bf16 output adds its own rounding: half an ulp, 2^-9 of the value; with V scaled
        # by v_scale the bar scales with it, plus half an fp16 ulp of the output
        tol = TOL * v_scale + (np.abs(ref) * 2.0 ** -9 if io_dtype == torch.bfloat16 else 0.0)
        if v_scale != 1.0:
            tol = tol + 0.5 * _ulp16(ref)
        err = np.abs(got[b] - ref)
        print("  b=%d max abs err %.3e" % (b, err.max()), flush=True)
        assert np.all(np.isfinite(got[b]))
        assert np.all(err <= tol)


def test_small_all_sources():
    print("case: prefill B=1 8/2 Sq=70 sink 20 + INT4 150 + recent 37 + causal", flush=True)
    _case(1, 1, 8, 2, 70, 20, [150], [37])


def test_gqa7_c5_geometry():
    print("case: prefill 28/4 Sq=33", flush=True)
    _case(2, 1, 28, 4, 33, 64, [300], [100])


def test_int4_only_no_causal():
    print("case: prefill INT4 only", flush=True)
    _case(3, 1, 4, 4, 50, 0, [500], [0], causal=False)


def test_causal_only_sharp():
    print("case: causal chunk only, sharp softmax", flush=True)
    _case(4, 1, 8, 2, 130, 0, [0], [0], q_scale=8.0)


def test_ragged_batch():
    print("case: prefill B=2 ragged", flush=True)
    _case(5, 2, 8, 2, 64, 64, [1000, 17], [200, 3])


def test_garbage_in_unused_tail_slots():
    print("case: prefill with NaN/inf scales and zero point 255 in the slots past each INT4 length", flush=True)
    _case(9, 2, 8, 2, 40, 16, [150, 33], [20, 5], poison=True)
    _case(10, 1, 4, 4, 20, 0, [7], [0], causal=False, poison=True)


def test_bf16_query_chunk_and_output():
    print("case: prefill with bf16 q, chunk and output, 16/4 Sq=100, sink 64 + INT4 300 + recent 50", flush=True)
    _case(11, 1, 16, 4, 100, 64, [300], [50], io_dtype=torch.bfloat16)
    _case(12, 2, 8, 8, 37, 0, [0, 70], [20, 0], io_dtype=torch.bfloat16)


def test_small_magnitude_keys():
    """K rows scaled by 3e-5, so nearly all INT4 K scales lie below fp16's normal range
    (2^-14), with q scaled so that the scores vary by a few log2 units.  The staging rounds
    each scale to fp16 (a subnormal here) and then the product; with the softmax scale on
    the queries, not folded into the keys, a CPU emulation of this case stays at 1.0e-4 of
    the float64 oracle (6.3e-4 with the scale folded into the keys, 7.5e-5 with every
    product rounded once from fp32)."""
    print("case: prefill with K scales below 2^-14 (K x 3e-5, q x 1e5), 8/2 Sq=48, 16 + 700 INT4 + 40", flush=True)
    _case(13, 1, 8, 2, 48, 16, [700], [40], causal=False, k_scale=3e-5, q_scale=1e5)


def test_small_magnitude_values():
    """V rows scaled by 3e-5 (V scales ~1e-5, below 2^-14): the output matches the oracle to
    2e-3 of the V scale plus half an fp16 ulp of the output."""
    print("case: prefill with V scales below 2^-14 (V x 3e-5), 8/2 Sq=48, 16 + 700 INT4 + 40", flush=True)
    _case(14, 1, 8, 2, 48, 16, [700], [40], causal=False, v_scale=3e-5)


def test_medium_c4_like():
    print("case: prefill 32/8 Sq=256, 64 + 4096 INT4 + 256 recent + causal", flush=True)
    _case(6, 1, 32, 8, 256, 64, [4096], [256])


def test_qwen2_7b_gqa_geometry():
    print("case: prefill 28/4 (n_rep 7) Sq=100, 64 + 600 INT4 + 300 recent + causal", flush=True)
    _case(8, 1, 28, 4, 100, 64, [600], [300])


def test_reference_api_fused_dequant_attn_forward():
    print("case: fused_dequant_attn_forward drop-in", flush=True)
    from heterokv import fused_dequant_attn_forward
    g = torch.Generator().manual_seed(7)
    H, S, Sq = 4, 333, 40
    q = torch.randn((1, H, Sq, 128), generator=g).half()
    K = torch.randn((1, H, S, 128), generator=g).half()
    V = torch.randn((1, H, S, 128), generator=g).half()
    kc, ks, kz = oc.compress(K.numpy(), 128)
    vc, vs, vz = oc.compress(V.numpy(), 128)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV)  # noqa: E731
    out = fused_dequant_attn_forward(q.to(DEV), t(kc), t(ks).reshape(1, H, S), t(kz).reshape(1, H, S).float(),
                                     t(vc), t(vs).reshape(1, H, S), t(vz).reshape(1, H, S).float())
    kd = oa.dequant_rows(kc[0], ks.reshape(H, S), kz.reshape(H, S))
    vd = oa.dequant_rows(vc[0], vs.reshape(H, S), vz.reshape(H, S))
    ref = oa.attend(q[0].double().numpy(), kd, vd)
    err = np.abs(out[0].float().cpu().numpy() - ref).max()
    print("  max abs err %.3e" % err, flush=True)
    assert out.shape == (1, H, Sq, 128) and err <= TOL


@pytest.mark.parametrize("seed", range(int(os.environ.get("HKV_PREFILL_RANDOM_CASES", "12"))))
def test_random_geometries(seed):
    """Seeded random shapes: batch 1-3, 1-4 kv heads, GQA ratio 1-8, 1-200 queries, ragged
    INT4 / recent lengths (zeros included), sink on or off, with or without the causal chunk,
    and a softmax sharpness between flat and sharp."""
    rng = np.random.default_rng(1000 + seed)
    B = int(rng.integers(1, 4))
    Hkv = int(rng.integers(1, 5))
    nrep = int(rng.integers(1, 9))
    Sq = int(rng.integers(1, 201))
    sink = int(rng.choice([0, 1, 17, 64, 80]))
    mids = [int(rng.choice([0, int(rng.integers(1, 700))])) for _ in range(B)]
    recents = [int(rng.integers(0, 300)) for _ in range(B)]
    causal = bool(rng.integers(0, 2))
    if not causal and (sink == 0 and min(m + r for m, r in zip(mids, recents)) == 0):
        causal = True   # every row must see at least one token
    q_scale = float(rng.choice([0.5, 1.0, 4.0]))
    print("case: prefill seed %d B=%d %d/%d Sq=%d sink %d mids %s recents %s causal %s q_scale %g" % (
        seed, B, Hkv * nrep, Hkv, Sq, sink, mids, recents, causal, q_scale), flush=True)
    _case(2000 + seed, B, Hkv * nrep, Hkv, Sq, sink, mids, recents, causal=causal, q_scale=q_scale)
