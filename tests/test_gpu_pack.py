"""GPU parity: the quantize+pack append kernel (hkv_pack_tokens), the reference-layout
repacker and unpacker, and the fp16 zone writer, byte for byte against the oracle's
compressor and its restatement of the documented record layout."""
import numpy as np
import pytest
import torch

from oracle import compressor as oc
from oracle import pool_format as pf

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _expected_pool(k, v, start, bt_row, num_blocks):
    """Records the pool must hold after packing k, v [H, T, 128] (fp16 numpy) at INT4
    slot `start` of a sequence whose block table row is bt_row (all else zero)."""
    H, T, _ = k.shape
    kc, ks, kz = oc.compress(k, 128)
    vc, vs, vz = oc.compress(v, 128)
    ks, kz, vs, vz = ks.reshape(H, T), kz.reshape(H, T), vs.reshape(H, T), vz.reshape(H, T)
    rb = pf.record_bytes(H)
    pool = np.zeros((num_blocks, rb), dtype=np.uint8)
    nlb = (start + T + 15) // 16
    for lb in range(start // 16, nlb):
        lo = max(start, lb * 16) - lb * 16
        hi = min(start + T, lb * 16 + 16) - lb * 16
        KC = np.zeros((H, 16, 128), np.uint8)
        VC = np.zeros((H, 16, 128), np.uint8)
        KS = np.zeros((H, 16), np.float32)
        VS = np.zeros((H, 16), np.float32)
        KZ = np.zeros((H, 16), np.uint8)
        VZ = np.zeros((H, 16), np.uint8)
        t0 = lb * 16 + lo - start
        t1 = lb * 16 + hi - start
        KC[:, lo:hi] = kc[:, t0:t1]
        VC[:, lo:hi] = vc[:, t0:t1]
        KS[:, lo:hi] = ks[:, t0:t1]
        VS[:, lo:hi] = vs[:, t0:t1]
        KZ[:, lo:hi] = kz[:, t0:t1]
        VZ[:, lo:hi] = vz[:, t0:t1]
        pool[bt_row[lb]] = pf.build_record(KC, VC, KS, VS, KZ, VZ)
    return pool, (kc, ks.reshape(-1), kz.reshape(-1)), (vc, vs.reshape(-1), vz.reshape(-1))


def _rand_kv(seed, H, T):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn((1, H, T, 128), generator=g)
    k[..., [7, 31, 64, 100]] *= 8
    v = torch.randn((1, H, T, 128), generator=g)
    return k.half(), v.half()


@pytest.mark.parametrize("H,T,start", [(8, 100, 5), (8, 4096, 0), (4, 33, 16), (2, 1, 31), (8, 16, 0)])
def test_pack_tokens_bytes(H, T, start):
    print("case: pack_tokens H=%d T=%d start=%d" % (H, T, start), flush=True)
    from heterokv import ops
    k, v = _rand_kv(H * 1000 + T, H, T)
    nlb = (start + T + 15) // 16
    nblocks = nlb + 3
    perm = torch.randperm(nblocks, generator=torch.Generator().manual_seed(T))[:nlb].to(torch.int32)
    pool = ops.Int4Pool(nblocks, H, DEV)
    ops.pack_tokens(pool, k.to(DEV), v.to(DEV), torch.tensor([start], dtype=torch.int32), perm[None])
    exp, kref, vref = _expected_pool(k[0].numpy(), v[0].numpy(), start, perm.numpy(), nblocks)
    got = pool.data.cpu().numpy()
    assert np.array_equal(got, exp)
    pool.check_errors()
    # unpack the sequence's INT4 slots [start, start+T) back to the reference layout
    for which, ref in ((0, kref), (1, vref)):
        codes, scales, zps = ops.unpack_tokens(pool, perm, start + T, which)
        assert np.array_equal(codes[:, start:].cpu().numpy(), ref[0])
        assert np.array_equal(scales.reshape(H, -1)[:, start:].cpu().numpy().reshape(-1), ref[1])
        assert np.array_equal(zps.reshape(H, -1)[:, start:].cpu().numpy().reshape(-1), ref[2])


def test_pack_tokens_bf16_rows():
    """bf16 K/V: the values widen to float32 exactly, so the records equal the oracle's
    compression of those float32 values."""
    print("case: pack_tokens bf16 H=4 T=77 start=3", flush=True)
    from heterokv import ops
    k, v = _rand_kv(4077, 4, 77)
    kb, vb = k.float().bfloat16(), v.float().bfloat16()
    start, nlb = 3, (3 + 77 + 15) // 16
    bt = torch.arange(nlb, dtype=torch.int32)
    pool = ops.Int4Pool(nlb, 4, DEV)
    ops.pack_tokens(pool, kb.to(DEV), vb.to(DEV), torch.tensor([start], dtype=torch.int32), bt[None])
    exp, _, _ = _expected_pool(kb[0].float().numpy(), vb[0].float().numpy(), start, bt.numpy(), nlb)
    assert np.array_equal(pool.data.cpu().numpy(), exp)
    pool.check_errors()


def test_pack_tokens_strided_rows_match_contiguous():
    """Rows 129 elements apart (no 16-byte alignment: the per-element load path) pack to
    the same bytes as the contiguous copy (the 16-byte load path)."""
    print("case: pack_tokens strided rows H=8 T=50 start=9", flush=True)
    from heterokv import ops
    g = torch.Generator().manual_seed(129)
    big_k = torch.randn((1, 8, 50, 129), generator=g).half().to(DEV)
    big_v = torch.randn((1, 8, 50, 129), generator=g).half().to(DEV)
    k, v = big_k[..., :128], big_v[..., :128]
    assert k.stride(2) == 129
    start, nlb = 9, (9 + 50 + 15) // 16
    bt = torch.arange(nlb, dtype=torch.int32)[None]
    sp = torch.tensor([start], dtype=torch.int32)
    p1, p2 = ops.Int4Pool(nlb, 8, DEV), ops.Int4Pool(nlb, 8, DEV)
    ops.pack_tokens(p1, k, v, sp, bt)
    ops.pack_tokens(p2, k.contiguous(), v.contiguous(), sp, bt)
    assert torch.equal(p1.data, p2.data)
    exp, _, _ = _expected_pool(k[0].cpu().numpy(), v[0].cpu().numpy(), start, bt[0].numpy(), nlb)
    assert np.array_equal(p1.data.cpu().numpy(), exp)
    p1.check_errors()


def test_pack_tokens_nan_and_inf_tokens():
    """A token row holding a NaN gets a NaN scale and zero codes/zp, as torch's min/max
    propagate NaN; rows with infinities follow the same float32 steps as the oracle."""
    print("case: pack_tokens NaN / inf rows", flush=True)
    from heterokv import ops
    H, T = 2, 20
    k, v = _rand_kv(77, H, T)
    k[0, 0, 3, 17] = float("nan")
    k[0, 1, 16, :] = float("nan")
    v[0, 0, 5, 0] = float("inf")
    v[0, 1, 19, 100] = float("-inf")
    k[0, 1, 2, 1], k[0, 1, 2, 2] = float("inf"), float("-inf")
    perm = torch.tensor([1, 0], dtype=torch.int32)
    pool = ops.Int4Pool(3, H, DEV)
    ops.pack_tokens(pool, k.to(DEV), v.to(DEV), torch.tensor([0], dtype=torch.int32), perm[None])
    pool.check_errors()
    for which, x in ((0, k), (1, v)):
        rc, rs, rz = oc.compress(x[0].numpy(), 128)
        codes, scales, zps = ops.unpack_tokens(pool, perm, T, which)
        got_s = scales.cpu().numpy().reshape(-1)
        assert np.array_equal(codes.cpu().numpy(), rc)
        assert np.array_equal(np.isnan(got_s), np.isnan(rs))
        assert np.array_equal(got_s[~np.isnan(rs)].view(np.uint32), rs[~np.isnan(rs)].view(np.uint32))
        assert np.array_equal(zps.cpu().numpy().reshape(-1), rz)
    assert np.isnan(ops.unpack_tokens(pool, perm, T, 0)[1].cpu().numpy().reshape(H, T)[[0, 1], [3, 16]]).all()


def test_incremental_append_equals_one_shot():
    print("case: pack in pieces 37 + 1 + 1 + 90 vs one shot", flush=True)
    from heterokv import ops
    H, T = 8, 129
    k, v = _rand_kv(7, H, T)
    nb = (T + 15) // 16
    bt = torch.arange(nb, dtype=torch.int32)[None]
    one = ops.Int4Pool(nb, H, DEV)
    ops.pack_tokens(one, k.to(DEV), v.to(DEV), [0], bt)
    inc = ops.Int4Pool(nb, H, DEV)
    pos = 0
    for n in (37, 1, 1, 90):
        ops.pack_tokens(inc, k[:, :, pos:pos + n].to(DEV), v[:, :, pos:pos + n].to(DEV), [pos], bt)
        pos += n
    assert torch.equal(one.data, inc.data)


def test_repack_reference_layout_equals_pack():
    print("case: repack_codes(oracle codes) == pack_tokens", flush=True)
    from heterokv import ops
    H, T = 8, 200
    k, v = _rand_kv(11, H, T)
    nb = (T + 15) // 16
    bt = torch.arange(nb, dtype=torch.int32)[None]
    a = ops.Int4Pool(nb, H, DEV)
    ops.pack_tokens(a, k.to(DEV), v.to(DEV), [0], bt)
    kc, ks, kz = oc.compress(k[0].numpy(), 128)
    vc, vs, vz = oc.compress(v[0].numpy(), 128)
    b = ops.Int4Pool(nb, H, DEV)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV)  # noqa: E731
    ops.repack_codes(b, t(kc)[None], t(vc)[None], t(ks).reshape(1, H, T), t(vs).reshape(1, H, T),
                     t(kz).reshape(1, H, T).float(), t(vz).reshape(1, H, T).float(), [0], bt)
    assert torch.equal(a.data, b.data)


def test_batched_pack_two_sequences():
    print("case: batch of 2 with different starts", flush=True)
    from heterokv import ops
    H, T = 4, 40
    g = torch.Generator().manual_seed(3)
    k = torch.randn((2, H, T, 128), generator=g).half()
    v = torch.randn((2, H, T, 128), generator=g).half()
    starts = [3, 20]
    bt = torch.tensor([[0, 1, 2, 3, 4], [9, 8, 7, 6, 5]], dtype=torch.int32)
    pool = ops.Int4Pool(10, H, DEV)
    ops.pack_tokens(pool, k.to(DEV), v.to(DEV), torch.tensor(starts, dtype=torch.int32), bt)
    got = pool.data.cpu().numpy()
    for b in range(2):
        exp, _, _ = _expected_pool(k[b].numpy(), v[b].numpy(), starts[b], bt[b].numpy(), 10)
        used = sorted(set(bt[b, starts[b] // 16:(starts[b] + T + 15) // 16].tolist()))
        assert np.array_equal(got[used], exp[used])


@pytest.mark.parametrize("start", [0, 21])
def test_start_by_value_equals_start_array(start):
    """One host start for every sequence is passed by value (no start array); the records
    equal those of the same start given as a device array."""
    print("case: pack start %d by value vs device array" % start, flush=True)
    from heterokv import ops
    H, T = 4, 50
    g = torch.Generator().manual_seed(5)
    k = torch.randn((2, H, T, 128), generator=g).half().to(DEV)
    v = torch.randn((2, H, T, 128), generator=g).half().to(DEV)
    bt = torch.tensor([[0, 1, 2, 3, 4, 5], [11, 10, 9, 8, 7, 6]], dtype=torch.int32)
    by_value = ops.Int4Pool(12, H, DEV)
    ops.pack_tokens(by_value, k, v, [start, start], bt)
    by_array = ops.Int4Pool(12, H, DEV)
    ops.pack_tokens(by_array, k, v, torch.tensor([start, start], dtype=torch.int32).to(DEV), bt)
    torch.cuda.synchronize()
    assert torch.equal(by_value.data, by_array.data)
    by_value.check_errors()
    by_array.check_errors()


def test_out_of_range_block_id_is_flagged_not_written():
    print("case: bad block id", flush=True)
    from heterokv import HeteroKVError, ops
    k, v = _rand_kv(5, 2, 16)
    pool = ops.Int4Pool(2, 2, DEV)
    ops.pack_tokens(pool, k.to(DEV), v.to(DEV), [0], torch.tensor([[7]], dtype=torch.int32))
    assert int(pool.data.abs().sum().item()) == 0
    with pytest.raises(HeteroKVError):
        pool.check_errors()


def test_f16_zone_write_read_and_ring():
    print("case: fp16 zone write/read", flush=True)
    from heterokv import ops
    H, cap = 4, 48
    g = torch.Generator().manual_seed(9)
    k = torch.randn((1, H, 40, 128), generator=g).half()
    v = torch.randn((1, H, 40, 128), generator=g).half()
    z = ops.F16Zone(1, H, cap, DEV)
    z.write(k.to(DEV), v.to(DEV), [0])
    rk, rv = z.read(40)
    assert torch.equal(rk.cpu(), k) and torch.equal(rv.cpu(), v)
    # V tiles follow the documented [g][c][n][i] layout
    tile = z.v[0, 1, 0].cpu().reshape(4, 16, 8, 4).numpy()
    assert np.array_equal(tile, pf.v_tile(v[0, 1, :16].numpy()))
    # ring: 20 more tokens at logical slot 40 wrap to slots 40..47, 0..11
    k2 = torch.randn((1, H, 20, 128), generator=g).half()
    v2 = torch.randn((1, H, 20, 128), generator=g).half()
    z.write(k2.to(DEV), v2.to(DEV), [40], ring=True)
    rk, rv = z.read(48)
    assert torch.equal(rk[0, :, 40:48].cpu(), k2[0, :, :8]) and torch.equal(rk[0, :, :12].cpu(), k2[0, :, 8:])
    assert torch.equal(rv[0, :, 12:40].cpu(), v[0, :, 12:40])


def test_f16_zone_write_per_sequence_slots_and_uniform_base():
    print("case: fp16 zone write, per-sequence slots vs by-value base", flush=True)
    from heterokv import ops
    B, H, cap = 3, 2, 32
    g = torch.Generator().manual_seed(10)
    k = torch.randn((B, H, 5, 128), generator=g).half()
    v = torch.randn((B, H, 5, 128), generator=g).half()
    z = ops.F16Zone(B, H, cap, DEV)
    z.write(k.to(DEV), v.to(DEV), torch.tensor([0, 7, 29], dtype=torch.int32), ring=True)
    rk, rv = z.read(cap)
    for b, s in enumerate([0, 7, 29]):
        slots = [(s + t) % cap for t in range(5)]
        assert torch.equal(rk[b][:, slots].cpu(), k[b]) and torch.equal(rv[b][:, slots].cpu(), v[b])
    z2 = ops.F16Zone(B, H, cap, DEV)
    z2.write(k.to(DEV), v.to(DEV), 11)
    z3 = ops.F16Zone(B, H, cap, DEV)
    z3.write(k.to(DEV), v.to(DEV), torch.tensor([11, 11, 11], dtype=torch.int32))
    assert torch.equal(z2.k, z3.k) and torch.equal(z2.v, z3.v)
    rk, _ = z2.read(16)
    assert torch.equal(rk[:, :, 11:16].cpu(), k)
