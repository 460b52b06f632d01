"""Pins the oracle's compressor restatement (oracle/hkv_oracle.c) to the reference
KVCompressor (src/quantization/kv_compressor.py:66-132) with hand-computed known
answers, invariants and library routines.  CPU only."""
import numpy as np
import pytest
import torch

from oracle import compressor as oc


def _row(vals, n=128, fill=0.0):
    r = np.full(n, fill, dtype=np.float32)
    r[: len(vals)] = vals
    return r


# ------------------------------------------------------------------ known answers
def test_kat_identity_row():
    # values 0..15 repeated: min 0, max 15 -> scale 1, zp 0, codes = values
    x = np.tile(np.arange(16, dtype=np.float32), 8)
    codes, scales, zps = oc.compress(x.astype(np.float16), 128)
    assert scales[0] == np.float32(1.0) and zps[0] == 0
    assert np.array_equal(codes, x.astype(np.uint8))


def test_kat_signed_row_half_even_and_clamp():
    # min -7.5, max 7.5: scale = 15/15 = 1; zp = round(7.5) = 8 (half to even);
    # code(-7.5) = round(0.5) = 0 (even); code(7.5) = round(15.5) = 16 -> clamp 15;
    # code(0) = 8; code(-5.5) = round(2.5) = 2; code(-4.5) = round(3.5) = 4; code(1.5) = round(9.5) = 10
    x = _row([-7.5, 7.5, 0.0, -5.5, -4.5, 1.5])
    codes, scales, zps = oc.compress(x, 128)
    assert scales[0] == np.float32(1.0)
    assert zps[0] == 8
    assert list(codes[:6]) == [0, 15, 8, 2, 4, 10]
    assert np.all(codes[6:] == 8)


def test_kat_zero_point_rounds_half_to_even_downwards():
    # min -2.5, max 12.5: scale 1, zp = round(2.5) = 2 (not 3); code(12.5) = round(14.5) = 14
    x = _row([-2.5, 12.5])
    codes, scales, zps = oc.compress(x, 128)
    assert zps[0] == 2 and scales[0] == np.float32(1.0)
    assert codes[0] == 0 and codes[1] == 14  # -2.5 + 2 = -0.5 -> -0 -> 0


def test_kat_constant_rows_saturate():
    # constant c over a full group: scale = max(0/15, 1e-8) = 1e-8 (float32);
    # c > 0: zp = clamp(round(-c/1e-8)) = 0, codes = clamp(round(c/1e-8)) = 15
    # c < 0: zp = 15, codes = clamp(round(c/1e-8 + 15)) = 0;  c = 0: zp 0, codes 0
    for c, zp, code in ((0.75, 0, 15), (-0.75, 15, 0), (0.0, 0, 0)):
        codes, scales, zps = oc.compress(np.full(128, c, dtype=np.float32), 128)
        assert scales[0] == np.float32(1e-8)
        assert zps[0] == zp and np.all(codes == code), (c, zps[0], codes[:4])


def test_kat_nonnegative_row_has_zero_zp():
    x = _row([1.0, 4.0, 16.0], fill=1.0)  # min 1 > 0 -> -min/scale < 0 -> zp clamps to 0
    codes, scales, zps = oc.compress(x, 128)
    assert zps[0] == 0
    assert scales[0] == np.float32(1.0)  # (16 - 1) / 15
    assert list(codes[:3]) == [1, 4, 15]  # round(16/1 + 0) = 16 -> 15


def test_kat_padding_takes_part_in_min_max():
    # shape (1,3,7,11): 231 values, group 128 -> group 1 holds 103 values + 25 zero pads.
    x = (np.arange(231, dtype=np.float32) + 10.0).reshape(1, 3, 7, 11)
    codes, scales, zps = oc.compress(x, 128)
    assert codes.shape == x.shape and scales.shape == (2,) and zps.shape == (2,)
    # group 0: min 10, max 137 (no padding) -> scale 127/15
    assert scales[0] == np.float32(np.float32(127.0) / np.float32(15.0))
    # group 1: real values 138..240 plus zeros -> min 0, max 240 -> scale 16 exactly, zp 0
    assert scales[1] == np.float32(16.0) and zps[1] == 0
    flat = codes.reshape(-1)
    assert flat[128] == 9  # round(138/16 = 8.625) = 9
    assert flat[230] == 15  # round(240/16 = 15)


def test_kat_group64():
    x = np.concatenate([np.linspace(0, 15, 64, dtype=np.float32), np.linspace(-3, 0, 64, dtype=np.float32)])
    codes, scales, zps = oc.compress(x, 64)
    assert scales.shape == (2,)
    assert scales[0] == np.float32(1.0) and zps[0] == 0
    assert scales[1] == np.float32(np.float32(3.0) / np.float32(15.0)) and zps[1] == 15


def test_kat_decompress():
    codes = np.array([0, 15, 8, 3], dtype=np.uint8)
    out = oc.decompress(codes, np.array([0.5], np.float32), np.array([8], np.uint8), group_size=4,
                        out_dtype=np.float32)
    assert list(out) == [-4.0, 3.5, 0.0, -2.5]
    # fp16 output rounds the float32 product to nearest even: (1-0)*(1+2^-11) -> 1.0
    s = np.float32(1.0 + 2.0 ** -11)
    o16 = oc.decompress(np.array([1], np.uint8), np.array([s]), np.array([0], np.uint8), group_size=1)
    assert o16.dtype == np.float16 and o16[0] == np.float16(1.0)
    s = np.float32(1.0 + 3 * 2.0 ** -11)  # halfway between 1+2^-10 and 1+2^-9 -> even (1+2^-9)
    o16 = oc.decompress(np.array([1], np.uint8), np.array([s]), np.array([0], np.uint8), group_size=1)
    assert o16[0] == np.float16(1.0 + 2.0 ** -9)


# ------------------------------------------------------------------ invariants
def test_invariants_random():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((1, 8, 256, 128)) * rng.uniform(0.1, 5, (1, 8, 256, 1))).astype(np.float16)
    codes, scales, zps = oc.compress(x, 128)
    g = x.astype(np.float32).reshape(-1, 128)
    mn, mx = g.min(1), g.max(1)
    assert codes.max() <= 15 and zps.max() <= 15
    assert np.all(scales >= np.float32(1e-8))
    assert np.array_equal(scales, np.maximum((mx - mn) / np.float32(15.0), np.float32(1e-8)))
    deq = oc.decompress(codes, scales, zps, 128, out_dtype=np.float32).reshape(-1, 128)
    # error bound: |x' - x| <= scale/2 wherever the zero point was not clamped
    unclamped = (np.rint(-mn / scales) >= 0) & (np.rint(-mn / scales) <= 15)
    err = np.abs(deq - g)[unclamped]
    bound = (scales[unclamped] / 2 * (1 + 1e-5) + 1e-6)[:, None]
    assert np.all(err <= np.broadcast_to(bound, err.shape))


def test_matches_torch_cpu_ops_random():
    """The same float32 operations spelled with torch's CPU kernels (the library the
    reference runs on): the C restatement must agree bit for bit."""
    rng = np.random.default_rng(1)
    for shape, gsz, dt in [((1, 32, 16, 128), 128, np.float16), ((1, 4, 1984, 64), 64, np.float16),
                           ((1, 8, 123, 128), 128, np.float32), ((1, 3, 7, 11), 128, np.float16),
                           ((1, 8, 1999, 64), 128, np.float16)]:
        x = (rng.standard_normal(shape) * 3).astype(dt)
        codes, scales, zps = oc.compress(x, gsz)
        t = torch.from_numpy(x).to(torch.float32).reshape(-1)
        pad = (gsz - t.numel() % gsz) % gsz
        t = torch.nn.functional.pad(t, (0, pad)).reshape(-1, gsz)
        s = torch.clamp((t.max(-1, keepdim=True).values - t.min(-1, keepdim=True).values) / 15, min=1e-8)
        z = torch.clamp(torch.round(-t.min(-1, keepdim=True).values / s), 0, 15).to(torch.uint8)
        q = torch.clamp(torch.round(t / s + z.float()), 0, 15).to(torch.uint8).reshape(-1)[: x.size]
        assert np.array_equal(scales, s.reshape(-1).numpy())
        assert np.array_equal(zps, z.reshape(-1).numpy())
        assert np.array_equal(codes.reshape(-1), q.numpy())


def test_nan_and_inf_rows_match_torch_ops():
    """torch's min/max propagate NaN (kv_compressor.py:76-77): a group holding a NaN gets
    a NaN scale, and its zero point and codes convert to 0 (torch's NaN -> uint8 is 0 on
    the CPU, checked here too).  Infinite values go through the same float32 steps."""
    assert torch.tensor([float("nan")]).to(torch.uint8).item() == 0
    rows = np.zeros((6, 128), np.float32)
    rows[0, 5] = np.nan
    rows[1] = np.linspace(-3, 3, 128)
    rows[1, 127] = np.nan
    rows[2, 0] = np.inf
    rows[3, 9] = -np.inf
    rows[4, 1], rows[4, 2] = np.inf, -np.inf
    rows[5] = np.nan
    codes, scales, zps = oc.compress(rows, 128)
    t = torch.from_numpy(rows)
    s = torch.clamp((t.max(-1, keepdim=True).values - t.min(-1, keepdim=True).values) / 15, min=1e-8)
    z = torch.clamp(torch.round(-t.min(-1, keepdim=True).values / s), 0, 15).to(torch.uint8)
    q = torch.clamp(torch.round(t / s + z.float()), 0, 15).to(torch.uint8)
    sr = s.reshape(-1).numpy()
    assert np.array_equal(np.isnan(scales), np.isnan(sr))
    assert np.array_equal(scales[~np.isnan(sr)], sr[~np.isnan(sr)])
    assert list(np.isnan(scales)) == [True, True, False, False, False, True]
    assert np.array_equal(zps, z.reshape(-1).numpy())
    assert np.array_equal(codes, q.numpy())
    assert not codes[[0, 1, 5]].any() and not zps[[0, 1, 5]].any()
    # decompress (kv_compressor.py:131): (q - zp) * scale, so a NaN group comes back
    # all NaN, and so does every 0-code element of a group with an infinite scale
    deq = oc.decompress(codes, scales, zps, 128, out_dtype=np.float32)
    ref = ((q.float() - z.float()) * s).numpy()
    assert np.array_equal(np.isnan(deq), np.isnan(ref))
    assert np.array_equal(deq[~np.isnan(ref)], ref[~np.isnan(ref)])
    assert np.isnan(deq[[0, 1, 5]]).all()


def test_bf16_input():
    rng = np.random.default_rng(2)
    x32 = rng.standard_normal(512).astype(np.float32)
    bf = oc.f32_to_bf16_bits(x32)
    assert np.array_equal(bf, torch.from_numpy(x32).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))
    codes, scales, zps = oc.compress(bf, 128)
    codes2, scales2, zps2 = oc.compress(oc.bf16_bits_to_f32(bf), 128)
    assert np.array_equal(codes, codes2) and np.array_equal(scales, scales2) and np.array_equal(zps, zps2)


# ------------------------------------------------------------------ conversions vs numpy
def test_f16_conversions_match_numpy():
    rng = np.random.default_rng(3)
    special = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 6.1e-5, 6.0e-8,
                        2.98e-8, 2.99e-8, 1e-10, np.inf, -np.inf, 5.96e-8, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11],
                       dtype=np.float32)
    vals = np.concatenate([special, rng.standard_normal(100000).astype(np.float32) * 10,
                           (rng.standard_normal(10000) * 1e-5).astype(np.float32)])
    got = oc.f32_to_f16_bits(vals)
    assert np.array_equal(got, vals.astype(np.float16).view(np.uint16))
    allbits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = oc.f16_bits_to_f32(allbits)
    ref = allbits.view(np.float16).astype(np.float32)
    same = (f == ref) | (np.isnan(f) & np.isnan(ref))
    assert np.all(same)


def test_relative_error_definition():
    x = np.tile(np.arange(16, dtype=np.float32), 8).astype(np.float16)
    codes, scales, zps = oc.compress(x, 128)
    assert oc.relative_error(x, codes, scales, zps) == pytest.approx(0.0, abs=1e-12)
    x2 = np.array([0.0, 1.0, 2.0, 3.1] + [0.0] * 124, dtype=np.float16)
    c2, s2, z2 = oc.compress(x2, 128)
    deq = oc.decompress(c2, s2, z2, 128).astype(np.float64)
    expect = np.abs(deq - x2.astype(np.float64)).mean() / (np.abs(x2.astype(np.float64)).mean() + 1e-8) * 100
    assert oc.relative_error(x2, c2, s2, z2) == pytest.approx(expect)
