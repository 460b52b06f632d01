"""GPU parity: KVCompressor (hkv_quantize_groups / hkv_dequantize_groups) against the
oracle restatement of kv_compressor.py:66-132, bit for bit."""
import numpy as np
import pytest
import torch

from oracle import compressor as oc

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
OUTLIER_CHANNELS = (7, 31, 64, 100)


def c1_inputs(seed=0, seq=4096):
    """Config 1: K, V [1, 8, seq, 128] fp16 from N(0,1), K channels 7/31/64/100 scaled x8."""
    g = torch.Generator().manual_seed(seed)
    k = torch.randn((1, 8, seq, 128), generator=g)
    v = torch.randn((1, 8, seq, 128), generator=g)
    k[..., list(OUTLIER_CHANNELS)] *= 8
    return k.to(torch.float16), v.to(torch.float16)


def _np_bits(t):
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def test_c1_round_trip_bit_exact():
    print("case: C1 [1,8,4096,128] quantize/dequantize vs oracle", flush=True)
    from heterokv import KVCompressor
    comp = KVCompressor(group_size=128)
    k, v = c1_inputs()
    for name, x in (("K", k), ("V", v)):
        codes, scales, zps = comp.compress(x.to(DEV))
        oc_codes, oc_scales, oc_zps = oc.compress(x.numpy(), 128)
        assert codes.shape == x.shape and scales.shape == (8 * 4096,) and zps.shape == (8 * 4096,)
        assert np.array_equal(codes.cpu().numpy(), oc_codes), name
        assert np.array_equal(scales.cpu().numpy().view(np.uint32), oc_scales.view(np.uint32)), name
        assert np.array_equal(zps.cpu().numpy(), oc_zps), name
        deq = comp.decompress(codes, scales, zps)
        assert np.array_equal(deq.cpu().numpy().view(np.uint16),
                              oc.decompress(oc_codes, oc_scales, oc_zps).view(np.uint16)), name
        rel = comp.relative_error(x.to(DEV), codes, scales, zps)
        rel_o = oc.relative_error(x.numpy(), oc_codes, oc_scales, oc_zps)
        assert rel == pytest.approx(rel_o, rel=1e-4), name
        print("  %s relative_error = %.3f%% (oracle %.3f%%)" % (name, rel, rel_o), flush=True)


# the reference's own test matrix (test_kv_compressor_fix.py:42-59)
SHAPES = [(1, 32, 16, 128), (1, 4, 1984, 64), (1, 8, 512, 64), (1, 8, 123, 128), (1, 8, 1, 128),
          (1, 8, 1999, 64), (1, 3, 7, 11)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("group_size", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_reference_shape_matrix(shape, group_size, dtype):
    print("case: compress", shape, group_size, dtype, flush=True)
    from heterokv import KVCompressor
    comp = KVCompressor(group_size=group_size)
    g = torch.Generator().manual_seed(hash((shape, group_size)) % 1000)
    x = torch.randn(shape, generator=g).to(dtype)
    codes, scales, zps = comp.compress(x.to(DEV))
    oc_codes, oc_scales, oc_zps = oc.compress(_np_bits(x), group_size)
    assert np.array_equal(codes.cpu().numpy(), oc_codes)
    assert np.array_equal(scales.cpu().numpy(), oc_scales)
    assert np.array_equal(zps.cpu().numpy(), oc_zps)
    out_dt = "bf16" if dtype == torch.bfloat16 else np.float16
    deq = comp.decompress(codes, scales, zps, target_dtype=dtype).cpu()
    assert np.array_equal(_np_bits(deq).view(np.uint16),
                          oc.decompress(oc_codes, oc_scales, oc_zps, group_size, out_dtype=out_dt).view(np.uint16))


def test_edge_rows():
    print("case: constant / tie / huge rows", flush=True)
    from heterokv import KVCompressor
    rows = np.zeros((6, 128), dtype=np.float32)
    rows[0] = 0.75
    rows[1] = -0.75
    rows[2, :6] = [-7.5, 7.5, 0.0, -5.5, -4.5, 1.5]
    rows[3] = np.linspace(-60000, 60000, 128)
    rows[4, :2] = [-2.5, 12.5]
    rows[5] = np.float32(1e-6) * np.arange(128)
    x = torch.from_numpy(rows)
    codes, scales, zps = KVCompressor().compress(x.to(DEV))
    oc_codes, oc_scales, oc_zps = oc.compress(rows, 128)
    assert np.array_equal(codes.cpu().numpy(), oc_codes)
    assert np.array_equal(scales.cpu().numpy(), oc_scales)
    assert np.array_equal(zps.cpu().numpy(), oc_zps)
    assert list(oc_codes[2, :6]) == [0, 15, 8, 2, 4, 10]


def _same_f32(a, b):
    """Bit-equal float32 arrays, except that NaN matches any NaN."""
    na, nb = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


def test_nan_and_inf_rows():
    """torch's min/max propagate NaN: a NaN group has a NaN scale and zero codes/zp."""
    print("case: NaN / inf rows (compress, decompress)", flush=True)
    from heterokv import KVCompressor
    rows = np.zeros((7, 128), np.float32)
    rows[0, 5] = np.nan
    rows[1] = np.linspace(-3, 3, 128)
    rows[1, 127] = np.nan
    rows[2, 0] = np.inf
    rows[3, 9] = -np.inf
    rows[4, 1], rows[4, 2] = np.inf, -np.inf
    rows[5] = np.nan
    rows[6] = np.linspace(-3, 3, 128)
    for dt in (torch.float32, torch.float16):
        x = torch.from_numpy(rows).to(dt)
        comp = KVCompressor()
        codes, scales, zps = comp.compress(x.to(DEV))
        oc_codes, oc_scales, oc_zps = oc.compress(x.numpy(), 128)
        assert np.isnan(oc_scales[[0, 1, 5]]).all() and not np.isnan(oc_scales[[2, 3, 4, 6]]).any()
        assert np.array_equal(codes.cpu().numpy(), oc_codes), dt
        assert _same_f32(scales.cpu().numpy(), oc_scales), dt
        assert np.array_equal(zps.cpu().numpy(), oc_zps), dt
        deq = comp.decompress(codes, scales, zps, target_dtype=torch.float32).cpu().numpy()
        assert _same_f32(deq, oc.decompress(oc_codes, oc_scales, oc_zps, 128, out_dtype=np.float32)), dt


def test_division_edge_rows_and_random_fp32():
    """The per-element x / scale is computed from RN(1/scale) with one fma correction; rows
    that exercise it: infinite values (the plain-division path), values whose residual
    underflows (tiny fp32 beside ordinary ones), huge-over-tiny ranges, and 2M random
    finite fp32 bit patterns; every code, scale and zero point against the oracle."""
    print("case: quantizer division edge rows + random fp32 bits", flush=True)
    from heterokv import KVCompressor
    rows = np.zeros((6, 128), dtype=np.float32)
    rows[0] = np.linspace(-3, 3, 128)
    rows[0, 5] = np.inf
    rows[1] = np.linspace(-3, 3, 128)
    rows[1, 9] = -np.inf
    rows[2] = np.float32(1e-40) * np.arange(128)            # subnormal inputs
    rows[3] = np.linspace(-1.0, 1.0, 128)
    rows[3, :8] = np.float32(3e-39) * np.arange(1, 9)        # quotients whose residual underflows
    rows[4] = np.float32(1e30) * np.linspace(-1, 1, 128)
    rows[4, 3] = np.float32(1e-30)
    rows[5] = np.float32(2.0 ** -120) * np.linspace(-1, 1, 128)
    g = np.random.default_rng(7)
    bits = g.integers(0, 2 ** 32, size=(16384, 128), dtype=np.uint64).astype(np.uint32)
    rnd = bits.view(np.float32)
    rnd = np.where(np.isfinite(rnd), rnd, np.float32(0.0)).astype(np.float32)
    for x_np in (rows, rnd):
        codes, scales, zps = KVCompressor().compress(torch.from_numpy(x_np).to(DEV))
        oc_codes, oc_scales, oc_zps = oc.compress(x_np, 128)
        assert np.array_equal(codes.cpu().numpy(), oc_codes)
        assert np.array_equal(scales.cpu().numpy().view(np.uint32), oc_scales.view(np.uint32))
        assert np.array_equal(zps.cpu().numpy(), oc_zps)


def test_cpu_tensor_is_rejected():
    from heterokv import HeteroKVError, KVCompressor
    with pytest.raises(HeteroKVError):
        KVCompressor().compress(torch.zeros(128, dtype=torch.float16))
