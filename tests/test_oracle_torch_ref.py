"""The float32 torch restatement (oracle/torch_ref.py, the bench's CPU baseline) against the
C compressor oracle (bit for bit) and the float64 attention oracle.  No GPU."""
import math

import numpy as np
import torch

from oracle import attention as oa
from oracle import compressor as oc
from oracle import torch_ref as tr


def _rows(seed, shape, outliers=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g)
    if outliers:
        x[..., [7, 31, 64, 100]] *= 8
    return x


def test_compress_matches_c_oracle_bitwise():
    for dtype in (torch.float16, torch.float32):
        x = _rows(1, (2, 3, 257, 128)).to(dtype)
        c, s, z = tr.compress(x, 128)
        c2, s2, z2 = oc.compress(x.numpy(), 128)
        assert np.array_equal(c.numpy(), c2)
        assert np.array_equal(s.numpy().view(np.uint32), s2.view(np.uint32))
        assert np.array_equal(z.numpy(), z2)


def test_compress_edge_rows_and_padding():
    # constant rows, non-negative rows, exact .5 ties, a tail that needs zero padding
    x = torch.zeros(4, 128)
    x[1] = 3.25
    x[2] = torch.arange(128, dtype=torch.float32) / 127.0
    x[3] = torch.tensor([(i % 16) * 0.5 - 3.75 for i in range(128)])
    flat = torch.cat([x.reshape(-1), torch.tensor([0.5, -1.5, 2.5])])
    for t in (x, flat):
        c, s, z = tr.compress(t, 128)
        c2, s2, z2 = oc.compress(t.numpy().astype(np.float32), 128)
        assert np.array_equal(c.numpy(), c2) and np.array_equal(s.numpy(), s2) and np.array_equal(z.numpy(), z2)


def test_decompress_matches_c_oracle_bitwise():
    x = _rows(2, (8, 64, 128)).half()
    c, s, z = oc.compress(x.numpy(), 128)
    for dtype, want in ((torch.float16, oc.decompress(c, s, z, 128)),
                        (torch.float32, oc.decompress(c, s, z, 128, out_dtype=np.float32))):
        got = tr.decompress(torch.from_numpy(c), torch.from_numpy(s), torch.from_numpy(z), 128, dtype)
        assert np.array_equal(got.numpy().view(np.uint8), want.view(np.uint8))


def test_attend_matches_float64_oracle():
    g = torch.Generator().manual_seed(3)
    q = torch.randn((28, 5, 128), generator=g) / math.sqrt(128)
    k = torch.randn((4, 300, 128), generator=g)
    v = torch.randn((4, 300, 128), generator=g)
    got = tr.attend(q, k, v).numpy()
    want = oa.attend(q.double().numpy(), k.double().numpy(), v.double().numpy())
    assert np.abs(got - want).max() < 1e-5
    # causal chunk: row i sees keys [0, 290 + i]
    got = tr.attend(q, k, v, causal_from=290).numpy()
    mask = np.arange(300)[None, :] <= 290 + np.arange(5)[:, None]
    want = oa.attend(q.double().numpy(), k.double().numpy(), v.double().numpy(), mask=mask)
    assert np.abs(got - want).max() < 1e-5
    # rows at chunk positions 0, 3, 4: the same rows of the contiguous call
    sel = tr.attend(q[:, [0, 3, 4]], k, v, causal_from=290, rows=[0, 3, 4]).numpy()
    assert np.abs(sel - got[:, [0, 3, 4]]).max() < 1e-6


def test_path_c_keys_order_and_rounding():
    x = _rows(4, (2, 40, 128)).half()
    c, s, z = oc.compress(x.numpy(), 128)
    zone = torch.randn((2, 7, 128)).half()
    keys = tr.path_c_keys(torch.from_numpy(c), torch.from_numpy(s), torch.from_numpy(z), [zone])
    assert keys.shape == (2, 47, 128) and keys.dtype == torch.float16
    assert np.array_equal(keys[:, :40].numpy(), oc.decompress(c, s, z, 128))
    assert torch.equal(keys[:, 40:], zone)
