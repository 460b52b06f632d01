"""Pins the float64 dequantize-then-attend oracle (oracle/attention.py) with closed
forms and torch's own SDPA.  CPU only."""
import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import compressor as oc


def test_zero_query_gives_mean_of_values():
    rng = np.random.default_rng(0)
    k = rng.standard_normal((2, 50, 128))
    v = rng.standard_normal((2, 50, 128))
    q = np.zeros((4, 1, 128))
    out = oa.attend(q, k, v)
    for i in range(4):
        assert np.allclose(out[i, 0], v[i // 2].mean(0), atol=1e-12)


def test_one_hot_key_selects_its_value():
    rng = np.random.default_rng(1)
    k = rng.standard_normal((1, 40, 128)) * 0.01
    k[0, 17] = 0.0
    k[0, 17, 5] = 1000.0
    q = np.zeros((1, 1, 128))
    q[0, 0, 5] = 1.0
    v = rng.standard_normal((1, 40, 128))
    out = oa.attend(q, k, v)
    assert np.allclose(out[0, 0], v[0, 17], atol=1e-9)


def test_gqa_uses_head_div_nrep():
    # kv head h has constant V = h; q head i must see kv head i // n_rep (not i % n_kv)
    hkv, nrep = 4, 3
    k = np.random.default_rng(2).standard_normal((hkv, 10, 128))
    v = np.broadcast_to(np.arange(hkv, dtype=np.float64)[:, None, None], (hkv, 10, 128))
    q = np.random.default_rng(3).standard_normal((hkv * nrep, 1, 128))
    out = oa.attend(q, k, v)
    for i in range(hkv * nrep):
        assert np.allclose(out[i], i // nrep)


def test_matches_torch_sdpa_float64():
    rng = np.random.default_rng(4)
    q = rng.standard_normal((8, 3, 128))
    k = rng.standard_normal((2, 77, 128))
    v = rng.standard_normal((2, 77, 128))
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q)[None], torch.from_numpy(np.repeat(k, 4, 0))[None],
        torch.from_numpy(np.repeat(v, 4, 0))[None])[0].numpy()
    assert np.allclose(oa.attend(q, k, v), ref, atol=1e-12)
    mask = np.tril(np.ones((3, 77), dtype=bool), k=74)
    ref_m = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q)[None], torch.from_numpy(np.repeat(k, 4, 0))[None],
        torch.from_numpy(np.repeat(v, 4, 0))[None], attn_mask=torch.from_numpy(mask))[0].numpy()
    assert np.allclose(oa.attend(q, k, v, mask=mask), ref_m, atol=1e-12)


def test_token_order_does_not_matter_and_split_merge_identity():
    rng = np.random.default_rng(5)
    q = rng.standard_normal((4, 128))
    k = rng.standard_normal((1, 300, 128))
    v = rng.standard_normal((1, 300, 128))
    full = oa.attend(q[:, None], k, v)[:, 0]
    perm = rng.permutation(300)
    assert np.allclose(oa.attend(q[:, None], k[:, perm], v[:, perm])[:, 0], full, atol=1e-12)
    parts = [oa.partial_state(q, k[:, a:b], v[:, a:b]) for a, b in ((0, 64), (64, 250), (250, 300))]
    assert np.allclose(oa.merge_states(parts), full, atol=1e-12)
    # dropping a zone changes the answer (the merge is not vacuous)
    assert not np.allclose(oa.merge_states(parts[:2]), full, atol=1e-6)


def test_sm_scale_is_applied():
    rng = np.random.default_rng(6)
    q = rng.standard_normal((1, 1, 128))
    k = rng.standard_normal((1, 20, 128))
    v = rng.standard_normal((1, 20, 128))
    a = oa.attend(q, k, v, sm_scale=0.5)
    b = oa.attend(q * 0.5 * np.sqrt(128), k, v)
    assert np.allclose(a, b, atol=1e-12)


def test_dequant_rows_path_c_fp16_rounding():
    codes = np.array([[[3] * 128]], dtype=np.uint8)
    scales = np.array([[np.float32(1.0 + 2.0 ** -11)]], dtype=np.float32)
    zps = np.array([[0]], dtype=np.uint8)
    d16 = oa.dequant_rows(codes, scales, zps, out_fp16=True)
    d32 = oa.dequant_rows(codes, scales, zps, out_fp16=False)
    assert d32[0, 0, 0] == np.float64(np.float32(3 * (1.0 + 2.0 ** -11)))
    assert d16[0, 0, 0] == float(np.float16(d32[0, 0, 0]))
    c, s, z = oc.compress(np.random.default_rng(7).standard_normal((3, 128)).astype(np.float16), 128)
    assert oa.dequant_rows(c, s, z).shape == (3, 128)
