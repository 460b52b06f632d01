"""The reference's INT4-KV path in plain float32 torch on the CPU (TEST INFRASTRUCTURE ONLY,
see oracle/__init__.py): the CPU baseline bench.py times beside the GPU, and a second
restatement the tests pin against the C oracle and the float64 attention.

Followed line by line, with the same torch operations:
  src/quantization/kv_compressor.py:66-98    compress: flat float32, zero pad to a multiple
                                             of the group, per-group min/max, scale =
                                             clamp((max - min) / 15, 1e-8), zp = clamp(round(
                                             -min / scale), 0, 15), code = clamp(round(x /
                                             scale + zp), 0, 15) (round half to even)
  src/quantization/kv_compressor.py:119-132  decompress: (code - zp) * scale, cast to the
                                             target dtype (fp16 by default)
  src/memory/manager.py:779-821              Path C: every INT4 token of the layer
                                             dequantized to fp16 and concatenated before the
                                             fp16 zones
  src/quantization/fused_dequant_attn.py:242-247
                                             softmax(q K^T * sm_scale) V, float32 here,
                                             GQA by repeat_kv (q head i reads kv head i // n_rep)
"""
import math

import torch


def compress(x, group_size=128):
    """kv_compressor.py:66-98: (codes uint8 shaped like x, scales float32 [G], zps uint8 [G])."""
    flat = x.float().reshape(-1)
    n = flat.numel()
    pad = (-n) % group_size
    if pad:
        flat = torch.cat([flat, torch.zeros(pad, dtype=flat.dtype)])
    g = flat.view(-1, group_size)
    mn = g.min(dim=1, keepdim=True).values
    mx = g.max(dim=1, keepdim=True).values
    scale = ((mx - mn) / 15).clamp(min=1e-8)
    zp = (-mn / scale).round().clamp(0, 15)
    q = (g / scale + zp).round().clamp(0, 15).to(torch.uint8)
    return q.reshape(-1)[:n].reshape(x.shape), scale.reshape(-1), zp.to(torch.uint8).reshape(-1)


def decompress(codes, scales, zps, group_size=128, dtype=torch.float16):
    """kv_compressor.py:119-132."""
    n = codes.numel()
    c = codes.reshape(-1).float()
    pad = (-n) % group_size
    if pad:
        c = torch.cat([c, torch.zeros(pad)])
    out = (c.view(-1, group_size) - zps.float()[:, None]) * scales.float()[:, None]
    return out.reshape(-1)[:n].reshape(codes.shape).to(dtype)


def attend(q, k, v, sm_scale=None, causal_from=None, rows=None):
    """float32 softmax(q k^T * sm_scale) v with GQA.  q [Hq, Sq, D]; k, v [Hkv, S, D].
    causal_from: key index of the first chunk key; query row i, at chunk position rows[i]
    (default i), then sees keys [0, causal_from + rows[i]] (the chunk causally)."""
    Hq, Sq, D = q.shape
    Hkv = k.shape[0]
    rep = Hq // Hkv
    kk = k.float().repeat_interleave(rep, dim=0)
    vv = v.float().repeat_interleave(rep, dim=0)
    s = torch.matmul(q.float(), kk.transpose(1, 2)) * (sm_scale if sm_scale is not None else 1.0 / math.sqrt(D))
    if causal_from is not None:
        S = k.shape[1]
        pos = (torch.arange(Sq) if rows is None else torch.as_tensor(rows))[:, None]
        cols = torch.arange(S)[None, :]
        s = s.masked_fill(cols > causal_from + pos, float("-inf"))
    return torch.matmul(torch.softmax(s, dim=-1), vv)


def path_c_keys(codes, scales, zps, zones):
    """Path C's attended keys or values for one sequence: the INT4 tokens (codes [H, T, D],
    one scale / zp per (head, token) row) dequantized to fp16, then the fp16 zone tokens
    ([H, S_z, D] each), concatenated along the token axis."""
    deq = decompress(codes, scales, zps, codes.shape[-1], torch.float16)
    return torch.cat([deq] + list(zones), dim=1)
