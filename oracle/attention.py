"""Dequantize-then-attend restatement in float64 (TEST INFRASTRUCTURE ONLY, see oracle/__init__.py).

Follows the reference's torch path, the formula its fused kernels are meant to
compute:
  src/quantization/fused_dequant_attn.py:242-247 / :326-331
      K = (Kq - zp) * s ; V = (Vq - zp) * s           (_dequant_tensor, :388-390)
      P = softmax(q K^T * sm_scale) ; O = P V         (sm_scale default 1/sqrt(d), :189-190)
  GQA as transformers' repeat_kv: query head i reads kv head i // n_rep.
  Zone merge (src/core/fused_attention_patch.py:127-196): one joint softmax over
  [HBM fp16 tokens || DRAM INT4 tokens].
Path C materialises the dequantized DRAM tokens as fp16
(src/memory/manager.py:806-807) before SDPA; ``dequant_fp16`` reproduces that
rounding exactly through the C restatement.
"""
import numpy as np

from . import compressor


def dequant_rows(codes, scales, zps, out_fp16=True):
    """Rows of 128 codes with one (scale, zp) per row -> float64 values.

    codes: [..., T, D] uint8; scales/zps: [..., T].  With out_fp16 the value is
    rounded to fp16 first (Path C), else it is the float32 product.
    """
    codes = np.asarray(codes)
    shp = codes.shape
    d = shp[-1]
    flat_c = codes.reshape(-1)
    s = np.asarray(scales, dtype=np.float32).reshape(-1)
    z = np.asarray(zps, dtype=np.uint8).reshape(-1)
    out = compressor.decompress(flat_c, s, z, group_size=d,
                                out_dtype=np.float16 if out_fp16 else np.float32)
    return out.reshape(shp).astype(np.float64)


def attend(q, k, v, sm_scale=None, mask=None):
    """float64 softmax(q k^T * sm_scale) v with GQA.

    q: [Hq, Sq, D]; k, v: [Hkv, S, D]; mask: optional bool [Sq, S] (True = attend).
    Returns [Hq, Sq, D] float64.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    hq, sq, d = q.shape
    hkv = k.shape[0]
    if hq % hkv:
        raise ValueError("num_q_heads must be a multiple of num_kv_heads")
    n_rep = hq // hkv
    if sm_scale is None:
        sm_scale = 1.0 / np.sqrt(d)
    out = np.empty((hq, sq, d), dtype=np.float64)
    for i in range(hq):
        kv = i // n_rep
        s = (q[i] @ k[kv].T) * sm_scale
        if mask is not None:
            s = np.where(mask, s, -np.inf)
        mx = s.max(axis=-1, keepdims=True)
        mx = np.where(np.isfinite(mx), mx, 0.0)
        p = np.exp(s - mx)
        den = p.sum(axis=-1, keepdims=True)
        out[i] = (p @ v[kv]) / np.where(den > 0, den, 1.0)
    return out


def partial_state(q, k, v, sm_scale=None):
    """Per-head (m, l, o) of one key range: m = max score, l = sum exp(s - m), o = sum exp(s - m) v."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    hq, d = q.shape
    n_rep = hq // k.shape[0]
    if sm_scale is None:
        sm_scale = 1.0 / np.sqrt(d)
    m = np.empty(hq)
    l = np.empty(hq)
    o = np.empty((hq, d))
    for i in range(hq):
        s = (k[i // n_rep] @ q[i]) * sm_scale
        m[i] = s.max()
        e = np.exp(s - m[i])
        l[i] = e.sum()
        o[i] = e @ v[i // n_rep]
    return m, l, o


def merge_states(states):
    """Combine partial states of disjoint key ranges into softmax attention outputs."""
    ms = np.stack([s[0] for s in states])
    M = ms.max(axis=0)
    w = np.exp(ms - M)
    L = sum(w[j] * states[j][1] for j in range(len(states)))
    O = sum(w[j][:, None] * states[j][2] for j in range(len(states)))
    return O / L[:, None]
