"""Fused dequant-attention entry points on the GPU.

Drop-ins for the reference's src/quantization/kernels/fused_dequant_attn.py:301-368
(``fused_dequant_attn_decode``) and :371-435 (``fused_dequant_attn_forward``) with the
numerics of its torch path
(src/quantization/fused_dequant_attn.py:326-331,388-390):
    K = (Kq - zp) * s, V = (Vq - zp) * s, out = softmax(q K^T * sm_scale) V,
sm_scale defaulting to 1/sqrt(head_dim).  Unlike the reference's Triton kernel
(which drops sm_scale and mis-addresses K, see its :69-78,353-365) this computes
exactly that formula, and it also accepts GQA (q heads a multiple of kv heads).

The reference passes unpacked codes (one uint8 per value) with per-token
scales/zps [B, H, S]; they are repacked into INT4 block records on the device
(hkv_repack_codes) and attended by the split-K decode kernel (hkv_decode_attn) or the
MFMA prefill kernel (hkv_prefill_attn).  q may be fp16 or bf16 (bf16 is narrowed to
fp16 operands exactly within the fp16 range).  Device errors (an out-of-range bf16
value, a decode placement failure) go to a per-device error word that is read without
blocking at the next call -- a later call raises HeteroKVError -- or at once by
check_errors().
"""
import math
from typing import Optional

import torch

from . import _lib, ops
from ._lib import BLOCK_TOKENS, HeteroKVError


_ERR = {}   # device -> ErrorWord shared by the calls on that device
_WS = {}    # device -> DecodeWorkspace shared by the decode calls on that device


def _errword(device):
    w = _ERR.get(device)
    if w is None:
        w = _ERR[device] = ops.ErrorWord(device)
        _WS[device] = ops.DecodeWorkspace(device)
        w.on_error = lambda bits: _WS[device].placement_failed() if bits & _lib.ERR_BIT_PLACEMENT else None
    return w


def check_errors(device=None) -> None:
    """Raise HeteroKVError if a call on `device` (default: every device used) reported a
    device error (synchronizes)."""
    for d, w in list(_ERR.items()):
        if device is None or torch.device(device) == d:
            w.check()


def _as_4d(t):
    if t.dim() == 2:
        return t.unsqueeze(0).unsqueeze(0)
    if t.dim() == 3:
        return t.unsqueeze(0)
    return t


def _as_kernel_q(q: torch.Tensor, err) -> torch.Tensor:
    """q in a dtype the kernels take: fp16 and bf16 as they are (the kernels range-check a
    bf16 q themselves); any other floating dtype is rounded to fp16, and a finite value
    beyond the fp16 range (which would become inf) sets HKV_ERR_BIT_RANGE in `err` on the
    device, reported like the kernels' own range errors (no host synchronization)."""
    if q.dtype in (torch.float16, torch.bfloat16):
        return q
    over = (q.abs() > 65504.0) & torch.isfinite(q)
    torch.bitwise_or(err.dev, over.any().to(torch.int32) * _lib.ERR_BIT_RANGE, out=err.dev)
    return q.to(torch.float16)


def fused_dequant_attn_decode(q: torch.Tensor, k_data: torch.Tensor, k_scales: torch.Tensor,
                              k_zps: torch.Tensor, v_data: torch.Tensor, v_scales: torch.Tensor,
                              v_zps: torch.Tensor, sm_scale: Optional[float] = None) -> torch.Tensor:
    """q [B, Hq, 1, D] fp16; k/v_data uint8 [B, Hkv, S, D]; scales/zps [B, Hkv, S] -> [B, Hq, 1, D] in q.dtype."""
    if q.dim() != 4 or q.shape[2] != 1:
        raise HeteroKVError(-1, "Decode expects [B,H,1,D], got %s" % (tuple(q.shape),))
    B, Hq, _, D = q.shape
    kd, vd = _as_4d(k_data), _as_4d(v_data)
    if kd.dim() == 4 and kd.shape[0] != B:
        raise HeteroKVError(-1, "batch mismatch between q and k_data")
    Hkv, S = kd.shape[1], kd.shape[2]
    ks = k_scales.reshape(B, Hkv, S)
    vs = v_scales.reshape(B, Hkv, S)
    kz = k_zps.reshape(B, Hkv, S)
    vz = v_zps.reshape(B, Hkv, S)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    nblk = (S + BLOCK_TOKENS - 1) // BLOCK_TOKENS
    err = _errword(q.device)
    err.poll()
    pool = ops.Int4Pool(B * nblk, Hkv, q.device)
    bt = torch.arange(B * nblk, dtype=torch.int32, device=q.device).reshape(B, nblk)
    start = torch.zeros(B, dtype=torch.int32, device=q.device)
    ops.repack_codes(pool, kd, vd, ks, vs, kz, vz, start, bt, err=err)
    qq = _as_kernel_q(q, err)
    out = ops.decode_attention(qq, zones=(), pool=pool, block_table=bt, int4_lens=None, int4_max_len=S,
                               sm_scale=sm_scale, workspace=_WS[q.device], err=err, out_dtype=qq.dtype)
    err.post()
    return out.to(q.dtype)


def _repack_reference(q, k_data, k_scales, k_zps, v_data, v_scales, v_zps, err):
    B = q.shape[0]
    kd, vd = _as_4d(k_data), _as_4d(v_data)
    Hkv, S = kd.shape[1], kd.shape[2]
    nblk = (S + BLOCK_TOKENS - 1) // BLOCK_TOKENS
    pool = ops.Int4Pool(B * nblk, Hkv, q.device)
    bt = torch.arange(B * nblk, dtype=torch.int32, device=q.device).reshape(B, nblk)
    start = torch.zeros(B, dtype=torch.int32, device=q.device)
    ops.repack_codes(pool, kd, vd, k_scales.reshape(B, Hkv, S), v_scales.reshape(B, Hkv, S),
                     k_zps.reshape(B, Hkv, S), v_zps.reshape(B, Hkv, S), start, bt, err=err)
    return pool, bt, S


def fused_dequant_attn_forward(q: torch.Tensor, k_data: torch.Tensor, k_scales: torch.Tensor,
                               k_zps: torch.Tensor, v_data: torch.Tensor, v_scales: torch.Tensor,
                               v_zps: torch.Tensor, sm_scale: Optional[float] = None) -> torch.Tensor:
    """q [B, Hq, Sq, D] fp16/bf16 against quantized K/V [B, Hkv, S, D] (all keys visible,
    as the reference's torch path) -> [B, Hq, Sq, D] in q.dtype."""
    if q.dim() != 4:
        raise HeteroKVError(-1, "Forward expects [B,H,S,D], got %s" % (tuple(q.shape),))
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(q.shape[-1])
    err = _errword(q.device)
    err.poll()
    pool, bt, S = _repack_reference(q, k_data, k_scales, k_zps, v_data, v_scales, v_zps, err)
    qq = _as_kernel_q(q, err)
    out = ops.prefill_attention(qq, pool=pool, block_table=bt, int4_max_len=S, sm_scale=sm_scale, err=err,
                                out_dtype=qq.dtype)
    err.post()
    return out.to(q.dtype)
