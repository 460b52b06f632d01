"""This build's packed INT4 block records and fp16 zone tiles, restated in numpy
from their specification in include/heterokv.h (TEST INFRASTRUCTURE ONLY, see
oracle/__init__.py).  Used to check the HIP packer byte for byte.

Block record (16 tokens, H kv heads, head_dim 128): H contiguous 2208-byte head parts,
part i at i*2208 = [K codes 1024][V codes 1024][K scales 16 f32][V scales 16 f32][K zps 16][V zps 16]
Packed word: 8 codes x0..x7, x_k at bit (k%2)*16 + (k//2)*4.
  K: word j of a token row = dims 8j..8j+7.
  V: word (g*16+c)*4+m of a head = tokens 4g..4g+3 at dim c+32m (x0..x3) and c+32m+16 (x4..x7).
fp16 V tile (16 tokens): [g 4][c 16][n 8][i 4] = V[4g+i][c+16n].
"""
import numpy as np

D = 128
BT = 16


def nib_shift(k):
    return (k % 2) * 16 + (k // 2) * 4


def record_bytes(h):
    return h * 2208


PART_BYTES = 2208
PART = dict(kc=0, vc=1024, ks=2048, vs=2112, kz=2176, vz=2192)


def offsets(i):
    """Byte offsets of head i's K codes, V codes, K scales, V scales, K zps, V zps."""
    return {k: i * PART_BYTES + v for k, v in PART.items()}


def pack_k_rows(codes):
    """codes [..., 128] uint8 -> [..., 64] bytes."""
    c = np.asarray(codes, dtype=np.uint32).reshape(-1, 16, 8)
    w = np.zeros(c.shape[:2], dtype=np.uint32)
    for k in range(8):
        w |= c[:, :, k] << nib_shift(k)
    return w.astype("<u4").view(np.uint8).reshape(np.asarray(codes).shape[:-1] + (64,))


def pack_v_block(codes):
    """codes [16 tokens, 128] uint8 (one head) -> 1024 bytes."""
    c = np.asarray(codes, dtype=np.uint32)
    w = np.zeros(256, dtype=np.uint32)
    for g in range(4):
        for cc in range(16):
            for m in range(4):
                word = 0
                for k in range(8):
                    tok = 4 * g + (k & 3)
                    dim = cc + 32 * m + (k >> 2) * 16
                    word |= int(c[tok, dim]) << nib_shift(k)
                w[(g * 16 + cc) * 4 + m] = word
    return w.astype("<u4").view(np.uint8)


def unpack_k_rows(packed):
    p = np.asarray(packed, dtype=np.uint8)
    w = p.reshape(-1, 16, 4).copy().view("<u4").reshape(-1, 16)
    out = np.zeros((w.shape[0], 16, 8), dtype=np.uint8)
    for k in range(8):
        out[:, :, k] = (w >> nib_shift(k)) & 0xF
    return out.reshape(p.shape[:-1] + (128,))


def unpack_v_block(packed):
    w = np.asarray(packed, dtype=np.uint8).copy().view("<u4")
    out = np.zeros((16, 128), dtype=np.uint8)
    for g in range(4):
        for cc in range(16):
            for m in range(4):
                word = int(w[(g * 16 + cc) * 4 + m])
                for k in range(8):
                    out[4 * g + (k & 3), cc + 32 * m + (k >> 2) * 16] = (word >> nib_shift(k)) & 0xF
    return out


def build_record(kcodes, vcodes, kscales, vscales, kzps, vzps):
    """Per-head arrays for one block ([H,16,128] codes, [H,16] meta) -> record bytes."""
    h = kcodes.shape[0]
    rec = np.zeros(record_bytes(h), dtype=np.uint8)
    ks = np.asarray(kscales, dtype="<f4").reshape(h, 16)
    vs = np.asarray(vscales, dtype="<f4").reshape(h, 16)
    kz = np.asarray(kzps, dtype=np.uint8).reshape(h, 16)
    vz = np.asarray(vzps, dtype=np.uint8).reshape(h, 16)
    for i in range(h):
        off = offsets(i)
        rec[off["kc"]: off["kc"] + 1024] = pack_k_rows(kcodes[i]).reshape(-1)
        rec[off["vc"]: off["vc"] + 1024] = pack_v_block(vcodes[i])
        rec[off["ks"]: off["ks"] + 64] = ks[i].view(np.uint8)
        rec[off["vs"]: off["vs"] + 64] = vs[i].view(np.uint8)
        rec[off["kz"]: off["kz"] + 16] = kz[i]
        rec[off["vz"]: off["vz"] + 16] = vz[i]
    return rec


def v_tile(vals):
    """fp16 V of 16 tokens [16, 128] -> transposed tile [4, 16, 8, 4]."""
    v = np.asarray(vals)
    t = np.empty((4, 16, 8, 4), dtype=v.dtype)
    for g in range(4):
        for i in range(4):
            for n in range(8):
                t[g, :, n, i] = v[4 * g + i, 16 * n: 16 * n + 16]
    return t
