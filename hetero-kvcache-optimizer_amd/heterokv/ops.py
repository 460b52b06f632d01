"""Tensor-level wrappers over the libheterokv C ABI.

Every function here takes torch tensors that live on a ROCm GPU, passes raw
pointers and torch's current stream to the library, and raises HeteroKVError on
any failure.  Nothing falls back to the CPU.
"""
import ctypes
import functools
import math

import torch

from . import _lib
from ._lib import BLOCK_TOKENS, HEAD_DIM, HeteroKVError, check, load, stream_ptr

_DTYPES = {torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_F32}


def _require_gpu(*ts):
    for t in ts:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
            raise HeteroKVError(-1, "heterokv kernels need tensors on a ROCm GPU (got %s)" %
                                (t.device if isinstance(t, torch.Tensor) else type(t)))


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _aligned16(t):
    """16-byte aligned base and strides (in elements) that are multiples of 8, unit last stride."""
    return t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all(st % 8 == 0 for st in t.stride()[:-1])


_F16_OR_BF16 = (torch.float16, torch.bfloat16)


class ErrorWord:
    """A device int32 that kernels OR HKV_ERR_BIT_* into, with a pinned host mirror.

    post() enqueues a copy of the word to the mirror and records an event on the current
    stream; poll() looks at the last posted copy only if that event has completed (it
    never blocks) and raises HeteroKVError if a bit was set; check() synchronizes.  A
    raised error clears the word."""

    def __init__(self, device):
        self.device = torch.device(device)
        self.dev = torch.zeros(1, dtype=torch.int32, device=self.device)
        self.host = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        self._event = None
        self.on_error = None   # optional callback(bits) run before the exception

    def ptr(self):
        return self.dev.data_ptr()

    def post(self):
        self.host.copy_(self.dev, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(self.device))
        self._event = ev

    def poll(self):
        ev = self._event
        if ev is None or not ev.query():
            return
        self._event = None
        bits = int(self.host[0])
        if bits:
            self._fail(bits)

    def check(self):
        self._event = None
        bits = int(self.dev.item())
        if bits:
            self._fail(bits)

    def _fail(self, bits):
        self.dev.zero_()
        self.host.zero_()
        if self.on_error is not None:
            self.on_error(bits)
        raise HeteroKVError(_lib.ERR_DEVICE, "device error word 0x%x: %s" % (bits, _lib.describe_error_bits(bits)))


def record_bytes(num_kv_heads, head_dim=HEAD_DIM):
    n = load().hkv_block_bytes(num_kv_heads, head_dim)
    if n < 0:
        raise HeteroKVError(-4, "unsupported block geometry (heads=%d, head_dim=%d)" % (num_kv_heads, head_dim))
    return int(n)


# ----------------------------------------------------------------------- reference layout
def quantize_groups(x, group_size=128):
    """KVCompressor.compress on the GPU: (codes uint8 like x, scales f32 [G], zps u8 [G])."""
    _require_gpu(x)
    if x.dtype not in _DTYPES:
        raise HeteroKVError(-1, "quantize_groups: unsupported dtype %s" % x.dtype)
    xc = x.contiguous()
    n = xc.numel()
    ng = (n + group_size - 1) // group_size
    codes = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    scales = torch.empty(ng, dtype=torch.float32, device=x.device)
    zps = torch.empty(ng, dtype=torch.uint8, device=x.device)
    check(load().hkv_quantize_groups(_p(xc), _DTYPES[x.dtype], n, group_size, _p(codes), _p(scales),
                                     _p(zps), stream_ptr(x.device)), "hkv_quantize_groups")
    return codes, scales, zps


def dequantize_groups(codes, scales, zps, group_size=128, dtype=torch.float16):
    """KVCompressor.decompress on the GPU."""
    _require_gpu(codes, scales, zps)
    if dtype not in _DTYPES:
        raise HeteroKVError(-1, "dequantize_groups: unsupported dtype %s" % dtype)
    c = codes.contiguous()
    s = scales.contiguous().to(torch.float32)
    z = zps.contiguous()
    if z.dtype != torch.uint8:
        z = z.to(torch.uint8)
    n = c.numel()
    ng = (n + group_size - 1) // group_size
    if s.numel() < ng or z.numel() < ng:
        raise HeteroKVError(-3, "dequantize_groups: %d groups need %d scales/zps, got %d/%d" %
                            (ng, ng, s.numel(), z.numel()))
    out = torch.empty(codes.shape, dtype=dtype, device=codes.device)
    check(load().hkv_dequantize_groups(_p(c), _p(s), _p(z), n, group_size, _p(out), _DTYPES[dtype],
                                       stream_ptr(codes.device)), "hkv_dequantize_groups")
    return out


# ----------------------------------------------------------------------- INT4 block pool
class Int4Pool:
    """Device array of INT4 block records: uint8 [num_blocks, record_bytes]."""

    def __init__(self, num_blocks, num_kv_heads, device, head_dim=HEAD_DIM):
        if head_dim != HEAD_DIM:
            raise HeteroKVError(-4, "Int4Pool: head_dim must be 128")
        self.num_kv_heads = num_kv_heads
        self.record_bytes = record_bytes(num_kv_heads)
        self.num_blocks = num_blocks
        self.data = torch.zeros((max(num_blocks, 1), self.record_bytes), dtype=torch.uint8, device=device)
        self.err = torch.zeros(1, dtype=torch.int32, device=device)

    @property
    def device(self):
        return self.data.device

    def check_errors(self):
        """Raise if a pack kernel met a bad block id or slot (synchronizes)."""
        e = int(self.err.item())
        if e:
            self.err.zero_()
            why = []
            if e & 1:
                why.append("a block table held an id outside [0, %d)" % self.num_blocks)
            if e & 2:
                why.append("a token slot lay beyond its block table row")
            raise HeteroKVError(-1, "; ".join(why))


def h2d(t, device):
    """Host tensor t on `device`.  A copy from pageable memory waits for every kernel
    already queued on the stream; this one goes through pinned memory (held by torch's
    caching host allocator until the copy has run) and does not wait."""
    device = torch.device(device)
    if t.device.type != "cpu" or device.type != "cuda" or torch.cuda.is_current_stream_capturing():
        return t.to(device)
    return t.pin_memory().to(device, non_blocking=True)


def _i32(t, device):
    if not isinstance(t, torch.Tensor):
        t = torch.tensor(t, dtype=torch.int32)
    if t.device.type == "cpu":
        return h2d(t.to(torch.int32).contiguous(), device)
    return t.to(device=device, dtype=torch.int32).contiguous()


def _check_table(bt, sp, B, T, what):
    nsp = sp.numel() if sp is not None else B
    if bt.shape[0] < B or nsp < B:
        raise HeteroKVError(-1, "%s: block table / start positions cover %d / %d sequences, need %d" %
                            (what, bt.shape[0], nsp, B))


def _uniform_start(start_pos, B):
    """The common start of every sequence when start_pos is host data (an int, a list, or
    a CPU tensor) with one value for all B sequences, else None."""
    if isinstance(start_pos, int):
        return start_pos
    if isinstance(start_pos, torch.Tensor):
        if start_pos.device.type != "cpu" or start_pos.numel() < B:
            return None
        start_pos = start_pos.reshape(-1)[:B].tolist()
    elif isinstance(start_pos, (list, tuple)):
        start_pos = list(start_pos)[:B]
    else:
        return None
    if len(start_pos) == B and all(int(x) == int(start_pos[0]) for x in start_pos):
        return int(start_pos[0])
    return None


def pack_tokens(pool, k, v, start_pos, block_table, err=None):
    """Quantize + pack k, v [B, H, T, 128] (fp16/bf16) into `pool` at INT4 slots start_pos[b] + t.
    start_pos: an int (every sequence), a host list / CPU tensor, or a device int32 tensor
    [B]; one host value for every sequence reaches the kernel by value.  Bad block ids /
    slots are reported in `err` (an ErrorWord; default the pool's word)."""
    _require_gpu(k, v)
    if k.shape != v.shape or k.dim() != 4 or k.shape[-1] != HEAD_DIM:
        raise HeteroKVError(-1, "pack_tokens: k/v must both be [B, H, T, 128], got %s / %s" %
                            (tuple(k.shape), tuple(v.shape)))
    if k.dtype != v.dtype or k.dtype not in (torch.float16, torch.bfloat16):
        raise HeteroKVError(-1, "pack_tokens: k/v must be fp16 or bf16")
    if k.stride() != v.stride() or k.stride(-1) != 1:
        k, v = k.contiguous(), v.contiguous()
    B, H, T, _ = k.shape
    if H != pool.num_kv_heads:
        raise HeteroKVError(-1, "pack_tokens: %d heads, pool has %d" % (H, pool.num_kv_heads))
    # one host start for every sequence goes by value: no copy, and no read in the kernel
    base = _uniform_start(start_pos, B)
    sp = _i32(start_pos, k.device) if base is None else None
    bt = _i32(block_table, k.device)
    if bt.dim() == 1:
        bt = bt.unsqueeze(0)
    _check_table(bt, sp, B, T, "pack_tokens")
    a = _lib.PackArgs(k=k.data_ptr(), v=v.data_ptr(), dtype=_DTYPES[k.dtype],
                      src_stride_b=k.stride(0), src_stride_h=k.stride(1), src_stride_t=k.stride(2),
                      batch=B, num_kv_heads=H, head_dim=HEAD_DIM, num_tokens=T,
                      start_pos=sp.data_ptr() if sp is not None else None, block_table=bt.data_ptr(),
                      bt_stride=bt.shape[1], pool=pool.data.data_ptr(), pool_blocks=pool.num_blocks,
                      err_flag=err.ptr() if err is not None else pool.err.data_ptr(),
                      start_base=base if base is not None else 0)
    check(load().hkv_pack_tokens(ctypes.byref(a), stream_ptr(k.device)), "hkv_pack_tokens")


def repack_codes(pool, k_codes, v_codes, k_scales, v_scales, k_zps, v_zps, start_pos, block_table, err=None):
    """Reference-layout INT4 (codes uint8 [B,H,T,128], scales/zps [B,H,T]) -> pool records."""
    _require_gpu(k_codes, v_codes, k_scales, v_scales, k_zps, v_zps)
    B, H, T, D = k_codes.shape
    if D != HEAD_DIM or v_codes.shape != k_codes.shape:
        raise HeteroKVError(-1, "repack_codes: codes must be [B, H, T, 128]")
    kc, vc = k_codes.contiguous(), v_codes.contiguous()
    ks = k_scales.reshape(B, H, T).to(torch.float32).contiguous()
    vs = v_scales.reshape(B, H, T).to(torch.float32).contiguous()
    zdt = torch.uint8 if k_zps.dtype == torch.uint8 else torch.float32
    kz = k_zps.reshape(B, H, T).to(zdt).contiguous()
    vz = v_zps.reshape(B, H, T).to(zdt).contiguous()
    sp = _i32(start_pos, kc.device)
    bt = _i32(block_table, kc.device)
    if bt.dim() == 1:
        bt = bt.unsqueeze(0)
    _check_table(bt, sp, B, T, "repack_codes")
    a = _lib.RepackArgs(k_codes=kc.data_ptr(), v_codes=vc.data_ptr(),
                        code_stride_b=kc.stride(0), code_stride_h=kc.stride(1), code_stride_t=kc.stride(2),
                        k_scales=ks.data_ptr(), v_scales=vs.data_ptr(), k_zps=kz.data_ptr(), v_zps=vz.data_ptr(),
                        zp_dtype=_lib.DTYPE_U8 if zdt == torch.uint8 else _lib.DTYPE_F32,
                        meta_stride_b=ks.stride(0), meta_stride_h=ks.stride(1), meta_stride_t=ks.stride(2),
                        batch=B, num_kv_heads=H, head_dim=HEAD_DIM, num_tokens=T,
                        start_pos=sp.data_ptr(), block_table=bt.data_ptr(), bt_stride=bt.shape[1],
                        pool=pool.data.data_ptr(), pool_blocks=pool.num_blocks,
                        err_flag=err.ptr() if err is not None else pool.err.data_ptr())
    check(load().hkv_repack_codes(ctypes.byref(a), stream_ptr(kc.device)), "hkv_repack_codes")


def unpack_tokens(pool, block_table_row, num_tokens, which):
    """Pool -> reference layout for one sequence: (codes [H,T,128], scales [H*T], zps [H*T])."""
    dev = pool.device
    bt = _i32(block_table_row, dev).reshape(-1)
    if bt.numel() * BLOCK_TOKENS < num_tokens:
        raise HeteroKVError(-3, "unpack_tokens: block table row covers %d slots, need %d" %
                            (bt.numel() * BLOCK_TOKENS, num_tokens))
    H = pool.num_kv_heads
    codes = torch.empty((H, num_tokens, HEAD_DIM), dtype=torch.uint8, device=dev)
    scales = torch.empty(H * num_tokens, dtype=torch.float32, device=dev)
    zps = torch.empty(H * num_tokens, dtype=torch.uint8, device=dev)
    check(load().hkv_unpack_tokens(_p(pool.data), pool.num_blocks, _p(bt), H, HEAD_DIM, num_tokens,
                                   0 if which in (0, "k", "K") else 1, _p(codes), _p(scales), _p(zps),
                                   stream_ptr(dev)), "hkv_unpack_tokens")
    return codes, scales, zps


# ----------------------------------------------------------------------- fp16 zones
class F16Zone:
    """fp16 zone storage: K [B, H, cap, 128] row-major, V in 16-token transposed tiles."""

    def __init__(self, batch, num_kv_heads, capacity, device):
        cap = int(math.ceil(max(capacity, 1) / BLOCK_TOKENS) * BLOCK_TOKENS)
        self.batch, self.num_kv_heads, self.capacity = batch, num_kv_heads, cap
        self.k = torch.zeros((batch, num_kv_heads, cap, HEAD_DIM), dtype=torch.float16, device=device)
        self.v = torch.zeros((batch, num_kv_heads, cap // BLOCK_TOKENS, BLOCK_TOKENS * HEAD_DIM),
                             dtype=torch.float16, device=device)

    @property
    def device(self):
        return self.k.device

    def write(self, k, v, slot_start, ring=0, err=None):
        """Write k, v [B, H, T, 128] (fp16, or bf16 narrowed to fp16 with a range check that
        sets HKV_ERR_BIT_RANGE in `err`, an ErrorWord) at slots slot_start[b] + t (mod `ring`
        if ring > 0; ring=True means the whole capacity).  An int slot_start (or a list of
        equal ints) is passed by value: no host-to-device copy."""
        _require_gpu(k, v)
        if k.dtype != v.dtype or k.dtype not in _F16_OR_BF16:
            raise HeteroKVError(-1, "F16Zone.write: k/v must both be fp16 or bf16")
        if k.shape != v.shape or k.dim() != 4 or k.shape[-1] != HEAD_DIM:
            raise HeteroKVError(-1, "F16Zone.write: k/v must be [B, H, T, 128]")
        if k.stride() != v.stride() or not _aligned16(k) or not _aligned16(v):
            k, v = k.contiguous(), v.contiguous()
        B, H, T, _ = k.shape
        if B != self.batch or H != self.num_kv_heads:
            raise HeteroKVError(-1, "F16Zone.write: shape %s does not match zone [%d, %d]" %
                                (tuple(k.shape), self.batch, self.num_kv_heads))
        if isinstance(slot_start, (list, tuple)) and slot_start and all(s == slot_start[0] for s in slot_start):
            slot_start = int(slot_start[0])
        ss, base = None, 0
        if isinstance(slot_start, int):
            base = slot_start
        else:
            ss = _i32(slot_start, k.device)
            if ss.numel() < B:
                raise HeteroKVError(-1, "F16Zone.write: %d start slots for %d sequences" % (ss.numel(), B))
        a = _lib.ZoneWriteArgs(k=k.data_ptr(), v=v.data_ptr(), src_stride_b=k.stride(0),
                               src_stride_h=k.stride(1), src_stride_t=k.stride(2), batch=B, num_kv_heads=H,
                               head_dim=HEAD_DIM, num_tokens=T, slot_start=ss.data_ptr() if ss is not None else None,
                               capacity=self.capacity, ring=(self.capacity if ring is True else int(ring)),
                               zone_k=self.k.data_ptr(), zone_v=self.v.data_ptr(), slot_base=base,
                               dtype=_DTYPES[k.dtype], err_flag=err.ptr() if err is not None else None)
        check(load().hkv_zone_write(ctypes.byref(a), stream_ptr(k.device)), "hkv_zone_write")

    def copy_to(self, dst, src_slot, dst_slot, n):
        """Copy slots [src_slot, src_slot + n) to dst's [dst_slot, dst_slot + n) (no wrap)."""
        check(load().hkv_zone_copy(_p(self.k), _p(self.v), self.capacity, src_slot, _p(dst.k), _p(dst.v),
                                   dst.capacity, dst_slot, self.batch, self.num_kv_heads, HEAD_DIM, n,
                                   stream_ptr(self.device)), "hkv_zone_copy")

    def step(self, hh, k, v, ring, hh_budget, state, tail_lens=None, hh_lens=None, err=None):
        """Device-stepped decode update (hkv_zone_step) of this ring zone and the heavy-hitter
        zone hh: k, v [B, H, 1, 128] fp16 or bf16 (range-checked into `err`); state int32 [4]
        (ring head, ring length, heavy-hitter length, dropped) is read and advanced on the
        GPU; tail_lens / hh_lens (int32 [B]) receive the new lengths."""
        _require_gpu(k, v, state)
        if k.dtype != v.dtype or k.dtype not in _F16_OR_BF16 or k.shape != v.shape or k.shape[2] != 1:
            raise HeteroKVError(-1, "F16Zone.step: k/v must be fp16 or bf16 [B, H, 1, 128]")
        if k.stride() != v.stride() or k.stride(-1) != 1:
            k, v = k.contiguous(), v.contiguous()
        a = _lib.ZoneStepArgs(k=k.data_ptr(), v=v.data_ptr(), src_stride_b=k.stride(0), src_stride_h=k.stride(1),
                              batch=self.batch, num_kv_heads=self.num_kv_heads, head_dim=HEAD_DIM,
                              tail_k=_p(self.k), tail_v=_p(self.v), tail_capacity=self.capacity, tail_ring=int(ring),
                              hh_k=_p(hh.k) if hh is not None else None, hh_v=_p(hh.v) if hh is not None else None,
                              hh_capacity=hh.capacity if hh is not None else 0, hh_budget=int(hh_budget),
                              state=state.data_ptr(), tail_lens=_p(tail_lens) if tail_lens is not None else None,
                              hh_lens=_p(hh_lens) if hh_lens is not None else None, dtype=_DTYPES[k.dtype],
                              err_flag=err.ptr() if err is not None else None)
        check(load().hkv_zone_step(ctypes.byref(a), stream_ptr(k.device)), "hkv_zone_step")

    def read(self, n):
        """Slots [0, n) as row-major (K, V) [B, H, n, 128]."""
        ok = torch.empty((self.batch, self.num_kv_heads, n, HEAD_DIM), dtype=torch.float16, device=self.device)
        ov = torch.empty_like(ok)
        check(load().hkv_zone_read(_p(self.k), _p(self.v), self.batch, self.num_kv_heads, HEAD_DIM,
                                   self.capacity, n, _p(ok), _p(ov), stream_ptr(self.device)), "hkv_zone_read")
        return ok, ov


# ----------------------------------------------------------------------- decode attention
def decode_workspace_bytes(batch, num_q_heads, num_kv_heads, int4_max_len, f16_max_lens):
    return _decode_workspace_bytes(int(batch), int(num_q_heads), int(num_kv_heads), int(int4_max_len),
                                   tuple(int(x) for x in f16_max_lens))


@functools.lru_cache(maxsize=256)
def _decode_workspace_bytes(batch, num_q_heads, num_kv_heads, int4_max_len, f16_max_lens):
    arr = (ctypes.c_int32 * max(len(f16_max_lens), 1))(*f16_max_lens)
    n = load().hkv_decode_workspace_bytes(batch, num_q_heads, num_kv_heads, HEAD_DIM, int4_max_len,
                                          ctypes.cast(arr, ctypes.c_void_p), len(f16_max_lens))
    if n == 0:
        raise HeteroKVError(-1, "decode_workspace_bytes: unsupported geometry")
    return int(n)


class DecodeWorkspace:
    """Zero-initialised scratch for hkv_decode_attn; grows on demand (re-zeroed when it
    grows).  Its ticket area has the same offsets for every geometry and the kernels leave
    it zero, so it serves launches of any geometry in any order, graph replays included.

    agent_handoff: launches on this workspace combine their ranges through device-scope
    memory (HKV_DECODE_AGENT_HANDOFF).  It is switched on by placement_failed(), which
    callers run when a launch reported HKV_ERR_BIT_PLACEMENT."""

    def __init__(self, device, agent_handoff=False):
        self.device = torch.device(device)
        self.buf = None
        self.agent_handoff = bool(agent_handoff)

    def get(self, nbytes):
        if self.buf is None or self.buf.numel() < nbytes:
            self.buf = torch.zeros(max(nbytes, 4096), dtype=torch.uint8, device=self.device)
        return self.buf

    def placement_failed(self):
        """A launch's ranges did not share one XCD: its tickets may be left inconsistent.
        Clear the workspace and use the device-scope hand-off from now on."""
        self.agent_handoff = True
        if self.buf is not None:
            self.buf.zero_()

    def error_flag(self):
        """Error bits (HKV_ERR_BIT_*) that launches without their own error word left in the
        workspace's first word since the last call (synchronizes); clears them."""
        if self.buf is None:
            return 0
        v = int(self.buf[:4].view(torch.int32).item())
        if v:
            self.buf[:4].zero_()
            if v & _lib.ERR_BIT_PLACEMENT:
                self.placement_failed()
        return v


def _int4_source(pool, staging):
    src = pool if pool is not None else staging
    return src.num_kv_heads if src is not None else None


def decode_attention(q, zones=(), pool=None, block_table=None, int4_lens=None, int4_max_len=0,
                     sm_scale=None, workspace=None, out=None, splits=0, staging=None, deterministic=False,
                     scores=None, score_stats=None, err=None, out_dtype=None, noalloc=False,
                     agent_handoff=False):
    """Split-K decode attention over fp16 zones and the INT4 pool.

    q: [B, Hq, 128] or [B, Hq, 1, 128] fp16 or bf16 (bf16 is range-checked into the error
    word).  out_dtype: fp16 or bf16 (default: q's dtype).  err: ErrorWord for
    HKV_ERR_BIT_* (default: the workspace's first word).
    noalloc: launch through hkv_decode_attn_noalloc, which takes no workspace (its scratch
    is a static device array of HKV_DECODE_SCRATCH_BYTES shared by every such call on
    the GPU) and allocates nothing; agent_handoff then selects the device-scope combine.
    zones: sequence of (F16Zone, lens int32 [B] or None, max_len).
    pool / block_table [B, nblk] / int4_lens [B] / int4_max_len: the INT4 zone.
    staging: Int4Pool whose record i a block-table entry ~i (negative) names.
    splits: ranges per (sequence, kv head); 0 lets the library choose (about one
    workgroup per CU).
    deterministic: fixed block-to-wave assignment, bitwise reproducible output.  The
    default hands blocks to waves on demand (faster); outputs can then differ from
    run to run in the last bits.
    scores / score_stats: optional fp32 outputs [B, Hq, n_items] (n_items >= int4_max_len
    plus the zones' max lengths; item order INT4 tokens, then each zone's slots) and
    [B, Hq, 2]: the log2-domain score of every item and each row's softmax max and sum
    (feeds attn_weights).  Items past a sequence's lengths are left untouched.
    Returns fp16 [B, Hq, 128] (or [B, Hq, 1, 128] if q was 4-D).
    """
    _require_gpu(q)
    squeeze = q.dim() == 4
    q3 = q.reshape(q.shape[0], q.shape[1], q.shape[-1]) if squeeze else q
    if q3.dtype not in _F16_OR_BF16 or q3.shape[-1] != HEAD_DIM:
        raise HeteroKVError(-1, "decode_attention: q must be fp16 or bf16 [B, Hq, 128]")
    if out_dtype is None:
        out_dtype = q3.dtype if out is None else out.dtype
    if out_dtype not in _F16_OR_BF16:
        raise HeteroKVError(-1, "decode_attention: out dtype must be fp16 or bf16")
    if q3.stride(-1) != 1 or q3.data_ptr() % 16 or q3.stride(0) % 8 or q3.stride(1) % 8:
        q3 = q3.contiguous()
    B, Hq, _ = q3.shape
    if len(zones) > _lib.MAX_F16_ZONES:
        raise HeteroKVError(-1, "decode_attention: at most %d fp16 zones" % _lib.MAX_F16_ZONES)
    Hkv = _int4_source(pool, staging) or (zones[0][0].num_kv_heads if zones else None)
    if Hkv is None:
        raise HeteroKVError(-1, "decode_attention: no key/value zone given")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(HEAD_DIM)
    dev = q3.device
    if out is None:
        out = torch.empty((B, Hq, HEAD_DIM), dtype=out_dtype, device=dev)
    elif out.dtype != out_dtype:
        raise HeteroKVError(-1, "decode_attention: out is %s, out_dtype %s" % (out.dtype, out_dtype))
    a = _lib.DecodeArgs()
    a.q_dtype, a.out_dtype = _DTYPES[q3.dtype], _DTYPES[out_dtype]
    a.err_flag = err.ptr() if err is not None else None
    a.batch, a.num_q_heads, a.num_kv_heads, a.head_dim = B, Hq, Hkv, HEAD_DIM
    a.sm_scale = float(sm_scale)
    a.q, a.q_stride_b, a.q_stride_h = q3.data_ptr(), q3.stride(0), q3.stride(1)
    a.num_f16_zones = len(zones)
    keep = []
    zl = []
    for i, (z, lens, max_len) in enumerate(zones):
        if z.batch != B or z.num_kv_heads != Hkv:
            raise HeteroKVError(-1, "decode_attention: zone %d geometry mismatch" % i)
        lt = None
        if lens is not None:
            lt = _i32(lens, dev)
            keep.append(lt)
        a.f16[i] = _lib.F16Zone(k=z.k.data_ptr(), v=z.v.data_ptr(), capacity=z.capacity, max_len=int(max_len),
                                lens=lt.data_ptr() if lt is not None else 0)
        zl.append(int(max_len))
    if int4_max_len > 0:
        if (pool is None and staging is None) or block_table is None:
            raise HeteroKVError(-1, "decode_attention: INT4 zone needs a pool and a block table")
        bt = _i32(block_table, dev)
        if bt.dim() == 1:
            bt = bt.unsqueeze(0)
        keep.append(bt)
        if pool is not None:
            a.pool, a.pool_blocks = pool.data.data_ptr(), pool.num_blocks
        if staging is not None:
            a.staging, a.staging_blocks = staging.data.data_ptr(), staging.num_blocks
        a.block_table, a.bt_stride = bt.data_ptr(), bt.shape[1]
        if int4_lens is not None:
            il = _i32(int4_lens, dev)
            keep.append(il)
            a.int4_lens = il.data_ptr()
    a.int4_max_len = int(int4_max_len)
    a.out, a.out_stride_b, a.out_stride_h = out.data_ptr(), out.stride(0), out.stride(1)
    a.splits_hint = int(splits)
    if noalloc:
        a.workspace, a.workspace_bytes = None, 0
    else:
        nbytes = decode_workspace_bytes(B, Hq, Hkv, int(int4_max_len), zl)
        if workspace is None:
            workspace = DecodeWorkspace(dev)
        ws = workspace.get(nbytes)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
        agent_handoff = agent_handoff or workspace.agent_handoff
    a.flags = (_lib.DECODE_DETERMINISTIC if deterministic else 0) | \
        (_lib.DECODE_AGENT_HANDOFF if agent_handoff else 0)
    if scores is not None:
        _require_gpu(scores, score_stats)
        if score_stats is None or scores.dtype != torch.float32 or score_stats.dtype != torch.float32:
            raise HeteroKVError(-1, "decode_attention: scores and score_stats must be fp32 tensors")
        if scores.dim() != 3 or tuple(scores.shape[:2]) != (B, Hq) or scores.stride(2) != 1 or \
                tuple(score_stats.shape) != (B, Hq, 2) or not score_stats.is_contiguous():
            raise HeteroKVError(-1, "decode_attention: scores [B, Hq, n] (unit item stride) and "
                                    "score_stats [B, Hq, 2] expected")
        a.scores, a.scores_stride_b, a.scores_stride_h = scores.data_ptr(), scores.stride(0), scores.stride(1)
        a.score_stats = score_stats.data_ptr()
    if noalloc:
        check(load().hkv_decode_attn_noalloc(ctypes.byref(a), stream_ptr(dev)), "hkv_decode_attn_noalloc")
    else:
        check(load().hkv_decode_attn(ctypes.byref(a), stream_ptr(dev)), "hkv_decode_attn")
    return out.unsqueeze(2) if squeeze else out


# ----------------------------------------------------------------------- record gather
def gather_blocks(src, ids, dst, staging=None, dst_offset=0, err=None):
    """dst record dst_offset + i = record ids[i] of src (ids >= 0) or of staging (~ids[i]).

    src / staging / dst: Int4Pool with the same record size.  ids: int32 (device or host)."""
    _require_gpu(dst.data)
    dev = dst.device
    ids = _i32(ids, dev).reshape(-1)
    n = ids.numel()
    if n == 0:
        return dst
    rb = dst.record_bytes
    for other in (src, staging):
        if other is not None and other.record_bytes != rb:
            raise HeteroKVError(-1, "gather_blocks: record sizes differ")
    if dst_offset < 0 or dst_offset + n > dst.num_blocks:
        raise HeteroKVError(-3, "gather_blocks: %d records at %d exceed the %d-record destination" %
                            (n, dst_offset, dst.num_blocks))
    check(load().hkv_gather_blocks(src.data.data_ptr() if src is not None else None,
                                   src.num_blocks if src is not None else 0,
                                   staging.data.data_ptr() if staging is not None else None,
                                   staging.num_blocks if staging is not None else 0,
                                   ids.data_ptr(), n, rb, dst.data[dst_offset].data_ptr(),
                                   err.ptr() if err is not None else dst.err.data_ptr(),
                                   stream_ptr(dev)), "hkv_gather_blocks")
    return dst


# ----------------------------------------------------------------------- heavy-hitter scoring
def attn_weights(scores, score_stats, order=None, out=None, accumulate=False):
    """Attention weights of the newest token averaged over heads (hkv_attn_weights).

    scores [B, H, n] / score_stats [B, H, 2]: a decode launch's score outputs.  order:
    optional int64 [m] item indices (negative: weight 0).  Returns fp32 [B, m] (or adds
    into out when accumulate)."""
    _require_gpu(scores, score_stats)
    B, H, n = scores.shape
    dev = scores.device
    if order is not None:
        order = order.to(device=dev, dtype=torch.int64).contiguous().reshape(-1)
        m = order.numel()
    else:
        m = n
    if out is None:
        out = torch.empty((B, m), dtype=torch.float32, device=dev)
        accumulate = False
    if out.dtype != torch.float32 or out.dim() != 2 or out.shape[0] != B or out.shape[1] < m or out.stride(1) != 1:
        raise HeteroKVError(-1, "attn_weights: out must be fp32 [B, >= %d] with unit stride" % m)
    check(load().hkv_attn_weights(scores.data_ptr(), scores.stride(0), scores.stride(1), score_stats.data_ptr(),
                                  B, H, m, order.data_ptr() if order is not None else None, out.data_ptr(),
                                  out.stride(0), 1 if accumulate else 0, stream_ptr(dev)), "hkv_attn_weights")
    return out


def block_scores(token_scores, seq_len, block_size):
    """Mean score of each block of block_size tokens (hkv_block_scores): fp32 [ceil(seq_len / bs)]."""
    _require_gpu(token_scores)
    ts = token_scores.contiguous()
    if ts.dtype != torch.float32 or ts.numel() < seq_len:
        raise HeteroKVError(-1, "block_scores: fp32 token scores with at least seq_len entries expected")
    nb = (seq_len + block_size - 1) // block_size
    out = torch.empty(nb, dtype=torch.float32, device=ts.device)
    check(load().hkv_block_scores(ts.data_ptr(), seq_len, block_size, out.data_ptr(), stream_ptr(ts.device)),
          "hkv_block_scores")
    return out


def eviction_candidates(token_scores, seq_len, block_size, sink_tokens, local_window, max_blocks):
    """Lowest-mean unprotected blocks, ascending (hkv_eviction_candidates): int64 [k]."""
    _require_gpu(token_scores)
    ts = token_scores.contiguous()
    if ts.dtype != torch.float32 or ts.numel() < seq_len:
        raise HeteroKVError(-1, "eviction_candidates: fp32 token scores with at least seq_len entries expected")
    lib = load()
    wsb = lib.hkv_eviction_workspace_bytes(seq_len, block_size, sink_tokens, local_window, max_blocks)
    ws = torch.empty(max(wsb, 8), dtype=torch.uint8, device=ts.device)
    out = torch.empty(max(max_blocks, 1), dtype=torch.int64, device=ts.device)
    k = _lib.i32(0)
    check(lib.hkv_eviction_candidates(ts.data_ptr(), seq_len, block_size, sink_tokens, local_window, max_blocks,
                                      out.data_ptr(), ctypes.byref(k), ws.data_ptr(), ws.numel(),
                                      stream_ptr(ts.device)), "hkv_eviction_candidates")
    return out[:k.value]


# ----------------------------------------------------------------------- prefill attention
_PREFILL_WS = {}


def _prefill_workspace(dev, nbytes):
    """Per-device scratch for the chunk in the zone layout and the zone kernel's softmax
    state (no zero fill needed); grown on demand.  Calls that share it are ordered on the
    device's current stream."""
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    buf = _PREFILL_WS.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(max(nbytes, 4096), dtype=torch.uint8, device=dev)
        _PREFILL_WS[key] = buf
    return buf


def prefill_attention(q, zones=(), pool=None, block_table=None, int4_lens=None, int4_max_len=0,
                      chunk_k=None, chunk_v=None, sm_scale=None, out=None, staging=None, err=None,
                      out_dtype=None, workspace=None):
    """Chunked-prefill attention (hkv_prefill_attn).

    q: [B, Hq, Sq, 128] fp16 or bf16.  Every query attends to all fp16-zone tokens and all
    INT4 tokens, plus -- when chunk_k/chunk_v [B, Hkv, Sq, 128] (fp16 or bf16) are given --
    causally to the chunk itself.  bf16 inputs are range-checked into the error word
    (err: ErrorWord; default: the INT4 pool's).  Returns [B, Hq, Sq, 128] in out_dtype
    (default q's dtype).  workspace: a uint8 device tensor of at least
    hkv_prefill_workspace_bytes(B, Hq, Sq) bytes, used with a causal chunk or with INT4 and
    zone keys (default: a cached per-device buffer, for calls ordered on one stream).
    """
    _require_gpu(q, chunk_k, chunk_v)
    if q.dtype not in _F16_OR_BF16 or q.dim() != 4 or q.shape[-1] != HEAD_DIM:
        raise HeteroKVError(-1, "prefill_attention: q must be fp16 or bf16 [B, Hq, Sq, 128]")
    if out_dtype is None:
        out_dtype = q.dtype if out is None else out.dtype
    if out_dtype not in _F16_OR_BF16:
        raise HeteroKVError(-1, "prefill_attention: out dtype must be fp16 or bf16")
    if q.stride(-1) != 1 or q.data_ptr() % 16 or any(st % 8 for st in q.stride()[:3]):
        q = q.contiguous()
    B, Hq, Sq, _ = q.shape
    Hkv = _int4_source(pool, staging) or (zones[0][0].num_kv_heads if zones else
                                          (chunk_k.shape[1] if chunk_k is not None else None))
    if Hkv is None:
        raise HeteroKVError(-1, "prefill_attention: no key/value source given")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(HEAD_DIM)
    dev = q.device
    if out is None:
        out = torch.empty((B, Hq, Sq, HEAD_DIM), dtype=out_dtype, device=dev)
    elif out.dtype != out_dtype:
        raise HeteroKVError(-1, "prefill_attention: out is %s, out_dtype %s" % (out.dtype, out_dtype))
    a = _lib.PrefillArgs()
    a.q_dtype, a.out_dtype = _DTYPES[q.dtype], _DTYPES[out_dtype]
    a.chunk_dtype = _DTYPES[chunk_k.dtype] if chunk_k is not None else _lib.DTYPE_F16
    a.batch, a.num_q_heads, a.num_kv_heads, a.head_dim, a.num_queries = B, Hq, Hkv, HEAD_DIM, Sq
    a.sm_scale = float(sm_scale)
    a.q, a.q_stride_b, a.q_stride_h, a.q_stride_t = q.data_ptr(), q.stride(0), q.stride(1), q.stride(2)
    keep = []
    a.num_f16_zones = len(zones)
    for i, (z, lens, max_len) in enumerate(zones):
        lt = None
        if lens is not None:
            lt = _i32(lens, dev)
            keep.append(lt)
        a.f16[i] = _lib.F16Zone(k=z.k.data_ptr(), v=z.v.data_ptr(), capacity=z.capacity, max_len=int(max_len),
                                lens=lt.data_ptr() if lt is not None else 0)
    pool_err = None
    if int4_max_len > 0:
        bt = _i32(block_table, dev)
        if bt.dim() == 1:
            bt = bt.unsqueeze(0)
        keep.append(bt)
        if pool is None and staging is None:
            raise HeteroKVError(-1, "prefill_attention: INT4 zone needs a pool and a block table")
        if pool is not None:
            a.pool, a.pool_blocks = pool.data.data_ptr(), pool.num_blocks
        if staging is not None:
            a.staging, a.staging_blocks = staging.data.data_ptr(), staging.num_blocks
        a.block_table, a.bt_stride = bt.data_ptr(), bt.shape[1]
        pool_err = (pool if pool is not None else staging).err
        if int4_lens is not None:
            il = _i32(int4_lens, dev)
            keep.append(il)
            a.int4_lens = il.data_ptr()
    a.int4_max_len = int(int4_max_len)
    if chunk_k is not None:
        if chunk_k.shape != (B, Hkv, Sq, HEAD_DIM) or chunk_v.shape != chunk_k.shape:
            raise HeteroKVError(-1, "prefill_attention: chunk K/V must be [B, Hkv, Sq, 128]")
        if chunk_k.dtype != chunk_v.dtype or chunk_k.dtype not in _F16_OR_BF16:
            raise HeteroKVError(-1, "prefill_attention: chunk K/V must both be fp16 or bf16")
        if chunk_k.stride() != chunk_v.stride() or not _aligned16(chunk_k) or not _aligned16(chunk_v):
            chunk_k, chunk_v = chunk_k.contiguous(), chunk_v.contiguous()
        a.chunk_k, a.chunk_v = chunk_k.data_ptr(), chunk_v.data_ptr()
        a.chunk_stride_b, a.chunk_stride_h, a.chunk_stride_t = chunk_k.stride(0), chunk_k.stride(1), chunk_k.stride(2)
    a.out, a.out_stride_b, a.out_stride_h, a.out_stride_t = out.data_ptr(), out.stride(0), out.stride(1), out.stride(2)
    if err is not None:
        a.err_flag = err.ptr()
    else:
        a.err_flag = pool_err.data_ptr() if pool_err is not None else 0
    zone_keys = chunk_k is not None or any(int(mx) > 0 for (_, _, mx) in zones)
    if chunk_k is not None or (zone_keys and int4_max_len > 0):
        need = load().hkv_prefill_workspace_bytes(B, Hq, Sq)
        ws = workspace if workspace is not None else _prefill_workspace(dev, need)
        if ws.device != dev or ws.dtype != torch.uint8 or ws.numel() < need:
            raise HeteroKVError(-1, "prefill_attention: workspace must be a uint8 tensor of %d bytes on %s" % (need, dev))
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    check(load().hkv_prefill_attn(ctypes.byref(a), stream_ptr(dev)), "hkv_prefill_attn")
    return out
