"""Host tier: pinned arena + side-stream prefetcher, and the reference's host-tier classes.

* `Prefetcher` wraps the native handle (hkv_pf_*): a hipHostMalloc arena, a
  default-priority side stream and per-slot events.  The manager's host tier
  keeps every offloaded INT4 block record of a layer contiguously in the arena
  and pulls them into an HBM staging buffer one layer ahead.
* `DRAMStorageManager` mirrors src/memory/dram_storage.py:20-222 (pinned-host
  dict of compressed chunks, byte accounting, optional caps).
* `AsyncPrefetcher` mirrors src/policy/prefetcher.py:21-123 (side-stream H2D +
  dequantize to bf16, fetch_if_ready makes the current stream wait).
* `AdaptivePrefetchController` mirrors src/policy/adaptive_prefetch_controller.py:33-143
  (window size w_t from attention volatility and miss rate).
"""
import collections
import ctypes
import math
from typing import Any, Dict, List, Optional, Tuple

import torch

from . import _lib
from ._lib import HeteroKVError, check, load, stream_ptr


class Prefetcher:
    """Native host-tier prefetcher (hkv_pf_create ... hkv_pf_destroy)."""

    def __init__(self, device, arena_bytes: int, num_slots: int = 2):
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise HeteroKVError(-1, "Prefetcher needs a ROCm GPU device, got %s" % self.device)
        idx = self.device.index if self.device.index is not None else torch.cuda.current_device()
        self.device = torch.device("cuda", idx)
        h = ctypes.c_void_p()
        check(load().hkv_pf_create(idx, int(arena_bytes), int(num_slots), ctypes.byref(h)), "hkv_pf_create")
        self._h = h
        self.arena_bytes = int(arena_bytes)
        self.num_slots = int(num_slots)
        self._side = None

    # ------------------------------------------------------------------ arena
    def host_ptr(self, offset: int = 0) -> int:
        p = load().hkv_pf_host_ptr(self._h, int(offset))
        if not p:
            raise HeteroKVError(-3, "arena offset %d outside the %d-byte arena" % (offset, self.arena_bytes))
        return p

    def host_tensor(self, offset: int, nbytes: int) -> torch.Tensor:
        """uint8 CPU tensor aliasing arena bytes [offset, offset + nbytes) (valid until close())."""
        if offset < 0 or nbytes < 0 or offset + nbytes > self.arena_bytes:
            raise HeteroKVError(-3, "arena range [%d, %d) outside the %d-byte arena" %
                                (offset, offset + nbytes, self.arena_bytes))
        if nbytes == 0:
            return torch.empty(0, dtype=torch.uint8)
        buf = (ctypes.c_uint8 * nbytes).from_address(self.host_ptr(offset))
        return torch.frombuffer(buf, dtype=torch.uint8)

    def stage_out(self, src: torch.Tensor, offset: int, stream=None) -> None:
        """Device -> arena copy of a contiguous device tensor's bytes, on `stream` (current)."""
        if src.device.type != "cuda" or not src.is_contiguous():
            raise HeteroKVError(-1, "stage_out: source must be a contiguous device tensor")
        nbytes = src.numel() * src.element_size()
        sp = stream_ptr(self.device) if stream is None else ctypes.c_void_p(stream.cuda_stream)
        check(load().hkv_pf_stage_out(self._h, src.data_ptr(), int(offset), nbytes, sp), "hkv_pf_stage_out")

    # ------------------------------------------------------------------ schedule
    def submit(self, copies: List[Tuple[int, int, int]], slot: int, after_slot: int = -1) -> None:
        """Side stream: wait for after_slot's "free" mark, copy (device_dst_ptr, host_src_ptr,
        nbytes) triples, record slot's "ready"."""
        n = len(copies)
        arr = (_lib.CopyDesc * max(n, 1))()
        for i, (dst, src, nb) in enumerate(copies):
            arr[i].dst, arr[i].src, arr[i].bytes = int(dst), int(src), int(nb)
        check(load().hkv_pf_submit(self._h, arr, n, int(slot), int(after_slot)), "hkv_pf_submit")

    def record(self, slot: int) -> None:
        check(load().hkv_pf_record(self._h, int(slot)), "hkv_pf_record")

    def wait(self, slot: int, stream=None) -> None:
        sp = stream_ptr(self.device) if stream is None else ctypes.c_void_p(stream.cuda_stream)
        check(load().hkv_pf_wait(self._h, int(slot), sp), "hkv_pf_wait")

    def mark(self, slot: int, stream=None) -> None:
        sp = stream_ptr(self.device) if stream is None else ctypes.c_void_p(stream.cuda_stream)
        check(load().hkv_pf_mark(self._h, int(slot), sp), "hkv_pf_mark")

    def stall_ms(self, slot: int) -> float:
        v = ctypes.c_float()
        check(load().hkv_pf_stall_ms(self._h, int(slot), ctypes.byref(v)), "hkv_pf_stall_ms")
        return float(v.value)

    def stats(self) -> Dict[str, int]:
        st = _lib.PfStats()
        check(load().hkv_pf_stats(self._h, ctypes.byref(st)), "hkv_pf_stats")
        return {"bytes_h2d": st.bytes_h2d, "copies_h2d": st.copies_h2d, "bytes_d2h": st.bytes_d2h,
                "arena_bytes": st.arena_bytes}

    def synchronize(self) -> None:
        check(load().hkv_pf_synchronize(self._h), "hkv_pf_synchronize")

    @property
    def side_stream(self) -> torch.cuda.ExternalStream:
        """The side stream as a torch stream (for work added after a submit)."""
        if self._side is None:
            self._side = torch.cuda.ExternalStream(load().hkv_pf_stream(self._h), device=self.device)
        return self._side

    def close(self) -> None:
        if self._h is not None and self._h.value:
            load().hkv_pf_destroy(self._h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


_ENTRY_KEYS = ("k_data", "k_scales", "k_zps", "v_data", "v_scales", "v_zps")


class DRAMStorageManager:
    """Pinned-host store of compressed chunks (dram_storage.py:20-222).

    Each entry's six tensors live in one pinned allocation (a new pinned tensor,
    not a page-locked copy of a pageable one), viewed as the six tensors."""

    def __init__(self, max_entries: Optional[int] = None, max_bytes: Optional[int] = None):
        self.max_entries = max_entries
        self.max_bytes = max_bytes
        self._table: Dict[str, Dict[str, torch.Tensor]] = {}
        self._total_bytes = 0

    @staticmethod
    def _nbytes(t: torch.Tensor) -> int:
        return t.element_size() * t.nelement()

    def _pin_entry(self, entry: Dict[str, torch.Tensor]) -> Dict[str, torch.Tensor]:
        sizes = [(self._nbytes(entry[k]) + 15) // 16 * 16 for k in _ENTRY_KEYS]
        slab = torch.empty(sum(sizes), dtype=torch.uint8, pin_memory=True)
        out, off = {}, 0
        for k, sz in zip(_ENTRY_KEYS, sizes):
            t = entry[k]
            view = slab[off:off + self._nbytes(t)].view(t.dtype).view(t.shape)
            view.copy_(t)
            out[k] = view
            off += sz
        return out

    def _fits(self, entry_bytes: int, key: str) -> bool:
        # the caps count the replaced entry too, as dram_storage.py:126-129 does
        if self.max_entries is not None and len(self._table) >= self.max_entries:
            return False
        if self.max_bytes is not None and self._total_bytes + entry_bytes > self.max_bytes:
            return False
        return True

    def store(self, chunk_key: str, q_k, k_scales, k_zps, q_v, v_scales, v_zps) -> bool:
        return self.store_entry(chunk_key, {"k_data": q_k, "k_scales": k_scales, "k_zps": k_zps,
                                            "v_data": q_v, "v_scales": v_scales, "v_zps": v_zps})

    def store_entry(self, chunk_key: str, entry: Dict[str, torch.Tensor]) -> bool:
        if not all(k in entry for k in _ENTRY_KEYS):
            raise ValueError("Entry missing required keys. Need: %s" % (_ENTRY_KEYS,))
        entry_bytes = sum(self._nbytes(entry[k]) for k in _ENTRY_KEYS)
        if not self._fits(entry_bytes, chunk_key):
            return False
        if chunk_key in self._table:
            self._total_bytes -= self._entry_bytes(chunk_key)
        self._table[chunk_key] = self._pin_entry(entry)
        self._total_bytes += entry_bytes
        return True

    def retrieve(self, chunk_key: str) -> Optional[Dict[str, torch.Tensor]]:
        return self._table.get(chunk_key)

    def remove(self, chunk_key: str) -> Optional[Dict[str, torch.Tensor]]:
        entry = self._table.pop(chunk_key, None)
        if entry is not None:
            self._total_bytes -= sum(self._nbytes(t) for t in entry.values())
        return entry

    def contains(self, chunk_key: str) -> bool:
        return chunk_key in self._table

    def transfer_to_device(self, chunk_key: str, device, non_blocking: bool = True):
        entry = self._table.get(chunk_key)
        if entry is None:
            return None
        return {k: entry[k].to(device, non_blocking=non_blocking) for k in _ENTRY_KEYS}

    def _entry_bytes(self, chunk_key: str) -> int:
        return sum(self._nbytes(t) for t in self._table[chunk_key].values())

    @property
    def table(self) -> Dict[str, Dict[str, torch.Tensor]]:
        return self._table

    @property
    def total_bytes(self) -> int:
        return self._total_bytes

    @property
    def num_entries(self) -> int:
        return len(self._table)

    @property
    def keys(self) -> List[str]:
        """Chunk keys in insertion order (a property, as dram_storage.py:211-213)."""
        return list(self._table.keys())

    def memory_summary(self) -> Dict[str, Any]:
        """Entry count and stored bytes (dram_storage.py:217-222); the bytes are the
        entries' tensor bytes, not the 16-byte-rounded pinned slabs holding them."""
        return {"num_entries": len(self._table), "total_bytes": self._total_bytes,
                "total_mb": self._total_bytes / (1024 * 1024)}

    def clear(self) -> None:
        self._table.clear()
        self._total_bytes = 0


class AsyncPrefetcher:
    """Side-stream chunk prefetch (prefetcher.py:21-123): H2D of the six entry tensors and
    dequantize to bf16 on the native prefetcher's side stream; fetch_if_ready makes the
    current stream wait for that chunk's "ready" event only."""

    _SLOTS = 256

    def __init__(self, device):
        self.device = torch.device(device)
        self._pf = Prefetcher(self.device, 0, self._SLOTS) if self.device.type == "cuda" else None
        self.prefetch_stream = self._pf.side_stream if self._pf is not None else None
        self.buffer: Dict[str, Tuple[torch.Tensor, torch.Tensor]] = {}
        self._slot_of: Dict[str, int] = {}
        self._free_slots = list(range(self._SLOTS))

    @property
    def free_slots(self) -> int:
        """Chunks that can still be submitted before one is fetched or cleared."""
        return len(self._free_slots)

    def submit_prefetch_task(self, chunk_key: str, dram_data: Dict[str, Any], compressor) -> None:
        """prefetcher.py:47-98.  Entries held in host memory are copied on the side stream
        first; entries already on this device (the GPU manager's chunks) are dequantized
        there directly."""
        if chunk_key in self.buffer:
            return
        split = "k_data" in dram_data and "v_data" in dram_data
        merged = "q_data" in dram_data
        if not split and not merged:
            return
        if self._pf is None:
            raise HeteroKVError(-1, "AsyncPrefetcher needs a ROCm GPU device")
        if not self._free_slots:
            raise HeteroKVError(-3, "AsyncPrefetcher: more than %d chunks pending" % self._SLOTS)
        names = _ENTRY_KEYS if split else ("q_data", "scales", "zps")
        on_device = all(dram_data[k].device == self.device for k in names)
        dev_t, copies = {}, []
        for k in names:
            src = dram_data[k]
            if on_device:
                dev_t[k] = (None, src)
                continue
            if src.device.type != "cpu":
                src = src.cpu()
            src = src.contiguous()
            dst = torch.empty(src.shape, dtype=src.dtype, device=self.device)
            dst.record_stream(self._pf.side_stream)
            copies.append((dst.data_ptr(), src.data_ptr(), src.numel() * src.element_size()))
            dev_t[k] = (src, dst)
        slot = self._free_slots.pop()
        side = self._pf.side_stream
        # the destinations (or the device entry) come from the current stream: the side
        # stream must not touch them before that stream reaches this point
        side.wait_stream(torch.cuda.current_stream(self.device))
        self._pf.submit(copies, slot)
        with torch.cuda.stream(side):
            if on_device:
                for _, t in dev_t.values():
                    t.record_stream(side)
            if split:
                rk = compressor.decompress(dev_t["k_data"][1], dev_t["k_scales"][1], dev_t["k_zps"][1]).to(torch.bfloat16)
                rv = compressor.decompress(dev_t["v_data"][1], dev_t["v_scales"][1], dev_t["v_zps"][1]).to(torch.bfloat16)
            else:
                rk = compressor.decompress(dev_t["q_data"][1], dev_t["scales"][1], dev_t["zps"][1]).to(torch.bfloat16)
                rv = rk
        self._pf.record(slot)
        # keep host sources alive until the copies are done (consumed at fetch)
        self._host_refs = getattr(self, "_host_refs", {})
        self._host_refs[chunk_key] = [s for s, _ in dev_t.values() if s is not None]
        self.buffer[chunk_key] = (rk, rv)
        self._slot_of[chunk_key] = slot

    def fetch_if_ready(self, chunk_key: str) -> Optional[Tuple[torch.Tensor, torch.Tensor]]:
        if chunk_key not in self.buffer:
            return None
        slot = self._slot_of.pop(chunk_key)
        cur = torch.cuda.current_stream(self.device)
        self._pf.wait(slot)
        k, v = self.buffer.pop(chunk_key)
        k.record_stream(cur)
        if v is not k:
            v.record_stream(cur)
        self._host_refs.pop(chunk_key, None)
        self._free_slots.append(slot)
        return k, v

    def clear(self) -> None:
        if self._pf is not None:
            self._pf.synchronize()
        self.buffer.clear()
        for k in list(self._slot_of):
            self._free_slots.append(self._slot_of.pop(k))
        getattr(self, "_host_refs", {}).clear()

    @property
    def pending_keys(self):
        return list(self.buffer.keys())


class AdaptivePrefetchController:
    """Prefetch window w_t (adaptive_prefetch_controller.py:33-143):
    raw = w_min + clip((sigma_t / sigma_ref - 1) * alpha, +-delta_max) + beta * miss_rate * w_max,
    w = clamp(round(raw), w_min, w_max) moved by at most 1 per step; sigma_ref is an EMA of the
    attention-weight standard deviation (torch.std, unbiased)."""

    def __init__(self, w_min: int = 2, w_max: int = 8, alpha: float = 1.5, beta: float = 0.5,
                 delta_max: float = 2.0, ema_decay: float = 0.9, miss_window_size: int = 16):
        self.w_min, self.w_max = w_min, w_max
        self.alpha, self.beta = alpha, beta
        self.delta_max, self.ema_decay = delta_max, ema_decay
        self.miss_window_size = miss_window_size
        self._window = float(w_min)                      # the last window handed out
        self._ema_sigma: Optional[float] = None          # None until the first weights arrive
        self._misses = collections.deque(maxlen=max(1, miss_window_size))
        self._calls = 0

    def _miss_rate(self) -> float:
        return sum(self._misses) / len(self._misses) if self._misses else 0.0

    def _volatility(self, attention_weights: Optional[torch.Tensor]) -> float:
        """Clipped relative deviation of this step's weight spread from its running mean."""
        if attention_weights is None or attention_weights.numel() <= 1:
            return 0.0
        sigma = float(attention_weights.detach().cpu().std())
        if self._ema_sigma is None:
            self._ema_sigma = sigma
        else:
            self._ema_sigma = self.ema_decay * self._ema_sigma + (1.0 - self.ema_decay) * sigma
        rel = sigma / self._ema_sigma - 1.0 if self._ema_sigma > 1e-8 else 0.0
        return min(self.delta_max, max(-self.delta_max, rel * self.alpha))

    def compute_window(self, attention_weights: Optional[torch.Tensor] = None, cache_miss: bool = False) -> int:
        self._calls += 1
        self._misses.append(bool(cache_miss))
        target = self.w_min + self._volatility(attention_weights) + self.beta * self._miss_rate() * self.w_max
        w = min(self.w_max, max(self.w_min, round(target)))
        # the window moves by at most one per step
        step = w - self._window
        if abs(step) > 1:
            w = int(self._window + (1 if step > 0 else -1))
        self._window = float(w)
        return int(w)

    @property
    def stats(self) -> Dict[str, float]:
        """The reference's report keys: current window, reference spread, miss rate, steps."""
        return {"current_w": self._window, "sigma_ref": self._ema_sigma if self._ema_sigma is not None else 0.0,
                "miss_rate": self._miss_rate(), "step": self._calls}
