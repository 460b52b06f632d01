"""HeteroKVManager: three-zone KV storage on the GPU.

Drop-in for src/memory/manager.py:30-1299 of the reference.  Per layer:
  * sink zone      -- the first `sink_tokens` tokens, fp16           (manager.py:462-466)
  * tail zone      -- the most recent `hbm_budget_tokens - sink_tokens`
                      tokens, fp16, kept as a ring                    (manager.py:480-485,618-664)
  * heavy hitters  -- tokens slid out of the tail at decode, fp16     (manager.py:686-715)
  * INT4 middle    -- every token evicted at prefill, quantized and
                      nibble-packed into 16-token block records by the
                      append kernel, in eviction order                (manager.py:1231-1299)
The reference keeps the middle in pinned host memory and copies + dequantizes
all of it to fp16 on every decode step (manager.py:779-821); here it stays INT4
in HBM and the split-K kernel reads it in place (`attend_decode`).

Index semantics follow the reference exactly (zone boundaries, eviction
ranges, chunk keys "l{layer}_e{counter}" with the counter moving only on layer
0, FIFO heavy-hitter fill, count_dram_tokens).  `positions(layer)` returns the
absolute token positions in the order the reference returns K/V, for index
parity checks.  Deliberate differences, all on paths that cannot change an
attended token: tokens that the reference leaves in its competition queue after
the heavy-hitter zone is full are not retained (they are never attended again);
the queue is kept per layer (equal to the reference's shared queue when layers
update in lockstep, the only way transformers drives a cache); zones store
fp16: bf16 inputs are narrowed by the zone kernels, exactly for magnitudes in
[2^-14, 65504], and a finite value beyond the fp16 range is reported as a
HeteroKVError (the manager's device error word, read without a per-launch sync
at the next step, or at once by check_errors()).
"""
from collections import OrderedDict, deque
from typing import Any, Dict, List, Optional, Tuple

import numpy as np
import torch

from . import ops
from . import _lib
from ._lib import BLOCK_TOKENS, HEAD_DIM, HeteroKVError
from .heavy_hitter import HeavyHitterOracle
from .kv_compressor import KVCompressor
from .prefetcher import AdaptivePrefetchController, AsyncPrefetcher, Prefetcher


class _Scores(dict):
    """Chunk scores that count their writes, so that a layer's cached ranking is rebuilt
    after any change."""
    epoch = 0

    def __setitem__(self, k, v):
        self.epoch += 1
        super().__setitem__(k, v)

    def __delitem__(self, k):
        self.epoch += 1
        super().__delitem__(k)

    def update(self, *a, **kw):
        self.epoch += 1
        super().update(*a, **kw)

    def pop(self, *a):
        self.epoch += 1
        return super().pop(*a)

    def popitem(self):
        self.epoch += 1
        return super().popitem()

    def setdefault(self, k, d=None):
        self.epoch += 1
        return super().setdefault(k, d)

    def clear(self):
        self.epoch += 1
        super().clear()


class _LayerState:
    def __init__(self, B, H, device, dtype, sink_tokens, tail_budget, hh_budget, err):
        self.B, self.H, self.device, self.dtype = B, H, device, dtype
        self.err = err                             # the manager's ErrorWord
        self.sink = ops.F16Zone(B, H, max(sink_tokens, 1), device)
        self.sink_len = 0
        self.sink_pos: List[int] = []
        self.ring = max(tail_budget, 1)
        self.tail = ops.F16Zone(B, H, self.ring, device)
        self.tail_head = 0
        self.tail_len = 0
        self.tail_pos = deque()
        self.tail_started = False
        self.hh = ops.F16Zone(B, H, max(hh_budget, 1), device)
        self.hh_len = 0
        self.hh_pos: List[int] = []
        self.hh_started = False
        # device copies of (tail_head, tail_len, hh_len, dropped) and the per-sequence zone
        # lengths, used by device-stepped decode (None: not in sync with the host values)
        self.dev_state: Optional[torch.Tensor] = None
        self.dev_tail_lens: Optional[torch.Tensor] = None
        self.dev_hh_lens: Optional[torch.Tensor] = None
        self.pool: Optional[ops.Int4Pool] = None
        self.pool_used = 0                         # pool records in use
        self.bt: Optional[torch.Tensor] = None     # device int32 [B, cap]: logical block -> record id
        self.bt_host: Optional[np.ndarray] = None  # host mirror of bt
        self.nb = 0                                # logical blocks allocated per sequence
        self.int4_len = 0
        self.int4_pos: List[int] = []
        self.prefilled = False
        self.seq_offset = 0
        # host tier: records ~0 .. ~(n_host-1) live in the pinned arena at host_off, in
        # (logical block, sequence) order; host_lbs[k] is the logical block of record k
        self.n_host = 0
        self.host_off = 0
        self.host_lbs: Optional[np.ndarray] = None
        self.version = 0                           # bumped whenever bt or pool change
        self.resident_cache = None
        self.runs_cache = None                     # (version, selection, host runs)
        # deferred write of a prefill chunk into the tail ring: (k, v, first chunk token
        # written, its ring slot, tail length before the chunk); see _incremental_prefill
        self.pending = None

    # -------------------------------------------------------------- INT4 pool
    def ensure_int4(self, n_tokens):
        """Allocate pool records for logical blocks up to n_tokens (new records are
        appended; earlier ones, resident or host, keep their ids)."""
        need = (n_tokens + BLOCK_TOKENS - 1) // BLOCK_TOKENS
        if need <= self.nb:
            return
        B = self.B
        cap = self.bt_host.shape[1] if self.bt_host is not None else 0
        if need > cap:
            bh = np.zeros((B, max(need, 2 * cap, 64)), dtype=np.int32)
            if cap:
                bh[:, :cap] = self.bt_host
            self.bt_host = bh
        add = need - self.nb
        used = self.pool_used + B * add
        pcap = self.pool.num_blocks if self.pool is not None else 0
        if used > pcap:
            pool = ops.Int4Pool(max(used, 2 * pcap, 64 * B), self.H, self.device)
            if self.pool is not None and self.pool_used:
                pool.data[:self.pool_used].copy_(self.pool.data[:self.pool_used])
            self.pool = pool
        self.bt_host[:, self.nb:need] = (self.pool_used + np.arange(B, dtype=np.int32)[:, None] * add +
                                         np.arange(add, dtype=np.int32)[None, :])
        self.pool_used, self.nb = used, need
        self.bt = ops.h2d(torch.from_numpy(self.bt_host), self.device)
        self.version += 1

    # -------------------------------------------------------------- tail ring
    def flush(self):
        """Apply a deferred prefill-chunk write to the tail ring."""
        if self.pending is None:
            return
        k, v, i0, slot, _ = self.pending
        self.pending = None
        if k.shape[2] > i0:
            self.tail.write(k[:, :, i0:], v[:, :, i0:], slot, ring=self.ring, err=self.err)

    def tail_tensors(self, i0=0, i1=None):
        """Tail tokens [i0, i1) in logical (oldest first) order, fp16 [B, H, i1 - i0, 128]."""
        self.flush()
        i1 = self.tail_len if i1 is None else i1
        n = i1 - i0
        if n <= 0:
            e = torch.empty((self.B, self.H, 0, HEAD_DIM), dtype=torch.float16, device=self.device)
            return e, e.clone()
        s0 = self.tail_head + i0
        if s0 % self.ring + n <= self.ring and s0 < self.ring:
            if s0 == 0:
                return self.tail.read(n)
            k, v = self.tail.read(s0 + n)
            return k[:, :, s0:], v[:, :, s0:]
        k, v = self.tail.read(self.ring)
        idx = (torch.arange(n, device=self.device) + s0) % self.ring
        return k.index_select(2, idx), v.index_select(2, idx)

    def write_tail(self, k, v):
        """Replace the tail with k, v (logical order), starting at ring slot 0."""
        self.pending = None
        n = k.shape[2]
        if n:
            self.tail.write(k, v, 0, err=self.err)
        self.tail_head, self.tail_len = 0, n
        self.dev_state = None


class HeteroKVManager:
    """Tiered KV manager with the reference's constructor and public methods."""

    def __init__(self, num_layers: int, sink_tokens: int = 64, hbm_budget_tokens: int = 8192,
                 device: str = "cuda", enable_quant: bool = True, enable_prefetch: bool = True,
                 group_size: int = 128, bits: int = 4, bandwidth_limiter=None,
                 enable_method_d: bool = False, method_d_alpha: float = 1.0):
        if group_size != HEAD_DIM or bits != 4:
            raise HeteroKVError(-4, "HeteroKVManager stores one INT4 group per 128-value token row "
                                    "(group_size=128, bits=4); got group_size=%d bits=%d" % (group_size, bits))
        if enable_method_d:
            raise HeteroKVError(-4, "query-aware retrieval (Method D) is not part of this library")
        self.num_layers = num_layers
        self.sink_tokens = sink_tokens
        self.hbm_budget_tokens = hbm_budget_tokens
        self.device = torch.device(device)
        self.enable_quant = enable_quant
        self.enable_prefetch = enable_prefetch
        self.group_size = group_size
        self.bits = bits
        self._bandwidth_limiter = bandwidth_limiter
        self._heavyhitter_budget = max(hbm_budget_tokens // 2, 2048)
        self._compressor = KVCompressor(group_size=group_size, bits=bits)
        self._layers: List[Optional[_LayerState]] = [None] * num_layers
        # chunk key -> (layer, first INT4 slot, token count), in eviction order
        self._chunks: "OrderedDict[str, Tuple[int, int, int]]" = OrderedDict()
        self._chunk_eviction_order: List[str] = []
        # the same keys per layer, in eviction order (decode looks a layer's chunks up every
        # step; scanning every layer's keys cost ~4 ms per token at 128K over 28 layers)
        self._layer_keys: Dict[int, List[str]] = {}
        # a layer's chunk keys by descending score, and the selection per window size,
        # kept until the layer's chunks or any chunk score change
        self._ranked: Dict[int, Tuple[int, List[str]]] = {}
        self._sel_cache: Dict[Tuple[int, int], Tuple[int, Tuple[str, ...]]] = {}
        self._chunk_attention_scores: Dict[str, float] = _Scores()
        self._eviction_counter = 0
        self._queued_tokens = 0      # tokens the reference would leave in its competition queue
        self._workspace = None
        self._err: Optional[ops.ErrorWord] = None
        self._async_pf: Optional[AsyncPrefetcher] = None
        self._top_layer = -1         # highest layer index attended so far (end of a decode step)
        # True: decode launches use the fixed block-to-wave schedule (bitwise
        # reproducible); False: blocks go to waves on demand (faster)
        self.deterministic_decode = False
        # host tier (offload_to_host) and its prefetch schedule
        self._pf: Optional[Prefetcher] = None
        self._staging: List[ops.Int4Pool] = []
        self._buf_owner: List[int] = []
        self._next_buf = 0
        # layer -> (staging buffer, selection, event slot).  Each layer owns two event slots
        # (2 * layer + parity) used alternately, so the events of one step's wait survive
        # the look-ahead submission of the next step until prefetch_stats reads them.
        self._pending: Dict[int, Tuple[int, Any, int]] = {}
        self._slot_parity: Dict[int, int] = {}
        self._waited: List[int] = []
        # host-tier copies of a decode step under graph capture (begin_graph_staging):
        # gather kernels on the capturing stream instead of the native side stream
        self._graph_staging = False
        self._graph_ids: Optional[torch.Tensor] = None
        self._selection_of: Dict[int, Any] = {}
        self._window_tables: Dict[Any, Tuple[torch.Tensor, int]] = {}
        self._selection_b: Dict[int, List[str]] = {}
        # retrieval of the INT4 middle at decode: None = every chunk (decompress_dram_chunks,
        # manager.py:779-821); an int or "adaptive" = the top-w chunks by score
        # (get_dram_chunks_quantized_adaptive, manager.py:931-1056)
        self._retrieval_window: Any = None
        self._adaptive_controller = AdaptivePrefetchController()
        self._last_attention_weights: Optional[torch.Tensor] = None
        # device-stepped decode (enable_device_decode): zone decisions and lengths on the GPU
        self.device_decode = False
        # cumulative attention scores (manager.py:102-106); fed by update_attention_scores
        # or attend_decode(feed_oracle=True)
        self._oracle = HeavyHitterOracle(block_size=16, sink_tokens=sink_tokens, local_window=hbm_budget_tokens)

    # ---------------------------------------------------------------- helpers
    @property
    def retrieval_window(self) -> Any:
        """None: every INT4 chunk joins decode attention (Path C, manager.py:779-821); an int
        or "adaptive": the top-w chunks by score (Path A, manager.py:931-1056)."""
        return self._retrieval_window

    @retrieval_window.setter
    def retrieval_window(self, w: Any) -> None:
        # selections made ahead of time by the look-ahead belong to the old window
        self._selection_of.clear()
        self._selection_b.clear()
        self._retrieval_window = w

    @property
    def tail_budget(self) -> int:
        return self.hbm_budget_tokens - self.sink_tokens

    # ---------------------------------------------------------------- device error word
    def _errword(self) -> "ops.ErrorWord":
        """The device int32 every kernel of this manager reports HKV_ERR_BIT_* into."""
        if self._err is None:
            self._err = ops.ErrorWord(self.device)
            self._err.on_error = self._on_device_error
        return self._err

    def _on_device_error(self, bits: int) -> None:
        if bits & _lib.ERR_BIT_PLACEMENT and self._workspace is not None:
            self._workspace.placement_failed()

    def check_errors(self) -> None:
        """Raise HeteroKVError if any kernel of this manager reported a device error
        (bad block id, slot, decode placement, bf16 range) since the last check.  This
        synchronizes; attend_decode checks without blocking (one step late)."""
        if self._err is not None:
            self._err.check()

    def _state(self, layer_idx, key_states) -> _LayerState:
        if layer_idx < 0:
            raise ValueError("Invalid layer %d" % layer_idx)
        while len(self._layers) <= layer_idx:
            self._layers.append(None)
        st = self._layers[layer_idx]
        if st is None:
            B, H, _, D = key_states.shape
            if D != HEAD_DIM:
                raise HeteroKVError(-4, "head_dim must be 128, got %d" % D)
            st = _LayerState(B, H, key_states.device, key_states.dtype, self.sink_tokens, self.tail_budget,
                             self._heavyhitter_budget, self._errword())
            self._layers[layer_idx] = st
        return st

    def _check_input(self, key_states, value_states):
        if key_states.device.type != "cuda":
            raise HeteroKVError(-1, "HeteroKVManager keeps KV on a ROCm GPU; got a %s tensor" % key_states.device)
        if key_states.dim() != 4 or key_states.shape != value_states.shape:
            raise HeteroKVError(-1, "key/value states must both be [B, H, S, 128]")

    # ---------------------------------------------------------------- public API
    def allocate(self, layer: int, budget: Optional[int] = None) -> bool:
        """manager.py:152-170: pools are created lazily; optionally changes the budget."""
        if layer < 0 or layer >= self.num_layers:
            raise ValueError("Invalid layer %d, num_layers=%d" % (layer, self.num_layers))
        if budget is not None:
            self.hbm_budget_tokens = budget
        return True

    def update(self, layer_idx: int, key_states: torch.Tensor, value_states: torch.Tensor,
               mode: str = "prefill", seq_offset: int = 0, materialize: bool = True
               ) -> Tuple[Optional[torch.Tensor], Optional[torch.Tensor]]:
        """manager.py:175-204.  Returns the K/V the reference would hand to attention
        (prefill: the full input or sink + old tail + chunk; decode: sink + tail + heavy
        hitters).  With materialize=False the bookkeeping is done and (None, None) is
        returned, for callers that attend with `attend_decode` / `attend_prefill`: a later
        prefill chunk then leaves the old tail in place for attend_prefill and writes the
        chunk into the tail ring after it (or at the layer's next operation)."""
        if mode not in ("prefill", "decode"):
            raise ValueError("Unknown mode: %s" % mode)
        self._check_input(key_states, value_states)
        st = self._state(layer_idx, key_states)
        st.flush()
        if mode == "prefill":
            st.dev_state = None
            if st.prefilled:
                return self._incremental_prefill(layer_idx, st, key_states, value_states, seq_offset, materialize)
            return self._first_prefill(layer_idx, st, key_states, value_states, seq_offset)
        return self._decode(layer_idx, st, key_states, value_states, seq_offset, materialize)

    def _first_prefill(self, layer, st, k, v, seq_offset):
        n = k.shape[2]
        sink_amt = min(n, self.sink_tokens)
        if sink_amt:
            st.sink.write(k[:, :, :sink_amt], v[:, :, :sink_amt], 0, err=st.err)
        st.sink_len = sink_amt
        st.sink_pos = list(range(seq_offset, seq_offset + sink_amt))
        tail_amt = min(n - sink_amt, self.tail_budget)
        st.write_tail(k[:, :, n - tail_amt:], v[:, :, n - tail_amt:])
        st.tail_pos = deque(range(seq_offset + n - tail_amt, seq_offset + n))
        st.tail_started = True
        body0, body1 = sink_amt, n - tail_amt
        if self.enable_quant and body1 > body0:
            self._evict(layer, st, k[:, :, body0:body1], v[:, :, body0:body1], seq_offset + body0)
        st.hh_len, st.hh_pos, st.hh_started = 0, [], True
        st.prefilled = True
        st.seq_offset = seq_offset + n
        return k, v

    def _incremental_prefill(self, layer, st, k, v, seq_offset, materialize=True):
        if not materialize:
            return self._incremental_prefill_deferred(layer, st, k, v, seq_offset)
        n = k.shape[2]
        old_k, old_v = st.tail_tensors()
        old_pos = list(st.tail_pos)
        combined_k = torch.cat([old_k.to(k.dtype), k], dim=2)
        combined_v = torch.cat([old_v.to(v.dtype), v], dim=2)
        sk, sv = st.sink.read(st.sink_len) if st.sink_len else (combined_k[:, :, :0], combined_v[:, :, :0])
        ret_k = torch.cat([sk.to(k.dtype), combined_k], dim=2)
        ret_v = torch.cat([sv.to(v.dtype), combined_v], dim=2)
        combined_pos = old_pos + list(range(seq_offset, seq_offset + n))
        total = combined_k.shape[2]
        if total > self.tail_budget:
            e = total - self.tail_budget
            if self.enable_quant:
                self._evict(layer, st, combined_k[:, :, :e], combined_v[:, :, :e], combined_pos[:e])
            st.write_tail(combined_k[:, :, e:], combined_v[:, :, e:])
            st.tail_pos = deque(combined_pos[e:])
        else:
            st.write_tail(combined_k, combined_v)
            st.tail_pos = deque(combined_pos)
        st.seq_offset = seq_offset + n
        return ret_k, ret_v

    def _incremental_prefill_deferred(self, layer, st, k, v, seq_offset):
        """_incremental_prefill_update (manager.py:537-586) without materializing
        sink + old tail + chunk: the oldest tokens of [old tail | chunk] beyond the tail
        budget are evicted now, and the chunk's surviving tokens are written into the
        tail ring in place -- after attend_prefill has read the old tail (or at this
        layer's next operation).  While the write is pending the ring still holds the
        old tail: either it is not full and its tokens sit in slots [0, len), or it is
        full and every slot is valid, which is all attend_prefill needs."""
        n = k.shape[2]
        L, R = st.tail_len, st.ring
        old_pos = list(st.tail_pos)
        combined_pos = old_pos + list(range(seq_offset, seq_offset + n))
        total = L + n
        e = max(0, total - self.tail_budget)
        if e and self.enable_quant:
            eo = min(e, L)
            parts_k, parts_v = [], []
            if eo:
                ok, ov = st.tail_tensors(0, eo)
                parts_k.append(ok.to(k.dtype))
                parts_v.append(ov.to(v.dtype))
            if e > L:
                parts_k.append(k[:, :, :e - L])
                parts_v.append(v[:, :, :e - L])
            ek = parts_k[0] if len(parts_k) == 1 else torch.cat(parts_k, dim=2)
            ev = parts_v[0] if len(parts_v) == 1 else torch.cat(parts_v, dim=2)
            self._evict(layer, st, ek, ev, combined_pos[:e])
        i0 = max(0, e - L)                          # chunk tokens [i0, n) survive into the tail
        slot = (st.tail_head + L + i0) % R
        st.pending = (k, v, i0, slot, L)
        if e:
            st.tail_head = (st.tail_head + e) % R
            st.tail_len = R
        else:
            st.tail_len = total
        st.tail_pos = deque(combined_pos[e:])
        st.seq_offset = seq_offset + n
        return None, None

    def _decode(self, layer, st, k, v, seq_offset, materialize):
        if k.shape[2] != 1:
            raise HeteroKVError(-1, "decode expects one new token, got %d" % k.shape[2])
        if self.device_decode:
            if st.dev_state is None:
                self._sync_device_state(st)
            st.tail.step(st.hh, k, v, st.ring, self._heavyhitter_budget, st.dev_state, st.dev_tail_lens,
                         st.dev_hh_lens, err=st.err)
        self._decode_host(st, seq_offset, k, v, launch=not self.device_decode)
        if not materialize:
            return None, None
        kk, vv = self.get_hbm_kv(layer)
        return kk.to(k.dtype), vv.to(v.dtype)

    def _decode_host(self, st, seq_offset, k, v, launch):
        """The decode step's zone decision (manager.py:588-674 as this library keeps it), with
        its kernels when `launch` (device-stepped decode takes the same decision on the GPU)."""
        pos = seq_offset
        if st.tail_len < self.tail_budget:
            if launch:
                st.tail.write(k, v, st.tail_head + st.tail_len, ring=st.ring, err=st.err)
            st.tail_len += 1
            st.tail_pos.append(pos)
        else:
            # the oldest tail token leaves: into the heavy-hitter zone while it has room
            # (manager.py:645-664, 686-715), else it stays queued in the reference and is never
            # attended again
            old = st.tail_pos.popleft()
            if st.hh_len < self._heavyhitter_budget:
                if launch:
                    st.tail.copy_to(st.hh, st.tail_head, st.hh_len, 1)
                st.hh_len += 1
                st.hh_pos.append(old)
            else:
                self._queued_tokens += 1
            if launch:
                st.tail.write(k, v, st.tail_head, ring=st.ring, err=st.err)
            st.tail_head = (st.tail_head + 1) % st.ring
            st.tail_pos.append(pos)
        st.tail_started = True
        st.hh_started = True
        st.seq_offset = seq_offset + 1

    # ---------------------------------------------------------------- device-stepped decode
    def enable_device_decode(self, on: bool = True) -> None:
        """Take each decode step's zone decision on the GPU (hkv_zone_step) and let decode
        attention read the recent-window and heavy-hitter lengths from device counters.  A
        decode step then has no kernel argument that depends on host state, so it can be
        captured once in a HIP graph and replayed (DecodeGraph).  The host copies of the
        lengths and positions keep following the same rules."""
        if on and self.tail_budget < 1:
            raise HeteroKVError(-4, "device-stepped decode needs a recent window of at least one token")
        self.device_decode = bool(on)
        for st in self._layers:
            if st is not None:
                st.dev_state = None

    def _sync_device_state(self, st) -> None:
        dev = self.device
        st.dev_state = torch.tensor([st.tail_head, st.tail_len, st.hh_len, 0], dtype=torch.int32, device=dev)
        st.dev_tail_lens = torch.full((st.B,), st.tail_len, dtype=torch.int32, device=dev)
        st.dev_hh_lens = torch.full((st.B,), st.hh_len, dtype=torch.int32, device=dev)

    def advance_decode_host(self, layer_idx: int, seq_offset: int) -> None:
        """The host half of one decode step of a layer, without kernels: what a replayed
        decode graph did on the GPU."""
        st = self._layers[layer_idx]
        if st is None:
            raise RuntimeError("Layer %d has not been allocated yet." % layer_idx)
        self._decode_host(st, seq_offset, None, None, launch=False)

    def _evict(self, layer, st, k, v, first_pos):
        """manager.py:1231-1299: quantize + pack into the layer's INT4 blocks, record the chunk."""
        n = k.shape[2]
        st.ensure_int4(st.int4_len + n)
        ops.pack_tokens(st.pool, k, v, st.int4_len, st.bt, err=st.err)   # one start, by value
        key = "l%d_e%d" % (layer, self._eviction_counter)
        self._chunks[key] = (layer, st.int4_len, n)
        self._layer_keys.setdefault(layer, []).append(key)
        self._forget_ranking(layer)
        if isinstance(first_pos, int):
            st.int4_pos.extend(range(first_pos, first_pos + n))
        else:
            st.int4_pos.extend(first_pos)
        st.int4_len += n
        self._chunk_eviction_order.append(key)
        scores = self._oracle.token_scores
        if scores is not None:
            # manager.py:1262-1268: the mean oracle score of tokens [counter * n, +n)
            part = scores[self._eviction_counter * n:(self._eviction_counter + 1) * n]
            self._chunk_attention_scores[key] = float(part.mean().item()) if part.numel() > 0 else 0.0
        else:
            self._chunk_attention_scores[key] = 1.0 / (self._eviction_counter + 1)
        if layer == 0:
            self._eviction_counter += 1

    def compress(self, layer: int, device: str = "DRAM") -> int:
        """manager.py:206-233: move every HBM token after the sink to the INT4 tier."""
        if device.upper() != "DRAM":
            raise NotImplementedError("Only DRAM compression is currently supported.")
        st = self._layers[layer] if layer < len(self._layers) else None
        if st is None:
            return 0
        kk, vv = self.get_hbm_kv(layer)
        total = kk.shape[2]
        if total <= self.sink_tokens:
            return 0
        pos = self.positions(layer, include_dram=False)
        ks, vs = kk[:, :, self.sink_tokens:], vv[:, :, self.sink_tokens:]
        self._evict(layer, st, ks, vs, pos[self.sink_tokens:])
        # the reference keeps only the sink as its concatenated cache; all zones after it empty
        st.tail_head, st.tail_len, st.tail_pos = 0, 0, deque()
        st.hh_len, st.hh_pos = 0, []
        st.dev_state = None
        if st.sink_len > self.sink_tokens:
            st.sink_len = self.sink_tokens
        return total - self.sink_tokens

    def get_hbm_kv(self, layer_idx: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """manager.py:294-299: sink + tail + heavy hitters (fp16 [B, H, S, 128])."""
        st = self._layers[layer_idx] if layer_idx < len(self._layers) else None
        if st is None:
            raise RuntimeError("Layer %d has not been allocated yet." % layer_idx)
        parts_k, parts_v = [], []
        if st.sink_len:
            a, b = st.sink.read(st.sink_len)
            parts_k.append(a)
            parts_v.append(b)
        tk, tv = st.tail_tensors()
        parts_k.append(tk)
        parts_v.append(tv)
        if st.hh_len:
            a, b = st.hh.read(st.hh_len)
            parts_k.append(a)
            parts_v.append(b)
        return torch.cat(parts_k, dim=2), torch.cat(parts_v, dim=2)

    def get_seq_offset(self, layer_idx: int) -> int:
        st = self._layers[layer_idx] if layer_idx < len(self._layers) else None
        return st.seq_offset if st is not None else 0

    def hbm_length(self, layer_idx: int) -> Optional[int]:
        """Length of the reference's concatenated HBM cache for this layer (None before use)."""
        st = self._layers[layer_idx] if layer_idx < len(self._layers) else None
        if st is None:
            return None
        return st.sink_len + st.tail_len + st.hh_len

    def tail_length(self, layer_idx: int) -> Optional[int]:
        st = self._layers[layer_idx] if layer_idx < len(self._layers) else None
        return None if st is None or not st.tail_started else st.tail_len

    def positions(self, layer_idx: int, include_dram: bool = False) -> List[int]:
        """Absolute positions of the tokens the reference returns for this layer, in its
        order: [DRAM chunks in eviction order] + sink + tail (oldest first) + heavy hitters."""
        st = self._layers[layer_idx]
        pre = list(st.int4_pos) if include_dram else []
        return pre + list(st.sink_pos) + list(st.tail_pos) + list(st.hh_pos)

    # ---------------------------------------------------------------- DRAM tier views
    @property
    def _dram_table(self) -> "DramTableView":
        return DramTableView(self)

    def count_dram_tokens(self, layer_idx: int = 0) -> int:
        """manager.py:1218-1229: #chunks of the layer times the first chunk's token count."""
        keys = self._layer_keys.get(layer_idx)
        if not keys:
            return 0
        return len(keys) * self._chunks[keys[0]][2]

    def dram_tokens(self, layer_idx: int) -> int:
        """Exact number of INT4 tokens held for the layer."""
        st = self._layers[layer_idx] if layer_idx < len(self._layers) else None
        return 0 if st is None else st.int4_len

    def chunk_codes(self, key: str) -> Dict[str, torch.Tensor]:
        """Reference-layout view of one evicted chunk (kv_compressor.compress of [B,H,T,128]):
        k_data/v_data uint8 [B,H,T,128], *_scales float32 [B*H*T], *_zps uint8 [B*H*T]."""
        layer, start, n = self._chunks[key]
        st = self._layers[layer]
        pool, bt = self._resident_view(st)
        out = {}
        for which, name in ((0, "k"), (1, "v")):
            cs, ss, zs = [], [], []
            for b in range(st.B):
                c, s, z = ops.unpack_tokens(pool, bt[b], start + n, which)
                cs.append(c[:, start:start + n])
                ss.append(s.view(st.H, -1)[:, start:start + n].reshape(-1))
                zs.append(z.view(st.H, -1)[:, start:start + n].reshape(-1))
            out[name + "_data"] = torch.stack(cs)
            out[name + "_scales"] = torch.cat(ss)
            out[name + "_zps"] = torch.cat(zs)
        return out

    def decompress_dram_chunks(self, layer_idx: int):
        """manager.py:779-821 (Path C): every INT4 token of the layer dequantized to fp16,
        in eviction order.  Returns (K, V, count) or (None, None, 0)."""
        st = self._layers[layer_idx] if layer_idx < len(self._layers) else None
        if st is None or st.int4_len == 0:
            return None, None, 0
        pool, bt = self._resident_view(st)
        outs = []
        for which in (0, 1):
            per_b = []
            for b in range(st.B):
                c, s, z = ops.unpack_tokens(pool, bt[b], st.int4_len, which)
                per_b.append(self._compressor.decompress(c, s, z, target_dtype=torch.float16))
            outs.append(torch.stack(per_b))
        return outs[0], outs[1], st.int4_len

    def _adaptive_selection(self, layer_idx: int, window_size: Optional[int]) -> List[str]:
        """The chunk keys manager.py:857-878 / :966-978 select: w = window_size, or the
        controller's w_t (one compute_window call) clamped to [1, #chunks] when None; the
        top w by chunk score (stable descending sort), returned in eviction order."""
        keys = self._layer_chunks(layer_idx)
        if not keys:
            return []
        if window_size is None:
            w_t = int(self._adaptive_controller.compute_window(attention_weights=self._last_attention_weights,
                                                               cache_miss=False))
            window_size = max(1, min(w_t, len(keys)))
        return list(self._top_chunks(layer_idx, keys, int(window_size)))

    def get_dram_chunks_quantized_adaptive(self, layer_idx: int, window_size: Optional[int] = None
                                           ) -> Optional[Dict[str, torch.Tensor]]:
        """manager.py:931-1056 (Path A gather): the INT4 tokens of the top-w chunks, not
        dequantized, as the six reference-layout tensors: k_data/v_data uint8 [B, H, T, 128]
        concatenated along the token axis in eviction order, the 1-D scales and zero points
        concatenated chunk after chunk.  window_size None: w_t from the adaptive controller.
        (The reference indexes its ranked list by eviction-list positions when it
        concatenates, :1012-1017, which only returns the selected chunks when they are the
        first ones in eviction order -- always the case under its default 1/(c+1) chunk
        scores; this returns the selected chunks in eviction order for any scores.)"""
        keys = self._adaptive_selection(layer_idx, window_size)
        if not keys:
            return None
        parts = [self.chunk_codes(k) for k in keys]
        return {name: torch.cat([p[name] for p in parts], dim=2 if name.endswith("_data") else 0)
                for name in parts[0]}

    def decompress_dram_chunks_adaptive(self, layer_idx: int, window_size: Optional[int] = None):
        """manager.py:823-929 (Path B): the top-w chunks dequantized to bf16
        (KVCompressor.decompress(..., target_dtype=bf16)), concatenated in eviction order.
        Returns (K, V, count) or (None, None, 0)."""
        return self._decompress_keys(self._adaptive_selection(layer_idx, window_size))

    def _decompress_keys(self, keys):
        if not keys:
            return None, None, 0
        ks, vs = [], []
        for key in keys:
            e = self.chunk_codes(key)
            ks.append(self._compressor.decompress(e["k_data"], e["k_scales"], e["k_zps"], target_dtype=torch.bfloat16))
            vs.append(self._compressor.decompress(e["v_data"], e["v_scales"], e["v_zps"], target_dtype=torch.bfloat16))
        K = ks[0] if len(ks) == 1 else torch.cat(ks, dim=-2)
        V = vs[0] if len(vs) == 1 else torch.cat(vs, dim=-2)
        return K, V, K.shape[-2]

    def _path_b_keys(self, layer_idx: int) -> List[str]:
        """The chunks Path B attends at this decode step, chosen once per layer and step
        (one compute_window call, as decompress_dram_chunks_adaptive makes), so that
        get_mask_sizes and update agree."""
        keys = self._selection_b.get(layer_idx)
        if keys is None:
            keys = self._selection_b[layer_idx] = self._adaptive_selection(layer_idx, None)
        return keys

    def selected_tokens(self, layer_idx: int) -> int:
        """INT4 tokens of the chunks Path B attends at this step."""
        return sum(self._chunks[k][2] for k in self._path_b_keys(layer_idx))

    def decompress_selected(self, layer_idx: int):
        """Path B for this step: the chosen chunks as bf16 (K, V, count)."""
        keys = self._path_b_keys(layer_idx)
        self._selection_b.pop(layer_idx, None)
        return self._decompress_keys(keys)

    @property
    def heavy_hitter_budget(self) -> int:
        return self._heavyhitter_budget

    def heavy_hitter_length(self, layer_idx: int) -> int:
        st = self._layers[layer_idx] if layer_idx < len(self._layers) else None
        return 0 if st is None else st.hh_len

    # ---------------------------------------------------------------- per-chunk swap-in
    def swap_in_quantized(self, layer_idx: int, chunk_key: str) -> Optional[Dict[str, torch.Tensor]]:
        """manager.py:233-263: one chunk's INT4 data on the device without dequantizing
        (k_data, k_scales, k_zps, v_data, v_scales, v_zps), or None; the chunk stays."""
        if chunk_key not in self._chunks:
            return None
        return self.chunk_codes(chunk_key)

    def schedule_prefetch(self, chunk_key: str) -> None:
        """manager.py:335-350: dequantize the chunk to bf16 on the prefetcher's side stream
        (AsyncPrefetcher) so that a later swap_in finds it ready.  The prefetcher holds at
        most AsyncPrefetcher._SLOTS chunks not yet fetched; a key scheduled while it is full
        is skipped (its swap_in dequantizes it then), where the reference's buffer grows
        without bound."""
        if not self.enable_prefetch or chunk_key not in self._chunks:
            return
        if self._async_pf is None:
            self._async_pf = AsyncPrefetcher(self.device)
        # a chunk already dequantized is skipped by the prefetcher: skip it before its
        # codes are gathered (that gather is a kernel launch and a host round trip)
        if chunk_key in self._async_pf.buffer or self._async_pf.free_slots == 0:
            return
        self._async_pf.submit_prefetch_task(chunk_key, self.chunk_codes(chunk_key), self._compressor)

    def swap_in(self, layer_idx: int, chunk_key: str) -> Optional[Tuple[torch.Tensor, torch.Tensor]]:
        """manager.py:265-292: remove the chunk from the INT4 tier and return its K, V as
        bf16 [B, H, T, 128] (decompress to fp16, then .to(bf16), as the reference), from a
        finished schedule_prefetch when there is one.  Later Path C gathers no longer see
        the chunk.  None if the key is unknown."""
        if chunk_key not in self._chunks:
            return None
        got = self._async_pf.fetch_if_ready(chunk_key) if self._async_pf is not None else None
        if got is None:
            e = self.chunk_codes(chunk_key)
            k = self._compressor.decompress(e["k_data"], e["k_scales"], e["k_zps"]).to(torch.bfloat16)
            v = self._compressor.decompress(e["v_data"], e["v_scales"], e["v_zps"]).to(torch.bfloat16)
        else:
            k, v = got
        self._remove_chunk(chunk_key)
        return k, v

    def _remove_chunk(self, key: str) -> None:
        """Drop one chunk from its layer's INT4 tier.  A chunk that starts on a block
        boundary and ends on one (or at the layer's end) leaves by a block-table edit;
        otherwise the later tokens move down by unpack + repack (per-token groups, so the
        codes are unchanged)."""
        layer, start, n = self._chunks.pop(key)
        self._layer_keys[layer].remove(key)
        self._forget_ranking(layer)
        # as the reference's _dram.remove: the chunk's eviction-order entry and score stay
        st = self._layers[layer]
        for k2, (l2, s2, n2) in list(self._chunks.items()):
            if l2 == layer and s2 > start:
                self._chunks[k2] = (l2, s2 - n, n2)
        del st.int4_pos[start:start + n]
        end = start + n
        if start % BLOCK_TOKENS == 0 and (n % BLOCK_TOKENS == 0 or end == st.int4_len):
            lb0, lb1 = start // BLOCK_TOKENS, (end + BLOCK_TOKENS - 1) // BLOCK_TOKENS
            d = lb1 - lb0
            st.bt_host[:, lb0:st.nb - d] = st.bt_host[:, lb1:st.nb].copy()
            st.nb -= d
            if st.host_lbs is not None:
                hl = st.host_lbs
                st.host_lbs = np.where(hl >= lb1, hl - d, np.where(hl >= lb0, lb0, hl))
        else:
            if st.n_host:
                raise HeteroKVError(-4, "swap_in: chunk %s is not block aligned (%d+%d) and its layer has "
                                        "records in host memory" % (key, start, n))
            rest = st.int4_len - end
            if rest:
                pieces = {}
                for which, name in ((0, "k"), (1, "v")):
                    cs, ss, zs = [], [], []
                    for b in range(st.B):
                        c, sc, z = ops.unpack_tokens(st.pool, st.bt[b], st.int4_len, which)
                        cs.append(c[:, end:])
                        ss.append(sc.view(st.H, -1)[:, end:])
                        zs.append(z.view(st.H, -1)[:, end:])
                    pieces[name] = (torch.stack(cs), torch.stack(ss), torch.stack(zs))
                ops.repack_codes(st.pool, pieces["k"][0], pieces["v"][0], pieces["k"][1], pieces["v"][1],
                                 pieces["k"][2], pieces["v"][2], torch.full((st.B,), start, dtype=torch.int32),
                                 st.bt, err=st.err)
            st.nb = (st.int4_len - n + BLOCK_TOKENS - 1) // BLOCK_TOKENS
        st.int4_len -= n
        st.bt = ops.h2d(torch.from_numpy(np.ascontiguousarray(st.bt_host)), self.device)
        st.version += 1
        st.resident_cache = None
        self._window_tables = {k2: v for k2, v in self._window_tables.items() if k2[0] != layer}

    # ---------------------------------------------------------------- host tier
    def offload_to_host(self, fraction: float, seed: int = 0, layers: Optional[List[int]] = None) -> int:
        """Move a seeded random `fraction` of each layer's INT4 block records to a pinned host
        arena (the reference's DRAM tier, dram_storage.py:106-138, as one contiguous run per
        layer).  Only full blocks move, so later appends always land in HBM.  The records
        chosen for layer l are those of numpy.random.default_rng([seed, l]).choice over the
        layer's full blocks.  Returns the number of records moved.  One call per manager."""
        if self._pf is not None:
            raise HeteroKVError(-1, "offload_to_host: the host tier is already set up")
        if not 0.0 <= fraction <= 1.0:
            raise ValueError("fraction must be in [0, 1]")
        if layers is None:
            layers = [i for i, st in enumerate(self._layers) if st is not None]
        plan = []
        for li in layers:
            st = self._layers[li]
            if st is None or st.int4_len == 0:
                continue
            full = st.int4_len // BLOCK_TOKENS
            total = st.B * st.nb
            n_host = min(int(round(fraction * total)), st.B * full)
            if n_host == 0:
                continue
            rng = np.random.default_rng([seed, li])
            chosen = np.sort(rng.choice(st.B * full, size=n_host, replace=False))   # c = lb * B + b
            plan.append((li, st, chosen))
        if not plan:
            return 0
        rb = ops.record_bytes(plan[0][1].H)
        arena = sum(len(c) * ops.record_bytes(st.H) for _, st, c in plan)
        self._pf = Prefetcher(self.device, arena, num_slots=2 * max(len(self._layers), 1))
        off = 0
        moved = 0
        for li, st, chosen in plan:
            rb = ops.record_bytes(st.H)
            lb, b = chosen // st.B, chosen % st.B
            is_host = np.zeros((st.B, st.nb), dtype=bool)
            is_host[b, lb] = True
            tmp = ops.Int4Pool(len(chosen), st.H, self.device)
            ops.gather_blocks(st.pool, st.bt_host[b, lb], tmp)
            self._pf.stage_out(tmp.data[:len(chosen)], off)
            rb_idx, rl_idx = np.nonzero(~is_host)                                  # resident, row-major
            res_ids = st.bt_host[rb_idx, rl_idx]
            pool = ops.Int4Pool(max(len(res_ids), st.B * 64), st.H, self.device)
            ops.gather_blocks(st.pool, res_ids, pool)
            bh = st.bt_host.copy()
            bh[rb_idx, rl_idx] = np.arange(len(res_ids), dtype=np.int32)
            bh[b, lb] = ~np.arange(len(chosen), dtype=np.int32)
            torch.cuda.current_stream(self.device).synchronize()
            for pl in (tmp, pool):
                pl.check_errors()
            st.pool, st.pool_used, st.bt_host = pool, len(res_ids), bh
            st.bt = ops.h2d(torch.from_numpy(bh), self.device)
            st.n_host, st.host_off, st.host_lbs = len(chosen), off, lb.astype(np.int64)
            st.version += 1
            st.resident_cache = None
            off += len(chosen) * rb
            moved += len(chosen)
        biggest = max(st.n_host for _, st, _ in plan)
        self._staging = [ops.Int4Pool(biggest, plan[0][1].H, self.device) for _ in range(2)]
        self._buf_owner = [-1, -1]
        return moved

    def host_blocks(self, layer_idx: int) -> int:
        st = self._layers[layer_idx] if layer_idx < len(self._layers) else None
        return 0 if st is None else st.n_host

    def _resident_view(self, st: _LayerState):
        """(pool, block table) holding every INT4 record of the layer in HBM: the layer's
        own when nothing is on the host, else a gathered copy (for inspection paths)."""
        if st.n_host == 0:
            return st.pool, st.bt
        if st.resident_cache is not None and st.resident_cache[0] == st.version:
            return st.resident_cache[1], st.resident_cache[2]
        rb = ops.record_bytes(st.H)
        stage = ops.Int4Pool(st.n_host, st.H, self.device)
        stage.data.view(-1)[:st.n_host * rb].copy_(self._pf.host_tensor(st.host_off, st.n_host * rb))
        full = ops.Int4Pool(st.B * st.nb, st.H, self.device)
        ops.gather_blocks(st.pool, st.bt_host[:, :st.nb].reshape(-1), full, staging=stage)
        full.check_errors()
        bt = torch.arange(st.B * st.nb, dtype=torch.int32, device=self.device).view(st.B, st.nb)
        st.resident_cache = (st.version, full, bt)
        return full, bt

    def _layer_chunks(self, layer_idx: int) -> List[str]:
        return list(self._layer_keys.get(layer_idx, ()))

    def _forget_ranking(self, layer_idx: int) -> None:
        self._ranked.pop(layer_idx, None)
        self._sel_cache = {k: v for k, v in self._sel_cache.items() if k[0] != layer_idx}

    def _top_chunks(self, layer_idx: int, keys: List[str], w: int) -> Tuple[str, ...]:
        """The top w of the layer's chunks by score (stable descending sort), in eviction
        order."""
        # scores replaced by a plain dict count no writes: nothing is cached then
        epoch = getattr(self._chunk_attention_scores, "epoch", None)
        hit = self._sel_cache.get((layer_idx, w)) if epoch is not None else None
        if hit is not None and hit[0] == epoch:
            return hit[1]
        ranked = self._ranked.get(layer_idx) if epoch is not None else None
        if ranked is None or ranked[0] != epoch:
            ranked = (epoch, sorted(keys, key=lambda k: self._chunk_attention_scores.get(k, 0.0), reverse=True))
            self._ranked[layer_idx] = ranked
        chosen = set(ranked[1][:max(0, w)])
        sel = tuple(k for k in keys if k in chosen)   # the layer's keys are in eviction order
        self._sel_cache[(layer_idx, w)] = (epoch, sel)
        return sel

    def _selection(self, layer_idx: int):
        """Chunk keys attended at this decode step (None = all), computed once per layer
        and step: the window size comes from retrieval_window or, for "adaptive", from the
        controller (called once per layer, as manager.py:965-968 does)."""
        if layer_idx in self._selection_of:
            return self._selection_of[layer_idx]
        sel = None
        if self.retrieval_window is not None:
            keys = self._layer_chunks(layer_idx)
            if keys:
                if self.retrieval_window == "adaptive":
                    w = int(self._adaptive_controller.compute_window(
                        attention_weights=self._last_attention_weights, cache_miss=False))
                else:
                    w = int(self.retrieval_window)
                w = max(1, min(w, len(keys)))
                sel = self._top_chunks(layer_idx, keys, w)
        self._selection_of[layer_idx] = sel
        return sel

    def _window_table(self, layer_idx: int, st: _LayerState, sel):
        """Block table over the selected chunks' blocks, in eviction order, and their token
        count.  Chunks must start on a block boundary and, except the layer's last, end on one."""
        key = (layer_idx, sel, st.version)
        hit = self._window_tables.get(key)
        if hit is not None:
            return hit
        lbs, n4 = [], 0
        for k in sel:
            _, start, n = self._chunks[k]
            if start % BLOCK_TOKENS or (n % BLOCK_TOKENS and start + n != st.int4_len):
                raise HeteroKVError(-4, "windowed retrieval needs 16-token aligned chunks (%s: %d+%d)" %
                                    (k, start, n))
            if lbs and n4 % BLOCK_TOKENS:
                raise HeteroKVError(-4, "windowed retrieval: only the last selected chunk may be partial")
            lbs.extend(range(start // BLOCK_TOKENS, (start + n + BLOCK_TOKENS - 1) // BLOCK_TOKENS))
            n4 += n
        bt = ops.h2d(torch.from_numpy(np.ascontiguousarray(st.bt_host[:, lbs])), self.device)
        self._window_tables = {k2: v for k2, v in self._window_tables.items() if k2[0] != layer_idx}
        self._window_tables[key] = (bt, n4)
        return bt, n4

    def _host_runs(self, st: _LayerState, sel) -> List[Tuple[int, int]]:
        """Ranges [k0, k1) of the layer's host records needed for selection `sel`."""
        if sel is None:
            return [(0, st.n_host)]
        c = st.runs_cache
        if c is not None and c[0] == st.version and c[1] == sel:
            return c[2]
        runs = []
        for k in sel:
            _, start, n = self._chunks[k]
            lb0, lb1 = start // BLOCK_TOKENS, (start + n + BLOCK_TOKENS - 1) // BLOCK_TOKENS
            k0 = int(np.searchsorted(st.host_lbs, lb0, "left"))
            k1 = int(np.searchsorted(st.host_lbs, lb1, "left"))
            if k1 > k0:
                if runs and runs[-1][1] == k0:
                    runs[-1] = (runs[-1][0], k1)
                else:
                    runs.append((k0, k1))
        st.runs_cache = (st.version, sel, runs)
        return runs

    def _submit(self, layer_idx: int, sel, avoid_buf: Optional[int] = None) -> Tuple[int, Any, int]:
        """Copy the layer's host runs into the next staging buffer (never `avoid_buf`, the one
        the layer being attended reads: its "free" mark is only recorded after its kernel, so
        a copy into it would race that kernel)."""
        st = self._layers[layer_idx]
        buf = self._next_buf
        if buf == avoid_buf:
            buf = (buf + 1) % len(self._staging)
        self._next_buf = (buf + 1) % len(self._staging)
        prev_slot = self._buf_owner[buf]
        prev = prev_slot // 2 if prev_slot >= 0 else -1
        if prev >= 0 and self._pending.get(prev, (None,))[0] == buf:
            del self._pending[prev]        # its copy is overwritten before use: fetch again later
        parity = self._slot_parity.get(layer_idx, 0)
        self._slot_parity[layer_idx] = parity ^ 1
        slot = 2 * layer_idx + parity
        rb = ops.record_bytes(st.H)
        dst = self._staging[buf].data
        copies = [(dst[k0].data_ptr(), self._pf.host_ptr(st.host_off + k0 * rb), (k1 - k0) * rb)
                  for k0, k1 in self._host_runs(st, sel)]
        self._pf.submit(copies, slot=slot, after_slot=prev_slot)
        self._buf_owner[buf] = slot
        self._pending[layer_idx] = (buf, sel, slot)
        return self._pending[layer_idx]

    def _prefetch_after(self, layer_idx: int, avoid_buf: Optional[int] = None) -> None:
        """Submit the copies of the next layer (cyclically) that holds host records."""
        L = len(self._layers)
        for d in range(1, L):
            j = (layer_idx + d) % L
            st = self._layers[j]
            if st is None or st.n_host == 0:
                continue
            sel = self._selection(j)
            p = self._pending.get(j)
            if p is None or p[1] != sel:
                self._submit(j, sel, avoid_buf)
            return

    # ------------------------------------------------- host tier under graph capture
    def begin_graph_staging(self) -> None:
        """Make the host-tier copies of the next captured decode step part of the graph.

        The native prefetcher's side stream and events cannot join a capture, so while
        this is on, attend_decode under capture gathers each staged layer's host runs from
        the pinned arena (hipHostMalloc memory is device-accessible) into staging buffer 0
        with the block-gather kernel, on the capturing stream right before the layer's
        decode kernel.  Stream order keeps the next layer's gather behind this layer's
        kernel.  A forked stream gains nothing here: the replayed graph ran its branches one
        after the other, and its host-side launch took 3.3 ms instead of well under one.
        Captured host-to-device memcpy nodes were slower than the kernel.  The eager
        schedule's pending copies are dropped first (the graph rewrites its buffer)."""
        if self._pf is not None:
            self._pf.synchronize()
        torch.cuda.current_stream(self.device).synchronize()
        self._pending.clear()
        self._buf_owner = [-1] * len(self._staging)
        n = max([st.n_host for st in self._layers if st is not None] + [1])
        if self._graph_ids is None or self._graph_ids.numel() < n:
            self._graph_ids = torch.arange(n, dtype=torch.int32, device=self.device)
        self._graph_staging = True

    def end_graph_staging(self) -> None:
        """Back to the native prefetch schedule (after every replay has finished)."""
        torch.cuda.synchronize(self.device)
        self._graph_staging = False

    def _graph_stage(self, layer_idx: int, sel) -> int:
        """Under capture: gather layer_idx's host runs into staging buffer 0 on the current
        stream; returns the buffer."""
        st = self._layers[layer_idx]
        rb = ops.record_bytes(st.H)
        dst = self._staging[0]
        sp = _lib.stream_ptr(self.device)
        for k0, k1 in self._host_runs(st, sel):
            _lib.check(_lib.load().hkv_gather_blocks(self._pf.host_ptr(st.host_off + k0 * rb), k1 - k0, None, 0,
                                                     self._graph_ids.data_ptr(), k1 - k0, rb,
                                                     dst.data[k0].data_ptr(), dst.err.data_ptr(), sp),
                       "hkv_gather_blocks")
        return 0

    def prefetch_stats(self, reset: bool = True) -> Dict[str, Any]:
        """Stall of every layer that waited for host records since the last call: per layer
        max(0, t(copies done) - t(kernel needs them)) in ms (synchronizes on those events,
        and raises if a kernel reported a device error meanwhile)."""
        self.check_errors()
        per = [(slot // 2, self._pf.stall_ms(slot)) for slot in self._waited] if self._pf is not None else []
        if reset:
            self._waited = []
        out = {"stall_ms": sum(ms for _, ms in per), "per_layer": per}
        if self._pf is not None:
            out.update(self._pf.stats())
        return out

    # ---------------------------------------------------------------- fused decode
    def attend_decode(self, layer_idx: int, query_states: torch.Tensor, sm_scale: Optional[float] = None,
                      include_dram: bool = True, feed_oracle: bool = False) -> torch.Tensor:
        """softmax(q K^T * sm_scale) V over [INT4 middle (if include_dram) | sink | tail |
        heavy hitters] of the layer, in one split-K launch (hkv_decode_attn).  With a host
        tier, the layer's host records are copied into a staging buffer on the prefetcher's
        side stream (normally already submitted while the previous layer ran) and the next
        host-tier layer's copies are submitted before this layer's kernel.
        query_states: [B, Hq, 1, 128]; returns [B, Hq, 1, 128] in the query's dtype."""
        st = self._layers[layer_idx]
        if st is None:
            raise RuntimeError("Layer %d has not been allocated yet." % layer_idx)
        st.flush()
        if self._workspace is None:
            self._workspace = ops.DecodeWorkspace(self.device)
        err = self._errword()
        capturing = torch.cuda.is_current_stream_capturing()
        if layer_idx == 0 and not capturing:
            err.poll()           # a step's errors surface at the next step's first layer
        if feed_oracle and self.device_decode:
            raise HeteroKVError(-1, "attend_decode: feed_oracle needs host-stepped decode")
        zones = []
        if st.sink_len:
            zones.append((st.sink, None, st.sink_len))
        if self.device_decode:
            # lengths from the device counters, bounds by value: the same launch serves
            # every step
            if st.dev_state is None:
                self._sync_device_state(st)
            zones.append((st.tail, st.dev_tail_lens, st.ring))
            if self._heavyhitter_budget > 0:
                zones.append((st.hh, st.dev_hh_lens, self._heavyhitter_budget))
        else:
            if st.tail_len:
                zones.append((st.tail, None, st.tail_len))
            if st.hh_len:
                zones.append((st.hh, None, st.hh_len))
        n4 = st.int4_len if include_dram else 0
        bt = st.bt
        sel = None
        if n4:
            sel = self._selection(layer_idx)
            if sel is not None:
                bt, n4 = self._window_table(layer_idx, st, sel)
        staged = n4 > 0 and st.n_host > 0 and bool(self._host_runs(st, sel))
        buf = slot = None
        graph_staged = capturing and self._graph_staging
        if graph_staged:
            if staged:
                buf = self._graph_stage(layer_idx, sel)
        elif staged:
            p = self._pending.get(layer_idx)
            if p is None or p[1] != sel:
                p = self._submit(layer_idx, sel)
            buf, _, slot = p
        if self._pf is not None and self.enable_prefetch and not graph_staged:
            self._prefetch_after(layer_idx, buf)
        if staged and not graph_staged:
            self._pf.wait(slot)
        q = query_states
        scores = stats = None
        if feed_oracle:
            n_items = n4 + sum(z[2] for z in zones)
            scores = torch.full((q.shape[0], q.shape[1], max(n_items, 1)), float("-inf"),
                                dtype=torch.float32, device=q.device)
            stats = torch.empty((q.shape[0], q.shape[1], 2), dtype=torch.float32, device=q.device)
        out = ops.decode_attention(q, zones=zones, pool=st.pool if n4 else None,
                                   block_table=bt if n4 else None, int4_max_len=n4,
                                   sm_scale=sm_scale, workspace=self._workspace,
                                   staging=self._staging[buf] if staged else None,
                                   deterministic=self.deterministic_decode, scores=scores, score_stats=stats,
                                   err=err, out_dtype=q.dtype)
        if feed_oracle:
            w = ops.attn_weights(scores[:1], stats[:1], order=self._score_order(st, n4))
            self.update_attention_scores(w[0])
        if staged and not graph_staged:
            self._pf.mark(slot)
            self._pending.pop(layer_idx, None)
            self._waited.append(slot)
        self._selection_of.pop(layer_idx, None)
        if layer_idx >= self._top_layer and not capturing:
            self._top_layer = layer_idx
            err.post()           # the step's last layer: its error word heads back to the host
        return out

    # ---------------------------------------------------------------- fused prefill
    def attend_prefill(self, layer_idx: int, query_states: torch.Tensor, key_states: torch.Tensor,
                       value_states: torch.Tensor, sm_scale: Optional[float] = None) -> torch.Tensor:
        """Attention of a prefill chunk exactly as the reference hands it to SDPA
        (manager.py:533-535,562-563), on the MFMA prefill kernel: every query sees the sink
        and the tail as they were before this chunk, and the chunk causally.  The chunk's
        K/V are those just given to update(..., materialize=False); its deferred tail write
        happens right after.  query [B, Hq, S, 128]; returns [B, Hq, S, 128] in its dtype."""
        st = self._layers[layer_idx]
        if st is None:
            raise RuntimeError("Layer %d has not been allocated yet." % layer_idx)
        zones = []
        if st.pending is not None:
            old_len = st.pending[4]
            if st.sink_len:
                zones.append((st.sink, None, st.sink_len))
            if old_len:
                zones.append((st.tail, None, old_len))
        out = ops.prefill_attention(query_states, zones=zones, chunk_k=key_states, chunk_v=value_states,
                                    sm_scale=sm_scale, err=self._errword(), out_dtype=query_states.dtype)
        st.flush()
        return out

    # ---------------------------------------------------------------- heavy-hitter scores
    def update_attention_scores(self, attention_weights: torch.Tensor) -> None:
        """manager.py:319-329: feed the newest token's attention weights to the oracle and
        keep them for the adaptive window controller."""
        self._oracle.update(attention_weights)
        self._last_attention_weights = attention_weights.detach().clone()

    def get_oracle_scores(self) -> Optional[torch.Tensor]:
        """manager.py:331-333: the oracle's cumulative per-token scores."""
        return self._oracle.token_scores

    def _score_order(self, st: "_LayerState", n4: int) -> torch.Tensor:
        """Decode score items in the order the reference concatenates the attended tokens:
        the INT4 tokens (eviction order), the sink, the recent window oldest first, the
        heavy hitters.  Items are indexed as attend_decode lays them out: INT4 tokens,
        then the sink, tail-ring and heavy-hitter slots."""
        dev = self.device   # built on the device: no host-to-device copy per step
        parts = [torch.arange(n4, dtype=torch.int64, device=dev)]
        base = n4
        if st.sink_len:
            parts.append(torch.arange(base, base + st.sink_len, dtype=torch.int64, device=dev))
            base += st.sink_len
        if st.tail_len:
            parts.append(base + (torch.arange(st.tail_head, st.tail_head + st.tail_len, dtype=torch.int64,
                                              device=dev) % st.ring))
            base += st.tail_len
        if st.hh_len:
            parts.append(torch.arange(base, base + st.hh_len, dtype=torch.int64, device=dev))
        return torch.cat(parts)

    # ---------------------------------------------------------------- summaries
    def memory_summary(self) -> Dict[str, Any]:
        """manager.py:387-401.  dram_bytes counts this library's packed INT4 storage (HBM and
        host records alike); host_bytes the part in the pinned host arena."""
        hbm = sum((st.sink_len + st.tail_len + st.hh_len) for st in self._layers if st is not None)
        dram_bytes = 0
        for st in self._layers:
            if st is not None:
                dram_bytes += st.B * st.H * st.int4_len * 2 * (HEAD_DIM // 2 + 5)
        host = sum(st.n_host * ops.record_bytes(st.H) for st in self._layers if st is not None)
        return {"hbm_tokens": hbm, "dram_entries": len(self._chunks), "dram_bytes": dram_bytes,
                "host_bytes": host, "max_hbm_tokens": self.max_hbm_tokens()}

    def max_hbm_tokens(self) -> int:
        return self.sink_tokens + self.hbm_budget_tokens + self._heavyhitter_budget


class DramTableView:
    """Read-only mapping chunk key -> reference-layout entry (k_data, k_scales, k_zps,
    v_data, v_scales, v_zps), materialized on access (dram_storage.py:140-147)."""

    def __init__(self, mgr: HeteroKVManager):
        self._m = mgr

    def keys(self):
        return list(self._m._chunks.keys())

    def __iter__(self):
        return iter(self.keys())

    def __len__(self):
        return len(self._m._chunks)

    def __contains__(self, key):
        return key in self._m._chunks

    def __getitem__(self, key):
        return self._m.chunk_codes(key)

    def items(self):
        return [(k, self[k]) for k in self.keys()]
