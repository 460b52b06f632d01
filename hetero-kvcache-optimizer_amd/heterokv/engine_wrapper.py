"""FusedHeteroCache: HuggingFace cache adapter over the GPU HeteroKVManager.

Drop-in for src/core/engine_wrapper.py:32-539 of the reference: same constructor
arguments, update / get_seq_length / get_mask_sizes / seen_tokens / dram_table /
memory_summary, ChunkedPrefillEngine and build_fused_cache.

Attention routes.
  * Prefill (new_len > 1): the reference hands transformers the full chunk (first
    chunk) or sink + old tail + chunk (later chunks) and lets SDPA attend
    (manager.py:533-535,562-563); the same tensors are returned here.  With
    fused_prefill=True update() returns the chunk itself, tagged, and the registered
    attention function runs the MFMA prefill kernel over the manager's own sink and
    tail zones (as they were before the chunk) plus the chunk causally -- the
    attention SDPA computes on the reference's tensors for an unpadded batch, with
    nothing concatenated or copied; the chunk enters the tail ring afterwards.
  * Decode, default (Path C, engine_wrapper.py:236-245): the reference prepends every
    DRAM token, dequantized to fp16, to sink + tail + heavy hitters.  With
    fused_decode=True (default) update() returns the new token's K/V tagged with a
    route, and the attention function registered as "heterokv" computes the same
    attention directly over the INT4 pool and the fp16 zones (one split-K launch);
    nothing is dequantized or concatenated.  With fused_decode=False the reference's
    concatenated tensors are materialized and returned.
The Path C gate is the reference's: DRAM tokens join a layer's attention only
while _swap_in_tokens > 0, which layer 0 refreshes after its own update.
adaptive_self_healing=True selects the reference's Path A (engine_wrapper.py:204-222):
only the top-w_t chunks by score join, w_t from AdaptivePrefetchController, attended
in place by the fused kernel; with enable_triton=False (or fused_decode=False) it is
Path B (:223-234): the chosen chunks are dequantized to bf16 and concatenated.

Sequence lengths.  By default get_seq_length is the number of tokens the layer has
seen (what transformers derives cache_position and RoPE positions from, as its
sliding-window layers do), get_mask_sizes the exact key length update() returns,
and the DRAM-tier gate counts the exact INT4 tokens and is refreshed after prefill
too.  reference_lengths=True keeps the reference's arithmetic instead
(engine_wrapper.py:256-301, manager.py:1218-1229): the HBM length plus #chunks x
first chunk size, refreshed only by layer 0's decode updates -- 3,904 tokens short
at 128K with keep_tail=4160, and no DRAM tokens for layer 0's first decode step.
"""
import gc
import math
from typing import Any, Dict, Optional, Tuple

import torch
from transformers.cache_utils import DynamicCache

from ._lib import HeteroKVError
from .manager import HeteroKVManager

ATTN_IMPLEMENTATION = "heterokv"


class FusedHeteroCache(DynamicCache):
    """HF DynamicCache subclass backed by HeteroKVManager (engine_wrapper.py:32-110)."""

    def __init__(self, num_layers: Optional[int] = None, sink_tokens: int = 64, keep_tail: int = 8192,
                 chunk_size: int = 2048, device: str = "cuda:0", group_size: int = 128,
                 enable_quant: bool = True, enable_prefetch: bool = True, enable_triton: bool = True,
                 bandwidth_limiter=None, self_healing: bool = True, adaptive_self_healing: bool = False,
                 enable_method_d: bool = False, method_d_alpha: float = 1.0, fused_decode: bool = True,
                 fused_prefill: bool = False, track_attention: bool = False, reference_lengths: bool = False):
        super().__init__()
        self.sink_tokens = sink_tokens
        self.keep_tail = keep_tail
        self.chunk_size = chunk_size
        self.device = device
        self.enable_quant = enable_quant
        self.enable_triton = enable_triton
        self.enable_prefetch = enable_prefetch
        self.group_size = group_size
        self._bandwidth_limiter = bandwidth_limiter
        self.self_healing = self_healing
        self.adaptive_self_healing = adaptive_self_healing
        self.enable_method_d = enable_method_d
        self.method_d_alpha = method_d_alpha
        # Path B (adaptive retrieval without the fused kernel) concatenates bf16 K/V
        self.fused_decode = fused_decode and not (adaptive_self_healing and not enable_triton)
        self.fused_prefill = fused_prefill
        self.reference_lengths = reference_lengths
        # feed the heavy-hitter oracle with the last layer's decode attention weights
        # (engine_wrapper.py:165-180 intends this; the reference's patch never sets them)
        self.track_attention = track_attention
        self._num_layers = num_layers
        self._manager: Optional[HeteroKVManager] = None
        self.real_seq_len: int = 0
        self._swap_in_tokens: int = 0
        self._layer_seen: Dict[int, int] = {}    # tokens each layer has been given

    def _ensure_manager(self, layer_idx: int) -> HeteroKVManager:
        if self._manager is not None:
            return self._manager
        num_layers = self._num_layers if self._num_layers is not None else (layer_idx + 1)
        self._manager = HeteroKVManager(num_layers=num_layers, sink_tokens=self.sink_tokens,
                                        hbm_budget_tokens=self.keep_tail, device=self.device,
                                        enable_quant=self.enable_quant, enable_prefetch=self.enable_prefetch,
                                        group_size=self.group_size, bandwidth_limiter=self._bandwidth_limiter,
                                        enable_method_d=self.enable_method_d, method_d_alpha=self.method_d_alpha)
        if self.adaptive_self_healing and self.fused_decode:
            self._manager.retrieval_window = "adaptive"
        return self._manager

    # ------------------------------------------------------------------ DynamicCache interface
    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int,
               cache_kwargs: Optional[Dict[str, Any]] = None, *args, **kwargs) -> Tuple[torch.Tensor, torch.Tensor]:
        """engine_wrapper.py:137-254."""
        manager = self._ensure_manager(layer_idx)
        new_len = key_states.shape[-2]
        mode = "prefill" if new_len > 1 else "decode"
        include_dram = mode == "decode" and self.self_healing and self._swap_in_tokens > 0
        if mode == "decode" and self.fused_decode:
            manager.update(layer_idx, key_states, value_states, mode="decode", seq_offset=self.real_seq_len,
                           materialize=False)
            out_k, out_v = key_states, value_states
            route = (self, layer_idx, include_dram)
            out_k._hkv_route = route
            out_v._hkv_route = route
        elif mode == "prefill" and self.fused_prefill:
            # the chunk is attended by attend_prefill over the manager's own zones: nothing
            # is concatenated
            manager.update(layer_idx, key_states, value_states, mode="prefill", seq_offset=self.real_seq_len,
                           materialize=False)
            out_k, out_v = key_states, value_states
            tag = (self, layer_idx)
            out_k._hkv_prefill = tag
            out_v._hkv_prefill = tag
        else:
            out_k, out_v = manager.update(layer_idx, key_states, value_states, mode=mode,
                                          seq_offset=self.real_seq_len)
            if include_dram:
                if self.adaptive_self_healing:
                    # Path B (engine_wrapper.py:223-234): top-w_t chunks as bf16
                    dram_k, dram_v, count = manager.decompress_selected(layer_idx)
                else:
                    dram_k, dram_v, count = manager.decompress_dram_chunks(layer_idx)
                if dram_k is not None and count > 0:
                    out_k = torch.cat([dram_k.to(out_k.dtype), out_k], dim=-2)
                    out_v = torch.cat([dram_v.to(out_v.dtype), out_v], dim=-2)
        self._layer_seen[layer_idx] = self._layer_seen.get(layer_idx, 0) + new_len
        if layer_idx == 0:
            self.real_seq_len += new_len
            if self.self_healing and (mode == "decode" or not self.reference_lengths):
                self._refresh_swap_count()
        return out_k, out_v

    def get_seq_length(self, layer_idx: int = 0, *args, **kwargs) -> int:
        """Tokens the layer has seen (its next token's position).  With
        reference_lengths=True: engine_wrapper.py:256-264, the HBM length plus the DRAM
        swap-in count."""
        if self._manager is None:
            return 0
        n = self._manager.hbm_length(layer_idx)
        if n is None:
            return 0
        if not self.reference_lengths:
            return self._layer_seen.get(layer_idx, 0)
        return n + self._swap_in_tokens

    @property
    def seen_tokens(self) -> int:
        return self.real_seq_len

    def get_mask_sizes(self, query, layer_idx: int = 0, *args, **kwargs) -> Tuple[int, int]:
        """(key length update() will return, key offset) for a query of this length,
        computed before the update as transformers does (engine_wrapper.py:274-301 with
        exact counts; reference_lengths=True keeps its arithmetic).  The offset pairs with
        get_query_offset so that a prefill query sees the cached prefix and the chunk
        causally and a decode query sees every key.  `query` is the query length
        (transformers >= 5) or the cache_position tensor (4.57, as the reference was
        written for)."""
        query_len = int(query.shape[0]) if isinstance(query, torch.Tensor) else int(query)
        mgr = self._manager
        if mgr is None:
            return query_len, 0
        phys = mgr.hbm_length(layer_idx)
        if phys is None:
            return query_len, 0
        if self.reference_lengths:
            if query_len > 1:
                return phys + query_len, 0
            tail = mgr.tail_length(layer_idx)
            if tail is not None and tail >= mgr.tail_budget:
                return phys + self._swap_in_tokens, 0
            return phys + self._swap_in_tokens + 1, 0
        shift = self._dram_shift(layer_idx)
        if query_len > 1:
            # keys = [sink | old tail | chunk]; query i sits at key phys + i, which with
            # get_query_offset = phys + shift needs kv_offset = shift
            return phys + query_len, shift
        tail = mgr.tail_length(layer_idx)
        grows = tail is None or tail < mgr.tail_budget or mgr.heavy_hitter_length(layer_idx) < mgr.heavy_hitter_budget
        dram = 0
        if shift:
            dram = mgr.selected_tokens(layer_idx) if (self.adaptive_self_healing and not self.fused_decode) else shift
        return phys + (1 if grows else 0) + dram, 0

    def _dram_shift(self, layer_idx: int) -> int:
        """INT4 tokens of the layer while the DRAM tier is attended at decode (else 0)."""
        if not (self.self_healing and self._swap_in_tokens > 0) or self._manager is None:
            return 0
        return self._manager.dram_tokens(layer_idx)

    def get_query_offset(self, layer_idx: int = 0) -> int:
        """Offset of the first query among the keys update() returns, as transformers' mask
        builder reads it (it defaults to get_seq_length, which here counts seen tokens):
        the cached prefix plus the DRAM tokens a decode step would prepend -- every key is
        then visible to a decode query, and a prefill chunk's mask keeps its causal
        alignment through the matching kv_offset of get_mask_sizes."""
        if self.reference_lengths:
            return self.get_seq_length(layer_idx)
        if self._manager is None:
            return 0
        phys = self._manager.hbm_length(layer_idx)
        if phys is None:
            return 0
        return phys + self._dram_shift(layer_idx)

    def _refresh_swap_count(self) -> None:
        if self._manager is not None:
            self._swap_in_tokens = (self._manager.count_dram_tokens(layer_idx=0) if self.reference_lengths
                                    else self._manager.dram_tokens(0))

    @property
    def is_compileable(self) -> bool:
        return False

    # ------------------------------------------------------------------ tiered storage passthrough
    def allocate(self, layer_idx: int, seq_len: int = 0, budget_tokens: Optional[int] = None) -> bool:
        return self._ensure_manager(layer_idx).allocate(layer_idx, budget_tokens)

    def compress(self, layer_idx: int, device: str = "DRAM") -> int:
        return self._ensure_manager(layer_idx).compress(layer_idx, device)

    def memory_summary(self) -> Dict[str, Any]:
        if self._manager is None:
            return {"hbm_tokens": 0, "dram_entries": 0, "dram_bytes": 0,
                    "max_hbm_tokens": self.sink_tokens + self.keep_tail}
        return self._manager.memory_summary()

    @property
    def dram_table(self):
        if self._manager is None:
            return {}
        return self._manager._dram_table

    def offload_to_host(self, fraction: float, seed: int = 0) -> int:
        """Move a seeded `fraction` of every layer's INT4 block records to pinned host memory;
        decode then prefetches each layer's records one layer ahead (HeteroKVManager.offload_to_host)."""
        if self._manager is None:
            return 0
        return self._manager.offload_to_host(fraction, seed)

    @property
    def retrieval_window(self):
        """None: attend every INT4 chunk (Path C); int or "adaptive": top-w chunks (Path A)."""
        return None if self._manager is None else self._manager.retrieval_window

    @retrieval_window.setter
    def retrieval_window(self, w):
        self._ensure_manager(0).retrieval_window = w

    def prefetch_stats(self, reset: bool = True) -> Dict[str, Any]:
        if self._manager is None:
            return {"stall_ms": 0.0, "per_layer": []}
        return self._manager.prefetch_stats(reset)

    def schedule_prefetch(self, chunk_key: str) -> None:
        """engine_wrapper.py:332-336: dequantize a chunk on the prefetcher's side stream."""
        if self._manager is not None:
            self._manager.schedule_prefetch(chunk_key)

    def swap_in_chunk(self, chunk_key: str) -> Optional[Tuple[torch.Tensor, torch.Tensor]]:
        """engine_wrapper.py:338-344: remove a chunk from the INT4 tier, returning bf16 K/V."""
        if self._manager is None:
            return None
        return self._manager.swap_in(0, chunk_key)

    def swap_in_quantized(self, chunk_key: str) -> Optional[Dict[str, torch.Tensor]]:
        """engine_wrapper.py:346-355: a chunk's INT4 data without dequantizing it."""
        if self._manager is None:
            return None
        return self._manager.swap_in_quantized(0, chunk_key)

    def check_errors(self) -> None:
        """Raise HeteroKVError if a kernel reported a device error (synchronizes)."""
        if self._manager is not None:
            self._manager.check_errors()

    def fused_attn_on_swapped(self, q: torch.Tensor, chunk_key: str,
                              sm_scale: Optional[float] = None) -> Optional[torch.Tensor]:
        """engine_wrapper.py:357-404: attention of q over one chunk's INT4 tokens."""
        from .fused_dequant_attn import fused_dequant_attn_decode
        data = self.swap_in_quantized(chunk_key)
        if data is None:
            return None
        B, H, T, _ = data["k_data"].shape
        return fused_dequant_attn_decode(q, data["k_data"], data["k_scales"].view(B, H, T), data["k_zps"].view(B, H, T),
                                         data["v_data"], data["v_scales"].view(B, H, T), data["v_zps"].view(B, H, T),
                                         sm_scale=sm_scale)


def heterokv_attention_forward(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    """Attention function registered with transformers as "heterokv".

    Decode tokens tagged by FusedHeteroCache.update attend through the manager's
    fused INT4/fp16 kernel, prefill chunks tagged by a fused_prefill cache through the
    MFMA prefill kernel; every other call goes to transformers' SDPA attention on the
    tensors the cache returned, as in the reference."""
    route = getattr(key, "_hkv_route", None)
    if route is not None and query.shape[2] == 1:
        cache, layer_idx, include_dram = route
        feed = cache.track_attention and cache._num_layers is not None and layer_idx == cache._num_layers - 1
        out = cache._manager.attend_decode(layer_idx, query, sm_scale=scaling, include_dram=include_dram,
                                           feed_oracle=feed)
        return out.transpose(1, 2).contiguous(), None
    pre = getattr(key, "_hkv_prefill", None)
    if pre is not None and query.shape[2] == key.shape[2]:
        cache, layer_idx = pre
        out = cache._manager.attend_prefill(layer_idx, query, key, value, sm_scale=scaling)
        return out.transpose(1, 2).contiguous(), None
    from transformers.integrations.sdpa_attention import sdpa_attention_forward
    return sdpa_attention_forward(module, query, key, value, attention_mask, scaling=scaling, dropout=dropout,
                                  **kwargs)


def register_attention() -> str:
    """Register heterokv_attention_forward with transformers; returns its name."""
    from transformers import AttentionInterface
    AttentionInterface.register(ATTN_IMPLEMENTATION, heterokv_attention_forward)
    try:
        from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS, sdpa_mask
        ALL_MASK_ATTENTION_FUNCTIONS.register(ATTN_IMPLEMENTATION, sdpa_mask)
    except Exception:  # older transformers: masks are built per implementation name elsewhere
        pass
    return ATTN_IMPLEMENTATION


class ChunkedPrefillEngine:
    """engine_wrapper.py:411-496: feeds a long prompt through the model in chunks.

    After every chunk it schedules a prefetch of every chunk key in the DRAM table, as the
    reference does (:484-486), so the prefetcher's side stream dequantizes the stored
    chunks while the next chunk runs; prefetch_after_chunk=False skips that (the
    attention outputs are the same either way)."""

    def __init__(self, model, cache: FusedHeteroCache, chunk_size: int = 2048, verbose: bool = False,
                 prefetch_after_chunk: bool = True):
        self.model = model
        self.cache = cache
        self.chunk_size = chunk_size
        self.verbose = verbose
        self.prefetch_after_chunk = prefetch_after_chunk

    @torch.inference_mode()
    def prefill(self, input_ids: torch.Tensor, position_ids: Optional[torch.Tensor] = None,
                attention_mask: Optional[torch.Tensor] = None):
        total_len = input_ids.shape[-1]
        device = input_ids.device
        last = None
        chunk_idx = 0
        for start in range(0, total_len, self.chunk_size):
            end = min(start + self.chunk_size, total_len)
            chunk_ids = input_ids[:, start:end]
            chunk_pos = (position_ids[:, start:end] if position_ids is not None
                         else torch.arange(start, end, dtype=torch.long, device=device).unsqueeze(0))
            # The cache returns [sink | old tail | chunk] for a later chunk, so the chunk's
            # queries sit after the `phys` cached tokens; the reference restarts
            # cache_position at 0 for every chunk (:455-460), which under transformers >= 5
            # lines the causal mask up with the start of that tensor instead.
            mgr = self.cache._manager
            phys = (mgr.hbm_length(0) or 0) if mgr is not None else 0
            chunk_cache_pos = torch.arange(phys, phys + end - start, dtype=torch.long, device=device)
            chunk_mask = attention_mask[:, :end] if attention_mask is not None else None
            last = self.model(input_ids=chunk_ids, past_key_values=self.cache, use_cache=True,
                              position_ids=chunk_pos, attention_mask=chunk_mask, cache_position=chunk_cache_pos)
            if self.verbose:
                print("  chunk [%6d:%6d] dram_entries=%d" % (start, end, len(self.cache.dram_table)), flush=True)
            if self.prefetch_after_chunk and self.cache._manager is not None:
                for key in list(self.cache.dram_table.keys()):
                    self.cache.schedule_prefetch(key)
            chunk_idx += 1
            # The reference collects every 4 chunks (:491-494).  A full collection walks
            # every tracked object of the process (~430K with transformers loaded, ~140 ms),
            # so the chunks in between collect the young generations only, where a chunk's
            # transient objects live; the last chunk still runs a full collection.
            if end == total_len:
                gc.collect()
            elif chunk_idx % 4 == 0:
                gc.collect(1)
        return last


class DecodeGraph:
    """One decode step of `model` over a FusedHeteroCache, captured in a HIP graph and
    replayed for every later token.

    The cache's manager switches to device-stepped decode (enable_device_decode): the
    zone decision of each step and the zone lengths decode attention reads live on the
    GPU, so no kernel argument of a step depends on host state.  The first step runs
    eagerly (it also sizes the decode workspace and settles the DRAM-tier gate, which
    layer 0 refreshes after its own update); the second is captured and replayed; from
    then on a step copies the token ids and positions into the graph's input buffers,
    advances the host copies of the zone bookkeeping exactly as an eager step would and
    replays.  The returned logits live in the graph's memory pool and are overwritten
    by the next step.

    A host tier's copies join the graph (HeteroKVManager.begin_graph_staging): each
    staged layer's host runs are gathered from the pinned arena by a kernel captured
    before the layer's decode kernel, in stream order, with nothing overlapping them; it
    suits a retrieval window (a few chunks per layer), while full retrieval runs faster
    eagerly, where the native side stream overlaps the copies with compute.  With a retrieval window the chunk selection is made on the
    host before every step, as an eager step makes it; a step whose selection differs
    from the captured one drops the graph and captures again.  Not for caches whose
    decode step does host work that has no graph form: attention tracking, adaptive
    self-healing.  The INT4 tier may not change while the graph lives (decode never adds
    to it)."""

    def __init__(self, model, cache: FusedHeteroCache):
        if not cache.fused_decode:
            raise HeteroKVError(-4, "DecodeGraph needs fused_decode=True")
        if cache.adaptive_self_healing or cache.track_attention:
            raise HeteroKVError(-4, "DecodeGraph: adaptive retrieval and attention tracking run host logic per step")
        self.model = model
        self.cache = cache
        self.graph = None
        self.steps = 0
        self._ids = self._pos = self._logits = None
        self._int4 = None
        self._sels = None
        self._staging = False

    def _check(self):
        mgr = self.cache._manager
        if mgr is None:
            raise HeteroKVError(-1, "DecodeGraph: prefill the cache before decoding")
        int4 = [0 if st is None else st.int4_len for st in mgr._layers]
        if self._int4 is not None and int4 != self._int4:
            raise HeteroKVError(-1, "DecodeGraph: the INT4 tier changed since the graph was captured")
        self._int4 = int4
        return mgr

    def _select(self, mgr):
        """This step's chunk selection of every layer (None without a retrieval window),
        made on the host once per layer as an eager step makes it and left for
        attend_decode; the window block tables are built here, outside any capture."""
        if mgr.retrieval_window is None:
            return None
        sels = []
        for li, st in enumerate(mgr._layers):
            sel = mgr._selection(li) if st is not None and st.int4_len else None
            if sel is not None:
                mgr._window_table(li, st, sel)
            sels.append(sel)
        return tuple(sels)

    def _drop(self):
        torch.cuda.synchronize()
        self.graph = None
        self._logits = None

    def _forward(self, ids, pos):
        return self.model(input_ids=ids, position_ids=pos, past_key_values=self.cache, use_cache=True).logits

    def _advance_host(self, mgr):
        """What FusedHeteroCache.update does on the host for one decode token, layer by layer."""
        cache = self.cache
        for li in range(mgr.num_layers):
            mgr.advance_decode_host(li, cache.real_seq_len)
            cache._layer_seen[li] = cache._layer_seen.get(li, 0) + 1
            if li == 0:
                cache.real_seq_len += 1
                if cache.self_healing:
                    cache._refresh_swap_count()

    @torch.inference_mode()
    def step(self, input_ids: torch.Tensor, position_ids: torch.Tensor) -> torch.Tensor:
        """input_ids, position_ids: [B, 1] on the cache's device; returns logits [B, 1, vocab]."""
        mgr = self._check()
        sels = self._select(mgr)
        if self.graph is not None and sels != self._sels:
            self._drop()              # another chunk selection: capture again
        if self.steps == 0:
            mgr.enable_device_decode(True)
            out = self._forward(input_ids, position_ids)
        elif self.graph is None:
            self._ids = input_ids.clone()
            self._pos = position_ids.clone()
            self._sels = sels
            if any(st is not None and st.n_host > 0 for st in mgr._layers):
                mgr.begin_graph_staging()
                self._staging = True
            g = torch.cuda.CUDAGraph()
            # capturing runs the step's host logic once (the host state advances here);
            # its kernels run at the first replay
            with torch.cuda.graph(g):
                self._logits = self._forward(self._ids, self._pos)
            g.replay()
            mgr._errword().post()
            self.graph = g
            out = self._logits
        else:
            # The kernels of a replay report into the manager's error word like eager steps
            # do; the word is read back here, at the next step, without blocking.  A step
            # that reported an error had its flags fixed at capture, so the graph is
            # dropped and a later step captures again (after a placement failure the
            # workspace has switched to the device-scope hand-off by then).
            err = mgr._errword()
            try:
                err.poll()
            except HeteroKVError:
                self.graph = None
                self._logits = None
                raise
            self._ids.copy_(input_ids)
            self._pos.copy_(position_ids)
            self._advance_host(mgr)
            mgr._selection_of.clear()     # read by the captured step, not again by a replay
            self.graph.replay()
            err.post()
            out = self._logits
        self.steps += 1
        return out

    def close(self) -> None:
        """Drop the graph and return the manager to host-stepped decode (and a host tier
        to the native prefetch schedule)."""
        self._drop()
        if self.cache._manager is not None:
            if self._staging:
                self.cache._manager.end_graph_staging()
                self._staging = False
            self.cache._manager.enable_device_decode(False)


def build_fused_cache(num_layers: Optional[int] = None, device: str = "cuda:0", sink_tokens: int = 64,
                      keep_tail: int = 8192, chunk_size: int = 2048, group_size: int = 128,
                      enable_quant: bool = True, enable_prefetch: bool = True, enable_triton: bool = True,
                      bandwidth_limiter=None, self_healing: bool = True,
                      adaptive_self_healing: bool = False) -> FusedHeteroCache:
    """engine_wrapper.py:503-539."""
    return FusedHeteroCache(num_layers=num_layers, sink_tokens=sink_tokens, keep_tail=keep_tail,
                            chunk_size=chunk_size, device=device, group_size=group_size,
                            enable_quant=enable_quant, enable_prefetch=enable_prefetch,
                            enable_triton=enable_triton, bandwidth_limiter=bandwidth_limiter,
                            self_healing=self_healing, adaptive_self_healing=adaptive_self_healing)
