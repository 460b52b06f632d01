"""Token-position restatement of the reference HeteroKVManager / FusedHeteroCache
bookkeeping (TEST INFRASTRUCTURE ONLY, see oracle/__init__.py).

Every token is represented by its absolute position; the restatement tracks
which positions sit in which zone and in which order the reference returns them,
so the build's manager can be checked index for index.  Followed line by line:

  src/memory/manager.py
    __init__ budgets              :67,88   tail budget = hbm_budget - sink;
                                           heavy-hitter budget = max(hbm_budget // 2, 2048)
    _prefill_update (first chunk) :454-535 sink = first min(N, sink); tail = last
                                           min(N - sink_amt, tail_budget); body -> DRAM;
                                           returns the full input
    _incremental_prefill_update   :537-586 combined = tail + chunk; returns sink + combined;
                                           evicts combined[:len - tail_budget] to DRAM
    _decode_update                :588-674 tail grows to tail_budget, then its oldest token
                                           goes to the competition queue and the tail slides;
                                           returns sink + tail + heavy hitters
    _process_competition_queue    :686-715 up to (hh_budget - |hh|) queued tokens, highest
                                           score first (stable), join the heavy-hitter zone
    _update_legacy_cache          :752-777 _key_cache = sink + tail + hh
    decompress_dram_chunks        :779-821 every "l{layer}_" chunk in dict (eviction) order
    count_dram_tokens             :1218-1229 #chunks(layer) * |first chunk|
    decompress_dram_chunks_adaptive / get_dram_chunks_quantized_adaptive
                                  :857-878,966-978 the layer's chunks in dict order, ranked
                                           by chunk score descending (stable), the first w
                                           kept, returned in eviction order
    swap_in                       :265-278 the chunk leaves the DRAM table (its eviction-order
                                           entry and score stay)
    _evict_to_dram                :1231-1299 key "l{layer}_e{counter}"; score 1/(counter+1)
                                           without oracle scores; counter += 1 only on layer 0
  src/memory/attention_competition_queue.py
    enqueue / dequeue_top_k       :34-107  one shared queue for all layers, sorted by score,
                                           ties in insertion order (Python's stable sort)
  src/core/engine_wrapper.py
    update                        :137-254 prefill if new_len > 1; Path C (default) prepends
                                           the layer's DRAM tokens at decode when
                                           _swap_in_tokens > 0; layer 0 bumps real_seq_len and,
                                           at decode, refreshes _swap_in_tokens afterwards
    get_seq_length                :256-264 |_key_cache| + _swap_in_tokens
    get_mask_sizes                :274-301 prefill: physical + q_len; decode: physical + swap
                                           (+1 while the tail still grows)

The attention scores that would come from HeavyHitterOracle are never produced
on the reference's decode path (its SDPA patch is inert, fused_attention_patch.py:24-30),
so every queued token carries score 1.0 (manager.py:643-644) and the order is FIFO.
"""
from collections import OrderedDict


class ManagerOracle:
    def __init__(self, num_layers, sink_tokens=64, hbm_budget_tokens=8192, enable_quant=True):
        self.num_layers = num_layers
        self.sink_tokens = sink_tokens
        self.hbm_budget_tokens = hbm_budget_tokens
        self.enable_quant = enable_quant
        self.tail_budget = hbm_budget_tokens - sink_tokens
        self.hh_budget = max(hbm_budget_tokens // 2, 2048)
        self.sink = [None] * num_layers
        self.tail = [None] * num_layers
        self.hh = [None] * num_layers
        self.key_cache = [None] * num_layers
        self.seq_offsets = [0] * num_layers
        self.dram = OrderedDict()          # chunk key -> list of positions
        self.chunk_order = []
        self.chunk_scores = {}
        self.eviction_counter = 0
        self.queue = OrderedDict()         # token id -> (layer, position, score)
        self.token_counter = 0

    # ------------------------------------------------------------ manager.py
    def update(self, layer, positions, mode, seq_offset=0):
        positions = list(positions)
        if mode == "prefill":
            if self.sink[layer] is not None:
                return self._incremental(layer, positions, seq_offset)
            n = len(positions)
            sink_amt = min(n, self.sink_tokens)
            self.sink[layer] = positions[:sink_amt]
            tail_amt = min(n - sink_amt, self.tail_budget)
            self.tail[layer] = positions[n - tail_amt:] if tail_amt > 0 else []
            body = positions[sink_amt:n - tail_amt]
            if self.enable_quant and body:
                self._evict(layer, body)
            self.hh[layer] = []
            self._legacy(layer)
            self.seq_offsets[layer] = seq_offset + n
            return positions
        if mode == "decode":
            assert len(positions) == 1
            if self.tail[layer] is None:
                self.tail[layer] = list(positions)
            elif len(self.tail[layer]) < self.tail_budget:
                self.tail[layer] = self.tail[layer] + positions
            else:
                evicted = self.tail[layer][0]
                self._enqueue(layer, evicted, 1.0)
                self.tail[layer] = self.tail[layer][1:] + positions
            self._process_queue(layer)
            self._legacy(layer)
            self.seq_offsets[layer] = seq_offset + 1
            return list(self.key_cache[layer])
        raise ValueError("Unknown mode: %s" % mode)

    def _incremental(self, layer, positions, seq_offset):
        combined = self.tail[layer] + positions
        ret = self.sink[layer] + combined
        if len(combined) > self.tail_budget:
            e = len(combined) - self.tail_budget
            if self.enable_quant and e > 0:
                self._evict(layer, combined[:e])
            self.tail[layer] = combined[e:]
        else:
            self.tail[layer] = combined
        self._legacy(layer)
        self.seq_offsets[layer] = seq_offset + len(positions)
        return ret

    def _enqueue(self, layer, position, score):
        tid = "tail_evict_%d_%d" % (layer, self.token_counter)
        self.queue[tid] = (layer, position, score)
        self.token_counter += 1

    def _process_queue(self, layer):
        cur = len(self.hh[layer]) if self.hh[layer] is not None else 0
        avail = self.hh_budget - cur
        if avail > 0 and self.queue:
            items = sorted(self.queue.items(), key=lambda kv: kv[1][2], reverse=True)[:avail]
            got = [it[1][1] for it in items]
            for tid, _ in items:
                del self.queue[tid]
            self.hh[layer] = (self.hh[layer] or []) + got

    def _legacy(self, layer):
        self.key_cache[layer] = (self.sink[layer] or []) + (self.tail[layer] or []) + (self.hh[layer] or [])

    def _evict(self, layer, chunk):
        key = "l%d_e%d" % (layer, self.eviction_counter)
        self.dram[key] = list(chunk)
        self.chunk_order.append(key)
        self.chunk_scores[key] = 1.0 / (self.eviction_counter + 1)
        if layer == 0:
            self.eviction_counter += 1

    def dram_positions(self, layer):
        pre = "l%d_" % layer
        out = []
        for k, v in self.dram.items():
            if k.startswith(pre):
                out.extend(v)
        return out

    def select_chunks(self, layer, window_size):
        pre = "l%d_" % layer
        keys = [k for k in self.dram if k.startswith(pre)]
        ranked = sorted(keys, key=lambda k: self.chunk_scores.get(k, 0.0), reverse=True)
        chosen = ranked[:window_size]
        return sorted(chosen, key=lambda k: self.chunk_order.index(k))

    def remove_chunk(self, key):
        return self.dram.pop(key, None)

    def count_dram_tokens(self, layer=0):
        pre = "l%d_" % layer
        keys = [k for k in self.dram if k.startswith(pre)]
        if not keys:
            return 0
        return len(keys) * len(self.dram[keys[0]])

    def max_hbm_tokens(self):
        return self.sink_tokens + self.hbm_budget_tokens + self.hh_budget


class CacheOracle:
    """FusedHeteroCache bookkeeping with the default Path C (engine_wrapper.py:137-301)."""

    def __init__(self, num_layers, sink_tokens=64, keep_tail=8192, self_healing=True):
        self.m = ManagerOracle(num_layers, sink_tokens, keep_tail)
        self.num_layers = num_layers
        self.self_healing = self_healing
        self.real_seq_len = 0
        self.swap_in_tokens = 0

    def update(self, layer, positions):
        n = len(positions)
        mode = "prefill" if n > 1 else "decode"
        out = self.m.update(layer, positions, mode, seq_offset=self.real_seq_len)
        if mode == "decode" and self.self_healing and self.swap_in_tokens > 0:
            dram = self.m.dram_positions(layer)
            if dram:
                out = dram + out
        if layer == 0:
            self.real_seq_len += n
            if mode == "decode" and self.self_healing:
                self.swap_in_tokens = self.m.count_dram_tokens(0)
        return out

    def get_seq_length(self, layer=0):
        kc = self.m.key_cache[layer] if layer < len(self.m.key_cache) else None
        if kc is None:
            return 0
        return len(kc) + self.swap_in_tokens

    def get_mask_sizes(self, query_len, layer=0):
        kc = self.m.key_cache[layer] if layer < len(self.m.key_cache) else None
        if kc is None:
            return query_len, 0
        phys = len(kc)
        if query_len > 1:
            return phys + query_len, 0
        tail = self.m.tail[layer]
        if tail is not None and len(tail) >= self.m.tail_budget:
            return phys + self.swap_in_tokens, 0
        return phys + self.swap_in_tokens + 1, 0
