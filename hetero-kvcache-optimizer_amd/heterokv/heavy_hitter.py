"""HeavyHitterOracle and compute_block_scores on the GPU.

Mirrors src/policy/heavy_hitter.py:8-101 and src/kernels/oracle_triton.py:60-79: the
same constructor, update / get_eviction_candidates and return types.  The block means
and the protected bottom-k run in libheterokv (hkv_block_scores,
hkv_eviction_candidates); the attention weights that feed update() can come straight
from a decode launch (hkv_attn_weights, see HeteroKVManager.attend_decode).

Fixed where the reference leaves it open: a block mean sums its tokens in index
order in fp32; equal block means are returned in index order.
"""
import math

import torch

from . import ops


def compute_block_scores(token_scores: torch.Tensor, current_seq_len: int, block_size: int) -> torch.Tensor:
    """oracle_triton.py:60-79: mean score of each of ceil(current_seq_len / block_size) blocks."""
    if block_size == 1:
        return token_scores[:current_seq_len].clone()
    return ops.block_scores(_board(token_scores, current_seq_len), current_seq_len, block_size)


def _board(token_scores: torch.Tensor, n: int) -> torch.Tensor:
    """The score board padded with zeros to n entries (tokens never scored count 0)."""
    ts = token_scores.to(torch.float32)
    if ts.shape[0] >= n:
        return ts
    out = torch.zeros(n, dtype=torch.float32, device=ts.device)
    out[:ts.shape[0]] = ts
    return out


class HeavyHitterOracle:
    """heavy_hitter.py:8-101: cumulative attention scores and eviction candidates."""

    def __init__(self, block_size: int = 16, sink_tokens: int = 32, local_window: int = 128):
        self.block_size = block_size
        self.sink_tokens = sink_tokens
        self.local_window = local_window
        self.token_scores = None

    def update(self, recent_attention: torch.Tensor) -> None:
        """heavy_hitter.py:26-37: token_scores[:n] += recent_attention (growing the board)."""
        n = recent_attention.shape[0]
        self._ensure(n, recent_attention.device)
        self.token_scores[:n] += recent_attention.to(torch.float32)

    def _ensure(self, n: int, device) -> None:
        if self.token_scores is None or self.token_scores.shape[0] < n:
            new = torch.zeros(n, dtype=torch.float32, device=device)
            if self.token_scores is not None:
                new[:self.token_scores.shape[0]] = self.token_scores
            self.token_scores = new

    def update_from_decode(self, scores: torch.Tensor, score_stats: torch.Tensor, order: torch.Tensor) -> None:
        """update() with the newest token's weights of sequence 0, computed from a decode
        launch's score outputs and added into the board in one kernel."""
        n = order.numel()
        self._ensure(n, scores.device)
        ops.attn_weights(scores[:1], score_stats[:1], order=order, out=self.token_scores.view(1, -1),
                         accumulate=True)

    def get_eviction_candidates(self, current_seq_len: int, evict_num_blocks: int) -> torch.Tensor:
        """heavy_hitter.py:43-101.  Cold start (no scores yet): the oldest blocks after the
        sink, as a CPU tensor; otherwise the lowest-mean unprotected blocks on the GPU."""
        if current_seq_len <= self.sink_tokens + self.local_window:
            dev = self.token_scores.device if self.token_scores is not None else torch.device("cpu")
            return torch.empty(0, dtype=torch.long, device=dev)
        num_blocks = math.ceil(current_seq_len / self.block_size)
        sink_blocks = math.ceil(self.sink_tokens / self.block_size)
        local_blocks = math.ceil(self.local_window / self.block_size)
        if self.token_scores is None:
            first, last = sink_blocks, num_blocks - local_blocks
            count = max(0, min(evict_num_blocks, last - first))
            if count <= 0:
                return torch.empty(0, dtype=torch.long, device="cpu")
            return torch.arange(first, first + count, dtype=torch.long, device="cpu")
        return ops.eviction_candidates(_board(self.token_scores, current_seq_len), current_seq_len,
                                       self.block_size, self.sink_tokens, self.local_window, evict_num_blocks)
