"""Heavy-hitter scoring restatement (TEST INFRASTRUCTURE ONLY, see oracle/__init__.py).

Follows the reference's HeavyHitterOracle and its block-mean kernel:
  src/policy/heavy_hitter.py:26-37   update: token_scores[:n] += recent_attention
  src/policy/heavy_hitter.py:43-101  get_eviction_candidates: protected sink / local
      blocks, +inf on them, bottom-k of the block means, ascending
  src/kernels/oracle_triton.py:16-79 compute_block_scores: per-block mean of the
      token scores (the last block may be partial)
  src/core/fused_attention_patch.py:104-107  the vector fed to update(): softmax
      weights of the newest query row, averaged over the heads

Choices the reference leaves open, fixed here (and by the HIP kernels):
  * a block mean is the float32 sum of its tokens in index order divided by the count
    in float32 (the reference's Triton kernel reduces its 256-lane vector in an order
    it does not specify; results can differ from it by float32 rounding);
  * equal means are ordered by block index (torch.topk leaves the order of ties open).
"""
import numpy as np


def block_scores(token_scores, seq_len, block_size):
    """oracle_triton.py:60-79: mean token score of each of ceil(seq_len / bs) blocks."""
    ts = np.asarray(token_scores, dtype=np.float32)
    nb = (seq_len + block_size - 1) // block_size
    out = np.empty(nb, dtype=np.float32)
    for i in range(nb):
        t0, t1 = i * block_size, min((i + 1) * block_size, seq_len)
        acc = np.float32(0.0)
        for t in range(t0, t1):
            acc = np.float32(acc + ts[t])
        out[i] = np.float32(acc / np.float32(max(t1 - t0, 1)))
    return out


def eviction_plan(seq_len, block_size, sink_tokens, local_window, evict_num_blocks):
    """heavy_hitter.py:51-92: (num_blocks, first protected-at-end block, count k)."""
    if seq_len <= sink_tokens + local_window:
        return 0, 0, 0, 0
    nb = -(-seq_len // block_size)
    sb = -(-sink_tokens // block_size)
    lb = -(-local_window // block_size)
    unsafe = max(0, nb - sb - lb)
    return nb, sb, max(0, nb - lb), min(evict_num_blocks, unsafe)


def eviction_candidates(token_scores, seq_len, block_size, sink_tokens, local_window, evict_num_blocks):
    """heavy_hitter.py:43-101 with scores present: block indices, ascending by (mean, index)."""
    nb, lo, hi, k = eviction_plan(seq_len, block_size, sink_tokens, local_window, evict_num_blocks)
    if k <= 0:
        return []
    means = block_scores(token_scores, seq_len, block_size).astype(np.float64)
    means[:lo] = np.inf
    means[hi:] = np.inf
    order = sorted(range(nb), key=lambda i: (means[i], i))
    return order[:k]


def cold_start_candidates(seq_len, block_size, sink_tokens, local_window, evict_num_blocks):
    """heavy_hitter.py:63-74: no scores yet -> the oldest blocks after the sink (FIFO)."""
    if seq_len <= sink_tokens + local_window:
        return []
    nb = -(-seq_len // block_size)
    first = -(-sink_tokens // block_size)
    last = nb - (-(-local_window // block_size))
    count = max(0, min(evict_num_blocks, last - first))
    return list(range(first, first + count))


def newest_token_weights(scores_log2):
    """fused_attention_patch.py:101,104-107: softmax over each head's scores (given in
    the log2 domain), averaged over heads.  scores_log2: [H, n] (-inf = masked)."""
    s = np.asarray(scores_log2, dtype=np.float64)
    mx = s.max(axis=1, keepdims=True)
    e = np.where(np.isfinite(s), np.exp2(s - mx), 0.0)
    return (e / e.sum(axis=1, keepdims=True)).mean(axis=0)
