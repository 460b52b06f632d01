"""heterokv: MI355X-native INT4-KV hot path (HIP kernels for gfx950 behind a C ABI).

Drop-in names of the reference's quantized-KV path:
  KVCompressor                 (src/quantization/kv_compressor.py)
  fused_dequant_attn_decode    (src/quantization/kernels/fused_dequant_attn.py)
  HeteroKVManager              (src/memory/manager.py)
  FusedHeteroCache, ChunkedPrefillEngine, build_fused_cache   (src/core/engine_wrapper.py)
  DRAMStorageManager           (src/memory/dram_storage.py)
  AsyncPrefetcher              (src/policy/prefetcher.py)
  AdaptivePrefetchController   (src/policy/adaptive_prefetch_controller.py)
  HeavyHitterOracle            (src/policy/heavy_hitter.py)
  compute_block_scores         (src/kernels/oracle_triton.py)
plus the block-pool / fp16-zone primitives in ``heterokv.ops``.
"""
from ._lib import HeteroKVError, load  # noqa: F401
from .kv_compressor import KVCompressor  # noqa: F401
from .fused_dequant_attn import fused_dequant_attn_decode, fused_dequant_attn_forward  # noqa: F401
from . import ops  # noqa: F401
from .prefetcher import (Prefetcher, DRAMStorageManager, AsyncPrefetcher,  # noqa: F401
                         AdaptivePrefetchController)
from .heavy_hitter import HeavyHitterOracle, compute_block_scores  # noqa: F401
from .manager import HeteroKVManager  # noqa: F401
from .engine_wrapper import (FusedHeteroCache, ChunkedPrefillEngine, DecodeGraph, build_fused_cache,  # noqa: F401
                             register_attention)

__all__ = ["HeavyHitterOracle", "compute_block_scores", "HeteroKVError", "KVCompressor", "fused_dequant_attn_decode", "fused_dequant_attn_forward", "ops", "load", "HeteroKVManager",
           "FusedHeteroCache", "ChunkedPrefillEngine", "DecodeGraph", "build_fused_cache", "register_attention",
           "Prefetcher", "DRAMStorageManager", "AsyncPrefetcher", "AdaptivePrefetchController"]
