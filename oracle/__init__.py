"""Oracle: CPU restatement of the reference's INT4-KV hot path.

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import anything from this package, and
only as the reference results that GPU outputs are compared with (or, for the
bench, as the timed CPU baseline).  The product path (the ``heterokv`` package)
never imports it and fails loudly when its HIP library is missing.

Modules
  compressor   -- KVCompressor.compress/decompress/relative_error
                  (src/quantization/kv_compressor.py:50-154), via the C file
                  hkv_oracle.c; pinned by hand-computed known answers and
                  invariants in tests/test_oracle_compressor.py.
  attention    -- dequantize-then-attend in float64 with GQA
                  (src/quantization/fused_dequant_attn.py:242-247,326-331,388-390;
                  zone merge src/core/fused_attention_patch.py:127-196); pinned by
                  closed forms and torch SDPA in tests/test_oracle_attention.py.
  pool_format  -- the packed INT4 block-record and fp16-zone layouts of this
                  build, written from their specification in include/heterokv.h.
  torch_ref    -- the same compress / decompress / Path C / attention in float32 torch
                  on the CPU, with the reference's own torch operations: the bench's
                  CPU baseline; pinned bit for bit against the C compressor and against
                  the float64 attention in tests/test_oracle_torch_ref.py.
  manager      -- HeteroKVManager zone / eviction / gather index arithmetic
                  (src/memory/manager.py:416-674,686-777,779-821,1218-1299);
                  pinned by hand-derived traces in tests/test_oracle_manager.py.
"""
