/*
 * heterokv.h -- C ABI of libheterokv.so, the MI355X (gfx950) INT4-KV hot path.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t passed
 * as `void*` (NULL = the default stream).  Nothing here allocates device memory:
 * the caller owns every buffer, including the decode workspace.  Every entry
 * point returns HKV_OK (0) or a negative HKV_ERR_* code; hkv_last_error() then
 * holds a message for the calling thread.  There is no fallback path: a call
 * that cannot run on the GPU fails.
 *
 * Reference interfaces replaced (paths are inside kldxg123/Hetero-KVCache-Optimizer):
 *   KVCompressor.compress          src/quantization/kv_compressor.py:50-98
 *   KVCompressor.decompress        src/quantization/kv_compressor.py:100-132
 *   fused_dequant_attn_decode      src/quantization/kernels/fused_dequant_attn.py:301-368
 *                                  (numerics: src/quantization/fused_dequant_attn.py:326-331,388-390)
 *   HeteroKVManager zone storage   src/memory/manager.py:416-674 (sink / tail / heavy-hitter)
 *   _evict_to_dram + DRAM chunks   src/memory/manager.py:1231-1299, src/memory/dram_storage.py:106-138
 *   decompress_dram_chunks (Path C gather order)   src/memory/manager.py:779-821
 *   DRAMStorageManager (host tier)                 src/memory/dram_storage.py:20-222
 *   AsyncPrefetcher (side-stream H2D)              src/policy/prefetcher.py:21-123
 *
 * INT4 block pool.  Tokens of the quantized middle zone live in 16-token
 * blocks.  One block record holds every kv head of those 16 tokens as H
 * contiguous 2208-byte head parts (part h at byte h*2208), so the reader of one
 * kv head streams one contiguous run per block:
 *
 *   offset in a head part      contents
 *   0                          K codes  [16 tokens][64 B]       (packed, see below)
 *   1024                       V codes  [1024 B]                (packed, transposed tiles)
 *   2048                       K scales [16] float32
 *   2112                       V scales [16] float32
 *   2176                       K zero points [16] uint8
 *   2192                       V zero points [16] uint8
 *   record size = H * 2208 bytes                                 (head_dim 128)
 *
 * A token's 128 values form one quantization group, exactly as the reference
 * compressor's default group_size=128 over a [B,H,S,128] tensor: scale =
 * max((max-min)/15, 1e-8) in float32, zp = clamp(rint(-min/scale),0,15),
 * code = clamp(rint(x/scale + zp),0,15) (round half to even).
 *
 * Nibble packing.  A 32-bit little-endian word holds 8 codes x0..x7 with
 * x_k at bit (k%2)*16 + (k/2)*4, so (w >> 4i) & 0x000F000F yields the pair
 * (x_2i, x_2i+1) as two 16-bit lanes.
 *   K: word j of a token row (j=0..15) holds dims 8j..8j+7 as x0..x7.
 *   V: word (g*16+c)*4+m of a head part's 1024 B holds, for tokens 4g..4g+3,
 *      x0..x3 = dim c+32m and x4..x7 = dim c+32m+16   (g<4, c<16, m<4).
 *
 * Host tier.  A block-table entry id >= 0 names record `id` of `pool`; an entry
 * id < 0 names record ~id (= -id-1) of `staging`, an HBM buffer that the
 * prefetcher below fills from pinned host memory before the kernel runs.  The
 * append kernels (hkv_pack_tokens, hkv_repack_codes) only write pool records.
 *
 * fp16 zones (sink, recent window, heavy hitters).  K is row-major
 * [B][H][cap][128]; V is stored in 16-token transposed tiles
 * [B][H][cap/16][4 g][16 c][8 n][4 i] fp16 holding V[token 4g+i][dim c+16n].
 * Slots [0, len) of a zone are attended; their order does not matter.
 *
 * bfloat16 models.  Entry points that take model activations (zone writes, the
 * decode query and output, the prefill query, chunk and output) accept bf16 as well
 * as fp16.  Zones and MFMA operands stay fp16: a bf16 value converts to fp16
 * exactly when its magnitude lies in [2^-14, 65504] (bf16 carries 8 significant
 * bits, fp16 11), smaller magnitudes lose at most 2^-25 absolutely, and a finite
 * value beyond the fp16 range becomes +-inf and sets HKV_ERR_BIT_RANGE in the
 * call's error word.  Results are written in the requested output dtype.
 *
 * Device error words.  Kernels that can meet bad data report it by OR-ing bits
 * into a caller-owned device int32 instead of faulting or failing silently; the
 * caller reads it at a synchronization point it already has and clears it (the
 * HKV_ERR_BIT_* values below).
 */
#ifndef HETEROKV_H
#define HETEROKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HKV_ABI_VERSION 9

/* dtype codes */
#define HKV_DTYPE_F16  0
#define HKV_DTYPE_BF16 1
#define HKV_DTYPE_F32  2
#define HKV_DTYPE_U8   3

/* return codes */
#define HKV_OK               0
#define HKV_ERR_ARG         -1   /* bad argument (shape, null pointer, size) */
#define HKV_ERR_HIP         -2   /* a HIP runtime call failed */
#define HKV_ERR_CAPACITY    -3   /* a caller buffer or pool is too small */
#define HKV_ERR_UNSUPPORTED -4   /* shape the kernels do not handle (e.g. head_dim != 128) */
#define HKV_ERR_DEVICE      -5   /* reserved for bindings: a device error word read non-zero */

/* device error-word bits */
#define HKV_ERR_BIT_BLOCK_ID  1   /* a block-table id outside the pool / staging records
                                     (a valid record was read in its place) */
#define HKV_ERR_BIT_SLOT      2   /* a token slot beyond its block-table row (nothing written) */
#define HKV_ERR_BIT_PLACEMENT 4   /* decode: the ranges of one (sequence, kv head) ran on more
                                     than one XCD while the launch relied on an XCD-local
                                     hand-off; that launch's output is invalid.  Pass
                                     HKV_DECODE_AGENT_HANDOFF from then on. */
#define HKV_ERR_BIT_RANGE     8   /* a finite bf16 value beyond the fp16 range was narrowed */

#define HKV_BLOCK_TOKENS 16
#define HKV_MAX_F16_ZONES 3

/* Version of this ABI (HKV_ABI_VERSION). */
int hkv_abi_version(void);

/* Message for the last failed call on this thread ("" if none). */
const char* hkv_last_error(void);

/* Bytes of one INT4 block record for `num_kv_heads` heads (head_dim must be 128). */
int64_t hkv_block_bytes(int32_t num_kv_heads, int32_t head_dim);

/*
 * KVCompressor.compress over a flat tensor (kv_compressor.py:66-98).
 * x: n elements of `dtype` (F16/BF16/F32), contiguous.  The tail is
 * zero-padded to a multiple of group_size exactly as the reference does.
 * codes: n uint8 (one code per byte, the reference's unpacked layout);
 * scales/zps: ceil(n/group_size) entries.
 */
int hkv_quantize_groups(const void* x, int32_t dtype, int64_t n, int32_t group_size,
                        uint8_t* codes, float* scales, uint8_t* zps, void* stream);

/*
 * KVCompressor.decompress (kv_compressor.py:119-132):
 * out[i] = dtype((float(codes[i]) - float(zps[g])) * scales[g]), g = i / group_size.
 */
int hkv_dequantize_groups(const uint8_t* codes, const float* scales, const uint8_t* zps,
                          int64_t n, int32_t group_size, void* out, int32_t out_dtype,
                          void* stream);

/*
 * Quantize `num_tokens` consecutive tokens of every sequence and pack them into
 * INT4 block records (the quantize+pack append kernel).  Token t of sequence b
 * (source K/V at k + b*src_stride_b + h*src_stride_h + t*src_stride_t) goes to
 * INT4 slot p = start_pos[b] + t (start_base + t when start_pos is NULL): record
 * block_table[b*bt_stride + p/16], row p%16.  Rows of a block outside the written
 * range keep their contents.
 */
typedef struct HkvPackArgs {
    const void* k;
    const void* v;
    int32_t dtype;                 /* F16 or BF16 */
    int64_t src_stride_b, src_stride_h, src_stride_t;   /* elements */
    int32_t batch, num_kv_heads, head_dim, num_tokens;
    const int32_t* start_pos;      /* [batch], device; NULL: every sequence starts at start_base */
    const int32_t* block_table;    /* [batch][bt_stride], device */
    int32_t bt_stride;
    uint8_t* pool;                 /* block records */
    int64_t pool_blocks;
    int32_t* err_flag;             /* optional device int: bit 0 = a block id outside the pool,
                                      bit 1 = a slot beyond the block table row (nothing written) */
    int32_t start_base;            /* first slot of every sequence when start_pos is NULL (by
                                      value: the kernel reads no start position from memory) */
} HkvPackArgs;

int hkv_pack_tokens(const HkvPackArgs* args, void* stream);

/*
 * Pack tokens that are already quantized in the reference layout (one code per
 * byte, per-token scale and zero point, as fused_dequant_attn_decode's
 * k_data/k_scales/k_zps, kernels/fused_dequant_attn.py:301-310) into block
 * records, with the same placement rules as hkv_pack_tokens.  Zero points may
 * be uint8 (HKV_DTYPE_U8) or float32 holding integers (HKV_DTYPE_F32).
 */
typedef struct HkvRepackArgs {
    const uint8_t* k_codes;
    const uint8_t* v_codes;
    int64_t code_stride_b, code_stride_h, code_stride_t;     /* bytes; dims contiguous */
    const float* k_scales;
    const float* v_scales;
    const void* k_zps;
    const void* v_zps;
    int32_t zp_dtype;
    int64_t meta_stride_b, meta_stride_h, meta_stride_t;     /* elements */
    int32_t batch, num_kv_heads, head_dim, num_tokens;
    const int32_t* start_pos;
    const int32_t* block_table;
    int32_t bt_stride;
    uint8_t* pool;
    int64_t pool_blocks;
    int32_t* err_flag;
} HkvRepackArgs;

int hkv_repack_codes(const HkvRepackArgs* args, void* stream);

/*
 * Unpack INT4 slots [0, num_tokens) of one sequence into the reference's
 * layout: codes [H][num_tokens][128] uint8, scales/zps [H*num_tokens]
 * (flattened (head, token) order, as compress() of a [1,H,T,128] chunk).
 * Any of codes/scales/zps may be NULL.
 */
int hkv_unpack_tokens(const uint8_t* pool, int64_t pool_blocks, const int32_t* block_table,
                      int32_t num_kv_heads, int32_t head_dim, int32_t num_tokens,
                      int32_t which /* 0 = K, 1 = V */,
                      uint8_t* codes, float* scales, uint8_t* zps, void* stream);

/*
 * Write `num_tokens` fp16 or bf16 tokens into an fp16 zone (sink / recent window /
 * heavy hitters).  Token t of sequence b goes to slot slot_start[b] + t (or
 * slot_base + t when slot_start is NULL), taken modulo `ring` when ring > 0 (a
 * ring of that many slots, ring <= capacity).  K rows are copied; V goes to
 * transposed tiles.
 */
typedef struct HkvZoneWriteArgs {
    const uint16_t* k;             /* source tokens, dtype below */
    const uint16_t* v;
    int64_t src_stride_b, src_stride_h, src_stride_t;
    int32_t batch, num_kv_heads, head_dim, num_tokens;
    const int32_t* slot_start;     /* [batch], device; NULL -> slot_base for every sequence */
    int32_t capacity;              /* slots per (b,h); multiple of 16 */
    int32_t ring;                  /* 0 = no wrap, else ring length (<= capacity) */
    uint16_t* zone_k;              /* [batch][H][capacity][128] */
    uint16_t* zone_v;              /* [batch][H][capacity/16][4096 B tiles] */
    int32_t slot_base;
    int32_t dtype;                 /* source dtype: F16 or BF16 */
    int32_t* err_flag;             /* optional device int: HKV_ERR_BIT_RANGE */
} HkvZoneWriteArgs;

int hkv_zone_write(const HkvZoneWriteArgs* args, void* stream);

/* Read slots [0,n) of an fp16 zone back as row-major K and V [batch][H][n][128]. */
int hkv_zone_read(const uint16_t* zone_k, const uint16_t* zone_v, int32_t batch,
                  int32_t num_kv_heads, int32_t head_dim, int32_t capacity, int32_t n,
                  uint16_t* out_k, uint16_t* out_v, void* stream);

/*
 * Copy n consecutive slots of one fp16 zone to another (both K rows and V
 * tiles), slot src_slot + i -> dst_slot + i for every sequence and head.  Used
 * to move a token evicted from the recent window into the heavy-hitter zone
 * (manager.py:645-664 and :686-715).  Ranges must not wrap and must lie inside
 * both capacities.
 */
int hkv_zone_copy(const uint16_t* src_k, const uint16_t* src_v, int32_t src_capacity, int32_t src_slot,
                  uint16_t* dst_k, uint16_t* dst_v, int32_t dst_capacity, int32_t dst_slot,
                  int32_t batch, int32_t num_kv_heads, int32_t head_dim, int32_t n, void* stream);

/*
 * Device-stepped decode update of the recent-window ring and the heavy-hitter zone:
 * the manager's decode step (src/memory/manager.py:588-674 as this library keeps it)
 * with its decision taken on the GPU from `state`, so that a captured graph can
 * replay it.  state = device int32 [4]: ring head, ring length, heavy-hitter length,
 * dropped tokens.  If the ring is not full the new token goes to slot
 * (head + length) % ring; otherwise the token at `head` moves to heavy-hitter slot
 * hh_len while hh_len < hh_budget (else it is dropped), the new token takes `head`
 * and head advances.  tail_lens / hh_lens (device int32 [batch], may be NULL)
 * receive the new lengths, as zone lengths for hkv_decode_attn.
 */
typedef struct HkvZoneStepArgs {
    const uint16_t* k;             /* new token [batch][num_kv_heads][1][128], dtype below */
    const uint16_t* v;
    int64_t src_stride_b, src_stride_h;
    int32_t batch, num_kv_heads, head_dim;
    uint16_t* tail_k;
    uint16_t* tail_v;
    int32_t tail_capacity, tail_ring;
    uint16_t* hh_k;
    uint16_t* hh_v;
    int32_t hh_capacity, hh_budget;
    int32_t* state;
    int32_t* tail_lens;
    int32_t* hh_lens;
    int32_t dtype;                 /* F16 or BF16 */
    int32_t* err_flag;             /* optional device int: HKV_ERR_BIT_RANGE */
} HkvZoneStepArgs;

int hkv_zone_step(const HkvZoneStepArgs* args, void* stream);

/*
 * Split-K decode attention over [fp16 zones || INT4 pool] for one query token per
 * sequence (fused_dequant_attn_decode with GQA: q head i uses kv head i / n_rep,
 * n_rep = num_q_heads / num_kv_heads).  One launch: partial results of the splits
 * are combined in-kernel by the last workgroup of each (sequence, kv head).
 * out = softmax(q K^T * sm_scale) V  over every valid token, fp16, fp32 accumulation.
 */
typedef struct HkvF16Zone {
    const uint16_t* k;             /* [batch][H][capacity][128] */
    const uint16_t* v;             /* transposed tiles */
    int32_t capacity;              /* multiple of 16 */
    int32_t max_len;               /* upper bound of lens[] (sizes the grid) */
    const int32_t* lens;           /* [batch] device; NULL -> every sequence has max_len */
} HkvF16Zone;

typedef struct HkvDecodeArgs {
    int32_t batch, num_q_heads, num_kv_heads, head_dim;
    float sm_scale;
    const uint16_t* q;             /* q_dtype [batch][num_q_heads][128] with strides below */
    int64_t q_stride_b, q_stride_h;
    int32_t num_f16_zones;
    HkvF16Zone f16[HKV_MAX_F16_ZONES];
    const uint8_t* pool;           /* INT4 block records (may be NULL if int4_max_len == 0) */
    int64_t pool_blocks;
    const int32_t* block_table;    /* [batch][bt_stride] */
    int32_t bt_stride;
    const int32_t* int4_lens;      /* [batch] device; NULL -> int4_max_len */
    int32_t int4_max_len;
    uint16_t* out;                 /* out_dtype [batch][num_q_heads][128] */
    int64_t out_stride_b, out_stride_h;
    void* workspace;               /* hkv_decode_workspace_bytes(), 256-byte aligned; see below */
    size_t workspace_bytes;
    int32_t splits_hint;           /* 0 = auto */
    const uint8_t* staging;        /* records addressed by negative block ids (may be NULL) */
    int64_t staging_blocks;
    int32_t flags;                 /* HKV_DECODE_* bits */
    /* Optional score output (NULL: none).  Row (b, q head) at scores + b * scores_stride_b
     * + head * scores_stride_h receives the log2-domain score (q.k * sm_scale * log2 e) of
     * every item: INT4 tokens [0, int4_max_len), then each fp16 zone's slots
     * [0, f16[i].max_len) in zone order.  Items past a sequence's lengths are not written.
     * score_stats [batch][num_q_heads][2] receives each row's softmax max and sum, so that
     * exp2(score - max) / sum is the attention probability.  Feeds hkv_attn_weights. */
    float* scores;
    int64_t scores_stride_b, scores_stride_h;
    float* score_stats;
    int32_t q_dtype;               /* F16 or BF16 */
    int32_t out_dtype;             /* F16 or BF16 */
    int32_t* err_flag;             /* device int for HKV_ERR_BIT_*; NULL: the workspace's first word */
} HkvDecodeArgs;

/* Decode flag: every wave of a range takes a fixed subset of the range's blocks, so
 * the output is bitwise reproducible from run to run.  Without it the blocks are
 * handed out to the waves on demand, which keeps all of them busy to the end (faster
 * on long contexts and large batches) and changes the summation order, so outputs
 * can differ in the last bits between runs. */
#define HKV_DECODE_DETERMINISTIC 1
/* Decode flag: combine the ranges of a (sequence, kv head) through device-coherent
 * memory.  Without it, when (batch x kv heads) is a multiple of the XCD count, the
 * combine stays in one XCD's L2, relying on the dispatcher placing workgroup ids of
 * one residue modulo the XCD count on one XCD; every launch checks that with one
 * device-scope atomic per workgroup and reports a violation as HKV_ERR_BIT_PLACEMENT. */
#define HKV_DECODE_AGENT_HANDOFF 2

/* Workspace rules.  The workspace must be zero-filled before its first use.  Its
 * ticket area sits at fixed offsets for up to 1024 split (sequence, kv head) pairs,
 * whatever the launch geometry, and the kernels leave every ticket at a zero count after
 * a launch, so one workspace serves launches of any geometry in any order (graph replays
 * included) with no clearing in between.  A launch that splits more than 1024 pairs
 * (possible only with splits_hint) fails with HKV_ERR_CAPACITY.  Launches that share a
 * workspace must be ordered on one stream. */

size_t hkv_decode_workspace_bytes(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                                  int32_t head_dim, int32_t int4_max_len,
                                  const int32_t* f16_max_lens, int32_t num_f16_zones);

int hkv_decode_attn(const HkvDecodeArgs* args, void* stream);

/*
 * hkv_decode_attn without a workspace: no counterpart in the reference.  It is for
 * callers that cannot allocate device memory -- code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc.  args->workspace must be NULL and
 * workspace_bytes 0; the partial states and tickets live in a library-owned static
 * device array of HKV_DECODE_SCRATCH_BYTES per GPU (held until the process ends), and
 * a geometry whose hkv_decode_workspace_bytes-style need exceeds it fails with
 * HKV_ERR_CAPACITY.  Every call on one GPU shares that array: calls that overlap on one
 * GPU (two streams, two threads) race.  Pass err_flag to see HKV_ERR_BIT_* reports.
 */
#define HKV_DECODE_SCRATCH_BYTES (8u << 20)
int hkv_decode_attn_noalloc(const HkvDecodeArgs* args, void* stream);

/*
 * Chunked-prefill attention (fused_dequant_attn_forward with GQA, kernels/
 * fused_dequant_attn.py:371-435; numerics fused_dequant_attn.py:242-247): every
 * query row of q attends to all tokens of the fp16 zones and of the INT4 pool
 * (dequantized to fp16 exactly as KVCompressor.decompress) and, when chunk_k/chunk_v
 * are given, causally to the chunk's own tokens (row i sees chunk rows 0..i).
 * q, chunk and out are fp16 or bf16 (see "bfloat16 models"); fp32 accumulation on MFMA.
 */
typedef struct HkvPrefillArgs {
    int32_t batch, num_q_heads, num_kv_heads, head_dim, num_queries;
    float sm_scale;
    const uint16_t* q;             /* [batch][num_q_heads][num_queries][128] with strides */
    int64_t q_stride_b, q_stride_h, q_stride_t;
    int32_t num_f16_zones;
    HkvF16Zone f16[HKV_MAX_F16_ZONES];
    const uint8_t* pool;
    int64_t pool_blocks;
    const int32_t* block_table;
    int32_t bt_stride;
    const int32_t* int4_lens;
    int32_t int4_max_len;
    const uint16_t* chunk_k;       /* optional causal chunk [batch][num_kv_heads][num_queries][128] */
    const uint16_t* chunk_v;
    int64_t chunk_stride_b, chunk_stride_h, chunk_stride_t;
    uint16_t* out;                 /* [batch][num_q_heads][num_queries][128] with strides */
    int64_t out_stride_b, out_stride_h, out_stride_t;
    int32_t* err_flag;             /* optional: HKV_ERR_BIT_BLOCK_ID, HKV_ERR_BIT_RANGE */
    const uint8_t* staging;        /* records addressed by negative block ids (may be NULL) */
    int64_t staging_blocks;
    int32_t q_dtype;               /* F16 or BF16 */
    int32_t chunk_dtype;           /* F16 or BF16 */
    int32_t out_dtype;             /* F16 or BF16 */
    /* Needed with a causal chunk, or with INT4 tokens and zone tokens: the chunk's K/V
     * are rewritten here in the zone layout, and the zone kernel leaves each query row's
     * partial softmax state here for the INT4 kernel.  16-byte aligned,
     * hkv_prefill_workspace_bytes() bytes; no zero fill needed.  NULL otherwise. */
    void* workspace;
    size_t workspace_bytes;
} HkvPrefillArgs;

size_t hkv_prefill_workspace_bytes(int32_t batch, int32_t num_q_heads, int32_t num_queries);
int hkv_prefill_attn(const HkvPrefillArgs* args, void* stream);

/*
 * Host-tier prefetcher (replaces DRAMStorageManager's per-tensor pinned dict,
 * dram_storage.py:106-194, and AsyncPrefetcher's side stream, prefetcher.py:33-111).
 * A handle owns a pinned host arena (hipHostMalloc), a side stream created at
 * the default priority, and `num_slots` event sets ("ready", "need", "free").  A
 * slot names one prefetch (typically one per layer); the HBM staging buffers it
 * fills are the caller's.  With two staging buffers reused across layers:
 *   hkv_pf_submit(slot l+1, after slot l-1)  while layer l computes: the copies
 *                                            wait for layer l-1's "free" mark
 *   hkv_pf_wait(slot l+1, compute stream)    before layer l+1's kernel
 *   hkv_pf_mark(slot l+1, compute stream)    after layer l+1's kernel
 * No call blocks the host except hkv_pf_stall_ms and hkv_pf_synchronize.  One
 * handle is used by one host thread.
 */
typedef struct HkvPrefetcher HkvPrefetcher;

typedef struct HkvCopyDesc {
    void* dst;                     /* device destination */
    const void* src;               /* host source (pinned arena memory for an async copy) */
    size_t bytes;
} HkvCopyDesc;

typedef struct HkvPfStats {
    uint64_t bytes_h2d;            /* bytes submitted host -> device */
    uint64_t copies_h2d;           /* copy descriptors submitted */
    uint64_t bytes_d2h;            /* bytes staged out device -> host */
    uint64_t arena_bytes;
} HkvPfStats;

/* arena_bytes may be 0 (no arena); num_slots in [1, 4096]. */
int hkv_pf_create(int32_t device, size_t arena_bytes, int32_t num_slots, HkvPrefetcher** out);
int hkv_pf_destroy(HkvPrefetcher* pf);
/* Host address of arena byte `offset` (NULL if outside the arena). */
void* hkv_pf_host_ptr(HkvPrefetcher* pf, size_t offset);
/* The side stream (hipStream_t as void*), for work the caller adds after a submit. */
void* hkv_pf_stream(HkvPrefetcher* pf);
/* Device -> arena copy of `bytes` at arena offset `host_offset`, on `stream`. */
int hkv_pf_stage_out(HkvPrefetcher* pf, const void* src_device, size_t host_offset, size_t bytes,
                     void* stream);
/* Side stream: wait for slot after_slot's last "free" mark (after_slot < 0: no wait),
 * copy the descriptors, record `slot`'s "ready". */
int hkv_pf_submit(HkvPrefetcher* pf, const HkvCopyDesc* descs, int32_t n, int32_t slot,
                  int32_t after_slot);
/* Side stream: record the slot's "ready" event again (after caller work on hkv_pf_stream). */
int hkv_pf_record(HkvPrefetcher* pf, int32_t slot);
/* Compute stream: record "need" and wait for the slot's "ready". */
int hkv_pf_wait(HkvPrefetcher* pf, int32_t slot, void* compute_stream);
/* Compute stream: record the slot's "free" mark after the kernels that read it. */
int hkv_pf_mark(HkvPrefetcher* pf, int32_t slot, void* compute_stream);
/* Blocks until the slot's events complete; *ms = max(0, ready - need) of its last wait
 * (the time the compute stream sat waiting for the copies); 0 if either is missing. */
int hkv_pf_stall_ms(HkvPrefetcher* pf, int32_t slot, float* ms);
int hkv_pf_stats(HkvPrefetcher* pf, HkvPfStats* out);
int hkv_pf_synchronize(HkvPrefetcher* pf);

/*
 * Block gather (index kernel): dst record i = src record ids[i] for i < n, where
 * an id < 0 names record ~id of `src_staging`.  Used to compact a pool and to
 * collect the records that leave for the host tier into one contiguous run.
 */
int hkv_gather_blocks(const uint8_t* src_pool, int64_t src_blocks, const uint8_t* src_staging,
                      int64_t staging_blocks, const int32_t* ids, int64_t n, int64_t record_bytes,
                      uint8_t* dst, int32_t* err_flag, void* stream);

/*
 * Heavy-hitter scoring (src/policy/heavy_hitter.py:26-101, src/kernels/oracle_triton.py:16-79).
 *
 * hkv_attn_weights: the attention weights of the newest token, averaged over heads,
 * from a decode launch's scores and score_stats (HkvDecodeArgs):
 *   out[b][t] (+)= (1/num_heads) sum_h exp2(scores[b][h][order[t]] - max[b][h]) / sum[b][h]
 * for t < n_items (order NULL: the identity; order[t] < 0: weight 0).  With
 * accumulate != 0 the weights are added to out (HeavyHitterOracle.update); otherwise
 * they replace it.  This is the [seq_len] vector the reference's attention patch hands
 * to the oracle (fused_attention_patch.py:104-107), one row per sequence.
 */
int hkv_attn_weights(const float* scores, int64_t scores_stride_b, int64_t scores_stride_h,
                     const float* score_stats, int32_t batch, int32_t num_heads, int64_t n_items,
                     const int64_t* order, float* out, int64_t out_stride_b, int32_t accumulate,
                     void* stream);

/* compute_block_scores: out[i] = mean of token_scores over block i of block_size tokens
 * (the last block may be partial); ceil(seq_len / block_size) outputs. */
int hkv_block_scores(const float* token_scores, int64_t seq_len, int32_t block_size, float* out, void* stream);

/* HeavyHitterOracle.get_eviction_candidates with scores present: the max_blocks blocks
 * with the lowest mean score, ascending (equal means: lower index first), never one of
 * the first ceil(sink_tokens / block_size) or last ceil(local_window / block_size)
 * blocks.  *num_out (set on the host, no sync) = min(max_blocks, unprotected blocks),
 * 0 when seq_len <= sink_tokens + local_window; out receives that many int64 block
 * indices.  The workspace is hkv_eviction_workspace_bytes(...) bytes, 8-byte aligned. */
size_t hkv_eviction_workspace_bytes(int64_t seq_len, int32_t block_size, int32_t sink_tokens,
                                    int32_t local_window, int32_t max_blocks);
int hkv_eviction_candidates(const float* token_scores, int64_t seq_len, int32_t block_size,
                            int32_t sink_tokens, int32_t local_window, int32_t max_blocks, int64_t* out,
                            int32_t* num_out, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HETEROKV_H */
