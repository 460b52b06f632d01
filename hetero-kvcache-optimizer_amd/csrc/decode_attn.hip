// Split-K INT4/fp16 decode attention for gfx950 (one query token per sequence).
//
// Math (fused_dequant_attn.py:326-331,388-390 with GQA as HF repeat_kv):
//   out[b, qh] = softmax_t( q[b,qh] . K[b, qh/n_rep, t] * sm_scale ) . V[b, qh/n_rep, t]
// over every valid token t of the fp16 zones and of the INT4 pool, where an
// INT4 value dequantizes to (code - zp) * scale.
//
// Mapping.  One wavefront handles one kv head and all n_rep (<=16) query heads
// of its GQA group, so every K/V byte is read once.  Per 16-token tile:
//   QK : 4 x v_mfma_f32_16x16x32_f16, A = K tile (rows = tokens, k = dims),
//        B = q^T (cols = heads).  Lane (c, g) = lane%16, lane/16 ends up with the
//        scores of head c for tokens 4g..4g+3.
//   PV : 8 x v_mfma_f32_16x16x16_f16, A = V^T (rows = 16 dims, k = tokens),
//        B = P^T.  The QK result layout is exactly the PV B-operand layout, so no
//        shuffle is needed between the two products.
// INT4 codes become fp16 operands with one AND-OR per two codes: a nibble n
// placed in the mantissa of 0x6400 is the fp16 value 1024 + n; subtracting the
// pair (1024 + zp) leaves the exact integer code - zp.  The K scale multiplies
// the score, the V scale multiplies the probability, both in fp32.
//
// Work split.  Every (sequence, kv head) pair is cut into S byte-balanced
// ranges (S chosen so that S x pairs is about one workgroup per CU); a range is
// a run of items in the order [INT4 blocks | fp16 zone tiles], and each of the
// 8 waves of the workgroup takes a contiguous piece of it.  Waves merge through
// LDS, workgroups through a workspace: the last workgroup of a pair to finish
// (atomic ticket after a release fence) merges the S partial states with
// independent loads and writes the output, so the whole op is one launch.  When every
// range of a pair is resident (the grid fits the CUs), each range instead waits
// (bounded) for the pair's arrival count and merges one slice of the output, in the
// XCD's L2 with the XCD-local hand-off and through memory otherwise (the kernel's tail
// describes both).
// Workgroup ids interleave the pairs so that all ranges of a pair land on one
// XCD: dispatch is round-robin over XCDs by workgroup id (the XCD that takes
// workgroup 0 rotates from launch to launch, so only the id modulo the XCD count
// is fixed).  When every range of a pair shares an XCD (pairs a multiple of the
// XCD count), the hand-off stays in that XCD's L2: plain stores, an L2 atomic
// ticket and group-scope loads.  Otherwise (or with HKV_DECODE_AGENT_HANDOFF) it
// goes through memory with agent-scope (sc1) accesses.  The placement is checked
// on every launch: each workgroup ORs its XCD bit into a device-scope mask of its
// pair when its streaming ends and reads the old mask back at its ticket; a foreign
// bit (or a ticket beyond the range count, left by such a launch) sets
// HKV_ERR_BIT_PLACEMENT.  The merging workgroup clears the mask.
#include "hkv_internal.h"
#include "nibble_decode.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>

namespace hkv {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

constexpr int kWaves = 8;                 // waves per workgroup
constexpr int kThreads = kWaves * 64;
constexpr int kPartStride = kHeadDim + 4;  // o[128], m, l, 2 pad (16-byte rows)
static_assert((kHeadDim * 4) % 8 == 0 && (kPartStride * 4) % 16 == 0, "m, l load as one aligned 8-byte pair");
#ifndef HKV_DECODE_PREFETCH
#define HKV_DECODE_PREFETCH 2
#endif
constexpr int kPrefetch = HKV_DECODE_PREFETCH;  // INT4 block pairs in flight per wave
// fp16 zone tiles in flight per wave: one (an 8 KB tile per wave is already as much in
// flight as two INT4 block pairs; two tiles measured ~1% slower on the 32K decode)
#ifndef HKV_DECODE_F16_DEPTH
#define HKV_DECODE_F16_DEPTH 1
#endif
constexpr int kF16Depth = HKV_DECODE_F16_DEPTH;
constexpr int kMaxSplits = 64;
constexpr int kLineWords = 64;           // ints per 256-byte hand-off line
// Slice merge: the pair's arrival word holds the arrivals of the current launch in bits
// 0-15, a generation in bits 16-29 that the last arrival advances (clearing the count),
// and a bit set by a range that stopped waiting.
constexpr int kArrivedMask = 0xffff;
constexpr int kGenOne = 1 << 16;
constexpr int kGenMask = 0x3fff << 16;
constexpr int kGoneBit = 1 << 30;
// Bound of a range's wait in the slice merge: 25 us of the 100 MHz constant clock.  Waits
// on the 32K decode are under ~4 us; a wait that runs out only hands the whole merge to
// the last arrival (~3 us), and a short bound limits what two decodes running at once on
// one GPU (neither kernel's ranges all resident) cost each other.
constexpr unsigned long long kMergeWaitTicks = 2500;
// INT4 tokens, and fp16 tokens over all zones, per sequence: 2^22 items of 16 tokens
// keep the range arithmetic in 32 bits.
constexpr int kMaxZoneTokens = 1 << 26;
constexpr int kIdWindow = 1024;           // INT4 block ids staged in LDS at a time
constexpr int kIdPerThread = kIdWindow / kThreads;
static_assert(kIdWindow % kThreads == 0, "whole id entries per thread");
constexpr float kLog2e = 1.4426950408889634f;

// Timeline build (HKV_DECODE_TIMELINE, libheterokv_timeline.so, for measurement only):
// every wave records the 100 MHz constant clock at the phase boundaries below and lane 0
// writes them, with the wave's XCD and range, as eight words at exit.
//   [0] start  [1] first id window in LDS  [2] streaming done  [3] partial state stored
//   [4] ticket known  [5] final merge loads done  [6] output written  [7] info
//   [8] first unit's data consumed (end of the first step)
//   [9] fp16 prologue loads arrived, [10] INT4 prologue loads arrived (only with
//       HKV_TIMELINE_WAITS=1 in the environment: the wave then waits for both slots before
//       its first step, which the measured kernel does not)
#ifdef HKV_DECODE_TIMELINE
constexpr int kTlMaxWaves = 16384;
constexpr int kTlWords = 16;
#define TL_MARK(i) (tl_t[i] = __builtin_amdgcn_s_memrealtime())
#define TL_FLUSH(info)                                                                              \
    do {                                                                                            \
        if (lane == 0 && p.tl && blockIdx.x * kWaves + wave < kTlMaxWaves) {                        \
            unsigned long long* _d = p.tl + ((size_t)blockIdx.x * kWaves + wave) * kTlWords;         \
            for (int _i = 0; _i < 7; ++_i) _d[_i] = tl_t[_i];                                       \
            _d[7] = (info);                                                                         \
            _d[8] = tl_t[7];                                                                        \
            _d[9] = tl_w[0];                                                                        \
            _d[10] = tl_w[1];                                                                       \
        }                                                                                           \
    } while (0)
#else
#define TL_MARK(i) ((void)0)
#define TL_FLUSH(info) ((void)0)
#endif
// Bytes one kv head reads per item (the weights that balance the ranges).
constexpr int64_t kInt4ItemBytes = kBlockTokens * (kHeadDim / 2 + 5) * 2;   // 2208
constexpr int64_t kF16ItemBytes = kBlockTokens * kHeadDim * 2 * 2;           // 8192
// Balance weight of an INT4 block against an fp16 tile (8192): its 2208 bytes plus the
// block-id indirection (INT4-only ranges start streaming only when their first ids are in
// LDS, ~2.5 us into the 32K decode) and the nibble decode; fitted on the 32K decode,
// where 3300 gives 24 INT4-only and 8 fp16-only ranges per (sequence, kv head).
#ifndef HKV_INT4_COST
#define HKV_INT4_COST 3300
#endif
constexpr int64_t kInt4Cost = HKV_INT4_COST;

struct ZoneP {
    const uint16_t* k;
    const uint16_t* v;
    int cap;
    int max_len;
    const int32_t* lens;
};

struct DecodeParams {
    int B, Hkv, nrep;
    float scale_log2;
    int q_bf16, out_bf16;     // q / out dtype is bfloat16 (else fp16)
    const uint16_t* q;
    int64_t q_sb, q_sh;
    int nz;
    ZoneP z[HKV_MAX_F16_ZONES];
    const uint8_t* pool;
    int64_t pool_blocks;
    const uint8_t* staging;   // records addressed by negative block ids
    int64_t staging_blocks;
    int fallback_id;          // id substituted for an out-of-range one (a valid record)
    const int32_t* bt;
    int bt_stride;
    const int32_t* int4_lens;
    int int4_max_len;
    uint16_t* out;
    int64_t o_sb, o_sh;
    int* err;
    // Hand-off words, one 256-byte line (kLineWords ints) per pair and kind, so that the
    // atomics of different pairs do not queue at one cache line:
    int* counters;            // agent-scope ticket: word 0 of the pair's agent line
    unsigned* owners;         // agent-scope XCD mask (placement check): word 1 of the same line
    int* counters_l2;         // XCD-local line: [0] slice-merge arrivals, [1] ticket
    float* partials;
    int max_splits;
    int64_t part_pair_stride;  // floats between the partial blocks of consecutive pairs (256-byte multiple)
    int xcc_local;             // 1: all ranges of a pair run on one XCD (see above)
    int nxcc;                  // XCDs the dispatcher round-robins over
    int coop;                  // 1: slice merge by every range of a pair (see the kernel's tail)
    int slice_outputs;         // slice merge: outputs per slice, ceil(n_rep * 128 / ranges)
    unsigned long long merge_wait;   // slice merge: constant-clock ticks a range waits for the others
    // optional score output (kScores): row (b, q head) holds the log2-domain score of
    // every item [INT4 tokens | zone 0 | zone 1 | zone 2]; zone z starts at sc_zone[z]
    float* scores;
    int64_t sc_sb, sc_sh;
    int sc_zone[HKV_MAX_F16_ZONES];
    float* stats;              // [B][Hq][2]: the softmax max and sum of each row
#ifdef HKV_DECODE_TIMELINE
    unsigned long long* tl;    // per-wave phase timestamps (timeline build only)
    int tl_waits;              // 1: also wait for the prologue loads and stamp their arrival
#endif
};

// Partial states cross workgroups (and XCDs) through agent-scope relaxed atomic
// loads and stores: those are coherent at the device level by themselves, so the
// hand-off needs no L2 writeback or invalidate.  Ordering comes from waiting for
// the stores to complete (s_waitcnt) before the workgroup barrier and the ticket
// increment, and from the ticket's return value before the loads.
__device__ __forceinline__ void st_agent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Group-scope (sc0) loads through a buffer resource.  They can be served from this
// CU's L1, which every kernel starts with empty; the merging workgroup reads the pair's
// partial states only after its ticket shows them all final and has read none of their
// lines before, so every line it loads comes from the XCD's L2 in its final state.
__device__ __forceinline__ float ld_l2(__amdgpu_buffer_rsrc_t r, int byte_off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, 1));
}
__device__ __forceinline__ f4 ld_l2_f4(__amdgpu_buffer_rsrc_t r, int byte_off) {
    return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 1));
}
__device__ __forceinline__ f2 ld_l2_f2(__amdgpu_buffer_rsrc_t r, int byte_off) {
    return __builtin_bit_cast(f2, __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, 1));
}
// The same loads at device scope (sc1: coherent with other XCDs' device-scope stores).
constexpr int kAuxL2 = 1, kAuxDevice = 16;

// Slice merge: the (m, l) pair and output d of eight partial states (splits q + base,
// q + base + 4, ...), with loads of cache policy kAux.
template <int kAux>
__device__ __forceinline__ void load_slice8(__amdgpu_buffer_rsrc_t prs, int q, int base, int nsplit, int nrep, int hd,
                                            int d, float (&ms)[8], float (&ls)[8], float (&os)[8]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int sj = q + base + 4 * j;
        const int off = min(sj, nsplit - 1) * (nrep * kPartStride) + hd * kPartStride;
        const f2 ml = __builtin_bit_cast(f2, __builtin_amdgcn_raw_buffer_load_b64(prs, (off + kHeadDim) * 4, 0, kAux));
        ms[j] = sj < nsplit ? ml.x : -INFINITY;
        ls[j] = ml.y;
        os[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(prs, (off + d) * 4, 0, kAux));
    }
}

// Slice merge: a range's arrival (one thread), with atomics of scope kScope on the pair's
// arrival word.  Returns 0 (the wait ran out: leave), 1 (merge this range's slice) or 2
// (merge every slice: the last arrival, after some range stopped waiting).  The last
// arrival resets the word at once (generation advanced, count cleared, one store) and
// clears `mask` (the placement check's, or null); *overrun reports a count at or past the
// range count at arrival.
template <int kScope>
__device__ __forceinline__ int slice_arrival(int* arrived, int nsplit, unsigned long long merge_wait,
                                             unsigned* mask, bool* overrun) {
    const int old = __hip_atomic_fetch_add(arrived, 1, __ATOMIC_RELAXED, kScope);
    const int gen = old & kGenMask;
    // a count at or past the range count is what a launch whose ranges did not share one
    // L2 leaves behind: reported, and the word starts a new generation
    *overrun = (old & kArrivedMask) >= nsplit;
    if ((old & kArrivedMask) == nsplit - 1 || *overrun) {
        __hip_atomic_store(arrived, (gen + kGenOne) & kGenMask, __ATOMIC_RELAXED, kScope);
        // every range has arrived, so every mask update is done
        if (mask) __hip_atomic_store(mask, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return (old & kGoneBit) ? 2 : 1;
    }
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    for (;;) {
        // an OR of zero, performed where the others' arrivals are (a load could be served
        // from this CU's L1); the zero is opaque so that the compiler keeps the atomic
        int zero;
        asm volatile("s_mov_b32 %0, 0" : "=s"(zero));
        int v = __hip_atomic_fetch_or(arrived, zero, __ATOMIC_RELAXED, kScope);
        if ((v & kGenMask) != gen || (v & kArrivedMask) >= nsplit) return 1;
        if (__builtin_amdgcn_s_memrealtime() - t0 > merge_wait) {
            // stop waiting: set kGoneBit in this generation's word while its count is
            // short (then the last arrival sees it), unless the count completed meanwhile
            for (;;) {
                if ((v & kGenMask) != gen || (v & kArrivedMask) >= nsplit) return 1;
                if (__hip_atomic_compare_exchange_strong(arrived, &v, v | kGoneBit, __ATOMIC_RELAXED,
                                                         __ATOMIC_RELAXED, kScope))
                    return 0;
            }
        }
        __builtin_amdgcn_s_sleep(2);
    }
}

__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }

// The value of lane (lane ^ x) of the same quad, x = 1 or 2 (DPP quad_perm [1,0,3,2] or
// [2,3,0,1]); every lane of the quad must be active.
__device__ __forceinline__ float quad_xor(float v, int x) {
    const int i = __builtin_bit_cast(int, v);
    return __builtin_bit_cast(float, x == 1 ? __builtin_amdgcn_mov_dpp(i, 0xB1, 0xF, 0xF, false)
                                            : __builtin_amdgcn_mov_dpp(i, 0x4E, 0xF, 0xF, false));
}

struct Int4Blk {
    u4 k;         // K codes of token (lane%16), dims 32g..32g+31
    u4 v;         // V codes: tokens 4g..4g+3, dims c+16n (n=0..7)
    f4 ks;        // K scales of tokens 4g..4g+3
    f4 vs;        // V scales of tokens 4g..4g+3
    uint32_t kz;  // K zero points of tokens 4(c/4)..+3 (bytes); token c's is byte c%4
    uint32_t vz;  // V zero points of tokens 4g..4g+3 (bytes)
};

struct F16Tile {
    u4 k[4];      // K row of token (lane%16), dims 32g + 8j .. +8
    u4 v[4];      // V^T tile: halves [n][i] for tokens 4g+i, dims c+16n
};

// Loads go through a buffer resource per block whose size is 0 for a slot with
// nothing to read: such a load returns zeros without a memory access, so the
// refills issued past the end of a range cost no traffic and no wait.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
__device__ __forceinline__ u4 ld16(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ uint32_t ld4(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

// `phys` is the (already validated, wave-uniform) block id: >= 0 a pool record,
// < 0 staging record ~phys.  Every load of a block is issued back to back so
// several blocks stay in flight.
__device__ __forceinline__ void load_int4(const DecodeParams& p, int h, int phys, bool valid, int c, int g,
                                          Int4Blk& d) {
    const int64_t rb = (int64_t)p.Hkv * kHeadPartBytes;
    const uint8_t* part = (phys >= 0 ? p.pool + (int64_t)phys * rb : p.staging + (int64_t)(~phys) * rb) +
                          RecordLayout::part(h);
    const __amdgpu_buffer_rsrc_t r = rsrc(part, valid ? kHeadPartBytes : 0);
    d.k = ld16(r, kPartKc + c * kCodeRowBytes + g * 16);
    d.v = ld16(r, kPartVc + (g * 16 + c) * 16);
    d.ks = __builtin_bit_cast(f4, ld16(r, kPartKs + g * 16));
    d.vs = __builtin_bit_cast(f4, ld16(r, kPartVs + g * 16));
    d.kz = ld4(r, kPartKz + (c & ~3));   // a full word: no byte value lives across the loop
    d.vz = ld4(r, kPartVz + g * 4);
}

// Block ids of logical blocks [lb0, lb0 + n) of sequence b, padded to an even
// count by repeating the last one: thread t requests entries t, t + kThreads.
__device__ __forceinline__ void fetch_block_ids(const DecodeParams& p, int b, int lb0, int n, int (&r)[kIdPerThread]) {
    const int n2 = (n + 1) & ~1;
#pragma unroll
    for (int j = 0; j < kIdPerThread; ++j) {
        const int i = threadIdx.x + j * kThreads;
        r[j] = i < n2 ? p.bt[(int64_t)b * p.bt_stride + lb0 + min(i, n - 1)] : 0;
    }
}

// Writes the fetched ids to LDS, with out-of-range ids replaced by a valid one and
// reported through p.err.
__device__ __forceinline__ void commit_block_ids(const DecodeParams& p, int n, const int (&r)[kIdPerThread], int* sm) {
    const int n2 = (n + 1) & ~1;
    bool bad_any = false;
#pragma unroll
    for (int j = 0; j < kIdPerThread; ++j) {
        const int i = threadIdx.x + j * kThreads;
        if (i < n2) {
            int id = r[j];
            const bool bad = id >= 0 ? (int64_t)id >= p.pool_blocks : (int64_t)(~id) >= p.staging_blocks;
            if (bad) {
                id = p.fallback_id;
                bad_any = true;
            }
            sm[i] = id;
        }
    }
    if (__ballot(bad_any) && (threadIdx.x & 63) == 0 && p.err) atomicOr(p.err, 1);
}

// Next unit of a workgroup counter, wave-uniform.
__device__ __forceinline__ int grab(int* ctr) {
    int v = 0;
    if ((threadIdx.x & 63) == 0) v = atomicAdd(ctr, 1);
    return __builtin_amdgcn_readfirstlane(v);
}

__device__ __forceinline__ u2 read_pair_ids(const int* sm, int pair) { return *(const u2*)(sm + 2 * pair); }

__device__ __forceinline__ void load_f16(const ZoneP& z, int64_t bh, int tile, bool valid, int c, int g, F16Tile& d) {
    constexpr int kTileBytes = kBlockTokens * kHeadDim * 2;   // 4 KB of K rows, 4 KB of V^T
    const __amdgpu_buffer_rsrc_t rk = rsrc(z.k + (bh * z.cap + (int64_t)tile * kBlockTokens) * kHeadDim, valid ? kTileBytes : 0);
    const __amdgpu_buffer_rsrc_t rv =
        rsrc(z.v + (bh * (z.cap / kBlockTokens) + tile) * (kBlockTokens * kHeadDim), valid ? kTileBytes : 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        d.k[j] = ld16(rk, (c * kHeadDim + 32 * g + 8 * j) * 2);
        d.v[j] = ld16(rv, ((g * 16 + c) * 32 + 8 * j) * 2);
    }
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Online-softmax update for N log2-domain scores per lane (-inf = masked).  The
// running max m is kept equal on the 4 lanes of a head; the cross-lane reduction
// and the rescale of acc/l run only when some lane sees a score above it, so the
// common step has no shuffle at all.  Returns exp2(s - m) in pr.
template <int N>
__device__ __forceinline__ void softmax_update(const float (&s)[N], f4 (&acc)[8], float& m, float& l,
                                               float (&pr)[N]) {
    float mt = s[0];
#pragma unroll
    for (int i = 1; i < N; ++i) mt = fmaxf(mt, s[i]);
    if (__ballot(mt > m)) {
        mt = fmaxf(mt, __shfl_xor(mt, 16));
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float m_new = fmaxf(m, mt);
        const float alpha = (m_new > m) ? fast_exp2(m - m_new) : 1.0f;
#pragma unroll
        for (int n = 0; n < 8; ++n) acc[n] *= alpha;
        l *= alpha;
        m = m_new;
    }
    const float msafe = (m == -INFINITY) ? 0.0f : m;
#pragma unroll
    for (int v = 0; v < N; ++v) {
        pr[v] = fast_exp2(s[v] - msafe);
        l += pr[v];
    }
}

// K operand of one packed word (dims 8j..8j+7 of token lane%16): exact code - zp.
__device__ __forceinline__ h8 k_operand(uint32_t w, h2 kz1024, h2 kz64) {
    const NibPairs a = unpack_word(w, kz1024, kz64);
    return h8{a.p0[0], a.p0[1], a.p1[0], a.p1[1], a.p2[0], a.p2[1], a.p3[0], a.p3[1]};
}

// Two INT4 blocks (32 tokens) per step: the two QK chains interleave, and one
// 16x16x32 MFMA per 16 dims does PV for both blocks (k slots 0..3 = block A
// tokens 4g..4g+3, slots 4..7 = block B tokens 4g..4g+3).
// With kScores, lanes of a valid head store the pair's eight scores (4 consecutive
// tokens of each block) at sA / sB.
template <bool kScores = false>
__device__ __forceinline__ void step_int4_pair(const Int4Blk& A, const Int4Blk& B, int nA, int nB, int g, int kzsh,
                                               const h8 (&qf)[4], float scale_log2, f4 (&acc)[8], float& m,
                                               float& l, bool store = false, float* sA = nullptr,
                                               float* sB = nullptr) {
    const uint32_t kza = __builtin_amdgcn_ubfe(A.kz, kzsh, 8), kzb = __builtin_amdgcn_ubfe(B.kz, kzsh, 8);
    const h2 kA1024 = zp1024(kza, kza), kA64 = zp64(kza, kza);
    const h2 kB1024 = zp1024(kzb, kzb), kB64 = zp64(kzb, kzb);
    const uint32_t kwA[4] = {A.k.x, A.k.y, A.k.z, A.k.w};
    const uint32_t kwB[4] = {B.k.x, B.k.y, B.k.z, B.k.w};
    f4 SA = {0.f, 0.f, 0.f, 0.f}, SB = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        SA = __builtin_amdgcn_mfma_f32_16x16x32_f16(k_operand(kwA[j], kA1024, kA64), qf[j], SA, 0, 0, 0);
        SB = __builtin_amdgcn_mfma_f32_16x16x32_f16(k_operand(kwB[j], kB1024, kB64), qf[j], SB, 0, 0, 0);
    }
    // V operands are unpacked while the QK products are in flight (they do not depend
    // on the scores).  V zero points of tokens 4g..4g+3: pairs (x0,x1), (x4,x5) are
    // tokens 4g, 4g+1; pairs (x2,x3), (x6,x7) are tokens 4g+2, 4g+3.
    const h2 zA01 = zp1024(A.vz & 0xffu, (A.vz >> 8) & 0xffu), zA23 = zp64((A.vz >> 16) & 0xffu, A.vz >> 24);
    const h2 zB01 = zp1024(B.vz & 0xffu, (B.vz >> 8) & 0xffu), zB23 = zp64((B.vz >> 16) & 0xffu, B.vz >> 24);
    const uint32_t vwA[4] = {A.v.x, A.v.y, A.v.z, A.v.w};
    const uint32_t vwB[4] = {B.v.x, B.v.y, B.v.z, B.v.w};
    h8 V0[4], V1[4];
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) {
        const NibPairs a = unpack_word(vwA[mm], zA01, zA23);
        const NibPairs bq = unpack_word(vwB[mm], zB01, zB23);
        V0[mm] = h8{a.p0[0], a.p0[1], a.p1[0], a.p1[1], bq.p0[0], bq.p0[1], bq.p1[0], bq.p1[1]};   // dims c + 32mm
        V1[mm] = h8{a.p2[0], a.p2[1], a.p3[0], a.p3[1], bq.p2[0], bq.p2[1], bq.p3[0], bq.p3[1]};   // dims c + 32mm + 16
    }
    float s[8];
    const bool full = nA >= kBlockTokens && nB >= kBlockTokens;
    if (full) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            s[v] = SA[v] * (A.ks[v] * scale_log2);
            s[4 + v] = SB[v] * (B.ks[v] * scale_log2);
        }
    } else {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            s[v] = (4 * g + v < nA) ? SA[v] * (A.ks[v] * scale_log2) : -INFINITY;
            s[4 + v] = (4 * g + v < nB) ? SB[v] * (B.ks[v] * scale_log2) : -INFINITY;
        }
    }
    if constexpr (kScores) {
        if (store) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                if (4 * g + v < nA) sA[v] = s[v];
                if (4 * g + v < nB) sB[v] = s[4 + v];
            }
        }
    }
    float pr[8];
    softmax_update<8>(s, acc, m, l, pr);
    h8 P;
    if (full) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            P[v] = (_Float16)(pr[v] * A.vs[v]);
            P[4 + v] = (_Float16)(pr[4 + v] * B.vs[v]);
        }
    } else {
        // masked tokens get exactly 0 (their scale may be anything)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            P[v] = (_Float16)((4 * g + v < nA) ? pr[v] * A.vs[v] : 0.0f);
            P[4 + v] = (_Float16)((4 * g + v < nB) ? pr[4 + v] * B.vs[v] : 0.0f);
        }
    }
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) {
        acc[2 * mm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(V0[mm], P, acc[2 * mm], 0, 0, 0);
        acc[2 * mm + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(V1[mm], P, acc[2 * mm + 1], 0, 0, 0);
    }
}

template <bool kScores = false>
__device__ __forceinline__ void step_f16(F16Tile& d, int nvalid, int g, const h8 (&qf)[4],
                                         float scale_log2, f4 (&acc)[8], float& m, float& l, bool store = false,
                                         float* sp = nullptr) {
    f4 S = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) S = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, d.k[j]), qf[j], S, 0, 0, 0);
    float s[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) s[v] = (4 * g + v < nvalid) ? S[v] * scale_log2 : -INFINITY;
    if constexpr (kScores) {
        if (store) {
#pragma unroll
            for (int v = 0; v < 4; ++v)
                if (4 * g + v < nvalid) sp[v] = s[v];
        }
    }
    float pr[4];
    softmax_update<4>(s, acc, m, l, pr);
    h4 P;
#pragma unroll
    for (int v = 0; v < 4; ++v) P[v] = (_Float16)((4 * g + v < nvalid) ? pr[v] : 0.0f);
    if (nvalid < kBlockTokens) {
        // Slots past the zone length may hold anything; clear them so 0 * V stays 0.
        const uint32_t m01 = (4 * g + 0 < nvalid ? 0x0000FFFFu : 0u) | (4 * g + 1 < nvalid ? 0xFFFF0000u : 0u);
        const uint32_t m23 = (4 * g + 2 < nvalid ? 0x0000FFFFu : 0u) | (4 * g + 3 < nvalid ? 0xFFFF0000u : 0u);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            d.v[j].x &= m01;
            d.v[j].y &= m23;
            d.v[j].z &= m01;
            d.v[j].w &= m23;
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const h4 A0 = __builtin_bit_cast(h4, u2{d.v[j].x, d.v[j].y});
        const h4 A1 = __builtin_bit_cast(h4, u2{d.v[j].z, d.v[j].w});
        acc[2 * j] = __builtin_amdgcn_mfma_f32_16x16x16f16(A0, P, acc[2 * j], 0, 0, 0);
        acc[2 * j + 1] = __builtin_amdgcn_mfma_f32_16x16x16f16(A1, P, acc[2 * j + 1], 0, 0, 0);
    }
}

// Tile counts of the fp16 zones of one sequence; tiles are numbered over zones
// 0, 1, 2 in order.
struct ZoneTiles {
    int nt[HKV_MAX_F16_ZONES];
    __device__ int total() const { return nt[0] + nt[1] + nt[2]; }
};

// Zone, valid length and tile of fp16 tile t counted over zones 0, 1, 2 in order.
static_assert(HKV_MAX_F16_ZONES == 3, "locate_tile walks three zones");
__device__ __forceinline__ void locate_tile(const DecodeParams& p, const ZoneTiles& im, const int (&lenz)[HKV_MAX_F16_ZONES],
                                            int t, ZoneP& z, int& len, int& tile) {
    z = p.z[0];
    len = lenz[0];
    if (t >= im.nt[0]) {
        t -= im.nt[0];
        z = p.z[1];
        len = lenz[1];
        if (t >= im.nt[1]) {
            t -= im.nt[1];
            z = p.z[2];
            len = lenz[2];
        }
    }
    tile = t;
}

// kDynamic: the workgroup's units are handed to its waves from LDS counters, so
// every wave stays busy until the workgroup's share is done (the two waves sharing
// a SIMD do not progress at the same rate: the older one wins issue).  The result
// then depends on which wave took which unit, in the last bits.  Otherwise wave w
// takes units w, w + kWaves, ... and the result is bitwise reproducible.
// Zone and tile of fp16 tile t counted over zones 0, 1, 2 in order.
__device__ __forceinline__ void locate_zone(const ZoneTiles& im, int t, int& zi, int& tile) {
    zi = 0;
    if (t >= im.nt[0]) {
        t -= im.nt[0];
        zi = 1;
        if (t >= im.nt[1]) {
            t -= im.nt[1];
            zi = 2;
        }
    }
    tile = t;
}

template <bool kDynamic>
__device__ __forceinline__ int next_unit(int* ctr, int& seq) {
    if constexpr (kDynamic) {
        return grab(ctr);
    } else {
        const int u = seq;
        seq += kWaves;
        return u;
    }
}

// Splits that stream only INT4 blocks when a pair's ranges are made of one kind
// each, or 0 when every range takes the same share of both kinds.  Ranges of one
// kind avoid a second pipeline start inside a range; they are used when the
// rounding of nsplit into two groups costs at most ~6% over an even share.  Costs:
// an INT4 block counts kInt4Cost bytes (its 2208 bytes, plus the block-id
// indirection and the nibble decode), an fp16 tile its 8192 bytes.
//
// Every workgroup computes the plan before its first load, so it uses float costs
// and 32-bit range bounds: a 64-bit division expands to ~130 instructions.
__device__ __forceinline__ int int4_splits(int nb4, int ntf, int nsplit) {
    if (nb4 == 0 || ntf == 0 || nsplit < 2) return 0;
    const float c4 = (float)nb4 * (float)kInt4Cost, cf = (float)ntf * (float)kF16ItemBytes, ct = c4 + cf;
    int s4 = (int)(c4 * (float)nsplit / ct + 0.5f);
    s4 = min(max(s4, 1), nsplit - 1);
    const float worst = fmaxf(c4 / (float)s4, cf / (float)(nsplit - s4));
    return worst * 16.0f <= ct / (float)nsplit * 17.0f ? s4 : 0;
}

// floor(n i / d) for the range bounds: n < 2^22 items (host-checked), i <= d <= 64,
// so the product fits 32 bits and the division is exact.
__device__ __forceinline__ int part_point(int n, int i, int d) {
    return (int)(((uint32_t)n * (uint32_t)i) / (uint32_t)d);
}

// Partial states s0 + j K (j < 8) of head hd for the final merge: m, l and
// float4 d4 of o.  Splits past the end read the last split again and get
// m = -inf, so that every load is issued unconditionally.  kL2: XCD-local
// hand-off (group-scope buffer loads), else agent-scope loads.
template <bool kL2>
__device__ __forceinline__ void load_partials(__amdgpu_buffer_rsrc_t prs, const float* parts, int s0, int K,
                                              int nsplit, int nrep, int hd, int d4, float* ms, float* ls, f4* os) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int sj = s0 + j * K;
        const int off = min(sj, nsplit - 1) * (nrep * kPartStride) + hd * kPartStride;
        if constexpr (kL2) {
            const f2 ml = ld_l2_f2(prs, (off + kHeadDim) * 4);   // m, l side by side (8-byte aligned)
            ms[j] = sj < nsplit ? ml.x : -INFINITY;
            ls[j] = ml.y;
            os[j] = ld_l2_f4(prs, (off + d4) * 4);
        } else {
            const float* ps = parts + off;
            ms[j] = sj < nsplit ? ld_agent(ps + kHeadDim) : -INFINITY;
            ls[j] = ld_agent(ps + kHeadDim + 1);
            os[j] = f4{ld_agent(ps + d4), ld_agent(ps + d4 + 1), ld_agent(ps + d4 + 2), ld_agent(ps + d4 + 3)};
        }
    }
}

// kL2: the XCD-local hand-off (p.xcc_local), a template parameter so that each hand-off's
// kernel carries only its own tail code.
template <bool kDynamic, bool kScores, bool kL2>
__global__ __launch_bounds__(kThreads) void decode_attn_kernel(DecodeParams p) {
    touch_kernel_args(p);   // the range plan below reads the arguments in a dependent chain
    const int BH = p.B * p.Hkv;
    const int bh = blockIdx.x % BH;
    const int split = blockIdx.x / BH;
    const int nsplit = p.max_splits;
    const int b = bh / p.Hkv, h = bh % p.Hkv;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: buffer resources stay scalar
    const int c = lane & 15, g = lane >> 4;
    const int kzsh = 8 * (c & 3);
    const int nrep = p.nrep;
    unsigned owner_old = 0u, owner_bit = 0u;   // placement check (below, after the streaming)
#ifdef HKV_DECODE_TIMELINE
    unsigned long long tl_t[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    unsigned long long tl_w[2] = {0, 0};
    TL_MARK(0);
#endif

    // per-sequence lengths: wave-uniform scalar loads (the kernel does not write them)
    const int len4 = p.int4_lens ? min(max(load_uniform_i32(p.int4_lens, b), 0), p.int4_max_len) : p.int4_max_len;
    int lenz[HKV_MAX_F16_ZONES];
    ZoneTiles zt;
#pragma unroll
    for (int zi = 0; zi < HKV_MAX_F16_ZONES; ++zi) {
        lenz[zi] = 0;
        if (zi < p.nz)
            lenz[zi] = p.z[zi].lens ? min(max(load_uniform_i32(p.z[zi].lens, b), 0), p.z[zi].max_len) : p.z[zi].max_len;
        zt.nt[zi] = (lenz[zi] + kBlockTokens - 1) / kBlockTokens;
    }
    // Range `split` of this (sequence, kv head): INT4 blocks [a0, a1) and fp16
    // tiles [f0, f0 + nf).
    const int nb4 = (len4 + kBlockTokens - 1) / kBlockTokens, ntf = zt.total();
    int a0, a1, f0, nf;
    {
        const int s4 = int4_splits(nb4, ntf, nsplit);
        if (s4 > 0 && s4 < nsplit) {
            // splits [0, s4) stream INT4 blocks only, the others fp16 tiles only
            const bool is4 = split < s4;
            const int si = is4 ? split : split - s4, sn = is4 ? s4 : nsplit - s4, n = is4 ? nb4 : ntf;
            const int u0 = part_point(n, si, sn), u1 = part_point(n, si + 1, sn);
            a0 = is4 ? u0 : 0;
            a1 = is4 ? u1 : 0;
            f0 = is4 ? 0 : u0;
            nf = is4 ? 0 : u1 - u0;
        } else {
            // every split takes the same share of both kinds
            a0 = part_point(nb4, split, nsplit);
            a1 = part_point(nb4, split + 1, nsplit);
            f0 = part_point(ntf, split, nsplit);
            nf = part_point(ntf, split + 1, nsplit) - f0;
        }
    }

    // The block ids of the first INT4 window are requested before anything else;
    // the fp16 tiles are streamed while they are on their way.
    int idr[kIdPerThread];
    fetch_block_ids(p, b, a0, min(kIdWindow, a1 - a0), idr);
    __builtin_amdgcn_sched_barrier(0);

    // q fragments: lane (c, g) holds q[head c][32g + 8j .. +8] for step j.
    h8 qf[4];
    {
        const bool has = c < nrep;
        const uint16_t* qp = p.q + (int64_t)b * p.q_sb + (int64_t)(h * nrep + (has ? c : 0)) * p.q_sh + 32 * g;
        bool over = false;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            u4 w = has ? *(const u4*)(qp + 8 * j) : u4{0u, 0u, 0u, 0u};
            if (p.q_bf16) {
                // bf16 -> fp16: exact in [2^-14, 65504]; a finite value beyond becomes inf
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float lo = __uint_as_float(w[e] << 16), hi = __uint_as_float(w[e] & 0xffff0000u);
                    const uint32_t a = f2h_rn(lo), bb = f2h_rn(hi);
                    over |= (((a & 0x7fffu) == 0x7c00u) && fabsf(lo) < INFINITY) ||
                            (((bb & 0x7fffu) == 0x7c00u) && fabsf(hi) < INFINITY);
                    w[e] = a | (bb << 16);
                }
            }
            qf[j] = __builtin_bit_cast(h8, w);
        }
        if (__ballot(over) && lane == 0 && p.err) atomicOr(p.err, HKV_ERR_BIT_RANGE);
    }

    f4 acc[8];
#pragma unroll
    for (int n = 0; n < 8; ++n) acc[n] = f4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.0f;
    float* srow = nullptr;   // this lane's score row (kScores)
    if constexpr (kScores) srow = p.scores + (int64_t)b * p.sc_sb + (int64_t)(h * nrep + min(c, nrep - 1)) * p.sc_sh;

    __shared__ __align__(16) int sm_ids[kIdWindow + 2];
    __shared__ int sm_ctr[2];   // next INT4 pair, next fp16 tile (kDynamic)
    if (kDynamic && threadIdx.x == 0) {
        sm_ctr[0] = kPrefetch * kWaves;   // the first round of each window is static
        sm_ctr[1] = kF16Depth * kWaves;
    }

    // ---- fp16 zone tiles f0 .. f0 + nf, depth 2.  Every slot of a round is
    // consumed (an empty one with no valid token, which contributes nothing), and
    // the only exit is at the back edge; units only grow, so an empty slot 0 means
    // every later slot is empty too.  An exit from inside the round would add a path
    // on which the later slots were not refilled, and the waits at the loop head
    // would then drain every slot.
    if (nf > 0) {
        F16Tile buf[kF16Depth];
        int tq[kF16Depth];
        ZoneP zq[kF16Depth];
        int lq[kF16Depth];
        int seq = wave + kF16Depth * kWaves;
#pragma unroll
        for (int k = 0; k < kF16Depth; ++k) {
            tq[k] = wave + k * kWaves;
            int t;
            locate_tile(p, zt, lenz, f0 + min(tq[k], nf - 1), zq[k], lq[k], t);
            __builtin_amdgcn_sched_barrier(0);
            load_f16(zq[k], bh, t, tq[k] < nf, c, g, buf[k]);
            __builtin_amdgcn_sched_barrier(0);
            lq[k] -= t * kBlockTokens;
        }
#ifdef HKV_DECODE_TIMELINE
        if (p.tl_waits) {
            __builtin_amdgcn_s_waitcnt(0);
            tl_w[0] = __builtin_amdgcn_s_memrealtime();
        }
#endif
        // the first INT4 window's ids arrive with these tiles (they were requested
        // first); they and the counters are published before the loop starts
        if (a1 > a0) commit_block_ids(p, min(kIdWindow, a1 - a0), idr, sm_ids);
        __syncthreads();
        TL_MARK(1);
        if (tq[0] < nf) {
            do {
#pragma unroll
                for (int k = 0; k < kF16Depth; ++k) {
                    if constexpr (kScores) {
                        int zi, t;
                        locate_zone(zt, f0 + min(tq[k], nf - 1), zi, t);
                        float* sp = srow + (zi == 0 ? p.sc_zone[0] : zi == 1 ? p.sc_zone[1] : p.sc_zone[2]) +
                                    t * kBlockTokens + 4 * g;
                        step_f16<true>(buf[k], tq[k] < nf ? min(kBlockTokens, lq[k]) : 0, g, qf, p.scale_log2, acc,
                                       m, l, c < nrep, sp);
                    } else {
                        step_f16(buf[k], tq[k] < nf ? min(kBlockTokens, lq[k]) : 0, g, qf, p.scale_log2, acc, m, l);
                    }
#ifdef HKV_DECODE_TIMELINE
                    if (tl_t[7] == 0) TL_MARK(7);
#endif
                    tq[k] = next_unit<kDynamic>(&sm_ctr[1], seq);
                    int t;
                    locate_tile(p, zt, lenz, f0 + min(tq[k], nf - 1), zq[k], lq[k], t);
                    __builtin_amdgcn_sched_barrier(0);
                    load_f16(zq[k], bh, t, tq[k] < nf, c, g, buf[k]);
                    __builtin_amdgcn_sched_barrier(0);
                    lq[k] -= t * kBlockTokens;
                }
            } while (tq[0] < nf);
        }
    }

    // ---- INT4 blocks a0 .. a1, two per step, in windows of kIdWindow block ids
    // staged in LDS (same loop shape).  An empty slot re-reads the window's last
    // pair, an in-bounds address.
    if (nf <= 0 && a1 > a0) {
        commit_block_ids(p, min(kIdWindow, a1 - a0), idr, sm_ids);
        __syncthreads();
        TL_MARK(1);
    }
    for (int wb = a0; wb < a1; wb += kIdWindow) {
        const int wn = min(kIdWindow, a1 - wb);
        if (wb != a0) {
            fetch_block_ids(p, b, wb, wn, idr);
            commit_block_ids(p, wn, idr, sm_ids);
            __syncthreads();
        }
        const int npairs = (wn + 1) >> 1;
        Int4Blk bufA[kPrefetch], bufB[kPrefetch];
        int pk[kPrefetch];
        int seq = wave + kPrefetch * kWaves;
        // sched_barrier keeps each slot's loads together and in slot order, in the
        // prologue as in the loop, so the waits before a slot's use only cover that
        // slot and the later slots stay in flight
#pragma unroll
        for (int k = 0; k < kPrefetch; ++k) {
            pk[k] = wave + k * kWaves;
            const u2 id = read_pair_ids(sm_ids, min(pk[k], npairs - 1));
            __builtin_amdgcn_sched_barrier(0);
            load_int4(p, h, __builtin_amdgcn_readfirstlane((int)id.x), pk[k] < npairs, c, g, bufA[k]);
            load_int4(p, h, __builtin_amdgcn_readfirstlane((int)id.y), 2 * pk[k] + 1 < wn, c, g, bufB[k]);
            __builtin_amdgcn_sched_barrier(0);
        }
#ifdef HKV_DECODE_TIMELINE
        if (p.tl_waits && wb == a0) {
            __builtin_amdgcn_s_waitcnt(0);
            tl_w[1] = __builtin_amdgcn_s_memrealtime();
        }
#endif
        int nxt = next_unit<kDynamic>(&sm_ctr[0], seq);
        u2 nid = read_pair_ids(sm_ids, min(nxt, npairs - 1));
        if (pk[0] < npairs) {
            do {
#pragma unroll
                for (int k = 0; k < kPrefetch; ++k) {
                    const int lb = wb + 2 * pk[k];
                    const int nA = pk[k] < npairs ? min(kBlockTokens, len4 - lb * kBlockTokens) : 0;
                    const int nB = (2 * pk[k] + 1 < wn) ? min(kBlockTokens, len4 - (lb + 1) * kBlockTokens) : 0;
                    if constexpr (kScores)
                        step_int4_pair<true>(bufA[k], bufB[k], nA, nB, g, kzsh, qf, p.scale_log2, acc, m, l, c < nrep,
                                             srow + lb * kBlockTokens + 4 * g,
                                             srow + (lb + 1) * kBlockTokens + 4 * g);
                    else
                        step_int4_pair(bufA[k], bufB[k], nA, nB, g, kzsh, qf, p.scale_log2, acc, m, l);
#ifdef HKV_DECODE_TIMELINE
                    if (tl_t[7] == 0) TL_MARK(7);
#endif
                    pk[k] = nxt;
                    __builtin_amdgcn_sched_barrier(0);
                    load_int4(p, h, __builtin_amdgcn_readfirstlane((int)nid.x), nxt < npairs, c, g, bufA[k]);
                    load_int4(p, h, __builtin_amdgcn_readfirstlane((int)nid.y), 2 * nxt + 1 < wn, c, g, bufB[k]);
                    __builtin_amdgcn_sched_barrier(0);
                    nxt = next_unit<kDynamic>(&sm_ctr[0], seq);
                    nid = read_pair_ids(sm_ids, min(nxt, npairs - 1));
                }
            } while (pk[0] < npairs);
        }
        if (wb + kIdWindow < a1) {
            __syncthreads();   // every wave is done with this window's ids and counter
            if (kDynamic && threadIdx.x == 0) sm_ctr[0] = kPrefetch * kWaves;
        }
    }

    TL_MARK(2);
#ifdef HKV_DECODE_TIMELINE
    const unsigned long long tl_info = ((unsigned long long)(__builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 15) << 56) |
                                       ((unsigned long long)(unsigned)(a1 - a0) << 24) | (unsigned)max(nf, 0);
#endif
    // XCD-local hand-off: OR this workgroup's XCD bit (HW_REG_XCC_ID) into the pair's
    // device-scope mask; the old mask is examined at the ticket.  Issued here, its round
    // trip overlaps the merge below.  (At the start of the kernel it cost ~1.7 us on the
    // 32K decode: the pair's 32 atomics serialize on one address, and loads issued after
    // one complete after it.)  Of any two workgroups of a pair on different XCDs, the
    // later OR returns the other's bit, so a split placement is always reported.
    // The last refills (zero-sized past the range's end) complete first, so that the OR
    // below is the one load in flight when the merge starts: with refills still pending on
    // the path that skips the OR, the compiler waited for all loads, the OR included,
    // before the first shuffle of the merge.
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    if (kL2 && threadIdx.x == 0) {
        owner_bit = 1u << (__builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 15);
        owner_old = __hip_atomic_fetch_or(&p.owners[bh * kLineWords], owner_bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // ---- merge the waves of this workgroup through LDS
    // the row sum over the four 16-lane rows, by lane swaps (the operands of each add are
    // the same on both lanes of a swapped pair, so every lane gets the same bits)
    {
        const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(l), __float_as_uint(l), false, false);
        l = __uint_as_float(s16[0]) + __uint_as_float(s16[1]);
        const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(l), __float_as_uint(l), false, false);
        l = __uint_as_float(s32[0]) + __uint_as_float(s32[1]);
    }
    extern __shared__ float smem[];
    float* sm_o = smem;                                   // [kWaves][nrep][128]
    float* sm_m = sm_o + kWaves * nrep * kHeadDim;        // [kWaves][nrep]
    float* sm_l = sm_m + kWaves * 16;                     // [kWaves][nrep]
    __shared__ int sm_ticket;
    if (c < nrep) {
        float* o = sm_o + (wave * nrep + c) * kHeadDim;
#pragma unroll
        for (int n = 0; n < 8; ++n)
#pragma unroll
            for (int v = 0; v < 4; ++v) o[16 * n + 4 * g + v] = acc[n][v];
        if (g == 0) {
            sm_m[wave * 16 + c] = m;
            sm_l[wave * 16 + c] = l;
        }
    }
    __syncthreads();

    const int nout = nrep * kHeadDim;
    // the pair's partial states, computed once and held in registers (opaque to the
    // compiler, which would otherwise read the arguments again after the arrival wait)
    float* parts = p.partials + (int64_t)bh * p.part_pair_stride;
    uint16_t* obase = p.out + (int64_t)b * p.o_sb + (int64_t)(h * nrep) * p.o_sh;   // this kv head's outputs
    int64_t osh = p.o_sh;
    int obf16 = p.out_bf16, slice_outputs = p.slice_outputs;
    asm volatile("" : "+s"(parts), "+s"(obase), "+s"(osh), "+s"(obf16), "+s"(slice_outputs));
    float* part = parts + (int64_t)split * (nrep * kPartStride);
    for (int idx = threadIdx.x; idx < nout; idx += kThreads) {
        const int hd = idx >> 7, d = idx & (kHeadDim - 1);
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) M = fmaxf(M, sm_m[w * 16 + hd]);
        float O = 0.f, L = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float mw = sm_m[w * 16 + hd];
            const float e = (mw == -INFINITY) ? 0.f : fast_exp2(mw - M);
            O += sm_o[(w * nrep + hd) * kHeadDim + d] * e;
            L += sm_l[w * 16 + hd] * e;
        }
        if (nsplit == 1) {
            const float r = L > 0.f ? O / L : 0.f;
            obase[(int64_t)hd * osh + d] = obf16 ? f2bf_rn(r) : f2h_rn(r);
            if (kScores && d == 0) {
                float* st = p.stats + ((int64_t)b * p.Hkv * nrep + h * nrep + hd) * 2;
                st[0] = M;
                st[1] = L;
            }
        } else if (kL2) {
            part[hd * kPartStride + d] = O;
            if (d == 0) {
                part[hd * kPartStride + kHeadDim] = M;
                part[hd * kPartStride + kHeadDim + 1] = L;
            }
        } else {
            st_agent(part + hd * kPartStride + d, O);
            if (d == 0) {
                st_agent(part + hd * kPartStride + kHeadDim, M);
                st_agent(part + hd * kPartStride + kHeadDim + 1, L);
            }
        }
    }
    TL_MARK(3);
    if (nsplit == 1) {
        TL_FLUSH(tl_info);
        return;
    }
    // every lane waits until its agent-coherent stores have completed, then the
    // barrier makes that true for the whole workgroup before the ticket is taken
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __syncthreads();
    if (p.coop) {
        // ---- slice merge (every range of the pair resident; atomics and loads in the
        // XCD's L2 with the XCD-local hand-off, at device scope otherwise).  Each
        // range adds itself to the pair's arrival count, waits until the count is complete
        // (bounded), then merges one slice of the pair's output from all nsplit partial
        // states, so that the end of the kernel is one small load round trip after the
        // last arrival instead of one workgroup loading every state.  A range whose wait
        // runs out sets kGoneBit and leaves; the last arrival, seeing it, merges every
        // slice (the same code, so a slice written twice gets the same bits).  The last
        // arrival also resets the pair's words at once: it advances the generation and
        // clears the count in one store, so a range still waiting sees the launch
        // complete either way (count full, or generation moved on), and no range needs
        // another round trip to the word before its slice.
        __shared__ int sm_slices;   // 0: none, 1: this range's slice, 2: every slice
        if (threadIdx.x == 0) {
            bool overrun;
            const int slices =
                kL2
                    ? slice_arrival<__HIP_MEMORY_SCOPE_WORKGROUP>(&p.counters_l2[bh * kLineWords], nsplit, p.merge_wait,
                                                                  &p.owners[bh * kLineWords], &overrun)
                    : slice_arrival<__HIP_MEMORY_SCOPE_AGENT>(&p.counters[bh * kLineWords + 2], nsplit, p.merge_wait,
                                                              nullptr, &overrun);
            const bool bad = (owner_old & ~owner_bit) != 0u || overrun;
            if (bad && p.err)
                __hip_atomic_fetch_or(p.err, HKV_ERR_BIT_PLACEMENT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            sm_slices = slices;
        }
        __syncthreads();
        TL_MARK(4);
        const int slices = sm_slices;
        if (slices == 0) {
            TL_FLUSH(tl_info);
            return;
        }
        // slice sl = outputs [sl S, sl S + S) of the pair's nout (head-major: head, dim);
        // 4 threads per output, thread q of an output taking splits q, q + 4, ...
        const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)parts, 0, (int)(nsplit * nrep * kPartStride * sizeof(float)), 0x00020000);
        const int S = slice_outputs;
        const int sl0 = slices == 2 ? 0 : split, sl1 = slices == 2 ? nsplit : split + 1;
        for (int sl = sl0; sl < sl1; ++sl) {
            for (int t = threadIdx.x; t < 4 * S; t += kThreads) {
                const int o = sl * S + (t >> 2), q = t & 3;
                const bool live = o < nout;
                const int hd = min(o, nout - 1) >> 7, d = min(o, nout - 1) & (kHeadDim - 1);
                float M = -INFINITY, L = 0.f, O = 0.f;
                for (int base = 0; q + base < nsplit; base += 32) {
                    float ms[8], ls[8], os[8];
                    if (kL2)
                        load_slice8<kAuxL2>(prs, q, base, nsplit, nrep, hd, d, ms, ls, os);
                    else
                        load_slice8<kAuxDevice>(prs, q, base, nsplit, nrep, hd, d, ms, ls, os);
                    float Mc = ms[0];
#pragma unroll
                    for (int j = 1; j < 8; ++j) Mc = fmaxf(Mc, ms[j]);
                    if (Mc > -INFINITY) {
                        const float Mn = fmaxf(M, Mc);
                        const float a = (M == -INFINITY) ? 0.f : fast_exp2(M - Mn);
                        float Oc = 0.f, Lc = 0.f;
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            const float e = (ms[j] == -INFINITY) ? 0.f : fast_exp2(ms[j] - Mn);
                            Oc += os[j] * e;
                            Lc += ls[j] * e;
                        }
                        O = O * a + Oc;
                        L = L * a + Lc;
                        M = Mn;
                    }
                }
                // the output's four threads are one quad of lanes: exchanged with DPP quad
                // permutes (lane ^ 1, then lane ^ 2), no LDS round trip
#pragma unroll
                for (int x = 1; x < 4; x <<= 1) {
                    const float M2 = quad_xor(M, x), L2 = quad_xor(L, x), O2 = quad_xor(O, x);
                    const float Mn = fmaxf(M, M2);
                    const float a = (M == -INFINITY) ? 0.f : fast_exp2(M - Mn);
                    const float c = (M2 == -INFINITY) ? 0.f : fast_exp2(M2 - Mn);
                    O = O * a + O2 * c;
                    L = L * a + L2 * c;
                    M = Mn;
                }
                if (live && q == 0) {
                    const float r = L > 0.f ? O / L : 0.f;
                    obase[(int64_t)hd * osh + d] = obf16 ? f2bf_rn(r) : f2h_rn(r);
                    if (kScores && d == 0) {
                        float* st = p.stats + ((int64_t)b * p.Hkv * nrep + h * nrep + hd) * 2;
                        st[0] = M;
                        st[1] = L;
                    }
                }
            }
        }
        TL_MARK(5);
        TL_MARK(6);
        TL_FLUSH(tl_info | (1ull << 48));
        return;
    }
    if (threadIdx.x == 0) {
        // the stores above have completed (in L2, or in memory for sc1 stores)
        int tk;
        if (kL2)
            tk = __hip_atomic_fetch_add(&p.counters_l2[bh * kLineWords + 1], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        else
            tk = __hip_atomic_fetch_add(&p.counters[bh * kLineWords], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // another XCD's bit in the mask: this pair's ranges did not share one L2.  A
        // ticket beyond the range count is what such a launch leaves behind; it is
        // reset so that later launches count from zero again.
        const bool foreign = (owner_old & ~owner_bit) != 0u;
        if (tk >= nsplit) {
            if (kL2)
                __hip_atomic_store(&p.counters_l2[bh * kLineWords + 1], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            else
                __hip_atomic_store(&p.counters[bh * kLineWords], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if ((foreign || tk >= nsplit) && p.err)
            __hip_atomic_fetch_or(p.err, HKV_ERR_BIT_PLACEMENT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sm_ticket = tk;
    }
    __syncthreads();
    TL_MARK(4);
    if (sm_ticket != nsplit - 1) {
        TL_FLUSH(tl_info);
        return;
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");

    // ---- last workgroup of this pair: merge the nsplit partial states in one
    // memory round trip.  Thread t owns float4 `u` of one head and the splits
    // s = k, k + K, k + 2K, ... (K = threads per unit); all its loads are
    // independent.  The K per-thread states then merge through LDS.
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)parts, 0, (int)(nsplit * nrep * kPartStride * sizeof(float)), 0x00020000);
    const int units = nrep * (kHeadDim / 4);
    const int K = kThreads / units;                  // >= 1 because nrep <= 16
    float* sm = smem;                                // [K][units][6] = (M, L, O[4])
    if (threadIdx.x < K * units) {
        const int u = threadIdx.x % units, k = threadIdx.x / units;
        const int hd = u / (kHeadDim / 4), d4 = (u % (kHeadDim / 4)) * 4;
        float M = -INFINITY, L = 0.f;
        f4 O = {0.f, 0.f, 0.f, 0.f};
        for (int s0 = k; s0 < nsplit; s0 += 8 * K) {
            float ms[8], ls[8];
            f4 os[8];
            if (kL2)
                load_partials<true>(prs, parts, s0, K, nsplit, nrep, hd, d4, ms, ls, os);
            else
                load_partials<false>(prs, parts, s0, K, nsplit, nrep, hd, d4, ms, ls, os);
            // the eight states merge with independent terms against their common max
            float Mc = ms[0];
#pragma unroll
            for (int j = 1; j < 8; ++j) Mc = fmaxf(Mc, ms[j]);
            if (Mc > -INFINITY) {
                const float Mn = fmaxf(M, Mc);
                const float a = (M == -INFINITY) ? 0.f : fast_exp2(M - Mn);
                f4 Oc = {0.f, 0.f, 0.f, 0.f};
                float Lc = 0.f;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float e = (ms[j] == -INFINITY) ? 0.f : fast_exp2(ms[j] - Mn);
                    Oc += os[j] * e;
                    Lc += ls[j] * e;
                }
                O = O * a + Oc;
                L = L * a + Lc;
                M = Mn;
            }
        }
        float* w = sm + (k * units + u) * 6;
        w[0] = M;
        w[1] = L;
        w[2] = O[0];
        w[3] = O[1];
        w[4] = O[2];
        w[5] = O[3];
    }
    __syncthreads();
    TL_MARK(5);
    if (threadIdx.x < units) {
        const int u = threadIdx.x;
        const int hd = u / (kHeadDim / 4), d4 = (u % (kHeadDim / 4)) * 4;
        float M = -INFINITY;
        for (int k = 0; k < K; ++k) M = fmaxf(M, sm[(k * units + u) * 6]);
        float L = 0.f;
        f4 O = {0.f, 0.f, 0.f, 0.f};
        for (int k = 0; k < K; ++k) {
            const float* w = sm + (k * units + u) * 6;
            if (w[0] == -INFINITY) continue;
            const float e = fast_exp2(w[0] - M);
            L += w[1] * e;
            O += f4{w[2], w[3], w[4], w[5]} * e;
        }
        const float inv = L > 0.f ? 1.0f / L : 0.f;
        uint16_t* op = obase + (int64_t)hd * osh + d4;
#pragma unroll
        for (int v = 0; v < 4; ++v) op[v] = obf16 ? f2bf_rn(O[v] * inv) : f2h_rn(O[v] * inv);
        if (kScores && d4 == 0) {
            float* st = p.stats + ((int64_t)b * p.Hkv * nrep + h * nrep + hd) * 2;
            st[0] = M;
            st[1] = L;
        }
    }
    TL_MARK(6);
    TL_FLUSH(tl_info | (1ull << 48));
    // last in the kernel, so that no barrier waits for these stores: every workgroup of
    // the pair has taken its ticket, so its mask update is done
    if (threadIdx.x == 0) {
        if (kL2) {
            __hip_atomic_store(&p.counters_l2[bh * kLineWords + 1], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            __hip_atomic_store(&p.owners[bh * kLineWords], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            __hip_atomic_store(&p.counters[bh * kLineWords], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// Clears a workspace's ticket area (int words) before a launch whose geometry differs
// from the previous launch on the same workspace.
__global__ __launch_bounds__(256) void clear_words_kernel(int* w, int64_t n) {
    for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) w[i] = 0;
}

constexpr size_t kWsHeader = 256;

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

int num_cus() {
    static std::atomic<int> cached[64];   // per device (partition modes can differ)
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    const int c = cached[dev & 63].load(std::memory_order_relaxed);
    if (c > 0) return c;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
    cached[dev & 63].store(n, std::memory_order_relaxed);
    return n;
}

// Ranges per (sequence, kv head): about one 8-wave workgroup per CU for the
// whole launch, each reading at least ~96 KB, at most kMaxSplits.
int choose_splits(int BH, int int4_max_len, const int32_t* f16_max_lens, int nz, int hint) {
    if (hint > 0) return hint < kMaxSplits ? hint : kMaxSplits;
    int64_t bytes = (int64_t)((int4_max_len + kBlockTokens - 1) / kBlockTokens) * kInt4ItemBytes;
    for (int i = 0; i < nz; ++i) bytes += (int64_t)((f16_max_lens[i] + kBlockTokens - 1) / kBlockTokens) * kF16ItemBytes;
    const int cus = num_cus();
    int64_t s = (cus + BH - 1) / BH;                       // fill the chip once
    const int64_t by_size = (bytes + 96 * 1024 - 1) / (96 * 1024);
    if (s > by_size) s = by_size;                           // small problems: fewer, fuller ranges
    if (s < 1) s = 1;
    if (s > kMaxSplits) s = kMaxSplits;
    return (int)s;
}

// Workspace: [header (error word) | agent lines (ticket, XCD mask) | XCD-local lines
// (256 B each) | partial states, one 256-byte aligned block per (sequence, kv head)].
// One line per pair: packed one word per pair, the 256 atomics of a 32K decode's 8 pairs
// went to one cache line and queued there (the placement check then cost ~0.6 us per launch).
// The ticket area holds kHandoffPairs slots of each kind at fixed offsets, whatever the
// launch geometry, so the partial states of one launch never overlap the tickets of
// another launch on the same workspace: the kernels leave every ticket at zero, and a
// workspace (or a graph replaying launches on it) stays valid across geometries with
// no clearing between launches.  A launch that splits more pairs than that is
// rejected.
constexpr int64_t kHandoffPairs = 1024;

size_t pair_part_bytes(int nrep, int nsplit) { return align256((size_t)nsplit * nrep * kPartStride * sizeof(float)); }

constexpr size_t kTicketAreaEnd = kWsHeader + 2 * kHandoffPairs * 256;
static_assert(kTicketAreaEnd % 256 == 0, "partial states start 256-byte aligned");

size_t workspace_bytes(int B, int Hq, int Hkv, int nsplit) {
    const size_t BH = (size_t)B * Hkv;
    const int nrep = Hq / Hkv;
    return kTicketAreaEnd + BH * pair_part_bytes(nrep, nsplit);
}

// XCDs that workgroups are dispatched over round-robin: gfx950 has 32 CUs per
// XCD, so a partition with N CUs spans N / 32 of them.
int num_xcc() {
    static std::atomic<int> cached[64];   // per device (partition modes can differ)
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 1;
    const int c = cached[dev & 63].load(std::memory_order_relaxed);
    if (c > 0) return c;
    hipDeviceProp_t prop;
    int n = 1;
    if (hipGetDeviceProperties(&prop, dev) == hipSuccess && strncmp(prop.gcnArchName, "gfx950", 6) == 0 &&
        prop.multiProcessorCount % 32 == 0 && prop.multiProcessorCount >= 32)
        n = prop.multiProcessorCount / 32;
    cached[dev & 63].store(n, std::memory_order_relaxed);
    return n;
}

size_t lds_bytes(int nrep) {
    const size_t merge = ((size_t)kWaves * nrep * kHeadDim + 2 * kWaves * 16) * sizeof(float);
    const size_t units = (size_t)nrep * (kHeadDim / 4);
    const size_t combine = (kThreads / units) * units * 6 * sizeof(float);
    return merge > combine ? merge : combine;
}

}  // namespace
}  // namespace hkv

using namespace hkv;

extern "C" size_t hkv_decode_workspace_bytes(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                                             int32_t head_dim, int32_t int4_max_len,
                                             const int32_t* f16_max_lens, int32_t num_f16_zones) {
    if (batch <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0 || head_dim != kHeadDim ||
        num_f16_zones < 0 || num_f16_zones > HKV_MAX_F16_ZONES || (num_f16_zones > 0 && !f16_max_lens))
        return 0;
    return workspace_bytes(batch, num_q_heads, num_kv_heads, kMaxSplits);
}

#ifdef HKV_DECODE_TIMELINE
static __device__ unsigned long long g_timeline[kTlMaxWaves * kTlWords];
static int64_t g_timeline_waves = 0;

// Copies the timestamps of the last decode launch (16 words per wave, workgroup-major)
// into `host` (room for max_waves waves); returns the number of waves copied.  Waits for
// the device.  Timeline build only.
extern "C" int64_t hkv_decode_timeline_read(unsigned long long* host, int64_t max_waves) {
    int64_t n = g_timeline_waves < max_waves ? g_timeline_waves : max_waves;
    if (n > kTlMaxWaves) n = kTlMaxWaves;
    if (!host || n <= 0) return 0;
    if (hipDeviceSynchronize() != hipSuccess) return -1;
    if (hipMemcpyFromSymbol(host, HIP_SYMBOL(g_timeline), (size_t)n * kTlWords * sizeof(unsigned long long), 0,
                            hipMemcpyDeviceToHost) != hipSuccess)
        return -1;
    return n;
}
#endif

// The launch behind both decode entry points: `wsp` / `ws_bytes` is the caller's
// workspace (hkv_decode_attn) or this device's static scratch (hkv_decode_attn_noalloc).
static int decode_launch(const HkvDecodeArgs* a, void* wsp, size_t ws_bytes, void* stream) {
    HKV_REQUIRE(a->head_dim == kHeadDim, HKV_ERR_UNSUPPORTED, "hkv_decode_attn: head_dim %d != 128", a->head_dim);
    HKV_REQUIRE(a->batch > 0 && a->num_kv_heads > 0 && a->num_q_heads > 0, HKV_ERR_ARG,
                "hkv_decode_attn: bad batch/heads");
    HKV_REQUIRE(a->num_q_heads % a->num_kv_heads == 0, HKV_ERR_ARG,
                "hkv_decode_attn: num_q_heads %d not a multiple of num_kv_heads %d", a->num_q_heads,
                a->num_kv_heads);
    const int nrep = a->num_q_heads / a->num_kv_heads;
    HKV_REQUIRE(nrep <= 16, HKV_ERR_UNSUPPORTED, "hkv_decode_attn: n_rep %d > 16", nrep);
    HKV_REQUIRE(a->num_f16_zones >= 0 && a->num_f16_zones <= HKV_MAX_F16_ZONES, HKV_ERR_ARG,
                "hkv_decode_attn: num_f16_zones %d out of range", a->num_f16_zones);
    HKV_REQUIRE((a->flags & ~(HKV_DECODE_DETERMINISTIC | HKV_DECODE_AGENT_HANDOFF)) == 0, HKV_ERR_ARG,
                "hkv_decode_attn: unknown flags 0x%x", (unsigned)a->flags);
    HKV_REQUIRE((a->q_dtype == HKV_DTYPE_F16 || a->q_dtype == HKV_DTYPE_BF16) &&
                    (a->out_dtype == HKV_DTYPE_F16 || a->out_dtype == HKV_DTYPE_BF16),
                HKV_ERR_ARG, "hkv_decode_attn: q/out dtype must be fp16 or bf16 (got %d / %d)", a->q_dtype,
                a->out_dtype);
    if (a->scores) {
        HKV_REQUIRE(a->score_stats != nullptr, HKV_ERR_ARG, "hkv_decode_attn: scores without score_stats");
        int64_t row = a->int4_max_len;
        for (int i = 0; i < a->num_f16_zones; ++i) row += a->f16[i].max_len;
        HKV_REQUIRE(a->scores_stride_h >= row && a->scores_stride_b >= (int64_t)a->num_q_heads * a->scores_stride_h,
                    HKV_ERR_ARG, "hkv_decode_attn: score strides too small for %lld items per row", (long long)row);
    }
    HKV_REQUIRE(a->q && a->out && wsp, HKV_ERR_ARG, "hkv_decode_attn: null q/out/workspace");
    HKV_REQUIRE((((uintptr_t)a->q) & 15) == 0 && (a->q_stride_b % 8) == 0 && (a->q_stride_h % 8) == 0,
                HKV_ERR_ARG, "hkv_decode_attn: q must be 16-byte aligned with strides multiple of 8");
    HKV_REQUIRE(a->int4_max_len >= 0 && a->int4_max_len <= kMaxZoneTokens, HKV_ERR_ARG,
                "hkv_decode_attn: int4_max_len %d outside [0, %d]", a->int4_max_len, kMaxZoneTokens);
    if (a->int4_max_len > 0) {
        HKV_REQUIRE(a->block_table && ((a->pool && a->pool_blocks > 0) || (a->staging && a->staging_blocks > 0)),
                    HKV_ERR_ARG, "hkv_decode_attn: INT4 zone without pool/staging records or block table");
        HKV_REQUIRE(a->pool_blocks >= 0 && a->staging_blocks >= 0 && a->staging_blocks <= (1ll << 31),
                    HKV_ERR_ARG, "hkv_decode_attn: bad pool/staging block counts");
        HKV_REQUIRE(a->staging_blocks == 0 || (((uintptr_t)a->staging) & 15) == 0, HKV_ERR_ARG,
                    "hkv_decode_attn: staging must be 16-byte aligned");
        HKV_REQUIRE((int64_t)a->bt_stride * kBlockTokens >= a->int4_max_len, HKV_ERR_CAPACITY,
                    "hkv_decode_attn: block table stride %d too small for %d INT4 tokens", a->bt_stride,
                    a->int4_max_len);
        HKV_REQUIRE((((uintptr_t)a->pool) & 15) == 0, HKV_ERR_ARG, "hkv_decode_attn: pool must be 16-byte aligned");
    }
    int32_t zl[HKV_MAX_F16_ZONES] = {0, 0, 0};
    for (int i = 0; i < a->num_f16_zones; ++i) {
        const HkvF16Zone& z = a->f16[i];
        HKV_REQUIRE(z.max_len >= 0 && z.max_len <= z.capacity, HKV_ERR_ARG,
                    "hkv_decode_attn: zone %d max_len %d exceeds capacity %d", i, z.max_len, z.capacity);
        HKV_REQUIRE(z.capacity % kBlockTokens == 0, HKV_ERR_ARG, "hkv_decode_attn: zone %d capacity not a multiple of 16", i);
        if (z.max_len > 0) {
            HKV_REQUIRE(z.k && z.v, HKV_ERR_ARG, "hkv_decode_attn: zone %d has null k/v", i);
            HKV_REQUIRE((((uintptr_t)z.k | (uintptr_t)z.v) & 15) == 0, HKV_ERR_ARG,
                        "hkv_decode_attn: zone %d k/v must be 16-byte aligned", i);
        }
        zl[i] = z.max_len;
    }
    HKV_REQUIRE((int64_t)zl[0] + zl[1] + zl[2] <= kMaxZoneTokens, HKV_ERR_ARG,
                "hkv_decode_attn: fp16 zones hold more than %d tokens", kMaxZoneTokens);
    const int64_t BH = (int64_t)a->batch * a->num_kv_heads;
    HKV_REQUIRE(BH < 65536, HKV_ERR_ARG, "hkv_decode_attn: batch x kv heads too large");
    const int ms = choose_splits((int)BH, a->int4_max_len, zl, a->num_f16_zones, a->splits_hint);
    HKV_REQUIRE(ms == 1 || BH <= kHandoffPairs, HKV_ERR_CAPACITY,
                "hkv_decode_attn: %d ranges per pair for %lld (sequence, kv head) pairs; a split launch hands off "
                "at most %lld pairs", ms, (long long)BH, (long long)kHandoffPairs);
    const size_t need = workspace_bytes(a->batch, a->num_q_heads, a->num_kv_heads, ms);
    HKV_REQUIRE(ws_bytes >= need, HKV_ERR_CAPACITY, "hkv_decode_attn: workspace %zu bytes, need %zu", ws_bytes, need);
    HKV_REQUIRE((((uintptr_t)wsp) & 255) == 0, HKV_ERR_ARG, "hkv_decode_attn: workspace must be 256-byte aligned");

    DecodeParams p;
    p.B = a->batch;
    p.Hkv = a->num_kv_heads;
    p.nrep = nrep;
    p.scale_log2 = a->sm_scale * kLog2e;
    p.q_bf16 = a->q_dtype == HKV_DTYPE_BF16;
    p.out_bf16 = a->out_dtype == HKV_DTYPE_BF16;
    p.q = a->q;
    p.q_sb = a->q_stride_b;
    p.q_sh = a->q_stride_h;
    p.nz = a->num_f16_zones;
    for (int i = 0; i < HKV_MAX_F16_ZONES; ++i) {
        const HkvF16Zone& z = a->f16[i];
        p.z[i].k = i < p.nz ? z.k : nullptr;
        p.z[i].v = i < p.nz ? z.v : nullptr;
        p.z[i].cap = i < p.nz ? z.capacity : 0;
        p.z[i].max_len = i < p.nz ? z.max_len : 0;
        p.z[i].lens = i < p.nz ? z.lens : nullptr;
    }
    p.pool = a->pool;
    p.pool_blocks = a->pool ? a->pool_blocks : 0;
    p.staging = a->staging;
    p.staging_blocks = a->staging ? a->staging_blocks : 0;
    p.fallback_id = p.pool_blocks > 0 ? 0 : -1;
    p.bt = a->block_table;
    p.bt_stride = a->bt_stride;
    p.int4_lens = a->int4_lens;
    p.int4_max_len = a->int4_max_len;
    p.out = a->out;
    p.o_sb = a->out_stride_b;
    p.o_sh = a->out_stride_h;
    char* ws = (char*)wsp;
    p.err = a->err_flag ? (int*)a->err_flag : (int*)ws;
    p.counters = (int*)(ws + kWsHeader);
    p.owners = (unsigned*)(ws + kWsHeader) + 1;
    p.counters_l2 = (int*)(ws + kWsHeader + kHandoffPairs * 256);
    p.partials = (float*)(ws + kTicketAreaEnd);
    p.part_pair_stride = (int64_t)(pair_part_bytes(nrep, ms) / sizeof(float));
    p.nxcc = num_xcc();
    // one range per pair needs no hand-off (and must not leave a mask bit behind)
    p.xcc_local = (BH % p.nxcc) == 0 && ms > 1 && !(a->flags & HKV_DECODE_AGENT_HANDOFF) ? 1 : 0;
    p.max_splits = ms;
    {
        // slice merge: every range of a pair must be resident while it waits for the
        // others (one 8-wave workgroup per CU: the grid fits the CUs); a slice has at most
        // 128 outputs (4 threads each).  With the XCD-local hand-off it runs in the XCD's
        // L2, otherwise through memory with device-scope accesses (a pair's ranges then
        // span XCDs, as with 4 kv heads on 8 XCDs).  Each output is
        // merged by one quad in a fixed split order, so the deterministic schedule keeps
        // bitwise reproducible outputs with it.  HKV_DECODE_MERGE_WAIT_TICKS shortens the bounded wait (tests force the
        // path where ranges stop waiting and the last arrival merges every slice).
        const int nout = nrep * kHeadDim;
        const int S = (nout + ms - 1) / ms;
        p.coop = (ms > 1 && (int64_t)BH * ms <= num_cus() && S <= 128 && ms < kArrivedMask) ? 1 : 0;
        p.slice_outputs = S;
        const char* mw = getenv("HKV_DECODE_MERGE_WAIT_TICKS");
        p.merge_wait = (mw && mw[0]) ? strtoull(mw, nullptr, 10) : kMergeWaitTicks;
    }
#ifdef HKV_DECODE_TIMELINE
    {
        static unsigned long long* tl_ptr[64] = {};
        int dev = 0;
        HKV_HIP_CHECK(hipGetDevice(&dev));
        HKV_REQUIRE(dev >= 0 && dev < 64, HKV_ERR_UNSUPPORTED, "timeline: device %d", dev);
        if (!tl_ptr[dev]) HKV_HIP_CHECK(hipGetSymbolAddress((void**)&tl_ptr[dev], HIP_SYMBOL(g_timeline)));
        p.tl = tl_ptr[dev];
        const char* w = getenv("HKV_TIMELINE_WAITS");
        p.tl_waits = (w && w[0] == '1') ? 1 : 0;
        g_timeline_waves = (int64_t)BH * ms * kWaves;
    }
#endif
    p.scores = a->scores;
    p.sc_sb = a->scores_stride_b;
    p.sc_sh = a->scores_stride_h;
    p.stats = a->score_stats;
    {
        int base = a->int4_max_len;
        for (int i = 0; i < HKV_MAX_F16_ZONES; ++i) {
            p.sc_zone[i] = base;
            if (i < a->num_f16_zones) base += a->f16[i].max_len;
        }
    }
    const size_t lds = lds_bytes(nrep);
    const bool det = (a->flags & HKV_DECODE_DETERMINISTIC) != 0;
    const bool sc = a->scores != nullptr;
    const int var = (det ? 0 : 1) + (sc ? 2 : 0) + (p.xcc_local ? 4 : 0);
#define HKV_DECODE_FN(v) decode_attn_kernel<((v) & 1) != 0, ((v) & 2) != 0, ((v) & 4) != 0>
    static const void* const fns[8] = {(const void*)HKV_DECODE_FN(0), (const void*)HKV_DECODE_FN(1),
                                       (const void*)HKV_DECODE_FN(2), (const void*)HKV_DECODE_FN(3),
                                       (const void*)HKV_DECODE_FN(4), (const void*)HKV_DECODE_FN(5),
                                       (const void*)HKV_DECODE_FN(6), (const void*)HKV_DECODE_FN(7)};
    static std::atomic<uint64_t> raised[8];   // the merge area plus the static id window can exceed 64 KB
    HKV_RAISE_LDS(fns[var], 96 * 1024, raised[var]);
    const dim3 grid((unsigned)(BH * ms)), block(kThreads);
    switch (var) {
        case 0: hipLaunchKernelGGL((HKV_DECODE_FN(0)), grid, block, lds, (hipStream_t)stream, p); break;
        case 1: hipLaunchKernelGGL((HKV_DECODE_FN(1)), grid, block, lds, (hipStream_t)stream, p); break;
        case 2: hipLaunchKernelGGL((HKV_DECODE_FN(2)), grid, block, lds, (hipStream_t)stream, p); break;
        case 3: hipLaunchKernelGGL((HKV_DECODE_FN(3)), grid, block, lds, (hipStream_t)stream, p); break;
        case 4: hipLaunchKernelGGL((HKV_DECODE_FN(4)), grid, block, lds, (hipStream_t)stream, p); break;
        case 5: hipLaunchKernelGGL((HKV_DECODE_FN(5)), grid, block, lds, (hipStream_t)stream, p); break;
        case 6: hipLaunchKernelGGL((HKV_DECODE_FN(6)), grid, block, lds, (hipStream_t)stream, p); break;
        default: hipLaunchKernelGGL((HKV_DECODE_FN(7)), grid, block, lds, (hipStream_t)stream, p); break;
    }
#undef HKV_DECODE_FN
    HKV_LAUNCH_CHECK("decode_attn_kernel");
    return HKV_OK;
}

extern "C" int hkv_decode_attn(const HkvDecodeArgs* a, void* stream) {
    clear_error();
    HKV_REQUIRE(a != nullptr, HKV_ERR_ARG, "hkv_decode_attn: null args");
    return decode_launch(a, a->workspace, a->workspace_bytes, stream);
}

// ---- allocation-free variant: the partial states, tickets and XCD masks live in a
// file-scope device array instead of a caller workspace.  Each device holds its own
// copy (resolved with hipGetSymbolAddress on the first call made with that device
// current); the first launch on a device clears its ticket area, like a new workspace.
static __device__ __align__(256) unsigned char scratch[HKV_DECODE_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

extern "C" int hkv_decode_attn_noalloc(const HkvDecodeArgs* a, void* stream) {
    clear_error();
    HKV_REQUIRE(a != nullptr, HKV_ERR_ARG, "hkv_decode_attn_noalloc: null args");
    HKV_REQUIRE(a->workspace == nullptr && a->workspace_bytes == 0, HKV_ERR_ARG,
                "hkv_decode_attn_noalloc: takes no workspace (pass NULL / 0)");
    int dev = 0;
    HKV_HIP_CHECK(hipGetDevice(&dev));
    HKV_REQUIRE(dev >= 0 && dev < kMaxDevices, HKV_ERR_UNSUPPORTED, "hkv_decode_attn_noalloc: device %d", dev);
    void* ptr = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        if (!g_scratch_ptr[dev]) {
            void* p = nullptr;
            HKV_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
            HKV_REQUIRE(p != nullptr, HKV_ERR_HIP, "hkv_decode_attn_noalloc: no scratch address on device %d", dev);
            // the ticket area starts at zero, like a new workspace (a fill kernel, not a memset,
            // so that a first call made under graph capture records nothing a replay mishandles)
            const int64_t words = (int64_t)(kTicketAreaEnd - kWsHeader) / 4;
            hipLaunchKernelGGL(clear_words_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0,
                               (hipStream_t)stream, (int*)((char*)p + kWsHeader), words);
            HKV_LAUNCH_CHECK("clear_words_kernel");
            g_scratch_ptr[dev] = p;
        }
        ptr = g_scratch_ptr[dev];
    }
    return decode_launch(a, ptr, HKV_DECODE_SCRATCH_BYTES, stream);
}
