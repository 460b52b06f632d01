// Chunked-prefill attention over [INT4 pool | fp16 zones | causal chunk] on MFMA: the
// entry point, and the INT4 kernel (the zone kernel is prefill_zones.hip; the tile loop
// both run is prefill_flat.h).
//
// Math (fused_dequant_attn.py:242-247,385-390; kernels/fused_dequant_attn.py:371-435
// is the reference entry point): out[q] = softmax_t(q . K_t * sm_scale) V_t over every
// INT4 token (dequantized as (code - zero point) x scale), every fp16 zone token and the
// chunk's own tokens t <= q (causal), GQA q head i -> kv head i / n_rep.
//
// INT4 tiles are staged into LDS as fp16 K rows (code - zero point) x K scale and V^T
// rows (code - zero point) x V scale; the queries carry sm_scale x log2 e (rounded to
// fp16 once, as in the zone kernel), so the scores come out of the MFMAs in the log2
// domain.  The staging rounds the scale to fp16 and then the product: two roundings,
// within about 1.5 fp16 ulps of the Path C dequantization's one while the scale is at
// least 2^-14 (store_k4 / store_v4).
#include "nibble_decode.h"
#include "prefill_flat.h"

#include <math.h>

#include <algorithm>
#include <type_traits>

namespace hkv {
namespace {

typedef pu4 u4;
typedef pf4 f4;
typedef pu2 u2;
typedef fh2 h2;

// Staging of INT4 tile x: wave wt of a team handles block wt of the tile (4 blocks of
// 16 tokens), so the block id and record address are wave-uniform (scalar registers,
// one buffer resource per block).  Waves 0-3 lane i: K codes of token i/4, dims
// 32(i%4)..+32, with that row's scale and zero point.  Waves 4-7 lane i: V word
// 4i..4i+3, with the V scales and zero points of tokens 4g..4g+3, g = i/16.
struct SlotK {
    u4 w;
    float ks;
    uint32_t kz;   // zero point in the low byte
};
struct SlotV {
    u4 w;
    f4 vs;
    uint32_t vz;   // zero points of tokens 4g..4g+3 (bytes)
};

// Block id of this wave's block of INT4 tile x (clamped to the last block), the same in
// every lane.  It stays a vector register until it is used two tiles later, so no wait
// for this load sits behind the record loads issued before it.
__device__ __forceinline__ int block_id4(const PrefillParams& p, int nb, int b, int x, int wt) {
    const int lb = min(x * 4 + wt, nb - 1);
    return p.bt[(int64_t)b * p.bt_stride + lb];
}
// Buffer resource over this wave's head part of record `id` (an out-of-range id is
// reported and replaced by a valid record).  The range check is a 32-bit unsigned
// compare of a wave-uniform value, and the id used is read back from lane 0, so it and
// the resource stay in scalar registers (a resource the compiler takes for divergent
// wraps every load in a readfirstlane loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t part_rsrc(const PrefillParams& p, int h, int id_v) {
    const int id = __builtin_amdgcn_readfirstlane(id_v);
    const bool ok = id >= 0 ? (uint32_t)id < p.pool_blocks : (uint32_t)(~id) < p.staging_blocks;
    const int phys = __builtin_amdgcn_readfirstlane(ok ? id : p.fallback_id);
    if (!ok && p.err && (threadIdx.x & 63) == 0) atomicOr(p.err, 1);
    const int64_t rb = (int64_t)p.Hkv * kHeadPartBytes;
    const uint8_t* part = (phys >= 0 ? p.pool + (int64_t)phys * rb : p.staging + (int64_t)(~phys) * rb) +
                          RecordLayout::part(h);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(part), 0, kHeadPartBytes, 0x00020000);
}
__device__ __forceinline__ u4 bld16(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ uint32_t bld4(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ void load_k4(const PrefillParams& p, int h, int id, int lane, SlotK& s) {
    const __amdgpu_buffer_rsrc_t r = part_rsrc(p, h, id);
    const int rr = lane >> 2, pt = lane & 3;
    s.w = bld16(r, kPartKc + rr * 64 + pt * 16);
    s.ks = __uint_as_float(bld4(r, kPartKs + rr * 4));
    s.kz = bld4(r, kPartKz + (rr & ~3)) >> (8 * (rr & 3));   // a word load, no byte value
}
__device__ __forceinline__ void load_v4(const PrefillParams& p, int h, int id, int lane, SlotV& s) {
    const __amdgpu_buffer_rsrc_t r = part_rsrc(p, h, id);
    const int g = lane >> 4;
    s.w = bld16(r, kPartVc + lane * 16);
    s.vs = __builtin_bit_cast(f4, bld16(r, kPartVs + g * 16));
    s.vz = bld4(r, kPartVz + g * 4);
}
// Writes a staged block into LDS: K as (code - zero point) x K scale with the per-token
// biases, V as (code - zero point) x V scale (the queries carry sm_scale x log2 e, so the
// scores come out of the MFMAs in the log2 domain); `valid` = valid tokens of the block.
// Tokens past it get scale 0 (their codes are finite, their scales may be anything) and
// bias -inf.
//
// Rounding.  The products are formed in packed fp16: the scale is rounded to fp16, then
// each product, so a staged element lies within about 1.5 fp16 ulps of the reference's
// dequantized value ((code - zp) x scale in float32, then .to(float16),
// kv_compressor.py:129-132) while the scale is at least 2^-14.  A smaller scale becomes
// an fp16 subnormal with fewer significant bits (about 2% error at 1e-6).  Keeping the
// softmax scale on the queries (not folded into K, which would make every K scale 8x
// smaller) keeps K's scales as far from that range as the reference's own fp16 keys.
__device__ __forceinline__ void store_k4(const SlotK& s, uint8_t* lds, uint8_t* bias, int wt, int lane, int valid) {
    const int rr = lane >> 2, pt = lane & 3;
    const int tok = wt * 16 + rr;
    const uint32_t kz = s.kz & 0xFFu;
    const h2 kz1024 = zp1024(kz, kz), kz64 = zp64(kz, kz);
    const _Float16 f = (_Float16)(rr < valid ? s.ks : 0.0f);
    const h2 f2 = {f, f};
    const uint32_t w4[4] = {s.w.x, s.w.y, s.w.z, s.w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {          // word j: dims 32pt + 8j .. +8
        const NibPairs a = unpack_word(w4[j], kz1024, kz64);
        *(u4*)(lds + k_addr(tok, pt * 4 + j)) =
            u4{__builtin_bit_cast(uint32_t, a.p0 * f2), __builtin_bit_cast(uint32_t, a.p1 * f2),
               __builtin_bit_cast(uint32_t, a.p2 * f2), __builtin_bit_cast(uint32_t, a.p3 * f2)};
    }
    if (pt == 0) ((float*)bias)[tok] = rr < valid ? 0.0f : -INFINITY;
}
__device__ __forceinline__ void store_v4(const SlotV& s, uint8_t* lds, int wt, int lane, int valid) {
    // V word 4 lane + mm: x0..x3 = tokens 4g..4g+3 at dim c+32mm, x4..x7 at +16
    const int g = lane >> 4, c = lane & 15;
    const h2 z01 = zp1024(s.vz & 0xFFu, (s.vz >> 8) & 0xFFu), z23 = zp64((s.vz >> 16) & 0xFFu, s.vz >> 24);
    const int t0 = 4 * g;
    const h2 vs01 = {(_Float16)(t0 < valid ? s.vs.x : 0.f), (_Float16)(t0 + 1 < valid ? s.vs.y : 0.f)};
    const h2 vs23 = {(_Float16)(t0 + 2 < valid ? s.vs.z : 0.f), (_Float16)(t0 + 3 < valid ? s.vs.w : 0.f)};
    const uint32_t v4[4] = {s.w.x, s.w.y, s.w.z, s.w.w};
    const int unit = wt * 4 + g;
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) {
        const NibPairs a = unpack_word(v4[mm], z01, z23);
        const int d1 = c + 32 * mm, d2 = d1 + 16;
        *(u2*)(lds + vt_addr(d1, unit)) =
            u2{__builtin_bit_cast(uint32_t, a.p0 * vs01), __builtin_bit_cast(uint32_t, a.p1 * vs23)};
        *(u2*)(lds + vt_addr(d2, unit)) =
            u2{__builtin_bit_cast(uint32_t, a.p2 * vs01), __builtin_bit_cast(uint32_t, a.p3 * vs23)};
    }
}

// The INT4 staging policy of the tile loop: two register slots per wave (the records
// of tiles t+2 and t+3 in flight while tile t is attended), block ids fetched one slot
// cycle ahead of their records.
template <int kTeam>
struct Int4Stage {
    static constexpr int kRing = 2;
    typedef typename std::conditional<kTeam == 0, SlotK, SlotV>::type Slot;
    const PrefillParams& p;
    const TileMap& tm;
    const FlatWave& w;
    int nb4;
    Slot ring[kRing];
    int idn[kRing];   // block id of the tile next loaded into each slot

    __device__ Int4Stage(const PrefillParams& p_, const TileMap& tm_, const FlatWave& w_)
        : p(p_), tm(tm_), w(w_), nb4((tm_.len4 + kBlockTokens - 1) / kBlockTokens) {}
    // valid tokens of this wave's block of tile x and of tile x, branch-free (0 past the end)
    __device__ int valid(int x) const { return min(kBlockTokens, max(0, tm.len4 - (x * 4 + w.wt) * kBlockTokens)); }
    __device__ int tvalid(int x) const { return min(kPfT, max(0, tm.len4 - x * kPfT)); }
    __device__ void load(int id, Slot& sl) const {
        if constexpr (kTeam == 0) load_k4(p, w.h, id, w.lane, sl);
        else load_v4(p, w.h, id, w.lane, sl);
    }
    __device__ void stage(int s, uint8_t* buf, uint8_t* bias, int x) const {
        if constexpr (kTeam == 0) store_k4(ring[s], buf, bias, w.wt, w.lane, valid(x));
        else store_v4(ring[s], buf, w.wt, w.lane, valid(x));
    }
    __device__ void refill(int s, int x) {   // tile x just staged from slot s
        load(idn[s], ring[s]);
        idn[s] = block_id4(p, nb4, w.b, x + 2 * kRing, w.wt);
    }
    __device__ void start(uint8_t* lds) {
#pragma unroll
        for (int x = 0; x < kRing; ++x) {
            load(block_id4(p, nb4, w.b, x, w.wt), ring[x]);
            idn[x] = block_id4(p, nb4, w.b, x + kRing, w.wt);
        }
#pragma unroll
        for (int x = 0; x < kRing; ++x) {
            stage(x, flat_buf(lds, x), flat_bias(lds, x), x);
            refill(x, x);
        }
    }
    __device__ void mask(int, pf16v (&)[2]) const {}
};

// One workgroup per CU: 8 waves (two per SIMD), up to 256 registers per wave, over one
// kv head and 64 query rows; waves 0-3 stage K, waves 4-7 stage V^T.
__global__ __launch_bounds__(kFlatThreads, 1) void prefill_attn_kernel(PrefillParams p) {
    touch_kernel_args(p);
    extern __shared__ __align__(16) uint8_t lds_raw[];
    const int b = blockIdx.z;
    const FlatBlock blk = flat_block();
    const int ngrp = (p.nrep + 3) / 4;
    const int h = blk.hg / ngrp, grp = blk.hg % ngrp;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int team = wave >> 2, wt = wave & 3;
    const int n = lane & 31, hh = lane >> 5;
    const int rep = grp * 4 + wt;
    const bool head_ok = rep < p.nrep;
    const int qh = h * p.nrep + (head_ok ? rep : 0);
    const int qrow = blk.qb * kFlatQ + team * kPfQ + n;

    TileMap tm;
    make_tile_map(p, b, blk.qb * kFlatQ + kFlatQ, tm);
    // a sequence with no INT4 token was finished by the zone kernel
    if (tm.n4 == 0) return;

    ph8 qf[8];
    flat_load_q(p, b, qh, head_ok && qrow < p.Sq, qrow, hh, p.scale_log2, qf);   // q carries sm_scale x log2 e
    pf16v acc[4];
    float m = -INFINITY, l = 0.f;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
    const FlatWave fw{b, h, wt, lane, n, hh, qrow, blk.qb};
    const int T = (tm.n4 + kFlatBufs - 1) / kFlatBufs * kFlatBufs;
    if (team == 0) {
        Int4Stage<0> pol(p, tm, fw);
        flat_tiles(pol, fw, lds_raw, qf, acc, m, l, T);
    } else {
        // waves 4-7 (the V^T staging, the larger share of VALU work) win issue ties
        // against the older waves 0-3 on their SIMDs
        __builtin_amdgcn_s_setprio(1);
        Int4Stage<1> pol(p, tm, fw);
        flat_tiles(pol, fw, lds_raw, qf, acc, m, l, T);
        __builtin_amdgcn_s_setprio(0);
    }

    l += __shfl_xor(l, 32);
    if (!(head_ok && qrow < p.Sq)) return;
    if (tm.nf() > 0) {
        // merge the zone kernel's state of this row (O relative to its max mz, sums of
        // both lane halves) with this kernel's: rescale both to the common max
        const float* st_row = state_row(p, b, qh, qrow);
        const float mz = st_row[kHeadDim];
        const float lz = st_row[kHeadDim + 1] + st_row[kHeadDim + 2];
        const float mn = fmaxf(m, mz);
        const float fa = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mn);
        const float fz = mz == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mz - mn);
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const f4 oz = *(const f4*)(st_row + 32 * db + 8 * j + 4 * hh);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[db][4 * j + i] = acc[db][4 * j + i] * fa + oz[i] * fz;
            }
        l = l * fa + lz * fz;
    }
    write_out(p, b, qh, qrow, hh, acc, l);
}

}  // namespace
}  // namespace hkv

using namespace hkv;

extern "C" int hkv_prefill_attn(const HkvPrefillArgs* a, void* stream) {
    clear_error();
    HKV_REQUIRE(a != nullptr, HKV_ERR_ARG, "hkv_prefill_attn: null args");
    HKV_REQUIRE(a->head_dim == kHeadDim, HKV_ERR_UNSUPPORTED, "hkv_prefill_attn: head_dim %d != 128", a->head_dim);
    HKV_REQUIRE(a->batch > 0 && a->num_kv_heads > 0 && a->num_q_heads > 0 && a->num_queries > 0, HKV_ERR_ARG,
                "hkv_prefill_attn: bad sizes");
    HKV_REQUIRE(a->num_q_heads % a->num_kv_heads == 0, HKV_ERR_ARG,
                "hkv_prefill_attn: num_q_heads %d not a multiple of num_kv_heads %d", a->num_q_heads,
                a->num_kv_heads);
    HKV_REQUIRE(a->num_f16_zones >= 0 && a->num_f16_zones <= HKV_MAX_F16_ZONES, HKV_ERR_ARG,
                "hkv_prefill_attn: num_f16_zones out of range");
    HKV_REQUIRE(a->q && a->out, HKV_ERR_ARG, "hkv_prefill_attn: null q/out");
    HKV_REQUIRE((a->q_dtype == HKV_DTYPE_F16 || a->q_dtype == HKV_DTYPE_BF16) &&
                    (a->chunk_dtype == HKV_DTYPE_F16 || a->chunk_dtype == HKV_DTYPE_BF16) &&
                    (a->out_dtype == HKV_DTYPE_F16 || a->out_dtype == HKV_DTYPE_BF16),
                HKV_ERR_ARG, "hkv_prefill_attn: q/chunk/out dtype must be fp16 or bf16");
    HKV_REQUIRE((((uintptr_t)a->q) & 15) == 0 && a->q_stride_b % 8 == 0 && a->q_stride_h % 8 == 0 &&
                    a->q_stride_t % 8 == 0,
                HKV_ERR_ARG, "hkv_prefill_attn: q must be 16-byte aligned with strides multiple of 8");
    HKV_REQUIRE((((uintptr_t)a->out) & 7) == 0 && a->out_stride_b % 4 == 0 && a->out_stride_h % 4 == 0 &&
                    a->out_stride_t % 4 == 0,
                HKV_ERR_ARG, "hkv_prefill_attn: out must be 8-byte aligned with strides multiple of 4");
    if (a->chunk_k || a->chunk_v) {
        HKV_REQUIRE(a->chunk_k && a->chunk_v, HKV_ERR_ARG, "hkv_prefill_attn: chunk K and V must both be given");
        HKV_REQUIRE((((uintptr_t)a->chunk_k | (uintptr_t)a->chunk_v) & 15) == 0 && a->chunk_stride_b % 8 == 0 &&
                        a->chunk_stride_h % 8 == 0 && a->chunk_stride_t % 8 == 0,
                    HKV_ERR_ARG, "hkv_prefill_attn: chunk K/V must be 16-byte aligned, strides multiple of 8");
    }
    HKV_REQUIRE(a->int4_max_len >= 0, HKV_ERR_ARG, "hkv_prefill_attn: int4_max_len < 0");
    if (a->int4_max_len > 0) {
        HKV_REQUIRE(a->block_table && ((a->pool && a->pool_blocks > 0) || (a->staging && a->staging_blocks > 0)),
                    HKV_ERR_ARG, "hkv_prefill_attn: INT4 zone without pool/staging records or block table");
        HKV_REQUIRE(a->pool_blocks >= 0 && a->staging_blocks >= 0 && a->staging_blocks <= (1ll << 31),
                    HKV_ERR_ARG, "hkv_prefill_attn: bad pool/staging block counts");
        HKV_REQUIRE((((uintptr_t)a->pool | (uintptr_t)a->staging) & 15) == 0, HKV_ERR_ARG,
                    "hkv_prefill_attn: pool/staging must be 16-byte aligned");
        HKV_REQUIRE((int64_t)a->bt_stride * kBlockTokens >= a->int4_max_len, HKV_ERR_CAPACITY,
                    "hkv_prefill_attn: block table stride too small");
    }
    for (int i = 0; i < a->num_f16_zones; ++i) {
        const HkvF16Zone& z = a->f16[i];
        HKV_REQUIRE(z.max_len >= 0 && z.max_len <= z.capacity && z.capacity % kBlockTokens == 0, HKV_ERR_ARG,
                    "hkv_prefill_attn: zone %d length/capacity invalid", i);
        if (z.max_len > 0)
            HKV_REQUIRE(z.k && z.v && (((uintptr_t)z.k | (uintptr_t)z.v) & 15) == 0, HKV_ERR_ARG,
                        "hkv_prefill_attn: zone %d k/v null or misaligned", i);
    }
    const int nrep = a->num_q_heads / a->num_kv_heads;
    const int ngrp = (nrep + 3) / 4;
    // the kernels' linear workgroup id (query block, head group) is a 32-bit int
    const int64_t qblocks = ((int64_t)a->num_queries + kFlatQ - 1) / kFlatQ;
    HKV_REQUIRE((int64_t)a->num_kv_heads * ngrp < 65536 && a->batch < 65536 &&
                    qblocks * a->num_kv_heads * ngrp < (1ll << 31),
                HKV_ERR_ARG, "hkv_prefill_attn: grid too large");
    PrefillParams p;
    p.B = a->batch;
    p.Hkv = a->num_kv_heads;
    p.nrep = nrep;
    p.Sq = a->num_queries;
    p.scale_log2 = a->sm_scale * kPfLog2e;
    p.q_bf16 = a->q_dtype == HKV_DTYPE_BF16;
    p.c_bf16 = a->chunk_dtype == HKV_DTYPE_BF16;
    p.out_bf16 = a->out_dtype == HKV_DTYPE_BF16;
    p.q = a->q;
    p.q_sb = a->q_stride_b;
    p.q_sh = a->q_stride_h;
    p.q_st = a->q_stride_t;
    p.nz = a->num_f16_zones;
    for (int i = 0; i < HKV_MAX_F16_ZONES; ++i) {
        const bool on = i < p.nz;
        p.z[i].k = on ? a->f16[i].k : nullptr;
        p.z[i].v = on ? a->f16[i].v : nullptr;
        p.z[i].cap = on ? a->f16[i].capacity : 0;
        p.z[i].max_len = on ? a->f16[i].max_len : 0;
        p.z[i].lens = on ? a->f16[i].lens : nullptr;
    }
    p.pool = a->pool;
    p.pool_blocks = a->pool ? (uint32_t)std::min<int64_t>(a->pool_blocks, 1ll << 31) : 0u;
    p.staging = a->staging;
    p.staging_blocks = a->staging ? (uint32_t)std::min<int64_t>(a->staging_blocks, 1ll << 31) : 0u;
    p.fallback_id = p.pool_blocks > 0 ? 0 : -1;
    p.bt = a->block_table;
    p.bt_stride = a->bt_stride;
    p.int4_lens = a->int4_lens;
    p.int4_max_len = a->int4_max_len;
    p.ck = a->chunk_k;
    p.cv = a->chunk_v;
    p.c_sb = a->chunk_stride_b;
    p.c_sh = a->chunk_stride_h;
    p.c_st = a->chunk_stride_t;
    p.out = a->out;
    p.o_sb = a->out_stride_b;
    p.o_sh = a->out_stride_h;
    p.o_st = a->out_stride_t;
    p.err = a->err_flag;
    // Which kernels run: the zone kernel whenever a sequence may have zone or chunk keys
    // or no INT4 token (it then writes the output), the INT4 kernel whenever there are
    // INT4 tokens; with both kinds of keys the zone kernel's state crosses the workspace.
    // The workspace holds that state, then the chunk's K/V in the zone layout (K rows,
    // 16-token V tiles), written by the zone writer before the zone kernel runs.
    bool zone_keys = a->chunk_k != nullptr;
    for (int i = 0; i < a->num_f16_zones; ++i) zone_keys = zone_keys || a->f16[i].max_len > 0;
    const bool int4_keys = a->int4_max_len > 0;
    const bool run_zones = zone_keys || !int4_keys || a->int4_lens != nullptr;
    const size_t state_bytes = (size_t)a->batch * a->num_q_heads * a->num_queries * kStateFloats * sizeof(float);
    const int ccap = (a->num_queries + kBlockTokens - 1) / kBlockTokens * kBlockTokens;
    const size_t chunk_bytes = (size_t)a->batch * a->num_kv_heads * ccap * kHeadDim * 2;
    if (a->chunk_k != nullptr || (zone_keys && int4_keys)) {
        const size_t need = hkv_prefill_workspace_bytes(a->batch, a->num_q_heads, a->num_queries);
        HKV_REQUIRE(a->workspace != nullptr && a->workspace_bytes >= need && (((uintptr_t)a->workspace) & 15) == 0,
                    HKV_ERR_ARG, "hkv_prefill_attn: a causal chunk, or INT4 and zone keys, need a 16-byte aligned "
                    "workspace of %zu bytes (hkv_prefill_workspace_bytes), got %zu", need,
                    a->workspace ? a->workspace_bytes : 0);
    }
    p.state = (float*)a->workspace;
    p.czk = nullptr;
    p.czv = nullptr;
    p.ccap = ccap;
    for (int i = 0; i < HKV_MAX_F16_ZONES; ++i)
        p.src[i] = PfSrc{p.z[i].k, p.z[i].v, p.z[i].k ? p.z[i].cap : 16, 0};
    p.src[HKV_MAX_F16_ZONES] = PfSrc{nullptr, nullptr, 16, 0};
    if (a->chunk_k != nullptr) {
        uint8_t* ws = (uint8_t*)a->workspace + state_bytes;
        p.czk = (const uint16_t*)ws;
        p.czv = (const uint16_t*)(ws + chunk_bytes);
        p.src[HKV_MAX_F16_ZONES] = PfSrc{p.czk, p.czv, ccap, 0};
        HkvZoneWriteArgs zw = {};
        zw.k = a->chunk_k;
        zw.v = a->chunk_v;
        zw.src_stride_b = a->chunk_stride_b;
        zw.src_stride_h = a->chunk_stride_h;
        zw.src_stride_t = a->chunk_stride_t;
        zw.batch = a->batch;
        zw.num_kv_heads = a->num_kv_heads;
        zw.head_dim = kHeadDim;
        zw.num_tokens = a->num_queries;
        zw.slot_start = nullptr;
        zw.capacity = ccap;
        zw.ring = 0;
        zw.zone_k = (uint16_t*)ws;
        zw.zone_v = (uint16_t*)(ws + chunk_bytes);
        zw.slot_base = 0;
        zw.dtype = a->chunk_dtype;
        zw.err_flag = a->err_flag;
        const int rc = hkv_zone_write(&zw, stream);
        if (rc != HKV_OK) return rc;
    }
    if (run_zones) {
        const int rc = launch_prefill_zones(p, ngrp, (hipStream_t)stream);
        if (rc != HKV_OK) return rc;
    }
    if (int4_keys) {
        const dim3 grid((a->num_queries + kFlatQ - 1) / kFlatQ, a->num_kv_heads * ngrp, a->batch);
        static std::atomic<uint64_t> raised{0};   // four tile buffers exceed the 64 KB default
        HKV_RAISE_LDS(prefill_attn_kernel, kFlatLdsBytes, raised);
        hipLaunchKernelGGL(prefill_attn_kernel, grid, dim3(kFlatThreads), kFlatLdsBytes, (hipStream_t)stream, p);
        HKV_LAUNCH_CHECK("prefill_attn_kernel");
    }
    return HKV_OK;
}

// The state of every (sequence, query head, query row), then the causal chunk's K rows
// and V tiles in the zone layout (sized with the query heads, which bound the kv heads).
extern "C" size_t hkv_prefill_workspace_bytes(int32_t batch, int32_t num_q_heads, int32_t num_queries) {
    if (batch <= 0 || num_q_heads <= 0 || num_queries <= 0) return 0;
    const size_t ccap = ((size_t)num_queries + kBlockTokens - 1) / kBlockTokens * kBlockTokens;
    return (size_t)batch * (size_t)num_q_heads * (size_t)num_queries * kStateFloats * sizeof(float) +
           2 * (size_t)batch * (size_t)num_q_heads * ccap * kHeadDim * 2;
}
