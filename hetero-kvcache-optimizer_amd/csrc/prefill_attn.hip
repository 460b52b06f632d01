// Chunked-prefill attention over [INT4 pool | fp16 zones | causal chunk] on MFMA.
//
// Math (fused_dequant_attn.py:242-247,388-390; kernels/fused_dequant_attn.py:371-435
// is the reference entry point): out[q] = softmax_t(q . K_t * sm_scale) V_t over every
// INT4 token (dequantized exactly as KVCompressor.decompress to fp16), every fp16 zone
// token and the chunk's own tokens t <= q (causal), GQA q head i -> kv head i / n_rep.
//
// Mapping.  A workgroup = 4 wavefronts = 4 query heads of one kv head (a GQA group)
// x 32 query rows; the group shares each 64-token K/V tile, which all 256 lanes
// dequantize / copy into LDS (double buffered, next tile's global loads in flight
// during the current tile's math).  Per wave and tile, with v_mfma_f32_32x32x16_f16:
//   S^T[64 tok x 32 q] = K[tok][d] . Q^T      (2 token blocks x 8 k-steps)
//   O^T[128 d x 32 q] += V^T[d][tok] . P^T    (4 dim blocks x 4 token steps)
// The S^T accumulator of lane (query n, half h) holds tokens 8j + 4h + i, exactly
// the 8-token k-slices the P^T operand needs, so P never leaves registers.  LDS rows
// are XOR-swizzled (16-byte chunks for K, 8-byte units for V^T) against bank conflicts.
#include "hkv_internal.h"
#include "nibble_decode.h"

#include <math.h>

namespace hkv {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

constexpr int kQ = 32;            // query rows per wave
constexpr int kT = 64;            // tokens per tile
constexpr int kWavesP = 4;
constexpr int kThreadsP = 256;
constexpr int kTileBytes = kT * kHeadDim * 2;     // 16 KB for K, 16 KB for V^T
// One LDS tile buffer: K rows, V^T, then per token the K factor (K scale x sm_scale x
// log2 e) and the V scale, fp32.  INT4 tiles hold exact (code - zero point) values and
// the scales are applied to the scores and the probabilities; fp16 tiles hold K and V
// with factors (sm_scale x log2 e, 1).
// A third per-token array holds the score bias: 0, or -inf past the valid length.
constexpr int kSkOff = 2 * kTileBytes, kSvOff = kSkOff + kT * 4, kSbOff = kSvOff + kT * 4;
constexpr int kBufBytes = kSbOff + kT * 4;
constexpr float kLog2eP = 1.4426950408889634f;

struct ZoneP {
    const uint16_t* k;
    const uint16_t* v;
    int cap;
    int max_len;
    const int32_t* lens;
};

struct PrefillParams {
    int B, Hkv, nrep, Sq;
    float scale_log2;
    int q_bf16, c_bf16, out_bf16;   // q / chunk / out dtype is bfloat16 (else fp16)
    const uint16_t* q;
    int64_t q_sb, q_sh, q_st;
    int nz;
    ZoneP z[HKV_MAX_F16_ZONES];
    const uint8_t* pool;
    int64_t pool_blocks;
    const uint8_t* staging;      // records addressed by negative block ids
    int64_t staging_blocks;
    int fallback_id;             // id substituted for an out-of-range one (a valid record)
    const int32_t* bt;
    int bt_stride;
    const int32_t* int4_lens;
    int int4_max_len;
    const uint16_t* ck;          // causal chunk K/V [B][Hkv][Sq][128] (may be null)
    const uint16_t* cv;
    int64_t c_sb, c_sh, c_st;
    uint16_t* out;
    int64_t o_sb, o_sh, o_st;
    int* err;
};

// LDS addresses (bytes) of the swizzled tiles.
__device__ __forceinline__ int k_addr(int tok, int chunk) { return tok * 256 + ((chunk ^ (tok & 15)) << 4); }
// V^T rows hold the tile's 64 tokens in 8-byte units of 4 tokens.  Within each
// 16-token group the units are stored in the order 0, 2, 1, 3, so that the 8 tokens
// one lane feeds to a P.V product (tokens 4hh..4hh+3 and 8+4hh..8+4hh+3 of a group)
// are one 16-byte read; the 16-byte pairs are XOR-swizzled by row against bank
// conflicts.  vt_addr takes the natural unit index (token / 4).
__device__ __forceinline__ int vt_unit(int unit) { return (unit & ~3) | ((unit & 1) << 1) | ((unit >> 1) & 1); }
__device__ __forceinline__ int vt_addr(int dim, int unit) {
    const int su = vt_unit(unit);
    return kTileBytes + dim * 128 + ((((su >> 1) ^ (dim & 7)) << 4) | ((su & 1) << 3));
}
// The 16 bytes holding natural units 4gr + hh and 4gr + 2 + hh (gr = 16-token group).
__device__ __forceinline__ int vt_pair_addr(int dim, int gr, int hh) {
    return kTileBytes + dim * 128 + (((2 * gr + hh) ^ (dim & 7)) << 4);
}

__device__ __forceinline__ uint32_t pack2(float a, float b) {
    return (uint32_t)f2h_rn(a) | ((uint32_t)f2h_rn(b) << 16);
}
__device__ __forceinline__ uint32_t pack2bf(float a, float b) {
    return (uint32_t)f2bf_rn(a) | ((uint32_t)f2bf_rn(b) << 16);
}

// Eight bf16 values to fp16: exact in [2^-14, 65504]; `over` is set when a finite
// value leaves the fp16 range (it becomes +-inf).
__device__ __forceinline__ u4 bf16x8_to_f16(u4 w, bool& over) {
    u4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float lo = __uint_as_float(w[e] << 16), hi = __uint_as_float(w[e] & 0xffff0000u);
        const uint32_t a = f2h_rn(lo), b = f2h_rn(hi);
        over |= (((a & 0x7fffu) == 0x7c00u) && fabsf(lo) < INFINITY) ||
                (((b & 0x7fffu) == 0x7c00u) && fabsf(hi) < INFINITY);
        r[e] = a | (b << 16);
    }
    return r;
}

// Staged global data of one tile for one thread (all tile kinds).
struct Stage {
    u4 a[4];      // K: 4 x 16 B row pieces
    u4 b[4];      // V: 4 x 16 B
    int kind;     // 1 = zone tile, 2 = chunk rows, 3 = empty
    int valid;    // tokens valid in this thread's slice
};

// Tile enumeration: INT4 tiles, then each zone's tiles, then the causal chunk's tiles
// (the generic staging below handles the last two kinds).
struct TileMap {
    int n4, nz_t[HKV_MAX_F16_ZONES], nc;
    int len4, lenz[HKV_MAX_F16_ZONES];
};

__device__ __forceinline__ void stage_load(const PrefillParams& p, const TileMap& tm, int b, int h, int tile,
                                           Stage& s) {
    const int t = threadIdx.x;
    s.kind = 3;
    s.valid = 0;
    int x = tile;
    x -= tm.n4;
#pragma unroll
    for (int zi = 0; zi < HKV_MAX_F16_ZONES; ++zi) {
        if (zi < p.nz && x >= 0 && x < tm.nz_t[zi]) {
            const ZoneP& z = p.z[zi];
            const int64_t bh = (int64_t)b * p.Hkv + h;
            const int tok = x * kT + (t >> 2);        // K row of this thread
            s.kind = 1;
            s.valid = tm.lenz[zi] - x * kT;           // tokens valid in the tile (may exceed 64)
            if (tok < tm.lenz[zi]) {
                const uint16_t* kp = z.k + (bh * z.cap + tok) * kHeadDim + (t & 3) * 32;
#pragma unroll
                for (int j = 0; j < 4; ++j) s.a[j] = *(const u4*)(kp + 8 * j);
            }
            // V: zone tile zt = t/64 of the four 16-token tiles, (g, c) = t%64: 32 halves
            const int zt = x * 4 + (t >> 6);
            if (zt * kBlockTokens < tm.lenz[zi]) {
                const uint16_t* vp = z.v + (bh * (z.cap / kBlockTokens) + zt) * (kBlockTokens * kHeadDim) + (t & 63) * 32;
#pragma unroll
                for (int j = 0; j < 4; ++j) s.b[j] = *(const u4*)(vp + 8 * j);
            }
            x = -1;
        }
        if (zi < p.nz && x >= 0) x -= tm.nz_t[zi];
    }
    if (x >= 0 && x < tm.nc && p.ck) {
        const int tok = x * kT + (t >> 2);
        s.kind = 2;
        s.valid = p.Sq - x * kT;
        if (tok < p.Sq) {
            const uint16_t* kp = p.ck + (int64_t)b * p.c_sb + (int64_t)h * p.c_sh + (int64_t)tok * p.c_st + (t & 3) * 32;
            const uint16_t* vp = p.cv + (int64_t)b * p.c_sb + (int64_t)h * p.c_sh + (int64_t)tok * p.c_st + (t & 3) * 32;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                s.a[j] = *(const u4*)(kp + 8 * j);
                s.b[j] = *(const u4*)(vp + 8 * j);
            }
        }
    }
}

// Writes the staged data of one tile into LDS buffer `lds` (K rows + V^T), zeros for
// slots past the valid length so that masked probabilities multiply finite values.
__device__ __forceinline__ void stage_store(Stage& s, uint8_t* lds, float scale_log2, bool chunk_bf16, int* err) {
    const int t = threadIdx.x;
    if (chunk_bf16 && s.kind == 2) {
        // rows past the chunk were not loaded: converted (and later zeroed), never checked
        bool over = false;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            s.a[j] = bf16x8_to_f16(s.a[j], over);
            s.b[j] = bf16x8_to_f16(s.b[j], over);
        }
        over = over && (t >> 2) < s.valid;
        if (__ballot(over) && (t & 63) == 0 && err) atomicOr(err, HKV_ERR_BIT_RANGE);
    }
    if (t < kT) {
        ((float*)(lds + kSkOff))[t] = scale_log2;
        ((float*)(lds + kSvOff))[t] = 1.0f;
        ((float*)(lds + kSbOff))[t] = s.kind != 3 && t < s.valid ? 0.0f : -INFINITY;
    }
    {
        const int tok = t >> 2, pt = t & 3;
        const bool okk = s.kind != 3 && tok < s.valid;
#pragma unroll
        for (int j = 0; j < 4; ++j) *(u4*)(lds + k_addr(tok, pt * 4 + j)) = okk ? s.a[j] : u4{0u, 0u, 0u, 0u};
        if (s.kind == 1) {
            // zone V tile zt: halves [n][i] = V[4g+i][c+16n] -> V^T rows c+16n, unit zt*4+g
            const int zt = t >> 6, g = (t & 63) >> 4, c = t & 15;
            const int base_tok = zt * 16 + 4 * g;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const int n = 2 * j + e;
                    u2 val = e == 0 ? u2{s.b[j].x, s.b[j].y} : u2{s.b[j].z, s.b[j].w};
                    // clear tokens past the length
                    const uint32_t m01 = (base_tok + 0 < s.valid ? 0x0000FFFFu : 0u) | (base_tok + 1 < s.valid ? 0xFFFF0000u : 0u);
                    const uint32_t m23 = (base_tok + 2 < s.valid ? 0x0000FFFFu : 0u) | (base_tok + 3 < s.valid ? 0xFFFF0000u : 0u);
                    val.x &= m01;
                    val.y &= m23;
                    *(u2*)(lds + vt_addr(c + 16 * n, zt * 4 + g)) = val;
                }
            }
        } else {
            // row-major V (chunk) or empty: scatter 32 dims of token `tok` into V^T
#pragma unroll
            for (int e = 0; e < 32; ++e) {
                const int d = pt * 32 + e;
                const uint32_t w = s.b[e >> 3][(e >> 1) & 3];
                const uint16_t v = okk ? (uint16_t)(w >> ((e & 1) * 16)) : (uint16_t)0;
                *(uint16_t*)(lds + vt_addr(d, tok >> 2) + (tok & 3) * 2) = v;
            }
        }
    }
}

// Compact staged data of one INT4 tile for one thread (the INT4 phase keeps kRing of
// them in flight).  Each stage also carries the block id of the tile kRing further on,
// so no load ever waits for a block id issued after other loads.
struct Stage4 {
    u4 k;         // K codes: token (t/4)%16 of block t/64, dims 32(t%4) .. +32
    u4 v;         // V words (t%64)*4 .. +3 of block t/64
    f4 vs;        // V scales of tokens 4g..4g+3, g = (t%64)/16
    float ks;     // K scale of the K row
    uint32_t kz;  // K zero point of the K row (low byte)
    uint32_t vz;  // V zero points of tokens 4g..4g+3 (bytes)
    int valid;    // valid tokens of block t/64 (0 past the end)
    int next_id;  // block id of this thread's block in tile + kRing
};
constexpr int kRing = 2;          // INT4 tiles in flight per thread (4 measured slower: register pressure)

// Block id of this thread's block (t/64) of INT4 tile x, clamped to the last block.
__device__ __forceinline__ int block_id4(const PrefillParams& p, int nb, int b, int x) {
    const int lb = min(x * 4 + (int)(threadIdx.x >> 6), nb - 1);
    return p.bt[(int64_t)b * p.bt_stride + lb];
}

// Loads INT4 tile `tile` (past the end it re-reads the last block and carries no valid
// token) from block id `id`, and the id of tile + kRing.
__device__ __forceinline__ void load4(const PrefillParams& p, int n4, int len4, int b, int h, int tile, int id,
                                      Stage4& s) {
    const int t = threadIdx.x;
    const int nb = (len4 + kBlockTokens - 1) / kBlockTokens;
    int phys = id;
    if (phys >= 0 ? (int64_t)phys >= p.pool_blocks : (int64_t)(~phys) >= p.staging_blocks) {
        if (p.err) atomicOr(p.err, 1);
        phys = p.fallback_id;
    }
    const int64_t rb = (int64_t)p.Hkv * kHeadPartBytes;
    const uint8_t* part = (phys >= 0 ? p.pool + (int64_t)phys * rb : p.staging + (int64_t)(~phys) * rb) +
                          RecordLayout::part(h);
    const int rr = (t >> 2) & 15, pt = t & 3, g = (t & 63) >> 4;
    const int lbt = tile * 4 + (t >> 6);
    s.valid = (tile < n4 && lbt < nb) ? min(kBlockTokens, len4 - lbt * kBlockTokens) : 0;
    s.k = *(const u4*)(part + kPartKc + rr * 64 + pt * 16);
    s.ks = *(const float*)(part + kPartKs + rr * 4);
    s.kz = *(const uint32_t*)(part + kPartKz + (rr & ~3)) >> (8 * (rr & 3));   // a word load, no byte value
    s.v = *(const u4*)(part + kPartVc + (t & 63) * 16);
    s.vs = *(const f4*)(part + kPartVs + g * 16);
    s.vz = *(const uint32_t*)(part + kPartVz + g * 4);
    s.next_id = block_id4(p, nb, b, min(tile + kRing, n4 - 1));
}

// Writes a staged INT4 tile into LDS buffer `lds`: K rows and V^T as exact fp16
// (code - zero point) values, and the per-token factors.  Tokens past the valid
// length hold finite values (their block is a valid record) and are masked in the
// scores.
__device__ __forceinline__ void store4(const Stage4& s, uint8_t* lds, float scale_log2) {
    const int t = threadIdx.x;
    const int blk = t >> 6, rr = (t >> 2) & 15, pt = t & 3;
    const int tok = blk * 16 + rr;
    const uint32_t kz = s.kz & 0xFFu;
    const h2 kz1024 = zp1024(kz, kz), kz64 = zp64(kz, kz);
    const uint32_t w4[4] = {s.k.x, s.k.y, s.k.z, s.k.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {          // word j: dims 32pt + 8j .. +8
        const NibPairs a = unpack_word(w4[j], kz1024, kz64);
        *(u4*)(lds + k_addr(tok, pt * 4 + j)) =
            u4{__builtin_bit_cast(uint32_t, a.p0), __builtin_bit_cast(uint32_t, a.p1),
               __builtin_bit_cast(uint32_t, a.p2), __builtin_bit_cast(uint32_t, a.p3)};
    }
    if (pt == 0) {
        ((float*)(lds + kSkOff))[tok] = s.ks * scale_log2;
        ((float*)(lds + kSbOff))[tok] = rr < s.valid ? 0.0f : -INFINITY;
    }
    // V word (t%64)*4 + mm: x0..x3 = tokens 4g..4g+3 at dim c+32mm, x4..x7 at +16
    const int g = (t & 63) >> 4, c = t & 15;
    const h2 z01 = zp1024(s.vz & 0xFFu, (s.vz >> 8) & 0xFFu), z23 = zp64((s.vz >> 16) & 0xFFu, s.vz >> 24);
    const uint32_t v4[4] = {s.v.x, s.v.y, s.v.z, s.v.w};
    const int unit = blk * 4 + g;
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) {
        const NibPairs a = unpack_word(v4[mm], z01, z23);
        const int d1 = c + 32 * mm, d2 = d1 + 16;
        *(u2*)(lds + vt_addr(d1, unit)) = u2{__builtin_bit_cast(uint32_t, a.p0), __builtin_bit_cast(uint32_t, a.p1)};
        *(u2*)(lds + vt_addr(d2, unit)) = u2{__builtin_bit_cast(uint32_t, a.p2), __builtin_bit_cast(uint32_t, a.p3)};
    }
    if (c == 0) *(f4*)(lds + kSvOff + (blk * 16 + 4 * g) * 4) = s.vs;
}

// One 64-token tile of attention for this wave's 32 query rows: S^T = K.Q^T, masked
// online softmax, O^T += V^T.P^T.  `cur` holds the tile's K rows and V^T in LDS.
// kCausal: the tile is a piece of the causal chunk starting at chunk position
// causal_base; token t is visible to query row qrow when t < tvalid and
// causal_base + t <= qrow.  Otherwise the tile's bias array masks it.
template <bool kCausal>
__device__ __forceinline__ void attend_tile(const uint8_t* cur, int tvalid, int causal_base, int n, int hh,
                                            int qrow, const h8 (&qf)[8], f16v (&acc)[4], float& m, float& l) {
    // Phases are kept apart (sched_barrier) so that at most one token block's operands
    // are live at a time: the kernel then fits two waves per SIMD.
    f16v S[2];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) S[tb][r] = 0.f;
        const int tok = tb * 32 + n;
        h8 a[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) a[s] = __builtin_bit_cast(h8, *(const u4*)(cur + k_addr(tok, 2 * s + hh)));
#pragma unroll
        for (int s = 0; s < 8; ++s) S[tb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[s], qf[s], S[tb], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
    }
    // lane (n, hh) holds tokens tb*32 + 8j + 4hh + i for r = 4j + i: four consecutive
    // tokens per j, whose factors are one 16-byte LDS read
    float mt = -INFINITY;
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
        f4 fk[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) fk[j] = *(const f4*)(cur + kSkOff + (tb * 32 + 8 * j + 4 * hh) * 4);
        if constexpr (kCausal) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int tok = tb * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
                const bool ok = tok < tvalid && causal_base + tok <= qrow;
                S[tb][r] = ok ? S[tb][r] * fk[r >> 2][r & 3] : -INFINITY;
                mt = fmaxf(mt, S[tb][r]);
            }
        } else {
            f4 fb[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) fb[j] = *(const f4*)(cur + kSbOff + (tb * 32 + 8 * j + 4 * hh) * 4);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                S[tb][r] = __builtin_fmaf(S[tb][r], fk[r >> 2][r & 3], fb[r >> 2][r & 3]);
                mt = fmaxf(mt, S[tb][r]);
            }
        }
    }
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    if (__ballot(mt > m)) {
        const float m_new = fmaxf(m, mt);
        const float alpha = (m_new > m) ? __builtin_amdgcn_exp2f(m - m_new) : 1.0f;
#pragma unroll
        for (int db = 0; db < 4; ++db) acc[db] *= alpha;
        l *= alpha;
        m = m_new;
    }
    const float msafe = (m == -INFINITY) ? 0.f : m;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
        f4 fv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) fv[j] = *(const f4*)(cur + kSvOff + (tb * 32 + 8 * j + 4 * hh) * 4);
        h8 P[2];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int jj = 0; jj < 2; ++jj)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = 4 * (2 * u + jj) + i;
                    const float pv = __builtin_amdgcn_exp2f(S[tb][r] - msafe);
                    l += pv;
                    P[u][jj * 4 + i] = (_Float16)(pv * fv[r >> 2][r & 3]);
                }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            // tokens tb*32 + 16u + 4hh .. +3 and +8 .. +11: 16-token group 2tb + u
            h8 a[4];
#pragma unroll
            for (int db = 0; db < 4; ++db)
                a[db] = __builtin_bit_cast(h8, *(const u4*)(cur + vt_pair_addr(32 * db + n, 2 * tb + u, hh)));
#pragma unroll
            for (int db = 0; db < 4; ++db) acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[db], P[u], acc[db], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Two workgroups per CU (two waves per SIMD): one wave's MFMA chains overlap the
// other's dequantization and softmax.  This caps a wave at 256 registers; the few
// values spilled are kernel-wide addresses read outside the INT4 tile loop.
__global__ __launch_bounds__(kThreadsP, 2) void prefill_attn_kernel(PrefillParams p) {
    extern __shared__ __align__(16) uint8_t lds_raw[];
    const int b = blockIdx.z;
    const int ngrp = (p.nrep + kWavesP - 1) / kWavesP;
    const int h = blockIdx.y / ngrp, grp = blockIdx.y % ngrp;
    const int q0 = blockIdx.x * kQ;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 31, hh = lane >> 5;
    const int rep = grp * kWavesP + wave;
    const bool head_ok = rep < p.nrep;
    const int qh = h * p.nrep + (head_ok ? rep : 0);
    const int qrow = q0 + n;

    TileMap tm;
    tm.len4 = p.int4_lens ? min(max(p.int4_lens[b], 0), p.int4_max_len) : p.int4_max_len;
    tm.n4 = (tm.len4 + kT - 1) / kT;
#pragma unroll
    for (int zi = 0; zi < HKV_MAX_F16_ZONES; ++zi) {
        tm.lenz[zi] = 0;
        if (zi < p.nz) tm.lenz[zi] = p.z[zi].lens ? min(max(p.z[zi].lens[b], 0), p.z[zi].max_len) : p.z[zi].max_len;
        tm.nz_t[zi] = (tm.lenz[zi] + kT - 1) / kT;
    }
    // causal chunk tiles up to the last query row of this block
    tm.nc = p.ck ? (min(q0 + kQ, p.Sq) + kT - 1) / kT : 0;
    int ntiles = tm.n4 + tm.nc;
#pragma unroll
    for (int zi = 0; zi < HKV_MAX_F16_ZONES; ++zi) ntiles += (zi < p.nz) ? tm.nz_t[zi] : 0;
    const int first_chunk_tile = ntiles - tm.nc;

    // Q^T fragments: lane (query n, half hh) step s -> q[qrow][16s + 8hh .. +8]
    h8 qf[8];
    {
        const bool ok = head_ok && qrow < p.Sq;
        const uint16_t* qp = p.q + (int64_t)b * p.q_sb + (int64_t)qh * p.q_sh + (int64_t)(ok ? qrow : 0) * p.q_st + 8 * hh;
        bool over = false;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            u4 w = ok ? *(const u4*)(qp + 16 * s) : u4{0u, 0u, 0u, 0u};
            if (p.q_bf16) w = bf16x8_to_f16(w, over);
            qf[s] = __builtin_bit_cast(h8, w);
        }
        if (__ballot(over) && lane == 0 && p.err) atomicOr(p.err, HKV_ERR_BIT_RANGE);
    }
    f16v acc[4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
    float m = -INFINITY, l = 0.f;

    // ---- INT4 tiles: kRing staged tiles in flight; tile t is computed from LDS buffer
    // t % 2 while tile t + 1 is dequantized into the other buffer.  The tile count is
    // padded to a multiple of kRing (padding tiles carry no valid token) so the ring
    // slots stay compile-time registers.
    const int n4 = tm.n4;
    const int n4p = n4 > 0 ? (n4 + kRing - 1) / kRing * kRing : 0;
    if (n4 > 0) {
        Stage4 ring[kRing];
        const int nb4 = (tm.len4 + kBlockTokens - 1) / kBlockTokens;
        int id0[kRing];
#pragma unroll
        for (int u = 0; u < kRing; ++u) id0[u] = block_id4(p, nb4, b, min(u, n4 - 1));
#pragma unroll
        for (int u = 0; u < kRing - 1; ++u) {
            __builtin_amdgcn_sched_barrier(0);
            load4(p, n4, tm.len4, b, h, u, id0[u], ring[u]);
            __builtin_amdgcn_sched_barrier(0);
        }
        ring[kRing - 1].next_id = id0[kRing - 1];
        store4(ring[0], lds_raw, p.scale_log2);
        __syncthreads();
        for (int t0 = 0; t0 < n4p; t0 += kRing) {
#pragma unroll
            for (int u = 0; u < kRing; ++u) {
                const int tile = t0 + u;
                __builtin_amdgcn_sched_barrier(0);
                Stage4& slot = ring[(u + kRing - 1) % kRing];
                load4(p, n4, tm.len4, b, h, tile + kRing - 1, slot.next_id, slot);
                __builtin_amdgcn_sched_barrier(0);
                const int tvalid = min(kT, tm.len4 - tile * kT);
                attend_tile<false>(lds_raw + (tile & 1) * kBufBytes, tvalid, -1, n, hh, qrow, qf, acc, m, l);
                store4(ring[(u + 1) % kRing], lds_raw + ((tile + 1) & 1) * kBufBytes, p.scale_log2);
                __syncthreads();
            }
        }
    }

    // ---- fp16 zone tiles and the causal chunk: one staged tile in flight
    Stage st;
    const int par0 = n4p;   // LDS buffer parity continues after the INT4 tiles
    if (ntiles > n4) {
        stage_load(p, tm, b, h, n4, st);
        stage_store(st, lds_raw + (par0 & 1) * kBufBytes, p.scale_log2, p.c_bf16 != 0, p.err);
    }
    __syncthreads();
    for (int tile = n4; tile < ntiles; ++tile) {
        const int par = par0 + (tile - n4);
        uint8_t* cur = lds_raw + (par & 1) * kBufBytes;
        uint8_t* nxt = lds_raw + ((par + 1) & 1) * kBufBytes;
        if (tile + 1 < ntiles) stage_load(p, tm, b, h, tile + 1, st);

        // valid tokens of this tile and causal limit
        int tvalid = kT;
        int causal_base = -1;  // chunk position of token 0 of this tile, or -1
        {
            int x = tile - tm.n4;
            bool found = false;
#pragma unroll
            for (int zi = 0; zi < HKV_MAX_F16_ZONES; ++zi) {
                if (!found && zi < p.nz) {
                    if (x < tm.nz_t[zi]) {
                        tvalid = min(kT, tm.lenz[zi] - x * kT);
                        found = true;
                    } else {
                        x -= tm.nz_t[zi];
                    }
                }
            }
            if (!found) {
                tvalid = min(kT, p.Sq - x * kT);
                causal_base = x * kT;
            }
        }
        if (causal_base >= 0)
            attend_tile<true>(cur, tvalid, causal_base, n, hh, qrow, qf, acc, m, l);
        else
            attend_tile<false>(cur, tvalid, causal_base, n, hh, qrow, qf, acc, m, l);
        if (tile + 1 < ntiles) stage_store(st, nxt, p.scale_log2, p.c_bf16 != 0, p.err);
        __syncthreads();
    }
    (void)first_chunk_tile;

    l += __shfl_xor(l, 32);
    if (head_ok && qrow < p.Sq) {
        const float inv = l > 0.f ? 1.0f / l : 0.f;
        uint16_t* op = p.out + (int64_t)b * p.o_sb + (int64_t)qh * p.o_sh + (int64_t)qrow * p.o_st;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d = 32 * db + 8 * j + 4 * hh;
                if (p.out_bf16)
                    *(u2*)(op + d) = u2{pack2bf(acc[db][4 * j + 0] * inv, acc[db][4 * j + 1] * inv),
                                        pack2bf(acc[db][4 * j + 2] * inv, acc[db][4 * j + 3] * inv)};
                else
                    *(u2*)(op + d) = u2{pack2(acc[db][4 * j + 0] * inv, acc[db][4 * j + 1] * inv),
                                        pack2(acc[db][4 * j + 2] * inv, acc[db][4 * j + 3] * inv)};
            }
    }
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
    const int ngrp = (nrep + kWavesP - 1) / kWavesP;
    HKV_REQUIRE((int64_t)a->num_kv_heads * ngrp < 65536 && a->batch < 65536, HKV_ERR_ARG,
                "hkv_prefill_attn: grid too large");
    PrefillParams p;
    p.B = a->batch;
    p.Hkv = a->num_kv_heads;
    p.nrep = nrep;
    p.Sq = a->num_queries;
    p.scale_log2 = a->sm_scale * kLog2eP;
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
    p.pool_blocks = a->pool ? a->pool_blocks : 0;
    p.staging = a->staging;
    p.staging_blocks = a->staging ? a->staging_blocks : 0;
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
    const dim3 grid((a->num_queries + kQ - 1) / kQ, a->num_kv_heads * ngrp, a->batch);
    static bool raised = false;   // two tile buffers are a little over 64 KB
    if (!raised) {
        HKV_HIP_CHECK(hipFuncSetAttribute((const void*)prefill_attn_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                          2 * kBufBytes));
        raised = true;
    }
    hipLaunchKernelGGL(prefill_attn_kernel, grid, dim3(kThreadsP), 2 * kBufBytes, (hipStream_t)stream, p);
    HKV_LAUNCH_CHECK("prefill_attn_kernel");
    return HKV_OK;
}
