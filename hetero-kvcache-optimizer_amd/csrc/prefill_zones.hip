// Chunked prefill, zone kernel: the fp16 zone tiles and the causal chunk of every
// sequence (fused_dequant_attn.py:242-247 with kernels/fused_dequant_attn.py:371-435 as
// the entry point; the INT4 tiles are prefill_attn.hip's).  When the sequence also has
// INT4 tokens, it leaves its online-softmax state for the INT4 kernel; otherwise it
// writes the output.
//
// Mapping.  A workgroup = 4 wavefronts = 4 query heads of one kv head (a GQA group)
// x 32 query rows; the group shares each 64-token K/V tile, which all 256 lanes copy
// into LDS (double buffered, next tile's global loads in flight during the current
// tile's math).  Per wave and tile, with v_mfma_f32_32x32x16_f16:
//   S^T[64 tok x 32 q] = K[tok][d] . Q^T      (2 token blocks x 8 k-steps)
//   O^T[128 d x 32 q] += V^T[d][tok] . P^T    (4 dim blocks x 4 token steps)
// The S^T accumulator of lane (query n, half h) holds tokens 8j + 4h + i, exactly
// the 8-token k-slices the P^T operand needs, so P never leaves registers.  LDS rows
// are XOR-swizzled (16-byte chunks for K, 8-byte units for V^T) against bank conflicts.
#include "prefill_common.h"

#include <math.h>

namespace hkv {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef PfZone ZoneP;

constexpr int kQ = kPfQ;          // query rows per wave
constexpr int kT = kPfT;          // tokens per tile
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

// Staged global data of one tile for one thread (all tile kinds).
struct Stage {
    u4 a[4];      // K: 4 x 16 B row pieces
    u4 b[4];      // V: 4 x 16 B
    int kind;     // 1 = zone tile, 2 = chunk rows, 3 = empty
    int valid;    // tokens valid in this thread's slice
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

__global__ __launch_bounds__(kThreadsP, 2) void prefill_zones_kernel(PrefillParams p) {
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
    make_tile_map(p, b, q0 + kQ, tm);
    const int nf = tm.nf();
    // Sequences with INT4 tokens and no zone or chunk tile: the INT4 kernel starts at zero
    if (tm.n4 > 0 && nf == 0) return;
    const int ntiles = tm.n4 + nf;

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

    // ---- fp16 zone tiles and the causal chunk: one staged tile in flight
    Stage st;
    if (nf > 0) {
        stage_load(p, tm, b, h, tm.n4, st);
        stage_store(st, lds_raw, p.scale_log2, p.c_bf16 != 0, p.err);
    }
    __syncthreads();
    for (int tile = tm.n4; tile < ntiles; ++tile) {
        const int par = tile - tm.n4;
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
    if (tm.n4 > 0) {
        // INT4 tokens follow in the INT4 kernel: leave this lane's state (O relative to m,
        // m, and its half-row sum l) for it
        if (head_ok && qrow < p.Sq) {
            float* st_row = state_row(p, b, qh, qrow);
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    *(f4*)(st_row + 32 * db + 8 * j + 4 * hh) =
                        f4{acc[db][4 * j + 0], acc[db][4 * j + 1], acc[db][4 * j + 2], acc[db][4 * j + 3]};
            st_row[kHeadDim + 1 + hh] = l;
            if (hh == 0) st_row[kHeadDim] = m;
        }
        return;
    }
    l += __shfl_xor(l, 32);
    if (head_ok && qrow < p.Sq) write_out(p, b, qh, qrow, hh, acc, l);
}

}  // namespace

int launch_prefill_zones(const PrefillParams& p, int ngrp, hipStream_t stream) {
    const dim3 grid((p.Sq + kQ - 1) / kQ, p.Hkv * ngrp, p.B);
    static bool raised = false;   // two tile buffers are a little over 64 KB
    if (!raised) {
        HKV_HIP_CHECK(hipFuncSetAttribute((const void*)prefill_zones_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                          2 * kBufBytes));
        raised = true;
    }
    hipLaunchKernelGGL(prefill_zones_kernel, grid, dim3(kThreadsP), 2 * kBufBytes, stream, p);
    HKV_LAUNCH_CHECK("prefill_zones_kernel");
    return HKV_OK;
}

}  // namespace hkv
