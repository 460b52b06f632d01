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
// Work split: a "unit" (8 INT4 blocks or 2 fp16 tiles, ~17 KB) per wave, 4 waves
// per workgroup; a workgroup's waves merge through LDS, workgroups of one
// (sequence, kv head) merge through a workspace, and the last workgroup to
// finish (atomic ticket) writes the output.  Workgroup ids interleave the
// (sequence, kv head) pairs so that all splits of a pair land on one XCD.
#include "hkv_internal.h"

#include <math.h>

namespace hkv {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;
constexpr int kUnitInt4Blocks = 8;
constexpr int kUnitF16Tiles = 2;
constexpr int kPartStride = kHeadDim + 2;  // o[128], m, l
constexpr int kPrefetch = 3;
constexpr float kLog2e = 1.4426950408889634f;

__host__ __device__ inline int units_int4(int len) {
    const int nb = (len + kBlockTokens - 1) / kBlockTokens;
    return (nb + kUnitInt4Blocks - 1) / kUnitInt4Blocks;
}
__host__ __device__ inline int units_f16(int len) {
    const int nt = (len + kBlockTokens - 1) / kBlockTokens;
    return (nt + kUnitF16Tiles - 1) / kUnitF16Tiles;
}

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
    const uint16_t* q;
    int64_t q_sb, q_sh;
    int nz;
    ZoneP z[HKV_MAX_F16_ZONES];
    const uint8_t* pool;
    int64_t pool_blocks;
    const int32_t* bt;
    int bt_stride;
    const int32_t* int4_lens;
    int int4_max_len;
    uint16_t* out;
    int64_t o_sb, o_sh;
    int* err;
    int* counters;
    float* partials;
    int max_splits;
};

__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }

// (w >> 4i) & 0x000F000F | 0x6400_6400  ->  fp16 pair (1024 + x_2i, 1024 + x_2i+1)
__device__ __forceinline__ uint32_t nib_pair(uint32_t w, int i) {
    return ((w >> (4 * i)) & 0x000F000Fu) | 0x64006400u;
}

struct Int4Blk {
    u4 k;         // K codes of token (lane%16), dims 32g..32g+31
    u4 v;         // V codes: tokens 4g..4g+3, dims c+16n (n=0..7)
    f4 ks;        // K scales of tokens 4g..4g+3
    f4 vs;        // V scales of tokens 4g..4g+3
    uint32_t kz;  // K zero point of token (lane%16)
    uint32_t vz;  // V zero points of tokens 4g..4g+3 (bytes)
};

struct F16Tile {
    u4 k[4];      // K row of token (lane%16), dims 32g + 8j .. +8
    u4 v[4];      // V^T tile: halves [n][i] for tokens 4g+i, dims c+16n
};

__device__ __forceinline__ void load_int4(const DecodeParams& p, int b, int h, int lb, int c, int g,
                                          Int4Blk& d) {
    int phys = p.bt[(int64_t)b * p.bt_stride + lb];
    if (phys < 0 || (int64_t)phys >= p.pool_blocks) {
        if (p.err) atomicOr(p.err, 1);
        phys = 0;
    }
    const int H = p.Hkv;
    const uint8_t* rec = p.pool + (int64_t)phys * ((int64_t)H * 2208);
    d.k = *(const u4*)(rec + h * kHeadCodeBytes + c * kCodeRowBytes + g * 16);
    d.v = *(const u4*)(rec + (int64_t)H * 1024 + h * kHeadCodeBytes + (g * 16 + c) * 16);
    d.ks = *(const f4*)(rec + (int64_t)H * 2048 + h * 64 + g * 16);
    d.vs = *(const f4*)(rec + (int64_t)H * 2112 + h * 64 + g * 16);
    d.kz = rec[(int64_t)H * 2176 + h * 16 + c];
    d.vz = *(const uint32_t*)(rec + (int64_t)H * 2192 + h * 16 + g * 4);
}

__device__ __forceinline__ void load_f16(const ZoneP& z, int64_t bh, int tile, int c, int g, F16Tile& d) {
    const uint16_t* kp = z.k + ((bh * z.cap + (int64_t)tile * kBlockTokens + c) * kHeadDim) + 32 * g;
    const uint16_t* vp = z.v + (bh * (z.cap / kBlockTokens) + tile) * (kBlockTokens * kHeadDim) +
                         (g * 16 + c) * 32;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        d.k[j] = *(const u4*)(kp + 8 * j);
        d.v[j] = *(const u4*)(vp + 8 * j);
    }
}

// Online-softmax update shared by both tile kinds.  s[] are log2-domain scores
// (-inf for masked tokens); returns the probabilities for tokens 4g..4g+3.
__device__ __forceinline__ void softmax_update(float (&s)[4], f4 (&acc)[8], float& m, float& l,
                                               float (&pr)[4]) {
    float mt = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    mt = fmaxf(mt, __shfl_xor(mt, 16));
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    const float m_new = fmaxf(m, mt);
    if (__ballot(m_new > m)) {
        const float alpha = (m_new > m) ? exp2f(m - m_new) : 1.0f;
#pragma unroll
        for (int n = 0; n < 8; ++n) acc[n] *= alpha;
        l *= alpha;
        m = m_new;
    }
    const float msafe = (m == -INFINITY) ? 0.0f : m;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        pr[v] = exp2f(s[v] - msafe);
        l += pr[v];
    }
}

__device__ __forceinline__ void step_int4(const Int4Blk& d, int nvalid, int g, const h8 (&qf)[4],
                                          float scale_log2, f4 (&acc)[8], float& m, float& l) {
    // ---- scores
    const _Float16 kzz = (_Float16)(1024.0f + (float)d.kz);
    const h2 kz2 = {kzz, kzz};
    const uint32_t kw[4] = {d.k.x, d.k.y, d.k.z, d.k.w};
    f4 S = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const h2 a0 = as_h2(nib_pair(kw[j], 0)) - kz2;
        const h2 a1 = as_h2(nib_pair(kw[j], 1)) - kz2;
        const h2 a2 = as_h2(nib_pair(kw[j], 2)) - kz2;
        const h2 a3 = as_h2(nib_pair(kw[j], 3)) - kz2;
        const h8 a = {a0[0], a0[1], a1[0], a1[1], a2[0], a2[1], a3[0], a3[1]};
        S = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[j], S, 0, 0, 0);
    }
    float s[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) s[v] = (4 * g + v < nvalid) ? S[v] * (d.ks[v] * scale_log2) : -INFINITY;
    float pr[4];
    softmax_update(s, acc, m, l, pr);
    // ---- P' = p * v_scale (exactly 0 for masked tokens)
    h4 P;
#pragma unroll
    for (int v = 0; v < 4; ++v) P[v] = (_Float16)((4 * g + v < nvalid) ? pr[v] * d.vs[v] : 0.0f);
    const _Float16 z0 = (_Float16)(1024.0f + (float)(d.vz & 0xff));
    const _Float16 z1 = (_Float16)(1024.0f + (float)((d.vz >> 8) & 0xff));
    const _Float16 z2 = (_Float16)(1024.0f + (float)((d.vz >> 16) & 0xff));
    const _Float16 z3 = (_Float16)(1024.0f + (float)(d.vz >> 24));
    const h2 zz01 = {z0, z1}, zz23 = {z2, z3};
    const uint32_t vw[4] = {d.v.x, d.v.y, d.v.z, d.v.w};
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) {
        const h2 e0 = as_h2(nib_pair(vw[mm], 0)) - zz01;
        const h2 e1 = as_h2(nib_pair(vw[mm], 1)) - zz23;
        const h2 o0 = as_h2(nib_pair(vw[mm], 2)) - zz01;
        const h2 o1 = as_h2(nib_pair(vw[mm], 3)) - zz23;
        const h4 A0 = {e0[0], e0[1], e1[0], e1[1]};
        const h4 A1 = {o0[0], o0[1], o1[0], o1[1]};
        acc[2 * mm] = __builtin_amdgcn_mfma_f32_16x16x16f16(A0, P, acc[2 * mm], 0, 0, 0);
        acc[2 * mm + 1] = __builtin_amdgcn_mfma_f32_16x16x16f16(A1, P, acc[2 * mm + 1], 0, 0, 0);
    }
}

__device__ __forceinline__ void step_f16(F16Tile& d, int nvalid, int g, const h8 (&qf)[4],
                                         float scale_log2, f4 (&acc)[8], float& m, float& l) {
    f4 S = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) S = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, d.k[j]), qf[j], S, 0, 0, 0);
    float s[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) s[v] = (4 * g + v < nvalid) ? S[v] * scale_log2 : -INFINITY;
    float pr[4];
    softmax_update(s, acc, m, l, pr);
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

__global__ __launch_bounds__(256) void decode_attn_kernel(DecodeParams p) {
    const int BH = p.B * p.Hkv;
    const int bh = blockIdx.x % BH;
    const int split = blockIdx.x / BH;
    const int b = bh / p.Hkv, h = bh % p.Hkv;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 15, g = lane >> 4;
    const int nrep = p.nrep;

    const int len4 = p.int4_lens ? min(max(p.int4_lens[b], 0), p.int4_max_len) : p.int4_max_len;
    const int n4 = units_int4(len4);
    int lenz[HKV_MAX_F16_ZONES], nzu[HKV_MAX_F16_ZONES];
    int total = n4;
#pragma unroll
    for (int zi = 0; zi < HKV_MAX_F16_ZONES; ++zi) {
        lenz[zi] = 0;
        nzu[zi] = 0;
        if (zi < p.nz) {
            lenz[zi] = p.z[zi].lens ? min(max(p.z[zi].lens[b], 0), p.z[zi].max_len) : p.z[zi].max_len;
            nzu[zi] = units_f16(lenz[zi]);
            total += nzu[zi];
        }
    }
    const int nsplit = max((total + kWaves - 1) / kWaves, 1);
    if (split >= nsplit) return;

    // q fragments: lane (c, g) holds q[head c][32g + 8j .. +8] for step j.
    h8 qf[4];
    {
        const bool has = c < nrep;
        const uint16_t* qp = p.q + (int64_t)b * p.q_sb + (int64_t)(h * nrep + (has ? c : 0)) * p.q_sh + 32 * g;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const u4 w = has ? *(const u4*)(qp + 8 * j) : u4{0u, 0u, 0u, 0u};
            qf[j] = __builtin_bit_cast(h8, w);
        }
    }

    f4 acc[8];
#pragma unroll
    for (int n = 0; n < 8; ++n) acc[n] = f4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.0f;

    int u = split * kWaves + wave;
    if (u < n4) {
        const int nb = (len4 + kBlockTokens - 1) / kBlockTokens;
        const int lb0 = u * kUnitInt4Blocks;
        const int lb1 = min(lb0 + kUnitInt4Blocks, nb);
        Int4Blk buf[kPrefetch];
#pragma unroll
        for (int k = 0; k < kPrefetch; ++k)
            if (lb0 + k < lb1) load_int4(p, b, h, lb0 + k, c, g, buf[k]);
        for (int base = lb0; base < lb1; base += kPrefetch) {
#pragma unroll
            for (int k = 0; k < kPrefetch; ++k) {
                const int lb = base + k;
                if (lb < lb1) {
                    step_int4(buf[k], min(kBlockTokens, len4 - lb * kBlockTokens), g, qf, p.scale_log2, acc, m, l);
                    if (lb + kPrefetch < lb1) load_int4(p, b, h, lb + kPrefetch, c, g, buf[k]);
                }
            }
        }
    } else {
        u -= n4;
        for (int zi = 0; zi < p.nz; ++zi) {
            if (u < nzu[zi]) {
                const ZoneP& z = p.z[zi];
                const int nt = (lenz[zi] + kBlockTokens - 1) / kBlockTokens;
                const int t0 = u * kUnitF16Tiles;
                const int t1 = min(t0 + kUnitF16Tiles, nt);
                F16Tile buf[2];
                if (t0 < t1) load_f16(z, bh, t0, c, g, buf[0]);
                if (t0 + 1 < t1) load_f16(z, bh, t0 + 1, c, g, buf[1]);
                for (int base = t0; base < t1; base += 2) {
#pragma unroll
                    for (int k = 0; k < 2; ++k) {
                        const int t = base + k;
                        if (t < t1) {
                            step_f16(buf[k], min(kBlockTokens, lenz[zi] - t * kBlockTokens), g, qf, p.scale_log2, acc, m, l);
                            if (t + 2 < t1) load_f16(z, bh, t + 2, c, g, buf[k]);
                        }
                    }
                }
                break;
            }
            u -= nzu[zi];
        }
    }

    // ---- merge the waves of this workgroup
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    __shared__ float sm_o[kWaves][16][kHeadDim];
    __shared__ float sm_m[kWaves][16], sm_l[kWaves][16];
    __shared__ int sm_ticket;
    if (c < nrep) {
#pragma unroll
        for (int n = 0; n < 8; ++n)
#pragma unroll
            for (int v = 0; v < 4; ++v) sm_o[wave][c][16 * n + 4 * g + v] = acc[n][v];
        if (g == 0) {
            sm_m[wave][c] = m;
            sm_l[wave][c] = l;
        }
    }
    __syncthreads();

    const int nout = nrep * kHeadDim;
    if (nsplit == 1) {
        for (int idx = threadIdx.x; idx < nout; idx += blockDim.x) {
            const int hd = idx >> 7, d = idx & (kHeadDim - 1);
            float M = -INFINITY;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) M = fmaxf(M, sm_m[w][hd]);
            float O = 0.f, L = 0.f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const float e = (sm_m[w][hd] == -INFINITY) ? 0.f : exp2f(sm_m[w][hd] - M);
                O += sm_o[w][hd][d] * e;
                L += sm_l[w][hd] * e;
            }
            p.out[(int64_t)b * p.o_sb + (int64_t)(h * nrep + hd) * p.o_sh + d] = f2h_rn(L > 0.f ? O / L : 0.f);
        }
        return;
    }

    float* part = p.partials + ((int64_t)bh * p.max_splits + split) * (nrep * kPartStride);
    for (int idx = threadIdx.x; idx < nout; idx += blockDim.x) {
        const int hd = idx >> 7, d = idx & (kHeadDim - 1);
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) M = fmaxf(M, sm_m[w][hd]);
        float O = 0.f, L = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float e = (sm_m[w][hd] == -INFINITY) ? 0.f : exp2f(sm_m[w][hd] - M);
            O += sm_o[w][hd][d] * e;
            L += sm_l[w][hd] * e;
        }
        part[hd * kPartStride + d] = O;
        if (d == 0) {
            part[hd * kPartStride + kHeadDim] = M;
            part[hd * kPartStride + kHeadDim + 1] = L;
        }
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) sm_ticket = atomicAdd(&p.counters[bh], 1);
    __syncthreads();
    if (sm_ticket != nsplit - 1) return;
    __threadfence();

    // ---- last workgroup of this (sequence, kv head): merge every split.
    const float* parts = p.partials + (int64_t)bh * p.max_splits * (nrep * kPartStride);
    for (int idx = threadIdx.x; idx < nout; idx += blockDim.x) {
        const int hd = idx >> 7, d = idx & (kHeadDim - 1);
        float M = -INFINITY, O = 0.f, L = 0.f;
        for (int s = 0; s < nsplit; ++s) {
            const float* ps = parts + (int64_t)s * (nrep * kPartStride) + hd * kPartStride;
            const float ms = ps[kHeadDim];
            if (ms == -INFINITY) continue;
            const float os = ps[d];
            const float ls = ps[kHeadDim + 1];
            if (ms > M) {
                const float a = (M == -INFINITY) ? 0.f : exp2f(M - ms);
                O *= a;
                L *= a;
                M = ms;
            }
            const float e = exp2f(ms - M);
            O += os * e;
            L += ls * e;
        }
        p.out[(int64_t)b * p.o_sb + (int64_t)(h * nrep + hd) * p.o_sh + d] = f2h_rn(L > 0.f ? O / L : 0.f);
    }
    if (threadIdx.x == 0) p.counters[bh] = 0;
}

constexpr size_t kWsHeader = 256;

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

int max_splits_for(int int4_max_len, const int32_t* f16_max_lens, int nz) {
    int total = units_int4(int4_max_len);
    for (int i = 0; i < nz; ++i) total += units_f16(f16_max_lens[i]);
    const int s = (total + kWaves - 1) / kWaves;
    return s > 1 ? s : 1;
}

size_t workspace_bytes(int B, int Hq, int Hkv, int max_splits) {
    const size_t BH = (size_t)B * Hkv;
    const int nrep = Hq / Hkv;
    return kWsHeader + align256(BH * sizeof(int)) + BH * (size_t)max_splits * nrep * kPartStride * sizeof(float);
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
    const int ms = max_splits_for(int4_max_len, f16_max_lens, num_f16_zones);
    return workspace_bytes(batch, num_q_heads, num_kv_heads, ms);
}

extern "C" int hkv_decode_attn(const HkvDecodeArgs* a, void* stream) {
    clear_error();
    HKV_REQUIRE(a != nullptr, HKV_ERR_ARG, "hkv_decode_attn: null args");
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
    HKV_REQUIRE(a->q && a->out && a->workspace, HKV_ERR_ARG, "hkv_decode_attn: null q/out/workspace");
    HKV_REQUIRE((((uintptr_t)a->q) & 15) == 0 && (a->q_stride_b % 8) == 0 && (a->q_stride_h % 8) == 0,
                HKV_ERR_ARG, "hkv_decode_attn: q must be 16-byte aligned with strides multiple of 8");
    HKV_REQUIRE(a->int4_max_len >= 0, HKV_ERR_ARG, "hkv_decode_attn: int4_max_len < 0");
    if (a->int4_max_len > 0) {
        HKV_REQUIRE(a->pool && a->block_table && a->pool_blocks > 0, HKV_ERR_ARG,
                    "hkv_decode_attn: INT4 zone without pool/block table");
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
    const int ms = max_splits_for(a->int4_max_len, zl, a->num_f16_zones);
    const size_t need = workspace_bytes(a->batch, a->num_q_heads, a->num_kv_heads, ms);
    HKV_REQUIRE(a->workspace_bytes >= need, HKV_ERR_CAPACITY,
                "hkv_decode_attn: workspace %zu bytes, need %zu", a->workspace_bytes, need);
    HKV_REQUIRE((((uintptr_t)a->workspace) & 255) == 0, HKV_ERR_ARG, "hkv_decode_attn: workspace must be 256-byte aligned");
    const int64_t BH = (int64_t)a->batch * a->num_kv_heads;
    HKV_REQUIRE(BH * ms < 2147483647LL, HKV_ERR_ARG, "hkv_decode_attn: grid too large");

    DecodeParams p;
    p.B = a->batch;
    p.Hkv = a->num_kv_heads;
    p.nrep = nrep;
    p.scale_log2 = a->sm_scale * kLog2e;
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
    p.pool_blocks = a->pool_blocks;
    p.bt = a->block_table;
    p.bt_stride = a->bt_stride;
    p.int4_lens = a->int4_lens;
    p.int4_max_len = a->int4_max_len;
    p.out = a->out;
    p.o_sb = a->out_stride_b;
    p.o_sh = a->out_stride_h;
    char* ws = (char*)a->workspace;
    p.err = (int*)ws;
    p.counters = (int*)(ws + kWsHeader);
    p.partials = (float*)(ws + kWsHeader + align256((size_t)BH * sizeof(int)));
    p.max_splits = ms;
    hipLaunchKernelGGL(decode_attn_kernel, dim3((unsigned)(BH * ms)), dim3(256), 0, (hipStream_t)stream, p);
    HKV_LAUNCH_CHECK("decode_attn_kernel");
    return HKV_OK;
}
