// Shared by the two chunked-prefill kernels (prefill_zones.hip: fp16 zone tiles and
// the causal chunk; prefill_attn.hip: INT4 tiles and the entry point).
//
// A launch with both kinds of keys runs the zone kernel first.  It leaves, per
// (sequence, query head, query row), the online-softmax state of the zone and chunk
// tokens in a workspace -- the unnormalized output O (relative to the running max m),
// m, and the running sums of the two lane halves -- and the INT4 kernel starts from that
// state, so the result is the softmax over all keys as from one pass.
#pragma once

#include "hkv_internal.h"

namespace hkv {

typedef _Float16 ph8 __attribute__((ext_vector_type(8)));
typedef float pf16v __attribute__((ext_vector_type(16)));
typedef float pf4 __attribute__((ext_vector_type(4)));
typedef uint32_t pu4 __attribute__((ext_vector_type(4)));
typedef uint32_t pu2 __attribute__((ext_vector_type(2)));

constexpr int kPfQ = 32;             // query rows per wave
constexpr int kPfT = 64;             // tokens per tile
constexpr float kPfLog2e = 1.4426950408889634f;
constexpr int kStateFloats = 132;    // O[128], m, l (lanes 0-31), l (lanes 32-63), pad

struct PfZone {
    const uint16_t* k;
    const uint16_t* v;
    int cap;
    int max_len;
    const int32_t* lens;
};

// Where the zone kernel reads the fp16 tiles of one source (a zone, or the causal chunk
// in the zone layout): K rows [B*Hkv][cap][128], V tiles [B*Hkv][cap/16][16 x 128].
struct PfSrc {
    const uint16_t* k;
    const uint16_t* v;
    int cap;
    int pad;
};

struct PrefillParams {
    int B, Hkv, nrep, Sq;
    float scale_log2;
    int q_bf16, c_bf16, out_bf16;   // q / chunk / out dtype is bfloat16 (else fp16)
    const uint16_t* q;
    int64_t q_sb, q_sh, q_st;
    int nz;
    PfZone z[HKV_MAX_F16_ZONES];
    const uint8_t* pool;
    uint32_t pool_blocks;        // record counts capped at 2^31 (block ids are int32), so the
    const uint8_t* staging;      // range check is a 32-bit scalar compare; staging records are
    uint32_t staging_blocks;     // addressed by negative block ids
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
    float* state;                // [B][Hq][Sq][kStateFloats] zone-kernel state (may be null)
    const uint16_t* czk;         // the causal chunk in the zone layout: K rows [B*Hkv][ccap][128]
    const uint16_t* czv;         // and V tiles [B*Hkv][ccap/16][16 x 128] (null without a chunk)
    int ccap;
    // the zone kernel's sources in tile order: zones 0..2 (unused ones empty), then the
    // chunk; indexed at run time, so that no source's pointers stay in registers
    PfSrc src[HKV_MAX_F16_ZONES + 1];
};

// Tile counts of one sequence: INT4 tiles, each zone's tiles, and the causal chunk's
// tiles up to query row q_end (exclusive).
struct TileMap {
    int n4, nz_t[HKV_MAX_F16_ZONES], nc;
    int len4, lenz[HKV_MAX_F16_ZONES];
    __device__ int nf() const { return nz_t[0] + nz_t[1] + nz_t[2] + nc; }
};

__device__ __forceinline__ void make_tile_map(const PrefillParams& p, int b, int q_end, TileMap& tm) {
    tm.len4 = p.int4_lens ? min(max(p.int4_lens[b], 0), p.int4_max_len) : p.int4_max_len;
    tm.n4 = (tm.len4 + kPfT - 1) / kPfT;
#pragma unroll
    for (int zi = 0; zi < HKV_MAX_F16_ZONES; ++zi) {
        tm.lenz[zi] = 0;
        if (zi < p.nz) tm.lenz[zi] = p.z[zi].lens ? min(max(p.z[zi].lens[b], 0), p.z[zi].max_len) : p.z[zi].max_len;
        tm.nz_t[zi] = (tm.lenz[zi] + kPfT - 1) / kPfT;
    }
    tm.nc = p.ck ? (min(q_end, p.Sq) + kPfT - 1) / kPfT : 0;
}

// The state of query row `qrow` of query head `qh` of sequence b.
__device__ __forceinline__ float* state_row(const PrefillParams& p, int b, int qh, int qrow) {
    return p.state + (((int64_t)b * p.Hkv * p.nrep + qh) * p.Sq + qrow) * kStateFloats;
}

__device__ __forceinline__ uint32_t pack2(float a, float b) {
    return (uint32_t)f2h_rn(a) | ((uint32_t)f2h_rn(b) << 16);
}
__device__ __forceinline__ uint32_t pack2bf(float a, float b) {
    return (uint32_t)f2bf_rn(a) | ((uint32_t)f2bf_rn(b) << 16);
}

// Eight bf16 values to fp16: exact in [2^-14, 65504]; `over` is set when a finite
// value leaves the fp16 range (it becomes +-inf).
__device__ __forceinline__ pu4 bf16x8_to_f16(pu4 w, bool& over) {
    pu4 r;
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

// Writes this lane's final output: acc[db][4j + i] is O^T[dim 32db + 8j + 4hh + i][its
// query row], l the row's softmax sum.
__device__ __forceinline__ void write_out(const PrefillParams& p, int b, int qh, int qrow, int hh,
                                          const pf16v (&acc)[4], float l) {
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    uint16_t* op = p.out + (int64_t)b * p.o_sb + (int64_t)qh * p.o_sh + (int64_t)qrow * p.o_st;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int d = 32 * db + 8 * j + 4 * hh;
            if (p.out_bf16)
                *(pu2*)(op + d) = pu2{pack2bf(acc[db][4 * j + 0] * inv, acc[db][4 * j + 1] * inv),
                                      pack2bf(acc[db][4 * j + 2] * inv, acc[db][4 * j + 3] * inv)};
            else
                *(pu2*)(op + d) = pu2{pack2(acc[db][4 * j + 0] * inv, acc[db][4 * j + 1] * inv),
                                      pack2(acc[db][4 * j + 2] * inv, acc[db][4 * j + 3] * inv)};
        }
}

// Launches the zone kernel (fp16 zone tiles and the causal chunk) over every sequence.
int launch_prefill_zones(const PrefillParams& p, int ngrp, hipStream_t stream);

}  // namespace hkv
