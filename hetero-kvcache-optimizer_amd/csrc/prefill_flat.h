// The tile loop shared by the two chunked-prefill kernels (prefill_attn.hip: INT4
// tiles; prefill_zones.hip: fp16 zone tiles and the causal chunk).  A workgroup is 8
// waves over one kv head: wave w takes query head 4 grp + (w & 3) of the GQA group and
// query rows q0 + 32 (w >> 2) .. +31 (kPfQ rows per wave, 64 per workgroup).  Per
// 64-token tile t every wave runs, with v_mfma_f32_32x32x16_f16,
//   A: S(t+1)^T = K(t+1) . Q^T (16 MFMAs) beside the softmax of S(t) -> P(t)
//   B: O^T += V(t)^T . P(t)^T (16 MFMAs) beside the staging of tile t+2 (this wave's
//      16-token quarter of the K rows, waves 0-3, or of the V^T rows, waves 4-7) and
//      the row sum of P(t)
// and one workgroup barrier ends the tile.  A wave can issue a few VALU instructions
// while each of its MFMAs executes, so the softmax and the staging mostly hide behind
// the MFMAs; sched_group_barrier asks the scheduler for that interleave.  Four LDS
// tile buffers rotate (tile t: V^T and biases read; t+1: K rows read; t+2: written).
// Tiles past the last one are empty (valid length 0), so every tile does the same work
// and no MFMA or accumulator update sits behind a branch.
//
// The S^T accumulator of lane (query n, half hh) holds tokens 8j + 4hh + i of each
// 32-token block, exactly the 8-token k-slices the P^T operand needs, so P never
// leaves registers.
#pragma once

#include "prefill_common.h"

namespace hkv {

typedef _Float16 fh2 __attribute__((ext_vector_type(2)));

// One LDS tile buffer: K rows (64 tokens, 256 bytes of fp16 each, padded to 272 bytes),
// then V^T rows (128 dims, 64 tokens of fp16 each, padded to 144 bytes).  The padding
// keeps the 16-byte operand reads of 8 consecutive lanes on distinct banks, and each
// lane reads all its operands of a tile at immediate offsets from one address.  The
// per-token score biases (0, or -inf past the valid length) of the four buffers sit
// together at the start of LDS, so every bias read is an immediate offset too.
constexpr int kFlatBufs = 4;
constexpr int kFlatWaves = 8;
constexpr int kFlatThreads = kFlatWaves * 64;
constexpr int kFlatQ = 2 * kPfQ;                     // query rows per workgroup
constexpr int kKRow = kHeadDim * 2 + 16;
constexpr int kVRow = kPfT * 2 + 16;
constexpr int kVOff = kPfT * kKRow;
constexpr int kDataBytes = kVOff + kHeadDim * kVRow;
constexpr int kFacBytes = kPfT * 4;
constexpr int kFlatLdsBytes = kFlatBufs * (kFacBytes + kDataBytes);

__device__ __forceinline__ uint8_t* flat_buf(uint8_t* lds, int i) { return lds + kFlatBufs * kFacBytes + i * kDataBytes; }
__device__ __forceinline__ uint8_t* flat_bias(uint8_t* lds, int i) { return lds + i * kFacBytes; }

// LDS addresses (bytes) inside a tile buffer.  K: 16-byte chunk `chunk` (dims
// 8 chunk .. +8) of token `tok`.  V^T rows hold the tile's 64 tokens in 8-byte units
// of 4 tokens; within each 16-token group the units are stored in the order 0, 2, 1,
// 3, so that the 8 tokens one lane feeds to a P.V product (tokens 4hh..4hh+3 and
// 8+4hh..8+4hh+3 of a group) are one 16-byte read.  vt_addr takes the natural unit
// index (token / 4).
__device__ __forceinline__ int k_addr(int tok, int chunk) { return tok * kKRow + chunk * 16; }
__device__ __forceinline__ int vt_unit(int unit) { return (unit & ~3) | ((unit & 1) << 1) | ((unit >> 1) & 1); }
__device__ __forceinline__ int vt_addr(int dim, int unit) { return kVOff + dim * kVRow + vt_unit(unit) * 8; }
// The 16 bytes holding natural units 4gr + hh and 4gr + 2 + hh (gr = 16-token group).
__device__ __forceinline__ int vt_pair_addr(int dim, int gr, int hh) { return kVOff + dim * kVRow + (2 * gr + hh) * 16; }

// The end of one tile: the scheduling barriers keep each tile's work on its side of the
// workgroup barrier.
__device__ __forceinline__ void flat_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
}

struct FlatWave {
    int b, h, wt, lane, n, hh, qrow, qb;
};

// The workgroup's query block and (kv head, GQA group) index.  Dispatch goes round-robin
// over the 8 XCDs by linear workgroup id, so with qb = lin / HG and hg = lin % HG (HG =
// gridDim.y, the head-group count) every workgroup of one head group runs on the same XCD
// when HG is a multiple of 8, and the query blocks reading that head's tiles share an L2.
struct FlatBlock {
    int qb, hg;
};
__device__ __forceinline__ FlatBlock flat_block() {
    const int lin = (int)blockIdx.x + (int)gridDim.x * (int)blockIdx.y;
    return FlatBlock{lin / (int)gridDim.y, lin % (int)gridDim.y};
}

// QK: S^T[64 tok x 32 q] = K . Q^T + c0.  The two token blocks' accumulators are two
// independent MFMA chains, started at c0 (minus the lane's running max, so the scores
// come out relative to it); each step's K operands are read two steps ahead.
__device__ __forceinline__ void qk_begin(const uint8_t* kt, int n, int hh, ph8 (&a0)[3], ph8 (&a1)[3], pf16v (&S)[2],
                                         float c0) {
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int r = 0; r < 16; ++r) S[tb][r] = c0;
    const uint8_t* k0 = kt + k_addr(n, hh);
    const uint8_t* k1 = kt + k_addr(32 + n, hh);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        a0[s] = __builtin_bit_cast(ph8, *(const pu4*)(k0 + 32 * s));
        a1[s] = __builtin_bit_cast(ph8, *(const pu4*)(k1 + 32 * s));
    }
}
template <int kS0, int kS1>
__device__ __forceinline__ void qk_steps(const uint8_t* kt, int n, int hh, const ph8 (&qf)[8], ph8 (&a0)[3],
                                         ph8 (&a1)[3], pf16v (&S)[2]) {
    const uint8_t* k0 = kt + k_addr(n, hh);
    const uint8_t* k1 = kt + k_addr(32 + n, hh);
#pragma unroll
    for (int s = kS0; s < kS1; ++s) {
        if (s + 2 < 8) {
            a0[(s + 2) % 3] = __builtin_bit_cast(ph8, *(const pu4*)(k0 + 32 * (s + 2)));
            a1[(s + 2) % 3] = __builtin_bit_cast(ph8, *(const pu4*)(k1 + 32 * (s + 2)));
        }
        S[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0[s % 3], qf[s], S[0], 0, 0, 0);
        S[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1[s % 3], qf[s], S[1], 0, 0, 0);
    }
}

// Softmax pieces.  Lane (n, hh) holds tokens tb*32 + 8j + 4hh + i for r = 4j + i: four
// consecutive tokens per j, whose biases are one 16-byte LDS read.  Only tiles with
// fewer than 64 valid tokens (tvalid, wave-uniform) read and add the biases.
__device__ __forceinline__ void sm_bias(const uint8_t* bias, int tvalid, int hh, pf16v (&S)[2]) {
    if (tvalid < kPfT) {
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const pf4 fb = *(const pf4*)(bias + (tb * 32 + 8 * j + 4 * hh) * 4);
#pragma unroll
                for (int i = 0; i < 4; ++i) S[tb][4 * j + i] += fb[i];
            }
    }
}
// The row max of S over both lane halves (four independent max chains, then a lane
// swap, not an LDS permute, for the other half of the row).
__device__ __forceinline__ float sm_max(const pf16v (&S)[2]) {
    float mx[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx[r & 3] = fmaxf(mx[r & 3], S[tb][r]);
    const float mt = fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3]));
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
    return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
}
// P = exp2(S), S already relative to the running max, as the P^T operands (P[2 tb + u]:
// tokens tb*32 + 16u + 4hh .. +3 and +8 .. +11) in fp16.
__device__ __forceinline__ void sm_exp(const pf16v (&S)[2], ph8 (&P)[4]) {
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int jj = 0; jj < 2; ++jj)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    P[2 * tb + u][jj * 4 + i] = (_Float16)__builtin_amdgcn_exp2f(S[tb][4 * (2 * u + jj) + i]);
}
// The row sum adds the fp16 P values (two per v_dot2), the same numbers P.V weighs.
__device__ __forceinline__ void sm_sum(const ph8 (&P)[4], float& l) {
    const fh2 one2 = {(_Float16)1.0f, (_Float16)1.0f};
    float ls[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        ls[k] = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) ls[k] = __builtin_amdgcn_fdot2(fh2{P[k][2 * e], P[k][2 * e + 1]}, one2, ls[k], false);
    }
    l += (ls[0] + ls[1]) + (ls[2] + ls[3]);
}
// PV: O^T[128 d x 32 q] += V^T . P^T, four independent accumulator chains (dim blocks);
// each token group's V^T operands are read one group ahead.
__device__ __forceinline__ void pv_flat(const uint8_t* vt, int n, int hh, const ph8 (&P)[4], pf16v (&acc)[4]) {
    ph8 a[2][4];
#pragma unroll
    for (int db = 0; db < 4; ++db) a[0][db] = __builtin_bit_cast(ph8, *(const pu4*)(vt + vt_pair_addr(32 * db + n, 0, hh)));
#pragma unroll
    for (int gr = 0; gr < 4; ++gr) {
        if (gr + 1 < 4) {
#pragma unroll
            for (int db = 0; db < 4; ++db)
                a[(gr + 1) & 1][db] =
                    __builtin_bit_cast(ph8, *(const pu4*)(vt + vt_pair_addr(32 * db + n, gr + 1, hh)));
        }
#pragma unroll
        for (int db = 0; db < 4; ++db) acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[gr & 1][db], P[gr], acc[db], 0, 0, 0);
    }
}

// The tile loop over tiles 0 .. T-1 (T a multiple of kFlatBufs).  The staging policy
// `pol` provides
//   kRing                      register slots of staged records in flight
//   start(lds)                 loads and stages tiles 0 and 1, fills the slots
//   stage(slot, buf, bias, x)  writes tile x from register slot `slot` into LDS and
//                              refills the slot with tile x + kRing
//   tvalid(x)                  valid tokens of tile x (0 for an empty tile)
//   mask(x, S)                 extra per-score masking of tile x (the causal chunk's
//                              diagonal tile), a wave-uniform branch
// and (m, l, acc) carry the online softmax of this wave's rows in and out.
template <class Pol>
__device__ __forceinline__ void flat_tiles(Pol& pol, const FlatWave& w, uint8_t* lds, const ph8 (&qf)[8],
                                           pf16v (&acc)[4], float& m, float& l, int T) {
    pol.start(lds);
    flat_barrier();
    pf16v Sx[2][2];
    ph8 P[4];
    ph8 a0[3], a1[3];
    // The QK chains start at -msafe (msafe = m, or 0 while m is -inf), so the scores come
    // out relative to the running max and a tile with no new row max exponentiates them
    // as they are (on C4, 4.29 vs 4.33 ms per call).  When the max moves, S(t) and the
    // partial S(t+1) are rebased on the new msafe.
    float msafe = (m == -INFINITY) ? 0.f : m;
    qk_begin(flat_buf(lds, 0), w.n, w.hh, a0, a1, Sx[0], -msafe);
    qk_steps<0, 8>(flat_buf(lds, 0), w.n, w.hh, qf, a0, a1, Sx[0]);
    __builtin_amdgcn_sched_barrier(0);
    for (int t0 = 0; t0 < T; t0 += kFlatBufs) {
#pragma unroll
        for (int uu = 0; uu < kFlatBufs; ++uu) {
            const int t = t0 + uu;
            pf16v (&Sc)[2] = Sx[uu & 1];
            pf16v (&Sn)[2] = Sx[(uu + 1) & 1];
            const uint8_t* const bt = flat_buf(lds, uu);
            const uint8_t* const bn = flat_buf(lds, (uu + 1) % kFlatBufs);
            sm_bias(flat_bias(lds, uu), pol.tvalid(t), w.hh, Sc);
            pol.mask(t, Sc);
            __builtin_amdgcn_sched_barrier(0);
            // A: QK(t+1) beside the softmax of S(t)
            qk_begin(bn, w.n, w.hh, a0, a1, Sn, -msafe);
            qk_steps<0, 2>(bn, w.n, w.hh, qf, a0, a1, Sn);
            const float mt = sm_max(Sc) + msafe;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);   // up to six VALU
            }
            if (__ballot(mt > m)) {
                const float m_new = fmaxf(m, mt);
                const float alpha = (m_new > m) ? __builtin_amdgcn_exp2f(m - m_new) : 1.0f;
#pragma unroll
                for (int db = 0; db < 4; ++db) acc[db] *= alpha;
                l *= alpha;
                m = m_new;
                const float ms_new = (m == -INFINITY) ? 0.f : m;
                const float d = ms_new - msafe;
                msafe = ms_new;
#pragma unroll
                for (int tb = 0; tb < 2; ++tb) {
                    Sc[tb] -= d;
                    Sn[tb] -= d;
                }
            }
            qk_steps<2, 8>(bn, w.n, w.hh, qf, a0, a1, Sn);
            sm_exp(Sc, P);
#pragma unroll
            for (int k = 0; k < 12; ++k) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 7, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            // B: PV(t) beside the staging of tile t+2 and the row sum
            pv_flat(bt, w.n, w.hh, P, acc);
            pol.stage(uu % Pol::kRing, flat_buf(lds, (uu + 2) % kFlatBufs), flat_bias(lds, (uu + 2) % kFlatBufs), t + 2);
            sm_sum(P, l);
            asm volatile("" ::"v"(l));   // keep the row sum beside this tile's MFMAs
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            pol.refill(uu % Pol::kRing, t + 2);
            flat_barrier();
        }
    }
}

// Loads this wave's Q^T fragments (lane (query n, half hh), step s -> q[qrow][16s + 8hh
// .. +8]) as fp16, each element times `mul` (1, or the fp16 factor folded into Q).
__device__ __forceinline__ void flat_load_q(const PrefillParams& p, int b, int qh, bool ok, int qrow, int hh,
                                            float mul, ph8 (&qf)[8]) {
    const uint16_t* qp = p.q + (int64_t)b * p.q_sb + (int64_t)qh * p.q_sh + (int64_t)(ok ? qrow : 0) * p.q_st + 8 * hh;
    bool over = false;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        pu4 w = ok ? *(const pu4*)(qp + 16 * s) : pu4{0u, 0u, 0u, 0u};
        if (p.q_bf16) w = bf16x8_to_f16(w, over);
        qf[s] = __builtin_bit_cast(ph8, w);
        if (mul != 1.0f) {
#pragma unroll
            for (int e = 0; e < 8; ++e) qf[s][e] = (_Float16)((float)qf[s][e] * mul);
        }
    }
    if (__ballot(over) && (threadIdx.x & 63) == 0 && p.err) atomicOr(p.err, HKV_ERR_BIT_RANGE);
}

}  // namespace hkv
