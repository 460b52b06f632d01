// Chunked-prefill attention over [INT4 pool | fp16 zones | causal chunk] on MFMA: the
// entry point, and the INT4 kernel (the zone kernel is prefill_zones.hip).
//
// Math (fused_dequant_attn.py:242-247,385-390; kernels/fused_dequant_attn.py:371-435
// is the reference entry point): out[q] = softmax_t(q . K_t * sm_scale) V_t over every
// INT4 token (dequantized as (code - zero point) x scale in fp32), every fp16 zone token
// and the chunk's own tokens t <= q (causal), GQA q head i -> kv head i / n_rep.  The
// INT4 operands are the exact integers code - zero point; the K scale multiplies the
// score and the V scale the probability, in fp32.
//
// INT4 kernel.  Per wave and 64-token tile, with v_mfma_f32_32x32x16_f16:
//   S^T[64 tok x 32 q] = K[tok][d] . Q^T      (2 token blocks x 8 k-steps)
//   O^T[128 d x 32 q] += V^T[d][tok] . P^T    (4 dim blocks x 4 token steps)
// The S^T accumulator of lane (query n, half h) holds tokens 8j + 4h + i, exactly the
// 8-token k-slices the P^T operand needs, so P never leaves registers.  The workgroup
// schedule (two teams in ping-pong) is described below.
#include "nibble_decode.h"
#include "prefill_common.h"

#include <math.h>

#include <algorithm>
#include <type_traits>

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
// One LDS tile buffer: K rows (64 tokens, 256 bytes of fp16 each, rows padded to
// 272 bytes), V^T rows (128 dims, 64 tokens of fp16 each, padded to 144 bytes), then
// per token the score bias (0, or -inf past the valid length), fp32.  K rows hold
// (code - zero point) x K scale x sm_scale x log2 e and V^T rows (code - zero point) x
// V scale, in fp16, so the scores come out of the MFMAs in the log2 domain (the fp16
// rounding of each dequantized element is the one fp16 dequantization makes).  Tokens
// past the valid length get K and V scale 0, so whatever their record slots hold, their
// scores are 0 until the bias masks them, and their V^T rows are 0.  The padding keeps the
// 16-byte operand reads of 8 consecutive lanes on distinct banks, and each lane reads
// all its operands of a tile at immediate offsets from one address.
constexpr int kKRow = kHeadDim * 2 + 16;
constexpr int kVRow = kT * 2 + 16;
constexpr int kVOff = kT * kKRow;
constexpr int kDataBytes = kVOff + kHeadDim * kVRow;   // K rows + V^T rows of one tile
// The per-token biases of the tile buffers sit together at the start of LDS, so every
// bias read is an immediate offset from one address (offsets stop at 65535).
constexpr int kSbOff = 0;
constexpr int kFacBytes = kT * 4;

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

// ---- Ping-pong schedule.  A workgroup = 8 waves = two teams of 4 waves over the same
// kv head: team 0 takes query rows q0 .. q0 + 31, team 1 rows q0 + 32 .. q0 + 63, and
// wave w of a team takes query head 4 grp + w of the GQA group.  Waves w and w + 4 share
// a SIMD.  Per 64-token tile t, each team runs
//   QK(t): S^T = K . Q^T      (16 MFMAs)
//   SM(t): scale, mask, online softmax, P = exp2(S - m) x V scale   (VALU)
//   PV(t): O^T += V^T . P^T   (16 MFMAs)
// and the teams are half an iteration apart, so one team's MFMAs run beside the
// other's VALU work on every SIMD:
//   phase X:  team 0: PV(t-1), QK(t), stage K of tile t+1     team 1: SM(t-1)
//   phase Y:  team 0: SM(t)     team 1: PV(t-1), QK(t), stage V of tile t+1
// with a workgroup barrier after each phase.  Three LDS tile buffers rotate: tile t-1
// (its V^T and biases still read), tile t, and tile t+1 being staged.  The staging of
// a tile is split between the teams (team 0 the K rows and the token biases, team 1 the
// V^T rows), so every wave dequantizes an eighth of each tile.
constexpr int kTeamWaves = 4;
constexpr int kThreadsPP = 2 * kTeamWaves * 64;
constexpr int kQB = 2 * kQ;                  // query rows per workgroup
constexpr int kNumBufs = 3;
constexpr int kLdsBytes = kNumBufs * (kFacBytes + kDataBytes);
constexpr int kRing4 = 3;                    // INT4 half-tiles per thread: one staged, two in flight

// Staging of INT4 tile x: wave w of a team handles block w of the tile (4 blocks of 16
// tokens), so the block id and record address are wave-uniform (scalar registers,
// one buffer resource per block).  Team 0 lane i: K codes of token i/4, dims
// 32(i%4)..+32, with that row's scale and zero point.  Team 1 lane i: V word 4i..4i+3,
// with the V scales and zero points of tokens 4g..4g+3, g = i/16.
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
// every lane.  It stays a vector register until it is used, kRing4 tiles later, so no
// wait for this load sits behind the record loads issued before it.
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
// Writes a staged block into LDS buffer `lds`: K as (code - zero point) x K scale x
// sm_scale x log2 e with the per-token biases, V as (code - zero point) x V scale;
// `valid` = valid tokens of the block.  Tokens past it get scale 0 (their codes are
// finite, their scales may be anything) and bias -inf.
__device__ __forceinline__ void store_k4(const SlotK& s, uint8_t* lds, uint8_t* fac, float scale_log2, int wt, int lane,
                                         int valid) {
    const int rr = lane >> 2, pt = lane & 3;
    const int tok = wt * 16 + rr;
    const uint32_t kz = s.kz & 0xFFu;
    const h2 kz1024 = zp1024(kz, kz), kz64 = zp64(kz, kz);
    const _Float16 f = (_Float16)(rr < valid ? s.ks * scale_log2 : 0.0f);
    const h2 f2 = {f, f};
    const uint32_t w4[4] = {s.w.x, s.w.y, s.w.z, s.w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {          // word j: dims 32pt + 8j .. +8
        const NibPairs a = unpack_word(w4[j], kz1024, kz64);
        *(u4*)(lds + k_addr(tok, pt * 4 + j)) =
            u4{__builtin_bit_cast(uint32_t, a.p0 * f2), __builtin_bit_cast(uint32_t, a.p1 * f2),
               __builtin_bit_cast(uint32_t, a.p2 * f2), __builtin_bit_cast(uint32_t, a.p3 * f2)};
    }
    if (pt == 0) ((float*)(fac + kSbOff))[tok] = rr < valid ? 0.0f : -INFINITY;
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

// QK(t): S^T[64 tok x 32 q] = K . Q^T for this wave's 32 query rows.  The two token
// blocks' accumulators form two independent MFMA chains, issued alternately, and each
// step's K operands are read two steps ahead, so neither the chain's result latency
// nor the LDS latency stalls the MFMA pipe.  (Scheduling barriers keep this order.)
__device__ __forceinline__ void qk_tile(const uint8_t* cur, int n, int hh, const h8 (&qf)[8], f16v (&S)[2]) {
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int r = 0; r < 16; ++r) S[tb][r] = 0.f;
    const uint8_t* k0 = cur + k_addr(n, hh);          // token n, chunk hh; step s adds 32 s bytes
    const uint8_t* k1 = cur + k_addr(32 + n, hh);
    h8 a0[3], a1[3];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        a0[s] = __builtin_bit_cast(h8, *(const u4*)(k0 + 32 * s));
        a1[s] = __builtin_bit_cast(h8, *(const u4*)(k1 + 32 * s));
    }
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        if (s + 2 < 8) {
            a0[(s + 2) % 3] = __builtin_bit_cast(h8, *(const u4*)(k0 + 32 * (s + 2)));
            a1[(s + 2) % 3] = __builtin_bit_cast(h8, *(const u4*)(k1 + 32 * (s + 2)));
        }
        S[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0[s % 3], qf[s], S[0], 0, 0, 0);
        S[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1[s % 3], qf[s], S[1], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// SM(t): masked online softmax of S; P = exp2(S - m) as the P^T operands (P[2 tb + u]:
// tokens tb*32 + 16u + 4hh .. +3 and +8 .. +11) in fp16, and the row sum adds those
// fp16 values (two per v_dot2), the same numbers the P.V product weighs.  Lane (n, hh)
// holds tokens tb*32 + 8j + 4hh + i for r = 4j + i: four consecutive tokens per j, whose
// biases are one 16-byte LDS read.  `tvalid` (wave-uniform) is the tile's count of
// valid tokens; only a sequence's last INT4 tile and the empty tiles have fewer than 64,
// and only they add the per-token bias (-inf past the valid length).
__device__ __forceinline__ void softmax_tile(const uint8_t* fac, int tvalid, int hh, f16v (&S)[2], f16v (&acc)[4],
                                             float& m, float& l, h8 (&P)[4]) {
    if (tvalid < kT) {
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const f4 fb = *(const f4*)(fac + kSbOff + (tb * 32 + 8 * j + 4 * hh) * 4);
#pragma unroll
                for (int i = 0; i < 4; ++i) S[tb][4 * j + i] += fb[i];
            }
    }
    // four independent max chains, so the reduction is not one 16-deep dependency chain
    float mx[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx[r & 3] = fmaxf(mx[r & 3], S[tb][r]);
    float mt = fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3]));
    // the other half of the row (lanes n and n + 32) by a lane swap, not an LDS permute
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
    mt = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
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
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const int j = 2 * u + jj;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    P[2 * tb + u][jj * 4 + i] = (_Float16)__builtin_amdgcn_exp2f(S[tb][4 * j + i] - msafe);
            }
        __builtin_amdgcn_sched_barrier(0);
    }
    const h2 one2 = {(_Float16)1.0f, (_Float16)1.0f};
    float ls[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        ls[k] = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) ls[k] = __builtin_amdgcn_fdot2(h2{P[k][2 * e], P[k][2 * e + 1]}, one2, ls[k], false);
    }
    l += (ls[0] + ls[1]) + (ls[2] + ls[3]);
}

// PV(t): O^T[128 d x 32 q] += V^T . P^T: four independent accumulator chains (dim
// blocks); each token group's V^T operands are read one group ahead.
__device__ __forceinline__ void pv_tile(const uint8_t* cur, int n, int hh, const h8 (&P)[4], f16v (&acc)[4]) {
    h8 a[2][4];
#pragma unroll
    for (int db = 0; db < 4; ++db) a[0][db] = __builtin_bit_cast(h8, *(const u4*)(cur + vt_pair_addr(32 * db + n, 0, hh)));
#pragma unroll
    for (int gr = 0; gr < 4; ++gr) {
        if (gr + 1 < 4) {
#pragma unroll
            for (int db = 0; db < 4; ++db)
                a[(gr + 1) & 1][db] = __builtin_bit_cast(h8, *(const u4*)(cur + vt_pair_addr(32 * db + n, gr + 1, hh)));
        }
#pragma unroll
        for (int db = 0; db < 4; ++db) acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[gr & 1][db], P[gr], acc[db], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// One ping-pong iteration boundary.  The scheduling barrier keeps each phase's work on
// its side of the workgroup barrier.
__device__ __forceinline__ void phase_end() {
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
}

struct WaveCtx {
    int b, h, wt, lane, n, hh, qrow;
};
#define HKV_BUF(i) (lds + kNumBufs * kFacBytes + (i) * kDataBytes)
#define HKV_FAC(i) (lds + (i) * kFacBytes)

// INT4 tiles 0 .. n4-1 for one team; iteration t (0 .. n4) runs phases X and Y.  The
// loop is unrolled by 3 from multiples of 3, so tile t's LDS buffer (t % 3) and staging
// slot are compile-time.  Both teams execute the same number of barriers.
template <int kTeam>
__device__ __forceinline__ void int4_tiles(const PrefillParams& p, const TileMap& tm, const WaveCtx& w, uint8_t* lds,
                                           const h8 (&qf)[8], f16v (&acc)[4], float& m, float& l, f16v (&S)[2],
                                           h8 (&P)[4]) {
    typedef typename std::conditional<kTeam == 0, SlotK, SlotV>::type Slot;
    const int n4 = tm.n4;
    const int nb4 = (tm.len4 + kBlockTokens - 1) / kBlockTokens;
    auto valid_of = [&](int x) {
        const int lbt = x * 4 + w.wt;
        return (x < n4 && lbt < nb4) ? min(kBlockTokens, tm.len4 - lbt * kBlockTokens) : 0;
    };
    auto tvalid_of = [&](int x) { return (x >= 0 && x < n4) ? min(kT, tm.len4 - x * kT) : 0; };
    auto load = [&](int id, Slot& sl) {
        if constexpr (kTeam == 0) load_k4(p, w.h, id, w.lane, sl);
        else load_v4(p, w.h, id, w.lane, sl);
    };
    auto store = [&](const Slot& sl, uint8_t* dst, uint8_t* fac, int x) {
        if constexpr (kTeam == 0) store_k4(sl, dst, fac, p.scale_log2, w.wt, w.lane, valid_of(x));
        else store_v4(sl, dst, w.wt, w.lane, valid_of(x));
    };
    Slot ring[kRing4];
    int idn[kRing4];   // block id of tile x + kRing4 for the slot holding tile x
#pragma unroll
    for (int x = 0; x < kRing4; ++x) {
        load(block_id4(p, nb4, w.b, x, w.wt), ring[x]);
        idn[x] = block_id4(p, nb4, w.b, x + kRing4, w.wt);
    }
    store(ring[0], HKV_BUF(0), HKV_FAC(0), 0);
    load(idn[0], ring[0]);
    idn[0] = block_id4(p, nb4, w.b, 2 * kRing4, w.wt);
    phase_end();
    // Every iteration does the same work: the first reads the empty tile -1 (buffer 2),
    // and iterations past the last tile read empty tiles (re-read records, no valid
    // token), so no MFMA or accumulator update sits behind a branch.
    for (int t0 = 0; t0 <= n4; t0 += kNumBufs) {
#pragma unroll
        for (int uu = 0; uu < kNumBufs; ++uu) {
            const int t = t0 + uu;
            const int ks = (uu + 1) % kRing4;   // slot of tile t + 1
            uint8_t* const prv = HKV_BUF((uu + kNumBufs - 1) % kNumBufs);
            uint8_t* const cur = HKV_BUF(uu);
            uint8_t* const nxt = HKV_BUF((uu + 1) % kNumBufs);
            uint8_t* const prv_f = HKV_FAC((uu + kNumBufs - 1) % kNumBufs);
            uint8_t* const cur_f = HKV_FAC(uu);
            uint8_t* const nxt_f = HKV_FAC((uu + 1) % kNumBufs);
            // A team's MFMA phase also stages its half of tile t+1 (buffer (t+1) % 3 held
            // tile t-2, whose last reads ended in the previous iteration) and issues the
            // loads of tile t+1+kRing4: that VALU and LDS work runs while its MFMAs
            // execute, and the other phase is the softmax alone.
            if constexpr (kTeam == 0) {
                // X: PV(t-1), QK(t), stage tile t+1
                pv_tile(prv, w.n, w.hh, P, acc);
                qk_tile(cur, w.n, w.hh, qf, S);
                store(ring[ks], nxt, nxt_f, t + 1);
                __builtin_amdgcn_sched_barrier(0);
                load(idn[ks], ring[ks]);
                idn[ks] = block_id4(p, nb4, w.b, t + 1 + 2 * kRing4, w.wt);
                phase_end();
                // Y: SM(t)
                softmax_tile(cur_f, tvalid_of(t), w.hh, S, acc, m, l, P);
                phase_end();
            } else {
                // X: SM(t-1)
                softmax_tile(prv_f, tvalid_of(t - 1), w.hh, S, acc, m, l, P);
                phase_end();
                // Y: PV(t-1), QK(t), stage tile t+1
                pv_tile(prv, w.n, w.hh, P, acc);
                qk_tile(cur, w.n, w.hh, qf, S);
                store(ring[ks], nxt, nxt_f, t + 1);
                __builtin_amdgcn_sched_barrier(0);
                load(idn[ks], ring[ks]);
                idn[ks] = block_id4(p, nb4, w.b, t + 1 + 2 * kRing4, w.wt);
                phase_end();
            }
        }
    }
}

#undef HKV_BUF
#undef HKV_FAC

// One workgroup per CU, 8 waves (two per SIMD), up to 256 registers per wave.
__global__ __launch_bounds__(kThreadsPP, 1) void prefill_attn_kernel(PrefillParams p) {
    extern __shared__ __align__(16) uint8_t lds_raw[];
    const int b = blockIdx.z;
    const int ngrp = (p.nrep + kTeamWaves - 1) / kTeamWaves;
    const int h = blockIdx.y / ngrp, grp = blockIdx.y % ngrp;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int team = wave >> 2, wt = wave & 3;
    const int q0 = blockIdx.x * kQB + team * kQ;
    const int n = lane & 31, hh = lane >> 5;
    const int rep = grp * kTeamWaves + wt;
    const bool head_ok = rep < p.nrep;
    const int qh = h * p.nrep + (head_ok ? rep : 0);
    const int qrow = q0 + n;

    TileMap tm;
    make_tile_map(p, b, (int)blockIdx.x * kQB + kQB, tm);
    // a sequence with no INT4 token was finished by the zone kernel
    if (tm.n4 == 0) return;

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
    float m = -INFINITY, l = 0.f;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
    // S and P start at zero and LDS buffer 2 as an empty tile (finite values, every token
    // masked): the first iteration's softmax and P.V of tile -1 then change nothing.
    f16v S[2];
    h8 P[4];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int r = 0; r < 16; ++r) S[tb][r] = 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int i = 0; i < 8; ++i) P[u][i] = (_Float16)0.f;
    for (int o = threadIdx.x * 16; o < kDataBytes; o += kThreadsPP * 16)
        *(u4*)(lds_raw + kNumBufs * kFacBytes + 2 * kDataBytes + o) = u4{0u, 0u, 0u, 0u};
    __syncthreads();
    if (threadIdx.x < kT) ((float*)(lds_raw + 2 * kFacBytes + kSbOff))[threadIdx.x] = -INFINITY;
    // The teams run mirrored loops (team 0 is half an iteration ahead); they meet at
    // every phase barrier.
    const WaveCtx wc{b, h, wt, lane, n, hh, qrow};
    if (team == 0) int4_tiles<0>(p, tm, wc, lds_raw, qf, acc, m, l, S, P);
    else int4_tiles<1>(p, tm, wc, lds_raw, qf, acc, m, l, S, P);

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
    const int ngrp = (nrep + kTeamWaves - 1) / kTeamWaves;
    HKV_REQUIRE((int64_t)a->num_kv_heads * ngrp < 65536 && a->batch < 65536, HKV_ERR_ARG,
                "hkv_prefill_attn: grid too large");
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
    p.state = (float*)a->workspace;
    // Which kernels run: the zone kernel whenever a sequence may have zone or chunk keys
    // or no INT4 token (it then writes the output), the INT4 kernel whenever there are
    // INT4 tokens; with both kinds of keys the zone kernel's state crosses the workspace.
    bool zone_keys = a->chunk_k != nullptr;
    for (int i = 0; i < a->num_f16_zones; ++i) zone_keys = zone_keys || a->f16[i].max_len > 0;
    const bool int4_keys = a->int4_max_len > 0;
    const bool run_zones = zone_keys || !int4_keys || a->int4_lens != nullptr;
    if (zone_keys && int4_keys) {
        const size_t need = hkv_prefill_workspace_bytes(a->batch, a->num_q_heads, a->num_queries);
        HKV_REQUIRE(a->workspace != nullptr && a->workspace_bytes >= need && (((uintptr_t)a->workspace) & 15) == 0,
                    HKV_ERR_ARG, "hkv_prefill_attn: INT4 and zone/chunk keys need a 16-byte aligned workspace of "
                    "%zu bytes (hkv_prefill_workspace_bytes), got %zu", need, a->workspace ? a->workspace_bytes : 0);
    }
    if (run_zones) {
        const int rc = launch_prefill_zones(p, ngrp, (hipStream_t)stream);
        if (rc != HKV_OK) return rc;
    }
    if (int4_keys) {
        const dim3 grid((a->num_queries + kQB - 1) / kQB, a->num_kv_heads * ngrp, a->batch);
        static bool raised = false;   // three tile buffers exceed the 64 KB default
        if (!raised) {
            HKV_HIP_CHECK(hipFuncSetAttribute((const void*)prefill_attn_kernel,
                                              hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes));
            raised = true;
        }
        hipLaunchKernelGGL(prefill_attn_kernel, grid, dim3(kThreadsPP), kLdsBytes, (hipStream_t)stream, p);
        HKV_LAUNCH_CHECK("prefill_attn_kernel");
    }
    return HKV_OK;
}

extern "C" size_t hkv_prefill_workspace_bytes(int32_t batch, int32_t num_q_heads, int32_t num_queries) {
    if (batch <= 0 || num_q_heads <= 0 || num_queries <= 0) return 0;
    return (size_t)batch * (size_t)num_q_heads * (size_t)num_queries * kStateFloats * sizeof(float);
}
