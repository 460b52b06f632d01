// Chunked prefill, zone kernel: the fp16 zone tiles and the causal chunk of every
// sequence (fused_dequant_attn.py:242-247 with kernels/fused_dequant_attn.py:371-435 as
// the entry point; the INT4 tiles are prefill_attn.hip's).  When the sequence also has
// INT4 tokens, it leaves its online-softmax state for the INT4 kernel; otherwise it
// writes the output.
//
// It runs the tile loop of prefill_flat.h over the zones in order, then the chunk.  The
// entry point has written the chunk in the zone layout (K rows [tok][128], 16-token V
// tiles), so every tile is staged the same way: waves 0-3 copy their 16 K rows, waves
// 4-7 turn their 16-token V tile into V^T rows.  Q carries sm_scale x log2 e (one fp16
// rounding per element), so the scores come out of the MFMAs in the log2 domain.  The
// chunk's diagonal tile (the tile of the workgroup's own 64 query rows) is the only one
// with a per-query causal mask.
#include "prefill_flat.h"

#include <math.h>

namespace hkv {
namespace {

typedef pu4 u4;
typedef pu2 u2;

// The fp16 staging policy of the tile loop: one register slot per wave (64 bytes per
// lane: a quarter of a tile's K rows or of its V tiles).
template <int kTeam>
struct F16Stage {
    static constexpr int kRing = 1;
    const PrefillParams& p;
    const TileMap& tm;
    const FlatWave& w;
    int zone_tiles;   // tiles of all zones; the chunk's tiles follow
    int diag;         // tile index of the chunk's diagonal tile (-1: none)
    u4 slot[4];

    __device__ F16Stage(const PrefillParams& p_, const TileMap& tm_, const FlatWave& w_)
        : p(p_), tm(tm_), w(w_) {
        zone_tiles = tm.nz_t[0] + tm.nz_t[1] + tm.nz_t[2];
        diag = tm.nc > 0 ? zone_tiles + w.qb : -1;
    }
    // Source of tile x: K rows, V tiles, capacity, valid length, tile index in the source.
    // The source index is found from the tile counts and the source read from the
    // argument block at that (wave-uniform) index: holding every source's pointers in
    // registers across the tile loop spilled ~100 scalar registers into vector lanes
    // (~55 lane moves per tile).
    __device__ void source(int x, const uint16_t*& k, const uint16_t*& v, int& cap, int& len, int& xl) const {
        int si = 0;
        xl = x;
#pragma unroll
        for (int zi = 0; zi < HKV_MAX_F16_ZONES; ++zi) {
            if (si == zi && xl >= tm.nz_t[zi]) {   // zones beyond p.nz have no tiles
                xl -= tm.nz_t[zi];
                si = zi + 1;
            }
        }
        const bool ok = si < HKV_MAX_F16_ZONES || xl < tm.nc;
        const PfSrc& s = p.src[si];
        k = s.k;
        v = s.v;
        cap = s.cap;
        len = !ok ? 0 : si == 0 ? tm.lenz[0] : si == 1 ? tm.lenz[1] : si == 2 ? tm.lenz[2] : p.Sq;
        if (!ok) xl = 0;
    }
    __device__ int tvalid(int x) const {
        const uint16_t *k, *v;
        int cap, len, xl;
        source(x, k, v, cap, len, xl);
        return min(kPfT, max(0, len - xl * kPfT));
    }
    __device__ void load(int x) { load_into(x, slot); }
    __device__ void load_into(int x, u4 (&dst)[4]) const {
        const uint16_t *k, *v;
        int cap, len, xl;
        source(x, k, v, cap, len, xl);
        const int64_t bh = (int64_t)w.b * p.Hkv + w.h;
        if constexpr (kTeam == 0) {
            // K row of token 16 wt + lane/4, dims 32 (lane % 4) .. +32
            const int tok = xl * kPfT + w.wt * 16 + (w.lane >> 2);
            if (tok < len) {
                const uint16_t* kp = k + (bh * cap + tok) * kHeadDim + (w.lane & 3) * 32;
#pragma unroll
                for (int j = 0; j < 4; ++j) dst[j] = *(const u4*)(kp + 8 * j);
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) dst[j] = u4{0u, 0u, 0u, 0u};
            }
        } else {
            // 64 bytes of the 16-token V tile 4 xl + wt: halves [n][i] = V[4g + i][c + 16n]
            const int ztl = xl * 4 + w.wt;
            if (ztl * kBlockTokens < len) {
                const uint16_t* vp = v + (bh * (cap / kBlockTokens) + ztl) * (kBlockTokens * kHeadDim) + w.lane * 32;
#pragma unroll
                for (int j = 0; j < 4; ++j) dst[j] = *(const u4*)(vp + 8 * j);
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) dst[j] = u4{0u, 0u, 0u, 0u};
            }
        }
    }
    __device__ void stage(int, uint8_t* buf, uint8_t* bias, int x) const {
        const uint16_t *k, *v;
        int cap, len, xl;
        source(x, k, v, cap, len, xl);
        if constexpr (kTeam == 0) {
            const int tok = w.wt * 16 + (w.lane >> 2), pt = w.lane & 3;
            const bool ok = xl * kPfT + tok < len;
#pragma unroll
            for (int j = 0; j < 4; ++j) *(u4*)(buf + k_addr(tok, pt * 4 + j)) = ok ? slot[j] : u4{0u, 0u, 0u, 0u};
            if (pt == 0) ((float*)bias)[tok] = ok ? 0.0f : -INFINITY;
        } else {
            // V^T rows c + 16n, unit 4 wt + g (tokens 16 wt + 4g .. +3); tokens past the
            // length are cleared so masked probabilities multiply finite values
            const int g = w.lane >> 4, c = w.lane & 15;
            const int base = xl * kPfT + w.wt * 16 + 4 * g;
            const uint32_t m01 = (base + 0 < len ? 0x0000FFFFu : 0u) | (base + 1 < len ? 0xFFFF0000u : 0u);
            const uint32_t m23 = (base + 2 < len ? 0x0000FFFFu : 0u) | (base + 3 < len ? 0xFFFF0000u : 0u);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                *(u2*)(buf + vt_addr(c + 32 * j, w.wt * 4 + g)) = u2{slot[j].x & m01, slot[j].y & m23};
                *(u2*)(buf + vt_addr(c + 32 * j + 16, w.wt * 4 + g)) = u2{slot[j].z & m01, slot[j].w & m23};
            }
        }
    }
    __device__ void refill(int, int x) { load(x + kRing); }
    __device__ void start(uint8_t* lds) {
        // tiles 0 and 1 requested together: one load round trip before the loop, not two
        u4 next[4];
        load(0);
        load_into(1, next);
        stage(0, flat_buf(lds, 0), flat_bias(lds, 0), 0);
#pragma unroll
        for (int j = 0; j < 4; ++j) slot[j] = next[j];
        stage(0, flat_buf(lds, 1), flat_bias(lds, 1), 1);
        load(2);
    }
    // The chunk's diagonal tile: token t (chunk position xl * 64 + t) is visible to query
    // row qrow when xl * 64 + t <= qrow.
    __device__ void mask(int x, pf16v (&S)[2]) const {
        if (x == diag) {
            const int lim = w.qrow - (x - zone_tiles) * kPfT;
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (tb * 32 + 8 * (r >> 2) + 4 * w.hh + (r & 3) > lim) S[tb][r] = -INFINITY;
        }
    }
};

// One workgroup per CU: 8 waves (two per SIMD) over one kv head and 64 query rows.
__global__ __launch_bounds__(kFlatThreads, 1) void prefill_zones_kernel(PrefillParams p) {
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
    const int nf = tm.nf();
    // Sequences with INT4 tokens and no zone or chunk tile: the INT4 kernel starts at zero
    if (tm.n4 > 0 && nf == 0) return;

    ph8 qf[8];
    flat_load_q(p, b, qh, head_ok && qrow < p.Sq, qrow, hh, p.scale_log2, qf);
    pf16v acc[4];
    float m = -INFINITY, l = 0.f;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[db][r] = 0.f;
    const FlatWave fw{b, h, wt, lane, n, hh, qrow, blk.qb};
    const int T = (nf + kFlatBufs - 1) / kFlatBufs * kFlatBufs;
    if (team == 0) {
        F16Stage<0> pol(p, tm, fw);
        flat_tiles(pol, fw, lds_raw, qf, acc, m, l, T);
    } else {
        // waves 4-7 (the V^T staging, the larger share of VALU work) win issue ties
        // against the older waves 0-3 on their SIMDs
        __builtin_amdgcn_s_setprio(1);
        F16Stage<1> pol(p, tm, fw);
        flat_tiles(pol, fw, lds_raw, qf, acc, m, l, T);
        __builtin_amdgcn_s_setprio(0);
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
                    *(pf4*)(st_row + 32 * db + 8 * j + 4 * hh) =
                        pf4{acc[db][4 * j + 0], acc[db][4 * j + 1], acc[db][4 * j + 2], acc[db][4 * j + 3]};
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
    const dim3 grid((p.Sq + kFlatQ - 1) / kFlatQ, p.Hkv * ngrp, p.B);
    static std::atomic<uint64_t> raised{0};   // four tile buffers exceed the 64 KB default
    HKV_RAISE_LDS(prefill_zones_kernel, kFlatLdsBytes, raised);
    hipLaunchKernelGGL(prefill_zones_kernel, grid, dim3(kFlatThreads), kFlatLdsBytes, stream, p);
    HKV_LAUNCH_CHECK("prefill_zones_kernel");
    return HKV_OK;
}

}  // namespace hkv
