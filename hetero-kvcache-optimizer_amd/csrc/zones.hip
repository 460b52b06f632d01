// fp16 zone storage (sink, recent window, heavy hitters) and the library's common
// entry points (version, last error, record size).
#include "hkv_internal.h"

#include <string.h>

namespace hkv {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

namespace {

// Halves offset of V[token s][dim d] inside a 16-token transposed tile:
// [g = s/4][c = d%16][n = d/16][i = s%4].
typedef uint32_t u4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int vtile_off(int s, int d) {
    return (((s >> 2) * 16 + (d & 15)) * 8 + (d >> 4)) * 4 + (s & 3);
}

struct ZoneWriteParams {
    const uint16_t* k;
    const uint16_t* v;
    int64_t sb, sh, st;
    int H, T;
    const int32_t* slot_start;
    int slot_base;
    int cap, ring;
    uint16_t* zk;
    uint16_t* zv;
    int bf16;      // source is bfloat16 (converted to fp16, range-checked)
    int* err;
};

// fp16 bits of a source element; sets `over` when a finite bf16 value leaves the fp16
// range (it becomes +-inf).  In range the conversion is exact (8 significant bits fit
// in 11) down to 2^-14; below that fp16 subnormals round to 2^-24.
__device__ __forceinline__ uint16_t to_f16(uint16_t x, bool bf16, bool& over) {
    if (!bf16) return x;
    const float f = bf2f(x);
    const uint16_t h = f2h_rn(f);
    over |= ((h & 0x7fffu) == 0x7c00u) && fabsf(f) < INFINITY;
    return h;
}

__device__ __forceinline__ void report_range(bool over, int* err) {
    if (__ballot(over) && (threadIdx.x & 63) == 0 && err) atomicOr(err, HKV_ERR_BIT_RANGE);
}

// One workgroup of 256 lanes per 16 source tokens (and head, sequence): lane t moves
// 16 bytes (8 dims) of token t/16.  K rows are copied with 16-byte accesses.  When the
// 16 tokens fill one whole V tile (their slots are 16 consecutive slots starting at a
// multiple of 16), the tile is transposed through LDS and written with one 16-byte
// store per lane; otherwise each lane writes its 8 V values into their tile slots.
__global__ __launch_bounds__(256) void zone_write_kernel(ZoneWriteParams p) {
    touch_kernel_args(p);
    __shared__ __align__(16) uint16_t sv[kBlockTokens][kHeadDim + 8];   // +8 halves: rows start on different banks
    const int j = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int t = threadIdx.x, r = t >> 4, q = t & 15;
    const int base = p.slot_start ? p.slot_start[b] : p.slot_base;
    auto slot_of = [&](int ts) {
        int s = base + ts;
        if (p.ring > 0) {
            s %= p.ring;
            if (s < 0) s += p.ring;
        }
        return s;
    };
    const int ts = j * kBlockTokens + r;
    const int s0 = slot_of(j * kBlockTokens);
    const bool whole_tile = j * kBlockTokens + kBlockTokens <= p.T && (s0 & (kBlockTokens - 1)) == 0 &&
                            s0 >= 0 && s0 + kBlockTokens <= p.cap && (p.ring == 0 || s0 + kBlockTokens <= p.ring);
    const int64_t bh = (int64_t)b * p.H + h;
    bool over = false;
    uint16_t vv[8];
    int slot = -1;
    if (ts < p.T) {
        const int64_t src = (int64_t)b * p.sb + (int64_t)h * p.sh + (int64_t)ts * p.st + 8 * q;
        const u4v kw = *(const u4v*)(p.k + src);
        const u4v vw = *(const u4v*)(p.v + src);
        const bool bf = p.bf16 != 0;
        u4v ko;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t lo = to_f16((uint16_t)(kw[e] & 0xffffu), bf, over);
            const uint32_t hi = to_f16((uint16_t)(kw[e] >> 16), bf, over);
            ko[e] = lo | (hi << 16);
            vv[2 * e] = to_f16((uint16_t)(vw[e] & 0xffffu), bf, over);
            vv[2 * e + 1] = to_f16((uint16_t)(vw[e] >> 16), bf, over);
        }
        slot = slot_of(ts);
        if (slot >= 0 && slot < p.cap) *(u4v*)(p.zk + (bh * p.cap + slot) * kHeadDim + 8 * q) = ko;
    }
    report_range(over, p.err);
    if (whole_tile) {
        u4v pw;
#pragma unroll
        for (int e = 0; e < 4; ++e) pw[e] = (uint32_t)vv[2 * e] | ((uint32_t)vv[2 * e + 1] << 16);
        *(u4v*)&sv[r][8 * q] = pw;
        __syncthreads();
        // 16-byte piece t of the tile: halves [g][c][n][i] with g = t/64, c = (t/4)%16,
        // n = 2(t%4) + {0,1}, i = 0..3, i.e. V[4g+i][c+16n]
        const int g = t >> 6, c = (t >> 2) & 15, n0 = 2 * (t & 3);
        uint16_t o[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) o[u] = sv[4 * g + (u & 3)][c + 16 * (n0 + (u >> 2))];
        u4v w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = (uint32_t)o[2 * e] | ((uint32_t)o[2 * e + 1] << 16);
        const int64_t tile = bh * (p.cap / kBlockTokens) + s0 / kBlockTokens;
        *(u4v*)(p.zv + tile * (kBlockTokens * kHeadDim) + 8 * t) = w;
    } else if (ts < p.T && slot >= 0 && slot < p.cap) {
        const int64_t tile = bh * (p.cap / kBlockTokens) + slot / kBlockTokens;
#pragma unroll
        for (int e = 0; e < 8; ++e) p.zv[tile * (kBlockTokens * kHeadDim) + vtile_off(slot & 15, 8 * q + e)] = vv[e];
    }
}

// Copies and reads work on 16-slot tiles: one 256-thread workgroup per tile of the slot
// range, thread (r, q) = (t / 16, t % 16) owns slot r of the tile and dims 8q .. 8q+7.
// K rows move as 16-byte pieces.  V tiles are stored transposed (vtile_off), so a V
// read stages the whole 4 KB tile in LDS with 16-byte loads and writes row-major
// 16-byte pieces; a copy between tile-aligned ranges moves whole tiles as 16-byte
// pieces, any other copy moves V element by element.
__global__ __launch_bounds__(256) void zone_copy_kernel(const uint16_t* __restrict__ sk,
                                                        const uint16_t* __restrict__ sv, int scap, int s0,
                                                        uint16_t* __restrict__ dk, uint16_t* __restrict__ dv,
                                                        int dcap, int d0, int n, int H) {
    const int tile = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int t = threadIdx.x, r = t >> 4, q = t & 15;
    const int64_t bh = (int64_t)b * H + h;
    const int i = tile * kBlockTokens + r;   // slot of the copy range
    if (i < n)
        *(u4v*)(dk + (bh * dcap + d0 + i) * kHeadDim + 8 * q) = *(const u4v*)(sk + (bh * scap + s0 + i) * kHeadDim + 8 * q);
    if (s0 % kBlockTokens == 0 && d0 % kBlockTokens == 0 && tile * kBlockTokens + kBlockTokens <= n) {
        const int64_t st = bh * (scap / kBlockTokens) + (s0 / kBlockTokens + tile);
        const int64_t dt = bh * (dcap / kBlockTokens) + (d0 / kBlockTokens + tile);
        *(u4v*)(dv + dt * (kBlockTokens * kHeadDim) + 8 * t) = *(const u4v*)(sv + st * (kBlockTokens * kHeadDim) + 8 * t);
    } else if (i < n) {
        const int ss = s0 + i, ds = d0 + i;
        const uint16_t* src = sv + (bh * (scap / kBlockTokens) + ss / kBlockTokens) * (kBlockTokens * kHeadDim);
        uint16_t* dst = dv + (bh * (dcap / kBlockTokens) + ds / kBlockTokens) * (kBlockTokens * kHeadDim);
#pragma unroll
        for (int e = 0; e < 8; ++e) dst[vtile_off(ds & 15, 8 * q + e)] = src[vtile_off(ss & 15, 8 * q + e)];
    }
}

__global__ __launch_bounds__(256) void zone_read_kernel(const uint16_t* __restrict__ zk,
                                                        const uint16_t* __restrict__ zv, int H,
                                                        int cap, int n, uint16_t* __restrict__ ok,
                                                        uint16_t* __restrict__ ov) {
    const int tile = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int t = threadIdx.x, r = t >> 4, q = t & 15;
    const int64_t bh = (int64_t)b * H + h;
    const int s = tile * kBlockTokens + r;
    if (ok && s < n) *(u4v*)(ok + (bh * n + s) * kHeadDim + 8 * q) = *(const u4v*)(zk + (bh * cap + s) * kHeadDim + 8 * q);
    if (ov) {
        __shared__ __align__(16) uint16_t sv[kBlockTokens * kHeadDim];
        *(u4v*)&sv[8 * t] = *(const u4v*)(zv + (bh * (cap / kBlockTokens) + tile) * (kBlockTokens * kHeadDim) + 8 * t);
        __syncthreads();
        if (s < n) {
            u4v w;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                w[e] = (uint32_t)sv[vtile_off(r, 8 * q + 2 * e)] | ((uint32_t)sv[vtile_off(r, 8 * q + 2 * e + 1)] << 16);
            *(u4v*)(ov + (bh * n + s) * kHeadDim + 8 * q) = w;
        }
    }
}

// ---- device-stepped decode update: the decision of the manager's decode step
// (manager.py:588-674 as this library keeps it) taken on the GPU from `state`, so the
// step can be replayed from a captured graph.
struct ZoneStepParams {
    const uint16_t* k;
    const uint16_t* v;
    int64_t sb, sh;
    int H;
    uint16_t* tk;
    uint16_t* tv;
    int tcap, ring;
    uint16_t* hk;
    uint16_t* hv;
    int hcap, hbudget;
    int* state;   // tail_head, tail_len, hh_len, dropped
    int* tail_lens;
    int* hh_lens;
    int B;
    int bf16;
    int* err;
};

__device__ __forceinline__ int64_t vtile_index(int64_t bh, int cap, int slot, int d) {
    return (bh * (cap / kBlockTokens) + slot / kBlockTokens) * (kBlockTokens * kHeadDim) + vtile_off(slot & 15, d);
}

__device__ inline bool state_ok(const ZoneStepParams& p, int head, int len, int hh) {
    return head >= 0 && head < p.ring && len >= 0 && len <= p.ring && hh >= 0 && hh <= p.hbudget;
}

// One workgroup of 128 lanes (lane = dim) per (kv head, sequence): when the ring is
// full its oldest token moves to the heavy-hitter zone (while it has room) before
// the new token takes its slot.  Every lane reads and writes only its own dim.
__global__ __launch_bounds__(128) void zone_step_kernel(ZoneStepParams p) {
    touch_kernel_args(p);
    const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
    const int head = p.state[0], len = p.state[1], hh = p.state[2];
    if (!state_ok(p, head, len, hh)) return;   // a state no step produced: write nothing
    const int64_t bh = (int64_t)b * p.H + h;
    int slot = head;
    if (len < p.ring) {
        slot = (head + len) % p.ring;
    } else if (hh < p.hbudget) {
        p.hk[(bh * p.hcap + hh) * kHeadDim + d] = p.tk[(bh * p.tcap + head) * kHeadDim + d];
        p.hv[vtile_index(bh, p.hcap, hh, d)] = p.tv[vtile_index(bh, p.tcap, head, d)];
    }
    const int64_t src = (int64_t)b * p.sb + (int64_t)h * p.sh + d;
    bool over = false;
    p.tk[(bh * p.tcap + slot) * kHeadDim + d] = to_f16(p.k[src], p.bf16 != 0, over);
    p.tv[vtile_index(bh, p.tcap, slot, d)] = to_f16(p.v[src], p.bf16 != 0, over);
    report_range(over, p.err);
}

// Advances the state after the step and publishes the zone lengths per sequence.
__global__ __launch_bounds__(256) void zone_advance_kernel(ZoneStepParams p) {
    touch_kernel_args(p);
    int head = p.state[0], len = p.state[1], hh = p.state[2], dropped = p.state[3];
    if (!state_ok(p, head, len, hh)) return;
    if (len < p.ring) {
        ++len;
    } else {
        if (hh < p.hbudget)
            ++hh;
        else
            ++dropped;
        head = (head + 1) % p.ring;
    }
    for (int b = threadIdx.x; b < p.B; b += 256) {
        if (p.tail_lens) p.tail_lens[b] = len;
        if (p.hh_lens) p.hh_lens[b] = hh;
    }
    __syncthreads();   // every lane has read the old state
    if (threadIdx.x == 0) {
        p.state[0] = head;
        p.state[1] = len;
        p.state[2] = hh;
        p.state[3] = dropped;
    }
}

}  // namespace
}  // namespace hkv

using namespace hkv;

extern "C" int hkv_zone_step(const HkvZoneStepArgs* a, void* stream) {
    clear_error();
    HKV_REQUIRE(a != nullptr, HKV_ERR_ARG, "hkv_zone_step: null args");
    HKV_REQUIRE(a->head_dim == kHeadDim, HKV_ERR_UNSUPPORTED, "hkv_zone_step: head_dim %d != 128", a->head_dim);
    HKV_REQUIRE(a->batch > 0 && a->batch <= 65535 && a->num_kv_heads > 0 && a->num_kv_heads <= 65535, HKV_ERR_ARG,
                "hkv_zone_step: bad sizes");
    HKV_REQUIRE(a->k && a->v && a->tail_k && a->tail_v && a->state, HKV_ERR_ARG, "hkv_zone_step: null pointer");
    HKV_REQUIRE(a->dtype == HKV_DTYPE_F16 || a->dtype == HKV_DTYPE_BF16, HKV_ERR_ARG,
                "hkv_zone_step: dtype %d is neither fp16 nor bf16", a->dtype);
    HKV_REQUIRE(a->tail_capacity > 0 && a->tail_capacity % kBlockTokens == 0 && a->tail_ring > 0 &&
                    a->tail_ring <= a->tail_capacity,
                HKV_ERR_ARG, "hkv_zone_step: tail ring %d / capacity %d", a->tail_ring, a->tail_capacity);
    HKV_REQUIRE(a->hh_budget >= 0 && (a->hh_budget == 0 || (a->hh_k && a->hh_v && a->hh_capacity >= a->hh_budget &&
                                                              a->hh_capacity % kBlockTokens == 0)),
                HKV_ERR_ARG, "hkv_zone_step: heavy-hitter budget %d / capacity %d", a->hh_budget, a->hh_capacity);
    ZoneStepParams p;
    p.k = a->k;
    p.v = a->v;
    p.sb = a->src_stride_b;
    p.sh = a->src_stride_h;
    p.H = a->num_kv_heads;
    p.tk = a->tail_k;
    p.tv = a->tail_v;
    p.tcap = a->tail_capacity;
    p.ring = a->tail_ring;
    p.hk = a->hh_k;
    p.hv = a->hh_v;
    p.hcap = a->hh_capacity;
    p.hbudget = a->hh_budget;
    p.state = a->state;
    p.tail_lens = a->tail_lens;
    p.hh_lens = a->hh_lens;
    p.B = a->batch;
    p.bf16 = a->dtype == HKV_DTYPE_BF16;
    p.err = a->err_flag;
    hipLaunchKernelGGL(zone_step_kernel, dim3(a->num_kv_heads, a->batch), dim3(128), 0, (hipStream_t)stream, p);
    HKV_LAUNCH_CHECK("zone_step_kernel");
    hipLaunchKernelGGL(zone_advance_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, p);
    HKV_LAUNCH_CHECK("zone_advance_kernel");
    return HKV_OK;
}

extern "C" int hkv_abi_version(void) { return HKV_ABI_VERSION; }

extern "C" const char* hkv_last_error(void) { return g_last_error; }

extern "C" int64_t hkv_block_bytes(int32_t num_kv_heads, int32_t head_dim) {
    if (num_kv_heads <= 0 || head_dim != kHeadDim) return -1;
    return RecordLayout(num_kv_heads).bytes;
}

extern "C" int hkv_zone_write(const HkvZoneWriteArgs* a, void* stream) {
    clear_error();
    HKV_REQUIRE(a != nullptr, HKV_ERR_ARG, "hkv_zone_write: null args");
    HKV_REQUIRE(a->head_dim == kHeadDim, HKV_ERR_UNSUPPORTED, "hkv_zone_write: head_dim %d != 128", a->head_dim);
    HKV_REQUIRE(a->capacity > 0 && a->capacity % kBlockTokens == 0, HKV_ERR_ARG,
                "hkv_zone_write: capacity %d must be a positive multiple of 16", a->capacity);
    HKV_REQUIRE(a->batch >= 0 && a->num_kv_heads > 0 && a->num_tokens >= 0, HKV_ERR_ARG,
                "hkv_zone_write: bad sizes");
    if (a->batch == 0 || a->num_tokens == 0) return HKV_OK;
    HKV_REQUIRE(a->k && a->v && a->zone_k && a->zone_v, HKV_ERR_ARG,
                "hkv_zone_write: null pointer");
    HKV_REQUIRE(a->num_kv_heads <= 65535 && a->batch <= 65535, HKV_ERR_ARG, "hkv_zone_write: grid too large");
    HKV_REQUIRE(a->ring >= 0 && a->ring <= a->capacity, HKV_ERR_ARG,
                "hkv_zone_write: ring %d must be in [0, capacity %d]", a->ring, a->capacity);
    HKV_REQUIRE(a->dtype == HKV_DTYPE_F16 || a->dtype == HKV_DTYPE_BF16, HKV_ERR_ARG,
                "hkv_zone_write: dtype %d is neither fp16 nor bf16", a->dtype);
    HKV_REQUIRE((((uintptr_t)a->k | (uintptr_t)a->v) & 15) == 0 && a->src_stride_b % 8 == 0 &&
                    a->src_stride_h % 8 == 0 && a->src_stride_t % 8 == 0,
                HKV_ERR_ARG, "hkv_zone_write: k/v must be 16-byte aligned with strides multiple of 8");
    ZoneWriteParams p;
    p.k = a->k;
    p.v = a->v;
    p.sb = a->src_stride_b;
    p.sh = a->src_stride_h;
    p.st = a->src_stride_t;
    p.H = a->num_kv_heads;
    p.T = a->num_tokens;
    p.slot_start = a->slot_start;
    p.slot_base = a->slot_base;
    p.cap = a->capacity;
    p.ring = a->ring;
    p.zk = a->zone_k;
    p.zv = a->zone_v;
    p.bf16 = a->dtype == HKV_DTYPE_BF16;
    p.err = a->err_flag;
    hipLaunchKernelGGL(zone_write_kernel, dim3((a->num_tokens + kBlockTokens - 1) / kBlockTokens, a->num_kv_heads,
                                               a->batch),
                       dim3(256), 0, (hipStream_t)stream, p);
    HKV_LAUNCH_CHECK("zone_write_kernel");
    return HKV_OK;
}

extern "C" int hkv_zone_read(const uint16_t* zone_k, const uint16_t* zone_v, int32_t batch,
                             int32_t num_kv_heads, int32_t head_dim, int32_t capacity, int32_t n,
                             uint16_t* out_k, uint16_t* out_v, void* stream) {
    clear_error();
    HKV_REQUIRE(head_dim == kHeadDim, HKV_ERR_UNSUPPORTED, "hkv_zone_read: head_dim %d != 128", head_dim);
    HKV_REQUIRE(capacity > 0 && capacity % kBlockTokens == 0, HKV_ERR_ARG,
                "hkv_zone_read: capacity must be a positive multiple of 16");
    HKV_REQUIRE(n >= 0 && n <= capacity && batch >= 0 && num_kv_heads > 0, HKV_ERR_ARG,
                "hkv_zone_read: bad sizes");
    if (n == 0 || batch == 0) return HKV_OK;
    HKV_REQUIRE(zone_k && zone_v && (out_k || out_v), HKV_ERR_ARG, "hkv_zone_read: null pointer");
    HKV_REQUIRE((((uintptr_t)zone_k | (uintptr_t)zone_v | (uintptr_t)out_k | (uintptr_t)out_v) & 15) == 0, HKV_ERR_ARG,
                "hkv_zone_read: zone and output pointers must be 16-byte aligned");
    hipLaunchKernelGGL(zone_read_kernel, dim3((n + kBlockTokens - 1) / kBlockTokens, num_kv_heads, batch), dim3(256), 0,
                       (hipStream_t)stream, zone_k, zone_v, num_kv_heads, capacity, n, out_k, out_v);
    HKV_LAUNCH_CHECK("zone_read_kernel");
    return HKV_OK;
}

extern "C" int hkv_zone_copy(const uint16_t* src_k, const uint16_t* src_v, int32_t src_capacity,
                             int32_t src_slot, uint16_t* dst_k, uint16_t* dst_v, int32_t dst_capacity,
                             int32_t dst_slot, int32_t batch, int32_t num_kv_heads, int32_t head_dim,
                             int32_t n, void* stream) {
    clear_error();
    HKV_REQUIRE(head_dim == kHeadDim, HKV_ERR_UNSUPPORTED, "hkv_zone_copy: head_dim %d != 128", head_dim);
    HKV_REQUIRE(src_capacity > 0 && src_capacity % kBlockTokens == 0 && dst_capacity > 0 &&
                    dst_capacity % kBlockTokens == 0,
                HKV_ERR_ARG, "hkv_zone_copy: capacities must be positive multiples of 16");
    HKV_REQUIRE(n >= 0 && batch >= 0 && num_kv_heads > 0 && num_kv_heads <= 65535 && batch <= 65535, HKV_ERR_ARG,
                "hkv_zone_copy: bad sizes");
    HKV_REQUIRE(src_slot >= 0 && dst_slot >= 0 && (int64_t)src_slot + n <= src_capacity &&
                    (int64_t)dst_slot + n <= dst_capacity,
                HKV_ERR_CAPACITY, "hkv_zone_copy: slot range outside a zone");
    if (n == 0 || batch == 0) return HKV_OK;
    HKV_REQUIRE(src_k && src_v && dst_k && dst_v, HKV_ERR_ARG, "hkv_zone_copy: null pointer");
    HKV_REQUIRE((((uintptr_t)src_k | (uintptr_t)src_v | (uintptr_t)dst_k | (uintptr_t)dst_v) & 15) == 0, HKV_ERR_ARG,
                "hkv_zone_copy: zone pointers must be 16-byte aligned");
    hipLaunchKernelGGL(zone_copy_kernel, dim3((n + kBlockTokens - 1) / kBlockTokens, num_kv_heads, batch), dim3(256), 0,
                       (hipStream_t)stream, src_k, src_v, src_capacity, src_slot, dst_k, dst_v, dst_capacity, dst_slot,
                       n, num_kv_heads);
    HKV_LAUNCH_CHECK("zone_copy_kernel");
    return HKV_OK;
}
