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
};

// One workgroup of 128 lanes per (token, head, sequence); lane = dim.
__global__ __launch_bounds__(128) void zone_write_kernel(ZoneWriteParams p) {
    const int t = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int d = threadIdx.x;
    int slot = (p.slot_start ? p.slot_start[b] : p.slot_base) + t;
    if (p.ring > 0) {
        slot %= p.ring;
        if (slot < 0) slot += p.ring;
    }
    if (slot < 0 || slot >= p.cap) return;
    const int64_t src = (int64_t)b * p.sb + (int64_t)h * p.sh + (int64_t)t * p.st + d;
    const int64_t bh = (int64_t)b * p.H + h;
    p.zk[(bh * p.cap + slot) * kHeadDim + d] = p.k[src];
    const int64_t tile = bh * (p.cap / kBlockTokens) + slot / kBlockTokens;
    p.zv[tile * (kBlockTokens * kHeadDim) + vtile_off(slot & 15, d)] = p.v[src];
}

__global__ __launch_bounds__(128) void zone_copy_kernel(const uint16_t* __restrict__ sk,
                                                        const uint16_t* __restrict__ sv, int scap, int s0,
                                                        uint16_t* __restrict__ dk, uint16_t* __restrict__ dv,
                                                        int dcap, int d0, int H) {
    const int i = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int d = threadIdx.x;
    const int64_t bh = (int64_t)b * H + h;
    const int ss = s0 + i, ds = d0 + i;
    dk[(bh * dcap + ds) * kHeadDim + d] = sk[(bh * scap + ss) * kHeadDim + d];
    dv[(bh * (dcap / kBlockTokens) + ds / kBlockTokens) * (kBlockTokens * kHeadDim) + vtile_off(ds & 15, d)] =
        sv[(bh * (scap / kBlockTokens) + ss / kBlockTokens) * (kBlockTokens * kHeadDim) + vtile_off(ss & 15, d)];
}

__global__ __launch_bounds__(128) void zone_read_kernel(const uint16_t* __restrict__ zk,
                                                        const uint16_t* __restrict__ zv, int H,
                                                        int cap, int n, uint16_t* __restrict__ ok,
                                                        uint16_t* __restrict__ ov) {
    const int s = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int d = threadIdx.x;
    const int64_t bh = (int64_t)b * H + h;
    const int64_t dst = (bh * n + s) * kHeadDim + d;
    if (ok) ok[dst] = zk[(bh * cap + s) * kHeadDim + d];
    if (ov) {
        const int64_t tile = bh * (cap / kBlockTokens) + s / kBlockTokens;
        ov[dst] = zv[tile * (kBlockTokens * kHeadDim) + vtile_off(s & 15, d)];
    }
}

}  // namespace
}  // namespace hkv

using namespace hkv;

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
    hipLaunchKernelGGL(zone_write_kernel, dim3(a->num_tokens, a->num_kv_heads, a->batch), dim3(128), 0,
                       (hipStream_t)stream, p);
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
    hipLaunchKernelGGL(zone_read_kernel, dim3(n, num_kv_heads, batch), dim3(128), 0, (hipStream_t)stream,
                       zone_k, zone_v, num_kv_heads, capacity, n, out_k, out_v);
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
    hipLaunchKernelGGL(zone_copy_kernel, dim3(n, num_kv_heads, batch), dim3(128), 0, (hipStream_t)stream, src_k,
                       src_v, src_capacity, src_slot, dst_k, dst_v, dst_capacity, dst_slot, num_kv_heads);
    HKV_LAUNCH_CHECK("zone_copy_kernel");
    return HKV_OK;
}
