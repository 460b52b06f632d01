// INT4 asymmetric group quantizer: the reference-layout compress/decompress
// (kv_compressor.py:50-132) and the quantize+pack kernel that appends tokens to
// the INT4 block pool.
#include "hkv_internal.h"

#include <math.h>

namespace hkv {
namespace {

// --------------------------------------------------------------------------
// Reference layout: one wavefront per group of `G` flattened elements; the last
// group is zero-padded (kv_compressor.py:70-74), so padding takes part in min/max.
// min/max are IEEE minimum/maximum (v_minimum3/v_maximum3), which propagate NaN as
// torch's min/max do: a group holding a NaN gets a NaN scale, and its zero point
// and codes are 0 (NaN clamps to 0 here; torch's .to(uint8) gives 0).
__global__ __launch_bounds__(256) void quantize_groups_kernel(
    const void* __restrict__ x, int dtype, int64_t n, int G, int64_t ngroups,
    uint8_t* __restrict__ codes, float* __restrict__ scales, uint8_t* __restrict__ zps) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) >> 6;
    for (int64_t g = wave; g < ngroups; g += nwaves) {
        const int64_t base = g * (int64_t)G;
        float mn = INFINITY, mx = -INFINITY;
        for (int i = lane; i < G; i += 64) {
            const int64_t idx = base + i;
            const float v = idx < n ? load_as_float(x, dtype, idx) : 0.0f;
            mn = __builtin_elementwise_minimum(mn, v);
            mx = __builtin_elementwise_maximum(mx, v);
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            mn = __builtin_elementwise_minimum(mn, __shfl_xor(mn, off));
            mx = __builtin_elementwise_maximum(mx, __shfl_xor(mx, off));
        }
        const QParams q = qparams_from_minmax(mn, mx);
        if (lane == 0) {
            scales[g] = q.scale;
            zps[g] = q.zp;
        }
        for (int i = lane; i < G; i += 64) {
            const int64_t idx = base + i;
            if (idx < n) codes[idx] = (uint8_t)quant_code(load_as_float(x, dtype, idx), q);
        }
    }
}

// kv_compressor.py:131-132: (q - zp) * scale in float32, then cast (round to nearest
// even).  One wavefront per group (as the quantizer), so the group's scale and zero
// point are read once and no element needs an index division.
__global__ __launch_bounds__(256) void dequantize_groups_kernel(
    const uint8_t* __restrict__ codes, const float* __restrict__ scales,
    const uint8_t* __restrict__ zps, int64_t n, int G, int64_t ngroups, void* __restrict__ out, int out_dtype) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) >> 6;
    for (int64_t g = wave; g < ngroups; g += nwaves) {
        const float zp = (float)zps[g], sc = scales[g];
        const int64_t base = g * (int64_t)G;
        for (int i = lane; i < G; i += 64) {
            const int64_t idx = base + i;
            if (idx >= n) break;
            const float v = ((float)codes[idx] - zp) * sc;
            if (out_dtype == HKV_DTYPE_F16) ((uint16_t*)out)[idx] = f2h_rn(v);
            else if (out_dtype == HKV_DTYPE_BF16) ((uint16_t*)out)[idx] = f2bf_rn(v);
            else ((float*)out)[idx] = v;
        }
    }
}

// --------------------------------------------------------------------------
// Quantize + pack into block records.  One workgroup per (logical block, head,
// sequence).  Phase 1: 8 lanes per token row (K rows 0..15, V rows 16..31) compute
// min/max, scale, zp and the codes; K words, scales and zero points go straight into
// the record part assembled in LDS, V codes into an LDS byte array.  Phase 2: every lane
// assembles one V word of the part.  Phase 3: the part is written with 16-byte stores
// (~1% slower than 4-byte stores straight from phase 1 and 2 on the 8 x 4096-token K+V
// pack, 8.30-8.34 vs 8.21-8.30 us; having 64 lanes build the V pieces themselves instead
// of the third barrier: 9.1 us).
struct PackParams {
    const void* k;
    const void* v;
    int dtype;
    int64_t sb, sh, st;
    int H, T;
    const int32_t* start_pos;    // null: every sequence starts at start_base
    const int32_t* bt;
    int bt_stride;
    uint8_t* pool;
    int64_t pool_blocks;
    int32_t* err;
    int vec_ok;  // 16-byte aligned rows: use 128-bit loads
    int start_base;
};

// Values p[0..7] and p[64..71] of a token row, as 16-bit words (w[i] = values 2i, 2i + 1
// of the 16).  The 8 lanes of a row read dims 8 part .. +7 and 64 + 8 part .. +7, so each
// of the two 16-byte loads of a wave fills whole 128-byte lines (the first or second half
// of 8 rows): 8.17-8.24 vs 8.37-8.41 us on the 8x4096-token K+V pack.  The rows are read
// once: non-temporal loads (8.8 vs 9.0 us).  The words are converted to float by
// row_values, apart from the loads, so that other loads can be issued in between.
__device__ __forceinline__ void load_row_halves(const void* src, int64_t off, int vec_ok, uint32_t (&w)[8]) {
    const uint16_t* p = (const uint16_t*)src + off;
    if (vec_ok) {
        typedef unsigned int nv4 __attribute__((ext_vector_type(4)));
        const nv4 a = __builtin_nontemporal_load((const nv4*)p);
        const nv4 b = __builtin_nontemporal_load((const nv4*)(p + 64));
        w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
        w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int e = 2 * i < 8 ? 2 * i : 56 + 2 * i;
            w[i] = (uint32_t)p[e] | ((uint32_t)p[e + 1] << 16);
        }
    }
}
__device__ __forceinline__ void row_values(const uint32_t (&w)[8], int dtype, float (&vals)[16]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint16_t lo = (uint16_t)(w[i] & 0xffffu), hi = (uint16_t)(w[i] >> 16);
        vals[2 * i] = dtype == HKV_DTYPE_F16 ? h2f(lo) : bf2f(lo);
        vals[2 * i + 1] = dtype == HKV_DTYPE_F16 ? h2f(hi) : bf2f(hi);
    }
}

// Phase 2 of the reference-layout repacker: every lane of the 256 assembles one K word
// and one V word of head h's part of the record from codes staged in LDS; rows outside
// [lo, hi) keep their previous contents.
__device__ __forceinline__ void write_block_words(const uint8_t (&codes)[2][kBlockTokens][kHeadDim],
                                                  int lo, int hi, uint8_t* rec, const RecordLayout& L,
                                                  int h) {
    const int t = threadIdx.x;
    // K word t: token r, dims 8j..8j+7.
    {
        const int r = t >> 4, j = t & 15;
        if (r >= lo && r < hi) {
            uint32_t w = 0;
#pragma unroll
            for (int k = 0; k < 8; ++k) w |= (uint32_t)codes[0][r][8 * j + k] << nib_shift(k);
            *(uint32_t*)(rec + L.kc(h) + r * kCodeRowBytes + j * 4) = w;
        }
    }
    // V word t = (g*16 + c)*4 + m: tokens 4g..4g+3, dims c+32m (x0..x3) and c+32m+16 (x4..x7).
    {
        const int g = t >> 6, c = (t >> 2) & 15, m = t & 3;
        uint32_t w = 0, mask = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int tok = 4 * g + (k & 3);
            const int dim = c + 32 * m + (k >> 2) * 16;
            if (tok >= lo && tok < hi) {
                w |= (uint32_t)codes[1][tok][dim] << nib_shift(k);
                mask |= 0xFu << nib_shift(k);
            }
        }
        if (mask) {
            uint32_t* dst = (uint32_t*)(rec + L.vc(h)) + t;
            if (mask != 0xFFFFFFFFu) w |= (*dst & ~mask);
            *dst = w;
        }
    }
}

// The record part of head h (kHeadPartBytes, 16-byte aligned) is assembled in LDS and
// written with one 16-byte store per lane (138 lanes).  A block the call fills only in
// part first loads the part's current bytes, so rows outside [lo, hi) keep them.
constexpr int kPartVecs = kHeadPartBytes / 16;
static_assert(kHeadPartBytes % 16 == 0 && kPartVecs <= 256, "one 16-byte store per lane");

__global__ __launch_bounds__(256) void pack_tokens_kernel(PackParams p) {
    touch_kernel_args(p);
    const int b = blockIdx.z, h = blockIdx.y;
    // a start passed by value saves the kernel its first memory round trip
    const int start = p.start_pos ? load_uniform_i32(p.start_pos, b) : p.start_base;
    const int lb = start / kBlockTokens + (int)blockIdx.x;
    const int lo = max(start, lb * kBlockTokens) - lb * kBlockTokens;
    const int hi = min(start + p.T, lb * kBlockTokens + kBlockTokens) - lb * kBlockTokens;
    if (lo >= hi) return;

    __shared__ __align__(16) uint8_t codes[kBlockTokens][kHeadDim];   // V codes, one byte each
    __shared__ __align__(16) uint8_t part[kHeadPartBytes];            // the record part being built

    // The block-table read and the block's rows (tokens lo..hi-1 of the input, in bounds
    // whatever the block table holds) are in flight together: the table entry is requested
    // first, so that its check waits for it alone (read unconditionally, at column 0 when lb
    // is outside the row: bt_stride > 0 is checked on the host).
    const bool lb_ok = lb >= 0 && lb < p.bt_stride;
    const int bt_entry = load_uniform_i32(p.bt, (int64_t)b * p.bt_stride + (lb_ok ? lb : 0));
    const int phys = lb_ok ? bt_entry : -1;
    const int t = threadIdx.x;
    const int row = t >> 3;
    const int kv = row >> 4, slot = row & 15, pt = t & 7;
    const bool active = slot >= lo && slot < hi;
    uint32_t raw[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
    if (active) {
        const int tok = lb * kBlockTokens + slot - start;
        const int64_t off = (int64_t)b * p.sb + (int64_t)h * p.sh + (int64_t)tok * p.st + pt * 8;
        load_row_halves(kv ? p.v : p.k, off, p.vec_ok, raw);
    }
    if (!lb_ok || phys < 0 || (int64_t)phys >= p.pool_blocks) {
        if (threadIdx.x == 0 && p.err) atomicOr(p.err, lb_ok ? 1 : 2);
        return;
    }
    const RecordLayout L(p.H);
    uint4* gpart = (uint4*)(p.pool + (int64_t)phys * L.bytes + RecordLayout::part(h));

    const bool whole = lo == 0 && hi == kBlockTokens;
    if (!whole && t < kPartVecs) ((uint4*)part)[t] = gpart[t];   // visible after the barrier below
    float vals[16];
    row_values(raw, p.dtype, vals);
    float mn = INFINITY, mx = -INFINITY;
    if (active) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            mn = __builtin_elementwise_minimum(mn, vals[i]);
            mx = __builtin_elementwise_maximum(mx, vals[i]);
        }
    }
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) {
        mn = __builtin_elementwise_minimum(mn, __shfl_xor(mn, off));
        mx = __builtin_elementwise_maximum(mx, __shfl_xor(mx, off));
    }
    if (!whole) __syncthreads();   // the loaded part is in LDS before rows are written into it
    if (active) {
        const QParams q = qparams_from_minmax(mn, mx);
        float tv[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) tv[i] = quant_unrounded(vals[i], q);
        if (kv == 0) {
            // this lane's 16 K codes are K words pt and 8 + pt of the row: codes 2j and
            // 2j + 1 of a word go to bytes 0 and 2 of x[j], and the word is
            // x0 | x1 << 4 | x2 << 8 | x3 << 12 (nib_shift order)
            uint32_t kw[2];
#pragma unroll
            for (int hw = 0; hw < 2; ++hw) {
                uint32_t x[4];
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    x[j] = code_into(tv[8 * hw + 2 * j + 1], 2u, code_into(tv[8 * hw + 2 * j], 0u, 0u));
                kw[hw] = x[0] | (x[1] << 4) | (x[2] << 8) | (x[3] << 12);
            }
            uint32_t* krow = (uint32_t*)(part + kPartKc + slot * kCodeRowBytes);
            krow[pt] = kw[0];
            krow[8 + pt] = kw[1];
        } else {
            // V words mix four tokens: the codes go through LDS (one byte each), two
            // 8-byte writes
            uint32_t b4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint32_t w = 0u;
#pragma unroll
                for (int e = 0; e < 4; ++e) w = code_into(tv[4 * i + e], (uint32_t)e, w);
                b4[i] = w;
            }
            *(uint2*)&codes[slot][pt * 8] = make_uint2(b4[0], b4[1]);
            *(uint2*)&codes[slot][64 + pt * 8] = make_uint2(b4[2], b4[3]);
        }
        if (pt == 0) {
            *(float*)(part + (kv ? kPartVs : kPartKs) + slot * 4) = q.scale;
            part[(kv ? kPartVz : kPartKz) + slot] = q.zp;
        }
    }
    __syncthreads();
    {
        // V word t = (g*16 + c)*4 + m: tokens 4g..4g+3, dims c+32m (x0..x3) and c+32m+16
        // (x4..x7); rows outside [lo, hi) keep the loaded bits
        const int g = t >> 6, c = (t >> 2) & 15, m = t & 3;
        uint32_t w = 0, mask = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int tok = 4 * g + (k & 3);
            const int dim = c + 32 * m + (k >> 2) * 16;
            if (tok >= lo && tok < hi) {
                w |= (uint32_t)codes[tok][dim] << nib_shift(k);
                mask |= 0xFu << nib_shift(k);
            }
        }
        uint32_t* dst = (uint32_t*)(part + kPartVc) + t;
        if (mask != 0xFFFFFFFFu) w |= (*dst & ~mask);
        *dst = w;
    }
    __syncthreads();
    if (t < kPartVecs) gpart[t] = ((const uint4*)part)[t];
}

// Already-quantized tokens in the reference layout (codes uint8 [.., T, 128] and
// per-token scale/zp) -> block records.  Same placement rules as pack_tokens_kernel.
struct RepackParams {
    const uint8_t* kc;
    const uint8_t* vc;
    int64_t cb, ch, ct;            // code strides (bytes)
    const float* ks;
    const float* vs;
    const void* kz;
    const void* vz;
    int zp_is_float;
    int64_t mb, mh, mt;            // scale / zp strides (elements)
    int H, T;
    const int32_t* start_pos;
    const int32_t* bt;
    int bt_stride;
    uint8_t* pool;
    int64_t pool_blocks;
    int32_t* err;
};

__global__ __launch_bounds__(256) void repack_codes_kernel(RepackParams p) {
    touch_kernel_args(p);
    const int b = blockIdx.z, h = blockIdx.y;
    const int start = p.start_pos[b];
    const int lb = start / kBlockTokens + (int)blockIdx.x;
    const int lo = max(start, lb * kBlockTokens) - lb * kBlockTokens;
    const int hi = min(start + p.T, lb * kBlockTokens + kBlockTokens) - lb * kBlockTokens;
    if (lo >= hi) return;
    if (lb < 0 || lb >= p.bt_stride) {
        if (threadIdx.x == 0 && p.err) atomicOr(p.err, 2);
        return;
    }
    const int phys = p.bt[(int64_t)b * p.bt_stride + lb];
    if (phys < 0 || (int64_t)phys >= p.pool_blocks) {
        if (threadIdx.x == 0 && p.err) atomicOr(p.err, 1);
        return;
    }
    const RecordLayout L(p.H);
    uint8_t* rec = p.pool + (int64_t)phys * L.bytes;
    __shared__ uint8_t codes[2][kBlockTokens][kHeadDim];
    const int t = threadIdx.x;
    const int row = t >> 3;
    const int kv = row >> 4, slot = row & 15, part = t & 7;
    if (slot >= lo && slot < hi) {
        const int tok = lb * kBlockTokens + slot - start;
        const uint8_t* src = (kv ? p.vc : p.kc) + (int64_t)b * p.cb + (int64_t)h * p.ch + (int64_t)tok * p.ct + part * 16;
#pragma unroll
        for (int i = 0; i < 16; ++i) codes[kv][slot][part * 16 + i] = src[i] & 0xF;
        if (part == 0) {
            const int64_t mi = (int64_t)b * p.mb + (int64_t)h * p.mh + (int64_t)tok * p.mt;
            const float sc = (kv ? p.vs : p.ks)[mi];
            const void* zsrc = kv ? p.vz : p.kz;
            const uint8_t zp = p.zp_is_float ? (uint8_t)((const float*)zsrc)[mi] : ((const uint8_t*)zsrc)[mi];
            ((float*)(rec + (kv ? L.vs(h) : L.ks(h))))[slot] = sc;
            (rec + (kv ? L.vz(h) : L.kz(h)))[slot] = zp;
        }
    }
    __syncthreads();
    write_block_words(codes, lo, hi, rec, L, h);
}

// Pool -> reference layout.  Thread (token, j) of head blockIdx.y writes the eight
// codes of dims 8j..8j+7 (one 8-byte store); lane j == 0 also writes the token's
// scale and zero point.
__global__ __launch_bounds__(256) void unpack_tokens_kernel(
    const uint8_t* __restrict__ pool, int64_t pool_blocks, const int32_t* __restrict__ bt, int H,
    int T, int which, uint8_t* __restrict__ codes, float* __restrict__ scales,
    uint8_t* __restrict__ zps) {
    const int h = blockIdx.y;
    const int u = blockIdx.x * blockDim.x + threadIdx.x;
    const int tok = u >> 4, j = u & 15;
    if (tok >= T) return;
    const int phys = bt[tok / kBlockTokens];
    if (phys < 0 || (int64_t)phys >= pool_blocks) return;
    const RecordLayout L(H);
    const uint8_t* rec = pool + (int64_t)phys * L.bytes;
    const int s = tok % kBlockTokens;
    uint32_t lo = 0, hi = 0;   // codes of dims 8j..8j+3 and 8j+4..8j+7, one per byte
    if (which == 0) {
        const uint32_t w = *(const uint32_t*)(rec + L.kc(h) + s * kCodeRowBytes + j * 4);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t code = (w >> nib_shift(e)) & 0xFu;
            if (e < 4) lo |= code << (8 * e);
            else hi |= code << (8 * (e - 4));
        }
    } else {
        // dim d = c + 16 n: word (g * 16 + c) * 4 + n / 2, nibble (s % 4) + 4 (n % 2)
        const int g = s >> 2, ii = s & 3;
        const uint32_t* vw = (const uint32_t*)(rec + L.vc(h));
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int d = 8 * j + e, c = d & 15, n = d >> 4;
            const uint32_t w = vw[(g * 16 + c) * 4 + (n >> 1)];
            const uint32_t code = (w >> nib_shift(ii + (n & 1) * 4)) & 0xFu;
            if (e < 4) lo |= code << (8 * e);
            else hi |= code << (8 * (e - 4));
        }
    }
    const int64_t row = (int64_t)h * T + tok;
    if (codes) *(uint2*)(codes + row * kHeadDim + 8 * j) = make_uint2(lo, hi);
    if (j == 0) {
        if (scales) scales[row] = ((const float*)(rec + (which ? L.vs(h) : L.ks(h))))[s];
        if (zps) zps[row] = (rec + (which ? L.vz(h) : L.kz(h)))[s];
    }
}

// The same for group sizes and lengths that are multiples of 8 with 8-byte aligned
// codes and 16-byte aligned output: thread t converts codes 8t..8t+7 (one group),
// one 8-byte load and one or two 16-byte stores.
__global__ __launch_bounds__(256) void dequantize_groups8_kernel(
    const uint8_t* __restrict__ codes, const float* __restrict__ scales,
    const uint8_t* __restrict__ zps, int64_t n8, int G8, void* __restrict__ out, int out_dtype) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < n8; t += stride) {
        const int64_t g = n8 <= 0x7fffffff ? (int64_t)((uint32_t)t / (uint32_t)G8) : t / G8;
        const float zp = (float)zps[g], sc = scales[g];
        const uint2 w = *(const uint2*)(codes + 8 * t);
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = ((float)(((e < 4 ? w.x : w.y) >> (8 * (e & 3))) & 0xffu) - zp) * sc;
        if (out_dtype == HKV_DTYPE_F32) {
            float4* o = (float4*)out + 2 * t;
            o[0] = make_float4(v[0], v[1], v[2], v[3]);
            o[1] = make_float4(v[4], v[5], v[6], v[7]);
        } else {
            uint32_t h[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t a = out_dtype == HKV_DTYPE_F16 ? f2h_rn(v[2 * e]) : f2bf_rn(v[2 * e]);
                const uint32_t b = out_dtype == HKV_DTYPE_F16 ? f2h_rn(v[2 * e + 1]) : f2bf_rn(v[2 * e + 1]);
                h[e] = a | (b << 16);
            }
            ((uint4*)out)[t] = make_uint4(h[0], h[1], h[2], h[3]);
        }
    }
}

int grid_for(int64_t work, int per_block) {
    int64_t g = (work + per_block - 1) / per_block;
    if (g < 1) g = 1;
    if (g > 65536) g = 65536;
    return (int)g;
}

}  // namespace
}  // namespace hkv

using namespace hkv;

extern "C" int hkv_quantize_groups(const void* x, int32_t dtype, int64_t n, int32_t group_size,
                                   uint8_t* codes, float* scales, uint8_t* zps, void* stream) {
    clear_error();
    HKV_REQUIRE(n >= 0, HKV_ERR_ARG, "hkv_quantize_groups: n < 0");
    HKV_REQUIRE(group_size > 0, HKV_ERR_ARG, "hkv_quantize_groups: group_size must be > 0");
    HKV_REQUIRE(dtype == HKV_DTYPE_F16 || dtype == HKV_DTYPE_BF16 || dtype == HKV_DTYPE_F32,
                HKV_ERR_ARG, "hkv_quantize_groups: unsupported dtype %d", dtype);
    if (n == 0) return HKV_OK;
    HKV_REQUIRE(x && codes && scales && zps, HKV_ERR_ARG, "hkv_quantize_groups: null pointer");
    const int64_t ngroups = (n + group_size - 1) / group_size;
    const int blocks = grid_for(ngroups, 4);
    hipLaunchKernelGGL(quantize_groups_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, x,
                       dtype, n, group_size, ngroups, codes, scales, zps);
    HKV_LAUNCH_CHECK("quantize_groups_kernel");
    return HKV_OK;
}

extern "C" int hkv_dequantize_groups(const uint8_t* codes, const float* scales, const uint8_t* zps,
                                     int64_t n, int32_t group_size, void* out, int32_t out_dtype,
                                     void* stream) {
    clear_error();
    HKV_REQUIRE(n >= 0, HKV_ERR_ARG, "hkv_dequantize_groups: n < 0");
    HKV_REQUIRE(group_size > 0, HKV_ERR_ARG, "hkv_dequantize_groups: group_size must be > 0");
    HKV_REQUIRE(out_dtype == HKV_DTYPE_F16 || out_dtype == HKV_DTYPE_BF16 || out_dtype == HKV_DTYPE_F32,
                HKV_ERR_ARG, "hkv_dequantize_groups: unsupported dtype %d", out_dtype);
    if (n == 0) return HKV_OK;
    HKV_REQUIRE(codes && scales && zps && out, HKV_ERR_ARG, "hkv_dequantize_groups: null pointer");
    if (group_size % 8 == 0 && n % 8 == 0 && ((uintptr_t)codes & 7) == 0 && ((uintptr_t)out & 15) == 0) {
        const int64_t n8 = n / 8;
        hipLaunchKernelGGL(dequantize_groups8_kernel, dim3(grid_for(n8, 256)), dim3(256), 0, (hipStream_t)stream,
                           codes, scales, zps, n8, group_size / 8, out, out_dtype);
        HKV_LAUNCH_CHECK("dequantize_groups8_kernel");
        return HKV_OK;
    }
    const int64_t ngroups = (n + group_size - 1) / group_size;
    const int blocks = grid_for(ngroups, 4);
    hipLaunchKernelGGL(dequantize_groups_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                       codes, scales, zps, n, group_size, ngroups, out, out_dtype);
    HKV_LAUNCH_CHECK("dequantize_groups_kernel");
    return HKV_OK;
}

extern "C" int hkv_pack_tokens(const HkvPackArgs* a, void* stream) {
    clear_error();
    HKV_REQUIRE(a != nullptr, HKV_ERR_ARG, "hkv_pack_tokens: null args");
    HKV_REQUIRE(a->head_dim == kHeadDim, HKV_ERR_UNSUPPORTED, "hkv_pack_tokens: head_dim %d != 128",
                a->head_dim);
    HKV_REQUIRE(a->dtype == HKV_DTYPE_F16 || a->dtype == HKV_DTYPE_BF16, HKV_ERR_ARG,
                "hkv_pack_tokens: dtype must be F16 or BF16");
    HKV_REQUIRE(a->batch >= 0 && a->num_kv_heads > 0 && a->num_tokens >= 0, HKV_ERR_ARG,
                "hkv_pack_tokens: bad batch/heads/tokens");
    if (a->batch == 0 || a->num_tokens == 0) return HKV_OK;
    HKV_REQUIRE(a->k && a->v && a->block_table && a->pool, HKV_ERR_ARG, "hkv_pack_tokens: null pointer");
    HKV_REQUIRE(a->pool_blocks > 0 && a->bt_stride > 0, HKV_ERR_ARG, "hkv_pack_tokens: empty pool/table");
    HKV_REQUIRE(a->batch <= 65535 && a->num_kv_heads <= 65535, HKV_ERR_ARG, "hkv_pack_tokens: grid too large");
    PackParams p;
    p.k = a->k;
    p.v = a->v;
    p.dtype = a->dtype;
    p.sb = a->src_stride_b;
    p.sh = a->src_stride_h;
    p.st = a->src_stride_t;
    p.H = a->num_kv_heads;
    p.T = a->num_tokens;
    p.start_pos = a->start_pos;
    p.start_base = a->start_base;
    p.bt = a->block_table;
    p.bt_stride = a->bt_stride;
    p.pool = a->pool;
    p.pool_blocks = a->pool_blocks;
    p.err = a->err_flag;
    const bool aligned = (((uintptr_t)a->k | (uintptr_t)a->v) & 15) == 0 &&
                         ((a->src_stride_b | a->src_stride_h | a->src_stride_t) & 7) == 0;
    p.vec_ok = aligned ? 1 : 0;
    // A run of T tokens starting anywhere touches at most ceil(T/16)+1 blocks.
    const int nblk = (a->num_tokens + kBlockTokens - 1) / kBlockTokens + 1;
    hipLaunchKernelGGL(pack_tokens_kernel, dim3(nblk, a->num_kv_heads, a->batch), dim3(256), 0,
                       (hipStream_t)stream, p);
    HKV_LAUNCH_CHECK("pack_tokens_kernel");
    return HKV_OK;
}

extern "C" int hkv_unpack_tokens(const uint8_t* pool, int64_t pool_blocks, const int32_t* block_table,
                                 int32_t num_kv_heads, int32_t head_dim, int32_t num_tokens,
                                 int32_t which, uint8_t* codes, float* scales, uint8_t* zps,
                                 void* stream) {
    clear_error();
    HKV_REQUIRE(head_dim == kHeadDim, HKV_ERR_UNSUPPORTED, "hkv_unpack_tokens: head_dim %d != 128", head_dim);
    HKV_REQUIRE(which == 0 || which == 1, HKV_ERR_ARG, "hkv_unpack_tokens: which must be 0 (K) or 1 (V)");
    HKV_REQUIRE(num_kv_heads > 0 && num_tokens >= 0, HKV_ERR_ARG, "hkv_unpack_tokens: bad sizes");
    if (num_tokens == 0) return HKV_OK;
    HKV_REQUIRE(pool && block_table && pool_blocks > 0, HKV_ERR_ARG, "hkv_unpack_tokens: null pool/table");
    HKV_REQUIRE(num_kv_heads <= 65535 && num_tokens <= (1 << 26), HKV_ERR_ARG, "hkv_unpack_tokens: grid too large");
    HKV_REQUIRE(codes == nullptr || ((uintptr_t)codes & 7) == 0, HKV_ERR_ARG,
                "hkv_unpack_tokens: codes must be 8-byte aligned");
    const int64_t threads = (int64_t)num_tokens * 16;
    hipLaunchKernelGGL(unpack_tokens_kernel, dim3((unsigned)((threads + 255) / 256), num_kv_heads), dim3(256), 0,
                       (hipStream_t)stream, pool, pool_blocks, block_table, num_kv_heads, num_tokens,
                       which, codes, scales, zps);
    HKV_LAUNCH_CHECK("unpack_tokens_kernel");
    return HKV_OK;
}

extern "C" int hkv_repack_codes(const HkvRepackArgs* a, void* stream) {
    clear_error();
    HKV_REQUIRE(a != nullptr, HKV_ERR_ARG, "hkv_repack_codes: null args");
    HKV_REQUIRE(a->head_dim == kHeadDim, HKV_ERR_UNSUPPORTED, "hkv_repack_codes: head_dim %d != 128",
                a->head_dim);
    HKV_REQUIRE(a->zp_dtype == HKV_DTYPE_U8 || a->zp_dtype == HKV_DTYPE_F32, HKV_ERR_ARG,
                "hkv_repack_codes: zp dtype must be U8 or F32");
    HKV_REQUIRE(a->batch >= 0 && a->num_kv_heads > 0 && a->num_tokens >= 0, HKV_ERR_ARG,
                "hkv_repack_codes: bad batch/heads/tokens");
    if (a->batch == 0 || a->num_tokens == 0) return HKV_OK;
    HKV_REQUIRE(a->k_codes && a->v_codes && a->k_scales && a->v_scales && a->k_zps && a->v_zps &&
                    a->start_pos && a->block_table && a->pool,
                HKV_ERR_ARG, "hkv_repack_codes: null pointer");
    HKV_REQUIRE(a->pool_blocks > 0 && a->bt_stride > 0, HKV_ERR_ARG, "hkv_repack_codes: empty pool/table");
    HKV_REQUIRE(a->batch <= 65535 && a->num_kv_heads <= 65535, HKV_ERR_ARG, "hkv_repack_codes: grid too large");
    RepackParams p;
    p.kc = a->k_codes;
    p.vc = a->v_codes;
    p.cb = a->code_stride_b;
    p.ch = a->code_stride_h;
    p.ct = a->code_stride_t;
    p.ks = a->k_scales;
    p.vs = a->v_scales;
    p.kz = a->k_zps;
    p.vz = a->v_zps;
    p.zp_is_float = a->zp_dtype == HKV_DTYPE_F32 ? 1 : 0;
    p.mb = a->meta_stride_b;
    p.mh = a->meta_stride_h;
    p.mt = a->meta_stride_t;
    p.H = a->num_kv_heads;
    p.T = a->num_tokens;
    p.start_pos = a->start_pos;
    p.bt = a->block_table;
    p.bt_stride = a->bt_stride;
    p.pool = a->pool;
    p.pool_blocks = a->pool_blocks;
    p.err = a->err_flag;
    const int nblk = (a->num_tokens + kBlockTokens - 1) / kBlockTokens + 1;
    hipLaunchKernelGGL(repack_codes_kernel, dim3(nblk, a->num_kv_heads, a->batch), dim3(256), 0,
                       (hipStream_t)stream, p);
    HKV_LAUNCH_CHECK("repack_codes_kernel");
    return HKV_OK;
}
