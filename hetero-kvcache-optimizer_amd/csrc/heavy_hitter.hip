// Heavy-hitter scoring: attention weights of the newest token from the decode
// kernel's scores, per-block mean scores, and the eviction candidates (the lowest
// block means outside the protected sink and local windows).
//
// Reference: HeavyHitterOracle.update / get_eviction_candidates
// (src/policy/heavy_hitter.py:26-101), compute_block_scores / _block_mean_kernel
// (src/kernels/oracle_triton.py:16-79), and the weights the reference's attention
// patch would hand to the oracle: softmax weights of the last query row averaged over
// heads (src/core/fused_attention_patch.py:104-107).
#include "hkv_internal.h"

#include <math.h>

namespace hkv {
namespace {

constexpr int kSortThreads = 1024;
constexpr int kSortMax = 16384;          // keys one workgroup sorts in LDS (128 KB)

// ---- attention weights: out[b][t] (+)= mean_h exp2(s[b][h][order(t)] - M) / L
struct WeightsParams {
    const float* scores;
    int64_t sb, sh;
    const float* stats;
    int B, H;
    int64_t n;
    const int64_t* order;
    float* out;
    int64_t ob;
    int accumulate;
};

constexpr int kMaxWeightHeads = 256;

__global__ __launch_bounds__(256) void attn_weights_kernel(WeightsParams p) {
    touch_kernel_args(p);
    // each row's max and 1 / sum, once per workgroup
    __shared__ float sm_m[kMaxWeightHeads], sm_inv[kMaxWeightHeads];
    const int b = blockIdx.y;
    for (int h = threadIdx.x; h < p.H; h += 256) {
        const float* st = p.stats + ((int64_t)b * p.H + h) * 2;
        const float L = st[1];
        sm_m[h] = st[0];
        sm_inv[h] = L > 0.f ? 1.0f / L : 0.f;
    }
    __syncthreads();
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= p.n) return;
    const int64_t item = p.order ? p.order[t] : t;
    float w = 0.f;
    if (item >= 0) {
        const float* s = p.scores + (int64_t)b * p.sb + item;
#pragma unroll 8
        for (int h = 0; h < p.H; ++h) {
            const float x = s[(int64_t)h * p.sh];
            // exp2(-inf) = 0: masked items add nothing
            w += __builtin_amdgcn_exp2f(x - sm_m[h]) * sm_inv[h];
        }
        w *= 1.0f / (float)p.H;
    }
    float* o = p.out + (int64_t)b * p.ob + t;
    *o = p.accumulate ? *o + w : w;
}

// ---- block means: the tokens of each block summed in order, then divided by
// their count (exact IEEE fp32 division)
__device__ __forceinline__ float block_mean(const float* ts, int64_t seq_len, int bs, int64_t blk) {
    const int64_t t0 = blk * bs;
    const int64_t t1 = t0 + bs < seq_len ? t0 + bs : seq_len;
    float acc = 0.f;
    for (int64_t t = t0; t < t1; ++t) acc += ts[t];
    const int64_t cnt = t1 - t0;
    return acc / (float)(cnt > 0 ? cnt : 1);
}

__global__ __launch_bounds__(256) void block_mean_kernel(const float* __restrict__ ts, int64_t seq_len, int bs,
                                                         int64_t nblocks, float* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < nblocks) out[i] = block_mean(ts, seq_len, bs, i);
}

// Sort key of a block: the mean's bits made order-preserving as unsigned, then the
// block index, so equal means keep index order.  Protected blocks get +inf.
__device__ __forceinline__ uint64_t sort_key(float v, uint32_t idx) {
    uint32_t u = __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)u << 32) | idx;
}

__global__ __launch_bounds__(256) void block_keys_kernel(const float* __restrict__ ts, int64_t seq_len, int bs,
                                                         int64_t nblocks, int64_t prot_lo, int64_t prot_hi,
                                                         uint64_t* __restrict__ keys) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= nblocks) return;
    const bool prot = i < prot_lo || i >= prot_hi;
    keys[i] = sort_key(prot ? INFINITY : block_mean(ts, seq_len, bs, i), (uint32_t)i);
}

// One workgroup sorts keys [c * chunk, min(n, (c + 1) * chunk)) ascending in LDS
// (bitonic, padded to a power of two with the largest key) and writes the first
// `take`: block indices to out_idx (final pass) or keys to out_keys.
__global__ __launch_bounds__(kSortThreads) void sort_take_kernel(const uint64_t* __restrict__ keys, int64_t n,
                                                                 int chunk, int pow2, int take,
                                                                 uint64_t* __restrict__ out_keys,
                                                                 int64_t* __restrict__ out_idx) {
    extern __shared__ uint64_t sk[];
    const int64_t base = (int64_t)blockIdx.x * chunk;
    const int64_t cnt = n - base < chunk ? n - base : chunk;
    for (int i = threadIdx.x; i < pow2; i += kSortThreads) sk[i] = i < cnt ? keys[base + i] : ~0ull;
    __syncthreads();
    for (int size = 2; size <= pow2; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < pow2; i += kSortThreads) {
                const int j = i ^ stride;
                if (j > i) {
                    const uint64_t a = sk[i], c = sk[j];
                    const bool up = (i & size) == 0;
                    if ((a > c) == up) {
                        sk[i] = c;
                        sk[j] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
    const int m = take < cnt ? take : (int)cnt;
    for (int i = threadIdx.x; i < take; i += kSortThreads) {
        const uint64_t key = i < m ? sk[i] : ~0ull;
        if (out_idx)
            out_idx[i] = (int64_t)(uint32_t)key;
        else
            out_keys[(int64_t)blockIdx.x * take + i] = key;
    }
}

int pow2_at_least(int64_t x) {
    int p = 64;
    while (p < x) p <<= 1;
    return p;
}

// Candidate count and protected range, as get_eviction_candidates decides them, and
// the sort layout: chunks of `chunk` keys sorted by one workgroup each; with more than
// one chunk, each keeps its first k keys and one more workgroup sorts those.
struct EvictPlan {
    int64_t nblocks, prot_lo, prot_hi;
    int k;
    int chunk;
    int64_t nchunks;
};

EvictPlan plan_eviction(int64_t seq_len, int bs, int sink, int local, int k) {
    EvictPlan e{0, 0, 0, 0};
    if (seq_len <= (int64_t)sink + local) return e;
    e.nblocks = (seq_len + bs - 1) / bs;
    const int64_t sb = ((int64_t)sink + bs - 1) / bs, lb = ((int64_t)local + bs - 1) / bs;
    e.prot_lo = sb;
    e.prot_hi = e.nblocks - lb > 0 ? e.nblocks - lb : 0;
    const int64_t unsafe = e.nblocks - sb - lb > 0 ? e.nblocks - sb - lb : 0;
    e.k = (int)(k < unsafe ? k : unsafe);
    // small chunks sort in parallel; a chunk holds at least 8k keys so that the merge
    // pass stays small
    int c = 512;
    while (c < kSortMax && c < 8ll * e.k) c <<= 1;
    while (c < kSortMax && ((e.nblocks + c - 1) / c) * (int64_t)e.k > kSortMax) c <<= 1;
    e.chunk = c;
    e.nchunks = e.k > 0 ? (e.nblocks + c - 1) / c : 0;
    return e;
}

size_t evict_workspace(const EvictPlan& e) {
    if (e.k <= 0) return 0;
    return (size_t)e.nblocks * 8 + (e.nchunks > 1 ? (size_t)e.nchunks * e.k * 8 : 0);
}

std::atomic<uint64_t> sort_lds_raised{0};

}  // namespace
}  // namespace hkv

using namespace hkv;

extern "C" int hkv_attn_weights(const float* scores, int64_t scores_stride_b, int64_t scores_stride_h,
                                const float* score_stats, int32_t batch, int32_t num_heads, int64_t n_items,
                                const int64_t* order, float* out, int64_t out_stride_b, int32_t accumulate,
                                void* stream) {
    clear_error();
    HKV_REQUIRE(batch > 0 && num_heads > 0 && n_items >= 0, HKV_ERR_ARG, "hkv_attn_weights: bad sizes");
    if (n_items == 0) return HKV_OK;
    HKV_REQUIRE(scores && score_stats && out, HKV_ERR_ARG, "hkv_attn_weights: null pointer");
    HKV_REQUIRE(out_stride_b >= n_items, HKV_ERR_ARG, "hkv_attn_weights: out stride %lld < %lld items",
                (long long)out_stride_b, (long long)n_items);
    HKV_REQUIRE(batch < 65536, HKV_ERR_ARG, "hkv_attn_weights: batch too large");
    HKV_REQUIRE(num_heads <= kMaxWeightHeads, HKV_ERR_UNSUPPORTED, "hkv_attn_weights: more than %d heads",
                kMaxWeightHeads);
    WeightsParams p{scores, scores_stride_b, scores_stride_h, score_stats, batch, num_heads, n_items,
                    order, out, out_stride_b, accumulate ? 1 : 0};
    hipLaunchKernelGGL(attn_weights_kernel, dim3((unsigned)((n_items + 255) / 256), (unsigned)batch), dim3(256), 0,
                       (hipStream_t)stream, p);
    HKV_LAUNCH_CHECK("attn_weights_kernel");
    return HKV_OK;
}

extern "C" int hkv_block_scores(const float* token_scores, int64_t seq_len, int32_t block_size, float* out,
                                void* stream) {
    clear_error();
    HKV_REQUIRE(seq_len >= 0 && block_size > 0, HKV_ERR_ARG, "hkv_block_scores: bad sizes");
    if (seq_len == 0) return HKV_OK;
    HKV_REQUIRE(token_scores && out, HKV_ERR_ARG, "hkv_block_scores: null pointer");
    const int64_t nb = (seq_len + block_size - 1) / block_size;
    hipLaunchKernelGGL(block_mean_kernel, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       token_scores, seq_len, (int)block_size, nb, out);
    HKV_LAUNCH_CHECK("block_mean_kernel");
    return HKV_OK;
}

extern "C" size_t hkv_eviction_workspace_bytes(int64_t seq_len, int32_t block_size, int32_t sink_tokens,
                                               int32_t local_window, int32_t max_blocks) {
    if (seq_len < 0 || block_size <= 0 || sink_tokens < 0 || local_window < 0 || max_blocks < 0) return 0;
    return evict_workspace(plan_eviction(seq_len, block_size, sink_tokens, local_window, max_blocks));
}

extern "C" int hkv_eviction_candidates(const float* token_scores, int64_t seq_len, int32_t block_size,
                                       int32_t sink_tokens, int32_t local_window, int32_t max_blocks,
                                       int64_t* out, int32_t* num_out, void* workspace, size_t workspace_bytes,
                                       void* stream) {
    clear_error();
    HKV_REQUIRE(seq_len >= 0 && block_size > 0 && sink_tokens >= 0 && local_window >= 0 && max_blocks >= 0,
                HKV_ERR_ARG, "hkv_eviction_candidates: bad sizes");
    HKV_REQUIRE(num_out != nullptr, HKV_ERR_ARG, "hkv_eviction_candidates: null num_out");
    const EvictPlan e = plan_eviction(seq_len, block_size, sink_tokens, local_window, max_blocks);
    *num_out = e.k;
    if (e.k <= 0) return HKV_OK;
    HKV_REQUIRE(token_scores && out, HKV_ERR_ARG, "hkv_eviction_candidates: null pointer");
    HKV_REQUIRE(workspace && workspace_bytes >= evict_workspace(e) && (((uintptr_t)workspace) & 7) == 0,
                HKV_ERR_CAPACITY, "hkv_eviction_candidates: workspace %zu bytes, need %zu (8-byte aligned)",
                workspace_bytes, evict_workspace(e));
    HKV_REQUIRE(e.nblocks < (1ll << 32), HKV_ERR_UNSUPPORTED, "hkv_eviction_candidates: too many blocks");
    const int64_t nchunks = e.nchunks;
    HKV_REQUIRE(nchunks == 1 || nchunks * e.k <= kSortMax, HKV_ERR_UNSUPPORTED,
                "hkv_eviction_candidates: %lld blocks with %d candidates exceed one merge pass",
                (long long)e.nblocks, e.k);
    HKV_RAISE_LDS(sort_take_kernel, kSortMax * 8, sort_lds_raised);
    uint64_t* keys = (uint64_t*)workspace;
    hipLaunchKernelGGL(block_keys_kernel, dim3((unsigned)((e.nblocks + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, token_scores, seq_len, (int)block_size, e.nblocks, e.prot_lo, e.prot_hi,
                       keys);
    HKV_LAUNCH_CHECK("block_keys_kernel");
    if (nchunks == 1) {
        const int pw = pow2_at_least(e.nblocks);
        hipLaunchKernelGGL(sort_take_kernel, dim3(1), dim3(kSortThreads), (size_t)pw * 8, (hipStream_t)stream, keys,
                           e.nblocks, e.chunk, pw, e.k, (uint64_t*)nullptr, out);
        HKV_LAUNCH_CHECK("sort_take_kernel");
        return HKV_OK;
    }
    uint64_t* cand = keys + e.nblocks;
    hipLaunchKernelGGL(sort_take_kernel, dim3((unsigned)nchunks), dim3(kSortThreads), (size_t)e.chunk * 8,
                       (hipStream_t)stream, keys, e.nblocks, e.chunk, e.chunk, e.k, cand, (int64_t*)nullptr);
    HKV_LAUNCH_CHECK("sort_take_kernel");
    const int64_t nc = nchunks * e.k;
    const int pw = pow2_at_least(nc);
    hipLaunchKernelGGL(sort_take_kernel, dim3(1), dim3(kSortThreads), (size_t)pw * 8, (hipStream_t)stream, cand, nc,
                       kSortMax, pw, e.k, (uint64_t*)nullptr, out);
    HKV_LAUNCH_CHECK("sort_take_kernel");
    return HKV_OK;
}
