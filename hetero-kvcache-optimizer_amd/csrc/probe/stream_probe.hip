// Streaming-read probes: how fast one launch of a given shape can read a buffer of
// the decode's size from HBM, with no compute.  They bound what a single-pass
// reader such as the split-K decode kernel can reach at that size and shape.
//
//   contiguous: workgroup w reads bytes [w * chunk, (w + 1) * chunk); each wave
//               load is 64 lanes x 16 bytes = one 1 KB run, and wave j of a
//               workgroup takes runs j, j + waves, ...
//   parts:      the INT4 pool's access pattern: records of `heads` parts of
//               `part_bytes` each; workgroup (range s, head h) = id s * heads + h
//               reads part h of the records of range s (records split evenly over
//               grid / heads ranges), one part per wave step (three loads).
//
// Each wave keeps `depth` units in flight as a ring: it folds the oldest unit into
// an XOR accumulator and issues the next load into its slot.  Loads past a
// workgroup's share go through a zero-sized buffer resource and return zeros
// without a memory access.  The accumulator is stored only if it equals a value the
// host passes and never produces (the loads cannot be optimised away).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u4 ld16(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

template <int kW, int kD>
__global__ __launch_bounds__(kW * 64) void probe_contig_kernel(const uint8_t* src, int64_t chunk, int64_t total,
                                                               uint32_t magic, uint32_t* sink) {
    const int64_t base = (int64_t)blockIdx.x * chunk;
    const int64_t n = base < total ? (total - base < chunk ? total - base : chunk) : 0;
    const __amdgpu_buffer_rsrc_t r = rsrc(src + (n > 0 ? base : 0), n);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int units = (int)((n + 1023) >> 10);
    u4 buf[kD];
    u4 acc = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int d = 0; d < kD; ++d) {
        buf[d] = ld16(r, ((wave + d * kW) << 10) + lane * 16);
        __builtin_amdgcn_sched_barrier(0);
    }
    for (int u0 = wave; u0 < units; u0 += kD * kW) {
#pragma unroll
        for (int d = 0; d < kD; ++d) {
            acc ^= buf[d];
            buf[d] = ld16(r, ((u0 + (d + kD) * kW) << 10) + lane * 16);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int d = 0; d < kD; ++d) acc ^= buf[d];
    if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == magic) sink[(int64_t)blockIdx.x * kW * 64 + threadIdx.x] = 1u;
}

struct Part {
    u4 a, b, c;
};

__device__ __forceinline__ void load_part(const uint8_t* src, int64_t rec, int64_t nrec, int heads, int h,
                                          int part_bytes, int lane, Part& d) {
    const bool valid = rec < nrec;
    const __amdgpu_buffer_rsrc_t r = rsrc(src + (valid ? (rec * heads + h) * part_bytes : 0), valid ? part_bytes : 0);
    d.a = ld16(r, lane * 16);
    d.b = ld16(r, 1024 + lane * 16);
    d.c = ld16(r, 2048 + lane * 16);
}

template <int kW, int kD>
__global__ __launch_bounds__(kW * 64) void probe_parts_kernel(const uint8_t* src, int64_t nrec, int heads,
                                                              int part_bytes, int nsplit, uint32_t magic,
                                                              uint32_t* sink) {
    const int h = blockIdx.x % heads, split = blockIdx.x / heads;
    const int64_t r0 = nrec * split / nsplit, r1 = nrec * (split + 1) / nsplit;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    Part buf[kD];
    u4 acc = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int d = 0; d < kD; ++d) {
        load_part(src, r0 + wave + d * kW, r1, heads, h, part_bytes, lane, buf[d]);
        __builtin_amdgcn_sched_barrier(0);
    }
    for (int64_t u0 = r0 + wave; u0 < r1; u0 += kD * kW) {
#pragma unroll
        for (int d = 0; d < kD; ++d) {
            acc ^= buf[d].a ^ buf[d].b ^ buf[d].c;
            load_part(src, u0 + (d + kD) * kW, r1, heads, h, part_bytes, lane, buf[d]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int d = 0; d < kD; ++d) acc ^= buf[d].a ^ buf[d].b ^ buf[d].c;
    if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == magic) sink[(int64_t)blockIdx.x * kW * 64 + threadIdx.x] = 1u;
}

template <int kW, int kD>
hipError_t launch(int pattern, const uint8_t* src, int64_t bytes, int grid, int heads, int part_bytes,
                  uint32_t magic, uint32_t* sink, hipStream_t st) {
    if (pattern == 0) {
        const int64_t chunk = ((bytes + grid - 1) / grid + 1023) & ~(int64_t)1023;
        hipLaunchKernelGGL((probe_contig_kernel<kW, kD>), dim3(grid), dim3(kW * 64), 0, st, src, chunk, bytes, magic,
                           sink);
    } else {
        const int64_t nrec = bytes / ((int64_t)heads * part_bytes);
        hipLaunchKernelGGL((probe_parts_kernel<kW, kD>), dim3(grid), dim3(kW * 64), 0, st, src, nrec, heads,
                           part_bytes, grid / heads, magic, sink);
    }
    return hipGetLastError();
}

template <int kW>
hipError_t launch_d(int depth, int pattern, const uint8_t* src, int64_t bytes, int grid, int heads, int part_bytes,
                    uint32_t magic, uint32_t* sink, hipStream_t st) {
    switch (depth) {
        case 1: return launch<kW, 1>(pattern, src, bytes, grid, heads, part_bytes, magic, sink, st);
        case 2: return launch<kW, 2>(pattern, src, bytes, grid, heads, part_bytes, magic, sink, st);
        case 4: return launch<kW, 4>(pattern, src, bytes, grid, heads, part_bytes, magic, sink, st);
        default: return launch<kW, 8>(pattern, src, bytes, grid, heads, part_bytes, magic, sink, st);
    }
}

}  // namespace

// Returns 0, -1 for arguments outside the probe's limits, or -2 for a launch error.
// pattern 0 = contiguous, 1 = head parts; waves per workgroup 4, 8 or 16; depth
// 1, 2, 4 or 8 units in flight per wave; `sink` holds grid x waves x 64 words.
extern "C" int hkv_probe_stream(const void* src, int64_t bytes, int32_t pattern, int32_t grid, int32_t waves,
                                int32_t depth, int32_t heads, int32_t part_bytes, uint32_t magic, uint32_t* sink,
                                void* stream) {
    if (!src || !sink || bytes <= 0 || grid <= 0 || grid > (1 << 20)) return -1;
    if (waves != 4 && waves != 8 && waves != 16) return -1;
    if (depth != 1 && depth != 2 && depth != 4 && depth != 8) return -1;
    if (pattern == 0) {
        if ((bytes + grid - 1) / grid >= (int64_t)1 << 30) return -1;   // per-workgroup offsets stay in 31 bits
    } else if (pattern == 1) {
        if (heads <= 0 || grid % heads != 0 || part_bytes <= 0 || part_bytes > 3072) return -1;
        if (bytes < (int64_t)heads * part_bytes) return -1;
    } else {
        return -1;
    }
    const uint8_t* s = (const uint8_t*)src;
    hipStream_t st = (hipStream_t)stream;
    hipError_t e;
    switch (waves) {
        case 4: e = launch_d<4>(depth, pattern, s, bytes, grid, heads, part_bytes, magic, sink, st); break;
        case 8: e = launch_d<8>(depth, pattern, s, bytes, grid, heads, part_bytes, magic, sink, st); break;
        default: e = launch_d<16>(depth, pattern, s, bytes, grid, heads, part_bytes, magic, sink, st); break;
    }
    return e == hipSuccess ? 0 : -2;
}
