// Host-tier prefetcher: a pinned host arena holding offloaded INT4 block records and
// a side stream that copies them into HBM staging buffers ahead of the layer that
// attends them (the reference's DRAMStorageManager + AsyncPrefetcher,
// dram_storage.py:20-222 and prefetcher.py:21-123, without per-tensor pin_memory
// calls or a dequantize on the side stream: records stay INT4 end to end).
//
// Protocol (one prefetcher per device, used from one host thread):
//   hkv_pf_create                 pinned arena (hipHostMalloc) + side stream (default
//                                 priority) + three events per slot
//   hkv_pf_host_ptr               where the caller writes/reads arena bytes
//   hkv_pf_stage_out              D2H copy of device bytes into the arena (offload)
//   hkv_pf_submit(slot, after)    side stream waits for slot `after`'s last "free"
//                                 mark, copies the descriptors, records "ready"
//   hkv_pf_wait(slot, compute)    compute stream records "need", waits for "ready"
//   hkv_pf_mark(slot, compute)    compute stream records "free" after the kernels
//                                 that read the slot's buffer
// Stall accounting: hkv_pf_stall_ms reads max(0, ready - need) of a slot once both
// events have completed (event timestamps share one device clock).
//
// hkv_gather_blocks, the record gather used to compact pools and to collect the
// records that leave for the host into one contiguous run, is in this file too.
#include "hkv_internal.h"

#include <new>
#include <vector>

struct HkvPrefetcher {
    int device;
    void* arena;
    size_t arena_bytes;
    hipStream_t side;
    std::vector<hipEvent_t> ready, freed, need;
    std::vector<int> ready_valid, need_valid, freed_valid;
    uint64_t bytes_h2d, copies_h2d, bytes_d2h;
};

using namespace hkv;

namespace {

int check_slot(HkvPrefetcher* pf, int slot) {
    if (!pf) {
        set_error("prefetcher handle is null");
        return HKV_ERR_ARG;
    }
    if (slot < 0 || slot >= (int)pf->ready.size()) {
        set_error("slot %d out of range [0, %d)", slot, (int)pf->ready.size());
        return HKV_ERR_ARG;
    }
    return HKV_OK;
}

}  // namespace

extern "C" int hkv_pf_create(int device, size_t arena_bytes, int num_slots, HkvPrefetcher** out) {
    clear_error();
    HKV_REQUIRE(out != nullptr, HKV_ERR_ARG, "hkv_pf_create: null out");
    HKV_REQUIRE(num_slots > 0 && num_slots <= 4096, HKV_ERR_ARG, "hkv_pf_create: num_slots %d out of range", num_slots);
    *out = nullptr;
    HKV_HIP_CHECK(hipSetDevice(device));
    HkvPrefetcher* pf = new (std::nothrow) HkvPrefetcher();
    HKV_REQUIRE(pf != nullptr, HKV_ERR_CAPACITY, "hkv_pf_create: out of host memory");
    pf->device = device;
    pf->arena = nullptr;
    pf->arena_bytes = arena_bytes;
    pf->bytes_h2d = pf->copies_h2d = pf->bytes_d2h = 0;
    if (arena_bytes > 0) {
        hipError_t e = hipHostMalloc(&pf->arena, arena_bytes, hipHostMallocDefault);
        if (e != hipSuccess) {
            set_error("hkv_pf_create: hipHostMalloc(%zu) failed: %s", arena_bytes, hipGetErrorString(e));
            delete pf;
            return HKV_ERR_CAPACITY;
        }
    }
    hipError_t e = hipStreamCreateWithFlags(&pf->side, hipStreamNonBlocking);
    if (e != hipSuccess) {
        set_error("hkv_pf_create: hipStreamCreate failed: %s", hipGetErrorString(e));
        if (pf->arena) (void)hipHostFree(pf->arena);
        delete pf;
        return HKV_ERR_HIP;
    }
    pf->ready.assign(num_slots, nullptr);
    pf->freed.assign(num_slots, nullptr);
    pf->need.assign(num_slots, nullptr);
    pf->ready_valid.assign(num_slots, 0);
    pf->need_valid.assign(num_slots, 0);
    pf->freed_valid.assign(num_slots, 0);
    for (int i = 0; i < num_slots; ++i) {
        if (hipEventCreate(&pf->ready[i]) != hipSuccess || hipEventCreate(&pf->freed[i]) != hipSuccess ||
            hipEventCreate(&pf->need[i]) != hipSuccess) {
            for (int j = 0; j <= i; ++j) {
                if (pf->ready[j]) (void)hipEventDestroy(pf->ready[j]);
                if (pf->freed[j]) (void)hipEventDestroy(pf->freed[j]);
                if (pf->need[j]) (void)hipEventDestroy(pf->need[j]);
            }
            (void)hipStreamDestroy(pf->side);
            if (pf->arena) (void)hipHostFree(pf->arena);
            delete pf;
            set_error("hkv_pf_create: hipEventCreate failed");
            return HKV_ERR_HIP;
        }
    }
    *out = pf;
    return HKV_OK;
}

extern "C" int hkv_pf_destroy(HkvPrefetcher* pf) {
    clear_error();
    if (!pf) return HKV_OK;
    (void)hipSetDevice(pf->device);
    (void)hipStreamSynchronize(pf->side);
    for (size_t i = 0; i < pf->ready.size(); ++i) {
        (void)hipEventDestroy(pf->ready[i]);
        (void)hipEventDestroy(pf->freed[i]);
        (void)hipEventDestroy(pf->need[i]);
    }
    (void)hipStreamDestroy(pf->side);
    if (pf->arena) (void)hipHostFree(pf->arena);
    delete pf;
    return HKV_OK;
}

extern "C" void* hkv_pf_host_ptr(HkvPrefetcher* pf, size_t offset) {
    if (!pf || !pf->arena || offset > pf->arena_bytes) return nullptr;
    return (char*)pf->arena + offset;
}

extern "C" int hkv_pf_stage_out(HkvPrefetcher* pf, const void* src_device, size_t host_offset, size_t bytes,
                                void* stream) {
    clear_error();
    HKV_REQUIRE(pf && src_device, HKV_ERR_ARG, "hkv_pf_stage_out: null argument");
    HKV_REQUIRE(host_offset + bytes <= pf->arena_bytes, HKV_ERR_CAPACITY,
                "hkv_pf_stage_out: [%zu, %zu) outside the %zu-byte arena", host_offset, host_offset + bytes,
                pf->arena_bytes);
    if (bytes == 0) return HKV_OK;
    HKV_HIP_CHECK(hipMemcpyAsync((char*)pf->arena + host_offset, src_device, bytes, hipMemcpyDeviceToHost,
                                 (hipStream_t)stream));
    pf->bytes_d2h += bytes;
    return HKV_OK;
}

extern "C" void* hkv_pf_stream(HkvPrefetcher* pf) { return pf ? (void*)pf->side : nullptr; }

extern "C" int hkv_pf_submit(HkvPrefetcher* pf, const HkvCopyDesc* descs, int n, int slot, int after_slot) {
    clear_error();
    int rc = check_slot(pf, slot);
    if (rc) return rc;
    if (after_slot >= 0) {
        rc = check_slot(pf, after_slot);
        if (rc) return rc;
    }
    HKV_REQUIRE(n >= 0 && (n == 0 || descs), HKV_ERR_ARG, "hkv_pf_submit: bad descriptor list");
    for (int i = 0; i < n; ++i) {
        HKV_REQUIRE(descs[i].bytes == 0 || (descs[i].dst != nullptr && descs[i].src != nullptr), HKV_ERR_ARG,
                    "hkv_pf_submit: descriptor %d has a null pointer", i);
    }
    if (after_slot >= 0 && pf->freed_valid[after_slot])
        HKV_HIP_CHECK(hipStreamWaitEvent(pf->side, pf->freed[after_slot], 0));
    for (int i = 0; i < n; ++i) {
        if (descs[i].bytes == 0) continue;
        HKV_HIP_CHECK(hipMemcpyAsync(descs[i].dst, descs[i].src, descs[i].bytes, hipMemcpyHostToDevice, pf->side));
        pf->bytes_h2d += descs[i].bytes;
        pf->copies_h2d += 1;
    }
    HKV_HIP_CHECK(hipEventRecord(pf->ready[slot], pf->side));
    pf->ready_valid[slot] = 1;
    return HKV_OK;
}

extern "C" int hkv_pf_record(HkvPrefetcher* pf, int slot) {
    clear_error();
    int rc = check_slot(pf, slot);
    if (rc) return rc;
    HKV_HIP_CHECK(hipEventRecord(pf->ready[slot], pf->side));
    pf->ready_valid[slot] = 1;
    return HKV_OK;
}

extern "C" int hkv_pf_wait(HkvPrefetcher* pf, int slot, void* compute_stream) {
    clear_error();
    int rc = check_slot(pf, slot);
    if (rc) return rc;
    HKV_HIP_CHECK(hipEventRecord(pf->need[slot], (hipStream_t)compute_stream));
    pf->need_valid[slot] = 1;
    if (pf->ready_valid[slot]) HKV_HIP_CHECK(hipStreamWaitEvent((hipStream_t)compute_stream, pf->ready[slot], 0));
    return HKV_OK;
}

extern "C" int hkv_pf_mark(HkvPrefetcher* pf, int slot, void* compute_stream) {
    clear_error();
    int rc = check_slot(pf, slot);
    if (rc) return rc;
    HKV_HIP_CHECK(hipEventRecord(pf->freed[slot], (hipStream_t)compute_stream));
    pf->freed_valid[slot] = 1;
    return HKV_OK;
}

extern "C" int hkv_pf_stall_ms(HkvPrefetcher* pf, int slot, float* ms) {
    clear_error();
    int rc = check_slot(pf, slot);
    if (rc) return rc;
    HKV_REQUIRE(ms != nullptr, HKV_ERR_ARG, "hkv_pf_stall_ms: null out");
    *ms = 0.f;
    if (!pf->ready_valid[slot] || !pf->need_valid[slot]) return HKV_OK;
    HKV_HIP_CHECK(hipEventSynchronize(pf->ready[slot]));
    HKV_HIP_CHECK(hipEventSynchronize(pf->need[slot]));
    float d = 0.f;
    HKV_HIP_CHECK(hipEventElapsedTime(&d, pf->need[slot], pf->ready[slot]));
    *ms = d > 0.f ? d : 0.f;
    return HKV_OK;
}

extern "C" int hkv_pf_stats(HkvPrefetcher* pf, HkvPfStats* out) {
    clear_error();
    HKV_REQUIRE(pf && out, HKV_ERR_ARG, "hkv_pf_stats: null argument");
    out->bytes_h2d = pf->bytes_h2d;
    out->copies_h2d = pf->copies_h2d;
    out->bytes_d2h = pf->bytes_d2h;
    out->arena_bytes = pf->arena_bytes;
    return HKV_OK;
}

extern "C" int hkv_pf_synchronize(HkvPrefetcher* pf) {
    clear_error();
    HKV_REQUIRE(pf != nullptr, HKV_ERR_ARG, "hkv_pf_synchronize: null handle");
    HKV_HIP_CHECK(hipStreamSynchronize(pf->side));
    return HKV_OK;
}

// ---------------------------------------------------------------- record gather

// One workgroup per destination record; 16-byte vector copies (record sizes are
// multiples of 16: H * 2208).
__global__ void __launch_bounds__(256) gather_blocks_kernel(const uint8_t* __restrict__ src, int64_t src_blocks,
                                                            const uint8_t* __restrict__ staging,
                                                            int64_t staging_blocks, const int32_t* __restrict__ ids,
                                                            int64_t rb, uint8_t* __restrict__ dst, int* err) {
    const int64_t i = blockIdx.x;
    const int id = ids[i];
    const uint8_t* rec;
    if (id >= 0) {
        if ((int64_t)id >= src_blocks) {
            if (threadIdx.x == 0 && err) atomicOr(err, 1);
            return;
        }
        rec = src + (int64_t)id * rb;
    } else {
        const int64_t s = ~(int64_t)id;
        if (s >= staging_blocks) {
            if (threadIdx.x == 0 && err) atomicOr(err, 1);
            return;
        }
        rec = staging + s * rb;
    }
    uint8_t* out = dst + i * rb;
    for (int64_t o = (int64_t)threadIdx.x * 16; o < rb; o += 256 * 16)
        *(uint4*)(out + o) = *(const uint4*)(rec + o);
}

extern "C" int hkv_gather_blocks(const uint8_t* src_pool, int64_t src_blocks, const uint8_t* src_staging,
                                 int64_t staging_blocks, const int32_t* ids, int64_t n, int64_t record_bytes,
                                 uint8_t* dst, int32_t* err_flag, void* stream) {
    clear_error();
    HKV_REQUIRE(n >= 0 && n < (1ll << 31), HKV_ERR_ARG, "hkv_gather_blocks: n %lld out of range", (long long)n);
    if (n == 0) return HKV_OK;
    HKV_REQUIRE(ids && dst, HKV_ERR_ARG, "hkv_gather_blocks: null ids/dst");
    HKV_REQUIRE(record_bytes > 0 && record_bytes % 16 == 0, HKV_ERR_ARG,
                "hkv_gather_blocks: record_bytes %lld not a positive multiple of 16", (long long)record_bytes);
    HKV_REQUIRE(src_blocks >= 0 && staging_blocks >= 0, HKV_ERR_ARG, "hkv_gather_blocks: negative block counts");
    HKV_REQUIRE(src_blocks == 0 || src_pool, HKV_ERR_ARG, "hkv_gather_blocks: null src pool");
    HKV_REQUIRE(staging_blocks == 0 || src_staging, HKV_ERR_ARG, "hkv_gather_blocks: null staging");
    HKV_REQUIRE(((uintptr_t)dst & 15) == 0 && ((uintptr_t)src_pool & 15) == 0 && ((uintptr_t)src_staging & 15) == 0,
                HKV_ERR_ARG, "hkv_gather_blocks: buffers must be 16-byte aligned");
    hipLaunchKernelGGL(gather_blocks_kernel, dim3((unsigned)n), dim3(256), 0, (hipStream_t)stream, src_pool,
                       src_blocks, src_staging, staging_blocks, ids, record_bytes, dst, (int*)err_flag);
    HKV_LAUNCH_CHECK("gather_blocks_kernel");
    return HKV_OK;
}
