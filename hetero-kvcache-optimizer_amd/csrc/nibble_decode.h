// Fused INT4 nibble decode shared by the decode and prefill kernels: packed codes to
// exact fp16 (code - zero point) values with one v_and_or_b32 and one packed fp16
// op per two codes.
#pragma once
#include "hkv_internal.h"

namespace hkv {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// (a & m) | c in one VALU instruction (the compiler splits it when m, c are literals).
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t c) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(m), "s"(c));   // one scalar operand per VOP3
    return r;
}

// The eight codes x0..x7 of a packed word as exact fp16 (code - zero point) pairs.
// (w & 0x000F000F) | 0x6400_6400 is the fp16 pair (1024 + x0, 1024 + x1); the pair at
// bits 4..7 / 20..23 gives (1024 + 16 x2, 1024 + 16 x3), which one fma with 1/16 maps
// to (64 + x2, 64 + x3); w >> 8 repeats this for x4..x7.  z1024 holds 1024 + zp of the
// pairs (x0,x1) and (x4,x5), z64 holds 64 + zp of (x2,x3) and (x6,x7).  Every value is
// an integer below 2048, so all of it is exact in fp16.
struct NibPairs {
    h2 p0, p1, p2, p3;   // (x0,x1), (x2,x3), (x4,x5), (x6,x7) minus their zero points
};
__device__ __forceinline__ NibPairs unpack_word(uint32_t w, h2 z1024, h2 z64) {
    const uint32_t m0 = 0x000F000Fu, m1 = 0x00F000F0u, c = 0x64006400u;
    const h2 s16 = {(_Float16)0.0625f, (_Float16)0.0625f};
    const uint32_t w8 = w >> 8;
    NibPairs r;
    r.p0 = __builtin_bit_cast(h2, and_or(w, m0, c)) - z1024;
    r.p1 = __builtin_elementwise_fma(__builtin_bit_cast(h2, and_or(w, m1, c)), s16, -z64);
    r.p2 = __builtin_bit_cast(h2, and_or(w8, m0, c)) - z1024;
    r.p3 = __builtin_elementwise_fma(__builtin_bit_cast(h2, and_or(w8, m1, c)), s16, -z64);
    return r;
}
// fp16 pairs (1024 + a, 1024 + b) and (64 + a, 64 + b) of two zero points a, b <= 15
__device__ __forceinline__ h2 zp1024(uint32_t a, uint32_t b) { return __builtin_bit_cast(h2, 0x64006400u | a | (b << 16)); }
__device__ __forceinline__ h2 zp64(uint32_t a, uint32_t b) { return __builtin_bit_cast(h2, 0x54005400u | (a << 4) | (b << 20)); }

}  // namespace hkv
