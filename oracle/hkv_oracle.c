/*
 * CPU restatement of the reference INT4 group quantizer -- TEST INFRASTRUCTURE ONLY.
 *
 * The HIP kernels are compared with this file's results.  Only tests/, the smoke test and
 * the bench's cpu_baseline leg load it; the product path never does.
 *
 * It follows src/quantization/kv_compressor.py of kldxg123/Hetero-KVCache-Optimizer:
 *   compress   :66-98   flat = x.float().reshape(-1); zero-pad to a multiple of
 *                       group_size (:70-74); per-group min/max (:76-77);
 *                       scale = clamp((max-min)/15, min=1e-8) (:79-80);
 *                       zp = uint8(clamp(round(-min/scale), 0, 15)) (:82-84);
 *                       q = uint8(clamp(round(flat/scale + zp), 0, 15)) (:86-88);
 *                       crop to the input size (:91)
 *   decompress :119-132 ((float(q) - float(zp)) * scale).to(dtype)
 * torch.round is round-half-to-even, i.e. rintf under the default rounding mode;
 * every operation is single precision with IEEE division (built with
 * -ffp-contract=off and without -ffast-math, on SSE so there is no excess
 * precision).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define HKVO_F16 0
#define HKVO_BF16 1
#define HKVO_F32 2

static float bits_to_float(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint32_t float_to_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

/* IEEE binary16 -> binary32 (exact). */
float hkvo_h2f(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    if (e == 0) {
        const float v = (float)m * 5.9604644775390625e-08f; /* m * 2^-24, exact */
        return (h & 0x8000u) ? -v : v;
    }
    if (e == 31) return bits_to_float(sign | 0x7f800000u | (m << 13));
    return bits_to_float(sign | ((e + 112u) << 23) | (m << 13));
}

/* binary32 -> binary16, round to nearest even, overflow to inf. */
uint16_t hkvo_f2h(float f) {
    const uint32_t x = float_to_bits(f);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) {
        /* fp16 subnormal range: the result is round(|x| * 2^24) ulps of 2^-24 */
        const float r = rintf(fabsf(f) * 16777216.0f);
        return (uint16_t)(sign | (uint16_t)r);
    }
    uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float hkvo_bf2f(uint16_t b) { return bits_to_float((uint32_t)b << 16); }

/* binary32 -> bfloat16, round to nearest even (c10::BFloat16 semantics). */
uint16_t hkvo_f2bf(float f) {
    const uint32_t u = float_to_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

static float load_elem(const void* x, int dtype, int64_t i) {
    if (dtype == HKVO_F16) return hkvo_h2f(((const uint16_t*)x)[i]);
    if (dtype == HKVO_BF16) return hkvo_bf2f(((const uint16_t*)x)[i]);
    return ((const float*)x)[i];
}

/* kv_compressor.py:76-84 for one group's min and max. */
void hkvo_group_params(float mn, float mx, float* scale, uint8_t* zp) {
    float s = (mx - mn) / 15.0f;
    if (s < 1e-8f) s = 1e-8f;
    float z = rintf(-mn / s);
    if (!(z >= 0.0f)) z = 0.0f; /* NaN converts to 0, as torch's .to(uint8) does */
    if (z > 15.0f) z = 15.0f;
    *scale = s;
    *zp = (uint8_t)z;
}

/* kv_compressor.py:86-88 for one element. */
uint8_t hkvo_quant_code(float x, float scale, uint8_t zp) {
    float t = x / scale;
    t = t + (float)zp;
    t = rintf(t);
    if (!(t >= 0.0f)) t = 0.0f; /* NaN as above */
    if (t > 15.0f) t = 15.0f;
    return (uint8_t)t;
}

/* KVCompressor.compress over n flattened elements; returns the group count. */
int64_t hkvo_compress(const void* x, int dtype, int64_t n, int32_t group_size, uint8_t* codes,
                      float* scales, uint8_t* zps) {
    if (n <= 0 || group_size <= 0) return 0;
    const int64_t ngroups = (n + group_size - 1) / group_size;
    for (int64_t g = 0; g < ngroups; ++g) {
        const int64_t base = g * (int64_t)group_size;
        float mn = INFINITY, mx = -INFINITY;
        for (int32_t i = 0; i < group_size; ++i) {
            const int64_t idx = base + i;
            const float v = idx < n ? load_elem(x, dtype, idx) : 0.0f; /* zero padding */
            /* torch's min/max propagate NaN: one NaN makes the group's scale NaN,
               and its zero point and codes then convert to 0 */
            if (v != v || mn != mn) mn = mx = NAN;
            else {
                if (v < mn) mn = v;
                if (v > mx) mx = v;
            }
        }
        float s;
        uint8_t z;
        hkvo_group_params(mn, mx, &s, &z);
        scales[g] = s;
        zps[g] = z;
        for (int32_t i = 0; i < group_size; ++i) {
            const int64_t idx = base + i;
            if (idx < n) codes[idx] = hkvo_quant_code(load_elem(x, dtype, idx), s, z);
        }
    }
    return ngroups;
}

/* KVCompressor.decompress: out dtype F16 / BF16 / F32. */
void hkvo_decompress(const uint8_t* codes, const float* scales, const uint8_t* zps, int64_t n,
                     int32_t group_size, void* out, int out_dtype) {
    for (int64_t i = 0; i < n; ++i) {
        const int64_t g = i / group_size;
        const float v = ((float)codes[i] - (float)zps[g]) * scales[g];
        if (out_dtype == HKVO_F16) ((uint16_t*)out)[i] = hkvo_f2h(v);
        else if (out_dtype == HKVO_BF16) ((uint16_t*)out)[i] = hkvo_f2bf(v);
        else ((float*)out)[i] = v;
    }
}

/* Element-wise conversions exposed for the oracle's own tests. */
void hkvo_f2h_array(const float* in, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = hkvo_f2h(in[i]);
}

void hkvo_h2f_array(const uint16_t* in, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = hkvo_h2f(in[i]);
}

void hkvo_f2bf_array(const float* in, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = hkvo_f2bf(in[i]);
}
