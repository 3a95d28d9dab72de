// Shared definitions of the gfx950 FP8 paged KV-cache kernels.
//
// Number formats, exact conversions and the per-row quantization rule are
// written once here as __host__ __device__ code: the kernels use them on the
// GPU and the host test entry points run the very same code on the CPU.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/kvfp8.h"

#define KVFP8_HD __host__ __device__ __forceinline__

namespace kvfp8 {

// Largest finite float8_e4m3fn value (torch.finfo(float8_e4m3fn).max), the MAX
// constant of reference kernals/kv_cache/quantized_append.py:50-51.
constexpr float kFp8Max = 448.0f;

KVFP8_HD uint32_t f32_bits(float x) {
    union { float f; uint32_t u; } c;
    c.f = x;
    return c.u;
}

KVFP8_HD float bits_f32(uint32_t u) {
    union { float f; uint32_t u; } c;
    c.u = u;
    return c.f;
}

// ---------------------------------------------------------------------------
// OCP float8_e4m3fn: 1 sign bit, 4 exponent bits (bias 7), 3 mantissa bits,
// no infinities, S.1111.111 is NaN, largest finite value 448.
// ---------------------------------------------------------------------------

// float32 -> e4m3fn with round-to-nearest-even, non-saturating (torch's
// `.to(torch.float8_e4m3fn)`, applied by the reference oracle at
// tests/test_kv_cache_quantization.py:65): NaN keeps its sign (0x7F / 0xFF),
// magnitudes that round above 448 become NaN, zero keeps its sign.
KVFP8_HD uint8_t encode_e4m3fn(float x) {
    const uint32_t bits = f32_bits(x);
    const uint32_t sign = (bits >> 24) & 0x80u;
    const uint32_t mag = bits & 0x7FFFFFFFu;
    // |x| >= 2^-6 (normal e4m3): keep the top 3 of 23 mantissa bits and round
    // the 20 dropped bits half to even; a mantissa carry runs into the exponent
    // field, which is the next code. (Garbage below 2^-6, where it is not used.)
    const uint32_t kept = (mag >> 20) & 0x7u;
    const uint32_t dropped = mag & 0xFFFFFu;
    const uint32_t up = (dropped > 0x80000u) | ((dropped == 0x80000u) & kept);
    const uint32_t normal = ((mag >> 23) - 120u) * 8u + kept + up;
    // |x| < 2^-6: an integer number of 2^-9 steps; scaling by 2^9 is exact and
    // rintf rounds half to even; 8 steps is code 0x08 = 2^-6.
    const uint32_t subnormal = (uint32_t)rintf(bits_f32(mag < 0x3C800000u ? mag : 0u) * 512.0f);
    uint32_t code = mag >= 0x3C800000u ? normal : subnormal;
    // Rounds past 448 (0x7E), or inf/NaN input: NaN (e4m3fn has no infinity).
    code = (code > 0x7Eu || mag >= 0x7F800000u) ? 0x7Fu : code;
    return (uint8_t)(code | sign);
}

// e4m3fn -> float32 (exact).
KVFP8_HD float decode_e4m3fn(uint32_t code) {
    const uint32_t sign = (code & 0x80u) << 24;
    const uint32_t exponent = (code >> 3) & 0xFu;
    const uint32_t mantissa = code & 0x7u;
    float mag;
    if (exponent == 0) {
        mag = (float)mantissa * (1.0f / 512.0f);
    } else if (exponent == 0xF && mantissa == 0x7) {
        mag = bits_f32(0x7FC00000u);
    } else {
        mag = bits_f32(((exponent + 120u) << 23) | (mantissa << 20));
    }
    return bits_f32(f32_bits(mag) | sign);
}

// ---------------------------------------------------------------------------
// 16-bit float formats.
// ---------------------------------------------------------------------------

KVFP8_HD float bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

// Round-to-nearest-even narrowing, NaN kept quiet (torch's float -> bfloat16).
KVFP8_HD uint16_t f32_to_bf16(float x) {
    const uint32_t u = f32_bits(x);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    const uint32_t rounding = 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)((u + rounding) >> 16);
}

KVFP8_HD float f16_to_f32(uint16_t h) {
    union { uint16_t u; _Float16 f; } c;
    c.u = h;
    return (float)c.f;
}

KVFP8_HD uint16_t f32_to_f16(float x) {
    union { uint16_t u; _Float16 f; } c;
    c.f = (_Float16)x;
    return c.u;
}

template <int DT> struct Elem;
template <> struct Elem<KVFP8_F32> {
    using T = float;
    static KVFP8_HD float load(T v) { return v; }
    static KVFP8_HD T store(float x) { return x; }
};
template <> struct Elem<KVFP8_F16> {
    using T = uint16_t;
    static KVFP8_HD float load(T v) { return f16_to_f32(v); }
    static KVFP8_HD T store(float x) { return f32_to_f16(x); }
};
template <> struct Elem<KVFP8_BF16> {
    using T = uint16_t;
    static KVFP8_HD float load(T v) { return bf16_to_f32(v); }
    static KVFP8_HD T store(float x) { return f32_to_bf16(x); }
};

// ---------------------------------------------------------------------------
// The quantization rule of one (token, kv head) row, reference
// tests/test_kv_cache_quantization.py:20-32 and :60-66.
// ---------------------------------------------------------------------------

// |x| as bits: for non-negative floats the unsigned order is the float order,
// and every NaN pattern is above +inf, so an integer max propagates NaN the way
// torch.amax does.
KVFP8_HD uint32_t abs_bits(float x) { return f32_bits(x) & 0x7FFFFFFFu; }

// scale = amax / 448 (IEEE division) when amax > 0, else 1.0 (also for NaN amax).
KVFP8_HD float row_scale(uint32_t amax_bits) {
    const float amax = bits_f32(amax_bits);
    return amax > 0.0f ? amax / kFp8Max : 1.0f;
}

// clamp(q, -448, 448) keeping NaN (torch.clamp semantics), then RNE.
KVFP8_HD uint8_t clamp_encode(float q) {
    q = q > kFp8Max ? kFp8Max : q;
    q = q < -kFp8Max ? -kFp8Max : q;
    return encode_e4m3fn(q);
}

// clamp(x / scale, -448, 448) then RNE, with IEEE division.
KVFP8_HD uint8_t quantize_value(float x, float scale) { return clamp_encode(x / scale); }

// x / scale for every element of a row that shares one scale, equal to the IEEE
// float32 division. The reciprocal y = RN(1 / scale) is one correctly rounded
// division per row; each quotient then costs a product and two FMA corrections:
//   q0 = RN(x y),  q1 = RN(q0 + (x - scale q0) y),  q2 = RN(q1 + (x - scale q1) y).
// The remainders x - scale q are exact with an FMA, q1 is within one ulp of
// x / scale, and then the second correction gives RN(x / scale) (Markstein's
// theorem). That needs normal intermediates: scale in [2^-60, 2^100] keeps the
// remainders exact wherever |x / scale| >= 2^-11; smaller quotients round to a
// zero code either way, and the sign is taken from x so -0 stays -0. Rows outside
// that scale range (tiny, infinite or NaN scales) use the IEEE division.
struct RowDivider {
    float scale;
    float recip;
    bool fast;

    KVFP8_HD explicit RowDivider(float s) : scale(s), recip(0.0f), fast(s >= 0x1p-60f && s <= 0x1p100f) {
        if (fast) recip = 1.0f / s;
    }

    KVFP8_HD float corrected(float x) const {
        const float q0 = x * recip;
        const float q1 = fmaf(fmaf(-q0, scale, x), recip, q0);
        const float q2 = fmaf(fmaf(-q1, scale, x), recip, q1);
        return copysignf(q2, x);
    }

    KVFP8_HD float divide(float x) const { return fast ? corrected(x) : x / scale; }
};

}  // namespace kvfp8
