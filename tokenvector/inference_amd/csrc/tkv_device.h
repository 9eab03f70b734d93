// tkv_device.h -- device-side numeric helpers shared by the kernels.
//
// Every helper restates a rounding rule of the reference's scalar path so
// that GPU codes and scales are bit-identical to it:
//   round(x)  -> .NET Math.Round(double), half to even       (v_rndne_f64)
//   int(x)    -> .NET (>= 9) saturating conversion, NaN -> 0
// All arithmetic here must stay uncontracted (no FMA): files that include
// this header are compiled with -ffp-contract=off.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tkv {

// clamp(int(round(p)), lo, hi) with the reference's saturating conversion.
__device__ __forceinline__ int rne_clamp(double p, double lo, double hi) {
    double r = __builtin_rint(p);
    if (r != r) return 0;
    r = r < lo ? lo : r;
    r = r > hi ? hi : r;
    return (int)r;
}

// Round v >= 0 right by s bits, ties to even (types.tkv:71-93).  Callers pass
// v < 2^24, so every shift >= 25 yields 0, as the reference's does.
__device__ __forceinline__ uint32_t rne_rshift(uint32_t v, int s) {
    if (s >= 25) return 0;
    uint32_t q = v >> s;
    uint32_t rem = v & ((1u << s) - 1u);
    uint32_t half = 1u << (s - 1);
    return q + ((rem > half || (rem == half && (q & 1u))) ? 1u : 0u);
}

// e4m3 encode of the reference (types.tkv:154-191 with bias 7, 3 mantissa
// bits, emax field 15, no inf, saturation code 0x7E) on the binary32 bits.
// Its three departures from OCP e4m3fn are kept: |x| >= 248 -> 0x7E,
// subnormal round-up clamped to 0x07, and -0.0 -> 0x00 (f32_bits.tkv:19-20).
// NaN gives 0x38: f64_to_f32_bits(NaN) falls through both exponent loops and
// returns the bits of 1.0.  +-inf gives 0x7F|sign (the reference's loop never
// ends there).
__device__ __forceinline__ uint32_t e4m3_encode(float x) {
    uint32_t b = __float_as_uint(x);
    uint32_t mag = b & 0x7fffffffu;
    if (mag == 0) return 0;
    if (mag > 0x7f800000u) return 0x38;
    uint32_t sign = (b >> 24) & 0x80u;
    if (mag == 0x7f800000u) return sign | 0x7fu;
    uint32_t ex = mag >> 23;
    uint32_t man = mag & 0x7fffffu;
    int e = ex ? (int)ex - 127 : -126;
    uint32_t full = ex ? (man | 0x800000u) : man;
    int e8 = e + 7;
    if (e8 >= 15) return sign | 0x7eu;
    if (e8 <= 0) {
        uint32_t m = rne_rshift(full, 21 - e8);
        return sign | (m > 7u ? 7u : m);
    }
    uint32_t r = rne_rshift(full, 20);
    if (r >= 16u) {
        r = 8u;
        e8 += 1;
        if (e8 >= 15) return sign | 0x7eu;
    }
    return sign | ((uint32_t)e8 << 3) | (r - 8u);
}

// e4m3 decode of the reference (types.tkv:193-226 through f32_bits_to_f64,
// f32_bits.tkv:60-74), f32 result.  Differs from OCP in three places that the
// reference fixes: subnormal m decodes to m * 2^-10 (normalisation uses
// exponent 127 - bias - n), 0x7F / 0xFF decode to +-inf (the exponent-255
// branch ignores the mantissa) and 0x80 decodes to +0.0 (0.0 - 0.0).
__device__ __forceinline__ float e4m3_decode_ref(uint32_t v) {
    uint32_t sign = (v >> 7) & 1u;
    uint32_t e8 = (v >> 3) & 15u;
    uint32_t m8 = v & 7u;
    if (e8 == 15u && m8 == 7u) return sign ? -__builtin_inff() : __builtin_inff();
    if (e8 == 0u) {
        if (m8 == 0u) return 0.0f;
        float mag = (float)m8 * 0x1p-10f;
        return sign ? -mag : mag;
    }
    uint32_t bits = (sign << 31) | ((e8 + 120u) << 23) | (m8 << 20);
    return __uint_as_float(bits);
}

// Wave64 reductions.
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ unsigned long long wave_min_u64(unsigned long long v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        unsigned long long t = __shfl_xor(v, o, 64);
        v = t < v ? t : v;
    }
    return v;
}

}  // namespace tkv
