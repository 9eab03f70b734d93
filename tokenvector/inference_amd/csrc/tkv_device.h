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

// clamp(int(round(p)), lo, hi) with the reference's saturating conversion;
// lo and hi are integers within int32 range.  v_cvt_i32_f64 saturates
// out-of-range values (infinities included) to INT32_MIN / INT32_MAX and
// converts NaN to 0, so rint, the hardware conversion and an integer med3
// give the same result as clamping in f64 first.
__device__ __forceinline__ int rne_clamp(double p, double lo, double hi) {
    const double r = __builtin_rint(p);
    int i;
    asm("v_cvt_i32_f64 %0, %1" : "=v"(i) : "v"(r));
    const int l = (int)lo, h = (int)hi;
    return i < l ? l : (i > h ? h : i);
}

// clamp(int(round(x * inv)), -127, 127) for f32 x and inv.  Their product is
// exact in f64, so this equals rne_clamp((double)x * inv, -127, 127) with
// f32 operations only: one fma adds 1.5 * 2^23 to the exact product and
// rounds once, to nearest even, onto the integer grid of [2^23, 2^24), which
// is exact for |x * inv| < 2^22; the sum is clamped to 1.5 * 2^23 +- 127
// before its bits are read, so larger products and infinities saturate, and
// NaN gives 0, as the saturating conversion does.
__device__ __forceinline__ int rne_clamp127_f32(float x, float inv) {
    constexpr float kMagic = 12582912.0f;  // 1.5 * 2^23, bits 0x4B400000
    const float r = __builtin_fmaf(x, inv, kMagic);
    const float c = __builtin_amdgcn_fmed3f(r, kMagic - 127.0f, kMagic + 127.0f);
    const int i = __float_as_int(c) - 0x4B400000;
    return r != r ? 0 : i;
}

// e4m3 encode of the reference (types.tkv:154-191 with bias 7, 3 mantissa
// bits, emax field 15, no inf, saturation code 0x7E) on the binary32 bits.
// Its three departures from OCP e4m3fn are kept: |x| >= 248 -> 0x7E,
// subnormal round-up clamped to 0x07, and -0.0 -> 0x00 (f32_bits.tkv:19-20).
// NaN gives 0x38: f64_to_f32_bits(NaN) falls through both exponent loops and
// returns the bits of 1.0.  +-inf gives 0x7F|sign (the reference's loop never
// ends there).
//
// Branch-free form (checked against the scalar restatement on all 2^32
// inputs).  Normal range (|x| >= 2^-6): rounding the f32 magnitude bits to
// 3 mantissa bits, ties to even, carries into the exponent by itself, and
// rebiasing 127 -> 7 subtracts 120 << 3.  Subnormal range: the code is
// rne(|x| * 2^9) (exact scaling), clamped to 7 as the reference does.
__device__ __forceinline__ uint32_t e4m3_encode(float x) {
    const uint32_t b = __float_as_uint(x);
    const uint32_t mag = b & 0x7fffffffu, sign = (b >> 24) & 0x80u;
    uint32_t nc = ((mag + 0x7ffffu + ((mag >> 20) & 1u)) >> 20) - 960u;
    nc = mag >= 0x43780000u ? 0x7eu : nc;  // >= 248: rounds to exponent field 15
    const float s = __builtin_rintf(__uint_as_float(mag) * 512.0f);
    const uint32_t sc = s > 7.0f ? 7u : (uint32_t)s;
    uint32_t code = sign | (mag >= 0x3c800000u ? nc : sc);
    code = mag == 0u ? 0u : code;
    code = mag == 0x7f800000u ? (sign | 0x7fu) : code;
    return mag > 0x7f800000u ? 0x38u : code;
}

// The same codes through the hardware conversion.  The reference encoder is
// OCP e4m3 with round to nearest even everywhere except its three departures
// and the non-finite inputs above (the integer form above checks that on all
// 2^32 inputs), so the code of |x| comes from v_cvt_pk_fp8_f32 (OCP e4m3fn,
// nearest even) and only those cases are patched, on the magnitude bits:
//   |x| >= 248 -> 0x7E (the hardware gives 0x78 .. 0x7F there);
//   |x| < 2^-6 -> at most 0x07 (the hardware rounds [7.5 * 2^-9, 2^-6) up to
//                0x08, the reference clamps the subnormal round-up);
//   the sign bit unless x is +-0 (-0.0 -> 0x00; a nonzero value that rounds
//   to zero keeps its sign, 0x80, as in the reference);
//   +-inf -> 0x7F|sign, NaN -> 0x38.
// f32 subnormal inputs round to code 0 either way.
__device__ __forceinline__ uint32_t e4m3_fix(uint32_t bits, uint32_t c) {
    const uint32_t mag = bits & 0x7fffffffu, sign = (bits >> 24) & 0x80u;
    c = mag >= 0x43780000u ? 0x7eu : c;
    c = (mag < 0x3c800000u && c > 7u) ? 7u : c;
    c |= mag != 0u ? sign : 0u;
    c = mag == 0x7f800000u ? (sign | 0x7fu) : c;
    return mag > 0x7f800000u ? 0x38u : c;
}

// Four codes packed little-endian (a in bits 7:0).
__device__ __forceinline__ uint32_t e4m3_encode4(float a, float b, float c, float d) {
    const uint32_t ba = __float_as_uint(a), bb = __float_as_uint(b);
    const uint32_t bc = __float_as_uint(c), bd = __float_as_uint(d);
    int hw = __builtin_amdgcn_cvt_pk_fp8_f32(__uint_as_float(ba & 0x7fffffffu),
                                             __uint_as_float(bb & 0x7fffffffu), 0, false);
    hw = __builtin_amdgcn_cvt_pk_fp8_f32(__uint_as_float(bc & 0x7fffffffu),
                                         __uint_as_float(bd & 0x7fffffffu), hw, true);
    const uint32_t h = (uint32_t)hw;
    return e4m3_fix(ba, h & 0xffu) | (e4m3_fix(bb, (h >> 8) & 0xffu) << 8) |
           (e4m3_fix(bc, (h >> 16) & 0xffu) << 16) | (e4m3_fix(bd, h >> 24) << 24);
}

// The same codes for finite x with the fix-ups moved in front of the
// conversion: the magnitude is clamped where the reference departs from OCP
// (|x| >= 248 -> 448, coded 0x7E; |x| < 2^-6 -> at most 7 * 2^-9, coded at
// most 0x07) and +-0 becomes +0 (code 0x00), so the hardware code of the
// signed result is the reference's, sign included (a nonzero value that
// rounds to zero keeps 0x80).  +-inf and NaN are not covered: callers test
// for them (e4m3_special) and take e4m3_encode4 instead.
__device__ __forceinline__ float e4m3_pre(float x) {
    const float a = fabsf(x);
    float m = a < 0x1p-6f ? fminf(a, 0x1.cp-7f) : a;  // 0x1.cp-7 = 7 * 2^-9
    m = a >= 248.0f ? 448.0f : m;
    return a == 0.0f ? 0.0f : __builtin_copysignf(m, x);
}

__device__ __forceinline__ bool e4m3_special(float x) { return !(fabsf(x) < __builtin_inff()); }

__device__ __forceinline__ uint32_t e4m3_encode4_finite(float a, float b, float c, float d) {
    int hw = __builtin_amdgcn_cvt_pk_fp8_f32(e4m3_pre(a), e4m3_pre(b), 0, false);
    hw = __builtin_amdgcn_cvt_pk_fp8_f32(e4m3_pre(c), e4m3_pre(d), hw, true);
    return (uint32_t)hw;
}

__device__ __forceinline__ uint32_t e4m3_encode1(float a) {
    const uint32_t ba = __float_as_uint(a);
    const int hw = __builtin_amdgcn_cvt_pk_fp8_f32(__uint_as_float(ba & 0x7fffffffu), 0.0f, 0, false);
    return e4m3_fix(ba, (uint32_t)hw & 0xffu);
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
// Max over the wave of a non-negative, non-NaN value, returned to every
// lane: DPP row shifts and row broadcasts (VALU only) leave it in lane 63,
// then one readlane.  Lanes without a DPP source read 0, which such a max
// ignores.  wave_max's shuffles are ds_bpermute, one dependent LDS round trip
// per step.  The whole wave must be active.
__device__ __forceinline__ float wave_max_nonneg(float v) {
    int b = __float_as_int(v);
#define TKV_DPP_MAX(CTRL, ROWS)                                                       \
    b = __float_as_int(fmaxf(__int_as_float(b),                                        \
                             __int_as_float(__builtin_amdgcn_update_dpp(0, b, CTRL, ROWS, \
                                                                       0xf, false))))
    TKV_DPP_MAX(0x111, 0xf);  // row_shr:1
    TKV_DPP_MAX(0x112, 0xf);  // row_shr:2
    TKV_DPP_MAX(0x114, 0xf);  // row_shr:4
    TKV_DPP_MAX(0x118, 0xf);  // row_shr:8: lane 15 of each row holds its row's max
    TKV_DPP_MAX(0x142, 0xa);  // row_bcast:15 into rows 1 and 3
    TKV_DPP_MAX(0x143, 0xc);  // row_bcast:31 into rows 2 and 3: lane 63 holds the max
#undef TKV_DPP_MAX
    return __int_as_float(__builtin_amdgcn_readlane(b, 63));
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
