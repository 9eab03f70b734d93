// tkv_reduce.h -- device-side calibration finalize and the reduction of the
// per-block min / max partials, shared by the calibration kernels of
// quant.hip and calib.hip (header-only: the library is built without
// relocatable device code).
#pragma once

#include <hip/hip_runtime.h>

#include "tkv_device.h"
#include "tkv_internal.h"

namespace tkv {

constexpr int kBlock = 256;

// ---------------------------------------------------------------------------
// Calibration finalize (engine.tkv:13-36 and session.tkv:2853-2876).
// mn / mx are the reference's f64 locals holding f32 values.
// ---------------------------------------------------------------------------
__device__ inline void finalize_minmax(double mn, double mx, int mode, int recipe,
                                       tkv_hip_qparams_dev* out) {
    tkv_hip_qparams_dev p;
    p.reserved = 0.0;
    if (mode == MM_SYMMETRIC) {
        double am = fabs(mx);
        if (fabs(mn) > am) am = fabs(mn);
        if (am < 0.00000001) am = 0.00000001;
        float scale = (float)(am / 127.0);
        p.scale = scale;
        p.min_val = (float)(-am);
        p.max_val = (float)am;
        p.zero_point = 0;
        // quantize_int8_symmetric(x, q, p.scale): engine.tkv:219-222
        if ((double)scale > 0.00000001)
            p.inv = recipe == TKV_HIP_RECIPE_PRIMARY ? (double)(1.0f / scale) : 1.0 / (double)scale;
        else
            p.inv = 1.0 / 0.00000001;
    } else if (mode == MM_ASYMMETRIC) {
        if (fabs(mx - mn) < 0.00000001) mx = mn + 0.00000001;
        double sc = (mx - mn) / 255.0;
        double z = __builtin_rint(-mn / sc);
        if (z != z) z = 0.0;
        z = z - 128.0;
        z = z < -128.0 ? -128.0 : (z > 127.0 ? 127.0 : z);
        p.scale = (float)sc;
        p.zero_point = (int32_t)z;
        p.min_val = (float)mn;
        p.max_val = (float)mx;
        p.inv = 1.0 / sc;
    } else if (mode == MM_FP8) {
        // Per-tensor FP8 scale (extension, not in the reference): amax maps
        // to kFp8Target; inv is the f32 reciprocal the scaled encode uses.
        double am = fabs(mx);
        if (fabs(mn) > am) am = fabs(mn);
        if (am < 0.00000001) am = 0.00000001;
        float scale = (float)(am / (double)kFp8Target);
        p.scale = scale;
        p.min_val = (float)(-am);
        p.max_val = (float)am;
        p.zero_point = 0;
        p.inv = (double)(1.0f / scale);
    } else {  // MM_DYNAMIC_QL
        if (mn > 0.0) mn = 0.0;
        if (mx < 0.0) mx = 0.0;
        if (mx - mn < 0.00000001) mx = mn + 0.00000001;
        double sc = (mx - mn) / 255.0;
        double z = __builtin_rint(-mn / sc);
        if (z != z) z = 0.0;
        z = z < 0.0 ? 0.0 : (z > 255.0 ? 255.0 : z);
        p.scale = (float)sc;
        p.zero_point = (int32_t)z;
        p.min_val = (float)mn;
        p.max_val = (float)mx;
        p.inv = 1.0 / sc;
        p.reserved = sc;  // the unrounded f64 scale the node divides by
    }
    *out = p;
}

__device__ __forceinline__ void mm_acc(float v, int64_t idx, bool track_zero, float& mn,
                                       float& mx, unsigned long long& zi) {
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
    if (track_zero && v == 0.0f && (unsigned long long)idx < zi) zi = (unsigned long long)idx;
}

// calibrate_minmax and DynamicQuantizeLinear seed their min and max with
// x[0] and replace them only on a strict comparison (engine.tkv:16-23,
// session.tkv:2866-2872): a NaN first element stays the result, while NaN
// anywhere else never compares and is skipped, as fminf / fmaxf skip it.
__device__ __forceinline__ void nan_first(const float* x, double& dmn, double& dmx) {
    const float x0 = x[0];
    if (x0 != x0) dmn = dmx = (double)x0;
}

// Reduces the per-block partials (every thread of a kBlock-thread block
// takes part; the result is returned to all of them) to the reference's f64
// min / max locals.  The reference keeps the first element reaching an
// extreme; values that compare equal are bit-identical except +-0, so a zero
// extreme takes the sign of the first zero in index order.
__device__ inline void reduce_partials(const float* __restrict__ x, int nparts, int track_zero,
                                       const RedPartial* __restrict__ partials, double& dmn,
                                       double& dmx) {
    float mn = __builtin_inff(), mx = -__builtin_inff();
    unsigned long long zi = ~0ull;
    for (int b = threadIdx.x; b < nparts; b += kBlock) {
        RedPartial p = partials[b];
        mn = fminf(mn, p.mn);
        mx = fmaxf(mx, p.mx);
        zi = p.zidx < zi ? p.zidx : zi;
    }
    __shared__ float s_mn[kBlock / 64], s_mx[kBlock / 64];
    __shared__ unsigned long long s_zi[kBlock / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    mn = wave_min(mn);
    mx = wave_max(mx);
    zi = wave_min_u64(zi);
    if (lane == 0) {
        s_mn[wave] = mn;
        s_mx[wave] = mx;
        s_zi[wave] = zi;
    }
    __syncthreads();
    mn = s_mn[0];
    mx = s_mx[0];
    zi = s_zi[0];
    for (int w = 1; w < kBlock / 64; w++) {
        mn = fminf(mn, s_mn[w]);
        mx = fmaxf(mx, s_mx[w]);
        zi = s_zi[w] < zi ? s_zi[w] : zi;
    }
    dmn = mn;
    dmx = mx;
    if (track_zero && zi != ~0ull) {
        const double z = x[zi];
        if (mn == 0.0f) dmn = z;
        if (mx == 0.0f) dmx = z;
    }
}

}  // namespace tkv
