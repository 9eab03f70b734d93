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

// Cross-workgroup hand-off inside one kernel, without cache maintenance:
// values another workgroup will read are written with agent-scope atomic
// stores or device atomics and read with agent-scope atomic loads, which
// gfx950 performs at the device coherence point (sc1: not held in, or served
// from, an XCD's L2).  Every wave waits for its own writes to complete
// (vmcnt(0): such a write completes once it is performed there) before the
// workgroup barrier, and one arrival add on `counter` (zero on entry) follows
// that barrier.  Returns true in every thread of the workgroup that completes
// the count of `total`; its loads are issued after its arrival add returned,
// so every other workgroup's writes are in place.  That workgroup clears the
// counter (arrive_clear) for the next call.  A release add with an acquire
// fence would instead write back and invalidate a whole L2 per workgroup.
__device__ __forceinline__ bool arrive_last(unsigned* counter, unsigned total) {
    __shared__ int s_last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
        s_last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 total - 1;
    __syncthreads();
    return s_last != 0;
}

__device__ __forceinline__ void arrive_clear(unsigned* counter) {
    if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One partial as two agent-scope 8-byte stores / loads ({mn, mx}, zidx; the
// zero index only when it is tracked, TZ).
template <bool TZ = true>
__device__ __forceinline__ void store_partial_sc1(RedPartial* p, float mn, float mx,
                                                  unsigned long long zi) {
    const unsigned long long w = (unsigned long long)__float_as_uint(mn) |
                                 ((unsigned long long)__float_as_uint(mx) << 32);
    __hip_atomic_store(reinterpret_cast<unsigned long long*>(p), w, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    if constexpr (TZ) __hip_atomic_store(&p->zidx, zi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <bool SC1>
__device__ __forceinline__ RedPartial load_partial(const RedPartial* p) {
    if constexpr (SC1) {
        const unsigned long long w = __hip_atomic_load(
            reinterpret_cast<const unsigned long long*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        RedPartial r;
        r.mn = __uint_as_float((uint32_t)w);
        r.mx = __uint_as_float((uint32_t)(w >> 32));
        r.zidx = __hip_atomic_load(&p->zidx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return r;
    } else {
        return *p;
    }
}

// Reduces the per-block partials (every thread of a kBlock-thread block
// takes part; the result is returned to all of them) to the reference's f64
// min / max locals.  The reference keeps the first element reaching an
// extreme; values that compare equal are bit-identical except +-0, so a zero
// extreme takes the sign of the first zero in index order.  SC1: partials
// written by other workgroups of the running kernel (store_partial_sc1).
template <bool SC1 = false>
__device__ inline void reduce_partials(const float* __restrict__ x, int nparts, int track_zero,
                                       const RedPartial* __restrict__ partials, double& dmn,
                                       double& dmx) {
    float mn = __builtin_inff(), mx = -__builtin_inff();
    unsigned long long zi = ~0ull;
    for (int b = threadIdx.x; b < nparts; b += kBlock) {
        const RedPartial p = load_partial<SC1>(partials + b);
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

// reduce_partials for the last workgroup of a kernel whose workgroups stored
// their partials with store_partial_sc1<TZ>: every thread issues all of its
// agent-scope loads before reducing them, one round trip for up to
// kMaxReduceBlocks partials (indices past nparts reload the last partial,
// which min / max / first-index ignore; with a loop the compiler waited for
// each trip's loads in turn), and the zero index is loaded and reduced only
// when TZ.
template <bool TZ>
__device__ inline void reduce_partials_sc1(const float* __restrict__ x, int nparts,
                                           const RedPartial* __restrict__ partials, double& dmn,
                                           double& dmx) {
    constexpr int kPer = kMaxReduceBlocks / kBlock;
    unsigned long long w[kPer], z[kPer];
#pragma unroll
    for (int i = 0; i < kPer; i++) {
        int b = (int)threadIdx.x + i * kBlock;
        b = b < nparts ? b : nparts - 1;
        w[i] = __hip_atomic_load(reinterpret_cast<const unsigned long long*>(partials + b),
                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if constexpr (TZ)
            z[i] = __hip_atomic_load(&partials[b].zidx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    float mn = __builtin_inff(), mx = -__builtin_inff();
    unsigned long long zi = ~0ull;
#pragma unroll
    for (int i = 0; i < kPer; i++) {
        mn = fminf(mn, __uint_as_float((uint32_t)w[i]));
        mx = fmaxf(mx, __uint_as_float((uint32_t)(w[i] >> 32)));
        if constexpr (TZ) zi = z[i] < zi ? z[i] : zi;
    }
    __shared__ float s_mn[kBlock / 64], s_mx[kBlock / 64];
    __shared__ unsigned long long s_zi[kBlock / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    mn = wave_min(mn);
    mx = wave_max(mx);
    if constexpr (TZ) zi = wave_min_u64(zi);
    if (lane == 0) {
        s_mn[wave] = mn;
        s_mx[wave] = mx;
        if constexpr (TZ) s_zi[wave] = zi;
    }
    __syncthreads();
    mn = s_mn[0];
    mx = s_mx[0];
    if constexpr (TZ) zi = s_zi[0];
    for (int v = 1; v < kBlock / 64; v++) {
        mn = fminf(mn, s_mn[v]);
        mx = fmaxf(mx, s_mx[v]);
        if constexpr (TZ) zi = s_zi[v] < zi ? s_zi[v] : zi;
    }
    dmn = mn;
    dmx = mx;
    if constexpr (TZ) {
        if (zi != ~0ull) {
            const double zv = x[zi];
            if (mn == 0.0f) dmn = zv;
            if (mx == 0.0f) dmx = zv;
        }
    }
}

// The reference's selection loop `if v[c] < best: best = v[c]; pick c` over
// c ascending from best = 1e45, on a kBlock-thread block (every thread calls
// it; the pick, or -1 for none, is returned to all).  Its pick is the
// smallest index holding the least value below 1e45 (`<`, so NaN never
// counts and +-0 tie): each thread takes the first strict minimum of its
// indices c = tid (mod kBlock), and pairs combine to the smaller value, or on
// == values to the smaller index.  The values are read with agent-scope
// loads (written by other workgroups of the running kernel).
__device__ inline int block_first_min(const double* v, int count) {
    __shared__ double s_b[kBlock / 64];
    __shared__ int s_i[kBlock / 64];
    double best = 1e45;
    int bi = 0x7fffffff;
    for (int c = threadIdx.x; c < count; c += kBlock) {
        const double x = __hip_atomic_load(v + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (x < best) {
            best = x;
            bi = c;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const double ob = __shfl_xor(best, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (ob < best || (ob == best && oi < bi)) {
            best = ob;
            bi = oi;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        s_b[threadIdx.x >> 6] = best;
        s_i[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    best = s_b[0];
    bi = s_i[0];
    for (int w = 1; w < kBlock / 64; w++)
        if (s_b[w] < best || (s_b[w] == best && s_i[w] < bi)) {
            best = s_b[w];
            bi = s_i[w];
        }
    return bi == 0x7fffffff ? -1 : bi;
}

}  // namespace tkv
