// calib.hip -- the heavier calibrators of the PTQ path on gfx950
// (tv/quantization/engine.tkv:42-197), all on device data, no host sync:
//
//   calibrate_kl          max|x| from the min / max partials, a num_bins
//                         histogram of |x| (LDS per block, 64-bit global
//                         atomics), then the threshold search: one candidate
//                         threshold per wave, its kl sum added in the
//                         reference's sequential order.
//   calibrate_percentile  the k-th smallest |x| by radix select on its f32 bit
//                         pattern (non-negative floats order as integers):
//                         three histogram passes of 11 / 11 / 10 bits, each
//                         followed by a one-block digit pick; the asymmetric
//                         form clips the min / max partials.
//   calibrate_mse         passes over x of 16 candidate thresholds each,
//                         summing squared quantization errors per block
//                         (f64), one block per candidate reducing those
//                         sums, then the reference's first-minimum pick.
//
// Numerics follow the reference's f64 locals.  Sums whose order the
// reference fixes are reproduced in that order where they decide the result
// bit for bit (the KL candidates); the MSE partial sums are grouped per block
// (a different order than the reference's single loop), which can only
// matter for candidates within rounding of each other.
#include <float.h>

#include <utility>

#include "tkv_device.h"
#include "tkv_internal.h"
#include "tkv_reduce.h"

namespace tkv {

namespace {

constexpr int kCalBlock = 256;
constexpr int kRadixBits = 11;
constexpr int kRadixBins = 1 << kRadixBits;  // 2048
constexpr int kMseChunk = 16;  // most candidates per pass: their scale / inv pairs fit in SGPRs

// Device-side state of one calibration call (in a context workspace).
struct CalibState {
    double am, bw, mn, mx;  // max|x|, bin width; min / max (f64 locals)
    uint32_t prefix;        // radix select: bits of the k-th |x| found so far
    uint32_t pad;
    int64_t rank;           // radix select: rank within the current prefix
};

__device__ __forceinline__ void write_sym(double thr, tkv_hip_qparams_dev* out) {
    tkv_hip_qparams_dev p;
    const float scale = (float)(thr / 127.0);
    p.scale = scale;
    p.min_val = (float)(-thr);
    p.max_val = (float)thr;
    p.zero_point = 0;
    p.inv = (double)scale > 0.00000001 ? (double)(1.0f / scale) : 1.0 / 0.00000001;
    p.reserved = 0.0;
    *out = p;
}

// Shared first step: reduce the min / max partials, keep max|x| and bw.
__global__ __launch_bounds__(kBlock) void k_cal_prep(const float* __restrict__ x, int nparts,
                                                     int track_zero,
                                                     const RedPartial* __restrict__ partials,
                                                     int64_t num_bins, CalibState* st,
                                                     unsigned long long* __restrict__ hist,
                                                     int64_t hist_len, int64_t rank) {
    double dmn, dmx;
    reduce_partials(x, nparts, track_zero, partials, dmn, dmx);
    for (int64_t i = threadIdx.x; i < hist_len; i += kBlock) hist[i] = 0;
    if (threadIdx.x == 0) {
        // max|x| from 0 (engine.tkv:45-49, 170-174) skips NaN; all NaN gives
        // 0 (the partials then hold min +inf > max -inf).  mn / mx feed the
        // calibrate_minmax fallback, seeded by x[0].
        const double am = dmn <= dmx ? fmax(fabs(dmn), fabs(dmx)) : 0.0;
        nan_first(x, dmn, dmx);
        st->am = am;
        st->bw = num_bins > 0 ? am / (double)num_bins : 0.0;
        st->mn = dmn;
        st->mx = dmx;
        st->prefix = 0;
        st->pad = 0;
        st->rank = rank;
    }
}

// ---------------------------------------------------------------------------
// calibrate_kl (engine.tkv:42-123)
// ---------------------------------------------------------------------------

// bin = int(|x| / bw) with the reference's saturating conversion (NaN -> 0),
// clamped to num_bins - 1.  |x| * (1 / bw) is within a few ulps of the
// quotient, so its truncation is the quotient's unless an integer lies within
// 1e-12 (relative) of it; only those elements pay for the f64 division.
__device__ __forceinline__ int kl_bin(float xv, double bw, double inv_bw, int num_bins) {
    const double a = (double)fabsf(xv);
    double q = a * inv_bw;
    const double t = __builtin_trunc(q);
    const double margin = 1e-12 * (q + 1.0);
    if (!(q - t > margin && t + 1.0 - q > margin)) q = a / bw;  // near an integer, or NaN
    if (q != q) return 0;
    if (q >= (double)num_bins) return num_bins - 1;
    return (int)q;
}

// Each wave counts into its own LDS histogram (num_bins x 4 waves), merged
// into the 64-bit global one at the end.
__global__ __launch_bounds__(kCalBlock) void k_kl_hist(const float* __restrict__ x, int64_t n,
                                                       int vec, int num_bins,
                                                       const CalibState* __restrict__ st,
                                                       unsigned long long* __restrict__ hist) {
    extern __shared__ unsigned int s_hist[];  // [kCalBlock / 64][num_bins]
    for (int i = threadIdx.x; i < num_bins * (kCalBlock / 64); i += kCalBlock) s_hist[i] = 0;
    __syncthreads();
    unsigned int* wh = s_hist + (threadIdx.x >> 6) * num_bins;
    const double bw = st->bw, inv_bw = 1.0 / bw;
    const int64_t stride = (int64_t)gridDim.x * kCalBlock;
    const int64_t tid = (int64_t)blockIdx.x * kCalBlock + threadIdx.x;
    const int64_t n4 = vec ? n / 4 : 0;
    const float4* __restrict__ x4 = reinterpret_cast<const float4*>(x);
    int64_t i = tid;
    for (; i + stride < n4; i += 2 * stride) {
        const float4 u = x4[i], v = x4[i + stride];
        atomicAdd(&wh[kl_bin(u.x, bw, inv_bw, num_bins)], 1u);
        atomicAdd(&wh[kl_bin(u.y, bw, inv_bw, num_bins)], 1u);
        atomicAdd(&wh[kl_bin(u.z, bw, inv_bw, num_bins)], 1u);
        atomicAdd(&wh[kl_bin(u.w, bw, inv_bw, num_bins)], 1u);
        atomicAdd(&wh[kl_bin(v.x, bw, inv_bw, num_bins)], 1u);
        atomicAdd(&wh[kl_bin(v.y, bw, inv_bw, num_bins)], 1u);
        atomicAdd(&wh[kl_bin(v.z, bw, inv_bw, num_bins)], 1u);
        atomicAdd(&wh[kl_bin(v.w, bw, inv_bw, num_bins)], 1u);
    }
    for (; i < n4; i += stride) {
        const float4 u = x4[i];
        atomicAdd(&wh[kl_bin(u.x, bw, inv_bw, num_bins)], 1u);
        atomicAdd(&wh[kl_bin(u.y, bw, inv_bw, num_bins)], 1u);
        atomicAdd(&wh[kl_bin(u.z, bw, inv_bw, num_bins)], 1u);
        atomicAdd(&wh[kl_bin(u.w, bw, inv_bw, num_bins)], 1u);
    }
    for (int64_t j = n4 * 4 + tid; j < n; j += stride)
        atomicAdd(&wh[kl_bin(x[j], bw, inv_bw, num_bins)], 1u);
    __syncthreads();
    for (int b = threadIdx.x; b < num_bins; b += kCalBlock) {
        unsigned int c = 0;
        for (int w = 0; w < kCalBlock / 64; w++) c += s_hist[w * num_bins + b];
        if (c) atomicAdd(&hist[b], (unsigned long long)c);
    }
}

// Candidate th = target + 16 * blockIdx.x, one wave each.  Every candidate's
// total s equals the histogram total (the tail is merged into p[th - 1]), so
// p[i] = hist[i] / s for i < th - 1 and p[th - 1] = (tail sum) / s, as the
// reference's own arithmetic gives; the total and the tail are integer sums,
// exact in f64 in any order.  Lanes form the block shares (each block's mass
// summed in index order) and the kl terms in parallel; lane 0 adds the terms
// in index order, so kl is the reference's sequential sum bit for bit (terms
// the reference skips are +0.0).
__global__ __launch_bounds__(64) void k_kl_candidate(int num_bins, int target_bins,
                                                     const unsigned long long* __restrict__ hist,
                                                     double* __restrict__ kl_out) {
    extern __shared__ double s_dyn[];  // [num_bins] p, then [target_bins] shares
    double* s_p = s_dyn;
    double* s_share = s_dyn + num_bins;
    __shared__ double s_t[64];
    const int lane = threadIdx.x;
    const int th = target_bins + 16 * (int)blockIdx.x;
    unsigned long long tot = 0, tail = 0;
    for (int i = lane; i < num_bins; i += 64) {
        const unsigned long long h = hist[i];
        tot += h;
        if (i >= th - 1) tail += h;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        tot += __shfl_xor(tot, o, 64);
        tail += __shfl_xor(tail, o, 64);
    }
    const double total = (double)tot;
    for (int i = lane; i < th - 1; i += 64) s_p[i] = (double)hist[i] / total;
    if (lane == 0) s_p[th - 1] = (double)tail / total;
    __syncthreads();
    const int per = th / target_bins;
    for (int b = lane; b < target_bins; b += 64) {
        const int start = b * per;
        const int end = (b == target_bins - 1) ? th : start + per;
        double mass = 0.0;
        for (int i = start; i < end; i++) mass = mass + s_p[i];
        int span = end - start;
        if (span < 1) span = 1;
        s_share[b] = mass / (double)span;
    }
    __syncthreads();
    double kl = 0.0;
    for (int i0 = 0; i0 < th; i0 += 64) {
        const int i = i0 + lane;
        double t = 0.0;
        if (i < th) {
            const int b = i / per < target_bins - 1 ? i / per : target_bins - 1;
            const double pi = s_p[i], sh = s_share[b];
            if (pi > 0.000000000001 && sh > 0.000000000001) t = pi * log(pi / sh);
        }
        s_t[lane] = t;
        __syncthreads();
        if (lane == 0) {
            const int cnt = th - i0 < 64 ? th - i0 : 64;
            for (int l = 0; l < cnt; l++) kl = kl + s_t[l];
        }
        __syncthreads();
    }
    if (lane == 0) kl_out[blockIdx.x] = kl;
}

// The first strict minimum over th ascending (the reference's loop), then the
// parameters: thr = best_bin * bw, or calibrate_minmax below max|x| 1e-8.
__global__ void k_kl_select(int ncand, int num_bins, int target_bins,
                            const double* __restrict__ kl, const CalibState* __restrict__ st,
                            tkv_hip_qparams_dev* __restrict__ out) {
    double best = 1e45;
    int best_bin = num_bins;
    for (int c = 0; c < ncand; c++)
        if (kl[c] < best) {
            best = kl[c];
            best_bin = target_bins + 16 * c;
        }
    if (st->am < 0.00000001)
        finalize_minmax(st->mn, st->mx, MM_SYMMETRIC, TKV_HIP_RECIPE_PRIMARY, out);
    else
        write_sym((double)best_bin * st->bw, out);
}

// ---------------------------------------------------------------------------
// calibrate_percentile (engine.tkv:126-162)
// ---------------------------------------------------------------------------

// Histogram of digit (bits(|x|) >> shift) & (bins - 1) over the elements
// whose bits above the digit equal the prefix found so far; per-wave LDS
// histograms, 16-byte loads.
__device__ __forceinline__ void radix_count(unsigned int* wh, float xv, uint32_t prefix,
                                            uint32_t hi_mask, int shift, uint32_t dmask) {
    const uint32_t v = __float_as_uint(xv) & 0x7fffffffu;
    if (((v ^ prefix) & hi_mask) == 0) atomicAdd(&wh[(v >> shift) & dmask], 1u);
}

__global__ __launch_bounds__(kCalBlock) void k_radix_hist(const float* __restrict__ x, int64_t n,
                                                          int vec, int shift, int bits,
                                                          const CalibState* __restrict__ st,
                                                          unsigned long long* __restrict__ hist) {
    __shared__ unsigned int s_hist[kCalBlock / 64][kRadixBins];
    for (int i = threadIdx.x; i < kRadixBins * (kCalBlock / 64); i += kCalBlock)
        (&s_hist[0][0])[i] = 0;
    __syncthreads();
    unsigned int* wh = s_hist[threadIdx.x >> 6];
    const uint32_t hi_mask = (shift + bits >= 32) ? 0u : ~((1u << (shift + bits)) - 1u);
    const uint32_t prefix = st->prefix;
    const uint32_t dmask = (1u << bits) - 1u;
    const int64_t stride = (int64_t)gridDim.x * kCalBlock;
    const int64_t tid = (int64_t)blockIdx.x * kCalBlock + threadIdx.x;
    const int64_t n4 = vec ? n / 4 : 0;
    const float4* __restrict__ x4 = reinterpret_cast<const float4*>(x);
    int64_t i = tid;
    for (; i + stride < n4; i += 2 * stride) {
        const float4 u = x4[i], v = x4[i + stride];
        radix_count(wh, u.x, prefix, hi_mask, shift, dmask);
        radix_count(wh, u.y, prefix, hi_mask, shift, dmask);
        radix_count(wh, u.z, prefix, hi_mask, shift, dmask);
        radix_count(wh, u.w, prefix, hi_mask, shift, dmask);
        radix_count(wh, v.x, prefix, hi_mask, shift, dmask);
        radix_count(wh, v.y, prefix, hi_mask, shift, dmask);
        radix_count(wh, v.z, prefix, hi_mask, shift, dmask);
        radix_count(wh, v.w, prefix, hi_mask, shift, dmask);
    }
    for (; i < n4; i += stride) {
        const float4 u = x4[i];
        radix_count(wh, u.x, prefix, hi_mask, shift, dmask);
        radix_count(wh, u.y, prefix, hi_mask, shift, dmask);
        radix_count(wh, u.z, prefix, hi_mask, shift, dmask);
        radix_count(wh, u.w, prefix, hi_mask, shift, dmask);
    }
    for (int64_t j = n4 * 4 + tid; j < n; j += stride) radix_count(wh, x[j], prefix, hi_mask, shift, dmask);
    __syncthreads();
    for (int b = threadIdx.x; b < kRadixBins; b += kCalBlock) {
        unsigned int c = 0;
        for (int w = 0; w < kCalBlock / 64; w++) c += s_hist[w][b];
        if (c) atomicAdd(&hist[b], (unsigned long long)c);
    }
}

// Digit holding the element of rank st->rank (block prefix sum over the
// 2048 digit counts, 8 per thread); clears the histogram after.
__global__ __launch_bounds__(kCalBlock) void k_radix_pick(int shift, CalibState* st,
                                                          unsigned long long* __restrict__ hist) {
    constexpr int kPer = kRadixBins / kCalBlock;
    __shared__ unsigned long long s_scan[kCalBlock];
    unsigned long long h[kPer], sum = 0;
#pragma unroll
    for (int j = 0; j < kPer; j++) {
        h[j] = hist[threadIdx.x * kPer + j];
        hist[threadIdx.x * kPer + j] = 0;
        sum += h[j];
    }
    s_scan[threadIdx.x] = sum;
    __syncthreads();
    for (int o = 1; o < kCalBlock; o <<= 1) {  // inclusive scan
        const unsigned long long v = threadIdx.x >= o ? s_scan[threadIdx.x - o] : 0ull;
        __syncthreads();
        s_scan[threadIdx.x] += v;
        __syncthreads();
    }
    const int64_t rank = st->rank;
    const unsigned long long before = threadIdx.x ? s_scan[threadIdx.x - 1] : 0ull;
    const unsigned long long upto = s_scan[threadIdx.x];
    __syncthreads();  // every thread has read st->rank before it is rewritten
    // a rank past the total lands in the last digit, as a sequential walk ends
    if ((unsigned long long)rank >= before &&
        ((unsigned long long)rank < upto || threadIdx.x == kCalBlock - 1)) {
        int64_t r = rank - (int64_t)before;
        int d = 0;
        for (; d < kPer - 1; d++) {
            if (r < (int64_t)h[d]) break;
            r -= (int64_t)h[d];
        }
        st->rank = r;
        st->prefix |= (uint32_t)(threadIdx.x * kPer + d) << shift;
    }
}

// clip = the selected |x| (>= 1e-8); symmetric, or the reference's
// asymmetric loop: data[0] unclipped, every later value clipped, so
// min = data[0] < clip(min x) ? ... with the first-minimum rule (the partials
// keep the sign of the first zero in index order).
__global__ void k_pct_final(const float* __restrict__ x, int symmetric,
                            const CalibState* __restrict__ st,
                            tkv_hip_qparams_dev* __restrict__ out) {
    double clip = (double)__uint_as_float(st->prefix);
    if (clip <= 0.00000001) clip = 0.00000001;
    if (symmetric) {
        write_sym(clip, out);
        return;
    }
    const double d0 = (double)x[0];
    double vmn = st->mn, vmx = st->mx;
    if (vmn < -clip) vmn = -clip;
    if (vmn > clip) vmn = clip;
    if (vmx < -clip) vmx = -clip;
    if (vmx > clip) vmx = clip;
    const double mn = vmn < d0 ? vmn : d0;
    const double mx = vmx > d0 ? vmx : d0;
    finalize_minmax(mn, mx, MM_ASYMMETRIC, TKV_HIP_RECIPE_PRIMARY, out);
}

// ---------------------------------------------------------------------------
// calibrate_mse (engine.tkv:165-197)
// ---------------------------------------------------------------------------

// Candidate c (1-based) of num_candidates: thr = am * c / nc, scale = thr /
// 127, inv = 1 / scale (f64, as the reference's locals).  Entries up to npad
// (whole chunks) past nc repeat the last candidate; their sums are dropped.
__global__ __launch_bounds__(kCalBlock) void k_mse_table(int nc, int npad,
                                                         const CalibState* __restrict__ st,
                                                         double* __restrict__ table) {
    for (int c = threadIdx.x; c < npad; c += kCalBlock) {
        const int cc = c < nc ? c : nc - 1;
        const double thr = st->am * (double)(cc + 1) / (double)nc;
        const double scale = thr / 127.0;
        table[3 * c + 0] = thr;
        table[3 * c + 1] = scale;
        table[3 * c + 2] = 1.0 / scale;
    }
}

// Squared error of one element against candidate (scale, inv), on a = |x|.
// The reference clamps x to [-thr, thr], rounds x * inv half to even and
// clamps the code to [-127, 127].  Since fl(thr * inv) lies within a few ulps
// of 127, min(rint(|x| * inv), 127) is that code's magnitude for every x, and
// the error of -x is the negated error of x, so its square is the same.  NaN
// stays NaN (a - q * scale).  Built without contraction, q * scale, the
// difference, its square and the sum each round once, as in the reference.
__device__ __forceinline__ double mse_term(double a, double scale, double inv) {
    const double q = __builtin_fmin(__builtin_rint(a * inv), 127.0);
    const double d = a - q * scale;
    return d * d;
}

// Squared error of candidates [c0, c0 + CH) summed over this block's
// elements: partial[block * nc + c] for c < nc.  Each thread sums its
// elements in index order, four per float4.
template <int CH>
__global__ __launch_bounds__(kCalBlock) void k_mse_partials(const float* __restrict__ x, int64_t n,
                                                            int vec, int nc, int c0,
                                                            const double* __restrict__ table,
                                                            double* __restrict__ partial) {
    __shared__ double s_red[kCalBlock / 64][CH];
    double sc[CH], iv[CH], acc[CH];
#pragma unroll
    for (int c = 0; c < CH; c++) {
        sc[c] = table[3 * (c0 + c) + 1];
        iv[c] = table[3 * (c0 + c) + 2];
        acc[c] = 0.0;
    }
    const int64_t stride = (int64_t)gridDim.x * kCalBlock;
    const int64_t tid = (int64_t)blockIdx.x * kCalBlock + threadIdx.x;
    const int64_t n4 = vec ? n / 4 : 0;
    const float4* __restrict__ x4 = reinterpret_cast<const float4*>(x);
    for (int64_t i = tid; i < n4; i += stride) {
        const float4 u = x4[i];
        const double a0 = __builtin_fabs((double)u.x), a1 = __builtin_fabs((double)u.y);
        const double a2 = __builtin_fabs((double)u.z), a3 = __builtin_fabs((double)u.w);
#pragma unroll
        for (int c = 0; c < CH; c++) {
            acc[c] = acc[c] + mse_term(a0, sc[c], iv[c]);
            acc[c] = acc[c] + mse_term(a1, sc[c], iv[c]);
            acc[c] = acc[c] + mse_term(a2, sc[c], iv[c]);
            acc[c] = acc[c] + mse_term(a3, sc[c], iv[c]);
        }
    }
    for (int64_t i = 4 * n4 + tid; i < n; i += stride) {
        const double a = __builtin_fabs((double)x[i]);
#pragma unroll
        for (int c = 0; c < CH; c++) acc[c] = acc[c] + mse_term(a, sc[c], iv[c]);
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        double a = acc[c];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) a = a + __shfl_xor(a, o, 64);
        if (lane == 0) s_red[wave][c] = a;
    }
    __syncthreads();
    if (threadIdx.x < CH && c0 + (int)threadIdx.x < nc) {
        double a = 0.0;
        for (int w = 0; w < kCalBlock / 64; w++) a = a + s_red[w][threadIdx.x];
        partial[(int64_t)blockIdx.x * nc + c0 + threadIdx.x] = a;
    }
}

using MsePartialsFn = void (*)(const float*, int64_t, int, int, int, const double*, double*);

template <int... CH>
constexpr MsePartialsFn mse_partials_for(int ch, std::integer_sequence<int, CH...>) {
    constexpr MsePartialsFn fns[] = {k_mse_partials<CH + 1>...};
    return fns[ch - 1];
}

// mse[c] = (sum over the per-block partials, a fixed tree order) / n.
__global__ __launch_bounds__(kCalBlock) void k_mse_reduce(int64_t n, int nc, int nblocks,
                                                          const double* __restrict__ partial,
                                                          double* __restrict__ mse) {
    __shared__ double s_red[kCalBlock / 64];
    const int c = blockIdx.x;
    double a = 0.0;
    for (int b = threadIdx.x; b < nblocks; b += kCalBlock) a = a + partial[(int64_t)b * nc + c];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) a = a + __shfl_xor(a, o, 64);
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = a;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        for (int w = 0; w < kCalBlock / 64; w++) t = t + s_red[w];
        mse[c] = t / (double)n;
    }
}

// The first strict minimum over c ascending, as in the reference's loop.
__global__ void k_mse_select(int nc, const double* __restrict__ table,
                             const double* __restrict__ mse, const CalibState* __restrict__ st,
                             tkv_hip_qparams_dev* __restrict__ out) {
    double best = 1e45;
    int bc = -1;
    for (int c = 0; c < nc; c++)
        if (mse[c] < best) {
            best = mse[c];
            bc = c;
        }
    if (st->am < 0.00000001)
        finalize_minmax(st->mn, st->mx, MM_SYMMETRIC, TKV_HIP_RECIPE_PRIMARY, out);
    else
        write_sym(bc >= 0 ? table[3 * bc] : st->am, out);
}

int64_t cal_grid(Ctx* c, int64_t n) {
    int64_t blocks = ceil_div(n, (int64_t)kCalBlock * 4);
    const int64_t cap = (int64_t)c->num_cus * 2;
    if (blocks > cap) blocks = cap;
    return blocks < 1 ? 1 : blocks;
}

// Workspace slot 9: [CalibState][histogram or MSE table + partials].
int cal_workspace(Ctx* c, size_t extra, CalibState** st, void** rest) {
    void* w;
    TKV_RC_TRY(ctx_workspace(c, 9, 256 + extra, &w));
    *st = static_cast<CalibState*>(w);
    *rest = static_cast<char*>(w) + 256;
    return TKV_HIP_OK;
}

}  // namespace

int launch_calibrate_kl(Ctx* c, const float* x, int64_t n, int64_t num_bins, int64_t target_bins,
                        tkv_hip_qparams_dev* out) {
    if (n <= 0 || num_bins < 1 || num_bins > kMaxKlBins || target_bins < 1 ||
        target_bins > kMaxKlBins)
        return set_error(TKV_HIP_BAD_ARG,
                         "calibrate_kl: needs n > 0, 1 <= num_bins <= 4096, target_bins >= 1");
    CalibState* st;
    void* rest;
    const int ncand = num_bins >= target_bins ? (int)((num_bins - target_bins) / 16 + 1) : 0;
    TKV_RC_TRY(cal_workspace(c, (size_t)num_bins * 16 + (size_t)ncand * 8 + 8, &st, &rest));
    auto* hist = static_cast<unsigned long long*>(rest);
    double* kl = reinterpret_cast<double*>(hist + num_bins);
    int64_t nparts;
    TKV_RC_TRY(launch_partials(c, x, n, 0, &nparts));
    hipLaunchKernelGGL(k_cal_prep, dim3(1), dim3(kBlock), 0, c->stream, x, (int)nparts, 0,
                       c->partials, num_bins, st, hist, num_bins, (int64_t)0);
    TKV_LAUNCH_CHECK();
    const int vec = aligned(x, 16) ? 1 : 0;
    hipLaunchKernelGGL(k_kl_hist, dim3((unsigned)cal_grid(c, n)), dim3(kCalBlock),
                       (size_t)num_bins * 4 * (kCalBlock / 64), c->stream, x, n, vec,
                       (int)num_bins, st, hist);
    TKV_LAUNCH_CHECK();
    if (ncand > 0) {
        hipLaunchKernelGGL(k_kl_candidate, dim3((unsigned)ncand), dim3(64),
                           (size_t)(num_bins + target_bins) * 8, c->stream, (int)num_bins,
                           (int)target_bins, hist, kl);
        TKV_LAUNCH_CHECK();
    }
    hipLaunchKernelGGL(k_kl_select, dim3(1), dim3(1), 0, c->stream, ncand, (int)num_bins,
                       (int)target_bins, kl, st, out);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

int64_t percentile_rank(int64_t n, float percentile) {
    const int64_t nab = n - 1 < 0 ? 0 : n - 1;
    const double t = (double)percentile / 100.0 * (double)n;
    const double lim = (double)nab < t ? (double)nab : t;
    return (int64_t)lim;  // t > 0, below 2^63: plain truncation
}

int launch_calibrate_percentile(Ctx* c, const float* x, int64_t n, float percentile,
                                int symmetric, tkv_hip_qparams_dev* out) {
    if (n <= 0) return set_error(TKV_HIP_BAD_ARG, "calibrate_percentile: empty input");
    if (!(percentile > 0.0f && percentile <= 100.0f))
        return set_error(TKV_HIP_BAD_ARG, "percentile must be in (0, 100]");
    CalibState* st;
    void* rest;
    TKV_RC_TRY(cal_workspace(c, (size_t)kRadixBins * 8, &st, &rest));
    auto* hist = static_cast<unsigned long long*>(rest);
    int64_t nparts;
    TKV_RC_TRY(launch_partials(c, x, n, symmetric ? 0 : 1, &nparts));
    hipLaunchKernelGGL(k_cal_prep, dim3(1), dim3(kBlock), 0, c->stream, x, (int)nparts,
                       symmetric ? 0 : 1, c->partials, (int64_t)0, st, hist, (int64_t)kRadixBins,
                       percentile_rank(n, percentile));
    TKV_LAUNCH_CHECK();
    const int grid = (int)cal_grid(c, n);
    const int vec = aligned(x, 16) ? 1 : 0;
    const int shifts[3] = {21, 10, 0}, widths[3] = {11, 11, 10};
    for (int r = 0; r < 3; r++) {
        hipLaunchKernelGGL(k_radix_hist, dim3((unsigned)grid), dim3(kCalBlock), 0, c->stream, x,
                           n, vec, shifts[r], widths[r], st, hist);
        TKV_LAUNCH_CHECK();
        hipLaunchKernelGGL(k_radix_pick, dim3(1), dim3(kCalBlock), 0, c->stream, shifts[r], st,
                           hist);
        TKV_LAUNCH_CHECK();
    }
    hipLaunchKernelGGL(k_pct_final, dim3(1), dim3(1), 0, c->stream, x, symmetric, st, out);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

int launch_calibrate_mse(Ctx* c, const float* x, int64_t n, int64_t num_candidates,
                         tkv_hip_qparams_dev* out) {
    if (n <= 0 || num_candidates > kMaxMseCandidates)
        return set_error(TKV_HIP_BAD_ARG, "calibrate_mse: needs n > 0, num_candidates <= 4096");
    const int nc = (int)(num_candidates < 4 ? 4 : num_candidates);
    // passes of ch <= kMseChunk candidates, as even as whole passes allow
    const int passes = (int)ceil_div((int64_t)nc, (int64_t)kMseChunk);
    const int ch = (int)ceil_div((int64_t)nc, (int64_t)passes);
    const int npad = passes * ch;
    // compute-bound: up to 8 blocks per CU
    int64_t blocks = ceil_div(n, (int64_t)kCalBlock * 4);
    if (blocks > (int64_t)c->num_cus * 8) blocks = (int64_t)c->num_cus * 8;
    const int grid = blocks < 1 ? 1 : (int)blocks;
    const int vec = aligned(x, 16) ? 1 : 0;
    CalibState* st;
    void* rest;
    TKV_RC_TRY(cal_workspace(c, (size_t)npad * 24 + (size_t)nc * 8 + (size_t)grid * nc * 8, &st,
                             &rest));
    auto* table = static_cast<double*>(rest);
    double* mse = table + 3 * npad;
    double* partial = mse + nc;
    int64_t nparts;
    TKV_RC_TRY(launch_partials(c, x, n, 0, &nparts));
    hipLaunchKernelGGL(k_cal_prep, dim3(1), dim3(kBlock), 0, c->stream, x, (int)nparts, 0,
                       c->partials, (int64_t)0, st, (unsigned long long*)nullptr, (int64_t)0,
                       (int64_t)0);
    TKV_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_mse_table, dim3(1), dim3(kCalBlock), 0, c->stream, nc, npad, st, table);
    TKV_LAUNCH_CHECK();
    const MsePartialsFn fn = mse_partials_for(ch, std::make_integer_sequence<int, kMseChunk>());
    for (int c0 = 0; c0 < nc; c0 += ch) {
        hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(kCalBlock), 0, c->stream,
                           x, n, vec, nc, c0, table, partial);
        TKV_LAUNCH_CHECK();
    }
    hipLaunchKernelGGL(k_mse_reduce, dim3((unsigned)nc), dim3(kCalBlock), 0, c->stream, n, nc,
                       grid, partial, mse);
    TKV_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_mse_select, dim3(1), dim3(1), 0, c->stream, nc, table, mse, st, out);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

}  // namespace tkv
