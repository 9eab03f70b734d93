// calib.hip -- the heavier calibrators of the PTQ path on gfx950
// (tv/quantization/engine.tkv:42-197), all on device data, no host sync:
//
//   calibrate_kl          max|x| from the min / max partials, a num_bins
//                         histogram of |x| (LDS per block, 64-bit global
//                         atomics), then the threshold search: one candidate
//                         threshold per block, its kl sum added in the
//                         reference's sequential order; the last block to
//                         finish picks the threshold.
//   calibrate_percentile  the k-th smallest |x| by radix select on its f32 bit
//                         pattern (non-negative floats order as integers):
//                         three histogram passes of 11 / 11 / 10 bits, the
//                         last block of each picking the digit; the
//                         asymmetric form clips the min / max partials.
//   calibrate_mse         passes over x of 16 candidate thresholds each,
//                         summing squared quantization errors per block
//                         (f64), one block per candidate reducing those
//                         sums, the last of them making the reference's
//                         first-minimum pick.
//
// The histogram and the "last block" arrival counts are the context's
// calibration scratch (cal_hist, cal_arrivals): zero at creation, and each
// call's last block clears what it used.
//
// Numerics follow the reference's f64 locals.  Sums whose order the
// reference fixes are reproduced in that order where they decide the result
// bit for bit (the KL candidates); the MSE partial sums are grouped per block
// (a different order than the reference's single loop), which can only
// matter for candidates within rounding of each other.
#include <float.h>
#include <limits.h>

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
    uint32_t spill;         // radix select: a workgroup's staged elements overflowed
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

constexpr int kKlVec = 4;     // float4 loads per lane per trip, all issued before any count
constexpr int kKlCopies = 2;  // LDS histogram copies per block (copy = lane parity)

// The |x| histogram: kKlCopies LDS histograms per block, pitch num_bins + 1
// (a bin's copies in different banks), merged into the 64-bit global one at
// the end.  Each element's bin comes from two f32 quotients that bracket
// |x| / bw: |x| * fl(inv_bw (1 - 2^-22)) and |x| * fl(inv_bw (1 + 2^-22)) lie
// below and above the exact quotient by more than 2^-23 of it (two f32
// roundings of 2^-24 at most), so equal truncations below num_bins are the
// bin of the exact quotient and of its f64 rounding alike.  An element whose
// truncations differ (a bin edge within ~2^-22 of it, the clamp at num_bins,
// NaN or inf) takes kl_bin instead, each on its own branch, which a wave
// skips unless one of its lanes needs it; so does every element when 1 / bw
// is outside the f32 normal range.
//   Every block reduces the min / max partials itself for max|x| and bw (a
// few KB from L2); block 0 also records them, with the first-element NaN rule
// for the calibrate_minmax fallback, in st.
__global__ __launch_bounds__(kCalBlock) void k_kl_hist(const float* __restrict__ x, int64_t n,
                                                       int vec, int num_bins, int nparts,
                                                       const RedPartial* __restrict__ partials,
                                                       CalibState* __restrict__ st,
                                                       unsigned long long* __restrict__ hist) {
    extern __shared__ unsigned int s_hist[];  // [kKlCopies][num_bins + 1]
    const int pitch = num_bins + 1;
    for (int i = threadIdx.x; i < pitch * kKlCopies; i += kCalBlock) s_hist[i] = 0;
    double dmn, dmx;
    reduce_partials(x, nparts, 0, partials, dmn, dmx);  // its barrier also orders the clear
    // max|x| from 0 (engine.tkv:45-49, 170-174) skips NaN; all NaN gives 0
    // (the partials then hold min +inf > max -inf)
    const double am = dmn <= dmx ? fmax(fabs(dmn), fabs(dmx)) : 0.0;
    const double bw = am / (double)num_bins, inv_bw = 1.0 / bw;
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        nan_first(x, dmn, dmx);
        st->am = am;
        st->bw = bw;
        st->mn = dmn;
        st->mx = dmx;
    }
    unsigned int* h = s_hist + (threadIdx.x % kKlCopies) * pitch;
    const bool fast = inv_bw >= 0x1p-125 && inv_bw <= 0x1p+125;
    const float inv_lo = (float)(inv_bw * (1.0 - 0x1p-22));
    const float inv_hi = (float)(inv_bw * (1.0 + 0x1p-22));
    const float fbins = (float)num_bins;
    const int64_t stride = (int64_t)gridDim.x * kCalBlock;
    const int64_t tid = (int64_t)blockIdx.x * kCalBlock + threadIdx.x;
    const int64_t n4 = vec ? n / 4 : 0;
    const float4* __restrict__ x4 = reinterpret_cast<const float4*>(x);
    int64_t i = tid;
    for (; i + (kKlVec - 1) * stride < n4; i += kKlVec * stride) {
        float v[kKlVec * 4];
#pragma unroll
        for (int k = 0; k < kKlVec; k++) {
            const float4 u = x4[i + k * stride];
            v[4 * k] = u.x;
            v[4 * k + 1] = u.y;
            v[4 * k + 2] = u.z;
            v[4 * k + 3] = u.w;
        }
        int b[kKlVec * 4];
        unsigned slow = fast ? 0u : ~0u;
#pragma unroll
        for (int e = 0; e < kKlVec * 4; e++) {
            const float a = fabsf(v[e]);
            const float tl = __builtin_truncf(a * inv_lo), qh = a * inv_hi;
            const bool ok = tl == __builtin_truncf(qh) && qh < fbins;
            slow |= ok ? 0u : 1u << e;
            b[e] = ok ? (int)tl : 0;
        }
        if (slow) {
#pragma unroll
            for (int e = 0; e < kKlVec * 4; e++)
                if (slow & (1u << e)) b[e] = kl_bin(v[e], bw, inv_bw, num_bins);
        }
#pragma unroll
        for (int e = 0; e < kKlVec * 4; e++) atomicAdd(&h[b[e]], 1u);
    }
    for (; i < n4; i += stride) {
        const float4 u = x4[i];
        atomicAdd(&h[kl_bin(u.x, bw, inv_bw, num_bins)], 1u);
        atomicAdd(&h[kl_bin(u.y, bw, inv_bw, num_bins)], 1u);
        atomicAdd(&h[kl_bin(u.z, bw, inv_bw, num_bins)], 1u);
        atomicAdd(&h[kl_bin(u.w, bw, inv_bw, num_bins)], 1u);
    }
    for (int64_t j = n4 * 4 + tid; j < n; j += stride)
        atomicAdd(&h[kl_bin(x[j], bw, inv_bw, num_bins)], 1u);
    __syncthreads();
    for (int b = threadIdx.x; b < num_bins; b += kCalBlock) {
        unsigned int c = 0;
#pragma unroll
        for (int w = 0; w < kKlCopies; w++) c += s_hist[w * pitch + b];
        if (c) atomicAdd(&hist[b], (unsigned long long)c);
    }
}

static_assert(kMaxKlBins <= kCalHistBins && kRadixBins <= kCalHistBins,
              "the context's calibration histogram holds every histogram");
constexpr int kKlCandBlock = 256;
constexpr int kKlHistPerThread = (int)(kMaxKlBins / kKlCandBlock);
static_assert(kKlCandBlock == kBlock, "block_first_min runs on kBlock threads");

// kl of candidate threshold th (returned in thread 0).  Every candidate's
// total s equals the histogram total (the tail is merged into p[th - 1]), so
// p[i] = hist[i] / s for i < th - 1 and p[th - 1] = (tail sum) / s, as the
// reference's own arithmetic gives; the total and the tail are integer sums,
// exact in f64 in any order.  Threads form the block shares (each block's
// mass summed in index order) and the kl terms in parallel, the terms
// overwriting p in LDS; thread 0 then adds them in index order, so kl is the
// reference's sequential sum bit for bit (terms the reference skips, and the
// padding to a multiple of 64, are +0.0, which leaves a sum that started at
// +0.0 unchanged).
//   s_dyn: [num_bins rounded up to 64] p, then [max(target_bins, 8)] shares;
// the wave totals sit in the shares' place until those are formed, so the
// largest call (4096 bins and targets) stays within 64 KB of LDS.
__device__ double candidate_kl(int num_bins, int target_bins, int th,
                               const unsigned long long* __restrict__ hist, double* s_dyn) {
    const int tid = threadIdx.x;
    const int nb64 = (num_bins + 63) & ~63;
    double* s_p = s_dyn;
    double* s_share = s_dyn + nb64;
    unsigned long long(*s_red)[kKlCandBlock / 64] =
        reinterpret_cast<unsigned long long(*)[kKlCandBlock / 64]>(s_share);
    unsigned long long h[kKlHistPerThread];
#pragma unroll
    for (int k = 0; k < kKlHistPerThread; k++) {
        const int i = tid + k * kKlCandBlock;
        h[k] = i < num_bins ? hist[i] : 0ull;
    }
    unsigned long long tot = 0, tail = 0;
#pragma unroll
    for (int k = 0; k < kKlHistPerThread; k++) {
        tot += h[k];
        tail += tid + k * kKlCandBlock >= th - 1 ? h[k] : 0ull;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        tot += __shfl_xor(tot, o, 64);
        tail += __shfl_xor(tail, o, 64);
    }
    if ((tid & 63) == 0) {
        s_red[0][tid >> 6] = tot;
        s_red[1][tid >> 6] = tail;
    }
    __syncthreads();
    tot = 0;
    tail = 0;
#pragma unroll
    for (int w = 0; w < kKlCandBlock / 64; w++) {
        tot += s_red[0][w];
        tail += s_red[1][w];
    }
    const double total = (double)tot;
#pragma unroll
    for (int k = 0; k < kKlHistPerThread; k++) {
        const int i = tid + k * kKlCandBlock;
        if (i < th - 1) s_p[i] = (double)h[k] / total;
    }
    if (tid == 0) s_p[th - 1] = (double)tail / total;
    __syncthreads();
    const int per = th / target_bins;
    for (int b = tid; b < target_bins; b += kKlCandBlock) {
        const int start = b * per;
        const int end = (b == target_bins - 1) ? th : start + per;
        double mass = 0.0;
        int i = start;
        for (; i + 8 <= end; i += 8) {
            double v[8];
#pragma unroll
            for (int k = 0; k < 8; k++) v[k] = s_p[i + k];
#pragma unroll
            for (int k = 0; k < 8; k++) mass = mass + v[k];
        }
        for (; i < end; i++) mass = mass + s_p[i];
        int span = end - start;
        if (span < 1) span = 1;
        s_share[b] = mass / (double)span;
    }
    __syncthreads();
    const int th64 = (th + 63) & ~63;
    for (int i = tid; i < th64; i += kKlCandBlock) {
        double t = 0.0;
        if (i < th) {
            const int b = i / per < target_bins - 1 ? i / per : target_bins - 1;
            const double pi = s_p[i], sh = s_share[b];
            if (pi > 0.000000000001 && sh > 0.000000000001) t = pi * log(pi / sh);
        }
        s_p[i] = t;
    }
    __syncthreads();
    double kl = 0.0;
    if (tid == 0) {
        const double2* t2 = reinterpret_cast<const double2*>(s_p);
        for (int j = 0; j < th64 / 2; j += 16) {
            double2 v[16];
#pragma unroll
            for (int k = 0; k < 16; k++) v[k] = t2[j + k];
#pragma unroll
            for (int k = 0; k < 16; k++) {
                kl = kl + v[k].x;
                kl = kl + v[k].y;
            }
        }
    }
    return kl;
}

// Candidate th = target + 16 * blockIdx.x, one block each.  The block that
// arrives last (arrive_last) makes the selection, writes the parameters and
// clears the histogram for the next call; with no candidate (num_bins <
// target_bins) a single block only does that.
__global__ __launch_bounds__(kKlCandBlock) void k_kl_candidate(
    int num_bins, int target_bins, int ncand, unsigned long long* __restrict__ hist,
    double* __restrict__ kl_out, const CalibState* __restrict__ st, unsigned* __restrict__ arrivals,
    tkv_hip_qparams_dev* __restrict__ out) {
    extern __shared__ double s_dyn[];
    if (ncand > 0) {
        const double kl =
            candidate_kl(num_bins, target_bins, target_bins + 16 * (int)blockIdx.x, hist, s_dyn);
        if (threadIdx.x == 0)
            __hip_atomic_store(kl_out + blockIdx.x, kl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (!arrive_last(arrivals, gridDim.x)) return;
    // the first strict minimum over th ascending (the reference's loop), then
    // thr = best_bin * bw, or calibrate_minmax below max|x| 1e-8
    const int pick = block_first_min(kl_out, ncand);
    for (int i = threadIdx.x; i < num_bins; i += kKlCandBlock) hist[i] = 0;
    if (threadIdx.x == 0) {
        const int best_bin = pick < 0 ? num_bins : target_bins + 16 * pick;
        if (st->am < 0.00000001)
            finalize_minmax(st->mn, st->mx, MM_SYMMETRIC, TKV_HIP_RECIPE_PRIMARY, out);
        else
            write_sym((double)best_bin * st->bw, out);
    }
    arrive_clear(arrivals);
}

// ---------------------------------------------------------------------------
// calibrate_percentile (engine.tkv:126-162)
// ---------------------------------------------------------------------------

// Elements a workgroup of the second radix pass stages for the third.
constexpr int kPctStage = 2048;

// One radix pass: the digit (bits(|x|) >> shift) & (2^bits - 1) counted over
// the elements whose higher bits equal the prefix found so far (one LDS
// histogram per block, kKlVec float4 per lane per trip), merged into the
// global histogram.  The block that arrives last (arrive_last) finds the
// digit holding the element of the wanted rank (block prefix sum over the
// 2048 digit counts, 8 per thread), records prefix and rank in st, clears
// the histogram, and after the last pass writes the parameters.
//   The second pass also stages the bits of every element it counts (those
// whose top 11 bits match) in LDS and writes them to its own kPctStage-entry
// region of `stage`, with their number in `staged`; the third pass then reads
// only those, block for block on the same grid, instead of all of x.  A
// workgroup with more than kPctStage of them sets st->spill, and the third
// pass reads x as the others do (the first pass's last block clears it).
__device__ __forceinline__ void radix_count(unsigned int* h, float xv, uint32_t prefix,
                                            uint32_t hi_mask, int shift, uint32_t dmask) {
    const uint32_t v = __float_as_uint(xv) & 0x7fffffffu;
    if (((v ^ prefix) & hi_mask) == 0) atomicAdd(&h[(v >> shift) & dmask], 1u);
}

__device__ __forceinline__ void radix_count_stage(unsigned int* h, uint32_t* stage,
                                                  unsigned int* n_staged, float xv,
                                                  uint32_t prefix, uint32_t hi_mask, int shift,
                                                  uint32_t dmask) {
    const uint32_t v = __float_as_uint(xv) & 0x7fffffffu;
    if (((v ^ prefix) & hi_mask) == 0) {
        atomicAdd(&h[(v >> shift) & dmask], 1u);
        const unsigned int i = atomicAdd(n_staged, 1u);
        if (i < (unsigned)kPctStage) stage[i] = v;
    }
}

template <int PASS>  // 0, 1, 2
__global__ __launch_bounds__(kCalBlock) void k_radix_pass(
    const float* __restrict__ x, int64_t n, int vec, int64_t rank0, int symmetric, int nparts,
    const RedPartial* __restrict__ partials, CalibState* __restrict__ st,
    unsigned long long* __restrict__ hist, uint32_t* __restrict__ stage,
    uint32_t* __restrict__ staged, unsigned* __restrict__ arrivals,
    tkv_hip_qparams_dev* __restrict__ out) {
    constexpr int shift = PASS == 0 ? 21 : (PASS == 1 ? 10 : 0);
    constexpr int bits = PASS == 2 ? 10 : 11;
    constexpr uint32_t hi_mask = (shift + bits >= 32) ? 0u : ~((1u << (shift + bits)) - 1u);
    constexpr uint32_t dmask = (1u << bits) - 1u;
    __shared__ unsigned int s_h[kRadixBins];
    __shared__ uint32_t s_stage[PASS == 1 ? kPctStage : 1];
    __shared__ unsigned int s_nst;
    for (int i = threadIdx.x; i < kRadixBins; i += kCalBlock) s_h[i] = 0;
    if (threadIdx.x == 0) s_nst = 0;
    __syncthreads();
    const uint32_t prefix = PASS == 0 ? 0u : st->prefix;
    const int64_t stride = (int64_t)gridDim.x * kCalBlock;
    const int64_t tid = (int64_t)blockIdx.x * kCalBlock + threadIdx.x;
    auto count = [&](float v) {
        if constexpr (PASS == 1)
            radix_count_stage(s_h, s_stage, &s_nst, v, prefix, hi_mask, shift, dmask);
        else
            radix_count(s_h, v, prefix, hi_mask, shift, dmask);
    };
    // arrivals expected at the end: the whole grid, or in the third pass on
    // staged elements only its first kStagedBlocks workgroups, each taking
    // every kStagedBlocks-th region (a few elements each, typically: the
    // others return at once, so the arrival adds do not pile up behind them)
    unsigned int arriving = gridDim.x;
    if (PASS == 2 && st->spill == 0) {
        constexpr unsigned int kStagedBlocks = 64;
        arriving = gridDim.x < kStagedBlocks ? gridDim.x : kStagedBlocks;
        if (blockIdx.x >= arriving) return;
        for (unsigned int g = blockIdx.x; g < gridDim.x; g += arriving) {
            const uint32_t* __restrict__ mine = stage + (int64_t)g * kPctStage;
            const unsigned int cnt = staged[g];
            for (unsigned int i = threadIdx.x; i < cnt; i += kCalBlock)
                radix_count(s_h, __uint_as_float(mine[i]), prefix, hi_mask, shift, dmask);
        }
    } else {
        const int64_t n4 = vec ? n / 4 : 0;
        const float4* __restrict__ x4 = reinterpret_cast<const float4*>(x);
        int64_t i = tid;
        for (; i + (kKlVec - 1) * stride < n4; i += kKlVec * stride) {
            float4 u[kKlVec];
#pragma unroll
            for (int k = 0; k < kKlVec; k++) u[k] = x4[i + k * stride];
#pragma unroll
            for (int k = 0; k < kKlVec; k++) {
                count(u[k].x);
                count(u[k].y);
                count(u[k].z);
                count(u[k].w);
            }
        }
        for (; i < n4; i += stride) {
            const float4 u = x4[i];
            count(u.x);
            count(u.y);
            count(u.z);
            count(u.w);
        }
        for (int64_t j = n4 * 4 + tid; j < n; j += stride) count(x[j]);
    }
    __syncthreads();
    if constexpr (PASS == 1) {
        const unsigned int cnt = s_nst;
        const unsigned int keep = cnt < (unsigned)kPctStage ? cnt : (unsigned)kPctStage;
        uint32_t* __restrict__ mine = stage + (int64_t)blockIdx.x * kPctStage;
        for (unsigned int i = threadIdx.x; i < keep; i += kCalBlock) mine[i] = s_stage[i];
        if (threadIdx.x == 0) {
            staged[blockIdx.x] = cnt;
            if (cnt > (unsigned)kPctStage) st->spill = 1;
        }
    }
    for (int b = threadIdx.x; b < kRadixBins; b += kCalBlock) {
        const unsigned int c = s_h[b];
        if (c) atomicAdd(&hist[b], (unsigned long long)c);
    }
    if (!arrive_last(arrivals, arriving)) return;

    constexpr int kPer = kRadixBins / kCalBlock;
    __shared__ unsigned long long s_wsum[kCalBlock / 64];
    __shared__ uint32_t s_prefix;
    unsigned long long h[kPer], sum = 0;
#pragma unroll
    for (int j = 0; j < kPer; j++) {
        h[j] = __hip_atomic_load(hist + threadIdx.x * kPer + j, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
        sum += h[j];
    }
#pragma unroll
    for (int j = 0; j < kPer; j++) hist[threadIdx.x * kPer + j] = 0;
    // inclusive scan of the per-thread sums: within each wave by shuffles,
    // then the totals of the waves before
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    unsigned long long upto = sum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const unsigned long long v = __shfl_up(upto, o, 64);
        if (lane >= o) upto += v;
    }
    if (lane == 63) s_wsum[wave] = upto;
    const int64_t rank = PASS == 0 ? rank0 : st->rank;
    __syncthreads();  // also: every thread has read st->rank before it is rewritten
    for (int w = 0; w < wave; w++) upto += s_wsum[w];
    const unsigned long long before = upto - sum;
    // a rank past the total lands in the last digit, as a sequential walk ends
    if ((unsigned long long)rank >= before &&
        ((unsigned long long)rank < upto || threadIdx.x == kCalBlock - 1)) {
        int64_t r = rank - (int64_t)before;
        int d = 0;
        for (; d < kPer - 1; d++) {
            if (r < (int64_t)h[d]) break;
            r -= (int64_t)h[d];
        }
        const uint32_t np = prefix | ((uint32_t)(threadIdx.x * kPer + d) << shift);
        st->rank = r;
        st->prefix = np;
        s_prefix = np;
    }
    if (PASS == 0 && threadIdx.x == 0) st->spill = 0;
    if constexpr (PASS == 2) {
        // clip = the selected |x| (>= 1e-8); symmetric, or the reference's
        // asymmetric loop: data[0] unclipped, every later value clipped, so
        // min = data[0] < clip(min x) ? ... with the first-minimum rule (the
        // partials keep the sign of the first zero in index order).
        __syncthreads();
        double dmn = 0.0, dmx = 0.0;
        if (!symmetric) {
            reduce_partials(x, nparts, 1, partials, dmn, dmx);
            nan_first(x, dmn, dmx);
        }
        if (threadIdx.x == 0) {
            double clip = (double)__uint_as_float(s_prefix);
            if (clip <= 0.00000001) clip = 0.00000001;
            if (symmetric) {
                write_sym(clip, out);
            } else {
                const double d0 = (double)x[0];
                double vmn = dmn, vmx = dmx;
                if (vmn < -clip) vmn = -clip;
                if (vmn > clip) vmn = clip;
                if (vmx < -clip) vmx = -clip;
                if (vmx > clip) vmx = clip;
                const double mn = vmn < d0 ? vmn : d0;
                const double mx = vmx > d0 ? vmx : d0;
                finalize_minmax(mn, mx, MM_ASYMMETRIC, TKV_HIP_RECIPE_PRIMARY, out);
            }
        }
    }
    arrive_clear(arrivals);
}

// ---------------------------------------------------------------------------
// calibrate_mse (engine.tkv:165-197)
// ---------------------------------------------------------------------------

// Candidate c (1-based) of num_candidates: thr = am * c / nc, scale = thr /
// 127, inv = 1 / scale (f64, as the reference's locals).  Entries up to npad
// (whole chunks) past nc repeat the last candidate; their sums are dropped.
// The block first reduces the min / max partials to max|x| (NaN skipped, 0
// when all are NaN) and records them in st for the selection.
__global__ __launch_bounds__(kCalBlock) void k_mse_table(const float* __restrict__ x, int nparts,
                                                         const RedPartial* __restrict__ partials,
                                                         int nc, int npad,
                                                         CalibState* __restrict__ st,
                                                         double* __restrict__ table) {
    double dmn, dmx;
    reduce_partials(x, nparts, 0, partials, dmn, dmx);
    const double am = dmn <= dmx ? fmax(fabs(dmn), fabs(dmx)) : 0.0;
    if (threadIdx.x == 0) {
        nan_first(x, dmn, dmx);
        st->am = am;
        st->mn = dmn;
        st->mx = dmx;
    }
    for (int c = threadIdx.x; c < npad; c += kCalBlock) {
        const int cc = c < nc ? c : nc - 1;
        const double thr = am * (double)(cc + 1) / (double)nc;
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

// mse[c] = (sum over the per-block partials, a fixed tree order) / n.  The
// block that arrives last (arrive_last) makes the reference's first-minimum
// pick over c ascending and writes the parameters.
__global__ __launch_bounds__(kCalBlock) void k_mse_reduce(int64_t n, int nc, int nblocks,
                                                          const double* __restrict__ partial,
                                                          double* __restrict__ mse,
                                                          const double* __restrict__ table,
                                                          const CalibState* __restrict__ st,
                                                          unsigned* __restrict__ arrivals,
                                                          tkv_hip_qparams_dev* __restrict__ out) {
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
        __hip_atomic_store(mse + c, t / (double)n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (!arrive_last(arrivals, gridDim.x)) return;
    const int bc = block_first_min(mse, nc);
    if (threadIdx.x == 0) {
        if (st->am < 0.00000001)
            finalize_minmax(st->mn, st->mx, MM_SYMMETRIC, TKV_HIP_RECIPE_PRIMARY, out);
        else
            write_sym(bc >= 0 ? table[3 * bc] : st->am, out);
    }
    arrive_clear(arrivals);
}

// Histogram passes (KL, radix), each lane taking kKlVec float4 per trip: two
// blocks per CU, the fastest shape measured on MI355X for the LDS-atomic-bound
// passes and for the stream-bound ones alike.
int64_t hist_grid(Ctx* c, int64_t n) {
    int64_t blocks = ceil_div(n, (int64_t)kCalBlock * 4 * kKlVec);
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

// The calibrators finish inside their last kernels (arrive_last), on the
// context's calibration histogram and counters.
static int need_cal_scratch(Ctx* c, const char* what) {
    if (c->cal_hist && c->cal_arrivals) return TKV_HIP_OK;
    return set_error(TKV_HIP_UNSUPPORTED,
                     std::string(what) + ": this context has no calibration scratch");
}

int launch_calibrate_kl(Ctx* c, const float* x, int64_t n, int64_t num_bins, int64_t target_bins,
                        tkv_hip_qparams_dev* out) {
    if (n <= 0 || num_bins < 1 || num_bins > kMaxKlBins || target_bins < 1 ||
        target_bins > kMaxKlBins)
        return set_error(TKV_HIP_BAD_ARG,
                         "calibrate_kl: needs n > 0, 1 <= num_bins <= 4096, target_bins >= 1");
    TKV_RC_TRY(need_cal_scratch(c, "calibrate_kl"));
    CalibState* st;
    void* rest;
    const int ncand = num_bins >= target_bins ? (int)((num_bins - target_bins) / 16 + 1) : 0;
    TKV_RC_TRY(cal_workspace(c, (size_t)(ncand > 0 ? ncand : 1) * 8, &st, &rest));
    double* kl = static_cast<double*>(rest);
    int64_t nparts;
    TKV_RC_TRY(launch_partials(c, x, n, 0, &nparts));
    const int vec = aligned(x, 16) ? 1 : 0;
    hipLaunchKernelGGL(k_kl_hist, dim3((unsigned)hist_grid(c, n)), dim3(kCalBlock),
                       (size_t)(num_bins + 1) * 4 * kKlCopies, c->stream, x, n, vec,
                       (int)num_bins, (int)nparts, c->partials, st, c->cal_hist);
    TKV_LAUNCH_CHECK();
    const size_t lds = (size_t)(((num_bins + 63) & ~63) + (target_bins > 8 ? target_bins : 8)) * 8;
    hipLaunchKernelGGL(k_kl_candidate, dim3((unsigned)(ncand > 0 ? ncand : 1)),
                       dim3(kKlCandBlock), ncand > 0 ? lds : 0, c->stream, (int)num_bins,
                       (int)target_bins, ncand, c->cal_hist, kl, st, c->cal_arrivals + 1, out);
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
    TKV_RC_TRY(need_cal_scratch(c, "calibrate_percentile"));
    CalibState* st;
    void* rest;
    const int grid = (int)hist_grid(c, n);
    TKV_RC_TRY(cal_workspace(c, (size_t)grid * (kPctStage + 1) * 4, &st, &rest));
    uint32_t* staged = static_cast<uint32_t*>(rest);
    uint32_t* stage = staged + grid;
    // the min / max partials only feed the asymmetric parameters
    int64_t nparts = 0;
    if (!symmetric) TKV_RC_TRY(launch_partials(c, x, n, 1, &nparts));
    const int vec = aligned(x, 16) ? 1 : 0;
    const int64_t rank = percentile_rank(n, percentile);
#define TKV_RADIX(PASS)                                                                          \
    hipLaunchKernelGGL(k_radix_pass<PASS>, dim3((unsigned)grid), dim3(kCalBlock), 0, c->stream, \
                       x, n, vec, rank, symmetric ? 1 : 0, (int)nparts, c->partials, st,        \
                       c->cal_hist, stage, staged, c->cal_arrivals + 2, out);                   \
    TKV_LAUNCH_CHECK()
    TKV_RADIX(0);
    TKV_RADIX(1);
    TKV_RADIX(2);
#undef TKV_RADIX
    return TKV_HIP_OK;
}

int launch_calibrate_mse(Ctx* c, const float* x, int64_t n, int64_t num_candidates,
                         tkv_hip_qparams_dev* out) {
    if (n <= 0 || num_candidates > kMaxMseCandidates)
        return set_error(TKV_HIP_BAD_ARG, "calibrate_mse: needs n > 0, num_candidates <= 4096");
    TKV_RC_TRY(need_cal_scratch(c, "calibrate_mse"));
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
    hipLaunchKernelGGL(k_mse_table, dim3(1), dim3(kCalBlock), 0, c->stream, x, (int)nparts,
                       c->partials, nc, npad, st, table);
    TKV_LAUNCH_CHECK();
    const MsePartialsFn fn = mse_partials_for(ch, std::make_integer_sequence<int, kMseChunk>());
    for (int c0 = 0; c0 < nc; c0 += ch) {
        hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(kCalBlock), 0, c->stream,
                           x, n, vec, nc, c0, table, partial);
        TKV_LAUNCH_CHECK();
    }
    hipLaunchKernelGGL(k_mse_reduce, dim3((unsigned)nc), dim3(kCalBlock), 0, c->stream, n, nc,
                       grid, partial, mse, table, st, c->cal_arrivals + 3, out);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

}  // namespace tkv
