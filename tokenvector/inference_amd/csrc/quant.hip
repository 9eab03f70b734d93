// quant.hip -- HBM-bound kernels of the PTQ path on gfx950:
//   absmax / min-max calibration (per tensor, per row), f32 -> int8 quantize
//   (per tensor, per channel, dynamic per row), f32 -> e4m3 encode,
//   dequantize, and code-layout conversions for the host-pointer mirrors.
//
// Layout: f32 inputs are read as 16-byte float4 loads, four per thread per
// loop trip for memory-level parallelism; int8 / e4m3 outputs leave as one
// 32-bit store per float4.  The streaming grids are two 256-thread blocks
// per CU, the shape that measured highest on MI355X HBM (about 6.8 TB/s
// read-only with nontemporal loads, 6.5 TB/s for the 16 B in / 4 B out
// quantize stream, against 5.3 TB/s from 16 blocks per CU).  Loads are
// nontemporal for tensors beyond kCacheableBytes, which no cache level
// holds; smaller ones load through the caches, so the quantize pass that
// follows calibration finds x in the 256 MB Infinity Cache.  Codes are
// stored through the caches too: the GEMM reads them next.  Reductions use
// wave64 shuffles, then
// LDS, then one partial per block; the consumer of the partials (a one-block
// finalize, or every block of the quantize kernel) reduces them after the
// kernel boundary, which orders them across XCDs without device-scope fences.
//
// Numerics restate tv/quantization/engine.tkv and types.tkv exactly: f64
// products and reciprocals where the reference computes in f64, round half to
// even, saturating clamp.  Compiled with -ffp-contract=off.
#include <float.h>
#include <cstdlib>

#include "gemm_tile.h"
#include "tkv_device.h"
#include "tkv_internal.h"
#include "tkv_reduce.h"

namespace tkv {

constexpr int kRedBlock = 256;   // calibration partial blocks
constexpr int kBlocksPerCu = 2;  // streaming grids: blocks per CU
constexpr int kUnroll = 4;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int64_t kCacheableBytes = 128ll << 20;

template <bool NT = true>
__device__ __forceinline__ float4 ld4(const float4* p) {
    if constexpr (NT) {
        const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
        return make_float4(v.x, v.y, v.z, v.w);
    } else {
        return *p;
    }
}

// Per-tensor min / max (+ first zero): one partial per block.  Consumers
// either reduce the partials themselves (the quantize kernels, every block),
// or (FIN) the last block to arrive reduces them and writes the QuantParams:
// the partials then go through the device coherence point (store_partial_sc1,
// arrive_last), so no finalize kernel and no cache maintenance is needed.
// Without FIN the kernel boundary orders the partial stores before the
// consumer's reads.
template <bool TRACK_ZERO, bool NT, bool FIN = false>
__global__ __launch_bounds__(kRedBlock) void k_minmax_partials(const float* __restrict__ x,
                                                               int64_t n, int vec,
                                                               RedPartial* __restrict__ partials,
                                                               unsigned* __restrict__ arrivals = nullptr,
                                                               int mode = 0, int recipe = 0,
                                                               tkv_hip_qparams_dev* __restrict__ out = nullptr) {
    float mn = __builtin_inff(), mx = -__builtin_inff();
    unsigned long long zi = ~0ull;
    // x[0] for the first-element NaN rule, loaded early: the last block's
    // finalize would otherwise wait for it at the end of the kernel
    float x0 = 0.0f;
    if (FIN && threadIdx.x == 0) x0 = x[0];
    const int64_t stride = (int64_t)gridDim.x * kRedBlock;
    const int64_t tid = (int64_t)blockIdx.x * kRedBlock + threadIdx.x;
    int64_t n4 = vec ? n / 4 : 0;
    const float4* __restrict__ x4 = reinterpret_cast<const float4*>(x);
    int64_t i = tid;
    for (; i + (kUnroll - 1) * stride < n4; i += kUnroll * stride) {
        float4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; u++) v[u] = ld4<NT>(x4 + i + u * stride);
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            int64_t b = (i + u * stride) * 4;
            mm_acc(v[u].x, b + 0, TRACK_ZERO, mn, mx, zi);
            mm_acc(v[u].y, b + 1, TRACK_ZERO, mn, mx, zi);
            mm_acc(v[u].z, b + 2, TRACK_ZERO, mn, mx, zi);
            mm_acc(v[u].w, b + 3, TRACK_ZERO, mn, mx, zi);
        }
    }
    for (; i < n4; i += stride) {
        float4 v = ld4<NT>(x4 + i);
        mm_acc(v.x, i * 4 + 0, TRACK_ZERO, mn, mx, zi);
        mm_acc(v.y, i * 4 + 1, TRACK_ZERO, mn, mx, zi);
        mm_acc(v.z, i * 4 + 2, TRACK_ZERO, mn, mx, zi);
        mm_acc(v.w, i * 4 + 3, TRACK_ZERO, mn, mx, zi);
    }
    for (int64_t j = n4 * 4 + tid; j < n; j += stride) mm_acc(x[j], j, TRACK_ZERO, mn, mx, zi);

    __shared__ float s_mn[kRedBlock / 64], s_mx[kRedBlock / 64];
    __shared__ unsigned long long s_zi[kRedBlock / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    mn = wave_min(mn);
    mx = wave_max(mx);
    if (TRACK_ZERO) zi = wave_min_u64(zi);
    if (lane == 0) {
        s_mn[wave] = mn;
        s_mx[wave] = mx;
        s_zi[wave] = zi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kRedBlock / 64; w++) {
            mn = fminf(mn, s_mn[w]);
            mx = fmaxf(mx, s_mx[w]);
            zi = s_zi[w] < zi ? s_zi[w] : zi;
        }
        if constexpr (FIN) {
            store_partial_sc1<TRACK_ZERO>(partials + blockIdx.x, mn, mx, zi);
        } else {
            RedPartial p;
            p.mn = mn;
            p.mx = mx;
            p.zidx = zi;
            partials[blockIdx.x] = p;
        }
    }
    if constexpr (FIN) {
        if (!arrive_last(arrivals, gridDim.x)) return;
        double dmn, dmx;
        reduce_partials_sc1<TRACK_ZERO>(x, (int)gridDim.x, partials, dmn, dmx);
        if (threadIdx.x == 0) {
            if (x0 != x0) dmn = dmx = (double)x0;  // nan_first
            finalize_minmax(dmn, dmx, mode, recipe, out);
        }
        arrive_clear(arrivals);
    }
}

__global__ __launch_bounds__(kBlock) void k_minmax_finalize(const float* __restrict__ x,
                                                            int nparts, int track_zero, int mode,
                                                            int recipe,
                                                            const RedPartial* __restrict__ partials,
                                                            tkv_hip_qparams_dev* __restrict__ out) {
    double dmn, dmx;
    reduce_partials(x, nparts, track_zero, partials, dmn, dmx);
    nan_first(x, dmn, dmx);
    if (threadIdx.x == 0) finalize_minmax(dmn, dmx, mode, recipe, out);
}

// kBlocksPerCu partials per CU: few enough that every block of a consumer
// kernel can reduce them itself.
static int64_t partial_blocks(Ctx* c, int64_t work, int vec) {
    int64_t blocks = ceil_div(work, (int64_t)kRedBlock * kUnroll);
    const int64_t want = (int64_t)c->num_cus * (vec ? kBlocksPerCu : 8);
    const int64_t cap = want < kMaxReduceBlocks ? want : kMaxReduceBlocks;
    if (blocks > cap) blocks = cap;
    return blocks < 1 ? 1 : blocks;
}

int launch_partials(Ctx* c, const float* x, int64_t n, int track_zero, int64_t* nparts) {
    const int vec = aligned(x, 16) ? 1 : 0;
    const int64_t blocks = partial_blocks(c, vec ? n / 4 : n, vec);
    const bool nt = n * 4 > kCacheableBytes;
#define TKV_PARTIALS(TZ, NT)                                                                     \
    hipLaunchKernelGGL((k_minmax_partials<TZ, NT>), dim3((unsigned)blocks), dim3(kRedBlock), 0, \
                       c->stream, x, n, vec, c->partials)
    if (track_zero) {
        if (nt) TKV_PARTIALS(true, true);
        else TKV_PARTIALS(true, false);
    } else {
        if (nt) TKV_PARTIALS(false, true);
        else TKV_PARTIALS(false, false);
    }
#undef TKV_PARTIALS
    TKV_LAUNCH_CHECK();
    *nparts = blocks;
    return TKV_HIP_OK;
}

int launch_minmax_tensor(Ctx* c, const float* x, int64_t n, int mode, int recipe,
                         tkv_hip_qparams_dev* out) {
    // the kernels read x[0] (the first-element NaN rule): an empty tensor is
    // the callers' case (the host entry points return the identity params)
    if (n <= 0 || !x) return set_error(TKV_HIP_BAD_ARG, "min/max of an empty or NULL tensor");
    // Only the asymmetric QuantParams expose the sign of a zero extreme.
    const int track_zero = (mode == MM_ASYMMETRIC) ? 1 : 0;
    if (c->cal_arrivals) {  // one kernel: its last block finalizes
        const int vec = aligned(x, 16) ? 1 : 0;
        const int64_t blocks = partial_blocks(c, vec ? n / 4 : n, vec);
        const bool nt = n * 4 > kCacheableBytes;
        unsigned* arr = c->cal_arrivals + 0;
#define TKV_PARTIALS_FIN(TZ, NT)                                                           \
    hipLaunchKernelGGL((k_minmax_partials<TZ, NT, true>), dim3((unsigned)blocks),         \
                       dim3(kRedBlock), 0, c->stream, x, n, vec, c->partials, arr, mode, \
                       recipe, out)
        if (track_zero) {
            if (nt) TKV_PARTIALS_FIN(true, true);
            else TKV_PARTIALS_FIN(true, false);
        } else {
            if (nt) TKV_PARTIALS_FIN(false, true);
            else TKV_PARTIALS_FIN(false, false);
        }
#undef TKV_PARTIALS_FIN
        TKV_LAUNCH_CHECK();
        return TKV_HIP_OK;
    }
    int64_t nparts;
    TKV_RC_TRY(launch_partials(c, x, n, track_zero, &nparts));
    hipLaunchKernelGGL(k_minmax_finalize, dim3(1), dim3(kBlock), 0, c->stream, x, (int)nparts,
                       track_zero, mode, recipe, c->partials, out);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

// ---------------------------------------------------------------------------
// Per-tensor int8 quantize: q = clamp(rne(x * inv), +-127), inv from params
// (engine.tkv:216-226).  OUT_I32 writes the reference's int32 codes.
// ---------------------------------------------------------------------------
// Low bytes of a, b, c, d as one little-endian word: two byte permutes
// (selector 0x0c yields a zero byte) and an or.
__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    const uint32_t lo = __builtin_amdgcn_perm((uint32_t)b, (uint32_t)a, 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm((uint32_t)d, (uint32_t)c, 0x04000c0cu);
    return lo | hi;
}

template <bool OUT_I32>
__device__ __forceinline__ void store4(void* q, int64_t i4, int a, int b, int c, int d) {
    if (OUT_I32) {
        reinterpret_cast<int4*>(q)[i4] = make_int4(a, b, c, d);
    } else {
        reinterpret_cast<uint32_t*>(q)[i4] = pack4(a, b, c, d);
    }
}

template <bool OUT_I32>
__device__ __forceinline__ void store1(void* q, int64_t i, int a) {
    if (OUT_I32)
        reinterpret_cast<int32_t*>(q)[i] = a;
    else
        reinterpret_cast<int8_t*>(q)[i] = (int8_t)a;
}

// FUSED: the scale is computed here from the calibration partials (every
// block reduces them itself, so no finalize kernel runs in between); block 0
// also publishes the QuantParams to *p.  Otherwise *p is read.
template <bool OUT_I32, bool FUSED, bool NT>
__global__ __launch_bounds__(kBlock) void k_quant_i8_tensor(const float* __restrict__ x,
                                                            int64_t n, int vec,
                                                            tkv_hip_qparams_dev* __restrict__ p,
                                                            void* __restrict__ q, int nparts,
                                                            int recipe,
                                                            const RedPartial* __restrict__ partials) {
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    const int64_t tid = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    int64_t n4 = vec ? n / 4 : 0;
    const float4* __restrict__ x4 = reinterpret_cast<const float4*>(x);
    int64_t i = tid;
    double inv;
    if constexpr (FUSED) {
        // The partials are loaded first and the first trip of x right after;
        // loads complete in issue order, so waiting for the partials leaves
        // the x loads in flight and the two latencies overlap.  The reduction
        // is reduce_partials' (exact min / max, so its order does not matter).
        // Both groups of loads are issued unconditionally (indices clamped:
        // a repeated partial leaves min / max unchanged; past the float4s of
        // x, or with none, the x loads read a valid dummy), because a branch
        // around either would make the wait for the partials drain both.
        const float x0 = x[0];  // the first-element NaN rule (nan_first)
        constexpr int kPp = kMaxReduceBlocks / kBlock;
        float pmn[kPp], pmx[kPp];
#pragma unroll
        for (int j = 0; j < kPp; j++) {
            const int b = (int)threadIdx.x + j * kBlock;
            const RedPartial* pp = partials + (b < nparts ? b : nparts - 1);
            pmn[j] = pp->mn;
            pmx[j] = pp->mx;
        }
        float4 v0[kUnroll];
        const bool pre = i + (kUnroll - 1) * stride < n4;
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            const int64_t j = i + u * stride < n4 ? i + u * stride : n4 - 1;
            v0[u] = ld4<NT>(n4 > 0 ? x4 + j : reinterpret_cast<const float4*>(partials));
        }
        __builtin_amdgcn_sched_barrier(0);  // every load above is issued before the reduction
        float mn = pmn[0], mx = pmx[0];
#pragma unroll
        for (int j = 1; j < kPp; j++) {
            mn = fminf(mn, pmn[j]);
            mx = fmaxf(mx, pmx[j]);
        }
        __shared__ float s_mn[kBlock / 64], s_mx[kBlock / 64];
        mn = wave_min(mn);
        mx = wave_max(mx);
        if ((threadIdx.x & 63) == 0) {
            s_mn[threadIdx.x >> 6] = mn;
            s_mx[threadIdx.x >> 6] = mx;
        }
        __syncthreads();
        mn = s_mn[0];
        mx = s_mx[0];
        for (int w = 1; w < kBlock / 64; w++) {
            mn = fminf(mn, s_mn[w]);
            mx = fmaxf(mx, s_mx[w]);
        }
        double dmn = mn, dmx = mx;
        if (x0 != x0) dmn = dmx = (double)x0;
        tkv_hip_qparams_dev prm;
        finalize_minmax(dmn, dmx, MM_SYMMETRIC, recipe, &prm);
        inv = prm.inv;
        if (blockIdx.x == 0 && threadIdx.x == 0) *p = prm;
        if (pre) {
            // pins the first use of the early loads here, so the compiler
            // cannot convert them (and wait for them) before the reduction
#pragma unroll
            for (int u = 0; u < kUnroll; u++)
                asm volatile("" : "+v"(v0[u].x), "+v"(v0[u].y), "+v"(v0[u].z), "+v"(v0[u].w));
#pragma unroll
            for (int u = 0; u < kUnroll; u++)
                store4<OUT_I32>(q, i + u * stride, rne_clamp((double)v0[u].x * inv, -127.0, 127.0),
                                rne_clamp((double)v0[u].y * inv, -127.0, 127.0),
                                rne_clamp((double)v0[u].z * inv, -127.0, 127.0),
                                rne_clamp((double)v0[u].w * inv, -127.0, 127.0));
            i += kUnroll * stride;
        }
    } else {
        inv = p->inv;
    }
    for (; i + (kUnroll - 1) * stride < n4; i += kUnroll * stride) {
        float4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; u++) v[u] = ld4<NT>(x4 + i + u * stride);
#pragma unroll
        for (int u = 0; u < kUnroll; u++)
            store4<OUT_I32>(q, i + u * stride, rne_clamp((double)v[u].x * inv, -127.0, 127.0),
                            rne_clamp((double)v[u].y * inv, -127.0, 127.0),
                            rne_clamp((double)v[u].z * inv, -127.0, 127.0),
                            rne_clamp((double)v[u].w * inv, -127.0, 127.0));
    }
    for (; i < n4; i += stride) {
        float4 v = ld4<NT>(x4 + i);
        store4<OUT_I32>(q, i, rne_clamp((double)v.x * inv, -127.0, 127.0),
                        rne_clamp((double)v.y * inv, -127.0, 127.0),
                        rne_clamp((double)v.z * inv, -127.0, 127.0),
                        rne_clamp((double)v.w * inv, -127.0, 127.0));
    }
    for (int64_t j = n4 * 4 + tid; j < n; j += stride)
        store1<OUT_I32>(q, j, rne_clamp((double)x[j] * inv, -127.0, 127.0));
}

// Grid of the float4 streaming kernels; `vec` 0 (misaligned input, one
// element per trip) takes the scalar kernels' wider grid.
static int64_t stream_blocks(Ctx* c, int64_t work, int vec) {
    int64_t blocks = ceil_div(work, (int64_t)kBlock * kUnroll);
    int64_t cap = (int64_t)c->num_cus * (vec ? kBlocksPerCu : 16);
    if (blocks > cap) blocks = cap;
    return blocks < 1 ? 1 : blocks;
}

// Grid for the one-element-per-trip kernels (dequantize, decode, layout
// conversions): enough resident waves to cover the load latency.
static int64_t scalar_blocks(Ctx* c, int64_t work) {
    int64_t blocks = ceil_div(work, (int64_t)kBlock * kUnroll);
    int64_t cap = (int64_t)c->num_cus * 16;
    if (blocks > cap) blocks = cap;
    return blocks < 1 ? 1 : blocks;
}

template <bool FUSED>
static void launch_quant_kernel(Ctx* c, const float* x, int64_t n, tkv_hip_qparams_dev* p,
                                void* q, bool out_i32, int nparts, int recipe) {
    const int vec = (aligned(x, 16) && aligned(q, out_i32 ? 16 : 4)) ? 1 : 0;
    const dim3 grid((unsigned)stream_blocks(c, vec ? n / 4 : n, vec)), block(kBlock);
    const bool nt = n * 4 > kCacheableBytes;
#define TKV_QUANT(OI, NT)                                                                        \
    hipLaunchKernelGGL((k_quant_i8_tensor<OI, FUSED, NT>), grid, block, 0, c->stream, x, n, vec, \
                       p, q, nparts, recipe, c->partials)
    if (out_i32) {
        if (nt) TKV_QUANT(true, true);
        else TKV_QUANT(true, false);
    } else {
        if (nt) TKV_QUANT(false, true);
        else TKV_QUANT(false, false);
    }
#undef TKV_QUANT
}

int launch_quant_i8_tensor(Ctx* c, const float* x, int64_t n, const tkv_hip_qparams_dev* p,
                           void* q, bool out_i32) {
    if (n <= 0) return TKV_HIP_OK;
    auto* pp = const_cast<tkv_hip_qparams_dev*>(p);  // read only when not fused
    launch_quant_kernel<false>(c, x, n, pp, q, out_i32, 0, 0);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

// ---------------------------------------------------------------------------
// Single-pass per-tensor calibrate + quantize for large tensors
// (calibrate_minmax(x, 1), then quantize_int8_symmetric: engine.tkv:13-36,
// 216-226).  One workgroup per CU keeps its share of x on chip: kResRegs
// float4 per thread in registers and kResLds in LDS (filled by direct-to-LDS
// loads), up to 100.7 MB on 256 CUs.  The workgroups exchange their absmax
// through a grid barrier and form the codes from the on-chip copy, so x
// crosses HBM once.  The two-kernel path reads it twice: at 8192 x 3072 it
// takes 17.9 + 20.7 us, this kernel ~26 us (timestamped probe: loads 15-16
// us at 6.3-6.8 TB/s, barrier ~3 us, codes ~7 us).  For a 25 MB tensor the
// two were equal, so the kernel is used from kResMinElems up.
//
// Symmetric calibration needs only max(|min|, |max|), the absmax of the
// elements that are not NaN (fmaxf skips NaN, as the reference's strict
// comparisons do); nan_first applies the reference's NaN-first-element rule,
// so the QuantParams equal the two-kernel path's bit for bit.
//
// The barrier is a slot array in context memory: workgroup b owns the 64-bit
// slot b = (generation << 32) | absmax bits.  It reads its own slot and
// stores the next generation with its absmax (one relaxed agent-scope atomic
// store).  Workgroup 0 polls every slot until all carry that generation,
// takes the max of their absmaxes and stores it, with the generation, in the
// result word (the last slot); the other workgroups poll only that word.
// Every launch advances every slot by one, so the slots hold equal
// generations whenever no launch is running, and a replayed graph needs
// nothing from the host.  Data and flag are one atomic word, performed at
// the device coherence point: no fences, no cache maintenance, and no shared
// counter (256 agent-scope adds on one word serialize, ~10 us).  The grid is
// one workgroup per CU (the LDS share leaves room for no second), so every
// workgroup is resident once the CUs are free of earlier work.  The wait is
// bounded all the same: a workgroup that gives up (kResSpin polls, or the
// context's TKV_HIP_TUNE_GRID_SPIN override) takes the absmax of the whole
// tensor itself, which gives the same scale (max is exact in any order), so
// the result never depends on the barrier completing and no workgroup can
// wait forever.
// ---------------------------------------------------------------------------
constexpr int kResBlock = 768;
constexpr int kResRegs = 19;   // float4 per thread in registers (164 VGPRs in all)
constexpr int kResLds = 13;    // float4 per thread in LDS (159,744 bytes)
constexpr int kResSpin = 1 << 20;
constexpr int64_t kResMinElems = 16ll << 20;  // 64 MB of f32

__device__ __forceinline__ float absmax4(float m, const float4 v) {
    return fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
}

// Block-wide max of a non-negative value, returned to every thread.
__device__ __forceinline__ float block_max_res(float v, float* s) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_max(v);
    __syncthreads();  // s free from any earlier use
    if (lane == 0) s[wave] = v;
    __syncthreads();
    float r = s[0];
#pragma unroll
    for (int w = 1; w < kResBlock / 64; w++) r = fmaxf(r, s[w]);
    return r;
}

template <bool OUT_I32>
__global__ __launch_bounds__(kResBlock, 3) void k_quant_i8_resident(
    const float* __restrict__ x, int64_t n, tkv_hip_qparams_dev* __restrict__ p,
    void* __restrict__ q, int recipe, unsigned long long* __restrict__ slots, int spin) {
    __shared__ float4 s_x[kResLds * kResBlock];
    __shared__ float s_red[kResBlock / 64];
    __shared__ float s_all;
    __shared__ int s_ok;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t n4 = n / 4;
    const int64_t stride = (int64_t)gridDim.x * kResBlock;
    const int64_t tid = (int64_t)blockIdx.x * kResBlock + threadIdx.x;
    const float4* __restrict__ x4 = reinterpret_cast<const float4*>(x);
    float4 v[kResRegs];
#pragma unroll
    for (int u = 0; u < kResRegs; u++) {
        const int64_t i = tid + u * stride;
        v[u] = i < n4 ? ld4<true>(x4 + i) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    // the LDS share: lane l's 16 bytes land at s_x[u * kResBlock + 64 * wave + l]
#pragma unroll
    for (int u = 0; u < kResLds; u++) {
        int64_t i = tid + (kResRegs + u) * stride;
        if (i >= n4) i = n4 - 1;  // in bounds; the element is not used
        __builtin_amdgcn_global_load_lds(
            (const void*)(x4 + i),
            (__attribute__((address_space(3))) void*)(s_x + u * kResBlock + 64 * wave), 16, 0, 0);
    }
    float am = 0.0f;
#pragma unroll
    for (int u = 0; u < kResRegs; u++) am = absmax4(am, v[u]);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's LDS share has landed
#pragma unroll
    for (int u = 0; u < kResLds; u++)
        if (tid + (kResRegs + u) * stride < n4) am = absmax4(am, s_x[u * kResBlock + threadIdx.x]);
    am = block_max_res(am, s_red);
    if (wave == 0) {
        unsigned gen = 0;
        if (lane == 0) {
            unsigned long long* mine = slots + blockIdx.x;
            gen = (unsigned)(__hip_atomic_load(mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >> 32) + 1u;
            __hip_atomic_store(mine, ((unsigned long long)gen << 32) | __float_as_uint(am),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        gen = __shfl(gen, 0, 64);
        unsigned long long* result = slots + (kMaxGridSlots - 1);
        float g = 0.0f;
        int ok = 0;
        if (blockIdx.x == 0) {
            // the leader gathers every slot, then publishes the max
            for (int it = 0; it < spin; it++) {
                int ready = 1;
                float gg = 0.0f;
                for (int b = lane; b < (int)gridDim.x; b += 64) {
                    const unsigned long long sv =
                        __hip_atomic_load(slots + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    ready &= (unsigned)(sv >> 32) == gen;
                    gg = fmaxf(gg, __uint_as_float((unsigned)sv));
                }
                if (__all(ready)) {
                    g = wave_max(gg);
                    ok = 1;
                    break;
                }
            }
            if (ok && lane == 0)
                __hip_atomic_store(result, ((unsigned long long)gen << 32) | __float_as_uint(g),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else if (lane == 0) {
            for (int it = 0; it < spin; it++) {
                const unsigned long long rv =
                    __hip_atomic_load(result, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if ((unsigned)(rv >> 32) == gen) {
                    g = __uint_as_float((unsigned)rv);
                    ok = 1;
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
        }
        if (lane == 0) {
            s_all = g;
            s_ok = ok;
        }
    }
    __syncthreads();
    float g = s_all;
    if (!s_ok) {
        // barrier gave up: the absmax of the whole tensor, read by this workgroup
        g = 0.0f;
        for (int64_t i = threadIdx.x; i < n4; i += kResBlock) g = absmax4(g, ld4<true>(x4 + i));
        g = block_max_res(g, s_red);
    }
    double dmn = 0.0, dmx = (double)g;
    nan_first(x, dmn, dmx);
    tkv_hip_qparams_dev prm;
    finalize_minmax(dmn, dmx, MM_SYMMETRIC, recipe, &prm);
    const double inv = prm.inv;
    if (blockIdx.x == 0 && threadIdx.x == 0) *p = prm;
    auto store_codes = [&](auto&& code) {
#pragma unroll
        for (int u = 0; u < kResRegs; u++) {
            const int64_t i = tid + u * stride;
            if (i < n4)
                store4<OUT_I32>(q, i, code(v[u].x), code(v[u].y), code(v[u].z), code(v[u].w));
        }
#pragma unroll
        for (int u = 0; u < kResLds; u++) {
            const int64_t i = tid + (kResRegs + u) * stride;
            if (i < n4) {
                const float4 w = s_x[u * kResBlock + threadIdx.x];
                store4<OUT_I32>(q, i, code(w.x), code(w.y), code(w.z), code(w.w));
            }
        }
    };
    // The store phase is VALU-bound: with an f32 reciprocal (the primary
    // recipe's fl32(1 / scale)) the codes take the f32 form of the rounding
    // (8192 x 3072: ~1.5 us per call less in a timing probe with a cheaper
    // rounding); otherwise the f64 one.
    const float invf = (float)inv;
    if ((double)invf == inv)
        store_codes([&](float a) { return rne_clamp127_f32(a, invf); });
    else
        store_codes([&](float a) { return rne_clamp((double)a * inv, -127.0, 127.0); });
}

// TKV_HIP_UNSUPPORTED when the tensor is outside the single-pass kernel's
// range (size, alignment, a tail of fewer than 4 elements) or the context
// has no barrier slots.
static int launch_quant_i8_resident(Ctx* c, const float* x, int64_t n, int recipe,
                                    tkv_hip_qparams_dev* p, void* q, bool out_i32) {
    const int64_t g = c->num_cus;
    if (!c->grid_slots || g > kMaxGridSlots - 1 || n < kResMinElems || n % 4 != 0 ||
        !aligned(x, 16) || !aligned(q, out_i32 ? 16 : 4) ||
        n / 4 > g * kResBlock * (kResRegs + kResLds))
        return TKV_HIP_UNSUPPORTED;
    const int spin = tuned(c, TKV_HIP_TUNE_GRID_SPIN) >= 0 ? (int)tuned(c, TKV_HIP_TUNE_GRID_SPIN)
                                                           : kResSpin;
    if (out_i32)
        hipLaunchKernelGGL((k_quant_i8_resident<true>), dim3((unsigned)g), dim3(kResBlock), 0,
                           c->stream, x, n, p, q, recipe, c->grid_slots, spin);
    else
        hipLaunchKernelGGL((k_quant_i8_resident<false>), dim3((unsigned)g), dim3(kResBlock), 0,
                           c->stream, x, n, p, q, recipe, c->grid_slots, spin);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

// calibrate_minmax(x, 1) then quantize_int8_symmetric(x, q, scale): the
// single-pass kernel for large tensors that fit it, else two kernels
// (per-CU partials, then the quantize kernel finalizing the scale in every
// block).  *p receives the QuantParams.
int launch_quant_i8_dynamic(Ctx* c, const float* x, int64_t n, int recipe,
                            tkv_hip_qparams_dev* p, void* q, bool out_i32) {
    if (n <= 0) return launch_minmax_tensor(c, x, n, MM_SYMMETRIC, recipe, p);
    if (tuned(c, TKV_HIP_TUNE_QUANT_TWO_PASS) != 1) {
        const int rc = launch_quant_i8_resident(c, x, n, recipe, p, q, out_i32);
        if (rc != TKV_HIP_UNSUPPORTED) return rc;
    }
    int64_t nparts;
    TKV_RC_TRY(launch_partials(c, x, n, 0, &nparts));
    launch_quant_kernel<true>(c, x, n, p, q, out_i32, (int)nparts, recipe);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

// ---------------------------------------------------------------------------
// Row kernels: one wave64 per row.
//   RM_DYNAMIC        quantize_dynamic_int8_rowwise   engine.tkv:266-285
//   RM_PER_CHANNEL    quantize_int8_per_channel       engine.tkv:237-250
//   RM_CALIBRATE      symmetric per-row scales        engine.tkv:202-213
//   RM_CALIBRATE_FULL calibrate_minmax per row (both modes), full params
// The second pass re-reads the row from cache (rows are 3-12 KB).
// ---------------------------------------------------------------------------
template <bool OUT_I32>
__global__ __launch_bounds__(kBlock) void k_rows(const float* __restrict__ x, int64_t rows,
                                                 int64_t cols, int vec, int mode,
                                                 const float* __restrict__ scales_in,
                                                 void* __restrict__ q,
                                                 float* __restrict__ scales_out,
                                                 tkv_hip_qparams_dev* __restrict__ row_params,
                                                 int symmetric) {
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
    if (r >= rows) return;
    const float* __restrict__ xr = x + r * cols;
    double inv = 0.0;
    if (mode != RM_PER_CHANNEL) {
        float mn = FLT_MAX * 2.0f, mx = -FLT_MAX * 2.0f;
        unsigned long long zi = ~0ull;
        const bool tz = (mode == RM_CALIBRATE_FULL && !symmetric);
        if (vec) {
            const float4* __restrict__ x4 = reinterpret_cast<const float4*>(xr);
            for (int64_t c4 = lane; c4 < cols / 4; c4 += 64) {
                float4 v = x4[c4];
                mm_acc(v.x, c4 * 4 + 0, tz, mn, mx, zi);
                mm_acc(v.y, c4 * 4 + 1, tz, mn, mx, zi);
                mm_acc(v.z, c4 * 4 + 2, tz, mn, mx, zi);
                mm_acc(v.w, c4 * 4 + 3, tz, mn, mx, zi);
            }
        } else {
            for (int64_t c = lane; c < cols; c += 64) mm_acc(xr[c], c, tz, mn, mx, zi);
        }
        mn = wave_min(mn);
        mx = wave_max(mx);
        double dmn = mn, dmx = mx;
        if (mode == RM_CALIBRATE_FULL) {
            zi = wave_min_u64(zi);
            if (lane == 0) {
                if (tz && zi != ~0ull) {
                    double z = xr[zi];
                    if (mn == 0.0f) dmn = z;
                    if (mx == 0.0f) dmx = z;
                }
                nan_first(xr, dmn, dmx);
                finalize_minmax(dmn, dmx, symmetric ? MM_SYMMETRIC : MM_ASYMMETRIC,
                                TKV_HIP_RECIPE_PRIMARY, row_params + r);
            }
            return;
        }
        double am;
        if (mode == RM_CALIBRATE) {
            // calibrate_minmax per row: the row's first element seeds min / max.
            nan_first(xr, dmn, dmx);
            am = fabs(dmx);
            if (fabs(dmn) > am) am = fabs(dmn);
        } else {
            // RM_DYNAMIC: am = max |x| from 0 (engine.tkv:272-276), so NaN is
            // skipped and a row of NaN only gives 0 (min +inf > max -inf).
            am = mn <= mx ? fmax(fabs(dmn), fabs(dmx)) : 0.0;
        }
        if (am < 0.00000001) am = 0.00000001;
        double sc = am / 127.0;
        if (mode == RM_CALIBRATE) {
            if (lane == 0) scales_out[r] = (float)sc;
            return;
        }
        if (lane == 0) scales_out[r] = (float)sc;  // RM_DYNAMIC
        inv = 1.0 / sc;
    } else {
        double sc = (double)scales_in[r];
        if (sc <= 0.00000001) sc = 0.00000001;
        inv = 1.0 / sc;
    }
    if (vec) {
        const float4* __restrict__ x4 = reinterpret_cast<const float4*>(xr);
        const int64_t base4 = r * (cols / 4);
        for (int64_t c4 = lane; c4 < cols / 4; c4 += 64) {
            float4 v = x4[c4];
            store4<OUT_I32>(q, base4 + c4, rne_clamp((double)v.x * inv, -127.0, 127.0),
                            rne_clamp((double)v.y * inv, -127.0, 127.0),
                            rne_clamp((double)v.z * inv, -127.0, 127.0),
                            rne_clamp((double)v.w * inv, -127.0, 127.0));
        }
    } else {
        for (int64_t c = lane; c < cols; c += 64)
            store1<OUT_I32>(q, r * cols + c, rne_clamp((double)xr[c] * inv, -127.0, 127.0));
    }
}

// quantize_dynamic_int8_rowwise (engine.tkv:266-285) with the row held in
// registers: each wave64 walks rows r, r + waves, ... with C4 float4 per
// lane (lane + 64 c), so every row is read from HBM once; with PIPE the next
// row's loads are issued before the current row is reduced and quantized.
// Same numerics as k_rows' RM_DYNAMIC branch.
//
// The loop body is kept free of branches so the next row's loads stay in
// flight while the current row is processed (a load or store under a lane
// guard makes the wait before the current row's first use drain every
// outstanding load and store):
//  * FULL (cols / 4 == 64 * C4): every lane owns C4 float4, no guard at all;
//  * otherwise lanes past the row end load the row's last float4 again
//    (a duplicate element leaves the row's min and max unchanged) and only
//    the stores are guarded;
//  * the prefetch past the last row re-reads row rows - 1;
//  * every lane stores the row's scale (one value, one address).
template <int C4, bool FULL>
__device__ __forceinline__ void load_row(const float* x, int64_t r, int64_t cols,
                                         int lane, float4 (&v)[C4]) {
    const int64_t cols4 = cols / 4;
    const float4* xr = reinterpret_cast<const float4*>(x + r * cols);
#pragma unroll
    for (int c = 0; c < C4; c++) {
        int64_t i = lane + 64 * c;
        if constexpr (!FULL) i = i < cols4 ? i : cols4 - 1;
        v[c] = ld4<true>(xr + i);
    }
}

template <int C4, bool FULL, bool OUT_I32>
__device__ __forceinline__ void quant_row(const float4 (&v)[C4], int64_t r, int64_t cols, int lane,
                                          void* q, float* scales_out) {
    const int64_t cols4 = cols / 4;
    // am = max |x| from 0 (engine.tkv:272-276): fmaxf skips NaN as the
    // reference's strict comparison does, and a row of NaN gives 0.
    float al = 0.0f;
#pragma unroll
    for (int c = 0; c < C4; c++)
        al = fmaxf(fmaxf(al, fabsf(v[c].x)),
                   fmaxf(fabsf(v[c].y), fmaxf(fabsf(v[c].z), fabsf(v[c].w))));
    double am = (double)wave_max_nonneg(al);
    if (am < 0.00000001) am = 0.00000001;
    const double sc = am / 127.0;
    if (lane == 0) scales_out[r] = (float)sc;
    const double inv = 1.0 / sc;
    const int64_t base4 = r * cols4;
#pragma unroll
    for (int c = 0; c < C4; c++)
        if (FULL || lane + 64 * c < cols4)
            store4<OUT_I32>(q, base4 + lane + 64 * c, rne_clamp((double)v[c].x * inv, -127.0, 127.0),
                            rne_clamp((double)v[c].y * inv, -127.0, 127.0),
                            rne_clamp((double)v[c].z * inv, -127.0, 127.0),
                            rne_clamp((double)v[c].w * inv, -127.0, 127.0));
}

template <int C4, bool FULL, bool OUT_I32, bool PIPE>
__global__ __launch_bounds__(kBlock) void k_rows_dynamic(const float* x, int64_t rows,
                                                         int64_t cols, void* q,
                                                         float* scales_out) {
    const int lane = threadIdx.x & 63;
    const int64_t nw = (int64_t)gridDim.x * (kBlock / 64);
    const int64_t r0 = (int64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
    if (r0 >= rows) return;
    float4 a[C4];
    load_row<C4, FULL>(x, r0, cols, lane, a);
    if constexpr (PIPE) {
        // Two register sets in turn: each row's loads are issued one row
        // ahead and no copy between the sets waits on them.  The pointers
        // are deliberately not __restrict__: the row's stores may then alias
        // the input, which keeps the compiler from sinking the prefetch below
        // them.  The loop is entered after the first row so that at its head
        // the same memory operations are outstanding on both incoming paths
        // (the next row's loads, then this row's stores), and the wait for
        // the next row need not drain the stores.
        float4 b[C4];
        load_row<C4, FULL>(x, r0 + nw < rows ? r0 + nw : rows - 1, cols, lane, b);
        quant_row<C4, FULL, OUT_I32>(a, r0, cols, lane, q, scales_out);
        for (int64_t r = r0 + nw; r < rows; r += 2 * nw) {
            load_row<C4, FULL>(x, r + nw < rows ? r + nw : rows - 1, cols, lane, a);
            quant_row<C4, FULL, OUT_I32>(b, r, cols, lane, q, scales_out);
            if (r + nw >= rows) break;
            load_row<C4, FULL>(x, r + 2 * nw < rows ? r + 2 * nw : rows - 1, cols, lane, b);
            quant_row<C4, FULL, OUT_I32>(a, r + nw, cols, lane, q, scales_out);
        }
    } else {
        for (int64_t r = r0; r < rows; r += nw) {
            if (r != r0) load_row<C4, FULL>(x, r, cols, lane, a);
            quant_row<C4, FULL, OUT_I32>(a, r, cols, lane, q, scales_out);
        }
    }
}

template <bool OUT_I32>
static bool launch_rows_dynamic(Ctx* c, const float* x, int64_t rows, int64_t cols, void* q,
                                float* scales_out) {
    const int64_t per_lane = ceil_div(cols / 4, 64);
    int64_t blocks = ceil_div(rows, kBlock / 64);
    // 2 to 24 blocks per CU all measured 42.2-44.5 us at 65536 x 768 (one
    // box, three interleaved rounds): the grid is not what limits it
    const int64_t cap = (int64_t)c->num_cus * 8;
    if (blocks > cap) blocks = cap;
    const dim3 grid((unsigned)blocks), block(kBlock);
#define TKV_ROWS_DYN(C4, PIPE)                                                                 \
    do {                                                                                       \
        if (cols / 4 == 64 * (C4))                                                             \
            hipLaunchKernelGGL((k_rows_dynamic<C4, true, OUT_I32, PIPE>), grid, block, 0,      \
                               c->stream, x, rows, cols, q, scales_out);                       \
        else                                                                                   \
            hipLaunchKernelGGL((k_rows_dynamic<C4, false, OUT_I32, PIPE>), grid, block, 0,     \
                               c->stream, x, rows, cols, q, scales_out);                       \
    } while (0)
    if (per_lane <= 1) TKV_ROWS_DYN(1, true);
    else if (per_lane <= 2) TKV_ROWS_DYN(2, true);
    else if (per_lane <= 3) TKV_ROWS_DYN(3, true);
    else if (per_lane <= 4) TKV_ROWS_DYN(4, true);
    else if (per_lane <= 6) TKV_ROWS_DYN(6, true);
    else if (per_lane <= 8) TKV_ROWS_DYN(8, false);
    else if (per_lane <= 12) TKV_ROWS_DYN(12, false);
    else if (per_lane <= 16) TKV_ROWS_DYN(16, false);
    else return false;
#undef TKV_ROWS_DYN
    return true;
}

int launch_quant_rows(Ctx* c, const float* x, int64_t rows, int64_t cols, int mode,
                      const float* scales_in, void* q, bool out_i32, float* scales_out,
                      tkv_hip_qparams_dev* row_params, int symmetric) {
    if (rows <= 0 || cols <= 0) return TKV_HIP_OK;
    bool q_ok = (mode == RM_CALIBRATE || mode == RM_CALIBRATE_FULL) ? true
                                                                     : aligned(q, out_i32 ? 16 : 4);
    int vec = (cols % 4 == 0 && aligned(x, 16) && q_ok) ? 1 : 0;
    if (mode == RM_DYNAMIC && vec) {
        const bool done = out_i32 ? launch_rows_dynamic<true>(c, x, rows, cols, q, scales_out)
                                  : launch_rows_dynamic<false>(c, x, rows, cols, q, scales_out);
        if (done) {
            TKV_LAUNCH_CHECK();
            return TKV_HIP_OK;
        }
    }
    int64_t blocks = ceil_div(rows, kBlock / 64);
    if (out_i32)
        hipLaunchKernelGGL(k_rows<true>, dim3((unsigned)blocks), dim3(kBlock), 0, c->stream, x,
                           rows, cols, vec, mode, scales_in, q, scales_out, row_params, symmetric);
    else
        hipLaunchKernelGGL(k_rows<false>, dim3((unsigned)blocks), dim3(kBlock), 0, c->stream, x,
                           rows, cols, vec, mode, scales_in, q, scales_out, row_params, symmetric);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

// ---------------------------------------------------------------------------
// Dequantize: y = fl32(q * s) with the product in f64 (engine.tkv:229-262).
// ---------------------------------------------------------------------------
template <bool IN_I32>
__global__ __launch_bounds__(kBlock) void k_dequant_i8(const void* __restrict__ q, int64_t rows,
                                                       int64_t cols, float scale,
                                                       const float* __restrict__ scales,
                                                       float* __restrict__ y) {
    const int64_t n = rows * cols;
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        int v = IN_I32 ? reinterpret_cast<const int32_t*>(q)[i]
                       : (int)reinterpret_cast<const int8_t*>(q)[i];
        float s = scales ? scales[i / cols] : scale;
        y[i] = (float)((double)v * (double)s);
    }
}

int launch_dequant_i8(Ctx* c, const void* q, bool in_i32, int64_t rows, int64_t cols,
                      float scale, const float* scales, float* y) {
    int64_t n = rows * cols;
    if (n <= 0) return TKV_HIP_OK;
    int64_t blocks = scalar_blocks(c, n / 4 + 1);
    if (in_i32)
        hipLaunchKernelGGL(k_dequant_i8<true>, dim3((unsigned)blocks), dim3(kBlock), 0, c->stream,
                           q, rows, cols, scale, scales, y);
    else
        hipLaunchKernelGGL(k_dequant_i8<false>, dim3((unsigned)blocks), dim3(kBlock), 0,
                           c->stream, q, rows, cols, scale, scales, y);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

// ---------------------------------------------------------------------------
// e4m3 encode (matmul.tkv:60-66 / types.tkv:154-191).  Raw bytes out, or the
// reference's int32 codes (byte - 128).  With `scaled` the input is first
// multiplied by fl32(1 / scale) in f32 (extension for per-tensor FP8).
// ---------------------------------------------------------------------------
// Four packed e4m3 bytes (element 0 in bits 7:0) as raw bytes (FP8_BYTES),
// as the reference's int32 codes (byte - 128, FP8_I32), or as their exact
// reference decode in f16, pre-scaled by 2^-8 (FP8_F16: what the
// reference-products GEMM multiplies).
enum { FP8_BYTES = 0, FP8_I32 = 1, FP8_F16 = 2 };

template <int OUT>
__device__ __forceinline__ void store_fp8x4(void* q, int64_t i4, uint32_t w) {
    if constexpr (OUT == FP8_I32)
        reinterpret_cast<int4*>(q)[i4] =
            make_int4((int)(w & 0xffu) - 128, (int)((w >> 8) & 0xffu) - 128,
                      (int)((w >> 16) & 0xffu) - 128, (int)(w >> 24) - 128);
    else if constexpr (OUT == FP8_F16)
        reinterpret_cast<uint2*>(q)[i4] =
            make_uint2(gemm::dec2_f16(__builtin_amdgcn_perm(0u, w, 0x0c010c00u)),
                       gemm::dec2_f16(__builtin_amdgcn_perm(0u, w, 0x0c030c02u)));
    else
        reinterpret_cast<uint32_t*>(q)[i4] = w;
}

template <int OUT>
__device__ __forceinline__ void store_fp8x1(void* q, int64_t j, uint32_t e) {
    if constexpr (OUT == FP8_I32)
        reinterpret_cast<int32_t*>(q)[j] = (int)e - 128;
    else if constexpr (OUT == FP8_F16)
        reinterpret_cast<uint16_t*>(q)[j] = (uint16_t)(gemm::dec2_f16(e) & 0xffffu);
    else
        reinterpret_cast<uint8_t*>(q)[j] = (uint8_t)e;
}

template <int OUT>
__global__ __launch_bounds__(kBlock) void k_fp8_encode(const float* __restrict__ x, int64_t n,
                                                       int vec,
                                                       const tkv_hip_qparams_dev* __restrict__ sp,
                                                       void* __restrict__ q) {
    const float mul = sp ? 1.0f / sp->scale : 1.0f;
    const bool scaled = sp != nullptr;
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    const int64_t tid = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    int64_t n4 = vec ? n / 4 : 0;
    const float4* __restrict__ x4 = reinterpret_cast<const float4*>(x);
    int64_t i = tid;
    for (; i + (kUnroll - 1) * stride < n4; i += kUnroll * stride) {
        float4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; u++) v[u] = ld4(x4 + i + u * stride);
        uint32_t w[kUnroll];
        int special = 0;
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            if (scaled) {
                v[u].x *= mul;
                v[u].y *= mul;
                v[u].z *= mul;
                v[u].w *= mul;
            }
            special |= (int)e4m3_special(v[u].x) | (int)e4m3_special(v[u].y) |
                       (int)e4m3_special(v[u].z) | (int)e4m3_special(v[u].w);
            w[u] = e4m3_encode4_finite(v[u].x, v[u].y, v[u].z, v[u].w);
        }
        if (special) {  // +-inf or NaN in this lane's trip: the patched form
#pragma unroll
            for (int u = 0; u < kUnroll; u++) w[u] = e4m3_encode4(v[u].x, v[u].y, v[u].z, v[u].w);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; u++) store_fp8x4<OUT>(q, i + u * stride, w[u]);
    }
    for (; i < n4; i += stride) {
        float4 v = ld4(x4 + i);
        if (scaled) {
            v.x *= mul;
            v.y *= mul;
            v.z *= mul;
            v.w *= mul;
        }
        store_fp8x4<OUT>(q, i, e4m3_encode4(v.x, v.y, v.z, v.w));
    }
    for (int64_t j = n4 * 4 + tid; j < n; j += stride) {
        float v = x[j];
        if (scaled) v *= mul;
        store_fp8x1<OUT>(q, j, e4m3_encode1(v));
    }
}

static int launch_fp8_encode_as(Ctx* c, const float* x, int64_t n,
                                const tkv_hip_qparams_dev* scaled, void* q, int out) {
    if (n <= 0) return TKV_HIP_OK;
    const int qalign = out == FP8_I32 ? 16 : (out == FP8_F16 ? 8 : 4);
    int vec = (aligned(x, 16) && aligned(q, qalign)) ? 1 : 0;
    // The e4m3 encode costs more ALU work per element than the int8 quantize
    // (~11 operations per element: the magnitude clamps in front of the
    // hardware conversion): three blocks per CU overlap it with the loads at
    // least as well as two, and better than four (at 201 MB: 41.6-42.7 us
    // against 41.4-43.6 / 46.2-47.0 us, three interleaved rounds on one box).
    // Four float4 per thread per trip: 42.6 us median against 43.4 / 43.8 us
    // with two / eight (four interleaved rounds on one box).
    int64_t blocks = ceil_div(vec ? n / 4 : n, (int64_t)kBlock * kUnroll);
    const int64_t cap = (int64_t)c->num_cus * (vec ? 3 : 16);
    if (blocks > cap) blocks = cap;
    if (blocks < 1) blocks = 1;
    if (out == FP8_I32)
        hipLaunchKernelGGL(k_fp8_encode<FP8_I32>, dim3((unsigned)blocks), dim3(kBlock), 0,
                           c->stream, x, n, vec, scaled, q);
    else if (out == FP8_F16)
        hipLaunchKernelGGL(k_fp8_encode<FP8_F16>, dim3((unsigned)blocks), dim3(kBlock), 0,
                           c->stream, x, n, vec, scaled, q);
    else
        hipLaunchKernelGGL(k_fp8_encode<FP8_BYTES>, dim3((unsigned)blocks), dim3(kBlock), 0,
                           c->stream, x, n, vec, scaled, q);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

int launch_fp8_encode(Ctx* c, const float* x, int64_t n, const tkv_hip_qparams_dev* scaled,
                      void* q, bool out_i32) {
    return launch_fp8_encode_as(c, x, n, scaled, q, out_i32 ? FP8_I32 : FP8_BYTES);
}

// Per-tensor FP8 activation quantize: the MM_FP8 scale, then the scaled
// encode reading it from *p.
int launch_quant_fp8_dynamic(Ctx* c, const float* x, int64_t n, tkv_hip_qparams_dev* p, void* q,
                             bool out_i32) {
    TKV_RC_TRY(launch_minmax_tensor(c, x, n, MM_FP8, TKV_HIP_RECIPE_PRIMARY, p));
    return launch_fp8_encode(c, x, n, p, q, out_i32);
}

// The same, writing the codes' reference decode in f16 (for the
// reference-products GEMM) instead of the codes.
int launch_quant_fp8_dynamic_f16(Ctx* c, const float* x, int64_t n, tkv_hip_qparams_dev* p,
                                 void* h16) {
    TKV_RC_TRY(launch_minmax_tensor(c, x, n, MM_FP8, TKV_HIP_RECIPE_PRIMARY, p));
    return launch_fp8_encode_as(c, x, n, p, h16, FP8_F16);
}

template <bool IN_I32>
__global__ __launch_bounds__(kBlock) void k_fp8_decode(const void* __restrict__ q, int64_t n,
                                                       float* __restrict__ y) {
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        uint32_t v = IN_I32 ? (uint32_t)(reinterpret_cast<const int32_t*>(q)[i] + 128)
                            : (uint32_t)reinterpret_cast<const uint8_t*>(q)[i];
        y[i] = e4m3_decode_ref(v & 0xffu);
    }
}

int launch_fp8_decode(Ctx* c, const void* q, bool in_i32, int64_t n, float* y) {
    if (n <= 0) return TKV_HIP_OK;
    int64_t blocks = scalar_blocks(c, n / 4 + 1);
    if (in_i32)
        hipLaunchKernelGGL(k_fp8_decode<true>, dim3((unsigned)blocks), dim3(kBlock), 0, c->stream,
                           q, n, y);
    else
        hipLaunchKernelGGL(k_fp8_decode<false>, dim3((unsigned)blocks), dim3(kBlock), 0,
                           c->stream, q, n, y);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

// ---------------------------------------------------------------------------
// Row sums of int8 codes (the zero-point corrections of QLinearMatMul): rows
// [0, rows_a) of A into out_a, then rows [0, rows_w) of W into out_w, in one
// launch.  With 16-byte
// rows (cols % 16 == 0, aligned) a wave64 sums R rows, 64 / R lanes each;
// each lane issues up to four 16-byte loads at once and adds their bytes with
// v_dot4_i32_i8 against 0x01010101.  Otherwise one wave per row, byte by
// byte.  A row sum is at most 128 * cols in magnitude, exact in int32.
// ---------------------------------------------------------------------------
template <int R>  // rows per wave (64 / R lanes each) in the 16-byte form
__global__ __launch_bounds__(kBlock) void k_row_sums_i8(const int8_t* __restrict__ a,
                                                        int64_t rows_a,
                                                        const int8_t* __restrict__ w,
                                                        int64_t rows_w, int64_t cols, int vec,
                                                        int32_t* __restrict__ out_a,
                                                        int32_t* __restrict__ out_w) {
    constexpr int L = 64 / R;
    const int lane = threadIdx.x & 63;
    const int64_t wave = (int64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
    const int64_t r = vec ? wave * R + lane / L : wave;
    const int64_t rows = rows_a + rows_w;
    const bool live = r < rows;
    const int8_t* __restrict__ row =
        !live ? a : (r < rows_a ? a + r * cols : w + (r - rows_a) * cols);
    int sum = 0;
    if (vec) {
        const v4i* __restrict__ r16 = reinterpret_cast<const v4i*>(row);
        const int64_t n16 = live ? cols / 16 : 0;
        const int sub = lane % L;
        for (int64_t c0 = 0; c0 < n16; c0 += 4 * L) {
            v4i v[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int64_t c = c0 + sub + u * L;
                v[u] = c < n16 ? r16[c] : v4i{0, 0, 0, 0};
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                sum = __builtin_amdgcn_sdot4(v[u].x, 0x01010101, sum, false);
                sum = __builtin_amdgcn_sdot4(v[u].y, 0x01010101, sum, false);
                sum = __builtin_amdgcn_sdot4(v[u].z, 0x01010101, sum, false);
                sum = __builtin_amdgcn_sdot4(v[u].w, 0x01010101, sum, false);
            }
        }
#pragma unroll
        for (int o = L / 2; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
        if (live && lane % L == 0) (r < rows_a ? out_a + r : out_w + (r - rows_a))[0] = sum;
    } else {
        if (!live) return;
        for (int64_t c = lane; c < cols; c += 64) sum += row[c];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
        if (lane == 0) (r < rows_a ? out_a + r : out_w + (r - rows_a))[0] = sum;
    }
}

int launch_row_sums_i8(Ctx* c, const int8_t* a, int64_t rows_a, const int8_t* w, int64_t rows_w,
                       int64_t cols, int32_t* out_a, int32_t* out_w) {
    const int64_t rows = rows_a + rows_w;
    if (rows <= 0) return TKV_HIP_OK;
    const int vec = (cols % 16 == 0 && aligned(a, 16) && aligned(w, 16)) ? 1 : 0;
    // Rows of up to 1 KB take 16 lanes and rows of up to 2 KB 32 lanes: a
    // wave then sums several rows and each lane issues all its loads (at
    // most four) at once.  Longer rows take a whole wave: 32 lanes with two
    // rounds of loads measured slower at 3 KB rows (6.1 against 5.0 us).
    const int R = !vec ? 1 : (cols <= 1024 ? 4 : (cols <= 2048 ? 2 : 1));
    const int64_t waves = ceil_div(rows, (int64_t)R);
    const dim3 grid((unsigned)ceil_div(waves, kBlock / 64)), block(kBlock);
    if (R == 4)
        hipLaunchKernelGGL(k_row_sums_i8<4>, grid, block, 0, c->stream, a, rows_a, w, rows_w, cols,
                           vec, out_a, out_w);
    else if (R == 2)
        hipLaunchKernelGGL(k_row_sums_i8<2>, grid, block, 0, c->stream, a, rows_a, w, rows_w, cols,
                           vec, out_a, out_w);
    else
        hipLaunchKernelGGL(k_row_sums_i8<1>, grid, block, 0, c->stream, a, rows_a, w, rows_w, cols,
                           vec, out_a, out_w);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

// ---------------------------------------------------------------------------
// Code layout conversions for the host mirrors: int32 codes (List<int>) to
// packed int8 rows with a padded leading dimension, and back.  code_bias
// +128 maps the reference's FP8 codes to raw e4m3 bytes.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void k_i32_to_i8(const int32_t* __restrict__ src,
                                                      int64_t rows, int64_t cols, int64_t ld_src,
                                                      int8_t* __restrict__ dst, int64_t ld_dst,
                                                      int code_bias) {
    const int64_t n = rows * ld_dst;
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        int64_t r = i / ld_dst, cidx = i - r * ld_dst;
        int v = cidx < cols ? src[r * ld_src + cidx] + code_bias : 0;
        dst[i] = (int8_t)v;
    }
}

int launch_i32_to_i8(Ctx* c, const int32_t* src, int64_t rows, int64_t cols, int64_t ld_src,
                     int8_t* dst, int64_t ld_dst, int code_bias) {
    int64_t n = rows * ld_dst;
    if (n <= 0) return TKV_HIP_OK;
    int64_t blocks = scalar_blocks(c, n / 4 + 1);
    hipLaunchKernelGGL(k_i32_to_i8, dim3((unsigned)blocks), dim3(kBlock), 0, c->stream, src, rows,
                       cols, ld_src, dst, ld_dst, code_bias);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

__global__ __launch_bounds__(kBlock) void k_i8_to_i32(const int8_t* __restrict__ src, int64_t n,
                                                      int32_t* __restrict__ dst, int code_bias) {
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride)
        dst[i] = (int32_t)src[i] + code_bias;
}

int launch_i8_to_i32(Ctx* c, const int8_t* src, int64_t n, int32_t* dst, int code_bias) {
    if (n <= 0) return TKV_HIP_OK;
    int64_t blocks = scalar_blocks(c, n / 4 + 1);
    hipLaunchKernelGGL(k_i8_to_i32, dim3((unsigned)blocks), dim3(kBlock), 0, c->stream, src, n,
                       dst, code_bias);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

// src int32 [rows, cols] (row-major) -> dst int8 [cols, ld_dst] (transposed,
// zero-padded to ld_dst >= rows).  32x32 tiles through LDS.
__global__ __launch_bounds__(kBlock) void k_i32_to_i8_transpose(const int32_t* __restrict__ src,
                                                                int64_t rows, int64_t cols,
                                                                int8_t* __restrict__ dst,
                                                                int64_t ld_dst) {
    __shared__ int8_t tile[32][33];
    const int64_t r0 = (int64_t)blockIdx.y * 32, c0 = (int64_t)blockIdx.x * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
    for (int j = ty; j < 32; j += 8) {
        int64_t r = r0 + j, cc = c0 + tx;
        tile[j][tx] = (r < rows && cc < cols) ? (int8_t)src[r * cols + cc] : (int8_t)0;
    }
    __syncthreads();
    for (int j = ty; j < 32; j += 8) {
        int64_t orow = c0 + j, ocol = r0 + tx;  // dst[orow][ocol] = src[ocol][orow]
        if (orow < cols && ocol < ld_dst) dst[orow * ld_dst + ocol] = tile[tx][j];
    }
}

int launch_i32_to_i8_transpose(Ctx* c, const int32_t* src, int64_t rows, int64_t cols,
                               int8_t* dst, int64_t ld_dst) {
    if (rows <= 0 || cols <= 0) return TKV_HIP_OK;
    dim3 grid((unsigned)ceil_div(cols, 32), (unsigned)ceil_div(ld_dst, 32));
    hipLaunchKernelGGL(k_i32_to_i8_transpose, grid, dim3(kBlock), 0, c->stream, src, rows, cols,
                       dst, ld_dst);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

}  // namespace tkv
