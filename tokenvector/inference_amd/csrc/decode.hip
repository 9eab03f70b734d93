// decode.hip -- the per-token W8A8 linear of decode batches (M <= 32) as
// one kernel: per-token absmax + int8 quantize of the activation rows
// (quantize_dynamic_int8_rowwise, tv/quantization/engine.tkv:266-285), the
// INT8 GEMM against a resident per-channel weight (matmul_int8_per_channel,
// tv/quantization/matmul.tkv:17-29, _dot_int8 :116-127) and the dequant +
// bias epilogue with the token's scale (the per-token form of the R11 chain:
// y = fl32(fl64(fl64(acc * sa[m]) * sw[n]) + b[n]), sa[m] = fl32(am / 127)).
//
// Workgroup (cb, rg) owns output columns [16 NCB cb, 16 NCB (cb + 1)) (NCB
// 16-column blocks, one MFMA each per k-step) and token rows [RG rg, RG rg +
// RG).  It needs its rows' full activation (the token scale
// is the row's absmax over all of K) and its columns' full weight rows, so
// it reads both itself and nothing crosses workgroups: no atomics, no
// barrier, no scratch memory, and the result does not depend on scheduling.
//   * Every load is issued at the start: the activation fragments (16 f32
//     per lane per k-step, the A operand's elements before quantization),
//     then the workgroup's weight rows, copied straight into LDS (direct DMA,
//     whole 128-byte lines of 8 rows per instruction); the row scales are
//     formed while the weight lines land, and the B operands of
//     v_mfma_i32_16x16x64_i8 are read from LDS.
//   * Wave w takes the contiguous k-steps [KSW w, KSW w + KSW); the row
//     absmax is reduced over the 4 lanes sharing a row (shuffles) and then
//     over the waves (LDS), then each wave quantizes its fragments in
//     registers and runs its MFMAs.
//   * The waves' INT32 partial tiles are summed exactly with LDS atomics and
//     wave c % waves runs the epilogue of column block c.
// Splitting the tokens into row groups keeps the activation bytes per
// workgroup near its weight bytes (16 K each at RG = 4): a CU then moves
// ~32 K bytes per workgroup whatever M is, instead of 4 M K.
// Workgroups sharing a column block sit on one XCD (consecutive tile ids per
// XCD), so their repeated weight reads come from that XCD's L2.
#include <cstdlib>

#include "gemm_tile.h"
#include "tkv_device.h"
#include "tkv_internal.h"

namespace tkv {
namespace {

using gemm::v4i;
using gemm::wave_id;
using gemm::barrier;
using gemm::xcd_tile;

constexpr int kKsw = 3;         // 64-deep k-steps per wave
constexpr int kMaxWaves = 16;   // K <= 16 * 3 * 64 = 3072
constexpr int kDecodeMaxM = 32;

// Four f32 -> int8 codes (rne, clamp +-127, NaN -> 0) packed little-endian.
__device__ __forceinline__ int quant4(const float4 v, double inv) {
    const int a = rne_clamp((double)v.x * inv, -127.0, 127.0);
    const int b = rne_clamp((double)v.y * inv, -127.0, 127.0);
    const int c = rne_clamp((double)v.z * inv, -127.0, 127.0);
    const int d = rne_clamp((double)v.w * inv, -127.0, 127.0);
    const uint32_t lo = __builtin_amdgcn_perm((uint32_t)b, (uint32_t)a, 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm((uint32_t)d, (uint32_t)c, 0x04000c0cu);
    return (int)(lo | hi);
}

__device__ __forceinline__ float amax4(float m, const float4 v) {
    return fmaxf(fmaxf(m, fabsf(v.x)), fmaxf(fmaxf(fabsf(v.y), fabsf(v.z)), fabsf(v.w)));
}

// x f32 [M, K] (16-byte aligned rows, K % 64 == 0, K <= KMAX), W int8 [N,
// ldk] (K-major, ldk % 128 == 0: rows are read in whole 128-byte lines, the
// padding past K included), sw f32 [N], bias f32 [N] or null, y f32 [M, N].
// ncb = ceil(N / (16 NCB)) column groups, ngr = ceil(M / RG) row groups.
//
// Weight rows in LDS (dynamic, NCB 16 nl 128 bytes, nl = ceil(K / 128)):
// the workgroup's 16 NCB rows of W arrive by direct DMA, one 1 KB
// instruction per 128-byte line of 8 rows.  Instruction d = (c nl + p) 2 + h
// holds line p of rows 16 c + 8 h + r, r = 0 .. 7, lane 8 r + q taking the
// line's 16-byte chunk q ^ w_swz(8 h + r).  Whole lines per instruction: the
// 64-byte halves that a B-operand load per lane reads (16 rows per
// instruction) measured 1.1-1.3x slower per call at M = 16 and 32 (kernel
// trace, one box).  The swizzle makes a 16-lane read of one chunk of the 16
// rows hit 16 distinct 16-byte bank groups (and any 8 consecutive lanes of
// it 8 distinct ones).  Each wave issues DPW instructions per column block,
// the last ones clamped to the final instruction (repeats write the same
// bytes).  With little weight per workgroup and at most one workgroup per
// CU (qkv and mlp_up at M <= 4: 12 KB) the LDS hop costs more than the whole
// lines save (4.1-4.5 against 4.4-4.8 us cold), so those launches load each
// lane's B operand straight into registers (DPW = 0, no weight LDS).
//
// The activation is quantized only for the group's valid rows: chunk
// c < nks * 4 * rows is 16 consecutive elements of row c % rows at k =
// 16 (c / rows); a lane holds up to kChunks chunks in registers, the row
// absmax is reduced with LDS atomics on the f32 bits (non-negative, NaN
// already skipped), threads 0 .. rows - 1 form the row's reciprocal once,
// and each chunk's 16 codes are written to LDS where the MFMA A fragment of
// its k-step expects them: 16 bytes at ((ks * 4 + kg) * 16 + row) * 16.
// (Measured against one float4 per thread per row with DPP row maxima and
// swizzled 4-byte code stores: the chunk form was 0.5-1.4 us faster per call
// up to M = 16 in a kernel trace of both on one box.)
constexpr int kChunks = 3;  // 16 rows * 3072 / (16 elements * 1024 threads) = 3

__device__ __forceinline__ int w_swz(int row) { return (row & 7) ^ (row >> 3); }

template <int NCB, int KMAX, int DPW>
__global__ __launch_bounds__(kMaxWaves * 64) void k_decode_i8(
    const float* __restrict__ x, const uint8_t* __restrict__ W, int M, int N, int K, int ldk,
    int RG, int ncb, int ngr, const float* __restrict__ sw, const float* __restrict__ bias,
    float* __restrict__ y) {
    extern __shared__ __attribute__((aligned(16))) uint8_t s_w[];
    // The activation codes are an array of their own: the compiler then
    // knows that their stores and loads cannot touch the weight DMA's bytes
    // and does not wait for it there.
    __shared__ __attribute__((aligned(16))) uint8_t s_a[16 * KMAX];
    __shared__ uint32_t s_am[16];
    __shared__ double s_inv[16];
    __shared__ float s_sa[16];
    __shared__ int32_t s_acc[256 * NCB];
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int nthreads = (int)blockDim.x;
    const int t = xcd_tile((int)blockIdx.x, ncb * ngr);
    const int cb = t / ngr, rg = t % ngr;
    const int n0 = cb * 16 * NCB, r0 = rg * RG;
    const int rows = M - r0 < RG ? M - r0 : RG;  // valid rows of this group (1 .. 16)
    const int nks = K / 64, nl = (K + 127) / 128;
    const int lr = lane & 15, kg = lane >> 4;
    const int ks0 = wave * kKsw;

    // Register form (DPW == 0): the weight loads are unconditional, from a
    // clamped k-step (fragments past nks are never used: the MFMA loop skips
    // them): under the wave-uniform branch they had, the compiler left a
    // register copy where the branches join and waited there (vmcnt(0)) for
    // the load, a memory round trip in the middle of issuing the loads.  The
    // activation loads stay lane-masked (clamped, every thread past nchunks
    // would load), with no value for the masked lanes, which nothing reads: a
    // zero there made the same join copy and wait.
    // weight fragments (B operand): column n0 + 16 c + lr, bytes [64 ks + 16 kg, +16)
    v4i wf[NCB][kKsw];
    if constexpr (DPW == 0) {
#pragma unroll
        for (int c = 0; c < NCB; c++) {
            const int wcol = n0 + 16 * c + lr < N ? n0 + 16 * c + lr : N - 1;
            const uint8_t* __restrict__ wp = W + (int64_t)wcol * ldk + kg * 16;
#pragma unroll
            for (int s = 0; s < kKsw; s++) {
                const int ks = ks0 + s < nks ? ks0 + s : nks - 1;
                wf[c][s] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wp + ks * 64));
            }
        }
    }
    // activation chunks of the valid rows
    const int nchunks = nks * 4 * rows;
    float4 xv[kChunks][4];
    int crow[kChunks], ck16[kChunks];
#pragma unroll
    for (int j = 0; j < kChunks; j++) {
        const int c = (int)threadIdx.x + j * nthreads;
        crow[j] = c % rows;
        ck16[j] = c / rows;
        const float4* xp = reinterpret_cast<const float4*>(x + (int64_t)(r0 + crow[j]) * K +
                                                           (int64_t)ck16[j] * 16);
        if (c < nchunks) {
#pragma unroll
            for (int q = 0; q < 4; q++) xv[j][q] = xp[q];
        }
    }
    // DMA form: the weight lines, unconditional DMAs from clamped rows and
    // instruction indices (no branch, and nothing lands in registers).  Lines
    // past K are the rows' zero padding; the MFMA loop never reads them.
    if constexpr (DPW > 0) {
        const int r = lane >> 3, q = lane & 7;
#pragma unroll
        for (int c = 0; c < NCB; c++) {
#pragma unroll
            for (int i = 0; i < DPW; i++) {
                const int d0 = wave * DPW + i;
                const int d = d0 < 2 * nl ? d0 : 2 * nl - 1;
                const int row = 8 * (d & 1) + r;
                const int col = n0 + 16 * c + row < N ? n0 + 16 * c + row : N - 1;
                const uint8_t* g =
                    W + (int64_t)col * ldk + (d >> 1) * 128 + ((q ^ w_swz(row)) << 4);
                __builtin_amdgcn_global_load_lds(
                    (const void*)g, (gemm::lds_ptr)(s_w + ((c * nl) * 2 + d) * 1024), 16, 0, 0);
            }
        }
    }
    if (threadIdx.x < 16) s_am[threadIdx.x] = 0u;
    for (int i = threadIdx.x; i < 256 * NCB; i += nthreads) s_acc[i] = 0;
    // Raw barriers (gemm::barrier: lgkmcnt(0), then s_barrier) until the
    // MFMAs: __syncthreads() is a release fence, which would wait for the
    // weight DMA (an outstanding LDS write) at the first barrier.
    barrier();
    // row absmax from 0 (engine.tkv:272-276: NaN never compares greater;
    // fmaxf skips it, so the bits compared below are those of a finite or
    // infinite non-negative value, ordered as unsigned integers)
#pragma unroll
    for (int j = 0; j < kChunks; j++) {
        const int c = (int)threadIdx.x + j * nthreads;
        if (c < nchunks) {
            float am = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; q++) am = amax4(am, xv[j][q]);
            atomicMax(&s_am[crow[j]], __float_as_uint(am));
        }
    }
    barrier();
    if (threadIdx.x < rows) {
        double dam = (double)__uint_as_float(s_am[threadIdx.x]);
        if (dam < 0.00000001) dam = 0.00000001;
        const double sc = dam / 127.0;  // unrounded f64 scale (engine.tkv:277-279)
        s_inv[threadIdx.x] = 1.0 / sc;
        s_sa[threadIdx.x] = (float)sc;
    }
    barrier();
#pragma unroll
    for (int j = 0; j < kChunks; j++) {
        const int c = (int)threadIdx.x + j * nthreads;
        if (c < nchunks) {
            const double inv = s_inv[crow[j]];
            const v4i q = {quant4(xv[j][0], inv), quant4(xv[j][1], inv), quant4(xv[j][2], inv),
                           quant4(xv[j][3], inv)};
            // ck16 = ks * 4 + kg
            *reinterpret_cast<v4i*>(s_a + ((ck16[j] * 16 + crow[j]) << 4)) = q;
        }
    }
    // every wave's weight DMAs have landed (vmcnt counts them) before any
    // wave reads the lines, some of which other waves copied
    if constexpr (DPW > 0) gemm::wait_vmcnt<0>();
    barrier();

    v4i acc[NCB];
#pragma unroll
    for (int c = 0; c < NCB; c++) acc[c] = v4i{0, 0, 0, 0};
    // B operand of k-step ks, column block c: chunk 4 (ks & 1) + kg of line
    // ks >> 1 of row lr
    const int wrow = ((lr >> 3) << 10) + ((lr & 7) << 7);
    const int wsw = w_swz(lr);
#pragma unroll
    for (int s = 0; s < kKsw; s++) {
        const int ks = ks0 + s;
        if (ks < nks) {
            const v4i af = lr < rows
                               ? *reinterpret_cast<const v4i*>(s_a + (((ks * 4 + kg) * 16 + lr) << 4))
                               : v4i{0, 0, 0, 0};
            const int woff = ((ks >> 1) << 11) + wrow + (((4 * (ks & 1) + kg) ^ wsw) << 4);
#pragma unroll
            for (int c = 0; c < NCB; c++) {
                v4i b;
                if constexpr (DPW > 0)
                    b = *reinterpret_cast<const v4i*>(s_w + ((c * nl) << 11) + woff);
                else
                    b = wf[c][s];
                acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, b, acc[c], 0, 0, 0);
            }
        }
    }
    // 16 x 16 result per column block: lane holds column lane & 15, rows
    // 4 (lane >> 4) + i
#pragma unroll
    for (int c = 0; c < NCB; c++)
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (4 * kg + i < rows) atomicAdd(&s_acc[c * 256 + (4 * kg + i) * 16 + lr], acc[c][i]);
    __syncthreads();
    auto store_block = [&](int c) {
        const int col = n0 + 16 * c + lr;
        if (col >= N) return;
        const double swc = (double)sw[col];
        const double bc = bias ? (double)bias[col] : 0.0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = 4 * kg + i;
            if (r < rows) {
                double v = (double)s_acc[c * 256 + r * 16 + lr] * (double)s_sa[r];
                v = v * swc;
                v = v + bc;
                __builtin_nontemporal_store((float)v, y + (int64_t)(r0 + r) * N + col);
            }
        }
    };
    if constexpr (NCB == 1) {
        if (wave == 0) store_block(0);
    } else {
        // wave w stores column blocks w, w + waves, ... (a workgroup may have
        // fewer waves than column blocks)
        for (int c = wave; c < NCB; c += nthreads / 64) store_block(c);
    }
}

// Row stride (in groups) of the Q8_0 decode's dots and scales: nkb (even)
// rounded up to twice an odd number, so 16 rows of it start 16 distinct
// even banks apart and float2 reads of the 16 columns do not conflict.
__host__ __device__ constexpr int q8_decode_stride(int nkb) { return (nkb / 2) % 2 ? nkb : nkb + 2; }
__host__ __device__ constexpr int64_t q8_decode_lds(int64_t k, int64_t rg) {
    return rg * k + (rg * 64 + 64) * q8_decode_stride((int)(k / 32));
}

// GGUF Q8_0 weights (extension; the reference decodes them to f32,
// gguf.tkv:284-290) for decode batches: the per-token quantize of
// k_decode_i8, then for 16 columns and a row group
//   dot_g = sum over block g's 32 k of a[m, k] q[n, k]   (exact INT32)
//   acc   = 0;  acc = fma(float(dot_g), d[n, g], acc)  for g = 0, 1, ... in order
//   y     = fl32(fl64(fl64(acc) * sa[m]) + b[n])
// -- the recipe of the Q8_0 tile GEMM, so results are the same bits.  Each
// wave multiplies its 6 groups (3 64-deep k-steps) with one
// v_mfma_i32_16x16x32_i8 each into a zero accumulator and keeps every
// group's dots in LDS; after a barrier one thread per output runs the fma
// chain over all groups in order (the order fixes the rounding, so the
// groups cannot be summed per wave) and the epilogue.
// x f32 [M, K] (16-byte aligned rows, K % 64 == 0), W int8 [N, ldk], gs f32
// [N, ldk / 32], bias f32 [N] or null, y f32 [M, N]; RG <= 16 tokens per
// group.  Dynamic LDS (q8_decode_lds): RG K code bytes (16-byte chunks of
// 16 k, the group's rows interleaved per chunk); the dots [RG][16][nkp] and
// scales [16][nkp], output-major so that a chain reads two groups per LDS
// load, nkp = K / 32 rounded up to twice an odd number so that the 16
// columns' rows start in distinct banks.  Dots are kept as f32 (exact, |dot|
// < 2^24), converted by the waves that form them.
template <int DPW>
__global__ __launch_bounds__(kMaxWaves * 64) void k_decode_q8(
    const float* __restrict__ x, const uint8_t* __restrict__ W, const float* __restrict__ gs,
    int M, int N, int K, int ldk, int RG, int ncb, int ngr, const float* __restrict__ bias,
    float* __restrict__ y) {
    extern __shared__ __attribute__((aligned(16))) uint8_t s_dyn[];
    const int nks = K / 64, nkb = K / 32, nkp = q8_decode_stride(nkb), nl = (K + 127) / 128;
    // lines form (DPW > 0): the 16 weight rows first, laid out as in k_decode_i8
    const int wb = DPW > 0 ? 16 * nl * 128 : 0;
    uint8_t* s_w = s_dyn;
    uint8_t* s_a = s_dyn + wb;                                                   // [K / 16][RG][16]
    float* s_p = reinterpret_cast<float*>(s_dyn + wb + RG * K);                  // [RG][16][nkp]
    float* s_d = reinterpret_cast<float*>(s_dyn + wb + RG * K + RG * 64 * nkp);  // [16][nkp]
    __shared__ uint32_t s_am[16];
    __shared__ double s_inv[16];
    __shared__ float s_sa[16];
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int nthreads = (int)blockDim.x;
    const int t = xcd_tile((int)blockIdx.x, ncb * ngr);
    const int cb = t / ngr, rg = t % ngr;
    const int n0 = cb * 16, r0 = rg * RG;
    const int rows = M - r0 < RG ? M - r0 : RG;
    const int lr = lane & 15, kg = lane >> 4;
    const int ks0 = wave * kKsw;
    const int gstride = ldk / 32;

    // Loads as in k_decode_i8 (unconditional weights from a clamped k-step,
    // lane-masked activation chunks with no default).  Register form: lane
    // (lr, kg) loads bytes [64 ks + 16 kg, +16) of column n0 + lr per 64-deep
    // k-step, one 16-byte load for two groups (8-byte loads per group, twice
    // the load instructions, measured 1.6-1.9x this kernel's INT8
    // counterpart at K = 3072, M = 1).  Lines form: the weight rows are
    // copied into LDS after the activation loads, whole 128-byte lines of 8
    // rows per DMA.  Each thread also takes up to two of the 16 columns'
    // group scales (16 * K / 32 <= 1.5 threads' worth), stored to LDS once
    // the loads are all issued.
    v4i wq[kKsw];
    if constexpr (DPW == 0) {
        const int wcol = n0 + lr < N ? n0 + lr : N - 1;
        const uint8_t* __restrict__ wp = W + (int64_t)wcol * ldk + 16 * kg;
#pragma unroll
        for (int s = 0; s < kKsw; s++) {
            const int ks = ks0 + s < nks ? ks0 + s : nks - 1;
            wq[s] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wp + ks * 64));
        }
    }
    // scale i is group i % nkb of column i / nkb: consecutive threads read
    // consecutive groups of one column (coalesced)
    float dv[2];
#pragma unroll
    for (int q = 0; q < 2; q++) {
        int i = (int)threadIdx.x + q * nthreads;
        i = i < 16 * nkb ? i : 16 * nkb - 1;
        const int c = i / nkb, g = i - c * nkb;
        const int col = n0 + c < N ? n0 + c : N - 1;
        dv[q] = gs[(int64_t)col * gstride + g];
    }
    const int nchunks = nks * 4 * rows;
    float4 xv[kChunks][4];
    int crow[kChunks], ck16[kChunks];
#pragma unroll
    for (int j = 0; j < kChunks; j++) {
        const int c = (int)threadIdx.x + j * nthreads;
        crow[j] = c % rows;
        ck16[j] = c / rows;
        const float4* xp = reinterpret_cast<const float4*>(x + (int64_t)(r0 + crow[j]) * K +
                                                           (int64_t)ck16[j] * 16);
        if (c < nchunks) {
#pragma unroll
            for (int q = 0; q < 4; q++) xv[j][q] = xp[q];
        }
    }
    if constexpr (DPW > 0) {
        const int r = lane >> 3, q = lane & 7;
#pragma unroll
        for (int i = 0; i < DPW; i++) {
            const int d0 = wave * DPW + i;
            const int d = d0 < 2 * nl ? d0 : 2 * nl - 1;
            const int row = 8 * (d & 1) + r;
            const int col = n0 + row < N ? n0 + row : N - 1;
            const uint8_t* g = W + (int64_t)col * ldk + (d >> 1) * 128 + ((q ^ w_swz(row)) << 4);
            __builtin_amdgcn_global_load_lds((const void*)g, (gemm::lds_ptr)(s_w + d * 1024), 16,
                                             0, 0);
        }
    }
    if (threadIdx.x < 16) s_am[threadIdx.x] = 0u;
    // raw barriers up to the MFMAs: __syncthreads() would wait for the
    // weight DMA (an outstanding LDS write) at each one
    barrier();
#pragma unroll
    for (int j = 0; j < kChunks; j++) {
        const int c = (int)threadIdx.x + j * nthreads;
        if (c < nchunks) {
            float am = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; q++) am = amax4(am, xv[j][q]);
            atomicMax(&s_am[crow[j]], __float_as_uint(am));
        }
    }
#pragma unroll
    for (int q = 0; q < 2; q++) {
        const int i = (int)threadIdx.x + q * nthreads;
        if (i < 16 * nkb) s_d[(i / nkb) * nkp + i % nkb] = dv[q];
    }
    barrier();
    if (threadIdx.x < rows) {
        double dam = (double)__uint_as_float(s_am[threadIdx.x]);
        if (dam < 0.00000001) dam = 0.00000001;
        const double sc = dam / 127.0;  // engine.tkv:277-279
        s_inv[threadIdx.x] = 1.0 / sc;
        s_sa[threadIdx.x] = (float)sc;
    }
    barrier();
#pragma unroll
    for (int j = 0; j < kChunks; j++) {
        const int c = (int)threadIdx.x + j * nthreads;
        if (c < nchunks) {
            const double inv = s_inv[crow[j]];
            const v4i q = {quant4(xv[j][0], inv), quant4(xv[j][1], inv), quant4(xv[j][2], inv),
                           quant4(xv[j][3], inv)};
            *reinterpret_cast<v4i*>(s_a + ((ck16[j] * RG + crow[j]) << 4)) = q;
        }
    }
    if constexpr (DPW > 0) gemm::wait_vmcnt<0>();  // every wave's weight lines have landed
    barrier();
    // Group dots.  Lane kg < 2 holds 16 bytes of group 2 ks, lane kg >= 2 of
    // group 2 ks + 1; lanes l and l ^ 32 swap one 8-byte half, after which
    // every lane holds one 8-byte piece of each group: kg 0..3 hold bytes
    // [8 j, +8) of both groups with j = 0, 2, 1, 3 (low half: group 2 ks,
    // high half: group 2 ks + 1).  A dot product only needs A and B in the
    // same k order, so the A operand of group g is row lr's codes at that same
    // offset, 32 g + 8 j: the first or second half (kg / 2) of 16-byte chunk
    // 2 g + (kg & 1).  Rows past the group read 0.  The result holds column
    // lr, rows 4 kg + i.
    // (the swaps run for every k-step, including clamped ones past nks,
    // before any MFMA: outside the k-step branch they are issued together)
    // Lines form: the B operand of group g is row lr's bytes [32 g + 8 kg,
    // +8) (16-byte chunk 2 (g & 3) + kg / 2 of line g / 4, half kg & 1), the
    // k order unpermuted, so A reads the same offset of its row's codes.
    const v4i zero = {0, 0, 0, 0};
    const bool lo_half = kg < 2;
    int64_t wf[kKsw][2];
#pragma unroll
    for (int s = 0; s < kKsw && DPW == 0; s++) {
        v4i w = wq[s];
        const int r0 = __shfl_xor(lo_half ? w.z : w.x, 32);
        const int r1 = __shfl_xor(lo_half ? w.w : w.y, 32);
        if (lo_half) {
            w.z = r0;
            w.w = r1;
        } else {
            w.x = r0;
            w.y = r1;
        }
        wf[s][0] = (int64_t)(uint32_t)w.x | ((int64_t)w.y << 32);
        wf[s][1] = (int64_t)(uint32_t)w.z | ((int64_t)w.w << 32);
    }
#pragma unroll
    for (int s = 0; s < kKsw; s++) {
        const int ks = ks0 + s;
        if (ks < nks) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int g = 2 * ks + h;
                int64_t af, bw;
                if constexpr (DPW > 0) {
                    af = lr < rows ? *reinterpret_cast<const int64_t*>(
                                         s_a + (((2 * g + (kg >> 1)) * RG + lr) << 4) + 8 * (kg & 1))
                                   : 0;
                    const int ch = 2 * (g & 3) + (kg >> 1);
                    bw = *reinterpret_cast<const int64_t*>(
                        s_w + ((((g >> 2) << 1) + (lr >> 3)) << 10) +
                        ((((lr & 7) << 3) + (ch ^ w_swz(lr))) << 4) + 8 * (kg & 1));
                } else {
                    af = lr < rows ? *reinterpret_cast<const int64_t*>(
                                         s_a + (((2 * g + (kg & 1)) * RG + lr) << 4) + 8 * (kg >> 1))
                                   : 0;
                    bw = wf[s][h];
                }
                const v4i p = __builtin_amdgcn_mfma_i32_16x16x32_i8(af, bw, zero, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (4 * kg + i < rows) s_p[((4 * kg + i) * 16 + lr) * nkp + g] = (float)p[i];
            }
        }
    }
    __syncthreads();
    if ((int)threadIdx.x < rows * 16) {
        const int r = (int)threadIdx.x >> 4, c = (int)threadIdx.x & 15;
        // the chain's LDS reads are issued 8 groups at a time (float2 loads),
        // so one LDS latency covers 8 dependent fmas instead of each
        const float2* pp = reinterpret_cast<const float2*>(s_p + (r * 16 + c) * nkp);
        const float2* dp = reinterpret_cast<const float2*>(s_d + c * nkp);
        constexpr int U = 4;  // float2 pairs per batch
        float acc = 0.0f;
        int h = 0;
        for (; h + U <= nkb / 2; h += U) {
            float2 pv[U], dw[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                pv[u] = pp[h + u];
                dw[u] = dp[h + u];
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                acc = __builtin_fmaf(pv[u].x, dw[u].x, acc);
                acc = __builtin_fmaf(pv[u].y, dw[u].y, acc);
            }
        }
        for (; h < nkb / 2; h++) {
            const float2 pv = pp[h], dw = dp[h];
            acc = __builtin_fmaf(pv.x, dw.x, acc);
            acc = __builtin_fmaf(pv.y, dw.y, acc);
        }
        const int col = n0 + c;
        if (col < N) {
            double v = (double)acc * (double)s_sa[r];
            v = v + (bias ? (double)bias[col] : 0.0);
            __builtin_nontemporal_store((float)v, y + (int64_t)(r0 + r) * N + col);
        }
    }
}

}  // namespace

// Tokens per row group: all of them up to 4; 4 up to 16 tokens, which keeps
// a workgroup's activation bytes (RG K 4) at its weight bytes (16 K); 8
// beyond, where more groups cost more in workgroup dispatch than their
// bytes save (trace of the three decode shapes at M = 32, RG 4 / 8 / 16:
// 7.7 / 7.0 / 7.4, 9.4 / 7.0 / 7.6, 11.4 / 9.6 / 12.7 us).  When the column
// blocks and those groups would keep fewer than half of the CUs busy (N = 768
// gives 48 blocks), the tokens are split into about 3/4 CUs / blocks groups
// instead: mlp_down at M = 8, 5.45 us with 2 tokens per group against 6.65
// with 4 (cold medians of three interleaved rounds, one box); qkv and mlp_up
// measured within 0.1 us of their best at any group size from 4 to 16.
// The context's TKV_HIP_TUNE_DECODE_GROUP override forces it (sweeps, tests).
static int decode_rows_per_group(const Ctx* c, int64_t m, int64_t ncb, int num_cus) {
    if (tuned(c, TKV_HIP_TUNE_DECODE_GROUP) >= 1) return (int)tuned(c, TKV_HIP_TUNE_DECODE_GROUP);
    int64_t rg = m <= 4 ? m : (m <= 16 ? 4 : 8);
    if (2 * ncb * ceil_div(m, rg) < num_cus) {
        const int64_t groups = ceil_div((int64_t)num_cus * 3 / 4, ncb);
        rg = ceil_div(m, groups);
    }
    return (int)rg;
}

int launch_decode_i8(Ctx* c, const float* x, int64_t m, int64_t k, const uint8_t* w, int64_t ldk,
                     int64_t n, const float* scales_w, const float* bias, float* y) {
    if (m < 1 || m > kDecodeMaxM || k % 64 != 0 || k / 64 > (int64_t)kMaxWaves * kKsw ||
        ldk % 128 != 0 || ldk < k || !aligned(x, 16) || !aligned(w, 16) || n < 1 ||
        n >= (1ll << 28))
        return TKV_HIP_UNSUPPORTED;
    // 16-column blocks per workgroup.  Above 16 tokens a workgroup's row
    // group is quantized once for several column blocks: 64 columns for K <=
    // 1024, else 32 (cold calls at M = 32, interleaved rounds on one box:
    // qkv 6.95 -> 6.76 us, mlp_up 7.08 -> 6.50, mlp_down 8.85 -> 8.44 with 32
    // columns and 11.0 with 64; at M = 16 two blocks measured 0.1-0.4 us
    // slower than one).
    int ncols = m <= 16 ? 1 : (k <= 1024 ? 4 : 2);
    const int64_t nl = ceil_div(k, (int64_t)128);
    const int64_t nw = ceil_div(k / 64, (int64_t)kKsw);
    const int kmax = k <= 1024 ? 1024 : 3072;
    // LDS: the activation codes and the partial tiles (fewer column blocks
    // per workgroup if the device's share is less), plus the weight lines
    // (dynamic) in the DMA form, which is taken only where they fit
    const int64_t max_lds = (int64_t)c->max_lds;
    auto lds_reg = [&](int nc) { return (int64_t)16 * kmax + 1024 * nc + 512; };
    auto lds_dma = [&](int nc) { return nc * 16 * nl * 128 + lds_reg(nc); };
    while (ncols > 1 && lds_reg(ncols) > max_lds) ncols /= 2;
    if (lds_reg(ncols) > max_lds) return TKV_HIP_UNSUPPORTED;
    const int64_t ncb = ceil_div(n, (int64_t)16 * ncols);
    const int rg = decode_rows_per_group(c, m, ncb, c->num_cus);
    const int64_t ngr = ceil_div(m, (int64_t)rg);
    // DMA instructions per wave and column block: 2 nl in all over nw waves
    // (3 for K = 768 and 3072; at most 4 for any K here).  The register form
    // (dpw 0) where a workgroup's weight rows are under 32 KB and the grid
    // fits the CUs in one pass (cold calls, same box, two alternating rounds:
    // mlp_down M = 32 8.18 -> 7.05 us and M = 1 4.98 -> 4.68 with the DMA;
    // qkv M = 16 5.94 -> 5.63, M = 32 6.72 -> 6.07; qkv and mlp_up at M <= 4
    // 4.1-4.5 us in registers against 4.4-4.8 through LDS).
    int dpw = 2 * nl > 3 * nw ? 4 : 3;
    if (tuned(c, TKV_HIP_TUNE_DECODE_DMA) == 0 ||
        (tuned(c, TKV_HIP_TUNE_DECODE_DMA) < 0 && ncols * 16 * nl * 128 < (32 << 10) &&
         ncb * ngr <= c->num_cus) ||
        dpw * nw < 2 * nl || lds_dma(ncols) > max_lds)
        dpw = 0;
    const dim3 grid((unsigned)(ncb * ngr)), block((unsigned)(nw * 64));
    const unsigned dyn = dpw ? (unsigned)(ncols * 16 * nl * 128) : 0u;
#define TKV_DEC(NC, KM)                                                                        \
    do {                                                                                       \
        if (dpw == 4)                                                                          \
            hipLaunchKernelGGL((k_decode_i8<NC, KM, 4>), grid, block, dyn, c->stream, x, w,   \
                               (int)m, (int)n, (int)k, (int)ldk, rg, (int)ncb, (int)ngr,      \
                               scales_w, bias, y);                                             \
        else if (dpw == 3)                                                                     \
            hipLaunchKernelGGL((k_decode_i8<NC, KM, 3>), grid, block, dyn, c->stream, x, w,   \
                               (int)m, (int)n, (int)k, (int)ldk, rg, (int)ncb, (int)ngr,      \
                               scales_w, bias, y);                                             \
        else                                                                                   \
            hipLaunchKernelGGL((k_decode_i8<NC, KM, 0>), grid, block, dyn, c->stream, x, w,   \
                               (int)m, (int)n, (int)k, (int)ldk, rg, (int)ncb, (int)ngr,      \
                               scales_w, bias, y);                                             \
    } while (0)
    if (kmax == 1024) {
        if (ncols == 4) TKV_DEC(4, 1024);
        else if (ncols == 2) TKV_DEC(2, 1024);
        else TKV_DEC(1, 1024);
    } else {
        if (ncols == 2) TKV_DEC(2, 3072);
        else TKV_DEC(1, 3072);
    }
#undef TKV_DEC
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

int launch_decode_q8(Ctx* c, const float* x, int64_t m, int64_t k, const uint8_t* w,
                     const float* gs, int64_t ldk, int64_t n, const float* bias, float* y) {
    if (m < 1 || m > kDecodeMaxM || k % 64 != 0 || k / 64 > (int64_t)kMaxWaves * kKsw ||
        ldk % 128 != 0 || ldk < k || !aligned(x, 16) || !aligned(w, 16) || n < 1 ||
        n >= (1ll << 28))
        return TKV_HIP_UNSUPPORTED;
    const int64_t ncb = ceil_div(n, (int64_t)16);
    int rg = decode_rows_per_group(c, m, ncb, c->num_cus);
    const int64_t nl = ceil_div(k, (int64_t)128);
    const int64_t nw = ceil_div(k / 64, (int64_t)kKsw);
    const int64_t max_lds = (int64_t)c->max_lds;
    // Lines form (the weight rows through LDS in whole lines, as in
    // k_decode_i8) by the same rule: 32 KB of weight rows per workgroup or
    // more workgroups than CUs, if it fits; the context knob forces either.
    const int dpw = 2 * nl > 3 * nw ? 4 : 3;
    const int64_t wbytes = 16 * nl * 128;
    const int64_t knob = tuned(c, TKV_HIP_TUNE_DECODE_DMA);
    bool lines = knob >= 0 ? knob == 1
                           : (wbytes >= (32 << 10) || ncb * ceil_div(m, (int64_t)rg) > c->num_cus);
    if (dpw * nw < 2 * nl) lines = false;
    // the group's codes, dots and scales (and the lines) must fit the
    // workgroup's LDS (1 KB kept for the kernel's static arrays): fewer
    // tokens per group otherwise
    auto lds_of = [&](int r) { return q8_decode_lds(k, r) + (lines ? wbytes : 0) + 1024; };
    if (lines && lds_of(1) > max_lds) lines = false;
    while (rg > 1 && lds_of(rg) > max_lds) rg--;
    if (lds_of(rg) > max_lds) return TKV_HIP_UNSUPPORTED;
    const int64_t ngr = ceil_div(m, (int64_t)rg);
    const dim3 grid((unsigned)(ncb * ngr)), block((unsigned)(nw * 64));
    const unsigned lds = (unsigned)(lds_of(rg) - 1024);
    if (!lines)
        hipLaunchKernelGGL(k_decode_q8<0>, grid, block, lds, c->stream, x, w, gs, (int)m, (int)n,
                           (int)k, (int)ldk, rg, (int)ncb, (int)ngr, bias, y);
    else if (dpw == 4)
        hipLaunchKernelGGL(k_decode_q8<4>, grid, block, lds, c->stream, x, w, gs, (int)m, (int)n,
                           (int)k, (int)ldk, rg, (int)ncb, (int)ngr, bias, y);
    else
        hipLaunchKernelGGL(k_decode_q8<3>, grid, block, lds, c->stream, x, w, gs, (int)m, (int)n,
                           (int)k, (int)ldk, rg, (int)ncb, (int)ngr, bias, y);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

}  // namespace tkv
