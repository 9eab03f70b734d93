// gemm_kernels.h -- INT8 and FP8 GEMM kernels of the PTQ path on gfx950, with
// the fused dequant epilogues of the reference's quantized linear, and their
// launchers (instantiated by gemm.hip, gemm_i8.hip and gemm_f8.hip).
//
//   INT8  (matmul_int8_per_channel / _symmetric, tv/quantization/matmul.tkv:4-29,
//          _dot_int8 :116-127): v_mfma_i32_32x32x32_i8, INT32 accumulators
//          exact, epilogue restating the reference's float typing:
//            per-channel: y = fl32(fl64(fl64(acc * sa) * sw[n]) + b[n])
//            symmetric:   y = fl32(fl64(acc * fl32(sa * sw)) + b[n])
//   FP8   (matmul_fp8_e4m3, matmul.tkv:46-58): y = fl32(fl64(acc) + b[n]),
//          optional per-token / per-channel scales (extension).
//          reference products: both operands decoded once by the reference's
//                       decoder into exact f16 (k_fp8_ref_to_f16), then
//                       PolicyF16 on the f16 MFMA (drop-in precision);
//          PolicyF8:    full-rate f8f6f4 MFMA (OCP decode, hardware rounding).
//
// Data movement and tiling live in gemm_tile.h.  All arithmetic here is
// compiled with -ffp-contract=off.
#pragma once

#include <cmath>
#include <cstdlib>
#include <type_traits>
#include <utility>

#include "gemm_tile.h"
#include "tkv_internal.h"

namespace tkv {
namespace gemm {

// 32x32 MFMA result layout: lane holds column (lane & 31); register r holds
// row (r / 4) * 8 + (lane / 32) * 4 + (r % 4).
__device__ __forceinline__ int acc_row(int r, int khalf) { return (r >> 2) * 8 + khalf * 4 + (r & 3); }

// Output stores bypass cache allocation: Y is written once and not re-read
// by this kernel, so it should not evict the A / W slices other tiles reuse.
template <class T>
__device__ __forceinline__ void put(T* p, T v) { __builtin_nontemporal_store(v, p); }

// An accumulator value as an opaque register: the epilogue arithmetic of a
// deferred tile then cannot be hoisted out of the next tile's K loop (where
// every converted value would occupy registers for the whole loop).
template <class T>
__device__ __forceinline__ T pin(T v) {
    asm volatile("" : "+v"(v));
    return v;
}

// Writes part of the calling wave's TM x TN blocks of 32 x 32 outputs of the
// tile at (m0, n0): parts P0 .. P0 + NP - 1, part p being accumulator register
// p % 16 of row block p / 16 (one output row per lane) across all TN column
// blocks; C::TM * 16 parts make the tile.  value(i, j, r) is the output held
// in accumulator register r of block (i, j).  Row bases are wave-uniform
// (scalar registers); the lane part is one 32-bit element offset (launchers
// keep N < 2^28).  Tiles fully inside [M, N] (all but the edges) store
// without any checks.
template <class C, int P0, int NP, class T, class F>
__device__ __forceinline__ void write_tile(T* __restrict__ Y, int m0, int n0, int M, int N,
                                           F&& value) {
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int wm = wave / C::WN, wn = wave % C::WN, khalf = lane >> 5, lc = lane & 31;
    const int rbase = m0 + wm * C::WTM, cbase = n0 + wn * C::WTN;
    const uint32_t loff = (uint32_t)(khalf * 4) * (uint32_t)N + (uint32_t)lc;
    auto body = [&](auto check) {
#pragma unroll
        for (int p = P0; p < P0 + NP; p++) {
            const int i = p / 16, r = p % 16;
            const int rrow = i * 32 + (r >> 2) * 8 + (r & 3);
            T* rowp = Y + (int64_t)(rbase + rrow) * N + cbase;
#pragma unroll
            for (int j = 0; j < C::TN; j++) {
                const T v = value(i, j, r);
                if (!decltype(check)::value ||
                    (rbase + rrow + khalf * 4 < M && cbase + j * 32 + lc < N))
                    put(rowp + loff + j * 32, v);
            }
        }
    };
    if (rbase + C::WTM <= M && cbase + C::WTN <= N)
        body(std::false_type{});
    else
        body(std::true_type{});
}

// INT8 dequant epilogue (MODE = EPI_*, RECIPE = TKV_HIP_RECIPE_*).
//   per-channel, primary:  y = fl32(fl64(fl64(acc * sa) * sw) + b)
//     When |acc| < 2^29 (K < 2^15) acc * sa is exact in f64 and so is
//     sa * sw (24 + 24 bits); then fl64(fl64(acc * sa) * sw) and
//     fl64(acc * fl64(sa * sw)) both round the same real number once, and the
//     per-column product c = sa * sw saves one f64 multiply per output
//     (per-tensor sa only: fold = 1).
//   symmetric, primary:    y = fl32(fl64(acc * fl32(sa * sw)) + b)
//   alternate recipes:     the same chains in f32.
// Per-tile epilogue operands: activation scale(s) of the lane's rows (one
// per-tensor value, or ROWS: one per accumulator row), weight scale and bias
// of its columns.  They are loaded when the tile starts: VMEM results retire
// in issue order, so loads issued before the K loop are complete by the
// epilogue instead of waiting there behind the previous tile's stores.
template <class C, bool ROWS>
struct EpiOperands {
    float sa_r[ROWS ? C::TM : 1][ROWS ? 16 : 1];
    float sw[C::TN], b[C::TN];
    __device__ __forceinline__ float sa(int i, int r) const {
        if constexpr (ROWS)
            return sa_r[i][r];
        else
            return sa_r[0][0];
    }
    // A copy whose values pass through an empty asm where the epilogue
    // starts.  The operands are loaded when the tile starts and used after its
    // K loop; without this the compiler hoists their first use (a conversion
    // to f64) next to the loads, and the wait for them there -- vmcnt retires
    // in issue order -- also waits for every output store of the previous
    // tile, serialising the stores with this tile's MFMAs.
    __device__ __forceinline__ EpiOperands pinned() const {
        EpiOperands o = *this;
#pragma unroll
        for (int i = 0; i < (ROWS ? C::TM : 1); i++)
#pragma unroll
            for (int r = 0; r < (ROWS ? 16 : 1); r++) o.sa_r[i][r] = pin(o.sa_r[i][r]);
#pragma unroll
        for (int j = 0; j < C::TN; j++) {
            o.sw[j] = pin(o.sw[j]);
            o.b[j] = pin(o.b[j]);
        }
        return o;
    }
};

// Rows past M read row M - 1 and columns past N column N - 1 (never stored).
template <class C, bool ROWS>
__device__ __forceinline__ void load_operands(const float* __restrict__ sa_ptr, int64_t stride,
                                              const float* __restrict__ scales_w,
                                              const float* __restrict__ bias, int m0, int n0,
                                              int M, int N, EpiOperands<C, ROWS>& o) {
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int wm = wave / C::WN, wn = wave % C::WN, khalf = lane >> 5;
    if (sa_ptr) {
        if constexpr (ROWS) {
#pragma unroll
            for (int i = 0; i < C::TM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = m0 + wm * C::WTM + i * 32 + acc_row(r, khalf);
                    o.sa_r[i][r] = sa_ptr[(int64_t)(row < M ? row : M - 1) * stride];
                }
        } else {
            o.sa_r[0][0] = sa_ptr[0];
        }
    }
#pragma unroll
    for (int j = 0; j < C::TN; j++) {
        int col = n0 + wn * C::WTN + j * 32 + (lane & 31);
        col = col < N ? col : N - 1;
        o.sw[j] = scales_w ? scales_w[col] : 1.0f;
        o.b[j] = bias ? bias[col] : 0.0f;
    }
}

template <int MODE, int RECIPE, bool ROWS>
struct EpiI8 {
    static constexpr bool kOut32 = true;  // 32-bit outputs (deferrable stores)
    const float* scale_a;
    int64_t scale_a_stride;
    float scale_w;
    const float* scales_w;
    const float* bias;
    int fold;

    template <class C>
    using Operands = EpiOperands<C, ROWS>;

    template <class C>
    __device__ __forceinline__ Operands<C> load(int m0, int n0, int M, int N) const {
        Operands<C> o;
        if (MODE != EPI_ACCUM_I32)
            load_operands<C, ROWS>(scale_a, scale_a_stride,
                                   MODE == EPI_PER_CHANNEL ? scales_w : nullptr, bias, m0, n0, M,
                                   N, o);
        return o;
    }

    // Calls f(value) once, value(i, j, r) being the 32 output bits of
    // accumulator register r of block (i, j): f32 bits, or the INT32 itself.
    template <class C, class P, class F>
    __device__ __forceinline__ void with_value(const typename P::Acc (&acc)[C::TM][C::TN],
                                               const Operands<C>& o_in, F&& f) const {
        const Operands<C> o = o_in.pinned();
        if constexpr (MODE == EPI_ACCUM_I32) {
            f([&](int i, int j, int r) { return (uint32_t)pin(acc[i][j][r]); });
        } else if constexpr (MODE == EPI_PER_CHANNEL && RECIPE == TKV_HIP_RECIPE_PRIMARY) {
            if (fold) {
                double c[C::TN];
#pragma unroll
                for (int j = 0; j < C::TN; j++) c[j] = (double)o.sa(0, 0) * (double)o.sw[j];
                f([&](int i, int j, int r) {
                    double v = (double)pin(acc[i][j][r]) * c[j];
                    v = v + (double)o.b[j];
                    return __float_as_uint((float)v);
                });
            } else {
                f([&](int i, int j, int r) {
                    double v = (double)pin(acc[i][j][r]) * (double)o.sa(i, r);
                    v = v * (double)o.sw[j];
                    v = v + (double)o.b[j];
                    return __float_as_uint((float)v);
                });
            }
        } else if constexpr (MODE == EPI_PER_CHANNEL) {
            f([&](int i, int j, int r) {
                float t = (float)pin(acc[i][j][r]) * o.sa(i, r);
                t = t * o.sw[j];
                return __float_as_uint(t + o.b[j]);
            });
        } else {
            f([&](int i, int j, int r) {
                const double s = RECIPE == TKV_HIP_RECIPE_PRIMARY
                                     ? (double)(o.sa(i, r) * scale_w)
                                     : (double)o.sa(i, r) * (double)scale_w;
                double v = (double)pin(acc[i][j][r]) * s;
                v = v + (double)o.b[j];
                return __float_as_uint((float)v);
            });
        }
    }

    template <class C, class P, int P0 = 0, int NP = C::TM * 16>
    __device__ __forceinline__ void store(const typename P::Acc (&acc)[C::TM][C::TN],
                                          const Operands<C>& o, int m0, int n0, int M, int N,
                                          void* __restrict__ Y) const {
        with_value<C, P>(acc, o, [&](auto&& value) {
            write_tile<C, P0, NP>(static_cast<uint32_t*>(Y), m0, n0, M, N, value);
        });
    }

    // The tile's outputs into registers (stored later with write_tile).
    template <class C, class P>
    __device__ __forceinline__ void values(const typename P::Acc (&acc)[C::TM][C::TN],
                                           const Operands<C>& o,
                                           uint32_t (&out)[C::TM][C::TN][16]) const {
        with_value<C, P>(acc, o, [&](auto&& value) {
#pragma unroll
            for (int i = 0; i < C::TM; i++)
#pragma unroll
                for (int j = 0; j < C::TN; j++)
#pragma unroll
                    for (int r = 0; r < 16; r++) out[i][j][r] = value(i, j, r);
        });
    }
};

// FP8 epilogue: y = fl32(fl64(acc) + b), or with per-token / per-channel
// scales y = fl32(fl64(fl64(fl64(acc) * sa) * sw) + b).  acc * kAccScale is
// exact (a power of two undoing the operand pre-scale).
template <bool SCALED, bool ROWS>
struct EpiF8 {
    static constexpr bool kOut32 = true;
    const float* scale_a;  // used when SCALED (extension epilogue)
    int64_t scale_a_stride;
    const float* scales_w;
    const float* bias;

    template <class C>
    using Operands = EpiOperands<C, ROWS>;

    template <class C>
    __device__ __forceinline__ Operands<C> load(int m0, int n0, int M, int N) const {
        Operands<C> o;
        load_operands<C, ROWS>(SCALED ? scale_a : nullptr, scale_a_stride,
                               SCALED ? scales_w : nullptr, bias, m0, n0, M, N, o);
        return o;
    }

    template <class C, class P, class F>
    __device__ __forceinline__ void with_value(const typename P::Acc (&acc)[C::TM][C::TN],
                                               const Operands<C>& o_in, F&& f) const {
        const Operands<C> o = o_in.pinned();
        f([&](int i, int j, int r) {
            double v = (double)(pin(acc[i][j][r]) * P::kAccScale);
            if (SCALED) {
                v = v * (double)o.sa(i, r);
                v = v * (double)o.sw[j];
            }
            v = v + (double)o.b[j];
            return __float_as_uint((float)v);
        });
    }

    template <class C, class P, int P0 = 0, int NP = C::TM * 16>
    __device__ __forceinline__ void store(const typename P::Acc (&acc)[C::TM][C::TN],
                                          const Operands<C>& o, int m0, int n0, int M, int N,
                                          void* __restrict__ Y) const {
        with_value<C, P>(acc, o, [&](auto&& value) {
            write_tile<C, P0, NP>(static_cast<uint32_t*>(Y), m0, n0, M, N, value);
        });
    }

    template <class C, class P>
    __device__ __forceinline__ void values(const typename P::Acc (&acc)[C::TM][C::TN],
                                           const Operands<C>& o,
                                           uint32_t (&out)[C::TM][C::TN][16]) const {
        with_value<C, P>(acc, o, [&](auto&& value) {
#pragma unroll
            for (int i = 0; i < C::TM; i++)
#pragma unroll
                for (int j = 0; j < C::TN; j++)
#pragma unroll
                    for (int r = 0; r < 16; r++) out[i][j][r] = value(i, j, r);
        });
    }
};

// QLinearMatMul requantizing epilogue (session.tkv:2016-2058), int8 out:
//   acc = sum_k (a - zpa)(w - zpw)
//       = sum_k a w - zpw * ra[m] - zpa * cw[n] + K * zpa * zpw
//   y   = clamp(rne(fl64(acc * mult)) + zpy, -128, 127)
// with ra / cw the row sums of A and W (the node's B transposed) and mult
// the host-computed multiplier; fl64(acc) is exact, so the product rounds
// once, as the reference's acc * mult does.
//   I32: the launcher has checked K (128 + |zpa|)(128 + |zpw|) < 2^31, so the
//        true acc fits int32 and two's-complement int32 arithmetic yields it
//        exactly whatever the intermediate wraps; the per-row term
//        K zpa zpw - zpw ra and the per-column term zpa cw are formed once per
//        tile.  The rounded product converts with saturation (NaN -> 0, as the
//        reference's saturating int()) before zpy is added and the result
//        clamped.
//   else: the same correction in f64, exact because the launcher keeps
//        |zp| <= 2^15 and K < 2^17 (every term below 2^53).
//   SUMS: ra / cw come from the accumulators of PolicyI8Q (each wave's own
//        per-lane partial sums of the fragments it multiplied, combined over
//        the two k-halves and moved into the accumulator layout with lane
//        shuffles at the tile's end) instead of a pre-pass; row_sums /
//        col_sums are not read.
__device__ __forceinline__ int32_t acc_int(const v16i& a, int r) { return a[r]; }
__device__ __forceinline__ int32_t acc_int(const AccQ& a, int r) { return a.v[r]; }

template <bool I32, bool SUMS = false>
struct EpiQL {
    static constexpr bool kOut32 = false;  // int8 outputs: stored at the tile's end
    const int32_t* row_sums;  // [M]
    const int32_t* col_sums;  // [N]
    int32_t zpa, zpw, zpy;
    int64_t kzz;              // K * zpa * zpw
    double mult;

    template <class C>
    struct Operands {
        int32_t rt[C::TM][16];  // I32: K zpa zpw - zpw ra; else ra
        int32_t ct[C::TN];      // I32: zpa cw; else cw
        // see EpiOperands::pinned
        __device__ __forceinline__ Operands pinned() const {
            Operands o = *this;
#pragma unroll
            for (int i = 0; i < C::TM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) o.rt[i][r] = pin(o.rt[i][r]);
#pragma unroll
            for (int j = 0; j < C::TN; j++) o.ct[j] = pin(o.ct[j]);
            return o;
        }
    };

    // Rows past M read row M - 1 and columns past N column N - 1 (never stored).
    template <class C>
    __device__ __forceinline__ Operands<C> load(int m0, int n0, int M, int N) const {
        Operands<C> o;
        if constexpr (SUMS) return o;
        const int lane = threadIdx.x & 63, wave = wave_id();
        const int wm = wave / C::WN, wn = wave % C::WN, khalf = lane >> 5;
#pragma unroll
        for (int i = 0; i < C::TM; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + wm * C::WTM + i * 32 + acc_row(r, khalf);
                const int32_t ra = row_sums[row < M ? row : M - 1];
                o.rt[i][r] = I32 ? (int32_t)((uint32_t)kzz - (uint32_t)zpw * (uint32_t)ra) : ra;
            }
#pragma unroll
        for (int j = 0; j < C::TN; j++) {
            const int col = n0 + wn * C::WTN + j * 32 + (lane & 31);
            const int32_t cw = col_sums[col < N ? col : N - 1];
            o.ct[j] = I32 ? (int32_t)((uint32_t)zpa * (uint32_t)cw) : cw;
        }
        return o;
    }

    // The row / column terms from PolicyI8Q's partial sums (SUMS).
    template <class C, class P>
    __device__ __forceinline__ Operands<C> from_sums(
        const typename P::Acc (&acc)[C::TM][C::TN]) const {
        Operands<C> o;
        const int khalf = (threadIdx.x & 63) >> 5;
#pragma unroll
        for (int i = 0; i < C::TM; i++) {
            const int part = acc[i][0].rs;
            const int full = part + __shfl_xor(part, 32, 64);  // row (lane % 32), all of K
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int32_t ra = __shfl(full, acc_row(r, khalf), 64);
                o.rt[i][r] = I32 ? (int32_t)((uint32_t)kzz - (uint32_t)zpw * (uint32_t)ra) : ra;
            }
        }
#pragma unroll
        for (int j = 0; j < C::TN; j++) {
            const int part = acc[0][j].cs;
            const int32_t cw = part + __shfl_xor(part, 32, 64);
            o.ct[j] = I32 ? (int32_t)((uint32_t)zpa * (uint32_t)cw) : cw;
        }
        return o;
    }

    template <class C, class P, class F>
    __device__ __forceinline__ void with_value(const typename P::Acc (&acc)[C::TM][C::TN],
                                               const Operands<C>& o_in, F&& f) const {
        Operands<C> o;
        if constexpr (SUMS)
            o = from_sums<C, P>(acc);
        else
            o = o_in.pinned();
        if constexpr (I32) {
            // clamp(rint(p) + zpy) == clamp(rint(p), -128 - zpy, 127 - zpy) + zpy for an
            // integer zpy; the launcher takes this path only for a finite mult, so p
            // is never NaN
            const double lo = -128.0 - (double)zpy, hi = 127.0 - (double)zpy;
            f([&](int i, int j, int r) {
                const int32_t a = (int32_t)((uint32_t)pin(acc_int(acc[i][j], r)) +
                                            (uint32_t)o.rt[i][r] - (uint32_t)o.ct[j]);
                double v = __builtin_rint((double)a * mult);
                v = v < lo ? lo : (v > hi ? hi : v);
                return (uint32_t)((int32_t)v + zpy);
            });
        } else {
            const double kzz_d = (double)kzz, zpw_d = (double)zpw, zpa_d = (double)zpa;
            f([&](int i, int j, int r) {
                const double row = kzz_d - zpw_d * (double)o.rt[i][r];
                const double a =
                    ((double)pin(acc_int(acc[i][j], r)) + row) - zpa_d * (double)o.ct[j];
                double v = __builtin_rint(a * mult);
                if (v != v) v = 0.0;
                v = v + (double)zpy;
                v = v < -128.0 ? -128.0 : (v > 127.0 ? 127.0 : v);
                return (uint32_t)(int32_t)v;
            });
        }
    }

    template <class C, class P, int P0 = 0, int NP = C::TM * 16>
    __device__ __forceinline__ void store(const typename P::Acc (&acc)[C::TM][C::TN],
                                          const Operands<C>& o, int m0, int n0, int M, int N,
                                          void* __restrict__ Y) const {
        with_value<C, P>(acc, o, [&](auto&& value) {
            write_tile<C, P0, NP>(static_cast<int8_t*>(Y), m0, n0, M, N, value);
        });
    }

    template <class C, class P>
    __device__ __forceinline__ void values(const typename P::Acc (&)[C::TM][C::TN],
                                           const Operands<C>&,
                                           uint32_t (&)[C::TM][C::TN][16]) const {}
};

// Persistent workgroups: workgroup b owns tiles b, b + G, b + 2G, ... (G =
// grid size, a multiple of the XCD count, so every tile a workgroup visits
// stays in its XCD's range).  The next tile's first slices are issued before
// the current tile's epilogue, so its DMA latency overlaps the output stores.
template <class C, class P, class E>
__global__ __launch_bounds__(C::THREADS) void k_gemm(const uint8_t* __restrict__ A,
                                                     const uint8_t* __restrict__ W, int M, int N,
                                                     int ldk, E ep, void* __restrict__ Y) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[C::LDS_BYTES];
    const int tiles_n = (N + C::BN - 1) / C::BN;
    const int tiles = ((M + C::BM - 1) / C::BM) * tiles_n;
    int v = blockIdx.x;
    int t = xcd_tile(v, tiles);
    int m0 = (t / tiles_n) * C::BM, n0 = (t % tiles_n) * C::BN;
    prologue<C>(A, W, M, N, ldk, m0, n0, smem);
    for (;;) {
        typename P::Acc acc[C::TM][C::TN];
#pragma unroll
        for (int i = 0; i < C::TM; i++)
#pragma unroll
            for (int j = 0; j < C::TN; j++) P::zero(acc[i][j]);
        const auto eo = ep.template load<C>(m0, n0, M, N);
        mainloop<C, P>(A, W, M, N, ldk, m0, n0, smem, acc);
        const int vn = v + (int)gridDim.x;
        const bool more = vn < tiles;
        int m0n = 0, n0n = 0;
        if (more) {
            const int tn = xcd_tile(vn, tiles);
            m0n = (tn / tiles_n) * C::BM;
            n0n = (tn % tiles_n) * C::BN;
            barrier();  // every wave is done reading the ring
            prologue<C>(A, W, M, N, ldk, m0n, n0n, smem);
        }
        ep.template store<C, P>(acc, eo, m0, n0, M, N, Y);
        if (!more) break;
        v = vn;
        m0 = m0n;
        n0 = n0n;
    }
}

// Stores part `part` (wave-uniform, run time, < C::TM * 16 <= 64) of a
// wave's finished output values, the wave's tile lying inside [M, N]: yw is
// the wave tile's first output, loff the lane's offset from it.  One scalar
// jump to the compile-time part, no bounds checks.
template <class C>
__device__ __forceinline__ void store_part_dyn(int part, const uint32_t (&v)[C::TM][C::TN][16],
                                               uint32_t* __restrict__ yw, int N, uint32_t loff) {
    static_assert(C::TM * 16 <= 64, "parts");
    switch (part) {
#define TKV_PART(p)                                                                      \
    case (p):                                                                            \
        if constexpr ((p) < C::TM * 16) {                                                \
            constexpr int i = (p) / 16 < C::TM ? (p) / 16 : 0, r = (p) % 16;            \
            uint32_t* rowp = yw + (int64_t)(i * 32 + (r >> 2) * 8 + (r & 3)) * N;        \
            _Pragma("unroll") for (int j = 0; j < C::TN; j++)                            \
                put(rowp + loff + j * 32, v[i][j][r]);                                   \
        }                                                                                \
        break;
#define TKV_PART8(p) TKV_PART(p) TKV_PART(p + 1) TKV_PART(p + 2) TKV_PART(p + 3) \
    TKV_PART(p + 4) TKV_PART(p + 5) TKV_PART(p + 6) TKV_PART(p + 7)
        TKV_PART8(0) TKV_PART8(8) TKV_PART8(16) TKV_PART8(24)
        TKV_PART8(32) TKV_PART8(40) TKV_PART8(48) TKV_PART8(56)
#undef TKV_PART8
#undef TKV_PART
        default: break;
    }
}

// Warp-specialised persistent GEMM (CfgWS).  Workgroup b owns tiles b, b + G,
// ...; its K slices form one stream s = 0 .. my_tiles * nk - 1 that the
// producer waves keep STAGES - 1 slices ahead of, across tile boundaries.
// Both roles pass one s_barrier per slice (plus one before the first):
//   producers: issue slice s + STAGES - 1 into the slot freed by slice s - 1,
//              wait (own vmcnt) for slice s + 1, barrier;
//   consumers: MFMAs on slice s, barrier; after a tile's last slice, the
//              epilogue.  They never wait on vmcnt for operand data, so the
//              epilogue's stores drain while the next tile's slices stream in.
// The barrier after slice s both publishes slice s + 1 to the consumers and
// tells the producers that slice s's slot is free again.
template <class C, class P, class E>
__global__ __launch_bounds__(C::THREADS, C::MIN_WAVES_EU) void k_gemm_ws(const uint8_t* __restrict__ A,
                                                        const uint8_t* __restrict__ W, int M,
                                                        int N, int ldk, E ep,
                                                        void* __restrict__ Y, int stagger) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[C::LDS_BYTES];
    const int tiles_n = (N + C::BN - 1) / C::BN;
    const int tiles = ((M + C::BM - 1) / C::BM) * tiles_n;
    const int G = (int)gridDim.x, b = (int)blockIdx.x;
    // Every other workgroup of each XCD starts `stagger` x 1024 cycles late
    // (see launch_ws).
    if ((b >> 3) & 1)
        for (int i = 0; i < stagger; i++) __builtin_amdgcn_s_sleep(16);
    const int my_tiles = b < tiles ? (tiles - 1 - b) / G + 1 : 0;
    const int nk = ldk / C::BK;
    const int total = my_tiles * nk;
    const int lane = threadIdx.x & 63, wave = wave_id();

    if (wave >= C::CW) {
        // Producer.  `ops` counts this wave's VMEM instructions; done[q % S]
        // holds the count right after slice q's DMAs, so waiting for slice q
        // is vmcnt(ops - done[q % S]) (vmcnt retires in issue order).  The
        // issue cursor (ti, kt) advances without divisions; lane offsets are
        // recomputed once per tile.
        const int pw = wave - C::CW;
        int issued = 0, ops = 0, ti = 0, kt = 0;
        int done[C::STAGES];
        WsLane<C> L;
        const uint8_t *a_tile = A, *w_tile = W;
        auto issue_next = [&]() {
            if (kt == 0) {
                const int t = xcd_tile(b + ti * G, tiles);
                const int tm = t / tiles_n;
                const int m0 = tm * C::BM, n0 = (t - tm * tiles_n) * C::BN;
                a_tile = A + (int64_t)m0 * ldk;
                w_tile = W + (int64_t)n0 * ldk;
                ws_lane_offsets<C>(M, N, ldk, m0, n0, pw, lane, L);
            }
            const int slot = issued % C::STAGES;
            ws_issue<C>(a_tile, w_tile, kt * C::BK, L, smem + slot * C::STAGE_BYTES, pw);
            ops += C::LPS;
#pragma unroll
            for (int i = 0; i < C::STAGES; i++)
                if (i == slot) done[i] = ops;
            issued++;
            if (++kt == nk) {
                kt = 0;
                ti++;
            }
        };
        auto wait_for = [&](int q) {
            int d = 0;
#pragma unroll
            for (int i = 0; i < C::STAGES; i++)
                if (i == q % C::STAGES) d = done[i];
            wait_vmcnt_dyn(ops - d);
        };
        while (issued < C::STAGES - 1 && issued < total) issue_next();
        if (total > 0) wait_for(0);
        barrier();
        for (int s = 0; s < total; s++) {
            if (issued < total) issue_next();
            if (s + 1 < total) wait_for(s + 1);
            barrier();
        }
        return;
    }

    const int wm = wave / C::WN, wn = wave % C::WN, khalf = lane >> 5;
    int a_row[C::TM], w_row[C::TN];
#pragma unroll
    for (int i = 0; i < C::TM; i++) a_row[i] = wm * C::WTM + i * 32 + (lane & 31);
#pragma unroll
    for (int j = 0; j < C::TN; j++) w_row[j] = wn * C::WTN + j * 32 + (lane & 31);
    barrier();
    int s = 0;
    if constexpr (!C::DEFER || !E::kOut32) {
        for (int ti = 0; ti < my_tiles; ti++) {
            const int t = xcd_tile(b + ti * G, tiles);
            const int m0 = (t / tiles_n) * C::BM, n0 = (t % tiles_n) * C::BN;
            typename P::Acc acc[C::TM][C::TN];
#pragma unroll
            for (int i = 0; i < C::TM; i++)
#pragma unroll
                for (int j = 0; j < C::TN; j++) P::zero(acc[i][j]);
            const auto eo = ep.template load<C>(m0, n0, M, N);
            for (int kt = 0; kt < nk; kt++, s++) {
                const uint8_t* sa = smem + (s % C::STAGES) * C::STAGE_BYTES;
                P::template slice<C>(sa, sa + C::A_BYTES, a_row, w_row, khalf, acc);
                if constexpr (shares_sums<P>::value)
                    if (kt == nk - 1) P::template publish<C>(acc, ti & 1);
                barrier();
            }
            if constexpr (shares_sums<P>::value) P::template gather<C>(acc, ti & 1);
            ep.template store<C, P>(acc, eo, m0, n0, M, N, Y);
        }
    } else {
        // Deferred stores: a finished tile is turned into its output values
        // (the epilogue arithmetic runs once, at the tile's end) and those are
        // stored during the next tile's K slices, one even share of the
        // C::TM * 16 parts after each slice's MFMAs, so the HBM writes drain
        // while the matrix cores work instead of stalling the consumers
        // between tiles.  Wave tiles crossing the M / N edge are stored at
        // once (with bounds checks); the last tile's values at the end.
        constexpr int NPART = C::TM * 16;
        uint32_t pv[C::TM][C::TN][16];
        uint32_t* Y32 = static_cast<uint32_t*>(Y);
        const uint32_t loff = (uint32_t)(khalf * 4) * (uint32_t)N + (uint32_t)(lane & 31);
        uint32_t* yw = Y32;
        bool have = false;
        for (int ti = 0; ti < my_tiles; ti++) {
            const int t = xcd_tile(b + ti * G, tiles);
            const int m0 = (t / tiles_n) * C::BM, n0 = (t % tiles_n) * C::BN;
            typename P::Acc acc[C::TM][C::TN];
#pragma unroll
            for (int i = 0; i < C::TM; i++)
#pragma unroll
                for (int j = 0; j < C::TN; j++) P::zero(acc[i][j]);
            const auto eo = ep.template load<C>(m0, n0, M, N);
            for (int kt = 0; kt < nk; kt++, s++) {
                const uint8_t* sa = smem + (s % C::STAGES) * C::STAGE_BYTES;
                P::template slice<C>(sa, sa + C::A_BYTES, a_row, w_row, khalf, acc);
                if (have)
                    for (int part = kt * NPART / nk; part < (kt + 1) * NPART / nk; part++)
                        store_part_dyn<C>(part, pv, yw, N, loff);
                barrier();
            }
            const int rbase = m0 + wm * C::WTM, cbase = n0 + wn * C::WTN;
            if (rbase + C::WTM <= M && cbase + C::WTN <= N) {
                ep.template values<C, P>(acc, eo, pv);
                yw = Y32 + (int64_t)rbase * N + cbase;
                have = true;
            } else {
                ep.template store<C, P>(acc, eo, m0, n0, M, N, Y);
                have = false;
            }
        }
        if (have)
            for (int part = 0; part < NPART; part++) store_part_dyn<C>(part, pv, yw, N, loff);
    }
}

// Fused-role persistent GEMM (Cfg): every wave both copies its share of the
// operand slices (LDS DMA) and runs MFMAs, two waves per SIMD.  A wave that
// issues a DMA instruction waits until the CU's address unit accepts it, and
// while any wave on a SIMD streams MFMAs, a separate DMA-only wave on that
// SIMD is served only in the gaps (timed on the box: 1 KB DMAs from L2 at
// 16.7 B/clk per CU beside four MFMA waves, against 51.8 B/clk alone).  So
// here the DMA instructions of slice kt + STAGES - 1 are spread one at a time
// between the MFMAs of slice kt: while one wave of a SIMD waits on its DMA
// issue, the other runs its MFMAs.  One barrier per slice, as in mainloop();
// the next tile's first slices are issued before the current tile's stores.
template <class C>
struct FusedDma {
    // per-lane byte offsets of the wave's DMA blocks from the tile's first
    // row (rows past M / N clamped), and their LDS offsets in a ring slot
    uint32_t off[C::A_DMA_W + C::W_DMA_W];
    uint32_t lds[C::A_DMA_W + C::W_DMA_W];
};

template <class C>
__device__ __forceinline__ void fused_offsets(int M, int N, int ldk, int m0, int n0, int wave,
                                              int lane, FusedDma<C>& F) {
    const int lrow = lane / C::CH, lch = lane % C::CH;
#pragma unroll
    for (int d = 0; d < C::A_DMA_W + C::W_DMA_W; d++) {
        const bool is_a = d < C::A_DMA_W;
        const int blk = is_a ? wave * C::A_DMA_W + d : wave * C::W_DMA_W + (d - C::A_DMA_W);
        const int row = blk * C::ROWS_PER_DMA + lrow;
        const int c = lch ^ swz<C::CH>(row);
        const int lim = is_a ? M - 1 - m0 : N - 1 - n0;
        F.off[d] = (uint32_t)(row < lim ? row : lim) * (uint32_t)ldk + (uint32_t)(c * 16);
        F.lds[d] = is_a ? blk * 1024 : C::A_BYTES + blk * 1024;
    }
}

template <class C>
__device__ __forceinline__ void fused_issue(const uint8_t* a_tile, const uint8_t* w_tile,
                                            const FusedDma<C>& F, int d, int kslice,
                                            uint8_t* smem) {
    const bool is_a = d < C::A_DMA_W;
    const uint8_t* g = (is_a ? a_tile : w_tile) + (int64_t)kslice * C::BK + F.off[d];
    uint8_t* dst = smem + (kslice % C::STAGES) * C::STAGE_BYTES + F.lds[d];
    __builtin_amdgcn_global_load_lds((const void*)g, (lds_ptr)dst, 16, 0, 0);
}

// One slice of INT8 MFMAs (as PolicyI8::slice) with the DMA blocks of slice
// `nxt` issued between them when `dma` is set: DMA d follows MFMA
// d * NMF / LPS of the NMF in the slice.
template <class C, class P>
__device__ __forceinline__ void fused_slice(const uint8_t* sa, const uint8_t* sw,
                                            const int (&a_row)[C::TM], const int (&w_row)[C::TN],
                                            int khalf, typename P::Acc (&acc)[C::TM][C::TN],
                                            bool dma, const uint8_t* a_tile,
                                            const uint8_t* w_tile, const FusedDma<C>& F, int nxt,
                                            uint8_t* smem) {
    constexpr int KS = C::BK / 32, D = C::FRAG_DEPTH;
    constexpr int LPS = C::A_DMA_W + C::W_DMA_W, NMF = KS * C::TM * C::TN;
    v4i af[KS][C::TM], bf[KS][C::TN];
    auto load = [&](int ks) {
        const int ch = ks * 2 + khalf;
#pragma unroll
        for (int i = 0; i < C::TM; i++) af[ks][i] = lds_chunk<C>(sa, a_row[i], ch);
#pragma unroll
        for (int j = 0; j < C::TN; j++) bf[ks][j] = lds_chunk<C>(sw, w_row[j], ch);
    };
#pragma unroll
    for (int ks = 0; ks < D - 1 && ks < KS; ks++) load(ks);
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
        if (ks + D - 1 < KS) load(ks + D - 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < C::TM; i++)
#pragma unroll
            for (int j = 0; j < C::TN; j++) {
                acc[i][j] = P::mfma(af[ks][i], bf[ks][j], acc[i][j]);
                const int f = (ks * C::TM + i) * C::TN + j;
#pragma unroll
                for (int d = 0; d < LPS; d++)
                    if (f == d * NMF / LPS) {
                        __builtin_amdgcn_sched_barrier(0);
                        if (dma) fused_issue<C>(a_tile, w_tile, F, d, nxt, smem);
                        __builtin_amdgcn_sched_barrier(0);
                    }
            }
        __builtin_amdgcn_sched_barrier(0);
    }
}

template <class C, class P, class E>
__global__ __launch_bounds__(C::THREADS, 2) void k_gemm_f(const uint8_t* __restrict__ A,
                                                          const uint8_t* __restrict__ W, int M,
                                                          int N, int ldk, E ep,
                                                          void* __restrict__ Y) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[C::LDS_BYTES];
    constexpr int LPS = C::A_DMA_W + C::W_DMA_W;
    const int tiles_n = (N + C::BN - 1) / C::BN;
    const int tiles = ((M + C::BM - 1) / C::BM) * tiles_n;
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int wm = wave / C::WN, wn = wave % C::WN, khalf = lane >> 5;
    const int nk = ldk / C::BK;
    int a_row[C::TM], w_row[C::TN];
#pragma unroll
    for (int i = 0; i < C::TM; i++) a_row[i] = wm * C::WTM + i * 32 + (lane & 31);
#pragma unroll
    for (int j = 0; j < C::TN; j++) w_row[j] = wn * C::WTN + j * 32 + (lane & 31);

    int v = blockIdx.x;
    if (v >= tiles) return;
    int t = xcd_tile(v, tiles);
    int m0 = (t / tiles_n) * C::BM, n0 = (t % tiles_n) * C::BN;
    FusedDma<C> F;
    fused_offsets<C>(M, N, ldk, m0, n0, wave, lane, F);
    const uint8_t* a_tile = A + (int64_t)m0 * ldk;
    const uint8_t* w_tile = W + (int64_t)n0 * ldk;
    auto prologue_f = [&]() {
#pragma unroll
        for (int s = 0; s < C::STAGES - 1; s++)
            if (s < nk)
#pragma unroll
                for (int d = 0; d < LPS; d++) fused_issue<C>(a_tile, w_tile, F, d, s, smem);
    };
    prologue_f();
    for (;;) {
        typename P::Acc acc[C::TM][C::TN];
#pragma unroll
        for (int i = 0; i < C::TM; i++)
#pragma unroll
            for (int j = 0; j < C::TN; j++) P::zero(acc[i][j]);
        const auto eo = ep.template load<C>(m0, n0, M, N);
        wait_slice<C>((C::STAGES - 2) < (nk - 1) ? (C::STAGES - 2) : (nk - 1));
        barrier();
        for (int kt = 0; kt < nk; kt++) {
            const int nxt = kt + C::STAGES - 1;
            const uint8_t* sa = smem + (kt % C::STAGES) * C::STAGE_BYTES;
            fused_slice<C, P>(sa, sa + C::A_BYTES, a_row, w_row, khalf, acc, nxt < nk, a_tile,
                              w_tile, F, nxt, smem);
            if (kt + 1 < nk) {
                const int last = nxt < nk ? nxt : nk - 1;
                wait_slice<C>(last - (kt + 1));
                barrier();
            }
        }
        const int vn = v + (int)gridDim.x;
        const bool more = vn < tiles;
        const int m0c = m0, n0c = n0;
        if (more) {
            const int tn = xcd_tile(vn, tiles);
            m0 = (tn / tiles_n) * C::BM;
            n0 = (tn % tiles_n) * C::BN;
            fused_offsets<C>(M, N, ldk, m0, n0, wave, lane, F);
            a_tile = A + (int64_t)m0 * ldk;
            w_tile = W + (int64_t)n0 * ldk;
            barrier();  // every wave is done reading the ring
            prologue_f();
        }
        ep.template store<C, P>(acc, eo, m0c, n0c, M, N, Y);
        if (!more) break;
        v = vn;
    }
}

// Skinny INT8 GEMM for decode batches (M <= 32): the weight is streamed
// from HBM once and every activation row is reused from L2.  Workgroup b owns
// output columns [32 b, 32 b + 32); its KW waves split the K steps (wave w
// takes steps w, w + KW, ...), each wave loads all of its A and W fragments
// before its MFMAs (v_mfma_i32_32x32x32_i8, A rows past M repeat row M - 1
// and are never stored), the partial INT32 tiles are summed exactly with LDS
// atomics, and wave 0 runs the same epilogue as the tiled kernels on the
// 32 x 32 tile.
__device__ __forceinline__ int lines_swz(int row) { return (row & 7) ^ (row >> 3); }

struct CfgGemv {
    static constexpr int BM = 32, BN = 32, WM = 1, WN = 1, WTM = 32, WTN = 32, TM = 1, TN = 1;
};
constexpr int kGemvMaxM = 32;
constexpr int kGemvUnroll = 8;

// LINES: the workgroup's 32 weight rows over its K range go into LDS first
// by direct DMA, whole 128-byte lines of 8 rows per 1 KB instruction (the
// rows' 16-byte chunks XOR-swizzled so that 16 lanes reading one chunk of 16
// rows hit distinct bank groups), and the B operands are read from there; a
// direct B load reads 32 bytes of each of 32 rows' lines per instruction.
// ldk % 128 == 0; dynamic LDS: 4 KB per 128-byte line of the K range.
// SPLIT: workgroup b takes column block b % ncb and the K steps of split
// b / ncb (of `splits`), so narrow N still spreads over the CUs.  Its INT32
// partial sums go into part[block][1024] with device-scope atomic adds (exact
// in any order); once those adds have completed it counts itself into
// arrivals[block] with another device-scope atomic.  The workgroup that
// completes the count takes the sums with an exchange that also clears them,
// clears the count, and runs the epilogue: no workgroup ever waits for
// another, and part / arrivals are zero again when the kernel ends (zeroed at
// context creation).
template <int KW, bool SPLIT, class E, bool LINES = false>
__global__ __launch_bounds__(KW * 64) void k_gemv_i8(const uint8_t* __restrict__ A,
                                                     const uint8_t* __restrict__ W, int M, int N,
                                                     int ldk, E ep, void* __restrict__ Y,
                                                     int splits, int32_t* __restrict__ part,
                                                     unsigned* __restrict__ arrivals) {
    __shared__ int32_t red[16 * 64];
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int ncb = (N + 31) / 32;
    const int cb = SPLIT ? (int)blockIdx.x % ncb : (int)blockIdx.x;
    const int sp = SPLIT ? (int)blockIdx.x / ncb : 0;
    const int n0 = cb * 32;
    const int r = lane & 31, kh = lane >> 5;
    for (int i = threadIdx.x; i < 16 * 64; i += KW * 64) red[i] = 0;
    const auto eo = ep.template load<CfgGemv>(0, n0, M, N);
    const uint8_t* arow = A + (int64_t)(r < M ? r : M - 1) * ldk + kh * 16;
    const uint8_t* wrow = W + (int64_t)(n0 + r < N ? n0 + r : N - 1) * ldk + kh * 16;
    const int nks = ldk / 32;
    const int k_lo = SPLIT ? (int)((int64_t)nks * sp / splits) : 0;
    const int k_hi = SPLIT ? (int)((int64_t)nks * (sp + 1) / splits) : nks;
    v16i acc;
#pragma unroll
    for (int i = 0; i < 16; i++) acc[i] = 0;
    // LINES: lines [p_lo, p_hi) of the K range; instruction d = 4 (p - p_lo)
    // + h holds rows 8 h .. 8 h + 7, lane 8 rr + q taking chunk q ^
    // lines_swz(8 h + rr)
    extern __shared__ __attribute__((aligned(16))) uint8_t s_wl[];
    const int p_lo = k_lo >> 2;
    auto wfrag = [&](int ks) -> v4i {
        if constexpr (LINES) {
            const int ch = 2 * (ks & 3) + kh;
            return *reinterpret_cast<const v4i*>(
                s_wl + ((4 * ((ks >> 2) - p_lo) + (r >> 3)) << 10) +
                ((((r & 7) << 3) + (ch ^ lines_swz(r & 15))) << 4));
        } else {
            return __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wrow + ks * 32));
        }
    };
    if constexpr (LINES) {
        const int nd = 4 * (((k_hi + 3) >> 2) - p_lo);
        const int rr = lane >> 3, q = lane & 7;
        for (int d = wave; d < nd; d += KW) {
            const int row = 8 * (d & 3) + rr;
            const int col = n0 + row < N ? n0 + row : N - 1;
            const uint8_t* g = W + (int64_t)col * ldk + (int64_t)(p_lo + (d >> 2)) * 128 +
                               ((q ^ lines_swz(row & 15)) << 4);
            __builtin_amdgcn_global_load_lds((const void*)g, (lds_ptr)(s_wl + d * 1024), 16, 0,
                                             0);
        }
        // each wave's DMAs have landed, then a raw barrier publishes them
        // all (__syncthreads() would also wait, being a release fence)
        wait_vmcnt<0>();
        barrier();
    }
    int ks = k_lo + wave;
    for (; ks + (kGemvUnroll - 1) * KW < k_hi; ks += kGemvUnroll * KW) {
        v4i af[kGemvUnroll], wf[kGemvUnroll];
#pragma unroll
        for (int u = 0; u < kGemvUnroll; u++) {
            af[u] = *reinterpret_cast<const v4i*>(arow + (ks + u * KW) * 32);
            wf[u] = wfrag(ks + u * KW);
        }
#pragma unroll
        for (int u = 0; u < kGemvUnroll; u++)
            acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[u], wf[u], acc, 0, 0, 0);
    }
    for (; ks < k_hi; ks += KW) {
        const v4i af = *reinterpret_cast<const v4i*>(arow + ks * 32);
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, wfrag(ks), acc, 0, 0, 0);
    }
    __syncthreads();  // red[] zeroed
    typename PolicyI8::Acc sum[1][1];
    if constexpr (KW == 1) {
        sum[0][0] = acc;
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) atomicAdd(&red[i * 64 + lane], acc[i]);
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int i = 0; i < 16; i++) sum[0][0][i] = red[i * 64 + lane];
    }
    if constexpr (SPLIT) {
        int32_t* pc = part + (int64_t)cb * 1024;
#pragma unroll
        for (int i = 0; i < 16; i++)
            __hip_atomic_fetch_add(pc + i * 64 + lane, sum[0][0][i], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        // Every access to part[] and arrivals[] is a device-scope atomic
        // (the adds, the count, the exchanges that read the sums), performed
        // where every XCD sees it.  The wave waits for its adds to complete
        // (vmcnt counts atomics and retires in issue order) before lane 0
        // issues the arrival, and the exchanges issue only after the
        // arrival has returned.  That is the hardware's ordering of this
        // wave's own memory operations, not a release / acquire pair of the
        // HIP memory model: agent-scope fences (an L2 writeback before the
        // arrival, an L2 invalidate before the exchanges) made the split
        // call 4.2 us slower (mlp_down decode shape, 6.6 -> 10.8 us at
        // M = 1, three interleaved rounds on one box), so they are not used.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        int last = 0;
        if (lane == 0)
            last = __hip_atomic_fetch_add(arrivals + cb, 1u, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(splits - 1);
        if (!__shfl(last, 0, 64)) return;
#pragma unroll
        for (int i = 0; i < 16; i++)
            sum[0][0][i] = __hip_atomic_exchange(pc + i * 64 + lane, 0, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
        if (lane == 0)
            __hip_atomic_store(arrivals + cb, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    ep.template store<CfgGemv, PolicyI8>(sum, eo, 0, n0, M, N, Y);
}

// ---- tile configurations ---------------------------------------------------
// K slices are 128 bytes: one full L2 line per row per DMA (64-byte slices
// fetch every line twice and halve the DMA throughput).
//            BM   BN  WM WN   BK  STAGES
typedef Cfg<64, 128, 2, 2, 128, 3> Cfg0;   //  72 KB, small M (tiles < CUs)
typedef Cfg<128, 192, 4, 2, 128, 3> Cfg1;  // 120 KB, 8 waves, 32x96 wave tiles
// warp-specialised:  BM   BN  WM WN   BK  STAGES PW DEFER FD
// (cfg 7 and 9 defer each tile's stores into the next tile's K slices; at
// M = 8192 they win on the N = 768 shapes by a few percent and lose on the
// wide ones, where the extra values cost fragment read-ahead: cfg 2 stays
// the default)
typedef CfgWS<128, 192, 4, 2, 128, 3, 4> Cfg2;     // 120 KB, 8 consumers (32x96) + 4 producers
typedef CfgWS<128, 192, 2, 2, 128, 3, 4> Cfg3;     // 120 KB, 4 consumers (64x96) + 4 producers
typedef CfgWS<128, 128, 2, 2, 128, 3, 4> Cfg4;     //  96 KB, 4 consumers (64x64) + 4 producers
typedef CfgWS<64, 128, 2, 2, 128, 3, 4> Cfg5;      //  72 KB, 4 consumers (32x64) + 4 producers
typedef CfgWS<128, 192, 4, 2, 128, 4, 4> Cfg6;     // 160 KB, 3 slices in flight
typedef CfgWS<128, 192, 4, 2, 128, 3, 4, 1, 1> Cfg7;  // Cfg2 + stores spread over the next tile
typedef CfgWS<128, 192, 4, 3, 128, 3, 4> Cfg8;     // 120 KB, 12 consumers (32x64) + 4 producers
typedef CfgWS<128, 192, 4, 3, 128, 3, 4, 1, 1> Cfg9;  // Cfg8 + stores spread over the next tile
// fused roles (k_gemm_f): every wave copies its share of the operands and
// runs MFMAs; 80 KB of LDS, so two workgroups share a CU and one's output
// stores overlap the other's K loop
typedef Cfg<128, 192, 2, 2, 128, 2> Cfg11;  //  80 KB, 4 waves (64x96), two workgroups per CU

constexpr int kBK = 128;

template <class C>
static int64_t tiles_of(int64_t m, int64_t n) {
    return ceil_div(m, C::BM) * ceil_div(n, C::BN);
}

// Tile choice: the largest tile that still gives every CU work; the
// context's TKV_HIP_TUNE_GEMM_CFG override (0..11; 2.. are the warp-
// specialised configurations, 10 the skinny kernel for INT8 with M <= 32, 11
// the fused-role kernel) forces one.
static inline int pick_cfg(Ctx* c, int64_t m, int64_t n) {
    const int64_t f = tuned(c, TKV_HIP_TUNE_GEMM_CFG);
    if (f >= 0) return (int)f;
    // Warp-specialised 128x192 tiles (cfg 2) measured best over the four
    // GPT-2 shapes at M = 8192 (warmed-up, interleaved medians); 64x128 tiles
    // keep every CU busy when M is small.  The switch is at three quarters of
    // the CUs: at M = 2048, qkv's 192 tiles ran 10.2 us with cfg 2 against
    // 11.4 (FP8) / 12.5 (INT8) with cfg 0, while attn_out and mlp_down (64
    // tiles) ran 6.2 / 13.8 us with cfg 0 against 8.9 / 19.1 (one box, two
    // rounds, HIP events).
    return tiles_of<Cfg2>(m, n) * 4 >= (int64_t)c->num_cus * 3 ? 2 : 0;
}

template <class C, class P, class E>
static int launch_cfg(Ctx* c, const uint8_t* a, const uint8_t* w, int64_t m, int64_t n,
                      int64_t ldk, const E& ep, void* y) {
    // one wave of resident workgroups (LDS-limited); a multiple of 8 (XCDs)
    // whenever tiles outnumber it
    const int64_t per_cu = 163840 / C::LDS_BYTES > 0 ? 163840 / C::LDS_BYTES : 1;
    const int64_t resident = (int64_t)c->num_cus * per_cu;
    const int64_t tiles = tiles_of<C>(m, n);
    const int64_t grid = tiles < resident ? tiles : resident;
    hipLaunchKernelGGL((k_gemm<C, P, E>), dim3((unsigned)grid), dim3(C::THREADS), 0, c->stream,
                       a, w, (int)m, (int)n, (int)ldk, ep, y);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

template <class C, class P, class E>
static int launch_f(Ctx* c, const uint8_t* a, const uint8_t* w, int64_t m, int64_t n,
                    int64_t ldk, const E& ep, void* y) {
    const int64_t per_cu = 163840 / C::LDS_BYTES > 0 ? 163840 / C::LDS_BYTES : 1;
    const int64_t resident = (int64_t)c->num_cus * per_cu;
    const int64_t tiles = tiles_of<C>(m, n);
    const int64_t grid = tiles < resident ? tiles : resident;
    hipLaunchKernelGGL((k_gemm_f<C, P, E>), dim3((unsigned)grid), dim3(C::THREADS), 0, c->stream,
                       a, w, (int)m, (int)n, (int)ldk, ep, y);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

// The fused-role kernel runs policies whose fragments are one 16-byte chunk
// per lane and k-step and that need nothing besides the MFMAs; the FP8
// full-rate policy and the row-summing PolicyI8Q take the plain tile kernel.
template <class C, class P, class E>
static int launch_fused(Ctx* c, const uint8_t* a, const uint8_t* w, int64_t m, int64_t n,
                        int64_t ldk, const E& ep, void* y) {
    if constexpr (std::is_same_v<P, PolicyF8> || std::is_same_v<P, PolicyI8Q>)
        return launch_cfg<C, P>(c, a, w, m, n, ldk, ep, y);
    else
        return launch_f<C, P>(c, a, w, m, n, ldk, ep, y);
}

// Start stagger of the persistent kernel, in units of s_sleep 16 (1024
// cycles, ~0.4 us).  Every workgroup runs the same sequence of equal tiles, so
// without it all CUs issue their output stores at the same moments: each
// burst saturates the HBM write path while the next tile's operand DMA waits
// behind the stores in the CU's memory pipeline.  Delaying every other
// workgroup of each XCD by ~1.7 us puts half of the machine's store bursts
// into the other half's K loops.  Measured over the four GPT-2 shapes at
// M = 8192 (sum of back-to-back GEMM times, interleaved medians, two boxes):
// 95.2 and 96.9 us against 97.8 and 99.2 us without; longer delays or four
// phase groups were slower.  Epilogues with int8 outputs (QLinearMatMul)
// store a quarter of the bytes and only lose the delay (attn_out 12.9 ->
// 15.2 us in a trace): they start unstaggered.  Results do not depend on it.
// A per-shape sweep of the delay (0, 1, 2, 4, 6, 8) over back-to-back GEMMs
// kept 4 for every shape.  Inside the bench step, where each GEMM follows its
// activation kernels, the launches with one tile per workgroup (attn_out and
// mlp_down, N = 768) only pay the delay: the step took 1.8672 ms with 4 on
// every shape, 1.8662 / 1.8575 ms with 4 on mlp_down / attn_out alone and
// 1.8523 / 1.8530 ms with 4 on qkv / mlp_up alone (5 interleaved rounds,
// one box), so the delay applies only when workgroups run several tiles.
constexpr int kStartStagger = 4;

template <class C, class P, class E>
static int launch_ws(Ctx* c, const uint8_t* a, const uint8_t* w, int64_t m, int64_t n,
                     int64_t ldk, const E& ep, void* y) {
    const int64_t per_cu = 163840 / C::LDS_BYTES > 0 ? 163840 / C::LDS_BYTES : 1;
    const int64_t resident = (int64_t)c->num_cus * per_cu;
    const int64_t tiles = tiles_of<C>(m, n);
    const int64_t grid = tiles < resident ? tiles : resident;
    int stagger = E::kOut32 && tiles > grid ? kStartStagger : 0;
    if (tuned(c, TKV_HIP_TUNE_GEMM_STAGGER) >= 0) stagger = (int)tuned(c, TKV_HIP_TUNE_GEMM_STAGGER);
    hipLaunchKernelGGL((k_gemm_ws<C, P, E>), dim3((unsigned)grid), dim3(C::THREADS), 0,
                       c->stream, a, w, (int)m, (int)n, (int)ldk, ep, y, stagger);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

// Waves per workgroup of the skinny kernel: enough workgroups x waves for
// the weight stream to fill the machine, but never more waves than K steps.
// When the column blocks cover at most a quarter of the CUs, K is split
// over workgroups too (SPLIT kernel): up to one workgroup per CU, at least 8
// K steps (two per wave) per split.  Per-token decode calls (quantize + GEMM,
// interleaved medians): mlp_down (N = 768, 24 blocks) 12.3 -> 9.1 us at M = 1
// and 17.2 -> 10.8 us at M = 32; splitting at half the CUs also took qkv and
// mlp_up (72 and 96 blocks), which lost 0.4-0.7 us.
template <class E>
static int launch_gemv(Ctx* c, const uint8_t* a, const uint8_t* w, int64_t m, int64_t n,
                       int64_t ldk, const E& ep, void* y) {
    const int64_t wgs = ceil_div(n, (int64_t)32);
    const int64_t nks = ldk / 32;
    // Weight path: whole lines through LDS wherever they fit (ldk % 128 == 0,
    // the K range's lines at 4 KB each within 128 KB), unless the context's
    // decode weight-path knob forces registers.  Cold weights, one box, two
    // rounds: unsplit launches (qkv / mlp_up shapes, 16 waves) 4.94 / 5.03 ->
    // 4.19 / 4.25 us at M = 1 and 5.48 / 5.72 -> 4.76 / 4.81 at M = 32; split
    // launches (mlp_down, 264 workgroups of 12 KB) within +-0.1 us.
    const bool want_lines = tuned(c, TKV_HIP_TUNE_DECODE_DMA) != 0 && ldk % 128 == 0;
    auto lines_lds = [&](int64_t span) { return 4096 * ((span + 3) / 4 + 1); };
    if (wgs * 4 <= c->num_cus && wgs <= kGemvSplitBlocks) {
        int64_t splits = ceil_div((int64_t)c->num_cus, wgs);
        if (splits > nks / 8) splits = nks / 8;
        if (splits >= 2) {
            const int64_t lds = lines_lds(ceil_div(nks, splits));
            if (want_lines && lds <= (128 << 10))
                hipLaunchKernelGGL((k_gemv_i8<4, true, E, true>), dim3((unsigned)(wgs * splits)),
                                   dim3(4 * 64), (unsigned)lds, c->stream, a, w, (int)m, (int)n,
                                   (int)ldk, ep, y, (int)splits, c->gemv_part, c->gemv_arrivals);
            else
                hipLaunchKernelGGL((k_gemv_i8<4, true, E>), dim3((unsigned)(wgs * splits)),
                                   dim3(4 * 64), 0, c->stream, a, w, (int)m, (int)n, (int)ldk, ep,
                                   y, (int)splits, c->gemv_part, c->gemv_arrivals);
            TKV_LAUNCH_CHECK();
            return TKV_HIP_OK;
        }
    }
    int64_t kw = ceil_div((int64_t)c->num_cus * 8, wgs);
    if (kw > nks) kw = nks;
    const int64_t lds = lines_lds(nks);
    const bool lines = want_lines && lds <= (128 << 10);
#define TKV_GEMV(KW)                                                                           \
    do {                                                                                       \
        if (lines)                                                                             \
            hipLaunchKernelGGL((k_gemv_i8<KW, false, E, true>), dim3((unsigned)wgs),          \
                               dim3(KW * 64), (unsigned)lds, c->stream, a, w, (int)m, (int)n, \
                               (int)ldk, ep, y, 1, nullptr, nullptr);                          \
        else                                                                                   \
            hipLaunchKernelGGL((k_gemv_i8<KW, false, E>), dim3((unsigned)wgs), dim3(KW * 64), \
                               0, c->stream, a, w, (int)m, (int)n, (int)ldk, ep, y, 1, nullptr, \
                               nullptr);                                                       \
    } while (0)
    if (kw >= 16)
        TKV_GEMV(16);
    else if (kw >= 8)
        TKV_GEMV(8);
    else if (kw >= 4)
        TKV_GEMV(4);
    else
        TKV_GEMV(1);
#undef TKV_GEMV
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

template <class P, class E>
static int launch_any(Ctx* c, const uint8_t* a, const uint8_t* w, int64_t m, int64_t n,
                      int64_t ldk, const E& ep, void* y) {
    const int cfg = pick_cfg(c, m, n);
    const bool forced = tuned(c, TKV_HIP_TUNE_GEMM_CFG) >= 0;
    // The split sums need the warp-specialised kernel and 2 (BM WN + BN WM)
    // ints of LDS beside its ring (all of cfg 6's LDS is ring); other
    // configurations sum in every wave (PolicyI8Q).
    if constexpr (std::is_same_v<P, PolicyI8QS>) {
        switch (cfg) {
            case 2: return launch_ws<Cfg2, P>(c, a, w, m, n, ldk, ep, y);
            case 3: return launch_ws<Cfg3, P>(c, a, w, m, n, ldk, ep, y);
            case 4: return launch_ws<Cfg4, P>(c, a, w, m, n, ldk, ep, y);
            case 5: return launch_ws<Cfg5, P>(c, a, w, m, n, ldk, ep, y);
            case 7: return launch_ws<Cfg7, P>(c, a, w, m, n, ldk, ep, y);
            case 8: return launch_ws<Cfg8, P>(c, a, w, m, n, ldk, ep, y);
            case 9: return launch_ws<Cfg9, P>(c, a, w, m, n, ldk, ep, y);
            default: return launch_any<PolicyI8Q>(c, a, w, m, n, ldk, ep, y);
        }
    }
    if constexpr (std::is_same_v<P, PolicyI8>) {
        if (m <= kGemvMaxM && (cfg == 10 || !forced))
            return launch_gemv(c, a, w, m, n, ldk, ep, y);
    }
    if constexpr (!std::is_same_v<P, PolicyI8QS>) switch (cfg) {
        case 0: return launch_cfg<Cfg0, P>(c, a, w, m, n, ldk, ep, y);
        case 1: return launch_cfg<Cfg1, P>(c, a, w, m, n, ldk, ep, y);
        case 2: return launch_ws<Cfg2, P>(c, a, w, m, n, ldk, ep, y);
        case 3: return launch_ws<Cfg3, P>(c, a, w, m, n, ldk, ep, y);
        case 4: return launch_ws<Cfg4, P>(c, a, w, m, n, ldk, ep, y);
        case 5: return launch_ws<Cfg5, P>(c, a, w, m, n, ldk, ep, y);
        case 6: return launch_ws<Cfg6, P>(c, a, w, m, n, ldk, ep, y);
        case 7: return launch_ws<Cfg7, P>(c, a, w, m, n, ldk, ep, y);
        case 8: return launch_ws<Cfg8, P>(c, a, w, m, n, ldk, ep, y);
        case 9: return launch_ws<Cfg9, P>(c, a, w, m, n, ldk, ep, y);
        case 11: return launch_fused<Cfg11, P>(c, a, w, m, n, ldk, ep, y);
        default: return launch_cfg<Cfg0, P>(c, a, w, m, n, ldk, ep, y);
    }
}

// Host helpers shared by the GEMM entry points (gemm.hip).
// Rows must start on 16-byte boundaries and K must be a multiple of the
// slice depth: otherwise both operands are repacked into zero-padded
// workspace; *ldk_out is the row stride the kernels then see.
int prepare_operands(Ctx* c, const void** a, const void** w, int64_t m, int64_t n, int64_t k,
                     int64_t* ldk_out);
int check_sizes(int64_t m, int64_t n, int64_t k, const char* what);

}  // namespace gemm
}  // namespace tkv
