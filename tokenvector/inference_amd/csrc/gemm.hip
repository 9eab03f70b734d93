// gemm.hip -- INT8 and FP8 GEMMs of the PTQ path on gfx950, with the fused
// dequant epilogues of the reference's quantized linear.
//
//   INT8  (matmul_int8_per_channel / _symmetric, tv/quantization/matmul.tkv:4-29,
//          _dot_int8 :116-127): v_mfma_i32_32x32x32_i8, INT32 accumulators
//          exact, epilogue restating the reference's float typing:
//            per-channel: y = fl32(fl64(fl64(acc * sa) * sw[n]) + b[n])
//            symmetric:   y = fl32(fl64(acc * fl32(sa * sw)) + b[n])
//   FP8   (matmul_fp8_e4m3, matmul.tkv:46-58): y = fl32(fl64(acc) + b[n]),
//          optional per-token / per-channel scales (extension).
//          PolicyF8Ref: reference decoder + f16 MFMA (drop-in precision);
//          PolicyF8:    full-rate f8f6f4 MFMA (OCP decode, hardware rounding).
//
// Data movement and tiling live in gemm_tile.h.  All arithmetic here is
// compiled with -ffp-contract=off.
#include <cstdlib>

#include "gemm_tile.h"
#include "tkv_internal.h"

namespace tkv {
namespace gemm {

// 32x32 MFMA result layout: lane holds column (lane & 31); register r holds
// row (r / 4) * 8 + (lane / 32) * 4 + (r % 4).
__device__ __forceinline__ int acc_row(int r, int khalf) { return (r >> 2) * 8 + khalf * 4 + (r & 3); }

// Activation scales of this lane's output rows, all loaded before any
// epilogue arithmetic so their latencies overlap (a single load when the
// scale is per tensor).
template <class C>
__device__ __forceinline__ void row_scales(const float* __restrict__ sa_ptr, int64_t stride, int m0,
                                           int M, int wm, int khalf, float (&sa)[C::TM][16]) {
    if (stride == 0) {
        const float s = sa_ptr[0];
#pragma unroll
        for (int i = 0; i < C::TM; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) sa[i][r] = s;
        return;
    }
#pragma unroll
    for (int i = 0; i < C::TM; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int row = m0 + wm * C::WTM + i * 32 + acc_row(r, khalf);
            sa[i][r] = row < M ? sa_ptr[(int64_t)row * stride] : 0.0f;
        }
}

// Output stores bypass cache allocation: Y is written once and not re-read
// by this kernel, so it should not evict the A / W slices other tiles reuse.
template <class T>
__device__ __forceinline__ void put(T* p, T v) { __builtin_nontemporal_store(v, p); }

template <int MODE, int RECIPE>
struct EpiI8 {
    const float* scale_a;
    int64_t scale_a_stride;
    float scale_w;
    const float* scales_w;
    const float* bias;

    template <class C, class P>
    __device__ __forceinline__ void store(const typename P::Acc (&acc)[C::TM][C::TN], int m0,
                                          int n0, int M, int N, void* __restrict__ Y) const {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        const int wm = wave / C::WN, wn = wave % C::WN, khalf = lane >> 5;
        float sa[C::TM][16];
        if (MODE != EPI_ACCUM_I32) row_scales<C>(scale_a, scale_a_stride, m0, M, wm, khalf, sa);
#pragma unroll
        for (int j = 0; j < C::TN; j++) {
            const int col = n0 + wn * C::WTN + j * 32 + (lane & 31);
            if (col >= N) continue;
            float sw = 0.0f, b = 0.0f;
            if (MODE == EPI_PER_CHANNEL) sw = scales_w[col];
            if (MODE != EPI_ACCUM_I32 && bias) b = bias[col];
#pragma unroll
            for (int i = 0; i < C::TM; i++) {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = m0 + wm * C::WTM + i * 32 + acc_row(r, khalf);
                    if (row >= M) continue;
                    const int64_t o = (int64_t)row * N + col;
                    const int32_t a = acc[i][j][r];
                    if (MODE == EPI_ACCUM_I32) {
                        put(reinterpret_cast<int32_t*>(Y) + o, a);
                        continue;
                    }
                    float y;
                    if (MODE == EPI_PER_CHANNEL) {
                        if (RECIPE == TKV_HIP_RECIPE_PRIMARY) {
                            double v = (double)a * (double)sa[i][r];
                            v = v * (double)sw;
                            v = v + (double)b;
                            y = (float)v;
                        } else {
                            float t = (float)a * sa[i][r];
                            t = t * sw;
                            y = t + b;
                        }
                    } else {
                        const double s = RECIPE == TKV_HIP_RECIPE_PRIMARY
                                             ? (double)(sa[i][r] * scale_w)
                                             : (double)sa[i][r] * (double)scale_w;
                        double v = (double)a * s;
                        v = v + (double)b;
                        y = (float)v;
                    }
                    put(reinterpret_cast<float*>(Y) + o, y);
                }
            }
        }
    }
};

template <bool SCALED>
struct EpiF8 {
    const float* scale_a;  // used when SCALED (extension epilogue)
    int64_t scale_a_stride;
    const float* scales_w;
    const float* bias;

    template <class C, class P>
    __device__ __forceinline__ void store(const typename P::Acc (&acc)[C::TM][C::TN], int m0,
                                          int n0, int M, int N, void* __restrict__ Y) const {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        const int wm = wave / C::WN, wn = wave % C::WN, khalf = lane >> 5;
        float sa[C::TM][16];
        if (SCALED) row_scales<C>(scale_a, scale_a_stride, m0, M, wm, khalf, sa);
#pragma unroll
        for (int j = 0; j < C::TN; j++) {
            const int col = n0 + wn * C::WTN + j * 32 + (lane & 31);
            if (col >= N) continue;
            const double b = bias ? (double)bias[col] : 0.0;
            const double sw = SCALED ? (double)scales_w[col] : 1.0;
#pragma unroll
            for (int i = 0; i < C::TM; i++) {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = m0 + wm * C::WTM + i * 32 + acc_row(r, khalf);
                    if (row >= M) continue;
                    double v = (double)(acc[i][j][r] * P::kAccScale);  // exact power of 2
                    if (SCALED) {
                        v = v * (double)sa[i][r];
                        v = v * sw;
                    }
                    v = v + b;
                    put(reinterpret_cast<float*>(Y) + (int64_t)row * N + col, (float)v);
                }
            }
        }
    }
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
            for (int j = 0; j < C::TN; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[i][j][r] = 0;
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
        ep.template store<C, P>(acc, m0, n0, M, N, Y);
        if (!more) break;
        v = vn;
        m0 = m0n;
        n0 = n0n;
    }
}

// ---- tile configurations ---------------------------------------------------
// K slices are 128 bytes: one full L2 line per row per DMA (64-byte slices
// fetch every line twice and halve the DMA throughput).
//            BM   BN  WM WN   BK  STAGES
typedef Cfg<128, 192, 2, 2, 128, 3> Cfg0;  // 120 KB
typedef Cfg<64, 192, 2, 2, 128, 3> Cfg1;   //  96 KB, fewer rows when tiles < CUs
typedef Cfg<128, 128, 2, 2, 128, 3> Cfg2;  //  96 KB, N not a multiple of 192
typedef Cfg<64, 128, 2, 2, 128, 3> Cfg3;   //  72 KB
typedef Cfg<128, 192, 2, 2, 128, 2> Cfg4;  //  80 KB, two workgroups per CU
typedef Cfg<128, 256, 4, 2, 128, 2> Cfg5;  //  96 KB, 8 waves, 32x128 wave tiles
typedef Cfg<256, 256, 4, 2, 128, 2> Cfg6;  // 128 KB, 8 waves, 64x128 wave tiles
typedef Cfg<256, 192, 4, 2, 128, 2> Cfg7;  // 112 KB, 8 waves, 64x96 wave tiles
typedef Cfg<128, 192, 4, 2, 128, 3> Cfg8;  // 120 KB, 8 waves, 32x96 wave tiles
typedef Cfg<128, 192, 2, 2, 64, 4> Cfg9;   //  80 KB, 64-byte slices

constexpr int kBK = 128;

template <class C>
static int64_t tiles_of(int64_t m, int64_t n) {
    return ceil_div(m, C::BM) * ceil_div(n, C::BN);
}

// Tile choice: the largest tile that still gives every CU work.  The
// environment variable TKV_GEMM_CFG (0..9) forces one (tuning sweeps).
static int pick_cfg(Ctx* c, int64_t m, int64_t n) {
    if (const char* v = getenv("TKV_GEMM_CFG")) {
        int f = atoi(v);
        if (f >= 0 && f <= 9) return f;
    }
    // 128x192 with 8 waves measured best on all four GPT-2 shapes at M=8192;
    // smaller 64x128 tiles keep every CU busy when M is small.
    return tiles_of<Cfg8>(m, n) >= c->num_cus ? 8 : 3;
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

template <class P, class E>
static int launch_any(Ctx* c, const uint8_t* a, const uint8_t* w, int64_t m, int64_t n,
                      int64_t ldk, const E& ep, void* y) {
    switch (pick_cfg(c, m, n)) {
        case 0: return launch_cfg<Cfg0, P>(c, a, w, m, n, ldk, ep, y);
        case 1: return launch_cfg<Cfg1, P>(c, a, w, m, n, ldk, ep, y);
        case 2: return launch_cfg<Cfg2, P>(c, a, w, m, n, ldk, ep, y);
        case 3: return launch_cfg<Cfg3, P>(c, a, w, m, n, ldk, ep, y);
        case 4: return launch_cfg<Cfg4, P>(c, a, w, m, n, ldk, ep, y);
        case 5: return launch_cfg<Cfg5, P>(c, a, w, m, n, ldk, ep, y);
        case 6: return launch_cfg<Cfg6, P>(c, a, w, m, n, ldk, ep, y);
        case 7: return launch_cfg<Cfg7, P>(c, a, w, m, n, ldk, ep, y);
        case 8: return launch_cfg<Cfg8, P>(c, a, w, m, n, ldk, ep, y);
        default: return launch_cfg<Cfg9, P>(c, a, w, m, n, ldk, ep, y);
    }
}

// Rows must start on 16-byte boundaries and K must be a multiple of the
// slice depth: otherwise repack both operands into zero-padded workspace.
static int prepare_operands(Ctx* c, const void** a, const void** w, int64_t m, int64_t n,
                            int64_t k, int64_t* ldk_out) {
    int64_t ldk = (k + kBK - 1) / kBK * kBK;
    if (ldk != k || !aligned(*a, 16) || !aligned(*w, 16)) {
        void *pa, *pw;
        TKV_RC_TRY(ctx_workspace(c, 2, (size_t)(m * ldk), &pa));
        TKV_RC_TRY(ctx_workspace(c, 3, (size_t)(n * ldk), &pw));
        TKV_HIP_TRY(hipMemsetAsync(pa, 0, (size_t)(m * ldk), c->stream));
        TKV_HIP_TRY(hipMemsetAsync(pw, 0, (size_t)(n * ldk), c->stream));
        TKV_HIP_TRY(hipMemcpy2DAsync(pa, (size_t)ldk, *a, (size_t)k, (size_t)k, (size_t)m,
                                     hipMemcpyDeviceToDevice, c->stream));
        TKV_HIP_TRY(hipMemcpy2DAsync(pw, (size_t)ldk, *w, (size_t)k, (size_t)k, (size_t)n,
                                     hipMemcpyDeviceToDevice, c->stream));
        *a = pa;
        *w = pw;
    }
    *ldk_out = ldk;
    return TKV_HIP_OK;
}

static int check_sizes(int64_t m, int64_t n, int64_t k, const char* what) {
    if (k <= 0 || m >= (1ll << 31) || n >= (1ll << 31) || k >= (1ll << 17))
        return set_error(TKV_HIP_UNSUPPORTED,
                         std::string(what) + ": K must be in [1, 2^17) and M, N < 2^31");
    return TKV_HIP_OK;
}

}  // namespace gemm

int64_t gemm_k_align() { return gemm::kBK; }

int launch_gemm_i8(Ctx* c, const int8_t* a, const int8_t* w, int64_t m, int64_t n, int64_t k,
                   const I8Epilogue& e, void* y) {
    if (m <= 0 || n <= 0) return TKV_HIP_OK;
    TKV_RC_TRY(gemm::check_sizes(m, n, k, "INT8 GEMM"));
    const void *pa = a, *pw = w;
    int64_t ldk;
    TKV_RC_TRY(gemm::prepare_operands(c, &pa, &pw, m, n, k, &ldk));
    const uint8_t* ua = static_cast<const uint8_t*>(pa);
    const uint8_t* uw = static_cast<const uint8_t*>(pw);
#define TKV_EPI(MODE, RECIPE)                                                                \
    gemm::launch_any<gemm::PolicyI8>(                                                        \
        c, ua, uw, m, n, ldk,                                                                \
        gemm::EpiI8<MODE, RECIPE>{e.scale_a, e.scale_a_stride, e.scale_w, e.scales_w, e.bias}, y)
    const bool primary = e.recipe == TKV_HIP_RECIPE_PRIMARY;
    switch (e.mode) {
        case EPI_PER_CHANNEL:
            return primary ? TKV_EPI(EPI_PER_CHANNEL, TKV_HIP_RECIPE_PRIMARY)
                           : TKV_EPI(EPI_PER_CHANNEL, TKV_HIP_RECIPE_ALTERNATE);
        case EPI_SYMMETRIC:
            return primary ? TKV_EPI(EPI_SYMMETRIC, TKV_HIP_RECIPE_PRIMARY)
                           : TKV_EPI(EPI_SYMMETRIC, TKV_HIP_RECIPE_ALTERNATE);
        default:
            return TKV_EPI(EPI_ACCUM_I32, TKV_HIP_RECIPE_PRIMARY);
    }
#undef TKV_EPI
}

int launch_gemm_f8(Ctx* c, const uint8_t* a, const uint8_t* w, int64_t m, int64_t n, int64_t k,
                   const float* scale_a, int64_t scale_a_stride, const float* scales_w,
                   const float* bias, float* y, bool fast) {
    if (m <= 0 || n <= 0) return TKV_HIP_OK;
    TKV_RC_TRY(gemm::check_sizes(m, n, k, "FP8 GEMM"));
    if ((scales_w == nullptr) != (scale_a == nullptr))
        return set_error(TKV_HIP_BAD_ARG, "FP8 GEMM: scale_a and scales_w go together");
    const void *pa = a, *pw = w;
    int64_t ldk;
    TKV_RC_TRY(gemm::prepare_operands(c, &pa, &pw, m, n, k, &ldk));
    const uint8_t* ua = static_cast<const uint8_t*>(pa);
    const uint8_t* uw = static_cast<const uint8_t*>(pw);
    if (scales_w) {
        gemm::EpiF8<true> ep{scale_a, scale_a_stride, scales_w, bias};
        return fast ? gemm::launch_any<gemm::PolicyF8>(c, ua, uw, m, n, ldk, ep, y)
                    : gemm::launch_any<gemm::PolicyF8Ref>(c, ua, uw, m, n, ldk, ep, y);
    }
    gemm::EpiF8<false> ep{nullptr, 0, nullptr, bias};
    return fast ? gemm::launch_any<gemm::PolicyF8>(c, ua, uw, m, n, ldk, ep, y)
                : gemm::launch_any<gemm::PolicyF8Ref>(c, ua, uw, m, n, ldk, ep, y);
}

}  // namespace tkv
