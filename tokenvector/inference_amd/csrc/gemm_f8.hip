// gemm_f8.hip -- FP8 (e4m3) x FP8 -> FP32 GEMM on CDNA4 MFMA
// (v_mfma_scale_f32_32x32x64_f8f6f4 with neutral E8M0 scales 2^0), gfx950.
//
// Reference: matmul_fp8_e4m3 (tv/quantization/matmul.tkv:46-58): every
// product of two decoded e4m3 values is exact in f32, the reference sums them
// in f64 (exactly, for K <= 2^17) and rounds acc + bias once to f32.  Here the
// MFMA accumulates in f32, so outputs agree within the summation bound
//   |y - y_ref| <= K * 2^-24 * sum_k |a_k w_k| + ulp(y_ref)
// that the parity tests state.  The epilogue adds the bias in f64 and rounds
// once, as the reference does.  Operands are raw e4m3 bytes (the reference's
// code + 128), K-major on both sides.
//
// Tiling mirrors gemm_i8.hip: 256 threads, 2 x 2 wave64, BK = 128-byte LDS
// stages double-buffered, XOR-swizzled 16-byte chunks; each MFMA fragment is
// two 16-byte LDS reads (32 consecutive K bytes per lane).
#include "tkv_device.h"
#include "tkv_internal.h"

namespace tkv {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

namespace gf8 {

constexpr int kThreads = 256;
constexpr int kBK = 128;
constexpr int kScaleOne = 127;  // E8M0 encoding of 2^0

__device__ __forceinline__ int swz(int row) { return (row ^ (row >> 3)) & 7; }

template <int BM, int BN>
__global__ __launch_bounds__(kThreads) void k_gemm_f8(const uint8_t* __restrict__ A,
                                                      const uint8_t* __restrict__ W, int M, int N,
                                                      int ldk, const float* __restrict__ scale_a,
                                                      int64_t scale_a_stride,
                                                      const float* __restrict__ scales_w,
                                                      const float* __restrict__ bias,
                                                      float* __restrict__ Y) {
    constexpr int WTM = BM / 2, WTN = BN / 2;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    constexpr int A_LOADS = BM * kBK / 16 / kThreads;
    constexpr int W_LOADS = BN * kBK / 16 / kThreads;

    __shared__ __attribute__((aligned(16))) uint8_t sA[2][BM * kBK];
    __shared__ __attribute__((aligned(16))) uint8_t sW[2][BN * kBK];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int tiles_n = (N + BN - 1) / BN;
    const int bm = blockIdx.x / tiles_n, bn = blockIdx.x - bm * tiles_n;
    const int m0 = bm * BM, n0 = bn * BN;

    const uint8_t* a_src[A_LOADS];
    const uint8_t* w_src[W_LOADS];
    int a_dst[A_LOADS], w_dst[W_LOADS], a_ch[A_LOADS], w_ch[W_LOADS];
#pragma unroll
    for (int i = 0; i < A_LOADS; i++) {
        int id = i * kThreads + tid, row = id >> 3, ch = id & 7;
        int gr = m0 + row < M ? m0 + row : M - 1;
        a_src[i] = A + (int64_t)gr * ldk + ch * 16;
        a_dst[i] = row * kBK + ((ch ^ swz(row)) << 4);
        a_ch[i] = ch * 16;
    }
#pragma unroll
    for (int i = 0; i < W_LOADS; i++) {
        int id = i * kThreads + tid, row = id >> 3, ch = id & 7;
        int gr = n0 + row < N ? n0 + row : N - 1;
        w_src[i] = W + (int64_t)gr * ldk + ch * 16;
        w_dst[i] = row * kBK + ((ch ^ swz(row)) << 4);
        w_ch[i] = ch * 16;
    }
    v4i ra[A_LOADS], rw[W_LOADS];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < A_LOADS; i++)
            ra[i] = (k0 + a_ch[i] < ldk) ? *reinterpret_cast<const v4i*>(a_src[i] + k0) : v4i{0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < W_LOADS; i++)
            rw[i] = (k0 + w_ch[i] < ldk) ? *reinterpret_cast<const v4i*>(w_src[i] + k0) : v4i{0, 0, 0, 0};
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_LOADS; i++) *reinterpret_cast<v4i*>(&sA[buf][a_dst[i]]) = ra[i];
#pragma unroll
        for (int i = 0; i < W_LOADS; i++) *reinterpret_cast<v4i*>(&sW[buf][w_dst[i]]) = rw[i];
    };

    v16f acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    int a_row[TM], w_row[TN];
#pragma unroll
    for (int i = 0; i < TM; i++) a_row[i] = wm * WTM + i * 32 + (lane & 31);
#pragma unroll
    for (int j = 0; j < TN; j++) w_row[j] = wn * WTN + j * 32 + (lane & 31);
    const int khalf = lane >> 5;

    const int nk = (ldk + kBK - 1) / kBK;
    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int buf = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * kBK);
#pragma unroll
        for (int ks = 0; ks < kBK / 64; ks++) {
            const int ch0 = ks * 4 + khalf * 2;
            v8i af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const uint8_t* base = &sA[buf][a_row[i] * kBK];
                v4i lo = *reinterpret_cast<const v4i*>(base + (((ch0) ^ swz(a_row[i])) << 4));
                v4i hi = *reinterpret_cast<const v4i*>(base + (((ch0 + 1) ^ swz(a_row[i])) << 4));
                af[i] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const uint8_t* base = &sW[buf][w_row[j] * kBK];
                v4i lo = *reinterpret_cast<const v4i*>(base + (((ch0) ^ swz(w_row[j])) << 4));
                v4i hi = *reinterpret_cast<const v4i*>(base + (((ch0 + 1) ^ swz(w_row[j])) << 4));
                bf[j] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                        af[i], bf[j], acc[i][j], 0, 0, 0, kScaleOne, 0, kScaleOne);
        }
        if (kt + 1 < nk) sstore(buf ^ 1);
        __syncthreads();
    }

    // Epilogue (32x32 result layout as in gemm_i8.hip); -ffp-contract=off
    // keeps the f64 steps separately rounded.
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int col = n0 + wn * WTN + j * 32 + (lane & 31);
        if (col >= N) continue;
        const double b = bias ? (double)bias[col] : 0.0;
        const double sw = scales_w ? (double)scales_w[col] : 1.0;
#pragma unroll
        for (int i = 0; i < TM; i++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + wm * WTM + i * 32 + (r >> 2) * 8 + khalf * 4 + (r & 3);
                if (row >= M) continue;
                double v = (double)acc[i][j][r];
                if (scales_w) {
                    v = v * (double)scale_a[(int64_t)row * scale_a_stride];
                    v = v * sw;
                }
                v = v + b;
                Y[(int64_t)row * N + col] = (float)v;
            }
        }
    }
}

}  // namespace gf8

int launch_gemm_f8(Ctx* c, const uint8_t* a, const uint8_t* w, int64_t m, int64_t n,
                   int64_t k, const float* scale_a, int64_t scale_a_stride,
                   const float* scales_w, const float* bias, float* y) {
    if (m <= 0 || n <= 0) return TKV_HIP_OK;
    if (k <= 0 || m >= (1ll << 31) || n >= (1ll << 31) || k >= (1ll << 17))
        return set_error(TKV_HIP_UNSUPPORTED, "FP8 GEMM: K must be in [1, 2^17) and M, N < 2^31");
    if ((scales_w == nullptr) != (scale_a == nullptr))
        return set_error(TKV_HIP_BAD_ARG, "FP8 GEMM: scale_a and scales_w go together");
    int64_t ldk = (k + 15) & ~int64_t(15);
    if (ldk != k || !aligned(a, 16) || !aligned(w, 16)) {
        void *pa, *pw;
        TKV_RC_TRY(ctx_workspace(c, 2, (size_t)(m * ldk), &pa));
        TKV_RC_TRY(ctx_workspace(c, 3, (size_t)(n * ldk), &pw));
        TKV_HIP_TRY(hipMemsetAsync(pa, 0, (size_t)(m * ldk), c->stream));
        TKV_HIP_TRY(hipMemsetAsync(pw, 0, (size_t)(n * ldk), c->stream));
        TKV_HIP_TRY(hipMemcpy2DAsync(pa, (size_t)ldk, a, (size_t)k, (size_t)k, (size_t)m,
                                     hipMemcpyDeviceToDevice, c->stream));
        TKV_HIP_TRY(hipMemcpy2DAsync(pw, (size_t)ldk, w, (size_t)k, (size_t)k, (size_t)n,
                                     hipMemcpyDeviceToDevice, c->stream));
        a = static_cast<const uint8_t*>(pa);
        w = static_cast<const uint8_t*>(pw);
    }
    constexpr int BM = 128, BN = 128;
    int64_t tiles = ceil_div(m, BM) * ceil_div(n, BN);
    hipLaunchKernelGGL((gf8::k_gemm_f8<BM, BN>), dim3((unsigned)tiles), dim3(gf8::kThreads), 0,
                       c->stream, a, w, (int)m, (int)n, (int)ldk, scale_a, scale_a_stride,
                       scales_w, bias, y);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

}  // namespace tkv
