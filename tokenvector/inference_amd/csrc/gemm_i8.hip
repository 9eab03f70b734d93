// gemm_i8.hip -- INT8 x INT8 -> INT32 GEMM with the fused dequant epilogue,
// on CDNA4 MFMA (v_mfma_i32_32x32x32_i8), for gfx950.
//
// Reference: matmul_int8_per_channel / matmul_int8_symmetric
// (tv/quantization/matmul.tkv:4-29) with _dot_int8 (:116-127) as the inner
// product.  Both operands are K-major (A[M,K], W[N,K], matmul.tkv:22), which
// is the layout MFMA consumes directly: no transposes.
//
// Tiling: a 256-thread workgroup (4 wave64, 2 x 2) owns a BM x BN output tile
// and walks K in BK = 128-byte stages.  Each stage is loaded from HBM/L2 with
// 16-byte loads into registers, then written to one of two LDS buffers
// (double buffering: the next stage's global loads are in flight while MFMA
// consumes the current LDS buffer).  LDS rows are 128 bytes; 16-byte chunks
// are XOR-swizzled by row so the ds_read_b128 fragment reads of 32 rows and
// the ds_write_b128 stores are bank-conflict free.
//
// INT32 accumulation is exact (|acc| <= 128^2 K < 2^31 for K < 2^17), so the
// result equals the reference's unbounded-integer sums bit for bit in any
// summation order.  The epilogue restates the reference's float typing in
// f64 with no contraction (compiled -ffp-contract=off):
//   per-channel: y = fl32(fl64(fl64(acc * sa) * sw[n]) + b[n])
//   symmetric:   y = fl32(fl64(acc * fl32(sa * sw)) + b[n])
#include "tkv_device.h"
#include "tkv_internal.h"

namespace tkv {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

namespace gi8 {

constexpr int kThreads = 256;
constexpr int kBK = 128;  // bytes of K per stage

// XOR swizzle of the 16-byte chunk index within a 128-byte LDS row.  For 8
// consecutive rows (32 banks) and for 16 consecutive rows (64 banks) the
// swizzled chunks land in distinct bank groups.
__device__ __forceinline__ int swz(int row) { return (row ^ (row >> 3)) & 7; }

struct Epi {
    int mode;
    int recipe;
    const float* scale_a;
    int64_t scale_a_stride;
    float scale_w;
    const float* scales_w;
    const float* bias;
};

template <int BM, int BN>
__global__ __launch_bounds__(kThreads) void k_gemm_i8(const int8_t* __restrict__ A,
                                                      const int8_t* __restrict__ W, int M, int N,
                                                      int ldk, Epi ep, void* __restrict__ Y) {
    constexpr int WTM = BM / 2;       // wave tile rows
    constexpr int WTN = BN / 2;       // wave tile cols
    constexpr int TM = WTM / 32;      // 32x32 MFMA tiles per wave (rows)
    constexpr int TN = WTN / 32;
    constexpr int A_LOADS = BM * kBK / 16 / kThreads;  // 16-byte chunks per thread
    constexpr int W_LOADS = BN * kBK / 16 / kThreads;
    static_assert(A_LOADS >= 1 && W_LOADS >= 1, "tile too small");

    __shared__ __attribute__((aligned(16))) int8_t sA[2][BM * kBK];
    __shared__ __attribute__((aligned(16))) int8_t sW[2][BN * kBK];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    const int tiles_n = (N + BN - 1) / BN;
    const int bm = blockIdx.x / tiles_n;
    const int bn = blockIdx.x - bm * tiles_n;
    const int m0 = bm * BM, n0 = bn * BN;

    // Global -> LDS mapping: chunk id = i * 256 + tid, row = id / 8, ch = id % 8.
    const int8_t* a_src[A_LOADS];
    const int8_t* w_src[W_LOADS];
    int a_dst[A_LOADS], w_dst[W_LOADS], a_ch[A_LOADS], w_ch[W_LOADS];
#pragma unroll
    for (int i = 0; i < A_LOADS; i++) {
        int id = i * kThreads + tid, row = id >> 3, ch = id & 7;
        int gr = m0 + row < M ? m0 + row : M - 1;  // clamp: rows >= M are never stored
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

    v16i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = v16i{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

    // Fragment rows of this lane (fixed across K).
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
        for (int ks = 0; ks < kBK / 32; ks++) {
            const int ch = ks * 2 + khalf;
            v4i af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; i++)
                af[i] = *reinterpret_cast<const v4i*>(
                    &sA[buf][a_row[i] * kBK + ((ch ^ swz(a_row[i])) << 4)]);
#pragma unroll
            for (int j = 0; j < TN; j++)
                bf[j] = *reinterpret_cast<const v4i*>(
                    &sW[buf][w_row[j] * kBK + ((ch ^ swz(w_row[j])) << 4)]);
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) sstore(buf ^ 1);
        __syncthreads();
    }

    // Epilogue.  32x32 MFMA result layout: lane holds column (lane & 31);
    // register r holds row (r / 4) * 8 + (lane / 32) * 4 + (r % 4).
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int col = n0 + wn * WTN + j * 32 + (lane & 31);
        if (col >= N) continue;
        float sw = 0.0f, b = 0.0f;
        if (ep.mode != EPI_ACCUM_I32) {
            if (ep.mode == EPI_PER_CHANNEL) sw = ep.scales_w[col];
            if (ep.bias) b = ep.bias[col];
        }
#pragma unroll
        for (int i = 0; i < TM; i++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + wm * WTM + i * 32 + (r >> 2) * 8 + khalf * 4 + (r & 3);
                if (row >= M) continue;
                const int64_t o = (int64_t)row * N + col;
                const int32_t a = acc[i][j][r];
                if (ep.mode == EPI_ACCUM_I32) {
                    reinterpret_cast<int32_t*>(Y)[o] = a;
                    continue;
                }
                const float sa = ep.scale_a[(int64_t)row * ep.scale_a_stride];
                float y;
                if (ep.mode == EPI_PER_CHANNEL) {
                    if (ep.recipe == TKV_HIP_RECIPE_PRIMARY) {
                        double v = (double)a * (double)sa;
                        v = v * (double)sw;
                        v = v + (double)b;
                        y = (float)v;
                    } else {
                        float t = (float)a * sa;
                        t = t * sw;
                        y = t + b;
                    }
                } else {
                    double s = ep.recipe == TKV_HIP_RECIPE_PRIMARY ? (double)(sa * ep.scale_w)
                                                                   : (double)sa * (double)ep.scale_w;
                    double v = (double)a * s;
                    v = v + (double)b;
                    y = (float)v;
                }
                reinterpret_cast<float*>(Y)[o] = y;
            }
        }
    }
}

}  // namespace gi8

int launch_gemm_i8(Ctx* c, const int8_t* a, const int8_t* w, int64_t m, int64_t n, int64_t k,
                   const I8Epilogue& e, void* y) {
    if (m <= 0 || n <= 0) return TKV_HIP_OK;
    if (k <= 0 || m >= (1ll << 31) || n >= (1ll << 31) || k >= (1ll << 17))
        return set_error(TKV_HIP_UNSUPPORTED, "INT8 GEMM: K must be in [1, 2^17) and M, N < 2^31");
    // Rows must start 16-byte aligned: repack with a zero-padded leading
    // dimension when K is not a multiple of 16 or a pointer is unaligned.
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
        a = static_cast<const int8_t*>(pa);
        w = static_cast<const int8_t*>(pw);
    }
    gi8::Epi ep{e.mode, e.recipe, e.scale_a, e.scale_a_stride, e.scale_w, e.scales_w, e.bias};
    constexpr int BM = 128, BN = 128;
    int64_t tiles = ceil_div(m, BM) * ceil_div(n, BN);
    hipLaunchKernelGGL((gi8::k_gemm_i8<BM, BN>), dim3((unsigned)tiles), dim3(gi8::kThreads), 0,
                       c->stream, a, w, (int)m, (int)n, (int)ldk, ep, y);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

}  // namespace tkv
