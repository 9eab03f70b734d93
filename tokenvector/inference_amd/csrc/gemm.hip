// gemm.hip -- host side shared by the GEMM entry points (operand padding,
// size checks) and QLinearMatMul's requantizing GEMM (session.tkv:1992-2071).
// The kernels and launchers are in gemm_kernels.h; the INT8 dequant GEMM is in
// gemm_i8.hip and the FP8 GEMM in gemm_f8.hip, so the three instantiation sets
// compile in parallel.
#include "gemm_kernels.h"

namespace tkv {
namespace gemm {

// dst[r * ldk + j] = j < k ? src[r * k + j] : 0 for r < rows, j < ldk
// (ldk a multiple of 16, dst 16-byte aligned): 16 output bytes per lane.
__global__ void __launch_bounds__(256) k_pad_rows(const uint8_t* __restrict__ src, int64_t k,
                                                  int64_t rows, int64_t ldk,
                                                  uint8_t* __restrict__ dst) {
    typedef unsigned char u8x16 __attribute__((ext_vector_type(16)));
    const int64_t n16 = rows * (ldk / 16);
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
        const int64_t r = i / (ldk / 16), j0 = (i % (ldk / 16)) * 16;
        const uint8_t* __restrict__ s = src + r * k;
        u8x16 v;
#pragma unroll
        for (int b = 0; b < 16; b++) v[b] = j0 + b < k ? s[j0 + b] : (uint8_t)0;
        *reinterpret_cast<u8x16*>(dst + 16 * i) = v;
    }
}

static int pad_rows(Ctx* c, const void* src, int64_t k, int64_t rows, int64_t ldk, void* dst) {
    const int64_t n16 = rows * (ldk / 16);
    const unsigned grid = (unsigned)std::min<int64_t>(ceil_div(n16 > 0 ? n16 : 1, 256),
                                                      (int64_t)c->num_cus * 8);
    hipLaunchKernelGGL(k_pad_rows, dim3(grid), dim3(256), 0, c->stream,
                       static_cast<const uint8_t*>(src), k, rows, ldk, static_cast<uint8_t*>(dst));
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

int prepare_operands(Ctx* c, const void** a, const void** w, int64_t m, int64_t n,
                            int64_t k, int64_t* ldk_out) {
    int64_t ldk = (k + kBK - 1) / kBK * kBK;
    if (ldk != k || !aligned(*a, 16) || !aligned(*w, 16)) {
        void *pa, *pw;
        TKV_RC_TRY(ctx_workspace(c, 2, (size_t)(m * ldk), &pa));
        TKV_RC_TRY(ctx_workspace(c, 3, (size_t)(n * ldk), &pw));
        TKV_RC_TRY(pad_rows(c, *a, k, m, ldk, pa));
        TKV_RC_TRY(pad_rows(c, *w, k, n, ldk, pw));
        *a = pa;
        *w = pw;
    }
    *ldk_out = ldk;
    return TKV_HIP_OK;
}

int check_sizes(int64_t m, int64_t n, int64_t k, const char* what) {
    if (k <= 0 || m >= (1ll << 31) || n >= (1ll << 28) || k >= (1ll << 17))
        return set_error(TKV_HIP_UNSUPPORTED,
                         std::string(what) + ": K must be in [1, 2^17), M < 2^31 and N < 2^28");
    return TKV_HIP_OK;
}

}  // namespace gemm

int64_t gemm_k_align() { return gemm::kBK; }

// QLinearMatMul: row sums of A and W first (zero padding past k adds
// nothing), then the GEMM with the requantizing epilogue.  The sums enter the
// corrections only through zpw * sum(a) and zpa * sum(w), so the rows of A are
// summed only for zpw != 0 and those of W only for zpa != 0; the epilogue
// reads the others (any int32 value) and multiplies them by zero.
int launch_gemm_qlinear(Ctx* c, const int8_t* a, const int8_t* w, int64_t m, int64_t n,
                        int64_t k, const QLinearParams& q, int8_t* y) {
    if (m <= 0 || n <= 0) return TKV_HIP_OK;
    TKV_RC_TRY(gemm::check_sizes(m, n, k, "QLinearMatMul"));
    auto small = [](int32_t v) { return v >= -32768 && v <= 32767; };
    if (!small(q.zpa) || !small(q.zpw))
        return set_error(TKV_HIP_UNSUPPORTED, "QLinearMatMul: input zero points beyond +-2^15");
    const void *pa = a, *pw = w;
    int64_t ldk;
    TKV_RC_TRY(gemm::prepare_operands(c, &pa, &pw, m, n, k, &ldk));
    const int64_t kzz = k * (int64_t)q.zpa * (int64_t)q.zpw;
    const int64_t bound = k * (128 + (int64_t)std::abs(q.zpa)) * (128 + (int64_t)std::abs(q.zpw));
    const auto* ua = static_cast<const uint8_t*>(pa);
    const auto* uw = static_cast<const uint8_t*>(pw);
    const bool i32 = bound < (1ll << 31) && std::isfinite(q.mult);
    // Tiled kernels can form the sums themselves.  Summed in every wave
    // (PolicyI8Q) that cost ~0.3 us per 128-deep K slice a workgroup runs;
    // split over the waves of the warp-specialised kernel (PolicyI8QS, each
    // byte summed once, partials exchanged through LDS at each tile's end)
    // it costs less per slice but adds an exchange per tile.  The pre-pass
    // costs ~4.5-7 us at M = 8192, growing with M K.  bench.py's qlinear
    // section, interleaved rounds on one box, split sums against the earlier
    // choice (pre-pass beyond 12 slices per workgroup, per-wave sums below):
    // attn_out 14.1 / 15.0 us, mlp_down (one tile of 24 slices per
    // workgroup) 29.8 / 32.4, qkv (three tiles of 6) 34.1 / 33.9, mlp_up
    // (four tiles of 6) 43.3 / 41.9.  So the GEMM sums whenever a workgroup
    // runs one tile, or few slices in all.
    const int64_t tiles = gemm::tiles_of<gemm::Cfg2>(m, n);
    const int64_t slices = ceil_div(tiles, (int64_t)c->num_cus) * (ldk / gemm::kBK);
    if (m > gemm::kGemvMaxM && (tiles <= c->num_cus || slices <= 12)) {
        if (i32)
            return gemm::launch_any<gemm::PolicyI8QS>(
                c, ua, uw, m, n, ldk,
                gemm::EpiQL<true, true>{nullptr, nullptr, q.zpa, q.zpw, q.zpy, kzz, q.mult}, y);
        return gemm::launch_any<gemm::PolicyI8QS>(
            c, ua, uw, m, n, ldk,
            gemm::EpiQL<false, true>{nullptr, nullptr, q.zpa, q.zpw, q.zpy, kzz, q.mult}, y);
    }
    void* sums;
    TKV_RC_TRY(ctx_workspace(c, 8, (size_t)(m + n) * 4, &sums));
    int32_t* ra = static_cast<int32_t*>(sums);
    TKV_RC_TRY(launch_row_sums_i8(c, a, q.zpw != 0 ? m : 0, w, q.zpa != 0 ? n : 0, k, ra,
                                  ra + m));
    if (i32)
        return gemm::launch_any<gemm::PolicyI8>(
            c, ua, uw, m, n, ldk, gemm::EpiQL<true>{ra, ra + m, q.zpa, q.zpw, q.zpy, kzz, q.mult},
            y);
    return gemm::launch_any<gemm::PolicyI8>(
        c, ua, uw, m, n, ldk, gemm::EpiQL<false>{ra, ra + m, q.zpa, q.zpw, q.zpy, kzz, q.mult}, y);
}

}  // namespace tkv
