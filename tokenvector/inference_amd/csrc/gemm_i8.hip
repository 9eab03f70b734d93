// gemm_i8.hip -- the INT8 GEMM with the fused dequant epilogue of
// matmul_int8_per_channel / _symmetric (tv/quantization/matmul.tkv:4-29) and
// the plain INT32 accumulator output (kernels in gemm_kernels.h).
#include "gemm_kernels.h"

namespace tkv {

int launch_gemm_i8(Ctx* c, const int8_t* a, const int8_t* w, int64_t m, int64_t n, int64_t k,
                   const I8Epilogue& e, void* y) {
    if (m <= 0 || n <= 0) return TKV_HIP_OK;
    TKV_RC_TRY(gemm::check_sizes(m, n, e.k_logical > 0 ? e.k_logical : k, "INT8 GEMM"));
    const void *pa = a, *pw = w;
    int64_t ldk;
    TKV_RC_TRY(gemm::prepare_operands(c, &pa, &pw, m, n, k, &ldk));
    const uint8_t* ua = static_cast<const uint8_t*>(pa);
    const uint8_t* uw = static_cast<const uint8_t*>(pw);
#define TKV_EPI(MODE, RECIPE, ROWS)                                                          \
    gemm::launch_any<gemm::PolicyI8>(c, ua, uw, m, n, ldk,                                   \
                                     gemm::EpiI8<MODE, RECIPE, ROWS>{e.scale_a, e.scale_a_stride, \
                                                                     e.scale_w, e.scales_w,   \
                                                                     e.bias, fold},           \
                                     y)
    const bool primary = e.recipe == TKV_HIP_RECIPE_PRIMARY;
    const bool rows = e.scale_a_stride != 0;
    // |acc| <= 128^2 * K < 2^29 makes acc * scale_a exact in f64
    const int fold = (!rows && k < (1 << 15)) ? 1 : 0;
    switch (e.mode) {
        case EPI_PER_CHANNEL:
            if (rows)
                return primary ? TKV_EPI(EPI_PER_CHANNEL, TKV_HIP_RECIPE_PRIMARY, true)
                               : TKV_EPI(EPI_PER_CHANNEL, TKV_HIP_RECIPE_ALTERNATE, true);
            return primary ? TKV_EPI(EPI_PER_CHANNEL, TKV_HIP_RECIPE_PRIMARY, false)
                           : TKV_EPI(EPI_PER_CHANNEL, TKV_HIP_RECIPE_ALTERNATE, false);
        case EPI_SYMMETRIC:
            if (rows)
                return primary ? TKV_EPI(EPI_SYMMETRIC, TKV_HIP_RECIPE_PRIMARY, true)
                               : TKV_EPI(EPI_SYMMETRIC, TKV_HIP_RECIPE_ALTERNATE, true);
            return primary ? TKV_EPI(EPI_SYMMETRIC, TKV_HIP_RECIPE_PRIMARY, false)
                           : TKV_EPI(EPI_SYMMETRIC, TKV_HIP_RECIPE_ALTERNATE, false);
        default:
            return TKV_EPI(EPI_ACCUM_I32, TKV_HIP_RECIPE_PRIMARY, false);
    }
#undef TKV_EPI
}

}  // namespace tkv
