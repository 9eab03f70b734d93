// gemm_f8.hip -- the FP8 e4m3 GEMM (matmul_fp8_e4m3, tv/quantization/matmul.tkv:46-58):
// reference-decoded f16 operands or the full-rate FP8 MFMA (kernels in
// gemm_kernels.h).
#include "gemm_kernels.h"

namespace tkv {

namespace gemm {

// Reference e4m3 decode of n4 * 16 bytes into halves (dec2_f16: exact, 2^-8
// pre-scaled), 16 codes per lane: the reference-products FP8 GEMM decodes each
// operand once here instead of in every consumer wave's fragments.
__global__ void __launch_bounds__(256) k_fp8_ref_to_f16(const uint8_t* __restrict__ src,
                                                      int64_t n16, uint8_t* __restrict__ dst) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
        const u32x4 x = reinterpret_cast<const u32x4*>(src)[i];
        u32x4 lo, hi;
#pragma unroll
        for (int e = 0; e < 2; e++) {
            lo[2 * e] = dec2_f16(__builtin_amdgcn_perm(0u, x[e], 0x0c010c00u));
            lo[2 * e + 1] = dec2_f16(__builtin_amdgcn_perm(0u, x[e], 0x0c030c02u));
            hi[2 * e] = dec2_f16(__builtin_amdgcn_perm(0u, x[e + 2], 0x0c010c00u));
            hi[2 * e + 1] = dec2_f16(__builtin_amdgcn_perm(0u, x[e + 2], 0x0c030c02u));
        }
        reinterpret_cast<u32x4*>(dst)[2 * i] = lo;
        reinterpret_cast<u32x4*>(dst)[2 * i + 1] = hi;
    }
}

static int decode_into(Ctx* c, const uint8_t* src, int64_t bytes, void* d) {
    const int64_t n16 = bytes / 16;  // rows are ldk (a multiple of 128) bytes
    const unsigned grid = (unsigned)std::min<int64_t>(ceil_div(n16 > 0 ? n16 : 1, 256),
                                                      (int64_t)c->num_cus * 8);
    hipLaunchKernelGGL(k_fp8_ref_to_f16, dim3(grid), dim3(256), 0, c->stream, src, n16,
                       static_cast<uint8_t*>(d));
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

static int decode_f16(Ctx* c, const uint8_t* src, int64_t bytes, int slot, uint8_t** out) {
    void* d;
    TKV_RC_TRY(ctx_workspace(c, slot, (size_t)bytes * 2, &d));
    TKV_RC_TRY(decode_into(c, src, bytes, d));
    *out = static_cast<uint8_t*>(d);
    return TKV_HIP_OK;
}

}  // namespace gemm

int launch_gemm_f8_decoded(Ctx* c, const void* a16, const void* w16, int64_t m, int64_t n,
                           int64_t k, const float* scale_a, const float* scales_w,
                           const float* bias, float* y) {
    if (m <= 0 || n <= 0) return TKV_HIP_OK;
    TKV_RC_TRY(gemm::check_sizes(m, n, k, "FP8 GEMM"));
    if (k % gemm::kBK != 0 || !aligned(a16, 16) || !aligned(w16, 16))
        return set_error(TKV_HIP_BAD_ARG, "FP8 GEMM (decoded): K or alignment");
    const auto* ha = static_cast<const uint8_t*>(a16);
    const auto* hw = static_cast<const uint8_t*>(w16);
    if (scales_w)
        return gemm::launch_any<gemm::PolicyF16>(
            c, ha, hw, m, n, 2 * k, gemm::EpiF8<true, false>{scale_a, 0, scales_w, bias}, y);
    return gemm::launch_any<gemm::PolicyF16>(c, ha, hw, m, n, 2 * k,
                                             gemm::EpiF8<false, false>{nullptr, 0, nullptr, bias},
                                             y);
}

int launch_fp8_ref_to_f16(Ctx* c, const uint8_t* src, int64_t bytes, void* dst) {
    if (bytes % 16 != 0) return set_error(TKV_HIP_BAD_ARG, "fp8 decode: bytes not a multiple of 16");
    return gemm::decode_into(c, src, bytes, dst);
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
    // Reference products: both operands decoded once into exact (pre-scaled)
    // f16, then the f16 MFMA over rows of 2 ldk bytes.
    auto run = [&](const auto& ep) -> int {
        if (fast) return gemm::launch_any<gemm::PolicyF8>(c, ua, uw, m, n, ldk, ep, y);
        uint8_t *ha, *hw;
        TKV_RC_TRY(gemm::decode_f16(c, ua, m * ldk, 10, &ha));
        TKV_RC_TRY(gemm::decode_f16(c, uw, n * ldk, 11, &hw));
        return gemm::launch_any<gemm::PolicyF16>(c, ha, hw, m, n, 2 * ldk, ep, y);
    };
    if (scales_w && scale_a_stride != 0)
        return run(gemm::EpiF8<true, true>{scale_a, scale_a_stride, scales_w, bias});
    if (scales_w) return run(gemm::EpiF8<true, false>{scale_a, 0, scales_w, bias});
    return run(gemm::EpiF8<false, false>{nullptr, 0, nullptr, bias});
}

}  // namespace tkv
