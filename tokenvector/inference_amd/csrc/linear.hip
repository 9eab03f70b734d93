// linear.hip -- device-resident quantized weights and the W8A8 linear that
// the reference's QuantizedGemm node runs (tv/runtime/session.tkv:678-697),
// as one call: activation calibrate + quantize, GEMM, dequant + bias.
//
// CS1 of the reference quantizes weights offline (calibrate_per_channel_minmax
// + quantize_int8_per_channel, engine.tkv:202-213,237-250) and activations
// per call (calibrate_minmax + quantize_int8_symmetric, :13-36,216-226).  A
// weight handle keeps the packed codes, per-channel scales and bias resident
// in HBM, as simd_gemm_packed_create keeps packed f32 tiles
// (docs/HANDOFF.md:1675).
#include <new>
#include <string>

#include "tkv_device.h"
#include "tkv_internal.h"

namespace tkv {

struct Weight {
    int device = 0;
    int format = TKV_HIP_WEIGHT_INT8;
    int64_t n = 0, k = 0, ldk = 0;
    void* codes = nullptr;   // [n, ldk] int8 or e4m3 bytes, zero-padded
    float* scales = nullptr; // [n] per-channel scales
    float* bias = nullptr;   // [n] or null
};

// Per-row scaled e4m3 encode: q[r, c] = encode(fl32(x[r, c] * fl32(1 / s[r]))),
// rows written with leading dimension ldq.  Extension (FP8 per-channel
// weights are not in the reference).
__global__ __launch_bounds__(256) void k_fp8_encode_rows(const float* __restrict__ x, int64_t rows,
                                                         int64_t cols,
                                                         const float* __restrict__ s,
                                                         uint8_t* __restrict__ q, int64_t ldq) {
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const float mul = 1.0f / s[r];
    for (int64_t c = lane; c < cols; c += 64) q[r * ldq + c] = (uint8_t)e4m3_encode(x[r * cols + c] * mul);
}

// FP8 per-channel scales: s[r] = fl32(max(|x[r,:]|, 1e-8) / kFp8Target).
__global__ __launch_bounds__(256) void k_fp8_row_scales(const float* __restrict__ x, int64_t rows,
                                                        int64_t cols, float* __restrict__ s) {
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    float am = 0.0f;
    for (int64_t c = lane; c < cols; c += 64) am = fmaxf(am, fabsf(x[r * cols + c]));
    am = wave_max(am);
    if (lane == 0) {
        double a = am < 0.00000001 ? 0.00000001 : (double)am;
        s[r] = (float)(a / (double)kFp8Target);
    }
}

static int weight_alloc(Ctx* c, Weight* wt, int64_t n, int64_t k, int format, const float* bias) {
    wt->device = c->device;
    wt->format = format;
    wt->n = n;
    wt->k = k;
    const int64_t ka = gemm_k_align();
    wt->ldk = (k + ka - 1) / ka * ka;  // the GEMM slice depth: no per-call repack
    TKV_HIP_TRY(hipMalloc(&wt->codes, (size_t)(n * wt->ldk)));
    TKV_HIP_TRY(hipMalloc(reinterpret_cast<void**>(&wt->scales), (size_t)n * 4));
    // zero padding past k (a kernel: the library records no memset nodes)
    TKV_RC_TRY(launch_fill(c, wt->codes, 0, n * wt->ldk));
    if (bias) {
        TKV_HIP_TRY(hipMalloc(reinterpret_cast<void**>(&wt->bias), (size_t)n * 4));
        TKV_HIP_TRY(hipMemcpyAsync(wt->bias, bias, (size_t)n * 4, hipMemcpyDeviceToDevice, c->stream));
    }
    return TKV_HIP_OK;
}

static void weight_release(Weight* wt) {
    if (!wt) return;
    // Teardown: errors here leave nothing the caller can act on.
    (void)hipSetDevice(wt->device);
    (void)hipDeviceSynchronize();
    if (wt->codes) (void)hipFree(wt->codes);
    if (wt->scales) (void)hipFree(wt->scales);
    if (wt->bias) (void)hipFree(wt->bias);
    delete wt;
}

// The per-call part of CS1 on context c: activation calibrate + quantize
// (per tensor or per token), GEMM, dequant + bias.
static int linear_forward(Ctx* c, Weight* wt, const float* x, int64_t m, int32_t act_mode,
                          float* y) {
    if (!wt || !x || !y || m < 0) return set_error(TKV_HIP_BAD_ARG, "linear_forward: bad arguments");
    if (m == 0) return TKV_HIP_OK;
    const int64_t k = wt->k;
    if (wt->format == TKV_HIP_WEIGHT_INT8 && act_mode == TKV_HIP_ACT_PER_TOKEN) {
        // decode batches: quantize + GEMM + epilogue in one kernel, reading
        // the weight through its padded row stride
        const int rc = launch_decode_i8(c, x, m, k, static_cast<const uint8_t*>(wt->codes),
                                        wt->ldk, wt->n, wt->scales, wt->bias, y);
        if (rc != TKV_HIP_UNSUPPORTED) return rc;
    }
    if (wt->ldk != k)
        return set_error(TKV_HIP_UNSUPPORTED, "linear_forward: K must be a multiple of the GEMM K step (128)");
    void* qa;
    TKV_RC_TRY(ctx_workspace(c, 0, (size_t)(m * k), &qa));
    tkv_hip_qparams_dev* ap = c->params + 1;
    if (wt->format == TKV_HIP_WEIGHT_INT8) {
        I8Epilogue ep;
        ep.mode = EPI_PER_CHANNEL;
        ep.recipe = TKV_HIP_RECIPE_PRIMARY;
        ep.scale_w = 0.0f;
        ep.scales_w = wt->scales;
        ep.bias = wt->bias;
        if (act_mode == TKV_HIP_ACT_PER_TENSOR) {
            TKV_RC_TRY(launch_quant_i8_dynamic(c, x, m * k, TKV_HIP_RECIPE_PRIMARY, ap, qa, false));
            ep.scale_a = &ap->scale;
            ep.scale_a_stride = 0;
        } else if (act_mode == TKV_HIP_ACT_PER_TOKEN) {
            void* sa;
            TKV_RC_TRY(ctx_workspace(c, 1, (size_t)m * 4, &sa));
            TKV_RC_TRY(launch_quant_rows(c, x, m, k, RM_DYNAMIC, nullptr, qa, false,
                                         static_cast<float*>(sa), nullptr, 1));
            ep.scale_a = static_cast<float*>(sa);
            ep.scale_a_stride = 1;
        } else {
            return set_error(TKV_HIP_BAD_ARG, "linear_forward: unknown act_mode");
        }
        return launch_gemm_i8(c, static_cast<int8_t*>(qa), static_cast<int8_t*>(wt->codes), m,
                              wt->n, k, ep, y);
    }
    if (act_mode != TKV_HIP_ACT_PER_TENSOR)
        return set_error(TKV_HIP_UNSUPPORTED, "linear_forward: FP8 weights take per-tensor activations");
    TKV_RC_TRY(launch_quant_fp8_dynamic(c, x, m * k, ap, qa, false));
    return launch_gemm_f8(c, static_cast<uint8_t*>(qa), static_cast<uint8_t*>(wt->codes), m, wt->n,
                          k, &ap->scale, 0, wt->scales, wt->bias, y,
                          wt->format == TKV_HIP_WEIGHT_FP8_FAST);
}

}  // namespace tkv

using namespace tkv;

extern "C" {

int32_t tkv_hip_weight_create(int64_t ctx, const float* w, int64_t n, int64_t k,
                              const float* bias, int32_t format, int64_t* handle_out) {
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    if (!w || !handle_out || n <= 0 || k <= 0)
        return set_error(TKV_HIP_BAD_ARG, "weight_create: empty weight or NULL output");
    if (c->capturing)
        return set_error(TKV_HIP_BAD_ARG, "weight_create: allocates and synchronizes, not inside a stream capture");
    if (format != TKV_HIP_WEIGHT_INT8 && format != TKV_HIP_WEIGHT_FP8 &&
        format != TKV_HIP_WEIGHT_FP8_FAST)
        return set_error(TKV_HIP_BAD_ARG, "weight_create: unknown format");
    Weight* wt = new (std::nothrow) Weight();
    if (!wt) return set_error(TKV_HIP_OOM, "weight_create: host allocation failed");
    int rc = weight_alloc(c, wt, n, k, format, bias);
    if (rc == TKV_HIP_OK) {
        if (format == TKV_HIP_WEIGHT_INT8) {
            // calibrate_per_channel_minmax (symmetric) + quantize_int8_per_channel
            rc = launch_quant_rows(c, w, n, k, RM_CALIBRATE, nullptr, nullptr, false, wt->scales,
                                   nullptr, 1);
            void* tmp = wt->codes;
            if (rc == TKV_HIP_OK && wt->ldk != k) rc = ctx_workspace(c, 2, (size_t)(n * k), &tmp);
            if (rc == TKV_HIP_OK)
                rc = launch_quant_rows(c, w, n, k, RM_PER_CHANNEL, wt->scales, tmp, false, nullptr,
                                       nullptr, 1);
            if (rc == TKV_HIP_OK && tmp != wt->codes) {
                hipError_t e = hipMemcpy2DAsync(wt->codes, (size_t)wt->ldk, tmp, (size_t)k,
                                                (size_t)k, (size_t)n, hipMemcpyDeviceToDevice,
                                                c->stream);
                if (e != hipSuccess) rc = fail_hip(e, "hipMemcpy2DAsync", __FILE__, __LINE__);
            }
        } else {
            int64_t blocks = ceil_div(n, 4);
            hipLaunchKernelGGL(k_fp8_row_scales, dim3((unsigned)blocks), dim3(256), 0, c->stream,
                               w, n, k, wt->scales);
            hipLaunchKernelGGL(k_fp8_encode_rows, dim3((unsigned)blocks), dim3(256), 0, c->stream,
                               w, n, k, wt->scales, static_cast<uint8_t*>(wt->codes), wt->ldk);
            hipError_t e = hipGetLastError();
            if (e != hipSuccess) rc = fail_hip(e, "fp8 weight pack", __FILE__, __LINE__);
        }
    }
    if (rc == TKV_HIP_OK) {
        hipError_t e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) rc = fail_hip(e, "hipStreamSynchronize", __FILE__, __LINE__);
    }
    if (rc != TKV_HIP_OK) {
        weight_release(wt);
        return rc;
    }
    *handle_out = reinterpret_cast<int64_t>(wt);
    return TKV_HIP_OK;
}

int32_t tkv_hip_weight_create_int8(int64_t ctx, const int8_t* codes, const float* scales,
                                   int64_t n, int64_t k, const float* bias, int64_t* handle_out) {
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    if (!codes || !scales || !handle_out || n <= 0 || k <= 0)
        return set_error(TKV_HIP_BAD_ARG, "weight_create_int8: bad arguments");
    if (c->capturing)
        return set_error(TKV_HIP_BAD_ARG, "weight_create_int8: allocates and synchronizes, not inside a stream capture");
    Weight* wt = new (std::nothrow) Weight();
    if (!wt) return set_error(TKV_HIP_OOM, "weight_create_int8: host allocation failed");
    int rc = weight_alloc(c, wt, n, k, TKV_HIP_WEIGHT_INT8, bias);
    if (rc == TKV_HIP_OK) {
        hipError_t e = hipMemcpy2DAsync(wt->codes, (size_t)wt->ldk, codes, (size_t)k, (size_t)k,
                                        (size_t)n, hipMemcpyDeviceToDevice, c->stream);
        if (e == hipSuccess)
            e = hipMemcpyAsync(wt->scales, scales, (size_t)n * 4, hipMemcpyDeviceToDevice, c->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) rc = fail_hip(e, "weight_create_int8 copy", __FILE__, __LINE__);
    }
    if (rc != TKV_HIP_OK) {
        weight_release(wt);
        return rc;
    }
    *handle_out = reinterpret_cast<int64_t>(wt);
    return TKV_HIP_OK;
}

int32_t tkv_hip_weight_free(int64_t handle) {
    weight_release(reinterpret_cast<Weight*>(handle));
    return TKV_HIP_OK;
}

int32_t tkv_hip_weight_info(int64_t handle, void** codes, float** scales, float** bias, int64_t* n,
                            int64_t* k, int32_t* format) {
    Weight* wt = reinterpret_cast<Weight*>(handle);
    if (!wt) return set_error(TKV_HIP_BAD_ARG, "NULL weight handle");
    if (codes) *codes = wt->codes;
    if (scales) *scales = wt->scales;
    if (bias) *bias = wt->bias;
    if (n) *n = wt->n;
    if (k) *k = wt->ldk;
    if (format) *format = wt->format;
    return TKV_HIP_OK;
}

int32_t tkv_hip_linear_forward(int64_t ctx, int64_t weight, const float* x, int64_t m,
                               int32_t act_mode, float* y) {
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    return linear_forward(c, reinterpret_cast<Weight*>(weight), x, m, act_mode, y);
}

}  // extern "C"
