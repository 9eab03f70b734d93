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
#include <mutex>
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
    void* codes16 = nullptr; // WEIGHT_FP8: [n, ldk] halves, the codes' reference decode
    float* scales = nullptr; // [n] per-channel scales
    float* gscales = nullptr;// WEIGHT_Q8_0: [n, ldk / 32] group scales (the blocks' d)
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
    for (int64_t c = lane; c < cols; c += 64) q[r * ldq + c] = (uint8_t)e4m3_encode1(x[r * cols + c] * mul);
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
    if (wt->codes16) (void)hipFree(wt->codes16);
    if (wt->gscales) (void)hipFree(wt->gscales);
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
    if (wt->format == TKV_HIP_WEIGHT_Q8_0 && act_mode == TKV_HIP_ACT_PER_TOKEN) {
        const int rc = launch_decode_q8(c, x, m, k, static_cast<const uint8_t*>(wt->codes),
                                        wt->gscales, wt->ldk, wt->n, wt->bias, y);
        if (rc != TKV_HIP_UNSUPPORTED) return rc;
    }
    if (wt->ldk != k)
        return set_error(TKV_HIP_UNSUPPORTED, "linear_forward: K must be a multiple of the GEMM K step (128)");
    void* qa;
    TKV_RC_TRY(ctx_workspace(c, 0, (size_t)(m * k), &qa));
    tkv_hip_qparams_dev* ap = c->params + 1;
    if (wt->format == TKV_HIP_WEIGHT_Q8_0) {
        // the INT8 path's activation quantizers, then the group-scaled GEMM
        const float* sa = &ap->scale;
        int64_t stride = 0;
        if (act_mode == TKV_HIP_ACT_PER_TENSOR) {
            TKV_RC_TRY(launch_quant_i8_dynamic(c, x, m * k, TKV_HIP_RECIPE_PRIMARY, ap, qa, false));
        } else if (act_mode == TKV_HIP_ACT_PER_TOKEN) {
            void* ws;
            TKV_RC_TRY(ctx_workspace(c, 1, (size_t)m * 4, &ws));
            TKV_RC_TRY(launch_quant_rows(c, x, m, k, RM_DYNAMIC, nullptr, qa, false,
                                         static_cast<float*>(ws), nullptr, 1));
            sa = static_cast<const float*>(ws);
            stride = 1;
        } else {
            return set_error(TKV_HIP_BAD_ARG, "linear_forward: unknown act_mode");
        }
        const int rc = launch_gemm_q8(c, static_cast<int8_t*>(qa), static_cast<int8_t*>(wt->codes),
                                      wt->gscales, m, wt->n, k, sa, stride, wt->bias, y);
        return rc == TKV_HIP_UNSUPPORTED
                   ? set_error(rc, "linear_forward: Q8_0 GEMM sizes out of range")
                   : rc;
    }
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
    if (wt->codes16) {
        // reference products: the activation's codes go straight to their
        // f16 decode, which the GEMM multiplies with the weight's
        void* ha;
        TKV_RC_TRY(ctx_workspace(c, 10, (size_t)(m * k) * 2, &ha));
        TKV_RC_TRY(launch_quant_fp8_dynamic_f16(c, x, m * k, ap, ha));
        return launch_gemm_f8_decoded(c, ha, wt->codes16, m, wt->n, k, &ap->scale, wt->scales,
                                      wt->bias, y);
    }
    TKV_RC_TRY(launch_quant_fp8_dynamic(c, x, m * k, ap, qa, false));
    return launch_gemm_f8(c, static_cast<uint8_t*>(qa), static_cast<uint8_t*>(wt->codes), m, wt->n,
                          k, &ap->scale, 0, wt->scales, wt->bias, y,
                          wt->format == TKV_HIP_WEIGHT_FP8_FAST);
}

// ---------------------------------------------------------------------------
// Fixed scratch of tkv_hip_linear_forward_static, for callers that cannot
// allocate: one area per device, in the code object's own device memory, so
// no call ever allocates.  Layout (256-byte aligned parts):
//   activation codes   TKV_HIP_STATIC_CODES_BYTES
//   per-token scales   kStaticMaxRows f32
//   calibration partials, per-call params
//   split-K partial sums and arrival counts (zero at load; every call that
//   can use them clears them first), the grid-barrier slots (zero at load;
//   every launch advances each slot it uses by one generation, and the clear
//   above resets all of them together)
// Host code never names `scratch` directly as an address (on the host it is
// a stand-in symbol): static_scratch() resolves each device's copy once with
// hipGetSymbolAddress and every launch takes that pointer.
// ---------------------------------------------------------------------------
constexpr int64_t kStaticMaxRows = 65536;
constexpr size_t kAlign256(size_t v) { return (v + 255) & ~size_t(255); }
constexpr size_t kOffCodes = 0;
constexpr size_t kOffScales = kAlign256(kOffCodes + (size_t)TKV_HIP_STATIC_CODES_BYTES);
constexpr size_t kOffPartials = kAlign256(kOffScales + (size_t)kStaticMaxRows * 4);
constexpr size_t kOffParams = kAlign256(kOffPartials + sizeof(RedPartial) * kMaxReduceBlocks);
constexpr size_t kOffGemv = kAlign256(kOffParams + sizeof(tkv_hip_qparams_dev) * 64);
constexpr size_t kOffArrivals = kOffGemv + (size_t)kGemvSplitBlocks * 1024 * sizeof(int32_t);
constexpr size_t kOffGridSlots = kAlign256(kOffArrivals + (size_t)kGemvSplitBlocks * sizeof(unsigned));
constexpr size_t kOffScratchEnd = kAlign256(kOffGridSlots + (size_t)kMaxGridSlots * 8);

static __device__ __align__(256) uint8_t scratch[kOffScratchEnd];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static uint8_t* g_scratch_ptr[kMaxDevices];
static int g_scratch_cus[kMaxDevices];
static size_t g_scratch_lds[kMaxDevices];

// The calling thread's current device must be `dev`.
static int static_scratch(int dev, uint8_t** out, int* cus, size_t* lds) {
    if (dev < 0 || dev >= kMaxDevices) return set_error(TKV_HIP_NO_DEVICE, "device index out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        TKV_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        int n = 0;
        TKV_HIP_TRY(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
        g_scratch_cus[dev] = n;
        int l = 0;
        TKV_HIP_TRY(hipDeviceGetAttribute(&l, hipDeviceAttributeMaxSharedMemoryPerBlock, dev));
        g_scratch_lds[dev] = (size_t)l;
        g_scratch_ptr[dev] = static_cast<uint8_t*>(p);
    }
    *out = g_scratch_ptr[dev];
    *cus = g_scratch_cus[dev];
    *lds = g_scratch_lds[dev];
    return TKV_HIP_OK;
}

static int linear_forward_static_on(Weight* wt, const float* x, int64_t m, int32_t act_mode,
                                    float* y, void* stream);

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
            // The reference-products GEMM multiplies the codes' exact f16
            // decode: done here once instead of in every call.
            if (rc == TKV_HIP_OK && format == TKV_HIP_WEIGHT_FP8) {
                e = hipMalloc(&wt->codes16, (size_t)(n * wt->ldk) * 2);
                if (e != hipSuccess)
                    rc = fail_hip(e, "hipMalloc", __FILE__, __LINE__);
                else
                    rc = launch_fp8_ref_to_f16(c, static_cast<const uint8_t*>(wt->codes),
                                               n * wt->ldk, wt->codes16);
            }
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

int32_t tkv_hip_weight_create_gguf_q8_0(int64_t ctx, const uint8_t* raw, int64_t n, int64_t k,
                                        const float* bias, int64_t* handle_out) {
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    if (!raw || !handle_out || n <= 0 || k <= 0 || k % 32 != 0 || n >= (1ll << 28))
        return set_error(TKV_HIP_BAD_ARG, "weight_create_gguf_q8_0: bad arguments (K % 32 != 0?)");
    if (c->capturing)
        return set_error(TKV_HIP_BAD_ARG, "weight_create_gguf_q8_0: allocates and synchronizes, not inside a stream capture");
    Weight* wt = new (std::nothrow) Weight();
    if (!wt) return set_error(TKV_HIP_OOM, "weight_create_gguf_q8_0: host allocation failed");
    int rc = weight_alloc(c, wt, n, k, TKV_HIP_WEIGHT_Q8_0, bias);
    if (rc == TKV_HIP_OK) {
        hipError_t e = hipMalloc(reinterpret_cast<void**>(&wt->gscales),
                                 (size_t)(n * (wt->ldk / 32)) * 4);
        if (e != hipSuccess)
            rc = fail_hip(e, "hipMalloc", __FILE__, __LINE__);
        else
            rc = launch_q8_0_unpack(c, raw, n, k, wt->ldk, static_cast<uint8_t*>(wt->codes),
                                    wt->gscales);
        if (rc == TKV_HIP_UNSUPPORTED)
            rc = set_error(TKV_HIP_BAD_ARG, "weight_create_gguf_q8_0: layout not supported");
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

int32_t tkv_hip_weight_free(int64_t handle) {
    weight_release(reinterpret_cast<Weight*>(handle));
    return TKV_HIP_OK;
}

int32_t tkv_hip_weight_info(int64_t handle, void** codes, float** scales, float** bias, int64_t* n,
                            int64_t* k, int32_t* format) {
    Weight* wt = reinterpret_cast<Weight*>(handle);
    if (!wt) return set_error(TKV_HIP_BAD_ARG, "NULL weight handle");
    if (codes) *codes = wt->codes;
    if (scales) *scales = wt->format == TKV_HIP_WEIGHT_Q8_0 ? wt->gscales : wt->scales;
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

int32_t tkv_hip_linear_forward_static(int64_t weight, const float* x, int64_t m,
                                      int32_t act_mode, float* y, void* stream) {
    Weight* wt = reinterpret_cast<Weight*>(weight);
    if (!wt || !x || !y || m < 0)
        return set_error(TKV_HIP_BAD_ARG, "linear_forward_static: bad arguments");
    if (wt->format != TKV_HIP_WEIGHT_INT8)
        return set_error(TKV_HIP_UNSUPPORTED, "linear_forward_static: INT8 weights only");
    if (m * wt->k > TKV_HIP_STATIC_CODES_BYTES || m > kStaticMaxRows)
        return set_error(TKV_HIP_BAD_ARG,
                         "linear_forward_static: m * k = " + std::to_string(m * wt->k) +
                             " activation codes (or m = " + std::to_string(m) +
                             " rows) exceed the static scratch (" +
                             std::to_string(TKV_HIP_STATIC_CODES_BYTES) + " bytes, " +
                             std::to_string(kStaticMaxRows) + " rows)");
    if (m == 0) return TKV_HIP_OK;
    // The weight's device is made current for the call and the caller's
    // current device restored before returning, whatever the outcome.
    int prev_dev = 0;
    TKV_HIP_TRY(hipGetDevice(&prev_dev));
    TKV_HIP_TRY(hipSetDevice(wt->device));
    const int rc = linear_forward_static_on(wt, x, m, act_mode, y, stream);
    const hipError_t e = hipSetDevice(prev_dev);
    if (rc != TKV_HIP_OK) return rc;
    if (e != hipSuccess) return fail_hip(e, "hipSetDevice(restore)", __FILE__, __LINE__);
    return TKV_HIP_OK;
}

}  // extern "C"

namespace tkv {

// The static entry's body, with wt->device current.
static int linear_forward_static_on(Weight* wt, const float* x, int64_t m, int32_t act_mode,
                                    float* y, void* stream) {
    uint8_t* base;
    int cus;
    size_t lds;
    TKV_RC_TRY(static_scratch(wt->device, &base, &cus, &lds));
    Ctx c;
    c.device = wt->device;
    c.num_cus = cus;
    if (lds) c.max_lds = lds;
    c.stream = static_cast<hipStream_t>(stream);
    c.own_stream = nullptr;
    c.no_alloc = true;
    c.partials = reinterpret_cast<RedPartial*>(base + kOffPartials);
    c.params = reinterpret_cast<tkv_hip_qparams_dev*>(base + kOffParams);
    c.gemv_part = reinterpret_cast<int32_t*>(base + kOffGemv);
    c.gemv_arrivals = reinterpret_cast<unsigned*>(base + kOffArrivals);
    c.grid_slots = reinterpret_cast<unsigned long long*>(base + kOffGridSlots);
    c.ws[0] = base + kOffCodes;
    c.ws_bytes[0] = (size_t)TKV_HIP_STATIC_CODES_BYTES;
    c.ws[1] = base + kOffScales;
    c.ws_bytes[1] = (size_t)kStaticMaxRows * 4;
    // The split-K skinny GEMM (per-tensor activations, m <= 32) needs its
    // partial sums and arrival counts at zero; its kernels leave them so,
    // but this area is shared by every call on the device: clear them (a
    // fill kernel, which a stream capture records as a kernel node).
    if (act_mode == TKV_HIP_ACT_PER_TENSOR && m <= 32)
        TKV_RC_TRY(launch_fill(&c, c.gemv_part, 0, kOffScratchEnd - kOffGemv));
    return linear_forward(&c, wt, x, m, act_mode, y);
}

}  // namespace tkv
