// capi.hip -- extern "C" entry points of libtkv_hip (declared in
// include/tkv_hip.h).  Host-pointer mirrors validate exactly where the .tkv
// functions raise ValueError (returning TKV_HIP_BAD_ARG), move the
// reference's int32-per-code lists to and from packed device codes, and run
// the same kernels as the device-pointer variants.
#include <climits>
#include <cstring>
#include <vector>

#include "tkv_internal.h"

using namespace tkv;

namespace {

// Host-mirror workspace slots (slots 2 and 3 belong to the GEMM launchers).
enum { WS_IN = 0, WS_OUT = 1, WS_A = 4, WS_W = 5, WS_SMALL = 6, WS_Y = 7 };

int begin_host(Ctx** c) {
    if (!hip_path_enabled())
        return set_error(TKV_HIP_UNSUPPORTED, "TKV_QUANT_HIP=0: HIP path disabled");
    return ctx_get(0, c);
}

int upload(Ctx* c, int slot, const void* h, size_t bytes, void** d) {
    TKV_RC_TRY(ctx_workspace(c, slot, bytes, d));
    if (bytes) TKV_HIP_TRY(hipMemcpyAsync(*d, h, bytes, hipMemcpyHostToDevice, c->stream));
    return TKV_HIP_OK;
}

int download(Ctx* c, void* h, const void* d, size_t bytes) {
    if (bytes) TKV_HIP_TRY(hipMemcpyAsync(h, d, bytes, hipMemcpyDeviceToHost, c->stream));
    TKV_HIP_TRY(hipStreamSynchronize(c->stream));
    return TKV_HIP_OK;
}

// int32 codes (List<int>) -> int8 rows padded to ldk (multiple of 16).
// Codes outside [lo, hi] cannot ride the int8 datapath: UNSUPPORTED, so the
// caller keeps its own loop.
int pack_codes(const int32_t* src, int64_t rows, int64_t k, int64_t ldk, int bias, int lo, int hi,
               std::vector<int8_t>& out) {
    out.assign((size_t)(rows * ldk), 0);
    for (int64_t r = 0; r < rows; r++) {
        const int32_t* s = src + r * k;
        int8_t* d = out.data() + r * ldk;
        for (int64_t i = 0; i < k; i++) {
            int v = s[i];
            if (v < lo || v > hi)
                return set_error(TKV_HIP_UNSUPPORTED, "code outside the int8 datapath range");
            d[i] = (int8_t)(v + bias);
        }
    }
    return TKV_HIP_OK;
}

int check_recipe(int32_t recipe) {
    if (recipe != TKV_HIP_RECIPE_PRIMARY && recipe != TKV_HIP_RECIPE_ALTERNATE)
        return set_error(TKV_HIP_BAD_ARG, "unknown recipe");
    return TKV_HIP_OK;
}

// Shared body of the INT8 GEMM host mirrors.
int host_gemm_i8(const int32_t* pa, const int32_t* pw, const float* pbias, int64_t n_bias,
                 void* py, bool accum, int64_t m, int64_t n, int64_t k, float scale_a,
                 float scale_w, const float* scales_w, int64_t n_scales, int32_t recipe) {
    if (m < 0 || n < 0 || k < 0) return set_error(TKV_HIP_BAD_ARG, "negative GEMM size");
    TKV_RC_TRY(check_recipe(recipe));
    if (!accum && n_bias > 0 && n_bias < n)
        return set_error(TKV_HIP_BAD_ARG, "bias shorter than N");
    Ctx* c;
    TKV_RC_TRY(begin_host(&c));
    if (m == 0 || n == 0) return TKV_HIP_OK;
    if (k == 0) {  // empty dot products (acc = 0): one zero term gives the same sums
        std::vector<int32_t> za((size_t)m, 0), zw((size_t)n, 0);
        return host_gemm_i8(za.data(), zw.data(), pbias, n_bias, py, accum, m, n, 1, scale_a,
                            scale_w, scales_w, n_scales, recipe);
    }
    const int64_t ka = gemm_k_align();
    int64_t ldk = (k + ka - 1) / ka * ka;  // zero-padded: no repack in the launcher
    std::vector<int8_t> ha, hw;
    TKV_RC_TRY(pack_codes(pa, m, k, ldk, 0, -128, 127, ha));
    TKV_RC_TRY(pack_codes(pw, n, k, ldk, 0, -128, 127, hw));
    void *da, *dw, *dsmall, *dy;
    TKV_RC_TRY(upload(c, WS_A, ha.data(), ha.size(), &da));
    TKV_RC_TRY(upload(c, WS_W, hw.data(), hw.size(), &dw));
    // small arrays: [scale_a][scales_w (n)][bias (n)]
    std::vector<float> small(1 + 2 * (size_t)n, 0.0f);
    small[0] = scale_a;
    if (scales_w) memcpy(&small[1], scales_w, sizeof(float) * (size_t)n);
    bool has_bias = !accum && n_bias > 0;
    if (has_bias) memcpy(&small[1 + n], pbias, sizeof(float) * (size_t)n);
    TKV_RC_TRY(upload(c, WS_SMALL, small.data(), small.size() * sizeof(float), &dsmall));
    size_t ybytes = (size_t)(m * n) * 4;
    TKV_RC_TRY(ctx_workspace(c, WS_Y, ybytes, &dy));
    const float* fs = static_cast<const float*>(dsmall);
    I8Epilogue ep;
    ep.mode = accum ? EPI_ACCUM_I32 : (scales_w ? EPI_PER_CHANNEL : EPI_SYMMETRIC);
    ep.recipe = recipe;
    ep.scale_a = fs;
    ep.scale_a_stride = 0;
    ep.scale_w = scale_w;
    ep.scales_w = scales_w ? fs + 1 : nullptr;
    ep.bias = has_bias ? fs + 1 + n : nullptr;
    ep.k_logical = k;  // rows are zero padded to ldk
    TKV_RC_TRY(launch_gemm_i8(c, static_cast<int8_t*>(da), static_cast<int8_t*>(dw), m, n, ldk,
                              ep, dy));
    return download(c, py, dy, ybytes);
}

// mult = sa * sw / sy of the QLinearMatMul node (session.tkv:2024-2027).
double qlinear_mult(float sa, float sw, float sy, int32_t recipe) {
    if (recipe == TKV_HIP_RECIPE_PRIMARY) {
        double dsy = (double)sy;
        if (dsy == 0.0) dsy = 1.0;
        return (double)sa * (double)sw / dsy;
    }
    const float fsy = sy == 0.0f ? 1.0f : sy;
    return (double)((sa * sw) / fsy);
}

}  // namespace

extern "C" {

// ===========================================================================
// Host-pointer mirrors
// ===========================================================================

}  // extern "C"

namespace {

// Host mirror of a heavier calibrator: n == 0 gives _quant_identity()
// (engine.tkv:9-10), as each of them returns first.
template <class F>
int32_t host_calibrate(const float* data, int64_t n, float* scale, int64_t* zero_point,
                       float* min_val, float* max_val, F&& launch) {
    if (n < 0) return set_error(TKV_HIP_BAD_ARG, "negative length");
    tkv_hip_qparams_dev p;
    if (n == 0) {
        p.scale = 1.0f;
        p.zero_point = 0;
        p.min_val = -3.4028234663852886e38f;
        p.max_val = 3.4028234663852886e38f;
    } else {
        void* dx;
        Ctx* c;
        TKV_RC_TRY(begin_host(&c));
        TKV_RC_TRY(upload(c, WS_IN, data, (size_t)n * 4, &dx));
        TKV_RC_TRY(launch(c, static_cast<const float*>(dx), c->params));
        TKV_RC_TRY(download(c, &p, c->params, sizeof(p)));
    }
    if (scale) *scale = p.scale;
    if (zero_point) *zero_point = p.zero_point;
    if (min_val) *min_val = p.min_val;
    if (max_val) *max_val = p.max_val;
    return TKV_HIP_OK;
}

}  // namespace

extern "C" {

int32_t tkv_hip_calibrate_kl(const float* data, int64_t n, int64_t num_bins,
                             int64_t target_bins, float* scale, int64_t* zero_point,
                             float* min_val, float* max_val) {
    return host_calibrate(data, n, scale, zero_point, min_val, max_val,
                          [&](Ctx* c, const float* x, tkv_hip_qparams_dev* o) {
                              return launch_calibrate_kl(c, x, n, num_bins, target_bins, o);
                          });
}

int32_t tkv_hip_calibrate_percentile(const float* data, int64_t n, float percentile,
                                     int32_t symmetric, float* scale, int64_t* zero_point,
                                     float* min_val, float* max_val) {
    if (n > 0 && !(percentile > 0.0f && percentile <= 100.0f))
        return set_error(TKV_HIP_BAD_ARG, "percentile must be in (0, 100]");
    return host_calibrate(data, n, scale, zero_point, min_val, max_val,
                          [&](Ctx* c, const float* x, tkv_hip_qparams_dev* o) {
                              return launch_calibrate_percentile(c, x, n, percentile, symmetric,
                                                                 o);
                          });
}

int32_t tkv_hip_calibrate_mse(const float* data, int64_t n, int64_t num_candidates,
                              float* scale, int64_t* zero_point, float* min_val,
                              float* max_val) {
    return host_calibrate(data, n, scale, zero_point, min_val, max_val,
                          [&](Ctx* c, const float* x, tkv_hip_qparams_dev* o) {
                              return launch_calibrate_mse(c, x, n, num_candidates, o);
                          });
}

int32_t tkv_hip_calibrate_minmax(const float* data, int64_t n, int32_t symmetric, float* scale,
                                 int64_t* zero_point, float* min_val, float* max_val) {
    if (n < 0) return set_error(TKV_HIP_BAD_ARG, "negative length");
    tkv_hip_qparams_dev p;
    if (n == 0) {  // _quant_identity(), engine.tkv:9-10
        p.scale = 1.0f;
        p.zero_point = 0;
        p.min_val = -3.4028234663852886e38f;
        p.max_val = 3.4028234663852886e38f;
    } else {
        void* dx;
        Ctx* c;
        TKV_RC_TRY(begin_host(&c));
        TKV_RC_TRY(upload(c, WS_IN, data, (size_t)n * 4, &dx));
        TKV_RC_TRY(launch_minmax_tensor(c, static_cast<float*>(dx), n,
                                        symmetric ? MM_SYMMETRIC : MM_ASYMMETRIC,
                                        TKV_HIP_RECIPE_PRIMARY, c->params));
        TKV_RC_TRY(download(c, &p, c->params, sizeof(p)));
    }
    if (scale) *scale = p.scale;
    if (zero_point) *zero_point = p.zero_point;
    if (min_val) *min_val = p.min_val;
    if (max_val) *max_val = p.max_val;
    return TKV_HIP_OK;
}

int32_t tkv_hip_calibrate_per_channel_minmax(const float* data, int64_t n_data, int64_t rows,
                                             int64_t cols, int32_t symmetric, float* scales,
                                             int64_t* zero_points, float* min_vals,
                                             float* max_vals) {
    if (rows <= 0 || cols <= 0) return set_error(TKV_HIP_BAD_ARG, "rows/cols must be > 0");
    if (n_data < rows * cols) return set_error(TKV_HIP_BAD_ARG, "data smaller than rows*cols");
    void *dx, *dp;
    Ctx* c;
    TKV_RC_TRY(begin_host(&c));
    TKV_RC_TRY(upload(c, WS_IN, data, (size_t)(rows * cols) * 4, &dx));
    TKV_RC_TRY(ctx_workspace(c, WS_OUT, sizeof(tkv_hip_qparams_dev) * (size_t)rows, &dp));
    auto* rp = static_cast<tkv_hip_qparams_dev*>(dp);
    TKV_RC_TRY(launch_quant_rows(c, static_cast<float*>(dx), rows, cols, RM_CALIBRATE_FULL,
                                 nullptr, nullptr, false, nullptr, rp, symmetric ? 1 : 0));
    std::vector<tkv_hip_qparams_dev> hp((size_t)rows);
    TKV_RC_TRY(download(c, hp.data(), rp, sizeof(tkv_hip_qparams_dev) * (size_t)rows));
    for (int64_t r = 0; r < rows; r++) {
        if (scales) scales[r] = hp[r].scale;
        if (zero_points) zero_points[r] = hp[r].zero_point;
        if (min_vals) min_vals[r] = hp[r].min_val;
        if (max_vals) max_vals[r] = hp[r].max_val;
    }
    return TKV_HIP_OK;
}

int32_t tkv_hip_quantize_int8_symmetric_recipe(const float* src, int64_t n_src, int32_t* dst,
                                               int64_t n_dst, float scale, int32_t recipe) {
    TKV_RC_TRY(check_recipe(recipe));
    if (n_src < 0 || n_dst < n_src) return set_error(TKV_HIP_BAD_ARG, "dst too small");
    if (n_src == 0) return TKV_HIP_OK;
    tkv_hip_qparams_dev p;
    memset(&p, 0, sizeof(p));
    p.scale = scale;
    // engine.tkv:219-222: f32 reciprocal (primary) or f64 (alternate)
    if ((double)scale > 0.00000001)
        p.inv = recipe == TKV_HIP_RECIPE_PRIMARY ? (double)(1.0f / scale) : 1.0 / (double)scale;
    else
        p.inv = 1.0 / 0.00000001;
    void *dx, *dq;
    Ctx* c;
    TKV_RC_TRY(begin_host(&c));
    TKV_RC_TRY(upload(c, WS_IN, src, (size_t)n_src * 4, &dx));
    TKV_HIP_TRY(hipMemcpyAsync(c->params, &p, sizeof(p), hipMemcpyHostToDevice, c->stream));
    TKV_RC_TRY(ctx_workspace(c, WS_OUT, (size_t)n_src * 4, &dq));
    TKV_RC_TRY(launch_quant_i8_tensor(c, static_cast<float*>(dx), n_src, c->params, dq, true));
    return download(c, dst, dq, (size_t)n_src * 4);
}

int32_t tkv_hip_quantize_int8_symmetric(const float* src, int64_t n_src, int32_t* dst,
                                        int64_t n_dst, float scale) {
    return tkv_hip_quantize_int8_symmetric_recipe(src, n_src, dst, n_dst, scale,
                                                  TKV_HIP_RECIPE_PRIMARY);
}

int32_t tkv_hip_dequantize_int8_symmetric(const int32_t* src, int64_t n_src, float* dst,
                                          int64_t n_dst, float scale) {
    if (n_src < 0 || n_dst < n_src) return set_error(TKV_HIP_BAD_ARG, "dst too small");
    if (n_src == 0) return TKV_HIP_OK;
    void *dq, *dy;
    Ctx* c;
    TKV_RC_TRY(begin_host(&c));
    TKV_RC_TRY(upload(c, WS_IN, src, (size_t)n_src * 4, &dq));
    TKV_RC_TRY(ctx_workspace(c, WS_OUT, (size_t)n_src * 4, &dy));
    TKV_RC_TRY(launch_dequant_i8(c, dq, true, 1, n_src, scale, nullptr, static_cast<float*>(dy)));
    return download(c, dst, dy, (size_t)n_src * 4);
}

int32_t tkv_hip_quantize_int8_per_channel(const float* src, int64_t n_src, int32_t* dst,
                                          int64_t n_dst, int64_t rows, int64_t cols,
                                          const float* scales, int64_t n_scales) {
    if (rows < 0 || cols < 0) return set_error(TKV_HIP_BAD_ARG, "negative rows/cols");
    if (n_dst < rows * cols || n_src < rows * cols) return set_error(TKV_HIP_BAD_ARG, "span too small");
    if (n_scales < rows) return set_error(TKV_HIP_BAD_ARG, "scales smaller than rows");
    if (rows * cols == 0) return TKV_HIP_OK;
    void *dx, *ds, *dq;
    Ctx* c;
    TKV_RC_TRY(begin_host(&c));
    TKV_RC_TRY(upload(c, WS_IN, src, (size_t)(rows * cols) * 4, &dx));
    TKV_RC_TRY(upload(c, WS_SMALL, scales, (size_t)rows * 4, &ds));
    TKV_RC_TRY(ctx_workspace(c, WS_OUT, (size_t)(rows * cols) * 4, &dq));
    TKV_RC_TRY(launch_quant_rows(c, static_cast<float*>(dx), rows, cols, RM_PER_CHANNEL,
                                 static_cast<float*>(ds), dq, true, nullptr, nullptr, 1));
    return download(c, dst, dq, (size_t)(rows * cols) * 4);
}

int32_t tkv_hip_dequantize_int8_per_channel(const int32_t* src, int64_t n_src, float* dst,
                                            int64_t n_dst, int64_t rows, int64_t cols,
                                            const float* scales, int64_t n_scales) {
    if (rows < 0 || cols < 0) return set_error(TKV_HIP_BAD_ARG, "negative rows/cols");
    if (n_dst < rows * cols || n_src < rows * cols) return set_error(TKV_HIP_BAD_ARG, "span too small");
    if (n_scales < rows) return set_error(TKV_HIP_BAD_ARG, "scales smaller than rows");
    if (rows * cols == 0) return TKV_HIP_OK;
    void *dq, *ds, *dy;
    Ctx* c;
    TKV_RC_TRY(begin_host(&c));
    TKV_RC_TRY(upload(c, WS_IN, src, (size_t)(rows * cols) * 4, &dq));
    TKV_RC_TRY(upload(c, WS_SMALL, scales, (size_t)rows * 4, &ds));
    TKV_RC_TRY(ctx_workspace(c, WS_OUT, (size_t)(rows * cols) * 4, &dy));
    TKV_RC_TRY(launch_dequant_i8(c, dq, true, rows, cols, 0.0f, static_cast<float*>(ds),
                                 static_cast<float*>(dy)));
    return download(c, dst, dy, (size_t)(rows * cols) * 4);
}

int32_t tkv_hip_quantize_dynamic_int8_rowwise(const float* src, int64_t n_src, int32_t* dst,
                                              int64_t n_dst, int64_t rows, int64_t cols,
                                              float* scales_out, int64_t n_scales_out) {
    if (rows < 0 || cols < 0) return set_error(TKV_HIP_BAD_ARG, "negative rows/cols");
    if (n_dst < rows * cols || n_src < rows * cols) return set_error(TKV_HIP_BAD_ARG, "span too small");
    if (n_scales_out < rows) return set_error(TKV_HIP_BAD_ARG, "scales_out smaller than rows");
    if (rows == 0) return TKV_HIP_OK;
    if (cols == 0) {  // am = 1e-8 floor for every row
        for (int64_t r = 0; r < rows; r++) scales_out[r] = (float)(0.00000001 / 127.0);
        return TKV_HIP_OK;
    }
    void *dx, *dq, *ds;
    Ctx* c;
    TKV_RC_TRY(begin_host(&c));
    TKV_RC_TRY(upload(c, WS_IN, src, (size_t)(rows * cols) * 4, &dx));
    TKV_RC_TRY(ctx_workspace(c, WS_OUT, (size_t)(rows * cols) * 4, &dq));
    TKV_RC_TRY(ctx_workspace(c, WS_SMALL, (size_t)rows * 4, &ds));
    TKV_RC_TRY(launch_quant_rows(c, static_cast<float*>(dx), rows, cols, RM_DYNAMIC, nullptr, dq,
                                 true, static_cast<float*>(ds), nullptr, 1));
    TKV_HIP_TRY(hipMemcpyAsync(scales_out, ds, (size_t)rows * 4, hipMemcpyDeviceToHost, c->stream));
    return download(c, dst, dq, (size_t)(rows * cols) * 4);
}

int32_t tkv_hip_quantize_fp8_e4m3(const float* src, int64_t n_src, int32_t* dst, int64_t n_dst) {
    if (n_src < 0 || n_dst < n_src) return set_error(TKV_HIP_BAD_ARG, "dst too small");
    if (n_src == 0) return TKV_HIP_OK;
    void *dx, *dq;
    Ctx* c;
    TKV_RC_TRY(begin_host(&c));
    TKV_RC_TRY(upload(c, WS_IN, src, (size_t)n_src * 4, &dx));
    TKV_RC_TRY(ctx_workspace(c, WS_OUT, (size_t)n_src * 4, &dq));
    TKV_RC_TRY(launch_fp8_encode(c, static_cast<float*>(dx), n_src, nullptr, dq, true));
    return download(c, dst, dq, (size_t)n_src * 4);
}

int32_t tkv_hip_dequantize_fp8_e4m3(const int32_t* src, int64_t n_src, float* dst,
                                    int64_t n_dst) {
    if (n_src < 0 || n_dst < n_src) return set_error(TKV_HIP_BAD_ARG, "dst too small");
    if (n_src == 0) return TKV_HIP_OK;
    void *dq, *dy;
    Ctx* c;
    TKV_RC_TRY(begin_host(&c));
    TKV_RC_TRY(upload(c, WS_IN, src, (size_t)n_src * 4, &dq));
    TKV_RC_TRY(ctx_workspace(c, WS_OUT, (size_t)n_src * 4, &dy));
    TKV_RC_TRY(launch_fp8_decode(c, dq, true, n_src, static_cast<float*>(dy)));
    return download(c, dst, dy, (size_t)n_src * 4);
}

int32_t tkv_hip_matmul_int8_symmetric(const int32_t* pa, const int32_t* pw, const float* pbias,
                                      int64_t n_bias, float* py, int64_t m, int64_t n, int64_t k,
                                      float scale_a, float scale_w) {
    return host_gemm_i8(pa, pw, pbias, n_bias, py, false, m, n, k, scale_a, scale_w, nullptr, 0,
                        TKV_HIP_RECIPE_PRIMARY);
}

int32_t tkv_hip_matmul_int8_per_channel(const int32_t* pa, const int32_t* pw, const float* pbias,
                                        int64_t n_bias, float* py, int64_t m, int64_t n,
                                        int64_t k, float scale_a, const float* scales_w,
                                        int64_t n_scales) {
    if (n_scales < n || !scales_w) return set_error(TKV_HIP_BAD_ARG, "scales_w smaller than N");
    return host_gemm_i8(pa, pw, pbias, n_bias, py, false, m, n, k, scale_a, 0.0f, scales_w,
                        n_scales, TKV_HIP_RECIPE_PRIMARY);
}

int32_t tkv_hip_matmul_int8_recipe(const int32_t* pa, const int32_t* pw, const float* pbias,
                                   int64_t n_bias, float* py, int64_t m, int64_t n, int64_t k,
                                   float scale_a, float scale_w, const float* scales_w,
                                   int64_t n_scales, int32_t recipe) {
    // n_scales == 0 selects the symmetric GEMM (len(scales_w) == 0)
    if (scales_w && n_scales > 0 && n_scales < n)
        return set_error(TKV_HIP_BAD_ARG, "scales_w smaller than N");
    return host_gemm_i8(pa, pw, pbias, n_bias, py, false, m, n, k, scale_a, scale_w,
                        n_scales > 0 ? scales_w : nullptr, n_scales, recipe);
}

int32_t tkv_hip_matmul_int8_accum(const int32_t* pa, const int32_t* pw, int32_t* acc, int64_t m,
                                  int64_t n, int64_t k) {
    return host_gemm_i8(pa, pw, nullptr, 0, acc, true, m, n, k, 0.0f, 0.0f, nullptr, 0,
                        TKV_HIP_RECIPE_PRIMARY);
}

int32_t tkv_hip_matmul_fp8_e4m3(const int32_t* pa, const int32_t* pw, const float* pbias,
                                int64_t n_bias, float* py, int64_t m, int64_t n, int64_t k) {
    if (m < 0 || n < 0 || k < 0) return set_error(TKV_HIP_BAD_ARG, "negative GEMM size");
    if (m == 0 || n == 0) return TKV_HIP_OK;
    if (n_bias > 0 && n_bias < n) return set_error(TKV_HIP_BAD_ARG, "bias shorter than N");
    int64_t kk = k > 0 ? k : 1;
    const int64_t ka = gemm_k_align();
    int64_t ldk = (kk + ka - 1) / ka * ka;
    std::vector<int8_t> ha, hw;
    if (k > 0) {
        // codes are e4m3 byte - 128: raw byte = code + 128 (0x00 is +0.0)
        TKV_RC_TRY(pack_codes(pa, m, k, ldk, 128, -128, 127, ha));
        TKV_RC_TRY(pack_codes(pw, n, k, ldk, 128, -128, 127, hw));
    } else {
        ha.assign((size_t)(m * ldk), 0);
        hw.assign((size_t)(n * ldk), 0);
    }
    void *da, *dw, *db = nullptr, *dy;
    Ctx* c;
    TKV_RC_TRY(begin_host(&c));
    TKV_RC_TRY(upload(c, WS_A, ha.data(), ha.size(), &da));
    TKV_RC_TRY(upload(c, WS_W, hw.data(), hw.size(), &dw));
    if (n_bias > 0) TKV_RC_TRY(upload(c, WS_SMALL, pbias, (size_t)n * 4, &db));
    size_t ybytes = (size_t)(m * n) * 4;
    TKV_RC_TRY(ctx_workspace(c, WS_Y, ybytes, &dy));
    TKV_RC_TRY(launch_gemm_f8(c, static_cast<uint8_t*>(da), static_cast<uint8_t*>(dw), m, n, ldk,
                              nullptr, 0, nullptr, static_cast<float*>(db),
                              static_cast<float*>(dy), false));
    return download(c, py, dy, ybytes);
}

int32_t tkv_hip_quantized_gemm(const int32_t* aq, const int32_t* wq, const float* bias,
                               int64_t n_bias, float* y, int64_t m, int64_t n, int64_t k,
                               float scale_a, float scale_b, const float* scales_w,
                               int64_t n_scales) {
    // session.tkv:693-696: per-channel iff len(scales_w) > 0
    if (n_scales > 0)
        return tkv_hip_matmul_int8_per_channel(aq, wq, bias, n_bias, y, m, n, k, scale_a,
                                               scales_w, n_scales);
    return tkv_hip_matmul_int8_symmetric(aq, wq, bias, n_bias, y, m, n, k, scale_a, scale_b);
}

int32_t tkv_hip_matmul_integer(const int32_t* a, int64_t na, const int32_t* b, int64_t nb,
                               int64_t* y, int64_t ny, int64_t m, int64_t n, int64_t k) {
    if (m < 0 || n < 0 || k < 0 || na < 0 || nb < 0 || ny < 0)
        return set_error(TKV_HIP_BAD_ARG, "negative size");
    if (m == 0 || n == 0) return TKV_HIP_OK;
    // Out-of-range reads are zero in the reference (session.tkv:2822-2836):
    // build A [m,k] and B^T [n,k] with those zeros, then one INT32 GEMM.
    int64_t kk = k > 0 ? k : 1;
    std::vector<int32_t> A((size_t)(m * kk), 0), Bt((size_t)(n * kk), 0);
    for (int64_t i = 0; i < m; i++)
        for (int64_t p = 0; p < k; p++) {
            int64_t ai = i * k + p;
            if (ai < na) A[(size_t)(i * kk + p)] = a[ai];
        }
    for (int64_t p = 0; p < k; p++)
        for (int64_t j = 0; j < n; j++) {
            int64_t bi = p * n + j;
            if (bi < nb) Bt[(size_t)(j * kk + p)] = b[bi];
        }
    std::vector<int32_t> acc((size_t)(m * n));
    TKV_RC_TRY(host_gemm_i8(A.data(), Bt.data(), nullptr, 0, acc.data(), true, m, n, kk, 0.0f,
                            0.0f, nullptr, 0, TKV_HIP_RECIPE_PRIMARY));
    int64_t lim = m * n < ny ? m * n : ny;
    for (int64_t i = 0; i < lim; i++) y[i] = acc[(size_t)i];
    return TKV_HIP_OK;
}

int32_t tkv_hip_qlinear_matmul(const int32_t* a, int64_t na, float sa, int64_t zpa,
                               const int32_t* b, int64_t nb, float sw, int64_t zpw, float sy,
                               int64_t zpy, int32_t* y, int64_t ny, int64_t m, int64_t n,
                               int64_t k, int32_t recipe) {
    if (m < 0 || n < 0 || k < 0 || na < 0 || nb < 0 || ny < 0)
        return set_error(TKV_HIP_BAD_ARG, "negative size");
    TKV_RC_TRY(check_recipe(recipe));
    if (m == 0 || n == 0 || ny == 0) return TKV_HIP_OK;
    auto fits8 = [](int64_t v) { return v >= -128 && v <= 127; };
    auto fits32 = [](int64_t v) { return v >= INT32_MIN && v <= INT32_MAX; };
    if (!fits32(zpa) || !fits32(zpw) || !fits32(zpy))
        return set_error(TKV_HIP_UNSUPPORTED, "QLinearMatMul: zero point beyond int32");
    // A value read past the end contributes 0 to the node's sum, which a code
    // equal to the zero point reproduces (k == 0: one such term, acc = 0).
    const bool pad_a = m * k > na || k == 0, pad_b = k * n > nb || k == 0;
    if ((pad_a && !fits8(zpa)) || (pad_b && !fits8(zpw)))
        return set_error(TKV_HIP_UNSUPPORTED, "QLinearMatMul: padding needs an int8 zero point");
    const int64_t kk = k > 0 ? k : 1;  // k == 0: one zero term (a = zpa) gives acc = 0
    std::vector<int8_t> A((size_t)(m * kk), (int8_t)(pad_a ? zpa : 0)),
        Wt((size_t)(n * kk), (int8_t)(pad_b ? zpw : 0));
    for (int64_t i = 0; i < m; i++)
        for (int64_t p = 0; p < k; p++) {
            const int64_t ai = i * k + p;
            if (ai < na) {
                if (!fits8(a[ai])) return set_error(TKV_HIP_BAD_ARG, "A code outside int8");
                A[(size_t)(i * kk + p)] = (int8_t)a[ai];
            }
        }
    for (int64_t p = 0; p < k; p++)
        for (int64_t j = 0; j < n; j++) {
            const int64_t bi = p * n + j;
            if (bi < nb) {
                if (!fits8(b[bi])) return set_error(TKV_HIP_BAD_ARG, "B code outside int8");
                Wt[(size_t)(j * kk + p)] = (int8_t)b[bi];
            }
        }
    Ctx* c;
    TKV_RC_TRY(begin_host(&c));
    void *da, *dw, *dy;
    TKV_RC_TRY(upload(c, WS_A, A.data(), A.size(), &da));
    TKV_RC_TRY(upload(c, WS_W, Wt.data(), Wt.size(), &dw));
    TKV_RC_TRY(ctx_workspace(c, WS_Y, (size_t)(m * n), &dy));
    QLinearParams q;
    q.zpa = (int32_t)zpa;
    q.zpw = (int32_t)zpw;
    q.zpy = (int32_t)zpy;
    q.mult = qlinear_mult(sa, sw, sy, recipe);
    TKV_RC_TRY(launch_gemm_qlinear(c, static_cast<int8_t*>(da), static_cast<int8_t*>(dw), m, n,
                                   kk, q, static_cast<int8_t*>(dy)));
    std::vector<int8_t> out((size_t)(m * n));
    TKV_RC_TRY(download(c, out.data(), dy, out.size()));
    const int64_t lim = m * n < ny ? m * n : ny;
    for (int64_t i = 0; i < lim; i++) y[i] = out[(size_t)i];
    return TKV_HIP_OK;
}

int32_t tkv_hip_quantize_linear(const float* x, int64_t nx, const float* scales, int64_t n_scales,
                                int64_t zero_point, int64_t outer, int64_t dim, int64_t inner,
                                int32_t* y) {
    if (nx < 0 || n_scales < 1) return set_error(TKV_HIP_BAD_ARG, "empty scale");
    if (n_scales != 1 && (outer < 0 || dim < 1 || inner < 1 || n_scales < dim ||
                          outer * dim * inner > nx))
        return set_error(TKV_HIP_BAD_ARG, "per-axis view does not fit the input");
    int64_t n = n_scales == 1 ? nx : outer * dim * inner;
    if (n == 0) return TKV_HIP_OK;
    void *dx, *ds, *dy;
    Ctx* c;
    TKV_RC_TRY(begin_host(&c));
    TKV_RC_TRY(upload(c, WS_IN, x, (size_t)n * 4, &dx));
    TKV_RC_TRY(upload(c, WS_SMALL, scales, (size_t)n_scales * 4, &ds));
    TKV_RC_TRY(ctx_workspace(c, WS_OUT, (size_t)n * 4, &dy));
    TKV_RC_TRY(launch_quantize_linear(c, static_cast<float*>(dx), n, static_cast<float*>(ds),
                                      n_scales, zero_point, dim, inner, static_cast<int32_t*>(dy)));
    return download(c, y, dy, (size_t)n * 4);
}

int32_t tkv_hip_dequantize_linear(const int32_t* x, int64_t nx, const float* scales,
                                  int64_t n_scales, int64_t zero_point, int64_t outer,
                                  int64_t dim, int64_t inner, float* y) {
    if (nx < 0 || n_scales < 1) return set_error(TKV_HIP_BAD_ARG, "empty scale");
    if (n_scales != 1 && (outer < 0 || dim < 1 || inner < 1 || n_scales < dim ||
                          outer * dim * inner > nx))
        return set_error(TKV_HIP_BAD_ARG, "per-axis view does not fit the input");
    int64_t n = n_scales == 1 ? nx : outer * dim * inner;
    if (n == 0) return TKV_HIP_OK;
    void *dx, *ds, *dy;
    Ctx* c;
    TKV_RC_TRY(begin_host(&c));
    TKV_RC_TRY(upload(c, WS_IN, x, (size_t)n * 4, &dx));
    TKV_RC_TRY(upload(c, WS_SMALL, scales, (size_t)n_scales * 4, &ds));
    TKV_RC_TRY(ctx_workspace(c, WS_OUT, (size_t)n * 4, &dy));
    TKV_RC_TRY(launch_dequantize_linear(c, static_cast<int32_t*>(dx), n, static_cast<float*>(ds),
                                        n_scales, zero_point, dim, inner, static_cast<float*>(dy)));
    return download(c, y, dy, (size_t)n * 4);
}

int32_t tkv_hip_dynamic_quantize_linear(const float* x, int64_t nx, int32_t* y, float* y_scale,
                                        float* y_zero_point) {
    if (nx <= 0) return set_error(TKV_HIP_BAD_ARG, "DynamicQuantizeLinear needs a non-empty input");
    void *dx, *dy;
    Ctx* c;
    TKV_RC_TRY(begin_host(&c));
    TKV_RC_TRY(upload(c, WS_IN, x, (size_t)nx * 4, &dx));
    TKV_RC_TRY(ctx_workspace(c, WS_OUT, (size_t)nx * 4, &dy));
    TKV_RC_TRY(launch_minmax_tensor(c, static_cast<float*>(dx), nx, MM_DYNAMIC_QL,
                                    TKV_HIP_RECIPE_PRIMARY, c->params));
    TKV_RC_TRY(launch_dynamic_ql(c, static_cast<float*>(dx), nx, c->params,
                                 static_cast<int32_t*>(dy)));
    tkv_hip_qparams_dev p;
    TKV_HIP_TRY(hipMemcpyAsync(&p, c->params, sizeof(p), hipMemcpyDeviceToHost, c->stream));
    TKV_RC_TRY(download(c, y, dy, (size_t)nx * 4));
    if (y_scale) *y_scale = p.scale;
    if (y_zero_point) *y_zero_point = (float)p.zero_point;
    return TKV_HIP_OK;
}

// ===========================================================================
// Device-pointer variants
// ===========================================================================

int32_t tkv_hip_dev_calibrate_minmax(int64_t ctx, const float* x, int64_t n, int32_t symmetric,
                                     tkv_hip_qparams_dev* params) {
    if (n <= 0 || !x || !params) return set_error(TKV_HIP_BAD_ARG, "empty input or NULL params");
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    return launch_minmax_tensor(c, x, n, symmetric ? MM_SYMMETRIC : MM_ASYMMETRIC,
                                TKV_HIP_RECIPE_PRIMARY, params);
}

int32_t tkv_hip_dev_calibrate_rows(int64_t ctx, const float* x, int64_t rows, int64_t cols,
                                   float* scales) {
    if (rows <= 0 || cols <= 0) return set_error(TKV_HIP_BAD_ARG, "rows/cols must be > 0");
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    return launch_quant_rows(c, x, rows, cols, RM_CALIBRATE, nullptr, nullptr, false, scales,
                             nullptr, 1);
}

int32_t tkv_hip_dev_quantize_int8_tensor(int64_t ctx, const float* x, int64_t n,
                                         const tkv_hip_qparams_dev* params, int8_t* q) {
    if (n < 0) return set_error(TKV_HIP_BAD_ARG, "negative length");
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    return launch_quant_i8_tensor(c, x, n, params, q, false);
}

int32_t tkv_hip_dev_calibrate_kl(int64_t ctx, const float* x, int64_t n, int64_t num_bins,
                                 int64_t target_bins, tkv_hip_qparams_dev* params) {
    if (!params) return set_error(TKV_HIP_BAD_ARG, "NULL params");
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    return launch_calibrate_kl(c, x, n, num_bins, target_bins, params);
}

int32_t tkv_hip_dev_calibrate_percentile(int64_t ctx, const float* x, int64_t n,
                                         float percentile, int32_t symmetric,
                                         tkv_hip_qparams_dev* params) {
    if (!params) return set_error(TKV_HIP_BAD_ARG, "NULL params");
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    return launch_calibrate_percentile(c, x, n, percentile, symmetric, params);
}

int32_t tkv_hip_dev_calibrate_mse(int64_t ctx, const float* x, int64_t n,
                                  int64_t num_candidates, tkv_hip_qparams_dev* params) {
    if (!params) return set_error(TKV_HIP_BAD_ARG, "NULL params");
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    return launch_calibrate_mse(c, x, n, num_candidates, params);
}

int32_t tkv_hip_dev_quantize_int8_dynamic_tensor(int64_t ctx, const float* x, int64_t n,
                                                 int8_t* q, tkv_hip_qparams_dev* params) {
    if (n <= 0 || !params) return set_error(TKV_HIP_BAD_ARG, "empty input or NULL params");
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    return launch_quant_i8_dynamic(c, x, n, TKV_HIP_RECIPE_PRIMARY, params, q, false);
}

int32_t tkv_hip_dev_quantize_int8_per_channel(int64_t ctx, const float* x, int64_t rows,
                                              int64_t cols, const float* scales, int8_t* q) {
    if (rows < 0 || cols < 0) return set_error(TKV_HIP_BAD_ARG, "negative rows/cols");
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    return launch_quant_rows(c, x, rows, cols, RM_PER_CHANNEL, scales, q, false, nullptr, nullptr,
                             1);
}

int32_t tkv_hip_dev_quantize_dynamic_int8_rowwise(int64_t ctx, const float* x, int64_t rows,
                                                  int64_t cols, int8_t* q, float* scales_out) {
    if (rows < 0 || cols <= 0) return set_error(TKV_HIP_BAD_ARG, "bad rows/cols");
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    return launch_quant_rows(c, x, rows, cols, RM_DYNAMIC, nullptr, q, false, scales_out, nullptr,
                             1);
}

int32_t tkv_hip_dev_dequantize_int8(int64_t ctx, const int8_t* q, int64_t rows, int64_t cols,
                                    float scale, const float* scales, float* y) {
    if (rows < 0 || cols < 0) return set_error(TKV_HIP_BAD_ARG, "negative rows/cols");
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    return launch_dequant_i8(c, q, false, rows, cols, scale, scales, y);
}

int32_t tkv_hip_dev_quantize_fp8_e4m3(int64_t ctx, const float* x, int64_t n, uint8_t* q) {
    if (n < 0) return set_error(TKV_HIP_BAD_ARG, "negative length");
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    return launch_fp8_encode(c, x, n, nullptr, q, false);
}

int32_t tkv_hip_dev_quantize_fp8_e4m3_scaled(int64_t ctx, const float* x, int64_t n,
                                             const tkv_hip_qparams_dev* params, uint8_t* q) {
    if (n < 0 || !params) return set_error(TKV_HIP_BAD_ARG, "negative length or NULL params");
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    return launch_fp8_encode(c, x, n, params, q, false);
}

int32_t tkv_hip_dev_quantize_fp8_e4m3_dynamic_tensor(int64_t ctx, const float* x, int64_t n,
                                                     uint8_t* q, tkv_hip_qparams_dev* params) {
    if (n <= 0 || !params) return set_error(TKV_HIP_BAD_ARG, "empty input or NULL params");
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    return launch_quant_fp8_dynamic(c, x, n, params, q, false);
}

int32_t tkv_hip_dev_dequantize_fp8_e4m3(int64_t ctx, const uint8_t* q, int64_t n, float* y) {
    if (n < 0) return set_error(TKV_HIP_BAD_ARG, "negative length");
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    return launch_fp8_decode(c, q, false, n, y);
}

int32_t tkv_hip_dev_matmul_int8(int64_t ctx, const int8_t* a, const int8_t* w, int64_t m,
                                int64_t n, int64_t k, const float* scale_a, int64_t scale_a_stride,
                                float scale_w, const float* scales_w, const float* bias, float* y,
                                int32_t recipe) {
    TKV_RC_TRY(check_recipe(recipe));
    if (m < 0 || n < 0 || k < 0 || !scale_a || scale_a_stride < 0)
        return set_error(TKV_HIP_BAD_ARG, "bad GEMM arguments");
    I8Epilogue ep;
    ep.mode = scales_w ? EPI_PER_CHANNEL : EPI_SYMMETRIC;
    ep.recipe = recipe;
    ep.scale_a = scale_a;
    ep.scale_a_stride = scale_a_stride;
    ep.scale_w = scale_w;
    ep.scales_w = scales_w;
    ep.bias = bias;
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    return launch_gemm_i8(c, a, w, m, n, k, ep, y);
}

int32_t tkv_hip_dev_qlinear_matmul(int64_t ctx, const int8_t* a, float sa, int32_t zpa,
                                   const int8_t* w, float sw, int32_t zpw, float sy, int32_t zpy,
                                   int8_t* y, int64_t m, int64_t n, int64_t k, int32_t recipe) {
    TKV_RC_TRY(check_recipe(recipe));
    if (m < 0 || n < 0 || k <= 0) return set_error(TKV_HIP_BAD_ARG, "bad QLinearMatMul sizes");
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    QLinearParams q;
    q.zpa = zpa;
    q.zpw = zpw;
    q.zpy = zpy;
    q.mult = qlinear_mult(sa, sw, sy, recipe);
    return launch_gemm_qlinear(c, a, w, m, n, k, q, y);
}

int32_t tkv_hip_dev_matmul_int8_accum(int64_t ctx, const int8_t* a, const int8_t* w, int64_t m,
                                      int64_t n, int64_t k, int32_t* acc) {
    if (m < 0 || n < 0 || k < 0) return set_error(TKV_HIP_BAD_ARG, "negative GEMM size");
    I8Epilogue ep;
    memset(&ep, 0, sizeof(ep));
    ep.mode = EPI_ACCUM_I32;
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    return launch_gemm_i8(c, a, w, m, n, k, ep, acc);
}

int32_t tkv_hip_dev_matmul_fp8_e4m3(int64_t ctx, const uint8_t* a, const uint8_t* w, int64_t m,
                                    int64_t n, int64_t k, const float* scale_a,
                                    int64_t scale_a_stride, const float* scales_w,
                                    const float* bias, float* y) {
    if (m < 0 || n < 0 || k < 0 || scale_a_stride < 0)
        return set_error(TKV_HIP_BAD_ARG, "bad GEMM arguments");
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    return launch_gemm_f8(c, a, w, m, n, k, scale_a, scale_a_stride, scales_w, bias, y, false);
}

int32_t tkv_hip_dev_matmul_fp8_e4m3_fast(int64_t ctx, const uint8_t* a, const uint8_t* w,
                                         int64_t m, int64_t n, int64_t k, const float* scale_a,
                                         int64_t scale_a_stride, const float* scales_w,
                                         const float* bias, float* y) {
    if (m < 0 || n < 0 || k < 0 || scale_a_stride < 0)
        return set_error(TKV_HIP_BAD_ARG, "bad GEMM arguments");
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    return launch_gemm_f8(c, a, w, m, n, k, scale_a, scale_a_stride, scales_w, bias, y, true);
}

int32_t tkv_hip_dev_matmul_q8_0(int64_t ctx, const int8_t* a, const int8_t* codes,
                                const float* group_scales, int64_t m, int64_t n, int64_t k,
                                const float* scale_a, int64_t scale_a_stride, const float* bias,
                                float* y) {
    if (m < 0 || n < 0 || k < 0 || (scale_a_stride != 0 && scale_a_stride != 1) || !scale_a)
        return set_error(TKV_HIP_BAD_ARG, "matmul_q8_0: bad arguments");
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    if (m == 0 || n == 0) return TKV_HIP_OK;
    if (!a || !codes || !group_scales || !y)
        return set_error(TKV_HIP_BAD_ARG, "matmul_q8_0: NULL operand");
    const int rc = launch_gemm_q8(c, a, codes, group_scales, m, n, k, scale_a, scale_a_stride,
                                  bias, y);
    return rc == TKV_HIP_UNSUPPORTED
               ? set_error(rc, "matmul_q8_0: K must be a positive multiple of 128, operands 16-byte aligned")
               : rc;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// grouped INT4 (int4.tkv) and GGUF blocks (gguf.tkv:284-313)
// ---------------------------------------------------------------------------

// Shape checks of the quantizers (int4.tkv:37-44); ZeroDivision for a group
// size of 0 reads as the same ValueError.
static int int4_quant_args(int64_t n_src, int64_t rows, int64_t cols, int64_t gs,
                           int64_t n_packed, int64_t n_groups_out) {
    if (rows < 0 || cols < 0 || gs <= 0) return set_error(TKV_HIP_BAD_ARG, "bad rows/cols/group_size");
    if (cols % gs != 0) return set_error(TKV_HIP_BAD_ARG, "cols must be a multiple of group_size");
    if (cols % 2 != 0) return set_error(TKV_HIP_BAD_ARG, "cols must be even for nibble packing");
    if (n_src < rows * cols) return set_error(TKV_HIP_BAD_ARG, "src smaller than rows*cols");
    if (n_packed < rows * (cols / 2)) return set_error(TKV_HIP_BAD_ARG, "packed_out too small");
    if (n_groups_out < rows * (cols / gs))
        return set_error(TKV_HIP_BAD_ARG, "scales_out smaller than rows*num_groups");
    return TKV_HIP_OK;
}

static int host_int4_quantize(const float* src, int64_t n_src, int64_t rows, int64_t cols,
                              int64_t gs, int32_t* packed_out, int64_t n_packed, float* scales_out,
                              int64_t* zps_out, int64_t n_groups_out) {
    TKV_RC_TRY(int4_quant_args(n_src, rows, cols, gs, n_packed, n_groups_out));
    Ctx* c;
    TKV_RC_TRY(begin_host(&c));
    memset(packed_out, 0, (size_t)n_packed * 4);  // the reference clears the whole list
    const int64_t bytes = rows * (cols / 2), groups = rows * (cols / gs);
    if (bytes == 0) return TKV_HIP_OK;
    void *dx, *dp, *ds, *dz = nullptr;
    TKV_RC_TRY(upload(c, WS_IN, src, (size_t)(rows * cols) * 4, &dx));
    TKV_RC_TRY(ctx_workspace(c, WS_OUT, (size_t)bytes * 4, &dp));
    TKV_RC_TRY(ctx_workspace(c, WS_SMALL, (size_t)groups * 4, &ds));
    if (zps_out) TKV_RC_TRY(ctx_workspace(c, WS_Y, (size_t)groups * 8, &dz));
    TKV_RC_TRY(launch_int4_quantize(c, static_cast<const float*>(dx), rows, cols, gs, zps_out != nullptr,
                                    dp, true, static_cast<float*>(ds), static_cast<int64_t*>(dz)));
    TKV_HIP_TRY(hipMemcpyAsync(packed_out, dp, (size_t)bytes * 4, hipMemcpyDeviceToHost, c->stream));
    if (zps_out)
        TKV_HIP_TRY(hipMemcpyAsync(zps_out, dz, (size_t)groups * 8, hipMemcpyDeviceToHost, c->stream));
    return download(c, scales_out, ds, (size_t)groups * 4);
}

// Dequantize: the pair at column c reads group r * ng + c / gs (flat, as the
// reference indexes); that index and the byte index must lie in the lists.
static int host_int4_dequantize(const int32_t* packed, int64_t n_packed, float* dst,
                                int64_t n_dst, int64_t rows, int64_t cols, int64_t gs,
                                const float* scales, const int64_t* zps, int64_t n_groups) {
    if (rows < 0 || cols < 0 || gs <= 0) return set_error(TKV_HIP_BAD_ARG, "bad rows/cols/group_size");
    if (cols % 2 != 0)
        return set_error(TKV_HIP_UNSUPPORTED, "odd cols: the reference's pairs overlap rows");
    const int64_t ng = cols / gs, half = cols / 2;
    if (n_dst < rows * cols) return set_error(TKV_HIP_BAD_ARG, "dst too small");
    if (n_groups < rows * ng) return set_error(TKV_HIP_BAD_ARG, "scales smaller than rows*num_groups");
    if (rows * half == 0) return TKV_HIP_OK;
    if ((rows - 1) * ng + (cols - 2) / gs >= n_groups || n_packed < rows * half)
        return set_error(TKV_HIP_BAD_ARG, "packed / scales index out of range");
    Ctx* c;
    TKV_RC_TRY(begin_host(&c));
    const int64_t groups = (rows - 1) * ng + (cols - 2) / gs + 1;
    void *dp, *ds, *dz = nullptr, *dy;
    TKV_RC_TRY(upload(c, WS_IN, packed, (size_t)(rows * half) * 4, &dp));
    TKV_RC_TRY(upload(c, WS_SMALL, scales, (size_t)groups * 4, &ds));
    if (zps) TKV_RC_TRY(upload(c, WS_A, zps, (size_t)groups * 8, &dz));
    TKV_RC_TRY(ctx_workspace(c, WS_OUT, (size_t)(rows * cols) * 4, &dy));
    TKV_RC_TRY(launch_int4_dequantize(c, dp, true, rows, cols, gs, static_cast<float*>(ds),
                                      static_cast<int64_t*>(dz), static_cast<float*>(dy)));
    return download(c, dst, dy, (size_t)(rows * cols) * 4);
}

static int host_permute(const float* src, int64_t n_src, int64_t rows, int64_t cols,
                        const int64_t* perm, int64_t n_perm, float* out, int64_t n_out,
                        bool inverse) {
    if (rows < 0 || cols < 0) return set_error(TKV_HIP_BAD_ARG, "negative rows/cols");
    if (n_perm != cols) return set_error(TKV_HIP_BAD_ARG, "perm length must equal cols");
    if (n_src < rows * cols || n_out < rows * cols) return set_error(TKV_HIP_BAD_ARG, "span too small");
    std::vector<char> seen((size_t)cols, 0);
    for (int64_t i = 0; i < cols; i++) {
        if (perm[i] < 0 || perm[i] >= cols) return set_error(TKV_HIP_BAD_ARG, "perm entry out of range");
        if (inverse && seen[(size_t)perm[i]]++)
            return set_error(TKV_HIP_UNSUPPORTED, "inverse of a non-permutation (ordered overwrites)");
    }
    if (rows * cols == 0) return TKV_HIP_OK;
    Ctx* c;
    TKV_RC_TRY(begin_host(&c));
    void *dx, *dp, *dy;
    TKV_RC_TRY(upload(c, WS_IN, src, (size_t)(rows * cols) * 4, &dx));
    TKV_RC_TRY(upload(c, WS_SMALL, perm, (size_t)cols * 8, &dp));
    TKV_RC_TRY(ctx_workspace(c, WS_OUT, (size_t)(rows * cols) * 4, &dy));
    TKV_RC_TRY(launch_permute_cols(c, static_cast<float*>(dx), rows, cols,
                                   static_cast<int64_t*>(dp), inverse, static_cast<float*>(dy)));
    return download(c, out, dy, (size_t)(rows * cols) * 4);
}

// matmul_int4_grouped(_ordered): the HIP path takes even K with whole groups
// (the reference's own quantizer produces nothing else) and perm entries in
// [0, K); anything else is UNSUPPORTED so the caller keeps its loop.
static int host_matmul_int4(const float* pa, int64_t n_a, const int32_t* packed_w,
                            int64_t n_packed, const float* pbias, int64_t n_bias, float* py,
                            int64_t n_y, int64_t m, int64_t n, int64_t k, int64_t gs,
                            const float* scales_w, int64_t n_scales, const int64_t* perm,
                            int64_t n_perm) {
    if (m < 0 || n < 0 || k < 0 || gs <= 0) return set_error(TKV_HIP_BAD_ARG, "bad GEMM arguments");
    const int64_t ng = k / gs, half = k / 2;
    if (!perm && n_scales < n * ng) return set_error(TKV_HIP_BAD_ARG, "scales_w smaller than N*num_groups");
    if (n_bias > 0 && n_bias < n) return set_error(TKV_HIP_BAD_ARG, "bias shorter than N");
    if (n_y < m * n || n_a < m * k || n_packed < n * half || n_scales < n * ng)
        return set_error(TKV_HIP_BAD_ARG, "span too small");
    if (k % 2 != 0 || k % gs != 0)
        return set_error(TKV_HIP_UNSUPPORTED, "matmul_int4: K must be even and a multiple of group_size");
    if (perm) {
        if (n_perm < k) return set_error(TKV_HIP_BAD_ARG, "perm shorter than K");
        for (int64_t i = 0; i < k; i++)
            if (perm[i] < 0 || perm[i] >= k)
                return set_error(TKV_HIP_UNSUPPORTED, "perm entry outside [0, K)");
    }
    Ctx* c;
    TKV_RC_TRY(begin_host(&c));
    if (m == 0 || n == 0) return TKV_HIP_OK;
    std::vector<uint8_t> wb((size_t)(n * half));
    for (size_t i = 0; i < wb.size(); i++) wb[i] = (uint8_t)packed_w[i];  // nibbles are bits 0-7
    void *da, *dw, *ds, *db = nullptr, *dp = nullptr, *dy;
    TKV_RC_TRY(upload(c, WS_A, pa, (size_t)(m * k) * 4, &da));
    TKV_RC_TRY(upload(c, WS_W, wb.data(), wb.size(), &dw));
    TKV_RC_TRY(upload(c, WS_SMALL, scales_w, (size_t)(n * ng) * 4, &ds));
    if (n_bias > 0) TKV_RC_TRY(upload(c, WS_IN, pbias, (size_t)n * 4, &db));
    if (perm) TKV_RC_TRY(upload(c, WS_OUT, perm, (size_t)k * 8, &dp));
    TKV_RC_TRY(ctx_workspace(c, WS_Y, (size_t)(m * n) * 4, &dy));
    TKV_RC_TRY(launch_matmul_int4(c, static_cast<float*>(da), static_cast<uint8_t*>(dw),
                                  static_cast<float*>(ds), static_cast<float*>(db),
                                  static_cast<int64_t*>(dp), static_cast<float*>(dy), m, n, k, gs));
    return download(c, py, dy, (size_t)(m * n) * 4);
}

extern "C" {

int32_t tkv_hip_quantize_int4_grouped(const float* src, int64_t n_src, int64_t rows, int64_t cols,
                                      int64_t group_size, int32_t* packed_out, int64_t n_packed,
                                      float* scales_out, int64_t n_scales_out) {
    return host_int4_quantize(src, n_src, rows, cols, group_size, packed_out, n_packed, scales_out,
                              nullptr, n_scales_out);
}

int32_t tkv_hip_dequantize_int4_grouped(const int32_t* packed, int64_t n_packed, float* dst,
                                        int64_t n_dst, int64_t rows, int64_t cols,
                                        int64_t group_size, const float* scales,
                                        int64_t n_scales) {
    return host_int4_dequantize(packed, n_packed, dst, n_dst, rows, cols, group_size, scales,
                                nullptr, n_scales);
}

int32_t tkv_hip_quantize_int4_grouped_asym(const float* src, int64_t n_src, int64_t rows,
                                           int64_t cols, int64_t group_size, int32_t* packed_out,
                                           int64_t n_packed, float* scales_out, int64_t* zps_out,
                                           int64_t n_groups_out) {
    if (!zps_out) return set_error(TKV_HIP_BAD_ARG, "zps_out is NULL");
    return host_int4_quantize(src, n_src, rows, cols, group_size, packed_out, n_packed, scales_out,
                              zps_out, n_groups_out);
}

int32_t tkv_hip_dequantize_int4_grouped_asym(const int32_t* packed, int64_t n_packed, float* dst,
                                             int64_t n_dst, int64_t rows, int64_t cols,
                                             int64_t group_size, const float* scales,
                                             const int64_t* zps, int64_t n_groups) {
    if (!zps) return set_error(TKV_HIP_BAD_ARG, "zps is NULL");
    return host_int4_dequantize(packed, n_packed, dst, n_dst, rows, cols, group_size, scales, zps,
                                n_groups);
}

int32_t tkv_hip_permute_cols(const float* src, int64_t n_src, int64_t rows, int64_t cols,
                             const int64_t* perm, int64_t n_perm, float* out, int64_t n_out) {
    return host_permute(src, n_src, rows, cols, perm, n_perm, out, n_out, false);
}

int32_t tkv_hip_inv_permute_cols(const float* src, int64_t n_src, int64_t rows, int64_t cols,
                                 const int64_t* perm, int64_t n_perm, float* out, int64_t n_out) {
    return host_permute(src, n_src, rows, cols, perm, n_perm, out, n_out, true);
}

int32_t tkv_hip_matmul_int4_grouped(const float* pa, int64_t n_a, const int32_t* packed_w,
                                    int64_t n_packed, const float* pbias, int64_t n_bias,
                                    float* py, int64_t n_y, int64_t m, int64_t n, int64_t k,
                                    int64_t group_size, const float* scales_w, int64_t n_scales) {
    return host_matmul_int4(pa, n_a, packed_w, n_packed, pbias, n_bias, py, n_y, m, n, k,
                            group_size, scales_w, n_scales, nullptr, 0);
}

int32_t tkv_hip_matmul_int4_grouped_ordered(const float* pa, int64_t n_a, const int32_t* packed_w,
                                            int64_t n_packed, const float* pbias, int64_t n_bias,
                                            float* py, int64_t n_y, int64_t m, int64_t n,
                                            int64_t k, int64_t group_size, const float* scales_w,
                                            int64_t n_scales, const int64_t* perm,
                                            int64_t n_perm) {
    if (!perm) return set_error(TKV_HIP_BAD_ARG, "perm is NULL");
    return host_matmul_int4(pa, n_a, packed_w, n_packed, pbias, n_bias, py, n_y, m, n, k,
                            group_size, scales_w, n_scales, perm, n_perm);
}

int32_t tkv_hip_dequantize_gguf(const uint8_t* raw, int64_t n_raw, int64_t n, int32_t dtype,
                                float* out, int64_t n_out) {
    const int64_t step = gguf_block_bytes(dtype);
    if (!step) return set_error(TKV_HIP_UNSUPPORTED, "gguf: only Q8_0, Q4_0 and Q4_1 blocks");
    if (n < 0 || n_out < n) return set_error(TKV_HIP_BAD_ARG, "bad n / out too small");
    if (n_raw < n / 32 * step) return set_error(TKV_HIP_BAD_ARG, "raw shorter than n / 32 blocks");
    if (n == 0) return TKV_HIP_OK;
    Ctx* c;
    TKV_RC_TRY(begin_host(&c));
    void *dr, *dy;
    TKV_RC_TRY(upload(c, WS_IN, raw, (size_t)(n / 32 * step), &dr));
    TKV_RC_TRY(ctx_workspace(c, WS_OUT, (size_t)n * 4, &dy));
    TKV_RC_TRY(launch_gguf_blocks(c, static_cast<uint8_t*>(dr), n, dtype, static_cast<float*>(dy)));
    return download(c, out, dy, (size_t)n * 4);
}

int32_t tkv_hip_dev_quantize_int4_grouped(int64_t ctx, const float* src, int64_t rows,
                                          int64_t cols, int64_t group_size, uint8_t* packed,
                                          float* scales, int64_t* zps) {
    TKV_RC_TRY(int4_quant_args(rows * cols, rows, cols, group_size, rows * (cols / 2),
                               group_size > 0 ? rows * (cols / group_size) : 0));
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    return launch_int4_quantize(c, src, rows, cols, group_size, zps != nullptr, packed, false,
                                scales, zps);
}

int32_t tkv_hip_dev_dequantize_int4_grouped(int64_t ctx, const uint8_t* packed, int64_t rows,
                                            int64_t cols, int64_t group_size, const float* scales,
                                            const int64_t* zps, float* dst) {
    if (rows < 0 || cols < 0 || group_size <= 0) return set_error(TKV_HIP_BAD_ARG, "bad rows/cols/group_size");
    if (cols % 2 != 0) return set_error(TKV_HIP_UNSUPPORTED, "odd cols");
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    return launch_int4_dequantize(c, packed, false, rows, cols, group_size, scales, zps, dst);
}

int32_t tkv_hip_dev_permute_cols(int64_t ctx, const float* src, int64_t rows, int64_t cols,
                                 const int64_t* perm, int32_t inverse, float* out) {
    if (rows < 0 || cols < 0) return set_error(TKV_HIP_BAD_ARG, "negative rows/cols");
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    return launch_permute_cols(c, src, rows, cols, perm, inverse != 0, out);
}

int32_t tkv_hip_dev_matmul_int4_grouped(int64_t ctx, const float* a, const uint8_t* packed_w,
                                        const float* scales_w, const float* bias,
                                        const int64_t* perm, float* y, int64_t m, int64_t n,
                                        int64_t k, int64_t group_size) {
    if (m < 0 || n < 0 || k < 0 || group_size <= 0) return set_error(TKV_HIP_BAD_ARG, "bad GEMM arguments");
    if (k % 2 != 0 || k % group_size != 0)
        return set_error(TKV_HIP_UNSUPPORTED, "matmul_int4: K must be even and a multiple of group_size");
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    return launch_matmul_int4(c, a, packed_w, scales_w, bias, perm, y, m, n, k, group_size);
}

int32_t tkv_hip_dev_dequantize_gguf(int64_t ctx, const uint8_t* raw, int64_t n, int32_t dtype,
                                    float* out) {
    if (!gguf_block_bytes(dtype)) return set_error(TKV_HIP_UNSUPPORTED, "gguf: only Q8_0, Q4_0 and Q4_1 blocks");
    if (n < 0) return set_error(TKV_HIP_BAD_ARG, "negative n");
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    return launch_gguf_blocks(c, raw, n, dtype, out);
}

}  // extern "C"
