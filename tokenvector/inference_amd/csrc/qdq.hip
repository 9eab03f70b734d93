// qdq.hip -- ONNX quantize / dequantize nodes of the reference graph runtime
// on gfx950 (elementwise, HBM-bound):
//   QuantizeLinear         tv/runtime/session.tkv:1896-1953
//   DequantizeLinear       tv/runtime/session.tkv:1955-1990
//   DynamicQuantizeLinear  tv/runtime/session.tkv:2853-2901 (min/max pass is
//                          the per-tensor reduction of quant.hip)
// These nodes divide by the scale in f64 (not a reciprocal multiply) and
// clamp after adding the zero point; integer sums are overflow-free in the
// reference, so the clamp is applied to the mathematical value.
#include "tkv_device.h"
#include "tkv_internal.h"

namespace tkv {

constexpr int kQBlock = 256;

__device__ __forceinline__ int32_t qlinear(float x, double s, int64_t zp, double lo, double hi) {
    double r = __builtin_rint((double)x / s);
    if (r != r) r = 0.0;
    r = r + (double)zp;  // |zp| is small: exact
    r = r < lo ? lo : (r > hi ? hi : r);
    return (int32_t)r;
}

__global__ __launch_bounds__(kQBlock) void k_quantize_linear(const float* __restrict__ x,
                                                             int64_t n,
                                                             const float* __restrict__ scales,
                                                             int per_axis, int64_t dim,
                                                             int64_t inner, int64_t zp,
                                                             int32_t* __restrict__ y) {
    const int64_t stride = (int64_t)gridDim.x * kQBlock;
    for (int64_t i = (int64_t)blockIdx.x * kQBlock + threadIdx.x; i < n; i += stride) {
        float sf = per_axis ? scales[(i / inner) % dim] : scales[0];
        double s = ((double)sf > 0.000000000001) ? (double)sf : 0.000000000001;
        y[i] = qlinear(x[i], s, zp, -128.0, 127.0);
    }
}

__global__ __launch_bounds__(kQBlock) void k_dequantize_linear(const int32_t* __restrict__ x,
                                                               int64_t n,
                                                               const float* __restrict__ scales,
                                                               int per_axis, int64_t dim,
                                                               int64_t inner, int64_t zp,
                                                               float* __restrict__ y) {
    const int64_t stride = (int64_t)gridDim.x * kQBlock;
    for (int64_t i = (int64_t)blockIdx.x * kQBlock + threadIdx.x; i < n; i += stride) {
        float sf = per_axis ? scales[(i / inner) % dim] : scales[0];
        y[i] = (float)((double)((int64_t)x[i] - zp) * (double)sf);
    }
}

__global__ __launch_bounds__(kQBlock) void k_dynamic_ql(const float* __restrict__ x, int64_t n,
                                                        const tkv_hip_qparams_dev* __restrict__ p,
                                                        int32_t* __restrict__ y) {
    const double sc = p->reserved;  // unrounded f64 scale
    const int64_t zp = p->zero_point;
    const int64_t stride = (int64_t)gridDim.x * kQBlock;
    for (int64_t i = (int64_t)blockIdx.x * kQBlock + threadIdx.x; i < n; i += stride)
        y[i] = qlinear(x[i], sc, zp, 0.0, 255.0) - 128;
}

static int64_t qdq_blocks(Ctx* c, int64_t n) {
    int64_t b = ceil_div(n, kQBlock * 4);
    int64_t cap = (int64_t)c->num_cus * 16;
    if (b > cap) b = cap;
    return b < 1 ? 1 : b;
}

int launch_quantize_linear(Ctx* c, const float* x, int64_t nx, const float* scales,
                           int64_t n_scales, int64_t zp, int64_t dim, int64_t inner,
                           int32_t* y) {
    if (nx <= 0) return TKV_HIP_OK;
    hipLaunchKernelGGL(k_quantize_linear, dim3((unsigned)qdq_blocks(c, nx)), dim3(kQBlock), 0,
                       c->stream, x, nx, scales, n_scales == 1 ? 0 : 1, dim, inner, zp, y);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

int launch_dequantize_linear(Ctx* c, const int32_t* x, int64_t nx, const float* scales,
                             int64_t n_scales, int64_t zp, int64_t dim, int64_t inner,
                             float* y) {
    if (nx <= 0) return TKV_HIP_OK;
    hipLaunchKernelGGL(k_dequantize_linear, dim3((unsigned)qdq_blocks(c, nx)), dim3(kQBlock), 0,
                       c->stream, x, nx, scales, n_scales == 1 ? 0 : 1, dim, inner, zp, y);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

int launch_dynamic_ql(Ctx* c, const float* x, int64_t nx, const tkv_hip_qparams_dev* p,
                      int32_t* y) {
    if (nx <= 0) return TKV_HIP_OK;
    hipLaunchKernelGGL(k_dynamic_ql, dim3((unsigned)qdq_blocks(c, nx)), dim3(kQBlock), 0,
                       c->stream, x, nx, p, y);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

}  // namespace tkv
