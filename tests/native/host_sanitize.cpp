// host_sanitize.cpp -- drives libtkv_hip's C ABI from a program whose host
// code (the library's and this driver's) is built with AddressSanitizer and
// UndefinedBehaviorSanitizer (csrc/Makefile: `make sanitize`; device code is
// built as usual).  Without a GPU it exercises the argument checks and the
// no-device error paths; with one it also runs small calls of every entry
// point family (host mirrors, device entry points, weights and linears, the
// static entry, graphs and the context / graph teardown orders), checking
// exact results where they are exact.  Exit status 0 = every check passed.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../include/tkv_hip.h"

static int g_fail = 0;
#define CHECK(cond, what)                                                  \
    do {                                                                   \
        if (!(cond)) {                                                     \
            char buf[256];                                                 \
            tkv_hip_last_error(buf, sizeof(buf));                          \
            fprintf(stderr, "host_sanitize: FAIL %s (last error: %s)\n", what, buf); \
            g_fail = 1;                                                    \
        }                                                                  \
    } while (0)

static uint32_t g_seed = 12345u;
static float frand() {
    g_seed = g_seed * 1103515245u + 12345u;
    return ((g_seed >> 8) & 0xFFFF) / 32768.0f - 1.0f;
}

// Calls that must be refused before any device is touched.
static void no_device_independent_checks() {
    char buf[8];
    CHECK(tkv_hip_last_error(buf, sizeof(buf)) >= 0, "last_error into a short buffer");
    CHECK(tkv_hip_last_error(nullptr, 0) >= 0, "last_error length only");
    CHECK(tkv_hip_version() > 0, "version");
    std::vector<int32_t> a(32, 1), q(8, 0);
    std::vector<float> x(16, 1.0f), y(16, 0.0f), sw(3, 1.0f);
    CHECK(tkv_hip_matmul_int8_per_channel(a.data(), a.data(), nullptr, 0, y.data(), 4, 4, 8, 1.0f,
                                          sw.data(), 3) == TKV_HIP_BAD_ARG,
          "per-channel scales shorter than N");
    CHECK(tkv_hip_quantize_int8_symmetric(x.data(), 16, q.data(), 8, 0.1f) == TKV_HIP_BAD_ARG,
          "quantize into a shorter list");
    CHECK(tkv_hip_weight_free(0) == TKV_HIP_OK, "weight_free(0)");
    CHECK(tkv_hip_graph_destroy(0) == TKV_HIP_OK, "graph_destroy(0)");
    CHECK(tkv_hip_ctx_destroy(0) == TKV_HIP_OK, "ctx_destroy(0)");
    CHECK(tkv_hip_linear_forward_static(0, nullptr, 1, 0, nullptr, nullptr) == TKV_HIP_BAD_ARG,
          "static entry with no weight");
    float one = 1.0f;
    CHECK(tkv_hip_dev_matmul_q8_0(0, nullptr, nullptr, nullptr, 4, 4, 128, &one, 2, nullptr,
                                  nullptr) == TKV_HIP_BAD_ARG,
          "q8_0 GEMM with scale stride 2");
    CHECK(tkv_hip_dev_matmul_q8_0(0, nullptr, nullptr, nullptr, 4, 4, 128, nullptr, 0, nullptr,
                                  nullptr) == TKV_HIP_BAD_ARG,
          "q8_0 GEMM without scale");
}

static void no_device_checks() {
    std::vector<float> x(64);
    for (auto& v : x) v = frand();
    float scale, mn, mx;
    int64_t zp;
    CHECK(tkv_hip_calibrate_minmax(x.data(), 64, 1, &scale, &zp, &mn, &mx) == TKV_HIP_NO_DEVICE,
          "calibrate without a device");
    int64_t h = 0;
    CHECK(tkv_hip_ctx_create(0, &h) == TKV_HIP_NO_DEVICE, "ctx_create without a device");
    CHECK(tkv_hip_ctx_set_tuning(0, 0, 2) == TKV_HIP_NO_DEVICE, "set_tuning without a device");
    std::vector<uint8_t> raw(34, 0);
    CHECK(tkv_hip_weight_create_gguf_q8_0(0, raw.data(), 1, 32, nullptr, &h) == TKV_HIP_NO_DEVICE,
          "q8_0 weight without a device");
}

static void device_checks() {
    int64_t ctx = 0;
    CHECK(tkv_hip_ctx_create(0, &ctx) == TKV_HIP_OK, "ctx_create");
    // host mirrors
    const int m = 37, n = 50, k = 256;  // linear_forward needs K % 128 == 0
    std::vector<float> x(m * k), w(n * k), bias(n), y(m * n);
    for (auto& v : x) v = frand();
    for (auto& v : w) v = 0.02f * frand();
    for (auto& v : bias) v = 0.01f * frand();
    float scale, mn, mx;
    int64_t zp;
    CHECK(tkv_hip_calibrate_minmax(x.data(), m * k, 1, &scale, &zp, &mn, &mx) == TKV_HIP_OK,
          "calibrate_minmax");
    float am = 0.0f;
    for (float v : x) am = std::fmax(am, std::fabs(v));
    CHECK(scale == (float)((double)am / 127.0), "calibrate scale = fl32(am / 127)");
    std::vector<int32_t> qa(m * k), qw(n * k);
    CHECK(tkv_hip_quantize_int8_symmetric(x.data(), m * k, qa.data(), m * k, scale) == TKV_HIP_OK,
          "quantize_int8_symmetric");
    for (int i = 0; i < n * k; i++) qw[i] = (int32_t)((i * 7) % 255) - 127;
    std::vector<int32_t> acc(m * n);
    CHECK(tkv_hip_matmul_int8_accum(qa.data(), qw.data(), acc.data(), m, n, k) == TKV_HIP_OK,
          "matmul_int8_accum");
    bool exact = true;
    for (int i = 0; i < m; i++)
        for (int j = 0; j < n; j++) {
            int64_t s = 0;
            for (int p = 0; p < k; p++) s += (int64_t)qa[i * k + p] * qw[j * k + p];
            exact &= acc[i * n + j] == s;
        }
    CHECK(exact, "INT32 accumulators exact");
    std::vector<float> sw(n, 1e-3f);
    CHECK(tkv_hip_matmul_int8_per_channel(qa.data(), qw.data(), bias.data(), n, y.data(), m, n, k,
                                          scale, sw.data(), n) == TKV_HIP_OK,
          "matmul_int8_per_channel");
    std::vector<int32_t> f8(m * k);
    std::vector<float> back(m * k);
    CHECK(tkv_hip_quantize_fp8_e4m3(x.data(), m * k, f8.data(), m * k) == TKV_HIP_OK, "fp8 quantize");
    CHECK(tkv_hip_dequantize_fp8_e4m3(f8.data(), m * k, back.data(), m * k) == TKV_HIP_OK,
          "fp8 dequantize");
    std::vector<float> rs(m);
    CHECK(tkv_hip_quantize_dynamic_int8_rowwise(x.data(), m * k, qa.data(), m * k, m, k, rs.data(),
                                                m) == TKV_HIP_OK,
          "rowwise quantize");
    std::vector<int64_t> y64(m * n);
    std::vector<int32_t> bkn(k * n);
    for (int p = 0; p < k; p++)
        for (int j = 0; j < n; j++) bkn[p * n + j] = qw[j * k + p];
    CHECK(tkv_hip_matmul_integer(qa.data(), m * k, bkn.data(), k * n, y64.data(), m * n, m, n, k) ==
              TKV_HIP_OK,
          "matmul_integer");
    std::vector<int32_t> yq(m * n);
    CHECK(tkv_hip_qlinear_matmul(qa.data(), m * k, 0.02f, 3, bkn.data(), k * n, 0.003f, -2, 0.05f, 1,
                                 yq.data(), m * n, m, n, k, 0) == TKV_HIP_OK,
          "qlinear_matmul");
    CHECK(tkv_hip_calibrate_kl(x.data(), m * k, 128, 64, &scale, &zp, &mn, &mx) == TKV_HIP_OK, "kl");
    CHECK(tkv_hip_calibrate_percentile(x.data(), m * k, 99.0f, 1, &scale, &zp, &mn, &mx) ==
              TKV_HIP_OK,
          "percentile");
    CHECK(tkv_hip_calibrate_mse(x.data(), m * k, 20, &scale, &zp, &mn, &mx) == TKV_HIP_OK, "mse");
    const int gs = 64;
    std::vector<int32_t> packed(n * k / 2);
    std::vector<float> gsc(n * k / gs), deq(n * k);
    CHECK(tkv_hip_quantize_int4_grouped(w.data(), n * k, n, k, gs, packed.data(), n * k / 2,
                                        gsc.data(), n * k / gs) == TKV_HIP_OK,
          "int4 quantize");
    CHECK(tkv_hip_dequantize_int4_grouped(packed.data(), n * k / 2, deq.data(), n * k, n, k, gs,
                                          gsc.data(), n * k / gs) == TKV_HIP_OK,
          "int4 dequantize");

    // device entry points, weights, linears, the static entry
    void *dx = nullptr, *dw = nullptr, *db = nullptr, *dy = nullptr, *dy2 = nullptr;
    CHECK(tkv_hip_malloc(ctx, m * k * 4, &dx) == TKV_HIP_OK, "malloc x");
    CHECK(tkv_hip_malloc(ctx, n * k * 4, &dw) == TKV_HIP_OK, "malloc w");
    CHECK(tkv_hip_malloc(ctx, n * 4, &db) == TKV_HIP_OK, "malloc b");
    CHECK(tkv_hip_malloc(ctx, m * n * 4, &dy) == TKV_HIP_OK, "malloc y");
    CHECK(tkv_hip_malloc(ctx, m * n * 4, &dy2) == TKV_HIP_OK, "malloc y2");
    CHECK(tkv_hip_memcpy_h2d(ctx, dx, x.data(), m * k * 4) == TKV_HIP_OK, "h2d x");
    CHECK(tkv_hip_memcpy_h2d(ctx, dw, w.data(), n * k * 4) == TKV_HIP_OK, "h2d w");
    CHECK(tkv_hip_memcpy_h2d(ctx, db, bias.data(), n * 4) == TKV_HIP_OK, "h2d b");
    int64_t wt = 0;
    CHECK(tkv_hip_weight_create(ctx, (const float*)dw, n, k, (const float*)db,
                                TKV_HIP_WEIGHT_INT8, &wt) == TKV_HIP_OK,
          "weight_create");
    for (int mode = 0; mode < 2; mode++) {
        std::vector<float> ya(m * n), yb(m * n);
        CHECK(tkv_hip_linear_forward(ctx, wt, (const float*)dx, m, mode, (float*)dy) == TKV_HIP_OK,
              "linear_forward");
        void* stream = nullptr;
        CHECK(tkv_hip_ctx_get_stream(ctx, &stream) == TKV_HIP_OK, "get_stream");
        CHECK(tkv_hip_linear_forward_static(wt, (const float*)dx, m, mode, (float*)dy2, stream) ==
                  TKV_HIP_OK,
              "linear_forward_static");
        CHECK(tkv_hip_ctx_synchronize(ctx) == TKV_HIP_OK, "synchronize");
        CHECK(tkv_hip_memcpy_d2h(ctx, ya.data(), dy, m * n * 4) == TKV_HIP_OK, "d2h y");
        CHECK(tkv_hip_memcpy_d2h(ctx, yb.data(), dy2, m * n * 4) == TKV_HIP_OK, "d2h y2");
        CHECK(memcmp(ya.data(), yb.data(), m * n * 4) == 0, "static entry equals linear_forward");
    }
    // FP8 weights: the reference-products handle (codes plus their f16
    // decode) and the full-rate one, per-tensor activations
    for (int32_t fmt : {TKV_HIP_WEIGHT_FP8, TKV_HIP_WEIGHT_FP8_FAST}) {
        int64_t wf = 0;
        CHECK(tkv_hip_weight_create(ctx, (const float*)dw, n, k, (const float*)db, fmt, &wf) ==
                  TKV_HIP_OK,
              "fp8 weight_create");
        CHECK(tkv_hip_linear_forward(ctx, wf, (const float*)dx, m, TKV_HIP_ACT_PER_TENSOR,
                                     (float*)dy) == TKV_HIP_OK,
              "fp8 linear_forward");
        CHECK(tkv_hip_linear_forward(ctx, wf, (const float*)dx, m, TKV_HIP_ACT_PER_TOKEN,
                                     (float*)dy) == TKV_HIP_UNSUPPORTED,
              "fp8 linear_forward refuses per-token activations");
        CHECK(tkv_hip_ctx_synchronize(ctx) == TKV_HIP_OK, "fp8 synchronize");
        CHECK(tkv_hip_weight_free(wf) == TKV_HIP_OK, "fp8 weight_free");
    }
    // GGUF Q8_0 weights (raw blocks on the device): both activation modes,
    // the raw GEMM entry on the handle's codes, and the refusals
    {
        const int kb = k / 32;
        std::vector<uint8_t> blocks((size_t)n * kb * 34);
        for (size_t i = 0; i < blocks.size(); i++) blocks[i] = (uint8_t)(i * 37 + 11);
        for (int b = 0; b < n * kb; b++) {  // f16 scales 2^-6 .. 2^-3, both signs
            blocks[(size_t)b * 34] = 0;
            blocks[(size_t)b * 34 + 1] = (uint8_t)(0x24 + 4 * (b % 4)) | (uint8_t)((b & 1) << 7);
        }
        void* draw = nullptr;
        CHECK(tkv_hip_malloc(ctx, blocks.size(), &draw) == TKV_HIP_OK, "malloc q8_0 blocks");
        CHECK(tkv_hip_memcpy_h2d(ctx, draw, blocks.data(), blocks.size()) == TKV_HIP_OK,
              "h2d q8_0 blocks");
        int64_t wq = 0;
        CHECK(tkv_hip_weight_create_gguf_q8_0(ctx, (const uint8_t*)draw, n, k - 16,
                                              (const float*)db, &wq) == TKV_HIP_BAD_ARG,
              "q8_0 weight with K % 32 != 0");
        CHECK(tkv_hip_weight_create_gguf_q8_0(ctx, (const uint8_t*)draw, n, k, (const float*)db,
                                              &wq) == TKV_HIP_OK,
              "q8_0 weight_create");
        for (int mode = 0; mode < 2; mode++)
            CHECK(tkv_hip_linear_forward(ctx, wq, (const float*)dx, m, mode, (float*)dy) ==
                      TKV_HIP_OK,
                  "q8_0 linear_forward");
        CHECK(tkv_hip_linear_forward(ctx, wq, (const float*)dx, 5, TKV_HIP_ACT_PER_TOKEN,
                                     (float*)dy) == TKV_HIP_OK,
              "q8_0 linear_forward, decode batch");
        void *codes = nullptr, *dqa = nullptr, *dsa = nullptr;
        float* gsc_dev = nullptr;
        int64_t wn = 0, wk = 0;
        int32_t wfmt = -1;
        CHECK(tkv_hip_weight_info(wq, &codes, &gsc_dev, nullptr, &wn, &wk, &wfmt) == TKV_HIP_OK &&
                  wfmt == TKV_HIP_WEIGHT_Q8_0 && wn == n && wk == k,
              "q8_0 weight_info");
        std::vector<int8_t> a8(m * k);
        for (int i = 0; i < m * k; i++) a8[i] = (int8_t)((i * 13) % 255 - 127);
        const float sa1 = 0.01f;
        CHECK(tkv_hip_malloc(ctx, m * k, &dqa) == TKV_HIP_OK, "malloc q8_0 a");
        CHECK(tkv_hip_malloc(ctx, 4, &dsa) == TKV_HIP_OK, "malloc q8_0 sa");
        CHECK(tkv_hip_memcpy_h2d(ctx, dqa, a8.data(), m * k) == TKV_HIP_OK, "h2d q8_0 a");
        CHECK(tkv_hip_memcpy_h2d(ctx, dsa, &sa1, 4) == TKV_HIP_OK, "h2d q8_0 sa");
        CHECK(tkv_hip_dev_matmul_q8_0(ctx, (const int8_t*)dqa, (const int8_t*)codes, gsc_dev, m, n,
                                      k, (const float*)dsa, 0, nullptr, (float*)dy) == TKV_HIP_OK,
              "q8_0 GEMM");
        CHECK(tkv_hip_dev_matmul_q8_0(ctx, (const int8_t*)dqa, (const int8_t*)codes, gsc_dev, m, n,
                                      k - 32, (const float*)dsa, 0, nullptr, (float*)dy) ==
                  TKV_HIP_UNSUPPORTED,
              "q8_0 GEMM with K % 128 != 0");
        CHECK(tkv_hip_linear_forward_static(wq, (const float*)dx, m, 0, (float*)dy, nullptr) ==
                  TKV_HIP_UNSUPPORTED,
              "static entry refuses Q8_0 weights");
        CHECK(tkv_hip_ctx_synchronize(ctx) == TKV_HIP_OK, "q8_0 synchronize");
        CHECK(tkv_hip_weight_free(wq) == TKV_HIP_OK, "q8_0 weight_free");
        for (void* p : {draw, dqa, dsa}) CHECK(tkv_hip_free(ctx, p) == TKV_HIP_OK, "free q8_0");
    }
    // tuning overrides: every configuration of the tiled GEMM on one product
    for (int cfg = 0; cfg <= 11; cfg++) {
        CHECK(tkv_hip_ctx_set_tuning(ctx, TKV_HIP_TUNE_GEMM_CFG, cfg) == TKV_HIP_OK, "set cfg");
        CHECK(tkv_hip_linear_forward(ctx, wt, (const float*)dx, m, 0, (float*)dy) == TKV_HIP_OK,
              "linear_forward under a forced configuration");
    }
    CHECK(tkv_hip_ctx_set_tuning(ctx, TKV_HIP_TUNE_GEMM_CFG, -1) == TKV_HIP_OK, "reset cfg");
    CHECK(tkv_hip_ctx_set_tuning(ctx, TKV_HIP_TUNE_GEMM_CFG, 12) == TKV_HIP_BAD_ARG, "cfg range");
    CHECK(tkv_hip_ctx_set_tuning(ctx, 99, 0) == TKV_HIP_BAD_ARG, "unknown knob");

    // graphs: capture, replay, workspace growth under a live graph, and a
    // context destroyed before its graph
    int64_t g = 0;
    CHECK(tkv_hip_capture_begin(ctx) == TKV_HIP_OK, "capture_begin");
    CHECK(tkv_hip_linear_forward(ctx, wt, (const float*)dx, m, 0, (float*)dy) == TKV_HIP_OK,
          "captured linear_forward");
    CHECK(tkv_hip_capture_end(ctx, &g) == TKV_HIP_OK && g != 0, "capture_end");
    CHECK(tkv_hip_graph_launch(ctx, g) == TKV_HIP_OK, "graph_launch");
    void* big = nullptr;
    const int mb = 4100, kb = 384;
    CHECK(tkv_hip_malloc(ctx, (int64_t)mb * kb * 4, &big) == TKV_HIP_OK, "malloc big");
    CHECK(tkv_hip_memset(ctx, big, 0, (int64_t)mb * kb * 4) == TKV_HIP_OK, "memset big");
    void* dw2 = nullptr;
    CHECK(tkv_hip_malloc(ctx, (int64_t)n * kb * 4, &dw2) == TKV_HIP_OK, "malloc w2");
    CHECK(tkv_hip_memset(ctx, dw2, 0, (int64_t)n * kb * 4) == TKV_HIP_OK, "memset w2");
    int64_t wt2 = 0;
    CHECK(tkv_hip_weight_create(ctx, (const float*)dw2, n, kb, nullptr, TKV_HIP_WEIGHT_INT8, &wt2) ==
              TKV_HIP_OK,
          "weight_create 2");
    void* ybig = nullptr;
    CHECK(tkv_hip_malloc(ctx, (int64_t)mb * n * 4, &ybig) == TKV_HIP_OK, "malloc ybig");
    CHECK(tkv_hip_linear_forward(ctx, wt2, (const float*)big, mb, 0, (float*)ybig) == TKV_HIP_OK,
          "workspace growth with a live graph");
    int64_t retired = -1;
    CHECK(tkv_hip_ctx_retired_buffers(ctx, &retired) == TKV_HIP_OK && retired > 0,
          "grown workspace retired, not freed");
    CHECK(tkv_hip_graph_launch(ctx, g) == TKV_HIP_OK, "replay after growth");
    CHECK(tkv_hip_ctx_synchronize(ctx) == TKV_HIP_OK, "synchronize after replay");
    for (void* p : {dx, dw, dw2, db, dy, dy2, big, ybig}) CHECK(tkv_hip_free(ctx, p) == TKV_HIP_OK, "free");
    CHECK(tkv_hip_weight_free(wt) == TKV_HIP_OK && tkv_hip_weight_free(wt2) == TKV_HIP_OK,
          "weight_free");
    CHECK(tkv_hip_ctx_destroy(ctx) == TKV_HIP_OK, "ctx_destroy with a live graph");
    int64_t other = 0;
    CHECK(tkv_hip_ctx_create(0, &other) == TKV_HIP_OK, "second context");
    CHECK(tkv_hip_graph_launch(other, g) == TKV_HIP_BAD_ARG, "detached graph refuses to launch");
    CHECK(tkv_hip_graph_destroy(g) == TKV_HIP_OK, "detached graph destroy");
    CHECK(tkv_hip_ctx_destroy(other) == TKV_HIP_OK, "second ctx_destroy");
}

int main() {
    no_device_independent_checks();
    const int devices = tkv_hip_device_count();
    if (devices < 1)
        no_device_checks();
    else
        device_checks();
    if (g_fail) return 1;
    printf("host_sanitize: all checks passed (%s)\n", devices < 1 ? "no device" : "device 0");
    return 0;
}
