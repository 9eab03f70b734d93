/* sanitize_check.c -- drives every entry point of the CPU oracle (test
 * infrastructure) on small, edge-case inputs so that it can run under
 * AddressSanitizer + UndefinedBehaviorSanitizer, and its threaded entry
 * points under ThreadSanitizer (oracle/Makefile: `make sanitize`).
 *
 * Every call also checks a property the mathematics fixes (codes in range,
 * round trips, agreement of the threaded and single-threaded forms, exact
 * integer sums), so a sanitizer-clean run is also a correct one.  Exit status
 * 0 = every check passed; the first failing check prints its name. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "tkv_oracle.h"

static int g_fail = 0;
#define CHECK(cond, name)                                   \
    do {                                                    \
        if (!(cond)) {                                      \
            fprintf(stderr, "sanitize_check: FAIL %s\n", name); \
            g_fail = 1;                                     \
        }                                                   \
    } while (0)

/* Exact-size heap buffers, so that any read or write past an end is an
 * AddressSanitizer report rather than a silent access to slack. */
static void* xmalloc(size_t n) {
    void* p = malloc(n ? n : 1);
    if (!p) {
        fprintf(stderr, "sanitize_check: out of memory\n");
        exit(2);
    }
    return p;
}

static float* noise(int64_t n, int64_t seed, double sigma) {
    float* x = (float*)xmalloc((size_t)n * sizeof(float));
    tkvo_gi_noise(x, n, seed, sigma);
    return x;
}

static void check_scalar_codecs(void) {
    /* f32 bit helpers: finite values (subnormals included) round trip; the
     * reference maps -0.0 to the bits of +0.0 and +-inf to 0x7F800000 /
     * 0xFF800000, which it decodes as +-2^128 */
    const double vals[] = {1.0, -2.5, 1e-40, 3.4e38};
    for (size_t i = 0; i < sizeof(vals) / sizeof(vals[0]); i++) {
        const int64_t b = tkvo_f64_to_f32_bits(vals[i]);
        CHECK(tkvo_f32_bits_to_f64(b) == (double)(float)vals[i], "f32 bits round trip");
    }
    CHECK(tkvo_f64_to_f32_bits(-0.0) == 0 && tkvo_f64_to_f32_bits(INFINITY) == 0x7F800000 &&
              (tkvo_f64_to_f32_bits(-INFINITY) & 0xFFFFFFFF) == 0xFF800000,
          "f32 bits of -0 and inf");
    CHECK(tkvo_rne_rshift(6, 2) == 2 && tkvo_rne_rshift(10, 2) == 2 && tkvo_rne_rshift(14, 2) == 4,
          "rne_rshift ties to even");
    for (int64_t c = 0; c < 256; c++) {
        const float d = tkvo_fp8_e4m3_decode(c);
        const int64_t ef = (c >> 3) & 15;
        /* normal codes below the encoder's 248 saturation point round trip
         * (subnormals decode halved and |x| >= 248 encodes as 0x7E, both
         * reference behaviours) */
        if (ef >= 1 && ef <= 14) CHECK(tkvo_fp8_e4m3_encode(d) == c, "e4m3 decode -> encode");
        (void)tkvo_fp8_e5m2_decode(c);
    }
    (void)tkvo_fp8_e5m2_encode(1.5f);
    (void)tkvo_fp8_encode(3.0f, 7, 3, 15, 0, 0x7E);
    (void)tkvo_fp8_decode(0x40, 7, 3, 15, 0);
    CHECK(tkvo_f16_to_f32(0x3C00) == 1.0f && tkvo_f16_to_f32(0xC000) == -2.0f, "f16 decode");
    CHECK(tkvo_pin_e4m3_spec_encode(1.0f) == tkvo_fp8_e4m3_encode(1.0f), "spec encoder agrees");
    const int64_t s = tkvo_lcg31(0);
    CHECK(s == 12345, "lcg31 first step");
}

static void check_calibration(void) {
    const int64_t n = 1000;
    float* x = noise(n, 5, 1.0);
    tkvo_add_outliers(x, n, 3, 3, 4, 20.0);
    x[17] = NAN;
    tkvo_qparams p = tkvo_calibrate_minmax(x, n, 1);
    CHECK(p.scale > 0.0f, "calibrate_minmax scale");
    p = tkvo_calibrate_minmax(x, n, 0);
    (void)tkvo_calibrate_minmax(x, 1, 1);
    (void)tkvo_quant_identity();
    (void)tkvo_calibrate_kl(x, n, 256, 128);
    int32_t err = 0;
    (void)tkvo_calibrate_percentile(x, n, 99.9f, 1, &err);
    (void)tkvo_calibrate_percentile(x, n, 50.0f, 0, &err);
    (void)tkvo_calibrate_mse(x, n, 20);
    const int64_t rows = 7, cols = 13;
    tkvo_qparams* pc = (tkvo_qparams*)xmalloc(sizeof(tkvo_qparams) * rows);
    CHECK(tkvo_calibrate_per_channel_minmax(x, rows * cols, rows, cols, 1, pc) == 0,
          "per-channel calibrate rc");
    for (int64_t r = 0; r < rows; r++) {
        const tkvo_qparams q = tkvo_calibrate_minmax(x + r * cols, cols, 1);
        CHECK(q.scale == pc[r].scale, "per-channel equals per-row calibrate_minmax");
    }
    free(pc);
    free(x);
}

static void check_int8(void) {
    const int64_t rows = 5, cols = 33, n = rows * cols;
    float* x = noise(n, 6, 1.0);
    x[3] = INFINITY;
    x[4] = -INFINITY;
    x[5] = NAN;
    int32_t* q = (int32_t*)xmalloc(sizeof(int32_t) * n);
    float* y = (float*)xmalloc(sizeof(float) * n);
    for (int recipe = 0; recipe < 2; recipe++) {
        CHECK(tkvo_quantize_int8_symmetric(x, n, q, 0.02f, recipe) == 0, "quantize rc");
        for (int64_t i = 0; i < n; i++) CHECK(q[i] >= -127 && q[i] <= 127, "codes in range");
    }
    CHECK(tkvo_dequantize_int8_symmetric(q, n, y, 0.02f) == 0, "dequantize rc");
    float* sc = (float*)xmalloc(sizeof(float) * rows);
    for (int64_t r = 0; r < rows; r++) sc[r] = 0.01f * (float)(r + 1);
    CHECK(tkvo_quantize_int8_per_channel(x, q, rows, cols, sc) == 0, "per-channel rc");
    CHECK(tkvo_dequantize_int8_per_channel(q, y, rows, cols, sc) == 0, "per-channel dq rc");
    CHECK(tkvo_quantize_dynamic_int8_rowwise(x + 6, q, rows - 1, cols, sc) == 0, "rowwise rc");
    free(sc);
    free(y);
    free(q);
    free(x);
}

/* Exact INT32 sums of the matmul forms, against a plain int64 triple loop. */
static void check_matmuls(void) {
    const int64_t m = 6, n = 9, k = 37;
    int32_t* a = (int32_t*)xmalloc(sizeof(int32_t) * m * k);
    int32_t* w = (int32_t*)xmalloc(sizeof(int32_t) * n * k);
    int64_t s = 11;
    for (int64_t i = 0; i < m * k; i++) { s = tkvo_lcg31(s); a[i] = (int32_t)(s % 255) - 127; }
    for (int64_t i = 0; i < n * k; i++) { s = tkvo_lcg31(s); w[i] = (int32_t)(s % 255) - 127; }
    int32_t* acc = (int32_t*)xmalloc(sizeof(int32_t) * m * n);
    CHECK(tkvo_matmul_int8_accum(a, w, acc, m, n, k) == 0, "accum rc");
    for (int64_t i = 0; i < m; i++)
        for (int64_t j = 0; j < n; j++) {
            int64_t t = 0;
            for (int64_t p = 0; p < k; p++) t += (int64_t)a[i * k + p] * w[j * k + p];
            CHECK(acc[i * n + j] == t, "INT32 accumulators exact");
            CHECK(tkvo_dot_int8(a, i * k, w, j * k, k) == t, "dot_int8 exact");
        }
    float* bias = noise(n, 2, 0.01);
    float* sw = (float*)xmalloc(sizeof(float) * n);
    for (int64_t j = 0; j < n; j++) sw[j] = 0.001f * (float)(j + 1);
    float* y = (float*)xmalloc(sizeof(float) * m * n);
    float* y2 = (float*)xmalloc(sizeof(float) * m * n);
    CHECK(tkvo_matmul_int8_symmetric(a, w, bias, n, y, m, n, k, 0.02f, 0.003f, 0) == 0, "sym rc");
    CHECK(tkvo_matmul_int8_per_channel(a, w, bias, n, y, m, n, k, 0.02f, sw, n, 0) == 0, "pc rc");
    CHECK(tkvo_matmul_int8_per_channel_mt(a, w, bias, n, y2, m, n, k, 0.02f, sw, n, 3) == 0,
          "pc mt rc");
    CHECK(memcmp(y, y2, sizeof(float) * m * n) == 0, "threaded per-channel matmul agrees");
    CHECK(tkvo_matmul_int8_per_channel(a, w, NULL, 0, y, m, n, k, 0.02f, sw, n, 1) == 0,
          "pc no bias rc");
    CHECK(tkvo_quantized_gemm_node(a, w, bias, n, y, m, n, k, 0.02f, 0.0f, sw, n, 0) == 0,
          "node rc");
    /* MatMulInteger reads B as [K, N] */
    int32_t* bt = (int32_t*)xmalloc(sizeof(int32_t) * k * n);
    for (int64_t j = 0; j < n; j++)
        for (int64_t p = 0; p < k; p++) bt[p * n + j] = w[j * k + p];
    int64_t* y64 = (int64_t*)xmalloc(sizeof(int64_t) * m * n);
    CHECK(tkvo_matmul_integer(a, m * k, bt, k * n, y64, m * n, m, n, k) == 0, "matmul_integer rc");
    for (int64_t i = 0; i < m * n; i++) CHECK(y64[i] == acc[i], "matmul_integer exact");
    int32_t* yq = (int32_t*)xmalloc(sizeof(int32_t) * m * n);
    CHECK(tkvo_qlinear_matmul(a, m * k, 0.02f, 3, bt, k * n, 0.003f, -2, 0.05f, 1, yq, m * n, m,
                              n, k, 0) == 0,
          "qlinear rc");
    for (int64_t i = 0; i < m * n; i++) CHECK(yq[i] >= -128 && yq[i] <= 127, "qlinear range");
    free(yq);
    free(y64);
    free(bt);
    free(y2);
    free(y);
    free(sw);
    free(bias);
    free(acc);
    free(w);
    free(a);
}

static void check_fp8(void) {
    const int64_t m = 4, n = 5, k = 19;
    float* xa = noise(m * k, 8, 1.0);
    float* xw = noise(n * k, 9, 0.02);
    int32_t* a = (int32_t*)xmalloc(sizeof(int32_t) * m * k);
    int32_t* w = (int32_t*)xmalloc(sizeof(int32_t) * n * k);
    float* back = (float*)xmalloc(sizeof(float) * m * k);
    CHECK(tkvo_quantize_fp8_e4m3(xa, m * k, a) == 0, "fp8 quantize rc");
    for (int64_t i = 0; i < m * k; i++) CHECK(a[i] >= -128 && a[i] <= 127, "fp8 offset codes");
    CHECK(tkvo_dequantize_fp8_e4m3(a, m * k, back) == 0, "fp8 dequantize rc");
    CHECK(tkvo_quantize_fp8_e4m3(xw, n * k, w) == 0, "fp8 quantize w rc");
    float* bias = noise(n, 3, 0.01);
    float* y = (float*)xmalloc(sizeof(float) * m * n);
    CHECK(tkvo_matmul_fp8_e4m3(a, w, bias, n, y, m, n, k) == 0, "fp8 matmul rc");
    int64_t* q20 = (int64_t*)xmalloc(sizeof(int64_t) * m * n);
    double* abs_sum = (double*)xmalloc(sizeof(double) * m * n);
    CHECK(tkvo_matmul_fp8_e4m3_exact(a, w, q20, abs_sum, m, n, k) == 0, "fp8 exact rc");
    float sa = 0.0f;
    CHECK(tkvo_quantize_fp8_e4m3_dynamic_tensor(xa, m * k, a, &sa) == 0, "fp8 dynamic rc");
    float* sw = (float*)xmalloc(sizeof(float) * n);
    CHECK(tkvo_fp8_weight_pack(xw, n, k, w, sw) == 0, "fp8 pack rc");
    CHECK(tkvo_matmul_fp8_e4m3_scaled(a, w, bias, n, y, m, n, k, &sa, 0, sw) == 0,
          "fp8 scaled rc");
    /* threaded bit encoder vs the scalar one */
    const int64_t nb = 4099;
    uint32_t* bits = (uint32_t*)xmalloc(sizeof(uint32_t) * nb);
    uint8_t* out = (uint8_t*)xmalloc(nb);
    int64_t st = 77;
    for (int64_t i = 0; i < nb; i++) {
        st = tkvo_lcg31(st);
        bits[i] = (uint32_t)st * 2654435761u;
    }
    CHECK(tkvo_fp8_e4m3_encode_bits(bits, nb, out, 4) == 0, "encode_bits rc");
    for (int64_t i = 0; i < nb; i++) {
        float f;
        memcpy(&f, &bits[i], 4);
        CHECK(out[i] == (uint8_t)tkvo_fp8_e4m3_encode(f), "threaded encoder agrees");
    }
    uint32_t first_bad = 0;
    CHECK(tkvo_pin_e4m3_exhaustive(126, 126, 3, &first_bad) == 0, "exhaustive slice agrees");
    free(out);
    free(bits);
    free(sw);
    free(abs_sum);
    free(q20);
    free(y);
    free(bias);
    free(back);
    free(w);
    free(a);
    free(xw);
    free(xa);
}

static void check_qdq(void) {
    const int64_t outer = 2, dim = 3, inner = 4, n = outer * dim * inner;
    float* x = noise(n, 12, 2.0);
    int32_t* q = (int32_t*)xmalloc(sizeof(int32_t) * n);
    float* y = (float*)xmalloc(sizeof(float) * n);
    const float s1 = 0.05f;
    const float s3[3] = {0.01f, 0.02f, 0.04f};
    CHECK(tkvo_quantize_linear(x, n, &s1, 1, 3, 1, n, 1, q) == 0, "QuantizeLinear rc");
    CHECK(tkvo_quantize_linear(x, n, s3, 3, 0, outer, dim, inner, q) == 0, "per-axis Q rc");
    for (int64_t i = 0; i < n; i++) CHECK(q[i] >= -128 && q[i] <= 127, "Q range");
    CHECK(tkvo_dequantize_linear(q, n, s3, 3, 0, outer, dim, inner, y) == 0, "DQ rc");
    float ys = 0.0f, yz = 0.0f;
    CHECK(tkvo_dynamic_quantize_linear(x, n, q, &ys, &yz) == 0, "DynamicQL rc");
    free(y);
    free(q);
    free(x);
}

static void check_int4_gguf(void) {
    const int64_t rows = 3, cols = 64, gs = 32, n = rows * cols;
    const int64_t npacked = n / 2, ngroups = n / gs;
    float* w = noise(n, 13, 0.02);
    int32_t* packed = (int32_t*)xmalloc(sizeof(int32_t) * npacked);
    float* sc = (float*)xmalloc(sizeof(float) * ngroups);
    int64_t* zp = (int64_t*)xmalloc(sizeof(int64_t) * ngroups);
    float* back = (float*)xmalloc(sizeof(float) * n);
    CHECK(tkvo_quantize_int4_grouped(w, n, rows, cols, gs, packed, npacked, sc) == 0, "int4 q rc");
    CHECK(tkvo_dequantize_int4_grouped(packed, npacked, back, n, rows, cols, gs, sc, ngroups) == 0,
          "int4 dq rc");
    CHECK(tkvo_quantize_int4_grouped_asym(w, n, rows, cols, gs, packed, npacked, sc, zp) == 0,
          "int4 asym q rc");
    CHECK(tkvo_dequantize_int4_grouped_asym(packed, npacked, back, n, rows, cols, gs, sc, zp,
                                            ngroups) == 0,
          "int4 asym dq rc");
    const int64_t m = 2;
    float* a = noise(m * cols, 14, 1.0);
    int64_t* perm = (int64_t*)xmalloc(sizeof(int64_t) * cols);
    for (int64_t i = 0; i < cols; i++) perm[i] = (i * 7) % cols;
    float* ap = (float*)xmalloc(sizeof(float) * m * cols);
    CHECK(tkvo_permute_cols(a, m, cols, perm, cols, 0, ap) == 0, "permute rc");
    float* a2 = (float*)xmalloc(sizeof(float) * m * cols);
    CHECK(tkvo_permute_cols(ap, m, cols, perm, cols, 1, a2) == 0, "inverse permute rc");
    CHECK(memcmp(a, a2, sizeof(float) * m * cols) == 0, "permute round trip");
    CHECK(tkvo_quantize_int4_grouped(w, n, rows, cols, gs, packed, npacked, sc) == 0, "int4 q2 rc");
    float* y = (float*)xmalloc(sizeof(float) * m * rows);
    CHECK(tkvo_matmul_int4_grouped(a, packed, NULL, 0, y, m, rows, cols, gs, sc, ngroups, perm) ==
              0,
          "int4 matmul rc");
    /* GGUF Q8_0: one 34-byte block (f16 scale 1.0, codes 0..31) */
    uint8_t blk[34];
    blk[0] = 0x00;
    blk[1] = 0x3C;
    for (int i = 0; i < 32; i++) blk[2 + i] = (uint8_t)i;
    float out[32];
    CHECK(tkvo_dequantize_gguf(blk, 34, 32, 8, out) == 0, "gguf q8_0 rc");
    for (int i = 0; i < 32; i++) CHECK(out[i] == (float)i, "gguf q8_0 values");
    /* Q8_0 linear on int8 codes: one row of ones against the block above
     * (d = 1): sum 0..31 = 496, times sa = 0.5, plus bias 1 */
    {
        int32_t ones[32];
        for (int i = 0; i < 32; i++) ones[i] = 1;
        const float sa_q8 = 0.5f, b_q8 = 1.0f;
        float yq;
        CHECK(tkvo_matmul_q8_0(ones, blk, 34, &sa_q8, 0, &b_q8, 1, &yq, 1, 1, 32) == 0,
              "q8_0 matmul rc");
        CHECK(yq == 249.0f, "q8_0 matmul value");
        CHECK(tkvo_matmul_q8_0(ones, blk, 33, &sa_q8, 0, NULL, 0, &yq, 1, 1, 32) != 0,
              "q8_0 matmul short raw");
    }
    free(y);
    free(a2);
    free(ap);
    free(perm);
    free(a);
    free(back);
    free(zp);
    free(sc);
    free(packed);
    free(w);
}

int main(void) {
    check_scalar_codecs();
    check_calibration();
    check_int8();
    check_matmuls();
    check_fp8();
    check_qdq();
    check_int4_gguf();
    if (g_fail) return 1;
    printf("sanitize_check: all checks passed\n");
    return 0;
}
