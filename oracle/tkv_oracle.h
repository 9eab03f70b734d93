/*
 * tkv_oracle.h -- CPU restatement of TokenVector.Inference's PTQ path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for
 * libtkv_hip: only tests/, __graft_entry__.smoke() and the cpu_baseline leg
 * of bench.py may load it.  The product library never links or calls it.
 *
 * Every function restates one scalar .tkv routine of the reference
 * (paths relative to the reference checkout):
 *   tv/quantization/engine.tkv   calibrate / quantize / dequantize
 *   tv/quantization/matmul.tkv   INT8 / FP8 GEMMs, FP8 pack
 *   tv/quantization/types.tkv    FP8 e4m3 / e5m2 codec
 *   tv/runtime/f32_bits.tkv      f32 <-> f64 bit reinterpretation
 *   tv/runtime/session.tkv       QuantizedGemm / MatMulInteger / ONNX Q-DQ nodes
 *   tv/quantization/int4.tkv     grouped INT4 (symmetric, AWQ-asym, act-order)
 *   tv/format/gguf.tkv           GGUF Q8_0 / Q4_0 / Q4_1 block decoding
 *   tv/training/gpt2_ref.tkv     LCG31 + Box-Muller input generator
 *
 * Codes are int32 per element, as the reference stores them (List<int>).
 * Floating-point typing follows the reference compiler's IL rules:
 * unannotated float locals are f64, f32 (+) f32 and literal (+) f32 are
 * computed in f32, and values are rounded to f32 at typed boundaries
 * (list[f32] stores, f32 fields and returns).  Where that typing cannot be
 * pinned without running the reference compiler, a recipe switch selects the
 * alternate reading (TKVO_RECIPE_*).
 *
 * Parity unpinned (compiler typing only; the arithmetic of both readings is
 * pinned by the tests):
 *   - tkvo_quantize_int8_symmetric: whether 1.0/scale (engine.tkv:219-222)
 *     is evaluated in f32 (primary) or f64 (TKVO_RECIPE_ALTERNATE);
 *   - tkvo_matmul_int8_per_channel / _symmetric: whether the i64 * f32
 *     epilogue chains (matmul.tkv:5,14 and :29) run in f64 (primary) or f32;
 *   - tkvo_qlinear_matmul: whether mult = sa * sw / sy (session.tkv:2027)
 *     runs on f64 locals (primary) or as an f32 chain;
 *   - tkvo_calibrate_kl: the natural log is the host libm's (the runtime's
 *     Math.Log), pinned only through the selected threshold.
 * No reference test reaches a rounding tie that separates the readings, and
 * the reference compiler (tkvc, .NET) is not available to run.
 */
#ifndef TKV_ORACLE_H
#define TKV_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* QuantParams record (tv/quantization/types.tkv:17-27), minus the _ok slot. */
typedef struct {
    float scale;
    int64_t zero_point;
    float min_val;
    float max_val;
} tkvo_qparams;

/* Recipe switches for typing the reference compiler leaves unpinned. */
enum {
    TKVO_RECIPE_PRIMARY = 0,   /* IL-derived reading (default)            */
    TKVO_RECIPE_ALTERNATE = 1  /* the other plausible reading             */
};

/* ---- f32_bits.tkv ---------------------------------------------------- */
int64_t tkvo_f64_to_f32_bits(double x);
double tkvo_f32_bits_to_f64(int64_t b);

/* ---- types.tkv: FP8 / FP16 codec ------------------------------------- */
int64_t tkvo_rne_rshift(int64_t v, int64_t s);
int64_t tkvo_fp8_encode(float x, int64_t bias, int64_t w, int64_t emax_field,
                        int64_t has_inf, int64_t sat_bits);
float tkvo_fp8_decode(int64_t v, int64_t bias, int64_t w, int64_t emax_field,
                      int64_t has_inf);
int64_t tkvo_fp8_e4m3_encode(float x);   /* byte 0..255 */
float tkvo_fp8_e4m3_decode(int64_t v);   /* v masked to 8 bits */
int64_t tkvo_fp8_e5m2_encode(float x);
float tkvo_fp8_e5m2_decode(int64_t v);

/* ---- engine.tkv ------------------------------------------------------ */
tkvo_qparams tkvo_quant_identity(void);
tkvo_qparams tkvo_calibrate_minmax(const float* data, int64_t n, int32_t symmetric);
/* engine.tkv:42-123: TensorRT-style KL calibration over a num_bins histogram
 * of |x|, thresholds target_bins, target_bins + 16, ..., num_bins. */
tkvo_qparams tkvo_calibrate_kl(const float* data, int64_t n, int64_t num_bins,
                               int64_t target_bins);
/* engine.tkv:126-162: clip at the percentile of |x| (sorted); *err = 1 where
 * the reference raises ValueError (percentile outside (0, 100]). */
tkvo_qparams tkvo_calibrate_percentile(const float* data, int64_t n, float percentile,
                                       int32_t symmetric, int32_t* err);
/* engine.tkv:165-197: MSE grid search over num_candidates thresholds. */
tkvo_qparams tkvo_calibrate_mse(const float* data, int64_t n, int64_t num_candidates);
/* returns 0, or -4 for the ValueError cases of engine.tkv:203-206 */
int32_t tkvo_calibrate_per_channel_minmax(const float* data, int64_t len, int64_t rows,
                                          int64_t cols, int32_t symmetric,
                                          tkvo_qparams* out);
int32_t tkvo_quantize_int8_symmetric(const float* src, int64_t n, int32_t* dst,
                                     float scale, int32_t recipe);
int32_t tkvo_dequantize_int8_symmetric(const int32_t* src, int64_t n, float* dst,
                                       float scale);
int32_t tkvo_quantize_int8_per_channel(const float* src, int32_t* dst, int64_t rows,
                                       int64_t cols, const float* scales);
int32_t tkvo_dequantize_int8_per_channel(const int32_t* src, float* dst, int64_t rows,
                                         int64_t cols, const float* scales);
int32_t tkvo_quantize_dynamic_int8_rowwise(const float* src, int32_t* dst, int64_t rows,
                                           int64_t cols, float* scales_out);

/* ---- matmul.tkv ------------------------------------------------------ */
int64_t tkvo_dot_int8(const int32_t* a, int64_t ao, const int32_t* b, int64_t bo,
                      int64_t k);
/* nbias == 0 means "no bias" (len(pbias) == 0). */
int32_t tkvo_matmul_int8_symmetric(const int32_t* a, const int32_t* w,
                                   const float* bias, int64_t nbias, float* y,
                                   int64_t m, int64_t n, int64_t k,
                                   float scale_a, float scale_w, int32_t recipe);
/* returns -4 when nscales < n (ValueError at matmul.tkv:18-19) */
int32_t tkvo_matmul_int8_per_channel(const int32_t* a, const int32_t* w,
                                     const float* bias, int64_t nbias, float* y,
                                     int64_t m, int64_t n, int64_t k, float scale_a,
                                     const float* scales_w, int64_t nscales,
                                     int32_t recipe);
/* INT32 accumulators only (the integer core shared by both INT8 GEMMs). */
int32_t tkvo_matmul_int8_accum(const int32_t* a, const int32_t* w, int32_t* acc,
                               int64_t m, int64_t n, int64_t k);
int32_t tkvo_quantize_fp8_e4m3(const float* src, int64_t n, int32_t* dst);
int32_t tkvo_dequantize_fp8_e4m3(const int32_t* src, int64_t n, float* dst);
int32_t tkvo_matmul_fp8_e4m3(const int32_t* a, const int32_t* w, const float* bias,
                             int64_t nbias, float* y, int64_t m, int64_t n, int64_t k);
/* Exact FP8 dot-product sum of matmul_fp8_e4m3 in units of 2^-20 (int64),
 * and sum |a_k w_k|.  Used to state error bounds for the f32-accumulating
 * GPU GEMM. */
int32_t tkvo_matmul_fp8_e4m3_exact(const int32_t* a, const int32_t* w, int64_t* acc_q20,
                                   double* abs_sum, int64_t m, int64_t n, int64_t k);

/* ---- FP8 W8A8 linear (R-ext, an extension defined on matmul.tkv) ------
 * The reference's FP8 GEMM has no scales; configs[3] needs per-tensor
 * activation and per-channel weight scales:
 *   s = fl32(max(am, 1e-8) / 240), codes = encode(fl32(x * fl32(1 / s))),
 *   y[m, n] = fl32(fl64(fl64(S * sa[m * sa_stride]) * sw[n]) + b[n])
 * with S the reference's exact product sum (matmul.tkv:52-55). */
int32_t tkvo_quantize_fp8_e4m3_dynamic_tensor(const float* x, int64_t n, int32_t* dst,
                                              float* scale_out);
int32_t tkvo_fp8_weight_pack(const float* w, int64_t rows, int64_t cols, int32_t* dst,
                             float* scales);
int32_t tkvo_matmul_fp8_e4m3_scaled(const int32_t* a, const int32_t* w, const float* bias,
                                    int64_t nbias, float* y, int64_t m, int64_t n, int64_t k,
                                    const float* sa, int64_t sa_stride, const float* sw);

/* ---- session.tkv nodes ----------------------------------------------- */
/* MatMulInteger (session.tkv:2789-2851): B is row-major [K,N]; reads outside
 * na/nb are zero and writes outside ny are dropped, as in the reference. */
int32_t tkvo_matmul_integer(const int32_t* a, int64_t na, const int32_t* b, int64_t nb,
                            int64_t* y, int64_t ny, int64_t m, int64_t n, int64_t k);
/* QLinearMatMul (session.tkv:1992-2071): y = clamp(round(acc * mult) + zpy,
 * -128, 127), acc = sum_p (a - zpa)(b - zpw) over in-range reads (others 0),
 * mult = sa * sw / sy with sy == 0 read as 1; B row-major [K,N]; writes
 * outside ny dropped.  recipe: TKVO_RECIPE_PRIMARY (f64 locals) or
 * TKVO_RECIPE_ALTERNATE (f32 chain for mult).  Parity unpinned for the
 * recipe choice (no reference test runs the node). */
int32_t tkvo_qlinear_matmul(const int32_t* a, int64_t na, float sa, int64_t zpa,
                            const int32_t* b, int64_t nb, float sw, int64_t zpw, float sy,
                            int64_t zpy, int32_t* y, int64_t ny, int64_t m, int64_t n,
                            int64_t k, int32_t recipe);
/* QuantizeLinear (session.tkv:1896-1953).  nscale == 1: per-tensor; else
 * per-axis with the tensor viewed as [outer, dim, inner]. */
int32_t tkvo_quantize_linear(const float* x, int64_t nx, const float* scales,
                             int64_t nscale, int64_t zero_point, int64_t outer,
                             int64_t dim, int64_t inner, int32_t* y);
int32_t tkvo_dequantize_linear(const int32_t* x, int64_t nx, const float* scales,
                               int64_t nscale, int64_t zero_point, int64_t outer,
                               int64_t dim, int64_t inner, float* y);
int32_t tkvo_dynamic_quantize_linear(const float* x, int64_t nx, int32_t* y,
                                     float* y_scale, float* y_zero_point);
/* QuantizedGemm node dispatch (session.tkv:678-697). */
int32_t tkvo_quantized_gemm_node(const int32_t* aq, const int32_t* wq,
                                 const float* bias, int64_t nbias, float* y,
                                 int64_t m, int64_t n, int64_t k, float scale_a,
                                 float scale_b, const float* scales_w,
                                 int64_t nscales, int32_t recipe);

/* ---- int4.tkv: grouped INT4 ------------------------------------------- */
int32_t tkvo_quantize_int4_grouped(const float* src, int64_t nsrc, int64_t rows, int64_t cols,
                                   int64_t group_size, int32_t* packed, int64_t npacked,
                                   float* scales);
int32_t tkvo_dequantize_int4_grouped(const int32_t* packed, int64_t npacked, float* dst,
                                     int64_t ndst, int64_t rows, int64_t cols,
                                     int64_t group_size, const float* scales, int64_t nscales);
int32_t tkvo_quantize_int4_grouped_asym(const float* src, int64_t nsrc, int64_t rows,
                                        int64_t cols, int64_t group_size, int32_t* packed,
                                        int64_t npacked, float* scales, int64_t* zps);
int32_t tkvo_dequantize_int4_grouped_asym(const int32_t* packed, int64_t npacked, float* dst,
                                          int64_t ndst, int64_t rows, int64_t cols,
                                          int64_t group_size, const float* scales,
                                          const int64_t* zps, int64_t ngroups);
int32_t tkvo_permute_cols(const float* src, int64_t rows, int64_t cols, const int64_t* perm,
                          int64_t nperm, int32_t inverse, float* out);
int32_t tkvo_matmul_int4_grouped(const float* a, const int32_t* packed_w, const float* bias,
                                 int64_t nbias, float* y, int64_t m, int64_t n, int64_t k,
                                 int64_t group_size, const float* scales_w, int64_t nscales,
                                 const int64_t* perm);

/* ---- gguf.tkv: block formats ----------------------------------------- */
float tkvo_f16_to_f32(int64_t h);
int32_t tkvo_dequantize_gguf(const uint8_t* raw, int64_t nraw, int64_t n, int32_t dtype,
                             float* out);
/* Extension (no reference counterpart): Q8_0 weights on int8 activation
 * codes with group scales; the recipe is stated at the definition. */
int32_t tkvo_matmul_q8_0(const int32_t* a, const uint8_t* raw, int64_t nraw, const float* sa,
                         int64_t sa_stride, const float* bias, int64_t nbias, float* y,
                         int64_t m, int64_t n, int64_t k);

/* ---- gpt2_ref.tkv input generator ------------------------------------ */
int64_t tkvo_lcg31(int64_t state);
void tkvo_gi_noise(float* out, int64_t n, int64_t seed, double sigma);
/* n_out positions of [0, n) chosen without replacement by LCG31 (seed),
 * each replaced by a sigma_out Gaussian draw (seed2). */
void tkvo_add_outliers(float* x, int64_t n, int64_t n_out, int64_t seed,
                       int64_t seed2, double sigma_out);

/* ---- pinning helpers (independent formulations) ---------------------- */
/* Spec encoder: nearest e4m3fn value by table search with ties to the even
 * code, then the reference's three documented deviations applied. */
int64_t tkvo_pin_e4m3_spec_encode(float x);
/* Exhaustive comparison of tkvo_fp8_e4m3_encode against the spec encoder over
 * every f32 bit pattern whose biased exponent lies in [elo, ehi], both signs.
 * Returns the number of mismatches; the first mismatching pattern goes to
 * *first_bad.  nthreads <= 0 picks the host core count. */
int64_t tkvo_pin_e4m3_exhaustive(int32_t elo, int32_t ehi, int32_t nthreads,
                                 uint32_t* first_bad);

/* tkvo_fp8_e4m3_encode over an array of f32 bit patterns, threaded. */
int32_t tkvo_fp8_e4m3_encode_bits(const uint32_t* bits, int64_t n, uint8_t* out,
                                  int32_t nthreads);

/* ---- threaded baseline helpers (timing only) ------------------------- */
/* OpenMP-free pthread split of matmul_int8_per_channel over rows. */
int32_t tkvo_matmul_int8_per_channel_mt(const int32_t* a, const int32_t* w,
                                        const float* bias, int64_t nbias, float* y,
                                        int64_t m, int64_t n, int64_t k, float scale_a,
                                        const float* scales_w, int64_t nscales,
                                        int32_t nthreads);

#ifdef __cplusplus
}
#endif
#endif
