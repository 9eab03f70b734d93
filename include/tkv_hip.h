/*
 * tkv_hip.h -- C ABI of libtkv_hip, the MI355X (gfx950) implementation of
 * TokenVector.Inference's post-training-quantization hot path.
 *
 * The reference (.tkv compiled to .NET IL) reaches native code only through
 * compiler builtins that P/Invoke a C export taking the backing arrays of
 * List<T> plus int64 sizes and returning an int32 rc
 * (docs/HANDOFF.md:1616,1643,2009,2563; the simd_gemm_* family).  This
 * library follows that convention:
 *
 *   - every entry point is extern "C", takes plain pointers and int64 sizes,
 *     and returns an int32 rc (TKV_HIP_OK or a negative code below);
 *   - on rc < 0 the caller runs its original .tkv loop (docs/HANDOFF.md:3649);
 *   - the caller owns every buffer; nothing is retained after return except
 *     through an explicit handle (context, weight) with create/destroy, as
 *     simd_gemm_packed_create/free do (docs/HANDOFF.md:1675);
 *   - entry points are re-entrant: state lives in contexts, never in
 *     process-wide mutable globals (the shared g_job of simd_gemm hung two
 *     callers, docs/COMPILER_TEAM_REQUEST2.md:46,91).
 *
 * Two families:
 *   tkv_hip_<fn>       host-pointer mirrors of the .tkv functions, with the
 *                      same argument order and meaning; codes are int32 per
 *                      element (List<int>), as the reference stores them.
 *   tkv_hip_dev_<fn>   device-pointer variants on packed codes (int8 for INT8,
 *                      raw e4m3 bytes for FP8) that run asynchronously on the
 *                      context's stream.
 *
 * Citations are path:line inside the reference checkout.
 */
#ifndef TKV_HIP_H
#define TKV_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- return codes ----------------------------------------------------- */
#define TKV_HIP_OK 0
#define TKV_HIP_UNSUPPORTED (-1) /* shape / layout not handled: fall back      */
#define TKV_HIP_NO_DEVICE (-2)   /* no usable gfx950 device                      */
#define TKV_HIP_OOM (-3)         /* device or pinned allocation failed           */
#define TKV_HIP_BAD_ARG (-4)     /* the cases where the .tkv raises ValueError   */
#define TKV_HIP_DEVICE_ERROR (-5)/* HIP runtime error (message in last_error)    */

/* Numeric recipe switches: typing the reference compiler leaves unpinned
 * (f32 vs f64 reciprocal in quantize_int8_symmetric, f64 vs f32 epilogue
 * chain in the INT8 GEMMs).  PRIMARY follows the IL typing rules of
 * docs/HANDOFF.md:1994-1999,3645,3663,3994-3997. */
#define TKV_HIP_RECIPE_PRIMARY 0
#define TKV_HIP_RECIPE_ALTERNATE 1

/* Per-tensor quantization parameters as kept in device memory, so that a
 * calibration can feed a quantize / GEMM without a host round trip.
 * scale/zero_point/min_val/max_val are the QuantParams fields
 * (tv/quantization/types.tkv:17-27); inv is the reciprocal the reference's
 * quantize loop multiplies by (f64). */
typedef struct {
    float scale;
    float min_val;
    float max_val;
    int32_t zero_point;
    double inv;
    double reserved;
} tkv_hip_qparams_dev;

/* ---- library / context -------------------------------------------------- */
/* No reference counterpart: library plumbing. */
int32_t tkv_hip_version(void);
/* Number of visible gfx950 devices (0 if none). */
int32_t tkv_hip_device_count(void);
/* Copies the calling thread's last error message; returns its length. */
int32_t tkv_hip_last_error(char* buf, int32_t len);
/* A context owns a HIP stream (or borrows the caller's) and a grow-only
 * device workspace.  Handles are int64 as the .tkv builtins pass them. */
int32_t tkv_hip_ctx_create(int32_t device, int64_t* ctx_out);
int32_t tkv_hip_ctx_destroy(int64_t ctx);
/* Use an external hipStream_t (e.g. torch's) for subsequent dev calls;
 * NULL restores the context's own stream.  The previous stream is drained
 * first: work on one context never runs on two streams at once (its calls
 * share workspaces and the split-K partial sums).  Calls that overlap on one
 * context from several host threads race on those buffers: drive a context
 * from one thread at a time. */
int32_t tkv_hip_ctx_set_stream(int64_t ctx, void* stream);
int32_t tkv_hip_ctx_get_stream(int64_t ctx, void** stream_out);
int32_t tkv_hip_ctx_synchronize(int64_t ctx);
/* Tuning and test overrides of one context.  No reference counterpart: the
 * library picks every launch shape itself; these exist for sweeps and for
 * tests that must reach a path the automatic choice avoids.  value -1
 * restores the automatic choice; anything outside a knob's range is
 * TKV_HIP_BAD_ARG.  Results are bit-identical under every setting except
 * TKV_HIP_TUNE_INT4_GEMV_WAVE, whose kernel adds the f64 products of the INT4
 * decode GEMV in another order (the same bound applies to both).
 *   GEMM_CFG        0..11  GEMM tile configuration of every INT8 / FP8
 *                          product (10: the skinny kernel, INT8 with M <= 32)
 *   GEMM_STAGGER    0..8   start delay of every other workgroup per XCD in
 *                          the warp-specialised GEMM (units of 1024 cycles)
 *   DECODE_GROUP    1..16  tokens per workgroup of the decode linear
 *   QUANT_TWO_PASS  0..1   1: per-tensor calibrate + quantize always takes
 *                          the two-kernel path (never the single pass)
 *   INT4_GEMV_WAVE  0..1   1: INT4 decode batches take the per-column kernel
 *   GRID_SPIN       0..2^20  polls a workgroup of the single-pass calibrate
 *                          + quantize makes at its grid barrier before it
 *                          scans the whole tensor itself (0: at once)
 *   DECODE_DMA      0..1   the weight path of the M <= 32 kernels (the
 *                          per-token decode linear with INT8 or GGUF Q8_0
 *                          weights, the skinny INT8 GEMM, the INT4 decode
 *                          kernel): 0 each lane's B operand loaded into
 *                          registers, 1 whole 128-byte lines copied into LDS */
enum {
    TKV_HIP_TUNE_GEMM_CFG = 0,
    TKV_HIP_TUNE_GEMM_STAGGER = 1,
    TKV_HIP_TUNE_DECODE_GROUP = 2,
    TKV_HIP_TUNE_QUANT_TWO_PASS = 3,
    TKV_HIP_TUNE_INT4_GEMV_WAVE = 4,
    TKV_HIP_TUNE_GRID_SPIN = 5,
    TKV_HIP_TUNE_DECODE_DMA = 6,
    TKV_HIP_TUNE_COUNT = 7
};
int32_t tkv_hip_ctx_set_tuning(int64_t ctx, int32_t knob, int64_t value);
/* Device memory and copies for callers without their own allocator (tests,
 * the .NET side).  Copies are ordered on the context's stream. */
int32_t tkv_hip_malloc(int64_t ctx, int64_t bytes, void** ptr_out);
int32_t tkv_hip_free(int64_t ctx, void* ptr);
int32_t tkv_hip_memcpy_h2d(int64_t ctx, void* dst, const void* src, int64_t bytes);
int32_t tkv_hip_memcpy_d2h(int64_t ctx, void* dst, const void* src, int64_t bytes);
/* Byte fill, asynchronous on the context's stream (a kernel, so it can be
 * captured). */
int32_t tkv_hip_memset(int64_t ctx, void* dst, int32_t value, int64_t bytes);
/* Device-to-device copy, asynchronous on the context's stream.  16-byte
 * aligned pointers and sizes run one plain streaming kernel (k_copy16) that
 * moves exactly `bytes` each way. */
int32_t tkv_hip_memcpy_d2d(int64_t ctx, void* dst, const void* src, int64_t bytes);
/* Stream-ordered event timing (bench harness). */
int32_t tkv_hip_event_create(int64_t* ev_out);
int32_t tkv_hip_event_destroy(int64_t ev);
int32_t tkv_hip_event_record(int64_t ctx, int64_t ev);
int32_t tkv_hip_event_elapsed_ms(int64_t ev_start, int64_t ev_end, float* ms_out);
/* Stream capture into a replayable HIP graph.  No reference counterpart (the
 * reference runs this path on the CPU); for callers that repeat a fixed
 * sequence of device entry points (a layer stack, a decode step) and want
 * one launch per sequence.  Between begin and end the context's stream
 * records instead of running; every entry point called in between must
 * find its workspace already sized by an identical earlier call (it fails
 * with TKV_HIP_BAD_ARG otherwise), and host-pointer entry points, weight
 * creation, stream switches, copies to or from the host and
 * synchronizations fail.  A graph replays the captured device pointers and
 * scalars as they were, workspace addresses included: while any graph of a
 * context is alive, a workspace that grows keeps its old buffer (it is
 * freed with the context's last graph, or with the context), so a replay
 * after a larger eager call still reads and writes valid memory.
 * Device-resident QuantParams are re-read on every replay.  Replays and
 * eager calls on one context are ordered on its stream.  A context destroyed
 * while some of its graphs are alive releases their executables and
 * detaches them: graph_launch then fails with TKV_HIP_BAD_ARG, and
 * graph_destroy only frees the handle, so either destruction order is safe. */
int32_t tkv_hip_capture_begin(int64_t ctx);
int32_t tkv_hip_capture_end(int64_t ctx, int64_t* graph_out);
int32_t tkv_hip_graph_launch(int64_t ctx, int64_t graph);
int32_t tkv_hip_graph_destroy(int64_t graph);
/* Number of workspace buffers kept alive for live graphs (diagnostics). */
int32_t tkv_hip_ctx_retired_buffers(int64_t ctx, int64_t* count_out);

/* ======================================================================== */
/* Host-pointer mirrors (one per .tkv function).  ctx-free: each calling    */
/* thread uses its own default context on device 0.                         */
/* ======================================================================== */

/* calibrate_minmax(data, symmetric) -> QuantParams   engine.tkv:13-36 */
int32_t tkv_hip_calibrate_minmax(const float* data, int64_t n, int32_t symmetric,
                                 float* scale, int64_t* zero_point, float* min_val,
                                 float* max_val);
/* calibrate_kl(data, num_bins, target_bins) -> QuantParams   engine.tkv:42-123
 * (TensorRT-style KL over a num_bins histogram of |x|; num_bins <= 4096). */
int32_t tkv_hip_calibrate_kl(const float* data, int64_t n, int64_t num_bins,
                             int64_t target_bins, float* scale, int64_t* zero_point,
                             float* min_val, float* max_val);
/* calibrate_percentile(data, percentile, symmetric) -> QuantParams
 * engine.tkv:126-162; TKV_HIP_BAD_ARG where the reference raises
 * ValueError (percentile outside (0, 100]). */
int32_t tkv_hip_calibrate_percentile(const float* data, int64_t n, float percentile,
                                     int32_t symmetric, float* scale, int64_t* zero_point,
                                     float* min_val, float* max_val);
/* calibrate_mse(data, num_candidates) -> QuantParams   engine.tkv:165-197
 * (num_candidates <= 4096; below 4 reads as 4, as in the reference). */
int32_t tkv_hip_calibrate_mse(const float* data, int64_t n, int64_t num_candidates,
                              float* scale, int64_t* zero_point, float* min_val,
                              float* max_val);
/* calibrate_per_channel_minmax(data, rows, cols, symmetric) engine.tkv:202-213;
 * outputs one QuantParams per row as four arrays (zero_points/min/max may be
 * NULL).  BAD_ARG where the .tkv raises (rows/cols <= 0, short data). */
int32_t tkv_hip_calibrate_per_channel_minmax(const float* data, int64_t n_data,
                                             int64_t rows, int64_t cols, int32_t symmetric,
                                             float* scales, int64_t* zero_points,
                                             float* min_vals, float* max_vals);
/* quantize_int8_symmetric(src, dst, scale)            engine.tkv:216-226 */
int32_t tkv_hip_quantize_int8_symmetric(const float* src, int64_t n_src, int32_t* dst,
                                        int64_t n_dst, float scale);
int32_t tkv_hip_quantize_int8_symmetric_recipe(const float* src, int64_t n_src,
                                               int32_t* dst, int64_t n_dst, float scale,
                                               int32_t recipe);
/* dequantize_int8_symmetric(src, dst, scale)          engine.tkv:229-234 */
int32_t tkv_hip_dequantize_int8_symmetric(const int32_t* src, int64_t n_src, float* dst,
                                          int64_t n_dst, float scale);
/* quantize_int8_per_channel(src, dst, rows, cols, scales) engine.tkv:237-250 */
int32_t tkv_hip_quantize_int8_per_channel(const float* src, int64_t n_src, int32_t* dst,
                                          int64_t n_dst, int64_t rows, int64_t cols,
                                          const float* scales, int64_t n_scales);
/* dequantize_int8_per_channel(...)                    engine.tkv:253-262 */
int32_t tkv_hip_dequantize_int8_per_channel(const int32_t* src, int64_t n_src, float* dst,
                                            int64_t n_dst, int64_t rows, int64_t cols,
                                            const float* scales, int64_t n_scales);
/* quantize_dynamic_int8_rowwise(src, dst, rows, cols, scales_out) engine.tkv:266-285 */
int32_t tkv_hip_quantize_dynamic_int8_rowwise(const float* src, int64_t n_src, int32_t* dst,
                                              int64_t n_dst, int64_t rows, int64_t cols,
                                              float* scales_out, int64_t n_scales_out);
/* quantize_fp8_e4m3(src, dst): dst = e4m3 byte - 128    matmul.tkv:60-66 */
int32_t tkv_hip_quantize_fp8_e4m3(const float* src, int64_t n_src, int32_t* dst,
                                  int64_t n_dst);
/* dequantize_fp8_e4m3(src, dst)                         matmul.tkv:68-73 */
int32_t tkv_hip_dequantize_fp8_e4m3(const int32_t* src, int64_t n_src, float* dst,
                                    int64_t n_dst);
/* matmul_int8_symmetric(pa, pw, pbias, py, m, n, k, scale_a, scale_w) matmul.tkv:4-15.
 * n_bias == 0 means no bias (len(pbias) == 0). */
int32_t tkv_hip_matmul_int8_symmetric(const int32_t* pa, const int32_t* pw,
                                      const float* pbias, int64_t n_bias, float* py,
                                      int64_t m, int64_t n, int64_t k, float scale_a,
                                      float scale_w);
/* matmul_int8_per_channel(pa, pw, pbias, py, m, n, k, scale_a, scales_w) matmul.tkv:17-29;
 * BAD_ARG when n_scales < n (matmul.tkv:18-19). */
int32_t tkv_hip_matmul_int8_per_channel(const int32_t* pa, const int32_t* pw,
                                        const float* pbias, int64_t n_bias, float* py,
                                        int64_t m, int64_t n, int64_t k, float scale_a,
                                        const float* scales_w, int64_t n_scales);
/* Same two GEMMs with the epilogue recipe selectable. */
int32_t tkv_hip_matmul_int8_recipe(const int32_t* pa, const int32_t* pw, const float* pbias,
                                   int64_t n_bias, float* py, int64_t m, int64_t n,
                                   int64_t k, float scale_a, float scale_w,
                                   const float* scales_w, int64_t n_scales, int32_t recipe);
/* The INT32 accumulators of the INT8 GEMM (matmul.tkv:116-127 per output). */
int32_t tkv_hip_matmul_int8_accum(const int32_t* pa, const int32_t* pw, int32_t* acc,
                                  int64_t m, int64_t n, int64_t k);
/* matmul_fp8_e4m3(pa, pw, pbias, py, m, n, k)           matmul.tkv:46-58 */
int32_t tkv_hip_matmul_fp8_e4m3(const int32_t* pa, const int32_t* pw, const float* pbias,
                                int64_t n_bias, float* py, int64_t m, int64_t n,
                                int64_t k);
/* QuantizedGemm node (session.tkv:678-697): per-channel iff n_scales > 0,
 * else symmetric with (scale_a, scale_b); M, K from A's shape, N from W's. */
int32_t tkv_hip_quantized_gemm(const int32_t* aq, const int32_t* wq, const float* bias,
                               int64_t n_bias, float* y, int64_t m, int64_t n, int64_t k,
                               float scale_a, float scale_b, const float* scales_w,
                               int64_t n_scales);
/* MatMulInteger node (session.tkv:2789-2851): Y[M,N] int64 = A[M,K] . B[K,N]
 * with B row-major [K,N]; reads past na/nb are 0, writes past ny dropped. */
int32_t tkv_hip_matmul_integer(const int32_t* a, int64_t na, const int32_t* b, int64_t nb,
                               int64_t* y, int64_t ny, int64_t m, int64_t n, int64_t k);
/* QLinearMatMul node (session.tkv:1992-2071, OperatorType_QLinearMatMul = 65):
 * y = clamp(round(acc * mult) + zpy, -128, 127) with
 * acc = sum_p (a[i,p] - zpa) (b[p,j] - zpw) and mult = sa * sw / sy (sy == 0
 * reads as 1).  B is row-major [K,N] as in the node.  recipe PRIMARY: sa, sw,
 * sy are f64 locals holding the f32 inputs (mult = fl64(sa*sw/sy)); ALTERNATE:
 * the f32 chain fl32(fl32(sa*sw)/sy).  Reads past na / nb contribute 0 as in
 * the node (TKV_HIP_UNSUPPORTED when a zero point outside [-128, 127] would be
 * needed to express that); writes past ny are dropped. */
int32_t tkv_hip_qlinear_matmul(const int32_t* a, int64_t na, float sa, int64_t zpa,
                               const int32_t* b, int64_t nb, float sw, int64_t zpw, float sy,
                               int64_t zpy, int32_t* y, int64_t ny, int64_t m, int64_t n,
                               int64_t k, int32_t recipe);
/* QuantizeLinear node (session.tkv:1896-1953): n_scales == 1 per-tensor, else
 * per-axis over the [outer, dim, inner] view of x. */
int32_t tkv_hip_quantize_linear(const float* x, int64_t nx, const float* scales,
                                int64_t n_scales, int64_t zero_point, int64_t outer,
                                int64_t dim, int64_t inner, int32_t* y);
/* DequantizeLinear node (session.tkv:1955-1990) */
int32_t tkv_hip_dequantize_linear(const int32_t* x, int64_t nx, const float* scales,
                                  int64_t n_scales, int64_t zero_point, int64_t outer,
                                  int64_t dim, int64_t inner, float* y);
/* DynamicQuantizeLinear node (session.tkv:2853-2901) */
int32_t tkv_hip_dynamic_quantize_linear(const float* x, int64_t nx, int32_t* y,
                                        float* y_scale, float* y_zero_point);

/* ======================================================================== */
/* Device-pointer variants (asynchronous on the context's stream).          */
/* ctx == 0 selects the calling thread's default context.                   */
/* ======================================================================== */

/* calibrate_minmax on device data; writes one tkv_hip_qparams_dev.
 * engine.tkv:13-36 */
int32_t tkv_hip_dev_calibrate_minmax(int64_t ctx, const float* x, int64_t n,
                                     int32_t symmetric, tkv_hip_qparams_dev* params);
/* The heavier calibrators on device data (engine.tkv:42-197), one
 * tkv_hip_qparams_dev each, no host sync; n > 0. */
int32_t tkv_hip_dev_calibrate_kl(int64_t ctx, const float* x, int64_t n, int64_t num_bins,
                                 int64_t target_bins, tkv_hip_qparams_dev* params);
int32_t tkv_hip_dev_calibrate_percentile(int64_t ctx, const float* x, int64_t n,
                                         float percentile, int32_t symmetric,
                                         tkv_hip_qparams_dev* params);
int32_t tkv_hip_dev_calibrate_mse(int64_t ctx, const float* x, int64_t n,
                                  int64_t num_candidates, tkv_hip_qparams_dev* params);
/* Per-row absmax scales (symmetric calibrate_per_channel_minmax, engine.tkv:202-213):
 * scales[r] = fl32(max(|x[r,:]|, 1e-8) / 127). */
int32_t tkv_hip_dev_calibrate_rows(int64_t ctx, const float* x, int64_t rows, int64_t cols,
                                   float* scales);
/* quantize_int8_symmetric with the scale read from params (device), so it
 * can follow tkv_hip_dev_calibrate_minmax without a sync.  engine.tkv:216-226 */
int32_t tkv_hip_dev_quantize_int8_tensor(int64_t ctx, const float* x, int64_t n,
                                         const tkv_hip_qparams_dev* params, int8_t* q);
/* calibrate_minmax(x, 1) + quantize_int8_symmetric(x, q, p.scale) fused:
 * the activation path of a W8A8 linear (two kernels, no host sync). */
int32_t tkv_hip_dev_quantize_int8_dynamic_tensor(int64_t ctx, const float* x, int64_t n,
                                                 int8_t* q, tkv_hip_qparams_dev* params);
/* quantize_int8_per_channel with device scales.  engine.tkv:237-250 */
int32_t tkv_hip_dev_quantize_int8_per_channel(int64_t ctx, const float* x, int64_t rows,
                                              int64_t cols, const float* scales, int8_t* q);
/* quantize_dynamic_int8_rowwise, one pass per row.  engine.tkv:266-285 */
int32_t tkv_hip_dev_quantize_dynamic_int8_rowwise(int64_t ctx, const float* x,
                                                  int64_t rows, int64_t cols, int8_t* q,
                                                  float* scales_out);
/* dequantize_int8_symmetric / _per_channel (scales == NULL -> per-tensor
 * `scale`).  engine.tkv:229-234,253-262 */
int32_t tkv_hip_dev_dequantize_int8(int64_t ctx, const int8_t* q, int64_t rows, int64_t cols,
                                    float scale, const float* scales, float* y);
/* quantize_fp8_e4m3: raw e4m3 bytes (the reference's code + 128).
 * matmul.tkv:60-66 */
int32_t tkv_hip_dev_quantize_fp8_e4m3(int64_t ctx, const float* x, int64_t n, uint8_t* q);
/* Extension for per-tensor-scaled FP8 (not in the reference): bytes of
 * encode(fl32(x * fl32(1 / scale))), scale read from params. */
int32_t tkv_hip_dev_quantize_fp8_e4m3_scaled(int64_t ctx, const float* x, int64_t n,
                                             const tkv_hip_qparams_dev* params, uint8_t* q);
/* Extension: per-tensor FP8 activation quantize (not in the reference):
 * params.scale = fl32(max|x| / 240) (floor 1e-8), then the scaled encode
 * above.  240 is the largest value the reference encoder reaches before its
 * >= 248 saturation step. */
int32_t tkv_hip_dev_quantize_fp8_e4m3_dynamic_tensor(int64_t ctx, const float* x, int64_t n,
                                                     uint8_t* q, tkv_hip_qparams_dev* params);
/* dequantize_fp8_e4m3 (reference decoder).  matmul.tkv:68-73 */
int32_t tkv_hip_dev_dequantize_fp8_e4m3(int64_t ctx, const uint8_t* q, int64_t n, float* y);

/* INT8 GEMM: A int8 [M,K] row-major, W int8 [N,K] row-major (both K-major,
 * matmul.tkv:22), INT32 accumulate, fused dequant epilogue, f32 Y [M,N].
 * Epilogue (matmul.tkv:14,28):
 *   scales_w != NULL: y = acc * sa * scales_w[n] + bias[n]   (per-channel)
 *   scales_w == NULL: y = acc * fl32(sa * scale_w) + bias[n] (symmetric)
 * sa = scale_a[m * scale_a_stride]: stride 0 per-tensor, 1 per-token (the
 * per-token form is an extension).  bias may be NULL. */
int32_t tkv_hip_dev_matmul_int8(int64_t ctx, const int8_t* a, const int8_t* w, int64_t m,
                                int64_t n, int64_t k, const float* scale_a,
                                int64_t scale_a_stride, float scale_w,
                                const float* scales_w, const float* bias, float* y,
                                int32_t recipe);
/* QLinearMatMul on device codes (session.tkv:1992-2071): a int8 [M,K], w int8
 * [N,K] (the node's B transposed: K-major, like every weight here), y int8
 * [M,N]; one GEMM with the zero-point corrections and the requantization
 * fused into its epilogue.  Same numerics and recipe switch as the mirror. */
int32_t tkv_hip_dev_qlinear_matmul(int64_t ctx, const int8_t* a, float sa, int32_t zpa,
                                   const int8_t* w, float sw, int32_t zpw, float sy, int32_t zpy,
                                   int8_t* y, int64_t m, int64_t n, int64_t k, int32_t recipe);
/* INT32 accumulators only (MatMulInteger core; exactness checks). */
int32_t tkv_hip_dev_matmul_int8_accum(int64_t ctx, const int8_t* a, const int8_t* w,
                                      int64_t m, int64_t n, int64_t k, int32_t* acc);
/* FP8 e4m3 GEMM: raw e4m3 bytes A [M,K], W [N,K]; y = fl32(acc + bias[n])
 * (matmul.tkv:46-58).  Products are the reference decoder's (decoded exactly
 * to f16, f16 MFMA), accumulated at f32-class precision.  With scale_a /
 * scales_w non-NULL the extension epilogue y = acc * sa * scales_w[n] + bias[n]. */
int32_t tkv_hip_dev_matmul_fp8_e4m3(int64_t ctx, const uint8_t* a, const uint8_t* w,
                                    int64_t m, int64_t n, int64_t k, const float* scale_a,
                                    int64_t scale_a_stride, const float* scales_w,
                                    const float* bias, float* y);
/* Same contract on the full-rate FP8 MFMA (v_mfma_scale_f32_32x32x64_f8f6f4):
 * hardware OCP e4m3 decode (subnormal codes read twice the reference's value)
 * and the MFMA's reduced-precision dot-product accumulation; outputs agree
 * with the reference within 2^-10 * sum_k |a_k w_k| per element. */
int32_t tkv_hip_dev_matmul_fp8_e4m3_fast(int64_t ctx, const uint8_t* a, const uint8_t* w,
                                         int64_t m, int64_t n, int64_t k, const float* scale_a,
                                         int64_t scale_a_stride, const float* scales_w,
                                         const float* bias, float* y);

/* ---- device-resident quantized weight (pack once, run many) ------------ */
/* Calibrates W f32 [N,K] (device pointer) per output channel and quantizes
 * it to int8 (format 0) or per-tensor-scaled e4m3 (format 1), keeping codes,
 * scales and an optional bias on the device.  Mirrors the offline
 * calibrate_per_channel_minmax + quantize_int8_per_channel steps of CS1. */
#define TKV_HIP_WEIGHT_INT8 0
#define TKV_HIP_WEIGHT_FP8 1      /* GEMM with the reference decoder's products */
#define TKV_HIP_WEIGHT_FP8_FAST 2 /* GEMM on the full-rate FP8 MFMA            */
int32_t tkv_hip_weight_create(int64_t ctx, const float* w, int64_t n, int64_t k,
                              const float* bias, int32_t format, int64_t* handle_out);
/* Pre-quantized int8 weight codes [N,K] + per-channel scales (device). */
int32_t tkv_hip_weight_create_int8(int64_t ctx, const int8_t* codes, const float* scales,
                                   int64_t n, int64_t k, const float* bias,
                                   int64_t* handle_out);
int32_t tkv_hip_weight_free(int64_t handle);
/* Read back the weight's codes / scales (device pointers owned by the handle).
 * *k is the codes' row stride (K rounded up to 128; rows are zero padded). */
int32_t tkv_hip_weight_info(int64_t handle, void** codes, float** scales, float** bias,
                            int64_t* n, int64_t* k, int32_t* format);
/* Quantized linear: y[M,N] = dequant(quant(x) . W^T) + bias.
 * act_mode 0: dynamic per-tensor activation scale (calibrate_minmax + R3);
 * act_mode 1: dynamic per-token scale (quantize_dynamic_int8_rowwise).
 * x, y are device pointers; the activation codes live in ctx workspace. */
#define TKV_HIP_ACT_PER_TENSOR 0
#define TKV_HIP_ACT_PER_TOKEN 1
int32_t tkv_hip_linear_forward(int64_t ctx, int64_t weight, const float* x, int64_t m,
                               int32_t act_mode, float* y);
/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): tkv_hip_linear_forward on the caller's stream (NULL:
 * the default stream) with every scratch buffer in one fixed area per GPU
 * inside the library's code object -- activation codes up to
 * TKV_HIP_STATIC_CODES_BYTES (m * k), per-token scales for up to 65536 rows,
 * calibration partials and per-call parameters.  It calls no hipMalloc,
 * hipFree or other allocating routine (the area is resolved once per device
 * on the first call).  INT8 weights only (FP8: TKV_HIP_UNSUPPORTED); larger
 * m * k or m: TKV_HIP_BAD_ARG.  Every call on a GPU shares that GPU's area,
 * which keeps the last call's contents: calls that overlap on one GPU (other
 * streams, other threads) race, so order them on one stream.  The weight's
 * device is made current for the call; the calling thread's current device
 * is restored before the call returns. */
#define TKV_HIP_STATIC_CODES_BYTES (32ll << 20)
int32_t tkv_hip_linear_forward_static(int64_t weight, const float* x, int64_t m,
                                      int32_t act_mode, float* y, void* stream);

/* ======================================================================== */
/* Grouped INT4 weights (tv/quantization/int4.tkv) and GGUF block formats   */
/* (tv/format/gguf.tkv).  Host mirrors carry the reference's lists: packed  */
/* codes as one int32 per byte (low nibble = even column), zero points as   */
/* int64; device variants take packed bytes [rows, cols / 2].               */
/* ======================================================================== */

/* quantize_int4_grouped(src, rows, cols, group_size, packed_out, scales_out)
 * int4.tkv:36-57: per (row, group) scale = fl32(max(max|x|, 1e-8) / 7), codes
 * clamp(round(x / scale), -8, 7) + 8, the pair (c, c + 1) coded with group
 * c / group_size; all n_packed entries are cleared first.  BAD_ARG where the
 * .tkv raises (cols % group_size, odd cols, short src / packed_out) and when
 * n_scales_out < rows * cols / group_size (the reference appends). */
int32_t tkv_hip_quantize_int4_grouped(const float* src, int64_t n_src, int64_t rows, int64_t cols,
                                      int64_t group_size, int32_t* packed_out, int64_t n_packed,
                                      float* scales_out, int64_t n_scales_out);
/* dequantize_int4_grouped(packed, dst, rows, cols, group_size, scales)
 * int4.tkv:60-73: dst = fl32((nibble - 8) * scale).  Odd cols: UNSUPPORTED. */
int32_t tkv_hip_dequantize_int4_grouped(const int32_t* packed, int64_t n_packed, float* dst,
                                        int64_t n_dst, int64_t rows, int64_t cols,
                                        int64_t group_size, const float* scales,
                                        int64_t n_scales);
/* quantize_int4_grouped_asym(src, rows, cols, group_size, packed_out,
 * scales_out, zps_out)   int4.tkv:77-157 (AWQ-style scale and zero point per
 * group, uint4 codes 0..15). */
int32_t tkv_hip_quantize_int4_grouped_asym(const float* src, int64_t n_src, int64_t rows,
                                           int64_t cols, int64_t group_size, int32_t* packed_out,
                                           int64_t n_packed, float* scales_out, int64_t* zps_out,
                                           int64_t n_groups_out);
/* dequantize_int4_grouped_asym(packed, dst, rows, cols, group_size, scales, zps)
 * int4.tkv:160-170: dst = fl32((nibble - zp) * scale). */
int32_t tkv_hip_dequantize_int4_grouped_asym(const int32_t* packed, int64_t n_packed, float* dst,
                                             int64_t n_dst, int64_t rows, int64_t cols,
                                             int64_t group_size, const float* scales,
                                             const int64_t* zps, int64_t n_groups);
/* permute_cols(src, rows, cols, perm) / inv_permute_cols   int4.tkv:175-192:
 * out[r, c] = src[r, perm[c]] (inverse: out[r, perm[c]] = src[r, c]).
 * BAD_ARG for len(perm) != cols and entries outside [0, cols); the inverse
 * of a non-permutation (ordered overwrites) is UNSUPPORTED. */
int32_t tkv_hip_permute_cols(const float* src, int64_t n_src, int64_t rows, int64_t cols,
                             const int64_t* perm, int64_t n_perm, float* out, int64_t n_out);
int32_t tkv_hip_inv_permute_cols(const float* src, int64_t n_src, int64_t rows, int64_t cols,
                                 const int64_t* perm, int64_t n_perm, float* out, int64_t n_out);
/* matmul_int4_grouped(pa, packed_w, pbias, py, m, n, k, group_size, scales_w)
 * int4.tkv:218-239: y = fl32(sum_k a * ((nibble - 8) * scale[n, k / gs]) +
 * bias) with f64 accumulation (exact products; only the order of the f64
 * additions differs from the reference's loop).  BAD_ARG when scales_w is
 * short (int4.tkv:220-221); odd K or K not a multiple of group_size:
 * UNSUPPORTED. */
int32_t tkv_hip_matmul_int4_grouped(const float* pa, int64_t n_a, const int32_t* packed_w,
                                    int64_t n_packed, const float* pbias, int64_t n_bias,
                                    float* py, int64_t n_y, int64_t m, int64_t n, int64_t k,
                                    int64_t group_size, const float* scales_w, int64_t n_scales);
/* matmul_int4_grouped_ordered(..., perm)   int4.tkv:195-215 (GPTQ act-order:
 * activation column perm[k] meets weight column k; entries outside [0, K)
 * are UNSUPPORTED). */
int32_t tkv_hip_matmul_int4_grouped_ordered(const float* pa, int64_t n_a, const int32_t* packed_w,
                                            int64_t n_packed, const float* pbias, int64_t n_bias,
                                            float* py, int64_t n_y, int64_t m, int64_t n,
                                            int64_t k, int64_t group_size, const float* scales_w,
                                            int64_t n_scales, const int64_t* perm,
                                            int64_t n_perm);
/* _dequant_tensor for GGUF dtype 8 (Q8_0), 2 (Q4_0), 3 (Q4_1)
 * gguf.tkv:284-313: n / 32 blocks of raw (34 / 18 / 20 bytes), elements past
 * the last whole block 0.  Other dtypes: UNSUPPORTED. */
#define TKV_HIP_GGUF_Q4_0 2
#define TKV_HIP_GGUF_Q4_1 3
#define TKV_HIP_GGUF_Q8_0 8
int32_t tkv_hip_dequantize_gguf(const uint8_t* raw, int64_t n_raw, int64_t n, int32_t dtype,
                                float* out, int64_t n_out);

/* Device-pointer variants (asynchronous on the context's stream).  packed:
 * bytes [rows, cols / 2]; zps NULL selects the symmetric form. */
int32_t tkv_hip_dev_quantize_int4_grouped(int64_t ctx, const float* src, int64_t rows,
                                          int64_t cols, int64_t group_size, uint8_t* packed,
                                          float* scales, int64_t* zps);
int32_t tkv_hip_dev_dequantize_int4_grouped(int64_t ctx, const uint8_t* packed, int64_t rows,
                                            int64_t cols, int64_t group_size, const float* scales,
                                            const int64_t* zps, float* dst);
int32_t tkv_hip_dev_permute_cols(int64_t ctx, const float* src, int64_t rows, int64_t cols,
                                 const int64_t* perm, int32_t inverse, float* out);
/* a f32 [M, K], packed_w bytes [N, K / 2], scales_w f32 [N, K / group_size],
 * bias and perm may be NULL (perm entries outside [0, K) read 0). */
int32_t tkv_hip_dev_matmul_int4_grouped(int64_t ctx, const float* a, const uint8_t* packed_w,
                                        const float* scales_w, const float* bias,
                                        const int64_t* perm, float* y, int64_t m, int64_t n,
                                        int64_t k, int64_t group_size);
int32_t tkv_hip_dev_dequantize_gguf(int64_t ctx, const uint8_t* raw, int64_t n, int32_t dtype,
                                    float* out);

/* ---- GGUF Q8_0 weights on the INT8 GEMM (extension) ------------------- */
/* No counterpart in the reference, which decodes Q8_0 blocks to f32
 * (_dequant_tensor, gguf.tkv:284-290) before any matmul.  A Q8_0 weight
 * [N, K] (N rows of K / 32 blocks of 34 bytes: f16 d, 32 int8 q) becomes
 * int8 codes [N, K] and f32 group scales [N, K / 32], and multiplies the
 * int8 codes a [M, K] of an activation whose scale is sa:
 *   dot_g = sum over block g's 32 k of a[m, k] q[n, k]          (exact)
 *   acc   = 0;  acc = fmaf((float)dot_g, d[n, g], acc)   g = 0, 1, ... in order
 *   y     = fl32(fl64(fl64(acc) * sa) + bias[n])              (bias 0 if NULL)
 * Against the reference's decode-then-multiply of the float activation x,
 * the int8 activation codes contribute at most (sa / 2) sum_k |d q[n, k]|
 * per output, and the f32 chain one rounding per group. */
#define TKV_HIP_WEIGHT_Q8_0 3
/* Weight handle from raw Q8_0 blocks (device bytes, row-major) for
 * tkv_hip_linear_forward: either act_mode, the activation quantized as for
 * INT8 weights (K % 128 == 0 there; per-token decode batches, M <= 32, run
 * one kernel with K % 64 == 0, K <= 3072, same results).  K % 32 != 0:
 * BAD_ARG.
 * tkv_hip_weight_info returns the group scales [N, k / 32] as `scales`
 * (k = the codes' padded row stride). */
int32_t tkv_hip_weight_create_gguf_q8_0(int64_t ctx, const uint8_t* raw, int64_t n, int64_t k,
                                        const float* bias, int64_t* handle_out);
/* The GEMM on device buffers: a int8 [M, K], codes int8 [N, K], group_scales
 * f32 [N, K / 32] (each 16-byte aligned), sa = scale_a[m * scale_a_stride]
 * (stride 0: per tensor, 1: per token).  K not a positive multiple of 128:
 * UNSUPPORTED. */
int32_t tkv_hip_dev_matmul_q8_0(int64_t ctx, const int8_t* a, const int8_t* codes,
                                const float* group_scales, int64_t m, int64_t n, int64_t k,
                                const float* scale_a, int64_t scale_a_stride, const float* bias,
                                float* y);

#ifdef __cplusplus
}
#endif
#endif
