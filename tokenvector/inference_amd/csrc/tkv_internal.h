// tkv_internal.h -- shared host/device internals of libtkv_hip (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstddef>
#include <string>
#include <vector>

#include "../../../include/tkv_hip.h"

namespace tkv {

// ---------------------------------------------------------------------------
// Errors: one message per calling thread, rc codes from tkv_hip.h.
// ---------------------------------------------------------------------------
int set_error(int rc, const std::string& msg);
int fail_hip(hipError_t e, const char* what, const char* file, int line);

#define TKV_HIP_TRY(expr)                                                  \
    do {                                                                   \
        hipError_t _tkv_e = (expr);                                        \
        if (_tkv_e != hipSuccess)                                          \
            return ::tkv::fail_hip(_tkv_e, #expr, __FILE__, __LINE__);     \
    } while (0)

#define TKV_RC_TRY(expr)              \
    do {                              \
        int _tkv_rc = (expr);         \
        if (_tkv_rc != TKV_HIP_OK)    \
            return _tkv_rc;           \
    } while (0)

#define TKV_LAUNCH_CHECK() TKV_HIP_TRY(hipGetLastError())

// ---------------------------------------------------------------------------
// Context: device, stream, grow-only workspaces.  A context is driven by one
// thread at a time; the default context of each thread is thread_local.
// ---------------------------------------------------------------------------
constexpr int kMaxReduceBlocks = 2048;
// Column blocks (32 columns each) of the split-K skinny GEMM's partial sums.
constexpr int kGemvSplitBlocks = 128;
// Workgroups of a grid-barrier kernel (one per CU) plus its result word.
constexpr int kMaxGridSlots = 1024;
// Arrival counts of the calibration kernels whose last workgroup finishes
// the call: 0 calibrate_minmax, 1 KL candidates, 2 radix passes, 3 MSE sums.
constexpr int kCalCounters = 4;
constexpr int64_t kCalHistBins = 4096;  // the largest KL histogram

struct Graph;

struct RedPartial {
    float mn;
    float mx;
    unsigned long long zidx;  // first index holding a zero (either sign)
};

struct Ctx {
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    int num_cus = 256;
    size_t max_lds = 65536;  // LDS bytes a workgroup may use (static + dynamic)
    // reduction scratch: kMaxReduceBlocks per-block partials (written by the
    // partials kernel, read by the finalize kernel; no clearing needed)
    RedPartial* partials = nullptr;
    tkv_hip_qparams_dev* params = nullptr;  // 64 slots of per-call params
    // Split-K skinny GEMM: kGemvSplitBlocks x 1024 INT32 partial sums and
    // kGemvSplitBlocks arrival counts, zeroed at creation and cleared again
    // by the kernel that uses them.
    int32_t* gemv_part = nullptr;
    unsigned* gemv_arrivals = nullptr;
    // Grid-barrier slots of the single-pass calibrate + quantize kernel: one
    // 64-bit word per workgroup and the result word (the last of
    // kMaxGridSlots), zero at creation; every launch advances each slot it
    // uses, and the result word, by one generation.
    unsigned long long* grid_slots = nullptr;
    // Calibration histogram (kCalHistBins 64-bit counts) and kCalCounters
    // arrival counts: zero at creation, and every calibration call that uses
    // them leaves them zero (its last workgroup clears what it used).
    // Contexts that do not run the calibrators leave them null.
    unsigned long long* cal_hist = nullptr;
    unsigned* cal_arrivals = nullptr;
    // grow-only workspaces
    static constexpr int kSlots = 13;  // 10, 11: f16-decoded FP8 operands; 12: INT4 split-K partials (either kernel)
    void* ws[kSlots] = {};
    size_t ws_bytes[kSlots] = {};
    bool capturing = false;  // between capture_begin and capture_end
    // Graphs captured on this context and not yet destroyed.  They replay
    // the workspace addresses they captured, so while any is alive a slot
    // that grows keeps its old buffer here (freed with the last graph, or
    // with the context) instead of freeing it.  Destroying the context
    // first releases every live graph's executable and detaches the graph
    // handles, which stay valid for graph_destroy (see runtime.hip).
    std::vector<Graph*> graphs;
    std::vector<void*> retired;
    // A context over caller-fixed memory (the static-scratch entry point):
    // its workspaces never grow; a call that would need more fails.
    bool no_alloc = false;
    // Tuning overrides (TKV_HIP_TUNE_*), -1 = automatic.
    int64_t tune[TKV_HIP_TUNE_COUNT] = {-1, -1, -1, -1, -1, -1, -1};
};

// The override of `knob` on context c, or -1 (automatic).
inline int64_t tuned(const Ctx* c, int knob) { return c->tune[knob]; }

int ctx_create(int device, Ctx** out);
int ctx_destroy(Ctx* c);
// ctx handle 0 -> calling thread's default context (device from
// TKV_HIP_DEVICE, default 0).
int ctx_get(int64_t handle, Ctx** out);
// Device workspace slot `slot` of at least `bytes` (contents undefined).
// Refuses to grow while the context's stream is being captured.
int ctx_workspace(Ctx* c, int slot, size_t bytes, void** out);
// Byte fill of [dst, dst + bytes) on the context's stream (a kernel).
int launch_fill(Ctx* c, void* dst, int value, int64_t bytes);
// Environment gate: TKV_QUANT_HIP=0 turns every host mirror into a
// TKV_HIP_UNSUPPORTED return so .tkv callers keep their own loops.
bool hip_path_enabled();

// ---------------------------------------------------------------------------
// Launch helpers
// ---------------------------------------------------------------------------
inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Kernel-family launchers (implemented in the .hip files).
// quant.hip
int launch_minmax_tensor(Ctx* c, const float* x, int64_t n, int mode, int recipe,
                         tkv_hip_qparams_dev* out);
// calib.hip: calibrate_kl / _percentile / _mse (engine.tkv:42-197) into *out.
constexpr int64_t kMaxKlBins = 4096;
constexpr int64_t kMaxMseCandidates = 4096;
int launch_calibrate_kl(Ctx* c, const float* x, int64_t n, int64_t num_bins, int64_t target_bins,
                        tkv_hip_qparams_dev* out);
int launch_calibrate_percentile(Ctx* c, const float* x, int64_t n, float percentile,
                                int symmetric, tkv_hip_qparams_dev* out);
int launch_calibrate_mse(Ctx* c, const float* x, int64_t n, int64_t num_candidates,
                         tkv_hip_qparams_dev* out);
// Per-block min / max (+ first zero when track_zero) partials of x into
// c->partials; *nparts = their count (reduced by reduce_partials, tkv_reduce.h).
int launch_partials(Ctx* c, const float* x, int64_t n, int track_zero, int64_t* nparts);
enum MinMaxMode { MM_SYMMETRIC = 0, MM_ASYMMETRIC = 1, MM_DYNAMIC_QL = 2, MM_FP8 = 3 };
// FP8 scaling target: amax maps to 240, the largest e4m3 value the
// reference encoder reaches without its >= 248 saturation step.
constexpr float kFp8Target = 240.0f;
int launch_quant_i8_tensor(Ctx* c, const float* x, int64_t n, const tkv_hip_qparams_dev* p,
                           void* q, bool out_i32);
// calibrate_minmax(x, 1) + quantize_int8_symmetric in two kernels; *p = QuantParams.
int launch_quant_i8_dynamic(Ctx* c, const float* x, int64_t n, int recipe,
                            tkv_hip_qparams_dev* p, void* q, bool out_i32);
// Per-tensor FP8 scale (MM_FP8) + scaled e4m3 encode; *p = QuantParams.
int launch_quant_fp8_dynamic(Ctx* c, const float* x, int64_t n, tkv_hip_qparams_dev* p,
                             void* q, bool out_i32);
// The same, writing each code's exact reference decode as f16 (pre-scaled by
// 2^-8, 2 bytes per element, 8-byte aligned h16) instead of the code.
int launch_quant_fp8_dynamic_f16(Ctx* c, const float* x, int64_t n, tkv_hip_qparams_dev* p,
                                 void* h16);
int launch_quant_rows(Ctx* c, const float* x, int64_t rows, int64_t cols, int mode,
                      const float* scales_in, void* q, bool out_i32, float* scales_out,
                      tkv_hip_qparams_dev* row_params, int symmetric);
enum RowMode { RM_DYNAMIC = 0, RM_PER_CHANNEL = 1, RM_CALIBRATE = 2, RM_CALIBRATE_FULL = 3 };
int launch_dequant_i8(Ctx* c, const void* q, bool in_i32, int64_t rows, int64_t cols,
                      float scale, const float* scales, float* y);
int launch_fp8_encode(Ctx* c, const float* x, int64_t n, const tkv_hip_qparams_dev* scaled,
                      void* q, bool out_i32);
int launch_fp8_decode(Ctx* c, const void* q, bool in_i32, int64_t n, float* y);
int launch_i32_to_i8(Ctx* c, const int32_t* src, int64_t rows, int64_t cols, int64_t ld_src,
                     int8_t* dst, int64_t ld_dst, int code_bias);
int launch_i8_to_i32(Ctx* c, const int8_t* src, int64_t n, int32_t* dst, int code_bias);
int launch_i32_to_i8_transpose(Ctx* c, const int32_t* src, int64_t rows, int64_t cols,
                               int8_t* dst, int64_t ld_dst);
// qdq.hip
int launch_quantize_linear(Ctx* c, const float* x, int64_t nx, const float* scales,
                           int64_t n_scales, int64_t zp, int64_t dim, int64_t inner,
                           int32_t* y);
int launch_dequantize_linear(Ctx* c, const int32_t* x, int64_t nx, const float* scales,
                             int64_t n_scales, int64_t zp, int64_t dim, int64_t inner,
                             float* y);
int launch_dynamic_ql(Ctx* c, const float* x, int64_t nx, const tkv_hip_qparams_dev* p,
                      int32_t* y);
// gemm.hip
struct I8Epilogue {
    int mode;                  // EPI_* below
    int recipe;                // TKV_HIP_RECIPE_*
    const float* scale_a;      // device, indexed by m * scale_a_stride
    int64_t scale_a_stride;
    float scale_w;             // symmetric weight scale
    const float* scales_w;     // device [N] (per-channel) or null
    const float* bias;         // device [N] or null
    // K of the caller's product when the operands arrive already zero padded
    // to a longer row stride (0: the stride is K); bounds |acc| < 2^31.
    int64_t k_logical = 0;
};
enum { EPI_PER_CHANNEL = 0, EPI_SYMMETRIC = 1, EPI_ACCUM_I32 = 2 };
int launch_gemm_i8(Ctx* c, const int8_t* a, const int8_t* w, int64_t m, int64_t n, int64_t k,
                   const I8Epilogue& ep, void* y);
// fast: full-rate FP8 MFMA (hardware OCP decode and rounding); otherwise the
// reference decoder's products on f16 MFMA.
int launch_gemm_f8(Ctx* c, const uint8_t* a, const uint8_t* w, int64_t m, int64_t n,
                   int64_t k, const float* scale_a, int64_t scale_a_stride,
                   const float* scales_w, const float* bias, float* y, bool fast);
// The reference e4m3 decode of `bytes` codes (a multiple of 16) into halves
// (exact, pre-scaled by 2^-8) at dst, on c's stream.
int launch_fp8_ref_to_f16(Ctx* c, const uint8_t* src, int64_t bytes, void* dst);
// The reference-products FP8 GEMM on operands already decoded that way:
// a16 [m, k] and w16 [n, k] halves, k a multiple of the GEMM K step, rows
// 16-byte aligned; per-tensor scale_a, per-channel scales_w, bias optional.
int launch_gemm_f8_decoded(Ctx* c, const void* a16, const void* w16, int64_t m, int64_t n,
                           int64_t k, const float* scale_a, const float* scales_w,
                           const float* bias, float* y);
// QLinearMatMul (session.tkv:1992-2071) on packed codes: A [m,k], W [n,k]
// (the node's B transposed), both with row stride k; y int8 [m,n].
struct QLinearParams {
    int32_t zpa, zpw, zpy;
    double mult;  // fl64(sa * sw / sy) (primary) or the f32 chain widened
};
int launch_gemm_qlinear(Ctx* c, const int8_t* a, const int8_t* w, int64_t m, int64_t n,
                        int64_t k, const QLinearParams& q, int8_t* y);
// Sums of each row's `cols` int8 codes: out_a[r] for the rows of A
// [rows_a, cols], out_w[r] for the rows of W [rows_w, cols] (both compact).
int launch_row_sums_i8(Ctx* c, const int8_t* a, int64_t rows_a, const int8_t* w, int64_t rows_w,
                       int64_t cols, int32_t* out_a, int32_t* out_w);

// Grouped INT4 (int4.hip).  packed: bytes, or int32 per byte (out32 / in32,
// the reference's list format); zps NULL selects the symmetric form.
int launch_int4_quantize(Ctx* c, const float* src, int64_t rows, int64_t cols, int64_t gs,
                         bool asym, void* packed, bool out32, float* scales, int64_t* zps);
int launch_int4_dequantize(Ctx* c, const void* packed, bool in32, int64_t rows, int64_t cols,
                           int64_t gs, const float* scales, const int64_t* zps, float* dst);
int launch_permute_cols(Ctx* c, const float* src, int64_t rows, int64_t cols, const int64_t* perm,
                        bool inverse, float* out);
// y[m, n] = fl32(sum_k a[m, perm[k]] * w[n, k] + bias[n]) in f64; K even,
// a multiple of gs (perm, bias may be NULL).
int launch_matmul_int4(Ctx* c, const float* a, const uint8_t* wp, const float* scales,
                       const float* bias, const int64_t* perm, float* y, int64_t m, int64_t n,
                       int64_t k, int64_t gs);
// GGUF block decoding, dtype 8 (Q8_0), 2 (Q4_0) or 3 (Q4_1); bytes per
// 32-element block (0 for any other dtype).
int launch_gguf_blocks(Ctx* c, const uint8_t* raw, int64_t n, int dtype, float* out);
int64_t gguf_block_bytes(int dtype);
// decode.hip: the per-token W8A8 linear of decode batches in one kernel
// (M <= 32, K % 64 == 0, K <= 3072, x 16-byte aligned; UNSUPPORTED
// otherwise, with nothing launched): rowwise absmax + int8 quantize of x,
// INT8 GEMM against W [n, ldk], y = fl32(fl64(fl64(acc * sa[m]) * sw[n]) + b[n]).
int launch_decode_i8(Ctx* c, const float* x, int64_t m, int64_t k, const uint8_t* w, int64_t ldk,
                     int64_t n, const float* scales_w, const float* bias, float* y);
// The same for GGUF Q8_0 weights (extension): codes w [n, ldk], group
// scales gs [n, ldk / 32], the Q8_0 GEMM's recipe (one fma per 32-element
// group, in order); ldk % 128 == 0.  UNSUPPORTED as above, with nothing
// launched.
int launch_decode_q8(Ctx* c, const float* x, int64_t m, int64_t k, const uint8_t* w,
                     const float* gs, int64_t ldk, int64_t n, const float* bias, float* y);
// gemm_q8.hip: GGUF Q8_0 weights on the INT8 MFMA (extension).
// Unpack n rows of k / 32 raw blocks (34 bytes) into codes [n, ldk] (16-byte
// aligned, padding left as it is) and group scales gs [n, ldk / 32] (padding
// groups 0).  k % 32 != 0, ldk % 128 != 0: UNSUPPORTED.
int launch_q8_0_unpack(Ctx* c, const uint8_t* raw, int64_t n, int64_t k, int64_t ldk,
                       uint8_t* codes, float* gs);
// y[m, n] = fl32(fl64(fl64(acc) * sa) + b[n]), acc the fma chain over the
// groups of fl32(dot_g) * gs[n, g]; a [m, ldk], w [n, ldk] int8 codes,
// sa = scale_a[m * scale_a_stride] (stride 0 or 1).  ldk % 128 != 0 or
// unaligned operands: UNSUPPORTED, nothing launched.
int launch_gemm_q8(Ctx* c, const int8_t* a, const int8_t* w, const float* gs, int64_t m,
                   int64_t n, int64_t ldk, const float* scale_a, int64_t scale_a_stride,
                   const float* bias, float* y);
// K granularity of the GEMM main loop: operands whose row stride is a
// multiple of it (and 16-byte aligned) run without repacking.
int64_t gemm_k_align();

}  // namespace tkv
