// runtime.hip -- contexts, errors, device memory and events of libtkv_hip.
//
// No reference counterpart: this is the plumbing the reference's native
// DLLs keep implicit (stream, workspace, error text).  State lives in
// explicit contexts; the only process-wide values are read-only after first
// use (the environment gate) or per-thread (last error, default context).
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <string>

#include "tkv_internal.h"

namespace tkv {

static thread_local std::string t_last_error;

int set_error(int rc, const std::string& msg) {
    t_last_error = msg;
    return rc;
}

int fail_hip(hipError_t e, const char* what, const char* file, int line) {
    char buf[512];
    snprintf(buf, sizeof(buf), "%s failed: %s (%s:%d)", what, hipGetErrorString(e), file, line);
    int rc = (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) ? TKV_HIP_OOM
                                                                          : TKV_HIP_DEVICE_ERROR;
    if (e == hipErrorNoDevice || e == hipErrorInvalidDevice) rc = TKV_HIP_NO_DEVICE;
    return set_error(rc, buf);
}

bool hip_path_enabled() {
    static const bool enabled = [] {
        const char* v = getenv("TKV_QUANT_HIP");
        return !(v && v[0] == '0' && v[1] == '\0');
    }();
    return enabled;
}

static int check_device(int device, int* num_cus, size_t* max_lds = nullptr) {
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0)
        return set_error(TKV_HIP_NO_DEVICE, "no HIP device visible");
    if (device < 0 || device >= count)
        return set_error(TKV_HIP_NO_DEVICE, "device index out of range");
    hipDeviceProp_t prop;
    TKV_HIP_TRY(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return set_error(TKV_HIP_NO_DEVICE,
                         std::string("libtkv_hip is built for gfx950, device is ") + prop.gcnArchName);
    *num_cus = prop.multiProcessorCount;
    if (max_lds) *max_lds = prop.sharedMemPerBlock;
    return TKV_HIP_OK;
}

int ctx_create(int device, Ctx** out) {
    int cus = 0;
    size_t lds = 0;
    TKV_RC_TRY(check_device(device, &cus, &lds));
    TKV_HIP_TRY(hipSetDevice(device));
    Ctx* c = new Ctx();
    c->device = device;
    c->num_cus = cus;
    if (lds) c->max_lds = lds;
    hipError_t e = hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete c;
        return fail_hip(e, "hipStreamCreateWithFlags", __FILE__, __LINE__);
    }
    c->stream = c->own_stream;
    const size_t gemv_bytes = (size_t)kGemvSplitBlocks * 1024 * sizeof(int32_t);
    size_t red_bytes = sizeof(RedPartial) * kMaxReduceBlocks + 256 + sizeof(tkv_hip_qparams_dev) * 64 +
                       256 + gemv_bytes + (size_t)kGemvSplitBlocks * sizeof(unsigned) + 256 +
                       (size_t)kMaxGridSlots * 8 + (size_t)kCalHistBins * 8 +
                       (size_t)kCalCounters * sizeof(unsigned);
    void* red = nullptr;
    e = hipMalloc(&red, red_bytes);
    if (e != hipSuccess) {
        (void)hipStreamDestroy(c->own_stream);
        delete c;
        return fail_hip(e, "hipMalloc(reduction scratch)", __FILE__, __LINE__);
    }
    c->partials = static_cast<RedPartial*>(red);
    c->params = reinterpret_cast<tkv_hip_qparams_dev*>(static_cast<char*>(red) +
                                                       sizeof(RedPartial) * kMaxReduceBlocks + 256);
    c->gemv_part = reinterpret_cast<int32_t*>(reinterpret_cast<char*>(c->params + 64) + 256);
    c->gemv_arrivals = reinterpret_cast<unsigned*>(reinterpret_cast<char*>(c->gemv_part) + gemv_bytes);
    {   // next 256-byte boundary past the arrival counts
        const uintptr_t end = reinterpret_cast<uintptr_t>(c->gemv_arrivals + kGemvSplitBlocks);
        c->grid_slots = reinterpret_cast<unsigned long long*>((end + 255) & ~uintptr_t(255));
    }
    c->cal_hist = c->grid_slots + kMaxGridSlots;
    c->cal_arrivals = reinterpret_cast<unsigned*>(c->cal_hist + kCalHistBins);
    // One-time zeroing at creation, so params read before any calibration
    // are defined (never inside a caller's stream capture).
    e = hipMemset(red, 0, red_bytes);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        (void)hipFree(red);
        (void)hipStreamDestroy(c->own_stream);
        delete c;
        return fail_hip(e, "hipMemset(reduction scratch)", __FILE__, __LINE__);
    }
    *out = c;
    return TKV_HIP_OK;
}

// A captured graph and the context whose workspaces it replays (null once
// that context has been destroyed: the graph is then detached, its
// executable released, and only the handle itself is left to free).
struct Graph {
    hipGraphExec_t exec = nullptr;
    Ctx* ctx = nullptr;
};

int ctx_destroy(Ctx* c) {
    if (!c) return TKV_HIP_OK;
    // Teardown: errors here leave nothing the caller can act on.
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    // Graphs still alive replay this context's workspaces: release their
    // executables now and detach the handles, so that a later graph_destroy
    // frees only the handle and never touches the freed context.
    for (Graph* g : c->graphs) {
        if (g->exec) (void)hipGraphExecDestroy(g->exec);
        g->exec = nullptr;
        g->ctx = nullptr;
    }
    c->graphs.clear();
    for (int i = 0; i < Ctx::kSlots; i++)
        if (c->ws[i]) (void)hipFree(c->ws[i]);
    for (void* p : c->retired) (void)hipFree(p);
    if (c->partials) (void)hipFree(c->partials);
    if (c->own_stream) (void)hipStreamDestroy(c->own_stream);
    delete c;
    return TKV_HIP_OK;
}

// Default contexts are per thread and intentionally never destroyed: HIP's
// own teardown at process exit may run before thread_local destructors.
static thread_local Ctx* t_default_ctx = nullptr;

int ctx_get(int64_t handle, Ctx** out) {
    if (handle != 0) {
        *out = reinterpret_cast<Ctx*>(handle);
        TKV_HIP_TRY(hipSetDevice((*out)->device));
        return TKV_HIP_OK;
    }
    if (!t_default_ctx) {
        int dev = 0;
        if (const char* v = getenv("TKV_HIP_DEVICE")) dev = atoi(v);
        TKV_RC_TRY(ctx_create(dev, &t_default_ctx));
    }
    *out = t_default_ctx;
    TKV_HIP_TRY(hipSetDevice(t_default_ctx->device));
    return TKV_HIP_OK;
}

int ctx_workspace(Ctx* c, int slot, size_t bytes, void** out) {
    if (bytes == 0) bytes = 256;
    if (c->ws_bytes[slot] < bytes && c->no_alloc)
        return set_error(TKV_HIP_BAD_ARG, "workspace slot " + std::to_string(slot) + " needs " +
                                              std::to_string(bytes) +
                                              " bytes, beyond this call's fixed scratch");
    if (c->ws_bytes[slot] < bytes) {
        // growing synchronizes the stream and reallocates: not capturable
        if (c->capturing)
            return set_error(TKV_HIP_BAD_ARG,
                             "workspace slot " + std::to_string(slot) +
                                 " would grow inside a stream capture: make the same calls "
                                 "once before capturing");
        if (c->ws[slot]) {
            if (!c->graphs.empty()) {
                // a live graph may replay into the old buffer: keep it
                c->retired.push_back(c->ws[slot]);
            } else {
                TKV_HIP_TRY(hipStreamSynchronize(c->stream));
                TKV_HIP_TRY(hipFree(c->ws[slot]));
            }
            c->ws[slot] = nullptr;
            c->ws_bytes[slot] = 0;
        }
        size_t sz = (bytes + 0xFFFFF) & ~size_t(0xFFFFF);
        TKV_HIP_TRY(hipMalloc(&c->ws[slot], sz));
        c->ws_bytes[slot] = sz;
    }
    *out = c->ws[slot];
    return TKV_HIP_OK;
}

// Plain streaming copy: 16 B per lane, grid-stride.  It reads and writes
// exactly `n16 * 16` bytes each, which makes it the known-size yardstick that
// HBM counters (FETCH_SIZE / WRITE_SIZE) are scaled against.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(256) k_copy16(const u32x4* __restrict__ src,
                                               u32x4* __restrict__ dst, int64_t n16) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
        __builtin_nontemporal_store(__builtin_nontemporal_load(&src[i]), &dst[i]);
}

// Byte fill: 16 B per lane over the 16-byte aligned middle, bytes at the
// ragged ends.  A kernel rather than hipMemsetAsync, so that a captured stream
// records a kernel node.
__global__ void __launch_bounds__(256) k_fill(uint8_t* __restrict__ dst, int64_t head,
                                              int64_t n16, int64_t bytes, uint32_t word) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    u32x4* __restrict__ d16 = reinterpret_cast<u32x4*>(dst + head);
    const u32x4 v = {word, word, word, word};
    for (int64_t i = t; i < n16; i += stride) d16[i] = v;
    const int64_t tail0 = head + 16 * n16;
    for (int64_t i = t; i < head + (bytes - tail0); i += stride) {
        const int64_t j = i < head ? i : tail0 + (i - head);
        dst[j] = (uint8_t)word;
    }
}

int launch_fill(Ctx* c, void* dst, int value, int64_t bytes) {
    if (bytes <= 0) return TKV_HIP_OK;
    const uintptr_t p = reinterpret_cast<uintptr_t>(dst);
    int64_t head = (int64_t)((16 - (p & 15)) & 15);
    if (head > bytes) head = bytes;
    const int64_t n16 = (bytes - head) / 16;
    const int64_t work = n16 > 0 ? n16 : 1;
    const unsigned grid = (unsigned)std::min<int64_t>((work + 255) / 256, (int64_t)c->num_cus * 8);
    const uint32_t b = (uint8_t)value;
    k_fill<<<grid, 256, 0, c->stream>>>(static_cast<uint8_t*>(dst), head, n16, bytes,
                                         b * 0x01010101u);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

}  // namespace tkv

using namespace tkv;

extern "C" {

int32_t tkv_hip_version(void) { return 100; }

int32_t tkv_hip_device_count(void) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess) return 0;
    int n = 0;
    for (int i = 0; i < count; i++) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, i) == hipSuccess &&
            strncmp(prop.gcnArchName, "gfx950", 6) == 0)
            n++;
    }
    return n;
}

int32_t tkv_hip_last_error(char* buf, int32_t len) {
    const std::string& s = t_last_error;
    if (buf && len > 0) {
        size_t n = s.size() < (size_t)(len - 1) ? s.size() : (size_t)(len - 1);
        memcpy(buf, s.data(), n);
        buf[n] = '\0';
    }
    return (int32_t)s.size();
}

int32_t tkv_hip_ctx_create(int32_t device, int64_t* ctx_out) {
    if (!ctx_out) return set_error(TKV_HIP_BAD_ARG, "ctx_out is NULL");
    Ctx* c = nullptr;
    TKV_RC_TRY(ctx_create(device, &c));
    *ctx_out = reinterpret_cast<int64_t>(c);
    return TKV_HIP_OK;
}

int32_t tkv_hip_ctx_destroy(int64_t ctx) {
    if (ctx == 0) return TKV_HIP_OK;
    return ctx_destroy(reinterpret_cast<Ctx*>(ctx));
}

int32_t tkv_hip_ctx_set_stream(int64_t ctx, void* stream) {
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    if (c->capturing) return set_error(TKV_HIP_BAD_ARG, "set_stream: context is capturing");
    hipStream_t next = stream ? static_cast<hipStream_t>(stream) : c->own_stream;
    // Work already queued on the previous stream shares this context's
    // workspaces and split-K buffers with what the next stream will run:
    // drain it so the two never overlap.
    if (next != c->stream) TKV_HIP_TRY(hipStreamSynchronize(c->stream));
    c->stream = next;
    return TKV_HIP_OK;
}

int32_t tkv_hip_ctx_get_stream(int64_t ctx, void** stream_out) {
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    *stream_out = c->stream;
    return TKV_HIP_OK;
}

int32_t tkv_hip_ctx_set_tuning(int64_t ctx, int32_t knob, int64_t value) {
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    static const int64_t hi[TKV_HIP_TUNE_COUNT] = {11, 8, 16, 1, 1, 1 << 20, 1};
    static const int64_t lo[TKV_HIP_TUNE_COUNT] = {0, 0, 1, 0, 0, 0, 0};
    if (knob < 0 || knob >= TKV_HIP_TUNE_COUNT)
        return set_error(TKV_HIP_BAD_ARG, "set_tuning: unknown knob " + std::to_string(knob));
    if (value != -1 && (value < lo[knob] || value > hi[knob]))
        return set_error(TKV_HIP_BAD_ARG, "set_tuning: value " + std::to_string(value) +
                                              " outside knob " + std::to_string(knob) +
                                              "'s range [" + std::to_string(lo[knob]) + ", " +
                                              std::to_string(hi[knob]) + "] (or -1)");
    c->tune[knob] = value;
    return TKV_HIP_OK;
}

int32_t tkv_hip_ctx_synchronize(int64_t ctx) {
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    TKV_HIP_TRY(hipStreamSynchronize(c->stream));
    return TKV_HIP_OK;
}

int32_t tkv_hip_malloc(int64_t ctx, int64_t bytes, void** ptr_out) {
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    if (bytes < 0 || !ptr_out) return set_error(TKV_HIP_BAD_ARG, "bad malloc arguments");
    TKV_HIP_TRY(hipMalloc(ptr_out, bytes > 0 ? (size_t)bytes : 256));
    return TKV_HIP_OK;
}

int32_t tkv_hip_free(int64_t ctx, void* ptr) {
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    if (ptr) {
        TKV_HIP_TRY(hipStreamSynchronize(c->stream));
        TKV_HIP_TRY(hipFree(ptr));
    }
    return TKV_HIP_OK;
}

int32_t tkv_hip_memcpy_h2d(int64_t ctx, void* dst, const void* src, int64_t bytes) {
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    if (bytes <= 0) return TKV_HIP_OK;
    TKV_HIP_TRY(hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyHostToDevice, c->stream));
    TKV_HIP_TRY(hipStreamSynchronize(c->stream));
    return TKV_HIP_OK;
}

int32_t tkv_hip_memcpy_d2h(int64_t ctx, void* dst, const void* src, int64_t bytes) {
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    if (bytes <= 0) return TKV_HIP_OK;
    TKV_HIP_TRY(hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyDeviceToHost, c->stream));
    TKV_HIP_TRY(hipStreamSynchronize(c->stream));
    return TKV_HIP_OK;
}

int32_t tkv_hip_memcpy_d2d(int64_t ctx, void* dst, const void* src, int64_t bytes) {
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    if (bytes <= 0) return TKV_HIP_OK;
    if (!dst || !src) return set_error(TKV_HIP_BAD_ARG, "memcpy_d2d: NULL pointer");
    const bool aligned = ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src) |
                           (uintptr_t)bytes) & 15) == 0;
    if (!aligned) {
        TKV_HIP_TRY(hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyDeviceToDevice, c->stream));
        return TKV_HIP_OK;
    }
    const int64_t n16 = bytes / 16;
    const int64_t want = (n16 + 255) / 256;
    const unsigned grid = (unsigned)std::min<int64_t>(want, (int64_t)c->num_cus * 8);
    k_copy16<<<grid, 256, 0, c->stream>>>(static_cast<const u32x4*>(src), static_cast<u32x4*>(dst),
                                          n16);
    TKV_LAUNCH_CHECK();
    return TKV_HIP_OK;
}

int32_t tkv_hip_memset(int64_t ctx, void* dst, int32_t value, int64_t bytes) {
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    if (bytes <= 0) return TKV_HIP_OK;
    if (!dst) return set_error(TKV_HIP_BAD_ARG, "memset: NULL pointer");
    return launch_fill(c, dst, value, bytes);
}

int32_t tkv_hip_capture_begin(int64_t ctx) {
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    if (c->capturing) return set_error(TKV_HIP_BAD_ARG, "capture_begin: already capturing");
    TKV_HIP_TRY(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    c->capturing = true;
    return TKV_HIP_OK;
}

int32_t tkv_hip_capture_end(int64_t ctx, int64_t* graph_out) {
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    if (!graph_out) return set_error(TKV_HIP_BAD_ARG, "capture_end: graph_out is NULL");
    *graph_out = 0;
    if (!c->capturing) return set_error(TKV_HIP_BAD_ARG, "capture_end: no capture in progress");
    c->capturing = false;
    hipGraph_t g = nullptr;
    TKV_HIP_TRY(hipStreamEndCapture(c->stream, &g));
    hipGraphExec_t x = nullptr;
    const hipError_t e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return fail_hip(e, "hipGraphInstantiate", __FILE__, __LINE__);
    Graph* gr = new (std::nothrow) Graph();
    if (!gr) {
        (void)hipGraphExecDestroy(x);
        return set_error(TKV_HIP_OOM, "capture_end: host allocation failed");
    }
    gr->exec = x;
    gr->ctx = c;
    c->graphs.push_back(gr);
    *graph_out = reinterpret_cast<int64_t>(gr);
    return TKV_HIP_OK;
}

int32_t tkv_hip_graph_launch(int64_t ctx, int64_t graph) {
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    if (!graph) return set_error(TKV_HIP_BAD_ARG, "graph_launch: NULL graph");
    if (c->capturing) return set_error(TKV_HIP_BAD_ARG, "graph_launch: context is capturing");
    const Graph* gr = reinterpret_cast<const Graph*>(graph);
    if (!gr->exec)
        return set_error(TKV_HIP_BAD_ARG, "graph_launch: the graph's context has been destroyed");
    TKV_HIP_TRY(hipGraphLaunch(gr->exec, c->stream));
    return TKV_HIP_OK;
}

int32_t tkv_hip_graph_destroy(int64_t graph) {
    Graph* gr = reinterpret_cast<Graph*>(graph);
    if (!gr) return TKV_HIP_OK;
    Ctx* c = gr->ctx;
    if (!c) {  // detached by ctx_destroy, which released the executable
        delete gr;
        return TKV_HIP_OK;
    }
    TKV_HIP_TRY(hipSetDevice(c->device));
    // replays already queued must finish before the graph or the buffers
    // it reads go away
    TKV_HIP_TRY(hipStreamSynchronize(c->stream));
    TKV_HIP_TRY(hipGraphExecDestroy(gr->exec));
    c->graphs.erase(std::find(c->graphs.begin(), c->graphs.end(), gr));
    delete gr;
    if (c->graphs.empty()) {
        for (void* p : c->retired) TKV_HIP_TRY(hipFree(p));
        c->retired.clear();
    }
    return TKV_HIP_OK;
}

int32_t tkv_hip_ctx_retired_buffers(int64_t ctx, int64_t* count_out) {
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    if (!count_out) return set_error(TKV_HIP_BAD_ARG, "retired_buffers: NULL output");
    *count_out = (int64_t)c->retired.size();
    return TKV_HIP_OK;
}

int32_t tkv_hip_event_create(int64_t* ev_out) {
    hipEvent_t e;
    TKV_HIP_TRY(hipEventCreate(&e));
    *ev_out = reinterpret_cast<int64_t>(e);
    return TKV_HIP_OK;
}

int32_t tkv_hip_event_destroy(int64_t ev) {
    if (ev) TKV_HIP_TRY(hipEventDestroy(reinterpret_cast<hipEvent_t>(ev)));
    return TKV_HIP_OK;
}

int32_t tkv_hip_event_record(int64_t ctx, int64_t ev) {
    Ctx* c;
    TKV_RC_TRY(ctx_get(ctx, &c));
    TKV_HIP_TRY(hipEventRecord(reinterpret_cast<hipEvent_t>(ev), c->stream));
    return TKV_HIP_OK;
}

int32_t tkv_hip_event_elapsed_ms(int64_t ev_start, int64_t ev_end, float* ms_out) {
    TKV_HIP_TRY(hipEventSynchronize(reinterpret_cast<hipEvent_t>(ev_end)));
    TKV_HIP_TRY(hipEventElapsedTime(ms_out, reinterpret_cast<hipEvent_t>(ev_start),
                                    reinterpret_cast<hipEvent_t>(ev_end)));
    return TKV_HIP_OK;
}

}  // extern "C"
