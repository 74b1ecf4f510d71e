// C ABI of libsamhip (include/samhip.h): contexts, validation, dispatch.
#include "samhip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "internal.hpp"

using namespace samhip;

namespace {

thread_local std::string g_last_error;

int fail(int status, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return status;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(e == hipErrorOutOfMemory ? SAMHIP_ERR_OUT_OF_MEMORY : SAMHIP_ERR_DEVICE, "%s: %s", what,
                hipGetErrorString(e));
}

#define HIP_TRY(expr, what)                         \
    do {                                            \
        hipError_t e_ = (expr);                     \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

bool is_weight_type(int t) { return t == T_Q8_0 || t == T_Q4_K || t == T_Q5_K || t == T_Q6_K; }

// Activation packing type for a weight type: ggml's CPU vec_dot_type
// (src/runtime/ggml/backends/cpu.hpp:13-23).
int vec_dot_type(int wtype) { return wtype == T_Q8_0 ? T_Q8_0 : T_Q8_K; }

size_t row_bytes(int t, int64_t k) { return size_t(k / block_elems(t)) * size_t(block_bytes(t)); }

}  // namespace

struct samhip_graph {
    samhip_context* ctx;
    hipGraphExec_t exec;
};

namespace {

// Fixed device scratch of samhip_mul_mat_noalloc: one array per device,
// allocated with the code object and kept until the process ends.  Host code
// never uses the array's name as an address: each device's own address comes
// from hipGetSymbolAddress once, with that device current, at context
// creation.
constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;
__device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;

// Per device: the scratch address, and what orders the calls that use it.
// `last` is recorded on a call's stream after its kernels, and the next call
// (on any context, any stream of that device) waits for it before its own,
// so calls made one after another on the host also run one after another on
// the GPU; `call` keeps two host threads from interleaving that wait/record.
struct FixedScratch {
    void* ptr = nullptr;
    hipEvent_t last = nullptr;
    std::mutex call;
};
FixedScratch g_fixed[kMaxDevices];

// The current device's scratch (looked up on its first use, with the
// ordering event created then; neither allocates device memory later).
hipError_t device_scratch(int device, void** out) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    FixedScratch& f = g_fixed[device];
    if (!f.ptr) {
        void* p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        hipEvent_t ev = nullptr;
        e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (e != hipSuccess) return e;
        f.last = ev;
        f.ptr = p;
    }
    *out = f.ptr;
    return hipSuccess;
}

}  // namespace

struct samhip_context {
    int device = 0;
    int compute = SAMHIP_COMPUTE_Q8_NATIVE;
    int q8_rounding = SAMHIP_Q8_ROUND_X86;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    // staged fp16 activations [M][K], F32 row scales [M] and, on the tall
    // path, the call's fp16 weights [N][K]
    void* staging = nullptr;
    size_t staging_bytes = 0;
    int* flag = nullptr;   // device error flag (get_rows id range)
    // this device's fixed scratch (samhip_mul_mat_noalloc); while such a call
    // runs, `staging` points at it and `no_alloc` forbids growing it
    void* fixed_scratch = nullptr;
    bool no_alloc = false;
    // tall-path selection: M at or above `tall_m` uses dequant + fp16 GEMM;
    // gemm_cfg >= 0 forces one fp16 GEMM tile configuration (SAMHIP_GEMM_CONFIG)
    int cus = 256;             // compute units of the device
    int tall_m = 256;
    int gemm_cfg = -1;
    bool fused_skinny = true;   // SAMHIP_FUSED_SKINNY=0 routes M < 256 through staging + the skinny kernel
    int strip_skinny = 1;       // SAMHIP_STRIP_SKINNY: 0 never, 1 where preferred, 2 every M < 256 product
    int attn_splits = 0;        // SAMHIP_ATTN_SPLITS: key splits of the attention kernel (0: by grid size)
    int fused_max_splits = 16;  // SAMHIP_FUSED_MAX_SPLITS: cap on the fused kernel's K splits
    bool check_activations = false;   // samhip_context_set_activation_check
    bool tall_int8 = false;     // SAMHIP_TALL_INT8=1: tall Q8_0 products on the exact int8 GEMM
    bool tall_decode = false;   // SAMHIP_TALL_DECODE=1: tall products on the in-loader weight-decode GEMM
    bool tall_small = true;     // SAMHIP_TALL_SMALL=0 keeps M >= 256 products with small weights on the fused kernel
    int int8_strip = 1;         // SAMHIP_INT8_STRIP: 0 keeps M < 256 products on the fp16 kernels; 1 sends Q8_0
                                // ones, and K-quant ones where that measured faster, to the int8 kernels; 2
                                // sends every K-quant one there as well
    bool kq_isum = false;       // SAMHIP_KQ_ISUM=1: the K-quant int8 strip kernel in its integer form (per
                                // super-block integer sums, ggml's F32 steps in K order: the oracle's bits with
                                // one K slice; measured 5 % slower on the Q4_K text stream)
    int strip_rows = 0;         // SAMHIP_I8_STRIP_ROWS: weight rows per workgroup of the int8 strip kernels,
                                // 32 or 64 (64 only for K slices of at most 256 values); 0: 64 where that
                                // brings the grid into one round
    bool vit_fc1_codes = false; // SAMHIP_VIT_FC1_CODES=1: with a Q8_0 fc2, an encoder block's fc1 epilogue
                                // applies the erf-GELU and writes fc2's Q8_0 codes (same bits; measured no
                                // faster: the GEMM gains the GELU's VALU work, the staging loses the F32 reads)
    samhip_exec_info info{};
    // per-launch event trace (samhip_trace_begin / samhip_trace_end)
    struct TraceRecord {
        const char* kernel;
        int weight_type;
        int64_t m, n, k;
        hipEvent_t start, stop;
    };
    bool tracing = false;        // a trace is open (trace_begin .. trace_end)
    bool trace_paused = false;   // open but not bracketing (samhip_trace_pause)
    // stream capture: staging buffers that captured graphs still use
    bool capturing = false;
    int live_graphs = 0;
    std::vector<void*> retired_staging;
    std::string trace_filter;
    std::vector<TraceRecord> trace;
    std::vector<hipEvent_t> event_pool;
    // vision-encoder intermediates (samhip_vit_block / samhip_vit_prefix /
    // samhip_flash_attn); grown on demand, never while capturing
    void* work = nullptr;
    size_t work_bytes = 0;
    // window-unpartition row table of the last (grid_w, grid_h, window)
    int* row_map = nullptr;
    int row_map_key[3] = {0, 0, 0};
};

namespace {

// Entry points that synchronize or allocate cannot be recorded into a graph.
#define SAMHIP_NOT_WHILE_CAPTURING(ctx, what)                                                  \
    do {                                                                                      \
        if ((ctx)->capturing) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "%s cannot be called while a capture is open", what); \
    } while (0)

int set_device(samhip_context* ctx) {
    HIP_TRY(hipSetDevice(ctx->device), "hipSetDevice");
    return SAMHIP_OK;
}

int ensure_staging(samhip_context* ctx, size_t bytes) {
    if (bytes <= ctx->staging_bytes) return SAMHIP_OK;
    if (ctx->no_alloc)
        return fail(SAMHIP_ERR_INVALID_ARGUMENT,
                    "mul_mat_noalloc: this product needs %zu bytes of scratch; the fixed scratch holds %zu", bytes,
                    ctx->staging_bytes);
    if (ctx->capturing)
        return fail(SAMHIP_ERR_INVALID_ARGUMENT,
                    "capture: this product needs %zu bytes of staging but %zu are reserved; run it once before "
                    "capturing", bytes, ctx->staging_bytes);
    if (ctx->staging) {
        HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
        if (ctx->live_graphs > 0) {
            ctx->retired_staging.push_back(ctx->staging);   // still named by captured graphs
        } else {
            HIP_TRY(hipFree(ctx->staging), "hipFree");
        }
        ctx->staging = nullptr;
        ctx->staging_bytes = 0;
    }
    const size_t rounded = (bytes + (size_t(1) << 20) - 1) & ~((size_t(1) << 20) - 1);
    HIP_TRY(hipMalloc(&ctx->staging, rounded), "hipMalloc staging");
    ctx->staging_bytes = rounded;
    ctx->info.activation_allocation_peak_bytes =
        std::max<uint64_t>(ctx->info.activation_allocation_peak_bytes, rounded);
    return SAMHIP_OK;
}

constexpr size_t kMaxTraceRecords = size_t(1) << 20;

hipEvent_t pooled_event(samhip_context* ctx) {
    if (!ctx->event_pool.empty()) {
        hipEvent_t e = ctx->event_pool.back();
        ctx->event_pool.pop_back();
        return e;
    }
    // timing only (trace_end synchronizes the stream before reading them):
    // no system-scope fence, so recording one does not write back and
    // invalidate the caches between the launches it brackets
    hipEvent_t e = nullptr;
    if (hipEventCreateWithFlags(&e, hipEventDisableSystemFence) != hipSuccess) return nullptr;
    return e;
}

// Launches `body` on the context stream, bracketed by events when tracing.
template <class Body>
int traced(samhip_context* ctx, const char* kernel, int wt, int64_t m, int64_t n, int64_t k, Body body) {
    hipEvent_t a = nullptr, b = nullptr;
    const bool record = ctx->tracing && !ctx->trace_paused && ctx->trace.size() < kMaxTraceRecords &&
                        (ctx->trace_filter.empty() || std::strstr(kernel, ctx->trace_filter.c_str()) != nullptr);
    if (record) {
        a = pooled_event(ctx);
        b = pooled_event(ctx);
        if (!a || !b) return fail(SAMHIP_ERR_DEVICE, "hipEventCreate failed");
        HIP_TRY(hipEventRecord(a, ctx->stream), "hipEventRecord");
    }
    const int rc = body();
    if (record) {
        HIP_TRY(hipEventRecord(b, ctx->stream), "hipEventRecord");
        ctx->trace.push_back({kernel, wt, m, n, k, a, b});
    }
    return rc;
}

const char* dequant_name(int wtype) {
    return wtype == T_Q8_0 ? "dequant_w_f16_q8_0" : wtype == T_Q4_K ? "dequant_w_f16_q4_k"
         : wtype == T_Q5_K ? "dequant_w_f16_q5_k" : "dequant_w_f16_q6_k";
}

int env_int(const char* name, int fallback) {
    const char* v = std::getenv(name);
    if (!v || !*v) return fallback;
    char* end = nullptr;
    const long x = std::strtol(v, &end, 10);
    return (end && *end == '\0') ? int(x) : fallback;
}

const char* prep_name(int mode) {
    return mode == T_F16 ? "stage_dequant_f16" : mode == T_Q8_0 ? "stage_dequant_q8_0" : "stage_dequant_q8_k";
}

const char* stage_name(int mode) {
    return mode == T_F16 ? "stage_rows_f16" : mode == T_Q8_0 ? "stage_rows_q8_0" : "stage_rows_q8_k";
}

const char* profile_name(int compute) {
    return compute == SAMHIP_COMPUTE_F16 ? "samhip-f16-f16mfma-v1" : "samhip-q8-native-f16mfma-v1";
}

// Returns 0 when supported, else a reason string (checked without touching
// device memory).
const char* mul_mat_problem(const samhip_tensor* w, const samhip_tensor* x, const samhip_tensor* y) {
    if (!w || !x || !y) return "null tensor descriptor";
    if (!is_weight_type(w->type)) return "weight type must be Q8_0, Q4_K, Q5_K or Q6_K";
    if (x->type != T_F32 || y->type != T_F32) return "activation and output must be F32";
    const int64_t K = w->ne[0], N = w->ne[1], M = x->ne[1];
    if (K <= 0 || N <= 0 || M <= 0) return "empty operand";
    for (int i = 2; i < 4; ++i)
        if (w->ne[i] != 1 || x->ne[i] != 1 || y->ne[i] != 1) return "only 2-D operands are supported";
    if (K % block_elems(w->type)) return "K is not a multiple of the weight block size";
    if (x->ne[0] != K) return "activation width differs from weight width";
    if (y->ne[0] != N || y->ne[1] != M) return "output shape must be [N, M]";
    if (w->nb[0] != size_t(block_bytes(w->type))) return "weight nb[0] must equal the block size";
    if (w->nb[1] < row_bytes(w->type, K)) return "weight rows overlap";
    if (x->nb[0] != 4 || x->nb[1] < size_t(4 * K) || x->nb[1] % 4) return "activation rows must be F32-contiguous";
    if (y->nb[0] != 4 || y->nb[1] < size_t(4 * N) || y->nb[1] % 4) return "output rows must be F32-contiguous";
    if (!w->data || !x->data || !y->data) return "null data pointer";
    if (reinterpret_cast<uintptr_t>(w->data) % 2 || w->nb[1] % 2) return "packed weight rows must be 2-byte aligned";
    if (reinterpret_cast<uintptr_t>(x->data) % 4 || reinterpret_cast<uintptr_t>(y->data) % 4)
        return "F32 operands must be 4-byte aligned";
    if (K > (int64_t(1) << 24) || N > (int64_t(1) << 30) || M > (int64_t(1) << 30)) return "dimension too large";
    return nullptr;
}

}  // namespace

extern "C" {

int samhip_abi_version(void) { return SAMHIP_ABI_VERSION; }

int samhip_device_count(int* count) {
    if (!count) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "null count");
    int n = 0;
    const hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) n = 0;
    *count = n;
    return SAMHIP_OK;
}

int samhip_context_create(const samhip_options* options, samhip_context** out) {
    if (!out) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "null output context");
    *out = nullptr;
    samhip_options o{SAMHIP_ABI_VERSION, 0, SAMHIP_COMPUTE_Q8_NATIVE, SAMHIP_Q8_ROUND_X86};
    if (options) o = *options;
    if (o.version != SAMHIP_ABI_VERSION) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "unsupported samhip ABI version %u", o.version);
    if (o.compute != SAMHIP_COMPUTE_Q8_NATIVE && o.compute != SAMHIP_COMPUTE_F16)
        return fail(SAMHIP_ERR_INVALID_ARGUMENT, "unknown HIP compute mode");
    if (o.q8_rounding != SAMHIP_Q8_ROUND_X86 && o.q8_rounding != SAMHIP_Q8_ROUND_REF)
        return fail(SAMHIP_ERR_INVALID_ARGUMENT, "unknown Q8 rounding mode");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return fail(SAMHIP_ERR_DEVICE, "no HIP device is visible");
    if (o.device < 0 || o.device >= n) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "HIP device %d out of range [0, %d)", o.device, n);
    samhip_context* ctx = new (std::nothrow) samhip_context;
    if (!ctx) return fail(SAMHIP_ERR_OUT_OF_MEMORY, "context allocation failed");
    ctx->device = o.device;
    ctx->compute = o.compute;
    ctx->q8_rounding = o.q8_rounding;
    ctx->info.version = SAMHIP_ABI_VERSION;
    ctx->info.device = o.device;
    std::snprintf(ctx->info.arithmetic_profile, sizeof(ctx->info.arithmetic_profile), "%s", profile_name(o.compute));
    hipDeviceProp_t prop;
    if (hipSetDevice(o.device) != hipSuccess || hipGetDeviceProperties(&prop, o.device) != hipSuccess ||
        hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking) != hipSuccess ||
        hipMalloc(reinterpret_cast<void**>(&ctx->flag), sizeof(int)) != hipSuccess) {
        samhip_context_destroy(ctx);
        return fail(SAMHIP_ERR_DEVICE, "HIP context initialization failed");
    }
    if (const hipError_t e = device_scratch(o.device, &ctx->fixed_scratch); e != hipSuccess) {
        samhip_context_destroy(ctx);
        return fail(SAMHIP_ERR_DEVICE, "fixed scratch address of device %d: %s", o.device, hipGetErrorString(e));
    }
    std::snprintf(ctx->info.device_name, sizeof(ctx->info.device_name), "%s (%s)", prop.name, prop.gcnArchName);
    ctx->cus = std::max(1, prop.multiProcessorCount);
    ctx->stream = ctx->own_stream;
    // kernel-variant forcing for tuning runs (SAMHIP_* environment variables)
    ctx->tall_m = std::max(1, env_int("SAMHIP_TALL_M", ctx->tall_m));
    ctx->fused_skinny = env_int("SAMHIP_FUSED_SKINNY", 1) != 0;
    ctx->strip_skinny = env_int("SAMHIP_STRIP_SKINNY", 1);
    ctx->attn_splits = std::max(0, env_int("SAMHIP_ATTN_SPLITS", 0));
    ctx->fused_max_splits = std::max(1, env_int("SAMHIP_FUSED_MAX_SPLITS", 16));
    ctx->int8_strip = env_int("SAMHIP_INT8_STRIP", 1);
    ctx->strip_rows = env_int("SAMHIP_I8_STRIP_ROWS", 0);
    ctx->kq_isum = env_int("SAMHIP_KQ_ISUM", 0) != 0;
    ctx->vit_fc1_codes = env_int("SAMHIP_VIT_FC1_CODES", 0) != 0;
    ctx->tall_small = env_int("SAMHIP_TALL_SMALL", 1) != 0;
    ctx->tall_int8 = env_int("SAMHIP_TALL_INT8", 0) != 0;
    ctx->tall_decode = env_int("SAMHIP_TALL_DECODE", 0) != 0;
    const int cfg = env_int("SAMHIP_GEMM_CONFIG", -1);
    ctx->gemm_cfg = (cfg >= 0 && cfg < gemm_f16_config_count()) ? cfg : -1;
    *out = ctx;
    return SAMHIP_OK;
}

void samhip_context_destroy(samhip_context* ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->capturing) {
        hipGraph_t g = nullptr;
        (void)hipStreamEndCapture(ctx->stream, &g);
        if (g) (void)hipGraphDestroy(g);
    }
    if (ctx->own_stream) (void)hipStreamSynchronize(ctx->own_stream);
    if (ctx->stream && ctx->stream != ctx->own_stream) (void)hipStreamSynchronize(ctx->stream);
    if (ctx->staging) (void)hipFree(ctx->staging);
    if (ctx->work) (void)hipFree(ctx->work);
    if (ctx->row_map) (void)hipFree(ctx->row_map);
    for (void* p : ctx->retired_staging) (void)hipFree(p);
    if (ctx->flag) (void)hipFree(ctx->flag);
    for (auto& r : ctx->trace) {
        (void)hipEventDestroy(r.start);
        (void)hipEventDestroy(r.stop);
    }
    for (hipEvent_t e : ctx->event_pool) (void)hipEventDestroy(e);
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
    delete ctx;
}

int samhip_context_set_stream(samhip_context* ctx, void* hip_stream) {
    if (!ctx) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "null context");
    SAMHIP_NOT_WHILE_CAPTURING(ctx, "context_set_stream");
    ctx->stream = hip_stream ? static_cast<hipStream_t>(hip_stream) : ctx->own_stream;
    return SAMHIP_OK;
}

int samhip_synchronize(samhip_context* ctx) {
    if (!ctx) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "null context");
    SAMHIP_NOT_WHILE_CAPTURING(ctx, "synchronize");
    if (int rc = set_device(ctx)) return rc;
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return SAMHIP_OK;
}

int samhip_buffer_alloc(samhip_context* ctx, size_t bytes, void** device_ptr) {
    if (!ctx || !device_ptr || bytes == 0) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "invalid buffer request");
    SAMHIP_NOT_WHILE_CAPTURING(ctx, "buffer_alloc");
    if (int rc = set_device(ctx)) return rc;
    HIP_TRY(hipMalloc(device_ptr, bytes), "hipMalloc");
    return SAMHIP_OK;
}

int samhip_buffer_free(samhip_context* ctx, void* device_ptr) {
    if (!ctx) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "null context");
    SAMHIP_NOT_WHILE_CAPTURING(ctx, "buffer_free");
    if (!device_ptr) return SAMHIP_OK;
    if (int rc = set_device(ctx)) return rc;
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    HIP_TRY(hipFree(device_ptr), "hipFree");
    return SAMHIP_OK;
}

int samhip_tensor_set(samhip_context* ctx, void* device_dst, const void* host_src, size_t bytes) {
    if (!ctx || (bytes && (!device_dst || !host_src))) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "invalid tensor_set");
    SAMHIP_NOT_WHILE_CAPTURING(ctx, "tensor_set");
    if (!bytes) return SAMHIP_OK;
    if (int rc = set_device(ctx)) return rc;
    HIP_TRY(hipMemcpyAsync(device_dst, host_src, bytes, hipMemcpyHostToDevice, ctx->stream), "hipMemcpyAsync H2D");
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return SAMHIP_OK;
}

int samhip_tensor_get(samhip_context* ctx, void* host_dst, const void* device_src, size_t bytes) {
    if (!ctx || (bytes && (!device_src || !host_dst))) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "invalid tensor_get");
    SAMHIP_NOT_WHILE_CAPTURING(ctx, "tensor_get");
    if (!bytes) return SAMHIP_OK;
    if (int rc = set_device(ctx)) return rc;
    HIP_TRY(hipMemcpyAsync(host_dst, device_src, bytes, hipMemcpyDeviceToHost, ctx->stream), "hipMemcpyAsync D2H");
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    return SAMHIP_OK;
}

int samhip_supports_mul_mat(const samhip_tensor* w, const samhip_tensor* x, const samhip_tensor* y) {
    return mul_mat_problem(w, x, y) == nullptr ? 1 : 0;
}

namespace {

// Trace name of an attention launch: the key-split count when it splits.
const char* attention_name(int splits) {
    switch (splits) {
        case 2: return "vit_attention_split2";
        case 3: return "vit_attention_split3";
        case 4: return "vit_attention_split4";
        default: return "vit_attention";
    }
}

// Reads back the device flag a range check or D4 staging launch raised.
int read_range_flag(samhip_context* ctx) {
    int bad = 0;
    HIP_TRY(hipMemcpyAsync(&bad, ctx->flag, sizeof(int), hipMemcpyDeviceToHost, ctx->stream), "hipMemcpyAsync");
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    if (bad)
        return fail(SAMHIP_ERR_INVALID_ARGUMENT,
                    "native Q8 activations require finite F32 and each nonzero block maximum in [1e-30,1e30]");
    return SAMHIP_OK;
}

int check_q8_rhs(samhip_context* ctx, const float* x, int64_t x_stride, int rows, int K) {
    HIP_TRY(hipMemsetAsync(ctx->flag, 0, sizeof(int), ctx->stream), "hipMemsetAsync");
    launch_q8_rhs_check(x, x_stride, rows, K, ctx->flag, ctx->stream);
    HIP_TRY(hipGetLastError(), "activation check launch");
    return read_range_flag(ctx);
}

}  // namespace

int samhip_context_set_activation_check(samhip_context* ctx, int enabled) {
    if (!ctx) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "null context");
    ctx->check_activations = enabled != 0;
    return SAMHIP_OK;
}

int samhip_mul_mat_noalloc(samhip_context* ctx, const samhip_tensor* w, const samhip_tensor* x,
                           const samhip_tensor* y) {
    if (!ctx) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "null context");
    if (!ctx->fixed_scratch) return fail(SAMHIP_ERR_DEVICE, "mul_mat_noalloc: no fixed scratch on this device");
    FixedScratch& f = g_fixed[ctx->device];
    std::lock_guard<std::mutex> lock(f.call);
    if (int rc = set_device(ctx)) return rc;
    // stream order behind the previous call on this device's scratch (not
    // while capturing: a graph's own replays are the caller's to order)
    if (!ctx->capturing) HIP_TRY(hipStreamWaitEvent(ctx->stream, f.last, 0), "hipStreamWaitEvent");
    void* const staging = ctx->staging;
    const size_t staging_bytes = ctx->staging_bytes;
    ctx->staging = ctx->fixed_scratch;
    ctx->staging_bytes = kNoAllocScratchBytes;
    ctx->no_alloc = true;
    const int rc = samhip_mul_mat(ctx, w, x, y);
    ctx->no_alloc = false;
    ctx->staging = staging;
    ctx->staging_bytes = staging_bytes;
    if (!ctx->capturing) HIP_TRY(hipEventRecord(f.last, ctx->stream), "hipEventRecord");
    return rc;
}

int samhip_mul_mat(samhip_context* ctx, const samhip_tensor* w, const samhip_tensor* x, const samhip_tensor* y) {
    if (!ctx) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "null context");
    if (const char* why = mul_mat_problem(w, x, y)) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "mul_mat: %s", why);
    const int K = int(w->ne[0]), N = int(w->ne[1]), M = int(x->ne[1]);
    if (int rc = set_device(ctx)) return rc;
    if (ctx->check_activations && ctx->compute == SAMHIP_COMPUTE_Q8_NATIVE) {
        SAMHIP_NOT_WHILE_CAPTURING(ctx, "mul_mat with the activation check");
        if (int rc = check_q8_rhs(ctx, static_cast<const float*>(x->data), int64_t(x->nb[1] / 4), M, K)) return rc;
    }
    // tall products with a 256x256-sized weight (the fusion / decoder image
    // tokens' q, k, v, out projections) take one launch: the small-weight
    // int8 kernels in native compute, the fused kernel otherwise
    const bool small_w = ctx->fused_skinny && int64_t(N) * K <= kFusedSmallW;
    // SAMHIP_TALL_DECODE=1 sends the tall products to the GEMM that decodes
    // the packed weight while staging it into LDS (gemm_kernel, one pass over
    // the weight) instead of weight decode in the preparation + fp16 GEMM
    const bool tall = M >= ctx->tall_m && gemm_f16_supported(M, N, K, K, K) && !small_w && !ctx->tall_decode;
    const bool kquant = (w->type == T_Q4_K || w->type == T_Q5_K || w->type == T_Q6_K) &&
                        (ctx->int8_strip == 2 || kq_strip_i8_preferred(w->type, M, N, K, ctx->cus, ctx->strip_rows != 32));
    const bool tall_small_q8 = w->type == T_Q8_0 && tall_small_i8_supported(M, N, K, w->data, int64_t(w->nb[1]));
    const bool tall_small_kq = tall_small_kq_i8_supported(w->type, M, N, K, w->data, int64_t(w->nb[1]));
    if (small_w && M >= kStripMaxM && (tall_small_q8 || tall_small_kq) && ctx->compute == SAMHIP_COMPUTE_Q8_NATIVE &&
        ctx->tall_small) {
        // many rows against a weight that fits in LDS: exact int8, one
        // workgroup per CU, no staging
        const char* variant = tall_small_q8 ? tall_small_i8_variant() : tall_small_kq_i8_variant(w->type);
        int rc = traced(ctx, variant, w->type, M, N, K, [&]() -> int {
            const float* xp = static_cast<const float*>(x->data);
            float* yp = static_cast<float*>(y->data);
            const char* ok =
                tall_small_q8
                    ? launch_tall_small_i8(xp, int64_t(x->nb[1] / 4), w->data, int64_t(w->nb[1]), yp,
                                           int64_t(y->nb[1] / 4), M, N, K,
                                           ctx->q8_rounding == SAMHIP_Q8_ROUND_X86 ? 1 : 0, ctx->cus, ctx->stream)
                    : launch_tall_small_kq_i8(w->type, xp, int64_t(x->nb[1] / 4), w->data, int64_t(w->nb[1]), yp,
                                              int64_t(y->nb[1] / 4), M, N, K, ctx->cus, ctx->stream);
            if (!ok) return fail(SAMHIP_ERR_UNSUPPORTED, "mul_mat: no small-weight kernel for this shape");
            HIP_TRY(hipGetLastError(), "small-weight launch");
            return SAMHIP_OK;
        });
        if (rc) return rc;
        ctx->info.mul_mat_calls++;
        ctx->info.skinny_launches++;
        std::snprintf(ctx->info.kernel_variant, sizeof(ctx->info.kernel_variant), "%s", variant);
        return SAMHIP_OK;
    }
    if (!tall && M < kStripMaxM && (w->type == T_Q8_0 || kquant) && ctx->compute == SAMHIP_COMPUTE_Q8_NATIVE &&
        ctx->int8_strip && ctx->fused_skinny) {
        // exact int8 block dots in blocks of 32 activation rows (the text
        // encoder, the decoder's queries and prompt); K slices of 256-1024
        // values, and a reduce launch when there is more than one
        const int slice_sb = i8_strip_slice_sb(w->type, M, N, K, ctx->cus);
        if (int rc = ensure_staging(ctx, std::max<size_t>(i8_strip_part_bytes(M, N, K, slice_sb), 256))) return rc;
        const char* variant = kquant ? kq_strip_i8_variant(w->type) : q8_strip_i8_variant();
        int rc = traced(ctx, variant, w->type, M, N, K, [&]() -> int {
            const float* xp = static_cast<const float*>(x->data);
            float* yp = static_cast<float*>(y->data);
            float* part = static_cast<float*>(ctx->staging);
            const bool two_tiles = ctx->strip_rows == 64 ||
                                   (ctx->strip_rows != 32 && i8_strip_two_tiles_preferred(M, N, K, slice_sb, ctx->cus));
            const char* ok = kquant
                ? launch_kq_strip_i8(w->type, xp, int64_t(x->nb[1] / 4), w->data, int64_t(w->nb[1]), yp,
                                     int64_t(y->nb[1] / 4), part, M, N, K, slice_sb, two_tiles, ctx->kq_isum,
                                     ctx->stream)
                : launch_q8_strip_i8(xp, int64_t(x->nb[1] / 4), w->data, int64_t(w->nb[1]), yp, int64_t(y->nb[1] / 4),
                                     part, M, N, K, slice_sb, ctx->q8_rounding == SAMHIP_Q8_ROUND_X86 ? 1 : 0,
                                     two_tiles, ctx->stream);
            if (!ok) return fail(SAMHIP_ERR_UNSUPPORTED, "mul_mat: no int8 strip kernel for this shape");
            HIP_TRY(hipGetLastError(), "int8 strip launch");
            return SAMHIP_OK;
        });
        if (rc) return rc;
        ctx->info.mul_mat_calls++;
        ctx->info.skinny_launches++;
        std::snprintf(ctx->info.kernel_variant, sizeof(ctx->info.kernel_variant), "%s", variant);
        return SAMHIP_OK;
    }
    if (!tall && M < kStripMaxM && ctx->fused_skinny && ctx->strip_skinny &&
        (ctx->strip_skinny == 2 || strip_skinny_preferred(w->type, M, K))) {
        // one launch per product (and a reduce when K > 1024): activation
        // packing in registers, weight decode and product
        const FusedPlan plan = strip_skinny_plan(M, N, K);
        if (int rc = ensure_staging(ctx, std::max<size_t>(plan.part_bytes, 256))) return rc;
        const char* variant = strip_skinny_variant(w->type);
        if (!variant) return fail(SAMHIP_ERR_UNSUPPORTED, "mul_mat: no kernel for weight type %d", w->type);
        int rc = traced(ctx, variant, w->type, M, N, K, [&]() -> int {
            if (!launch_strip_skinny(w->type, ctx->compute == SAMHIP_COMPUTE_F16, static_cast<const float*>(x->data),
                                     int64_t(x->nb[1] / 4), w->data, int64_t(w->nb[1]), static_cast<float*>(y->data),
                                     int64_t(y->nb[1] / 4), static_cast<float*>(ctx->staging), M, N, K,
                                     ctx->q8_rounding == SAMHIP_Q8_ROUND_X86 ? 1 : 0, ctx->stream))
                return fail(SAMHIP_ERR_UNSUPPORTED, "mul_mat: no strip kernel for this shape");
            HIP_TRY(hipGetLastError(), "strip skinny launch");
            return SAMHIP_OK;
        });
        if (rc) return rc;
        ctx->info.mul_mat_calls++;
        ctx->info.skinny_launches++;
        std::snprintf(ctx->info.kernel_variant, sizeof(ctx->info.kernel_variant), "%s", variant);
        return SAMHIP_OK;
    }
    if (!tall && (M <= kFusedMaxM || small_w) && ctx->fused_skinny) {
        // one launch: activation packing, weight decode and product
        const FusedPlan plan = fused_skinny_plan(M, N, K, ctx->fused_max_splits, ctx->cus);
        if (int rc = ensure_staging(ctx, std::max<size_t>(plan.part_bytes, 256))) return rc;
        const char* variant = fused_skinny_variant(w->type);
        if (!variant) return fail(SAMHIP_ERR_UNSUPPORTED, "mul_mat: no kernel for weight type %d", w->type);
        int rc = traced(ctx, variant, w->type, M, N, K, [&]() -> int {
            if (!launch_fused_skinny(w->type, ctx->compute == SAMHIP_COMPUTE_F16, static_cast<const float*>(x->data),
                                     int64_t(x->nb[1] / 4), w->data, int64_t(w->nb[1]), static_cast<float*>(y->data),
                                     int64_t(y->nb[1] / 4), static_cast<float*>(ctx->staging), M, N, K,
                                     ctx->q8_rounding == SAMHIP_Q8_ROUND_X86 ? 1 : 0, ctx->fused_max_splits,
                                     ctx->cus, ctx->stream))
                return fail(SAMHIP_ERR_UNSUPPORTED, "mul_mat: no fused kernel for this shape");
            HIP_TRY(hipGetLastError(), "fused skinny launch");
            return SAMHIP_OK;
        });
        if (rc) return rc;
        ctx->info.mul_mat_calls++;
        ctx->info.skinny_launches++;
        std::snprintf(ctx->info.kernel_variant, sizeof(ctx->info.kernel_variant), "%s", variant);
        return SAMHIP_OK;
    }
    if (M >= ctx->tall_m && !small_w && w->type == T_Q8_0 && ctx->compute == SAMHIP_COMPUTE_Q8_NATIVE &&
        ctx->tall_int8 && gemm_i8_supported(M, N, K)) {
        // exact: int8 codes and F32 block scales for both operands, int8 MFMA
        if (int rc = ensure_staging(ctx, gemm_i8_staging_bytes(M, N, K))) return rc;
        const char* variant = gemm_i8_variant();
        int rc = traced(ctx, variant, w->type, M, N, K, [&]() -> int {
            const char* prep = nullptr;
            if (!launch_gemm_i8(static_cast<const float*>(x->data), int64_t(x->nb[1] / 4), w->data, int64_t(w->nb[1]),
                                static_cast<float*>(y->data), int64_t(y->nb[1] / 4), M, N, K,
                                ctx->q8_rounding == SAMHIP_Q8_ROUND_X86 ? 1 : 0, ctx->staging, ctx->stream, &prep))
                return fail(SAMHIP_ERR_UNSUPPORTED, "mul_mat: no int8 GEMM for this shape");
            HIP_TRY(hipGetLastError(), "int8 GEMM launch");
            return SAMHIP_OK;
        });
        if (rc) return rc;
        ctx->info.mul_mat_calls++;
        ctx->info.activation_launches++;
        ctx->info.gemm_launches++;
        ctx->info.activation_payload_peak_bytes =
            std::max<uint64_t>(ctx->info.activation_payload_peak_bytes, uint64_t(M) * K + uint64_t(M) * (K / 32) * 4);
        std::snprintf(ctx->info.kernel_variant, sizeof(ctx->info.kernel_variant), "%s", variant);
        return SAMHIP_OK;
    }
    auto align256 = [](size_t v) { return (v + 255) & ~size_t(255); };
    const size_t a_bytes = size_t(M) * size_t(K) * 2;
    const size_t rs_offset = align256(a_bytes);
    const size_t w_offset = align256(rs_offset + size_t(M) * 4);
    const size_t need = tall ? w_offset + size_t(N) * size_t(K) * 2 : w_offset;
    if (int rc = ensure_staging(ctx, need)) return rc;
    uint8_t* base = static_cast<uint8_t*>(ctx->staging);
    _Float16* a = reinterpret_cast<_Float16*>(base);
    float* rs = reinterpret_cast<float*>(base + rs_offset);
    _Float16* wh = reinterpret_cast<_Float16*>(base + w_offset);
    const int mode = ctx->compute == SAMHIP_COMPUTE_F16 ? T_F16 : vec_dot_type(w->type);
    const bool aligned = reinterpret_cast<uintptr_t>(x->data) % 16 == 0 && x->nb[1] % 16 == 0;
    const int x86 = ctx->q8_rounding == SAMHIP_Q8_ROUND_X86 ? 1 : 0;
    const char* variant = gemm_variant(w->type);
    if (!variant) return fail(SAMHIP_ERR_UNSUPPORTED, "mul_mat: no kernel for weight type %d", w->type);
    int rc = SAMHIP_OK;
    // activation staging and weight decode in one launch (aligned rows, K <= 5120)
    bool prepared = false;
    if (tall && aligned && K <= 5120) {
        rc = traced(ctx, prep_name(mode), w->type, M, N, K, [&]() -> int {
            prepared = launch_prep(mode, w->type, static_cast<const float*>(x->data), int64_t(x->nb[1] / 4), M, K, a,
                                   K, rs, x86, w->data, int64_t(w->nb[1]), N, wh, K, ctx->stream);
            HIP_TRY(hipGetLastError(), "staging and weight decode launch");
            return prepared ? SAMHIP_OK : fail(SAMHIP_ERR_UNSUPPORTED, "mul_mat: no staging kernel for this shape");
        });
        if (rc) return rc;
    }
    if (!prepared) {
        rc = traced(ctx, stage_name(mode), w->type, M, N, K, [&]() -> int {
            launch_stage_rows(mode, aligned, static_cast<const float*>(x->data), int64_t(x->nb[1] / 4), M, K, a, K,
                              rs, x86, ctx->stream);
            HIP_TRY(hipGetLastError(), "activation staging launch");
            return SAMHIP_OK;
        });
        if (rc) return rc;
    }
    if (tall) {
        if (!prepared) {
            rc = traced(ctx, dequant_name(w->type), w->type, M, N, K, [&]() -> int {
                launch_dequant_w_f16(w->type, w->data, int64_t(w->nb[1]), N, K, wh, K, ctx->stream);
                HIP_TRY(hipGetLastError(), "weight dequant launch");
                return SAMHIP_OK;
            });
            if (rc) return rc;
        }
        const int cfg = ctx->gemm_cfg >= 0 ? ctx->gemm_cfg : gemm_f16_pick_plain(M, N, K, ctx->cus);
        variant = gemm_f16_config_name(cfg);
        rc = traced(ctx, variant, w->type, M, N, K, [&]() -> int {
            launch_gemm_f16(cfg, a, K, rs, wh, K, static_cast<float*>(y->data), int64_t(y->nb[1] / 4), M, N, K,
                            ctx->cus, ctx->stream);
            HIP_TRY(hipGetLastError(), "gemm launch");
            return SAMHIP_OK;
        });
    } else if (M <= kSkinnyMaxM) {
        variant = skinny_variant(w->type, M, N);
        rc = traced(ctx, variant, w->type, M, N, K, [&]() -> int {
            if (!launch_skinny(w->type, a, K, rs, w->data, int64_t(w->nb[1]), static_cast<float*>(y->data),
                               int64_t(y->nb[1] / 4), M, N, K, ctx->stream))
                return fail(SAMHIP_ERR_UNSUPPORTED, "mul_mat: no skinny kernel for this shape");
            HIP_TRY(hipGetLastError(), "skinny launch");
            return SAMHIP_OK;
        });
        if (!rc) ctx->info.skinny_launches++;
    } else {
        rc = traced(ctx, variant, w->type, M, N, K, [&]() -> int {
            if (!launch_gemm(w->type, a, K, rs, w->data, int64_t(w->nb[1]), static_cast<float*>(y->data),
                             int64_t(y->nb[1] / 4), M, N, K, ctx->stream))
                return fail(SAMHIP_ERR_UNSUPPORTED, "mul_mat: no GEMM kernel for this shape");
            HIP_TRY(hipGetLastError(), "gemm launch");
            return SAMHIP_OK;
        });
    }
    if (rc) return rc;
    ctx->info.mul_mat_calls++;
    ctx->info.activation_launches++;
    if (tall || M > kSkinnyMaxM) ctx->info.gemm_launches++;
    ctx->info.activation_payload_peak_bytes = std::max<uint64_t>(ctx->info.activation_payload_peak_bytes, a_bytes);
    std::snprintf(ctx->info.kernel_variant, sizeof(ctx->info.kernel_variant), "%s", variant);
    return SAMHIP_OK;
}

int samhip_get_rows(samhip_context* ctx, const samhip_tensor* src, const samhip_tensor* ids, const samhip_tensor* dst) {
    if (!ctx || !src || !ids || !dst) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "get_rows: null argument");
    SAMHIP_NOT_WHILE_CAPTURING(ctx, "get_rows");
    const int t = src->type;
    if (t != T_F32 && t != T_F16 && !is_weight_type(t)) return fail(SAMHIP_ERR_UNSUPPORTED, "get_rows: unsupported source type %d", t);
    if (ids->type != T_I32 || dst->type != T_F32) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "get_rows: ids must be I32 and dst F32");
    const int64_t K = src->ne[0], rows = src->ne[1], n = ids->ne[0];
    if (K <= 0 || rows <= 0 || n <= 0 || K % 32 || K % block_elems(t))
        return fail(SAMHIP_ERR_INVALID_ARGUMENT, "get_rows: row width must be a positive multiple of the block size and 32");
    if (dst->ne[0] != K || dst->ne[1] != n || ids->nb[0] != 4 || dst->nb[0] != 4 || dst->nb[1] < size_t(4 * K))
        return fail(SAMHIP_ERR_INVALID_ARGUMENT, "get_rows: dst must be [K, n] F32 and ids contiguous I32");
    if (src->nb[1] < row_bytes(t, K) || !src->data || !ids->data || !dst->data)
        return fail(SAMHIP_ERR_INVALID_ARGUMENT, "get_rows: invalid source rows");
    for (int i = 2; i < 4; ++i)
        if (src->ne[i] != 1 || ids->ne[i] != 1 || dst->ne[i] != 1) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "get_rows: 2-D only");
    if (int rc = set_device(ctx)) return rc;
    HIP_TRY(hipMemsetAsync(ctx->flag, 0, sizeof(int), ctx->stream), "hipMemsetAsync");
    launch_dequant_rows(t, src->data, int64_t(src->nb[1]), static_cast<const int32_t*>(ids->data), rows,
                        static_cast<float*>(dst->data), int64_t(dst->nb[1] / 4), int(n), int(K), ctx->flag, ctx->stream);
    HIP_TRY(hipGetLastError(), "get_rows launch");
    int bad = 0;
    HIP_TRY(hipMemcpyAsync(&bad, ctx->flag, sizeof(int), hipMemcpyDeviceToHost, ctx->stream), "hipMemcpyAsync");
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    ctx->info.get_rows_calls++;
    if (bad) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "get_rows: row id out of range [0, %lld)", (long long)rows);
    return SAMHIP_OK;
}

int samhip_quantize_rows(samhip_context* ctx, int32_t type, const float* src, size_t src_row_stride, void* dst,
                         int64_t rows, int64_t k, int32_t q8_rounding) {
    if (!ctx || !src || !dst || rows <= 0 || k <= 0) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "quantize_rows: invalid argument");
    if (type != T_F16 && type != T_Q8_0 && type != T_Q8_1 && type != T_Q8_K && type != T_Q4_K && type != T_Q5_K &&
        type != T_Q6_K)
        return fail(SAMHIP_ERR_UNSUPPORTED, "quantize_rows: unsupported type %d", type);
    if (k % block_elems(type)) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "quantize_rows: k must be a multiple of %d", block_elems(type));
    if (src_row_stride < size_t(4 * k) || src_row_stride % 4 || reinterpret_cast<uintptr_t>(src) % 4)
        return fail(SAMHIP_ERR_INVALID_ARGUMENT, "quantize_rows: invalid source stride");
    if (q8_rounding != SAMHIP_Q8_ROUND_X86 && q8_rounding != SAMHIP_Q8_ROUND_REF)
        return fail(SAMHIP_ERR_INVALID_ARGUMENT, "quantize_rows: unknown Q8 rounding");
    if ((type == T_Q8_K) && reinterpret_cast<uintptr_t>(dst) % 4) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "quantize_rows: Q8_K dst must be 4-byte aligned");
    if (rows > (int64_t(1) << 30) || k > (int64_t(1) << 24)) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "quantize_rows: too large");
    if ((type == T_F16 || type == T_Q8_1) && reinterpret_cast<uintptr_t>(dst) % 2)
        return fail(SAMHIP_ERR_INVALID_ARGUMENT, "quantize_rows: F16 and Q8_1 dst must be 2-byte aligned");
    if (int rc = set_device(ctx)) return rc;
    if (type == T_F16)
        launch_cast_f16(src, int64_t(src_row_stride / 4), int(rows), int(k), static_cast<_Float16*>(dst), ctx->stream);
    else if (type == T_Q8_0 || type == T_Q8_K)
        launch_quantize_act(type, src, int64_t(src_row_stride / 4), int(rows), int(k), dst,
                            q8_rounding == SAMHIP_Q8_ROUND_X86 ? 1 : 0, ctx->stream);
    else if (type == T_Q8_1)
        launch_quantize_q8_1(src, int64_t(src_row_stride / 4), int(rows), int(k), dst, ctx->stream);
    else
        launch_quantize_weights(type, src, int64_t(src_row_stride / 4), int(rows), int(k), dst, ctx->stream);
    HIP_TRY(hipGetLastError(), "quantize launch");
    return SAMHIP_OK;
}

size_t samhip_q8_1_mmq_bytes(int64_t rows, int64_t k) {
    if (rows <= 0 || k <= 0) return 0;
    return size_t((k + 511) / 512) * 4 * size_t(rows) * 144;
}

int samhip_quantize_rows_q8_1_mmq(samhip_context* ctx, const float* src, size_t src_row_stride, void* dst,
                                  int64_t rows, int64_t k) {
    if (!ctx || !src || !dst || rows <= 0 || k <= 0 || k % 32)
        return fail(SAMHIP_ERR_INVALID_ARGUMENT, "native MMQ Q8 RHS needs nonempty 32-aligned rows");
    if (src_row_stride < size_t(4 * k) || src_row_stride % 4 || reinterpret_cast<uintptr_t>(src) % 4 ||
        reinterpret_cast<uintptr_t>(dst) % 4)
        return fail(SAMHIP_ERR_INVALID_ARGUMENT, "quantize_rows_q8_1_mmq: invalid stride or alignment");
    if (rows > (int64_t(1) << 24) || k > (int64_t(1) << 24))
        return fail(SAMHIP_ERR_INVALID_ARGUMENT, "quantize_rows_q8_1_mmq: too large");
    SAMHIP_NOT_WHILE_CAPTURING(ctx, "quantize_rows_q8_1_mmq");
    if (int rc = set_device(ctx)) return rc;
    HIP_TRY(hipMemsetAsync(ctx->flag, 0, sizeof(int), ctx->stream), "hipMemsetAsync");
    launch_quantize_q8_1_mmq(src, int64_t(src_row_stride / 4), int(rows), int(k), dst, ctx->flag, ctx->stream);
    HIP_TRY(hipGetLastError(), "quantize_rows_q8_1_mmq launch");
    return read_range_flag(ctx);
}

int samhip_dequantize_rows(samhip_context* ctx, int32_t type, const void* src, size_t src_row_stride, float* dst,
                           int64_t rows, int64_t k) {
    if (!ctx || !src || !dst || rows <= 0 || k <= 0) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "dequantize_rows: invalid argument");
    if (!is_weight_type(type) && type != T_Q8_K && type != T_F16)
        return fail(SAMHIP_ERR_UNSUPPORTED, "dequantize_rows: unsupported type %d", type);
    if (type == T_F16 && (k % 32 || reinterpret_cast<uintptr_t>(src) % 2 || src_row_stride % 2))
        return fail(SAMHIP_ERR_INVALID_ARGUMENT, "dequantize_rows: F16 rows must be 32-value groups, 2-byte aligned");
    if (k % block_elems(type) || src_row_stride < row_bytes(type, k))
        return fail(SAMHIP_ERR_INVALID_ARGUMENT, "dequantize_rows: invalid row shape");
    if (rows > (int64_t(1) << 30) || k > (int64_t(1) << 24)) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "dequantize_rows: too large");
    if (int rc = set_device(ctx)) return rc;
    launch_dequant_rows(type, src, int64_t(src_row_stride), nullptr, rows, dst, k, int(rows), int(k), nullptr, ctx->stream);
    HIP_TRY(hipGetLastError(), "dequantize launch");
    return SAMHIP_OK;
}

int samhip_validate_quantized_payload(int32_t type, int64_t ne0, int64_t rows, const void* host_bytes, size_t bytes) {
    if (!is_weight_type(type)) return fail(SAMHIP_ERR_UNSUPPORTED, "invalid quantized SAM tensor layout");
    if (ne0 <= 0 || rows <= 0 || ne0 % block_elems(type)) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "invalid quantized SAM tensor layout");
    const size_t rb = row_bytes(type, ne0);
    if (size_t(rows) > SIZE_MAX / rb || size_t(rows) * rb != bytes || (!host_bytes && bytes))
        return fail(SAMHIP_ERR_INVALID_ARGUMENT, "quantized SAM tensor payload size does not match its shape");
    const uint8_t* p = static_cast<const uint8_t*>(host_bytes);
    const int bb = block_bytes(type), be = block_elems(type);
    auto half_value = [](const uint8_t* q) {
        const uint16_t h = uint16_t(q[0] | (q[1] << 8));
        const uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
        if (e == 0x1f) return m ? NAN : ((h & 0x8000) ? -INFINITY : INFINITY);
        float v = e ? std::ldexp(float(m | 0x400), int(e) - 25) : std::ldexp(float(m), -24);
        return (h & 0x8000) ? -v : v;
    };
    for (size_t b = 0; b < size_t(rows) * size_t(ne0 / be); ++b) {
        const uint8_t* blk = p + b * bb;
        const float d = half_value(blk + (type == T_Q6_K ? bb - 2 : 0));
        if (!std::isfinite(d)) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "non-finite quantized SAM block scale");
        if ((type == T_Q4_K || type == T_Q5_K) && !std::isfinite(half_value(blk + 2)))
            return fail(SAMHIP_ERR_INVALID_ARGUMENT, "non-finite quantized SAM block minimum scale");
        // With finite scales the decoded values of these formats are bounded
        // by |d| * 127 (Q8_0), |d| * 63 * 31 + |dmin| * 63 (Q4_K/Q5_K) and
        // |d| * 128 * 32 (Q6_K), all finite in F32.
    }
    return SAMHIP_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// SAM 3 vision encoder
// ---------------------------------------------------------------------------

namespace {

int ensure_work(samhip_context* ctx, size_t bytes) {
    if (bytes <= ctx->work_bytes) return SAMHIP_OK;
    if (ctx->work) {
        HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
        HIP_TRY(hipFree(ctx->work), "hipFree");
        ctx->work = nullptr;
        ctx->work_bytes = 0;
    }
    const size_t rounded = (bytes + (size_t(1) << 20) - 1) & ~((size_t(1) << 20) - 1);
    HIP_TRY(hipMalloc(&ctx->work, rounded), "hipMalloc vision workspace");
    ctx->work_bytes = rounded;
    return SAMHIP_OK;
}

// Carves aligned sub-buffers out of one allocation.
struct Carve {
    size_t used = 0;
    size_t take(size_t bytes) {
        const size_t at = used;
        used = (used + bytes + 255) & ~size_t(255);
        return at;
    }
};

bool layer_norm_supported(int64_t n) {
    return n >= 256 && n <= 2048 && n % 256 == 0 && n != 1792;
}

// Row r of a window-order product (ggml_win_part of a gw x gh grid) returns
// to grid row row_map[r] (ggml_win_unpart); built on the host once per shape.
int ensure_row_map(samhip_context* ctx, int gw, int gh, int ws) {
    if (ctx->row_map && ctx->row_map_key[0] == gw && ctx->row_map_key[1] == gh && ctx->row_map_key[2] == ws)
        return SAMHIP_OK;
    std::vector<int> map(size_t(gw) * gh);
    const int npx = gw / ws;
    for (int gy = 0; gy < gh; ++gy)
        for (int gx = 0; gx < gw; ++gx) {
            const int win = (gy / ws) * npx + gx / ws;
            map[size_t(win) * ws * ws + (gy % ws) * ws + gx % ws] = gy * gw + gx;
        }
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    if (ctx->row_map) HIP_TRY(hipFree(ctx->row_map), "hipFree");
    ctx->row_map = nullptr;
    HIP_TRY(hipMalloc(&ctx->row_map, map.size() * sizeof(int)), "hipMalloc row map");
    HIP_TRY(hipMemcpy(ctx->row_map, map.data(), map.size() * sizeof(int), hipMemcpyHostToDevice), "hipMemcpy row map");
    ctx->row_map_key[0] = gw;
    ctx->row_map_key[1] = gh;
    ctx->row_map_key[2] = ws;
    return SAMHIP_OK;
}

// Activation rows as Q8_0 codes [M][ld] and F32 block maxima [M][ld / 32]
// (what Epilogue::q8 writes).
struct CodeRows {
    const int8_t* codes = nullptr;
    const float* amax = nullptr;
    int64_t ld = 0;
};

// Tall product through staging (with the producing node folded in, `pre`;
// or from Q8_0 code rows, `in`) + weight decode + the fp16 GEMM with an
// epilogue; x rows are K contiguous floats (16-byte aligned), y rows ldy.
int linear(samhip_context* ctx, const samhip_tensor& w, const float* x, int M, float* y, int64_t ldy,
           const Epilogue& ep, const char* what, const RowPre& pre = RowPre{}, const CodeRows* in = nullptr) {
    const int K = int(w.ne[0]), N = int(w.ne[1]);
    auto align256 = [](size_t v) { return (v + 255) & ~size_t(255); };
    const size_t rs_offset = align256(size_t(M) * size_t(K) * 2);
    const size_t w_offset = align256(rs_offset + size_t(M) * 4);
    if (int rc = ensure_staging(ctx, w_offset + size_t(N) * size_t(K) * 2)) return rc;
    uint8_t* base = static_cast<uint8_t*>(ctx->staging);
    _Float16* a = reinterpret_cast<_Float16*>(base);
    float* rs = reinterpret_cast<float*>(base + rs_offset);
    _Float16* wh = reinterpret_cast<_Float16*>(base + w_offset);
    const int mode = ctx->compute == SAMHIP_COMPUTE_F16 ? T_F16 : vec_dot_type(w.type);
    const int x86 = ctx->q8_rounding == SAMHIP_Q8_ROUND_X86 ? 1 : 0;
    int rc = traced(ctx, in ? "stage_codes_q8_0" : prep_name(mode), w.type, M, N, K, [&]() -> int {
        const bool ok = in ? launch_prep_codes(in->codes, in->amax, in->ld, M, K, a, K, rs, w.type, w.data,
                                               int64_t(w.nb[1]), N, wh, K, ctx->stream)
                           : launch_prep(mode, w.type, x, K, M, K, a, K, rs, x86, w.data, int64_t(w.nb[1]), N, wh, K,
                                         ctx->stream, pre);
        if (!ok) return fail(SAMHIP_ERR_UNSUPPORTED, "%s: no staging kernel for K = %d", what, K);
        HIP_TRY(hipGetLastError(), "staging and weight decode launch");
        return SAMHIP_OK;
    });
    if (rc) return rc;
    rc = traced(ctx, what, w.type, M, N, K, [&]() -> int {
        if (!launch_gemm_f16_epi(a, K, rs, wh, K, y, ldy, M, N, K, ctx->cus, ep, ctx->stream))
            return fail(SAMHIP_ERR_UNSUPPORTED, "%s: no GEMM epilogue variant", what);
        HIP_TRY(hipGetLastError(), "gemm launch");
        return SAMHIP_OK;
    });
    if (rc) return rc;
    ctx->info.mul_mat_calls++;
    ctx->info.activation_launches++;
    ctx->info.gemm_launches++;
    return SAMHIP_OK;
}

// 0 when the packed weight fits the block, else a status with the message set.
int weight_check(const samhip_tensor& t, int64_t K, int64_t N, int64_t M, const char* name) {
    const char* why = nullptr;
    if (!is_weight_type(t.type)) why = "type must be Q8_0, Q4_K, Q5_K or Q6_K";
    else if (t.ne[0] != K || t.ne[1] != N || t.ne[2] != 1 || t.ne[3] != 1) why = "shape differs from the block's";
    else if (K % block_elems(t.type)) why = "width is not a multiple of its block";
    else if (t.nb[0] != size_t(block_bytes(t.type)) || t.nb[1] < row_bytes(t.type, K)) why = "bad strides";
    else if (!t.data || reinterpret_cast<uintptr_t>(t.data) % 2 || t.nb[1] % 2) why = "bad data pointer";
    if (why) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "vit_block: %s weight: %s", name, why);
    if (K > 5120 || !gemm_f16_supported(int(M), int(N), int(K), K, K))
        return fail(SAMHIP_ERR_UNSUPPORTED, "vit_block: %s weight: width %lld unsupported (multiple of 128, at most 5120)",
                    name, (long long)K);
    return SAMHIP_OK;
}

}  // namespace

extern "C" {

int samhip_layer_norm(samhip_context* ctx, const float* x, float* y, int64_t rows, int64_t n, const float* w,
                      const float* b, float eps) {
    if (!ctx) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "null context");
    SAMHIP_NOT_WHILE_CAPTURING(ctx, "layer_norm");
    if (!x || !y || rows <= 0 || rows > (int64_t(1) << 30)) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "layer_norm: bad operands");
    if (!layer_norm_supported(n)) return fail(SAMHIP_ERR_UNSUPPORTED, "layer_norm: row width %lld unsupported", (long long)n);
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(y) % 16)
        return fail(SAMHIP_ERR_INVALID_ARGUMENT, "layer_norm: rows must be 16-byte aligned");
    if (!(eps >= 0.f)) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "layer_norm: eps must be nonnegative");
    if (int rc = set_device(ctx)) return rc;
    return traced(ctx, "layer_norm", T_F32, rows, n, 0, [&]() -> int {
        launch_layer_norm(x, nullptr, 1, 1, int(rows), 0, w, b, eps, y, int(rows), int(n), ctx->stream);
        HIP_TRY(hipGetLastError(), "layer_norm launch");
        return SAMHIP_OK;
    });
}

int samhip_flash_attn(samhip_context* ctx, const float* q, const float* k, const float* v, int64_t ld, float* out,
                      int64_t batches, int64_t n, int32_t heads, int32_t head_dim, float scale) {
    if (!ctx) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "null context");
    SAMHIP_NOT_WHILE_CAPTURING(ctx, "flash_attn");
    if (!q || !k || !v || !out || batches <= 0 || n <= 0 || heads <= 0)
        return fail(SAMHIP_ERR_INVALID_ARGUMENT, "flash_attn: bad operands");
    if (head_dim != 64) return fail(SAMHIP_ERR_UNSUPPORTED, "flash_attn: head_dim %d unsupported (64)", head_dim);
    if (ld < int64_t(heads) * 64 || ld % 4 || batches * n > (int64_t(1) << 26) || heads > 4096 || batches > 65535)
        return fail(SAMHIP_ERR_INVALID_ARGUMENT, "flash_attn: bad row stride or sizes");
    for (const float* p : {q, k, v, static_cast<const float*>(out)})
        if (reinterpret_cast<uintptr_t>(p) % 16) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "flash_attn: 16-byte alignment");
    if (!std::isfinite(scale)) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "flash_attn: scale");
    if (int rc = set_device(ctx)) return rc;
    // F32-accurate, as the reference requests GGML_PREC_F32 for every
    // FLASH_ATTN_EXT node (src/runtime/ggml/graph.hpp:64)
    const int64_t np = (n + 63) / 64 * 64;
    const size_t packed = size_t(batches) * heads * np * 64 * 2;
    Carve c;
    size_t off[6];
    for (size_t& o : off) o = c.take(packed);
    const int splits = attention_splits(int(batches), heads, int(n), true, ctx->cus, ctx->attn_splits);
    const size_t att_bytes = attention_scratch_bytes(int(batches), heads, int(n), splits);
    const size_t o_att = c.take(att_bytes);
    if (int rc = ensure_work(ctx, c.used)) return rc;
    uint8_t* wb = static_cast<uint8_t*>(ctx->work);
    float* att_scratch = att_bytes ? reinterpret_cast<float*>(wb + o_att) : nullptr;
    AttnOperands ops;
    _Float16** parts[6] = {&ops.q, &ops.k, &ops.v, &ops.ql, &ops.kl, &ops.vl};
    for (int i = 0; i < 6; ++i) *parts[i] = reinterpret_cast<_Float16*>(wb + off[i]);
    int rc = traced(ctx, "vit_pack_qkv", T_F32, batches * n, heads * 64, 0, [&]() -> int {
        launch_pack_qkv(q, k, v, ld, nullptr, scale, ops, int(batches), heads, int(n), ctx->stream);
        HIP_TRY(hipGetLastError(), "pack launch");
        return SAMHIP_OK;
    });
    if (rc) return rc;
    return traced(ctx, attention_name(splits), T_F32, batches * n, heads * 64, n, [&]() -> int {
        if (!launch_attention(ops, out, int64_t(heads) * 64, int(batches), heads, int(n), splits, att_scratch,
                              att_bytes, ctx->stream))
            return fail(SAMHIP_ERR_UNSUPPORTED, "flash_attn: no attention launch for this grid");
        HIP_TRY(hipGetLastError(), "attention launch");
        return SAMHIP_OK;
    });
}

int samhip_vit_block(samhip_context* ctx, const samhip_vit_block_desc* d, float* x) {
    if (!ctx) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "null context");
    SAMHIP_NOT_WHILE_CAPTURING(ctx, "vit_block");
    if (!d || !x) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "vit_block: null argument");
    if (d->version != SAMHIP_ABI_VERSION) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "vit_block: descriptor version");
    const int64_t E = d->embed, H = d->heads, MLP = d->mlp, GW = d->grid_w, GH = d->grid_h, WS = d->window;
    if (E <= 0 || H <= 0 || MLP <= 0 || GW <= 0 || GH <= 0 || WS < 0 || GW * GH > (int64_t(1) << 22))
        return fail(SAMHIP_ERR_INVALID_ARGUMENT, "vit_block: nonpositive or oversized dimension");
    if (E != H * 64) return fail(SAMHIP_ERR_UNSUPPORTED, "vit_block: head_dim must be 64 (embed = 64 * heads)");
    if (!layer_norm_supported(E)) return fail(SAMHIP_ERR_UNSUPPORTED, "vit_block: embed must be a multiple of 256 up to 2048");
    if (WS > 0 && (GW % WS || GH % WS))
        return fail(SAMHIP_ERR_UNSUPPORTED, "vit_block: grid sides must be multiples of the window");
    if (!d->norm1_w || !d->norm1_b || !d->norm2_w || !d->norm2_b || !d->qkv_b || !d->proj_b || !d->fc1_b || !d->fc2_b)
        return fail(SAMHIP_ERR_INVALID_ARGUMENT, "vit_block: null norm or bias pointer");
    const struct { const samhip_tensor* t; int64_t k, n; const char* name; } weights[] = {
        {&d->qkv_w, E, 3 * E, "qkv"}, {&d->proj_w, E, E, "proj"}, {&d->fc1_w, E, MLP, "fc1"}, {&d->fc2_w, MLP, E, "fc2"}};
    for (const auto& w : weights)
        if (int rc = weight_check(*w.t, w.k, w.n, GW * GH, w.name)) return rc;
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(d->freqs_cis) % 16)
        return fail(SAMHIP_ERR_INVALID_ARGUMENT, "vit_block: x and freqs_cis must be 16-byte aligned");
    if (d->attention_type != T_F32 && d->attention_type != T_F16)
        return fail(SAMHIP_ERR_UNSUPPORTED, "vit_block: attention type must be F32 or F16");
    const bool precise = d->attention_type == T_F32;
    if (int rc = set_device(ctx)) return rc;

    const int64_t T = GW * GH, per = WS > 0 ? WS * WS : T, B = T / per, np = (per + 63) / 64 * 64;
    if (B * H * np * 64 >= (int64_t(1) << 31) || B > 65535)
        return fail(SAMHIP_ERR_UNSUPPORTED, "vit_block: grid too large");
    Carve c;
    const size_t o_ln = c.take(size_t(T * E) * 4), o_x1 = c.take(size_t(T * E) * 4),
                 o_h1 = c.take(size_t(T * MLP) * 4);
    const size_t packed = size_t(B * H * np * 64) * 2;
    size_t o_ops[6];
    for (int i = 0; i < (precise ? 6 : 3); ++i) o_ops[i] = c.take(packed);
    const int splits = attention_splits(int(B), int(H), int(per), precise, ctx->cus, ctx->attn_splits);
    const size_t att_bytes = attention_scratch_bytes(int(B), int(H), int(per), splits);
    const size_t o_att = c.take(att_bytes);
    if (int rc = ensure_work(ctx, c.used)) return rc;
    uint8_t* wb = static_cast<uint8_t*>(ctx->work);
    float* att_scratch = att_bytes ? reinterpret_cast<float*>(wb + o_att) : nullptr;
    float* ln = reinterpret_cast<float*>(wb + o_ln);
    float* x1 = reinterpret_cast<float*>(wb + o_x1);
    float* h1 = reinterpret_cast<float*>(wb + o_h1);
    AttnOperands ops;
    _Float16** parts[6] = {&ops.q, &ops.k, &ops.v, &ops.ql, &ops.kl, &ops.vl};
    for (int i = 0; i < (precise ? 6 : 3); ++i) *parts[i] = reinterpret_cast<_Float16*>(wb + o_ops[i]);
    const int iT = int(T);

    // attention half: LN1 folded into the qkv staging (rows leave in window
    // order), qkv + bias, RoPE and packing, attention, proj + bias +
    // unpartition + residual -> x1
    if (WS > 0)
        if (int rc = ensure_row_map(ctx, int(GW), int(GH), int(WS))) return rc;
    RowPre ln1;
    ln1.kind = PRE_LAYER_NORM;
    ln1.w = d->norm1_w;
    ln1.b = d->norm1_b;
    ln1.eps = 1e-5f;
    ln1.ws = int(WS);
    ln1.gw = int(GW);
    // qkv + bias, written by the product's epilogue as the per-head fp16
    // attention operands (RoPE on q and k, q times 1/8)
    Epilogue e_qkv;
    e_qkv.bias = d->qkv_b;
    e_qkv.pack[0] = ops.q;
    e_qkv.pack[1] = ops.k;
    e_qkv.pack[2] = ops.v;
    e_qkv.pack_lo[0] = ops.ql;
    e_qkv.pack_lo[1] = ops.kl;
    e_qkv.pack_lo[2] = ops.vl;
    e_qkv.freqs = d->freqs_cis;
    e_qkv.embed = int(E);
    e_qkv.per = int(per);
    e_qkv.np = int(np);
    e_qkv.heads = int(H);
    e_qkv.q_scale = 0.125f;
    int rc = linear(ctx, d->qkv_w, x, iT, nullptr, 3 * E, e_qkv, "vit_qkv", ln1);
    if (rc) return rc;
    if (np != per) {
        rc = traced(ctx, "vit_zero_pad", T_F32, T, E, per, [&]() -> int {
            launch_zero_pad(ops, int(B), int(H), int(per), ctx->stream);
            HIP_TRY(hipGetLastError(), "zero pad launch");
            return SAMHIP_OK;
        });
        if (rc) return rc;
    }
    rc = traced(ctx, attention_name(splits), T_F32, T, E, per, [&]() -> int {
        if (!launch_attention(ops, ln, E, int(B), int(H), int(per), splits, att_scratch, att_bytes, ctx->stream))
            return fail(SAMHIP_ERR_UNSUPPORTED, "vit_block: no attention launch for this grid");
        HIP_TRY(hipGetLastError(), "attention launch");
        return SAMHIP_OK;
    });
    if (rc) return rc;
    Epilogue e_proj;
    e_proj.bias = d->proj_b;
    e_proj.res = x;
    if (WS > 0) e_proj.row_map = ctx->row_map;
    if ((rc = linear(ctx, d->proj_w, ln, iT, x1, E, e_proj, "vit_proj"))) return rc;

    // MLP half: LN2 folded into the fc1 staging, fc1 + bias, erf-GELU folded
    // into the fc2 staging, fc2 + bias + residual -> x
    RowPre ln2 = ln1;
    ln2.w = d->norm2_w;
    ln2.b = d->norm2_b;
    ln2.ws = 0;
    Epilogue e_fc1;
    e_fc1.bias = d->fc1_b;
    Epilogue e_fc2;
    e_fc2.bias = d->fc2_b;
    e_fc2.res = x1;
    // Opt-in: with a Q8_0 fc2 in native compute, fc1's epilogue applies the
    // erf-GELU and packs fc2's Q8_0 blocks itself (codes and F32 block
    // maxima, 1.125 bytes per value in h1's space instead of 4), and fc2's
    // staging expands them: the same operand bits as staging the F32 rows.
    if (ctx->vit_fc1_codes && d->fc2_w.type == T_Q8_0 && ctx->compute != SAMHIP_COMPUTE_F16 && MLP % 32 == 0) {
        CodeRows rows;
        rows.codes = reinterpret_cast<const int8_t*>(h1);
        rows.amax = reinterpret_cast<const float*>(reinterpret_cast<const uint8_t*>(h1) +
                                                   ((size_t(T * MLP) + 255) & ~size_t(255)));
        rows.ld = MLP;
        e_fc1.gelu = true;
        e_fc1.q8 = const_cast<int8_t*>(rows.codes);
        e_fc1.q8_amax = const_cast<float*>(rows.amax);
        e_fc1.q8_ld = MLP;
        e_fc1.q8_x86 = ctx->q8_rounding == SAMHIP_Q8_ROUND_X86;
        if ((rc = linear(ctx, d->fc1_w, x1, iT, nullptr, MLP, e_fc1, "vit_fc1", ln2))) return rc;
        return linear(ctx, d->fc2_w, nullptr, iT, x, E, e_fc2, "vit_fc2", RowPre{}, &rows);
    }
    if ((rc = linear(ctx, d->fc1_w, x1, iT, h1, MLP, e_fc1, "vit_fc1", ln2))) return rc;
    RowPre gelu;
    gelu.kind = PRE_GELU;
    return linear(ctx, d->fc2_w, h1, iT, x, E, e_fc2, "vit_fc2", gelu);
}

int samhip_vit_prefix(samhip_context* ctx, const samhip_vit_prefix_desc* d, const float* image, float* x) {
    if (!ctx) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "null context");
    SAMHIP_NOT_WHILE_CAPTURING(ctx, "vit_prefix");
    if (!d || !image || !x) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "vit_prefix: null argument");
    if (d->version != SAMHIP_ABI_VERSION) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "vit_prefix: descriptor version");
    if (!d->patch_w || !d->pos_embed || !d->ln_pre_w || !d->ln_pre_b)
        return fail(SAMHIP_ERR_INVALID_ARGUMENT, "vit_prefix: null weight pointer");
    const int64_t img = d->image_size, p = d->patch, E = d->embed, pg = d->pos_grid;
    if (img <= 0 || p <= 0 || E <= 0 || pg <= 0 || img % p || img > 16384 || p > 64)
        return fail(SAMHIP_ERR_INVALID_ARGUMENT, "vit_prefix: image size must be a positive multiple of the patch");
    const int64_t grid = img / p;
    if (grid % pg) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "vit_prefix: grid must be a multiple of pos_grid");
    if (!layer_norm_supported(E)) return fail(SAMHIP_ERR_UNSUPPORTED, "vit_prefix: embed must be a multiple of 256 up to 2048");
    const int64_t kp = (3 * p * p + 127) / 128 * 128, T = grid * grid;
    if (3 * kp > 5120 * 4) return fail(SAMHIP_ERR_UNSUPPORTED, "vit_prefix: patch too large");
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(d->pos_embed) % 16)
        return fail(SAMHIP_ERR_INVALID_ARGUMENT, "vit_prefix: 16-byte alignment");
    if (int rc = set_device(ctx)) return rc;
    Carve c;
    const size_t o_a = c.take(size_t(T * 3 * kp) * 2), o_rs = c.take(size_t(T) * 4),
                 o_w = c.take(size_t(E * 3 * kp) * 2), o_conv = c.take(size_t(T * E) * 4);
    if (int rc = ensure_work(ctx, c.used)) return rc;
    uint8_t* wb = static_cast<uint8_t*>(ctx->work);
    _Float16* a = reinterpret_cast<_Float16*>(wb + o_a);
    float* rs = reinterpret_cast<float*>(wb + o_rs);
    _Float16* w = reinterpret_cast<_Float16*>(wb + o_w);
    float* conv = reinterpret_cast<float*>(wb + o_conv);
    int rc = traced(ctx, "vit_patch_operands", T_F32, T, E, 3 * kp, [&]() -> int {
        launch_patch_columns(image, int(img), int(p), a, rs, int(kp), ctx->stream);
        launch_patch_kernel(d->patch_w, int(E), int(p), w, int(kp), ctx->stream);
        HIP_TRY(hipGetLastError(), "patch operand launch");
        return SAMHIP_OK;
    });
    if (rc) return rc;
    rc = traced(ctx, "vit_patch_gemm", T_F32, T, E, 3 * kp, [&]() -> int {
        if (!launch_gemm_f16_epi(a, 3 * kp, rs, w, 3 * kp, conv, E, int(T), int(E), int(3 * kp), ctx->cus, Epilogue{},
                                 ctx->stream))
            return fail(SAMHIP_ERR_UNSUPPORTED, "vit_prefix: no GEMM variant");
        HIP_TRY(hipGetLastError(), "patch gemm launch");
        return SAMHIP_OK;
    });
    if (rc) return rc;
    return traced(ctx, "vit_layer_norm", T_F32, T, E, 0, [&]() -> int {
        launch_layer_norm(conv, d->pos_embed, int(pg), int(grid), int(grid), 0, d->ln_pre_w, d->ln_pre_b, 1e-5f, x,
                          int(T), int(E), ctx->stream);
        HIP_TRY(hipGetLastError(), "layer_norm launch");
        return SAMHIP_OK;
    });
}

int samhip_vit_neck(samhip_context* ctx, const samhip_vit_neck_desc* d, const float* x, float* level0, float* level1,
                    float* level2, float* level3) {
    if (!ctx) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "null context");
    SAMHIP_NOT_WHILE_CAPTURING(ctx, "vit_neck");
    if (!d || !x) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "vit_neck: null argument");
    if (d->version != SAMHIP_ABI_VERSION) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "vit_neck: descriptor version");
    if (d->columns_type != T_F32 && d->columns_type != T_F16)
        return fail(SAMHIP_ERR_UNSUPPORTED, "vit_neck: columns type must be F32 or F16");
    float* level[4] = {level0, level1, level2, level3};
    const int64_t g = d->grid, E = d->embed, mid = d->mid, D = d->dim;
    if (g <= 0 || g > 4096 || E <= 0 || mid <= 0 || D <= 0 || E > 8192 || mid > 8192 || D > 8192 || E % 4 ||
        mid % 4 || D % 4)
        return fail(SAMHIP_ERR_INVALID_ARGUMENT,
                    "vit_neck: grid (1..4096) and channel counts (multiples of 4, at most 8192) out of range");
    if (level[3] && g % 2) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "vit_neck: level 3 needs an even grid");
    if (reinterpret_cast<uintptr_t>(x) % 16) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "vit_neck: 16-byte alignment");
    for (float* p : level)
        if (reinterpret_cast<uintptr_t>(p) % 16) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "vit_neck: 16-byte alignment");
    const samhip_neck_scale* sc = d->scales;
    auto convs = [](const samhip_neck_scale& s) { return s.conv1x1_w && s.conv1x1_b && s.conv3x3_w && s.conv3x3_b; };
    if ((level[0] && !(convs(sc[0]) && sc[0].deconv1_w && sc[0].deconv1_b && sc[0].deconv2_w && sc[0].deconv2_b)) ||
        (level[1] && !(convs(sc[1]) && sc[1].deconv1_w && sc[1].deconv1_b)) || (level[2] && !convs(sc[2])) ||
        (level[3] && !convs(sc[3])))
        return fail(SAMHIP_ERR_INVALID_ARGUMENT, "vit_neck: null weight pointer for a requested level");
    if (!level[0] && !level[1] && !level[2] && !level[3]) return SAMHIP_OK;
    if (int rc = set_device(ctx)) return rc;

    // Operands.  Split (F32 columns) A rows are stored [hi | lo] and read as
    // [hi | hi | lo] (A_REPEAT) against B rows [hi | lo | hi]; F16 columns
    // are one fp16 part.  A 3x3 convolution over a map of 128k channels
    // gathers its im2col rows from the map's own operand rows (A_CONV3, one
    // power-of-two scale for the whole map); other channel counts build the
    // im2col rows.
    const bool f16 = d->columns_type == T_F16;
    const int64_t parts = f16 ? 1 : 3, stored = f16 ? 1 : 2;
    auto kpad = [](int64_t k) { return (k + 127) / 128 * 128; };
    const int64_t T = g * g, T2 = 4 * T, T4 = 16 * T, kpE = kpad(E), kpM = kpad(mid), kpD = kpad(D),
                  kp9 = kpad(9 * D);
    const bool gather3 = D % 128 == 0;
    constexpr int64_t kMaxOperand = 0x7fffffff;   // 32-bit buffer offsets of the GEMM
    auto chunk_rows = [&](int64_t rows, int64_t lda) {
        return std::min(rows, std::max<int64_t>(256, kMaxOperand / (lda * 2) / 256 * 256));
    };
    // (rows, stored row halves) of every A operand built into `at`: 1x1 and
    // pooled inputs in chunks, 3x3 inputs whole (gathered) or in chunks
    std::vector<std::pair<int64_t, int64_t>> conv_ops;
    const bool need_ax = level[0] || level[1] || (level[2] && !f16);
    auto add3 = [&](int64_t rows) {
        conv_ops.push_back(gather3 ? std::make_pair(rows, stored * D)
                                   : std::make_pair(chunk_rows(rows, stored * kp9), stored * kp9));
    };
    if (level[0]) {
        conv_ops.push_back({chunk_rows(T4, stored * kpD), stored * kpD});
        add3(T4);
    }
    if (level[1]) {
        conv_ops.push_back({chunk_rows(T2, stored * kpM), stored * kpM});
        add3(T2);
    }
    if (level[2]) {
        if (f16) conv_ops.push_back({T, kpE});
        add3(T);
    }
    if (level[3]) {
        conv_ops.push_back({chunk_rows(T / 4, stored * kpE), stored * kpE});
        add3(T / 4);
    }
    // whole-map operands: the split ViT output, the second deconvolution's
    // input and the gathered 3x3 inputs
    if ((need_ax && T * 2 * kpE * 2 > kMaxOperand) || (level[0] && T2 * 2 * kpM * 2 > kMaxOperand) ||
        (gather3 && (level[0] ? T4 : T2) * stored * D * 2 > kMaxOperand))
        return fail(SAMHIP_ERR_UNSUPPORTED, "vit_neck: map too large for one product");
    int64_t at_halves = level[0] ? T2 * 2 * kpM : 0, max_rows = level[0] ? T2 : 0;
    for (auto [rows, lda] : conv_ops) {
        at_halves = std::max(at_halves, rows * lda);
        max_rows = std::max(max_rows, rows);
    }
    const int64_t wb_halves = std::max({4 * mid * 3 * kpE, 4 * D * 3 * kpM, D * parts * kp9, D * parts * kpE,
                                        D * parts * kpM, D * parts * kpD});
    const int64_t t1_floats = std::max({level[0] || level[1] ? T2 * mid : 0, T * D, T / 4 * D});
    const int64_t t2_floats = level[0] ? T4 * D : T2 * D;
    const int64_t part_floats = std::max<int64_t>(1024, (std::max(E, mid) + 63) / 64 * 4 * std::max(mid, D));
    Carve c;
    const size_t o_ax = c.take(need_ax ? size_t(T * 2 * kpE) * 2 : 0), o_rsx = c.take(size_t(T) * 4),
                 o_at = c.take(size_t(at_halves) * 2), o_rst = c.take(size_t(max_rows) * 4),
                 o_wb = c.take(size_t(wb_halves) * 2), o_cs = c.take(size_t(4 * std::max(mid, D)) * 4),
                 o_part = c.take(size_t(part_floats) * 4), o_t1 = c.take(size_t(t1_floats) * 4),
                 o_t2 = c.take(size_t(t2_floats) * 4), o_t3 = c.take(level[0] ? size_t(T4 * D) * 4 : 0);
    if (int rc = ensure_work(ctx, c.used)) return rc;
    uint8_t* wk = static_cast<uint8_t*>(ctx->work);
    _Float16* ax = reinterpret_cast<_Float16*>(wk + o_ax);
    float* rsx = reinterpret_cast<float*>(wk + o_rsx);
    _Float16* at = reinterpret_cast<_Float16*>(wk + o_at);
    float* rst = reinterpret_cast<float*>(wk + o_rst);
    _Float16* wb = reinterpret_cast<_Float16*>(wk + o_wb);
    float* cs = reinterpret_cast<float*>(wk + o_cs);
    float* part = reinterpret_cast<float*>(wk + o_part);
    float* t1 = reinterpret_cast<float*>(wk + o_t1);
    float* t2 = reinterpret_cast<float*>(wk + o_t2);
    float* t3 = reinterpret_cast<float*>(wk + o_t3);

    auto columns = [&](int src, bool split, const float* in, int64_t W, int64_t H, int64_t C, int64_t kp,
                       int64_t row0, int64_t rows, _Float16* a, float* rs) -> int {
        return traced(ctx, "neck_columns", T_F32, rows, 0, kp, [&]() -> int {
            launch_neck_columns(src, split, in, int(W), int(H), int(C), int(kp), row0, int(rows), a, rs, ctx->stream);
            HIP_TRY(hipGetLastError(), "neck columns launch");
            return SAMHIP_OK;
        });
    };
    auto weights = [&](bool deconv, bool split, const float* w, int k, int64_t cin, int64_t cout, int64_t kp) -> int {
        return traced(ctx, "neck_weights", T_F32, deconv ? 4 * cout : cout, 0, kp, [&]() -> int {
            launch_neck_weights(deconv, split, w, k, int(cin), int(cout), int(kp), wb, cs, part, ctx->stream);
            HIP_TRY(hipGetLastError(), "neck weights launch");
            return SAMHIP_OK;
        });
    };
    // product of A (M rows of lda stored halves, read as K columns) with the
    // prepared B rows (K halves each)
    auto gemm = [&](const char* name, const _Float16* a, int64_t lda, int64_t K, const float* rs, float* y,
                    int64_t ldy, int64_t M, int64_t N, const Epilogue& ep, const AOperand& op) -> int {
        if (!gemm_f16_supported(int(M), int(N), int(K), lda, K))
            return fail(SAMHIP_ERR_UNSUPPORTED, "vit_neck: product %lld x %lld x %lld out of range", (long long)M,
                        (long long)N, (long long)K);
        return traced(ctx, name, T_F32, M, N, K, [&]() -> int {
            if (!launch_gemm_f16_epi(a, lda, rs, wb, K, y, ldy, int(M), int(N), int(K), ctx->cus, ep, ctx->stream, op))
                return fail(SAMHIP_ERR_UNSUPPORTED, "vit_neck: no GEMM variant");
            HIP_TRY(hipGetLastError(), "neck gemm launch");
            return SAMHIP_OK;
        });
    };
    auto repeat = [&](int64_t kp) {
        AOperand op;
        if (!f16) {
            op.mode = A_REPEAT;
            op.part = int(kp);
        }
        return op;
    };
    // k x k convolution (stride 1, padding k/2) of a W x H map of C channels
    // into D channels; NECK_POOL convolves the 2x2 max pool of the map.  With
    // split columns a 1x1 convolution of the ViT output reuses its operand.
    auto conv = [&](const char* name, int src, const float* in, int64_t W, int64_t H, int64_t C, const float* w,
                    const float* b, int k, float* out) -> int {
        Epilogue ep;
        ep.bias = b;
        ep.col_scale = cs;
        if (src == NECK_IM2COL3 && gather3) {
            const int64_t K = parts * 9 * C, rows = W * H;
            if (int rc = weights(false, !f16, w, k, C, D, 9 * C)) return rc;
            int rc = traced(ctx, "neck_columns", T_F32, rows, 0, C, [&]() -> int {
                launch_neck_pixels(!f16, in, rows, int(C), at, rst, part, ctx->stream);
                HIP_TRY(hipGetLastError(), "neck pixels launch");
                return SAMHIP_OK;
            });
            if (rc) return rc;
            AOperand op;
            op.mode = A_CONV3;
            op.part = int(C);
            op.width = int(W);
            op.height = int(H);
            return gemm(name, at, stored * C, K, rst, out, D, rows, D, ep, op);
        }
        const int64_t kp = kpad(src == NECK_IM2COL3 ? 9 * C : C), lda = stored * kp;
        const int64_t rows = src == NECK_POOL ? (W / 2) * (H / 2) : W * H, step = chunk_rows(rows, lda);
        if (int rc = weights(false, !f16, w, k, C, D, kp)) return rc;
        if (!f16 && in == x && src == NECK_ROWS) return gemm(name, ax, lda, parts * kp, rsx, out, D, rows, D, ep, repeat(kp));
        for (int64_t r0 = 0; r0 < rows; r0 += step) {
            const int64_t n = std::min(step, rows - r0);
            if (int rc = columns(src, !f16, in, W, H, C, kp, r0, n, at, rst)) return rc;
            if (int rc = gemm(name, at, lda, parts * kp, rst, out + r0 * D, D, n, D, ep, repeat(kp))) return rc;
        }
        return SAMHIP_OK;
    };
    // 2x2 stride-2 transposed convolution of split rows of a W x W map
    auto deconv = [&](const _Float16* a, const float* rs, int64_t W, int64_t cin, const float* w, const float* b,
                      int64_t cout, bool gelu, float* out) -> int {
        const int64_t kp = kpad(cin);
        if (int rc = weights(true, true, w, 2, cin, cout, kp)) return rc;
        Epilogue ep;
        ep.bias = b;
        ep.col_scale = cs;
        ep.shuffle_w = int(W);
        ep.shuffle_c = int(cout);
        ep.gelu = gelu;
        AOperand op;
        op.mode = A_REPEAT;
        op.part = int(kp);
        return gemm("neck_deconv", a, 2 * kp, 3 * kp, rs, out, cout, W * W, 4 * cout, ep, op);
    };

    int rc = SAMHIP_OK;
    if (need_ax && (rc = columns(NECK_ROWS, true, x, g, g, E, kpE, 0, T, ax, rsx))) return rc;
    if (level[0]) {
        const samhip_neck_scale& s = sc[0];
        if ((rc = deconv(ax, rsx, g, E, s.deconv1_w, s.deconv1_b, mid, true, t1)) ||
            (rc = columns(NECK_ROWS, true, t1, 2 * g, 2 * g, mid, kpM, 0, T2, at, rst)) ||
            (rc = deconv(at, rst, 2 * g, mid, s.deconv2_w, s.deconv2_b, D, false, t2)) ||
            (rc = conv("neck_conv1x1", NECK_ROWS, t2, 4 * g, 4 * g, D, s.conv1x1_w, s.conv1x1_b, 1, t3)) ||
            (rc = conv("neck_conv3x3", NECK_IM2COL3, t3, 4 * g, 4 * g, D, s.conv3x3_w, s.conv3x3_b, 3, level[0])))
            return rc;
    }
    if (level[1]) {
        const samhip_neck_scale& s = sc[1];
        if ((rc = deconv(ax, rsx, g, E, s.deconv1_w, s.deconv1_b, mid, false, t1)) ||
            (rc = conv("neck_conv1x1", NECK_ROWS, t1, 2 * g, 2 * g, mid, s.conv1x1_w, s.conv1x1_b, 1, t2)) ||
            (rc = conv("neck_conv3x3", NECK_IM2COL3, t2, 2 * g, 2 * g, D, s.conv3x3_w, s.conv3x3_b, 3, level[1])))
            return rc;
    }
    if (level[2]) {
        const samhip_neck_scale& s = sc[2];
        if ((rc = conv("neck_conv1x1", NECK_ROWS, x, g, g, E, s.conv1x1_w, s.conv1x1_b, 1, t1)) ||
            (rc = conv("neck_conv3x3", NECK_IM2COL3, t1, g, g, D, s.conv3x3_w, s.conv3x3_b, 3, level[2])))
            return rc;
    }
    if (level[3]) {
        const samhip_neck_scale& s = sc[3];
        if ((rc = conv("neck_conv1x1", NECK_POOL, x, g, g, E, s.conv1x1_w, s.conv1x1_b, 1, t1)) ||
            (rc = conv("neck_conv3x3", NECK_IM2COL3, t1, g / 2, g / 2, D, s.conv3x3_w, s.conv3x3_b, 3, level[3])))
            return rc;
    }
    return SAMHIP_OK;
}

int samhip_trace_begin(samhip_context* ctx, const char* kernel_filter) {
    if (!ctx) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "null context");
    SAMHIP_NOT_WHILE_CAPTURING(ctx, "trace_begin");
    ctx->trace_filter = kernel_filter ? kernel_filter : "";
    for (auto& r : ctx->trace) {
        ctx->event_pool.push_back(r.start);
        ctx->event_pool.push_back(r.stop);
    }
    ctx->trace.clear();
    ctx->tracing = true;
    ctx->trace_paused = false;
    return SAMHIP_OK;
}

int samhip_trace_pause(samhip_context* ctx, int paused) {
    if (!ctx) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "null context");
    if (!ctx->tracing) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "trace_pause: no trace is open");
    ctx->trace_paused = paused != 0;
    return SAMHIP_OK;
}

int samhip_trace_end(samhip_context* ctx, samhip_kernel_record* records, size_t capacity, size_t* count) {
    if (!ctx || (capacity && !records)) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "invalid trace_end argument");
    SAMHIP_NOT_WHILE_CAPTURING(ctx, "trace_end");
    ctx->tracing = false;
    ctx->trace_paused = false;
    if (int rc = set_device(ctx)) return rc;
    HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    for (size_t i = 0; i < ctx->trace.size() && i < capacity; ++i) {
        const auto& r = ctx->trace[i];
        samhip_kernel_record& o = records[i];
        std::snprintf(o.kernel, sizeof(o.kernel), "%s", r.kernel);
        o.weight_type = r.weight_type;
        o.m = r.m;
        o.n = r.n;
        o.k = r.k;
        HIP_TRY(hipEventElapsedTime(&o.ms, r.start, r.stop), "hipEventElapsedTime");
    }
    if (count) *count = ctx->trace.size();
    for (auto& r : ctx->trace) {
        ctx->event_pool.push_back(r.start);
        ctx->event_pool.push_back(r.stop);
    }
    ctx->trace.clear();
    return SAMHIP_OK;
}

int samhip_query(samhip_context* ctx, samhip_exec_info* info) {
    if (!ctx || !info) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "null query argument");
    *info = ctx->info;
    return SAMHIP_OK;
}

int samhip_capture_begin(samhip_context* ctx) {
    if (!ctx) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "null context");
    SAMHIP_NOT_WHILE_CAPTURING(ctx, "capture_begin");
    if (ctx->tracing) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "capture_begin: a trace is open");
    if (!ctx->stream) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "capture_begin: the null stream cannot be captured");
    if (int rc = set_device(ctx)) return rc;
    HIP_TRY(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    ctx->capturing = true;
    return SAMHIP_OK;
}

int samhip_capture_end(samhip_context* ctx, samhip_graph** graph) {
    if (!ctx || !graph) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "capture_end: null argument");
    *graph = nullptr;
    if (!ctx->capturing) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "capture_end: no capture is open");
    ctx->capturing = false;
    if (int rc = set_device(ctx)) return rc;
    hipGraph_t g = nullptr;
    HIP_TRY(hipStreamEndCapture(ctx->stream, &g), "hipStreamEndCapture");
    hipGraphExec_t exec = nullptr;
    const hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
    samhip_graph* out = new (std::nothrow) samhip_graph{ctx, exec};
    if (!out) {
        (void)hipGraphExecDestroy(exec);
        return fail(SAMHIP_ERR_OUT_OF_MEMORY, "graph allocation failed");
    }
    ctx->live_graphs++;
    *graph = out;
    return SAMHIP_OK;
}

int samhip_graph_launch(samhip_context* ctx, const samhip_graph* graph) {
    if (!ctx || !graph) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "graph_launch: null argument");
    SAMHIP_NOT_WHILE_CAPTURING(ctx, "graph_launch");
    if (graph->ctx != ctx) return fail(SAMHIP_ERR_INVALID_ARGUMENT, "graph_launch: graph belongs to another context");
    if (int rc = set_device(ctx)) return rc;
    HIP_TRY(hipGraphLaunch(graph->exec, ctx->stream), "hipGraphLaunch");
    return SAMHIP_OK;
}

void samhip_graph_destroy(samhip_graph* graph) {
    if (!graph) return;
    samhip_context* ctx = graph->ctx;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipGraphExecDestroy(graph->exec);
    if (--ctx->live_graphs == 0) {
        for (void* p : ctx->retired_staging) (void)hipFree(p);
        ctx->retired_staging.clear();
    }
    delete graph;
}

size_t samhip_last_error(char* buffer, size_t size) {
    if (buffer && size) {
        const size_t n = std::min(size - 1, g_last_error.size());
        std::memcpy(buffer, g_last_error.data(), n);
        buffer[n] = '\0';
    }
    return g_last_error.size();
}

}  // extern "C"
