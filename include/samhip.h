/*
 * samhip — MI355X (gfx950) quantized mul_mat backend, C ABI.
 *
 * Drop-in replacement for the ggml operators that SAM.cpp's quantized linears
 * reach (GGML_OP_MUL_MAT on GGUF-packed Q8_0/Q4_K/Q5_K/Q6_K weights against
 * F32 activations, and GGML_OP_GET_ROWS), keeping ggml's tensor semantics:
 *   W = src0 [ne0 = K, ne1 = N] packed rows, nb[0] = block bytes, nb[1] = row stride
 *   X = src1 [ne0 = K, ne1 = M] F32, nb[0] = 4, nb[1] >= 4*K (strided rows allowed)
 *   Y = dst  [ne0 = N, ne1 = M] F32, Y[m][n] = sum_k W[n][k] * X[m][k]
 * (reference: ggml_mul_mat as called by sam3_channel_projection,
 * src/models/sam3/ops.hpp:40-45; layout stated at
 * tools/benchmark/ggml_linear_probe.cpp:103).
 *
 * No C++ exception crosses this boundary: every entry point returns an int
 * status (0 = ok, negative = error class) and records a message readable with
 * samhip_last_error().  The C++ host layer maps SAMHIP_ERR_INVALID_ARGUMENT to
 * std::invalid_argument and every other error to std::runtime_error, as
 * src/runtime/ggml/workspace.hpp:174-177 and README.md:239-242 do.
 *
 * Threading: a context is single-threaded and stream-ordered (one HIP stream);
 * distinct contexts may be used from distinct threads.  Apart from the stream
 * given to samhip_context_set_stream (used until it is replaced) and the
 * device buffers named by captured graphs (used by every replay), the
 * library keeps no caller pointer after a call returns.
 */
#ifndef SAMHIP_H
#define SAMHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SAMHIP_ABI_VERSION 1

/* ggml / GGUF type ids used on the path (ggml.h enum ggml_type). */
enum samhip_type {
    SAMHIP_TYPE_F32 = 0,
    SAMHIP_TYPE_F16 = 1,
    SAMHIP_TYPE_Q8_0 = 8,
    SAMHIP_TYPE_Q8_1 = 9,
    SAMHIP_TYPE_Q4_K = 12,
    SAMHIP_TYPE_Q5_K = 13,
    SAMHIP_TYPE_Q6_K = 14,
    SAMHIP_TYPE_Q8_K = 15,
    SAMHIP_TYPE_I32 = 26
};

enum samhip_status {
    SAMHIP_OK = 0,
    SAMHIP_ERR_INVALID_ARGUMENT = -1, /* bad shape/type/pointer: std::invalid_argument */
    SAMHIP_ERR_UNSUPPORTED = -2,      /* no kernel for this operand combination */
    SAMHIP_ERR_DEVICE = -3,           /* HIP runtime failure */
    SAMHIP_ERR_OUT_OF_MEMORY = -4
};

/* Arithmetic contract of mul_mat (mirrors sam::CpuComputeMode /
 * sam::CudaComputeMode, include/sam/types.hpp:13-14):
 *  Q8_NATIVE: activations are packed per call to the weight's ggml
 *             vec_dot_type (Q8_0 for Q8_0 weights, Q8_K for K-quants),
 *             bit-exact with ggml's CPU from_float, then multiplied on fp16
 *             MFMA with F32 accumulation.  Compare with the CPU
 *             "ggml-quantized-cpu-native-v1" path.
 *  F16:       activations are rounded to fp16 directly; compare with the
 *             CPU "ggml-quantized-weights-f32-v1" (F32-decode) path.
 * In both, the weight operand is fp16(ggml to_float(W)). */
enum samhip_compute {
    SAMHIP_COMPUTE_Q8_NATIVE = 0,
    SAMHIP_COMPUTE_F16 = 1
};

/* Q8_0 activation rounding (tools/quantize/cache_quantization.py:76-95):
 * X86: ggml CPU from_float on x86-64 (scale 127/amax, ties to even),
 * REF: ggml quantize_row_q8_0_ref (scale 1/d, ties away from zero). */
enum samhip_q8_rounding {
    SAMHIP_Q8_ROUND_X86 = 0,
    SAMHIP_Q8_ROUND_REF = 1
};

/* ggml tensor descriptor: ne = elements per dimension, nb = byte strides,
 * data = device address.  Only 2-D operands (ne[2] = ne[3] = 1) are used. */
typedef struct samhip_tensor {
    int32_t type;
    int64_t ne[4];
    size_t nb[4];
    void* data;
} samhip_tensor;

typedef struct samhip_options {
    uint32_t version;     /* SAMHIP_ABI_VERSION */
    int32_t device;       /* HIP device index (BackendOptions::hip_device) */
    int32_t compute;      /* enum samhip_compute */
    int32_t q8_rounding;  /* enum samhip_q8_rounding */
} samhip_options;

/* Versioned execution counters, after ggml_cuda_sam_q8_rhs_query_v1's struct
 * {version, path, launches, payload_bytes, allocation_bytes}
 * (cmake/patches/ggml-native-activation.patch:13-26). */
typedef struct samhip_exec_info {
    uint32_t version;
    int32_t device;
    uint64_t mul_mat_calls;
    uint64_t gemm_launches;
    uint64_t skinny_launches;
    uint64_t activation_launches;
    uint64_t get_rows_calls;
    uint64_t activation_payload_peak_bytes;
    uint64_t activation_allocation_peak_bytes;
    char kernel_variant[64];      /* last mul_mat kernel */
    char arithmetic_profile[48];  /* e.g. "samhip-q8-native-f16mfma-v1" */
    char device_name[64];
} samhip_exec_info;

typedef struct samhip_context samhip_context;

/* --- identity and devices ------------------------------------------------ */
int samhip_abi_version(void);
int samhip_device_count(int* count);

/* --- context (one device, one stream) ------------------------------------ */
/* replaces make_cuda_backend(device, compute, ...) as the backend driver
 * factory (src/runtime/ggml/backends/cuda.hpp:156-189). */
int samhip_context_create(const samhip_options* options, samhip_context** out);
void samhip_context_destroy(samhip_context* ctx);
/* Run subsequent calls on `hip_stream` (a hipStream_t); NULL restores the
 * context's own stream. */
int samhip_context_set_stream(samhip_context* ctx, void* hip_stream);
int samhip_synchronize(samhip_context* ctx);

/* --- device memory (ggml_backend_alloc_ctx_tensors / tensor_set / get) --- */
int samhip_buffer_alloc(samhip_context* ctx, size_t bytes, void** device_ptr);
int samhip_buffer_free(samhip_context* ctx, void* device_ptr);
/* Synchronous copies, as ggml_backend_tensor_set/get (src/models/sam3/
 * model.hpp:130, src/runtime/ggml/host_tensor.hpp:18-33).  Packed weight
 * bytes are uploaded unchanged. */
int samhip_tensor_set(samhip_context* ctx, void* device_dst, const void* host_src, size_t bytes);
int samhip_tensor_get(samhip_context* ctx, void* host_dst, const void* device_src, size_t bytes);

/* --- operators ------------------------------------------------------------ */
/* The native activation's fail-closed range check for mul_mat (the
 * reference runs it on every native-activation product,
 * cmake/patches/ggml-native-activation.patch:148-171): when enabled, a
 * Q8_NATIVE mul_mat first checks X and returns INVALID_ARGUMENT, computing
 * nothing, if a value is non-finite or a nonzero 32-value block maximum lies
 * outside [1e-30, 1e30].  Off by default; the check synchronizes the stream,
 * so checked products cannot be captured. */
int samhip_context_set_activation_check(samhip_context* ctx, int enabled);

/* 1 if mul_mat(w, x, y) has a kernel, else 0; asked before execution so an
 * unsupported node is a runtime error, not a crash (ggml_backend_supports_op
 * at src/runtime/ggml/graph.hpp:65-78). */
int samhip_supports_mul_mat(const samhip_tensor* w, const samhip_tensor* x, const samhip_tensor* y);

/* GGML_OP_MUL_MAT (ggml_mul_mat; ggml-cuda mul_mat dispatch
 * tests/runtime/ggml/test_quantization.cpp:604-614).  w may be a row-offset
 * view of a larger packed tensor, x may have a row stride above 4*K. */
int samhip_mul_mat(samhip_context* ctx, const samhip_tensor* w, const samhip_tensor* x, const samhip_tensor* y);

/* samhip_mul_mat without any allocation: no reference counterpart; for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same operands,
 * kernels and results as samhip_mul_mat, but every intermediate (activation
 * staging, decoded weights, split-K partial sums) lives in one fixed 64 MiB
 * device array per GPU that the library holds until the process ends
 * (enough for every SAM 3 batch-1 linear; the largest, the ViT fc2 at
 * M = 5184, K = 4736, needs 59 MB).  A product that needs more returns
 * INVALID_ARGUMENT.  Calls on the same GPU share that array and keep no
 * state in it between calls.  The library orders them on the GPU: each call
 * waits (hipStreamWaitEvent, on its context's stream) for the previous
 * call's kernels on that GPU, whichever context, stream or host thread made
 * it, so calls made one after another on the host run one after another on
 * the GPU.  Calls recorded into a graph (samhip_capture_begin) are not
 * ordered that way: replays of such a graph race with any other call on the
 * array unless the caller orders them (same stream, or an event). */
int samhip_mul_mat_noalloc(samhip_context* ctx, const samhip_tensor* w, const samhip_tensor* x,
                           const samhip_tensor* y);

/* GGML_OP_GET_ROWS: dst row i = to_float(src row ids[i]) (ggml_get_rows,
 * src/models/sam3/text_encoder.hpp:158).  src type F32/F16/Q8_0/Q4_K/Q5_K/
 * Q6_K, ids I32, dst F32.  Out-of-range ids fail with INVALID_ARGUMENT. */
int samhip_get_rows(samhip_context* ctx, const samhip_tensor* src, const samhip_tensor* ids, const samhip_tensor* dst);

/* Row quantization on the device, bit-exact with ggml:
 *   F16:  ggml_cast F32 -> F16 (round to nearest even; the F16 feature cache)
 *   Q8_0: ggml from_float / quantize_row_q8_0_ref per `q8_rounding` (also
 *         ggml_cast F32 -> Q8_0 of the Q8_0 feature cache,
 *         src/models/sam3/execution.hpp:76-83)
 *   Q8_K: quantize_row_q8_K_ref (CPU activation packing for K weights)
 *   Q8_1: ggml-cuda's MMVQ right operand (quantize_row_q8_1_cuda, exported by
 *         the SAM-patched ggml and driven by tools/quantize/
 *         cuda_q8_rhs_probe.cu:15-20, 74-80): 36-byte blocks of half
 *         d = amax/127, half sum of the original values (32-lane xor-butterfly
 *         order), codes roundf(x/d); q8_rounding is ignored
 *   Q4_K, Q5_K, Q6_K: quantize_row_q*_K_ref (ggml_quantize_chunk without
 *         importance weights; tools/quantize/quantize_rows.cpp:210)
 * src rows have `src_row_stride` bytes, dst rows are packed back to back. */
int samhip_quantize_rows(samhip_context* ctx, int32_t type, const float* src, size_t src_row_stride,
                         void* dst, int64_t rows, int64_t k, int32_t q8_rounding);

/* ggml-cuda's MMQ right operand for Q8_0 weights in the D4 layout
 * (quantize_mmq_q8_1_cuda as patched at cmake/patches/ggml-precise-cuda.patch:
 * 622-633; layout tools/quantize/native_activation.py:13-20, 42-62): rows
 * padded with zeros to a multiple of 512 values, then for 128-value tile t of
 * row r, dst + (t*rows + r)*144 holds 4 F32 scales 1/d_inv (d_inv = 127/amax
 * per 32 values, correctly rounded) and the 128 codes roundf(x*d_inv).
 * Fails closed like sam_q8_rhs_validate
 * (cmake/patches/ggml-native-activation.patch:148-171): a non-finite value or
 * a nonzero 32-value block maximum outside [1e-30, 1e30] returns
 * INVALID_ARGUMENT (dst contents then unspecified).  Synchronizes the
 * stream; not capturable.  dst must be 4-byte aligned and hold
 * samhip_q8_1_mmq_bytes(rows, k) bytes. */
size_t samhip_q8_1_mmq_bytes(int64_t rows, int64_t k);
int samhip_quantize_rows_q8_1_mmq(samhip_context* ctx, const float* src, size_t src_row_stride, void* dst,
                                  int64_t rows, int64_t k);

/* ggml to_float on the device for F16/Q8_0/Q4_K/Q5_K/Q6_K/Q8_K rows
 * (bit-exact; F16 rows need k % 32 == 0). */
int samhip_dequantize_rows(samhip_context* ctx, int32_t type, const void* src, size_t src_row_stride,
                           float* dst, int64_t rows, int64_t k);

/* Host-side payload check run before upload, as validate_quantized_payload
 * (src/models/sam3/weights.hpp:384-425): non-finite d (offset 0, or
 * type_size-2 for Q6_K), non-finite dmin (offset 2 for Q4_K/Q5_K) or a
 * non-finite decoded value is rejected. */
int samhip_validate_quantized_payload(int32_t type, int64_t ne0, int64_t rows, const void* host_bytes, size_t bytes);

/* --- SAM 3 vision encoder ----------------------------------------------------
 * The ViT of sam3_build_vit_graph (src/models/sam3/vision.hpp:248-293) as two
 * fused subgraph operators on device buffers, for a backend that takes the
 * whole vision encoder instead of its ggml nodes.  Activations are
 * token-major F32 rows of `embed` floats, token (x, y) of the grid at row
 * y*grid_w + x (ggml ne = {embed, grid_w, grid_h}).  Linears run as
 * samhip_mul_mat does (same activation packing and arithmetic), with bias,
 * erf-GELU, window unpartition and residual folded into the product's store;
 * layer norms, RoPE and softmax are F32, attention products fp16 (MFMA) with
 * F32 accumulation.  Supported: head_dim 64, embed a multiple of 256 (at
 * most 2048), embed and mlp multiples of 128 (mlp at most 5120), grid sides
 * multiples of the window. */
typedef struct samhip_vit_block_desc {
    int32_t version;                                  /* SAMHIP_ABI_VERSION */
    int32_t embed, heads, mlp;                        /* SAM 3: 1024, 16, 4736 */
    int32_t grid_w, grid_h, window;                   /* 72, 72, 24; window 0 = global attention */
    const float *norm1_w, *norm1_b, *norm2_w, *norm2_b;   /* device F32 [embed] */
    samhip_tensor qkv_w, proj_w, fc1_w, fc2_w;        /* packed weights [embed->3*embed], [embed->embed],
                                                         [embed->mlp], [mlp->embed] (ggml ne = {K, N}) */
    const float *qkv_b, *proj_b, *fc1_b, *fc2_b;      /* device F32 [N] */
    const float* freqs_cis;                           /* device F32 [tokens per window (or grid)][head_dim/2][2]
                                                         (cos, sin); NULL = no RoPE */
    int32_t attention_type;                           /* SAMHIP_TYPE_F32 (0, default): F32-accurate attention, as
                                                         the reference's GGML_PREC_F32 (src/runtime/ggml/
                                                         graph.hpp:64), split fp16 operands at three times the
                                                         MFMA work; SAMHIP_TYPE_F16: fp16 operands */
} samhip_vit_block_desc;

/* sam3_vit_block_forward (src/models/sam3/vision.hpp:152-243): x (device F32
 * [grid_h*grid_w][embed]) is replaced by the block's output. */
int samhip_vit_block(samhip_context* ctx, const samhip_vit_block_desc* block, float* x);

typedef struct samhip_vit_prefix_desc {
    int32_t version;                                  /* SAMHIP_ABI_VERSION */
    int32_t image_size, patch, embed, pos_grid;       /* SAM 3: 1008, 14, 1024, 24 */
    const float* patch_w;                             /* device F32, ggml {patch, patch, 3, embed} */
    const float* pos_embed;                           /* device F32, ggml {embed, pos_grid, pos_grid} */
    const float *ln_pre_w, *ln_pre_b;                 /* device F32 [embed] */
} samhip_vit_prefix_desc;

/* sam3_build_vit_prefix_graph (src/models/sam3/vision.hpp:248-272): image
 * (device F32, ggml {image_size, image_size, 3}) -> x (device F32
 * [(image_size/patch)^2][embed]): patch convolution (F32-accurate: split
 * fp16 operands), tiled position embedding, ln_pre. */
int samhip_vit_prefix(samhip_context* ctx, const samhip_vit_prefix_desc* prefix, const float* image, float* x);

/* One scale of the SimpleFPN neck (sam3_neck_scale,
 * src/models/sam3/architecture.hpp:87-96): device F32 weights in their ggml
 * layouts, transposed convolutions {2, 2, Cout, Cin}, convolutions
 * {k, k, Cin, Cout}, biases [Cout].  Scale 0 uses every field; scale 1 no
 * deconv2; scales 2 and 3 neither deconvolution. */
typedef struct samhip_neck_scale {
    const float *deconv1_w, *deconv1_b;
    const float *deconv2_w, *deconv2_b;
    const float *conv1x1_w, *conv1x1_b;
    const float *conv3x3_w, *conv3x3_b;
} samhip_neck_scale;

typedef struct samhip_vit_neck_desc {
    int32_t version;                    /* SAMHIP_ABI_VERSION */
    int32_t grid, embed, mid, dim;      /* SAM 3: 72, 1024, 512 (deconvolution width), 256 (neck_dim) */
    /* im2col columns of the 1x1 and 3x3 convolutions (the runtime's
     * convolution_columns_type, src/models/sam3/ops.hpp:68-84):
     * SAMHIP_TYPE_F32 keeps F32 accuracy (split fp16 operands),
     * SAMHIP_TYPE_F16 rounds both operands to fp16.  The transposed
     * convolutions are F32-accurate either way (ops.hpp:107-108). */
    int32_t columns_type;
    samhip_neck_scale scales[4];
} samhip_vit_neck_desc;

/* sam3_build_neck_graph (src/models/sam3/vision.hpp:307-366) on the ViT
 * output x (device F32 [grid*grid][embed], 16-byte aligned): level i, when
 * its pointer is non-NULL, receives the (4, 2, 1, 1/2) x grid map as device
 * F32 [side*side][dim] (pixel rows, 16-byte aligned).  A NULL level is not
 * computed (the image path outputs levels 0-2, execution.hpp:73-83).
 * embed, mid and dim must be multiples of 4; level 3 needs an even grid. */
int samhip_vit_neck(samhip_context* ctx, const samhip_vit_neck_desc* neck, const float* x, float* level0,
                    float* level1, float* level2, float* level3);

/* Pieces of the same graph as single operators.
 * GGML_OP_NORM followed by the gain/bias of sam3_layer_norm
 * (src/models/sam3/ops.hpp:56-66): y = ggml_norm(x, eps) * w + b over rows of
 * n floats (n a multiple of 256, at most 2048; w, b may be NULL). */
int samhip_layer_norm(samhip_context* ctx, const float* x, float* y, int64_t rows, int64_t n, const float* w,
                      const float* b, float eps);
/* GGML_OP_FLASH_ATTN_EXT without mask (src/models/sam3/vision.hpp:214-218),
 * F32-accurate (GGML_PREC_F32):
 * per batch and head, out = softmax(scale * Q K^T) V over n tokens.  q, k, v
 * (device F32) rows b*n + t with stride ld floats, head h at columns
 * h*head_dim; out rows of heads*head_dim floats.  head_dim must be 64. */
int samhip_flash_attn(samhip_context* ctx, const float* q, const float* k, const float* v, int64_t ld, float* out,
                      int64_t batches, int64_t n, int32_t heads, int32_t head_dim, float scale);

/* --- diagnostics ------------------------------------------------------------ */
int samhip_query(samhip_context* ctx, samhip_exec_info* info);

/* Per-launch kernel timing, the device-side counterpart of the reference's
 * opt-in GraphObserver computing/computed callbacks
 * (src/runtime/ggml/observer.hpp:14-22; tools/benchmark/execution_cost.hpp:
 * 47-80): between trace_begin and trace_end every kernel launch of the context
 * is bracketed by HIP events on the context's stream.  trace_end waits for the
 * stream and copies up to `capacity` records; *count receives the number
 * recorded (which may exceed capacity).  A non-NULL `kernel_filter` limits
 * the bracketing to kernels whose name contains that text, so that a timed
 * run carries events around one kernel only. */
typedef struct samhip_kernel_record {
    char kernel[64];
    int32_t weight_type;
    int64_t m, n, k;
    float ms;
} samhip_kernel_record;
int samhip_trace_begin(samhip_context* ctx, const char* kernel_filter);
int samhip_trace_end(samhip_context* ctx, samhip_kernel_record* records, size_t capacity, size_t* count);
/* Pauses (paused != 0) or resumes the bracketing of an open trace without
 * synchronizing; records already taken are kept.  Each bracket adds two
 * event records to the stream (several microseconds of GPU time per launch),
 * so a timed run can bracket a sample of its steps.  No reference
 * counterpart (an observer is attached for a whole compute). */
int samhip_trace_pause(samhip_context* ctx, int paused);
/* --- stream capture (no reference counterpart) ----------------------------
 * For launch-bound streams of small products (the text encoder's 97 linears
 * at M = 32): the calls between capture_begin and capture_end are recorded
 * into a HIP graph instead of running, and graph_launch replays them on the
 * context's stream with one host call.  Only samhip_mul_mat,
 * samhip_quantize_rows and samhip_dequantize_rows may be captured; every
 * other entry point fails with INVALID_ARGUMENT while a capture is open.  A
 * captured call must fit the context's current staging (run the same
 * product once before capturing); staging that has to grow later is
 * reallocated without freeing the buffer that live graphs use.  Replays
 * read and write the device buffers named at capture time.  Destroy graphs
 * before their context. */
typedef struct samhip_graph samhip_graph;
int samhip_capture_begin(samhip_context* ctx);
int samhip_capture_end(samhip_context* ctx, samhip_graph** graph);
int samhip_graph_launch(samhip_context* ctx, const samhip_graph* graph);
void samhip_graph_destroy(samhip_graph* graph);

/* Copies the calling thread's last error message; returns its full length. */
size_t samhip_last_error(char* buffer, size_t size);

#ifdef __cplusplus
}
#endif

#endif /* SAMHIP_H */
