/*
 * CPU oracle for the quantized mul_mat path — TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of the arithmetic that SAM.cpp delegates to
 * ggml 0.26.0 (ggml-org/ggml @ d7cb574130e6f01ad25b3289685489200febcd74, not
 * vendored in the reference: cmake/ggml.cmake:10-14).  It is used only by
 * tests/, by __graft_entry__.smoke() as the checker, and by bench.py's
 * cpu_baseline leg.  The product (libsamhip.so) never links or calls it.
 *
 * Pinning status of each function (what checks it besides its own formula):
 *   fp16 <-> fp32        : numpy float16 conversion over all 65536 halves and
 *                          random/edge floats (tests/test_oracle.py).
 *   q8_0 quantize (ref)  : known-answer vector of
 *                          tests/tools/test_cache_quantization.py:26-43.
 *   q8_0 quantize (x86)  : known-answer vector of
 *                          tests/tools/test_cache_quantization.py:62-71.
 *   q8_K quantize        : layout invariants of
 *                          tools/benchmark/cpu_kernel_capture_probe.cpp:62-93
 *                          (f32 d at 0, codes at 4, bsums at 260 equal code
 *                          sums) plus closed-form bounds; the scale constant
 *                          and sign (iscale = -127/max) are ggml-internal:
 *                          "parity unpinned" for that constant.
 *   dequantize (4 types) : exact decode of blocks assembled field by field
 *                          by an independent numpy packer, brute force.
 *   q4_K/q5_K/q6_K weight quantizers : ggml's iterative scale search
 *                          (ggml-quants.c quantize_row_q*_K_ref) has no
 *                          golden vector in the reference: "parity unpinned";
 *                          checked only by round-trip error bounds.
 *   vec_dot / mul_mat    : double-precision brute force over decoded
 *                          operands (tests/runtime/ggml/test_quantization.cpp:
 *                          469-494; tools/benchmark/cpu_quantized_matmul.hpp:
 *                          195-222) and the exact-integer identity of block dots.
 */
#ifndef SAMHIP_ORACLE_GGML_ORACLE_H
#define SAMHIP_ORACLE_GGML_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (GGUF on-disk ids). */
enum { OR_F32 = 0, OR_F16 = 1, OR_Q8_0 = 8, OR_Q4_K = 12, OR_Q5_K = 13, OR_Q6_K = 14, OR_Q8_K = 15 };

/* Q8_0 activation rounding variants (tools/quantize/cache_quantization.py:76-95). */
enum { OR_Q8_ROUND_REF = 0, OR_Q8_ROUND_X86 = 1 };

int64_t or_block_elems(int type);
int64_t or_block_bytes(int type);
int64_t or_row_bytes(int type, int64_t k);

uint16_t or_fp32_to_fp16(float f);
float or_fp16_to_fp32(uint16_t h);
void or_fp32_to_fp16_rows(const float* x, uint16_t* y, int64_t n);
void or_fp16_to_fp32_rows(const uint16_t* x, float* y, int64_t n);

/* Portable N(mean, std^2) generator: splitmix64-seeded xoshiro256** and
 * Box-Muller in double, rounded to float. */
void or_rng_normal(uint64_t seed, float mean, float stddev, float* out, int64_t n);

/* Row quantizers: x[rows][k] -> packed rows. */
int or_quantize_q8_0(const float* x, void* y, int64_t rows, int64_t k, int rounding);
int or_quantize_q8_k(const float* x, void* y, int64_t rows, int64_t k);
int or_quantize_q4_k(const float* x, void* y, int64_t rows, int64_t k);
int or_quantize_q5_k(const float* x, void* y, int64_t rows, int64_t k);
int or_quantize_q6_k(const float* x, void* y, int64_t rows, int64_t k);
/* Weight quantizer dispatch as ggml_quantize_chunk without importance
 * weights (q8_0 uses the reference rounding). Returns bytes written or -1. */
int64_t or_quantize_chunk(int type, const float* x, void* y, int64_t rows, int64_t k);

/* First phase of the K-quant weight quantizers on one 256-value super-block,
 * exposed so tests can check it against the published candidate search:
 * Q4_K/Q5_K: scales[8], mins[8] (= -min >= 0) and codes[256] in [0, nmax]
 * of the weighted least-squares fit of each 32-element sub-block;
 * Q6_K: scales[16] and codes[256] (l + 32) of each 16-element sub-block's
 * symmetric fit (mins unused).  Returns -1 for other types. */
int or_kquant_fit(int type, const float* x, float* scales, float* mins, uint8_t* codes);

/* ggml-cuda right-operand formats: Q8_1 rows (36 B per 32 values: half d,
 * half original sum, 32 codes) and the MMQ D4 staging of Q8_0 products
 * ([ceil(k/512)*4 tiles][rows][144 B]; or_q8_1_mmq_bytes gives the size). */
int or_quantize_q8_1(const float* x, void* y, int64_t rows, int64_t k);
int64_t or_q8_1_mmq_bytes(int64_t rows, int64_t k);
int or_quantize_q8_1_mmq(const float* x, void* y, int64_t rows, int64_t k);
/* 1 when x is finite with every nonzero 32-value block maximum in
 * [1e-30, 1e30] (the native activation's fail-closed range rule). */
int or_q8_rhs_supported(const float* x, int64_t rows, int64_t k);

/* to_float for Q8_0/Q4_K/Q5_K/Q6_K/Q8_K rows. */
int or_dequantize(int type, const void* x, float* y, int64_t rows, int64_t k);

/* One row dot of a packed weight row with a packed activation row of the
 * matching vec_dot_type (Q8_0 for Q8_0, Q8_K for K types). */
float or_vec_dot(int wtype, const void* w_row, const void* x_row, int64_t k);

/* ggml mul_mat contract: W[n][k] packed with row stride w_stride bytes,
 * X[m][k] F32 with row stride x_stride floats, Y[m][n] F32 contiguous.
 * native: activations packed per call to the vec_dot_type, block integer
 *         dots, F32 accumulation ("ggml-quantized-cpu-native-v1").
 * decode: W dequantized to F32, F32 dot ("ggml-quantized-weights-f32-v1").
 * threads <= 0 uses OpenMP's default. */
int or_mul_mat_native(int wtype, const void* w, size_t w_stride, const float* x, size_t x_stride,
                      float* y, int64_t n, int64_t m, int64_t k, int q8_rounding, int threads);
int or_mul_mat_decode(int wtype, const void* w, size_t w_stride, const float* x, size_t x_stride,
                      float* y, int64_t n, int64_t m, int64_t k, int threads);

/* Double-precision brute force over F32 operands: y[m][n] = sum w[n][k] x[m][k]. */
void or_gemm_f64(const float* w, const float* x, double* y, int64_t n, int64_t m, int64_t k, int threads);

int or_max_threads(void);

#ifdef __cplusplus
}
#endif

#endif
