/*
 * CPU oracle for the SAM 3 vision encoder forward — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the ggml graph SAM.cpp builds for the ViT
 * (src/models/sam3/vision.hpp:152-293, src/models/sam3/ops.hpp:56-89): the
 * prefix (14x14 patch convolution, tiled 24x24 position embedding, ln_pre)
 * and the pre-LN block (LN, window partition, qkv linear + bias, axial RoPE
 * on Q/K, softmax attention, proj linear + bias, window unpartition,
 * residual, LN, fc1 + bias, erf-GELU, fc2 + bias, residual).  Linears use the
 * native quantized mul_mat of ggml_oracle.c.  Used only by tests/, the smoke
 * check and bench.py's cpu_baseline leg; the product never links it.
 *
 * Layout: activations are token-major rows of E floats, token (x, y) of a
 * W x H grid at row y*W + x (ggml ne = {E, W, H}).
 *
 * Pinning (tests/test_vit_oracle.py):
 *   layer norm      : numpy float64 mean/variance formula, and the invariant
 *                     that unit-gain output rows have mean 0, variance 1.
 *   erf-GELU        : scipy.special.erf in float64.
 *   win part/unpart : unpart(part(x)) == x, zero padding, and the window
 *                     order of ggml_win_part (window py*npx+px, token
 *                     i2*ws+i1) on a coordinate-encoded grid.
 *   RoPE            : numpy complex multiplication of (x[2i] + j x[2i+1]) by
 *                     (cos + j sin); norms of each pair preserved.
 *   attention       : numpy float64 softmax(scale * Q K^T) V.
 *   patch prefix    : numpy float64 convolution by explicit sum (einsum over
 *                     the 14x14x3 patch), tiling and layer norm.
 *   block           : a numpy composition of the pinned pieces in the
 *                     reference graph order (same oracle mul_mat for the
 *                     linears) at reduced width, windowed and global.
 */
#ifndef SAMHIP_ORACLE_VIT_ORACLE_H
#define SAMHIP_ORACLE_VIT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml_norm(x, eps) * w + b over rows of n (sums in double, as ggml's CPU
 * norm); w / b may be NULL (gain 1, bias 0). */
void or_layer_norm(const float* x, float* y, int64_t rows, int64_t n, const float* w, const float* b, float eps,
                   int threads);

/* 0.5 x (1 + erf(x / sqrt 2)) in float. */
void or_gelu_erf(const float* x, float* y, int64_t n);

/* ggml_win_part / ggml_win_unpart on a W x H grid of C channels, window ws:
 * windows ceil(W/ws) x ceil(H/ws) in order py*npx + px, tokens i2*ws + i1
 * inside a window, zero padding past the grid. */
void or_win_part(const float* x, float* y, int W, int H, int C, int ws);
void or_win_unpart(const float* y, float* x, int W, int H, int C, int ws);

/* Complex RoPE of sam3_apply_rope on the first `heads` head slices of each
 * token row (row stride ld floats, head h at columns h*hd..): pair i of a
 * head, (x[2i], x[2i+1]), is multiplied by freqs[t][i] = (cos, sin). */
void or_rope(float* x, int64_t ld, int64_t tokens, int heads, int hd, const float* freqs);

/* softmax(scale * Q K^T) V per head over `n` tokens of one window:
 * q/k/v rows of stride ld floats, head h at columns h*hd; out rows of
 * heads*hd floats.  Dots in float, softmax and the V sum in double. */
void or_attention(const float* q, const float* k, const float* v, int64_t ld, int64_t n, int heads, int hd,
                  float scale, float* out, int threads);

typedef struct {
    const float *norm1_w, *norm1_b, *norm2_w, *norm2_b;
    int qkv_type, proj_type, fc1_type, fc2_type;   /* OR_Q8_0 / OR_Q4_K / OR_Q5_K / OR_Q6_K */
    const void *qkv_w, *proj_w, *fc1_w, *fc2_w;    /* packed rows [3E][E], [E][E], [MLP][E], [E][MLP] */
    const float *qkv_b, *proj_b, *fc1_b, *fc2_b;
    const float* freqs;                            /* [tokens of a window (or the grid)][hd/2][2] */
} or_vit_block_weights;

/* One ViT block x_out = block(x_in) on a W x H grid of E channels with
 * `heads` heads; ws > 0 windows the attention, ws == 0 is global.  Linears
 * on the native quantized path with the given Q8_0 activation rounding
 * (decode == 0, "ggml-quantized-cpu-native-v1"), or weights decoded to F32
 * against F32 activations (decode != 0, "ggml-quantized-weights-f32-v1",
 * src/runtime/ggml/runtime.hpp:105-106). */
int or_vit_block(const or_vit_block_weights* wts, const float* x_in, float* x_out, int W, int H, int E, int heads,
                 int mlp, int ws, int q8_rounding, int decode, int threads);

/* The ViT prefix: image (ggml {img, img, 3}: x + img*(y + img*c)) through the
 * patch x patch stride-patch convolution with kernel (ggml {p, p, 3, E}:
 * kx + p*(ky + p*(c + 3*e))), the position embedding (ggml {E, pg, pg})
 * tiled over the grid, and ggml_norm(1e-5) * ln_w + ln_b.  out: grid^2 rows
 * of E floats, grid = img / patch. */
int or_vit_prefix(const float* image, int img, int patch, const float* kernel, const float* pos, int pos_grid,
                  const float* ln_w, const float* ln_b, int E, float* out, int threads);

/* ---- SimpleFPN neck (src/models/sam3/vision.hpp:307-366) ----------------
 * Feature maps are pixel-major rows of C floats: pixel (x, y) of a W x H
 * map at row y*W + x (ggml ne = {C, W, H}).  Sums in double. */

/* ConvTranspose2d k=2 s=2 (sam3_deconv_2x2, src/models/sam3/ops.hpp:96-121):
 * out[(2y+ky)*2W + 2x+kx][co] = b[co] + sum_ci w[kx + 2*(ky + 2*(co + Cout*ci))] * in[y*W+x][ci]
 * (weight ggml {2, 2, Cout, Cin}); b may be NULL. */
void or_deconv2x2(const float* in, int W, int H, int Cin, const float* w, const float* b, int Cout, float* out,
                  int threads);
/* Conv2d stride 1, k x k, zero padding k/2 (sam3_conv_2d, ops.hpp:71-94):
 * out[y*W+x][co] = b[co] + sum w[kx + k*(ky + k*(ci + Cin*co))] * in[(y+ky-p)*W + x+kx-p][ci]
 * (weight ggml {k, k, Cin, Cout}). */
void or_conv2d(const float* in, int W, int H, int Cin, const float* w, const float* b, int Cout, int k, float* out,
               int threads);
/* The same with F16 im2col columns when columns_f16 != 0: each input value
 * and each kernel value enters the product rounded to fp16 (the F16
 * convolution_columns_type, ops.hpp:68-84, whose product narrows the kernel
 * to the columns' type). */
void or_conv2d_cols(const float* in, int W, int H, int Cin, const float* w, const float* b, int Cout, int k,
                    int columns_f16, float* out, int threads);
/* ggml_pool_2d MAX 2x2 stride 2 (W, H even). */
void or_maxpool2x2(const float* in, int W, int H, int C, float* out);

typedef struct {
    /* scale 0: deconv (E -> mid), GELU, deconv (mid -> D), 1x1, 3x3 */
    const float *s0_dc1_w, *s0_dc1_b, *s0_dc2_w, *s0_dc2_b, *s0_c1_w, *s0_c1_b, *s0_c3_w, *s0_c3_b;
    /* scale 1: deconv (E -> mid), 1x1 (mid -> D), 3x3 */
    const float *s1_dc_w, *s1_dc_b, *s1_c1_w, *s1_c1_b, *s1_c3_w, *s1_c3_b;
    /* scale 2: 1x1 (E -> D), 3x3 */
    const float *s2_c1_w, *s2_c1_b, *s2_c3_w, *s2_c3_b;
    /* scale 3: maxpool, 1x1 (E -> D), 3x3 */
    const float *s3_c1_w, *s3_c1_b, *s3_c3_w, *s3_c3_b;
} or_neck_weights;

/* sam3_build_neck_graph on the ViT output x (grid x grid rows of E): out[i]
 * are (4, 2, 1, 0.5) x grid maps of D channels; a NULL out[i] is skipped.
 * Returns nonzero for an odd grid with out[3] requested. */
int or_neck(const or_neck_weights* w, const float* x, int grid, int E, int mid, int D, int columns_f16, float* out[4],
            int threads);

#ifdef __cplusplus
}
#endif

#endif
