/*
 * CPU oracle for the SAM 3 vision encoder forward — TEST INFRASTRUCTURE ONLY.
 * See vit_oracle.h for the graph it restates and what pins each function.
 */
#include "vit_oracle.h"
#include "ggml_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static void use_threads(int threads) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
}

/* ggml_norm (ggml-cpu ggml_compute_forward_norm_f32): mean and variance
 * accumulated in double, y = (x - mean) / sqrtf(var + eps) in float, then
 * the ggml_mul / ggml_add broadcasts of sam3_layer_norm
 * (src/models/sam3/ops.hpp:56-66). */
void or_layer_norm(const float* x, float* y, int64_t rows, int64_t n, const float* w, const float* b, float eps,
                   int threads) {
    use_threads(threads);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + r * n;
        float* yr = y + r * n;
        double sum = 0.0;
        for (int64_t i = 0; i < n; ++i) sum += (double)xr[i];
        const float mean = (float)(sum / (double)n);
        double sum2 = 0.0;
        for (int64_t i = 0; i < n; ++i) {
            const float v = xr[i] - mean;
            yr[i] = v;
            sum2 += (double)(v * v);
        }
        const float variance = (float)(sum2 / (double)n);
        const float scale = 1.0f / sqrtf(variance + eps);
        for (int64_t i = 0; i < n; ++i) {
            float v = yr[i] * scale;
            if (w) v = v * w[i];
            if (b) v = v + b[i];
            yr[i] = v;
        }
    }
}

/* ggml_gelu_erf on F32 (src/models/sam3/vision.hpp:238). */
void or_gelu_erf(const float* x, float* y, int64_t n) {
    const float inv_sqrt2 = 0.70710678118654752440f;
    for (int64_t i = 0; i < n; ++i) y[i] = 0.5f * x[i] * (1.0f + erff(x[i] * inv_sqrt2));
}

/* ggml_win_part / ggml_win_unpart (src/models/sam3/vision.hpp:172, 226). */
void or_win_part(const float* x, float* y, int W, int H, int C, int ws) {
    const int npx = (W + ws - 1) / ws, npy = (H + ws - 1) / ws;
    for (int py = 0; py < npy; ++py)
        for (int px = 0; px < npx; ++px)
            for (int i2 = 0; i2 < ws; ++i2)
                for (int i1 = 0; i1 < ws; ++i1) {
                    const int gy = py * ws + i2, gx = px * ws + i1;
                    float* dst = y + ((int64_t)(py * npx + px) * ws * ws + (int64_t)i2 * ws + i1) * C;
                    if (gy < H && gx < W) memcpy(dst, x + ((int64_t)gy * W + gx) * C, sizeof(float) * (size_t)C);
                    else memset(dst, 0, sizeof(float) * (size_t)C);
                }
}

void or_win_unpart(const float* y, float* x, int W, int H, int C, int ws) {
    const int npx = (W + ws - 1) / ws;
    for (int gy = 0; gy < H; ++gy)
        for (int gx = 0; gx < W; ++gx) {
            const int py = gy / ws, px = gx / ws, i2 = gy % ws, i1 = gx % ws;
            memcpy(x + ((int64_t)gy * W + gx) * C,
                   y + ((int64_t)(py * npx + px) * ws * ws + (int64_t)i2 * ws + i1) * C, sizeof(float) * (size_t)C);
        }
}

/* sam3_apply_rope (src/models/sam3/vision.hpp:109-152):
 *   out[2i] = x[2i] cos - x[2i+1] sin,  out[2i+1] = x[2i] sin + x[2i+1] cos,
 * each product rounded to float before the add, as the ggml_mul / ggml_sub /
 * ggml_add graph does. */
void or_rope(float* x, int64_t ld, int64_t tokens, int heads, int hd, const float* freqs) {
    const int half = hd / 2;
    for (int64_t t = 0; t < tokens; ++t)
        for (int h = 0; h < heads; ++h) {
            float* p = x + t * ld + (int64_t)h * hd;
            const float* f = freqs + t * half * 2;
            for (int i = 0; i < half; ++i) {
                const float re = p[2 * i], im = p[2 * i + 1], c = f[2 * i], s = f[2 * i + 1];
                const float a = re * c, bb = im * s, cc = re * s, d = im * c;
                p[2 * i] = a - bb;
                p[2 * i + 1] = cc + d;
            }
        }
}

/* ggml_flash_attn_ext(Q, K, V, no mask, scale) per window and head
 * (src/models/sam3/vision.hpp:214-218), computed as exact softmax. */
void or_attention(const float* q, const float* k, const float* v, int64_t ld, int64_t n, int heads, int hd,
                  float scale, float* out, int threads) {
    use_threads(threads);
#pragma omp parallel
    {
        double* p = (double*)malloc(sizeof(double) * (size_t)n);
        double* acc = (double*)malloc(sizeof(double) * (size_t)hd);
#pragma omp for schedule(static)
        for (int64_t task = 0; task < (int64_t)heads * n; ++task) {
            const int h = (int)(task / n);
            const int64_t i = task % n;
            const float* qi = q + i * ld + (int64_t)h * hd;
            double mx = -INFINITY;
            for (int64_t j = 0; j < n; ++j) {
                const float* kj = k + j * ld + (int64_t)h * hd;
                float s = 0.f;
                for (int d = 0; d < hd; ++d) s += qi[d] * kj[d];
                p[j] = (double)s * (double)scale;
                if (p[j] > mx) mx = p[j];
            }
            double sum = 0.0;
            for (int d = 0; d < hd; ++d) acc[d] = 0.0;
            for (int64_t j = 0; j < n; ++j) {
                const double e = exp(p[j] - mx);
                sum += e;
                const float* vj = v + j * ld + (int64_t)h * hd;
                for (int d = 0; d < hd; ++d) acc[d] += e * (double)vj[d];
            }
            float* o = out + i * (int64_t)heads * hd + (int64_t)h * hd;
            for (int d = 0; d < hd; ++d) o[d] = (float)(acc[d] / sum);
        }
        free(p);
        free(acc);
    }
}

static void add_bias(float* y, const float* b, int64_t rows, int64_t n) {
    if (!b) return;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < n; ++c) y[r * n + c] += b[c];
}

/* one linear y[m][n] = x[m][k] . W[n][k] on the selected CPU path */
static int linear(int type, const void* w, const float* x, float* y, int64_t n, int64_t m, int64_t k, int q8_rounding,
                  int decode, int threads) {
    const size_t ws = (size_t)or_row_bytes(type, k);
    return decode ? or_mul_mat_decode(type, w, ws, x, (size_t)k, y, n, m, k, threads)
                  : or_mul_mat_native(type, w, ws, x, (size_t)k, y, n, m, k, q8_rounding, threads);
}

/* sam3_vit_block_forward (src/models/sam3/vision.hpp:152-243). */
int or_vit_block(const or_vit_block_weights* wt, const float* x_in, float* x_out, int W, int H, int E, int heads,
                 int mlp, int ws, int q8_rounding, int decode, int threads) {
    const int hd = E / heads;
    const int64_t tokens = (int64_t)W * H;
    int64_t wtokens = tokens, nwin = 1, per = tokens;   /* windowed layout sizes */
    if (ws > 0) {
        const int npx = (W + ws - 1) / ws, npy = (H + ws - 1) / ws;
        nwin = (int64_t)npx * npy;
        per = (int64_t)ws * ws;
        wtokens = nwin * per;
    }
    const int64_t big = wtokens > tokens ? wtokens : tokens;
    float* ln = (float*)malloc(sizeof(float) * (size_t)(tokens * E));
    float* part = (float*)malloc(sizeof(float) * (size_t)(big * E));
    float* qkv = (float*)malloc(sizeof(float) * (size_t)(wtokens * 3 * E));
    float* att = (float*)malloc(sizeof(float) * (size_t)(wtokens * E));
    float* proj = (float*)malloc(sizeof(float) * (size_t)(wtokens * E));
    float* h1 = (float*)malloc(sizeof(float) * (size_t)(tokens * mlp));
    int rc = -1;
    if (!ln || !part || !qkv || !att || !proj || !h1) goto done;

    /* attention half */
    or_layer_norm(x_in, ln, tokens, E, wt->norm1_w, wt->norm1_b, 1e-5f, threads);
    const float* xa = ln;
    if (ws > 0) {
        or_win_part(ln, part, W, H, E, ws);
        xa = part;
    }
    if (linear(wt->qkv_type, wt->qkv_w, xa, qkv, 3 * E, wtokens, E, q8_rounding, decode, threads))
        goto done;
    add_bias(qkv, wt->qkv_b, wtokens, 3 * E);
    for (int64_t b = 0; b < nwin; ++b) {
        float* base = qkv + b * per * 3 * E;
        if (wt->freqs) {
            or_rope(base, 3 * E, per, heads, hd, wt->freqs);
            or_rope(base + E, 3 * E, per, heads, hd, wt->freqs);
        }
        or_attention(base, base + E, base + 2 * E, 3 * E, per, heads, hd, 1.0f / sqrtf((float)hd),
                     att + b * per * E, threads);
    }
    if (linear(wt->proj_type, wt->proj_w, att, proj, E, wtokens, E, q8_rounding, decode, threads))
        goto done;
    add_bias(proj, wt->proj_b, wtokens, E);
    const float* pa = proj;
    if (ws > 0) {
        or_win_unpart(proj, part, W, H, E, ws);
        pa = part;
    }
    for (int64_t i = 0; i < tokens * E; ++i) x_out[i] = x_in[i] + pa[i];

    /* MLP half */
    or_layer_norm(x_out, ln, tokens, E, wt->norm2_w, wt->norm2_b, 1e-5f, threads);
    if (linear(wt->fc1_type, wt->fc1_w, ln, h1, mlp, tokens, E, q8_rounding, decode, threads))
        goto done;
    add_bias(h1, wt->fc1_b, tokens, mlp);
    or_gelu_erf(h1, h1, tokens * mlp);
    if (linear(wt->fc2_type, wt->fc2_w, h1, proj, E, tokens, mlp, q8_rounding, decode, threads))
        goto done;
    add_bias(proj, wt->fc2_b, tokens, E);
    for (int64_t i = 0; i < tokens * E; ++i) x_out[i] += proj[i];
    rc = 0;
done:
    free(ln);
    free(part);
    free(qkv);
    free(att);
    free(proj);
    free(h1);
    return rc;
}

/* sam3_build_vit_prefix_graph (src/models/sam3/vision.hpp:248-272): the
 * im2col + F32 mul_mat convolution (src/models/sam3/ops.hpp:71-89) summed
 * in double, the ggml_repeat tiling of pos_embed, and ln_pre. */
int or_vit_prefix(const float* image, int img, int patch, const float* kernel, const float* pos, int pos_grid,
                  const float* ln_w, const float* ln_b, int E, float* out, int threads) {
    const int grid = img / patch;
    const int64_t tokens = (int64_t)grid * grid;
    const int kk = 3 * patch * patch;
    float* col = (float*)malloc(sizeof(float) * (size_t)(tokens * kk));
    if (!col) return -1;
    use_threads(threads);
    /* im2col: column index c*p*p + ky*p + kx, matching the kernel's ggml layout */
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < tokens; ++t) {
        const int ox = (int)(t % grid), oy = (int)(t / grid);
        for (int c = 0; c < 3; ++c)
            for (int ky = 0; ky < patch; ++ky)
                for (int kx = 0; kx < patch; ++kx)
                    col[t * kk + (c * patch + ky) * patch + kx] =
                        image[(int64_t)(oy * patch + ky) * img + ox * patch + kx + (int64_t)c * img * img];
    }
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < tokens; ++t) {
        const int ox = (int)(t % grid), oy = (int)(t / grid);
        const float* pr = pos + ((int64_t)(oy % pos_grid) * pos_grid + ox % pos_grid) * E;
        for (int e = 0; e < E; ++e) {
            double s = 0.0;
            const float* kr = kernel + (int64_t)e * kk;
            for (int i = 0; i < kk; ++i) s += (double)kr[i] * (double)col[t * kk + i];
            out[t * E + e] = (float)s + pr[e];
        }
    }
    free(col);
    or_layer_norm(out, out, tokens, E, ln_w, ln_b, 1e-5f, threads);
    return 0;
}

/* ---- SimpleFPN neck ------------------------------------------------------ */

void or_deconv2x2(const float* in, int W, int H, int Cin, const float* w, const float* b, int Cout, float* out,
                  int threads) {
    use_threads(threads);
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < (int64_t)W * H; ++p) {
        const int x = (int)(p % W), y = (int)(p / W);
        const float* ir = in + p * Cin;
        for (int ky = 0; ky < 2; ++ky)
            for (int kx = 0; kx < 2; ++kx) {
                float* orow = out + ((int64_t)(2 * y + ky) * 2 * W + 2 * x + kx) * Cout;
                for (int co = 0; co < Cout; ++co) {
                    double s = 0.0;
                    for (int ci = 0; ci < Cin; ++ci)
                        s += (double)w[kx + 2 * (ky + 2 * (co + (int64_t)Cout * ci))] * (double)ir[ci];
                    orow[co] = (float)s + (b ? b[co] : 0.f);
                }
            }
    }
}

static inline double conv_operand(float v, int columns_f16) {
    return columns_f16 ? (double)or_fp16_to_fp32(or_fp32_to_fp16(v)) : (double)v;
}

void or_conv2d(const float* in, int W, int H, int Cin, const float* w, const float* b, int Cout, int k, float* out,
               int threads) {
    or_conv2d_cols(in, W, H, Cin, w, b, Cout, k, 0, out, threads);
}

void or_conv2d_cols(const float* in, int W, int H, int Cin, const float* w, const float* b, int Cout, int k,
                    int columns_f16, float* out, int threads) {
    const int pad = k / 2;
    use_threads(threads);
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < (int64_t)W * H; ++p) {
        const int x = (int)(p % W), y = (int)(p / W);
        for (int co = 0; co < Cout; ++co) {
            double s = 0.0;
            for (int ky = 0; ky < k; ++ky) {
                const int iy = y + ky - pad;
                if (iy < 0 || iy >= H) continue;
                for (int kx = 0; kx < k; ++kx) {
                    const int ix = x + kx - pad;
                    if (ix < 0 || ix >= W) continue;
                    const float* ir = in + ((int64_t)iy * W + ix) * Cin;
                    for (int ci = 0; ci < Cin; ++ci)
                        s += conv_operand(w[kx + k * (ky + k * (ci + (int64_t)Cin * co))], columns_f16) *
                             conv_operand(ir[ci], columns_f16);
                }
            }
            out[p * Cout + co] = (float)s + (b ? b[co] : 0.f);
        }
    }
}

void or_maxpool2x2(const float* in, int W, int H, int C, float* out) {
    const int W2 = W / 2, H2 = H / 2;
    for (int y = 0; y < H2; ++y)
        for (int x = 0; x < W2; ++x)
            for (int c = 0; c < C; ++c) {
                float m = in[((int64_t)(2 * y) * W + 2 * x) * C + c];
                for (int d = 1; d < 4; ++d) {
                    const float v = in[((int64_t)(2 * y + d / 2) * W + 2 * x + d % 2) * C + c];
                    if (v > m) m = v;
                }
                out[((int64_t)y * W2 + x) * C + c] = m;
            }
}

/* sam3_build_neck_graph (src/models/sam3/vision.hpp:307-366). */
int or_neck(const or_neck_weights* w, const float* x, int grid, int E, int mid, int D, int columns_f16, float* out[4],
            int threads) {
    const int cf = columns_f16;
    const int64_t g = grid, g2 = 2 * g, g4 = 4 * g, gh = g / 2;
    const int64_t a_n = g2 * g2 * (mid > D ? mid : D), a_pool = gh * gh * E;
    float* a = (float*)malloc(sizeof(float) * (size_t)(a_n > a_pool ? a_n : a_pool));
    float* bb = (float*)malloc(sizeof(float) * (size_t)(g4 * g4 * D));
    float* c = (float*)malloc(sizeof(float) * (size_t)(g4 * g4 * D));
    int rc = -1;
    if (!a || !bb || !c) goto done;
    if (out[3] && grid % 2) goto done;
    /* scale 0 */
    if (out[0]) {
        or_deconv2x2(x, grid, grid, E, w->s0_dc1_w, w->s0_dc1_b, mid, a, threads);
        or_gelu_erf(a, a, g2 * g2 * mid);
        or_deconv2x2(a, (int)g2, (int)g2, mid, w->s0_dc2_w, w->s0_dc2_b, D, bb, threads);
        or_conv2d_cols(bb, (int)g4, (int)g4, D, w->s0_c1_w, w->s0_c1_b, D, 1, cf, c, threads);
        or_conv2d_cols(c, (int)g4, (int)g4, D, w->s0_c3_w, w->s0_c3_b, D, 3, cf, out[0], threads);
    }
    /* scale 1 */
    if (out[1]) {
        or_deconv2x2(x, grid, grid, E, w->s1_dc_w, w->s1_dc_b, mid, a, threads);
        or_conv2d_cols(a, (int)g2, (int)g2, mid, w->s1_c1_w, w->s1_c1_b, D, 1, cf, c, threads);
        or_conv2d_cols(c, (int)g2, (int)g2, D, w->s1_c3_w, w->s1_c3_b, D, 3, cf, out[1], threads);
    }
    /* scale 2 */
    if (out[2]) {
        or_conv2d_cols(x, grid, grid, E, w->s2_c1_w, w->s2_c1_b, D, 1, cf, c, threads);
        or_conv2d_cols(c, grid, grid, D, w->s2_c3_w, w->s2_c3_b, D, 3, cf, out[2], threads);
    }
    /* scale 3 */
    if (out[3]) {
        or_maxpool2x2(x, grid, grid, E, a);
        or_conv2d_cols(a, (int)gh, (int)gh, E, w->s3_c1_w, w->s3_c1_b, D, 1, cf, c, threads);
        or_conv2d_cols(c, (int)gh, (int)gh, D, w->s3_c3_w, w->s3_c3_b, D, 3, cf, out[3], threads);
    }
    rc = 0;
done:
    free(a);
    free(bb);
    free(c);
    return rc;
}
