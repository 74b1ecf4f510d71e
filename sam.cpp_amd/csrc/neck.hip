// SimpleFPN neck operands on gfx950 (sam3_build_neck_graph,
// src/models/sam3/vision.hpp:307-366).  Every convolution of the neck is a
// product on the fp16 MFMA GEMM:
//   * 2x2 stride-2 transposed convolutions (sam3_deconv_2x2, ops.hpp:96-121)
//     are one product per input pixel with 4*Cout columns (tap-major) whose
//     epilogue scatters each tap to its output pixel;
//   * 1x1 and 3x3 convolutions (sam3_conv_2d, ops.hpp:68-94) are products
//     of im2col rows (tap-major, channel-minor) with the rearranged kernel.
// F32 columns keep F32 accuracy with split operands: a value v scaled by a
// power of two 2^-e is hi + lo with hi = fp16(v 2^-e), lo = fp16(v 2^-e -
// hi); A rows [hi | hi | lo] against B rows [hi | lo | hi] sum hi*hi + hi*lo
// + lo*hi in F32, and the epilogue multiplies by the row's and the
// column's 2^e.  F16 columns are plain fp16 operands without scaling.
//
// Both operand builders give one wave to one output row: a first pass finds
// the row's largest magnitude (split only), a second reads the values again
// (from cache) and writes the halves.
#include "internal.hpp"
#include "q8stage.hpp"

namespace samhip {

namespace {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));

template <int SRC>
__device__ __forceinline__ floatx4 neck_fetch(const float* __restrict__ x, int W, int H, int C, int64_t p, int oy,
                                              int ox, int c) {
    if (SRC == NECK_ROWS) return load4f(x + p * C + c);
    if (SRC == NECK_POOL) {
        const float* q = x + (int64_t(2 * oy) * W + 2 * ox) * C + c;
        const int64_t down = int64_t(W) * C;
        const floatx4 v0 = load4f(q), v1 = load4f(q + C), v2 = load4f(q + down), v3 = load4f(q + down + C);
        floatx4 v;
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = fmaxf(fmaxf(v0[i], v1[i]), fmaxf(v2[i], v3[i]));
        return v;
    }
    const int tap = c / C, ci = c - tap * C, ky = tap / 3, kx = tap - 3 * ky;
    const int yy = oy + ky - 1, xx = ox + kx - 1;
    if (yy < 0 || yy >= H || xx < 0 || xx >= W) return floatx4{0.f, 0.f, 0.f, 0.f};
    return load4f(x + (int64_t(yy) * W + xx) * C + ci);
}

template <int SRC, bool SPLIT>
__global__ __launch_bounds__(256) void neck_columns_kernel(const float* __restrict__ x, int W, int H, int C, int kp,
                                                           int64_t row0, int rows, _Float16* __restrict__ a,
                                                           float* __restrict__ row_scale) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const int64_t p = row0 + r;
    const int K = SRC == NECK_IM2COL3 ? 9 * C : C;
    const int ow = SRC == NECK_POOL ? W / 2 : W;
    const int oy = int(p / ow), ox = int(p - int64_t(oy) * ow);
    int e = 0;
    if (SPLIT) {
        float amax = 0.f;
        for (int c = 4 * lane; c < K; c += 256) {
            const floatx4 v = neck_fetch<SRC>(x, W, H, C, p, oy, ox, c);
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
        }
        e = row_exponent(wave_max(amax));
    }
    const float down = exp2i(-e);
    _Float16* row = a + int64_t(r) * (SPLIT ? 3 : 1) * kp;
    for (int c = 4 * lane; c < kp; c += 256) {
        const floatx4 v = c < K ? neck_fetch<SRC>(x, W, H, C, p, oy, ox, c) : floatx4{0.f, 0.f, 0.f, 0.f};
        if (SPLIT) {
            half4_t hi, lo;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float s = v[i] * down;
                hi[i] = (_Float16)s;
                lo[i] = (_Float16)(s - (float)hi[i]);
            }
            *reinterpret_cast<half4_t*>(row + c) = hi;
            *reinterpret_cast<half4_t*>(row + kp + c) = hi;
            *reinterpret_cast<half4_t*>(row + 2 * kp + c) = lo;
        } else {
            *reinterpret_cast<half4_t*>(row + c) = half4_t{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
        }
    }
    if (lane == 0) row_scale[r] = exp2i(e);
}

template <bool DECONV>
__device__ __forceinline__ float neck_weight(const float* __restrict__ w, int k, int cin, int cout, int n, int c) {
    if (DECONV) {   // ggml {2, 2, Cout, Cin}: row n = tap*Cout + co, column ci
        const int tap = n / cout, co = n - tap * cout;
        return w[(tap & 1) + 2 * ((tap >> 1) + 2 * (co + int64_t(cout) * c))];
    }
    // ggml {k, k, Cin, Cout}: row co = n, column tap*Cin + ci
    const int tap = c / cin, ci = c - tap * cin, ky = tap / k, kx = tap - k * ky;
    return w[kx + k * (ky + k * (ci + int64_t(cin) * n))];
}

template <bool DECONV, bool SPLIT>
__global__ __launch_bounds__(256) void neck_weights_kernel(const float* __restrict__ w, int k, int cin, int cout,
                                                           int kp, _Float16* __restrict__ b,
                                                           float* __restrict__ col_scale) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int rows = DECONV ? 4 * cout : cout, K = DECONV ? cin : k * k * cin;
    if (n >= rows) return;
    int e = 0;
    if (SPLIT) {
        float amax = 0.f;
        for (int c = lane; c < K; c += 64) amax = fmaxf(amax, fabsf(neck_weight<DECONV>(w, k, cin, cout, n, c)));
        e = row_exponent(wave_max(amax));
    }
    const float down = exp2i(-e);
    _Float16* row = b + int64_t(n) * (SPLIT ? 3 : 1) * kp;
    for (int c = lane; c < kp; c += 64) {
        const float v = c < K ? neck_weight<DECONV>(w, k, cin, cout, n, c) : 0.f;
        if (SPLIT) {
            const float s = v * down;
            const _Float16 hi = (_Float16)s, lo = (_Float16)(s - (float)hi);
            row[c] = hi;
            row[kp + c] = lo;
            row[2 * kp + c] = hi;
        } else {
            row[c] = (_Float16)v;
        }
    }
    if (lane == 0) col_scale[n] = exp2i(e);
}

}  // namespace

void launch_neck_columns(int src, bool split, const float* x, int W, int H, int C, int kp, int64_t row0, int rows,
                         _Float16* a, float* row_scale, hipStream_t stream) {
    const dim3 grid(unsigned((rows + 3) / 4)), block(256);
#define SAMHIP_NECK_COLUMNS(S)                                                                                        \
    if (split) hipLaunchKernelGGL((neck_columns_kernel<S, true>), grid, block, 0, stream, x, W, H, C, kp, row0, rows, \
                                  a, row_scale);                                                                      \
    else hipLaunchKernelGGL((neck_columns_kernel<S, false>), grid, block, 0, stream, x, W, H, C, kp, row0, rows, a,   \
                            row_scale);
    switch (src) {
        case NECK_ROWS: SAMHIP_NECK_COLUMNS(NECK_ROWS) break;
        case NECK_POOL: SAMHIP_NECK_COLUMNS(NECK_POOL) break;
        case NECK_IM2COL3: SAMHIP_NECK_COLUMNS(NECK_IM2COL3) break;
        default: break;
    }
#undef SAMHIP_NECK_COLUMNS
}

void launch_neck_weights(bool deconv, bool split, const float* w, int k, int cin, int cout, int kp, _Float16* b,
                         float* col_scale, hipStream_t stream) {
    const int rows = deconv ? 4 * cout : cout;
    const dim3 grid(unsigned((rows + 3) / 4)), block(256);
    if (deconv && split)
        hipLaunchKernelGGL((neck_weights_kernel<true, true>), grid, block, 0, stream, w, k, cin, cout, kp, b, col_scale);
    else if (deconv)
        hipLaunchKernelGGL((neck_weights_kernel<true, false>), grid, block, 0, stream, w, k, cin, cout, kp, b, col_scale);
    else if (split)
        hipLaunchKernelGGL((neck_weights_kernel<false, true>), grid, block, 0, stream, w, k, cin, cout, kp, b, col_scale);
    else
        hipLaunchKernelGGL((neck_weights_kernel<false, false>), grid, block, 0, stream, w, k, cin, cout, kp, b, col_scale);
}

}  // namespace samhip
