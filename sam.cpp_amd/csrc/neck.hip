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
// hi); A rows stored [hi | lo] and read as [hi | hi | lo] against B rows
// [hi | lo | hi] sum hi*hi + hi*lo + lo*hi in F32, and the epilogue
// multiplies by the row's and the column's 2^e.  F16 columns are plain fp16
// operands without scaling.  A 3x3 convolution over 128k channels does not
// build im2col rows: the product gathers them from the map's own operand
// rows (scaled by one exponent for the whole map).
//
// The activation builder gives one wave to one output row: a first pass
// finds the row's largest magnitude (split only), a second reads the values
// again (from cache) and writes the halves.
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
    _Float16* row = a + int64_t(r) * (SPLIT ? 2 : 1) * kp;
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
            *reinterpret_cast<half4_t*>(row + kp + c) = lo;
        } else {
            *reinterpret_cast<half4_t*>(row + c) = half4_t{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
        }
    }
    if (lane == 0) row_scale[r] = exp2i(e);
}

// Operand rows of a whole map for the gathered 3x3 convolution: the map's
// largest magnitude (block maxima into `partial`, then combined by every
// block of the second kernel) gives one power-of-two scale, and each pixel
// row of C values becomes [hi | lo] (split) or [fp16] (unscaled).
__global__ __launch_bounds__(256) void neck_absmax_kernel(const float* __restrict__ x, int64_t n4,
                                                          float* __restrict__ partial) {
    __shared__ float part[4];
    float amax = 0.f;
    for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n4; i += int64_t(gridDim.x) * 256) {
        const floatx4 v = load4f(x + 4 * i);
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
    }
    amax = wave_max(amax);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = amax;
    __syncthreads();
    if (threadIdx.x == 0) partial[blockIdx.x] = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
}

template <bool SPLIT>
__global__ __launch_bounds__(256) void neck_pixels_kernel(const float* __restrict__ x, int64_t rows, int C,
                                                          const float* __restrict__ partial, int nparts,
                                                          _Float16* __restrict__ a, float* __restrict__ row_scale) {
#pragma clang fp contract(off)
    __shared__ float part[4];
    int e = 0;
    if (SPLIT) {
        float amax = 0.f;
        for (int i = threadIdx.x; i < nparts; i += 256) amax = fmaxf(amax, partial[i]);
        amax = wave_max(amax);
        if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = amax;
        __syncthreads();
        e = row_exponent(fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3])));
    }
    const float down = exp2i(-e), up = exp2i(e);
    const int c4 = C / 4;
    const int64_t n4 = rows * c4;
    for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n4; i += int64_t(gridDim.x) * 256) {
        const int64_t p = i / c4;
        const int c = int(i - p * c4) * 4;
        const floatx4 v = load4f(x + 4 * i);
        if (SPLIT) {
            half4_t hi, lo;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float s = v[q] * down;
                hi[q] = (_Float16)s;
                lo[q] = (_Float16)(s - (float)hi[q]);
            }
            *reinterpret_cast<half4_t*>(a + p * 2 * C + c) = hi;
            *reinterpret_cast<half4_t*>(a + p * 2 * C + C + c) = lo;
        } else {
            *reinterpret_cast<half4_t*>(a + p * C + c) =
                half4_t{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
        }
        if (c == 0) row_scale[p] = up;
    }
}

// Convolution kernel {k, k, Cin, Cout} -> B row co, column tap*Cin + ci
// (tap = k*ky + kx).  One workgroup per row: the row's k*k*Cin source
// values are contiguous (ci-major, taps inner), read coalesced for the
// magnitude pass and re-read from cache, k*k apart, for the permuted write.
template <bool SPLIT>
__global__ __launch_bounds__(256) void neck_conv_weights_kernel(const float* __restrict__ w, int kk, int cin, int kp,
                                                                _Float16* __restrict__ b,
                                                                float* __restrict__ col_scale) {
#pragma clang fp contract(off)
    __shared__ float part[4];
    const int co = blockIdx.x, t = threadIdx.x, K = kk * cin;
    const float* src = w + int64_t(co) * K;
    int e = 0;
    if (SPLIT) {
        float amax = 0.f;
        for (int c = t; c < K; c += 256) amax = fmaxf(amax, fabsf(src[c]));
        amax = wave_max(amax);
        if ((t & 63) == 0) part[t >> 6] = amax;
        __syncthreads();
        e = row_exponent(fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3])));
    }
    const float down = exp2i(-e);
    _Float16* row = b + int64_t(co) * (SPLIT ? 3 : 1) * kp;
    for (int c = t; c < kp; c += 256) {
        float v = 0.f;
        if (c < K) {
            const int tap = c / cin, ci = c - tap * cin;
            v = src[int64_t(ci) * kk + tap];
        }
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
    if (t == 0) col_scale[co] = exp2i(e);
}

// Transposed-convolution kernel {2, 2, Cout, Cin}: as a matrix S[ci][j]
// with j = 4*co + tap (tap = 2*ky + kx) it becomes B row n(j) = tap*Cout +
// co, column ci.  64 x 64 tiles of S: the first pass leaves each tile's
// column maxima in `partial` [Cin/64][4 Cout], the second combines a
// column's partials into its power-of-two scale and transposes the tile
// through LDS, so that both the reads of S and the writes of B are
// contiguous.
__device__ __forceinline__ int deconv_row(int j, int cout) { return (j & 3) * cout + (j >> 2); }

__global__ __launch_bounds__(256) void neck_deconv_max_kernel(const float* __restrict__ w, int cin, int cout,
                                                              float* __restrict__ partial) {
    __shared__ float part[4][64];
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const int J = 4 * cout, j = blockIdx.x * 64 + tx, ci0 = blockIdx.y * 64;
    float amax = 0.f;
    if (j < J)
#pragma unroll 4
        for (int r = ty; r < 64; r += 4)
            if (ci0 + r < cin) amax = fmaxf(amax, fabsf(w[int64_t(ci0 + r) * J + j]));
    part[ty][tx] = amax;
    __syncthreads();
    if (ty == 0 && j < J)
        partial[int64_t(blockIdx.y) * J + j] = fmaxf(fmaxf(part[0][tx], part[1][tx]), fmaxf(part[2][tx], part[3][tx]));
}

__global__ __launch_bounds__(256) void neck_deconv_pack_kernel(const float* __restrict__ w, int cin, int cout, int kp,
                                                               const float* __restrict__ partial,
                                                               _Float16* __restrict__ b, float* __restrict__ col_scale) {
#pragma clang fp contract(off)
    __shared__ float tile[64][65];
    __shared__ float down[64];
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const int J = 4 * cout, j0 = blockIdx.x * 64, ci0 = blockIdx.y * 64, tiles = (cin + 63) / 64;
#pragma unroll 4
    for (int r = ty; r < 64; r += 4) {
        const int ci = ci0 + r, j = j0 + tx;
        tile[r][tx] = (ci < cin && j < J) ? w[int64_t(ci) * J + j] : 0.f;
    }
    if (ty == 0) {
        const int j = j0 + tx;
        float amax = 0.f;
        if (j < J)
            for (int t = 0; t < tiles; ++t) amax = fmaxf(amax, partial[int64_t(t) * J + j]);
        const int e = row_exponent(amax);
        down[tx] = exp2i(-e);
        if (blockIdx.y == 0 && j < J) col_scale[deconv_row(j, cout)] = exp2i(e);
    }
    __syncthreads();
    const int ci = ci0 + tx;
#pragma unroll 4
    for (int jj = ty; jj < 64; jj += 4) {
        const int j = j0 + jj;
        if (j >= J) break;
        const float s = tile[tx][jj] * down[jj];
        const _Float16 hi = (_Float16)s, lo = (_Float16)(s - (float)hi);
        _Float16* row = b + int64_t(deconv_row(j, cout)) * 3 * kp;
        row[ci] = hi;
        row[kp + ci] = lo;
        row[2 * kp + ci] = hi;
    }
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

void launch_neck_pixels(bool split, const float* x, int64_t rows, int C, _Float16* a, float* row_scale,
                        float* partial, hipStream_t stream) {
    const int64_t n4 = rows * (C / 4);
    const int blocks = int(std::min<int64_t>(1024, (n4 + 255) / 256));
    if (split) {
        hipLaunchKernelGGL(neck_absmax_kernel, dim3(unsigned(blocks)), dim3(256), 0, stream, x, n4, partial);
        hipLaunchKernelGGL(neck_pixels_kernel<true>, dim3(unsigned(blocks)), dim3(256), 0, stream, x, rows, C, partial,
                           blocks, a, row_scale);
    } else {
        hipLaunchKernelGGL(neck_pixels_kernel<false>, dim3(unsigned(blocks)), dim3(256), 0, stream, x, rows, C,
                           partial, 0, a, row_scale);
    }
}

void launch_neck_weights(bool deconv, bool split, const float* w, int k, int cin, int cout, int kp, _Float16* b,
                         float* col_scale, float* partial, hipStream_t stream) {
    if (deconv) {   // always split (the transposed convolutions stay F32-accurate)
        const unsigned jt = unsigned((4 * cout + 63) / 64);
        hipLaunchKernelGGL(neck_deconv_max_kernel, dim3(jt, unsigned((cin + 63) / 64)), dim3(256), 0, stream, w, cin,
                           cout, partial);
        hipLaunchKernelGGL(neck_deconv_pack_kernel, dim3(jt, unsigned(kp / 64)), dim3(256), 0, stream, w, cin, cout,
                           kp, partial, b, col_scale);
        return;
    }
    if (split)
        hipLaunchKernelGGL(neck_conv_weights_kernel<true>, dim3(unsigned(cout)), dim3(256), 0, stream, w, k * k, cin,
                           kp, b, col_scale);
    else
        hipLaunchKernelGGL(neck_conv_weights_kernel<false>, dim3(unsigned(cout)), dim3(256), 0, stream, w, k * k, cin,
                           kp, b, col_scale);
}

}  // namespace samhip
