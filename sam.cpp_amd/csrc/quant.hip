// Activation staging (the per-call RHS packing of the mul_mat path), row
// quantizers in ggml wire format, and to_float / get_rows, for gfx950.
//
// Staging turns F32 activation rows into the fp16 MFMA A operand:
//   Q8_0 mode : value = fp16(to_float(q8_0 block) * 2^-e)  (Q8_0 weights)
//   Q8_K mode : value = fp16(to_float(q8_K block) * 2^-e)  (K-quant weights)
//   F16 mode  : value = fp16(x * 2^-e)
// where the Q8 blocks are bit-exact with ggml's CPU from_float for the
// weight's vec_dot_type (src/runtime/ggml/backends/cpu.hpp:13-23) and 2^e is
// a per-row power of two that keeps the row maximum inside fp16's range; the
// GEMM epilogue multiplies it back exactly.
#include "internal.hpp"
#include "q8stage.hpp"

#pragma clang fp contract(off)

namespace samhip {

namespace {

// Staging with each lane owning 8 consecutive values (a Q8_0 block spans 4
// lanes, a Q8_K block 32 lanes).  The row stays in registers (K <= 512*CH),
// so X is read once; every cross-lane reduction runs with all lanes active
// (lanes past K hold zeros).
template <int MODE, int CH, bool X86, int PRE = PRE_NONE>
__device__ __forceinline__ void stage8_row(const float* __restrict__ x, int64_t x_stride, int m, int K,
                                           _Float16* __restrict__ a, int64_t lda, float* __restrict__ row_scale,
                                           int lane, const RowPre& pre = RowPre{}) {
    const float* xr = x + int64_t(m) * x_stride;
    floatx8 v[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int k = 512 * c + 8 * lane;
        if (k < K) {
            const floatx4 lo = load4f_stream(xr + k), hi = load4f_stream(xr + k + 4);
            v[c] = floatx8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        } else {
            v[c] = floatx8{0, 0, 0, 0, 0, 0, 0, 0};
        }
    }
    int64_t dst = m;
    if (PRE == PRE_GELU) {
        // the F32 erf-GELU of the producing graph node, before packing
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int i = 0; i < 8; ++i) v[c][i] = gelu_erf(v[c][i]);   // gelu(0) = 0 keeps the padding
    } else if (PRE == PRE_LAYER_NORM) {
        // ggml_norm(x, eps) * w + b of the producing node, the row leaving in
        // window order when pre.ws > 0
        float s = 0.f;
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int i = 0; i < 8; ++i) s += v[c][i];
        const float mean = wave_sum(s) / float(K);
        float s2 = 0.f;
        if (K == 512 * CH) {   // every lane's values lie in the row
#pragma unroll
            for (int c = 0; c < CH; ++c)
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float d = v[c][i] - mean;
                    v[c][i] = d;
                    s2 += d * d;
                }
        } else {
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const bool live = 512 * c + 8 * lane < K;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float d = live ? v[c][i] - mean : 0.f;
                    v[c][i] = d;
                    s2 += d * d;
                }
            }
        }
        const float variance = wave_sum(s2) / float(K);
        const float scale = 1.0f / sqrtf(variance + pre.eps);
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int k = 512 * c + 8 * lane;
            if (k < K) {
                const floatx4 w0 = load4f(pre.w + k), w1 = load4f(pre.w + k + 4);
                const floatx4 b0 = load4f(pre.b + k), b1 = load4f(pre.b + k + 4);
                const floatx8 w{w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
                const floatx8 b{b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
#pragma unroll
                for (int i = 0; i < 8; ++i) v[c][i] = (v[c][i] * scale) * w[i] + b[i];
            }
        }
        if (pre.ws > 0) {
            const int gy = m / pre.gw, gx = m - gy * pre.gw;
            const int win = (gy / pre.ws) * (pre.gw / pre.ws) + gx / pre.ws;
            dst = int64_t(win) * pre.ws * pre.ws + (gy % pre.ws) * pre.ws + gx % pre.ws;
        }
    }
    float rmax = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int i = 0; i < 8; ++i) rmax = fmaxf(rmax, fabsf(v[c][i]));
    const float r32 = max32_lanes(rmax);
    rmax = fmaxf(r32, __shfl_xor(r32, 32, 64));
    const int e = row_exponent(rmax);
    const float down = exp2i(-e);
    if (lane == 0) row_scale[dst] = exp2i(e);
    _Float16* ar = a + dst * lda;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int k = 512 * c + 8 * lane;
        const half8 o = quant8<MODE, X86>(v[c], lane, down);
        if (k < K) *reinterpret_cast<half8*>(ar + k) = o;
    }
}

// Rows of up to 5120 values (fc2's 4736), optionally through erf-GELU: two
// waves per row (values [0, 2560) and [2560, K)), the row maximum combined
// through LDS, so each wave holds half the row in registers and the
// workgroup stages two rows.  Every wave of the workgroup must call it (one
// barrier).  Measured against the alternatives at K = 4736: 39 us without
// a PRE (one wave per row, 97 VGPRs: 41 us), 42 us with the erf-GELU (a
// chunked pass parking the Q8 codes in LDS until the row maximum is known:
// 43-44 us).
template <int MODE, bool X86, int PRE>
__device__ __forceinline__ void stage8_half_row(const float* __restrict__ x, int64_t x_stride, int m, int M, int K,
                                                _Float16* __restrict__ a, int64_t lda, float* __restrict__ row_scale,
                                                int lane, int wave, float* pair_max) {
    constexpr int CHH = 5;
    const int half = wave & 1;
    const bool live = m < M;
    const float* xr = x + int64_t(live ? m : 0) * x_stride;
    floatx8 v[CHH];
#pragma unroll
    for (int c = 0; c < CHH; ++c) {
        const int k = 2560 * half + 512 * c + 8 * lane;
        if (live && k < K) {
            const floatx4 lo = load4f_stream(xr + k), hi = load4f_stream(xr + k + 4);
            v[c] = floatx8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        } else {
            v[c] = floatx8{0, 0, 0, 0, 0, 0, 0, 0};
        }
    }
    if (PRE == PRE_GELU)
#pragma unroll
        for (int c = 0; c < CHH; ++c)
#pragma unroll
            for (int i = 0; i < 8; ++i) v[c][i] = gelu_erf(v[c][i]);   // gelu(0) = 0 keeps the padding
    float rmax = 0.f;
#pragma unroll
    for (int c = 0; c < CHH; ++c)
#pragma unroll
        for (int i = 0; i < 8; ++i) rmax = fmaxf(rmax, fabsf(v[c][i]));
    const float r32 = max32_lanes(rmax);
    rmax = fmaxf(r32, __shfl_xor(r32, 32, 64));
    if (lane == 0) pair_max[wave] = rmax;
    __syncthreads();
    rmax = fmaxf(pair_max[wave & ~1], pair_max[wave | 1]);
    const int e = row_exponent(rmax);
    const float down = exp2i(-e);
    if (live && half == 0 && lane == 0) row_scale[m] = exp2i(e);
    _Float16* ar = a + int64_t(live ? m : 0) * lda;
#pragma unroll
    for (int c = 0; c < CHH; ++c) {
        const int k = 2560 * half + 512 * c + 8 * lane;
        const half8 o = quant8<MODE, X86>(v[c], lane, down);
        if (live && k < K) *reinterpret_cast<half8*>(ar + k) = o;
    }
}

template <int MODE, int CH, bool X86>
__global__ __launch_bounds__(256) void stage8_kernel(const float* __restrict__ x, int64_t x_stride, int M, int K,
                                                     _Float16* __restrict__ a, int64_t lda,
                                                     float* __restrict__ row_scale) {
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (m >= M) return;
    stage8_row<MODE, CH, X86>(x, x_stride, m, K, a, lda, row_scale, threadIdx.x & 63);
}

// thread t: half (t & 1) of 32-value step of one weight row -> 16 fp16 values
template <int WT>
__device__ __forceinline__ void dequant_piece(const uint8_t* __restrict__ W, int64_t w_stride, int K, int64_t t,
                                              _Float16* __restrict__ out, int64_t ldo) {
    const int steps = K / 32;
    const int h = int(t & 1);
    const int64_t rs = t >> 1;
    const int row = int(rs / steps), step = int(rs % steps);
    WeightPiece<WT> piece;
    piece.load(W + int64_t(row) * w_stride, step, h);
    _Float16 v[16];
    piece.dequant(step, h, v);
    half8* o = reinterpret_cast<half8*>(out + int64_t(row) * ldo + 32 * step + 16 * h);
    o[0] = half8{v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]};
    o[1] = half8{v[8], v[9], v[10], v[11], v[12], v[13], v[14], v[15]};
}

// Both per-call preparations of a tall product in one launch: workgroups
// [0, stage_blocks) pack four activation rows each, the rest decode 256
// weight pieces each (the two roles touch disjoint memory).
template <int MODE, int CH, bool X86, int WT, int PRE = PRE_NONE>
__global__ __launch_bounds__(256) void prep_kernel(const float* __restrict__ x, int64_t x_stride, int M, int K,
                                                   _Float16* __restrict__ a, int64_t lda, float* __restrict__ row_scale,
                                                   int stage_blocks, const uint8_t* __restrict__ W, int64_t w_stride,
                                                   int N, _Float16* __restrict__ wout, int64_t ldo, RowPre pre) {
    // rows past 2048 values without a layer norm: two waves per row
    constexpr bool PAIR = CH > 4 && (PRE == PRE_NONE || PRE == PRE_GELU);
    if constexpr (PAIR) {
        if (int(blockIdx.x) < stage_blocks) {
            __shared__ float pair_max[4];
            const int wave = threadIdx.x >> 6;
            stage8_half_row<MODE, X86, PRE>(x, x_stride, blockIdx.x * 2 + (wave >> 1), M, K, a, lda, row_scale,
                                       threadIdx.x & 63, wave, pair_max);
            return;
        }
    }
    if (!PAIR && int(blockIdx.x) < stage_blocks) {
        const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
        if (m < M) {
            stage8_row<MODE, CH, X86, PRE>(x, x_stride, m, K, a, lda, row_scale, threadIdx.x & 63, pre);
        }
        return;
    }
    const int64_t t = int64_t(blockIdx.x - stage_blocks) * 256 + threadIdx.x;
    if (t < int64_t(N) * (K / 32) * 2) dequant_piece<WT>(W, w_stride, K, t, wout, ldo);
}

// One wave per row, 4 rows per 256-thread block.
template <int MODE>
__global__ __launch_bounds__(256) void stage_rows_kernel(const float* __restrict__ x, int64_t x_stride, int M, int K,
                                                         _Float16* __restrict__ a, int64_t lda,
                                                         float* __restrict__ row_scale, int x86) {
    const int lane = threadIdx.x & 63;
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (m >= M) return;
    const float* xr = x + int64_t(m) * x_stride;
    float rmax = 0.f;
    for (int k = 4 * lane; k < K; k += 256) {
        const floatx4 v = load4f(xr + k);
        rmax = fmaxf(rmax, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
    }
    rmax = wave_max(rmax);
    const int e = row_exponent(rmax);
    const float down = exp2i(-e);
    if (lane == 0) row_scale[m] = exp2i(e);
    _Float16* ar = a + int64_t(m) * lda;
    for (int k = 4 * lane; k < K; k += 256) {
        const floatx4 v = load4f(xr + k);
        _Float16 out[4];
        if (MODE == T_F16) {
            for (int i = 0; i < 4; ++i) out[i] = (_Float16)(v[i] * down);
        } else {
            float d;
            int q[4];
            if (MODE == T_Q8_0) {
                q8_0_codes(v, x86, d, q);
                d = half_bits_to_float(float_to_half_bits(d));   // stored fp16 scale
            } else {
                q8_k_codes(v, lane, d, q);
            }
            const float dd = d * down;
            for (int i = 0; i < 4; ++i) out[i] = (_Float16)((float)q[i] * dd);
        }
        typedef _Float16 half4 __attribute__((ext_vector_type(4)));
        *reinterpret_cast<half4*>(ar + k) = half4{out[0], out[1], out[2], out[3]};
    }
}

// Weight rows -> fp16(to_float(W)) [N][K]: thread (row, 32-element step,
// half) writes 16 consecutive halves, so a wave stores 1 KB contiguously.
template <int WT>
__global__ __launch_bounds__(256) void dequant_w_f16_kernel(const uint8_t* __restrict__ W, int64_t w_stride, int N,
                                                            int K, _Float16* __restrict__ out, int64_t ldo) {
    const int64_t t = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (t >= int64_t(N) * (K / 32) * 2) return;
    dequant_piece<WT>(W, w_stride, K, t, out, ldo);
}

// Scalar-load variant for rows that are not 16-byte aligned.
template <int MODE>
__global__ __launch_bounds__(256) void stage_rows_unaligned_kernel(const float* __restrict__ x, int64_t x_stride, int M,
                                                                   int K, _Float16* __restrict__ a, int64_t lda,
                                                                   float* __restrict__ row_scale, int x86) {
    const int lane = threadIdx.x & 63;
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (m >= M) return;
    const float* xr = x + int64_t(m) * x_stride;
    auto load = [&](int k) { return floatx4{xr[k], xr[k + 1], xr[k + 2], xr[k + 3]}; };
    float rmax = 0.f;
    for (int k = 4 * lane; k < K; k += 256) {
        const floatx4 v = load(k);
        rmax = fmaxf(rmax, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
    }
    rmax = wave_max(rmax);
    const int e = row_exponent(rmax);
    const float down = exp2i(-e);
    if (lane == 0) row_scale[m] = exp2i(e);
    _Float16* ar = a + int64_t(m) * lda;
    for (int k = 4 * lane; k < K; k += 256) {
        const floatx4 v = load(k);
        float d = 0.f;
        int q[4];
        if (MODE == T_Q8_0) {
            q8_0_codes(v, x86, d, q);
            d = half_bits_to_float(float_to_half_bits(d));
        } else if (MODE == T_Q8_K) {
            q8_k_codes(v, lane, d, q);
        }
        const float dd = d * down;
        for (int i = 0; i < 4; ++i)
            ar[k + i] = MODE == T_F16 ? (_Float16)(v[i] * down) : (_Float16)((float)q[i] * dd);
    }
}

// Q8_0 / Q8_K rows in ggml wire format.  One wave per row.
template <int TYPE>
__global__ __launch_bounds__(256) void quantize_act_kernel(const float* __restrict__ x, int64_t x_stride, int rows,
                                                           int K, uint8_t* __restrict__ dst, int x86) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const float* xr = x + int64_t(r) * x_stride;
    constexpr int BE = block_elems(TYPE), BB = block_bytes(TYPE);
    uint8_t* out = dst + int64_t(r) * (K / BE) * BB;
    for (int k = 4 * lane; k < K; k += 256) {
        const floatx4 v = floatx4{xr[k], xr[k + 1], xr[k + 2], xr[k + 3]};
        float d;
        int q[4];
        if (TYPE == T_Q8_0) q8_0_codes(v, x86, d, q);
        else q8_k_codes(v, lane, d, q);
        uint8_t* blk = out + (k / BE) * BB;
        const int within = k % BE;
        if (TYPE == T_Q8_0) {
            if (within == 0) {
                const uint16_t h = float_to_half_bits(d);
                blk[0] = uint8_t(h & 0xff);
                blk[1] = uint8_t(h >> 8);
            }
            for (int i = 0; i < 4; ++i) blk[2 + within + i] = uint8_t(int8_t(q[i]));
        } else {
            if (within == 0) *reinterpret_cast<float*>(blk) = d;
            for (int i = 0; i < 4; ++i) blk[4 + within + i] = uint8_t(int8_t(q[i]));
            const int s = group_sum<4>(q[0] + q[1] + q[2] + q[3]);
            if ((lane & 3) == 0) {
                const int16_t s16 = int16_t(s);
                blk[260 + 2 * (within / 16)] = uint8_t(uint16_t(s16) & 0xff);
                blk[260 + 2 * (within / 16) + 1] = uint8_t(uint16_t(s16) >> 8);
            }
        }
    }
}

// to_float of one 32-element group (a Q8_0 block, a Q4_K/Q5_K sub-block, two
// Q6_K sub-blocks, a quarter of a Q8_K block's codes).
template <int TYPE>
__device__ void dequant32(const uint8_t* row, int g, float* y) {
    if (TYPE == T_Q8_0) {
        const uint8_t* b = row + 34 * g;
        const float d = half_bits_to_float(load2_a2(b));
        for (int i = 0; i < 32; ++i) y[i] = d * (float)(int8_t)b[2 + i];
    } else if (TYPE == T_Q8_K) {
        const uint8_t* b = row + 292 * (g >> 3);
        const float d = __builtin_bit_cast(float, load4_a2(b));
        for (int i = 0; i < 32; ++i) y[i] = d * (float)(int8_t)b[4 + 32 * (g & 7) + i];
    } else if (TYPE == T_Q4_K || TYPE == T_Q5_K) {
        const int bb = TYPE == T_Q4_K ? 144 : 176;
        const uint8_t* b = row + bb * (g >> 3);
        const int j = g & 7;
        const uint32_t sc[3] = {load4_a2(b + 4), load4_a2(b + 8), load4_a2(b + 12)};
        int s, m;
        k4_scale_min(j, sc, s, m);
        const float dj = half_bits_to_float(load2_a2(b)) * (float)s;
        const float mj = half_bits_to_float(load2_a2(b + 2)) * (float)m;
        const uint8_t* qs = b + (TYPE == T_Q4_K ? 16 : 48) + 32 * (j >> 1);
        for (int l = 0; l < 32; ++l) {
            int v = (j & 1) ? (qs[l] >> 4) : (qs[l] & 0x0f);
            if (TYPE == T_Q5_K && ((b[16 + l] >> j) & 1)) v += 16;
            y[l] = dj * (float)v - mj;
        }
    } else if (TYPE == T_Q6_K) {
        const uint8_t* b = row + 210 * (g >> 3);
        const int j = g & 7, half = j >> 2, q4 = j & 3;
        const float d = half_bits_to_float(load2_a2(b + 208));
        for (int l = 0; l < 32; ++l) {
            const uint8_t lb = b[64 * half + 32 * (q4 & 1) + l];
            const int lo = (q4 < 2) ? (lb & 0x0f) : (lb >> 4);
            const int hi = (b[128 + 32 * half + l] >> (2 * q4)) & 3;
            const int sc = (int8_t)b[192 + 8 * half + 2 * q4 + l / 16];
            y[l] = d * (float)sc * (float)((lo | (hi << 4)) - 32);
        }
    }
}

template <int TYPE>
__global__ __launch_bounds__(256) void dequant_rows_kernel(const uint8_t* __restrict__ src, int64_t src_stride,
                                                           const int32_t* __restrict__ ids, int64_t src_rows,
                                                           float* __restrict__ dst, int64_t dst_stride, int rows,
                                                           int K, int* __restrict__ bad_id) {
    const int groups = K / 32;
    const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= int64_t(rows) * groups) return;
    const int r = int(t / groups), g = int(t % groups);
    int64_t sr = r;
    if (ids) {
        sr = ids[r];
        if (sr < 0 || sr >= src_rows) {
            if (g == 0) atomicOr(bad_id, 1);
            return;
        }
    }
    const uint8_t* row = src + sr * src_stride;
    float* y = dst + int64_t(r) * dst_stride + 32 * g;
    if (TYPE == T_F32) {
        const float* f = reinterpret_cast<const float*>(row) + 32 * g;
        for (int i = 0; i < 32; ++i) y[i] = f[i];
    } else if (TYPE == T_F16) {
        const _Float16* f = reinterpret_cast<const _Float16*>(row) + 32 * g;
        for (int i = 0; i < 32; ++i) y[i] = (float)f[i];
    } else {
        dequant32<TYPE>(row, g, y);
    }
}

// Staging of a product whose activation rows arrive as Q8_0 codes and F32
// block maxima (Epilogue::q8 of the producing GEMM): the fp16 operand and
// row scale that staging the F32 rows gives, bit for bit, since the row
// maximum is the largest block maximum, the block scale fp16(amax / 127) and
// each value fp16(q * (d * 2^-e)).  One wave per row, four rows per
// workgroup; lane l takes values 8l .. 8l + 7 of each 512-value chunk.  The
// workgroups past stage_blocks decode the weight as prep_kernel's do.
template <int WT>
__global__ __launch_bounds__(256) void prep_codes_kernel(const int8_t* __restrict__ codes,
                                                         const float* __restrict__ amax, int64_t ldc, int M, int K,
                                                         _Float16* __restrict__ a, int64_t lda,
                                                         float* __restrict__ row_scale, int stage_blocks,
                                                         const uint8_t* __restrict__ W, int64_t w_stride, int N,
                                                         _Float16* __restrict__ wout, int64_t ldo) {
#pragma clang fp contract(off)
    if (int(blockIdx.x) < stage_blocks) {
        const int lane = threadIdx.x & 63;
        const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
        if (m >= M) return;
        const float* am = amax + int64_t(m) * (ldc >> 5);
        float rmax = 0.f;
        for (int b = lane; b < K / 32; b += 64) rmax = fmaxf(rmax, am[b]);
        rmax = wave_max(rmax);
        const int e = row_exponent(rmax);
        const float down = exp2i(-e);
        if (lane == 0) row_scale[m] = exp2i(e);
        const int8_t* cr = codes + int64_t(m) * ldc;
        _Float16* ar = a + int64_t(m) * lda;
        for (int k = 8 * lane; k < K; k += 512) {
            const u32x2 w = *reinterpret_cast<const u32x2*>(cr + k);
            const float dd = half_bits_to_float(float_to_half_bits(am[k >> 5] / 127.f)) * down;
            half8 o;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int q = int(int8_t(uint8_t(w[i >> 2] >> (8 * (i & 3)))));
                o[i] = (_Float16)(float(q) * dd);
            }
            *reinterpret_cast<half8*>(ar + k) = o;
        }
        return;
    }
    const int64_t t = int64_t(blockIdx.x - stage_blocks) * 256 + threadIdx.x;
    if (t < int64_t(N) * (K / 32) * 2) dequant_piece<WT>(W, w_stride, K, t, wout, ldo);
}

}  // namespace

void launch_dequant_w_f16(int wtype, const void* w, int64_t w_stride, int N, int K, _Float16* out, int64_t ldo,
                          hipStream_t stream) {
    const int64_t threads = int64_t(N) * (K / 32) * 2;
    const dim3 grid(unsigned((threads + 255) / 256)), block(256);
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    switch (wtype) {
        case T_Q8_0: hipLaunchKernelGGL(dequant_w_f16_kernel<T_Q8_0>, grid, block, 0, stream, wb, w_stride, N, K, out, ldo); break;
        case T_Q4_K: hipLaunchKernelGGL(dequant_w_f16_kernel<T_Q4_K>, grid, block, 0, stream, wb, w_stride, N, K, out, ldo); break;
        case T_Q5_K: hipLaunchKernelGGL(dequant_w_f16_kernel<T_Q5_K>, grid, block, 0, stream, wb, w_stride, N, K, out, ldo); break;
        case T_Q6_K: hipLaunchKernelGGL(dequant_w_f16_kernel<T_Q6_K>, grid, block, 0, stream, wb, w_stride, N, K, out, ldo); break;
        default: break;
    }
}

bool launch_prep(int mode, int wtype, const float* x, int64_t x_stride, int M, int K, _Float16* a, int64_t lda,
                 float* row_scale, int x86, const void* w, int64_t w_stride, int N, _Float16* wout, int64_t ldo,
                 hipStream_t stream, const RowPre& pre) {
    if (K > 512 * 10 || reinterpret_cast<uintptr_t>(x) % 16 || x_stride % 4) return false;
    if (pre.kind == PRE_LAYER_NORM && (!pre.w || !pre.b || reinterpret_cast<uintptr_t>(pre.w) % 16 ||
                                       reinterpret_cast<uintptr_t>(pre.b) % 16 || K % 8))
        return false;
    const int64_t db = (int64_t(N) * (K / 32) * 2 + 255) / 256;
    const dim3 block(256);
    const uint8_t* wb = static_cast<const uint8_t*>(w);
#define SAMHIP_PREP(MODE, CH, X86, WT)                                                                               \
    do {                                                                                                             \
        /* staging workgroups: four rows each, two for long rows with no PRE */                                    \
        const int sb = (CH > 4 && pre.kind != PRE_LAYER_NORM) ? (M + 1) / 2 : (M + 3) / 4;                                  \
        const dim3 grid(unsigned(sb + db));                                                                          \
        if (pre.kind == PRE_GELU)                                                                                    \
            hipLaunchKernelGGL((prep_kernel<MODE, CH, X86, WT, PRE_GELU>), grid, block, 0, stream, x, x_stride, M, K, \
                               a, lda, row_scale, sb, wb, w_stride, N, wout, ldo, pre);                              \
        else if (pre.kind == PRE_LAYER_NORM)                                                                         \
            hipLaunchKernelGGL((prep_kernel<MODE, CH, X86, WT, PRE_LAYER_NORM>), grid, block, 0, stream, x, x_stride, \
                               M, K, a, lda, row_scale, sb, wb, w_stride, N, wout, ldo, pre);                        \
        else                                                                                                         \
            hipLaunchKernelGGL((prep_kernel<MODE, CH, X86, WT>), grid, block, 0, stream, x, x_stride, M, K, a, lda,  \
                               row_scale, sb, wb, w_stride, N, wout, ldo, pre);                                      \
    } while (0)
#define SAMHIP_PREP_CH(MODE, X86, WT)                    \
    do {                                                 \
        if (K <= 1024) SAMHIP_PREP(MODE, 2, X86, WT);    \
        else if (K <= 2048) SAMHIP_PREP(MODE, 4, X86, WT); \
        else SAMHIP_PREP(MODE, 10, X86, WT);             \
    } while (0)
    switch (wtype) {
        case T_Q8_0:
            if (mode == T_F16) SAMHIP_PREP_CH(T_F16, false, T_Q8_0);
            else if (x86) SAMHIP_PREP_CH(T_Q8_0, true, T_Q8_0);
            else SAMHIP_PREP_CH(T_Q8_0, false, T_Q8_0);
            break;
        case T_Q4_K:
            if (mode == T_F16) SAMHIP_PREP_CH(T_F16, false, T_Q4_K);
            else SAMHIP_PREP_CH(T_Q8_K, false, T_Q4_K);
            break;
        case T_Q5_K:
            if (mode == T_F16) SAMHIP_PREP_CH(T_F16, false, T_Q5_K);
            else SAMHIP_PREP_CH(T_Q8_K, false, T_Q5_K);
            break;
        case T_Q6_K:
            if (mode == T_F16) SAMHIP_PREP_CH(T_F16, false, T_Q6_K);
            else SAMHIP_PREP_CH(T_Q8_K, false, T_Q6_K);
            break;
        default: return false;
    }
#undef SAMHIP_PREP_CH
#undef SAMHIP_PREP
    return true;
}

bool launch_prep_codes(const int8_t* codes, const float* amax, int64_t ldc, int M, int K, _Float16* a, int64_t lda,
                       float* row_scale, int wtype, const void* w, int64_t w_stride, int N, _Float16* wout,
                       int64_t ldo, hipStream_t stream) {
    // 8-byte code loads and 16-byte operand stores
    if (wtype != T_Q8_0 || M < 1 || N < 1 || K < 32 || K % 32 || ldc % 32 || K > ldc || lda % 8 ||
        reinterpret_cast<uintptr_t>(codes) % 8 || reinterpret_cast<uintptr_t>(amax) % 4 ||
        reinterpret_cast<uintptr_t>(a) % 16)
        return false;
    const int sb = (M + 3) / 4;
    const int64_t db = (int64_t(N) * (K / 32) * 2 + 255) / 256;
    hipLaunchKernelGGL(prep_codes_kernel<T_Q8_0>, dim3(unsigned(sb + db)), dim3(256), 0, stream, codes, amax, ldc, M,
                       K, a, lda, row_scale, sb, static_cast<const uint8_t*>(w), w_stride, N, wout, ldo);
    return true;
}

void launch_stage_rows(int mode, bool aligned, const float* x, int64_t x_stride, int M, int K, _Float16* a,
                       int64_t lda, float* row_scale, int x86, hipStream_t stream) {
    const dim3 grid((M + 3) / 4), block(256);
    if (aligned && K <= 512 * 10) {
#define SAMHIP_STAGE8(MODE, CH)                                                                                 \
    do {                                                                                                        \
        if (MODE == T_Q8_0 && x86)                                                                              \
            hipLaunchKernelGGL((stage8_kernel<MODE, CH, true>), grid, block, 0, stream, x, x_stride, M, K, a,   \
                               lda, row_scale);                                                                 \
        else                                                                                                    \
            hipLaunchKernelGGL((stage8_kernel<MODE, CH, false>), grid, block, 0, stream, x, x_stride, M, K, a,  \
                               lda, row_scale);                                                                 \
    } while (0)
#define SAMHIP_STAGE8_MODE(MODE)                  \
    if (K <= 1024) SAMHIP_STAGE8(MODE, 2);        \
    else if (K <= 2048) SAMHIP_STAGE8(MODE, 4);   \
    else SAMHIP_STAGE8(MODE, 10);
        switch (mode) {
            case T_F16: SAMHIP_STAGE8_MODE(T_F16) break;
            case T_Q8_0: SAMHIP_STAGE8_MODE(T_Q8_0) break;
            case T_Q8_K: SAMHIP_STAGE8_MODE(T_Q8_K) break;
            default: break;
        }
#undef SAMHIP_STAGE8_MODE
#undef SAMHIP_STAGE8
        return;
    }
#define SAMHIP_STAGE(MODE)                                                                                      \
    if (aligned) hipLaunchKernelGGL(stage_rows_kernel<MODE>, grid, block, 0, stream, x, x_stride, M, K, a, lda, \
                                    row_scale, x86);                                                           \
    else hipLaunchKernelGGL(stage_rows_unaligned_kernel<MODE>, grid, block, 0, stream, x, x_stride, M, K, a, lda, \
                            row_scale, x86);
    switch (mode) {
        case T_F16: SAMHIP_STAGE(T_F16) break;
        case T_Q8_0: SAMHIP_STAGE(T_Q8_0) break;
        case T_Q8_K: SAMHIP_STAGE(T_Q8_K) break;
        default: break;
    }
#undef SAMHIP_STAGE
}

// F32 -> F16 rows (ggml_cast to F16: round to nearest even, overflow to inf).
__global__ __launch_bounds__(256) void cast_f16_kernel(const float* __restrict__ x, int64_t x_stride, int rows, int K,
                                                       _Float16* __restrict__ dst) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= int64_t(rows) * K) return;
    const int64_t r = i / K, c = i - r * K;
    dst[i] = (_Float16)x[r * x_stride + c];
}

void launch_cast_f16(const float* x, int64_t x_stride, int rows, int K, _Float16* dst, hipStream_t stream) {
    const int64_t n = int64_t(rows) * K;
    hipLaunchKernelGGL(cast_f16_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, stream, x, x_stride, rows, K,
                       dst);
}

void launch_quantize_act(int type, const float* x, int64_t x_stride, int rows, int K, void* dst, int x86,
                         hipStream_t stream) {
    const dim3 grid((rows + 3) / 4), block(256);
    if (type == T_Q8_0)
        hipLaunchKernelGGL(quantize_act_kernel<T_Q8_0>, grid, block, 0, stream, x, x_stride, rows, K,
                           static_cast<uint8_t*>(dst), x86);
    else
        hipLaunchKernelGGL(quantize_act_kernel<T_Q8_K>, grid, block, 0, stream, x, x_stride, rows, K,
                           static_cast<uint8_t*>(dst), x86);
}

// ---------------------------------------------------------------------------
// ggml-cuda's right-operand formats and the native-activation range rule.
// One lane per value, 32 lanes (half a wave) per 32-value block, so every
// reduction stays inside a lane group and whole groups leave together.
// ---------------------------------------------------------------------------

// 1 when a block of F32 values is outside the native activation's range:
// a non-finite value, or a nonzero block maximum outside [1e-30, 1e30],
// compared as bit patterns so subnormals are not flushed
// (cmake/patches/ggml-native-activation.patch:148-171).
__device__ __forceinline__ bool block_out_of_range(float v) {
    uint32_t bits = __builtin_bit_cast(uint32_t, v) & 0x7fffffffu;
    uint32_t bad = bits >= 0x7f800000u;
    for (int off = 16; off > 0; off >>= 1) {
        bits = max(bits, uint32_t(__shfl_xor(int(bits), off, 32)));
        bad |= uint32_t(__shfl_xor(int(bad), off, 32));
    }
    constexpr uint32_t lower = 0x0da24260u, upper = 0x7149f2cau;   // bits of 1e-30f, 1e30f
    return bad || bits > upper || (bits != 0 && bits < lower);
}

__device__ __forceinline__ float group32_absmax(float v) {
    float a = fabsf(v);
    for (int off = 16; off > 0; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, 32));
    return a;
}

// quantize_q8_1 (MMVQ right operand): d = amax/127, q = roundf(x/d), half d
// and half of the original values' sum in the 32-lane xor-butterfly order.
__global__ __launch_bounds__(256) void quantize_q8_1_kernel(const float* __restrict__ x, int64_t x_stride, int rows,
                                                            int K, uint8_t* __restrict__ dst) {
#pragma clang fp contract(off)
    const int64_t nb = K / 32;
    const int64_t blk = (int64_t(blockIdx.x) * 256 + threadIdx.x) >> 5;
    const int lane = threadIdx.x & 31;
    if (blk >= int64_t(rows) * nb) return;
    const int64_t r = blk / nb, b = blk - r * nb;
    const float v = x[r * x_stride + b * 32 + lane];
    const float amax = group32_absmax(v);
    float s = v;
    for (int off = 16; off > 0; off >>= 1) s = s + __shfl_xor(s, off, 32);
    const float d = amax / 127.f;
    const float qr = amax == 0.f ? 0.f : __builtin_roundf(v / d);
    const float q = qr == qr ? qr : 0.f;   // NaN -> code 0
    uint8_t* out = dst + blk * 36;
    out[4 + lane] = uint8_t(int8_t(q));
    if (lane == 0) {
        *reinterpret_cast<uint16_t*>(out) = float_to_half_bits(d);
        *reinterpret_cast<uint16_t*>(out + 2) = float_to_half_bits(s);
    }
}

// quantize_mmq_q8_1, D4 layout, for Q8_0 products: rows padded with zeros to
// kp (a multiple of 512) values, tile t of 128 values of row r at
// dst + (t*rows + r)*144 = 4 F32 scales, then 128 codes.  d_inv = 127/amax
// correctly rounded, q = roundf(x*d_inv), scale 1/d_inv.  Blocks outside the
// native range set *invalid.
__global__ __launch_bounds__(256) void quantize_q8_1_mmq_kernel(const float* __restrict__ x, int64_t x_stride,
                                                                int rows, int K, int kp, uint8_t* __restrict__ dst,
                                                                int* __restrict__ invalid) {
#pragma clang fp contract(off)
    const int64_t nb = kp / 32;
    const int64_t blk = (int64_t(blockIdx.x) * 256 + threadIdx.x) >> 5;
    const int lane = threadIdx.x & 31;
    if (blk >= int64_t(rows) * nb) return;
    const int64_t r = blk / nb, kb = blk - r * nb;
    const int64_t k = kb * 32 + lane;
    const float v = k < K ? x[r * x_stride + k] : 0.f;
    if (block_out_of_range(v) && lane == 0) atomicOr(invalid, 1);
    const float amax = group32_absmax(v);
    float q = 0.f, d = 0.f;
    if (amax != 0.f) {
        const float d_inv = 127.f / amax;
        const float r = __builtin_roundf(v * d_inv);
        q = r == r ? r : 0.f;   // NaN -> code 0 (such blocks also raise *invalid)
        d = 1.f / d_inv;
    }
    uint8_t* out = dst + ((kb >> 2) * rows + r) * 144;
    out[16 + 32 * (kb & 3) + lane] = uint8_t(int8_t(q));
    if (lane == 0) *reinterpret_cast<float*>(out + 4 * (kb & 3)) = d;
}

// The range rule alone over F32 rows (mul_mat's opt-in activation check).
__global__ __launch_bounds__(256) void q8_rhs_check_kernel(const float* __restrict__ x, int64_t x_stride, int rows,
                                                           int K, int* __restrict__ invalid) {
    const int64_t nb = K / 32;
    const int64_t blk = (int64_t(blockIdx.x) * 256 + threadIdx.x) >> 5;
    const int lane = threadIdx.x & 31;
    if (blk >= int64_t(rows) * nb) return;
    const int64_t r = blk / nb, b = blk - r * nb;
    if (block_out_of_range(x[r * x_stride + b * 32 + lane]) && lane == 0) atomicOr(invalid, 1);
}

void launch_quantize_q8_1(const float* x, int64_t x_stride, int rows, int K, void* dst, hipStream_t stream) {
    const int64_t lanes = int64_t(rows) * K;
    hipLaunchKernelGGL(quantize_q8_1_kernel, dim3(unsigned((lanes + 255) / 256)), dim3(256), 0, stream, x, x_stride,
                       rows, K, static_cast<uint8_t*>(dst));
}

void launch_quantize_q8_1_mmq(const float* x, int64_t x_stride, int rows, int K, void* dst, int* invalid,
                              hipStream_t stream) {
    const int kp = (K + 511) / 512 * 512;
    const int64_t lanes = int64_t(rows) * kp;
    hipLaunchKernelGGL(quantize_q8_1_mmq_kernel, dim3(unsigned((lanes + 255) / 256)), dim3(256), 0, stream, x,
                       x_stride, rows, K, kp, static_cast<uint8_t*>(dst), invalid);
}

void launch_q8_rhs_check(const float* x, int64_t x_stride, int rows, int K, int* invalid, hipStream_t stream) {
    const int64_t lanes = int64_t(rows) * K;
    hipLaunchKernelGGL(q8_rhs_check_kernel, dim3(unsigned((lanes + 255) / 256)), dim3(256), 0, stream, x, x_stride,
                       rows, K, invalid);
}

void launch_dequant_rows(int type, const void* src, int64_t src_stride, const int32_t* ids, int64_t src_rows,
                         float* dst, int64_t dst_stride, int rows, int K, int* bad_id, hipStream_t stream) {
    const int64_t threads = int64_t(rows) * (K / 32);
    const dim3 grid(unsigned((threads + 255) / 256)), block(256);
    const uint8_t* s = static_cast<const uint8_t*>(src);
#define SAMHIP_DQ(T) \
    hipLaunchKernelGGL(dequant_rows_kernel<T>, grid, block, 0, stream, s, src_stride, ids, src_rows, dst, dst_stride, rows, K, bad_id)
    switch (type) {
        case T_F32: SAMHIP_DQ(T_F32); break;
        case T_F16: SAMHIP_DQ(T_F16); break;
        case T_Q8_0: SAMHIP_DQ(T_Q8_0); break;
        case T_Q4_K: SAMHIP_DQ(T_Q4_K); break;
        case T_Q5_K: SAMHIP_DQ(T_Q5_K); break;
        case T_Q6_K: SAMHIP_DQ(T_Q6_K); break;
        case T_Q8_K: SAMHIP_DQ(T_Q8_K); break;
        default: break;
    }
#undef SAMHIP_DQ
}

}  // namespace samhip
