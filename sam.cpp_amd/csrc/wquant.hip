// K-quant weight packing on the device: ggml_quantize_chunk for Q4_K, Q5_K
// and Q6_K without importance weights, i.e. quantize_row_q{4,5,6}_K_ref
// (the path tools/quantize/quantize_rows.cpp:210 takes to pack SAM weights).
// One thread packs one 256-element super-block with the same serial scale
// search ggml runs on the CPU; contraction is disabled and division/sqrt are
// correctly rounded so the bytes match the CPU packer exactly.
#include "internal.hpp"

#pragma clang fp contract(off)

namespace samhip {

namespace {

__device__ __forceinline__ int round_even(float v) { return int(__builtin_rintf(v)); }

__device__ __forceinline__ void put_half(uint8_t* p, float v) {
    const uint16_t h = float_to_half_bits(v);
    p[0] = uint8_t(h & 0xff);
    p[1] = uint8_t(h >> 8);
}

__device__ __forceinline__ float get_half(const uint8_t* p) { return half_bits_to_float(uint32_t(p[0]) | (uint32_t(p[1]) << 8)); }

__device__ void scale_min_of(int j, const uint8_t* packed, int& sc, int& mn) {
    if (j < 4) {
        sc = packed[j] & 63;
        mn = packed[j + 4] & 63;
    } else {
        sc = (packed[j + 4] & 0x0f) | ((packed[j - 4] >> 6) << 4);
        mn = (packed[j + 4] >> 4) | ((packed[j] >> 6) << 4);
    }
}

// Weighted asymmetric fit of 32 values to [0, nmax] (see the CPU restatement).
__device__ float fit_scale_min(int nmax, const float* x, const float* w, uint8_t* codes, float* neg_min,
                               float rmin, int nstep) {
    float lo = x[0], hi = x[0];
    float sum_w = w[0], sum_x = w[0] * x[0];
    for (int i = 1; i < 32; ++i) {
        if (x[i] < lo) lo = x[i];
        if (x[i] > hi) hi = x[i];
        sum_w += w[i];
        sum_x += w[i] * x[i];
    }
    if (lo > 0) lo = 0;
    if (hi == lo) {
        for (int i = 0; i < 32; ++i) codes[i] = 0;
        *neg_min = -lo;
        return 0.f;
    }
    float iscale = nmax / (hi - lo);
    float scale = 1 / iscale;
    float best = 0;
    for (int i = 0; i < 32; ++i) {
        int l = round_even(iscale * (x[i] - lo));
        l = l < 0 ? 0 : (l > nmax ? nmax : l);
        codes[i] = uint8_t(l);
        const float diff = scale * codes[i] + lo - x[i];
        best += w[i] * diff * diff;
    }
    uint8_t trial[32];
    for (int step = 0; step <= nstep; ++step) {
        iscale = (rmin + 0.1f * step + nmax) / (hi - lo);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < 32; ++i) {
            int l = round_even(iscale * (x[i] - lo));
            l = l < 0 ? 0 : (l > nmax ? nmax : l);
            trial[i] = uint8_t(l);
            sum_l += w[i] * l;
            sum_l2 += w[i] * l * l;
            sum_xl += w[i] * l * x[i];
        }
        const float det = sum_w * sum_l2 - sum_l * sum_l;
        if (det > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / det;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / det;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float err = 0;
            for (int i = 0; i < 32; ++i) {
                const float diff = this_scale * trial[i] + this_min - x[i];
                err += w[i] * diff * diff;
            }
            if (err < best) {
                for (int i = 0; i < 32; ++i) codes[i] = trial[i];
                best = err;
                scale = this_scale;
                lo = this_min;
            }
        }
    }
    *neg_min = -lo;
    return scale;
}

// Q4_K / Q5_K: header (d, dmin, 12 scale bytes) and 256 codes in [0, nmax].
__device__ void asym_superblock(const float* x, uint8_t* header, int nmax, float rmin, int nstep, uint8_t* codes) {
    float scales[8], mins[8], weights[32];
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 8; ++j) {
        float sum_x2 = 0;
        for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
        const float av_x = __builtin_sqrtf(sum_x2 / 32);
        for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(x[32 * j + l]);
        scales[j] = fit_scale_min(nmax, x + 32 * j, weights, codes + 32 * j, &mins[j], rmin, nstep);
        if (scales[j] > max_scale) max_scale = scales[j];
        if (mins[j] > max_min) max_min = mins[j];
    }
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    for (int i = 0; i < 16; ++i) header[i] = 0;
    for (int j = 0; j < 8; ++j) {
        uint8_t ls = uint8_t(round_even(inv_scale * scales[j]));
        uint8_t lm = uint8_t(round_even(inv_min * mins[j]));
        ls = ls < 63 ? ls : 63;
        lm = lm < 63 ? lm : 63;
        uint8_t* s = header + 4;
        if (j < 4) {
            s[j] = ls;
            s[j + 4] = lm;
        } else {
            s[j + 4] = uint8_t((ls & 0x0f) | ((lm & 0x0f) << 4));
            s[j - 4] |= uint8_t((ls >> 4) << 6);
            s[j] |= uint8_t((lm >> 4) << 6);
        }
    }
    put_half(header, max_scale / 63.f);
    put_half(header + 2, max_min / 63.f);
    const float d = get_half(header), dmin = get_half(header + 2);
    for (int j = 0; j < 8; ++j) {
        int sc, m;
        scale_min_of(j, header + 4, sc, m);
        const float dj = d * sc;
        if (!dj) continue;
        const float mj = dmin * m;
        for (int i = 0; i < 32; ++i) {
            int l = round_even((x[32 * j + i] + mj) / dj);
            l = l < 0 ? 0 : (l > nmax ? nmax : l);
            codes[32 * j + i] = uint8_t(l);
        }
    }
}

// Symmetric fit of 16 values to [-32, 31] with x^2 weights, 19 candidates.
__device__ float fit_scale_sym16(const float* x, int8_t* codes) {
    const int nmax = 32;
    float amax = 0, smax = 0;
    for (int i = 0; i < 16; ++i) {
        const float a = fabsf(x[i]);
        if (a > amax) { amax = a; smax = x[i]; }
    }
    if (amax < 1e-15f) {
        for (int i = 0; i < 16; ++i) codes[i] = 0;
        return 0.f;
    }
    float iscale = -nmax / smax;
    float sum_lx = 0, sum_l2 = 0;
    for (int i = 0; i < 16; ++i) {
        int l = round_even(iscale * x[i]);
        l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
        codes[i] = int8_t(l + nmax);
        const float w = x[i] * x[i];
        sum_lx += w * x[i] * l;
        sum_l2 += w * l * l;
    }
    float scale = sum_l2 ? sum_lx / sum_l2 : 0.f;
    float best = scale * sum_lx;
    for (int step = -9; step <= 9; ++step) {
        if (step == 0) continue;
        iscale = -(nmax + 0.1f * step) / smax;
        sum_lx = sum_l2 = 0;
        for (int i = 0; i < 16; ++i) {
            int l = round_even(iscale * x[i]);
            l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
            const float w = x[i] * x[i];
            sum_lx += w * x[i] * l;
            sum_l2 += w * l * l;
        }
        if (sum_l2 > 0 && sum_lx * sum_lx > best * sum_l2) {
            for (int i = 0; i < 16; ++i) {
                int l = round_even(iscale * x[i]);
                l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
                codes[i] = int8_t(l + nmax);
            }
            scale = sum_lx / sum_l2;
            best = scale * sum_lx;
        }
    }
    return scale;
}

template <int TYPE>
__global__ __launch_bounds__(64) void quantize_weights_kernel(const float* __restrict__ x, int64_t x_stride, int rows,
                                                              int K, uint8_t* __restrict__ dst) {
    const int nb = K / 256;
    const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= int64_t(rows) * nb) return;
    const int r = int(t / nb), b = int(t % nb);
    const float* xb = x + int64_t(r) * x_stride + 256 * b;
    constexpr int BB = block_bytes(TYPE);
    uint8_t* out = dst + (int64_t(r) * nb + b) * BB;
    if (TYPE == T_Q4_K || TYPE == T_Q5_K) {
        uint8_t codes[256];
        uint8_t header[16];
        if (TYPE == T_Q4_K) asym_superblock(xb, header, 15, -1.f, 20, codes);
        else asym_superblock(xb, header, 31, -0.5f, 15, codes);
        for (int i = 0; i < 16; ++i) out[i] = header[i];
        if (TYPE == T_Q4_K) {
            for (int c = 0; c < 4; ++c)
                for (int l = 0; l < 32; ++l)
                    out[16 + 32 * c + l] = uint8_t(codes[64 * c + l] | (codes[64 * c + 32 + l] << 4));
        } else {
            uint8_t qh[32];
            for (int l = 0; l < 32; ++l) qh[l] = 0;
            for (int c = 0; c < 4; ++c) {
                for (int l = 0; l < 32; ++l) {
                    int lo = codes[64 * c + l], hi = codes[64 * c + 32 + l];
                    if (lo > 15) { lo -= 16; qh[l] |= uint8_t(1u << (2 * c)); }
                    if (hi > 15) { hi -= 16; qh[l] |= uint8_t(2u << (2 * c)); }
                    out[48 + 32 * c + l] = uint8_t(lo | (hi << 4));
                }
            }
            for (int l = 0; l < 32; ++l) out[16 + l] = qh[l];
        }
    } else {
        int8_t codes[256];
        float scales[16];
        float max_scale = 0, max_abs = 0;
        for (int s = 0; s < 16; ++s) {
            scales[s] = fit_scale_sym16(xb + 16 * s, codes + 16 * s);
            const float a = fabsf(scales[s]);
            if (a > max_abs) { max_abs = a; max_scale = scales[s]; }
        }
        for (int i = 0; i < 210; ++i) out[i] = 0;
        if (max_abs < 1e-15f) return;
        const float iscale = -128.f / max_scale;
        put_half(out + 208, 1 / iscale);
        int8_t* sc = reinterpret_cast<int8_t*>(out + 192);
        for (int s = 0; s < 16; ++s) {
            const int v = round_even(iscale * scales[s]);
            sc[s] = int8_t(v < 127 ? v : 127);
        }
        const float d = get_half(out + 208);
        for (int s = 0; s < 16; ++s) {
            const float ds = d * sc[s];
            if (!ds) continue;
            for (int i = 0; i < 16; ++i) {
                int l = round_even(xb[16 * s + i] / ds);
                l = l < -32 ? -32 : (l > 31 ? 31 : l);
                codes[16 * s + i] = int8_t(l + 32);
            }
        }
        for (int h = 0; h < 2; ++h) {
            const int8_t* c = codes + 128 * h;
            for (int l = 0; l < 32; ++l) {
                out[64 * h + l] = uint8_t((c[l] & 0x0f) | ((c[l + 64] & 0x0f) << 4));
                out[64 * h + 32 + l] = uint8_t((c[l + 32] & 0x0f) | ((c[l + 96] & 0x0f) << 4));
                out[128 + 32 * h + l] = uint8_t(((c[l] >> 4) & 3) | (((c[l + 32] >> 4) & 3) << 2) |
                                                (((c[l + 64] >> 4) & 3) << 4) | (((c[l + 96] >> 4) & 3) << 6));
            }
        }
    }
}

}  // namespace

void launch_quantize_weights(int type, const float* x, int64_t x_stride, int rows, int K, void* dst,
                             hipStream_t stream) {
    const int64_t threads = int64_t(rows) * (K / 256);
    const dim3 grid(unsigned((threads + 63) / 64)), block(64);
    uint8_t* d = static_cast<uint8_t*>(dst);
    switch (type) {
        case T_Q4_K: hipLaunchKernelGGL(quantize_weights_kernel<T_Q4_K>, grid, block, 0, stream, x, x_stride, rows, K, d); break;
        case T_Q5_K: hipLaunchKernelGGL(quantize_weights_kernel<T_Q5_K>, grid, block, 0, stream, x, x_stride, rows, K, d); break;
        case T_Q6_K: hipLaunchKernelGGL(quantize_weights_kernel<T_Q6_K>, grid, block, 0, stream, x, x_stride, rows, K, d); break;
        default: break;
    }
}

}  // namespace samhip
