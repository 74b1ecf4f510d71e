/*
 * CPU oracle for the quantized mul_mat path — TEST INFRASTRUCTURE ONLY.
 * See ggml_oracle.h for what pins each function.  Only tests/, the smoke
 * check and bench.py's cpu_baseline leg load this library.
 *
 * The algorithms restated here are ggml 0.26.0's (d7cb5741) CPU reference
 * routines, which the reference reaches through ggml_get_type_traits(_cpu)
 * (src/runtime/ggml/backends/cpu.hpp:13-23, tests/runtime/ggml/
 * test_quantization.cpp:46-68) and ggml_quantize_chunk
 * (tools/quantize/quantize_rows.cpp:210).  ggml itself is not present in the
 * reference tree, so each routine below is written from the published
 * algorithm, not copied.
 */
#include "ggml_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK8 32
#define QKK 256

/* ---- block layouts (byte offsets) -------------------------------------- */
/* Q8_0 : f16 d @0, i8 q[32] @2                              = 34 B / 32    */
/* Q8_K : f32 d @0, i8 q[256] @4, i16 bsums[16] @260          = 292 B / 256  */
/* Q4_K : f16 d @0, f16 dmin @2, u8 sc[12] @4, u8 qs[128] @16 = 144 B / 256  */
/* Q5_K : Q4_K header, u8 qh[32] @16, u8 qs[128] @48          = 176 B / 256  */
/* Q6_K : u8 ql[128] @0, u8 qh[64] @128, i8 sc[16] @192, f16 d @208 = 210 B  */

int64_t or_block_elems(int type) {
    switch (type) {
        case OR_F32: case OR_F16: return 1;
        case OR_Q8_0: return QK8;
        case OR_Q4_K: case OR_Q5_K: case OR_Q6_K: case OR_Q8_K: return QKK;
        default: return 0;
    }
}

int64_t or_block_bytes(int type) {
    switch (type) {
        case OR_F32: return 4;
        case OR_F16: return 2;
        case OR_Q8_0: return 34;
        case OR_Q4_K: return 144;
        case OR_Q5_K: return 176;
        case OR_Q6_K: return 210;
        case OR_Q8_K: return 292;
        default: return 0;
    }
}

int64_t or_row_bytes(int type, int64_t k) {
    const int64_t be = or_block_elems(type);
    if (be <= 0 || k <= 0 || k % be) return -1;
    return k / be * or_block_bytes(type);
}

int or_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

static void set_threads(int threads) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
}

/* ---- IEEE binary16 conversion, round to nearest even -------------------- */

uint16_t or_fp32_to_fp16(float f) {
    uint32_t bits;
    memcpy(&bits, &f, 4);
    const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    const uint32_t mag = bits & 0x7fffffffu;
    if (mag > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((mag >> 13) & 0x3ffu)); /* quiet NaN */
    if (mag >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  /* >= 65520 (and inf) -> inf */
    if (mag >= 0x38800000u) {                                   /* normal half */
        uint32_t h = (mag - 0x38000000u) >> 13;                 /* rebias 127 -> 15 */
        const uint32_t rest = mag & 0x1fffu;
        if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h;
        return (uint16_t)(sign | h);
    }
    if (mag < 0x33000000u) return sign;                         /* < 2^-25 -> zero */
    {
        /* subnormal half: units of 2^-24 */
        const uint32_t exponent = mag >> 23;
        const uint32_t significand = (mag & 0x7fffffu) | 0x800000u;
        const int shift = 126 - (int)exponent;                  /* 14 .. 24 */
        uint32_t q = significand >> shift;
        const uint32_t rest = significand & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1);
        if (rest > half || (rest == half && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
}

float or_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t exponent = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t mantissa = (uint32_t)h & 0x3ffu;
    uint32_t bits;
    if (exponent == 0x1f) {
        bits = sign | 0x7f800000u | (mantissa << 13);
    } else if (exponent != 0) {
        bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    } else if (mantissa == 0) {
        bits = sign;
    } else {
        /* subnormal: value = mantissa * 2^-24, exact in binary32 */
        float v = (float)mantissa * 5.9604644775390625e-8f;
        memcpy(&bits, &v, 4);
        bits |= sign;
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

void or_fp32_to_fp16_rows(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = or_fp32_to_fp16(x[i]);
}

void or_fp16_to_fp32_rows(const uint16_t* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = or_fp16_to_fp32(x[i]);
}

/* ---- portable normal generator ----------------------------------------- */

static uint64_t splitmix64_next(uint64_t* state) {
    uint64_t z = (*state += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

static inline uint64_t rotl64(uint64_t v, int s) { return (v << s) | (v >> (64 - s)); }

static uint64_t xoshiro_next(uint64_t s[4]) {
    const uint64_t result = rotl64(s[1] * 5u, 7) * 9u;
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl64(s[3], 45);
    return result;
}

void or_rng_normal(uint64_t seed, float mean, float stddev, float* out, int64_t n) {
    uint64_t sm = seed, s[4];
    for (int i = 0; i < 4; ++i) s[i] = splitmix64_next(&sm);
    const double two_pi = 6.283185307179586476925286766559;
    for (int64_t i = 0; i < n; i += 2) {
        const double u1 = ((double)(xoshiro_next(s) >> 11) + 1.0) * 0x1.0p-53; /* (0, 1] */
        const double u2 = (double)(xoshiro_next(s) >> 11) * 0x1.0p-53;         /* [0, 1) */
        const double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(mean + stddev * r * cos(two_pi * u2));
        if (i + 1 < n) out[i + 1] = (float)(mean + stddev * r * sin(two_pi * u2));
    }
}

/* ---- helpers ------------------------------------------------------------ */

/* ggml's nearest_int: round half to even for |v| < 2^22; a NaN gives 0, as
 * nearest_int's bit trick does ((0x7fc00000 & 0x7fffff) - 0x400000). */
static inline int round_even(float v) { return isnan(v) ? 0 : (int)rintf(v); }

static inline void put_f16(uint8_t* p, float v) {
    const uint16_t h = or_fp32_to_fp16(v);
    memcpy(p, &h, 2);
}

static inline float get_f16(const uint8_t* p) {
    uint16_t h;
    memcpy(&h, p, 2);
    return or_fp16_to_fp32(h);
}

/* 6-bit scale/min of sub-block j (0..7) from the 12 packed bytes of a
 * Q4_K/Q5_K super-block: j<4 keep their low 6 bits in bytes j and j+4;
 * j>=4 take a nibble from byte j+4 and two high bits from bytes j-4 / j. */
static inline void k4_scale_min(int j, const uint8_t* packed, int* scale, int* min) {
    if (j < 4) {
        *scale = packed[j] & 63;
        *min = packed[j + 4] & 63;
    } else {
        *scale = (packed[j + 4] & 0x0f) | ((packed[j - 4] >> 6) << 4);
        *min = (packed[j + 4] >> 4) | ((packed[j] >> 6) << 4);
    }
}

/* ---- Q8_0 / Q8_K activation & weight packing --------------------------- */

static void q8_0_block(const float* x, uint8_t* out, int rounding) {
    float amax = 0.f;
    for (int j = 0; j < QK8; ++j) {
        const float a = fabsf(x[j]);
        amax = a > amax ? a : amax;
    }
    const float d = amax / 127.f;
    float inv;
    if (rounding == OR_Q8_ROUND_X86) inv = amax != 0.f ? 127.f / amax : 0.f;
    else inv = d != 0.f ? 1.f / d : 0.f;
    put_f16(out, d);
    int8_t* q = (int8_t*)(out + 2);
    for (int j = 0; j < QK8; ++j) {
        const float v = x[j] * inv;
        const float r = rounding == OR_Q8_ROUND_X86 ? rintf(v) : roundf(v);
        q[j] = isnan(r) ? 0 : (int8_t)r;   /* NaN -> code 0: Q8_K's nearest_int rule, chosen for both Q8_0
                                              roundings (ggml's AVX2 packing would give -128 instead) */
    }
}

int or_quantize_q8_0(const float* x, void* y, int64_t rows, int64_t k, int rounding) {
    if (k <= 0 || k % QK8 || rows < 0) return -1;
    const int64_t nb = k / QK8;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t b = 0; b < nb; ++b)
            q8_0_block(x + r * k + b * QK8, (uint8_t*)y + (r * nb + b) * 34, rounding);
    return 0;
}

static void q8_k_block(const float* x, uint8_t* out) {
    float amax = 0.f, signed_max = 0.f;
    for (int j = 0; j < QKK; ++j) {
        const float a = fabsf(x[j]);
        if (a > amax) { amax = a; signed_max = x[j]; }
    }
    int8_t* q = (int8_t*)(out + 4);
    int16_t sums[16];
    if (amax == 0.f) {
        const float zero = 0.f;
        memcpy(out, &zero, 4);
        memset(q, 0, QKK);
        memset(sums, 0, sizeof(sums));
        memcpy(out + 260, sums, sizeof(sums));
        return;
    }
    const float iscale = -127.f / signed_max;
    for (int j = 0; j < QKK; ++j) {
        const int v = round_even(iscale * x[j]);
        q[j] = (int8_t)(v < 127 ? v : 127);
    }
    for (int g = 0; g < 16; ++g) {
        int s = 0;
        for (int i = 0; i < 16; ++i) s += q[16 * g + i];
        sums[g] = (int16_t)s;
    }
    const float d = 1.f / iscale;
    memcpy(out, &d, 4);
    memcpy(out + 260, sums, sizeof(sums));
}

int or_quantize_q8_k(const float* x, void* y, int64_t rows, int64_t k) {
    if (k <= 0 || k % QKK || rows < 0) return -1;
    const int64_t nb = k / QKK;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t b = 0; b < nb; ++b)
            q8_k_block(x + r * k + b * QKK, (uint8_t*)y + (r * nb + b) * 292);
    return 0;
}

/* ---- K-quant weight quantizers (ggml quantize_row_q{4,5,6}_K_ref) ------- */

/* Asymmetric fit of n values to [0, nmax] codes with a weighted least-squares
 * refinement over nstep+1 candidate inverse scales; returns the scale and
 * stores -min (>= 0) in *neg_min. */
static float fit_scale_min(int n, int nmax, const float* x, const float* w, uint8_t* codes,
                           float* neg_min, uint8_t* trial, float rmin, float rdelta, int nstep) {
    float lo = x[0], hi = x[0];
    float sum_w = w[0], sum_x = w[0] * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < lo) lo = x[i];
        if (x[i] > hi) hi = x[i];
        sum_w += w[i];
        sum_x += w[i] * x[i];
    }
    if (lo > 0) lo = 0;
    if (hi == lo) {
        for (int i = 0; i < n; ++i) codes[i] = 0;
        *neg_min = -lo;
        return 0.f;
    }
    float iscale = nmax / (hi - lo);
    float scale = 1 / iscale;
    float best = 0;
    for (int i = 0; i < n; ++i) {
        int l = round_even(iscale * (x[i] - lo));
        l = l < 0 ? 0 : (l > nmax ? nmax : l);
        codes[i] = (uint8_t)l;
        const float diff = scale * codes[i] + lo - x[i];
        best += w[i] * diff * diff;
    }
    for (int step = 0; step <= nstep; ++step) {
        iscale = (rmin + rdelta * step + nmax) / (hi - lo);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = round_even(iscale * (x[i] - lo));
            l = l < 0 ? 0 : (l > nmax ? nmax : l);
            trial[i] = (uint8_t)l;
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
            for (int i = 0; i < n; ++i) {
                const float diff = this_scale * trial[i] + this_min - x[i];
                err += w[i] * diff * diff;
            }
            if (err < best) {
                memcpy(codes, trial, (size_t)n);
                best = err;
                scale = this_scale;
                lo = this_min;
            }
        }
    }
    *neg_min = -lo;
    return scale;
}

/* Packs 8 (scale, min) 6-bit pairs into 12 bytes (inverse of k4_scale_min). */
static void pack_scale_min(const uint8_t ls[8], const uint8_t lm[8], uint8_t packed[12]) {
    for (int j = 0; j < 8; ++j) {
        if (j < 4) {
            packed[j] = ls[j];
            packed[j + 4] = lm[j];
        } else {
            packed[j + 4] = (uint8_t)((ls[j] & 0x0f) | ((lm[j] & 0x0f) << 4));
            packed[j - 4] |= (uint8_t)((ls[j] >> 4) << 6);
            packed[j] |= (uint8_t)((lm[j] >> 4) << 6);
        }
    }
}

/* First phase of the Q4_K/Q5_K quantizers: each 32-element sub-block fitted
 * with the weights sqrt(mean x^2) + |x| (scales[j], mins[j] = -min, codes). */
static void kquant_asym_fit(const float* x, int nmax, float rmin, int nstep, float scales[8], float mins[8],
                            uint8_t codes[QKK]) {
    float weights[32];
    uint8_t trial[32];
    for (int j = 0; j < 8; ++j) {
        float sum_x2 = 0;
        for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
        const float av_x = sqrtf(sum_x2 / 32);
        for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(x[32 * j + l]);
        scales[j] = fit_scale_min(32, nmax, x + 32 * j, weights, codes + 32 * j, &mins[j], trial, rmin, 0.1f, nstep);
    }
}

/* Shared body of the Q4_K/Q5_K reference quantizers: per 32-element
 * sub-block fit, 6-bit quantized scales/mins, then requantized codes. */
static void kquant_asym_block(const float* x, uint8_t* header, int nmax, float rmin, int nstep, uint8_t codes[QKK]) {
    float scales[8], mins[8];
    float max_scale = 0, max_min = 0;
    kquant_asym_fit(x, nmax, rmin, nstep, scales, mins, codes);
    for (int j = 0; j < 8; ++j) {
        if (scales[j] > max_scale) max_scale = scales[j];
        if (mins[j] > max_min) max_min = mins[j];
    }
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    uint8_t ls[8], lm[8];
    for (int j = 0; j < 8; ++j) {
        const uint8_t s = (uint8_t)round_even(inv_scale * scales[j]);
        const uint8_t m = (uint8_t)round_even(inv_min * mins[j]);
        ls[j] = s < 63 ? s : 63;
        lm[j] = m < 63 ? m : 63;
    }
    memset(header, 0, 16);
    pack_scale_min(ls, lm, header + 4);
    put_f16(header, max_scale / 63.f);
    put_f16(header + 2, max_min / 63.f);
    const float d = get_f16(header), dmin = get_f16(header + 2);
    for (int j = 0; j < 8; ++j) {
        int sc, m;
        k4_scale_min(j, header + 4, &sc, &m);
        const float dj = d * sc;
        if (!dj) continue;
        const float mj = dmin * m;
        for (int i = 0; i < 32; ++i) {
            int l = round_even((x[32 * j + i] + mj) / dj);
            l = l < 0 ? 0 : (l > nmax ? nmax : l);
            codes[32 * j + i] = (uint8_t)l;
        }
    }
}

int or_quantize_q4_k(const float* x, void* y, int64_t rows, int64_t k) {
    if (k <= 0 || k % QKK || rows < 0) return -1;
    const int64_t nb = k / QKK;
    uint8_t codes[QKK];
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t b = 0; b < nb; ++b) {
            uint8_t* out = (uint8_t*)y + (r * nb + b) * 144;
            kquant_asym_block(x + r * k + b * QKK, out, 15, -1.f, 20, codes);
            uint8_t* qs = out + 16;
            for (int c = 0; c < 4; ++c)             /* 64-element chunk c: low nibble first 32 */
                for (int l = 0; l < 32; ++l)
                    qs[32 * c + l] = (uint8_t)(codes[64 * c + l] | (codes[64 * c + 32 + l] << 4));
        }
    }
    return 0;
}

int or_quantize_q5_k(const float* x, void* y, int64_t rows, int64_t k) {
    if (k <= 0 || k % QKK || rows < 0) return -1;
    const int64_t nb = k / QKK;
    uint8_t codes[QKK];
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t b = 0; b < nb; ++b) {
            uint8_t* out = (uint8_t*)y + (r * nb + b) * 176;
            kquant_asym_block(x + r * k + b * QKK, out, 31, -0.5f, 15, codes);
            uint8_t* qh = out + 16;
            uint8_t* qs = out + 48;
            memset(qh, 0, 32);
            for (int c = 0; c < 4; ++c) {
                for (int l = 0; l < 32; ++l) {
                    int lo = codes[64 * c + l], hi = codes[64 * c + 32 + l];
                    if (lo > 15) { lo -= 16; qh[l] |= (uint8_t)(1u << (2 * c)); }
                    if (hi > 15) { hi -= 16; qh[l] |= (uint8_t)(2u << (2 * c)); }
                    qs[32 * c + l] = (uint8_t)(lo | (hi << 4));
                }
            }
        }
    }
    return 0;
}

/* Symmetric fit of n values to [-nmax, nmax-1] (ggml make_qx_quants with
 * rmse_type 1: weights x^2, 19 candidate scales). */
static float fit_scale_sym(int n, int nmax, const float* x, int8_t* codes) {
    float amax = 0, signed_max = 0;
    for (int i = 0; i < n; ++i) {
        const float a = fabsf(x[i]);
        if (a > amax) { amax = a; signed_max = x[i]; }
    }
    if (amax < 1e-15f) {
        for (int i = 0; i < n; ++i) codes[i] = 0;
        return 0.f;
    }
    float iscale = -nmax / signed_max;
    float sum_lx = 0, sum_l2 = 0;
    for (int i = 0; i < n; ++i) {
        int l = round_even(iscale * x[i]);
        l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
        codes[i] = (int8_t)(l + nmax);
        const float w = x[i] * x[i];
        sum_lx += w * x[i] * l;
        sum_l2 += w * l * l;
    }
    float scale = sum_l2 ? sum_lx / sum_l2 : 0.f;
    float best = scale * sum_lx;
    for (int step = -9; step <= 9; ++step) {
        if (step == 0) continue;
        iscale = -(nmax + 0.1f * step) / signed_max;
        sum_lx = sum_l2 = 0;
        for (int i = 0; i < n; ++i) {
            int l = round_even(iscale * x[i]);
            l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
            const float w = x[i] * x[i];
            sum_lx += w * x[i] * l;
            sum_l2 += w * l * l;
        }
        if (sum_l2 > 0 && sum_lx * sum_lx > best * sum_l2) {
            for (int i = 0; i < n; ++i) {
                int l = round_even(iscale * x[i]);
                l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
                codes[i] = (int8_t)(l + nmax);
            }
            scale = sum_lx / sum_l2;
            best = scale * sum_lx;
        }
    }
    return scale;
}

/* First phase of the Q6_K quantizer: each 16-element sub-block fitted
 * symmetrically (scales[s], codes l + 32). */
static void q6_k_fit(const float* xb, float scales[16], int8_t codes[QKK]) {
    for (int s = 0; s < 16; ++s) scales[s] = fit_scale_sym(16, 32, xb + 16 * s, codes + 16 * s);
}

int or_quantize_q6_k(const float* x, void* y, int64_t rows, int64_t k) {
    if (k <= 0 || k % QKK || rows < 0) return -1;
    const int64_t nb = k / QKK;
    int8_t codes[QKK];
    float scales[16];
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t b = 0; b < nb; ++b) {
            const float* xb = x + r * k + b * QKK;
            uint8_t* out = (uint8_t*)y + (r * nb + b) * 210;
            float max_scale = 0, max_abs = 0;
            q6_k_fit(xb, scales, codes);
            for (int s = 0; s < 16; ++s) {
                const float a = fabsf(scales[s]);
                if (a > max_abs) { max_abs = a; max_scale = scales[s]; }
            }
            memset(out, 0, 210);
            if (max_abs < 1e-15f) continue;                 /* all-zero block */
            const float iscale = -128.f / max_scale;
            put_f16(out + 208, 1 / iscale);
            int8_t* sc = (int8_t*)(out + 192);
            for (int s = 0; s < 16; ++s) {
                const int v = round_even(iscale * scales[s]);
                sc[s] = (int8_t)(v < 127 ? v : 127);
            }
            const float d = get_f16(out + 208);
            for (int s = 0; s < 16; ++s) {
                const float ds = d * sc[s];
                if (!ds) continue;
                for (int i = 0; i < 16; ++i) {
                    int l = round_even(xb[16 * s + i] / ds);
                    l = l < -32 ? -32 : (l > 31 ? 31 : l);
                    codes[16 * s + i] = (int8_t)(l + 32);
                }
            }
            uint8_t* ql = out;
            uint8_t* qh = out + 128;
            for (int h = 0; h < 2; ++h) {                    /* two 128-element halves */
                const int8_t* c = codes + 128 * h;
                for (int l = 0; l < 32; ++l) {
                    ql[64 * h + l] = (uint8_t)((c[l] & 0x0f) | ((c[l + 64] & 0x0f) << 4));
                    ql[64 * h + 32 + l] = (uint8_t)((c[l + 32] & 0x0f) | ((c[l + 96] & 0x0f) << 4));
                    qh[32 * h + l] = (uint8_t)(((c[l] >> 4) & 3) | (((c[l + 32] >> 4) & 3) << 2) |
                                               (((c[l + 64] >> 4) & 3) << 4) | (((c[l + 96] >> 4) & 3) << 6));
                }
            }
        }
    }
    return 0;
}

int or_kquant_fit(int type, const float* x, float* scales, float* mins, uint8_t* codes) {
    switch (type) {
        case OR_Q4_K: kquant_asym_fit(x, 15, -1.f, 20, scales, mins, codes); return 0;
        case OR_Q5_K: kquant_asym_fit(x, 31, -0.5f, 15, scales, mins, codes); return 0;
        case OR_Q6_K: q6_k_fit(x, scales, (int8_t*)codes); return 0;
        default: return -1;
    }
}

/* ---- ggml-cuda activation formats --------------------------------------- */

/* quantize_q8_1 (MMVQ right operand, as pinned by tools/validation/
 * verify_q8_rhs_staging.py:24-83): d = amax/127, q = roundf(x/d) (ties away),
 * zero block -> zeros; stored half d and half of the original values' sum,
 * reduced in the 32-lane xor-butterfly order (offsets 16, 8, 4, 2, 1). */
static void q8_1_block(const float* x, uint8_t* out) {
    float amax = 0.f;
    for (int j = 0; j < QK8; ++j) {
        const float a = fabsf(x[j]);
        amax = a > amax ? a : amax;
    }
    float lanes[QK8];
    memcpy(lanes, x, sizeof(lanes));
    for (int off = 16; off > 0; off >>= 1) {
        float next[QK8];
        for (int j = 0; j < QK8; ++j) next[j] = lanes[j] + lanes[j ^ off];
        memcpy(lanes, next, sizeof(lanes));
    }
    const float d = amax / 127.f;
    int8_t* q = (int8_t*)(out + 4);
    for (int j = 0; j < QK8; ++j) q[j] = (int8_t)(amax == 0.f ? 0.f : roundf(x[j] / d));
    put_f16(out, d);
    put_f16(out + 2, lanes[0]);
}

int or_quantize_q8_1(const float* x, void* y, int64_t rows, int64_t k) {
    if (k <= 0 || k % QK8 || rows < 0) return -1;
    const int64_t nb = k / QK8;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t b = 0; b < nb; ++b) q8_1_block(x + r * k + b * QK8, (uint8_t*)y + (r * nb + b) * 36);
    return 0;
}

/* The native-activation range rule (cmake/patches/ggml-native-activation.patch:
 * 148-171, tools/quantize/native_activation.py:24-40): finite values, and
 * each nonzero 32-value block maximum in [1e-30, 1e30], compared as F32 bit
 * patterns (no flush of subnormals).  1 when every block passes. */
int or_q8_rhs_supported(const float* x, int64_t rows, int64_t k) {
    if (k <= 0 || k % QK8 || rows < 0) return 0;
    uint32_t lower, upper;
    const float lo = 1.e-30f, hi = 1.e30f;
    memcpy(&lower, &lo, 4);
    memcpy(&upper, &hi, 4);
    for (int64_t i = 0; i < rows * k; i += QK8) {
        uint32_t maximum = 0;
        for (int j = 0; j < QK8; ++j) {
            uint32_t bits;
            memcpy(&bits, x + i + j, 4);
            bits &= 0x7fffffffu;
            if (bits >= 0x7f800000u) return 0;
            maximum = bits > maximum ? bits : maximum;
        }
        if (maximum > upper || (maximum != 0 && maximum < lower)) return 0;
    }
    return 1;
}

/* quantize_mmq_q8_1 with the D4 layout (ggml-cuda MMQ right operand for
 * Q8_0 weights, K padded to 512 with zeros; tools/quantize/
 * native_activation.py:42-62): d_inv = 127/amax (correctly rounded,
 * cmake/patches/ggml-precise-cuda.patch:627-633), q = roundf(x * d_inv),
 * stored F32 scale d = 1/d_inv, zero block -> zeros.  Layout [kp/128 tile]
 * [row][4 F32 scales | 128 codes] = 144 B per row and tile. */
int64_t or_q8_1_mmq_bytes(int64_t rows, int64_t k) { return (k + 511) / 512 * 4 * rows * 144; }

int or_quantize_q8_1_mmq(const float* x, void* y, int64_t rows, int64_t k) {
    if (k <= 0 || k % QK8 || rows < 0) return -1;
    const int64_t kp = (k + 511) / 512 * 512, tiles = kp / 128;
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t t = 0; t < tiles; ++t) {
            uint8_t* out = (uint8_t*)y + (t * rows + r) * 144;
            for (int s = 0; s < 4; ++s) {
                const int64_t k0 = t * 128 + s * 32;
                float v[QK8];
                for (int j = 0; j < QK8; ++j) v[j] = k0 + j < k ? x[r * k + k0 + j] : 0.f;
                float amax = 0.f;
                for (int j = 0; j < QK8; ++j) amax = fabsf(v[j]) > amax ? fabsf(v[j]) : amax;
                float d = 0.f;
                int8_t* q = (int8_t*)(out + 16 + 32 * s);
                if (amax != 0.f) {
                    const float d_inv = 127.f / amax;
                    for (int j = 0; j < QK8; ++j) q[j] = (int8_t)roundf(v[j] * d_inv);
                    d = 1.f / d_inv;
                } else {
                    memset(q, 0, QK8);
                }
                memcpy(out + 4 * s, &d, 4);
            }
        }
    }
    return 0;
}

int64_t or_quantize_chunk(int type, const float* x, void* y, int64_t rows, int64_t k) {
    int rc;
    switch (type) {
        case OR_Q8_0: rc = or_quantize_q8_0(x, y, rows, k, OR_Q8_ROUND_REF); break;
        case OR_Q4_K: rc = or_quantize_q4_k(x, y, rows, k); break;
        case OR_Q5_K: rc = or_quantize_q5_k(x, y, rows, k); break;
        case OR_Q6_K: rc = or_quantize_q6_k(x, y, rows, k); break;
        default: return -1;
    }
    return rc ? -1 : rows * or_row_bytes(type, k);
}

/* ---- to_float ----------------------------------------------------------- */

static void dequant_block(int type, const uint8_t* b, float* y) {
    switch (type) {
        case OR_Q8_0: {
            const float d = get_f16(b);
            const int8_t* q = (const int8_t*)(b + 2);
            for (int j = 0; j < QK8; ++j) y[j] = d * q[j];
            break;
        }
        case OR_Q8_K: {
            float d;
            memcpy(&d, b, 4);
            const int8_t* q = (const int8_t*)(b + 4);
            for (int j = 0; j < QKK; ++j) y[j] = d * q[j];
            break;
        }
        case OR_Q4_K:
        case OR_Q5_K: {
            const float d = get_f16(b), dmin = get_f16(b + 2);
            const uint8_t* qh = b + 16;
            const uint8_t* qs = b + (type == OR_Q4_K ? 16 : 48);
            for (int j = 0; j < 8; ++j) {
                int sc, m;
                k4_scale_min(j, b + 4, &sc, &m);
                const float dj = d * sc, mj = dmin * m;
                const uint8_t* q = qs + 32 * (j / 2);
                for (int l = 0; l < 32; ++l) {
                    int v = (j & 1) ? (q[l] >> 4) : (q[l] & 0x0f);
                    if (type == OR_Q5_K && ((qh[l] >> j) & 1)) v += 16;
                    y[32 * j + l] = dj * v - mj;
                }
            }
            break;
        }
        case OR_Q6_K: {
            const float d = get_f16(b + 208);
            const int8_t* sc = (const int8_t*)(b + 192);
            for (int e = 0; e < QKK; ++e) {
                const int h = e / 128, r = e % 128, g = r / 32, l = r % 32;
                const uint8_t lowbyte = b[64 * h + 32 * (g & 1) + l];
                const int low = (g < 2) ? (lowbyte & 0x0f) : (lowbyte >> 4);
                const int high = (b[128 + 32 * h + l] >> (2 * g)) & 3;
                const int q = (low | (high << 4)) - 32;
                y[e] = d * sc[8 * h + 2 * g + l / 16] * q;
            }
            break;
        }
        default: break;
    }
}

int or_dequantize(int type, const void* x, float* y, int64_t rows, int64_t k) {
    const int64_t be = or_block_elems(type), bb = or_block_bytes(type);
    if (type == OR_F32 || type == OR_F16 || be <= 0 || k <= 0 || k % be || rows < 0) return -1;
    const int64_t nb = k / be;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t b = 0; b < nb; ++b)
            dequant_block(type, (const uint8_t*)x + (r * nb + b) * bb, y + r * k + b * be);
    return 0;
}

/* ---- block dots (ggml vec_dot_*_q8_*) ----------------------------------- */

static float dot_q8_0(const uint8_t* w, const uint8_t* x, int64_t nb) {
    float sum = 0.f;
    for (int64_t b = 0; b < nb; ++b, w += 34, x += 34) {
        const int8_t* qw = (const int8_t*)(w + 2);
        const int8_t* qx = (const int8_t*)(x + 2);
        int isum = 0;
        for (int j = 0; j < QK8; ++j) isum += qw[j] * qx[j];
        sum += (float)isum * (get_f16(w) * get_f16(x));
    }
    return sum;
}

static inline float q8k_d(const uint8_t* x) {
    float d;
    memcpy(&d, x, 4);
    return d;
}

static inline int q8k_bsum(const uint8_t* x, int g) {
    int16_t s;
    memcpy(&s, x + 260 + 2 * g, 2);
    return s;
}

static float dot_q45_k(int type, const uint8_t* w, const uint8_t* x, int64_t nb) {
    const int bb = type == OR_Q4_K ? 144 : 176;
    float sum = 0.f;
    for (int64_t b = 0; b < nb; ++b, w += bb, x += 292) {
        const int8_t* qx = (const int8_t*)(x + 4);
        const uint8_t* qh = w + 16;
        const uint8_t* qs = w + (type == OR_Q4_K ? 16 : 48);
        int isum = 0, msum = 0;
        for (int j = 0; j < 8; ++j) {
            int sc, m;
            k4_scale_min(j, w + 4, &sc, &m);
            const uint8_t* q = qs + 32 * (j / 2);
            int part = 0;
            for (int l = 0; l < 32; ++l) {
                int v = (j & 1) ? (q[l] >> 4) : (q[l] & 0x0f);
                if (type == OR_Q5_K && ((qh[l] >> j) & 1)) v += 16;
                part += v * qx[32 * j + l];
            }
            isum += sc * part;
            msum += m * (q8k_bsum(x, 2 * j) + q8k_bsum(x, 2 * j + 1));
        }
        const float dx = q8k_d(x);
        sum += get_f16(w) * dx * (float)isum;
        sum -= get_f16(w + 2) * dx * (float)msum;
    }
    return sum;
}

static float dot_q6_k(const uint8_t* w, const uint8_t* x, int64_t nb) {
    float sum = 0.f;
    for (int64_t b = 0; b < nb; ++b, w += 210, x += 292) {
        const int8_t* qx = (const int8_t*)(x + 4);
        const int8_t* sc = (const int8_t*)(w + 192);
        int isum = 0;
        for (int s = 0; s < 16; ++s) {
            int part = 0;
            for (int i = 0; i < 16; ++i) {
                const int e = 16 * s + i;
                const int h = e / 128, r = e % 128, g = r / 32, l = r % 32;
                const uint8_t lowbyte = w[64 * h + 32 * (g & 1) + l];
                const int low = (g < 2) ? (lowbyte & 0x0f) : (lowbyte >> 4);
                const int high = (w[128 + 32 * h + l] >> (2 * g)) & 3;
                part += ((low | (high << 4)) - 32) * qx[e];
            }
            isum += sc[s] * part;
        }
        sum += get_f16(w + 208) * q8k_d(x) * (float)isum;
    }
    return sum;
}

float or_vec_dot(int wtype, const void* w_row, const void* x_row, int64_t k) {
    const uint8_t* w = (const uint8_t*)w_row;
    const uint8_t* x = (const uint8_t*)x_row;
    switch (wtype) {
        case OR_Q8_0: return dot_q8_0(w, x, k / QK8);
        case OR_Q4_K: case OR_Q5_K: return dot_q45_k(wtype, w, x, k / QKK);
        case OR_Q6_K: return dot_q6_k(w, x, k / QKK);
        default: return NAN;
    }
}

/* ---- mul_mat (ggml CPU paths) ------------------------------------------- */

static int supported_weight(int t) { return t == OR_Q8_0 || t == OR_Q4_K || t == OR_Q5_K || t == OR_Q6_K; }

int or_mul_mat_native(int wtype, const void* w, size_t w_stride, const float* x, size_t x_stride,
                      float* y, int64_t n, int64_t m, int64_t k, int q8_rounding, int threads) {
    if (!supported_weight(wtype) || k % or_block_elems(wtype) || n <= 0 || m <= 0) return -1;
    const int xtype = wtype == OR_Q8_0 ? OR_Q8_0 : OR_Q8_K;
    const int64_t xrow = or_row_bytes(xtype, k);
    uint8_t* packed = (uint8_t*)malloc((size_t)(xrow * m));
    if (!packed) return -1;
    set_threads(threads);
    /* activation packing per compute (ggml from_float of vec_dot_type) */
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < m; ++r) {
        if (xtype == OR_Q8_0) or_quantize_q8_0(x + r * x_stride, packed + r * xrow, 1, k, q8_rounding);
        else or_quantize_q8_k(x + r * x_stride, packed + r * xrow, 1, k);
    }
    const int64_t tm = 16, tn = 16;
    const int64_t tiles_m = (m + tm - 1) / tm, tiles_n = (n + tn - 1) / tn;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t t = 0; t < tiles_m * tiles_n; ++t) {
        const int64_t m0 = (t / tiles_n) * tm, n0 = (t % tiles_n) * tn;
        for (int64_t r = m0; r < m0 + tm && r < m; ++r)
            for (int64_t c = n0; c < n0 + tn && c < n; ++c)
                y[r * n + c] = or_vec_dot(wtype, (const uint8_t*)w + c * w_stride, packed + r * xrow, k);
    }
    free(packed);
    return 0;
}

static float dot_f32(const float* a, const float* b, int64_t k) {
    float acc[16] = {0};
    int64_t i = 0;
    for (; i + 16 <= k; i += 16)
        for (int j = 0; j < 16; ++j) acc[j] += a[i + j] * b[i + j];
    float s = 0.f;
    for (int j = 0; j < 16; ++j) s += acc[j];
    for (; i < k; ++i) s += a[i] * b[i];
    return s;
}

int or_mul_mat_decode(int wtype, const void* w, size_t w_stride, const float* x, size_t x_stride,
                      float* y, int64_t n, int64_t m, int64_t k, int threads) {
    if (!supported_weight(wtype) || k % or_block_elems(wtype) || n <= 0 || m <= 0) return -1;
    float* wf = (float*)malloc((size_t)(n * k) * sizeof(float));
    if (!wf) return -1;
    set_threads(threads);
#pragma omp parallel for schedule(static)
    for (int64_t c = 0; c < n; ++c) or_dequantize(wtype, (const uint8_t*)w + c * w_stride, wf + c * k, 1, k);
    const int64_t tm = 16, tn = 16;
    const int64_t tiles_m = (m + tm - 1) / tm, tiles_n = (n + tn - 1) / tn;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t t = 0; t < tiles_m * tiles_n; ++t) {
        const int64_t m0 = (t / tiles_n) * tm, n0 = (t % tiles_n) * tn;
        for (int64_t r = m0; r < m0 + tm && r < m; ++r)
            for (int64_t c = n0; c < n0 + tn && c < n; ++c)
                y[r * n + c] = dot_f32(wf + c * k, x + r * x_stride, k);
    }
    free(wf);
    return 0;
}

void or_gemm_f64(const float* w, const float* x, double* y, int64_t n, int64_t m, int64_t k, int threads) {
    set_threads(threads);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < m; ++r) {
        for (int64_t c = 0; c < n; ++c) {
            double s = 0.0;
            for (int64_t i = 0; i < k; ++i) s += (double)w[c * k + i] * (double)x[r * k + i];
            y[r * n + c] = s;
        }
    }
}
