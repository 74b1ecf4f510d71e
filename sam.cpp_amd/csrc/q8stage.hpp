// Activation packing shared by the staging kernels and the fused skinny
// kernel: lane-level reductions on the DPP network, the power-of-two operand
// scale, and the conversion of 8 consecutive F32 activations per lane into
// the fp16 MFMA operand
//   Q8_0 mode : fp16(to_float(q8_0 block) * 2^-e)   (Q8_0 weights)
//   Q8_K mode : fp16(to_float(q8_K block) * 2^-e)   (K-quant weights)
//   F16 mode  : fp16(x * 2^-e)
// with Q8 blocks bit-exact with ggml's CPU from_float for the weight's
// vec_dot_type (src/runtime/ggml/backends/cpu.hpp:13-23).
#pragma once

#include "blocks.hpp"

namespace samhip {


__device__ __forceinline__ float wave_sum(float v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// ggml_gelu_erf on one F32 value: 0.5 x (1 + erf(x / sqrt 2)), in ggml's
// order of operations (erf rounded to F32, then 1 + erf).  erf(t) is
// sign(t) (1 - erfc(a)), a = min(|t|, 4), with
//   erfc(a) = r exp(-a^2) P(r - 1),  r = 1 / (1 + 0.55 a),
// the form of Abramowitz & Stegun 7.1.26 with a degree-7 P fitted for this
// kernel (least squares on [0, 4] with Lawson's reweighting towards the
// largest relative error).  Evaluated in F32 (simulated with a correctly
// rounded reciprocal and exponential; the hardware's are within 1 ulp) it is
// within 2.7e-7 of erf everywhere and within a few 1e-9 for a >= 2, where
// 1 + erf is small.
// Past a = 4, 1 - erfc(a) rounds to 1, as F32 erf does.  The library erff
// costs ~50 VALU instructions here (the wave runs both halves of its range
// split) and made fc2's erf-GELU staging VALU-bound: 45-52 us per
// M = 5184, K = 4736 staging, against 29-30 us without the GELU.  This form
// needs ~20 instructions.  After Q8_0 packing, ~1e-6 of the codes and ~1e-5
// of the block scales differ from a correctly rounded erff's, simulated
// over 2^24 N(0, 1) values.
__device__ __forceinline__ float gelu_erf(float v) {
#pragma clang fp contract(off)
    const float t = v * 0.70710678118654752440f;
    const float a = fminf(fabsf(t), 4.f);
    const float r = __builtin_amdgcn_rcpf(__builtin_fmaf(a, 0.55f, 1.f));
    const float u = r - 1.f;
    float p = -0.07083717733621597f;
    p = __builtin_fmaf(p, u, -0.11515318602323532f);
    p = __builtin_fmaf(p, u, 0.034340959042310715f);
    p = __builtin_fmaf(p, u, -0.004200853407382965f);
    p = __builtin_fmaf(p, u, -0.2428262084722519f);
    p = __builtin_fmaf(p, u, 0.202457457780838f);
    p = __builtin_fmaf(p, u, 1.051594614982605f);
    p = __builtin_fmaf(p, u, 1.f);
    const float g = __builtin_amdgcn_exp2f((a * a) * -1.4426950408889634f);   // exp(-a^2), a^2 <= 16
    const float erfc_a = (r * g) * p;
    const float erf_t = __builtin_copysignf(1.f - erfc_a, t);
    return 0.5f * v * (1.0f + erf_t);
}

__device__ __forceinline__ float wave_max(float v) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// max over aligned groups of `width` lanes
template <int width>
__device__ __forceinline__ float group_max(float v) {
    for (int off = width / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

template <int width>
__device__ __forceinline__ int group_sum(int v) {
    for (int off = width / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// 2^e as a float for |e| <= 126.
__device__ __forceinline__ float exp2i(int e) { return __builtin_bit_cast(float, uint32_t(127 + e) << 23); }

// Row exponent e with rowmax * 2^-e in [2^14, 2^15), clamped to [-110, 110]
// so that both 2^e and 2^-e are normal floats.
__device__ __forceinline__ int row_exponent(float rowmax) {
    if (!(rowmax > 0.f) || !__builtin_isfinite(rowmax)) return 0;
    const int biased = int((__builtin_bit_cast(uint32_t, rowmax) >> 23) & 0xffu);
    int e = (biased == 0 ? -126 : biased - 127) - 14;
    return e < -110 ? -110 : (e > 110 ? 110 : e);
}

__device__ __forceinline__ floatx4 load4f(const float* p) { return *reinterpret_cast<const floatx4*>(p); }
// An integral float to int32 by the hardware conversion, which gives 0 for
// NaN (and saturates out of range).  NaN -> code 0 is this library's
// contract for a NaN activation in every Q8 packing: it is what ggml's
// nearest_int (Q8_K) and its scalar Q8_0 reference rounding give on x86,
// but not what ggml's AVX2 Q8_0 packing gives (its saturating packs turn
// the conversion's 0x80000000 into -128), so for the x86 rounding mode it is
// a deliberate choice, not parity with that SIMD code.
__device__ __forceinline__ int cvt_i32_nan0(float r) {
    int q;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(q) : "v"(r));
    return q;
}

// read-once data (activation rows being staged): a streaming load
__device__ __forceinline__ floatx4 load4f_stream(const float* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(p));
}

// Cross-lane steps on the DPP network (no LDS round trip): quad_perm swaps
// for lane ^ 1 and lane ^ 2, row rotations by 4 and 8 within 16 lanes.
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_ROR4 = 0x124, DPP_ROR8 = 0x128;

template <int CTRL>
__device__ __forceinline__ int dpp(int v) { return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false); }
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float max4_lanes(float v) {
    v = fmaxf(v, dpp<DPP_XOR1>(v));
    return fmaxf(v, dpp<DPP_XOR2>(v));
}
__device__ __forceinline__ float max32_lanes(float v) {
    v = max4_lanes(v);
    v = fmaxf(v, dpp<DPP_ROR4>(v));
    v = fmaxf(v, dpp<DPP_ROR8>(v));
    return fmaxf(v, __shfl_xor(v, 16, 64));
}
__device__ __forceinline__ int min32_lanes(int v) {
    v = min(v, dpp<DPP_XOR1>(v));
    v = min(v, dpp<DPP_XOR2>(v));
    v = min(v, dpp<DPP_ROR4>(v));
    v = min(v, dpp<DPP_ROR8>(v));
    return min(v, __shfl_xor(v, 16, 64));
}
typedef float floatx8 __attribute__((ext_vector_type(8)));

// x / 127 correctly rounded for x >= 0 (a Q8_0 block maximum): the product
// with fl(1/127) and one FMA correction of its residual give the quotient's
// bits for every non-negative float (checked exhaustively against IEEE
// division), except +inf, whose residual is NaN; 5 VALU operations against
// ~10 for a general division.
__device__ __forceinline__ float div127(float x) {
#pragma clang fp contract(off)
    const float r = 1.0f / 127.0f;
    const float q = x * r;
    const float e = __builtin_fmaf(-q, 127.0f, x);
    const float q2 = __builtin_fmaf(e, r, q);
    return x < __builtin_inff() ? q2 : x;
}

// The Q8 block packing of 8 consecutive activations held by each lane;
// lanes 4g..4g+3 hold one Q8_0 block, lanes 32h..32h+31 one Q8_K block.
// Every lane of the wave must call these (cross-lane reductions); lanes past
// the row's end hold zeros.  quant8_scale gives the block's decoded scale d
// (the stored fp16 for Q8_0) and the multiplier that takes a value to its
// unrounded code; quant8_codes and quant8_icodes give the codes in
// [-127, 127] as floats or as ints.  X86 selects the Q8_0 rounding of
// ggml's x86-64 from_float (scale 127/amax, ties to even) over the reference
// quantize_row_q8_0_ref (scale 1/d, ties away from zero).
template <int MODE, bool X86>
__device__ __forceinline__ void quant8_scale(const floatx8& v, int lane, float& d, float& mul) {
#pragma clang fp contract(off)
    d = 0.f;
    mul = 0.f;
    if (MODE == T_Q8_0) {
        float amax = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
        amax = max4_lanes(amax);
        const float dd = div127(amax);
        if (X86) mul = amax != 0.f ? 127.f / amax : 0.f;
        else mul = dd != 0.f ? 1.f / dd : 0.f;
        d = half_bits_to_float(float_to_half_bits(dd));   // stored fp16 scale
    } else {
        // Q8_K: first element of largest magnitude in the 256-value block
        const int base = 8 * (lane & 31);
        float la = 0.f, ls = 0.f;
        int li = 1 << 20;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float t = fabsf(v[i]);
            if (t > la) { la = t; ls = v[i]; li = base + i; }
        }
        // its sign rides in the low bit of the index minimum (the value at
        // the first maximum is +-amax), so no lane-to-lane read is needed
        const float amax = max32_lanes(la);
        const int key = min32_lanes(la == amax ? 2 * li + int(__float_as_uint(ls) >> 31) : (1 << 20));
        const float smax = (key & 1) ? -amax : amax;
        if (amax != 0.f) {
            // ggml clamps the code to 127; with |v| <= amax = |smax| the
            // product is at most 127 (1 + 2^-23), which rounds to 127, so
            // the clamp never acts (a non-finite amax makes the product NaN)
            mul = -127.f / smax;
            d = 1.f / mul;
        }
    }
}

// The rounding of a scaled value to its code.
template <int MODE, bool X86>
__device__ __forceinline__ float quant8_round(float s) {
    return (MODE == T_Q8_0 && !X86) ? __builtin_roundf(s) : __builtin_rintf(s);
}

template <int MODE, bool X86>
__device__ __forceinline__ void quant8_codes(const floatx8& v, int lane, float& d, float (&q)[8]) {
#pragma clang fp contract(off)
    float mul;
    quant8_scale<MODE, X86>(v, lane, d, mul);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float r = quant8_round<MODE, X86>(v[i] * mul);
        q[i] = r == r ? r : 0.f;   // a NaN activation packs as code 0 (this library's contract, above)
    }
}

// The same codes as integers (the int8 kernels): the conversion itself
// takes a NaN to 0.
template <int MODE, bool X86>
__device__ __forceinline__ void quant8_icodes(const floatx8& v, int lane, float& d, int (&c)[8]) {
#pragma clang fp contract(off)
    float mul;
    quant8_scale<MODE, X86>(v, lane, d, mul);
#pragma unroll
    for (int i = 0; i < 8; ++i) c[i] = cvt_i32_nan0(quant8_round<MODE, X86>(v[i] * mul));
}

// The fp16 MFMA operand of the same 8 activations:
//   Q8 modes: fp16(q * (d * down));  F16 mode: fp16(x * down)
// with `down` = 2^-e.  d * down is d scaled by a power of two, so
// q * (d * down) is fl(d * q) * down whenever d * q is a normal float (a
// subnormal d * q is below 2^-126, and such a value times down is below
// fp16's range unless the row maximum is below ~2^-87, where this form
// keeps more bits).
template <int MODE, bool X86>
__device__ __forceinline__ half8 quant8(const floatx8& v, int lane, float down) {
#pragma clang fp contract(off)
    half8 o;
    if (MODE == T_F16) {
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = (_Float16)(v[i] * down);
        return o;
    }
    float d, q[8];
    quant8_codes<MODE, X86>(v, lane, d, q);
    const float dd = d * down;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (_Float16)(q[i] * dd);
    return o;
}

// Q8_0 block: amax over 8 lanes x 4 values; returns fp16 d bits and codes.
__device__ __forceinline__ void q8_0_codes(const floatx4& v, int x86, float& d_out, int q[4]) {
#pragma clang fp contract(off)
    float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    amax = group_max<8>(amax);
    const float d = amax / 127.f;
    float inv;
    if (x86) inv = amax != 0.f ? 127.f / amax : 0.f;
    else inv = d != 0.f ? 1.f / d : 0.f;
    d_out = d;
    for (int i = 0; i < 4; ++i) {
        const float r = x86 ? __builtin_rintf(v[i] * inv) : __builtin_roundf(v[i] * inv);
        q[i] = r == r ? int(r) : 0;   // |r| <= 127 when finite; NaN -> 0
    }
}

// Q8_K block over the whole wave (64 lanes x 4 values = 256): ggml keeps the
// first element of largest magnitude as the signed maximum.
__device__ __forceinline__ void q8_k_codes(const floatx4& v, int lane, float& d_out, int q[4]) {
#pragma clang fp contract(off)
    float amax = 0.f, smax = 0.f;
    int idx = 1 << 30;
    for (int i = 0; i < 4; ++i) {
        const float a = fabsf(v[i]);
        if (a > amax) { amax = a; smax = v[i]; idx = 4 * lane + i; }
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float oa = __shfl_xor(amax, off, 64);
        const float os = __shfl_xor(smax, off, 64);
        const int oi = __shfl_xor(idx, off, 64);
        if (oa > amax || (oa == amax && oi < idx)) { amax = oa; smax = os; idx = oi; }
    }
    if (amax == 0.f) {
        d_out = 0.f;
        for (int i = 0; i < 4; ++i) q[i] = 0;
        return;
    }
    const float iscale = -127.f / smax;
    for (int i = 0; i < 4; ++i) {
        const float r = __builtin_rintf(iscale * v[i]);
        q[i] = r == r ? (r < 127.f ? int(r) : 127) : 0;   // NaN -> 0 (ggml nearest_int)
    }
    d_out = 1.f / iscale;
}

}  // namespace samhip
