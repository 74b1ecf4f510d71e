// GGUF block formats on the device: byte layouts, unaligned-safe loads and
// per-format dequantization to fp16 for the MFMA operand loaders.
//
// Layouts (ggml-common.h block_* structs; sizes pinned by
// tools/validation/verify_q8_mmq_dots.py:41, tools/benchmark/
// cpu_kernel_capture_probe.cpp:62-93, src/models/sam3/weights.hpp:411-418):
//   Q8_0 : f16 d @0, i8 q[32] @2                                 34 B / 32
//   Q8_K : f32 d @0, i8 q[256] @4, i16 bsums[16] @260            292 B / 256
//   Q4_K : f16 d @0, f16 dmin @2, u8 sc[12] @4, u8 qs[128] @16   144 B / 256
//   Q5_K : Q4_K header, u8 qh[32] @16, u8 qs[128] @48            176 B / 256
//   Q6_K : u8 ql[128] @0, u8 qh[64] @128, i8 sc[16] @192, f16 d @208  210 B / 256
//   Q8_1 : f16 d @0, f16 s @2, i8 q[32] @4                       36 B / 32
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace samhip {

enum : int { T_F32 = 0, T_F16 = 1, T_Q8_0 = 8, T_Q8_1 = 9, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_Q8_K = 15,
              T_I32 = 26 };

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__host__ __device__ constexpr int block_elems(int t) {
    return (t == T_Q8_0 || t == T_Q8_1) ? 32 : (t == T_Q4_K || t == T_Q5_K || t == T_Q6_K || t == T_Q8_K) ? 256 : 1;
}
__host__ __device__ constexpr int block_bytes(int t) {
    return t == T_Q8_0 ? 34 : t == T_Q8_1 ? 36 : t == T_Q4_K ? 144 : t == T_Q5_K ? 176 : t == T_Q6_K ? 210
         : t == T_Q8_K ? 292 : t == T_F16 ? 2 : 4;
}

__device__ __forceinline__ float half_bits_to_float(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// ({hi, lo} >> 8*shift)[31:0]
__device__ __forceinline__ uint32_t funnel_bytes(uint32_t hi, uint32_t lo, uint32_t shift) {
    return __builtin_amdgcn_alignbyte(hi, lo, shift);
}

// 16 bytes at a 2-byte aligned address, read as dword-aligned loads.  Every
// dword touched holds at least one requested byte, so no load crosses into
// memory past the requested range's last dword.
__device__ __forceinline__ u32x4 load16_a2(const uint8_t* p) {
    // the aligned address is formed from p itself (not from an integer), so
    // the compiler keeps p's global address space: global, not flat, loads
    const uint32_t sh = uint32_t(reinterpret_cast<uintptr_t>(p) & 3);
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p - sh);
    const uint32_t w0 = q[0], w1 = q[1], w2 = q[2], w3 = q[3];
    const uint32_t w4 = sh ? q[4] : 0u;
    return u32x4{funnel_bytes(w1, w0, sh), funnel_bytes(w2, w1, sh), funnel_bytes(w3, w2, sh), funnel_bytes(w4, w3, sh)};
}

// 4 bytes at a 2-byte aligned address.
__device__ __forceinline__ uint32_t load4_a2(const uint8_t* p) {
    const uint32_t sh = uint32_t(reinterpret_cast<uintptr_t>(p) & 3);
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p - sh);
    const uint32_t w0 = q[0];
    const uint32_t w1 = sh ? q[1] : 0u;
    return funnel_bytes(w1, w0, sh);
}

// 2 bytes at a 2-byte aligned address.
__device__ __forceinline__ uint32_t load2_a2(const uint8_t* p) {
    const uint32_t sh = uint32_t(reinterpret_cast<uintptr_t>(p) & 3);
    const uint32_t w = *reinterpret_cast<const uint32_t*>(p - sh);
    return (sh & 2) ? (w >> 16) : (w & 0xffffu);
}

// one byte
__device__ __forceinline__ uint32_t load1(const uint8_t* p) { return *p; }

// 6-bit (scale, min) of sub-block j of a Q4_K/Q5_K super-block from its 12
// packed bytes held as three little-endian dwords.
__device__ __forceinline__ void k4_scale_min(int j, const uint32_t s[3], int& sc, int& mn) {
    auto byte = [&](int i) -> int { return int((s[i >> 2] >> (8 * (i & 3))) & 0xffu); };
    if (j < 4) {
        sc = byte(j) & 63;
        mn = byte(j + 4) & 63;
    } else {
        sc = (byte(j + 4) & 0x0f) | ((byte(j - 4) >> 6) << 4);
        mn = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
    }
}

// Four unsigned bytes of w, each times a and plus b in f32 (one rounding:
// a*u is exact for the small codes used here), rounded to fp16.
__device__ __forceinline__ void fma_u8x4_to_half(uint32_t w, float a, float b, _Float16* out) {
    out[0] = (_Float16)__builtin_fmaf(a, (float)((w >> 0) & 0xffu), b);
    out[1] = (_Float16)__builtin_fmaf(a, (float)((w >> 8) & 0xffu), b);
    out[2] = (_Float16)__builtin_fmaf(a, (float)((w >> 16) & 0xffu), b);
    out[3] = (_Float16)__builtin_fmaf(a, (float)((w >> 24) & 0xffu), b);
}

// Four signed bytes of w, each times the fp16 scale d, in fp16 arithmetic:
// RNE(d*q) in binary16 equals the binary16 rounding of the exact f32 product.
__device__ __forceinline__ void mul_i8x4_to_half(uint32_t w, _Float16 d, _Float16* out) {
    // byte ^ 0x80 = q + 128; 0x6400 | u is the half 1024 + u.
    const uint32_t u = w ^ 0x80808080u;
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x07010700u);
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x07030702u);
    const half2v bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const half2v dd = {d, d};
    const half2v qlo = __builtin_bit_cast(half2v, lo) + bias;
    const half2v qhi = __builtin_bit_cast(half2v, hi) + bias;
    const half2v vlo = qlo * dd;
    const half2v vhi = qhi * dd;
    out[0] = vlo[0];
    out[1] = vlo[1];
    out[2] = vhi[0];
    out[3] = vhi[1];
}

// ---------------------------------------------------------------------------
// Byte readers over one packed weight row (offsets in bytes from the row
// start; 2-byte reads at even offsets, 4- and 16-byte reads at even offsets).
// ---------------------------------------------------------------------------

// A row in device memory at a 2-byte aligned address.
struct GlobalRow {
    const uint8_t* p;
    __device__ __forceinline__ uint32_t u8(int o) const { return load1(p + o); }
    __device__ __forceinline__ uint32_t u16(int o) const { return load2_a2(p + o); }
    __device__ __forceinline__ uint32_t u32(int o) const { return load4_a2(p + o); }
    __device__ __forceinline__ u32x4 u128(int o) const { return load16_a2(p + o); }
};

// A row copied into LDS as whole dwords: the row's first byte is byte `sh`
// (0 or 2) of dw[0].
struct LdsRow {
    const uint32_t* dw;
    int sh;
    __device__ __forceinline__ uint32_t word(int i) const { return dw[i]; }
    __device__ __forceinline__ uint32_t u8(int o) const {
        const int b = o + sh;
        return (dw[b >> 2] >> (8 * (b & 3))) & 0xffu;
    }
    __device__ __forceinline__ uint32_t u16(int o) const {
        const int b = o + sh;
        return (dw[b >> 2] >> (8 * (b & 2))) & 0xffffu;
    }
    __device__ __forceinline__ uint32_t u32(int o) const {
        const int b = o + sh, i = b >> 2;
        return funnel_bytes(dw[i + 1], dw[i], uint32_t(b & 3));
    }
    // five dword reads and four byte funnels, no branch on the alignment
    __device__ __forceinline__ u32x4 u128(int o) const {
        const int b = o + sh, i = b >> 2;
        const uint32_t s = uint32_t(b & 3);
        const uint32_t w0 = dw[i], w1 = dw[i + 1], w2 = dw[i + 2], w3 = dw[i + 3], w4 = dw[i + 4];
        return u32x4{funnel_bytes(w1, w0, s), funnel_bytes(w2, w1, s), funnel_bytes(w3, w2, s), funnel_bytes(w4, w3, s)};
    }
};

// ---------------------------------------------------------------------------
// Weight operand loaders: one thread owns 16 consecutive K elements (half h of
// a 32-element K step) of one weight row.  load() issues the reads,
// dequant() turns them into 16 fp16 values equal to fp16(ggml to_float(W)).
// ---------------------------------------------------------------------------

template <int WT> struct WeightPiece;

template <> struct WeightPiece<T_Q8_0> {
    u32x4 q;
    uint32_t d;
    template <class R>
    __device__ __forceinline__ void load(const R& r, int step, int h) {
        const int blk = 34 * step;
        d = r.u16(blk);
        q = r.u128(blk + 2 + 16 * h);
    }
    __device__ __forceinline__ void load(const uint8_t* row, int step, int h) { load(GlobalRow{row}, step, h); }
    __device__ __forceinline__ void dequant(int /*step*/, int /*h*/, _Float16* out) const {
        const _Float16 dh = __builtin_bit_cast(_Float16, (uint16_t)d);
        mul_i8x4_to_half(q[0], dh, out + 0);
        mul_i8x4_to_half(q[1], dh, out + 4);
        mul_i8x4_to_half(q[2], dh, out + 8);
        mul_i8x4_to_half(q[3], dh, out + 12);
    }
};

template <> struct WeightPiece<T_Q4_K> {
    uint32_t hdr, sc[3];
    u32x4 qs;
    template <class R>
    __device__ __forceinline__ void load(const R& r, int step, int h) {
        const int blk = 144 * (step >> 3);
        const int j = step & 7;
        hdr = r.u32(blk);
        sc[0] = r.u32(blk + 4);
        sc[1] = r.u32(blk + 8);
        sc[2] = r.u32(blk + 12);
        qs = r.u128(blk + 16 + 32 * (j >> 1) + 16 * h);
    }
    __device__ __forceinline__ void load(const uint8_t* row, int step, int h) { load(GlobalRow{row}, step, h); }
    __device__ __forceinline__ void dequant(int step, int /*h*/, _Float16* out) const {
        const int j = step & 7;
        int s, m;
        k4_scale_min(j, sc, s, m);
        const float dj = half_bits_to_float(hdr & 0xffffu) * (float)s;
        const float mj = half_bits_to_float(hdr >> 16) * (float)m;
        const int shift = (j & 1) * 4;
        for (int i = 0; i < 4; ++i) fma_u8x4_to_half((qs[i] >> shift) & 0x0f0f0f0fu, dj, -mj, out + 4 * i);
    }
};

template <> struct WeightPiece<T_Q5_K> {
    uint32_t hdr, sc[3];
    u32x4 qs, qh;
    template <class R>
    __device__ __forceinline__ void load(const R& r, int step, int h) {
        const int blk = 176 * (step >> 3);
        const int j = step & 7;
        hdr = r.u32(blk);
        sc[0] = r.u32(blk + 4);
        sc[1] = r.u32(blk + 8);
        sc[2] = r.u32(blk + 12);
        qh = r.u128(blk + 16 + 16 * h);
        qs = r.u128(blk + 48 + 32 * (j >> 1) + 16 * h);
    }
    __device__ __forceinline__ void load(const uint8_t* row, int step, int h) { load(GlobalRow{row}, step, h); }
    __device__ __forceinline__ void dequant(int step, int /*h*/, _Float16* out) const {
        const int j = step & 7;
        int s, m;
        k4_scale_min(j, sc, s, m);
        const float dj = half_bits_to_float(hdr & 0xffffu) * (float)s;
        const float mj = half_bits_to_float(hdr >> 16) * (float)m;
        const int shift = (j & 1) * 4;
        for (int i = 0; i < 4; ++i) {
            const uint32_t v = ((qs[i] >> shift) & 0x0f0f0f0fu) | (((qh[i] >> j) & 0x01010101u) << 4);
            fma_u8x4_to_half(v, dj, -mj, out + 4 * i);
        }
    }
};

template <> struct WeightPiece<T_Q6_K> {
    u32x4 ql, qh;
    uint32_t sc, d;
    template <class R>
    __device__ __forceinline__ void load(const R& r, int step, int h) {
        const int blk = 210 * (step >> 3);
        const int j = step & 7, half = j >> 2, g = j & 3;
        ql = r.u128(blk + 64 * half + 32 * (g & 1) + 16 * h);
        qh = r.u128(blk + 128 + 32 * half + 16 * h);
        sc = r.u8(blk + 192 + 8 * half + 2 * g + h);
        d = r.u16(blk + 208);
    }
    __device__ __forceinline__ void load(const uint8_t* row, int step, int h) { load(GlobalRow{row}, step, h); }
    __device__ __forceinline__ void dequant(int step, int /*h*/, _Float16* out) const {
        const int g = (step & 7) & 3;
        const float t = half_bits_to_float(d) * (float)(int8_t)sc;   // exact in f32
        const int lshift = (g >> 1) * 4, hshift = 2 * g;
        for (int i = 0; i < 4; ++i) {
            const uint32_t u = ((ql[i] >> lshift) & 0x0f0f0f0fu) | (((qh[i] >> hshift) & 0x03030303u) << 4);
            fma_u8x4_to_half(u, t, -32.0f * t, out + 4 * i);   // RNE(t*(u-32))
        }
    }
};

}  // namespace samhip
