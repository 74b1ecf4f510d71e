// SAM 3 vision-encoder kernels for gfx950: the non-linear parts of the ViT
// prefix and block (src/models/sam3/vision.hpp:152-272) around the quantized
// linears.
//   layer_norm_kernel : ggml_norm * w + b over one 1024-float row per wave,
//                       optionally adding the tiled position embedding first
//                       and writing rows in window order (ggml_win_part)
//   pack_qkv_kernel   : q/k/v columns -> per-head fp16 operands with the
//                       complex RoPE on q and k (the encoder block has the
//                       qkv product's epilogue write them instead)
//   attention_kernel  : softmax(Q K^T) V per window and head on
//                       v_mfma_f32_32x32x16_f16 with an online softmax in F32
//   patch_*_kernel    : the 14x14 patch convolution as a split-fp16 GEMM
// Arithmetic follows the reference graph's order (products rounded before
// adds, no contraction).  Built with MFMA results in VGPRs (Makefile): the
// softmax reads every score, so accumulation registers would cost a copy
// per value.
#include <algorithm>

#include "internal.hpp"

#pragma clang fp contract(off)

namespace samhip {

namespace {

typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float wave_sum(float v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ floatx4 ld4(const float* p) { return *reinterpret_cast<const floatx4*>(p); }

// ---------------------------------------------------------------------------
// Layer norm: one wave per row of E = 256 * CH floats.
// ---------------------------------------------------------------------------
template <int CH>
__global__ __launch_bounds__(256) void layer_norm_kernel(const float* __restrict__ x, const float* __restrict__ add,
                                                         int add_grid, int gw, int ws, const float* __restrict__ w,
                                                         const float* __restrict__ b, float eps, float* __restrict__ y,
                                                         int rows) {
    constexpr int E = 256 * CH;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const int lane = threadIdx.x & 63;
    const int gy = r / gw, gx = r - gy * gw;
    const float* xr = x + int64_t(r) * E;
    const float* ar = add ? add + int64_t((gy % add_grid) * add_grid + gx % add_grid) * E : nullptr;
    floatx4 v[CH];
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        v[c] = ld4(xr + 256 * c + 4 * lane);
        if (ar) {
            const floatx4 a = ld4(ar + 256 * c + 4 * lane);
#pragma unroll
            for (int i = 0; i < 4; ++i) v[c][i] = v[c][i] + a[i];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) s += v[c][i];
    }
    const float mean = wave_sum(s) / float(E);
    float s2 = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float d = v[c][i] - mean;
            v[c][i] = d;
            s2 += d * d;
        }
    const float variance = wave_sum(s2) / float(E);
    const float scale = 1.0f / sqrtf(variance + eps);
    int64_t dst = r;
    if (ws > 0) {
        const int win = (gy / ws) * (gw / ws) + gx / ws;
        dst = int64_t(win) * ws * ws + (gy % ws) * ws + gx % ws;
    }
    float* yr = y + dst * E;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int k = 256 * c + 4 * lane;
        floatx4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float t = v[c][i] * scale;
            if (w) t = t * w[k + i];
            if (b) t = t + b[k + i];
            o[i] = t;
        }
        *reinterpret_cast<floatx4*>(yr + k) = o;
    }
}

// ---------------------------------------------------------------------------
// q/k/v packing with RoPE.  Block: 64 tokens of one (batch, head); thread t
// owns token t/4 and the 16 head dims 16*(t%4)..
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pack_qkv_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                       const float* __restrict__ v, int64_t ld,
                                                       const float* __restrict__ freqs, float q_scale,
                                                       AttnOperands o_, int H, int N, int Np) {
    const int n0 = blockIdx.x * 64, h = blockIdx.y, b = blockIdx.z;
    const int t = threadIdx.x, tok = t >> 2, d0 = 16 * (t & 3);
    const int n = n0 + tok;
    const bool valid = n < N;
    const int64_t src = (int64_t(b) * N + n) * ld + h * 64 + d0;
    const int64_t dst = ((int64_t(b) * H + h) * Np + n) * 64 + d0;
#pragma unroll
    for (int which = 0; which < 3; ++which) {
        float xs[16];
        if (valid) {
            const float* p = (which == 0 ? q : which == 1 ? k : v) + src;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const floatx4 f = ld4(p + 4 * j);
                xs[4 * j] = f[0], xs[4 * j + 1] = f[1], xs[4 * j + 2] = f[2], xs[4 * j + 3] = f[3];
            }
            if (freqs && which < 2) {
                // pair i of the head: (x[2i], x[2i+1]) * (cos_i + j sin_i)
                const float* f = freqs + (int64_t(n) * 32 + d0 / 2) * 2;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float re = xs[2 * i], im = xs[2 * i + 1], c = f[2 * i], s = f[2 * i + 1];
                    const float a = re * c, bb = im * s, cc = re * s, dd = im * c;
                    xs[2 * i] = a - bb;
                    xs[2 * i + 1] = cc + dd;
                }
            }
            if (which == 0)
#pragma unroll
                for (int j = 0; j < 16; ++j) xs[j] = xs[j] * q_scale;
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) xs[j] = 0.f;
        }
        half8 h0, h1;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            h0[j] = (_Float16)xs[j];
            h1[j] = (_Float16)xs[8 + j];
        }
        half8* o = reinterpret_cast<half8*>((which == 0 ? o_.q : which == 1 ? o_.k : o_.v) + dst);
        o[0] = h0;
        o[1] = h1;
        _Float16* lo = which == 0 ? o_.ql : which == 1 ? o_.kl : o_.vl;
        if (lo) {   // remainders for the split products
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                h0[j] = (_Float16)(xs[j] - (float)h0[j]);
                h1[j] = (_Float16)(xs[8 + j] - (float)h1[j]);
            }
            half8* ol = reinterpret_cast<half8*>(lo + dst);
            ol[0] = h0;
            ol[1] = h1;
        }
    }
}

// Zero rows [N, Np) of packed operands [B*H][Np][64] (the padding of the
// last key tile when the qkv product wrote the packed rows itself).
__global__ __launch_bounds__(256) void zero_pad_kernel(AttnOperands o, int N, int Np) {
    const int64_t bh = blockIdx.y;
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;   // 8-half chunk of the pad rows
    if (i >= int64_t(Np - N) * 8) return;
    const int64_t off = (bh * Np + N) * 64 + 8 * i;
    const half8 z{0, 0, 0, 0, 0, 0, 0, 0};
    *reinterpret_cast<half8*>(o.q + off) = z;
    *reinterpret_cast<half8*>(o.k + off) = z;
    *reinterpret_cast<half8*>(o.v + off) = z;
    if (o.ql) *reinterpret_cast<half8*>(o.ql + off) = z;
    if (o.kl) *reinterpret_cast<half8*>(o.kl + off) = z;
    if (o.vl) *reinterpret_cast<half8*>(o.vl + off) = z;
}

// ---------------------------------------------------------------------------
// Attention.  Workgroup: 32 queries per wave, 4 waves, one (batch, head);
// 64-key tiles of K and V, both [key][d], double-buffered in LDS; the
// V^T fragments are read transposed (ds_read_b64_tr_b16).
// Each wave computes S^T = K Q^T (lane: query l%32, 16 keys per 32-key
// tile), so the softmax statistics of a query sit in one lane pair (l,
// l^32), and O^T = V^T P^T with P^T used as the B operand straight from the
// S^T accumulator registers (the K index of both operands is the same
// permutation of the tile's keys).
// PRECISE: every operand is split, v = hi + lo (lo = fp16(v - hi)), and each
// product sums hi*hi + lo*hi + hi*lo, with the weights P split the same way
// in registers: the scores and the output carry ~22 bits, as the reference
// computes attention in F32 (GGML_PREC_F32 on every FLASH_ATTN_EXT node,
// src/runtime/ggml/graph.hpp:64), at three times the MFMA work.
// ---------------------------------------------------------------------------
[[maybe_unused]] constexpr int RSRC_WORD3 = 0x00020000;   // raw buffer, 32-bit data format

// s_waitcnt vmcnt(0), expcnt/lgkmcnt left at their maximum (gfx9 encoding)
[[maybe_unused]] __device__ __forceinline__ void wait_vmcnt0() { __builtin_amdgcn_s_waitcnt(0x70 | 0xF00); }
// s_waitcnt vmcnt(N), expcnt/lgkmcnt left at their maximum (gfx9 encoding)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | 0xF00);
}

typedef short short4_t __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16: within each group of 16 lanes, lane i receives
// element (i % 4) of the 8-byte rows that lanes 4j + i/4 address, j = 0..3
// (lane layout measured on gfx950).  With lane r of a group addressing
// V[key0 + r/4][d0 + 4 (r % 4)] of a key-major tile, lane i holds
// V[key0 + j][d0 + i], j = 0..3: four consecutive keys of one column.
[[maybe_unused]] __device__ __forceinline__ half4 ds_read_tr(const uint8_t* p) {
    const short4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4_t*)(p));
    return __builtin_bit_cast(half4, v);
}
constexpr float LOG2E = 1.44269504088896340736f;

// slot permutation of a V tile row (the attention kernel's LDS layout)
__device__ __forceinline__ int v_swizzle(int r) { return 2 * (r & 3) + ((r >> 2) & 1); }

// LEVEL 0: fp16 operands; 1: split scores; 2: split scores and output.
template <int QW, int LEVEL>   // waves per workgroup (32 queries each), precision level
__global__ __launch_bounds__(64 * QW) void attention_kernel(AttnOperands op, float* __restrict__ out, int64_t ldo,
                                                            int H, int N, int Np, int S, float* __restrict__ part_o,
                                                            float* __restrict__ part_ml) {
#if defined(__HIP_DEVICE_COMPILE__)   // LDS-DMA builtins exist only in the device pass
    constexpr bool PRECISE = LEVEL > 0;         // split scores
    constexpr bool PRECISE_PV = LEVEL > 1;      // split weights and values too
    constexpr int P = PRECISE ? 2 : 1;          // parts of Q and K: hi (and lo)
    constexpr int PV = PRECISE_PV ? 2 : 1;      // parts of V
    static_assert(QW == 4, "the tile loads assume 4 waves");
    constexpr int TB = 64 * 128;   // bytes of one 64-key tile of one part
    // K tiles are double-buffered; with split V (LEVEL 2) the V tiles have a
    // single buffer, reloaded once every wave is past the tile's products, so
    // a workgroup takes 48 KB of LDS and three fit on a CU (two with 64 KB)
    constexpr int VB = PRECISE_PV ? 1 : 2;
    __shared__ __attribute__((aligned(1024))) uint8_t ktile[P][2][TB];
    __shared__ __attribute__((aligned(1024))) uint8_t vtile[PV][VB][TB];
    // grid z = window x key split: split sp takes key tiles [kb0, kb1)
    const int h = blockIdx.y, b = blockIdx.z / S, sp = blockIdx.z - b * S;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 31, hh = lane >> 5;
    const int64_t bh = int64_t(b) * H + h;
    const _Float16* Qg[2] = {op.q + bh * Np * 64, PRECISE ? op.ql + bh * Np * 64 : nullptr};
    const int q0 = blockIdx.x * (32 * QW) + wave * 32;
    const int qrow = min(q0 + li, Np - 1);

    half8 qf[P][4];
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
        for (int s = 0; s < 4; ++s)
            qf[p][s] = *reinterpret_cast<const half8*>(Qg[p] + int64_t(qrow) * 64 + 16 * s + 8 * hh);

    // K and V tiles go straight from HBM into LDS (buffer_load ... lds): a
    // tile's 512 16-byte chunks, two per lane; the chunk landing in slot c of
    // row r is the row's chunk c ^ swz(r).  K: swz(r) = r & 7, so that the
    // 16-byte fragment reads of 8 rows at one column hit 8 different slots.
    // V: its transposed reads take 32 bytes (a slot pair) from each of 4
    // consecutive rows per 16 lanes, so swz(r) = 2 (r & 3) + ((r >> 2) & 1)
    // puts those 4 rows' pairs in 4 different pairs of slots (with r & 7 two
    // rows shared a pair: a 2-way bank conflict on every V read).
    const uint32_t bytes = uint32_t(Np) * 128;
    __amdgpu_buffer_rsrc_t kr[P], vr[PV];
#pragma unroll
    for (int p = 0; p < P; ++p)
        kr[p] = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>((p ? op.kl : op.k) + bh * Np * 64), 0, bytes,
                                                  RSRC_WORD3);
#pragma unroll
    for (int p = 0; p < PV; ++p)
        vr[p] = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>((p ? op.vl : op.v) + bh * Np * 64), 0, bytes,
                                                  RSRC_WORD3);
    uint32_t goff[2], gofv[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int id = wave * 128 + i * 64 + lane, r = id >> 3, c = id & 7;
        goff[i] = uint32_t(r * 128 + ((c ^ (r & 7)) << 4));
        gofv[i] = uint32_t(r * 128 + ((c ^ v_swizzle(r)) << 4));
    }
    auto issue_k = [&](int kb, int buf) {   // 2 P loads per lane
        const int koff = kb * TB;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int p = 0; p < P; ++p)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    kr[p], (__attribute__((address_space(3))) void*)(ktile[p][buf] + (wave * 128 + i * 64) * 16), 16,
                    goff[i], koff, 0, 0);
    };
    auto issue_v = [&](int kb, int buf) {
        const int koff = kb * TB;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int p = 0; p < PV; ++p)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    vr[p], (__attribute__((address_space(3))) void*)(vtile[p][buf] + (wave * 128 + i * 64) * 16), 16,
                    gofv[i], koff, 0, 0);
    };

    floatx16 o0, o1;
#pragma unroll
    for (int r = 0; r < 16; ++r) o0[r] = o1[r] = 0.f;
    float mrun = -__builtin_inff(), lsum = 0.f;
    float one = 1.0f;
    asm("" : "+s"(one));   // 1.0 the compiler cannot see (the P split below)
    const int nkb = Np / 64, per_split = (nkb + S - 1) / S;
    const int kb0 = sp * per_split, kb1 = min(nkb, kb0 + per_split);

    issue_k(kb0, 0);
    issue_v(kb0, 0);
    wait_vmcnt0();
    __syncthreads();
    for (int kb = kb0; kb < kb1; ++kb) {
        const int buf = (kb - kb0) & 1, vbuf = VB == 2 ? buf : 0;
        if (kb + 1 < kb1) {   // that buffer's reads ended at the last barrier
            issue_k(kb + 1, buf ^ 1);
            if (VB == 2) issue_v(kb + 1, buf ^ 1);
        }
        floatx16 s0, s1;
#pragma unroll
        for (int r = 0; r < 16; ++r) s0[r] = s1[r] = 0.f;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            // rows li and 32 + li, chunk 2s + hh (same swizzle: (32 + li) & 7 == li & 7)
            const int kofs0 = li * 128 + (((2 * s + hh) ^ (li & 7)) << 4);
            const uint8_t* kt = ktile[0][buf];
            const half8 a0 = *reinterpret_cast<const half8*>(kt + kofs0);
            const half8 a1 = *reinterpret_cast<const half8*>(kt + kofs0 + 32 * 128);
            s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, qf[0][s], s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, qf[0][s], s1, 0, 0, 0);
            if (PRECISE) {
                const uint8_t* kl = ktile[P - 1][buf];
                const half8 l0 = *reinterpret_cast<const half8*>(kl + kofs0);
                const half8 l1 = *reinterpret_cast<const half8*>(kl + kofs0 + 32 * 128);
                s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(l0, qf[0][s], s0, 0, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(l1, qf[0][s], s1, 0, 0, 0);
                s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, qf[P - 1][s], s0, 0, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, qf[P - 1][s], s1, 0, 0, 0);
            }
        }
        // keys past N (only in the last tile)
        const int kbase = kb * 64;
        if (kbase + 64 > N) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = kbase + 8 * (r >> 2) + 4 * hh + (r & 3);
                if (key >= N) s0[r] = -__builtin_inff();
                if (key + 32 >= N) s1[r] = -__builtin_inff();
            }
        }
        // the tile's largest score per query: IEEE maximum (v_maximum3_f32,
        // a NaN score gives a NaN row either way), where fmaxf would first
        // quiet every MFMA result with a separate v_max
        float mx = -__builtin_inff();
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = __builtin_elementwise_maximum(mx, __builtin_elementwise_maximum(s0[r], s1[r]));
        mx = __builtin_elementwise_maximum(mx, __shfl_xor(mx, 32, 64));
        // Lazy rescaling: the exponent base mrun only moves when a score
        // exceeds it by more than 8 / log2(e), so the weights stay below 2^8
        // (fp16 keeps its full relative precision there) and most tiles skip
        // the rescale of O and of the running sum.
        if (__any(mx > mrun + 8.0f / LOG2E)) {
            const float mnew = fmaxf(mrun, mx);
            const float alpha = __builtin_amdgcn_exp2f((mrun - mnew) * LOG2E);
            mrun = mnew;
            lsum = lsum * alpha;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                o0[r] = o0[r] * alpha;
                o1[r] = o1[r] * alpha;
            }
        }
        const float mb = mrun * LOG2E;
        float ps = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            s0[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[r], LOG2E, -mb));
            s1[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[r], LOG2E, -mb));
            ps += s0[r] + s1[r];
        }
        lsum = lsum + ps;
        // P in fp16: hi = fp16(p) two at a time (v_cvt_pk_f16_f32) and, at
        // LEVEL 2, lo = fp16(p - hi) (exact difference, one rounding) by
        // v_fma_mixlo/mixhi_f16 reading hi's halves: fma(p, one, -hi) with
        // `one` opaque to the compiler, which would otherwise fold the fma
        // into a subtraction and convert hi back to F32 separately
        half8 pf[PV][4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
                const float2_t p{t < 2 ? s0[8 * t + j] : s1[8 * (t - 2) + j],
                                 t < 2 ? s0[8 * t + j + 1] : s1[8 * (t - 2) + j + 1]};
                const half2_t hi = __builtin_convertvector(p, half2_t);
                pf[0][t][j] = hi[0];
                pf[0][t][j + 1] = hi[1];
                if (PRECISE_PV) {
                    const float2_t hf = __builtin_convertvector(hi, float2_t);
                    pf[PV - 1][t][j] = (_Float16)__builtin_fmaf(p[0], one, -hf[0]);
                    pf[PV - 1][t][j + 1] = (_Float16)__builtin_fmaf(p[1], one, -hf[1]);
                }
            }
        }
        // V^T fragments of part p for 16-key step u (lane: dim l%32 of each
        // 32-dim half, keys kofs + 0..3 and kofs + 8..11, the P^T order),
        // read transposed out of the key-major tile
        auto vfrag = [&](int p, int u, half8& a0, half8& a1) {
            const int row = 32 * (u >> 1) + 16 * (u & 1) + 4 * hh + ((lane & 15) >> 2);
            const int cg = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1), sw = v_swizzle(row);   // row + 8 alike
            const uint8_t* at = vtile[p][vbuf] + row * 128 + 8 * (lane & 1);
            const half4 a_lo0 = ds_read_tr(at + ((cg ^ sw) << 4));
            const half4 a_hi0 = ds_read_tr(at + 8 * 128 + ((cg ^ sw) << 4));
            const half4 a_lo1 = ds_read_tr(at + (((cg + 4) ^ sw) << 4));
            const half4 a_hi1 = ds_read_tr(at + 8 * 128 + (((cg + 4) ^ sw) << 4));
            a0 = __builtin_shufflevector(a_lo0, a_hi0, 0, 1, 2, 3, 4, 5, 6, 7);
            a1 = __builtin_shufflevector(a_lo1, a_hi1, 0, 1, 2, 3, 4, 5, 6, 7);
        };
        if (VB == 1 && kb > kb0) {
            // V(kb), requested after the last barrier and before K(kb + 1):
            // this lane's part has landed once at most K(kb + 1)'s 2 P loads
            // are outstanding, every lane's after the barrier
            if (kb + 1 < kb1) wait_vmcnt<2 * P>();
            else wait_vmcnt0();
            __syncthreads();
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            half8 a0, a1;
            vfrag(0, u, a0, a1);
            o0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, pf[0][u], o0, 0, 0, 0);
            o1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, pf[0][u], o1, 0, 0, 0);
            if (PRECISE_PV) {
                o0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, pf[PV - 1][u], o0, 0, 0, 0);
                o1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, pf[PV - 1][u], o1, 0, 0, 0);
                half8 l0, l1;
                vfrag(PV - 1, u, l0, l1);
                o0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(l0, pf[0][u], o0, 0, 0, 0);
                o1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(l1, pf[0][u], o1, 0, 0, 0);
            }
        }
        if (kb + 1 < kb1) {
            wait_vmcnt0();   // this wave's loads of the next tile landed
            __syncthreads();
            if (VB == 1) issue_v(kb + 1, 0);   // every wave is past V(kb)
        }
    }
    const float ltot = lsum + __shfl_xor(lsum, 32, 64);
    const float inv = 1.0f / ltot;
    const int qo = q0 + li;
    if (qo < N) {
        // one split: the output; several: this split's normalized partial,
        // its exponent base and weight sum (attention_merge_kernel)
        float* orow = S == 1 ? out + (int64_t(b) * N + qo) * ldo + h * 64
                             : part_o + ((int64_t(sp) * gridDim.z / S + b) * N + qo) * (int64_t(H) * 64) + h * 64;
        if (S > 1 && hh == 0) {
            float* ml = part_ml + (((int64_t(sp) * gridDim.z / S + b) * N + qo) * H + h) * 2;
            ml[0] = mrun;
            ml[1] = ltot;
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d0 = 8 * g + 4 * hh;
            *reinterpret_cast<floatx4*>(orow + d0) =
                floatx4{o0[4 * g] * inv, o0[4 * g + 1] * inv, o0[4 * g + 2] * inv, o0[4 * g + 3] * inv};
            *reinterpret_cast<floatx4*>(orow + 32 + d0) =
                floatx4{o1[4 * g] * inv, o1[4 * g + 1] * inv, o1[4 * g + 2] * inv, o1[4 * g + 3] * inv};
        }
    }
#endif
}

// ---------------------------------------------------------------------------
// Patch convolution operands (split fp16): v = hi + lo with hi = fp16(v),
// lo = fp16(v - hi).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void patch_columns_kernel(const float* __restrict__ image, int img, int patch,
                                                            _Float16* __restrict__ a, float* __restrict__ row_scale,
                                                            int kp) {
    const int grid = img / patch, pp = patch * patch, kk = 3 * pp;
    const int64_t tokens = int64_t(grid) * grid;
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= tokens * kp) return;
    const int64_t t = i / kp;
    const int c = int(i - t * kp);
    float v = 0.f;
    if (c < kk) {
        const int ci = c / pp, rem = c - ci * pp, ky = rem / patch, kx = rem - ky * patch;
        const int oy = int(t / grid), ox = int(t - int64_t(oy) * grid);
        v = image[(int64_t(ci) * img + oy * patch + ky) * img + ox * patch + kx];
    }
    const _Float16 hi = (_Float16)v;
    const _Float16 lo = (_Float16)(v - (float)hi);
    _Float16* row = a + t * 3 * kp;
    row[c] = hi;
    row[kp + c] = hi;
    row[2 * kp + c] = lo;
    if (c == 0) row_scale[t] = 1.0f;
}

__global__ __launch_bounds__(256) void patch_kernel_kernel(const float* __restrict__ kernel, int E, int patch,
                                                           _Float16* __restrict__ w, int kp) {
    const int kk = 3 * patch * patch;
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= int64_t(E) * kp) return;
    const int64_t e = i / kp;
    const int c = int(i - e * kp);
    const float v = c < kk ? kernel[e * kk + c] : 0.f;
    const _Float16 hi = (_Float16)v;
    const _Float16 lo = (_Float16)(v - (float)hi);
    _Float16* row = w + e * 3 * kp;
    row[c] = hi;
    row[kp + c] = lo;
    row[2 * kp + c] = hi;
}

}  // namespace

void launch_layer_norm(const float* x, const float* add, int add_grid, int gw, int gh, int ws, const float* w,
                       const float* b, float eps, float* y, int rows, int E, hipStream_t stream) {
    (void)gh;
    const dim3 grid((rows + 3) / 4), block(256);
    switch (E / 256) {
        case 1: hipLaunchKernelGGL(layer_norm_kernel<1>, grid, block, 0, stream, x, add, add_grid, gw, ws, w, b, eps, y, rows); break;
        case 2: hipLaunchKernelGGL(layer_norm_kernel<2>, grid, block, 0, stream, x, add, add_grid, gw, ws, w, b, eps, y, rows); break;
        case 3: hipLaunchKernelGGL(layer_norm_kernel<3>, grid, block, 0, stream, x, add, add_grid, gw, ws, w, b, eps, y, rows); break;
        case 4: hipLaunchKernelGGL(layer_norm_kernel<4>, grid, block, 0, stream, x, add, add_grid, gw, ws, w, b, eps, y, rows); break;
        case 5: hipLaunchKernelGGL(layer_norm_kernel<5>, grid, block, 0, stream, x, add, add_grid, gw, ws, w, b, eps, y, rows); break;
        case 6: hipLaunchKernelGGL(layer_norm_kernel<6>, grid, block, 0, stream, x, add, add_grid, gw, ws, w, b, eps, y, rows); break;
        case 8: hipLaunchKernelGGL(layer_norm_kernel<8>, grid, block, 0, stream, x, add, add_grid, gw, ws, w, b, eps, y, rows); break;
        default: break;   // callers check layer_norm_supported
    }
}

void launch_pack_qkv(const float* q, const float* k, const float* v, int64_t ld, const float* freqs, float q_scale,
                     const AttnOperands& o, int B, int H, int N, hipStream_t stream) {
    const int np = (N + 63) / 64 * 64;
    hipLaunchKernelGGL(pack_qkv_kernel, dim3(unsigned(np / 64), unsigned(H), unsigned(B)), dim3(256), 0, stream, q, k,
                       v, ld, freqs, q_scale, o, H, N, np);
}

void launch_zero_pad(const AttnOperands& o, int B, int H, int N, hipStream_t stream) {
    const int np = (N + 63) / 64 * 64;
    if (np == N) return;
    const int64_t chunks = int64_t(np - N) * 8;
    hipLaunchKernelGGL(zero_pad_kernel, dim3(unsigned((chunks + 255) / 256), unsigned(B * H)), dim3(256), 0, stream, o,
                       N, np);
}

// O = sum_s w_s O_s / sum_s w_s with w_s = l_s exp(m_s - max m): the key
// splits of one (window, query, head) combined in split order.  One thread
// per 4 output values.
__global__ __launch_bounds__(256) void attention_merge_kernel(const float* __restrict__ part_o,
                                                              const float* __restrict__ part_ml,
                                                              float* __restrict__ out, int64_t ldo, int rows, int H,
                                                              int S) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;   // (row, head, 4-value group)
    if (i >= int64_t(rows) * H * 16) return;
    const int64_t row = i / (H * 16);
    const int hg = int(i - row * H * 16), h = hg >> 4, g = hg & 15;
    const int64_t plane_o = int64_t(rows) * H * 64, plane_ml = int64_t(rows) * H * 2;
    float mmax = -__builtin_inff();
    for (int sp = 0; sp < S; ++sp) mmax = fmaxf(mmax, part_ml[sp * plane_ml + (row * H + h) * 2]);
    floatx4 acc{0.f, 0.f, 0.f, 0.f};
    float wsum = 0.f;
    for (int sp = 0; sp < S; ++sp) {
        const float* ml = part_ml + sp * plane_ml + (row * H + h) * 2;
        const float w = ml[1] * __builtin_amdgcn_exp2f((ml[0] - mmax) * LOG2E);
        const floatx4 o = ld4(part_o + sp * plane_o + row * H * 64 + h * 64 + 4 * g);
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[q] = acc[q] + w * o[q];
        wsum = wsum + w;
    }
    const float inv = 1.0f / wsum;
    *reinterpret_cast<floatx4*>(out + row * ldo + h * 64 + 4 * g) =
        floatx4{acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
}

// Key splits for a grid of `wgs` workgroups: the S in 1..4 with the lowest
// cost below, each split keeping at least 8 key tiles.
int attention_splits(int B, int H, int N, bool precise, int cus, int force) {
    const int np = (N + 63) / 64 * 64, nkb = np / 64;
    // the grid's z dimension holds B * S and is limited to 65535
    const int cap = std::max(1, std::min(4, 65535 / std::max(B, 1)));
    if (force > 0) {
        // every split keeps at least one key tile
        int S = std::max(1, std::min(std::min(force, cap), nkb));
        while (S > 1 && (S - 1) * ((nkb + S - 1) / S) >= nkb) --S;
        return S;
    }
    // fp16 operands: cost = rounds of resident workgroups (four per CU) per
    // unit of work.  F32-accurate: three fit a CU and share its matrix cores,
    // so the cost is the most workgroups any CU runs per unit of work (SAM 3
    // global block, 656 workgroups of 81 key tiles: 3 splits 317 us, 4 324,
    // 2 335, whole 326 us)
    const int64_t wgs = int64_t((np + 127) / 128) * H * B, slots = precise ? int64_t(cus) : int64_t(4) * cus;
    int best = 1;
    double best_cost = double((wgs + slots - 1) / slots);
    for (int s = 2; s <= cap && nkb >= 8 * s; ++s) {
        const double cost = double((wgs * s + slots - 1) / slots) / s;
        if (cost < best_cost * 0.95) {
            best = s;
            best_cost = cost;
        }
    }
    return best;
}

size_t attention_scratch_bytes(int B, int H, int N, int S) {
    return S <= 1 ? 0 : size_t(S) * B * N * H * (64 + 2) * 4;
}

bool launch_attention(const AttnOperands& o, float* out, int64_t ldo, int B, int H, int N, int S, float* scratch,
                      size_t scratch_bytes, hipStream_t stream) {
    const int np = (N + 63) / 64 * 64;
    const bool precise = o.ql && o.kl && o.vl;
    if (S < 1 || int64_t(B) * S > 65535) return false;
    if (S > 1 && (!scratch || scratch_bytes < attention_scratch_bytes(B, H, N, S))) return false;
    float* part_o = S > 1 ? scratch : nullptr;
    float* part_ml = S > 1 ? scratch + size_t(S) * B * N * H * 64 : nullptr;
    // 128-query workgroups: measured on the SAM 3 shapes against 64, 96 and
    // 192 (windowed 34 / 42 / 35 / 41 us, global 206 / 294 / 213 / 267 us;
    // 96 and 192 tile 576 and 5184 queries exactly and still lose; 192 again
    // at 151 VGPRs, three waves per SIMD: windowed 54.7 against 52.2 us,
    // global 389 against 333 us)
    const dim3 grid(unsigned((np + 127) / 128), unsigned(H), unsigned(B * S));
    // (splitting the scores alone, level 1, measured 6e-4 relative error per
    // output row at 2.8 ms per SAM 3 image against 5e-6 at 3.9 ms for level 2
    // and 4e-3 at 1.9 ms for level 0)
    if (precise)
        hipLaunchKernelGGL((attention_kernel<4, 2>), grid, dim3(256), 0, stream, o, out, ldo, H, N, np, S, part_o,
                           part_ml);
    else
        hipLaunchKernelGGL((attention_kernel<4, 0>), grid, dim3(256), 0, stream, o, out, ldo, H, N, np, S, part_o,
                           part_ml);
    if (S > 1) {
        const int64_t n = int64_t(B) * N * H * 16;
        hipLaunchKernelGGL(attention_merge_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, stream, part_o,
                           part_ml, out, ldo, B * N, H, S);
    }
    return true;
}

void launch_patch_columns(const float* image, int img, int patch, _Float16* a, float* row_scale, int kp,
                          hipStream_t stream) {
    const int64_t grid = img / patch, n = grid * grid * kp;
    hipLaunchKernelGGL(patch_columns_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, stream, image, img, patch,
                       a, row_scale, kp);
}

void launch_patch_kernel(const float* kernel, int E, int patch, _Float16* w, int kp, hipStream_t stream) {
    const int64_t n = int64_t(E) * kp;
    hipLaunchKernelGGL(patch_kernel_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, stream, kernel, E, patch, w,
                       kp);
}

}  // namespace samhip
