// Exact tall products for Q8_0 weights on the int8 matrix cores (gfx950):
//   Y[m][n] = sum_b (d_w[n][b] d_x[m][b]) * sum_{k in b} q_x[m][k] q_w[n][k]
// per 32-value block b, in K order: ggml's native CPU arithmetic for Q8_0
// weights (vec_dot_q8_0_q8_0 on Q8_0 activation codes), the reference's
// `ggml-quantized-cpu-native-v1` profile (src/runtime/ggml/runtime.hpp:105).
//
// Two launches per product:
//  1. prep_q8_split_kernel: each activation row packed to Q8_0 codes and
//     fp16 block scales (ggml's from_float, bit-exact, both roundings), and
//     each packed weight row split the same way, into
//       codes [rows][K] int8 (16-byte aligned rows) and
//       scales [K/32][rows] F32 (a block's scales for consecutive rows
//       are contiguous, so a tile's scales are one direct-to-LDS load);
//  2. gemm_i8_kernel: BM x BN tiles, K in stages of two blocks through a
//     ring of LDS stages filled by direct-to-LDS loads (codes XOR-swizzled
//     by row so the 32 rows of a fragment read spread over the banks), one
//     v_mfma_i32_32x32x32_i8 per 32x32 tile and block, and the per-block
//     update acc = fma(d_w d_x, dot, acc) on the VALU (the next block's
//     MFMAs are issued before this block's update).
#include "internal.hpp"
#include "q8stage.hpp"

namespace samhip {

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
constexpr int RSRC_WORD3 = 0x00020000;   // raw buffer, 32-bit data format

// ---------------------------------------------------------------------------
// 1. Split staging.  Workgroups [0, ceil(M / 4)) take four activation rows
// (a wave per row; a lane owns 8 consecutive values, a block's four lanes
// meet on its maximum), the rest four weight rows (a lane per block).
// ---------------------------------------------------------------------------
template <bool X86, bool XVEC>
__global__ __launch_bounds__(256) void prep_q8_split_kernel(const float* __restrict__ X, int64_t ldx, int M, int K,
                                                            int8_t* __restrict__ ac, float* __restrict__ as,
                                                            const uint8_t* __restrict__ W, int64_t w_stride, int N,
                                                            int8_t* __restrict__ bc, float* __restrict__ bs) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nb = K / 32;
    const int arows_wg = (M + 3) / 4;
    if (int(blockIdx.x) < arows_wg) {
        const int m = blockIdx.x * 4 + wave;
        if (m >= M) return;
        const float* xr = X + int64_t(m) * ldx;
        for (int k0 = 0; k0 < K; k0 += 512) {
            const int k = k0 + 8 * lane;
            float v[8];
            if (k < K) {
                if (XVEC) {
                    const floatx4 t0 = load4f(xr + k), t1 = load4f(xr + k + 4);
                    v[0] = t0[0]; v[1] = t0[1]; v[2] = t0[2]; v[3] = t0[3];
                    v[4] = t1[0]; v[5] = t1[1]; v[6] = t1[2]; v[7] = t1[3];
                } else {
#pragma unroll
                    for (int i = 0; i < 8; ++i) v[i] = xr[k + i];
                }
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = 0.f;
            }
            float amax = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
            amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
            amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
            const float d = amax / 127.f;
            float inv;
            if (X86) inv = amax != 0.f ? 127.f / amax : 0.f;
            else inv = d != 0.f ? 1.f / d : 0.f;
            uint32_t q[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float s = v[i] * inv;
                q[i] = uint32_t(cvt_i32_nan0(X86 ? __builtin_rintf(s) : __builtin_roundf(s)));
            }
            const uint32_t w0 = __builtin_amdgcn_perm(__builtin_amdgcn_perm(q[3], q[2], 0x0c0c0400u),
                                                      __builtin_amdgcn_perm(q[1], q[0], 0x0c0c0400u), 0x05040100u);
            const uint32_t w1 = __builtin_amdgcn_perm(__builtin_amdgcn_perm(q[7], q[6], 0x0c0c0400u),
                                                      __builtin_amdgcn_perm(q[5], q[4], 0x0c0c0400u), 0x05040100u);
            if (k < K) {
                *reinterpret_cast<uint2*>(ac + int64_t(m) * K + k) = uint2{w0, w1};
                if ((lane & 3) == 0) as[int64_t(k / 32) * M + m] = half_bits_to_float(float_to_half_bits(d));
            }
        }
    } else {
        const int n = (blockIdx.x - arows_wg) * 4 + wave;
        if (n >= N) return;
        const uint8_t* wr = W + int64_t(n) * w_stride;
        for (int b = lane; b < nb; b += 64) {
            const uint8_t* blk = wr + 34 * b;
            const u32x4 lo = load16_a2(blk + 2), hi = load16_a2(blk + 18);
            u32x4* dst = reinterpret_cast<u32x4*>(bc + int64_t(n) * K + 32 * b);
            dst[0] = lo;
            dst[1] = hi;
            bs[int64_t(b) * N + n] = half_bits_to_float(load2_a2(blk));
        }
    }
}

// ---------------------------------------------------------------------------
// 2. The product.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int swz4(int r) { return (r >> 2) & 3; }

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | 0xF00);
}

template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN) void gemm_i8_kernel(const int8_t* __restrict__ ac, const float* __restrict__ as,
                                                             const int8_t* __restrict__ bc, const float* __restrict__ bs,
                                                             float* Y, int64_t ldy, int M, int N, int K, int tiles_m,
                                                             int tiles_n) {
#if defined(__HIP_DEVICE_COMPILE__)
#pragma clang fp contract(off)
    constexpr int STAGES = 3;
    constexpr int NW = WM * WN;
    constexpr int BK = 64;                           // codes per stage: two blocks
    constexpr int CODE_BYTES = (BM + BN) * BK;
    constexpr int STAGE_BYTES = CODE_BYTES + 2 * (BM + BN) * 4;
    constexpr int A_CODE_LOADS = BM / 16, B_CODE_LOADS = BN / 16;     // 1 KB = 16 rows per wave load
    constexpr int A_SC_LOADS = 2 * BM / 64, B_SC_LOADS = 2 * BN / 64; // 64 scales per wave load
    constexpr int ALL_LOADS = A_CODE_LOADS + B_CODE_LOADS + A_SC_LOADS + B_SC_LOADS;
    constexpr int LOADS = ALL_LOADS / NW;
    constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32;
    static_assert(LOADS * NW == ALL_LOADS, "the stage's loads split evenly over the waves");
    static_assert(BM % 64 == 0 && BN % 64 == 0 && FM >= 1 && FN >= 1, "tile shape");

    __shared__ __attribute__((aligned(1024))) uint8_t lds[STAGES * STAGE_BYTES];

    // XCD-aware tile order: a contiguous run of tiles per XCD, walked in
    // groups of 4 row tiles
    int tm, tn;
    {
        const int nblocks = gridDim.x, bid = blockIdx.x;
        const int per = nblocks / 8, rem = nblocks % 8;
        const int xcd = bid % 8, idx = bid / 8;
        const int t = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + idx;
        const int span = 4 * tiles_n;
        const int first = (t / span) * 4;
        const int gm = min(tiles_m - first, 4);
        const int within = t % span;
        tm = first + within % gm;
        tn = within / gm;
    }
    const int m0 = tm * BM, n0 = tn * BN;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int nb = K / 32;

    const uint32_t a_bytes = uint32_t(int64_t(M) * K), b_bytes = uint32_t(int64_t(N) * K);
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(ac), 0, a_bytes, RSRC_WORD3);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(bc), 0, b_bytes, RSRC_WORD3);
    const __amdgpu_buffer_rsrc_t rsa =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(as), 0, uint32_t(int64_t(nb) * M * 4), RSRC_WORD3);
    const __amdgpu_buffer_rsrc_t rsb =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(bs), 0, uint32_t(int64_t(nb) * N * 4), RSRC_WORD3);

    // the loads of one stage, listed as ALL_LOADS wave loads; wave w issues
    // w, w + NW, ...
    auto issue = [&](int s) {
        uint8_t* st = lds + (s % STAGES) * STAGE_BYTES;
#pragma unroll
        for (int j = 0; j < LOADS; ++j) {
            const int li = wave + NW * j;
            if (li < A_CODE_LOADS + B_CODE_LOADS) {
                const bool is_a = li < A_CODE_LOADS;
                const int blk = is_a ? li : li - A_CODE_LOADS;
                const int r = blk * 16 + lane / 4, slot = lane % 4, kc = slot ^ swz4(r);
                const int row = (is_a ? m0 : n0) + r;
                const int lim = is_a ? M : N;
                const uint32_t off = row < lim ? uint32_t(int64_t(row) * K + BK * s + 16 * kc) : (is_a ? a_bytes : b_bytes);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(is_a ? ra : rb,
                                                         (__attribute__((address_space(3))) void*)(st + (is_a ? 0 : BM * BK) + blk * 1024),
                                                         16, off, 0, 0, 0);
            } else {
                const int si = li - A_CODE_LOADS - B_CODE_LOADS;
                const bool is_a = si < A_SC_LOADS;
                const int sj = is_a ? si : si - A_SC_LOADS;
                const int rows = is_a ? BM : BN;
                const int bb = sj / (rows / 64), part = sj % (rows / 64);
                const int rr = part * 64 + lane;
                const int lim = is_a ? M : N;
                const int row = (is_a ? m0 : n0) + rr;
                // rows past the operand read the next block's scales or, in the
                // last block, zero: their codes are zero and their outputs unused
                const uint32_t off = uint32_t((int64_t(2 * s + bb) * lim + row) * 4);
                uint8_t* dst = st + CODE_BYTES + (is_a ? 0 : 2 * BM * 4) + (bb * rows + part * 64) * 4;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(is_a ? rsa : rsb, (__attribute__((address_space(3))) void*)dst, 4,
                                                         off, 0, 0, 0);
            }
        }
    };

    const int frow = lane & 31, h = lane >> 5;
    int a_row[FM], b_row[FN];
#pragma unroll
    for (int i = 0; i < FM; ++i) a_row[i] = wm * TM + i * 32 + frow;
#pragma unroll
    for (int j = 0; j < FN; ++j) b_row[j] = wn * TN + j * 32 + frow;

    floatx16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int nst = K / BK;
    auto enter = [&](int t) {
        const int later = min(STAGES - 2, nst - 1 - t);
        __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0)
        if (later >= 1) wait_vmcnt<LOADS>();
        else wait_vmcnt<0>();
        asm volatile("s_barrier" ::: "memory");
        if (t + STAGES - 1 < nst) issue(t + STAGES - 1);
    };
    // products of block bb of stage s
    auto mfmas = [&](int s, int bb, i32x16 (&dots)[FM][FN]) {
        const uint8_t* st = lds + (s % STAGES) * STAGE_BYTES;
        const int kc = 2 * bb + h;
        i32x4 fa[FM], fb[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
            fa[i] = *reinterpret_cast<const i32x4*>(st + a_row[i] * BK + 16 * (kc ^ swz4(a_row[i])));
#pragma unroll
        for (int j = 0; j < FN; ++j)
            fb[j] = *reinterpret_cast<const i32x4*>(st + BM * BK + b_row[j] * BK + 16 * (kc ^ swz4(b_row[j])));
        const i32x16 zero = {0};
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) dots[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], zero, 0, 0, 0);
    };
    // acc += d_w d_x dot for block bb of stage s (element r of lane l: row
    // 8 (r / 4) + 4 h + r % 4 of the fragment, column l % 32): a conversion,
    // a multiply and an fma per element.  (Forming the products d_x d_w of a
    // tile on the f32 matrix core instead, as the outer product of its 32 row
    // and 32 column scales, leaves two VALU operations per element but
    // measured slower on MI355X: ViT fc2 197 against 152 us per product.)
    auto update = [&](int s, int bb, const i32x16 (&dots)[FM][FN]) {
        const uint8_t* st = lds + (s % STAGES) * STAGE_BYTES;
        const float* sa = reinterpret_cast<const float*>(st + CODE_BYTES) + bb * BM;
        const float* sb = reinterpret_cast<const float*>(st + CODE_BYTES + 2 * BM * 4) + bb * BN;
        float dw[FN];
#pragma unroll
        for (int j = 0; j < FN; ++j) dw[j] = sb[b_row[j]];
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const floatx4 dx = *reinterpret_cast<const floatx4*>(sa + wm * TM + i * 32 + 8 * q + 4 * h);
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int p = 0; p < 4; ++p)
                        acc[i][j][4 * q + p] = __builtin_fmaf(dw[j] * dx[p], float(dots[i][j][4 * q + p]), acc[i][j][4 * q + p]);
            }
    };

#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
        if (s < nst) issue(s);
    i32x16 d0[FM][FN], d1[FM][FN];
    for (int s = 0; s < nst; ++s) {
        enter(s);
        mfmas(s, 0, d0);
        mfmas(s, 1, d1);
        update(s, 0, d0);
        update(s, 1, d1);
    }

    // output: each store instruction covers two 128-byte row segments
    const uint32_t y_bytes = uint32_t(min(int64_t(M) * ldy * 4, int64_t(0x7fffffff)));
    const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(Y, 0, y_bytes, RSRC_WORD3);
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int n = n0 + wn * TN + j * 32 + frow;
            const int mb = m0 + wm * TM + i * 32 + 4 * h;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = mb + 8 * (r >> 2) + (r & 3);
                const float val = acc[i][j][r];
                const uint32_t off = (m < M && n < N) ? uint32_t((int64_t(m) * ldy + n) * 4) : 0x80000000u;
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(val), ry, off, 0, 0);
            }
        }
    (void)nb;
#endif
}

}  // namespace

size_t gemm_i8_staging_bytes(int M, int N, int K) {
    auto align256 = [](size_t v) { return (v + 255) & ~size_t(255); };
    return align256(size_t(M) * K) + align256(size_t(K / 32) * M * 4) + align256(size_t(N) * K) +
           align256(size_t(K / 32) * N * 4);
}

bool gemm_i8_supported(int M, int N, int K) {
    return M >= 1 && N >= 1 && K >= 64 && K % 64 == 0 && int64_t(M) * K < 0x7fffffff && int64_t(N) * K < 0x7fffffff &&
           int64_t(K / 32) * M * 4 < 0x7fffffff && int64_t(K / 32) * N * 4 < 0x7fffffff;
}

const char* gemm_i8_variant() { return "gemm_i8mfma_q8_0_128x128x64"; }

const char* launch_gemm_i8(const float* x, int64_t ldx, const void* w, int64_t w_stride, float* y, int64_t ldy, int M,
                           int N, int K, int x86, void* staging, hipStream_t stream, const char** prep_name_out) {
    if (!gemm_i8_supported(M, N, K) || int64_t(M) * ldy * 4 > 0x7fffffff) return nullptr;
    auto align256 = [](size_t v) { return (v + 255) & ~size_t(255); };
    uint8_t* base = static_cast<uint8_t*>(staging);
    int8_t* ac = reinterpret_cast<int8_t*>(base);
    base += align256(size_t(M) * K);
    float* as = reinterpret_cast<float*>(base);
    base += align256(size_t(K / 32) * M * 4);
    int8_t* bc = reinterpret_cast<int8_t*>(base);
    base += align256(size_t(N) * K);
    float* bs = reinterpret_cast<float*>(base);
    const bool xvec = reinterpret_cast<uintptr_t>(x) % 16 == 0 && ldx % 4 == 0;
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    const dim3 pgrid(unsigned((M + 3) / 4 + (N + 3) / 4));
#define SAMHIP_PREP(X86V, XV)                                                                                       \
    hipLaunchKernelGGL((prep_q8_split_kernel<X86V, XV>), pgrid, dim3(256), 0, stream, x, ldx, M, K, ac, as, wb, \
                       w_stride, N, bc, bs)
    if (x86) {
        if (xvec) SAMHIP_PREP(true, true); else SAMHIP_PREP(true, false);
    } else {
        if (xvec) SAMHIP_PREP(false, true); else SAMHIP_PREP(false, false);
    }
#undef SAMHIP_PREP
    if (prep_name_out) *prep_name_out = "stage_split_q8_0";
    constexpr int BM = 128, BN = 128;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    hipLaunchKernelGGL((gemm_i8_kernel<BM, BN, 2, 4>), dim3(unsigned(tiles_m * tiles_n)), dim3(512), 0, stream, ac, as,
                       bc, bs, y, ldy, M, N, K, tiles_m, tiles_n);
    return gemm_i8_variant();
}

}  // namespace samhip
