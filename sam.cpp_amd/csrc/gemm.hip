// Quantized-weight GEMM for gfx950: Y[m][n] = rs[m] * sum_k A[m][k] * Wq[n][k]
//   A  : staged fp16 activations [M][K] (row scale rs[m] = 2^e)
//   Wq : GGUF-packed weight rows (Q8_0 / Q4_K / Q5_K / Q6_K), any row stride
//   Y  : F32 [M][N] with row stride ldy
// Weights are dequantized to fp16(ggml to_float(W)) while they travel from
// HBM to LDS; the product runs on v_mfma_f32_32x32x16_f16 with F32
// accumulation.  This replaces ggml's MUL_MAT kernels for packed weights
// (CPU vec_dot_* / CUDA MMQ, tests/runtime/ggml/test_quantization.cpp:604-614).
#include "internal.hpp"

namespace samhip {

namespace {

constexpr int BM = 128, BN = 128, BK = 32;
constexpr int LDS_STRIDE = BK + 8;   // halves; 80-byte rows keep 16-byte reads conflict-free
constexpr int GROUP_M = 8;

// Tile order: blocks are dispatched round-robin over the 8 XCDs, so give each
// XCD a contiguous range of tiles, and walk that range in groups of GROUP_M
// row-tiles so that concurrently resident tiles share A rows and W rows in
// the XCD's L2.
__device__ __forceinline__ void tile_of(int bid, int nblocks, int tiles_m, int tiles_n, int& tm, int& tn) {
    const int per = nblocks / 8, rem = nblocks % 8;
    const int xcd = bid % 8, idx = bid / 8;
    const int t = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + idx;
    const int span = GROUP_M * tiles_n;
    const int group = t / span, first = group * GROUP_M;
    const int gm = min(tiles_m - first, GROUP_M);
    const int within = t % span;
    tm = first + within % gm;
    tn = within / gm;
}

template <int WT>
__global__ __launch_bounds__(256, 2) void gemm_kernel(const _Float16* __restrict__ A, int64_t lda,
                                                      const float* __restrict__ row_scale,
                                                      const uint8_t* __restrict__ W, int64_t w_stride,
                                                      float* __restrict__ Y, int64_t ldy, int M, int N, int K,
                                                      int tiles_m, int tiles_n) {
    __shared__ _Float16 As[2][BM * LDS_STRIDE];
    __shared__ _Float16 Bs[2][BN * LDS_STRIDE];

    int tm, tn;
    tile_of(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    // loader role: row lr of the tile, 16-element half lh of the K step
    const int lr = tid >> 1, lh = tid & 1;
    const bool a_ok = m0 + lr < M;
    const bool b_ok = n0 + lr < N;
    const _Float16* a_src = A + int64_t(a_ok ? m0 + lr : 0) * lda + 16 * lh;
    const uint8_t* w_row = W + int64_t(b_ok ? n0 + lr : 0) * w_stride;

    floatx16 acc[2][2];
    for (int i = 0; i < 2; ++i)
        for (int j = 0; j < 2; ++j)
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    u32x4 a_reg[2];
    WeightPiece<WT> b_reg;

    auto global_load = [&](int step) {
        if (a_ok) {
            const u32x4* p = reinterpret_cast<const u32x4*>(a_src + BK * step);
            a_reg[0] = p[0];
            a_reg[1] = p[1];
        } else {
            a_reg[0] = u32x4{0, 0, 0, 0};
            a_reg[1] = u32x4{0, 0, 0, 0};
        }
        if (b_ok) b_reg.load(w_row, step, lh);
    };
    auto lds_store = [&](int buf, int step) {
        u32x4* ad = reinterpret_cast<u32x4*>(&As[buf][lr * LDS_STRIDE + 16 * lh]);
        ad[0] = a_reg[0];
        ad[1] = a_reg[1];
        _Float16 w[16];
        if (b_ok) {
            b_reg.dequant(step, lh, w);
        } else {
            for (int i = 0; i < 16; ++i) w[i] = (_Float16)0.f;
        }
        half8* bd = reinterpret_cast<half8*>(&Bs[buf][lr * LDS_STRIDE + 16 * lh]);
        bd[0] = half8{w[0], w[1], w[2], w[3], w[4], w[5], w[6], w[7]};
        bd[1] = half8{w[8], w[9], w[10], w[11], w[12], w[13], w[14], w[15]};
    };

    const int nsteps = K / BK;
    global_load(0);
    lds_store(0, 0);
    __syncthreads();

    const int frag_row = lane & 31, frag_k = 8 * (lane >> 5);
    for (int s = 0; s < nsteps; ++s) {
        const int buf = s & 1;
        if (s + 1 < nsteps) global_load(s + 1);
#pragma unroll
        for (int ks = 0; ks < BK; ks += 16) {
            half8 af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = *reinterpret_cast<const half8*>(&As[buf][(wm * 64 + i * 32 + frag_row) * LDS_STRIDE + ks + frag_k]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bf[j] = *reinterpret_cast<const half8*>(&Bs[buf][(wn * 64 + j * 32 + frag_row) * LDS_STRIDE + ks + frag_k]);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (s + 1 < nsteps) lds_store(buf ^ 1, s + 1);
        __syncthreads();
    }

    // 32x32 accumulator layout: lane l holds column l%32, rows 8*(r/4) + 4*(l/32) + r%4.
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (m >= M) continue;
            const float rs = row_scale[m];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int n = n0 + wn * 64 + j * 32 + (lane & 31);
                if (n < N) Y[int64_t(m) * ldy + n] = acc[i][j][r] * rs;
            }
        }
    }
}

}  // namespace

const char* gemm_variant(int wtype) {
    switch (wtype) {
        case T_Q8_0: return "gemm_f16mfma_128x128x32_q8_0";
        case T_Q4_K: return "gemm_f16mfma_128x128x32_q4_k";
        case T_Q5_K: return "gemm_f16mfma_128x128x32_q5_k";
        case T_Q6_K: return "gemm_f16mfma_128x128x32_q6_k";
        default: return nullptr;
    }
}

const char* launch_gemm(int wtype, const _Float16* a, int64_t lda, const float* row_scale, const void* w,
                        int64_t w_stride, float* y, int64_t ldy, int M, int N, int K, hipStream_t stream) {
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    const dim3 grid(unsigned(tiles_m * tiles_n)), block(256);
    const uint8_t* wb = static_cast<const uint8_t*>(w);
#define SAMHIP_GEMM(T)                                                                                             \
    hipLaunchKernelGGL(gemm_kernel<T>, grid, block, 0, stream, a, lda, row_scale, wb, w_stride, y, ldy, M, N, K, \
                       tiles_m, tiles_n)
    switch (wtype) {
        case T_Q8_0: SAMHIP_GEMM(T_Q8_0); break;
        case T_Q4_K: SAMHIP_GEMM(T_Q4_K); break;
        case T_Q5_K: SAMHIP_GEMM(T_Q5_K); break;
        case T_Q6_K: SAMHIP_GEMM(T_Q6_K); break;
        default: return nullptr;
    }
#undef SAMHIP_GEMM
    return gemm_variant(wtype);
}

}  // namespace samhip
