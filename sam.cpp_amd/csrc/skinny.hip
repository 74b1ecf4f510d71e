// Skinny and medium quantized-weight products (M < 256 activation rows):
//   Y[m][n] = rs[m] * sum_k A[m][k] * fp16(to_float(Wq[n][k]))
// the shapes of SAM 3's text encoder (M = 32), the K/V projections of text
// tokens (M = 33) and the decoder queries (M = 201), where every packed
// weight byte is read once and the product is HBM-bound (ggml's MMVQ / MMQ
// dispatch for these widths: tests/runtime/ggml/test_quantization.cpp:604-614;
// call sites src/models/sam3/text_encoder.hpp:83-174,
// src/models/sam3/detector.hpp:343-479).
//
// One workgroup owns 32 consecutive weight rows and the whole K range; its
// KSPLIT waves (4 to 16) take contiguous shares of the K steps.  Each
// lane decodes 16 weights of one row per 32-wide K step straight from the
// packed bytes into registers (the same fp16 operand as the tall path), and
// the wave multiplies them against up to eight 32-row activation tiles with
// v_mfma_f32_32x32x16_f16.  Lanes 0-31 take K elements 0-15 of the step and
// lanes 32-63 elements 16-31 (the A fragments follow the same permutation),
// so a lane's operands come from 16 contiguous bytes of codes.  The KSPLIT
// partial sums meet in LDS and leave as coalesced 128-byte row segments.
#include <algorithm>

#include "internal.hpp"
#include "q8stage.hpp"

namespace samhip {

namespace {

constexpr int ROWS = 32;            // weight rows per workgroup
constexpr int PART_STRIDE = 33;     // floats; padded LDS rows for the partial sums

template <int WT, int MT, int KSPLIT, int U>
__global__ __launch_bounds__(64 * KSPLIT) void skinny_kernel(const _Float16* __restrict__ A, int64_t lda,
                                                             const float* __restrict__ row_scale,
                                                             const uint8_t* __restrict__ W, int64_t w_stride,
                                                             float* __restrict__ Y, int64_t ldy, int M, int N,
                                                             int K) {
    __shared__ float part[KSPLIT][ROWS * PART_STRIDE];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n0 = blockIdx.x * ROWS;
    const int col = lane & 31, h = lane >> 5;
    const uint8_t* w_row = W + int64_t(min(n0 + col, N - 1)) * w_stride;
    const int nsteps = K / 32;
    const int per = (nsteps + KSPLIT - 1) / KSPLIT;
    const int s0 = min(nsteps, wave * per), s1 = min(nsteps, s0 + per);

    const _Float16* a_row[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) a_row[t] = A + int64_t(min(t * 32 + col, M - 1)) * lda + 16 * h;

    floatx16 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][r] = 0.f;

    // U steps per batch: every load of the batch is issued before the first
    // product, so each wave keeps U steps of weights and activations in flight
    for (int s = s0; s < s1; s += U) {
        WeightPiece<WT> wp[U];
        half8 a_lo[U][MT], a_hi[U][MT];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int st = min(s + u, s1 - 1);   // past the range: a repeat of the last step, never multiplied
            wp[u].load(w_row, st, h);
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const half8* p = reinterpret_cast<const half8*>(a_row[t] + 32 * st);
                a_lo[u][t] = p[0];
                a_hi[u][t] = p[1];
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (s + u >= s1) break;
            _Float16 wv[16];
            wp[u].dequant(s + u, h, wv);
            const half8 b_lo{wv[0], wv[1], wv[2], wv[3], wv[4], wv[5], wv[6], wv[7]};
            const half8 b_hi{wv[8], wv[9], wv[10], wv[11], wv[12], wv[13], wv[14], wv[15]};
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_lo[u][t], b_lo, acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_hi[u][t], b_hi, acc[t], 0, 0, 0);
            }
        }
    }

    // 32x32 accumulator layout: lane l holds column (weight row) l%32 and
    // activation rows 8*(r/4) + 4*(l/32) + r%4.
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        if (t * 32 >= M) break;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int ml = 8 * (r >> 2) + 4 * h + (r & 3);
            part[wave][ml * PART_STRIDE + col] = acc[t][r];
        }
        __syncthreads();
        for (int o = threadIdx.x; o < ROWS * 32; o += 64 * KSPLIT) {
            const int ml = o >> 5, nl = o & 31;
            const int m = t * 32 + ml, n = n0 + nl;
            float v = 0.f;
#pragma unroll
            for (int w = 0; w < KSPLIT; ++w) v += part[w][ml * PART_STRIDE + nl];
            if (m < M && n < N) Y[int64_t(m) * ldy + n] = v * row_scale[m];
        }
        __syncthreads();
    }
}

// Waves per workgroup and steps per batch: a grid with fewer workgroups than
// CUs gets more waves per workgroup (all on one CU) and deeper batches, sized
// so that the wave's registers still allow KSPLIT / 4 waves per SIMD.
template <int WT, int MT>
void launch_mt(const _Float16* a, int64_t lda, const float* rs, const uint8_t* w, int64_t w_stride, float* y,
               int64_t ldy, int M, int N, int K, bool wide, hipStream_t stream) {
    const dim3 grid(unsigned((N + ROWS - 1) / ROWS));
    constexpr int KS = MT == 1 ? 16 : MT == 2 ? 8 : 4;
    constexpr int UW = MT == 1 ? (WT == T_Q8_0 ? 4 : 2) : MT == 2 ? 4 : MT <= 4 ? 2 : 1;
    if (wide)
        hipLaunchKernelGGL((skinny_kernel<WT, MT, KS, UW>), grid, dim3(64 * KS), 0, stream, a, lda, rs, w, w_stride, y,
                           ldy, M, N, K);
    else
        hipLaunchKernelGGL((skinny_kernel<WT, MT, 4, MT <= 2 ? 2 : 1>), grid, dim3(256), 0, stream, a, lda, rs, w,
                           w_stride, y, ldy, M, N, K);
}

template <int WT>
void launch_wt(const _Float16* a, int64_t lda, const float* rs, const uint8_t* w, int64_t w_stride, float* y,
               int64_t ldy, int M, int N, int K, bool wide, hipStream_t stream) {
    switch ((M + 31) / 32) {
        case 1: launch_mt<WT, 1>(a, lda, rs, w, w_stride, y, ldy, M, N, K, wide, stream); break;
        case 2: launch_mt<WT, 2>(a, lda, rs, w, w_stride, y, ldy, M, N, K, wide, stream); break;
        case 3: launch_mt<WT, 3>(a, lda, rs, w, w_stride, y, ldy, M, N, K, wide, stream); break;
        case 4: launch_mt<WT, 4>(a, lda, rs, w, w_stride, y, ldy, M, N, K, wide, stream); break;
        case 5: launch_mt<WT, 5>(a, lda, rs, w, w_stride, y, ldy, M, N, K, wide, stream); break;
        case 6: launch_mt<WT, 6>(a, lda, rs, w, w_stride, y, ldy, M, N, K, wide, stream); break;
        case 7: launch_mt<WT, 7>(a, lda, rs, w, w_stride, y, ldy, M, N, K, wide, stream); break;
        default: launch_mt<WT, 8>(a, lda, rs, w, w_stride, y, ldy, M, N, K, wide, stream); break;
    }
}

// ---------------------------------------------------------------------------
// Fused path for M <= 256: one launch per product (two when K is split).  A
// workgroup of 8 waves owns 128 weight rows (a 32-row tile per wave pair),
// a block of up to 128 activation rows (the decoder's 201 queries take two
// blocks along the grid) and a range of 256-wide K chunks.  Per chunk:
//  * the waves copy the packed bytes of their tiles with coalesced dword
//    loads into LDS (rows padded to an odd dword count, so the per-lane piece
//    reads of one column are bank-conflict free);
//  * the workgroup packs the activation chunk (M rows x 256, F32) into the
//    fp16 operand in LDS with quant8 (Q8_0 / Q8_K blocks bit-exact with
//    ggml's from_float) under a power-of-two scale 2^-e per row and chunk;
//  * each wave decodes its pieces from LDS and runs 4 of the chunk's 8 K
//    steps of v_mfma_f32_32x32x16_f16, then adds the products times 2^e;
//    the wave pair's two sums meet in LDS at the end.
// When the K range is split over S workgroups, each writes its partial sums
// to scratch and splitk_reduce_kernel adds the S partials in split order
// (results do not depend on scheduling).  A reduction inside the kernel
// would need agent-scope release/acquire fences, which on gfx950 write back
// and invalidate the XCD's whole L2; the second launch is cheaper.
// ---------------------------------------------------------------------------

constexpr int FROWS = 128;          // weight rows per workgroup
constexpr int CHUNK = 256;          // K elements per chunk
constexpr int ALD = CHUNK + 8;      // halves per LDS activation row

template <int WT>
constexpr int chunk_bytes() { return WT == T_Q8_0 ? 8 * 34 : block_bytes(WT); }
// dwords per LDS weight row: the row's bytes start at byte 0 or 2 of the
// first dword; an odd count keeps column reads conflict free
template <int WT>
constexpr int wrow_dw() { return ((chunk_bytes<WT>() + 2 + 3) / 4) | 1; }

template <int WT, int MODE, bool X86, int MT, bool XVEC>
__global__ __launch_bounds__(512) void fused_skinny_kernel(const float* __restrict__ X, int64_t ldx,
                                                           const uint8_t* __restrict__ W, int64_t w_stride,
                                                           float* __restrict__ Y, int64_t ldy,
                                                           float* __restrict__ part, int M, int N, int K, int RG,
                                                           int S, int cps) {
    constexpr int WDW = wrow_dw<WT>();
    constexpr int CB = chunk_bytes<WT>();
    // the activation tile; after the last chunk it holds the K-half partial sums
    __shared__ __attribute__((aligned(16))) _Float16 As[MT * 32 * ALD];
    __shared__ __attribute__((aligned(16))) float escale[MT * 32];
    __shared__ __attribute__((aligned(16))) uint32_t Ws[4][32 * WDW];
    static_assert(MT * 32 * ALD * 2 >= 4 * MT * 1024 * 4, "partial-sum exchange must fit the activation tile");

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tile = wave & 3, kh = wave >> 2;   // 32-row tile, half of the chunk's K steps
    const int rg = blockIdx.x % RG, sp = (blockIdx.x / RG) % S, mb = blockIdx.x / (RG * S);
    const int n0 = rg * FROWS + 32 * tile;
    const int col = lane & 31, h = lane >> 5;
    const int nchunks = (K + CHUNK - 1) / CHUNK;
    const int c0 = sp * cps, c1 = min(nchunks, c0 + cps);
    // this workgroup's block of MT * 32 activation rows
    const int m0 = mb * (MT * 32), Mall = M;
    X += int64_t(m0) * ldx;
    Y += int64_t(m0) * ldy;
    M = min(M - m0, MT * 32);

    // this lane's weight row (for its pieces) and its byte shift in LDS
    const uint8_t* my_row = W + int64_t(min(n0 + col, N - 1)) * w_stride;

    floatx16 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][r] = 0.f;

    for (int c = c0; c < c1; ++c) {
        const int kc = c * CHUNK;
        const int steps = min(8, (K - kc) / 32);
        const int cb = WT == T_Q8_0 ? 34 * steps : CB;
        const int64_t off = int64_t(c) * CB;

        // 1. the activation rows are requested first (loads return in issue
        //    order, so they are packed while the weights are in flight),
        //    then the packed weight bytes: each wave copies 16 rows of its
        //    tile with coalesced dword loads (two rows per pass)
        auto load_x = [&](int pass) -> floatx8 {
            const int r = pass * 16 + wave * 2 + h;
            const int k = kc + 8 * col;
            floatx8 v{0, 0, 0, 0, 0, 0, 0, 0};
            if (r < M && k < K) {
                const float* xr = X + int64_t(r) * ldx + k;
                if (XVEC) {
                    const floatx4 lo = load4f(xr), hi = load4f(xr + 4);
                    v = floatx8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                } else {
#pragma unroll
                    for (int i = 0; i < 8; ++i) v[i] = xr[i];
                }
            }
            return v;
        };
        floatx8 xv[2 * MT];
#pragma unroll
        for (int p = 0; p < 2 * MT; ++p) xv[p] = load_x(p);
        constexpr int DPR = (CB + 2 + 3) / 4;   // dwords a row can span
        constexpr int RI = (DPR + 31) / 32;
        uint32_t wreg[8][RI];
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            const int r = 16 * kh + 2 * p + h;
            // (addressed through an integer, i.e. flat loads: global loads of
            // the same dwords measured ~1.5 % slower on the text Q4_K stream)
            const uintptr_t g = reinterpret_cast<uintptr_t>(W + int64_t(min(n0 + r, N - 1)) * w_stride + off);
            const uint32_t* src = reinterpret_cast<const uint32_t*>(g & ~uintptr_t(3));
            const int ndw = int(((g & 3) + cb + 3) >> 2);
#pragma unroll
            for (int q = 0; q < RI; ++q) {
                const int d = col + 32 * q;
                wreg[p][q] = d < ndw ? src[d] : 0u;
            }
        }

        // 2. activation chunk -> fp16 operand (two rows per wave per pass)
#pragma unroll
        for (int p = 0; p < 2 * MT; ++p) {
            const int r = p * 16 + wave * 2 + h;
            float rmax = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) rmax = fmaxf(rmax, fabsf(xv[p][i]));
            rmax = max32_lanes(rmax);
            const int e = row_exponent(rmax);
            const half8 o = quant8<MODE, X86>(xv[p], lane, exp2i(-e));
            *reinterpret_cast<half8*>(&As[r * ALD + 8 * col]) = o;
            if (col == 0) escale[r] = exp2i(e);
        }
#pragma unroll
        for (int p = 0; p < 8; ++p)
#pragma unroll
            for (int q = 0; q < RI; ++q) {
                const int d = col + 32 * q;
                if (d < WDW) Ws[tile][(16 * kh + 2 * p + h) * WDW + d] = wreg[p][q];
            }
        __syncthreads();

        // 3. products of this wave's K steps of the chunk
        floatx16 cacc[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) cacc[t][r] = 0.f;
        const LdsRow wrow{&Ws[tile][col * WDW], int((reinterpret_cast<uintptr_t>(my_row) + uintptr_t(off)) & 3)};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int s = 4 * kh + i;
            if (s >= steps) break;
            WeightPiece<WT> wp;
            wp.load(wrow, s, h);
            _Float16 wv[16];
            wp.dequant(s, h, wv);
            const half8 b_lo{wv[0], wv[1], wv[2], wv[3], wv[4], wv[5], wv[6], wv[7]};
            const half8 b_hi{wv[8], wv[9], wv[10], wv[11], wv[12], wv[13], wv[14], wv[15]};
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const half8* ap = reinterpret_cast<const half8*>(&As[(t * 32 + col) * ALD + 32 * s + 16 * h]);
                cacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ap[0], b_lo, cacc[t], 0, 0, 0);
                cacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ap[1], b_hi, cacc[t], 0, 0, 0);
            }
        }
        // accumulator element r of tile t is activation row t*32 + 8*(r/4) + 4*h + r%4
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const floatx4 sc = *reinterpret_cast<const floatx4*>(&escale[t * 32 + 8 * q + 4 * h]);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[t][4 * q + i] += cacc[t][4 * q + i] * sc[i];
            }
        __syncthreads();
    }

    // the second K half hands its sums to the first through LDS
    float* xch = reinterpret_cast<float*>(As);
    if (kh == 1) {
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) xch[((tile * MT + t) * 16 + r) * 64 + lane] = acc[t][r];
    }
    __syncthreads();
    if (kh == 1) return;

    // S == 1: the product; otherwise this split's partial sums
    const int n = n0 + col;
    float* out = part ? part + (int64_t(sp) * Mall + m0) * N : Y;
    const int64_t ld = part ? int64_t(N) : ldy;
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = t * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
            const float v = acc[t][r] + xch[((tile * MT + t) * 16 + r) * 64 + lane];
            if (m < M && n < N) out[int64_t(m) * ld + n] = v;
        }
}

// Y[m][n] = sum over q = 0 .. S-1 of part[q][m][n], in that order.  Up to
// 16 partials are loaded at once (one memory latency instead of S: the
// loads are issued before the first add).
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part, float* __restrict__ Y,
                                                            int64_t ldy, int M, int N, int S) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= int64_t(M) * N) return;
    const int m = int(i / N), n = int(i % N);
    const int64_t plane = int64_t(M) * N;
    float v = 0.f;
    for (int q = 0; q < S; q += 16) {
        float t[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) t[j] = q + j < S ? part[(q + j) * plane + i] : 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j)
            if (q + j < S) v += t[j];
    }
    Y[int64_t(m) * ldy + n] = v;
}

// ---------------------------------------------------------------------------
// Strip path for M < 256 (the text encoder's 32 tokens), in blocks of 32
// activation rows: one workgroup per 32-row strip of W, row block and group
// of four 256-wide K chunks, 16 waves, so that
// a product with K <= 1024 is one launch with no partial sums in memory.
//  * the waves copy the strip's packed bytes for the group with coalesced
//    dword loads into LDS (odd dword row stride: conflict-free piece reads);
//  * the four waves of chunk q pack its 32 activation rows (two rows per
//    wave per pass, 8 values per lane, requested before the weights) into
//    the fp16 operand with quant8 under a power-of-two scale per row and
//    chunk, as the fused kernel does;
//  * wave w runs steps 2 (w % 4) and 2 (w % 4) + 1 of chunk w / 4 (weights
//    decoded from LDS), scales by 2^e, and the 16 partial tiles are added in
//    LDS in a fixed order.
// With more than four chunks the groups go to `part` and
// splitk_reduce_kernel adds them.  Every workgroup packs the activation
// chunks it uses: VALU time per workgroup in place of a second launch and a
// round trip of partial sums through memory.
// ---------------------------------------------------------------------------
template <int WT>
constexpr int strip_wdw() { return ((4 * chunk_bytes<WT>() + 2 + 3) / 4) | 1; }

template <int WT, int MODE, bool X86, bool XVEC>
__global__ __launch_bounds__(1024) void strip_skinny_kernel(const float* __restrict__ X, int64_t ldx,
                                                            const uint8_t* __restrict__ W, int64_t w_stride,
                                                            float* __restrict__ Y, int64_t ldy,
                                                            float* __restrict__ part, int M, int N, int K, int RG,
                                                            int S) {
    constexpr int CB = chunk_bytes<WT>();
    constexpr int WDW = strip_wdw<WT>();
    constexpr int RI = (WDW + 31) / 32;
    // activation tiles of the four chunks; afterwards the 16 partial tiles
    __shared__ __attribute__((aligned(16))) _Float16 As[4][32 * ALD];
    __shared__ __attribute__((aligned(16))) uint32_t Ws[32 * WDW];
    __shared__ __attribute__((aligned(16))) float escale[4][32];
    static_assert(4 * 32 * ALD * 2 >= 16 * 16 * 64 * 4, "partial tiles must fit the activation tiles");
    float* red = reinterpret_cast<float*>(&As[0][0]);

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 31, h = lane >> 5;
    const int rg = blockIdx.x % RG, sp = (blockIdx.x / RG) % S, mb = blockIdx.x / (RG * S);
    const int n0 = rg * 32;
    const int nchunks = (K + 255) / 256;
    const int cq = wave >> 2, c = 4 * sp + cq;   // this wave's chunk
    // this workgroup's block of 32 activation rows
    const int m0 = mb * 32, Mall = M;
    X += int64_t(m0) * ldx;
    Y += int64_t(m0) * ldy;
    M = min(M - m0, 32);
    const bool active = c < nchunks;

    // 1. activations of chunk cq, rows 8 (w % 4) + 2 p + h, then the packed bytes
    const int kc = 256 * c;
    floatx8 xv[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const int r = 8 * (wave & 3) + 2 * p + h, k = kc + 8 * col;
        floatx8 v{0, 0, 0, 0, 0, 0, 0, 0};
        if (active && r < M && k < K) {
            const float* xr = X + int64_t(r) * ldx + k;
            if (XVEC) {
                const floatx4 lo = load4f(xr), hi = load4f(xr + 4);
                v = floatx8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = xr[i];
            }
        }
        xv[p] = v;
    }
    const int64_t off = int64_t(4 * sp) * CB;   // the group's first byte in a row
    const int gb = WT == T_Q8_0 ? 34 * min(32, K / 32 - 32 * sp) : CB * min(4, nchunks - 4 * sp);
    const int wr = 2 * wave + h;                  // the row this lane copies
    const uint8_t* rowp = W + int64_t(min(n0 + wr, N - 1)) * w_stride + off;
    const uint32_t sh = uint32_t(reinterpret_cast<uintptr_t>(rowp) & 3);
    const uint32_t* src = reinterpret_cast<const uint32_t*>(rowp - sh);
    const int ndw = int((sh + gb + 3) >> 2);
    uint32_t wreg[RI];
#pragma unroll
    for (int i = 0; i < RI; ++i) {
        const int d = col + 32 * i;
        wreg[i] = d < ndw ? src[d] : 0u;
    }

    // 2. the fp16 operand (two rows per pass), then the weight bytes to LDS
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const int r = 8 * (wave & 3) + 2 * p + h;
        float rmax = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) rmax = fmaxf(rmax, fabsf(xv[p][i]));
        rmax = max32_lanes(rmax);
        const int e = row_exponent(rmax);
        const half8 o = quant8<MODE, X86>(xv[p], lane, exp2i(-e));
        *reinterpret_cast<half8*>(&As[cq][r * ALD + 8 * col]) = o;
        if (col == 0) escale[cq][r] = exp2i(e);
    }
#pragma unroll
    for (int i = 0; i < RI; ++i) {
        const int d = col + 32 * i;
        if (d < WDW) Ws[wr * WDW + d] = wreg[i];
    }
    __syncthreads();

    // 3. this wave's two steps of its chunk
    floatx16 a0, a1;
#pragma unroll
    for (int r = 0; r < 16; ++r) a0[r] = a1[r] = 0.f;
    if (active) {
        const int steps = min(8, (K - kc) / 32);
        const LdsRow wrow{&Ws[col * WDW], int((reinterpret_cast<uintptr_t>(W + int64_t(min(n0 + col, N - 1)) * w_stride) +
                                               uintptr_t(off)) & 3)};
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int s = 2 * (wave & 3) + t;
            if (s >= steps) break;
            WeightPiece<WT> wp;
            wp.load(wrow, 8 * cq + s, h);
            _Float16 wv[16];
            wp.dequant(8 * cq + s, h, wv);
            const half8 b_lo{wv[0], wv[1], wv[2], wv[3], wv[4], wv[5], wv[6], wv[7]};
            const half8 b_hi{wv[8], wv[9], wv[10], wv[11], wv[12], wv[13], wv[14], wv[15]};
            const half8* ap = reinterpret_cast<const half8*>(&As[cq][col * ALD + 32 * s + 16 * h]);
            a0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ap[0], b_lo, a0, 0, 0, 0);
            a1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ap[1], b_hi, a1, 0, 0, 0);
        }
    }
    floatx16 acc;
    // accumulator element r is activation row 8 (r / 4) + 4 h + r % 4
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
        const floatx4 sc = *reinterpret_cast<const floatx4*>(&escale[cq][8 * qd + 4 * h]);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[4 * qd + i] = (a0[4 * qd + i] + a1[4 * qd + i]) * sc[i];
    }
    __syncthreads();   // the activation tiles are read; their LDS takes the partial tiles
#pragma unroll
    for (int r = 0; r < 16; ++r) red[(wave * 16 + r) * 64 + lane] = acc[r];
    __syncthreads();
    // wave w adds the 16 tiles' element (m, n), m = 2 w + h, n = n0 + col
    const int m = 2 * wave + h, n = n0 + col;
    const int ri = (4 * (m >> 3) + (m & 3)) * 64 + col + 32 * ((m >> 2) & 1);
    float v = 0.f;
#pragma unroll
    for (int t = 0; t < 16; ++t) v += red[t * 16 * 64 + ri];
    float* out = part ? part + (int64_t(sp) * Mall + m0) * N : Y;
    const int64_t ld = part ? int64_t(N) : ldy;
    if (m < M && n < N) out[int64_t(m) * ld + n] = v;
}

// ---------------------------------------------------------------------------
// Exact int8 strip path: Q8_0 weights against blocks of 32 activation rows
// (the text encoder's 32 tokens, the decoder's 201 queries) in
// COMPUTE_Q8_NATIVE, i.e. ggml's CPU
// native arithmetic on the matrix cores.  Per Q8_0 block the integer dot
// sum_k q_w q_x comes exactly out of v_mfma_i32_32x32x32_i8 (one 32-value
// block per instruction: the weight codes are the B operand as stored, no
// decode), and the block adds fma(float(dot), d_w * d_x, acc) in F32 as
// ggml's vec_dot_q8_0_q8_0 does; only the order of the block sums differs.
// One workgroup of 16 waves per 32 weight rows (CT = 1) or, for slices of
// at most 256 values, per 64 weight rows (CT = 2), 32 activation rows and K
// slice of up to 1024 values:
//  1. the strip's packed bytes for the slice go to LDS with coalesced dword
//     loads (rows of an odd dword count: conflict-free reads);
//  2. thread (m, b) packs activation row m, block b of the slice to Q8_0
//     (ggml's from_float, x86 or reference rounding) into LDS codes and
//     scales, so each workgroup packs its slice once, with one lane per
//     block and no cross-lane reductions;
//  3. CT = 1: wave w multiplies blocks w, w + 16 of the slice; CT = 2: wave
//     w multiplies block w % 8 of column tile w / 8, so all 16 waves have a
//     block and the activation slice is packed once per 64 weight rows;
//  4. each column tile's partial tiles are added in LDS in wave order.
// The host picks the slice width SL (256, 512 or 1024 values).  With more
// than one slice each workgroup writes its partial sums, which
// splitk_reduce_kernel adds in slice order.  Timed back to back on MI355X
// with the weight warm in L2: CT = 2 takes 3.85 against 7.3 us per launch at
// M = 201, N = 2048, K = 256 (224 workgroups in one round instead of 448 in
// two) and 3.6 against 4.2 us at M = 201 and 33 with N = K = 256; in the
// streams, with each product's weight read cold, only the first gained, so
// the host takes CT = 2 where it brings the grid into one round.  Both
// forms give the same bits.
// ---------------------------------------------------------------------------
constexpr int I8_XLD = kI8SliceK + 16;                                // bytes per LDS code row
constexpr int I8_WDW = (((kI8SliceK / 32) * 34 + 2 + 3) / 4) | 1;    // dwords per LDS weight row
constexpr int I8_WDW256 = ((8 * 34 + 2 + 3) / 4) | 1;                 // the same for slices of 256 values
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

template <bool X86, bool XVEC, int CT>
__global__ __launch_bounds__(1024) void q8_strip_i8_kernel(const float* __restrict__ X, int64_t ldx,
                                                           const uint8_t* __restrict__ W, int64_t w_stride,
                                                           float* __restrict__ Y, int64_t ldy, float* __restrict__ part,
                                                           int M, int N, int K, int RG, int S, int SL) {
#pragma clang fp contract(off)
    static_assert(CT == 1 || CT == 2, "one or two column tiles");
    constexpr int WP = CT == 2 ? I8_WDW256 : I8_WDW;   // dword pitch of an LDS weight row
    constexpr int TPR = 32 / CT;                        // threads per weight row in the load
    static_assert(32 * CT * WP <= 32 * I8_WDW, "the weight rows fit the LDS strip");
    __shared__ __attribute__((aligned(16))) int8_t Xq[32 * I8_XLD];
    __shared__ __attribute__((aligned(16))) float Xd[kI8SliceK / 32][32];
    __shared__ __attribute__((aligned(16))) uint32_t Ws[32 * I8_WDW];
    __shared__ __attribute__((aligned(16))) float red[16 * 16 * 64];
    constexpr int RI = (WP + TPR - 1) / TPR;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rg = blockIdx.x % RG, sp = (blockIdx.x / RG) % S, mb = blockIdx.x / (RG * S);
    const int n0 = rg * 32 * CT, k0 = sp * SL;
    const int nb = min(SL, K - k0) / 32;   // Q8_0 blocks in this slice (SL <= kI8SliceK)
    // this workgroup's block of 32 activation rows
    const int m0 = mb * 32, Mall = M;
    X += int64_t(m0) * ldx;
    Y += int64_t(m0) * ldy;
    M = min(M - m0, 32);

    // 1. packed weight bytes: thread (r, c) loads dwords c, c + 32, ... of
    // row r; the activation loads are issued before these go to LDS, so the
    // two latencies overlap (7.57 against 7.88 us per K = 1024 product)
    const int wr_r = tid / TPR, wr_c = tid % TPR;
    uint32_t wr[RI];
    {
        const uint8_t* rowp = W + int64_t(min(n0 + wr_r, N - 1)) * w_stride + int64_t(k0 / 32) * 34;
        const uint32_t sh = uint32_t(reinterpret_cast<uintptr_t>(rowp) & 3);
        const uint32_t* src = reinterpret_cast<const uint32_t*>(rowp - sh);
        const int ndw = int((sh + 34 * nb + 3) >> 2);   // <= WP (CT = 2: nb <= 8)
#pragma unroll
        for (int i = 0; i < RI; ++i) wr[i] = wr_c + TPR * i < ndw ? src[wr_c + TPR * i] : 0u;
    }
    // 2. activation rows -> Q8_0 codes and scales: wave w takes rows 2 w and
    // 2 w + 1 of the block, in SL / 256 passes of 512 values; lane l holds 8
    // consecutive values and lanes 4g..4g+3 one 32-value block (its maximum
    // over the quad by DPP), so a 16-byte load instruction touches 16 cache
    // lines instead of the 64 of a lane per block
    {
        const int passes = SL / 256;
        floatx8 v[kI8SliceK / 256];
#pragma unroll
        for (int p = 0; p < kI8SliceK / 256; ++p) {
            if (p >= passes) break;
            const int e = 512 * p + 8 * lane, pr = e >= SL, kl = e - pr * SL, m = 2 * wave + pr;
            if (m < M && kl < 32 * nb) {
                const float* xr = X + int64_t(m) * ldx + k0 + kl;
                if (XVEC) {
                    const floatx4 a = load4f(xr), c = load4f(xr + 4);
                    v[p] = floatx8{a[0], a[1], a[2], a[3], c[0], c[1], c[2], c[3]};
                } else {
#pragma unroll
                    for (int i = 0; i < 8; ++i) v[p][i] = xr[i];
                }
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) v[p][i] = 0.f;
            }
        }
#pragma unroll
        for (int i = 0; i < RI; ++i)
            if (wr_c + TPR * i < WP) Ws[wr_r * WP + wr_c + TPR * i] = wr[i];
#pragma unroll
        for (int p = 0; p < kI8SliceK / 256; ++p) {
            if (p >= passes) break;
            const int e = 512 * p + 8 * lane, pr = e >= SL, kl = e - pr * SL, m = 2 * wave + pr;
            // ggml's from_float on the block (x86 or reference rounding; NaN
            // -> code 0, this library's contract), the stored fp16 scale
            float d;
            int ci[8];
            quant8_icodes<T_Q8_0, X86>(v[p], lane, d, ci);
            uint32_t c[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) c[i] = uint32_t(ci[i]);
            const uint32_t lo = __builtin_amdgcn_perm(__builtin_amdgcn_perm(c[3], c[2], 0x0c0c0400u),
                                                      __builtin_amdgcn_perm(c[1], c[0], 0x0c0c0400u), 0x05040100u);
            const uint32_t hi = __builtin_amdgcn_perm(__builtin_amdgcn_perm(c[7], c[6], 0x0c0c0400u),
                                                      __builtin_amdgcn_perm(c[5], c[4], 0x0c0c0400u), 0x05040100u);
            if (kl < 32 * nb) {
                *reinterpret_cast<u32x2*>(&Xq[m * I8_XLD + kl]) = u32x2{lo, hi};
                if ((lane & 3) == 0) Xd[kl >> 5][m] = d;
            }
        }
    }
    __syncthreads();

    // 3. blocks wave, wave + 16 of the slice (CT = 2: block wave % 8 of
    // column tile wave / 8): activation row (A) and weight row (B) codes,
    // lanes 32h.. taking bytes 16h..16h+15 of both
    const int col = lane & 31, h = lane >> 5;
    const int tile = CT == 2 ? wave >> 3 : 0;
    const int wn = n0 + 32 * tile + col;
    const int wshift = int((reinterpret_cast<uintptr_t>(W + int64_t(min(wn, N - 1)) * w_stride) + k0 / 32 * 34) & 3);
    const uint32_t* wrow = &Ws[(32 * tile + col) * WP];
    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
    const i32x16 zero = {0};
    for (int b = CT == 2 ? wave & 7 : wave; b < nb; b += 16 / CT) {
        const i32x4 a = *reinterpret_cast<const i32x4*>(&Xq[col * I8_XLD + 32 * b + 16 * h]);
        // the row's bytes start at byte wshift (0 or 2) of its first dword;
        // every read stays inside the row's dwords
        const int sb = wshift + 34 * b, cb = sb + 2 + 16 * h;
        const int cd = cb >> 2, cs = cb & 3;
        const uint32_t c0 = wrow[cd], c1 = wrow[cd + 1], c2 = wrow[cd + 2], c3 = wrow[cd + 3];
        const uint32_t c4 = cs ? wrow[cd + 4] : 0u;
        const u32x4 wq{funnel_bytes(c1, c0, cs), funnel_bytes(c2, c1, cs), funnel_bytes(c3, c2, cs),
                       funnel_bytes(c4, c3, cs)};
        const float dw = half_bits_to_float((wrow[sb >> 2] >> (8 * (sb & 3))) & 0xffffu);
        const i32x16 dot = __builtin_amdgcn_mfma_i32_32x32x32_i8(
            a, i32x4{int(wq[0]), int(wq[1]), int(wq[2]), int(wq[3])}, zero, 0, 0, 0);
        // element r: activation row 8 (r / 4) + 4 h + r % 4, weight row col
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
            const floatx4 dx = *reinterpret_cast<const floatx4*>(&Xd[b][8 * qd + 4 * h]);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc[4 * qd + i] = __builtin_fmaf(dw * dx[i], float(dot[4 * qd + i]), acc[4 * qd + i]);
        }
    }
    // 4. partial tiles in wave order, per column tile
#pragma unroll
    for (int r = 0; r < 16; ++r) red[(wave * 16 + r) * 64 + lane] = acc[r];
    __syncthreads();
    const int m = tid >> 5, n = tid & 31;
    const int src = (4 * (m >> 3) + (m & 3)) * 64 + n + 32 * ((m >> 2) & 1);
#pragma unroll
    for (int t = 0; t < CT; ++t) {
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < 16 / CT; ++w) v += red[(t * (16 / CT) + w) * 16 * 64 + src];
        const int nn = n0 + 32 * t + n;
        if (m < M && nn < N) {
            if (part) part[(int64_t(sp) * Mall + m0 + m) * N + nn] = v;
            else __builtin_nontemporal_store(v, Y + int64_t(m) * ldy + nn);
        }
    }
}

// ---------------------------------------------------------------------------
// Many activation rows against a small Q8_0 weight (N <= 256, K = 256: the
// fusion encoder's and decoder's image-token projections, M = 5184), exact
// int8 as the strip kernel but shaped for a weight that fits in LDS whole:
//  1. one workgroup per CU, each with an even run of rows (M / grid: 20 or
//     21 of 5184), so every CU streams the same number of activation bytes;
//  2. waves 0-3 load the run's next 32 activation rows (a 32-value block per
//     thread) and pack them to Q8_0 codes and the block's fp16 scale (ggml's
//     from_float, bit-exact); meanwhile waves 4-7 bring 64 weight rows each
//     into LDS by direct-to-LDS loads (1 KB per wave instruction; a row is
//     272 bytes, so a wave's rows are 17 whole KB) and each lane re-lays its
//     row in place: the 32 codes of every block 16-byte aligned (a block is
//     34 bytes, so its codes sit 2 bytes off a dword in the packed row) and
//     the scales as floats, so every MFMA operand is one 16-byte LDS read;
//  3. wave w takes column tile w of 32 weight rows: all 8 blocks'
//     v_mfma_i32_32x32x32_i8 are issued before the first epilogue, then
//     acc = fma(d_w d_x, dot, acc) in K order (ggml's vec_dot_q8_0_q8_0
//     order of the block sums), and the 32x32 tile goes straight from the
//     accumulators to Y (a store covers two 128-byte row segments; stores
//     past the rows or past N are dropped by the bounds of a buffer clipped
//     to the rows).
// Timed with per-wave stamps on MI355X at M = 5184, N = K = 256: 9.7 us per
// launch with 4 waves reading the packed rows and one MFMA at a time, 8.2
// with 8 waves, 6.6 with the weight re-laid by a separate pass.
// ---------------------------------------------------------------------------
constexpr int TS_RB = (kTallSmallK / 32) * 34;          // 272 bytes per packed row
constexpr int TS_XLD = kTallSmallK + 16;                 // bytes per LDS code row
constexpr int TS_NB = kTallSmallK / 32;                  // 8 blocks per row
static_assert(TS_RB % 16 == 0 && 64 * TS_RB % 1024 == 0, "64 packed rows are whole KB of 16-byte aligned rows");

template <bool X86, bool XVEC, int NQD>
__global__ __launch_bounds__(512) void tall_small_i8_kernel(const float* __restrict__ X, int64_t ldx,
                                                            const uint8_t* __restrict__ W, float* __restrict__ Y,
                                                            int64_t ldy, int M, int N) {
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(16))) uint8_t Wl[kTallSmallMaxN * TS_RB];   // packed, then re-laid rows
    __shared__ __attribute__((aligned(16))) float Wd[TS_NB][kTallSmallMaxN];      // weight block scales
    __shared__ __attribute__((aligned(16))) int8_t Xq[32 * TS_XLD];
    __shared__ __attribute__((aligned(16))) float Xd[TS_NB][32];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = gridDim.x, g = blockIdx.x;
    const int r_begin = int(int64_t(M) * g / G), r_end = int(int64_t(M) * (g + 1) / G);
    const int col = lane & 31, h = lane >> 5;
    const int n = wave * 32 + col;          // this lane's weight row in the products
    const int nr = min(n, N - 1);
    for (int rt = r_begin; rt < r_end; rt += 32) {
        const int rows = min(32, r_end - rt);
        if (wave < 4) {
            // activation row qm, block qb -> Q8_0 codes and scale (zeros past the rows)
            const int qm = tid >> 3, qb = tid & 7;
            float v[32];
            if (qm < rows) {
                const float* xr = X + int64_t(rt + qm) * ldx + 32 * qb;
                if (XVEC) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const floatx4 t = load4f(xr + 4 * i);
                        v[4 * i] = t[0];
                        v[4 * i + 1] = t[1];
                        v[4 * i + 2] = t[2];
                        v[4 * i + 3] = t[3];
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 32; ++i) v[i] = xr[i];
                }
            } else {
#pragma unroll
                for (int i = 0; i < 32; ++i) v[i] = 0.f;
            }
            float amax = 0.f;
#pragma unroll
            for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
            const float d = div127(amax);
            float inv;
            if (X86) inv = amax != 0.f ? 127.f / amax : 0.f;
            else inv = d != 0.f ? 1.f / d : 0.f;
            uint32_t packed[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                uint32_t q[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float sv = v[4 * i + j] * inv;
                    q[j] = uint32_t(cvt_i32_nan0(X86 ? __builtin_rintf(sv) : __builtin_roundf(sv)));
                }
                const uint32_t lo = __builtin_amdgcn_perm(q[1], q[0], 0x0c0c0400u);
                const uint32_t hi = __builtin_amdgcn_perm(q[3], q[2], 0x0c0c0400u);
                packed[i] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
            }
            u32x4* dst = reinterpret_cast<u32x4*>(&Xq[qm * TS_XLD + 32 * qb]);
            dst[0] = u32x4{packed[0], packed[1], packed[2], packed[3]};
            dst[1] = u32x4{packed[4], packed[5], packed[6], packed[7]};
            Xd[qb][qm] = half_bits_to_float(float_to_half_bits(d));   // the stored fp16 scale
        } else if (rt == r_begin) {
            // weight rows 64 v .. 64 v + 63 (requests past N rows read as zero)
            const int v = wave - 4, wrow = 64 * v + lane;
            const __amdgpu_buffer_rsrc_t wd =
                __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(W), 0, uint32_t(N * TS_RB), 0x00020000);
#pragma unroll
            for (int c = 0; c < 64 * TS_RB / 1024; ++c)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    wd, (__attribute__((address_space(3))) void*)(Wl + 64 * v * TS_RB + c * 1024), 16,
                    uint32_t(64 * v * TS_RB + c * 1024 + 16 * lane), 0, 0, 0);
            __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's rows have landed
            __builtin_amdgcn_wave_barrier();
            if (wrow < N) {
                // the lane's packed row in registers, then its blocks' codes
                // back 16-byte aligned (block b at byte 32 b) and the scales out
                uint32_t rw[TS_RB / 4 + 1];
#pragma unroll
                for (int i = 0; i < TS_RB / 16; ++i) {
                    const u32x4 t = *reinterpret_cast<const u32x4*>(Wl + wrow * TS_RB + 16 * i);
                    rw[4 * i] = t[0];
                    rw[4 * i + 1] = t[1];
                    rw[4 * i + 2] = t[2];
                    rw[4 * i + 3] = t[3];
                }
                rw[TS_RB / 4] = 0u;
#pragma unroll
                for (int b = 0; b < TS_NB; ++b) {
                    const int sb = 34 * b, cb = sb + 2, cd = cb >> 2, cs = cb & 3;
                    Wd[b][wrow] = half_bits_to_float((rw[sb >> 2] >> (8 * (sb & 3))) & 0xffffu);
                    const u32x4 lo{funnel_bytes(rw[cd + 1], rw[cd], cs), funnel_bytes(rw[cd + 2], rw[cd + 1], cs),
                                   funnel_bytes(rw[cd + 3], rw[cd + 2], cs), funnel_bytes(rw[cd + 4], rw[cd + 3], cs)};
                    const u32x4 hi{funnel_bytes(rw[cd + 5], rw[cd + 4], cs), funnel_bytes(rw[cd + 6], rw[cd + 5], cs),
                                   funnel_bytes(rw[cd + 7], rw[cd + 6], cs), funnel_bytes(rw[cd + 8], rw[cd + 7], cs)};
                    u32x4* dst = reinterpret_cast<u32x4*>(Wl + wrow * TS_RB + 32 * b);
                    dst[0] = lo;
                    dst[1] = hi;
                }
            }
        }
        __syncthreads();
        // column tile `wave` of 32 weight rows against the 32 activation rows
        if (wave * 32 < N) {
            const __amdgpu_buffer_rsrc_t yd = __builtin_amdgcn_make_buffer_rsrc(
                Y + int64_t(rt) * ldy, 0, uint32_t(((rows - 1) * ldy + N) * 4), 0x00020000);
            const i32x16 zero = {0};
            i32x16 dots[TS_NB];
#pragma unroll
            for (int b = 0; b < TS_NB; ++b) {
                const i32x4 a = *reinterpret_cast<const i32x4*>(&Xq[col * TS_XLD + 32 * b + 16 * h]);
                const i32x4 w = *reinterpret_cast<const i32x4*>(Wl + nr * TS_RB + 32 * b + 16 * h);
                dots[b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, w, zero, 0, 0, 0);
            }
            // element r: activation row 8 (r / 4) + 4 h + r % 4, weight row n;
            // the host takes NQD = 3 when no run has more than 24 rows, so the
            // last group of 8 rows is neither scaled nor stored
            floatx16 acc;
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll
            for (int b = 0; b < TS_NB; ++b) {
                const float dw = Wd[b][nr];
#pragma unroll
                for (int qd = 0; qd < NQD; ++qd) {
                    const floatx4 dx = *reinterpret_cast<const floatx4*>(&Xd[b][8 * qd + 4 * h]);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        acc[4 * qd + i] = __builtin_fmaf(dw * dx[i], float(dots[b][4 * qd + i]), acc[4 * qd + i]);
                }
            }
            const uint32_t base = n < N ? uint32_t(4 * h * ldy + n) * 4 : 0x80000000u;
#pragma unroll
            for (int r = 0; r < 4 * NQD; ++r) {
                const float val = acc[r];
                const uint32_t dr = uint32_t(8 * (r >> 2) + (r & 3));
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(val), yd, base + dr * uint32_t(ldy) * 4, 0, 2);
            }
        }
        __syncthreads();   // the codes are read before the next rows overwrite them
    }
}

// ---------------------------------------------------------------------------
// The same shape for K-quant weights (Q4_K, Q5_K, Q6_K; K = 256, one
// super-block per row), with ggml's CPU native arithmetic reproduced
// exactly: each activation row is packed to Q8_K (quantize_row_q8_K, one
// F32 scale d_x), and for weight row n
//   Q4_K, Q5_K:  y = (d d_x) isum - (dmin d_x) msum,
//                isum = sum_j sc_j dot_j,  msum = sum_j m_j xs_j,
//   Q6_K:        y = (d d_x) isum,
//                isum = sum_s sc_s (dot_s - 32 xs_s),
// with the integer sums of vec_dot_q4_K/q5_K/q6_K_q8_K exact in int32
// (dot_j: the codes' dot over sub-block j, v_mfma_i32_32x32x32_i8; xs_j:
// the activation codes' sum over the sub-block; the F32 steps in ggml's
// order), so the result equals the CPU path's.
//  1. waves 4-7 copy the packed weight into LDS (direct-to-LDS loads, each
//     wave the whole KBs that cover its 64 rows) and each lane decodes one
//     row: its codes (0..15, 0..31 or 0..63) 16-byte aligned, its sub-block
//     scales (and Q4_K/Q5_K mins) as int8 rows, d (and dmin) as floats;
//     meanwhile waves 0-3 pack the next 32 activation rows to Q8_K codes,
//     d_x and the sub-block code sums, split as xs = 64 xh + xl (xl in
//     [0, 63], xh in [-64, 63]) so that sum_j m_j xs_j and sum_s sc_s xs_s
//     are two more int8 MFMAs against the mins (scales) as the B operand;
//  2. wave w takes column tile w of 32 weight rows: the sub-block dots,
//     isum by 24-bit integer multiply-adds in sub-block order, then the F32
//     steps and the stores.
// ---------------------------------------------------------------------------
template <int WT>
constexpr int tskq_pack_bytes() { return kTallSmallMaxN * block_bytes(WT) + 1024; }

template <int WT, bool XVEC, int NQD>
__global__ __launch_bounds__(512) void tall_small_kq_i8_kernel(const float* __restrict__ X, int64_t ldx,
                                                               const uint8_t* __restrict__ W, float* __restrict__ Y,
                                                               int64_t ldy, int M, int N) {
#pragma clang fp contract(off)
    constexpr int BB = block_bytes(WT);
    constexpr bool Q6 = WT == T_Q6_K;
    constexpr int NS = Q6 ? 16 : 8;                 // weight sub-blocks per row (16 or 32 values)
    __shared__ __attribute__((aligned(16))) uint8_t Wp[tskq_pack_bytes<WT>()];   // packed rows as stored
    __shared__ __attribute__((aligned(16))) uint8_t Wl[kTallSmallMaxN * TS_XLD]; // codes, 16-byte aligned rows
    __shared__ __attribute__((aligned(16))) int8_t Wsc[kTallSmallMaxN * 32];    // sub-block scales (zero padded)
    __shared__ __attribute__((aligned(16))) int8_t Wm[Q6 ? 16 : kTallSmallMaxN * 32];   // Q4_K/Q5_K mins
    __shared__ __attribute__((aligned(16))) float Wd[kTallSmallMaxN], Wdm[kTallSmallMaxN];
    __shared__ __attribute__((aligned(16))) int8_t Xq[32 * TS_XLD];
    __shared__ __attribute__((aligned(16))) int8_t Xsl[32 * 32], Xsh[32 * 32];
    __shared__ __attribute__((aligned(16))) float Xd[32];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = gridDim.x, g = blockIdx.x;
    const int r_begin = int(int64_t(M) * g / G), r_end = int(int64_t(M) * (g + 1) / G);
    const int col = lane & 31, h = lane >> 5;
    const int n = wave * 32 + col;          // this lane's weight row in the products
    const int nr = min(n, N - 1);
    for (int rt = r_begin; rt < r_end; rt += 32) {
        const int rows = min(32, r_end - rt);
        if (wave < 4) {
            // pass p: activation row 8 p + tid / 32, values 8 li .. 8 li + 7
            // (32 lanes per Q8_K block: the row's 256 values)
            const int li = tid & 31;
            floatx8 v[4];
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const int m = 8 * p + (tid >> 5);
                v[p] = floatx8{0, 0, 0, 0, 0, 0, 0, 0};
                if (m < rows) {
                    const float* xr = X + int64_t(rt + m) * ldx + 8 * li;
                    if (XVEC) {
                        const floatx4 a = load4f(xr), c = load4f(xr + 4);
                        v[p] = floatx8{a[0], a[1], a[2], a[3], c[0], c[1], c[2], c[3]};
                    } else {
#pragma unroll
                        for (int i = 0; i < 8; ++i) v[p][i] = xr[i];
                    }
                }
            }
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const int m = 8 * p + (tid >> 5);
                float d;
                int c[8], sum = 0;
                quant8_icodes<T_Q8_K, false>(v[p], lane, d, c);
#pragma unroll
                for (int i = 0; i < 8; ++i) sum += c[i];
                const uint32_t lo = __builtin_amdgcn_perm(
                    __builtin_amdgcn_perm(uint32_t(c[3]), uint32_t(c[2]), 0x0c0c0400u),
                    __builtin_amdgcn_perm(uint32_t(c[1]), uint32_t(c[0]), 0x0c0c0400u), 0x05040100u);
                const uint32_t hi = __builtin_amdgcn_perm(
                    __builtin_amdgcn_perm(uint32_t(c[7]), uint32_t(c[6]), 0x0c0c0400u),
                    __builtin_amdgcn_perm(uint32_t(c[5]), uint32_t(c[4]), 0x0c0c0400u), 0x05040100u);
                *reinterpret_cast<u32x2*>(&Xq[m * TS_XLD + 8 * li]) = u32x2{lo, hi};
                if (li == 0) Xd[m] = d;
                // code sum of the weight's sub-block: 4 lanes (32 values) or 2 (16)
                const int xs = group_sum<Q6 ? 2 : 4>(sum);
                const int sj = Q6 ? li >> 1 : li >> 2;   // sub-block of this lane
                const int xh = xs >> 6, xl = xs - 64 * xh;
                if ((li & (Q6 ? 1 : 3)) == 0) {
                    Xsl[m * 32 + sj] = int8_t(xl);
                    Xsh[m * 32 + sj] = int8_t(xh);
                }
                if (li >= NS) {   // the K padding of the sum operands
                    Xsl[m * 32 + li] = 0;
                    Xsh[m * 32 + li] = 0;
                }
            }
        } else if (rt == r_begin) {
            // the packed bytes of rows 64 v .. 64 v + 63, whole KBs from the
            // first (requests past the N rows read as zero)
            const int v = wave - 4, wrow = 64 * v + lane;
            constexpr int CH = (64 * BB + 1023) / 1024;
            const __amdgpu_buffer_rsrc_t wd =
                __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(W), 0, uint32_t(N * BB), 0x00020000);
#pragma unroll
            for (int c = 0; c < CH; ++c)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    wd, (__attribute__((address_space(3))) void*)(Wp + 64 * v * BB + c * 1024), 16,
                    uint32_t(64 * v * BB + c * 1024 + 16 * lane), 0, 0, 0);
            __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's rows have landed
            __builtin_amdgcn_wave_barrier();
            if (wrow < N) {
                if constexpr (BB % 16 != 0) {
                    // the buffer's range check zeroes a dword that crosses its
                    // end (N odd for the 210-byte Q6_K rows): the last row
                    // takes its bytes past the last whole 16 from memory
                    if (wrow == N - 1)
                        for (int o = (N * BB) & ~15; o < N * BB; o += 2)
                            *reinterpret_cast<uint16_t*>(Wp + o) = *reinterpret_cast<const uint16_t*>(W + o);
                }
                // the lane's packed row in registers (as dwords from its
                // 2-byte aligned start), then its decode
                const uint8_t* rp = Wp + wrow * BB;
                const uint32_t* rd = reinterpret_cast<const uint32_t*>(rp - (reinterpret_cast<uintptr_t>(rp) & 3));
                const uint32_t sh = uint32_t(reinterpret_cast<uintptr_t>(rp) & 3);
                constexpr int ND = (BB + 3) / 4 + 1;
                uint32_t rw[ND];
#pragma unroll
                for (int i = 0; i < ND; ++i) rw[i] = rd[i];
                auto word = [&](int o) -> uint32_t {   // bytes o .. o + 3 of the row, o a multiple of 4
                    return funnel_bytes(rw[(o >> 2) + 1], rw[o >> 2], (sh + uint32_t(o)) & 3u);
                };
                uint32_t* dst = reinterpret_cast<uint32_t*>(Wl + wrow * TS_XLD);
                if constexpr (Q6) {
                    // value e = 128 hf + 32 gq + l: low = nibble gq / 2 of ql[64 hf + 32 (gq & 1) + l],
                    // high = bits 2 gq of qh[32 hf + l]
#pragma unroll
                    for (int st = 0; st < 8; ++st) {
                        const int hf = st >> 2, gq = st & 3;
#pragma unroll
                        for (int t = 0; t < 8; ++t) {
                            const uint32_t ql = word(64 * hf + 32 * (gq & 1) + 4 * t);
                            const uint32_t qh = word(128 + 32 * hf + 4 * t);
                            dst[8 * st + t] =
                                ((ql >> (4 * (gq >> 1))) & 0x0f0f0f0fu) | (((qh >> (2 * gq)) & 0x03030303u) << 4);
                        }
                    }
                    const uint32_t s0 = word(192), s1 = word(196), s2 = word(200), s3 = word(204);
                    uint32_t* sd = reinterpret_cast<uint32_t*>(Wsc + wrow * 32);
                    sd[0] = s0; sd[1] = s1; sd[2] = s2; sd[3] = s3;
                    sd[4] = sd[5] = sd[6] = sd[7] = 0u;
                    Wd[wrow] = half_bits_to_float(word(208) & 0xffffu);
                } else {
                    // Q4_K: d @0, dmin @2, scales @4, qs @16; Q5_K: qh @16, qs @48
                    constexpr int QS = WT == T_Q5_K ? 48 : 16;
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) {
#pragma unroll
                        for (int t = 0; t < 8; ++t) {
                            uint32_t u = (word(QS + 32 * (jj >> 1) + 4 * t) >> (4 * (jj & 1))) & 0x0f0f0f0fu;
                            if constexpr (WT == T_Q5_K) u |= ((word(16 + 4 * t) >> jj) & 0x01010101u) << 4;
                            dst[8 * jj + t] = u;
                        }
                    }
                    const uint32_t scw[3] = {word(4), word(8), word(12)};
                    uint32_t scp[2] = {0u, 0u}, mnp[2] = {0u, 0u};
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) {
                        int sc, mn;
                        k4_scale_min(jj, scw, sc, mn);
                        scp[jj >> 2] |= uint32_t(sc) << (8 * (jj & 3));
                        mnp[jj >> 2] |= uint32_t(mn) << (8 * (jj & 3));
                    }
                    uint32_t* sd = reinterpret_cast<uint32_t*>(Wsc + wrow * 32);
                    uint32_t* md = reinterpret_cast<uint32_t*>(Wm + wrow * 32);
                    sd[0] = scp[0]; sd[1] = scp[1];
                    md[0] = mnp[0]; md[1] = mnp[1];
#pragma unroll
                    for (int i = 2; i < 8; ++i) sd[i] = md[i] = 0u;
                    const uint32_t hdr = word(0);
                    Wd[wrow] = half_bits_to_float(hdr & 0xffffu);
                    Wdm[wrow] = half_bits_to_float(hdr >> 16);
                }
            }
        }
        __syncthreads();
        // column tile `wave` of 32 weight rows against the 32 activation rows
        if (wave * 32 < N) {
            const __amdgpu_buffer_rsrc_t yd = __builtin_amdgcn_make_buffer_rsrc(
                Y + int64_t(rt) * ldy, 0, uint32_t(((rows - 1) * ldy + N) * 4), 0x00020000);
            const i32x16 zero = {0};
            // this lane's weight row: sub-block scales (unsigned 6-bit, or
            // int8 for Q6_K) in sub-block order
            const i32x4 scv = *reinterpret_cast<const i32x4*>(&Wsc[nr * 32]);
            auto sc_of = [&](int j) -> int {
                const uint32_t b = (uint32_t(scv[j >> 2]) >> (8 * (j & 3))) & 0xffu;
                return Q6 ? int(int8_t(b)) : int(b);
            };
            // the activation code sums against the mins (Q4_K/Q5_K) or the
            // scales (Q6_K): exact, as 64 xh + xl
            const i32x4 bsum_b = *reinterpret_cast<const i32x4*>(Q6 ? &Wsc[nr * 32 + 16 * h] : &Wm[nr * 32 + 16 * h]);
            const i32x16 cl = __builtin_amdgcn_mfma_i32_32x32x32_i8(
                *reinterpret_cast<const i32x4*>(&Xsl[col * 32 + 16 * h]), bsum_b, zero, 0, 0, 0);
            const i32x16 ch = __builtin_amdgcn_mfma_i32_32x32x32_i8(
                *reinterpret_cast<const i32x4*>(&Xsh[col * 32 + 16 * h]), bsum_b, zero, 0, 0, 0);
            i32x16 isum = zero;
            // sub-block dots four steps at a time, isum in sub-block order
#pragma unroll
            for (int q4 = 0; q4 < 2; ++q4) {
                i32x16 dots[4][Q6 ? 2 : 1];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int st = 4 * q4 + k;
                    const i32x4 a = *reinterpret_cast<const i32x4*>(&Xq[col * TS_XLD + 32 * st + 16 * h]);
                    const i32x4 w = *reinterpret_cast<const i32x4*>(&Wl[nr * TS_XLD + 32 * st + 16 * h]);
                    if constexpr (Q6) {
                        // each 16-value half against its own scale: the other
                        // half's weight codes zeroed
#pragma unroll
                        for (int hs = 0; hs < 2; ++hs)
                            dots[k][hs] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, h == hs ? w : i32x4{0, 0, 0, 0}, zero,
                                                                                0, 0, 0);
                    } else {
                        dots[k][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, w, zero, 0, 0, 0);
                    }
                }
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int st = 4 * q4 + k;
#pragma unroll
                    for (int hs = 0; hs < (Q6 ? 2 : 1); ++hs) {
                        const int scj = sc_of(Q6 ? 2 * st + hs : st);
#pragma unroll
                        for (int r = 0; r < 16; ++r) isum[r] = __mul24(scj, dots[k][hs][r]) + isum[r];
                    }
                }
            }
            const float dw = Wd[nr];
            const float dmw = Q6 ? 0.f : Wdm[nr];
            const uint32_t base = n < N ? uint32_t(4 * h * ldy + n) * 4 : 0x80000000u;
            // NQD = 3 (no run past 24 rows): the tile's last 8 rows are not stored
#pragma unroll
            for (int qd = 0; qd < NQD; ++qd) {
                const floatx4 dx = *reinterpret_cast<const floatx4*>(&Xd[8 * qd + 4 * h]);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = 4 * qd + i;
                    const int xsum = __mul24(64, ch[r]) + cl[r];   // sum over sub-blocks of (mins|scales) x code sums
                    float y;
                    if constexpr (Q6) {
                        const int is = isum[r] - 32 * xsum;
                        y = 0.f + (dw * dx[i]) * float(is);
                    } else {
                        y = 0.f + (dw * dx[i]) * float(isum[r]);
                        y = y - (dmw * dx[i]) * float(xsum);
                    }
                    const uint32_t dr = uint32_t(8 * (r >> 2) + (r & 3));
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(y), yd, base + dr * uint32_t(ldy) * 4, 0, 2);
                }
            }
        }
        __syncthreads();   // the codes are read before the next rows overwrite them
    }
}

// ---------------------------------------------------------------------------
// Exact int8 path for the K-quants: Q4_K, Q5_K and Q6_K weights against
// Q8_K activation codes, ggml's CPU native arithmetic (vec_dot_q*_K_q8_K)
// on the matrix cores, with the workgroup shape of the Q8_0 path (16 waves
// per 32 weight rows, 32 activation rows and a K slice of up to 1024 values):
//  1. the strip's packed bytes for the slice go to LDS with coalesced dword
//     loads (rows of an odd dword count);
//  2. each 256-value activation block of the slice is packed to Q8_K by 32
//     lanes of 8 values (ggml's quantize_row_q8_K: the first value of
//     largest magnitude sets iscale = -127 / max); the codes, the block's d
//     and the code sums of every weight sub-block (32 values; 16 for Q6_K)
//     go to LDS;
//  3. wave w takes the slice's 32-value steps w, w + 16, ...: the integer
//     dot of activation codes and the weight's unsigned 4/5/6-bit codes
//     comes out of v_mfma_i32_32x32x32_i8 (for Q6_K once per 16-value half,
//     the other half's weight codes set to zero), then in F32
//       Q4_K, Q5_K: acc += d_x ((d sc_j) dot - (dmin m_j) sum(codes_j))
//       Q6_K:       acc += (d sc) d_x (dot - 32 sum(codes))
//     (the same integer sums ggml forms; only the order of the F32 additions
//     differs);
//  4. the 16 partial tiles are added in LDS in wave order.
// The host picks the slice width (SK super-blocks of 256 values: 1, 2 or 4).
// With more than one slice each workgroup writes its partial sums, which
// splitk_reduce_kernel adds in slice order.  With slices of one super-block
// a workgroup can take 64 weight rows instead (CT = 2, as in the Q8_0
// kernel: wave w takes step w % 8 of column tile w / 8).
// ---------------------------------------------------------------------------
template <int WT>
constexpr int kq_wdw() { return (((kI8SliceK / 256) * block_bytes(WT) + 2 + 3) / 4) | 1; }
template <int WT>
constexpr int kq_wdw1() { return ((block_bytes(WT) + 2 + 3) / 4) | 1; }   // one super-block

template <int WT, bool XVEC, int CT>
__global__ __launch_bounds__(1024) void kq_strip_i8_kernel(const float* __restrict__ X, int64_t ldx,
                                                           const uint8_t* __restrict__ W, int64_t w_stride,
                                                           float* __restrict__ Y, int64_t ldy, float* __restrict__ part,
                                                           int M, int N, int K, int RG, int S, int SK) {
#pragma clang fp contract(off)
    static_assert(CT == 1 || CT == 2, "one or two column tiles");
    constexpr int WDW = CT == 2 ? kq_wdw1<WT>() : kq_wdw<WT>();   // dword pitch of an LDS weight row
    constexpr int TPR = 32 / CT;                                  // threads per weight row in the load
    static_assert(32 * CT * WDW <= 32 * kq_wdw<WT>(), "the weight rows fit the LDS strip");
    constexpr int BB = block_bytes(WT);
    constexpr int SUB = WT == T_Q6_K ? 16 : 32;     // values per weight scale
    constexpr int SPB = 256 / SUB;                  // sub-blocks per super-block
    constexpr int XSB = kI8SliceK / 256;            // super-blocks per full slice
    __shared__ __attribute__((aligned(16))) int8_t Xq[32 * I8_XLD];
    __shared__ __attribute__((aligned(16))) float Xd[XSB][32];
    __shared__ __attribute__((aligned(16))) float Xs[XSB * SPB][32];   // code sums per sub-block and row
    __shared__ __attribute__((aligned(16))) uint32_t Ws[32 * kq_wdw<WT>()];
    __shared__ __attribute__((aligned(16))) float red[16 * 16 * 64];
    constexpr int RI = (WDW + TPR - 1) / TPR;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rg = blockIdx.x % RG, sp = (blockIdx.x / RG) % S, mb = blockIdx.x / (RG * S);
    const int n0 = rg * 32 * CT, k0 = sp * 256 * SK;
    const int nsb = min(256 * SK, K - k0) / 256;    // super-blocks in this slice (SK <= XSB; CT = 2: 1)
    const int m0 = mb * 32, Mall = M;
    X += int64_t(m0) * ldx;
    Y += int64_t(m0) * ldy;
    M = min(M - m0, 32);

    // 1. packed weight bytes: thread (r, c) loads dwords c, c + TPR, ... of row r
    const int wr_r = tid / TPR, wr_c = tid % TPR;
    uint32_t wr[RI];
    {
        const uint8_t* rowp = W + int64_t(min(n0 + wr_r, N - 1)) * w_stride + int64_t(k0 / 256) * BB;
        const uint32_t sh = uint32_t(reinterpret_cast<uintptr_t>(rowp) & 3);
        const uint32_t* src = reinterpret_cast<const uint32_t*>(rowp - sh);
        const int ndw = int((sh + BB * nsb + 3) >> 2);
#pragma unroll
        for (int i = 0; i < RI; ++i) wr[i] = wr_c + TPR * i < ndw ? src[wr_c + TPR * i] : 0u;
    }
    // 2. activation block (row m, super-block b) by the 32 lanes of half hu
    // of a wave, 8 values per lane: unit u = m * nsb + b = 32 pass + 2 wave + hu
    const int hu = lane >> 5, li = lane & 31;
    floatx8 xv[XSB];
#pragma unroll
    for (int p = 0; p < XSB; ++p) {
        xv[p] = floatx8{0, 0, 0, 0, 0, 0, 0, 0};
        if (p < nsb) {
            const int u = 32 * p + 2 * wave + hu, m = u / nsb, b = u - m * nsb;
            if (m < M) {
                const float* xr = X + int64_t(m) * ldx + k0 + 256 * b + 8 * li;
                if (XVEC) {
                    const floatx4 lo = load4f(xr), hi = load4f(xr + 4);
                    xv[p] = floatx8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                } else {
#pragma unroll
                    for (int i = 0; i < 8; ++i) xv[p][i] = xr[i];
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < RI; ++i)
        if (wr_c + TPR * i < WDW) Ws[wr_r * WDW + wr_c + TPR * i] = wr[i];
#pragma unroll
    for (int p = 0; p < XSB; ++p) {
        if (p >= nsb) break;
        const int u = 32 * p + 2 * wave + hu, m = u / nsb, b = u - m * nsb;
        float d;
        int c[8], sum = 0;
        quant8_icodes<T_Q8_K, false>(xv[p], lane, d, c);
#pragma unroll
        for (int i = 0; i < 8; ++i) sum += c[i];
        const uint32_t lo = __builtin_amdgcn_perm(__builtin_amdgcn_perm(uint32_t(c[3]), uint32_t(c[2]), 0x0c0c0400u),
                                                  __builtin_amdgcn_perm(uint32_t(c[1]), uint32_t(c[0]), 0x0c0c0400u),
                                                  0x05040100u);
        const uint32_t hi = __builtin_amdgcn_perm(__builtin_amdgcn_perm(uint32_t(c[7]), uint32_t(c[6]), 0x0c0c0400u),
                                                  __builtin_amdgcn_perm(uint32_t(c[5]), uint32_t(c[4]), 0x0c0c0400u),
                                                  0x05040100u);
        *reinterpret_cast<uint2*>(&Xq[m * I8_XLD + 256 * b + 8 * li]) = uint2{lo, hi};
        if (li == 0) Xd[b][m] = d;
        // code sums of the weight's sub-blocks: 4 lanes (Q4_K, Q5_K) or 2 (Q6_K)
        sum = group_sum<SUB / 8>(sum);
        if (li % (SUB / 8) == 0) Xs[b * SPB + li / (SUB / 8)][m] = float(sum);
    }
    __syncthreads();

    // 3. this wave's 32-value steps (CT = 2: step wave % 8 of column tile
    // wave / 8); the activation rows of element r are 8 (r / 4) + 4 h + r % 4,
    // the weight row is the tile's row col
    const int col = lane & 31, h = lane >> 5;
    const int tile = CT == 2 ? wave >> 3 : 0;
    const int wshift = int((reinterpret_cast<uintptr_t>(W + int64_t(min(n0 + 32 * tile + col, N - 1)) * w_stride) +
                            (k0 / 256) * BB) &
                           3);
    const LdsRow wrow{&Ws[(32 * tile + col) * WDW], wshift};
    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
    const i32x16 zero = {0};
    const int nst = 8 * nsb;   // 32-value steps in the slice
    for (int st = CT == 2 ? wave & 7 : wave; st < nst; st += 16 / CT) {
        const int b = st >> 3, jj = st & 7;
        const i32x4 a = *reinterpret_cast<const i32x4*>(&Xq[col * I8_XLD + 32 * st + 16 * h]);
        floatx4 dx[4];
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) dx[qd] = *reinterpret_cast<const floatx4*>(&Xd[b][8 * qd + 4 * h]);
        WeightPiece<WT> wp;
        wp.load(wrow, st, h);
        if constexpr (WT == T_Q6_K) {
            // u = low 4 | high 2 << 4 in [0, 63]; value = d sc (u - 32)
            const int g = jj & 3;
            const int lshift = (g >> 1) * 4, hshift = 2 * g;
            u32x4 u;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                u[i] = ((wp.ql[i] >> lshift) & 0x0f0f0f0fu) | (((wp.qh[i] >> hshift) & 0x03030303u) << 4);
            const float d = half_bits_to_float(wp.d);
            // the two 16-value halves' scales of this weight row
            const int sbase = BB * b + 192 + 8 * (jj >> 2) + 2 * g;
            const float t0 = d * float(int8_t(wrow.u8(sbase))), t1 = d * float(int8_t(wrow.u8(sbase + 1)));
#pragma unroll
            for (int hs = 0; hs < 2; ++hs) {
                const i32x4 bq = h == hs ? i32x4{int(u[0]), int(u[1]), int(u[2]), int(u[3])} : i32x4{0, 0, 0, 0};
                const i32x16 dot = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bq, zero, 0, 0, 0);
                const float t = hs ? t1 : t0;
#pragma unroll
                for (int qd = 0; qd < 4; ++qd) {
                    const floatx4 cs = *reinterpret_cast<const floatx4*>(&Xs[2 * st + hs][8 * qd + 4 * h]);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float v = float(dot[4 * qd + i]) - 32.f * cs[i];   // exact integers
                        acc[4 * qd + i] = __builtin_fmaf(t * dx[qd][i], v, acc[4 * qd + i]);
                    }
                }
            }
        } else {
            const int shift = (jj & 1) * 4;
            u32x4 u;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                u[i] = (wp.qs[i] >> shift) & 0x0f0f0f0fu;
                if constexpr (WT == T_Q5_K) u[i] |= ((wp.qh[i] >> jj) & 0x01010101u) << 4;
            }
            int sc, mn;
            k4_scale_min(jj, wp.sc, sc, mn);
            const float ws = half_bits_to_float(wp.hdr & 0xffffu) * float(sc);
            const float wm = half_bits_to_float(wp.hdr >> 16) * float(mn);
            const i32x16 dot = __builtin_amdgcn_mfma_i32_32x32x32_i8(
                a, i32x4{int(u[0]), int(u[1]), int(u[2]), int(u[3])}, zero, 0, 0, 0);
            // acc += d_x (ws dot - wm csum): four VALU operations per element
#pragma unroll
            for (int qd = 0; qd < 4; ++qd) {
                const floatx4 cs = *reinterpret_cast<const floatx4*>(&Xs[st][8 * qd + 4 * h]);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float t = __builtin_fmaf(-wm, cs[i], ws * float(dot[4 * qd + i]));
                    acc[4 * qd + i] = __builtin_fmaf(dx[qd][i], t, acc[4 * qd + i]);
                }
            }
        }
    }
    // 4. partial tiles in wave order, per column tile
#pragma unroll
    for (int r = 0; r < 16; ++r) red[(wave * 16 + r) * 64 + lane] = acc[r];
    __syncthreads();
    const int m = tid >> 5, n = tid & 31;
    const int src = (4 * (m >> 3) + (m & 3)) * 64 + n + 32 * ((m >> 2) & 1);
#pragma unroll
    for (int t = 0; t < CT; ++t) {
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < 16 / CT; ++w) v += red[(t * (16 / CT) + w) * 16 * 64 + src];
        const int nn = n0 + 32 * t + n;
        if (m < M && nn < N) {
            if (part) part[(int64_t(sp) * Mall + m0 + m) * N + nn] = v;
            else __builtin_nontemporal_store(v, Y + int64_t(m) * ldy + nn);
        }
    }
}

template <int WT, bool XVEC, int CT>
__global__ __launch_bounds__(1024) void kq_strip_isum_kernel(const float* __restrict__ X, int64_t ldx,
                                                           const uint8_t* __restrict__ W, int64_t w_stride,
                                                           float* __restrict__ Y, int64_t ldy, float* __restrict__ part,
                                                           int M, int N, int K, int RG, int S, int SK) {
#pragma clang fp contract(off)
    static_assert(CT == 1 || CT == 2, "one or two column tiles");
    constexpr int WDW = CT == 2 ? kq_wdw1<WT>() : kq_wdw<WT>();   // dword pitch of an LDS weight row
    constexpr int TPR = 32 / CT;                                  // threads per weight row in the load
    static_assert(32 * CT * WDW <= 32 * kq_wdw<WT>(), "the weight rows fit the LDS strip");
    constexpr int BB = block_bytes(WT);
    constexpr int SUB = WT == T_Q6_K ? 16 : 32;     // values per weight scale
    constexpr int SPB = 256 / SUB;                  // sub-blocks per super-block
    constexpr int XSB = kI8SliceK / 256;            // super-blocks per full slice
    __shared__ __attribute__((aligned(16))) int8_t Xq[32 * I8_XLD];
    __shared__ __attribute__((aligned(16))) float Xd[XSB][32];
    // code sums per (super-block, row, sub-block) as xs = 64 xh + xl, the
    // K axis of the sum products padded to 32 with zeros
    __shared__ __attribute__((aligned(16))) int8_t Xsl[XSB][32][32], Xsh[XSB][32][32];
    __shared__ __attribute__((aligned(16))) uint32_t Ws[32 * kq_wdw<WT>()];
    __shared__ __attribute__((aligned(16))) int red[16 * 16 * 64];           // integer partial tiles
    __shared__ __attribute__((aligned(16))) int Mst[XSB][16 * 64];           // sum products per super-block
    __shared__ __attribute__((aligned(16))) float Dw[XSB][32], Dmw[XSB][32]; // d, dmin per weight row
    constexpr int RI = (WDW + TPR - 1) / TPR;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rg = blockIdx.x % RG, sp = (blockIdx.x / RG) % S, mb = blockIdx.x / (RG * S);
    const int n0 = rg * 32 * CT, k0 = sp * 256 * SK;
    const int nsb = min(256 * SK, K - k0) / 256;    // super-blocks in this slice (SK <= XSB; CT = 2: 1)
    const int m0 = mb * 32, Mall = M;
    X += int64_t(m0) * ldx;
    Y += int64_t(m0) * ldy;
    M = min(M - m0, 32);

    // 1. packed weight bytes: thread (r, c) loads dwords c, c + TPR, ... of row r
    const int wr_r = tid / TPR, wr_c = tid % TPR;
    uint32_t wr[RI];
    {
        const uint8_t* rowp = W + int64_t(min(n0 + wr_r, N - 1)) * w_stride + int64_t(k0 / 256) * BB;
        const uint32_t sh = uint32_t(reinterpret_cast<uintptr_t>(rowp) & 3);
        const uint32_t* src = reinterpret_cast<const uint32_t*>(rowp - sh);
        const int ndw = int((sh + BB * nsb + 3) >> 2);
#pragma unroll
        for (int i = 0; i < RI; ++i) wr[i] = wr_c + TPR * i < ndw ? src[wr_c + TPR * i] : 0u;
    }
    // 2. activation block (row m, super-block b) by the 32 lanes of half hu
    // of a wave, 8 values per lane: unit u = m * nsb + b = 32 pass + 2 wave + hu
    const int hu = lane >> 5, li = lane & 31;
    floatx8 xv[XSB];
#pragma unroll
    for (int p = 0; p < XSB; ++p) {
        xv[p] = floatx8{0, 0, 0, 0, 0, 0, 0, 0};
        if (p < nsb) {
            const int u = 32 * p + 2 * wave + hu, m = u / nsb, b = u - m * nsb;
            if (m < M) {
                const float* xr = X + int64_t(m) * ldx + k0 + 256 * b + 8 * li;
                if (XVEC) {
                    const floatx4 lo = load4f(xr), hi = load4f(xr + 4);
                    xv[p] = floatx8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                } else {
#pragma unroll
                    for (int i = 0; i < 8; ++i) xv[p][i] = xr[i];
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < RI; ++i)
        if (wr_c + TPR * i < WDW) Ws[wr_r * WDW + wr_c + TPR * i] = wr[i];
#pragma unroll
    for (int p = 0; p < XSB; ++p) {
        if (p >= nsb) break;
        const int u = 32 * p + 2 * wave + hu, m = u / nsb, b = u - m * nsb;
        float d;
        int c[8], sum = 0;
        quant8_icodes<T_Q8_K, false>(xv[p], lane, d, c);
#pragma unroll
        for (int i = 0; i < 8; ++i) sum += c[i];
        const uint32_t lo = __builtin_amdgcn_perm(__builtin_amdgcn_perm(uint32_t(c[3]), uint32_t(c[2]), 0x0c0c0400u),
                                                  __builtin_amdgcn_perm(uint32_t(c[1]), uint32_t(c[0]), 0x0c0c0400u),
                                                  0x05040100u);
        const uint32_t hi = __builtin_amdgcn_perm(__builtin_amdgcn_perm(uint32_t(c[7]), uint32_t(c[6]), 0x0c0c0400u),
                                                  __builtin_amdgcn_perm(uint32_t(c[5]), uint32_t(c[4]), 0x0c0c0400u),
                                                  0x05040100u);
        *reinterpret_cast<uint2*>(&Xq[m * I8_XLD + 256 * b + 8 * li]) = uint2{lo, hi};
        if (li == 0) Xd[b][m] = d;
        // code sums of the weight's sub-blocks: 4 lanes (Q4_K, Q5_K) or 2 (Q6_K)
        const int xs = group_sum<SUB / 8>(sum);
        const int xh = xs >> 6, xl = xs - 64 * xh;   // xl in [0, 63], xh in [-64, 63]
        if (li % (SUB / 8) == 0) {
            Xsl[b][m][li / (SUB / 8)] = int8_t(xl);
            Xsh[b][m][li / (SUB / 8)] = int8_t(xh);
        }
        if (li >= SPB) {   // the K padding
            Xsl[b][m][li] = 0;
            Xsh[b][m][li] = 0;
        }
    }
    __syncthreads();

    // 3. wave w takes steps st0 .. st0 + spw - 1 of one super-block (CT = 2:
    // step w % 8 of column tile w / 8) and sums sc_j dot_j in integers; the
    // wave that takes a super-block's first step also forms that super-block's
    // sum products sum_j c_j xs_j (c_j the mins, Q6_K the scales) by two int8
    // MFMAs, and its d (and dmin); the activation rows of element r are
    // 8 (r / 4) + 4 h + r % 4, the weight row is the tile's row col
    const int col = lane & 31, h = lane >> 5;
    const int tile = CT == 2 ? wave >> 3 : 0;
    const int wt = CT == 2 ? wave & 7 : wave;            // wave within its column tile
    const int nst = 8 * nsb;                             // 32-value steps in the slice
    const int spw = CT == 2 ? 1 : (nst + 15) / 16;       // steps per wave: 1 or 2 (a divisor of 8)
    const int st0 = wt * spw;
    const int wshift = int((reinterpret_cast<uintptr_t>(W + int64_t(min(n0 + 32 * tile + col, N - 1)) * w_stride) +
                            (k0 / 256) * BB) &
                           3);
    const LdsRow wrow{&Ws[(32 * tile + col) * WDW], wshift};
    const i32x16 zero = {0};
    i32x16 isum = zero;
    if (st0 < nst) {
        for (int st = st0; st < st0 + spw; ++st) {
            const int b = st >> 3, jj = st & 7;
            const i32x4 a = *reinterpret_cast<const i32x4*>(&Xq[col * I8_XLD + 32 * st + 16 * h]);
            WeightPiece<WT> wp;
            wp.load(wrow, st, h);
            if constexpr (WT == T_Q6_K) {
                // unsigned codes u = low 4 | high 2 << 4 in [0, 63]; value u - 32
                const int g = jj & 3;
                const int lshift = (g >> 1) * 4, hshift = 2 * g;
                u32x4 u;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    u[i] = ((wp.ql[i] >> lshift) & 0x0f0f0f0fu) | (((wp.qh[i] >> hshift) & 0x03030303u) << 4);
                const int sbase = BB * b + 192 + 8 * (jj >> 2) + 2 * g;
#pragma unroll
                for (int hs = 0; hs < 2; ++hs) {
                    const i32x4 bq = h == hs ? i32x4{int(u[0]), int(u[1]), int(u[2]), int(u[3])} : i32x4{0, 0, 0, 0};
                    const i32x16 dot = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bq, zero, 0, 0, 0);
                    const int sc = int(int8_t(wrow.u8(sbase + hs)));
#pragma unroll
                    for (int r = 0; r < 16; ++r) isum[r] = __mul24(sc, dot[r]) + isum[r];
                }
            } else {
                const int shift = (jj & 1) * 4;
                u32x4 u;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    u[i] = (wp.qs[i] >> shift) & 0x0f0f0f0fu;
                    if constexpr (WT == T_Q5_K) u[i] |= ((wp.qh[i] >> jj) & 0x01010101u) << 4;
                }
                int sc, mn;
                k4_scale_min(jj, wp.sc, sc, mn);
                const i32x16 dot = __builtin_amdgcn_mfma_i32_32x32x32_i8(
                    a, i32x4{int(u[0]), int(u[1]), int(u[2]), int(u[3])}, zero, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 16; ++r) isum[r] = __mul24(sc, dot[r]) + isum[r];
            }
        }
        if ((st0 & 7) == 0) {
            // this super-block's sum products for the tile and its d (dmin)
            const int b = st0 >> 3, slot = CT == 2 ? tile : b;
            uint32_t c0 = 0u, c1 = 0u, c2 = 0u, c3 = 0u;   // c_j as int8, j = 0 .. SPB - 1 (lanes h = 0)
            float dw, dmw = 0.f;
            if constexpr (WT == T_Q6_K) {
                const u32x4 scs = wrow.u128(BB * b + 192);
                c0 = scs[0]; c1 = scs[1]; c2 = scs[2]; c3 = scs[3];
                dw = half_bits_to_float(wrow.u16(BB * b + 208));
            } else {
                const uint32_t scw[3] = {wrow.u32(BB * b + 4), wrow.u32(BB * b + 8), wrow.u32(BB * b + 12)};
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    int sc, mn;
                    k4_scale_min(j, scw, sc, mn);
                    if (j < 4) c0 |= uint32_t(mn) << (8 * j);
                    else c1 |= uint32_t(mn) << (8 * (j - 4));
                }
                const uint32_t hdr = wrow.u32(BB * b);
                dw = half_bits_to_float(hdr & 0xffffu);
                dmw = half_bits_to_float(hdr >> 16);
            }
            const i32x4 cb = h == 0 ? i32x4{int(c0), int(c1), int(c2), int(c3)} : i32x4{0, 0, 0, 0};
            const i32x16 ml = __builtin_amdgcn_mfma_i32_32x32x32_i8(
                *reinterpret_cast<const i32x4*>(&Xsl[b][col][16 * h]), cb, zero, 0, 0, 0);
            const i32x16 mh = __builtin_amdgcn_mfma_i32_32x32x32_i8(
                *reinterpret_cast<const i32x4*>(&Xsh[b][col][16 * h]), cb, zero, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 16; ++r) Mst[slot][r * 64 + lane] = __mul24(64, mh[r]) + ml[r];
            if (h == 0) {
                Dw[slot][col] = dw;
                Dmw[slot][col] = dmw;
            }
        }
    }
    // 4. per column tile and super-block (in K order): the waves' integer
    // partials added, then ggml's F32 steps
    //   Q4_K, Q5_K: y += (d d_x) isum;  y -= (dmin d_x) msum
    //   Q6_K:       y += (d d_x) (isum - 32 sum_s sc_s xs_s)
#pragma unroll
    for (int r = 0; r < 16; ++r) red[(wave * 16 + r) * 64 + lane] = isum[r];
    __syncthreads();
    const int m = tid >> 5, n = tid & 31;
    const int src = (4 * (m >> 3) + (m & 3)) * 64 + n + 32 * ((m >> 2) & 1);
    const int wpb = 8 / spw;   // waves per super-block
#pragma unroll
    for (int t = 0; t < CT; ++t) {
        float v = 0.f;
        for (int b = 0; b < nsb; ++b) {
            const int slot = CT == 2 ? t : b, w0 = CT == 2 ? 8 * t : b * wpb;
            int is = 0;
            for (int w = 0; w < wpb; ++w) is += red[((w0 + w) * 16) * 64 + src];
            const int ms = Mst[slot][src];
            const float dx = Xd[b][m];
            if constexpr (WT == T_Q6_K) {
                v = v + (Dw[slot][n] * dx) * float(is - 32 * ms);
            } else {
                v = v + (Dw[slot][n] * dx) * float(is);
                v = v - (Dmw[slot][n] * dx) * float(ms);
            }
        }
        const int nn = n0 + 32 * t + n;
        if (m < M && nn < N) {
            if (part) part[(int64_t(sp) * Mall + m0 + m) * N + nn] = v;
            else __builtin_nontemporal_store(v, Y + int64_t(m) * ldy + nn);
        }
    }
}

template <int WT, int MODE, bool X86>
void launch_strip_mode(bool xvec, const float* x, int64_t ldx, const uint8_t* w, int64_t w_stride, float* y,
                       int64_t ldy, float* part, int M, int N, int K, int RG, int S, hipStream_t stream) {
    const dim3 grid(unsigned(RG * S * ((M + 31) / 32))), block(1024);
    if (xvec)
        hipLaunchKernelGGL((strip_skinny_kernel<WT, MODE, X86, true>), grid, block, 0, stream, x, ldx, w, w_stride, y,
                           ldy, part, M, N, K, RG, S);
    else
        hipLaunchKernelGGL((strip_skinny_kernel<WT, MODE, X86, false>), grid, block, 0, stream, x, ldx, w, w_stride,
                           y, ldy, part, M, N, K, RG, S);
}

template <int WT>
void launch_strip_wt(bool f16, int x86, bool xvec, const float* x, int64_t ldx, const uint8_t* w, int64_t w_stride,
                     float* y, int64_t ldy, float* part, int M, int N, int K, int RG, int S, hipStream_t stream) {
    constexpr int Q = WT == T_Q8_0 ? T_Q8_0 : T_Q8_K;
    if (f16)
        launch_strip_mode<WT, T_F16, false>(xvec, x, ldx, w, w_stride, y, ldy, part, M, N, K, RG, S, stream);
    else if (Q == T_Q8_0 && x86)
        launch_strip_mode<WT, Q, true>(xvec, x, ldx, w, w_stride, y, ldy, part, M, N, K, RG, S, stream);
    else
        launch_strip_mode<WT, Q, false>(xvec, x, ldx, w, w_stride, y, ldy, part, M, N, K, RG, S, stream);
}

template <int WT, int MODE, bool X86, int MT>
void launch_fused_mt(const float* x, int64_t ldx, bool xvec, const uint8_t* w, int64_t w_stride, float* y,
                     int64_t ldy, float* part, int M, int N, int K, int RG, int S, int cps, int x86,
                     hipStream_t stream) {
    const int MB = (M + MT * 32 - 1) / (MT * 32);
    const dim3 grid(unsigned(RG * S * MB)), block(512);
    if (xvec)
        hipLaunchKernelGGL((fused_skinny_kernel<WT, MODE, X86, MT, true>), grid, block, 0, stream, x, ldx, w, w_stride,
                           y, ldy, part, M, N, K, RG, S, cps);
    else
        hipLaunchKernelGGL((fused_skinny_kernel<WT, MODE, X86, MT, false>), grid, block, 0, stream, x, ldx, w, w_stride,
                           y, ldy, part, M, N, K, RG, S, cps);
}

template <int WT, int MODE, bool X86>
void launch_fused_mode(const float* x, int64_t ldx, bool xvec, const uint8_t* w, int64_t w_stride, float* y,
                       int64_t ldy, float* part, int M, int N, int K, int RG, int S, int cps, int MT, int x86,
                       hipStream_t stream) {
    switch (MT) {
        case 1: launch_fused_mt<WT, MODE, X86, 1>(x, ldx, xvec, w, w_stride, y, ldy, part, M, N, K, RG, S, cps, x86, stream); break;
        case 2: launch_fused_mt<WT, MODE, X86, 2>(x, ldx, xvec, w, w_stride, y, ldy, part, M, N, K, RG, S, cps, x86, stream); break;
        case 3: launch_fused_mt<WT, MODE, X86, 3>(x, ldx, xvec, w, w_stride, y, ldy, part, M, N, K, RG, S, cps, x86, stream); break;
        default: launch_fused_mt<WT, MODE, X86, 4>(x, ldx, xvec, w, w_stride, y, ldy, part, M, N, K, RG, S, cps, x86, stream); break;
    }
}

template <int WT>
void launch_fused_wt(bool f16, const float* x, int64_t ldx, bool xvec, const uint8_t* w, int64_t w_stride, float* y,
                     int64_t ldy, float* part, int M, int N, int K, int RG, int S, int cps, int MT, int x86,
                     hipStream_t stream) {
    constexpr int Q = WT == T_Q8_0 ? T_Q8_0 : T_Q8_K;
    if (f16)
        launch_fused_mode<WT, T_F16, false>(x, ldx, xvec, w, w_stride, y, ldy, part, M, N, K, RG, S, cps, MT, x86, stream);
    else if (Q == T_Q8_0 && x86)
        launch_fused_mode<WT, Q, true>(x, ldx, xvec, w, w_stride, y, ldy, part, M, N, K, RG, S, cps, MT, x86, stream);
    else
        launch_fused_mode<WT, Q, false>(x, ldx, xvec, w, w_stride, y, ldy, part, M, N, K, RG, S, cps, MT, x86, stream);
}

}  // namespace

const char* skinny_variant(int wtype, int M, int N) {
    const bool wide = (N + ROWS - 1) / ROWS < 256;
    static const char* names[4][2] = {
        {"skinny_f16mfma_q8_0", "skinny_f16mfma_q8_0_wide"},
        {"skinny_f16mfma_q4_k", "skinny_f16mfma_q4_k_wide"},
        {"skinny_f16mfma_q5_k", "skinny_f16mfma_q5_k_wide"},
        {"skinny_f16mfma_q6_k", "skinny_f16mfma_q6_k_wide"},
    };
    (void)M;
    switch (wtype) {
        case T_Q8_0: return names[0][wide];
        case T_Q4_K: return names[1][wide];
        case T_Q5_K: return names[2][wide];
        case T_Q6_K: return names[3][wide];
        default: return nullptr;
    }
}

const char* launch_skinny(int wtype, const _Float16* a, int64_t lda, const float* row_scale, const void* w,
                          int64_t w_stride, float* y, int64_t ldy, int M, int N, int K, hipStream_t stream) {
    if (M < 1 || M > kSkinnyMaxM || N < 1 || K < 32 || K % 32) return nullptr;
    const bool wide = (N + ROWS - 1) / ROWS < 256;
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    switch (wtype) {
        case T_Q8_0: launch_wt<T_Q8_0>(a, lda, row_scale, wb, w_stride, y, ldy, M, N, K, wide, stream); break;
        case T_Q4_K: launch_wt<T_Q4_K>(a, lda, row_scale, wb, w_stride, y, ldy, M, N, K, wide, stream); break;
        case T_Q5_K: launch_wt<T_Q5_K>(a, lda, row_scale, wb, w_stride, y, ldy, M, N, K, wide, stream); break;
        case T_Q6_K: launch_wt<T_Q6_K>(a, lda, row_scale, wb, w_stride, y, ldy, M, N, K, wide, stream); break;
        default: return nullptr;
    }
    return skinny_variant(wtype, M, N);
}

}  // namespace samhip

namespace samhip {

FusedPlan fused_skinny_plan(int M, int N, int K, int max_splits, int cus) {
    FusedPlan p{};
    p.rg = (N + FROWS - 1) / FROWS;
    const int round_wgs = std::max(1, cus);   // one round: a workgroup per CU
    // rows per block: the fewest (32, 64, 96 or 128) whose (row group, row
    // block) grid still fits one round of workgroups, so the
    // activation chunk is packed by as few workgroups as possible without a
    // second round.  Measured on MI355X against the earlier rule (64 or 256
    // workgroups wanted): the detector's 5184 image tokens on 256 x 256
    // weights 9.3 us with 64-row blocks (162 workgroups) instead of 11.0
    // with 32-row blocks (324: two rounds); its 201 queries on 2048 x 256
    // weights 6.4 us with 32-row blocks (112) instead of 8.6 with 64 (64).
    const int max_mt = std::min(4, (M + 31) / 32);
    p.mt = 1;
    while (p.mt < max_mt && int64_t(p.rg) * ((M + 32 * p.mt - 1) / (32 * p.mt)) > round_wgs)
        p.mt = std::min(2 * p.mt, max_mt);
    const int mb = (M + 32 * p.mt - 1) / (32 * p.mt);
    const int groups = p.rg * mb;
    const int nchunks = (K + CHUNK - 1) / CHUNK;
    const int S = std::min(std::min(nchunks, std::max(1, max_splits)),
                           std::max(1, (round_wgs + groups - 1) / groups));
    p.cps = (nchunks + S - 1) / S;
    p.splits = (nchunks + p.cps - 1) / p.cps;
    p.part_bytes = p.splits > 1 ? size_t(p.splits) * size_t(M) * size_t(N) * 4 : 0;
    return p;
}

FusedPlan strip_skinny_plan(int M, int N, int K) {
    FusedPlan p{};
    p.rg = (N + 31) / 32;
    const int nchunks = (K + 255) / 256;
    p.cps = 4;
    p.splits = (nchunks + 3) / 4;
    p.part_bytes = p.splits > 1 ? size_t(p.splits) * size_t(M) * size_t(N) * 4 : 0;
    (void)M;
    return p;
}

const char* strip_skinny_variant(int wtype) {
    switch (wtype) {
        case T_Q8_0: return "skinny_strip_q8_0";
        case T_Q4_K: return "skinny_strip_q4_k";
        case T_Q5_K: return "skinny_strip_q5_k";
        case T_Q6_K: return "skinny_strip_q6_k";
        default: return nullptr;
    }
}

const char* launch_strip_skinny(int wtype, bool f16, const float* x, int64_t ldx, const void* w, int64_t w_stride,
                                float* y, int64_t ldy, float* part, int M, int N, int K, int x86, hipStream_t stream) {
    if (M < 1 || M >= kStripMaxM || N < 1 || K < 32 || K % 32) return nullptr;
    const FusedPlan p = strip_skinny_plan(M, N, K);
    const bool xvec = reinterpret_cast<uintptr_t>(x) % 16 == 0 && ldx % 4 == 0;
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    float* pt = p.splits > 1 ? part : nullptr;
    switch (wtype) {
        case T_Q8_0: launch_strip_wt<T_Q8_0>(f16, x86, xvec, x, ldx, wb, w_stride, y, ldy, pt, M, N, K, p.rg, p.splits, stream); break;
        case T_Q4_K: launch_strip_wt<T_Q4_K>(f16, x86, xvec, x, ldx, wb, w_stride, y, ldy, pt, M, N, K, p.rg, p.splits, stream); break;
        case T_Q5_K: launch_strip_wt<T_Q5_K>(f16, x86, xvec, x, ldx, wb, w_stride, y, ldy, pt, M, N, K, p.rg, p.splits, stream); break;
        case T_Q6_K: launch_strip_wt<T_Q6_K>(f16, x86, xvec, x, ldx, wb, w_stride, y, ldy, pt, M, N, K, p.rg, p.splits, stream); break;
        default: return nullptr;
    }
    if (p.splits > 1) {
        const int64_t outs = int64_t(M) * N;
        hipLaunchKernelGGL(splitk_reduce_kernel, dim3(unsigned((outs + 255) / 256)), dim3(256), 0, stream, part, y, ldy,
                           M, N, p.splits);
    }
    return strip_skinny_variant(wtype);
}

const char* q8_strip_i8_variant() { return "skinny_i8mfma_q8_0"; }

const char* launch_q8_strip_i8(const float* x, int64_t ldx, const void* w, int64_t w_stride, float* y, int64_t ldy,
                               float* part, int M, int N, int K, int slice_sb, int x86, bool two_tiles,
                               hipStream_t stream) {
    if (M < 1 || N < 1 || K < 32 || K % 32) return nullptr;
    if (slice_sb != 1 && slice_sb != 2 && slice_sb != kI8SliceK / 256) return nullptr;
    const int SL = 256 * slice_sb;
    // two column tiles per workgroup when a slice holds at most 256 values
    const int CT = (SL == 256 || K <= 256) && two_tiles ? 2 : 1;
    const int RG = (N + 32 * CT - 1) / (32 * CT), S = (K + SL - 1) / SL, MB = (M + 31) / 32;
    if (S > 1 && !part) return nullptr;
    if (int64_t(RG) * S * MB > kMaxWorkgroups1024) return nullptr;
    const bool xvec = reinterpret_cast<uintptr_t>(x) % 16 == 0 && ldx % 4 == 0;
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    float* pt = S > 1 ? part : nullptr;
    const dim3 grid(unsigned(RG * S * MB)), block(1024);
#define SAMHIP_I8(X86V, XV, CTV)                                                                                   \
    hipLaunchKernelGGL((q8_strip_i8_kernel<X86V, XV, CTV>), grid, block, 0, stream, x, ldx, wb, w_stride, y, ldy, pt, \
                       M, N, K, RG, S, SL)
#define SAMHIP_I8_CT(X86V, XV)                              \
    do {                                                    \
        if (CT == 2) SAMHIP_I8(X86V, XV, 2);                \
        else SAMHIP_I8(X86V, XV, 1);                        \
    } while (0)
    if (x86) {
        if (xvec) SAMHIP_I8_CT(true, true); else SAMHIP_I8_CT(true, false);
    } else {
        if (xvec) SAMHIP_I8_CT(false, true); else SAMHIP_I8_CT(false, false);
    }
#undef SAMHIP_I8_CT
#undef SAMHIP_I8
    if (S > 1) {
        const int64_t outs = int64_t(M) * N;
        hipLaunchKernelGGL(splitk_reduce_kernel, dim3(unsigned((outs + 255) / 256)), dim3(256), 0, stream, part, y, ldy,
                           M, N, S);
    }
    return q8_strip_i8_variant();
}

const char* kq_strip_i8_variant(int wtype) {
    switch (wtype) {
        case T_Q4_K: return "skinny_i8mfma_q4_k";
        case T_Q5_K: return "skinny_i8mfma_q5_k";
        case T_Q6_K: return "skinny_i8mfma_q6_k";
        default: return nullptr;
    }
}

template <int WT>
void launch_kq_strip_wt(bool xvec, int CT, bool isum, const float* x, int64_t ldx, const uint8_t* w, int64_t w_stride,
                        float* y, int64_t ldy, float* part, int M, int N, int K, int RG, int S, int MB, int SK,
                        hipStream_t stream) {
    const dim3 grid(unsigned(RG * S * MB)), block(1024);
#define SAMHIP_KQ(KERN, XV, CTV)                                                                              \
    hipLaunchKernelGGL((KERN<WT, XV, CTV>), grid, block, 0, stream, x, ldx, w, w_stride, y, ldy, part, M, N, K, RG, \
                       S, SK)
#define SAMHIP_KQ_CT(KERN)                                                                       \
    do {                                                                                         \
        if (xvec) {                                                                              \
            if (CT == 2) SAMHIP_KQ(KERN, true, 2); else SAMHIP_KQ(KERN, true, 1);                \
        } else {                                                                                 \
            if (CT == 2) SAMHIP_KQ(KERN, false, 2); else SAMHIP_KQ(KERN, false, 1);              \
        }                                                                                        \
    } while (0)
    if (isum) SAMHIP_KQ_CT(kq_strip_isum_kernel);
    else SAMHIP_KQ_CT(kq_strip_i8_kernel);
#undef SAMHIP_KQ_CT
#undef SAMHIP_KQ
}

const char* launch_kq_strip_i8(int wtype, const float* x, int64_t ldx, const void* w, int64_t w_stride, float* y,
                               int64_t ldy, float* part, int M, int N, int K, int slice_sb, bool two_tiles, bool isum,
                               hipStream_t stream) {
    if (M < 1 || N < 1 || K < 256 || K % 256) return nullptr;
    if (slice_sb != 1 && slice_sb != 2 && slice_sb != kI8SliceK / 256) return nullptr;
    const int SK = slice_sb;
    // two column tiles per workgroup when a slice holds one super-block
    const int CT = (SK == 1 || K == 256) && two_tiles ? 2 : 1;
    const int RG = (N + 32 * CT - 1) / (32 * CT), S = (K + 256 * SK - 1) / (256 * SK), MB = (M + 31) / 32;
    if (S > 1 && !part) return nullptr;
    if (int64_t(RG) * S * MB > kMaxWorkgroups1024) return nullptr;
    const bool xvec = reinterpret_cast<uintptr_t>(x) % 16 == 0 && ldx % 4 == 0;
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    float* pt = S > 1 ? part : nullptr;
    switch (wtype) {
        case T_Q4_K: launch_kq_strip_wt<T_Q4_K>(xvec, CT, isum, x, ldx, wb, w_stride, y, ldy, pt, M, N, K, RG, S, MB, SK, stream); break;
        case T_Q5_K: launch_kq_strip_wt<T_Q5_K>(xvec, CT, isum, x, ldx, wb, w_stride, y, ldy, pt, M, N, K, RG, S, MB, SK, stream); break;
        case T_Q6_K: launch_kq_strip_wt<T_Q6_K>(xvec, CT, isum, x, ldx, wb, w_stride, y, ldy, pt, M, N, K, RG, S, MB, SK, stream); break;
        default: return nullptr;
    }
    if (S > 1) {
        const int64_t outs = int64_t(M) * N;
        hipLaunchKernelGGL(splitk_reduce_kernel, dim3(unsigned((outs + 255) / 256)), dim3(256), 0, stream, part, y, ldy,
                           M, N, S);
    }
    return kq_strip_i8_variant(wtype);
}

const char* tall_small_i8_variant() { return "tall_small_i8mfma_q8_0"; }

bool tall_small_kq_i8_supported(int wtype, int M, int N, int K, const void* w, int64_t w_stride) {
    return (wtype == T_Q4_K || wtype == T_Q5_K || wtype == T_Q6_K) && M >= 1 && N >= 1 && N <= kTallSmallMaxN &&
           K == kTallSmallK && w_stride == block_bytes(wtype) && reinterpret_cast<uintptr_t>(w) % 16 == 0;
}

const char* tall_small_kq_i8_variant(int wtype) {
    switch (wtype) {
        case T_Q4_K: return "tall_small_i8mfma_q4_k";
        case T_Q5_K: return "tall_small_i8mfma_q5_k";
        case T_Q6_K: return "tall_small_i8mfma_q6_k";
        default: return nullptr;
    }
}

const char* launch_tall_small_kq_i8(int wtype, const float* x, int64_t ldx, const void* w, int64_t w_stride, float* y,
                                    int64_t ldy, int M, int N, int K, int cus, hipStream_t stream) {
    if (!tall_small_kq_i8_supported(wtype, M, N, K, w, w_stride)) return nullptr;
    // 32-bit output offsets, also for the dropped stores of a partial 32-row tile
    if ((int64_t(std::max(M, 32)) * ldy + N) * 4 > 0x7fffffff) return nullptr;
    const int grid = std::max(1, std::min(cus, (M + 15) / 16));
    const bool xvec = reinterpret_cast<uintptr_t>(x) % 16 == 0 && ldx % 4 == 0;
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    // no run past 24 rows: the epilogue skips the tile's last 8 rows
    const bool short_runs = (M + grid - 1) / grid <= 24;
#define SAMHIP_TSK1(WT, XV)                                                                                      \
    do {                                                                                                        \
        if (short_runs)                                                                                         \
            hipLaunchKernelGGL((tall_small_kq_i8_kernel<WT, XV, 3>), dim3(unsigned(grid)), dim3(512), 0, stream, \
                               x, ldx, wb, y, ldy, M, N);                                                       \
        else                                                                                                    \
            hipLaunchKernelGGL((tall_small_kq_i8_kernel<WT, XV, 4>), dim3(unsigned(grid)), dim3(512), 0, stream, \
                               x, ldx, wb, y, ldy, M, N);                                                       \
    } while (0)
#define SAMHIP_TSK(WT)                                                                                          \
    do {                                                                                                        \
        if (xvec) SAMHIP_TSK1(WT, true); else SAMHIP_TSK1(WT, false);                                           \
    } while (0)
    switch (wtype) {
        case T_Q4_K: SAMHIP_TSK(T_Q4_K); break;
        case T_Q5_K: SAMHIP_TSK(T_Q5_K); break;
        case T_Q6_K: SAMHIP_TSK(T_Q6_K); break;
        default: return nullptr;
    }
#undef SAMHIP_TSK
#undef SAMHIP_TSK1
    return tall_small_kq_i8_variant(wtype);
}

bool tall_small_i8_supported(int M, int N, int K, const void* w, int64_t w_stride) {
    return M >= 1 && N >= 1 && N <= kTallSmallMaxN && K == kTallSmallK && w_stride == TS_RB &&
           reinterpret_cast<uintptr_t>(w) % 16 == 0;
}

const char* launch_tall_small_i8(const float* x, int64_t ldx, const void* w, int64_t w_stride, float* y, int64_t ldy,
                                 int M, int N, int K, int x86, int cus, hipStream_t stream) {
    if (!tall_small_i8_supported(M, N, K, w, w_stride)) return nullptr;
    // 32-bit output offsets, also for the dropped stores of a partial 32-row tile
    if ((int64_t(std::max(M, 32)) * ldy + N) * 4 > 0x7fffffff) return nullptr;
    // one workgroup per CU, each with an even run of rows (at least 16)
    const int grid = std::max(1, std::min(cus, (M + 15) / 16));
    const bool xvec = reinterpret_cast<uintptr_t>(x) % 16 == 0 && ldx % 4 == 0;
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    // no run past 24 rows: the epilogue skips the tile's last 8 rows
    const bool short_runs = (M + grid - 1) / grid <= 24;
#define SAMHIP_TS(X86V, XV)                                                                                          \
    do {                                                                                                             \
        if (short_runs)                                                                                              \
            hipLaunchKernelGGL((tall_small_i8_kernel<X86V, XV, 3>), dim3(unsigned(grid)), dim3(512), 0, stream, x, ldx, \
                               wb, y, ldy, M, N);                                                                    \
        else                                                                                                         \
            hipLaunchKernelGGL((tall_small_i8_kernel<X86V, XV, 4>), dim3(unsigned(grid)), dim3(512), 0, stream, x, ldx, \
                               wb, y, ldy, M, N);                                                                    \
    } while (0)
    if (x86) {
        if (xvec) SAMHIP_TS(true, true); else SAMHIP_TS(true, false);
    } else {
        if (xvec) SAMHIP_TS(false, true); else SAMHIP_TS(false, false);
    }
#undef SAMHIP_TS
    return tall_small_i8_variant();
}

const char* fused_skinny_variant(int wtype) {
    switch (wtype) {
        case T_Q8_0: return "skinny_fused_q8_0";
        case T_Q4_K: return "skinny_fused_q4_k";
        case T_Q5_K: return "skinny_fused_q5_k";
        case T_Q6_K: return "skinny_fused_q6_k";
        default: return nullptr;
    }
}

const char* launch_fused_skinny(int wtype, bool f16, const float* x, int64_t ldx, const void* w, int64_t w_stride,
                                float* y, int64_t ldy, float* part, int M, int N, int K, int x86, int max_splits,
                                int cus, hipStream_t stream) {
    if (M < 1 || (M > kFusedMaxM && int64_t(N) * K > kFusedSmallW) || N < 1 || K < 32 || K % 32) return nullptr;
    const FusedPlan p = fused_skinny_plan(M, N, K, max_splits, cus);
    const bool xvec = reinterpret_cast<uintptr_t>(x) % 16 == 0 && ldx % 4 == 0;
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    switch (wtype) {
        case T_Q8_0: launch_fused_wt<T_Q8_0>(f16, x, ldx, xvec, wb, w_stride, y, ldy, p.splits > 1 ? part : nullptr, M, N, K, p.rg, p.splits, p.cps, p.mt, x86, stream); break;
        case T_Q4_K: launch_fused_wt<T_Q4_K>(f16, x, ldx, xvec, wb, w_stride, y, ldy, p.splits > 1 ? part : nullptr, M, N, K, p.rg, p.splits, p.cps, p.mt, x86, stream); break;
        case T_Q5_K: launch_fused_wt<T_Q5_K>(f16, x, ldx, xvec, wb, w_stride, y, ldy, p.splits > 1 ? part : nullptr, M, N, K, p.rg, p.splits, p.cps, p.mt, x86, stream); break;
        case T_Q6_K: launch_fused_wt<T_Q6_K>(f16, x, ldx, xvec, wb, w_stride, y, ldy, p.splits > 1 ? part : nullptr, M, N, K, p.rg, p.splits, p.cps, p.mt, x86, stream); break;
        default: return nullptr;
    }
    if (p.splits > 1) {
        const int64_t outs = int64_t(M) * N;
        hipLaunchKernelGGL(splitk_reduce_kernel, dim3(unsigned((outs + 255) / 256)), dim3(256), 0, stream, part, y, ldy,
                           M, N, p.splits);
    }
    return fused_skinny_variant(wtype);
}

}  // namespace samhip
