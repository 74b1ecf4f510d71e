// fp16 x fp16 -> F32 GEMM for the tall (many-token) mul_mat shapes on gfx950:
//   Y[m][n] = rs[m] * sum_k A[m][k] * B[n][k]
// A = staged activations [M][K], B = weights dequantized per call to
// fp16(ggml to_float(W)) [N][K]; both K-contiguous, K a multiple of 2*BK.
//
// Per workgroup a BM x BN tile, WM x WN waves, each wave a grid of 32x32
// v_mfma_f32_32x32x16_f16 accumulators.  Operands go straight from HBM into
// a ring of XOR-swizzled LDS stages (buffer_load_dwordx4 ... lds, rows past
// M or N read as zero through the buffer bounds), one barrier per BK stage,
// and each wave interleaves the next substep's fragment reads with the
// current substep's MFMAs.  The epilogue goes through LDS so that each lane
// stores 16 contiguous bytes of Y.
#include "internal.hpp"
#include "q8stage.hpp"

namespace samhip {

namespace {

// Row tiles per group of the tile order.  An XCD's run of tiles covers about
// GROUP_M row tiles and (its tile count / GROUP_M) column tiles, whose A and
// B panels it reads into its own L2; at M = 5184, N = 1024, K = 4736 (216
// tiles of 192x128, 27 per XCD) 4 row tiles by ~7 column tiles read less than
// 8 by ~4: sweep 585-588 -> 590-595 TOPS and fc2 790-794 -> 799-812 TFLOP/s
// on one box, alternating the two libraries; the image encode unchanged.
constexpr int GROUP_M = 4;
[[maybe_unused]] constexpr int RSRC_WORD3 = 0x00020000;   // raw buffer, 32-bit data format

[[maybe_unused]] __device__ __forceinline__ void tile_order(int bid, int nblocks, int tiles_m, int tiles_n, int& tm, int& tn) {
    // Blocks are dispatched round-robin over the 8 XCDs: give XCD x a
    // contiguous run of tiles, walked in groups of GROUP_M row tiles.
    const int per = nblocks / 8, rem = nblocks % 8;
    const int xcd = bid % 8, idx = bid / 8;
    const int t = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + idx;
    const int span = GROUP_M * tiles_n;
    const int first = (t / span) * GROUP_M;
    const int gm = min(tiles_m - first, GROUP_M);
    const int within = t % span;
    tm = first + within % gm;
    tn = within / gm;
}

// Epilogue flags (EPI template bits) for Epilogue fields.
constexpr int EPI_BIAS = 1, EPI_RES = 4, EPI_REMAP = 8, EPI_PACK = 16, EPI_COLSCALE = 32, EPI_SHUFFLE = 64,
              EPI_GELU = 128, EPI_Q8 = 256, EPI_PACK_LO = 512;

// Epilogue of a wave's (32*FM) x (32*FN) tile at (row0, col0): each 32-row
// block goes through the wave's LDS slab (stride ES floats; accumulator
// element r of lane l sits on row 8*(r/4) + 4*(l/32) + r%4) and leaves as
// 16-byte row segments scaled by their row's 2^e.  A lane always owns the same 4 columns
// (64 % C4 == 0), so the bias is loaded once; each 32-row block's row
// scales, output rows and residuals are requested before its accumulators
// go through the slab.
template <int FM, int FN, int ES, int EPI>
__device__ __forceinline__ void store_tile_epi(floatx16 (&acc)[FM][FN], const float* row_scale, float* slab, int lane,
                                               int row0, int col0, int M, int N, float* Y, int64_t ldy,
                                               const Epilogue& ep) {
#pragma clang fp contract(off)
    constexpr int TN = 32 * FN, C4 = TN / 4, RSTEP = 64 / C4, IT = 32 / RSTEP;
    static_assert(64 % C4 == 0, "a lane keeps its columns");
    const bool vec_ok = (ldy % 4) == 0 && (reinterpret_cast<uintptr_t>(Y) % 16) == 0;
    const int c4 = lane % C4, r0 = lane / C4;
    const int n = col0 + 4 * c4;
    const bool full = n + 3 < N;
    // transposed-convolution scatter: the lane's 4 columns share one tap
    int ycol = n, sky = 0, skx = 0;
    if (EPI & EPI_SHUFFLE) {
        const int tap = n / ep.shuffle_c;
        ycol = n - tap * ep.shuffle_c;
        sky = tap >> 1;
        skx = tap & 1;
    }
    floatx4 bias{0.f, 0.f, 0.f, 0.f}, cs{1.f, 1.f, 1.f, 1.f};
    if (EPI & EPI_BIAS)
#pragma unroll
        for (int q = 0; q < 4; ++q) bias[q] = (full || n + q < N) ? ep.bias[ycol + q] : 0.f;
    if (EPI & EPI_COLSCALE)
#pragma unroll
        for (int q = 0; q < 4; ++q) cs[q] = (full || n + q < N) ? ep.col_scale[n + q] : 0.f;
    const float inv_sw = (EPI & EPI_SHUFFLE) ? 1.0f / float(ep.shuffle_w) : 0.f;
    // packed outputs: the wave's 64-aligned column block lies in one part and
    // one head (embed is a multiple of 64), so the part and its output
    // arrays are the same for every lane; element offsets are 32-bit (the
    // host keeps each part's array below 2^31 elements)
    const int part = (EPI & EPI_PACK) ? __builtin_amdgcn_readfirstlane(col0 / ep.embed) : 0;
    const float inv_per = (EPI & EPI_PACK) ? 1.0f / float(ep.per) : 0.f;
    const int head_off = (EPI & EPI_PACK) ? ((n - part * ep.embed) >> 6) * ep.np * 64 + (n & 63) : 0;
    _Float16* const pk_hi = (EPI & EPI_PACK) ? (part == 0 ? ep.pack[0] : part == 1 ? ep.pack[1] : ep.pack[2]) : nullptr;
    _Float16* const pk_lo =
        (EPI & EPI_PACK_LO) ? (part == 0 ? ep.pack_lo[0] : part == 1 ? ep.pack_lo[1] : ep.pack_lo[2]) : nullptr;
    const __amdgpu_buffer_rsrc_t pk_rsrc = __builtin_amdgcn_make_buffer_rsrc(pk_hi, 0, 0x7fffffff, RSRC_WORD3);
    const __amdgpu_buffer_rsrc_t pk_lo_rsrc = __builtin_amdgcn_make_buffer_rsrc(pk_lo, 0, 0x7fffffff, RSRC_WORD3);
    const bool rope = (EPI & EPI_PACK) && part < 2 && ep.freqs;
    // 1.0 the compiler cannot see: fma(v, one, -hi) stays one v_fma_mix
    // (v - hi is exact in F32, rounded once to fp16) instead of a conversion
    // of hi back to F32 and a subtraction
    float one = 1.0f;
    if (EPI & EPI_PACK_LO) asm("" : "+s"(one));
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        float sc[IT];
        int64_t dst[IT];
        floatx4 res[IT];
        floatx4 fq[IT];
#pragma unroll
        for (int t = 0; t < IT; ++t) {
            const int m = row0 + i * 32 + r0 + RSTEP * t;
            const bool live = m < M;
            sc[t] = live ? row_scale[m] : 0.f;
            if (EPI & EPI_PACK) {
                // window = m / per by a float reciprocal and one correction;
                // every factor is below 2^24 (24-bit multiplies)
                int w = int(float(m) * inv_per);
                int wp = int(__umul24(unsigned(w), unsigned(ep.per)));
                if (wp + ep.per <= m) {
                    ++w;
                    wp += ep.per;
                }
                if (wp > m) {
                    --w;
                    wp -= ep.per;
                }
                const int tok = live ? m - wp : 0;
                dst[t] = (int(__umul24(__umul24(unsigned(w), unsigned(ep.heads)), unsigned(ep.np))) + tok) * 64;
                if (rope) fq[t] = *reinterpret_cast<const floatx4*>(ep.freqs + (tok * 32 + ((n & 63) >> 1)) * 2);
            } else if (EPI & EPI_SHUFFLE) {
                // input pixel (x, y) = (m % shuffle_w, m / shuffle_w) by a float
                // reciprocal and one correction
                const int sw = ep.shuffle_w;
                int y = int(float(m) * inv_sw);
                y += (y + 1) * sw <= m;
                y -= y * sw > m;
                const int x = m - y * sw;
                dst[t] = live ? int64_t(2 * y + sky) * 2 * sw + 2 * x + skx : 0;
            } else {
                dst[t] = (EPI & EPI_REMAP) ? (live ? int64_t(ep.row_map[m]) : 0) : int64_t(m);
            }
        }
        if (EPI & EPI_RES) {
#pragma unroll
            for (int t = 0; t < IT; ++t) {
                const int m = row0 + i * 32 + r0 + RSTEP * t;
                const float* rp = ep.res + dst[t] * ldy + n;
                if (m < M && full && vec_ok) {
                    res[t] = *reinterpret_cast<const floatx4*>(rp);
                } else {
#pragma unroll
                    for (int q = 0; q < 4; ++q) res[t][q] = (m < M && n + q < N) ? rp[q] : 0.f;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                slab[(8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * ES + 32 * j + (lane & 31)] = acc[i][j][r];
        __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): the slab is written
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int t = 0; t < IT; ++t) {
            const int rr = r0 + RSTEP * t;
            if (row0 + i * 32 + rr >= M) continue;
            const floatx4 raw = *reinterpret_cast<const floatx4*>(slab + rr * ES + 4 * c4);
            floatx4 v;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                // the row scale is a power of two, so raw * sc is exact and
                // fma(raw, sc, bias) rounds as the product and the sum do
                float u;
                if ((EPI & EPI_BIAS) && !(EPI & EPI_COLSCALE)) {
                    u = __builtin_fmaf(raw[q], sc[t], bias[q]);
                } else {
                    u = raw[q] * sc[t];
                    if (EPI & EPI_COLSCALE) u = u * cs[q];
                    if (EPI & EPI_BIAS) u = u + bias[q];
                }
                if (EPI & EPI_GELU) u = gelu_erf(u);
                if (EPI & EPI_RES) u = res[t][q] + u;
                v[q] = u;
            }
            if constexpr ((EPI & EPI_Q8) != 0) {
                // Q8_0 packing of the row's 32-column block, held by the 8
                // lanes c4 = 8g .. 8g + 7 (C4 is a multiple of 8, col0 of 32):
                // ggml's from_float on these F32 values (x86 scale 127/amax
                // with ties to even, or the reference 1/d with ties away;
                // NaN packs as code 0); the block maximum leaves in F32
                float amax = 0.f;
#pragma unroll
                for (int q = 0; q < 4; ++q) amax = fmaxf(amax, fabsf(v[q]));
                amax = group_max<8>(amax);
                const float dd = amax / 127.f;
                float inv;
                if (ep.q8_x86) inv = amax != 0.f ? 127.f / amax : 0.f;
                else inv = dd != 0.f ? 1.f / dd : 0.f;
                uint32_t word = 0;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float sq = v[q] * inv;
                    const float r = ep.q8_x86 ? __builtin_rintf(sq) : __builtin_roundf(sq);
                    word |= (uint32_t(r == r ? int(r) : 0) & 0xffu) << (8 * q);
                }
                *reinterpret_cast<uint32_t*>(ep.q8 + dst[t] * ep.q8_ld + n) = word;
                if ((c4 & 7) == 0) ep.q8_amax[dst[t] * (ep.q8_ld >> 5) + (n >> 5)] = amax;
                continue;
            }
            if (EPI & EPI_PACK) {
                if (rope) {
#pragma unroll
                    for (int p2 = 0; p2 < 2; ++p2) {
                        const float re = v[2 * p2], im = v[2 * p2 + 1], c = fq[t][2 * p2], s = fq[t][2 * p2 + 1];
                        const float a = re * c, bb = im * s, cc = re * s, dd = im * c;
                        v[2 * p2] = a - bb;
                        v[2 * p2 + 1] = cc + dd;
                    }
                }
                if (part == 0)
#pragma unroll
                    for (int q = 0; q < 4; ++q) v[q] = v[q] * ep.q_scale;
                typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
                const half4_t hv = __builtin_convertvector(v, half4_t);
                // 8-byte stores at 32-bit byte offsets from the part's array
                const uint32_t off = uint32_t(head_off + int(dst[t])) * 2;
                __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, hv), pk_rsrc, off, 0, 0);
                if ((EPI & EPI_PACK_LO) && pk_lo) {
                    const half4_t lv{(_Float16)__builtin_fmaf(v[0], one, -(float)hv[0]),
                                     (_Float16)__builtin_fmaf(v[1], one, -(float)hv[1]),
                                     (_Float16)__builtin_fmaf(v[2], one, -(float)hv[2]),
                                     (_Float16)__builtin_fmaf(v[3], one, -(float)hv[3])};
                    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, lv), pk_lo_rsrc, off, 0, 0);
                }
                continue;
            }
            float* yp = Y + dst[t] * ldy + ycol;
            if (vec_ok && full) {
                __builtin_nontemporal_store(v, reinterpret_cast<floatx4*>(yp));
            } else {
                for (int q = 0; q < 4; ++q)
                    if (n + q < N) yp[q] = v[q];
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
}

// ---------------------------------------------------------------------------
// LDS layout: operands go HBM -> LDS with buffer_load_dwordx4 ... lds (no
// VGPR round trip, no ds_write), through a ring of STAGES buffers, so the
// loads of stage s+STAGES-1 are requested while stage s computes.  One
// wave-wide load fills 1 KB of LDS contiguously (lane l -> bytes 16l..16l+15);
// each lane picks the global chunk that belongs at its slot, which lays every
// tile row out with its 16-byte K chunks XOR-swizzled by the row index:
//   chunk kc of row r lives at slot kc ^ swz(r)
// so that the 32 rows an MFMA fragment read touches fall in distinct banks.
// ---------------------------------------------------------------------------

// LDS has 64 banks of 4 bytes, 256 bytes across.  A tile row of CPR 16-byte
// chunks is 16 * CPR bytes, so 16 / CPR consecutive rows share one 256-byte
// span of banks; the XOR pattern changes every 16 / CPR rows, so the same
// chunk of 32 consecutive rows (one fragment read) lands evenly on all
// sixteen 16-byte bank groups.
template <int CPR>
__device__ __forceinline__ int swz(int r) {
    return CPR == 16 ? (r & 15) : CPR == 8 ? ((r >> 1) & 7) : ((r >> 2) & 3);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    // s_waitcnt vmcnt(N), expcnt/lgkmcnt left at their maximum (gfx9 encoding)
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | 0xF00);
}

// ---------------------------------------------------------------------------
// The tall GEMM: every wave holds two sets of MFMA
// fragments, and the ds_reads of K substep kk+1 are interleaved with the
// MFMAs of substep kk (pinned with sched_group_barrier), so the matrix cores
// never wait on LDS latency inside a stage.  The stage hand-over (wait for
// this wave's loads of the next stage, a bare s_barrier, the next ring slot's
// loads and the first fragments of the next stage) sits between the two
// halves of the last substep's MFMAs.  WM x WN waves, each a (BM/WM) x
// (BN/WN) tile: 256x128 on 2x2 waves or 256x256 on 2x4 / 4x2 waves gives 8
// independent 32x32 accumulators per wave (8 waves: two per SIMD).
// ---------------------------------------------------------------------------

template <int BM, int BN, int BK, int STAGES, int WM, int WN, int EPI = 0, int AM = A_PLAIN>
__global__ __launch_bounds__(64 * WM * WN) void gemm_f16_pipe_kernel(const _Float16* __restrict__ A, int64_t lda,
                                                            const float* __restrict__ row_scale,
                                                            const _Float16* __restrict__ B, int64_t ldb,
                                                            float* Y, int64_t ldy, int M, int N, int K,
                                                            int tiles_m, int tiles_n, Epilogue ep, AOperand op) {
#if defined(__HIP_DEVICE_COMPILE__)
    constexpr int NW = WM * WN;
    constexpr int CPR = BK / 8, RB = BK * 2;
    constexpr int RPB = 64 / CPR;
    constexpr int A_BLOCKS = BM / RPB, B_BLOCKS = BN / RPB;
    constexpr int A_PER_WAVE = A_BLOCKS / NW, B_PER_WAVE = B_BLOCKS / NW;
    constexpr int LOADS = A_PER_WAVE + B_PER_WAVE;
    constexpr int STAGE_BYTES = (BM + BN) * RB;
    constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32;
    constexpr int KK = BK / 16;
    constexpr int NF = FM * FN;
    constexpr int ES = TN + 8;
    static_assert(A_PER_WAVE * NW == A_BLOCKS && B_PER_WAVE * NW == B_BLOCKS, "tile rows must split over the waves");
    static_assert(STAGES >= 2 && STAGES <= 6, "ring depth");
    static_assert(KK % 2 == 0, "fragment double buffer alternates per substep");
    static_assert(NW * 32 * ES * 4 <= STAGES * STAGE_BYTES, "epilogue staging must fit in LDS");

    __shared__ __attribute__((aligned(1024))) uint8_t lds[STAGES * STAGE_BYTES];

    int tm, tn;
    tile_order(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;

    const uint32_t a_bytes = uint32_t(min(int64_t(M) * lda * 2, int64_t(0x7fffffff)));
    const uint32_t b_bytes = uint32_t(min(int64_t(N) * ldb * 2, int64_t(0x7fffffff)));
    const __amdgpu_buffer_rsrc_t ra_desc = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(A), 0, a_bytes, RSRC_WORD3);
    const __amdgpu_buffer_rsrc_t rb_desc = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(B), 0, b_bytes, RSRC_WORD3);

    uint32_t a_off[A_PER_WAVE], b_off[B_PER_WAVE];
    int a_taps[A_PER_WAVE];   // A_CONV3: bit 3*ky+kx set when that neighbour lies in the map
#pragma unroll
    for (int i = 0; i < A_PER_WAVE; ++i) {
        const int blk = wave * A_PER_WAVE + i, r = blk * RPB + lane / CPR, slot = lane % CPR;
        const int kc = slot ^ swz<CPR>(r);
        a_off[i] = m0 + r < M ? uint32_t((int64_t(m0 + r) * lda + 8 * kc) * 2) : a_bytes;
        if (AM == A_CONV3) {
            const int m = m0 + r, y = m / op.width, x = m - y * op.width;
            int taps = 0;
#pragma unroll
            for (int t = 0; t < 9; ++t) {
                const int yy = y + t / 3 - 1, xx = x + t % 3 - 1;
                taps |= (m < M && yy >= 0 && yy < op.height && xx >= 0 && xx < op.width) ? 1 << t : 0;
            }
            a_taps[i] = taps;
        }
    }
#pragma unroll
    for (int i = 0; i < B_PER_WAVE; ++i) {
        const int blk = wave * B_PER_WAVE + i, r = blk * RPB + lane / CPR, slot = lane % CPR;
        const int kc = slot ^ swz<CPR>(r);
        b_off[i] = n0 + r < N ? uint32_t((int64_t(n0 + r) * ldb + 8 * kc) * 2) : b_bytes;
    }
    auto issue = [&](int s) {
        uint8_t* st = lds + (s % STAGES) * STAGE_BYTES;
        const int koff = s * RB;
        if (AM == A_CONV3) {
            // the stage's BK columns lie in one (part, tap) block of `part`
            // channels: one signed byte step from each lane's own pixel
            const int k = s * BK, span = 9 * op.part;
            const int p = k / span, rem = k - p * span, tap = rem / op.part, c0 = rem - tap * op.part;
            const int step = (((tap / 3 - 1) * op.width + tap % 3 - 1) * int(lda) + (p == 2 ? op.part : 0) + c0) * 2;
#pragma unroll
            for (int i = 0; i < A_PER_WAVE; ++i)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    ra_desc, (__attribute__((address_space(3))) void*)(st + (wave * A_PER_WAVE + i) * 1024), 16,
                    (a_taps[i] >> tap) & 1 ? uint32_t(int(a_off[i]) + step) : a_bytes, 0, 0, 0);
        } else {
            // A_REPEAT: logical columns [part, 2 part) re-read the hi half
            const int akoff = (AM == A_REPEAT && s * BK >= op.part) ? koff - op.part * 2 : koff;
#pragma unroll
            for (int i = 0; i < A_PER_WAVE; ++i)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    ra_desc, (__attribute__((address_space(3))) void*)(st + (wave * A_PER_WAVE + i) * 1024), 16,
                    a_off[i], akoff, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < B_PER_WAVE; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rb_desc, (__attribute__((address_space(3))) void*)(st + BM * RB + (wave * B_PER_WAVE + i) * 1024),
                16, b_off[i], koff, 0, 0);
    };

    // LDS byte offsets of this lane's fragment rows (stage 0, chunk 0); the
    // swizzle only depends on the row, so a substep adds 32 bytes XOR-ed
    const int frow = lane & 31, fhalf = lane >> 5;
    int a_row[FM], b_row[FN], a_sw[FM], b_sw[FN];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const int r = wm * TM + i * 32 + frow;
        a_row[i] = r * RB;
        a_sw[i] = swz<CPR>(r);
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int r = wn * TN + j * 32 + frow;
        b_row[j] = BM * RB + r * RB;
        b_sw[j] = swz<CPR>(r);
    }
    auto load_frags = [&](int s, int kk, half8* fa, half8* fb) {
        const uint8_t* st = lds + (s % STAGES) * STAGE_BYTES;
        const int kc = 2 * kk + fhalf;
#pragma unroll
        for (int i = 0; i < FM; ++i) fa[i] = *reinterpret_cast<const half8*>(st + a_row[i] + 16 * (kc ^ a_sw[i]));
#pragma unroll
        for (int j = 0; j < FN; ++j) fb[j] = *reinterpret_cast<const half8*>(st + b_row[j] + 16 * (kc ^ b_sw[j]));
    };

    floatx16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int nst = K / BK;
    // hand-over into stage t: this wave's reads of stage t-1 are complete and
    // its loads of stage t landed; after the barrier every wave's have, and
    // the ring slot of stage t-1 is refilled with stage t+STAGES-1
    auto enter = [&](int t) {
        const int later = min(STAGES - 2, nst - 1 - t);
        __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0)
        if (later >= 4) wait_vmcnt<4 * LOADS>();
        else if (later == 3) wait_vmcnt<3 * LOADS>();
        else if (later == 2) wait_vmcnt<2 * LOADS>();
        else if (later == 1) wait_vmcnt<LOADS>();
        else wait_vmcnt<0>();
        asm volatile("s_barrier" ::: "memory");
        if (t + STAGES - 1 < nst) issue(t + STAGES - 1);
    };

    half8 fa[2][FM], fb[2][FN];
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
        if (s < nst) issue(s);
    enter(0);
    load_frags(0, 0, fa[0], fb[0]);

    for (int s = 0; s < nst; ++s) {
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            const int cur = kk & 1;
            if (kk + 1 < KK) {
                load_frags(s, kk + 1, fa[cur ^ 1], fb[cur ^ 1]);
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[cur][i], fb[cur][j], acc[i][j], 0, 0, 0);
                // one fragment read between consecutive MFMAs, then the rest
#pragma unroll
                for (int q = 0; q < FM + FN; ++q) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
                __builtin_amdgcn_sched_group_barrier(0x008, NF - (FM + FN), 0);
            } else {
                // first half of the last substep's products, the hand-over,
                // then the second half while the next stage's fragments load
#pragma unroll
                for (int q = 0; q < NF / 2; ++q) {
                    const int i = q / FN, j = q % FN;
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[cur][i], fb[cur][j], acc[i][j], 0, 0, 0);
                }
                if (s + 1 < nst) {
                    enter(s + 1);
                    load_frags(s + 1, 0, fa[0], fb[0]);
                }
#pragma unroll
                for (int q = NF / 2; q < NF; ++q) {
                    const int i = q / FN, j = q % FN;
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[cur][i], fb[cur][j], acc[i][j], 0, 0, 0);
                }
            }
        }
    }
    __syncthreads();

    store_tile_epi<FM, FN, ES, EPI>(acc, row_scale, reinterpret_cast<float*>(lds) + wave * 32 * ES, lane,
                                    m0 + wm * TM, n0 + wn * TN, M, N, Y, ldy, ep);
#endif
}

// Dynamic LDS that keeps a second workgroup off a CU: when a grid has no
// more tiles than CUs, two resident workgroups per CU would leave other CUs
// idle (the dispatcher fills a CU before moving on).
constexpr size_t spread_pad(size_t static_lds) { return static_lds > 82944 ? 0 : 82944 - static_lds; }

template <int BM, int BN, int BK, int STAGES, int WM = 2, int WN = 2, int EPI = 0, int AM = A_PLAIN>
void launch_pipe(const _Float16* a, int64_t lda, const float* rs, const _Float16* b, int64_t ldb, float* y,
                 int64_t ldy, int M, int N, int K, bool spread, hipStream_t stream, const Epilogue& ep = Epilogue{},
                 const AOperand& op = AOperand{}) {
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    const size_t pad = spread ? spread_pad(size_t(STAGES) * (BM + BN) * BK * 2) : 0;
    hipLaunchKernelGGL((gemm_f16_pipe_kernel<BM, BN, BK, STAGES, WM, WN, EPI, AM>), dim3(unsigned(tiles_m * tiles_n)),
                       dim3(64 * WM * WN), pad, stream, a, lda, rs, b, ldb, y, ldy, M, N, K, tiles_m, tiles_n, ep, op);
}

// Configuration-table entry point (plain epilogue).
template <int BM, int BN, int BK, int STAGES, int WM = 2, int WN = 2>
void launch_pipe_plain(const _Float16* a, int64_t lda, const float* rs, const _Float16* b, int64_t ldb, float* y,
                       int64_t ldy, int M, int N, int K, bool spread, hipStream_t stream) {
    launch_pipe<BM, BN, BK, STAGES, WM, WN, 0>(a, lda, rs, b, ldb, y, ldy, M, N, K, spread, stream);
}

struct Cfg {
    const char* name;
    void (*launch)(const _Float16*, int64_t, const float*, const _Float16*, int64_t, float*, int64_t, int, int, int,
                   bool, hipStream_t);
    int bm, bn, bk, wm, wn;
};

#define SAMHIP_CFG(BM, BN, BK, S, WM, WN)                                                            \
    {"gemm_f16pipe_" #BM "x" #BN "x" #BK "_s" #S "_w" #WM "x" #WN, launch_pipe_plain<BM, BN, BK, S, WM, WN>, BM, \
     BN, BK, WM, WN}
// Every configuration runs the pipelined kernel; the ones the picks below
// do not take stay selectable through SAMHIP_GEMM_CONFIG for tile sweeps.
constexpr Cfg kConfigs[] = {
    SAMHIP_CFG(256, 256, 64, 2, 2, 4),   // qkv-like grids that fill the CUs
    SAMHIP_CFG(192, 128, 64, 2, 2, 4),   // the rest of the tall shapes
    SAMHIP_CFG(128, 128, 64, 3, 2, 4),   // plain products with small grids
    SAMHIP_CFG(256, 128, 64, 2, 2, 2),
    SAMHIP_CFG(256, 128, 32, 3, 2, 2),
    SAMHIP_CFG(128, 256, 32, 3, 2, 2),
    SAMHIP_CFG(256, 256, 32, 3, 2, 4),
    SAMHIP_CFG(256, 128, 64, 2, 4, 2),
    SAMHIP_CFG(128, 256, 64, 2, 2, 4),
    SAMHIP_CFG(128, 128, 128, 2, 2, 4),
    SAMHIP_CFG(192, 128, 64, 2, 2, 2),
    SAMHIP_CFG(64, 128, 64, 3, 2, 4),
    SAMHIP_CFG(128, 64, 64, 3, 4, 2),
    SAMHIP_CFG(64, 128, 64, 4, 2, 4),
};
#undef SAMHIP_CFG
constexpr int kCfgSquare = 0, kCfgWide = 1, kCfgSmall = 2, kCfgTiny = 11, kCfgTinyDeep = 13;
static_assert(kConfigs[kCfgSquare].bm == 256 && kConfigs[kCfgSquare].bn == 256 && kConfigs[kCfgWide].bm == 192 &&
                  kConfigs[kCfgWide].bn == 128 && kConfigs[kCfgSmall].bm == 128 && kConfigs[kCfgSmall].bn == 128 &&
                  kConfigs[kCfgTiny].bm == 64 && kConfigs[kCfgTiny].bn == 128 && kConfigs[kCfgTinyDeep].bm == 64 &&
                  kConfigs[kCfgTinyDeep].bn == 128,
              "the picks below name these entries");
constexpr int kNumConfigs = sizeof(kConfigs) / sizeof(kConfigs[0]);

}  // namespace

int gemm_f16_config_count() { return kNumConfigs; }

const char* gemm_f16_config_name(int cfg) { return cfg >= 0 && cfg < kNumConfigs ? kConfigs[cfg].name : nullptr; }

// The main loop walks K in pairs of stages, so K must be a multiple of 2*BK
// for every configuration (128 covers BK = 32 and 64); buffer offsets are
// 32-bit.
bool gemm_f16_supported(int M, int N, int K, int64_t lda, int64_t ldb) {
    return K % 128 == 0 && int64_t(M) * lda * 2 < 0x7fffffff && int64_t(N) * ldb * 2 < 0x7fffffff;
}

// Tile choice from measured sweeps on MI355X (kernel time, HIP events,
// random operands; differences below ~3 % are within run-to-run noise).
// Eight-wave workgroups win on every shape; what decides between the two
// remaining tiles is how evenly the grid fills the CUs.  256x256 tiles
// (2x4 waves, one workgroup per CU) are the most efficient per tile but
// come in coarse waves; 192x128 tiles (2x4 waves, 80 KB of LDS: two
// workgroups per CU) balance better.  256x256 is taken when its tiles fill
// at least 80 % of the CU waves they occupy:
//   M = 5184:  qkv N 3072 (252 tiles) 42.8 us vs 46.3; fc1 N 4736 (399
//              tiles) 72.9 vs 61.2 -> 192x128; N 1024 K 1024 / 4736 (proj,
//              fc2) 22.1 / 65.7 us with 192x128 vs 23.7 / 70.3 with 256x128;
//   M = 41472: N 3072 377 vs 408, N 4736 557 vs 579, N 1024 K 4736 495 vs
//              528 -> 256x256; N 1024 K 1024 117 vs 115.
int gemm_f16_pick(int M, int N, int /*K*/, int cus) {
    const int64_t tiles = int64_t((M + 255) / 256) * ((N + 255) / 256);
    const int64_t waves = (tiles + cus - 1) / cus;
    return tiles * 10 >= waves * cus * 8 ? kCfgSquare : kCfgWide;
}

// Plain products (mul_mat) also take 128x128x64 tiles on 2x4 waves (three
// stages) when even 192x128 tiles would leave half the CUs idle: M = 5184,
// N = 256 (the fusion / decoder image-token products) 9.5 vs 10.9 us at
// K = 256 and 23.5 vs 29.3 us at K = 2048; N = 2048 stays 192x128 (17.3 vs
// 22.1 us).
//
// 64x128 tiles (2x4 waves of 32x32) where even 128x128 tiles would leave
// half the CUs idle, and for K of at most 256 (four stages, too few to
// amortize a large tile's prologue and epilogue): M = 5184, N = 256,
// K = 2048 (the fusion encoder's FFN output product) 21.7 -> 17.1 us;
// N = 2048, K = 256 (its FFN input) 19.7 -> 18.7 us against 192x128.
// When those tiles take one workgroup per CU anyway and K is long, a
// four-deep ring (96 KB of LDS): the FFN output product 17.1 -> 16.3 us
// (five and six stages 18.5 and 17.9; 64x64 tiles on 2x2 waves 18.4, 17.1
// with four stages); at K = 256 the deep ring's second workgroup per CU is
// missed (18.7 -> 24.8 us).
int gemm_f16_pick_plain(int M, int N, int K, int cus) {
    const int64_t tiles = int64_t((M + 191) / 192) * ((N + 127) / 128);
    const int64_t small = int64_t((M + 127) / 128) * ((N + 127) / 128);
    const int64_t tiny = int64_t((M + 63) / 64) * ((N + 127) / 128);
    if (K >= 1024 && tiny <= cus && 2 * small <= cus && K % kConfigs[kCfgTinyDeep].bk == 0) return kCfgTinyDeep;
    if (K <= 256 || (2 * tiles <= cus && 2 * small <= cus)) return kCfgTiny;
    if (2 * tiles <= cus && K % kConfigs[kCfgSmall].bk == 0) return kCfgSmall;
    return gemm_f16_pick(M, N, K, cus);
}

// The two configurations gemm_f16_pick returns (256x256x64 and 192x128x64 on
// 2x4 waves) with each epilogue and operand mode the encoder uses.
template <int BM, int BN, int WM, int WN>
bool launch_epi(const _Float16* a, int64_t lda, const float* rs, const _Float16* b, int64_t ldb, float* y,
                int64_t ldy, int M, int N, int K, bool spread, const Epilogue& ep, const AOperand& op,
                hipStream_t stream) {
    const int flags = (ep.bias ? EPI_BIAS : 0) | (ep.res ? EPI_RES : 0) | (ep.row_map ? EPI_REMAP : 0) |
                      (ep.pack[0] ? EPI_PACK : 0) | (ep.col_scale ? EPI_COLSCALE : 0) |
                      (ep.shuffle_c > 0 ? EPI_SHUFFLE : 0) | (ep.gelu ? EPI_GELU : 0) |
                      (ep.pack_lo[0] ? EPI_PACK_LO : 0) | (ep.q8 ? EPI_Q8 : 0);
#define SAMHIP_EPI(E, AMODE)                                                                                     \
    launch_pipe<BM, BN, 64, 2, WM, WN, E, AMODE>(a, lda, rs, b, ldb, y, ldy, M, N, K, spread, stream, ep, op); \
    return true;
    constexpr int BC = EPI_BIAS | EPI_COLSCALE;
    if (op.mode == A_PLAIN) {
        switch (flags) {
            case 0: SAMHIP_EPI(0, A_PLAIN)
            case EPI_BIAS: SAMHIP_EPI(EPI_BIAS, A_PLAIN)
            case EPI_BIAS | EPI_RES: SAMHIP_EPI(EPI_BIAS | EPI_RES, A_PLAIN)
            case EPI_BIAS | EPI_PACK: SAMHIP_EPI(EPI_BIAS | EPI_PACK, A_PLAIN)
            case EPI_BIAS | EPI_PACK | EPI_PACK_LO: SAMHIP_EPI(EPI_BIAS | EPI_PACK | EPI_PACK_LO, A_PLAIN)
            case EPI_BIAS | EPI_RES | EPI_REMAP: SAMHIP_EPI(EPI_BIAS | EPI_RES | EPI_REMAP, A_PLAIN)
            case BC: SAMHIP_EPI(BC, A_PLAIN)
            case EPI_BIAS | EPI_GELU | EPI_Q8: SAMHIP_EPI(EPI_BIAS | EPI_GELU | EPI_Q8, A_PLAIN)
            default: return false;
        }
    }
    if (op.mode == A_REPEAT) {
        switch (flags) {
            case BC: SAMHIP_EPI(BC, A_REPEAT)
            case BC | EPI_SHUFFLE: SAMHIP_EPI(BC | EPI_SHUFFLE, A_REPEAT)
            case BC | EPI_SHUFFLE | EPI_GELU: SAMHIP_EPI(BC | EPI_SHUFFLE | EPI_GELU, A_REPEAT)
            default: return false;
        }
    }
    if (op.mode == A_CONV3 && flags == BC) {
        SAMHIP_EPI(BC, A_CONV3)
    }
#undef SAMHIP_EPI
    return false;   // combinations the encoder does not use
}

const char* launch_gemm_f16_epi(const _Float16* a, int64_t lda, const float* row_scale, const _Float16* b,
                                int64_t ldb, float* y, int64_t ldy, int M, int N, int K, int cus, const Epilogue& ep,
                                hipStream_t stream, const AOperand& op) {
    const int cfg = gemm_f16_pick(M, N, K, cus);
    const Cfg& c = kConfigs[cfg];
    const bool spread = int64_t((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn) <= cus;
    if (op.mode != A_PLAIN && (op.part % (op.mode == A_CONV3 ? 128 : 64) || op.part <= 0)) return nullptr;
    // Q8_0 blocks: whole 32-column blocks, 4-byte aligned code rows
    if (ep.q8 && (N % 32 || ep.q8_ld % 32 || ep.q8_ld < N || !ep.q8_amax ||
                  reinterpret_cast<uintptr_t>(ep.q8) % 4 || reinterpret_cast<uintptr_t>(ep.q8_amax) % 4))
        return nullptr;
    if (op.mode == A_CONV3 && (op.width <= 0 || op.height <= 0 || int64_t(op.width) * op.height != M)) return nullptr;
    const bool ok = cfg == kCfgSquare
        ? launch_epi<256, 256, 2, 4>(a, lda, row_scale, b, ldb, y, ldy, M, N, K, spread, ep, op, stream)
        : launch_epi<192, 128, 2, 4>(a, lda, row_scale, b, ldb, y, ldy, M, N, K, spread, ep, op, stream);
    return ok ? c.name : nullptr;
}

const char* launch_gemm_f16(int cfg, const _Float16* a, int64_t lda, const float* row_scale, const _Float16* b,
                            int64_t ldb, float* y, int64_t ldy, int M, int N, int K, int cus, hipStream_t stream) {
    if (cfg < 0 || cfg >= kNumConfigs || K % kConfigs[cfg].bk) cfg = gemm_f16_pick(M, N, K, cus);
    const Cfg& c = kConfigs[cfg];
    const int64_t tiles = int64_t((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn);
    c.launch(a, lda, row_scale, b, ldb, y, ldy, M, N, K, tiles <= cus, stream);
    return kConfigs[cfg].name;
}

}  // namespace samhip
