// Launchers shared between the kernel translation units and the C ABI layer.
#pragma once

#include "blocks.hpp"

namespace samhip {

// mode: T_F16 (direct), T_Q8_0 or T_Q8_K (native activation packing).
void launch_stage_rows(int mode, bool aligned, const float* x, int64_t x_stride, int M, int K, _Float16* a,
                       int64_t lda, float* row_scale, int x86, hipStream_t stream);

// Q8_0 / Q8_K activation rows in ggml wire format.
void launch_quantize_act(int type, const float* x, int64_t x_stride, int rows, int K, void* dst, int x86,
                         hipStream_t stream);

// ggml-cuda right-operand formats: Q8_1 rows (quantize_row_q8_1_cuda) and
// the MMQ D4 staging of Q8_0 products (quantize_mmq_q8_1_cuda; rows padded
// to a multiple of 512 values, [kp/128][rows][144 B]).  The D4 launch and
// the range check set *invalid for blocks outside the native activation's
// range (non-finite, or a nonzero block maximum outside [1e-30, 1e30]).
void launch_quantize_q8_1(const float* x, int64_t x_stride, int rows, int K, void* dst, hipStream_t stream);
void launch_quantize_q8_1_mmq(const float* x, int64_t x_stride, int rows, int K, void* dst, int* invalid,
                              hipStream_t stream);
void launch_q8_rhs_check(const float* x, int64_t x_stride, int rows, int K, int* invalid, hipStream_t stream);

// F32 -> F16 rows, packed (ggml_cast to F16).
void launch_cast_f16(const float* x, int64_t x_stride, int rows, int K, _Float16* dst, hipStream_t stream);

// Q4_K / Q5_K / Q6_K weight rows in ggml wire format (ggml_quantize_chunk).
void launch_quantize_weights(int type, const float* x, int64_t x_stride, int rows, int K, void* dst,
                             hipStream_t stream);

// to_float (ids == nullptr) or get_rows (ids != nullptr, bad_id flag set on
// an out-of-range id).
void launch_dequant_rows(int type, const void* src, int64_t src_stride, const int32_t* ids, int64_t src_rows,
                         float* dst, int64_t dst_stride, int rows, int K, int* bad_id, hipStream_t stream);

// Weight rows -> fp16(ggml to_float(W)) [N][K] with row stride ldo halves.
void launch_dequant_w_f16(int wtype, const void* w, int64_t w_stride, int N, int K, _Float16* out, int64_t ldo,
                          hipStream_t stream);

// fp16 x fp16 GEMM for tall shapes: Y = rs * A B^T.  cfg < 0 picks a tile
// configuration from the shape; returns the configuration's name.
int gemm_f16_config_count();
bool gemm_f16_supported(int M, int N, int K, int64_t lda, int64_t ldb);
const char* gemm_f16_config_name(int cfg);
int gemm_f16_pick(int M, int N, int K, int cus);
// gemm_f16_pick plus 128x128 tiles for small grids (plain products only).
int gemm_f16_pick_plain(int M, int N, int K, int cus);
// `cus`: compute units of the device; grids with at most that many tiles run
// one workgroup per CU.
const char* launch_gemm_f16(int cfg, const _Float16* a, int64_t lda, const float* row_scale, const _Float16* b,
                            int64_t ldb, float* y, int64_t ldy, int M, int N, int K, int cus, hipStream_t stream);

// Epilogue applied to the tall GEMM's tile before the store, in the order of
// the reference graph (src/models/sam3/vision.hpp:186-241):
//   v = rs[m] * acc;  v += bias[n];  y[d] = res[d] + v
// where d is the output row: m itself, or row_map[m] (the grid row that a
// window-order row returns to, ggml_win_unpart).  res may alias y.
// Per-head attention operands [B*H][Np][64] fp16 (hi), and for the
// F32-accurate attention their remainders fp16(v - hi) (lo, all three;
// else null).
struct AttnOperands {
    _Float16 *q = nullptr, *k = nullptr, *v = nullptr;
    _Float16 *ql = nullptr, *kl = nullptr, *vl = nullptr;
};

struct Epilogue {
    const float* bias = nullptr;
    const float* res = nullptr;   // row stride = ldy
    const int* row_map = nullptr;
    // Packed attention operands instead of Y (an encoder block's qkv
    // product): column n = part*embed + h*64 + d of row m (window m / per,
    // token t = m % per) goes to pack[part][((window*heads + h)*np + t)*64 +
    // d] in fp16, q and k rotated by freqs[t] (complex RoPE, products
    // rounded before the add), q multiplied by q_scale.
    _Float16* pack[3] = {nullptr, nullptr, nullptr};
    _Float16* pack_lo[3] = {nullptr, nullptr, nullptr};   // with pack: fp16(v - fp16(v)) too
    const float* freqs = nullptr;
    int embed = 0, per = 0, np = 0, heads = 0;
    float q_scale = 1.f;
    // Per-column scale (multiplies with the row scale before the bias).
    const float* col_scale = nullptr;
    // 2x2 stride-2 transposed convolution: column n = tap*shuffle_c + c
    // (tap = 2*ky + kx) of input pixel m = y*shuffle_w + x goes to row
    // (2y+ky)*2*shuffle_w + 2x+kx, column c of Y (ldy = shuffle_c); the bias
    // is indexed by c.
    int shuffle_w = 0, shuffle_c = 0;
    bool gelu = false;   // ggml_gelu_erf after the bias
    // Q8_0 blocks instead of Y (with bias and gelu: an encoder block's fc1,
    // whose output only feeds fc2's Q8_0 packing): the 32 values of row m,
    // columns 32b .. 32b + 31 leave as their ggml Q8_0 codes
    // q8[m * q8_ld + 32b ..] and their F32 maximum magnitude
    // q8_amax[m * (q8_ld / 32) + b]; N and q8_ld are multiples of 32.
    int8_t* q8 = nullptr;
    float* q8_amax = nullptr;
    int64_t q8_ld = 0;
    bool q8_x86 = true;   // x86 rounding (127/amax, ties to even) or ggml's reference (1/d, ties away)
};
// How the A tile loader reads row m, logical column k (K columns) of A:
//   A_PLAIN : A[m][k] (lda halves per row);
//   A_REPEAT: split rows stored [hi | lo] (part halves each, lda = 2*part)
//             read as [hi | hi | lo] (K = 3*part);
//   A_CONV3 : a 3x3, stride-1, zero-padded convolution gathered from pixel
//             rows of a width x height map: A rows hold [v] or [hi | lo] of
//             `part` channels each (lda = part or 2*part); logical column
//             k = ((p*9 + tap)*part + c) reads physical part (p == 2) of
//             pixel (y+ky-1, x+kx-1), tap = 3*ky + kx, zero outside the map
//             (K = 9*part for one part, 27*part for [hi | hi | lo]).
// part is a multiple of 64 (of 128 for A_CONV3).
constexpr int A_PLAIN = 0, A_REPEAT = 1, A_CONV3 = 2;
struct AOperand {
    int mode = A_PLAIN;
    int part = 0;
    int width = 0, height = 0;
};
// Same product as launch_gemm_f16 with the shape's picked configuration and
// the epilogue; returns the configuration's name, or nullptr for an
// epilogue / operand combination without a kernel (plain A with: bias;
// bias + res; bias + res + row_map; bias + pack; bias + col_scale;
// bias + gelu + q8; or none;
// repeated A with bias + col_scale (+ shuffle (+ gelu)); gathered A with
// bias + col_scale are built).
const char* launch_gemm_f16_epi(const _Float16* a, int64_t lda, const float* row_scale, const _Float16* b,
                                int64_t ldb, float* y, int64_t ldy, int M, int N, int K, int cus, const Epilogue& ep,
                                hipStream_t stream, const AOperand& op = AOperand{});

// SAM 3 vision-encoder kernels (vit.hip).
// Layer norm over rows of E floats (E a multiple of 256): y[dst(r)] =
// ggml_norm(x[r] + add[tile(r)], eps) * w + b, with `add` (nullable) tiled
// with period `add_grid` over the gw x gh grid, and dst(r) the window-order
// row of grid row r when ws > 0 (else r).
void launch_layer_norm(const float* x, const float* add, int add_grid, int gw, int gh, int ws, const float* w,
                       const float* b, float eps, float* y, int rows, int E, hipStream_t stream);
// q/k/v rows (row b*N + n, stride ld floats, head h at columns h*64) ->
// per-head operands [B][H][Np][64] fp16: Q (RoPE, times q_scale), K (RoPE),
// V, Np = N rounded up to 64 with zero padding; freqs (nullable):
// [N][32][2] (cos, sin).  With the lo pointers set each value v is also
// written as fp16(v - fp16(v)), for the F32-accurate attention.
void launch_pack_qkv(const float* q, const float* k, const float* v, int64_t ld, const float* freqs, float q_scale,
                     const AttnOperands& o, int B, int H, int N, hipStream_t stream);
// Zero the padding rows [N, Np) of the packed operands.
void launch_zero_pad(const AttnOperands& o, int B, int H, int N, hipStream_t stream);
// softmax(Q K^T) V per (batch, head) on the packed operands (head dim 64);
// out row b*N + n, columns h*64.. (row stride ldo floats).  F32-accurate
// (split operands, three products each) when o carries the lo parts.
// softmax(Q K^T) V; when the grid is small against the CUs (SAM 3's global
// blocks), the keys are split over S (up to 4) workgroups per query block
// whose partials go through `scratch` (attention_scratch_bytes(.., S) bytes)
// and are merged in split order by a second launch.  The caller picks S once
// with attention_splits (force > 0 fixes it: SAMHIP_ATTN_SPLITS; B * S stays
// within the grid's 65535 z limit) and sizes the scratch from the same S;
// launch_attention returns false, launching nothing, when the scratch is
// smaller or B * S exceeds the limit.
int attention_splits(int B, int H, int N, bool precise, int cus, int force);
size_t attention_scratch_bytes(int B, int H, int N, int S);
bool launch_attention(const AttnOperands& o, float* out, int64_t ldo, int B, int H, int N, int S, float* scratch,
                      size_t scratch_bytes, hipStream_t stream);
// Patch convolution operands as split fp16: A [T][3*Kp] = [hi | hi | lo] of
// the image patches, W [E][3*Kp] = [hi | lo | hi] of the kernel rows, so
// A W^T = hi*hi + hi*lo + lo*hi (F32-accurate); Kp = 3*p*p rounded up to 128.
void launch_patch_columns(const float* image, int img, int patch, _Float16* a, float* row_scale, int kp,
                          hipStream_t stream);
void launch_patch_kernel(const float* kernel, int E, int patch, _Float16* w, int kp, hipStream_t stream);

// SimpleFPN neck operands (neck.hip).  A rows: output row r of a chunk
// starting at row0 reads its K values from x (pixel rows of C floats, a W x
// H map) as
//   NECK_ROWS   : pixel row0 + r                                 (K = C)
//   NECK_POOL   : max over the 2x2 block of output pixel row0 + r (K = C,
//                 output map W/2 x H/2)
//   NECK_IM2COL3: column tap*C + c = pixel (y+ky-1, x+kx-1) channel c,
//                 zero outside the map, tap = 3*ky + kx          (K = 9 C)
// and writes, for split, [hi | lo] of v * 2^-e (e from the row's largest
// magnitude, hi = fp16, lo = fp16 of the remainder, row_scale = 2^e; rows of
// 2*kp halves, read as A_REPEAT), else fp16(v) (row_scale 1, rows of kp
// halves).
// Columns K..kp-1 are zero.  C is a multiple of 4.
constexpr int NECK_ROWS = 0, NECK_POOL = 1, NECK_IM2COL3 = 2;
void launch_neck_columns(int src, bool split, const float* x, int W, int H, int C, int kp, int64_t row0, int rows,
                         _Float16* a, float* row_scale, hipStream_t stream);
// Operand rows of a whole map (rows pixels of C floats, C a multiple of 4)
// for A_CONV3: split [hi | lo] of v * 2^-e with one e from the map's largest
// magnitude (row_scale = 2^e on every row; `partial` holds 1024 floats),
// else fp16(v) (row_scale 1).
void launch_neck_pixels(bool split, const float* x, int64_t rows, int C, _Float16* a, float* row_scale,
                        float* partial, hipStream_t stream);
// B rows from ggml convolution weights:
//   conv   {k, k, Cin, Cout}: row co, column tap*Cin + ci (tap = k*ky + kx)
//   deconv {2, 2, Cout, Cin}: row tap*Cout + co (tap = 2*ky + kx), column ci
// split: [hi | lo | hi] of w * 2^-e per row (col_scale = 2^e), else
// fp16(w) (col_scale 1).  Transposed convolutions are always split and use
// `partial` (ceil(Cin/64) * 4 * Cout floats) for their row maxima.
void launch_neck_weights(bool deconv, bool split, const float* w, int k, int cin, int cout, int kp, _Float16* b,
                         float* col_scale, float* partial, hipStream_t stream);

// The producing graph node folded into a tall product's activation staging:
// PRE_GELU stages gelu_erf(x) (ggml_gelu_erf), PRE_LAYER_NORM stages
// ggml_norm(x, eps) * w + b, its rows leaving in window order (ggml_win_part
// of a gw-wide grid) when ws > 0.  The packed operand is the one the
// separate node's F32 output would have produced.
constexpr int PRE_NONE = 0, PRE_GELU = 1, PRE_LAYER_NORM = 2;
struct RowPre {
    int kind = PRE_NONE;
    const float* w = nullptr;
    const float* b = nullptr;
    float eps = 0.f;
    int ws = 0, gw = 1;
};

// Activation staging and weight decode of a tall product in one launch
// (16-byte aligned activation rows, K <= 5120); false when not applicable.
bool launch_prep(int mode, int wtype, const float* x, int64_t x_stride, int M, int K, _Float16* a, int64_t lda,
                 float* row_scale, int x86, const void* w, int64_t w_stride, int N, _Float16* wout, int64_t ldo,
                 hipStream_t stream, const RowPre& pre = RowPre{});
// The same for a Q8_0 weight whose activation rows arrive as Q8_0 codes
// [M][ldc] and F32 block maxima [M][ldc / 32] (Epilogue::q8): the fp16
// operand and row scales launch_prep gives for the F32 rows these codes
// pack; false when not applicable.
bool launch_prep_codes(const int8_t* codes, const float* amax, int64_t ldc, int M, int K, _Float16* a, int64_t lda,
                       float* row_scale, int wtype, const void* w, int64_t w_stride, int N, _Float16* wout,
                       int64_t ldo, hipStream_t stream);

// Kernel variant name for a weight type, or nullptr when unsupported.
const char* gemm_variant(int wtype);

// Returns the kernel variant name, or nullptr for an unsupported type.
const char* launch_gemm(int wtype, const _Float16* a, int64_t lda, const float* row_scale, const void* w,
                        int64_t w_stride, float* y, int64_t ldy, int M, int N, int K, hipStream_t stream);

// Skinny / medium products (M <= kSkinnyMaxM): weights decoded in registers,
// one pass over the packed bytes.  Returns the variant name, or nullptr.
constexpr int kSkinnyMaxM = 256;
const char* skinny_variant(int wtype, int M, int N);
const char* launch_skinny(int wtype, const _Float16* a, int64_t lda, const float* row_scale, const void* w,
                          int64_t w_stride, float* y, int64_t ldy, int M, int N, int K, hipStream_t stream);

// Fused skinny products (M <= kFusedMaxM, in blocks of 128 activation rows):
// activation packing, weight decode and product in one launch; when the K
// range is split over workgroups their partial sums go through `part`
// (FusedPlan::part_bytes) and a second, small launch adds them.
constexpr int kFusedMaxM = 256;
// ... and any M when the weight has at most this many elements
constexpr int64_t kFusedSmallW = 256 * 256;
struct FusedPlan {
    int rg, splits, cps;
    int mt;               // 32-row activation tiles per row block (fused kernel)
    size_t part_bytes;
};
FusedPlan fused_skinny_plan(int M, int N, int K, int max_splits, int cus);
const char* fused_skinny_variant(int wtype);
const char* launch_fused_skinny(int wtype, bool f16, const float* x, int64_t ldx, const void* w, int64_t w_stride,
                                float* y, int64_t ldy, float* part, int M, int N, int K, int x86, int max_splits,
                                int cus, hipStream_t stream);

// Strip skinny products (M < kStripMaxM): one launch per product while
// K <= 1024 (four 256-wide chunks per workgroup), plus the split-K reduce
// beyond; partial sums go through `part` (FusedPlan::part_bytes).
// The dispatch counts work-items in 32 bits: a grid of 1024-thread
// workgroups may hold at most this many.
constexpr int64_t kMaxWorkgroups1024 = int64_t(0xffffffffu) / 1024;

// Many activation rows against a Q8_0 weight that fits in LDS whole (the
// fusion / decoder image-token projections, K = 256, N <= 256): exact int8,
// one workgroup per CU with an even run of rows.  The packed rows must be
// contiguous (w_stride = row bytes) and 16-byte aligned.
constexpr int kTallSmallMaxN = 256, kTallSmallK = 256;
bool tall_small_i8_supported(int M, int N, int K, const void* w, int64_t w_stride);
const char* tall_small_i8_variant();
const char* launch_tall_small_i8(const float* x, int64_t ldx, const void* w, int64_t w_stride, float* y, int64_t ldy,
                                 int M, int N, int K, int x86, int cus, hipStream_t stream);
// The same for Q4_K / Q5_K / Q6_K weights (one super-block per row), with
// ggml's native arithmetic (Q8_K activation codes, exact integer sums).
bool tall_small_kq_i8_supported(int wtype, int M, int N, int K, const void* w, int64_t w_stride);
const char* tall_small_kq_i8_variant(int wtype);
const char* launch_tall_small_kq_i8(int wtype, const float* x, int64_t ldx, const void* w, int64_t w_stride, float* y,
                                    int64_t ldy, int M, int N, int K, int cus, hipStream_t stream);

// Exact tall products for Q8_0 weights (gemm_i8.hip): activations and the
// weight split per call into int8 codes and F32 block scales (staging of
// gemm_i8_staging_bytes), then an int8-MFMA GEMM with ggml's per-block
// scaling in K order.  K a multiple of 64.  Returns the GEMM's name and the
// staging launch's name in *prep_name.
bool gemm_i8_supported(int M, int N, int K);
size_t gemm_i8_staging_bytes(int M, int N, int K);
const char* gemm_i8_variant();
const char* launch_gemm_i8(const float* x, int64_t ldx, const void* w, int64_t w_stride, float* y, int64_t ldy, int M,
                           int N, int K, int x86, void* staging, hipStream_t stream, const char** prep_name);

constexpr int kStripMaxM = 256;   // in blocks of 32 activation rows
// Where the strip kernel measured faster than the fused one: Q8_0 weights
// with K <= 1024 (one launch).  K-quant pieces are read with scattered
// per-lane loads and K > 1024 adds the reduce launch back.
inline bool strip_skinny_preferred(int wtype, int M, int K) { return wtype == T_Q8_0 && K <= 1024 && M <= 32; }
FusedPlan strip_skinny_plan(int M, int N, int K);
// Exact int8 products of Q8_0 weights in blocks of 32 activation rows
// (COMPUTE_Q8_NATIVE).  A workgroup takes a K slice of 256 * slice_sb values
// (slice_sb 1, 2 or 4, from i8_strip_slice_sb); with more than one slice the
// partial sums go through `part` (i8_strip_part_bytes) and a reduce launch.
constexpr int kI8SliceK = 1024;   // widest K slice
// 256-value units of K per workgroup (1, 2 or 4): the fewest whose grid of
// row groups x K slices x row blocks still fits one workgroup per CU, so a
// workgroup's chain of loads, packing and epilogue stays as short as the
// chip allows; 4 when no choice fits.  Q8_0 packs 32-value blocks, a short
// chain, so with K <= 1024 it keeps one slice unless 256-wide ones fit
// (graph replay, M = 32, K = 1024: N = 1024 7.6 -> 7.1 us with four slices;
// N = 4096 7.8 us in one slice, 8.8 in two plus the reduce launch; at
// K = 4096, N = 1024 512-wide slices take 8.8 us against 9.9).
inline int i8_strip_slice_sb(int wtype, int M, int N, int K, int cus) {
    const int64_t rows = int64_t((N + 31) / 32) * ((M + 31) / 32);
    const auto fits = [&](int sb) { return rows * ((K + 256 * sb - 1) / (256 * sb)) <= cus; };
    if (fits(1)) return 1;
    if (wtype == T_Q8_0 && K <= kI8SliceK) return kI8SliceK / 256;
    return fits(2) ? 2 : kI8SliceK / 256;
}
inline size_t i8_strip_part_bytes(int M, int N, int K, int slice_sb) {
    const int S = (K + 256 * slice_sb - 1) / (256 * slice_sb);
    return S > 1 ? size_t(S) * size_t(M) * size_t(N) * 4 : 0;
}
const char* q8_strip_i8_variant();
// two_tiles: 64 weight rows per workgroup when a K slice holds at most 256
// values (two 32-row column tiles; the same bits as 32 rows per workgroup).
// Taken where 32-row workgroups need a second round of the chip and 64-row
// ones fit one (the decoder's M = 201 FFN expansion, 256 -> 2048: 448
// workgroups become 224).  In the streams' replayed graphs, with each
// product's weight read cold, it measured slower where both fit one round
// (M = 201, 256x256: 0.241 -> 0.252 ms per step; text out_proj, four
// 256-wide slices: text stream 476 -> 472 GB/s).
inline bool i8_strip_two_tiles_preferred(int M, int N, int K, int slice_sb, int cus) {
    if (slice_sb != 1 && K > 256) return false;
    const int64_t blocks = int64_t((M + 31) / 32) * ((K + 256 * slice_sb - 1) / (256 * slice_sb));
    return blocks * ((N + 31) / 32) > cus && blocks * ((N + 63) / 64) <= cus;
}
const char* launch_q8_strip_i8(const float* x, int64_t ldx, const void* w, int64_t w_stride, float* y, int64_t ldy,
                               float* part, int M, int N, int K, int slice_sb, int x86, bool two_tiles,
                               hipStream_t stream);
// The same for Q4_K / Q5_K / Q6_K weights against Q8_K activation codes
// (K a multiple of 256; same partial-sum buffer, K slices of 256, 512 or 1024
// values).  Taken by default where it measured faster than the fused kernel
// (graph replay, one box): Q4_K and Q5_K when the grid of row groups x row
// blocks x 1024-wide K slices fits one workgroup per CU, e.g. the text
// encoder's M = 32 products (Q4_K K = 1024, N = 1024: 8.9 -> 7.3 us;
// N = 4096: 9.9 -> 9.6; K = 4096: 9.9 -> 9.6) and the decoder's M = 201 and
// M = 33 products on 256x256 weights (6.8 -> 5.0 us); Q6_K (two masked MFMAs
// per 32 values) only when 256-wide slices fit (N = 1024, K = 1024: 8.8 ->
// 7.7 us; with 512-wide slices N = 4096: 9.8 against 10.5 us).  A second
// round of workgroups makes it slower (Q4_K M = 201, N = 2048, K = 256: 9.2
// against 7.0 us).
// With K = 256 it also takes the products that fit one round only with 64
// weight rows per workgroup (the decoder's M = 201 FFN expansion, 256 ->
// 2048), two_tiles below.
inline bool kq_strip_i8_preferred(int wtype, int M, int N, int K, int cus, bool allow_two_tiles = true) {
    const int slice = wtype == T_Q6_K ? 256 : kI8SliceK;
    return int64_t((N + 31) / 32) * ((M + 31) / 32) * ((K + slice - 1) / slice) <= cus ||
           (allow_two_tiles && K == 256 && i8_strip_two_tiles_preferred(M, N, K, 1, cus));
}
const char* kq_strip_i8_variant(int wtype);
// two_tiles: 64 weight rows per workgroup when a K slice holds one
// super-block (two 32-row column tiles; the same bits as 32 rows).  isum:
// the integer form (per super-block integer sums, then ggml's F32 steps in
// K order: with one K slice the oracle's bits); otherwise F32 per sub-block.
const char* launch_kq_strip_i8(int wtype, const float* x, int64_t ldx, const void* w, int64_t w_stride, float* y,
                               int64_t ldy, float* part, int M, int N, int K, int slice_sb, bool two_tiles, bool isum,
                               hipStream_t stream);
const char* strip_skinny_variant(int wtype);
const char* launch_strip_skinny(int wtype, bool f16, const float* x, int64_t ldx, const void* w, int64_t w_stride,
                                float* y, int64_t ldy, float* part, int M, int N, int K, int x86, hipStream_t stream);

}  // namespace samhip
