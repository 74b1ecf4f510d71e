"""ctypes bridge to the CPU oracle (libggml_oracle.so) — TEST INFRASTRUCTURE ONLY.

The oracle restates ggml 0.26.0's CPU quantization and mul_mat arithmetic in C
(ggml_oracle.c) and the SAM 3 vision encoder graph built on it (vit_oracle.c).  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module; the product path never does.
"""

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libggml_oracle.so")

F32, F16, Q8_0, Q8_1, Q4_K, Q5_K, Q6_K, Q8_K = 0, 1, 8, 9, 12, 13, 14, 15
ROUND_REF, ROUND_X86 = 0, 1
BLOCK_ELEMS = {Q8_0: 32, Q8_1: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256, Q8_K: 256}
BLOCK_BYTES = {Q8_0: 34, Q8_1: 36, Q4_K: 144, Q5_K: 176, Q6_K: 210, Q8_K: 292}
NAMES = {Q8_0: "q8_0", Q8_1: "q8_1", Q4_K: "q4_K", Q5_K: "q5_K", Q6_K: "q6_K", Q8_K: "q8_K"}

_lib = None
_default_threads = None   # OpenMP's thread count when the library was loaded

NECK_FIELDS = ("s0_dc1_w", "s0_dc1_b", "s0_dc2_w", "s0_dc2_b", "s0_c1_w", "s0_c1_b", "s0_c3_w", "s0_c3_b",
               "s1_dc_w", "s1_dc_b", "s1_c1_w", "s1_c1_b", "s1_c3_w", "s1_c3_b",
               "s2_c1_w", "s2_c1_b", "s2_c3_w", "s2_c3_b", "s3_c1_w", "s3_c1_b", "s3_c3_w", "s3_c3_b")


class NeckWeights(ctypes.Structure):
    """or_neck_weights (vit_oracle.h)."""
    _fields_ = [(n, ctypes.c_void_p) for n in NECK_FIELDS]


class VitBlockWeights(ctypes.Structure):
    """or_vit_block_weights (vit_oracle.h)."""
    _fields_ = [(n, ctypes.c_void_p) for n in ("norm1_w", "norm1_b", "norm2_w", "norm2_b")] + \
               [(n, ctypes.c_int) for n in ("qkv_type", "proj_type", "fc1_type", "fc2_type")] + \
               [(n, ctypes.c_void_p) for n in ("qkv_w", "proj_w", "fc1_w", "fc2_w", "qkv_b", "proj_b", "fc1_b",
                                               "fc2_b", "freqs")]


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.or_fp32_to_fp16_rows.argtypes = [P, P, I64]
        L.or_fp16_to_fp32_rows.argtypes = [P, P, I64]
        L.or_rng_normal.argtypes = [ctypes.c_uint64, ctypes.c_float, ctypes.c_float, P, I64]
        L.or_quantize_q8_0.argtypes = [P, P, I64, I64, I]
        L.or_quantize_q8_k.argtypes = [P, P, I64, I64]
        L.or_quantize_chunk.argtypes = [I, P, P, I64, I64]
        L.or_quantize_chunk.restype = I64
        L.or_dequantize.argtypes = [I, P, P, I64, I64]
        L.or_kquant_fit.argtypes = [I, P, P, P, P]
        L.or_quantize_q8_1.argtypes = [P, P, I64, I64]
        L.or_q8_1_mmq_bytes.argtypes = [I64, I64]
        L.or_q8_1_mmq_bytes.restype = I64
        L.or_quantize_q8_1_mmq.argtypes = [P, P, I64, I64]
        L.or_q8_rhs_supported.argtypes = [P, I64, I64]
        L.or_vec_dot.argtypes = [I, P, P, I64]
        L.or_vec_dot.restype = ctypes.c_float
        L.or_mul_mat_native.argtypes = [I, P, ctypes.c_size_t, P, ctypes.c_size_t, P, I64, I64, I64, I, I]
        L.or_mul_mat_decode.argtypes = [I, P, ctypes.c_size_t, P, ctypes.c_size_t, P, I64, I64, I64, I]
        L.or_gemm_f64.argtypes = [P, P, P, I64, I64, I64, I]
        L.or_max_threads.restype = I
        L.or_layer_norm.argtypes = [P, P, I64, I64, P, P, ctypes.c_float, I]
        L.or_gelu_erf.argtypes = [P, P, I64]
        L.or_win_part.argtypes = [P, P, I, I, I, I]
        L.or_win_unpart.argtypes = [P, P, I, I, I, I]
        L.or_rope.argtypes = [P, I64, I64, I, I, P]
        L.or_attention.argtypes = [P, P, P, I64, I64, I, I, ctypes.c_float, P, I]
        L.or_vit_block.argtypes = [ctypes.POINTER(VitBlockWeights), P, P, I, I, I, I, I, I, I, I, I]
        L.or_vit_prefix.argtypes = [P, I, I, P, P, I, P, P, I, P, I]
        L.or_deconv2x2.argtypes = [P, I, I, I, P, P, I, P, I]
        L.or_conv2d.argtypes = [P, I, I, I, P, P, I, I, P, I]
        L.or_conv2d_cols.argtypes = [P, I, I, I, P, P, I, I, I, P, I]
        L.or_maxpool2x2.argtypes = [P, I, I, I, P]
        L.or_neck.argtypes = [ctypes.POINTER(NeckWeights), P, I, I, I, I, I, ctypes.POINTER(P), I]
        _lib = L
        # every entry point with threads > 0 calls omp_set_num_threads, which
        # persists: remember the process default before any call changes it
        global _default_threads
        _default_threads = L.or_max_threads()
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def row_bytes(qtype, k):
    return k // BLOCK_ELEMS[qtype] * BLOCK_BYTES[qtype]


def fp32_to_fp16_bits(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().or_fp32_to_fp16_rows(_ptr(x), _ptr(out), x.size)
    return out


def fp16_bits_to_fp32(h):
    h = np.ascontiguousarray(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().or_fp16_to_fp32_rows(_ptr(h), _ptr(out), h.size)
    return out


def rng_normal(seed, n, mean=0.0, std=1.0):
    out = np.empty(int(n), np.float32)
    lib().or_rng_normal(seed, mean, std, _ptr(out), out.size)
    return out


def quantize(qtype, x, rounding=ROUND_REF):
    """ggml quantize rows: Q8_0 (ref or x86 rounding), Q8_K, or the K-quant weight quantizers."""
    x = np.ascontiguousarray(x, np.float32)
    rows, k = x.shape
    out = np.zeros((rows, row_bytes(qtype, k)), np.uint8)
    if qtype == Q8_0:
        rc = lib().or_quantize_q8_0(_ptr(x), _ptr(out), rows, k, rounding)
    elif qtype == Q8_K:
        rc = lib().or_quantize_q8_k(_ptr(x), _ptr(out), rows, k)
    elif qtype == Q8_1:
        rc = lib().or_quantize_q8_1(_ptr(x), _ptr(out), rows, k)
    else:
        rc = 0 if lib().or_quantize_chunk(qtype, _ptr(x), _ptr(out), rows, k) == out.size else -1
    if rc:
        raise ValueError("oracle quantize rejected shape")
    return out


def kquant_fit(qtype, x256):
    """First phase of a K-quant weight quantizer on one super-block:
    (scales, mins, codes) — mins is None for Q6_K."""
    x = np.ascontiguousarray(x256, np.float32).reshape(256)
    n = 16 if qtype == Q6_K else 8
    scales = np.zeros(n, np.float32)
    mins = np.zeros(n, np.float32)
    codes = np.zeros(256, np.uint8)
    if lib().or_kquant_fit(qtype, _ptr(x), _ptr(scales), _ptr(mins), _ptr(codes)):
        raise ValueError("oracle kquant_fit: not a K-quant type")
    return scales, (None if qtype == Q6_K else mins), codes


def quantize_q8_1_mmq(x):
    """ggml-cuda MMQ D4 staging: bytes [ceil(k/512)*4][rows][144]."""
    x = np.ascontiguousarray(x, np.float32)
    rows, k = x.shape
    out = np.zeros(int(lib().or_q8_1_mmq_bytes(rows, k)), np.uint8)
    if lib().or_quantize_q8_1_mmq(_ptr(x), _ptr(out), rows, k):
        raise ValueError("oracle quantize_q8_1_mmq rejected shape")
    return out


def q8_rhs_supported(x):
    x = np.ascontiguousarray(x, np.float32)
    rows, k = x.shape
    return bool(lib().or_q8_rhs_supported(_ptr(x), rows, k))


def dequantize(qtype, packed, k):
    packed = np.ascontiguousarray(packed, np.uint8)
    rows = packed.size // row_bytes(qtype, k)
    out = np.empty((rows, k), np.float32)
    if lib().or_dequantize(qtype, _ptr(packed), _ptr(out), rows, k):
        raise ValueError("oracle dequantize rejected shape")
    return out


def mul_mat_native(qtype, w_packed, x, rounding=ROUND_X86, threads=0):
    w_packed = np.ascontiguousarray(w_packed, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    m, k = x.shape
    n = w_packed.shape[0]
    y = np.empty((m, n), np.float32)
    if lib().or_mul_mat_native(qtype, _ptr(w_packed), w_packed.shape[1], _ptr(x), k, _ptr(y), n, m, k,
                               rounding, threads):
        raise ValueError("oracle native mul_mat rejected shape")
    return y


def mul_mat_decode(qtype, w_packed, x, threads=0):
    w_packed = np.ascontiguousarray(w_packed, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    m, k = x.shape
    n = w_packed.shape[0]
    y = np.empty((m, n), np.float32)
    if lib().or_mul_mat_decode(qtype, _ptr(w_packed), w_packed.shape[1], _ptr(x), k, _ptr(y), n, m, k, threads):
        raise ValueError("oracle decode mul_mat rejected shape")
    return y


def gemm_f64(w, x, threads=0):
    w = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    n, k = w.shape
    m = x.shape[0]
    y = np.empty((m, n), np.float64)
    lib().or_gemm_f64(_ptr(w), _ptr(x), _ptr(y), n, m, k, threads)
    return y


def max_threads():
    """The host threads OpenMP would use by default (OMP_NUM_THREADS, else
    every core), as read when the library was loaded, so a call made with an
    explicit smaller count does not shrink what later callers get."""
    lib()
    return _default_threads


# ---- SAM 3 vision encoder pieces (vit_oracle.c) ----------------------------

def _f32(a):
    return np.ascontiguousarray(a, np.float32)


def layer_norm(x, w=None, b=None, eps=1e-5, threads=0):
    x = _f32(x)
    y = np.empty_like(x)
    n = x.shape[-1]
    lib().or_layer_norm(_ptr(x), _ptr(y), x.size // n, n, None if w is None else _ptr(_f32(w)),
                        None if b is None else _ptr(_f32(b)), eps, threads)
    return y


def gelu_erf(x):
    x = _f32(x)
    y = np.empty_like(x)
    lib().or_gelu_erf(_ptr(x), _ptr(y), x.size)
    return y


def win_part(x, W, H, ws):
    x = _f32(x)
    C = x.shape[-1]
    n = ((W + ws - 1) // ws) * ((H + ws - 1) // ws) * ws * ws
    y = np.empty((n, C), np.float32)
    lib().or_win_part(_ptr(x), _ptr(y), W, H, C, ws)
    return y


def win_unpart(y, W, H, ws):
    y = _f32(y)
    C = y.shape[-1]
    x = np.empty((W * H, C), np.float32)
    lib().or_win_unpart(_ptr(y), _ptr(x), W, H, C, ws)
    return x


def rope(x, heads, hd, freqs):
    """x: [tokens][ld] (first heads*hd columns roped, returned as a copy)."""
    x = _f32(x).copy()
    lib().or_rope(_ptr(x), x.shape[1], x.shape[0], heads, hd, _ptr(_f32(freqs)))
    return x


def attention(q, k, v, heads, hd, scale, threads=0):
    """q, k, v: [n][heads*hd] each."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    n, ld = q.shape
    assert k.shape == q.shape and v.shape == q.shape and ld == heads * hd
    out = np.empty((n, heads * hd), np.float32)
    lib().or_attention(_ptr(q), _ptr(k), _ptr(v), ld, n, heads, hd, scale, _ptr(out), threads)
    return out


def vit_block(weights, x, W, H, E, heads, mlp, ws, rounding=ROUND_X86, threads=0, decode=False):
    """weights: dict with norm1_w/b, norm2_w/b, {qkv,proj,fc1,fc2}_{type,w,b}, freqs (numpy arrays)."""
    keep = {}

    def p(name, dtype):
        a = weights.get(name)
        if a is None:
            return None
        a = np.ascontiguousarray(a, dtype)
        keep[name] = a
        return _ptr(a)

    s = VitBlockWeights()
    for n in ("norm1_w", "norm1_b", "norm2_w", "norm2_b", "qkv_b", "proj_b", "fc1_b", "fc2_b", "freqs"):
        setattr(s, n, p(n, np.float32))
    for n in ("qkv", "proj", "fc1", "fc2"):
        setattr(s, n + "_type", weights[n + "_type"])
        setattr(s, n + "_w", p(n + "_w", np.uint8))
    x = _f32(x)
    y = np.empty_like(x)
    if lib().or_vit_block(ctypes.byref(s), _ptr(x), _ptr(y), W, H, E, heads, mlp, ws, rounding, int(decode), threads):
        raise ValueError("oracle vit block rejected its arguments")
    return y


def vit_prefix(image, patch, kernel, pos, pos_grid, ln_w, ln_b, E, threads=0):
    """image: [3][img][img] (ggml {img, img, 3}); kernel: [E][3][p][p]; pos: [pg][pg][E]."""
    image = _f32(image)
    img = image.shape[-1]
    grid = img // patch
    out = np.empty((grid * grid, E), np.float32)
    if lib().or_vit_prefix(_ptr(image), img, patch, _ptr(_f32(kernel)), _ptr(_f32(pos)), pos_grid, _ptr(_f32(ln_w)),
                           _ptr(_f32(ln_b)), E, _ptr(out), threads):
        raise ValueError("oracle vit prefix rejected its arguments")
    return out


# ---- SimpleFPN neck ----------------------------------------------------------

def deconv2x2(x, W, H, w, b, cout, threads=0):
    """x: [H*W][Cin]; w: ggml {2, 2, Cout, Cin} flat."""
    x = _f32(x)
    out = np.empty((4 * W * H, cout), np.float32)
    lib().or_deconv2x2(_ptr(x), W, H, x.shape[1], _ptr(_f32(w)), None if b is None else _ptr(_f32(b)), cout,
                       _ptr(out), threads)
    return out


def conv2d(x, W, H, w, b, cout, k, threads=0, columns_f16=False):
    """x: [H*W][Cin]; w: ggml {k, k, Cin, Cout} flat; columns_f16 rounds both operands to fp16."""
    x = _f32(x)
    out = np.empty((W * H, cout), np.float32)
    lib().or_conv2d_cols(_ptr(x), W, H, x.shape[1], _ptr(_f32(w)), None if b is None else _ptr(_f32(b)), cout, k,
                         int(columns_f16), _ptr(out), threads)
    return out


def maxpool2x2(x, W, H):
    x = _f32(x)
    out = np.empty((W * H // 4, x.shape[1]), np.float32)
    lib().or_maxpool2x2(_ptr(x), W, H, x.shape[1], _ptr(out))
    return out


def neck(weights, x, grid, E, mid, D, threads=0, columns_f16=False, levels=(0, 1, 2, 3)):
    """weights: dict of NECK_FIELDS numpy arrays (ggml layouts; those of
    skipped levels may be absent); returns the 4 maps (None when skipped)."""
    keep = {n: _f32(weights[n]) for n in NECK_FIELDS if n in weights}
    s = NeckWeights(*[_ptr(keep[n]) if n in keep else None for n in NECK_FIELDS])
    sides = (4 * grid, 2 * grid, grid, grid // 2)
    outs = [np.empty((sides[i] ** 2, D), np.float32) if i in levels else None for i in range(4)]
    arr = (ctypes.c_void_p * 4)(*[None if o is None else _ptr(o) for o in outs])
    if lib().or_neck(ctypes.byref(s), _ptr(_f32(x)), grid, E, mid, D, int(columns_f16), arr, threads):
        raise ValueError("oracle neck rejected its arguments")
    return outs
