"""ctypes bridge to the CPU oracle (libggml_oracle.so) — TEST INFRASTRUCTURE ONLY.

The oracle restates ggml 0.26.0's CPU quantization and mul_mat arithmetic in C
(ggml_oracle.c).  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module; the product path never does.
"""

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libggml_oracle.so")

F32, F16, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K = 0, 1, 8, 12, 13, 14, 15
ROUND_REF, ROUND_X86 = 0, 1
BLOCK_ELEMS = {Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256, Q8_K: 256}
BLOCK_BYTES = {Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210, Q8_K: 292}
NAMES = {Q8_0: "q8_0", Q4_K: "q4_K", Q5_K: "q5_K", Q6_K: "q6_K", Q8_K: "q8_K"}

_lib = None


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
        L.or_vec_dot.argtypes = [I, P, P, I64]
        L.or_vec_dot.restype = ctypes.c_float
        L.or_mul_mat_native.argtypes = [I, P, ctypes.c_size_t, P, ctypes.c_size_t, P, I64, I64, I64, I, I]
        L.or_mul_mat_decode.argtypes = [I, P, ctypes.c_size_t, P, ctypes.c_size_t, P, I64, I64, I64, I]
        L.or_gemm_f64.argtypes = [P, P, P, I64, I64, I64, I]
        L.or_max_threads.restype = I
        _lib = L
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
    else:
        rc = 0 if lib().or_quantize_chunk(qtype, _ptr(x), _ptr(out), rows, k) == out.size else -1
    if rc:
        raise ValueError("oracle quantize rejected shape")
    return out


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
    return lib().or_max_threads()
