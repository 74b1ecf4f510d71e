"""ctypes binding of libsamhip (include/samhip.h) for tests and bench.py.

This is a thin veneer over the C ABI, in the manner of the reference's own
ctypes bridge to its native CUDA cache encoder
(tools/quantize/cache_quantization.py:26-49).  There is no fallback: if
libsamhip.so is missing or no HIP device is visible, calls raise.
"""

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsamhip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "samhip.h")

ABI_VERSION = 1
F32, F16, Q8_0, Q8_1, Q4_K, Q5_K, Q6_K, Q8_K, I32 = 0, 1, 8, 9, 12, 13, 14, 15, 26
COMPUTE_Q8_NATIVE, COMPUTE_F16 = 0, 1
ROUND_X86, ROUND_REF = 0, 1
OK, ERR_INVALID_ARGUMENT, ERR_UNSUPPORTED, ERR_DEVICE, ERR_OUT_OF_MEMORY = 0, -1, -2, -3, -4
BLOCK_ELEMS = {F32: 1, F16: 1, Q8_0: 32, Q8_1: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256, Q8_K: 256, I32: 1}
BLOCK_BYTES = {F32: 4, F16: 2, Q8_0: 34, Q8_1: 36, Q4_K: 144, Q5_K: 176, Q6_K: 210, Q8_K: 292, I32: 4}
TYPE_NAMES = {Q8_0: "q8_0", Q8_1: "q8_1", Q4_K: "q4_K", Q5_K: "q5_K", Q6_K: "q6_K", Q8_K: "q8_K", F32: "f32",
              F16: "f16"}

# Every entry point the header declares, with its ctypes signature.
_P, _I, _I32, _I64, _SZ, _U32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t, ctypes.c_uint32


class Tensor(ctypes.Structure):
    _fields_ = [("type", ctypes.c_int32), ("ne", ctypes.c_int64 * 4), ("nb", ctypes.c_size_t * 4), ("data", ctypes.c_void_p)]


class Options(ctypes.Structure):
    _fields_ = [("version", ctypes.c_uint32), ("device", ctypes.c_int32), ("compute", ctypes.c_int32),
                ("q8_rounding", ctypes.c_int32)]


class ExecInfo(ctypes.Structure):
    _fields_ = [("version", ctypes.c_uint32), ("device", ctypes.c_int32),
                ("mul_mat_calls", ctypes.c_uint64), ("gemm_launches", ctypes.c_uint64),
                ("skinny_launches", ctypes.c_uint64), ("activation_launches", ctypes.c_uint64),
                ("get_rows_calls", ctypes.c_uint64), ("activation_payload_peak_bytes", ctypes.c_uint64),
                ("activation_allocation_peak_bytes", ctypes.c_uint64), ("kernel_variant", ctypes.c_char * 64),
                ("arithmetic_profile", ctypes.c_char * 48), ("device_name", ctypes.c_char * 64)]


class KernelRecord(ctypes.Structure):
    _fields_ = [("kernel", ctypes.c_char * 64), ("weight_type", ctypes.c_int32), ("m", ctypes.c_int64),
                ("n", ctypes.c_int64), ("k", ctypes.c_int64), ("ms", ctypes.c_float)]


class VitBlockDesc(ctypes.Structure):
    """samhip_vit_block_desc."""
    _fields_ = [("version", ctypes.c_int32), ("embed", ctypes.c_int32), ("heads", ctypes.c_int32),
                ("mlp", ctypes.c_int32), ("grid_w", ctypes.c_int32), ("grid_h", ctypes.c_int32),
                ("window", ctypes.c_int32)] + \
               [(n, ctypes.c_void_p) for n in ("norm1_w", "norm1_b", "norm2_w", "norm2_b")] + \
               [(n, Tensor) for n in ("qkv_w", "proj_w", "fc1_w", "fc2_w")] + \
               [(n, ctypes.c_void_p) for n in ("qkv_b", "proj_b", "fc1_b", "fc2_b", "freqs_cis")] + \
               [("attention_type", ctypes.c_int32)]


NECK_SCALE_FIELDS = ("deconv1_w", "deconv1_b", "deconv2_w", "deconv2_b", "conv1x1_w", "conv1x1_b", "conv3x3_w",
                     "conv3x3_b")


class NeckScale(ctypes.Structure):
    """samhip_neck_scale."""
    _fields_ = [(n, ctypes.c_void_p) for n in NECK_SCALE_FIELDS]


class VitNeckDesc(ctypes.Structure):
    """samhip_vit_neck_desc."""
    _fields_ = [("version", ctypes.c_int32), ("grid", ctypes.c_int32), ("embed", ctypes.c_int32),
                ("mid", ctypes.c_int32), ("dim", ctypes.c_int32), ("columns_type", ctypes.c_int32),
                ("scales", NeckScale * 4)]


class VitPrefixDesc(ctypes.Structure):
    """samhip_vit_prefix_desc."""
    _fields_ = [("version", ctypes.c_int32), ("image_size", ctypes.c_int32), ("patch", ctypes.c_int32),
                ("embed", ctypes.c_int32), ("pos_grid", ctypes.c_int32)] + \
               [(n, ctypes.c_void_p) for n in ("patch_w", "pos_embed", "ln_pre_w", "ln_pre_b")]


SIGNATURES = {
    "samhip_abi_version": ([], _I),
    "samhip_device_count": ([_P], _I),
    "samhip_context_create": ([ctypes.POINTER(Options), ctypes.POINTER(_P)], _I),
    "samhip_context_destroy": ([_P], None),
    "samhip_context_set_stream": ([_P, _P], _I),
    "samhip_synchronize": ([_P], _I),
    "samhip_buffer_alloc": ([_P, _SZ, ctypes.POINTER(_P)], _I),
    "samhip_buffer_free": ([_P, _P], _I),
    "samhip_tensor_set": ([_P, _P, _P, _SZ], _I),
    "samhip_tensor_get": ([_P, _P, _P, _SZ], _I),
    "samhip_supports_mul_mat": ([ctypes.POINTER(Tensor)] * 3, _I),
    "samhip_mul_mat": ([_P] + [ctypes.POINTER(Tensor)] * 3, _I),
    "samhip_mul_mat_noalloc": ([_P] + [ctypes.POINTER(Tensor)] * 3, _I),
    "samhip_get_rows": ([_P] + [ctypes.POINTER(Tensor)] * 3, _I),
    "samhip_quantize_rows": ([_P, _I32, _P, _SZ, _P, _I64, _I64, _I32], _I),
    "samhip_q8_1_mmq_bytes": ([_I64, _I64], _SZ),
    "samhip_quantize_rows_q8_1_mmq": ([_P, _P, _SZ, _P, _I64, _I64], _I),
    "samhip_context_set_activation_check": ([_P, _I], _I),
    "samhip_dequantize_rows": ([_P, _I32, _P, _SZ, _P, _I64, _I64], _I),
    "samhip_validate_quantized_payload": ([_I32, _I64, _I64, _P, _SZ], _I),
    "samhip_query": ([_P, ctypes.POINTER(ExecInfo)], _I),
    "samhip_last_error": ([ctypes.c_char_p, _SZ], _SZ),
    "samhip_trace_begin": ([_P, ctypes.c_char_p], _I),
    "samhip_trace_end": ([_P, ctypes.POINTER(KernelRecord), _SZ, ctypes.POINTER(_SZ)], _I),
    "samhip_trace_pause": ([_P, ctypes.c_int], _I),
    "samhip_capture_begin": ([_P], _I),
    "samhip_capture_end": ([_P, ctypes.POINTER(_P)], _I),
    "samhip_graph_launch": ([_P, _P], _I),
    "samhip_graph_destroy": ([_P], None),
    "samhip_vit_block": ([_P, ctypes.POINTER(VitBlockDesc), _P], _I),
    "samhip_vit_prefix": ([_P, ctypes.POINTER(VitPrefixDesc), _P, _P], _I),
    "samhip_vit_neck": ([_P, ctypes.POINTER(VitNeckDesc), _P, _P, _P, _P, _P], _I),
    "samhip_layer_norm": ([_P, _P, _P, _I64, _I64, _P, _P, ctypes.c_float], _I),
    "samhip_flash_attn": ([_P, _P, _P, _P, _I64, _P, _I64, _I64, _I32, _I32, ctypes.c_float], _I),
}

_lib = None


def lib():
    """Load libsamhip.so; raises if it was not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"libsamhip.so is not built ({LIB_PATH}); run __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        if L.samhip_abi_version() != ABI_VERSION:
            raise RuntimeError("libsamhip ABI version mismatch")
        _lib = L
    return _lib


class SamhipError(RuntimeError):
    def __init__(self, status, message):
        super().__init__(f"samhip status {status}: {message}")
        self.status = status


class InvalidArgument(SamhipError, ValueError):
    pass


def last_error():
    buf = ctypes.create_string_buffer(1024)
    lib().samhip_last_error(buf, 1024)
    return buf.value.decode(errors="replace")


def check(status):
    if status != OK:
        cls = InvalidArgument if status == ERR_INVALID_ARGUMENT else SamhipError
        raise cls(status, last_error())
    return status


def row_bytes(qtype, k):
    return k // BLOCK_ELEMS[qtype] * BLOCK_BYTES[qtype]


def device_count():
    n = ctypes.c_int(0)
    check(lib().samhip_device_count(ctypes.byref(n)))
    return n.value


def tensor(qtype, ne0, ne1, data, nb1=None):
    """A 2-D ggml tensor descriptor over device address `data`."""
    t = Tensor()
    t.type = qtype
    t.ne[0], t.ne[1], t.ne[2], t.ne[3] = ne0, ne1, 1, 1
    nb0 = BLOCK_BYTES[qtype]
    rb = row_bytes(qtype, ne0)
    t.nb[0] = nb0
    t.nb[1] = rb if nb1 is None else nb1
    t.nb[2] = t.nb[1] * ne1
    t.nb[3] = t.nb[2]
    t.data = data
    return t


def validate_quantized_payload(qtype, ne0, rows, payload):
    payload = np.ascontiguousarray(payload, np.uint8)
    return check(lib().samhip_validate_quantized_payload(qtype, ne0, rows, payload.ctypes.data, payload.nbytes))


class Buffer:
    def __init__(self, ctx, nbytes):
        self.ctx, self.nbytes = ctx, int(nbytes)
        p = ctypes.c_void_p()
        check(lib().samhip_buffer_alloc(ctx.handle, self.nbytes, ctypes.byref(p)))
        self.ptr = p.value

    def free(self):
        if self.ptr:
            check(lib().samhip_buffer_free(self.ctx.handle, self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr and self.ctx.handle:
                lib().samhip_buffer_free(self.ctx.handle, self.ptr)
        except Exception:
            pass


class Graph:
    """A captured sequence of calls (samhip_capture_begin / _end)."""

    def __init__(self, ctx, handle):
        self.ctx, self.handle = ctx, handle

    def launch(self):
        check(lib().samhip_graph_launch(self.ctx.handle, self.handle))

    def destroy(self):
        if self.handle:
            lib().samhip_graph_destroy(self.handle)
            self.handle = None


class Context:
    def __init__(self, device=0, compute=COMPUTE_Q8_NATIVE, q8_rounding=ROUND_X86):
        o = Options(ABI_VERSION, device, compute, q8_rounding)
        h = ctypes.c_void_p()
        check(lib().samhip_context_create(ctypes.byref(o), ctypes.byref(h)))
        self.handle = h.value

    def close(self):
        if self.handle:
            lib().samhip_context_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def set_stream(self, stream_handle):
        check(lib().samhip_context_set_stream(self.handle, stream_handle))

    def synchronize(self):
        check(lib().samhip_synchronize(self.handle))

    def alloc(self, nbytes):
        return Buffer(self, nbytes)

    def upload(self, array):
        a = np.ascontiguousarray(array)
        b = Buffer(self, max(a.nbytes, 1))
        check(lib().samhip_tensor_set(self.handle, b.ptr, a.ctypes.data, a.nbytes))
        return b

    def write(self, buf, array, offset=0):
        a = np.ascontiguousarray(array)
        check(lib().samhip_tensor_set(self.handle, buf.ptr + offset, a.ctypes.data, a.nbytes))

    def download(self, buf, shape, dtype, offset=0):
        out = np.empty(shape, dtype)
        check(lib().samhip_tensor_get(self.handle, out.ctypes.data, buf.ptr + offset, out.nbytes))
        return out

    def mul_mat(self, w, x, y):
        check(lib().samhip_mul_mat(self.handle, ctypes.byref(w), ctypes.byref(x), ctypes.byref(y)))

    def get_rows(self, src, ids, dst):
        check(lib().samhip_get_rows(self.handle, ctypes.byref(src), ctypes.byref(ids), ctypes.byref(dst)))

    def quantize_rows(self, qtype, src_ptr, src_stride, dst_ptr, rows, k, q8_rounding=ROUND_X86):
        check(lib().samhip_quantize_rows(self.handle, qtype, src_ptr, src_stride, dst_ptr, rows, k, q8_rounding))

    def dequantize_rows(self, qtype, src_ptr, src_stride, dst_ptr, rows, k):
        check(lib().samhip_dequantize_rows(self.handle, qtype, src_ptr, src_stride, dst_ptr, rows, k))

    def query(self):
        info = ExecInfo()
        check(lib().samhip_query(self.handle, ctypes.byref(info)))
        return info

    def trace_begin(self, kernel_filter=None):
        """Bracket launches (all, or those whose name contains kernel_filter) with HIP events."""
        check(lib().samhip_trace_begin(self.handle, kernel_filter.encode() if kernel_filter else None))

    def trace_pause(self, paused=True):
        """Stops (or resumes) bracketing launches of the open trace, without synchronizing."""
        check(lib().samhip_trace_pause(self.handle, 1 if paused else 0))

    def trace_end(self, capacity=1 << 16):
        """Returns [(kernel, weight_type, m, n, k, ms)] of the launches since trace_begin."""
        recs = (KernelRecord * capacity)()
        count = ctypes.c_size_t(0)
        check(lib().samhip_trace_end(self.handle, recs, capacity, ctypes.byref(count)))
        return [(r.kernel.decode(), r.weight_type, r.m, r.n, r.k, r.ms) for r in recs[:min(count.value, capacity)]]

    def capture_begin(self):
        check(lib().samhip_capture_begin(self.handle))

    def capture_end(self):
        """Ends the open capture; returns a Graph replayable on this context."""
        g = ctypes.c_void_p()
        check(lib().samhip_capture_end(self.handle, ctypes.byref(g)))
        return Graph(self, g.value)

    # -- numpy conveniences used by the tests ------------------------------
    def quantize(self, qtype, x, q8_rounding=ROUND_X86):
        x = np.ascontiguousarray(x, np.float32)
        rows, k = x.shape
        src = self.upload(x)
        dst = self.alloc(rows * row_bytes(qtype, k))
        self.quantize_rows(qtype, src.ptr, 4 * k, dst.ptr, rows, k, q8_rounding)
        return self.download(dst, (rows, row_bytes(qtype, k)), np.uint8)

    def quantize_q8_1_mmq(self, x):
        """samhip_quantize_rows_q8_1_mmq on a device copy of numpy rows x."""
        x = np.ascontiguousarray(x, np.float32)
        rows, k = x.shape
        nbytes = lib().samhip_q8_1_mmq_bytes(rows, k)
        src = self.upload(x)
        dst = self.alloc(nbytes)
        check(lib().samhip_quantize_rows_q8_1_mmq(self.handle, src.ptr, 4 * k, dst.ptr, rows, k))
        return self.download(dst, (nbytes,), np.uint8)

    def set_activation_check(self, enabled):
        check(lib().samhip_context_set_activation_check(self.handle, 1 if enabled else 0))

    def dequantize(self, qtype, packed, k):
        packed = np.ascontiguousarray(packed, np.uint8)
        rows = packed.size // row_bytes(qtype, k)
        src = self.upload(packed)
        dst = self.alloc(rows * k * 4)
        self.dequantize_rows(qtype, src.ptr, row_bytes(qtype, k), dst.ptr, rows, k)
        return self.download(dst, (rows, k), np.float32)

    def layer_norm(self, x, w=None, b=None, eps=1e-5):
        """samhip_layer_norm on a device copy of numpy rows x [rows][n]."""
        x = np.ascontiguousarray(x, np.float32)
        rows, n = x.shape
        xb, yb = self.upload(x), self.alloc(x.nbytes)
        wb = self.upload(np.ascontiguousarray(w, np.float32)) if w is not None else None
        bb = self.upload(np.ascontiguousarray(b, np.float32)) if b is not None else None
        check(lib().samhip_layer_norm(self.handle, xb.ptr, yb.ptr, rows, n, wb.ptr if wb else None,
                                      bb.ptr if bb else None, eps))
        return self.download(yb, (rows, n), np.float32)

    def flash_attn(self, q, k, v, batches, heads, scale, head_dim=64):
        """samhip_flash_attn on device copies of q, k, v [batches*n][heads*head_dim]."""
        q, k, v = (np.ascontiguousarray(a, np.float32) for a in (q, k, v))
        rows, ld = q.shape
        qb, kb, vb, ob = self.upload(q), self.upload(k), self.upload(v), self.alloc(rows * heads * head_dim * 4)
        check(lib().samhip_flash_attn(self.handle, qb.ptr, kb.ptr, vb.ptr, ld, ob.ptr, batches, rows // batches,
                                      heads, head_dim, scale))
        return self.download(ob, (rows, heads * head_dim), np.float32)

    def matmul(self, qtype, w_packed, x, w_row_offset=0, w_rows=None, x_row_stride=None):
        """Y = X W^T through samhip_mul_mat on device copies of numpy inputs.

        w_packed: [rows, row_bytes] uint8 (the whole packed tensor); the
        product uses rows [w_row_offset, w_row_offset + w_rows) as a view.
        x: [M, K] F32; with x_row_stride (floats) > K the rows are strided.
        """
        w_packed = np.ascontiguousarray(w_packed, np.uint8)
        x = np.ascontiguousarray(x, np.float32)
        m, k = x.shape
        rb = row_bytes(qtype, k)
        n = w_packed.shape[0] - w_row_offset if w_rows is None else w_rows
        wb = self.upload(w_packed)
        xs = k if x_row_stride is None else x_row_stride
        if xs != k:
            xp = np.full((m, xs), 91.0, np.float32)
            xp[:, :k] = x
        else:
            xp = x
        xb = self.upload(xp)
        yb = self.alloc(m * n * 4)
        wt = tensor(qtype, k, n, wb.ptr + w_row_offset * rb, nb1=rb)
        xt = tensor(F32, k, m, xb.ptr, nb1=4 * xs)
        yt = tensor(F32, n, m, yb.ptr)
        self.mul_mat(wt, xt, yt)
        return self.download(yb, (m, n), np.float32)


class VitBlock:
    """One SAM 3 ViT block's weights on the device (numpy arrays in, as
    produced for the oracle: norm*_w/b, {qkv,proj,fc1,fc2}_{type,w,b},
    freqs) and its samhip_vit_block descriptor."""

    def __init__(self, ctx, weights, embed, heads, mlp, grid_w, grid_h, window, attention_type=F32):
        self.ctx = ctx
        self.buffers = {}
        d = VitBlockDesc()
        d.version = ABI_VERSION
        d.embed, d.heads, d.mlp, d.grid_w, d.grid_h, d.window = embed, heads, mlp, grid_w, grid_h, window
        d.attention_type = attention_type
        for n in ("norm1_w", "norm1_b", "norm2_w", "norm2_b", "qkv_b", "proj_b", "fc1_b", "fc2_b"):
            self.buffers[n] = ctx.upload(np.ascontiguousarray(weights[n], np.float32))
            setattr(d, n, self.buffers[n].ptr)
        if weights.get("freqs") is not None:
            self.buffers["freqs"] = ctx.upload(np.ascontiguousarray(weights["freqs"], np.float32))
            d.freqs_cis = self.buffers["freqs"].ptr
        shapes = {"qkv": (embed, 3 * embed), "proj": (embed, embed), "fc1": (embed, mlp), "fc2": (mlp, embed)}
        for n, (k, rows) in shapes.items():
            qt = weights[n + "_type"]
            self.buffers[n] = ctx.upload(np.ascontiguousarray(weights[n + "_w"], np.uint8))
            setattr(d, n + "_w", tensor(qt, k, rows, self.buffers[n].ptr))
        self.desc = d

    def forward(self, x_buf):
        """Runs the block in place on device buffer x_buf."""
        check(lib().samhip_vit_block(self.ctx.handle, ctypes.byref(self.desc), x_buf.ptr))

    def free(self):
        for b in self.buffers.values():
            b.free()
        self.buffers = {}


class VitPrefix:
    """The ViT prefix weights on the device: patch kernel [E][3][p][p]
    (ggml {p, p, 3, E}), pos_embed [pg][pg][E], ln_pre w/b."""

    def __init__(self, ctx, patch_w, pos_embed, ln_w, ln_b, image_size, patch, embed, pos_grid):
        self.ctx = ctx
        self.buffers = {n: ctx.upload(np.ascontiguousarray(a, np.float32))
                        for n, a in (("patch_w", patch_w), ("pos_embed", pos_embed), ("ln_pre_w", ln_w),
                                     ("ln_pre_b", ln_b))}
        d = VitPrefixDesc()
        d.version = ABI_VERSION
        d.image_size, d.patch, d.embed, d.pos_grid = image_size, patch, embed, pos_grid
        for n, b in self.buffers.items():
            setattr(d, n, b.ptr)
        self.desc = d

    def forward(self, image_buf, x_buf):
        check(lib().samhip_vit_prefix(self.ctx.handle, ctypes.byref(self.desc), image_buf.ptr, x_buf.ptr))

    def free(self):
        for b in self.buffers.values():
            b.free()
        self.buffers = {}


class VitNeck:
    """The SimpleFPN neck weights on the device.  `scales` is a list of 4
    dicts keyed by NECK_SCALE_FIELDS (ggml layouts, absent keys unused);
    columns_type F32 (F32-accurate) or F16 (fp16 im2col operands)."""

    def __init__(self, ctx, scales, grid, embed, mid, dim, columns_type=F32):
        self.ctx = ctx
        self.buffers = {}
        d = VitNeckDesc()
        d.version = ABI_VERSION
        d.grid, d.embed, d.mid, d.dim, d.columns_type = grid, embed, mid, dim, columns_type
        for i, sc in enumerate(scales):
            for n in NECK_SCALE_FIELDS:
                if sc.get(n) is not None:
                    b = ctx.upload(np.ascontiguousarray(sc[n], np.float32))
                    self.buffers[(i, n)] = b
                    setattr(d.scales[i], n, b.ptr)
        self.desc = d
        self.grid, self.dim = grid, dim

    def level_rows(self, level):
        side = (4 * self.grid) >> level
        return side * side

    def forward(self, x_buf, levels):
        """levels: 4 device buffers (or None) of level_rows(i) x dim floats."""
        ptrs = [None if b is None else b.ptr for b in levels]
        check(lib().samhip_vit_neck(self.ctx.handle, ctypes.byref(self.desc), x_buf.ptr, *ptrs))

    def free(self):
        for b in self.buffers.values():
            b.free()
        self.buffers = {}
