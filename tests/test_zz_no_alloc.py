"""samhip_mul_mat_noalloc (the entry point for callers that cannot allocate)
against samhip_mul_mat through the C ABI: the same kernels run on the fixed
per-GPU scratch instead of the context's staging, so results must be
bit-identical.  Two calls in a row, the second with a smaller input, so
stale scratch contents from the first call would show; a product that needs
more scratch than the fixed array holds is rejected before anything runs."""

import ctypes
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _case(oracle, seed, qtype, m, n, k):
    rng = np.random.default_rng(seed)
    w = oracle.quantize(qtype, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = rng.standard_normal((m, k)).astype(np.float32)
    return w, x


def _both(samhip, ctx, qtype, w, x, n):
    m, k = x.shape
    wb, xb = ctx.upload(w), ctx.upload(x)
    ya, yb = ctx.alloc(m * n * 4), ctx.alloc(m * n * 4)
    W = samhip.tensor(qtype, k, n, wb.ptr)
    X = samhip.tensor(samhip.F32, k, m, xb.ptr)
    Ya, Yb = samhip.tensor(samhip.F32, n, m, ya.ptr), samhip.tensor(samhip.F32, n, m, yb.ptr)
    ctx.mul_mat(W, X, Ya)
    samhip.check(samhip.lib().samhip_mul_mat_noalloc(ctx.handle, ctypes.byref(W), ctypes.byref(X), ctypes.byref(Yb)))
    a = ctx.download(ya, (m, n), np.float32)
    b = ctx.download(yb, (m, n), np.float32)
    for buf in (wb, xb, ya, yb):
        buf.free()
    return a, b


# (first call, second smaller call): tall GEMM path, the int8 kernels with
# K slices (Q8_0 and K-quant, 32 and 64 weight rows per workgroup), the
# small-weight int8 kernels, the fused skinny kernel
PAIRS = [
    (("Q4_K", 5184, 256, 256), ("Q6_K", 1000, 255, 256)),         # small-weight K-quant kernel, twice
    (("Q4_K", 201, 2048, 256), ("Q8_0", 300, 100, 256)),          # K-quant strip, 64-row workgroups; small-weight Q8_0
    (("Q8_0", 5184, 1024, 4736), ("Q8_0", 2048, 1024, 4736)),     # ViT fc2: 59 MB of scratch, then 24 MB
    (("Q4_K", 5184, 4736, 1024), ("Q5_K", 1024, 3072, 1024)),     # ViT fc1, then a smaller qkv
    (("Q8_0", 201, 2048, 256), ("Q6_K", 33, 256, 256)),           # decoder fc1, then a prompt K/V product
    (("Q8_0", 32, 4096, 1024), ("Q8_0", 32, 1024, 4096)),         # text fc1 (strip), then fc2 (split K)
    (("Q4_K", 32, 1024, 4096), ("Q4_K", 32, 1024, 1024)),         # text fc2: eight 512-wide K slices, then four 256-wide
    (("Q6_K", 32, 4096, 1024), ("Q6_K", 17, 96, 512)),            # fused kernel, then int8 in two K slices
]


@pytest.mark.parametrize("pair", PAIRS, ids=lambda p: f"{p[0][0]}-{p[0][1]}x{p[0][2]}x{p[0][3]}")
def test_noalloc_matches_mul_mat_twice(samhip, oracle, pair):
    with samhip.Context(0, samhip.COMPUTE_Q8_NATIVE, samhip.ROUND_X86) as ctx:
        for i, (tname, m, n, k) in enumerate(pair):
            say("case noalloc", i, tname, m, n, k)
            qtype = getattr(samhip, tname)
            w, x = _case(oracle, 100 * i + m + n, qtype, m, n, k)
            a, b = _both(samhip, ctx, qtype, w, x, n)
            assert np.isfinite(a).all()
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_noalloc_rejects_products_beyond_the_scratch(samhip, oracle):
    say("case noalloc too large")
    qtype, m, n, k = samhip.Q8_0, 8 * 5184, 1024, 4736     # batch-8 fc2: ~400 MB of staging
    with samhip.Context(0, samhip.COMPUTE_Q8_NATIVE, samhip.ROUND_X86) as ctx:
        wb = ctx.alloc(n * samhip.row_bytes(qtype, k))
        xb, yb = ctx.alloc(m * k * 4), ctx.alloc(m * n * 4)
        ctx.write(yb, np.full((m, n), 3.0, np.float32))
        W = samhip.tensor(qtype, k, n, wb.ptr)
        X = samhip.tensor(samhip.F32, k, m, xb.ptr)
        Y = samhip.tensor(samhip.F32, n, m, yb.ptr)
        rc = samhip.lib().samhip_mul_mat_noalloc(ctx.handle, ctypes.byref(W), ctypes.byref(X), ctypes.byref(Y))
        assert rc == samhip.ERR_INVALID_ARGUMENT
        assert "scratch" in samhip.last_error()
        assert (ctx.download(yb, (m, n), np.float32) == 3.0).all()


def test_noalloc_calls_from_two_contexts_run_in_order(samhip, oracle):
    """Two contexts (two streams) on one thread call the no-allocation entry
    point back to back with no synchronization between: the second call's
    staging would overwrite the first one's in the shared array if they
    overlapped on the GPU.  The library's per-device event puts them in
    order, so both match their own samhip_mul_mat results bit for bit."""
    cases = [("Q8_0", 5184, 1024, 4736), ("Q4_K", 5184, 4736, 1024), ("Q8_0", 2048, 3072, 1024)]
    with samhip.Context(0, samhip.COMPUTE_Q8_NATIVE, samhip.ROUND_X86) as ca, \
            samhip.Context(0, samhip.COMPUTE_Q8_NATIVE, samhip.ROUND_X86) as cb:
        runs = []
        for i, (tname, m, n, k) in enumerate(cases):
            ctx = (ca, cb)[i % 2]
            qtype = getattr(samhip, tname)
            w, x = _case(oracle, 500 + i, qtype, m, n, k)
            wb, xb = ctx.upload(w), ctx.upload(x)
            ya, yb = ctx.alloc(m * n * 4), ctx.alloc(m * n * 4)
            W = samhip.tensor(qtype, k, n, wb.ptr)
            X = samhip.tensor(samhip.F32, k, m, xb.ptr)
            Ya, Yb = samhip.tensor(samhip.F32, n, m, ya.ptr), samhip.tensor(samhip.F32, n, m, yb.ptr)
            ctx.mul_mat(W, X, Ya)
            ctx.synchronize()
            runs.append((ctx, W, X, Ya, Yb, (wb, xb, ya, yb), m, n))
        for rep in range(2):
            say("case noalloc two contexts, pass", rep)
            for ctx, W, X, _, Yb, _, _, _ in (runs if rep == 0 else runs[::-1]):
                samhip.check(samhip.lib().samhip_mul_mat_noalloc(ctx.handle, ctypes.byref(W), ctypes.byref(X),
                                                                 ctypes.byref(Yb)))
            for ctx, _, _, _, _, bufs, m, n in runs:
                a = ctx.download(bufs[2], (m, n), np.float32)
                b = ctx.download(bufs[3], (m, n), np.float32)
                assert np.isfinite(a).all()
                assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        for run in runs:
            for buf in run[5]:
                buf.free()
