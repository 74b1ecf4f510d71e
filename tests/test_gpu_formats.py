"""ggml-cuda's right-operand formats and the native activation's range rule on
the device, against the oracle, through the C ABI.

Bars: Q8_1 rows and the MMQ D4 staging are bit-exact with the oracle (which
the CPU suite pins to the reference's known answers and verifier rules); the
range rule rejects exactly the inputs the reference's fail-closed check
rejects (tests/tools/test_native_activation.py:140-147) and, when enabled on
mul_mat, computes nothing for them."""

import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _rows(seed, rows, k):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, k)) * np.exp(rng.uniform(-12, 12, (rows, 1)))).astype(np.float32)
    x[1, :32] = 0.0
    x[2, :32] = [127.0, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5] + [0.0] * 25       # ties
    x[3, :32] = 0.0
    x[3, 0], x[3, 16], x[3, 1] = 2048.0, -2048.0, 2.0 ** -13                 # order-dependent sum
    x[4, min(40, k - 1)] = 3e38 / 1e10
    return x


def test_quantize_q8_1_bit_exact(gpu_ctx, oracle, samhip):
    say("case quantize q8_1")
    x = _rows(31, 41, 1024)
    got = gpu_ctx.quantize(samhip.Q8_1, x)
    ref = oracle.quantize(oracle.Q8_1, x)
    assert got.shape == ref.shape == (41, 32 * 36)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("k", [32, 640, 1024, 4736])
def test_quantize_q8_1_mmq_bit_exact(gpu_ctx, oracle, samhip, k):
    say("case quantize q8_1 mmq k", k)
    x = _rows(32 + k, 19, k)
    x = np.clip(x, -1e29, 1e29)
    x[np.abs(x) < 1e-29] = 0.0
    got = gpu_ctx.quantize_q8_1_mmq(x)
    ref = oracle.quantize_q8_1_mmq(x)
    assert got.size == ref.size == (k + 511) // 512 * 4 * 19 * 144
    assert np.array_equal(got, ref)


def test_quantize_q8_1_mmq_strided_source(gpu_ctx, oracle, samhip):
    say("case quantize q8_1 mmq strided")
    x = _rows(77, 6, 320)
    src = gpu_ctx.upload(np.pad(x, ((0, 0), (0, 64))))        # row stride 384 floats
    nbytes = samhip.lib().samhip_q8_1_mmq_bytes(6, 320)
    dst = gpu_ctx.alloc(nbytes)
    samhip.check(samhip.lib().samhip_quantize_rows_q8_1_mmq(gpu_ctx.handle, src.ptr, 384 * 4, dst.ptr, 6, 320))
    got = gpu_ctx.download(dst, (nbytes,), np.uint8)
    assert np.array_equal(got, oracle.quantize_q8_1_mmq(x))


@pytest.mark.parametrize("value", [np.nan, np.inf, -np.inf, 1e31, 1e-31, float(np.finfo(np.float32).tiny)])
def test_q8_1_mmq_fails_closed(gpu_ctx, samhip, value):
    say("case mmq range reject", value)
    x = np.ones((3, 96), np.float32)
    x[2, 32:64] = value
    with pytest.raises(samhip.InvalidArgument):
        gpu_ctx.quantize_q8_1_mmq(x)


@pytest.mark.parametrize("value", [0.0, 1e-30, -1e-30, 1e30, -1e30])
def test_q8_1_mmq_accepts_range_edges(gpu_ctx, oracle, samhip, value):
    say("case mmq range accept", value)
    x = np.full((2, 32), value, np.float32)
    assert np.array_equal(gpu_ctx.quantize_q8_1_mmq(x), oracle.quantize_q8_1_mmq(x))


def test_mul_mat_activation_check(samhip, oracle):
    say("case mul_mat activation check")
    rng = np.random.default_rng(41)
    k, n, m = 512, 96, 300
    w = oracle.quantize(oracle.Q4_K, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = rng.standard_normal((m, k)).astype(np.float32)
    with samhip.Context(0, samhip.COMPUTE_Q8_NATIVE, samhip.ROUND_X86) as ctx:
        ref = ctx.matmul(samhip.Q4_K, w, x)
        ctx.set_activation_check(True)
        assert np.array_equal(ctx.matmul(samhip.Q4_K, w, x), ref)       # a valid X passes unchanged
        wb, xb, yb = ctx.upload(w), ctx.upload(x), ctx.alloc(m * n * 4)
        sentinel = np.full((m, n), 7.0, np.float32)
        ctx.write(yb, sentinel)
        for bad in (np.nan, np.inf, 1e31, 1e-31):
            x2 = x.copy()
            x2[m // 2, 64:96] = bad
            ctx.write(xb, x2)
            with pytest.raises(samhip.InvalidArgument):
                ctx.mul_mat(samhip.tensor(samhip.Q4_K, k, n, wb.ptr), samhip.tensor(samhip.F32, k, m, xb.ptr),
                            samhip.tensor(samhip.F32, n, m, yb.ptr))
            assert np.array_equal(ctx.download(yb, (m, n), np.float32), sentinel)   # nothing computed
        ctx.set_activation_check(False)
        x2 = x.copy()
        x2[0, 0] = np.inf
        ctx.write(xb, x2)
        ctx.mul_mat(samhip.tensor(samhip.Q4_K, k, n, wb.ptr), samhip.tensor(samhip.F32, k, m, xb.ptr),
                    samhip.tensor(samhip.F32, n, m, yb.ptr))              # off: no check, no error
