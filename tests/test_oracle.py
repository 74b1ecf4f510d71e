"""Pins the CPU oracle (a C restatement of ggml's CPU arithmetic) against the
reference's known-answer vectors, numpy's IEEE binary16 conversion, blocks
assembled field by field, closed-form bounds and double-precision brute force.
CPU only."""

import json
import os

import numpy as np
import pytest

from tests.reference_fixtures import (DECODED_TOL, NATIVE_TOL, matrix_values, probe_rhs, probe_weights, within)

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")))


def _block_from(spec, n=32):
    v = np.zeros(n, np.float32)
    for i, x in enumerate(spec):
        v[i] = np.nextafter(np.float32(0.5), np.float32(0)) if x == "nextafter(0.5,0)" else np.float32(x)
    return v


# ---- binary16 --------------------------------------------------------------

def test_fp16_to_fp32_exhaustive(oracle):
    h = np.arange(65536, dtype=np.uint16)
    got = oracle.fp16_bits_to_fp32(h)
    ref = h.view(np.float16).astype(np.float32)
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all()


def test_fp32_to_fp16_matches_numpy(oracle):
    rng = np.random.default_rng(0)
    x = rng.standard_normal(500_000).astype(np.float32) * (np.float32(10.0) ** rng.integers(-9, 6, 500_000)).astype(np.float32)
    edges = np.array([65504, 65519.996, 65520, 65536, 1e30, np.inf, -np.inf, 2.0 ** -25, 2.0 ** -24, 2.0 ** -14,
                      3 * 2.0 ** -26, 2.0 ** -25 * 1.0000001, -2.0 ** -25, 0.0, -0.0, 6.1e-5, 5.96e-8], np.float32)
    x = np.concatenate([x, edges])
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert (oracle.fp32_to_fp16_bits(x) == ref).all()


# ---- Q8_0 ------------------------------------------------------------------

@pytest.mark.parametrize("case", GOLDEN["q8_0_ref"])
def test_q8_0_reference_rounding_known_answers(oracle, case):
    x = np.zeros((1, 64), np.float32)
    x[0, :32] = _block_from(case["block"])
    if "second_block_linspace" in case:
        lo, hi = case["second_block_linspace"]
        x[0, 32:] = np.linspace(lo, hi, 32, dtype=np.float32)
    packed = oracle.quantize(oracle.Q8_0, x, oracle.ROUND_REF)
    assert packed.shape == (1, 68)
    codes = packed[0, 2:34].view(np.int8)
    assert codes[:len(case["codes"])].tolist() == case["codes"]


def test_q8_0_x86_rounding_known_answer(oracle):
    case = GOLDEN["q8_0_x86"][0]
    x = np.random.default_rng(39).normal(size=(1, 32)).astype(np.float32)
    x[0, :5] = case["block"]
    codes = oracle.quantize(oracle.Q8_0, x, oracle.ROUND_X86)[0, 2:34].view(np.int8)
    assert codes[:5].tolist() == case["codes"]
    # the reference rounding differs on the ties of this same block
    ref = oracle.quantize(oracle.Q8_0, x, oracle.ROUND_REF)[0, 2:34].view(np.int8)
    assert ref[:5].tolist() == [127, 1, -1, 2, -2]


@pytest.mark.parametrize("rounding", [0, 1])
def test_q8_0_extreme_known_answers(oracle, rounding):
    for blk in GOLDEN["q8_extremes"][0]["blocks"]:
        x = np.zeros((1, 32), np.float32)
        for i, v in blk["values"].items():
            x[0, int(i)] = v
        codes = oracle.quantize(oracle.Q8_0, x, rounding)[0, 2:34].view(np.int8)
        for i, c in blk["codes"].items():
            assert codes[int(i)] == c


@pytest.mark.parametrize("rounding", [0, 1])
def test_q8_0_closed_form_bounds(oracle, rounding):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((64, 256)) * np.exp(rng.uniform(-6, 6, (64, 1)))).astype(np.float32)
    packed = oracle.quantize(oracle.Q8_0, x, rounding).reshape(-1, 34)
    blocks = x.reshape(-1, 32)
    d = packed[:, :2].copy().view(np.float16).astype(np.float32)[:, 0]
    q = packed[:, 2:].view(np.int8).astype(np.int32)
    amax = np.abs(blocks).max(axis=1)
    assert np.array_equal(d, (amax / np.float32(127)).astype(np.float16).astype(np.float32))
    assert np.abs(q).max() <= 127
    arg = np.abs(blocks).argmax(axis=1)
    assert np.all(np.abs(q[np.arange(len(q)), arg]) == 127)
    # decoded error at most half a step of the unrounded scale (+ fp16 scale error)
    err = np.abs(q * (amax / 127)[:, None] - blocks)
    assert np.all(err <= (amax / 127)[:, None] * 0.5000001 + 1e-30)
    dec = oracle.dequantize(oracle.Q8_0, packed.reshape(64, -1), 256)
    assert np.array_equal(dec, (q * d[:, None]).astype(np.float32).reshape(64, 256))


def test_q8_0_requantize_is_idempotent(oracle):
    rng = np.random.default_rng(9)
    x = rng.standard_normal((32, 128)).astype(np.float32)
    p = oracle.quantize(oracle.Q8_0, x, oracle.ROUND_REF)
    p2 = oracle.quantize(oracle.Q8_0, oracle.dequantize(oracle.Q8_0, p, 128), oracle.ROUND_REF)
    assert np.array_equal(p, p2)


# ---- Q8_K ------------------------------------------------------------------

def test_q8_k_layout_and_invariants(oracle):
    lay = GOLDEN["q8_k_layout"]
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((16, 512)) * np.exp(rng.uniform(-5, 5, (16, 1)))).astype(np.float32)
    x[3, :256] = 0.0
    packed = oracle.quantize(oracle.Q8_K, x).reshape(-1, lay["block_bytes"])
    blocks = x.reshape(-1, 256)
    d = packed[:, 0:4].copy().view(np.float32)[:, 0]
    q = packed[:, 4:260].view(np.int8).astype(np.int32)
    sums = packed[:, 260:292].copy().view(np.int16).astype(np.int32)
    assert np.array_equal(sums, q.reshape(-1, 16, 16).sum(axis=2))
    assert q.max() <= 127 and q.min() >= -127
    zero = 6  # row 3, first block
    assert d[zero] == 0 and not q[zero].any()
    nz = np.arange(len(d)) != zero
    # first element of largest magnitude maps to -127; the scale is -max/127
    arg = np.abs(blocks).argmax(axis=1)
    smax = blocks[np.arange(len(d)), arg]
    assert np.all(q[nz, arg[nz]] == -127)
    assert np.allclose(d[nz], -smax[nz] / 127, rtol=2e-7)
    err = np.abs(d[:, None] * q - blocks)
    assert np.all(err[nz] <= np.abs(d[nz, None]) * 0.5000005)


def test_q8_k_sign_follows_first_maximum(oracle):
    x = np.zeros((2, 256), np.float32)
    x[0, 0], x[0, 1] = 5.0, -5.0
    x[1, 0], x[1, 1] = -5.0, 5.0
    p = oracle.quantize(oracle.Q8_K, x)
    q0, q1 = p[0, 4:6].view(np.int8), p[1, 4:6].view(np.int8)
    assert q0.tolist() == [-127, 127] and q1.tolist() == [-127, 127]
    assert p[0, :4].copy().view(np.float32)[0] < 0 < p[1, :4].copy().view(np.float32)[0]


# ---- K-quant block layouts (independent packer) ---------------------------

def _f16(v):
    return np.array([v], np.float16).view(np.uint8)


def _pack_scale_min_bits(sc, mn):
    """12 bytes: for j<4 the low 6 bits of byte j / j+4 hold scale/min j; for
    j>=4 byte j+4 holds their low nibbles and the top two bits of bytes j-4 / j
    hold their high bits."""
    out = np.zeros(12, np.uint8)
    for j in range(8):
        if j < 4:
            out[j] |= sc[j] & 63
            out[j + 4] |= mn[j] & 63
        else:
            out[j + 4] |= (sc[j] & 15) | ((mn[j] & 15) << 4)
            out[j - 4] |= (sc[j] >> 4) << 6
            out[j] |= (mn[j] >> 4) << 6
    return out


def _random_kblock(kind, rng):
    """Returns (packed block bytes, expected 256 values from the fields)."""
    d = np.float16(rng.uniform(0.001, 0.05))
    if kind in ("q4_K", "q5_K"):
        dmin = np.float16(rng.uniform(0.001, 0.05))
        sc = rng.integers(0, 64, 8)
        mn = rng.integers(0, 64, 8)
        nmax = 15 if kind == "q4_K" else 31
        codes = rng.integers(0, nmax + 1, 256)
        qs = np.zeros(128, np.uint8)
        qh = np.zeros(32, np.uint8)
        for e in range(256):
            j, l = e // 32, e % 32           # sub-block j covers elements 32j..32j+31
            byte = 32 * (j // 2) + l           # pairs of sub-blocks share 32 bytes
            qs[byte] |= (codes[e] & 15) << (4 * (j % 2))
            qh[l] |= ((codes[e] >> 4) & 1) << j
        blk = np.concatenate([_f16(d), _f16(dmin), _pack_scale_min_bits(sc, mn)] +
                             ([qh] if kind == "q5_K" else []) + [qs])
        expect = np.array([np.float32(np.float32(d) * sc[e // 32]) * np.float32(codes[e]) -
                           np.float32(np.float32(dmin) * mn[e // 32]) for e in range(256)], np.float32)
        return blk, expect
    # q6_K: 16 sub-blocks of 16 with signed 8-bit scales, 6-bit codes (q-32)
    sc = rng.integers(-128, 128, 16)
    codes = rng.integers(0, 64, 256)
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for e in range(256):
        half, r = e // 128, e % 128
        quarter, l = r // 32, r % 32
        ql[64 * half + 32 * (quarter % 2) + l] |= (codes[e] & 15) << (4 * (quarter // 2))
        qh[32 * half + l] |= ((codes[e] >> 4) & 3) << (2 * quarter)
    blk = np.concatenate([ql, qh, sc.astype(np.int8).view(np.uint8), _f16(d)])
    expect = np.array([np.float32(np.float32(d) * np.float32(sc[e // 16])) * np.float32(codes[e] - 32)
                       for e in range(256)], np.float32)
    return blk, expect


@pytest.mark.parametrize("kind", ["q4_K", "q5_K", "q6_K"])
def test_kquant_dequant_fields(oracle, kind):
    qtype = {"q4_K": oracle.Q4_K, "q5_K": oracle.Q5_K, "q6_K": oracle.Q6_K}[kind]
    rng = np.random.default_rng(hash(kind) % 1000)
    blocks, expects = zip(*[_random_kblock(kind, rng) for _ in range(24)])
    packed = np.concatenate(blocks).reshape(6, -1)
    assert packed.shape[1] == 4 * oracle.BLOCK_BYTES[qtype]
    got = oracle.dequantize(qtype, packed, 1024)
    assert np.array_equal(got.reshape(-1), np.concatenate(expects))


# ---- weight quantizers: round trip bounds (field-level pins: test_oracle_pins.py)

@pytest.mark.parametrize("qtype,bound", [(8, 0.012), (12, 0.12), (13, 0.06), (14, 0.03)])
def test_weight_quantizer_round_trip(oracle, qtype, bound):
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((48, 1024)) * 0.02).astype(np.float32)
    w[5] = 0.0
    w[7, :256] = 0.0
    packed = oracle.quantize(qtype, w, oracle.ROUND_REF)
    dec = oracle.dequantize(qtype, packed, 1024)
    assert np.all(dec[5] == 0) and np.all(dec[7, :256] == 0)
    rel = np.linalg.norm(dec - w, axis=1) / np.maximum(np.linalg.norm(w, axis=1), 1e-30)
    assert rel[np.linalg.norm(w, axis=1) > 0].max() < bound
    # deterministic
    assert np.array_equal(packed, oracle.quantize(qtype, w, oracle.ROUND_REF))


# ---- dots and mul_mat --------------------------------------------------------

def test_vec_dot_integer_identity(oracle):
    # d_w = d_x = 1: each Q8_0 block dot is the exact integer sum of products
    rng = np.random.default_rng(3)
    qa = rng.integers(-127, 128, (1, 256)).astype(np.int8)
    qb = rng.integers(-127, 128, (1, 256)).astype(np.int8)
    qb[0, ::32] = 127   # every activation block keeps amax 127, so repacking it is the identity
    def pack(q):
        out = np.zeros((8, 34), np.uint8)
        out[:, :2] = _f16(1.0)
        out[:, 2:] = q.reshape(8, 32).view(np.uint8)
        return out.reshape(1, -1)
    y = oracle.mul_mat_native(oracle.Q8_0, pack(qa), oracle.dequantize(oracle.Q8_0, pack(qb), 256))
    assert y[0, 0] == float(int((qa.astype(np.int64) * qb.astype(np.int64)).sum()))


@pytest.mark.parametrize("qtype", [8, 14, 13, 12])
@pytest.mark.parametrize("shape", [(256, 65, 1, "ordinary"), (256, 65, 8, "ordinary"), (256, 65, 17, "ordinary"),
                                   (1024, 33, 3, "outlier"), (256, 33, 3, "zero")])
def test_native_mul_mat_vs_decoded_bruteforce(oracle, qtype, shape):
    width, rows, columns, scenario = shape
    w = probe_weights(width, rows)
    x = probe_rhs(width, columns, scenario)
    packed = oracle.quantize(qtype, w, oracle.ROUND_REF)
    wd = oracle.dequantize(qtype, packed, width)
    xtype = oracle.Q8_0 if qtype == oracle.Q8_0 else oracle.Q8_K
    for rounding in (oracle.ROUND_X86, oracle.ROUND_REF):
        xd = oracle.dequantize(xtype, oracle.quantize(xtype, x, rounding), width)
        y = oracle.mul_mat_native(qtype, packed, x, rounding)
        ok, err = within(y, oracle.gemm_f64(wd, xd), NATIVE_TOL)
        assert ok, err
    if scenario == "outlier":   # native arithmetic really used quantized activations
        assert np.abs(y - oracle.gemm_f64(wd, x)).max() > 1e-4


def test_native_mul_mat_q8_0_short_and_4736(oracle):
    for width, rows, columns in ((32, 3, 3), (4736, 33, 3)):
        w = probe_weights(width, rows)
        x = probe_rhs(width, columns, "outlier" if width > 32 else "ordinary")
        packed = oracle.quantize(oracle.Q8_0, w)
        xd = oracle.dequantize(oracle.Q8_0, oracle.quantize(oracle.Q8_0, x, oracle.ROUND_X86), width)
        y = oracle.mul_mat_native(oracle.Q8_0, packed, x)
        ok, err = within(y, oracle.gemm_f64(oracle.dequantize(oracle.Q8_0, packed, width), xd), NATIVE_TOL)
        assert ok, err


@pytest.mark.parametrize("qtype", [8, 14, 13, 12])
@pytest.mark.parametrize("width", [256, 1024])
def test_decode_mul_mat_reference_fixture(oracle, qtype, width):
    # check_backend_quantized_math: QKV rows 3*width plus a 257-row tail, 3 columns
    x = matrix_values(width, 3, 3)
    for rows, salt in ((3 * width, 1), (257, 7)):
        w = matrix_values(width, rows, salt)
        packed = oracle.quantize(qtype, w)
        y = oracle.mul_mat_decode(qtype, packed, x)
        ok, err = within(y, oracle.gemm_f64(oracle.dequantize(qtype, packed, width), x), DECODED_TOL)
        assert ok, err


def test_decode_mul_mat_q8_0_4736_tail(oracle):
    x = matrix_values(4736, 3, 13)
    w = matrix_values(4736, 17, 17)
    packed = oracle.quantize(oracle.Q8_0, w)
    y = oracle.mul_mat_decode(oracle.Q8_0, packed, x)
    ok, err = within(y, oracle.gemm_f64(oracle.dequantize(oracle.Q8_0, packed, 4736), x), (1e-4, 1e-5))
    assert ok, err
