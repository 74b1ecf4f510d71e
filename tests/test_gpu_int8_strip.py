"""The exact int8 paths for Q8_0 weights (Q8_0 activation codes) and for
Q4_K / Q5_K / Q6_K weights (Q8_K activation codes) against fewer than 256
activation rows in blocks of 32 (the text encoder's 32 tokens, the
decoder's 201 queries and 33 prompt tokens), against the oracle's native
CPU path.

Both sides form the same Q8_0 activation codes and exact integer block dots;
only the F32 order in which the per-block terms d_w d_x dot are added
differs, so the bar is the exact-code bar of the reference's dot verifier,
max per-row relative L2 <= 2e-5 (tools/validation/verify_q8_mmq_dots.py:105),
well inside the product tolerance of 1e-3."""

import sys

import numpy as np
import pytest

from tests.reference_fixtures import max_row_rel_l2, probe_rhs, probe_weights

pytestmark = pytest.mark.gpu

EXACT = 2e-5


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


# text encoder (in_proj, out_proj, fc1, fc2, resizer) at M = 32, ragged M and
# N, K slices past 1024 (partial sums and the reduce launch), short K; the
# decoder's queries (M = 201: 256x256, FFN 256->2048 and 2048->256) and
# prompt (M = 33), several row blocks with ragged ends
SHAPES = [(32, 3072, 1024), (32, 1024, 1024), (32, 4096, 1024), (32, 1024, 4096), (32, 256, 1024),
          (1, 4096, 1024), (17, 96, 512), (31, 33, 2048), (32, 64, 32), (5, 1000, 1056),
          (201, 256, 256), (201, 2048, 256), (201, 256, 2048), (33, 256, 256), (255, 96, 1056), (64, 40, 64),
          (97, 33, 1024), (3, 1, 256)]


@pytest.mark.parametrize("rounding", ["x86", "ref"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_int8_strip_matches_native(samhip, oracle, shape, rounding):
    m, n, k = shape
    say("case int8 strip", shape, rounding)
    gmode = samhip.ROUND_X86 if rounding == "x86" else samhip.ROUND_REF
    cmode = oracle.ROUND_X86 if rounding == "x86" else oracle.ROUND_REF
    rng = np.random.default_rng(m * 7 + n + k)
    w = oracle.quantize(oracle.Q8_0, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = (rng.standard_normal((m, k)) * np.exp(rng.uniform(-4, 4, (m, 1)))).astype(np.float32)
    with samhip.Context(0, samhip.COMPUTE_Q8_NATIVE, gmode) as ctx:
        y = ctx.matmul(samhip.Q8_0, w, x, x_row_stride=k + 3 if n % 2 else None)
        assert ctx.query().kernel_variant == b"skinny_i8mfma_q8_0"
        again = ctx.matmul(samhip.Q8_0, w, x)
    ref = oracle.mul_mat_native(oracle.Q8_0, w, x, cmode)
    err = max_row_rel_l2(y, ref)
    say(f"  max row rel L2 {err:.2e}")
    assert np.isfinite(y).all() and err <= EXACT
    assert np.array_equal(y, again)                 # deterministic, strided or not


def test_int8_strip_two_column_tiles_same_bits(samhip, oracle, monkeypatch):
    """SAMHIP_I8_STRIP_ROWS=64 runs 64 weight rows per workgroup (two 32-row
    column tiles, all 16 waves busy) wherever the K slice holds at most 256
    values, =32 keeps 32 rows, and the default takes 64 only where that
    brings the grid into one round (M = 201, N = 2048, K = 256).  All give
    the same bits: K = 256 products with one and several row blocks, ragged
    N (one row, 33 rows: the second tile partly or wholly past N), K = 64,
    and 256-wide slices of K = 1024 with the reduce launch."""
    say("case int8 strip two column tiles")
    rng = np.random.default_rng(78)
    shapes = [(201, 256, 256), (201, 2048, 256), (33, 256, 256), (3, 1, 256), (17, 33, 256), (64, 40, 64),
              (32, 1024, 1024), (97, 33, 1024)]
    cases = []
    for m, n, k in shapes:
        w = oracle.quantize(oracle.Q8_0, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
        x = (rng.standard_normal((m, k)) * np.exp(rng.uniform(-4, 4, (m, 1)))).astype(np.float32)
        cases.append((w, x))
    outs = {}
    for rows in ("64", "32", None):
        if rows:
            monkeypatch.setenv("SAMHIP_I8_STRIP_ROWS", rows)
        else:
            monkeypatch.delenv("SAMHIP_I8_STRIP_ROWS", raising=False)
        with samhip.Context(0, samhip.COMPUTE_Q8_NATIVE) as ctx:
            outs[rows] = [ctx.matmul(samhip.Q8_0, w, x) for w, x in cases]
            assert ctx.query().kernel_variant == b"skinny_i8mfma_q8_0"
    for i, ((w, x), shp) in enumerate(zip(cases, shapes)):
        assert np.array_equal(outs["64"][i], outs["32"][i]), shp
        assert np.array_equal(outs[None][i], outs["32"][i]), shp
        assert max_row_rel_l2(outs["64"][i], oracle.mul_mat_native(oracle.Q8_0, w, x)) <= EXACT, shp


def test_int8_strip_views_and_reference_probe(gpu_ctx, oracle, samhip):
    """Row-offset views of a fused in-projection and the reference's probe
    fixture (tools/benchmark/cpu_quantized_matmul.hpp:63-75) with its outlier
    and zero activation columns."""
    say("case int8 strip views")
    d = 1024
    w = oracle.quantize(oracle.Q8_0, probe_weights(d, 3 * d))
    for scenario in ("ordinary", "outlier", "zero"):
        x = probe_rhs(d, 32, scenario)
        for part in range(3):
            y = gpu_ctx.matmul(samhip.Q8_0, w, x, w_row_offset=part * d, w_rows=d)
            ref = oracle.mul_mat_native(oracle.Q8_0, w[part * d:(part + 1) * d], x)
            if scenario == "zero":
                assert not y.any() and not ref.any()
            else:
                assert max_row_rel_l2(y, ref) <= EXACT


def test_int8_strip_repeats_and_replays(samhip, oracle):
    """Products with one and with several K slices (partial sums in the
    context's staging, added by the reduce launch) in alternating order,
    repeated eager calls and three replays of a captured stream, with eager
    work between them, all give the first call's bits."""
    say("case int8 tickets")
    rng = np.random.default_rng(77)
    shapes = [(32, 1024, 4096), (32, 3072, 1024), (7, 100, 1056), (32, 256, 512)]
    with samhip.Context(0, samhip.COMPUTE_Q8_NATIVE) as ctx:
        ops, bufs = [], []
        for m, n, k in shapes:
            w = oracle.quantize(oracle.Q8_0, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
            x = rng.standard_normal((m, k)).astype(np.float32)
            wb, xb, yb = ctx.upload(w), ctx.upload(x), ctx.alloc(m * n * 4)
            bufs += [wb, xb, yb]
            ops.append((samhip.tensor(samhip.Q8_0, k, n, wb.ptr), samhip.tensor(samhip.F32, k, m, xb.ptr),
                        samhip.tensor(samhip.F32, n, m, yb.ptr), yb, (m, n), w, x))
        for wt, xt, yt, *_ in ops:
            ctx.mul_mat(wt, xt, yt)
        assert ctx.query().kernel_variant == b"skinny_i8mfma_q8_0"
        first = [ctx.download(yb, shp, np.float32) for _, _, _, yb, shp, _, _ in ops]
        for (_, _, _, _, _, w, x), y in zip(ops, first):
            assert max_row_rel_l2(y, oracle.mul_mat_native(oracle.Q8_0, w, x)) <= EXACT
        for _ in range(3):
            for wt, xt, yt, *_ in reversed(ops):
                ctx.mul_mat(wt, xt, yt)
        for (_, _, _, yb, shp, _, _), y in zip(ops, first):
            assert np.array_equal(ctx.download(yb, shp, np.float32), y)
        ctx.capture_begin()
        for wt, xt, yt, *_ in ops:
            ctx.mul_mat(wt, xt, yt)
        g = ctx.capture_end()
        try:
            for rep in range(3):
                for _, _, _, yb, shp, _, _ in ops:
                    ctx.write(yb, np.zeros(shp, np.float32))
                wt, xt, yt = ops[1][:3]
                ctx.mul_mat(wt, xt, yt)                 # eager work between replays
                ctx.synchronize()
                g.launch()
                ctx.synchronize()
                for (_, _, _, yb, shp, _, _), y in zip(ops, first):
                    assert np.array_equal(ctx.download(yb, shp, np.float32), y), rep
        finally:
            g.destroy()


def test_small_weight_and_kquant_kernels_in_graph_replays(samhip, oracle):
    """The small-weight kernels (Q8_0 and Q4_K), the K-quant strip kernel
    (one and several K slices) and the 64-row Q8_0 strip workgroups,
    captured as one stream and replayed three times with eager work between
    the replays: every replay gives the eager call's bits."""
    say("case graph replays of the int8 kernels")
    rng = np.random.default_rng(81)
    cases = [(samhip.Q8_0, oracle.Q8_0, 5184, 256, 256), (samhip.Q4_K, oracle.Q4_K, 1000, 200, 256),
             (samhip.Q4_K, oracle.Q4_K, 32, 1024, 1024), (samhip.Q6_K, oracle.Q6_K, 33, 256, 256),
             (samhip.Q8_0, oracle.Q8_0, 201, 2048, 256)]
    with samhip.Context(0, samhip.COMPUTE_Q8_NATIVE) as ctx:
        ops = []
        for gt, ot, m, n, k in cases:
            w = oracle.quantize(ot, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
            x = rng.standard_normal((m, k)).astype(np.float32)
            wb, xb, yb = ctx.upload(w), ctx.upload(x), ctx.alloc(m * n * 4)
            ops.append((samhip.tensor(gt, k, n, wb.ptr), samhip.tensor(samhip.F32, k, m, xb.ptr),
                        samhip.tensor(samhip.F32, n, m, yb.ptr), (wb, xb, yb), (m, n), w, x, ot))
        first = []
        for wt, xt, yt, bufs, shp, w, x, ot in ops:
            ctx.mul_mat(wt, xt, yt)
            y = ctx.download(bufs[2], shp, np.float32)
            assert max_row_rel_l2(y, oracle.mul_mat_native(ot, w, x)) <= EXACT
            first.append(y)
        ctx.capture_begin()
        for wt, xt, yt, *_ in ops:
            ctx.mul_mat(wt, xt, yt)
        g = ctx.capture_end()
        try:
            for rep in range(3):
                for _, _, _, bufs, shp, *_ in ops:
                    ctx.write(bufs[2], np.zeros(shp, np.float32))
                wt, xt, yt = ops[2][:3]
                ctx.mul_mat(wt, xt, yt)                 # eager work between replays
                ctx.synchronize()
                g.launch()
                ctx.synchronize()
                for (_, _, _, bufs, shp, *_), y in zip(ops, first):
                    assert np.array_equal(ctx.download(bufs[2], shp, np.float32), y), (rep, shp)
        finally:
            g.destroy()
        for *_, bufs, _, _, _, _ in ops:
            for b in bufs:
                b.free()


@pytest.mark.parametrize("rounding", ["x86", "ref"])
def test_int8_strip_nan_activations(samhip, oracle, rounding):
    """A NaN activation packs as code 0 (the library's contract, as ggml's
    nearest_int gives; not ggml's AVX2 Q8_0 packing, which would give -128)
    and leaves its block's scale to the finite values: single NaNs, a NaN
    run across blocks and a whole NaN row, against the oracle."""
    say("case int8 strip NaN", rounding)
    gmode = samhip.ROUND_X86 if rounding == "x86" else samhip.ROUND_REF
    cmode = oracle.ROUND_X86 if rounding == "x86" else oracle.ROUND_REF
    rng = np.random.default_rng(91)
    m, n, k = 32, 256, 1024
    w = oracle.quantize(oracle.Q8_0, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[3, 5] = np.nan
    x[7, 100:140] = np.nan
    x[20, :] = np.nan
    x[29, 31] = np.nan
    with samhip.Context(0, samhip.COMPUTE_Q8_NATIVE, gmode) as ctx:
        y = ctx.matmul(samhip.Q8_0, w, x)
        assert ctx.query().kernel_variant == b"skinny_i8mfma_q8_0"
    ref = oracle.mul_mat_native(oracle.Q8_0, w, x, cmode)
    assert np.isfinite(ref).all() and np.isfinite(y).all()
    assert not y[20].any() and not ref[20].any()
    assert max_row_rel_l2(y, ref) <= EXACT


KQ_SHAPES = [(32, 1024, 1024), (32, 1024, 4096), (32, 4096, 1024), (201, 256, 2048), (201, 2048, 256),
             (33, 256, 256), (17, 96, 512), (255, 40, 1280), (1, 64, 256), (97, 33, 768), (3, 1, 512)]


@pytest.mark.parametrize("form", ["f32", "isum"])
@pytest.mark.parametrize("qtype", ["q4_K", "q5_K", "q6_K"])
@pytest.mark.parametrize("shape", KQ_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_kquant_int8_strip_matches_native(samhip, oracle, monkeypatch, shape, qtype, form):
    """K-quant weights on the int8 path (SAMHIP_INT8_STRIP=2 takes it for
    every shape; by default only where it is faster): the 4/5/6-bit codes and
    Q8_K activation codes meet in exact integer dots; the sub-block scales
    and minimums are applied in F32 per sub-block (form f32, the default) or
    in integers per super-block (form isum, SAMHIP_KQ_ISUM=1), so only the
    order of the F32 additions differs from the oracle's vec_dot (same bar
    as Q8_0; K slices past the first, K = 768 in three, among them)."""
    m, n, k = shape
    say("case int8 strip", qtype, shape)
    gt = {"q4_K": samhip.Q4_K, "q5_K": samhip.Q5_K, "q6_K": samhip.Q6_K}[qtype]
    ot = {"q4_K": oracle.Q4_K, "q5_K": oracle.Q5_K, "q6_K": oracle.Q6_K}[qtype]
    rng = np.random.default_rng(m * 13 + n + k + gt)
    w = oracle.quantize(ot, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = (rng.standard_normal((m, k)) * np.exp(rng.uniform(-4, 4, (m, 1)))).astype(np.float32)
    if m > 3:
        x[2, 7] = np.nan                      # packs as code 0
        x[3, :] = 0.0                         # an all-zero row: d = 0
    monkeypatch.setenv("SAMHIP_KQ_ISUM", "1" if form == "isum" else "0")
    monkeypatch.setenv("SAMHIP_INT8_STRIP", "2")
    with samhip.Context(0, samhip.COMPUTE_Q8_NATIVE) as ctx:
        y = ctx.matmul(gt, w, x, x_row_stride=k + 4 if n % 2 else None)
        assert ctx.query().kernel_variant == ("skinny_i8mfma_" + qtype.lower()).encode()
        again = ctx.matmul(gt, w, x)
    ref = oracle.mul_mat_native(ot, w, x)
    assert np.isfinite(ref).all() and np.isfinite(y).all()
    if m > 3:
        assert not y[3].any() and not ref[3].any()
    err = max_row_rel_l2(y, ref)
    say(f"  max row rel L2 {err:.2e}")
    assert err <= EXACT
    assert np.array_equal(y, again)


def test_kquant_int8_default_routing(samhip, oracle):
    """By default the K-quant int8 path takes the products whose grid of
    row groups x 32-row blocks x K slices fits one round of the chip's CUs,
    with 1024-wide slices for Q4_K / Q5_K (the text encoder's M = 32
    products, the decoder's 256x256 products at M = 201 and 33) and 256-wide
    ones for Q6_K, and with K = 256 those that fit one round with 64 weight
    rows per workgroup (the decoder's M = 201 FFN expansion to 2048); the
    rest (M = 201, N = 4096, K = 256; Q6_K M = 32, N = 4096, K = 1024) stays
    on the fused kernel."""
    rng = np.random.default_rng(5)
    with samhip.Context(0, samhip.COMPUTE_Q8_NATIVE) as ctx:
        for qt, m, n, k, exact in ((oracle.Q4_K, 201, 256, 256, True), (oracle.Q4_K, 33, 256, 256, True),
                                   (oracle.Q4_K, 32, 1024, 1024, True), (oracle.Q5_K, 32, 1024, 4096, True),
                                   (oracle.Q4_K, 201, 2048, 256, True), (oracle.Q4_K, 201, 4096, 256, False),
                                   (oracle.Q6_K, 32, 1024, 1024, True), (oracle.Q6_K, 32, 4096, 1024, False)):
            w = oracle.quantize(qt, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
            x = rng.standard_normal((m, k)).astype(np.float32)
            y = ctx.matmul(qt, w, x)
            name = ctx.query().kernel_variant.decode()
            tname = {oracle.Q4_K: "q4_k", oracle.Q5_K: "q5_k", oracle.Q6_K: "q6_k"}[qt]
            assert name == ("skinny_i8mfma_" if exact else "skinny_fused_") + tname, (name, m, n, k)
            assert max_row_rel_l2(y, oracle.mul_mat_native(qt, w, x)) <= (EXACT if exact else 1e-3)


@pytest.mark.parametrize("qtype", ["q4_K", "q5_K", "q6_K"])
def test_kquant_int8_strip_one_slice_bit_equal(samhip, oracle, monkeypatch, qtype):
    """In its integer form (SAMHIP_KQ_ISUM=1) the K-quant int8 kernel sums
    each super-block's sc_j dot_j and c_j xs_j in integers and then takes
    ggml's F32 steps per super-block in K order, the oracle's arithmetic:
    with the whole K in one slice the bits agree (K = 256 with one and
    several row blocks, ragged N, 64 weight rows per workgroup at N = 2048;
    K = 1024 in one 1024-wide slice at N = 8192; a NaN activation and an
    all-zero row)."""
    say("case kquant int8 strip bit-equal", qtype)
    qt = {"q4_K": oracle.Q4_K, "q5_K": oracle.Q5_K, "q6_K": oracle.Q6_K}[qtype]
    gt = {"q4_K": samhip.Q4_K, "q5_K": samhip.Q5_K, "q6_K": samhip.Q6_K}[qtype]
    rng = np.random.default_rng(80)
    monkeypatch.setenv("SAMHIP_INT8_STRIP", "2")
    monkeypatch.setenv("SAMHIP_KQ_ISUM", "1")
    with samhip.Context(0, samhip.COMPUTE_Q8_NATIVE) as ctx:
        for m, n, k in ((201, 256, 256), (33, 256, 256), (3, 1, 256), (17, 33, 256), (201, 2048, 256),
                        (32, 8192, 1024)):
            w = oracle.quantize(qt, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
            x = (rng.standard_normal((m, k)) * np.exp(rng.uniform(-4, 4, (m, 1)))).astype(np.float32)
            if m > 3:
                x[2, 7] = np.nan
                x[3, :] = 0.0
            y = ctx.matmul(gt, w, x, x_row_stride=k + 4 if n % 2 else None)
            assert ctx.query().kernel_variant == ("skinny_i8mfma_" + qtype.lower()).encode()
            ref = oracle.mul_mat_native(qt, w, x)
            assert np.array_equal(y, ref), (m, n, k, max_row_rel_l2(y, ref))


@pytest.mark.parametrize("qtype", ["q4_K", "q5_K", "q6_K"])
def test_kquant_int8_strip_two_column_tiles_same_bits(samhip, oracle, monkeypatch, qtype):
    """The K-quant int8 kernel with 64 weight rows per workgroup
    (SAMHIP_I8_STRIP_ROWS=64, slices of one super-block) gives the bits of
    32 rows (=32): one and several row blocks, ragged N, and 256-wide slices
    of K = 1024 with the reduce launch (SAMHIP_INT8_STRIP=2 keeps every
    product on the int8 kernel)."""
    say("case kquant int8 strip two column tiles", qtype)
    qt = {"q4_K": oracle.Q4_K, "q5_K": oracle.Q5_K, "q6_K": oracle.Q6_K}[qtype]
    gt = {"q4_K": samhip.Q4_K, "q5_K": samhip.Q5_K, "q6_K": samhip.Q6_K}[qtype]
    rng = np.random.default_rng(79)
    shapes = [(201, 256, 256), (201, 2048, 256), (33, 256, 256), (3, 1, 256), (17, 33, 256), (32, 1024, 1024),
              (97, 33, 1024)]
    cases = []
    for m, n, k in shapes:
        w = oracle.quantize(qt, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
        x = (rng.standard_normal((m, k)) * np.exp(rng.uniform(-4, 4, (m, 1)))).astype(np.float32)
        cases.append((w, x))
    monkeypatch.setenv("SAMHIP_INT8_STRIP", "2")
    outs = {}
    for rows in ("64", "32"):
        monkeypatch.setenv("SAMHIP_I8_STRIP_ROWS", rows)
        with samhip.Context(0, samhip.COMPUTE_Q8_NATIVE) as ctx:
            outs[rows] = [ctx.matmul(gt, w, x) for w, x in cases]
            assert ctx.query().kernel_variant == ("skinny_i8mfma_" + qtype.lower()).encode()
    for i, ((w, x), shp) in enumerate(zip(cases, shapes)):
        assert np.array_equal(outs["64"][i], outs["32"][i]), shp
        assert max_row_rel_l2(outs["64"][i], oracle.mul_mat_native(qt, w, x)) <= EXACT, shp


# many activation rows against a Q8_0 weight that fits in LDS (K = 256,
# N <= 256): the fusion encoder's and decoder's image tokens (M = 5184) on
# 256x256 weights, a batch of 8 images (several 32-row steps per
# workgroup), ragged M and N, an unaligned activation stride
TALL_SMALL = [(5184, 256, 256), (41472, 256, 256), (300, 100, 256), (1000, 255, 256), (257, 33, 256),
              (4097, 17, 256), (5184, 64, 256), (256, 200, 256)]


@pytest.mark.parametrize("rounding", ["x86", "ref"])
@pytest.mark.parametrize("shape", TALL_SMALL, ids=lambda s: "x".join(map(str, s)))
def test_tall_small_weight_int8_matches_native(samhip, oracle, shape, rounding):
    m, n, k = shape
    say("case tall small-weight int8", shape, rounding)
    gmode = samhip.ROUND_X86 if rounding == "x86" else samhip.ROUND_REF
    cmode = oracle.ROUND_X86 if rounding == "x86" else oracle.ROUND_REF
    rng = np.random.default_rng(m + 3 * n + k)
    w = oracle.quantize(oracle.Q8_0, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = (rng.standard_normal((m, k)) * np.exp(rng.uniform(-4, 4, (m, 1)))).astype(np.float32)
    with samhip.Context(0, samhip.COMPUTE_Q8_NATIVE, gmode) as ctx:
        y = ctx.matmul(samhip.Q8_0, w, x, x_row_stride=k + 1 if m % 2 else None)
        assert ctx.query().kernel_variant == b"tall_small_i8mfma_q8_0"
        again = ctx.matmul(samhip.Q8_0, w, x)
    ref = oracle.mul_mat_native(oracle.Q8_0, w, x, cmode)
    err = max_row_rel_l2(y, ref)
    say(f"  max row rel L2 {err:.2e}")
    assert np.isfinite(y).all() and err <= EXACT
    assert np.array_equal(y, again)


def test_tall_small_weight_other_widths_take_the_fused_kernel(samhip, oracle):
    """K other than 256 keeps the fused kernel (the small-weight kernel holds
    256-value rows only)."""
    rng = np.random.default_rng(92)
    with samhip.Context(0, samhip.COMPUTE_Q8_NATIVE, samhip.ROUND_X86) as ctx:
        for n, k in ((100, 224), (256, 128)):
            w = oracle.quantize(oracle.Q8_0, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
            x = rng.standard_normal((1000, k)).astype(np.float32)
            y = ctx.matmul(samhip.Q8_0, w, x)
            assert ctx.query().kernel_variant.startswith(b"skinny_fused")
            assert max_row_rel_l2(y, oracle.mul_mat_native(oracle.Q8_0, w, x, oracle.ROUND_X86)) <= 1e-3


def test_tall_small_weight_views_of_in_projection(samhip, oracle):
    """q / k / v as row-offset views of a fused [3 x 256, 256] in-projection
    (fusion_encoder.hpp:63-137), each against the oracle on its rows."""
    say("case tall small-weight views")
    rng = np.random.default_rng(91)
    w = oracle.quantize(oracle.Q8_0, (rng.standard_normal((768, 256)) * 0.02).astype(np.float32))
    x = rng.standard_normal((5184, 256)).astype(np.float32)
    with samhip.Context(0, samhip.COMPUTE_Q8_NATIVE, samhip.ROUND_X86) as ctx:
        for s in range(3):
            y = ctx.matmul(samhip.Q8_0, w, x, w_row_offset=256 * s, w_rows=256)
            assert ctx.query().kernel_variant == b"tall_small_i8mfma_q8_0"
            ref = oracle.mul_mat_native(oracle.Q8_0, w[256 * s:256 * (s + 1)], x, oracle.ROUND_X86)
            assert max_row_rel_l2(y, ref) <= EXACT


# the same shapes on K-quant weights: one 256-value super-block per row, the
# activations packed to Q8_K, ggml's integer dot of codes and scales
@pytest.mark.parametrize("qtype", ["Q4_K", "Q5_K", "Q6_K"])
@pytest.mark.parametrize("shape", TALL_SMALL, ids=lambda s: "x".join(map(str, s)))
def test_tall_small_kquant_int8_matches_native(samhip, oracle, shape, qtype):
    m, n, k = shape
    say("case tall small-weight kquant int8", shape, qtype)
    gt, ot = getattr(samhip, qtype), getattr(oracle, qtype)
    rng = np.random.default_rng(m + 5 * n + k + len(qtype) + ord(qtype[1]))
    w = oracle.quantize(ot, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = (rng.standard_normal((m, k)) * np.exp(rng.uniform(-4, 4, (m, 1)))).astype(np.float32)
    x[2, 7] = np.nan                          # packs as code 0
    x[3, :] = 0.0                             # an all-zero row: d = 0
    with samhip.Context(0, samhip.COMPUTE_Q8_NATIVE) as ctx:
        y = ctx.matmul(gt, w, x, x_row_stride=k + 1 if m % 2 else None)
        assert ctx.query().kernel_variant == ("tall_small_i8mfma_" + qtype.lower()).encode()
        again = ctx.matmul(gt, w, x)
    ref = oracle.mul_mat_native(ot, w, x)
    assert np.isfinite(ref).all() and np.isfinite(y).all()
    assert not y[3].any() and not ref[3].any()
    err = max_row_rel_l2(y, ref)
    say(f"  max row rel L2 {err:.2e}")
    # one super-block per row: the integer sums and the F32 steps in the
    # oracle's order, so the bits agree
    assert np.array_equal(y, ref), err
    assert np.array_equal(y, again)


def test_tall_small_kquant_views_and_switch(samhip, oracle, monkeypatch):
    """Row-offset views of a [768, 256] Q4_K weight take the small-weight
    kernel; SAMHIP_TALL_SMALL=0 puts the same products back on the fused
    kernel."""
    say("case tall small-weight kquant views")
    rng = np.random.default_rng(93)
    w = oracle.quantize(oracle.Q4_K, (rng.standard_normal((768, 256)) * 0.02).astype(np.float32))
    x = rng.standard_normal((5184, 256)).astype(np.float32)
    with samhip.Context(0, samhip.COMPUTE_Q8_NATIVE) as ctx:
        for s in range(3):
            y = ctx.matmul(samhip.Q4_K, w, x, w_row_offset=256 * s, w_rows=256)
            assert ctx.query().kernel_variant == b"tall_small_i8mfma_q4_k"
            ref = oracle.mul_mat_native(oracle.Q4_K, w[256 * s:256 * (s + 1)], x)
            assert max_row_rel_l2(y, ref) <= EXACT
    monkeypatch.setenv("SAMHIP_TALL_SMALL", "0")
    with samhip.Context(0, samhip.COMPUTE_Q8_NATIVE) as ctx:
        y = ctx.matmul(samhip.Q4_K, w, x, w_rows=256)
        assert ctx.query().kernel_variant == b"skinny_fused_q4_k"
        assert max_row_rel_l2(y, oracle.mul_mat_native(oracle.Q4_K, w[:256], x)) <= 1e-3


# the exact int8 GEMM for tall Q8_0 products (SAMHIP_TALL_INT8=1): ViT fc2
# (K = 4736) and fc1 (config 1) on every row, ragged M and N, a strided
# activation, a row-offset view, both roundings
TALL_I8 = [(5184, 1024, 4736), (5184, 4736, 1024), (300, 257, 1024), (1000, 96, 4736), (257, 1000, 128),
           (700, 3072, 64)]


@pytest.mark.parametrize("rounding", ["x86", "ref"])
@pytest.mark.parametrize("shape", TALL_I8, ids=lambda s: "x".join(map(str, s)))
def test_tall_int8_gemm_matches_native(samhip, oracle, monkeypatch, shape, rounding):
    m, n, k = shape
    say("case tall int8 gemm", shape, rounding)
    gmode = samhip.ROUND_X86 if rounding == "x86" else samhip.ROUND_REF
    cmode = oracle.ROUND_X86 if rounding == "x86" else oracle.ROUND_REF
    rng = np.random.default_rng(m + n + 7 * k)
    w = oracle.quantize(oracle.Q8_0, (rng.standard_normal((n + 5, k)) * 0.02).astype(np.float32))
    x = (rng.standard_normal((m, k)) * np.exp(rng.uniform(-4, 4, (m, 1)))).astype(np.float32)
    monkeypatch.setenv("SAMHIP_TALL_INT8", "1")
    with samhip.Context(0, samhip.COMPUTE_Q8_NATIVE, gmode) as ctx:
        y = ctx.matmul(samhip.Q8_0, w, x, w_row_offset=5, w_rows=n, x_row_stride=k + 4 if m % 2 else None)
        assert ctx.query().kernel_variant == b"gemm_i8mfma_q8_0_128x128x64"
        again = ctx.matmul(samhip.Q8_0, w, x, w_row_offset=5, w_rows=n)
    ref = oracle.mul_mat_native(oracle.Q8_0, w[5:5 + n], x, cmode)
    err = max_row_rel_l2(y, ref)
    say(f"  max row rel L2 {err:.2e} over {m} rows")
    assert np.isfinite(y).all() and err <= EXACT
    assert np.array_equal(y, again)


def test_tall_int8_gemm_nan_and_zero_rows(samhip, oracle, monkeypatch):
    """A NaN activation packs as code 0 and zero rows give zero outputs, as
    the oracle's native path does."""
    say("case tall int8 gemm NaN")
    rng = np.random.default_rng(95)
    w = oracle.quantize(oracle.Q8_0, (rng.standard_normal((256, 1024)) * 0.02).astype(np.float32))
    x = rng.standard_normal((300, 1024)).astype(np.float32)
    x[3, 7] = x[40, 300] = x[299, 1023] = np.nan
    x[10] = 0.0
    monkeypatch.setenv("SAMHIP_TALL_INT8", "1")
    with samhip.Context(0, samhip.COMPUTE_Q8_NATIVE, samhip.ROUND_X86) as ctx:
        y = ctx.matmul(samhip.Q8_0, w, x)
        assert ctx.query().kernel_variant == b"gemm_i8mfma_q8_0_128x128x64"
    assert np.isfinite(y).all() and not y[10].any()
    assert max_row_rel_l2(y, oracle.mul_mat_native(oracle.Q8_0, w, x, oracle.ROUND_X86)) <= EXACT
