"""SimpleFPN neck parity on the GPU: samhip_vit_neck against the oracle's
restatement of sam3_build_neck_graph (oracle/vit_oracle.c or_neck, pinned
against float64 numpy convolutions in tests/test_vit_oracle.py), on the same
seeded inputs and weights.

Tolerances (per output pixel, relative L2 against the oracle):
  * F32 columns: 5e-6 (measured up to 1.2e-6).  Split fp16 operands carry
    ~22 significant bits per value (hi + lo, scaled per row by a power of
    two), summed in F32; four chained products at level 0.
  * F16 columns against the oracle with fp16-rounded convolution operands:
    levels 2 and 3 (whose first convolution reads the exact ViT output)
    median 2e-6, levels 0 and 1 median 3e-5; max 1e-3 everywhere.  The
    operands agree except where an intermediate that differs in its last
    F32 bits lies within that much of an fp16 rounding boundary and rounds
    to the other neighbour (one step of 2^-11 in one of K products moves the
    output by about 2^-11 / sqrt(K) relative).  At levels 2 and 3 only the
    3x3 input can flip, rarely; at levels 0 and 1 the transposed
    convolutions' F32 round-off already flips some 1x1 inputs, whose
    outputs then flip more 3x3 inputs, so most pixels carry a few flips.
    F32 columns differ from F16 ones by ~4e-4 on every pixel.
The full-size case (SAM 3 at 1008 px: grid 72, embed 1024, mid 512, dim 256)
is checked on a crop: the neck's receptive field is one input pixel plus a
one-pixel ring at each level, so the oracle on an 8 x 8 crop at an even
offset gives every level's map exactly except its outermost ring.
"""

import numpy as np
import pytest

from tests.vit_fixtures import neck_scales, neck_weights

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def row_rel(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    return np.linalg.norm(got - ref, axis=1) / np.maximum(np.linalg.norm(ref, axis=1), 1e-30)


def run_neck(ctx, samhip, weights, x, grid, E, mid, D, columns_type, levels=(0, 1, 2, 3)):
    neck = samhip.VitNeck(ctx, neck_scales(weights), grid, E, mid, D, columns_type)
    xb = ctx.upload(np.ascontiguousarray(x, np.float32))
    bufs = [ctx.alloc(neck.level_rows(i) * D * 4) if i in levels else None for i in range(4)]
    try:
        neck.forward(xb, bufs)
        return [None if b is None else ctx.download(b, (neck.level_rows(i), D), np.float32)
                for i, b in enumerate(bufs)]
    finally:
        for b in bufs:
            if b is not None:
                b.free()
        xb.free()
        neck.free()


def case(seed, grid, E, mid, D):
    rng = np.random.default_rng(seed)
    w = neck_weights(rng, E, mid, D, scale=1.0 / np.sqrt(E))
    x = rng.standard_normal((grid * grid, E)).astype(np.float32)
    return w, x


# dim 128 and 256 gather the 3x3 im2col rows inside the product; 20 and 32
# build them
@pytest.mark.parametrize("grid,E,mid,D", [(8, 128, 64, 32), (6, 100, 36, 20), (4, 256, 128, 128), (6, 128, 64, 128)])
def test_neck_f32_columns(gpu_ctx, oracle, samhip, grid, E, mid, D):
    w, x = case(grid + E, grid, E, mid, D)
    say(f"vit_neck F32 columns grid={grid} E={E} mid={mid} D={D}")
    got = run_neck(gpu_ctx, samhip, w, x, grid, E, mid, D, samhip.F32)
    ref = oracle.neck(w, x, grid, E, mid, D)
    for i in range(4):
        rel = row_rel(got[i], ref[i])
        say(f"  level {i}: max {rel.max():.3g}")
        assert rel.max() < 5e-6, i


@pytest.mark.parametrize("grid,E,mid,D", [(8, 128, 64, 32), (6, 100, 36, 20), (6, 128, 64, 128)])
def test_neck_f16_columns(gpu_ctx, oracle, samhip, grid, E, mid, D):
    w, x = case(grid + E + 1, grid, E, mid, D)
    say(f"vit_neck F16 columns grid={grid} E={E} mid={mid} D={D}")
    got = run_neck(gpu_ctx, samhip, w, x, grid, E, mid, D, samhip.F16)
    ref = oracle.neck(w, x, grid, E, mid, D, columns_f16=True)
    exact = oracle.neck(w, x, grid, E, mid, D)
    stats = []
    for i in range(4):
        rel, f32 = row_rel(got[i], ref[i]), row_rel(ref[i], exact[i])
        say(f"  level {i}: median {np.median(rel):.3g} max {rel.max():.3g} "
            f"(F32 columns differ by median {np.median(f32):.3g})")
        stats.append((np.median(rel), rel.max(), np.median(f32)))
    for i, (med, mx, f32) in enumerate(stats):
        assert med < (3e-5 if i < 2 else 2e-6) and mx < 1e-3, i
        assert f32 > 10 * med   # the fp16 rounding is what is matched


def test_neck_levels_are_independent(gpu_ctx, samhip):
    grid, E, mid, D = 6, 64, 32, 16
    w, x = case(3, grid, E, mid, D)
    full = run_neck(gpu_ctx, samhip, w, x, grid, E, mid, D, samhip.F32)
    for lv in range(4):
        only = run_neck(gpu_ctx, samhip, w, x, grid, E, mid, D, samhip.F32, levels=(lv,))
        assert np.array_equal(only[lv], full[lv]), lv
        assert all(only[i] is None for i in range(4) if i != lv)


def test_neck_full_size_crop(gpu_ctx, oracle, samhip):
    grid, E, mid, D = 72, 1024, 512, 256
    w, x = case(72, grid, E, mid, D)
    say("vit_neck 1008px F32 columns (levels 0-3)")
    got = run_neck(gpu_ctx, samhip, w, x, grid, E, mid, D, samhip.F32)
    again = run_neck(gpu_ctx, samhip, w, x, grid, E, mid, D, samhip.F32)
    for i in range(4):
        assert np.isfinite(got[i]).all()
        assert np.array_equal(got[i], again[i]), i   # deterministic
    c, oy, ox = 8, 30, 16
    crop = x.reshape(grid, grid, E)[oy:oy + c, ox:ox + c].reshape(-1, E)
    ref = oracle.neck(w, crop, c, E, mid, D)
    for i in range(4):
        side, cs = (4 * grid) >> i, (4 * c) >> i
        y0, x0 = (4 * oy) >> i, (4 * ox) >> i
        g = got[i].reshape(side, side, D)[y0 + 1:y0 + cs - 1, x0 + 1:x0 + cs - 1].reshape(-1, D)
        r = ref[i].reshape(cs, cs, D)[1:-1, 1:-1].reshape(-1, D)
        rel = row_rel(g, r)
        say(f"  level {i} crop interior {cs - 2}^2: max {rel.max():.3g}")
        assert rel.max() < 5e-6, i


def test_neck_rejects(gpu_ctx, samhip):
    grid, E, mid, D = 6, 64, 32, 16
    w, x = case(5, grid, E, mid, D)
    with pytest.raises(samhip.SamhipError, match="columns type"):
        run_neck(gpu_ctx, samhip, w, x, grid, E, mid, D, samhip.Q8_0)
    with pytest.raises(samhip.SamhipError, match="even grid"):
        run_neck(gpu_ctx, samhip, w, x[:25], 5, E, mid, D, samhip.F32)
    w2 = dict(w)
    del w2["s0_dc2_w"]
    with pytest.raises(samhip.SamhipError, match="null weight"):
        run_neck(gpu_ctx, samhip, w2, x, grid, E, mid, D, samhip.F32, levels=(0,))
    run_neck(gpu_ctx, samhip, w2, x, grid, E, mid, D, samhip.F32, levels=(1, 2, 3))   # level 0 not requested
    with pytest.raises(samhip.SamhipError, match="multiples of 4"):
        run_neck(gpu_ctx, samhip, w, x, grid, E, mid, 18, samhip.F32)
