"""Pins of the vision-encoder oracle (oracle/vit_oracle.c) against
independent float64 restatements (numpy / scipy) and structural invariants,
each following the reference graph it restates
(src/models/sam3/vision.hpp:109-293, src/models/sam3/ops.hpp:56-89)."""

import numpy as np
import pytest
from scipy.special import erf

from tests.vit_fixtures import axial_rope_table, block_weights, neck_scales, neck_weights


def np_layer_norm(x, w=None, b=None, eps=1e-5):
    x = x.astype(np.float64)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    y = (x - mu) / np.sqrt(var + eps)
    if w is not None:
        y = y * w
    if b is not None:
        y = y + b
    return y


def test_layer_norm(oracle):
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((37, 1024)) * 3 + 1.5).astype(np.float32)
    w = rng.standard_normal(1024).astype(np.float32)
    b = rng.standard_normal(1024).astype(np.float32)
    y = oracle.layer_norm(x, w, b)
    assert np.abs(y - np_layer_norm(x, w, b)).max() < 2e-5
    u = oracle.layer_norm(x)                                     # unit gain: mean 0, variance 1 (minus eps)
    assert np.abs(u.mean(1)).max() < 1e-6
    assert np.abs(u.var(1) - 1).max() < 1e-4
    c = np.full((2, 64), 3.25, np.float32)                       # constant rows: (x - mean) = 0 exactly
    assert np.all(oracle.layer_norm(c) == 0)


def test_gelu_erf(oracle):
    x = np.concatenate([np.linspace(-8, 8, 4001), [0.0, -0.0, 1e-30, -40, 40]]).astype(np.float32)
    y = oracle.gelu_erf(x)
    ref = 0.5 * x.astype(np.float64) * (1 + erf(x.astype(np.float64) / np.sqrt(2)))
    assert np.abs(y - ref).max() < 2e-6 * max(1.0, np.abs(ref).max() / 8)
    assert y[-2] == 0 and y[-1] == 40


@pytest.mark.parametrize("W,H,ws", [(72, 72, 24), (10, 7, 4), (8, 8, 8)])
def test_win_part_order_and_round_trip(oracle, W, H, ws):
    """ggml_win_part: window py*npx + px, token i2*ws + i1 inside it, zeros
    past the grid; ggml_win_unpart inverts it."""
    gx, gy = np.meshgrid(np.arange(W), np.arange(H))
    x = np.stack([gx.ravel() + 1, gy.ravel() + 1, gx.ravel() * 1000 + gy.ravel()], 1).astype(np.float32)
    p = oracle.win_part(x, W, H, ws)
    npx, npy = -(-W // ws), -(-H // ws)
    assert p.shape == (npx * npy * ws * ws, 3)
    for py in range(npy):
        for px in range(npx):
            for i2 in range(ws):
                for i1 in range(ws):
                    row = p[(py * npx + px) * ws * ws + i2 * ws + i1]
                    X, Y = px * ws + i1, py * ws + i2
                    if X < W and Y < H:
                        assert row[0] == X + 1 and row[1] == Y + 1
                    else:
                        assert not row.any()
    assert np.array_equal(oracle.win_unpart(p, W, H, ws), x)


def test_rope_complex_product(oracle):
    rng = np.random.default_rng(1)
    heads, hd, n = 3, 64, 50
    x = rng.standard_normal((n, heads * hd + 5)).astype(np.float32)
    f = axial_rope_table(10, 5, hd)
    y = oracle.rope(x, heads, hd, f)
    fc = f[..., 0].astype(np.float64) + 1j * f[..., 1]
    for h in range(heads):
        z = x[:, h * hd:(h + 1) * hd:2].astype(np.float64) + 1j * x[:, h * hd + 1:(h + 1) * hd:2]
        out = z * fc
        assert np.abs(y[:, h * hd:(h + 1) * hd:2] - out.real).max() < 1e-5
        assert np.abs(y[:, h * hd + 1:(h + 1) * hd:2] - out.imag).max() < 1e-5
        yn = np.hypot(y[:, h * hd:(h + 1) * hd:2], y[:, h * hd + 1:(h + 1) * hd:2])
        assert np.allclose(yn, np.abs(z), rtol=1e-6, atol=1e-7)   # unit-modulus table keeps pair norms
    assert np.array_equal(y[:, heads * hd:], x[:, heads * hd:])    # columns past the heads untouched


def test_attention_against_float64_softmax(oracle):
    rng = np.random.default_rng(2)
    heads, hd, n = 2, 64, 97
    ld = 3 * heads * hd
    qkv = rng.standard_normal((n, ld)).astype(np.float32) * 2
    q, k, v = qkv[:, :heads * hd], qkv[:, heads * hd:2 * heads * hd], qkv[:, 2 * heads * hd:]
    out = oracle.attention(q, k, v, heads, hd, 0.125)
    for h in range(heads):
        s = q[:, h * hd:(h + 1) * hd].astype(np.float64) @ k[:, h * hd:(h + 1) * hd].T.astype(np.float64) * 0.125
        p = np.exp(s - s.max(1, keepdims=True))
        ref = (p / p.sum(1, keepdims=True)) @ v[:, h * hd:(h + 1) * hd].astype(np.float64)
        assert np.abs(out[:, h * hd:(h + 1) * hd] - ref).max() < 1e-5


def test_prefix_against_float64_convolution(oracle):
    rng = np.random.default_rng(3)
    img, patch, E, pg = 56, 14, 64, 2
    grid = img // patch
    image = rng.standard_normal((3, img, img)).astype(np.float32)
    kernel = (rng.standard_normal((E, 3, patch, patch)) * 0.02).astype(np.float32)
    pos = (rng.standard_normal((pg, pg, E)) * 0.1).astype(np.float32)
    lw, lb = rng.standard_normal(E).astype(np.float32), rng.standard_normal(E).astype(np.float32)
    out = oracle.vit_prefix(image, patch, kernel, pos, pg, lw, lb, E)
    patches = image.astype(np.float64).reshape(3, grid, patch, grid, patch)          # c, oy, ky, ox, kx
    conv = np.einsum("cykxl,eckl->yxe", patches, kernel.astype(np.float64))          # [oy][ox][E]
    tiled = np.tile(pos.astype(np.float64), (grid // pg, grid // pg, 1))
    ref = np_layer_norm((conv + tiled).reshape(grid * grid, E), lw, lb)
    assert np.abs(out - ref).max() < 1e-4


def np_block(oracle, w, x, W, H, E, heads, mlp, ws):
    """The reference block graph (src/models/sam3/vision.hpp:152-243) from
    numpy pieces and the oracle's native mul_mat."""
    hd = E // heads
    xs = x
    h = np_layer_norm(x, w["norm1_w"], w["norm1_b"]).astype(np.float32)
    if ws:
        h = oracle.win_part(h, W, H, ws)
        per = ws * ws
    else:
        per = W * H
    qkv = oracle.mul_mat_native(w["qkv_type"], w["qkv_w"], h) + w["qkv_b"]
    att = np.empty((qkv.shape[0], E), np.float32)
    fc = w["freqs"][..., 0].astype(np.float64) + 1j * w["freqs"][..., 1]
    for b in range(qkv.shape[0] // per):
        blk = qkv[b * per:(b + 1) * per].astype(np.float64)
        for hh in range(heads):
            def roped(col0):
                z = blk[:, col0 + hh * hd:col0 + (hh + 1) * hd:2] + 1j * blk[:, col0 + hh * hd + 1:col0 + (hh + 1) * hd:2]
                r = z * fc
                out = np.empty((per, hd))
                out[:, 0::2], out[:, 1::2] = r.real, r.imag
                return out
            q, k = roped(0), roped(E)
            v = blk[:, 2 * E + hh * hd:2 * E + (hh + 1) * hd]
            s = q @ k.T / np.sqrt(hd)
            p = np.exp(s - s.max(1, keepdims=True))
            att[b * per:(b + 1) * per, hh * hd:(hh + 1) * hd] = (p / p.sum(1, keepdims=True)) @ v
    pr = oracle.mul_mat_native(w["proj_type"], w["proj_w"], att) + w["proj_b"]
    if ws:
        pr = oracle.win_unpart(pr, W, H, ws)
    x1 = xs + pr
    h2 = np_layer_norm(x1, w["norm2_w"], w["norm2_b"]).astype(np.float32)
    f1 = oracle.mul_mat_native(w["fc1_type"], w["fc1_w"], h2) + w["fc1_b"]
    g = (0.5 * f1.astype(np.float64) * (1 + erf(f1.astype(np.float64) / np.sqrt(2)))).astype(np.float32)
    f2 = oracle.mul_mat_native(w["fc2_type"], w["fc2_w"], g) + w["fc2_b"]
    return x1 + f2


@pytest.mark.parametrize("ws", [4, 0])
def test_block_composition(oracle, ws):
    """The C block equals the numpy composition of the pinned pieces in the
    reference graph order (windowed ws=4 on an 8x8 grid, and global)."""
    W = H = 8
    E, heads, mlp = 256, 4, 512
    per_w = ws if ws else W
    w = block_weights(oracle, E, mlp, heads, per_w * per_w, per_w, seed=5)
    x = np.random.default_rng(6).standard_normal((W * H, E)).astype(np.float32)
    y = oracle.vit_block(w, x, W, H, E, heads, mlp, ws)
    ref = np_block(oracle, w, x, W, H, E, heads, mlp, ws)
    rel = np.linalg.norm(y - ref, axis=1) / np.linalg.norm(ref, axis=1)
    # float64 vs float32 pieces only; a Q8_K activation rounding flip in a
    # linear moves a row by ~1e-4 of its norm
    assert rel.max() < 5e-4, rel.max()
    assert np.median(rel) < 1e-5


# ---- SimpleFPN neck ----------------------------------------------------------

def np_deconv(x, W, H, w, b, cout):
    """ConvTranspose2d k=2 s=2 in float64 (PyTorch semantics; weight ggml {2,2,Cout,Cin} = torch [Cin][Cout][2][2])."""
    cin = x.shape[1]
    wt = w.reshape(cin, cout, 2, 2).astype(np.float64)           # [ci][co][ky][kx]
    img = x.reshape(H, W, cin).astype(np.float64)
    out = np.einsum("yxc,cokl->ykxlo", img, wt).reshape(2 * H, 2 * W, cout)
    return (out + (0 if b is None else b)).reshape(-1, cout)


def np_conv(x, W, H, w, b, cout, k):
    """Conv2d stride 1, padding k//2, in float64 (weight ggml {k,k,Cin,Cout} = torch [Cout][Cin][k][k])."""
    cin, p = x.shape[1], k // 2
    wt = w.reshape(cout, cin, k, k).astype(np.float64)
    img = np.pad(x.reshape(H, W, cin).astype(np.float64), ((p, p), (p, p), (0, 0)))
    out = np.zeros((H, W, cout))
    for ky in range(k):
        for kx in range(k):
            out += img[ky:ky + H, kx:kx + W] @ wt[:, :, ky, kx].T
    return (out + (0 if b is None else b)).reshape(-1, cout)


def test_deconv_conv_pool_against_float64(oracle):
    rng = np.random.default_rng(12)
    W, H, cin, cout = 6, 4, 12, 8
    x = rng.standard_normal((W * H, cin)).astype(np.float32)
    wd = rng.standard_normal(2 * 2 * cout * cin).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32)
    assert np.abs(oracle.deconv2x2(x, W, H, wd, b, cout) - np_deconv(x, W, H, wd, b, cout)).max() < 1e-5
    for k in (1, 3):
        wc = rng.standard_normal(k * k * cin * cout).astype(np.float32)
        assert np.abs(oracle.conv2d(x, W, H, wc, b, cout, k) - np_conv(x, W, H, wc, b, cout, k)).max() < 1e-5
    # a 3x3 kernel with only the centre tap equals the 1x1 convolution
    w1 = rng.standard_normal(cin * cout).astype(np.float32)
    w3 = np.zeros((cout, cin, 3, 3), np.float32)
    w3[:, :, 1, 1] = w1.reshape(cout, cin)
    assert np.array_equal(oracle.conv2d(x, W, H, w3.ravel(), b, cout, 3), oracle.conv2d(x, W, H, w1, b, cout, 1))
    # F16 columns: the same convolution of fp16-rounded operands
    wc = rng.standard_normal(9 * cin * cout).astype(np.float32)
    got = oracle.conv2d(x, W, H, wc, b, cout, 3, columns_f16=True)
    ref = np_conv(x.astype(np.float16).astype(np.float32), W, H, wc.astype(np.float16).astype(np.float32), b, cout, 3)
    assert np.abs(got - ref).max() < 1e-5
    assert np.abs(got - oracle.conv2d(x, W, H, wc, b, cout, 3)).max() > 1e-4   # the rounding is visible
    p = oracle.maxpool2x2(x, W, H)
    assert np.array_equal(p, x.reshape(H // 2, 2, W // 2, 2, cin).max(axis=(1, 3)).reshape(-1, cin))


def test_neck_composition(oracle):
    """or_neck equals the reference graph's order of the pinned pieces."""
    rng = np.random.default_rng(13)
    grid, E, mid, D = 4, 16, 12, 8
    w = neck_weights(rng, E, mid, D)
    x = rng.standard_normal((grid * grid, E)).astype(np.float32)
    outs = oracle.neck(w, x, grid, E, mid, D)
    g = grid
    s0 = np_deconv(x, g, g, w["s0_dc1_w"], w["s0_dc1_b"], mid)
    s0 = (0.5 * s0 * (1 + erf(s0 / np.sqrt(2))))
    s0 = np_deconv(s0, 2 * g, 2 * g, w["s0_dc2_w"], w["s0_dc2_b"], D)
    s0 = np_conv(s0, 4 * g, 4 * g, w["s0_c1_w"], w["s0_c1_b"], D, 1)
    s0 = np_conv(s0, 4 * g, 4 * g, w["s0_c3_w"], w["s0_c3_b"], D, 3)
    s1 = np_deconv(x, g, g, w["s1_dc_w"], w["s1_dc_b"], mid)
    s1 = np_conv(np_conv(s1, 2 * g, 2 * g, w["s1_c1_w"], w["s1_c1_b"], D, 1), 2 * g, 2 * g, w["s1_c3_w"],
                 w["s1_c3_b"], D, 3)
    s2 = np_conv(np_conv(x, g, g, w["s2_c1_w"], w["s2_c1_b"], D, 1), g, g, w["s2_c3_w"], w["s2_c3_b"], D, 3)
    xp = x.reshape(g // 2, 2, g // 2, 2, E).max(axis=(1, 3)).reshape(-1, E)
    s3 = np_conv(np_conv(xp, g // 2, g // 2, w["s3_c1_w"], w["s3_c1_b"], D, 1), g // 2, g // 2, w["s3_c3_w"],
                 w["s3_c3_b"], D, 3)
    for got, ref in zip(outs, (s0, s1, s2, s3)):
        assert np.abs(got - ref).max() < 1e-4 * max(1.0, np.abs(ref).max())


def test_neck_scales_mapping():
    w = neck_weights(np.random.default_rng(0), 8, 8, 4)
    s = neck_scales(w)
    assert s[0]["deconv2_w"] is w["s0_dc2_w"] and s[1]["deconv1_b"] is w["s1_dc_b"]
    assert s[3]["conv3x3_w"] is w["s3_c3_w"] and "deconv1_w" not in s[2]
    assert sum(len(x) for x in s) == len(w)


def test_neck_skips_levels(oracle):
    rng = np.random.default_rng(14)
    grid, E, mid, D = 4, 16, 12, 8
    w = neck_weights(rng, E, mid, D)
    x = rng.standard_normal((grid * grid, E)).astype(np.float32)
    full = oracle.neck(w, x, grid, E, mid, D)
    part = oracle.neck(w, x, grid, E, mid, D, levels=(1, 2))
    assert part[0] is None and part[3] is None
    assert np.array_equal(part[1], full[1]) and np.array_equal(part[2], full[2])
    with pytest.raises(ValueError):
        oracle.neck(w, x[:9], 3, E, mid, D)   # level 3 of an odd grid
    assert oracle.neck(w, x[:9], 3, E, mid, D, levels=(2,))[2].shape == (9, D)
