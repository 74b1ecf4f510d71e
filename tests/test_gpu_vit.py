"""Vision-encoder parity on the GPU: samhip_layer_norm, samhip_flash_attn,
samhip_vit_prefix and samhip_vit_block against the oracle's restatement of
the reference graph (oracle/vit_oracle.c, pinned in tests/test_vit_oracle.py),
on the same seeded inputs and packed weights.

Tolerances (per output row, relative L2 against the oracle):
  * layer norm: 2e-6 (F32 both sides; sums in a different order);
  * patch prefix: 1e-5 (split-fp16 operands carry ~22 bits);
  * attention (samhip_flash_attn, F32-accurate as the reference's
    GGML_PREC_F32): 1e-5 max / 2e-6 median: q, k, v and the softmax weights
    enter the products split into two fp16 halves (~22 bits), the oracle
    sums its scores in F32;
  * block, attention half (MLP weights zero): F32 attention 3e-4 max /
    1.2e-4 median (what remains is the linears' fp16 operands), fp16
    attention (attention_type F16: q, k, v and P rounded
    to fp16, unit roundoff 2^-11) 5e-4 / 2e-4, carried through proj into a
    residual stream that dominates the row norm;
  * block, F16 compute and fp16 attention against the oracle's F32-decode
    path: 1e-3 max / 3e-4 median (fp16 operands, no activation
    quantization);
  * block, native Q8 compute: 6e-3 max / 4e-3 median.  Both sides quantize
    each linear's input to 8-bit codes; where the inputs differ in low bits
    (fp16 weights and attention upstream) a code near a rounding boundary
    flips by one step d = amax/127.  For fc2 (K = 4736 Q8_0 inputs after
    GELU, about 1 % of codes flipping) that moves an output by about
    sqrt(0.01 * 4736) * d * |w| ~ 2e-3, i.e. ~3e-3 of the MLP branch.
"""

import numpy as np
import pytest

from tests.vit_fixtures import axial_rope_table, block_weights

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def row_rel(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    return np.linalg.norm(got - ref, axis=1) / np.maximum(np.linalg.norm(ref, axis=1), 1e-30)


@pytest.mark.parametrize("rows,n", [(5184, 1024), (37, 256), (3, 2048)])
def test_layer_norm(gpu_ctx, oracle, rows, n):
    rng = np.random.default_rng(rows)
    x = (rng.standard_normal((rows, n)) * 2 + 0.5).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    b = (0.1 * rng.standard_normal(n)).astype(np.float32)
    say(f"layer_norm rows={rows} n={n}")
    got = gpu_ctx.layer_norm(x, w, b)
    ref = oracle.layer_norm(x, w, b)
    assert row_rel(got, ref).max() < 2e-6
    assert np.array_equal(gpu_ctx.layer_norm(np.full((4, 256), 7.0, np.float32)), np.zeros((4, 256), np.float32))


@pytest.mark.parametrize("batches,n,heads", [(9, 576, 16), (3, 100, 2), (1, 5184, 2), (2, 64, 1), (1, 1, 3)])
def test_flash_attn(gpu_ctx, oracle, batches, n, heads):
    rng = np.random.default_rng(n + heads)
    hd = 64
    q, k, v = (rng.standard_normal((batches * n, heads * hd)).astype(np.float32) for _ in range(3))
    say(f"flash_attn batches={batches} n={n} heads={heads}")
    got = gpu_ctx.flash_attn(q, k, v, batches, heads, 0.125)
    ref = np.concatenate([oracle.attention(q[b * n:(b + 1) * n], k[b * n:(b + 1) * n], v[b * n:(b + 1) * n],
                                           heads, hd, 0.125) for b in range(batches)])
    rel = row_rel(got.reshape(-1, hd), ref.reshape(-1, hd))   # per (token, head)
    say(f"  max {rel.max():.3g} median {np.median(rel):.3g}")
    assert rel.max() < 1e-5 and np.median(rel) < 2e-6


@pytest.mark.parametrize("splits", [2, 3, 4])
def test_flash_attn_key_splits(samhip, oracle, monkeypatch, splits):
    """Keys split over several workgroups per query block and merged
    (SAMHIP_ATTN_SPLITS forces the count, which is cut back so that every
    split keeps a key tile: 9 tiles at n = 576, a ragged last tile at 1000,
    a peaked row): the merged result stays F32-accurate."""
    monkeypatch.setenv("SAMHIP_ATTN_SPLITS", str(splits))
    ctx = samhip.Context(0)
    try:
        for batches, n, heads in ((2, 576, 2), (1, 1000, 3), (1, 130, 1)):
            rng = np.random.default_rng(n + splits)
            q, k, v = (rng.standard_normal((batches * n, heads * 64)).astype(np.float32) for _ in range(3))
            q[0] *= 40   # one query with a dominant key
            say(f"flash_attn splits={splits} batches={batches} n={n} heads={heads}")
            got = ctx.flash_attn(q, k, v, batches, heads, 0.125)
            ref = np.concatenate([oracle.attention(q[b * n:(b + 1) * n], k[b * n:(b + 1) * n],
                                                   v[b * n:(b + 1) * n], heads, 64, 0.125) for b in range(batches)])
            rel = row_rel(got.reshape(-1, 64), ref.reshape(-1, 64))
            say(f"  max {rel.max():.3g} median {np.median(rel):.3g}")
            assert np.all(np.isfinite(got)) and rel.max() < 1e-5 and np.median(rel) < 2e-6
    finally:
        ctx.close()


@pytest.mark.parametrize("splits", [2, 3, 4])
def test_vit_block_fp16_attention_key_splits(samhip, oracle, monkeypatch, splits):
    """The fp16-operand attention (attention_type F16) with its keys split
    and merged inside a block, on ragged key tiles (20x20 grid: global, 400
    tokens = 7 tiles with a partial last one; window 10, 100 tokens = 2
    tiles): the trace names the split count that ran, and the block matches
    the oracle as the unsplit fp16 block does."""
    monkeypatch.setenv("SAMHIP_ATTN_SPLITS", str(splits))
    ctx = samhip.Context(0)
    try:
        for ws, tiles in ((0, 7), (10, 2)):
            say(f"vit_block fp16 attention splits={splits} window={ws}")
            per_w = ws if ws else 20
            w = block_weights(oracle, 256, 640, 4, per_w * per_w, per_w, seed=61 + ws)
            x = np.random.default_rng(62 + ws).standard_normal((400, 256)).astype(np.float32)
            blk = samhip.VitBlock(ctx, w, 256, 4, 640, 20, 20, ws, attention_type=samhip.F16)
            xb = ctx.upload(x)
            ctx.trace_begin()
            blk.forward(xb)
            names = [r[0] for r in ctx.trace_end()]
            got = ctx.download(xb, x.shape, np.float32)
            blk.free()
            want = f"vit_attention_split{min(splits, tiles)}"
            assert want in names, names
            ref = oracle.vit_block(w, x, 20, 20, 256, 4, 640, ws)
            rel = row_rel(got, ref)
            say(f"  ran {want}: max {rel.max():.3g} median {np.median(rel):.3g}")
            assert np.isfinite(got).all() and rel.max() < 6e-3 and np.median(rel) < 4e-3
    finally:
        ctx.close()


def test_flash_attn_rejects(gpu_ctx, samhip):
    x = np.zeros((64, 128), np.float32)
    with pytest.raises(samhip.SamhipError, match="head_dim"):
        gpu_ctx.flash_attn(x, x, x, 1, 4, 0.125, head_dim=32)


def test_flash_attn_peaked_softmax(gpu_ctx, oracle):
    """Large logits (one dominant key per query) and a constant row: the
    online softmax rescaling must keep the result F32-accurate."""
    n, heads, hd = 256, 1, 64
    rng = np.random.default_rng(7)
    k = rng.standard_normal((n, hd)).astype(np.float32)
    q = (k[rng.permutation(n)] * 4).astype(np.float32)    # logits up to ~4*64/8 = 32
    v = rng.standard_normal((n, hd)).astype(np.float32)
    q[0] = 0                                             # uniform weights over all keys
    got = gpu_ctx.flash_attn(q, k, v, 1, heads, 0.125)
    ref = oracle.attention(q, k, v, heads, hd, 0.125)
    rel = row_rel(got, ref)
    say(f"  peaked max {rel.max():.3g}")
    assert rel.max() < 1e-5
    assert np.allclose(got[0], v.mean(0), atol=1e-5)


def test_vit_prefix_full_size(gpu_ctx, oracle, samhip):
    img, patch, E, pg = 1008, 14, 1024, 24
    rng = np.random.default_rng(11)
    image = rng.standard_normal((3, img, img)).astype(np.float32)
    kernel = (rng.standard_normal((E, 3, patch, patch)) * 0.02).astype(np.float32)
    pos = (rng.standard_normal((pg, pg, E)) * 0.1).astype(np.float32)
    lw = (1 + 0.1 * rng.standard_normal(E)).astype(np.float32)
    lb = (0.1 * rng.standard_normal(E)).astype(np.float32)
    say("vit_prefix 1008px")
    pre = samhip.VitPrefix(gpu_ctx, kernel, pos, lw, lb, img, patch, E, pg)
    ib = gpu_ctx.upload(image)
    xb = gpu_ctx.alloc((img // patch) ** 2 * E * 4)
    pre.forward(ib, xb)
    got = gpu_ctx.download(xb, ((img // patch) ** 2, E), np.float32)
    ref = oracle.vit_prefix(image, patch, kernel, pos, pg, lw, lb, E)
    rel = row_rel(got, ref)
    say(f"  max {rel.max():.3g}")
    assert rel.max() < 1e-5
    pre.free()


@pytest.fixture(scope="module")
def f16_ctx(samhip):
    ctx = samhip.Context(0, samhip.COMPUTE_F16, samhip.ROUND_X86)
    yield ctx
    ctx.close()


def _block_case(ctx, oracle, samhip, grid, E, heads, mlp, ws, seed, types=None, zero_mlp=False, decode=False,
                attention=None):
    per_w = ws if ws else grid
    w = block_weights(oracle, E, mlp, heads, per_w * per_w, per_w, seed, types)
    if zero_mlp:
        w["fc1_w"] = np.zeros_like(w["fc1_w"])
        w["fc2_w"] = np.zeros_like(w["fc2_w"])
    x = (np.random.default_rng(seed + 100).standard_normal((grid * grid, E))).astype(np.float32)
    blk = samhip.VitBlock(ctx, w, E, heads, mlp, grid, grid, ws,
                          samhip.F32 if attention is None else attention)
    xb = ctx.upload(x)
    blk.forward(xb)
    got = ctx.download(xb, x.shape, np.float32)
    ref = oracle.vit_block(w, x, grid, grid, E, heads, mlp, ws, decode=decode)
    blk.free()
    return row_rel(got, ref), got


@pytest.mark.parametrize("ws", [24, 0])
def test_vit_block_full_size(gpu_ctx, oracle, samhip, ws):
    """SAM 3 block shapes: 72x72 tokens, width 1024, 16 heads, MLP 4736;
    Q4_K qkv/proj/fc1, Q8_0 fc2; windowed (24) and global."""
    say(f"vit_block 72x72 E=1024 window={ws}")
    rel, got = _block_case(gpu_ctx, oracle, samhip, 72, 1024, 16, 4736, ws, seed=21 + ws)
    say(f"  max {rel.max():.3g} median {np.median(rel):.3g}")
    assert np.isfinite(got).all()
    assert rel.max() < 6e-3 and np.median(rel) < 4e-3


@pytest.mark.parametrize("ws", [24, 0])
@pytest.mark.parametrize("attention", ["f32", "f16"])
def test_vit_block_attention_half(gpu_ctx, oracle, samhip, ws, attention):
    """Same block with the MLP weights zero, so the output is the attention
    half (LN1, window partition, qkv, RoPE, attention, proj, unpartition,
    residual) plus constant MLP terms: no 8-bit code flips downstream."""
    say(f"vit_block attention half window={ws} attention {attention}")
    rel, _ = _block_case(gpu_ctx, oracle, samhip, 72, 1024, 16, 4736, ws, seed=23 + ws, zero_mlp=True,
                         attention=samhip.F32 if attention == "f32" else samhip.F16)
    say(f"  max {rel.max():.3g} median {np.median(rel):.3g}")
    if attention == "f32":
        assert rel.max() < 3e-4 and np.median(rel) < 1.2e-4
    else:
        assert rel.max() < 5e-4 and np.median(rel) < 2e-4


@pytest.mark.parametrize("ws", [24, 0])
def test_vit_block_f16_compute(f16_ctx, oracle, samhip, ws):
    """F16 compute (fp16 activations, no 8-bit codes) with fp16 attention
    against the oracle's F32-decode linears: every op of the block with only
    fp16 rounding."""
    say(f"vit_block f16 compute window={ws}")
    rel, _ = _block_case(f16_ctx, oracle, samhip, 72, 1024, 16, 4736, ws, seed=25 + ws, decode=True,
                         attention=samhip.F16)
    say(f"  max {rel.max():.3g} median {np.median(rel):.3g}")
    assert rel.max() < 1e-3 and np.median(rel) < 3e-4


@pytest.mark.parametrize("types", ["q8_0", "q6_k"])
def test_vit_block_formats(gpu_ctx, oracle, samhip, types):
    """A reduced block (16x16 grid, window 8, width 256) in all-Q8_0 and
    Q6_K/Q8_0 storage."""
    t = {"q8_0": dict(qkv=oracle.Q8_0, proj=oracle.Q8_0, fc1=oracle.Q8_0, fc2=oracle.Q8_0),
         "q6_k": dict(qkv=oracle.Q6_K, proj=oracle.Q6_K, fc1=oracle.Q6_K, fc2=oracle.Q8_0)}[types]
    say(f"vit_block 16x16 E=256 {types}")
    rel, _ = _block_case(gpu_ctx, oracle, samhip, 16, 256, 4, 640, 8, seed=31, types=t)
    say(f"  max {rel.max():.3g} median {np.median(rel):.3g}")
    assert rel.max() < 6e-3 and np.median(rel) < 4e-3


def test_vit_block_is_deterministic(gpu_ctx, oracle, samhip):
    w = block_weights(oracle, 256, 640, 4, 64, 8, seed=41)
    x = np.random.default_rng(42).standard_normal((256, 256)).astype(np.float32)
    blk = samhip.VitBlock(gpu_ctx, w, 256, 4, 640, 16, 16, 8)
    outs = []
    for _ in range(2):
        xb = gpu_ctx.upload(x)
        blk.forward(xb)
        outs.append(gpu_ctx.download(xb, x.shape, np.float32))
    blk.free()
    assert np.array_equal(outs[0], outs[1])


def _block_run(ctx, samhip, w, x, E, heads, mlp, grid, ws):
    blk = samhip.VitBlock(ctx, w, E, heads, mlp, grid, grid, ws)
    xb = ctx.upload(x)
    ctx.trace_begin()
    blk.forward(xb)
    names = [r[0] for r in ctx.trace_end()]
    got = ctx.download(xb, x.shape, np.float32)
    blk.free()
    return got, names


@pytest.mark.parametrize("rounding", ["x86", "ref"])
@pytest.mark.parametrize("case", ["72x72_window24", "72x72_global", "16x16_wide_range"])
def test_vit_block_fc1_codes_same_bits(samhip, oracle, monkeypatch, rounding, case):
    """SAMHIP_VIT_FC1_CODES=1: with a Q8_0 fc2 in native compute, fc1's
    epilogue applies the erf-GELU and writes fc2's Q8_0 codes and F32 block
    maxima, and fc2's staging expands them (stage_codes_q8_0).  The block
    output must have the bits of the default path, which writes fc1's F32
    rows and packs them in fc2's staging, in both Q8_0 roundings: full SAM 3
    blocks, and a reduced block whose fc1 bias spreads the rows over ~5
    decades with one all-zero 32-column block (amax 0, codes 0)."""
    rnd = samhip.ROUND_X86 if rounding == "x86" else samhip.ROUND_REF
    if case.startswith("72x72"):
        grid, E, heads, mlp, ws = 72, 1024, 16, 4736, (24 if case.endswith("24") else 0)
    else:
        grid, E, heads, mlp, ws = 16, 256, 4, 640, 8
    per_w = ws if ws else grid
    w = block_weights(oracle, E, mlp, heads, per_w * per_w, per_w, seed=71 + ws)
    assert w["fc2_type"] == oracle.Q8_0
    if case == "16x16_wide_range":
        w["fc1_b"] = (w["fc1_b"] * np.where(np.arange(mlp) % 7 == 0, 4e3, 1.0)).astype(np.float32)
        fc1 = w["fc1_w"].reshape(mlp, -1).copy()
        fc1[64:96] = 0   # all-zero packed rows decode to 0
        w["fc1_w"] = fc1
        w["fc1_b"][64:96] = 0.0
    x = np.random.default_rng(72 + ws).standard_normal((grid * grid, E)).astype(np.float32)
    say(f"vit_block fc1 codes {case} rounding={rounding}")
    monkeypatch.setenv("SAMHIP_VIT_FC1_CODES", "1")
    ctx = samhip.Context(0, samhip.COMPUTE_Q8_NATIVE, rnd)
    try:
        got, names = _block_run(ctx, samhip, w, x, E, heads, mlp, grid, ws)
    finally:
        ctx.close()
    monkeypatch.delenv("SAMHIP_VIT_FC1_CODES")
    ctx = samhip.Context(0, samhip.COMPUTE_Q8_NATIVE, rnd)
    try:
        want, names_f32 = _block_run(ctx, samhip, w, x, E, heads, mlp, grid, ws)
    finally:
        ctx.close()
    assert "stage_codes_q8_0" in names and "stage_codes_q8_0" not in names_f32, (names, names_f32)
    assert np.isfinite(got).all()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_vit_block_kquant_fc2_keeps_f32_rows(samhip, oracle, monkeypatch):
    """Even with SAMHIP_VIT_FC1_CODES=1, a K-quant fc2 packs Q8_K blocks of
    256 values, which no fc1 tile holds: fc1 writes F32 rows and fc2's
    staging packs them."""
    t = dict(qkv=oracle.Q4_K, proj=oracle.Q4_K, fc1=oracle.Q4_K, fc2=oracle.Q6_K)
    w = block_weights(oracle, 256, 768, 4, 64, 8, seed=75, types=t)
    x = np.random.default_rng(76).standard_normal((256, 256)).astype(np.float32)
    monkeypatch.setenv("SAMHIP_VIT_FC1_CODES", "1")
    ctx = samhip.Context(0)
    try:
        _, names = _block_run(ctx, samhip, w, x, 256, 4, 768, 16, 8)
    finally:
        ctx.close()
    assert "stage_codes_q8_0" not in names and "stage_dequant_q8_k" in names, names


def test_vit_block_rejects(gpu_ctx, oracle, samhip):
    w = block_weights(oracle, 256, 640, 4, 64, 8, seed=51)
    x = gpu_ctx.upload(np.zeros((256, 256), np.float32))
    with pytest.raises(samhip.SamhipError, match="multiples of the window"):
        samhip.VitBlock(gpu_ctx, w, 256, 4, 640, 16, 16, 6).forward(x)
    with pytest.raises(samhip.SamhipError, match="head_dim"):
        samhip.VitBlock(gpu_ctx, w, 256, 2, 640, 16, 16, 8).forward(x)
    bad = dict(w)
    bad["fc1_w"] = w["fc1_w"][:320]                      # fewer rows than mlp
    blk = samhip.VitBlock(gpu_ctx, bad, 256, 4, 640, 16, 16, 8)
    blk.desc.fc1_w.ne[1] = 320
    with pytest.raises(samhip.SamhipError, match="fc1 weight: shape"):
        blk.forward(x)


def test_vit_block_rejects_attention_type(gpu_ctx, oracle, samhip):
    w = block_weights(oracle, 256, 640, 4, 64, 8, seed=52)
    x = gpu_ctx.upload(np.zeros((256, 256), np.float32))
    blk = samhip.VitBlock(gpu_ctx, w, 256, 4, 640, 16, 16, 8, attention_type=samhip.Q8_0)
    with pytest.raises(samhip.SamhipError, match="attention type"):
        blk.forward(x)
    blk.free()
    x.free()
