"""Synthetic SAM 3 vision-encoder weights and inputs for the ViT tests.

Shapes follow the reference's tensor registry (src/models/sam3/tensors.hpp:
95-127): per block norm1/norm2 (E), qkv (E -> 3E) + bias, proj (E -> E) +
bias, mlp lin1 (E -> MLP) + bias, lin2 (MLP -> E) + bias, and a RoPE table
freqs_cis [tokens][hd/2][2] (cos, sin).  Linear weights are N(0, 0.02^2)
quantized by the oracle's ggml quantizers; biases and norms are small random
values so that every term of the block contributes.
"""

import numpy as np


def axial_rope_table(width, height, hd, theta=10000.0):
    """Axial 2-D RoPE table of SAM-style ViTs: hd/4 frequencies per axis,
    token t = y*width + x, pairs [x-frequencies..., y-frequencies...] as
    (cos, sin).  Any unit-modulus table exercises the same arithmetic."""
    freqs = 1.0 / theta ** (np.arange(0, hd, 4)[: hd // 4].astype(np.float64) / hd)
    t = np.arange(width * height)
    tx, ty = (t % width).astype(np.float64), (t // width).astype(np.float64)
    ang = np.concatenate([np.outer(tx, freqs), np.outer(ty, freqs)], axis=1)      # [N][hd/2]
    return np.stack([np.cos(ang), np.sin(ang)], axis=-1).astype(np.float32)      # [N][hd/2][2]


def block_weights(oracle, E, mlp, heads, tokens_rope, rope_w, seed, types=None):
    """One block's weights as numpy arrays (packed rows for the linears).
    types: dict qkv/proj/fc1/fc2 -> oracle type id (default Q4_K, fc2 Q8_0
    when MLP is not a multiple of 256)."""
    rng = np.random.default_rng(seed)
    hd = E // heads
    if types is None:
        k_type = oracle.Q4_K
        types = {"qkv": k_type, "proj": k_type, "fc1": k_type,
                 "fc2": k_type if mlp % 256 == 0 else oracle.Q8_0}
    shapes = {"qkv": (3 * E, E), "proj": (E, E), "fc1": (mlp, E), "fc2": (E, mlp)}
    w = {}
    for i, (name, (n, k)) in enumerate(shapes.items()):
        wf = oracle.rng_normal(1000 * seed + i, n * k, 0.0, 0.02).reshape(n, k)
        w[name + "_type"] = types[name]
        w[name + "_w"] = oracle.quantize(types[name], wf)
        w[name + "_b"] = (rng.standard_normal(n) * 0.05).astype(np.float32)
    w["norm1_w"] = (1.0 + 0.1 * rng.standard_normal(E)).astype(np.float32)
    w["norm1_b"] = (0.05 * rng.standard_normal(E)).astype(np.float32)
    w["norm2_w"] = (1.0 + 0.1 * rng.standard_normal(E)).astype(np.float32)
    w["norm2_b"] = (0.05 * rng.standard_normal(E)).astype(np.float32)
    w["freqs"] = axial_rope_table(rope_w, tokens_rope // rope_w, hd)
    return w


def neck_weights(rng, E, mid, D, scale=0.05):
    """SimpleFPN weights in ggml layouts (flat), keyed as the oracle's
    or_neck_weights: deconvolutions {2, 2, Cout, Cin}, convolutions
    {k, k, Cin, Cout} (numpy shapes are the reversed ggml dims)."""
    def r(*shape):
        return (rng.standard_normal(shape) * scale).astype(np.float32).ravel()
    return {"s0_dc1_w": r(E, mid, 2, 2), "s0_dc1_b": r(mid), "s0_dc2_w": r(mid, D, 2, 2), "s0_dc2_b": r(D),
            "s0_c1_w": r(D, D), "s0_c1_b": r(D), "s0_c3_w": r(D, D, 3, 3), "s0_c3_b": r(D),
            "s1_dc_w": r(E, mid, 2, 2), "s1_dc_b": r(mid), "s1_c1_w": r(D, mid), "s1_c1_b": r(D),
            "s1_c3_w": r(D, D, 3, 3), "s1_c3_b": r(D), "s2_c1_w": r(D, E), "s2_c1_b": r(D),
            "s2_c3_w": r(D, D, 3, 3), "s2_c3_b": r(D), "s3_c1_w": r(D, E), "s3_c1_b": r(D),
            "s3_c3_w": r(D, D, 3, 3), "s3_c3_b": r(D)}


_NECK_SCALE_KEYS = {"dc1": "deconv1", "dc": "deconv1", "dc2": "deconv2", "c1": "conv1x1", "c3": "conv3x3"}


def neck_scales(weights):
    """The oracle-keyed neck weights as 4 per-scale dicts (samhip_neck_scale fields)."""
    scales = [{}, {}, {}, {}]
    for name, value in weights.items():
        level, part, kind = name.split("_")
        scales[int(level[1])][f"{_NECK_SCALE_KEYS[part]}_{kind}"] = value
    return scales
