"""GGUF reader, storage-profile checks and weight upload
(sam.cpp_amd/host/gguf_reader.hpp) through tests/host/_build/gguf_tool.

The rejection cases are the reference's loader contract test, byte for byte
(tests/api/test_contracts.cpp:364-460): the same probe fixture, the same
mutations at the same offsets.  Those offsets are computed from the GGUF
layout, so they also pin the independent Python writer (tests/gguf_fixture.py)
and the C++ reader to that layout.  Profile cases follow
src/models/sam3/weights.hpp:537-623; the GPU case loads a schema-3 Q4_K
checkpoint with ViT-shaped linears and checks the device bytes and products.
"""

import json
import struct
import os
import subprocess

import numpy as np
import pytest

from tests import gguf_fixture as gg

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TOOL = os.path.join(ROOT, "tests", "host", "_build", "gguf_tool")


def tool(*args, timeout=300):
    if not os.path.exists(TOOL):
        pytest.fail(f"{TOOL} is not built: run make -C tests/host")
    out = subprocess.run([TOOL, *map(str, args)], capture_output=True, text=True, timeout=timeout)
    return out


def inspect(path):
    out = tool("inspect", path)
    if out.returncode == 3:
        return None, json.loads(out.stdout)["error"]
    assert out.returncode == 0, out.stdout + out.stderr
    return json.loads(out.stdout), None


def write(tmp_path, data, name="container.gguf"):
    path = tmp_path / name
    path.write_bytes(bytes(data))
    return path


def test_probe_fixture_reads(tmp_path):
    path = write(tmp_path, gg.probe_fixture())
    info, err = inspect(path)
    assert err is None
    (t,) = info["tensors"]
    assert t["name"] == "probe.weight" and t["dims"] == [1, 3, 2] and t["ne"] == [1, 3, 2, 1]
    assert t["type"] == 0 and t["size"] == 24
    assert t["offset"] == info["data_offset"] and info["data_offset"] % 32 == 0
    assert info["size"] == info["data_offset"] + 32           # 24 bytes + 8 bytes of padding
    out = tool("contract", path)
    assert out.returncode == 0 and "contract: 0 failed" in out.stdout, out.stdout + out.stderr


def test_missing_file(tmp_path):
    _, err = inspect(tmp_path / "missing.gguf")
    assert "cannot open SAM checkpoint" in err


def _mut_alignment_field(data, value):
    gg.integer_at(data, gg.text_at(data, "general.alignment") + 17 + 4, value, 4)


# (mutation, second tensor, expected message fragment); mutations and
# offsets are those of tests/api/test_contracts.cpp:399-431
REJECTIONS = {
    "truncated header": (lambda b: b.__delitem__(slice(3, None)), False, "truncated GGUF checkpoint header"),
    "version 2": (lambda b: gg.integer_at(b, 4, 2, 4), False, "GGUF v3"),
    "tensor count 4097": (lambda b: gg.integer_at(b, 8, 4097), False, "count exceeds"),
    "key count 257": (lambda b: gg.integer_at(b, 16, 257), False, "count exceeds"),
    "truncated final padding": (lambda b: b.pop(), False, "truncated GGUF tensor range"),
    "nonzero padding": (lambda b: b.__setitem__(len(b) - 1, 1), False, "nonzero GGUF tensor padding"),
    "trailing payload": (lambda b: b.append(0), False, "unexpected data after"),
    "oversized array": (lambda b: gg.integer_at(b, gg.text_at(b, "probe.indices") + 13 + 8, 2**64 - 1),
                        False, "oversized GGUF array"),
    "oversized string": (lambda b: gg.integer_at(b, gg.text_at(b, "probe.label") + 11 + 4, 16 * 1024 * 1024 + 1),
                         False, "oversized GGUF metadata"),
    "NUL in value": (lambda b: b.__setitem__(gg.text_at(b, "labelx") + 5, 0), False, "NUL"),
    "NUL in tensor name": (lambda b: b.__setitem__(gg.text_at(b, "probe.weight") + 11, 0), False, "NUL"),
    "NUL in key": (lambda b: b.__setitem__(gg.text_at(b, "probe.label") + 10, 0), False, "NUL"),
    "zero dimension": (lambda b: gg.integer_at(b, gg.text_at(b, "probe.weight") + 12 + 4, 0), False,
                       "invalid or overflowing GGUF tensor dimensions"),
    "overflowing shape": (lambda b: (gg.integer_at(b, gg.text_at(b, "probe.weight") + 16, 1 << 32),
                                     gg.integer_at(b, gg.text_at(b, "probe.weight") + 24, 1 << 32)),
                          False, "invalid or overflowing GGUF tensor dimensions"),
    "unknown type": (lambda b: gg.integer_at(b, gg.text_at(b, "probe.weight") + 12 + 4 + 24, 255, 4), False,
                     "unsupported GGUF tensor type"),
    "overlapping offsets": (lambda b: gg.integer_at(b, gg.text_at(b, "other.weight") + 12 + 4 + 24 + 4, 0), True,
                            "overlapping"),
    "overflowing offset": (lambda b: gg.integer_at(b, gg.text_at(b, "other.weight") + 12 + 4 + 24 + 4, 2**64 - 1),
                           True, "overflowing"),
    "duplicate tensor names": (lambda b: b.__setitem__(slice(gg.text_at(b, "other.weight"),
                                                             gg.text_at(b, "other.weight") + 12), b"probe.weight"),
                               True, "duplicate GGUF tensor name"),
    "legacy magic": (lambda b: gg.integer_at(b, 0, 0x73616D33, 4), False, "original .pt"),
}


@pytest.mark.parametrize("case", sorted(REJECTIONS))
def test_reference_rejections(tmp_path, case):
    mutate, second, message = REJECTIONS[case]
    data = bytearray(gg.probe_fixture(second_tensor=second))
    assert inspect(write(tmp_path, data))[1] is None          # the unmutated file is valid
    mutate(data)
    info, err = inspect(write(tmp_path, data))
    assert info is None, f"{case} was accepted"
    assert message in err, err


@pytest.mark.parametrize("alignment", [0, 3, 64])
def test_alignment_must_be_32(tmp_path, alignment):
    data = bytearray(gg.probe_fixture(extra_kv=[("general.alignment", gg.U32, 32)]))
    assert inspect(write(tmp_path, data))[1] is None
    _mut_alignment_field(data, alignment)
    assert "32-byte alignment" in inspect(write(tmp_path, data))[1]


def test_misaligned_quantized_row_width(tmp_path, oracle):
    """A Q8_0 tensor whose element count is block-aligned but whose row
    width is not (32 x 2 rewritten as 16 x 4) is rejected
    (tests/api/test_contracts.cpp:386-394)."""
    row = (np.arange(32, dtype=np.float32) - 16) / 16
    packed = oracle.quantize(gg.GGML_Q8_0, np.stack([row, row]), rounding=oracle.ROUND_REF).tobytes()
    data = bytearray(gg.gguf_bytes([], [("probe.quant", (32, 2), gg.GGML_Q8_0, packed)]))
    assert inspect(write(tmp_path, data))[1] is None
    at = gg.text_at(data, "probe.quant") + len("probe.quant") + 4
    gg.integer_at(data, at, 16)
    gg.integer_at(data, at + 8, 4)
    assert "not quantization-block aligned" in inspect(write(tmp_path, data))[1]


def _raw_tensor_info_file(dims_written):
    """probe.weight with its tensor-info dims written as given (the writer
    drops trailing 1s; a file that keeps them is a noncanonical encoding)."""
    data = bytearray(gg.probe_fixture())
    at = gg.text_at(data, "probe.weight") + 12
    old_nd = int.from_bytes(data[at:at + 4], "little")
    new = len(dims_written).to_bytes(4, "little") + b"".join(int(d).to_bytes(8, "little") for d in dims_written)
    data[at:at + 4 + 8 * old_nd] = new
    # re-pad the metadata to 32 bytes and keep the blob
    blob = bytes(data[-32:])
    meta_end = at + len(new) + 4 + 8
    meta = bytes(data[:meta_end])
    return meta + b"\0" * ((-len(meta)) % 32) + blob


def test_trailing_unit_dimension_is_noncanonical(tmp_path):
    assert inspect(write(tmp_path, _raw_tensor_info_file([1, 3, 2])))[1] is None
    err = inspect(write(tmp_path, _raw_tensor_info_file([1, 3, 2, 1])))[1]
    assert "noncanonical" in err


def test_more_rejections(tmp_path):
    base = gg.probe_fixture()
    # duplicate key
    data = gg.probe_fixture(extra_kv=[("probe.scalar", gg.U32, 18)])
    assert "ambiguous GGUF metadata key" in inspect(write(tmp_path, data))[1]
    # a bool that is neither 0 nor 1
    data = bytearray(gg.probe_fixture(extra_kv=[("probe.flag", gg.BOOL, True)]))
    data[gg.text_at(data, "probe.flag") + 10 + 4] = 2
    assert "bool" in inspect(write(tmp_path, data))[1]
    # a nonzero byte in the padding between metadata and data
    data = bytearray(base)
    info, _ = inspect(write(tmp_path, data))
    assert data[info["data_offset"] - 1] == 0 and data[info["data_offset"] - 9:info["data_offset"]] == bytes(9)
    data[info["data_offset"] - 1] = 7
    assert "noncanonical" in inspect(write(tmp_path, data))[1]
    # metadata cut short
    assert "truncated" in inspect(write(tmp_path, base[:60]))[1]
    # tensor name of 64 bytes
    data = gg.gguf_bytes([], [("t" * 64, (4,), gg.GGML_F32, bytes(16))])
    assert "too long" in inspect(write(tmp_path, data))[1]
    data = gg.gguf_bytes([], [("t" * 63, (4,), gg.GGML_F32, bytes(16))])
    assert inspect(write(tmp_path, data))[1] is None
    # empty key
    data = gg.gguf_bytes([("", gg.U32, 1)], [("t", (4,), gg.GGML_F32, bytes(16))])
    assert "empty GGUF key" in inspect(write(tmp_path, data))[1]


def test_every_metadata_type_round_trips(tmp_path):
    """Every GGUF value type parses and re-serializes canonically (a float
    NaN payload and a negative zero included)."""
    kv = [("u8", gg.U8, 250), ("i8", gg.I8, -3), ("u16", gg.U16, 65000), ("i16", gg.I16, -30000),
          ("u32", gg.U32, 4000000000), ("i32", gg.I32, -2000000000), ("f32", gg.F32, -0.0),
          ("bool", gg.BOOL, True), ("str", gg.STRING, ""), ("u64", gg.U64, 2**63 + 5),
          ("i64", gg.I64, -2**62), ("f64", gg.F64, float("nan")),
          ("a.f32", gg.ARRAY, (gg.F32, [1.5, float("inf")])), ("a.str", gg.ARRAY, (gg.STRING, ["", "x"])),
          ("a.empty", gg.ARRAY, (gg.U8, [])), ("a.i64", gg.ARRAY, (gg.I64, [-1, 2]))]
    data = gg.gguf_bytes(kv, [("t", (32, 2), gg.GGML_F16, bytes(128))])
    info, err = inspect(write(tmp_path, data))
    assert err is None and info["tensors"][0]["size"] == 128


# ---------------------------------------------------------------------------
# Storage profiles
# ---------------------------------------------------------------------------

def _q(oracle, qtype, k, n, seed):
    w = oracle.rng_normal(seed, n * k, 0.0, 0.02).reshape(n, k)
    return oracle.quantize(qtype, w).tobytes()


def _image_kv(schema, profile, file_type, qversion=2, extra=()):
    kv = [("general.architecture", gg.STRING, "sam3"), ("sam.schema_version", gg.U32, schema),
          ("sam.task", gg.STRING, "text_image"), ("general.file_type", gg.U32, file_type)]
    if qversion is not None:
        kv.append(("general.quantization_version", gg.U32, qversion))
    if profile is not None:
        kv.append(("sam.storage_profile", gg.STRING, profile))
    return kv + list(extra)


def _image_tensors(oracle, rows=64, kq=gg.GGML_Q4_K):
    """ViT block-0 linears at their real row widths (ne[0] = K) with a few
    output rows each: qkv / proj / lin1 in the profile's K type, lin2
    (ne[0] = 4736) in the Q8_0 fallback, plus an F32 norm."""
    return [("vit.blocks.0.attn.qkv.weight", (1024, rows), kq, _q(oracle, kq, 1024, rows, 1)),
            ("vit.blocks.0.attn.proj.weight", (1024, rows), kq, _q(oracle, kq, 1024, rows, 2)),
            ("vit.blocks.0.mlp.lin1.weight", (1024, rows), kq, _q(oracle, kq, 1024, rows, 3)),
            ("vit.blocks.0.mlp.lin2.weight", (4736, rows), gg.GGML_Q8_0, _q(oracle, gg.GGML_Q8_0, 4736, rows, 4)),
            ("vit.blocks.0.norm1.weight", (1024,), gg.GGML_F32, np.ones(1024, np.float32).tobytes())]


def profile(path):
    out = tool("profile", path)
    if out.returncode == 3:
        return json.loads(out.stdout)["error"]
    assert out.returncode == 0, out.stdout + out.stderr
    return json.loads(out.stdout)


def test_schema3_profile_accepts_canonical_types(tmp_path, oracle):
    data = gg.gguf_bytes(_image_kv(3, "image-linear-q4_k-v1", 14), _image_tensors(oracle))
    assert profile(write(tmp_path, data)) == {"ok": True, "constrained": 5}


@pytest.mark.parametrize("change,message", [
    (dict(profile="image-linear-q8_0-v1"), "file type does not match"),
    (dict(profile="image-linear-q3_k-v1"), "storage profile"),
    (dict(profile=None), "missing its storage profile"),
    (dict(qversion=1), "quantization version"),
    (dict(qversion=None), "general.quantization_version"),
])
def test_schema3_profile_rejections(tmp_path, oracle, change, message):
    args = dict(profile="image-linear-q4_k-v1", qversion=2)
    args.update(change)
    data = gg.gguf_bytes(_image_kv(3, args["profile"], 14, args["qversion"]), _image_tensors(oracle))
    err = profile(write(tmp_path, data))
    assert isinstance(err, str) and message in err, err


def test_schema3_profile_rejects_wrong_tensor_type(tmp_path, oracle):
    """qkv stored as Q8_0 in a Q4_K file; a K-quant lin2 cannot exist
    (4736 is not a multiple of 256) and is rejected by the reader."""
    tensors = _image_tensors(oracle)
    tensors[0] = (tensors[0][0], (1024, 64), gg.GGML_Q8_0, _q(oracle, gg.GGML_Q8_0, 1024, 64, 1))
    err = profile(write(tmp_path, gg.gguf_bytes(_image_kv(3, "image-linear-q4_k-v1", 14), tensors)))
    assert "incompatible SAM 3 tensor precision: vit.blocks.0.attn.qkv.weight is q8_0" in err


def test_schema1_rejects_image_hybrid_profile(tmp_path):
    """tests/api/test_contracts.cpp:445-458: a video-only hybrid profile on
    an image container is rejected for its storage profile."""
    data = gg.probe_fixture(extra_kv=[("general.file_type", gg.U32, 1),
                                      ("sam.storage_profile", gg.STRING, "visual-tracker-f32-v1")])
    err = profile(write(tmp_path, data))
    assert "storage profile" in err


def test_schema4_modules(tmp_path, oracle):
    text = ("text.blocks.0.mlp.fc1.weight", (1024, 64), gg.GGML_Q8_0, _q(oracle, gg.GGML_Q8_0, 1024, 64, 5))
    vit = ("vit.blocks.0.attn.qkv.weight", (1024, 64), gg.GGML_Q8_0, _q(oracle, gg.GGML_Q8_0, 1024, 64, 6))
    f32_vit = ("vit.blocks.0.attn.qkv.weight", (1024, 64), gg.GGML_F32, bytes(1024 * 64 * 4))

    def run(modules, tensors, name="image-modules-linear-q8_0-v1"):
        kv = _image_kv(4, name, 7, extra=[("sam.quantization.modules", gg.STRING, modules)])
        return profile(write(tmp_path, gg.gguf_bytes(kv, tensors)))

    assert run("vision,text", [text, vit]) == {"ok": True, "constrained": 2}
    assert run("text", [text, f32_vit]) == {"ok": True, "constrained": 2}
    assert "incompatible SAM 3 tensor precision" in run("text", [text, vit])
    assert "canonical CSV" in run("text,vision", [text, vit])
    assert "canonical module list" in run("vision,text", [text, vit], "image-full-linear-q8_0-v1")


def test_payload_with_nonfinite_scale_rejected(tmp_path, oracle):
    tensors = _image_tensors(oracle)
    name, ne, t, payload = tensors[3]                     # Q8_0 lin2: fp16 scale at byte 0 of each block
    bad = bytearray(payload)
    bad[34 * 5:34 * 5 + 2] = np.array([np.inf], np.float16).tobytes()
    tensors[3] = (name, ne, t, bytes(bad))
    err = profile(write(tmp_path, gg.gguf_bytes(_image_kv(3, "image-linear-q4_k-v1", 14), tensors)))
    assert isinstance(err, str) and "vit.blocks.0.mlp.lin2.weight" in err, err


# ---------------------------------------------------------------------------
# Upload and products on the device
# ---------------------------------------------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("kq,file_type,profile_name", [(gg.GGML_Q4_K, 14, "image-linear-q4_k-v1"),
                                                       (gg.GGML_Q6_K, 18, "image-linear-q6_k-v1")])
def test_gguf_upload_and_products(tmp_path, oracle, kq, file_type, profile_name):
    """A schema-3 checkpoint with the ViT block's four linears at their real
    shapes (qkv 1024 -> 3072, proj 1024 -> 1024, lin1 1024 -> 4736 in the
    profile's K type, lin2 4736 -> 1024 in Q8_0) and a text fc1: loaded
    through DeviceWeights, the device bytes equal the file's and every
    product at M = 300 and M = 32 is within row relative L2 1e-3 of the
    oracle's native product."""
    tensors = [("vit.blocks.0.attn.qkv.weight", (1024, 3072), kq, _q(oracle, kq, 1024, 3072, 1)),
               ("vit.blocks.0.attn.proj.weight", (1024, 1024), kq, _q(oracle, kq, 1024, 1024, 2)),
               ("vit.blocks.0.mlp.lin1.weight", (1024, 4736), kq, _q(oracle, kq, 1024, 4736, 3)),
               ("vit.blocks.0.mlp.lin2.weight", (4736, 1024), gg.GGML_Q8_0,
                _q(oracle, gg.GGML_Q8_0, 4736, 1024, 4)),
               ("text.blocks.0.mlp.fc1.weight", (1024, 4096), kq, _q(oracle, kq, 1024, 4096, 5)),
               ("vit.blocks.0.norm1.weight", (1024,), gg.GGML_F32, np.ones(1024, np.float32).tobytes())]
    path = write(tmp_path, gg.gguf_bytes(_image_kv(3, profile_name, file_type), tensors))
    for m in (300, 32):
        print(f"gguf upload {profile_name} M={m}", flush=True)
        out = tool("gpu", path, m, timeout=120)
        assert out.returncode == 0, out.stdout + out.stderr
        res = json.loads(out.stdout)
        assert res["loaded"] == 5
        for p in res["products"]:
            print(p, flush=True)
            assert p["bytes_equal"], p
            assert p["max_row_rel_l2"] <= 1e-3, p


# ---------------------------------------------------------------------------
# The image encoder from a converted checkpoint
# ---------------------------------------------------------------------------

def _encoder_checkpoint(oracle, tmp_path):
    """A SAM 3-structured checkpoint at reduced size (168 px, patch 14 ->
    12 x 12 tokens, width 256, 4 heads, 2 blocks with block 1 global, MLP
    512, window 6, neck 64 -> 32): the reference's tensor names and ggml
    shapes (src/models/sam3/tensors.hpp:96-163) and sam3.vision.* metadata.
    Returns the path, the image, and the host weights for the oracle."""
    from tests.vit_fixtures import axial_rope_table, block_weights, neck_weights
    img, patch, E, heads, mlp, ws, D, mid, blocks, glob = 168, 14, 256, 4, 512, 6, 32, 64, 2, [1]
    G, pg = img // patch, img // patch // 3
    rng = np.random.default_rng(21)
    f32 = lambda a: np.ascontiguousarray(a, np.float32)
    kernel = f32(rng.standard_normal((E, 3, patch, patch)) * 0.02)
    pos = f32(rng.standard_normal((pg, pg, E)) * 0.1)
    lw, lb = f32(1 + 0.1 * rng.standard_normal(E)), f32(0.05 * rng.standard_normal(E))
    T = [("vit.patch_embed.proj.weight", (patch, patch, 3, E), gg.GGML_F32, kernel.tobytes()),
         ("vit.pos_embed", (E, pg, pg), gg.GGML_F32, pos.tobytes()),
         ("vit.ln_pre.weight", (E,), gg.GGML_F32, lw.tobytes()), ("vit.ln_pre.bias", (E,), gg.GGML_F32, lb.tobytes())]
    bw = []
    for i in range(blocks):
        g = i in glob
        w = block_weights(oracle, E, mlp, heads, G * G if g else ws * ws, G if g else ws, 30 + i,
                          {"qkv": oracle.Q4_K, "proj": oracle.Q4_K, "fc1": oracle.Q4_K, "fc2": oracle.Q8_0})
        bw.append(w)
        p = f"vit.blocks.{i}"
        for n, k, nn in (("attn.qkv", E, 3 * E), ("attn.proj", E, E), ("mlp.lin1", E, mlp), ("mlp.lin2", mlp, E)):
            key = {"attn.qkv": "qkv", "attn.proj": "proj", "mlp.lin1": "fc1", "mlp.lin2": "fc2"}[n]
            gt = {oracle.Q4_K: gg.GGML_Q4_K, oracle.Q8_0: gg.GGML_Q8_0}[w[key + "_type"]]
            T.append((f"{p}.{n}.weight", (k, nn), gt, w[key + "_w"].tobytes()))
            T.append((f"{p}.{n}.bias", (nn,), gg.GGML_F32, f32(w[key + "_b"]).tobytes()))
        for n in ("norm1", "norm2"):
            T.append((f"{p}.{n}.weight", (E,), gg.GGML_F32, f32(w[n + "_w"]).tobytes()))
            T.append((f"{p}.{n}.bias", (E,), gg.GGML_F32, f32(w[n + "_b"]).tobytes()))
        T.append((f"{p}.attn.freqs_cis", (2, 32, w["freqs"].shape[0]), gg.GGML_F32, f32(w["freqs"]).tobytes()))
    nw = neck_weights(rng, E, mid, D, scale=1.0 / np.sqrt(E))
    names = {"s0_dc1": ("0.dconv_2x2_0", (2, 2, mid, E)), "s0_dc2": ("0.dconv_2x2_1", (2, 2, D, mid)),
             "s0_c1": ("0.conv_1x1", (1, 1, D, D)), "s0_c3": ("0.conv_3x3", (3, 3, D, D)),
             "s1_dc": ("1.dconv_2x2", (2, 2, mid, E)), "s1_c1": ("1.conv_1x1", (1, 1, mid, D)),
             "s1_c3": ("1.conv_3x3", (3, 3, D, D)), "s2_c1": ("2.conv_1x1", (1, 1, E, D)),
             "s2_c3": ("2.conv_3x3", (3, 3, D, D)), "s3_c1": ("3.conv_1x1", (1, 1, E, D)),
             "s3_c3": ("3.conv_3x3", (3, 3, D, D))}
    for key, (n, shape) in names.items():
        T.append((f"neck.det.{n}.weight", shape, gg.GGML_F32, f32(nw[key + "_w"]).tobytes()))
        T.append((f"neck.det.{n}.bias", (shape[2] if "dconv" in n else shape[3],), gg.GGML_F32,
                  f32(nw[key + "_b"]).tobytes()))
    kv = [("general.architecture", gg.STRING, "sam3"), ("sam3.vision.image_size", gg.U32, img),
          ("sam3.vision.patch_size", gg.U32, patch), ("sam3.vision.embedding_length", gg.U32, E),
          ("sam3.vision.block_count", gg.U32, blocks), ("sam3.vision.attention.head_count", gg.U32, heads),
          ("sam3.vision.feed_forward_length", gg.U32, mlp), ("sam3.vision.window_size", gg.U32, ws),
          ("sam3.vision.global_attention_blocks", gg.ARRAY, (gg.U32, glob)),
          ("sam3.neck.embedding_length", gg.U32, D)]
    path = write(tmp_path, gg.gguf_bytes(kv, T))
    image = f32(np.random.default_rng(22).standard_normal((3, img, img)))
    host = {"img": img, "patch": patch, "E": E, "heads": heads, "mlp": mlp, "ws": ws, "D": D, "mid": mid,
            "glob": glob, "G": G, "pg": pg, "kernel": kernel, "pos": pos, "lw": lw, "lb": lb, "blocks": bw,
            "neck": nw}
    return path, image, host


def _row_rel(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    return np.linalg.norm(got - ref, axis=1) / np.maximum(np.linalg.norm(ref, axis=1), 1e-30)


@pytest.mark.gpu
@pytest.mark.parametrize("columns", ["f32", "f16"])
def test_image_encoder_from_checkpoint(tmp_path, oracle, columns):
    """The image encoder wired from a converted checkpoint's tensors
    (sam.cpp_amd/host/vision_encoder.hpp): its ViT output against the
    oracle's prefix and blocks on the same weights (native Q8 linears:
    median 2e-3, max 6e-3 per row over the two blocks, inside the one-block
    bar of tests/test_gpu_vit.py; measured 6e-4 / 9e-4), and its neck levels
    against the
    oracle's neck applied to that same ViT output (F32 columns 5e-6; F16
    columns median 3e-5, max 1e-3, as tests/test_gpu_neck.py)."""
    path, image, h = _encoder_checkpoint(oracle, tmp_path)
    image_path = str(tmp_path / "image.f32")
    image.tofile(image_path)
    prefix = str(tmp_path / "out")
    print(f"image encoder from checkpoint ({columns} columns)", flush=True)
    out = tool("encode", path, image_path, prefix, columns, timeout=120)
    assert out.returncode == 0, out.stdout + out.stderr
    res = json.loads(out.stdout)
    G, E, D = h["G"], h["E"], h["D"]
    assert res["grid"] == G and res["dim"] == D and res["levels"] == [4 * G, 2 * G, G, G // 2]
    x = np.fromfile(prefix + ".features.f32", np.float32).reshape(G * G, E)
    ref = oracle.vit_prefix(image, h["patch"], h["kernel"], h["pos"], h["pg"], h["lw"], h["lb"], E)
    for i, w in enumerate(h["blocks"]):
        ref = oracle.vit_block(w, ref, G, G, E, h["heads"], h["mlp"], 0 if i in h["glob"] else h["ws"])
    rel = _row_rel(x, ref)
    print(f"  ViT output: median {np.median(rel):.3g} max {rel.max():.3g}", flush=True)
    assert np.median(rel) < 2e-3 and rel.max() < 6e-3
    levels = oracle.neck(h["neck"], x, G, E, h["mid"], D, columns_f16=columns == "f16")
    for i, lref in enumerate(levels):
        got = np.fromfile(prefix + f".level{i}.f32", np.float32).reshape(-1, D)
        rel = _row_rel(got, lref)
        print(f"  level {i}: median {np.median(rel):.3g} max {rel.max():.3g}", flush=True)
        if columns == "f32":
            assert rel.max() < 5e-6, i
        else:
            assert np.median(rel) < (3e-5 if i < 2 else 2e-6) and rel.max() < 1e-3, i


def test_image_encoder_parameters_rejected(tmp_path, oracle):
    """VisionParameters checks the metadata before any device work: a
    non-64 head width is refused with the reference's message family."""
    path, image, h = _encoder_checkpoint(oracle, tmp_path)
    data = open(path, "rb").read()
    key = b"sam3.vision.attention.head_count"
    at = data.index(key) + len(key) + 4        # u32 value type, then the value
    bad = data[:at] + struct.pack("<I", 8) + data[at + 4:]
    p2 = tmp_path / "bad.gguf"
    p2.write_bytes(bad)
    out = tool("encode", str(p2), str(tmp_path / "none.f32"), str(tmp_path / "o"))
    assert out.returncode == 3 and "unsupported SAM 3 image encoder parameters" in out.stdout, out.stdout


SAM3_IMAGE_PARAMETERS = [("sam3.vision.image_size", 1008), ("sam3.vision.patch_size", 14),
                         ("sam3.vision.embedding_length", 1024), ("sam3.vision.block_count", 32),
                         ("sam3.vision.attention.head_count", 16), ("sam3.vision.feed_forward_length", 4736),
                         ("sam3.vision.window_size", 24), ("sam3.text.embedding_length", 1024),
                         ("sam3.text.attention.head_count", 16), ("sam3.text.block_count", 24),
                         ("sam3.text.context_length", 32), ("sam3.text.vocab_size", 49408),
                         ("sam3.text.output_length", 256), ("sam3.neck.embedding_length", 256),
                         ("sam3.fusion.block_count", 6), ("sam3.fusion.attention.head_count", 8),
                         ("sam3.fusion.feed_forward_length", 2048), ("sam3.decoder.block_count", 6),
                         ("sam3.decoder.attention.head_count", 8), ("sam3.decoder.feed_forward_length", 2048),
                         ("sam3.decoder.query_count", 200), ("sam3.geometry.block_count", 3)]


def _params_file(tmp_path, name, values, globals_=(7, 15, 23, 31), gtype=gg.U32):
    kv = [("general.alignment", gg.U32, 32)] + [(k, gg.U32, v) for k, v in values]
    kv.append(("sam3.vision.global_attention_blocks", gg.ARRAY, (gtype, list(globals_))))
    path = tmp_path / name
    path.write_bytes(gg.gguf_bytes(kv, [("vit.ln_pre.bias", (4,), gg.GGML_F32, np.zeros(4, np.float32).tobytes())]))
    return str(path)


def test_vision_parameters_strict_by_default(tmp_path):
    """The strict read mirrors the reference loader (src/models/sam3/
    weights.hpp:591-600): the 22 fixed SAM 3 image parameters and the global
    blocks {7, 15, 23, 31} as a U32 array; each deviation is refused with the
    reference's message, and the relaxed read accepts the same files."""
    good = _params_file(tmp_path, "sam3.gguf", SAM3_IMAGE_PARAMETERS)
    out = tool("vision-params", good)
    assert out.returncode == 0, out.stdout
    p = json.loads(out.stdout)
    assert (p["image_size"], p["embed"], p["blocks"], p["mlp"], p["window"], p["global_blocks"]) == \
        (1008, 1024, 32, 4736, 24, [7, 15, 23, 31])
    for i, (key, value) in enumerate(SAM3_IMAGE_PARAMETERS):
        if i % 3:
            continue   # a spread of keys across the vision, text, fusion and decoder groups
        values = list(SAM3_IMAGE_PARAMETERS)
        values[i] = (key, value * 2)
        path = _params_file(tmp_path, f"bad{i}.gguf", values)
        out = tool("vision-params", path)
        assert out.returncode == 3 and f"unsupported SAM 3 image parameter: {key}" in out.stdout, out.stdout
    for gl in ((7, 15, 23), (7, 15, 23, 30), (15, 7, 23, 31)):
        path = _params_file(tmp_path, "glob.gguf", SAM3_IMAGE_PARAMETERS, gl)
        out = tool("vision-params", path)
        assert out.returncode == 3 and "global attention block order" in out.stdout, (gl, out.stdout)
        relaxed = tool("vision-params", path, "relaxed")
        assert relaxed.returncode == (0 if gl[0] < gl[1] else 3), relaxed.stdout
    path = _params_file(tmp_path, "i32.gguf", SAM3_IMAGE_PARAMETERS, gtype=gg.I32)
    assert tool("vision-params", path).returncode == 3


def test_vision_parameters_reduced_checkpoint_needs_relaxed(tmp_path, oracle):
    """The reduced encoder checkpoint (168 px, 2 blocks) is not a SAM 3 file:
    strictly it is refused, relaxed it reads with its own structure."""
    path, _, _ = _encoder_checkpoint(oracle, tmp_path)
    out = tool("vision-params", path)
    assert out.returncode == 3 and "unsupported SAM 3 image parameter" in out.stdout, out.stdout
    out = tool("vision-params", path, "relaxed")
    assert out.returncode == 0, out.stdout
    p = json.loads(out.stdout)
    assert (p["image_size"], p["blocks"], p["global_blocks"]) == (168, 2, [1])
