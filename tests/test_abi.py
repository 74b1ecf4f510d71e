"""The C ABI library loads, exports every entry point include/samhip.h
declares, and its host-side checks behave as the reference's (no device
needed: nothing here launches a kernel)."""

import ctypes
import re
import subprocess

import numpy as np
import pytest


def _declared(header):
    text = open(header).read()
    return sorted(set(re.findall(r"^\s*(?:int|void|size_t)\s+(samhip_\w+)\s*\(", text, re.M)))


def test_header_symbols_exported(samhip):
    names = _declared(samhip.HEADER)
    assert len(names) >= 18
    out = subprocess.run(["nm", "-D", "--defined-only", samhip.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT\s+(samhip_\w+)", out))
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    # the binding declares a signature for every one of them
    assert sorted(samhip.SIGNATURES) == names


def test_abi_version(samhip):
    assert samhip.lib().samhip_abi_version() == samhip.ABI_VERSION == 1


def _descs(samhip, qtype=8, k=256, n=64, m=9, **over):
    base = 0x10000
    w = samhip.tensor(qtype, k, n, base)
    x = samhip.tensor(samhip.F32, k, m, base * 4)
    y = samhip.tensor(samhip.F32, n, m, base * 8)
    for key, val in over.items():
        obj, field = key.split("_", 1)
        t = {"w": w, "x": x, "y": y}[obj]
        if field.startswith("ne"):
            t.ne[int(field[2])] = val
        elif field.startswith("nb"):
            t.nb[int(field[2])] = val
        else:
            setattr(t, field, val)
    return w, x, y


def _supports(samhip, w, x, y):
    return samhip.lib().samhip_supports_mul_mat(ctypes.byref(w), ctypes.byref(x), ctypes.byref(y))


@pytest.mark.parametrize("qtype", [8, 12, 13, 14])
def test_supports_valid_operands(samhip, qtype):
    assert _supports(samhip, *_descs(samhip, qtype)) == 1
    # a row-offset view and a strided activation are supported
    w, x, y = _descs(samhip, qtype, x_nb1=2 * 4 * 256)
    w.data = 0x10000 + 3 * samhip.row_bytes(qtype, 256)
    assert _supports(samhip, w, x, y) == 1


@pytest.mark.parametrize("over", [
    {"w_type": 2},                 # Q4_0 is not on the path
    {"w_type": 0},                 # F32 weights are not a quantized matmul
    {"x_type": 1},                 # F16 activation (test_cpu_quantized_matmul.cpp:90-95)
    {"y_type": 1},
    {"x_ne0": 512},                # width mismatch
    {"y_ne0": 65},
    {"w_nb0": 32},                 # not row-contiguous packed blocks
    {"x_nb0": 8},
    {"x_nb1": 1000},               # rows overlap
    {"w_ne2": 2},
    {"w_data": 0},
    {"x_data": 0x40002},           # misaligned F32
])
def test_supports_rejects(samhip, over):
    assert _supports(samhip, *_descs(samhip, 8, **over)) == 0


def test_supports_rejects_non_block_width(samhip):
    assert _supports(samhip, *_descs(samhip, 12, k=4736)) == 0   # K-quants need K % 256 == 0
    assert _supports(samhip, *_descs(samhip, 8, k=4736)) == 1    # Q8_0 fallback width


def test_payload_validation(samhip, oracle):
    # tests/runtime/ggml/test_quantization.cpp:70-104
    for qtype in (8, 14, 13, 12):
        width = samhip.BLOCK_ELEMS[qtype]
        src = ((np.arange(width, dtype=np.float32) - width // 2) / width)[None, :]
        block = oracle.quantize(qtype, src).reshape(-1)
        samhip.validate_quantized_payload(qtype, width, 1, block)
        inf = np.array([0x7c00], np.uint16).view(np.uint8)
        if qtype == 14:   # Q6_K keeps d at the end: a half-infinity pattern in its prefix is valid
            b = block.copy()
            b[0:2] = inf
            samhip.validate_quantized_payload(qtype, width, 1, b)
        off = block.size - 2 if qtype == 14 else 0
        b = block.copy()
        b[off:off + 2] = inf
        with pytest.raises(samhip.InvalidArgument, match="scale"):
            samhip.validate_quantized_payload(qtype, width, 1, b)
        if qtype in (12, 13):
            b = block.copy()
            b[2:4] = inf
            with pytest.raises(samhip.InvalidArgument, match="minimum"):
                samhip.validate_quantized_payload(qtype, width, 1, b)
        with pytest.raises(samhip.InvalidArgument, match="size"):
            samhip.validate_quantized_payload(qtype, width, 2, block)


def test_context_without_device_fails_closed(samhip):
    if samhip.device_count() > 0:
        pytest.skip("a HIP device is visible")
    with pytest.raises(samhip.SamhipError, match="no HIP device"):
        samhip.Context(0)
    opts = samhip.Options(99, 0, 0, 0)
    h = ctypes.c_void_p()
    assert samhip.lib().samhip_context_create(ctypes.byref(opts), ctypes.byref(h)) == samhip.ERR_INVALID_ARGUMENT
    assert "ABI version" in samhip.last_error()


def test_invalid_options_rejected_before_device(samhip):
    for opts in (samhip.Options(1, 0, 7, 0), samhip.Options(1, 0, 0, 5)):
        h = ctypes.c_void_p()
        assert samhip.lib().samhip_context_create(ctypes.byref(opts), ctypes.byref(h)) == samhip.ERR_INVALID_ARGUMENT
