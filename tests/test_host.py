"""The C++17 host layer (sam.cpp_amd/host/sam_hip.hpp) through its C++ test
program tests/host/test_host (built by __graft_entry__.build() or
`make -C tests/host`)."""

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BINARY = os.path.join(ROOT, "tests", "host", "_build", "test_host")


def run(mode):
    if not os.path.exists(BINARY):
        pytest.fail(f"{BINARY} is not built: run make -C tests/host")
    out = subprocess.run([BINARY, mode], capture_output=True, text=True, timeout=300)
    print(out.stdout, out.stderr, flush=True)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "0 failed" in out.stdout


def test_host_layer_cpu():
    """Options and CLI validation, format policy, status mapping, graph
    prepare errors and the no-device error."""
    run("--cpu")


@pytest.mark.gpu
def test_host_layer_gpu():
    """HipBackend + HipGraphExecution on device 0 against the oracle."""
    run("--gpu")
