import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a visible HIP device (MI355X / gfx950)")


def _load(name, path):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o
    o.lib()
    return o


@pytest.fixture(scope="session")
def samhip():
    return _load("samhip", os.path.join(ROOT, "sam.cpp_amd", "samhip.py"))


@pytest.fixture(scope="session")
def gpu_ctx(samhip):
    ctx = samhip.Context(0, samhip.COMPUTE_Q8_NATIVE, samhip.ROUND_X86)
    yield ctx
    ctx.close()
