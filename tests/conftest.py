import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (HIP device)")


def read_bf16(name):
    return np.fromfile(os.path.join(GOLDEN, "dit_fixture", name), dtype="<u2")


def read_f32(name, sub="dit_fixture"):
    return np.fromfile(os.path.join(GOLDEN, sub, name), dtype="<f4")


def golden_json(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.sqrt(np.sum(b * b))
    return float(np.sqrt(np.sum((a - b) ** 2)) / (den if den > 0 else 1.0))


def cosine(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-300))


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o
    o.lib()
    return o


def load_qdit():
    """The product's ctypes binding (qwen-metal_amd/qdit.py)."""
    import importlib.util
    path = os.path.join(ROOT, "qwen-metal_amd", "qdit.py")
    spec = importlib.util.spec_from_file_location("qdit", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def qd():
    return load_qdit()


@pytest.fixture(scope="session")
def gpu(qd):
    g = qd.Gpu()
    yield g
    g.close()


def ulp_diff(a, b):
    """Distance in bf16 units between two bf16 bit arrays (sign-aware)."""
    def key(x):
        x = np.asarray(x, np.int32)
        return np.where(x & 0x8000, 0x8000 - (x & 0x7FFF), 0x8000 + (x & 0x7FFF))
    return np.abs(key(a) - key(b))


def bf16_neighbours(v):
    """The two bf16 values next to each element of v (bit patterns), by
    magnitude one step down and one step up; around zero, +-the smallest
    subnormal."""
    v = v.astype(np.uint16)
    mag = v & np.uint16(0x7FFF)
    zero = mag == 0
    down = np.where(zero, np.uint16(0x0001), v - np.uint16(1)).astype(np.uint16)
    up = np.where(zero, np.uint16(0x8001), v + np.uint16(1)).astype(np.uint16)
    return down, up
