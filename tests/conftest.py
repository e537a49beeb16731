"""Test configuration. `gpu` tests need an MI355X (gfx950) and the built HIP library; the rest run
on any CPU with the oracle built (make -C oracle)."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def reference():
    """The reference's own kernels (oracle/_ref), where they were built."""
    from oracle import Reference
    try:
        return Reference()
    except FileNotFoundError:
        pytest.skip("oracle/_ref not built (needs /root/reference at build time)")


@pytest.fixture(scope="session")
def backend():
    from fastgguf_amd.backend import Backend
    b = Backend(0)
    yield b
    b.close()


def golden(name):
    import numpy as np
    return np.load(os.path.join(ROOT, "tests", "golden", name), allow_pickle=False)


def rel_err(y, ref):
    """max |y - ref| / max |ref| over one output vector (the selftest metric, fastgguf.c:5723-5733)"""
    import numpy as np
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.abs(y - ref).max() / (np.abs(ref).max() + 1e-30))


def bits_equal_or_nan(a, b):
    """bits_equal, with any NaN matching any NaN: the CPU's fma(0, inf) gives the x86 default NaN
    (sign set), the GPU's the positive one."""
    import numpy as np
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    if a.shape != b.shape:
        return False
    na, nb = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32)))


def bits_equal(a, b):
    import numpy as np
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))
