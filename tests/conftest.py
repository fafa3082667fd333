import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (ROOT, os.path.join(ROOT, "oracle")):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: requires an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """Fail (not skip) when a gpu-marked test runs without a usable device."""
    import ctypes

    from maxsim_amd import _native

    lib = _native.load()  # raises NativeLibraryMissing when the .so is absent
    hip = ctypes.CDLL("libamdhip64.so")
    count = ctypes.c_int(0)
    status = hip.hipGetDeviceCount(ctypes.byref(count))
    assert status == 0 and count.value > 0, "gpu-marked test needs a visible HIP device"
    return lib


@pytest.fixture(scope="session")
def oracle():
    import oracle as orc

    orc.build()
    return orc


def ragged_fixture(num_docs, seed, lo=1, hi=8, empty=2, dim=128):
    """Ragged docs with lengths U{lo..hi} and one empty doc (tests/test_int4_int8q.py:29-35)."""
    rng = np.random.default_rng(seed)
    lengths = rng.integers(lo, hi + 1, size=num_docs)
    if empty is not None:
        lengths[min(empty, num_docs - 1)] = 0
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    docs = rng.standard_normal((int(offsets[-1]), dim)).astype(np.float32)
    return docs, offsets
