import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("esm-cpp_amd", "oracle", ""):
    p = os.path.join(ROOT, sub) if sub else ROOT
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    from pyoracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from pyoracle import REF_LIB, RefLib
    if not os.path.exists(REF_LIB):
        pytest.skip("oracle/_ref/libesmref.so not built (needs /root/reference at build time)")
    return RefLib(threads=4)


@pytest.fixture(scope="session")
def dev():
    import esm_gfx950
    d = esm_gfx950.Device(0)
    yield d
    d.close()


def rng(seed):
    return np.random.default_rng(seed)


def cu_from_lengths(lengths):
    cu = np.zeros(len(lengths) + 1, np.int32)
    cu[1:] = np.cumsum(lengths)
    return cu
