import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

# Parity bar stated for this path: rel-L2 <= 5e-3, cosine >= 0.9999.
REL_L2_TOL = 5e-3
COS_TOL = 0.9999


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) HIP device")


@pytest.fixture(scope="session")
def clib():
    import oracle
    return oracle.oracle_lib()


@pytest.fixture(scope="session")
def reflib():
    import oracle
    lib = oracle.reference_lib()
    if lib is None:
        pytest.skip("oracle/_ref/libmxfp4_ref.so not built (the reference source is only present "
                    "in the build container)")
    return lib


@pytest.fixture
def rng():
    return np.random.default_rng(1234)


def assert_close(got, want, label, rel=REL_L2_TOL, cos=COS_TOL):
    import oracle
    r, c = oracle.rel_l2(got, want), oracle.cosine(got, want)
    print(f"{label}: rel-L2 {r:.3e} cosine {c:.8f}")
    assert np.all(np.isfinite(np.asarray(got))), f"{label}: non-finite values"
    assert r <= rel, f"{label}: rel-L2 {r:.3e} > {rel:.1e}"
    assert c >= cos, f"{label}: cosine {c:.8f} < {cos}"
    return r, c
