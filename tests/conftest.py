import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI library)")
    config.addinivalue_line("markers", "slow: long-running CPU check")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle
    oracle.build()
    return oracle


@pytest.fixture(scope="session")
def golden():
    import numpy as np
    path = os.path.join(ROOT, "tests", "golden", "ref_moe_mul1_vectors.npz")
    return dict(np.load(path))


@pytest.fixture
def kernel_policy():
    """set(key, value) selects a kernel path (include/exl3_amd.h EXL3_AMD_POLICY_*) for the rest of
    the test; every key set is restored to its previous value afterwards."""
    from ampstein_amd import _lib
    saved = []

    def set_(key, value):
        saved.append((key, _lib.check(_lib.lib().exl3_amd_get_policy(key))))
        _lib.check(_lib.lib().exl3_amd_set_policy(key, value))

    yield set_
    for key, prev in reversed(saved):
        _lib.lib().exl3_amd_set_policy(key, prev)
