import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")


@pytest.fixture(scope="session")
def quant_golden():
    import numpy as np
    return np.load(os.path.join(GOLDEN, "quant_golden.npz"))


@pytest.fixture(scope="session")
def cache_golden():
    import numpy as np
    return np.load(os.path.join(GOLDEN, "cache_golden.npz"))


@pytest.fixture(scope="session")
def axes_golden():
    import numpy as np
    return np.load(os.path.join(GOLDEN, "axes_golden.npz"))


@pytest.fixture(scope="session")
def hybrid_ties():
    import numpy as np
    return np.load(os.path.join(GOLDEN, "hybrid_ties.npz"))
