import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X)")


@pytest.fixture(scope="session")
def orc():
    import oracle

    if not os.path.exists(oracle.ORACLE_SO):
        oracle.build()
    return oracle.oracle()


@pytest.fixture(scope="session")
def ref():
    import oracle

    r = oracle.reference()
    if r is None:
        pytest.skip("oracle/_ref (the compiled reference tmsample.h) is not built here")
    return r


@pytest.fixture(scope="session")
def golden():
    import numpy as np

    return np.load(os.path.join(ROOT, "tests", "golden", "sample_golden.npz"))


@pytest.fixture(scope="session", params=["auto", "general"])
def sampler(request):
    """The sampler twice: "auto" takes the top-k kernel for batches whose
    rows are all greedy or top-k <= 128; "general" always takes the general
    kernel, so every parity test covers both."""
    import torch

    from tensormark_amd import Sampler

    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    s = Sampler(max_batch=1024, max_vocab=262144, kernel=request.param)
    yield s
    s.close()
