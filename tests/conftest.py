import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu)")


@pytest.fixture(scope="session")
def orc():
    """The C restatement of the reference CPU quant path (the checker)."""
    import oracle
    return oracle.oracle()


@pytest.fixture(scope="session")
def golden():
    def load(name):
        return np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)
    return load


@pytest.fixture(scope="session")
def dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def nq():
    from nanoinfer_amd import quant
    return quant


# NQ_TEST_TIMES=<path>: append "<start_ns> <end_ns> <test id>" per test (CLOCK_MONOTONIC
# and CLOCK_BOOTTIME both, as "mono"/"boot" lines), so that a kernel trace of the
# same run (rocprofv3 --kernel-trace) can name the test that launched each kernel.
_TIMES = os.environ.get("NQ_TEST_TIMES")
if _TIMES:
    import time

    @pytest.hookimpl(hookwrapper=True)
    def pytest_runtest_call(item):
        t0m, t0b = time.clock_gettime_ns(time.CLOCK_MONOTONIC), time.clock_gettime_ns(time.CLOCK_BOOTTIME)
        yield
        try:
            import torch
            if torch.cuda.is_initialized():
                torch.cuda.synchronize()
        except Exception:
            pass
        t1m, t1b = time.clock_gettime_ns(time.CLOCK_MONOTONIC), time.clock_gettime_ns(time.CLOCK_BOOTTIME)
        with open(_TIMES, "a") as f:
            f.write(f"mono {t0m} {t1m} {item.nodeid}\nboot {t0b} {t1b} {item.nodeid}\n")
