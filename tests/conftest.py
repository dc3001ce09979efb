"""Shared test setup: marker registration, import paths, the GPU fixture."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")


@pytest.fixture(scope="session")
def device():
    """Opens device 0 through the arch guard; the HIP library must be built."""
    import kanjoos_amd as K

    caps = K.open_device(0)
    assert caps.gcn_arch.decode() == "gfx950"
    yield caps


def rel_rmse(got, want):
    """The reference's metric (tests/host_oracle.h:143-171): sqrt(sum d^2 / sum w^2)
    over the elements whose expected value is nonzero."""
    import numpy as np

    got = np.asarray(got, dtype=np.float64).ravel()
    want = np.asarray(want, dtype=np.float64).ravel()
    nz = want != 0
    den = float(np.sum(want[nz] ** 2))
    return float(np.sqrt(np.sum((got[nz] - want[nz]) ** 2) / den)) if den > 0 else 0.0


def progress(msg):
    """A progress line for long GPU tests: printed, and appended to
    gpurun_out/test_progress.log so a long test visibly makes progress even
    while pytest captures its output."""
    print(msg, flush=True)
    try:
        d = os.path.join(ROOT, "gpurun_out")
        os.makedirs(d, exist_ok=True)
        with open(os.path.join(d, "test_progress.log"), "a") as f:
            f.write(msg + "\n")
    except OSError:
        pass
