import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (ROOT, os.path.join(ROOT, "oracle")):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    import pyoracle
    return pyoracle.load_oracle()


@pytest.fixture(scope="session")
def ref():
    import pyoracle
    if not pyoracle.ref_available():
        pytest.skip("reference CPU library (oracle/_ref) is not built here")
    return pyoracle.load_ref()


@pytest.fixture(scope="session")
def gpu():
    """A context on cuda:0; fails loudly (no skip) when the library or the
    GPU is missing, since GPU tests are selected only on a machine with one."""
    import torch
    from adi_amd import hip
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    ctx = hip.Context(0)
    yield ctx
    ctx.synchronize()
    ctx.close()


def max_rel_error(got, want):
    """max_i |g_i - c_i| / max_i |c_i| over each output vector (last axis),
    the worst vector returned."""
    import numpy as np
    got = np.asarray(got, np.float64).reshape(-1, np.shape(want)[-1])
    want = np.asarray(want, np.float64).reshape(-1, np.shape(want)[-1])
    scale = np.maximum(np.abs(want).max(axis=1), 1e-30)
    return float((np.abs(got - want).max(axis=1) / scale).max())


def error_report(got, want):
    """The three output-error figures of the measurement contract, over the
    whole array: the max-normalised error (as max_rel_error), the normwise
    relative L2 error ||g - c|| / ||c||, and the largest elementwise relative
    error |g_i - c_i| / |c_i| over the elements with |c_i| >= 1% of max |c|."""
    import numpy as np
    g = np.asarray(got, np.float64).ravel()
    c = np.asarray(want, np.float64).ravel()
    scale = max(float(np.abs(c).max()), 1e-30)
    big = np.abs(c) >= 0.01 * scale
    return {
        "max_rel": float(np.abs(g - c).max() / scale),
        "l2_rel": float(np.linalg.norm(g - c) / max(float(np.linalg.norm(c)), 1e-30)),
        "elem_rel_1pct": float((np.abs(g - c)[big] / np.abs(c)[big]).max()) if big.any() else 0.0,
    }
