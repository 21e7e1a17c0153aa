import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    # tests/sanitize_host.py runs the CPU tests against sanitized builds of the
    # oracle and of libdscq's host side; these variables name those builds.
    if os.environ.get("DSCQ_TEST_ORACLE_LIB"):
        from oracle import native
        native.LIB_PATH = os.environ["DSCQ_TEST_ORACLE_LIB"]
    if os.environ.get("DSCQ_TEST_LIBDSCQ"):
        from dscquant_amd import _lib
        _lib.LIB_PATH = os.environ["DSCQ_TEST_LIBDSCQ"]


@pytest.fixture(scope="session", autouse=True)
def _oracle_built():
    """The C oracle is test infrastructure: build it if it is missing."""
    from oracle import native
    if not os.path.exists(native.LIB_PATH):
        native.build()


def sweep_size(n: int, seed: int):
    """(case count, seed) of a seeded random sweep.  DSCQ_SWEEP_SEED (added to
    every sweep's own seed) and DSCQ_SWEEP_SCALE (multiplying its case count)
    draw other or more cases; unset, every sweep keeps its committed cases."""
    shift = int(os.environ.get("DSCQ_SWEEP_SEED", "0"))
    scale = float(os.environ.get("DSCQ_SWEEP_SCALE", "1"))
    return max(1, int(round(n * scale))), seed + shift


def activations(M: int, K: int, seed: int = 0, outlier_frac: float = 0.01,
                outlier_scale: float = 50.0, dtype=np.float16) -> np.ndarray:
    """X ~ N(0,1) [M, K] with ceil(1%) of channels (seeded choice) scaled x50."""
    import torch
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    n_out = int(np.ceil(outlier_frac * K))
    if n_out:
        idx = torch.randperm(K, generator=torch.Generator().manual_seed(seed + 2))[:n_out]
        x[:, idx] *= outlier_scale
    return x.numpy().astype(dtype)


def weights(N: int, K: int, seed: int = 1, std: float = 0.02, dtype=np.float16) -> np.ndarray:
    """W ~ N(0, 0.02) [N, K]."""
    import torch
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(N, K, generator=g) * std).numpy().astype(dtype)


@pytest.fixture
def gpu():
    """cuda:0 after checking it is a gfx950 device with libdscq loaded."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    import dscquant_amd
    dscquant_amd._lib.require_gfx950(torch.device("cuda:0"))
    return torch.device("cuda:0")
