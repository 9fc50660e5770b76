import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "splatting-rs_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP library)")
    config.addinivalue_line("markers", "slow: full-size configuration (seconds to minutes of CPU oracle time)")


@pytest.fixture(scope="session")
def ctx():
    """One library context on cuda:0 for the whole GPU test session."""
    import splathip
    c = splathip.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="session")
def weights_dir(tmp_path_factory):
    return tmp_path_factory.mktemp("weights")


def report(name, **kw):
    """One line per case, flushed, so a failing GPU step names its case."""
    print(f"[case] {name} " + " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def rel_err(a, b, tau=0.01):
    """max |a-b| / (|b| + tau * max|b|): relative error floored at tau of the tensor's scale, so
    that entries near zero (raw logits) do not make the ratio ill-conditioned."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b) / (np.abs(b) + tau * np.max(np.abs(b)) + 1e-30)))


# Network outputs in the 16-bit dtypes against the fp32 oracle: (minimum cosine, maximum median
# relative depth error). f16 keeps 11 mantissa bits to bf16's 8: rounding errors 8x smaller, so
# 1 - cosine, quadratic in them, ~60x smaller.
H16 = {"bf16": (0.999, 1e-2), "f16": (0.9999, 2e-3)}


def cosine(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-300))
