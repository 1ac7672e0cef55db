import json
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def known_answers():
    with open(os.path.join(ROOT, "tests", "golden", "reference_known_answers.json")) as f:
        return json.load(f)


@pytest.fixture(scope="session")
def gpu():
    """Initialises device 0 through the C-ABI. GPU tests fail (not skip)
    when the library or the GPU is missing: they are only collected with
    -m gpu on a GPU box."""
    import torch

    from gorch_amd import hip

    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    hip.init(0)
    torch.cuda.set_device(0)
    return hip


def rel_err(got, ref):
    """max |got - ref| / max(RMS(ref), tiny) — the reference's
    |delta| <= tol * RMS(ref) metric (bf16_matmul_metal_test.go:20-48)."""
    import numpy as np

    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    rms = float(np.sqrt(np.mean(ref * ref))) if ref.size else 0.0
    return float(np.max(np.abs(got - ref))) / max(rms, 1e-30) if ref.size else 0.0
