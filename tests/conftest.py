import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: runs HIP kernels on an MI355X (cuda:0)")


@pytest.fixture(scope="session", autouse=True)
def _torch_initialises_the_gpu_first(request):
    """torch ships its own HIP runtime next to the system one the library links;
    torch finds the GPU only if it initialises the device first.  When any GPU
    test is selected, let torch do so before any test creates a model."""
    if any(item.get_closest_marker("gpu") for item in request.session.items):
        import torch
        torch.cuda.is_available()
    yield


_WEIGHTS = {}


@pytest.fixture(scope="session")
def weights_for():
    """Cached synthetic weights per model config."""
    from edgebert_amd import synth

    def get(cfg):
        if cfg not in _WEIGHTS:
            _WEIGHTS[cfg] = synth.make_weights(cfg)
        return _WEIGHTS[cfg]
    return get


def cosine_rows(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    return (a * b).sum(1) / (np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1))
