import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "rwkv-theseus_amd"))  # `import theseus` (the drop-in package)
sys.path.insert(0, str(ROOT))                       # `import oracle` (test infrastructure)

import numpy as np
import pytest
import torch


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(autouse=True)
def small_threads():
    # Same per-test determinism as the reference suite (tests/conftest.py:7-10).
    torch.set_num_threads(1)
    torch.manual_seed(123)


def _np(x):
    if isinstance(x, torch.Tensor):
        return x.detach().double().cpu().numpy()
    return np.asarray(x, dtype=np.float64)


def rel_l2(x, ref):
    x, ref = _np(x), _np(ref)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(x - ref) / (den if den > 0 else 1.0))


def max_abs(x, ref):
    x, ref = _np(x), _np(ref)
    return float(np.max(np.abs(x - ref))) if np.size(ref) else 0.0
