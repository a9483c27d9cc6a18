"""Shared fixtures.

Markers:
  gpu -- needs an MI355X (HIP device) and the built libmoeq.so; compares the
         HIP path with the CPU oracle.  Everything else runs on the CPU.
"""

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: requires a HIP GPU (MI355X) and libmoeq.so")


@pytest.fixture(scope="session")
def device():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")
    from robustgemq_amd import _lib
    _lib.lib()  # loud failure if the native library is missing
    return torch.device("cuda:0")


def relative_error(actual, reference):
    """Frobenius-norm relative error in float64 (tests/conftest.py:152-157 of the reference)."""
    a = np.asarray(actual, dtype=np.float64)
    r = np.asarray(reference, dtype=np.float64)
    return float(np.linalg.norm(a - r) / max(np.linalg.norm(r), 1e-30))


def to_np(t):
    """torch tensor (any device / dtype) -> numpy (fp16 kept, bf16 -> fp32)."""
    import torch
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        t = t.float()
    return t.numpy()


@pytest.fixture(autouse=True)
def _free_gpu():
    yield
    try:
        import gc

        import torch
        if torch.cuda.is_available():
            gc.collect()
            torch.cuda.empty_cache()
    except Exception:
        pass
