"""Shared helpers of the GPU tests: a GPU-only fixture that fails loudly when
the HIP library is missing."""
import pytest

from qwen_pkg import pyqwen


@pytest.fixture(scope="session")
def gpu():
    return pyqwen.gpu_lib()


def rel_err(got, ref):
    """max |got-ref| / max |ref| : the normwise relative error used by the parity bars."""
    import numpy as np
    ref = np.asarray(ref, np.float64)
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))
