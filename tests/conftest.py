import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built libqmm.so")


def rel_err(gpu: np.ndarray, ref: np.ndarray, floor_frac: float = 0.05) -> float:
    """Max elementwise relative error with the denominator floored at
    floor_frac * rms(ref): the integer dot products are exact on both sides,
    only the fp32 combine order differs, so outputs that are near zero from
    cancellation are judged against the output scale instead of themselves."""
    gpu = np.asarray(gpu, np.float64)
    ref = np.asarray(ref, np.float64)
    rms = float(np.sqrt(np.mean(ref * ref))) if ref.size else 0.0
    den = np.maximum(np.abs(ref), floor_frac * rms + 1e-30)
    return float(np.max(np.abs(gpu - ref) / den)) if ref.size else 0.0


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.lib()
    return oracle
