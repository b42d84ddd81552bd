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


def err_report(gpu: np.ndarray, ref: np.ndarray) -> dict:
    """The floored relative error (the bar) beside the unfloored one, and where the unfloored
    one passes 1e-3: how many outputs, and the largest |ref| among them as a fraction of the
    output rms (near-zero outputs from cancellation, whose absolute error is still ~1e-7 of
    the output scale)."""
    g = np.asarray(gpu, np.float64).ravel()
    r = np.asarray(ref, np.float64).ravel()
    rms = float(np.sqrt(np.mean(r * r))) if r.size else 0.0
    ad = np.abs(g - r)
    raw = ad / np.maximum(np.abs(r), 1e-30)
    over = raw > 1e-3
    return {"floored": rel_err(g, r), "unfloored": float(raw.max()) if r.size else 0.0,
            "n_over_1e-3": int(over.sum()), "n": int(r.size),
            "max_abs_ref_over_rms": float(np.abs(r[over]).max() / rms) if over.any() and rms else 0.0,
            "max_abs_err_over_rms": float(ad.max() / rms) if r.size and rms else 0.0}


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.lib()
    return oracle
