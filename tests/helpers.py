"""Shared test helpers: tolerance checks and numpy <-> torch transfers."""

from __future__ import annotations

import numpy as np

# The floating-point bar for layer outputs against an fp32 (here float64)
# matmul on the oracle-dequantized weights: max-abs-err 2e-2 and rel-L2 1e-3.
MAX_ABS = 2e-2
REL_L2 = 1e-3


def rel_l2(got: np.ndarray, ref: np.ndarray) -> float:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(got - ref) / (den if den > 0 else 1.0))


def assert_close(got, ref, max_abs=MAX_ABS, rel=REL_L2, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    mae = float(np.abs(got - ref).max()) if got.size else 0.0
    r = rel_l2(got, ref)
    assert mae <= max_abs and r <= rel, f"{what}: max_abs={mae:.3e} rel_l2={r:.3e}"
    return mae, r


def to_dev(a: np.ndarray, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)
